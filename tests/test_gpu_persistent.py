"""GPU: the persistent, graph-capturable plan (tonari_amd.persistent).

NeighborListPlan enqueues the count and the writing pass without waiting for
the pair count, into outputs of a fixed capacity, reading the plan and bins
on the device.  Its first E rows must be the public call's pairs (the same
(i, j, S) multiset, d/D within the stated tolerance) eagerly and when
captured in a HIP graph and replayed on new positions: every replay is
checked against an eager public call, with eager work between replays.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests._util import assert_same_keys, keys_of
from tonari_amd import neighbor_list
from tonari_amd import workloads as W
from tonari_amd.persistent import NeighborListPlan

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def tensors(cfg, dtype=None):
    t = {k: torch.as_tensor(cfg[k]).to(DEV) for k in ("positions", "cell", "pbc", "batch_ptr")}
    if dtype is not None:
        t["positions"] = t["positions"].to(dtype)
        t["cell"] = t["cell"].to(dtype)
    return t


def check_rows(plan, t, cfg, **kw):
    E = int(plan.n_pairs.item())
    assert E <= plan.capacity
    P, S, D = (x[:E] for x in plan.outputs)
    Pr, Sr, Dr = neighbor_list("PSD", t["positions"], t["cell"], t["pbc"], cfg["cutoff"],
                               t["batch_ptr"], **kw)
    assert_same_keys(keys_of(P, S), keys_of(Pr, Sr))
    # D of the same key in both
    a = np.column_stack([P.cpu().numpy(), S.cpu().numpy()])
    b = np.column_stack([Pr.cpu().numpy(), Sr.cpu().numpy()])
    ia, ib = np.lexsort(a.T[::-1]), np.lexsort(b.T[::-1])
    tol = 1e-5 if t["positions"].dtype == torch.float32 else 1e-12
    Da, Db = D.double().cpu().numpy()[ia], Dr.double().cpu().numpy()[ib]
    assert np.max(np.abs(Da - Db)) <= tol * max(1.0, float(np.max(np.abs(Db))))


@pytest.mark.parametrize("name,kw", [
    ("C4s", dict(algorithm="cell_list")),
    ("C2s", dict(algorithm="brute_force")),
    ("C3s", dict(algorithm="auto", half_list=True, sorted=True)),
])
def test_eager_rows_match_public_call(name, kw):
    cfg = {"C4s": lambda: W.c4(n_atoms=6000), "C2s": lambda: W.c2(n_structures=20),
           "C3s": lambda: W.c3(n_structures=40)}[name]()
    t = tensors(cfg)
    plan = NeighborListPlan("PSD", t["positions"], t["cell"], t["pbc"], cfg["cutoff"],
                            t["batch_ptr"], capacity=2_000_000, **kw)
    plan.run()
    E = plan.check()
    assert E > 0
    check_rows(plan, t, cfg, **kw)


def test_graph_replays_follow_new_positions():
    cfg = W.c4(n_atoms=8000)
    t = tensors(cfg)
    plan = NeighborListPlan("PSD", t["positions"], t["cell"], t["pbc"], cfg["cutoff"],
                            t["batch_ptr"], capacity=1_500_000, algorithm="cell_list")
    # warm-up on a side stream, as torch asks before a capture
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        plan.run()
    torch.cuda.current_stream().wait_stream(side)
    plan.check()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.run()
    base = plan.positions.clone()
    gen = torch.Generator(device=DEV).manual_seed(5)
    for replay in range(4):
        moved = base + 0.3 * torch.randn(base.shape, generator=gen, device=DEV,
                                         dtype=base.dtype)
        plan.positions.copy_(moved)
        graph.replay()
        torch.cuda.synchronize()
        check_rows(plan, dict(t, positions=moved.clone()), cfg, algorithm="cell_list")
        # eager work between replays
        neighbor_list("P", moved, t["cell"], t["pbc"], cfg["cutoff"], t["batch_ptr"])
        torch.cuda.synchronize()


def test_overflow_is_reported():
    cfg = W.c4(n_atoms=4000)
    t = tensors(cfg)
    plan = NeighborListPlan("PS", t["positions"], t["cell"], t["pbc"], cfg["cutoff"],
                            t["batch_ptr"], capacity=1000, algorithm="cell_list")
    plan.run()
    with pytest.raises(RuntimeError, match="exceeds the plan's capacity"):
        plan.check()
    assert int(plan.n_pairs.item()) > 1000
