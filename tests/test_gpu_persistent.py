"""GPU: the persistent, graph-capturable plan (tonari_amd.persistent).

NeighborListPlan enqueues the count and the writing pass without waiting for
the pair count, into outputs of a fixed capacity, reading the plan and bins
on the device (``tnr_emit`` with ``plan = -1``: the strided cell-list emit
``k_cell_emit<T, MODE, true>`` and the brute-force ``k_brute<write>`` over a
grid the device holds at once).  The reference lists this path as
unsupported (``docs/design.md:125-127``), so the CPU oracle is the only
anchor: the first E rows must be the oracle's (i, j, S) multiset bit for bit,
and D must follow the float64 reference formula within the stated tolerance
(1e-5 relative for float32, 1e-12 for float64), eagerly and in every replay
of a captured HIP graph on new positions (atoms moved across the cell
faces, so wrapped), with eager work between the replays.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests._util import assert_geometry_close, assert_same_keys, keys_of, oracle_call
from tonari_amd import neighbor_list
from tonari_amd import workloads as W
from tonari_amd.persistent import NeighborListPlan

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def tensors(cfg):
    return {k: torch.as_tensor(cfg[k]).to(DEV) for k in ("positions", "cell", "pbc", "batch_ptr")}


def check_against_oracle(plan, cfg, algorithm):
    """Rows [:E] of the plan against the oracle on cfg's inputs."""
    E = int(plan.n_pairs.item())
    assert 0 < E <= plan.capacity
    P, S, D = (x[:E] for x in plan.outputs)
    exp_p, exp_s = oracle_call(cfg, algorithm=algorithm)
    assert_same_keys(keys_of(P, S), keys_of(exp_p, exp_s))
    assert_geometry_close(P, S, None, D, cfg)
    return E


CASES = {
    # cell list, one structure, float32 (C4 at 6,000 atoms)
    "C4s": (lambda: W.c4(n_atoms=6000), dict(algorithm="cell_list")),
    # periodic brute force, a batch of triclinic crystals (C2's generator)
    "C2s": (lambda: W.c2(n_structures=20), dict(algorithm="brute_force")),
    # molecules, half list, sorted (C3's generator; auto plans them as brute force)
    "C3s": (lambda: W.c3(n_structures=40), dict(algorithm="auto", half_list=True, sorted=True)),
    # wrapped slabs, float64, include_self, sorted (C5's generator, small)
    "C5s": (lambda: W.c5(n_structures=3, n_min=400, n_max=1500),
            dict(algorithm="cell_list", include_self=True, sorted=True)),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_eager_rows_match_oracle(name):
    make, kw = CASES[name]
    cfg = dict(make(), **{k: v for k, v in kw.items() if k != "algorithm"})
    t = tensors(cfg)
    plan = NeighborListPlan("PSD", t["positions"], t["cell"], t["pbc"], cfg["cutoff"],
                            t["batch_ptr"], capacity=3_000_000, **kw)
    plan.run()
    E = plan.check()
    assert E == check_against_oracle(plan, cfg, kw["algorithm"])
    # twice on the same workspace: the second run starts from the first's state
    plan.run()
    assert plan.check() == E
    check_against_oracle(plan, cfg, kw["algorithm"])


@pytest.mark.parametrize("name,sigma", [("C4s", 0.3), ("C2s", 0.2), ("C3s", 0.2)])
def test_graph_replays_match_oracle(name, sigma):
    make, kw = CASES[name]
    cfg = dict(make(), **{k: v for k, v in kw.items() if k != "algorithm"})
    if name == "C4s":
        cfg = W.c4(n_atoms=8000)
    t = tensors(cfg)
    plan = NeighborListPlan("PSD", t["positions"], t["cell"], t["pbc"], cfg["cutoff"],
                            t["batch_ptr"], capacity=2_500_000, **kw)
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
    base = cfg["positions"].copy()
    rng = np.random.Generator(np.random.PCG64(5))
    for replay in range(3):
        moved = (base + sigma * rng.standard_normal(base.shape)).astype(base.dtype)
        plan.positions.copy_(torch.as_tensor(moved).to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        check_against_oracle(plan, dict(cfg, positions=moved), kw["algorithm"])
        # eager work between replays
        neighbor_list("P", plan.positions.clone(), t["cell"], t["pbc"], cfg["cutoff"],
                      t["batch_ptr"])
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
