"""GPU: the graph adapter (``tonari_amd.pyg``), the edge-first layout.

``neighbor_graph`` must give ``edge_index == P.T`` of the same search, with
D / d / S row-aligned to its columns, as the reference's PyTorch Geometric
example builds it (``README.md:81-99``), for brute-force and cell-list plans,
first and repeated calls (the repeated call writes into a buffer sized
before E is known), a pair count that outgrows the previous call's buffer,
gradients of the edge vectors, and seeded random batches with every option.
"""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from tests._util import assert_geometry_close, assert_same_keys, keys_of, oracle_call
from tonari_amd import neighbor_list
from tonari_amd import workloads as W
from tonari_amd.pyg import from_batch, neighbor_graph

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _t(cfg):
    return {k: torch.as_tensor(cfg[k]).to(DEV) for k in ("positions", "cell", "pbc", "batch_ptr")}


def _check(cfg, graph, **options):
    ei = graph.edge_index
    assert ei.dtype == torch.int64 and ei.dim() == 2 and ei.shape[0] == 2
    assert ei.is_contiguous()
    P = ei.T.contiguous()
    assert_same_keys(keys_of(P, graph.cell_shifts),
                     keys_of(*oracle_call(dict(cfg, **options), algorithm=cfg.get("algorithm"))))
    assert_geometry_close(P, graph.cell_shifts, graph.edge_lengths, graph.edge_vectors, cfg)


@pytest.mark.parametrize("name", ["C2", "C4"])
def test_graph_matches_the_oracle_first_and_repeated(name):
    cfg = W.c2(n_structures=32) if name == "C2" else W.c4(seed=41, n_atoms=8000)
    t = _t(cfg)
    for rep in range(3):
        print(f"[graph] {name} call {rep}", flush=True)
        g = neighbor_graph(t["positions"], t["cell"], t["pbc"], cfg["cutoff"], t["batch_ptr"],
                           lengths=True, shifts=True, algorithm=cfg["algorithm"])
        torch.cuda.synchronize()
        _check(cfg, g)


def test_graph_equals_the_transposed_pairs_of_the_same_call_shape():
    cfg = W.c2(n_structures=24)
    t = _t(cfg)
    P, D = neighbor_list("PD", t["positions"], t["cell"], t["pbc"], cfg["cutoff"],
                         t["batch_ptr"], algorithm="brute_force")
    g = neighbor_graph(t["positions"], t["cell"], t["pbc"], cfg["cutoff"], t["batch_ptr"],
                       algorithm="brute_force")
    torch.cuda.synchronize()
    # brute-force outputs come in source order; within a source compare sorted rows
    a = torch.cat([P, D], 1).cpu().numpy()
    b = torch.cat([g.edge_index.T.to(D.dtype), g.edge_vectors], 1).cpu().numpy()
    assert np.array_equal(a[np.lexsort(a.T[::-1])], b[np.lexsort(b.T[::-1])])
    assert g.edge_lengths is None and g.cell_shifts is None


def test_graph_when_the_pair_count_outgrows_the_last_buffer():
    sparse = W.c4(seed=42, n_atoms=5000, density=0.02)
    dense = W.c4(seed=43, n_atoms=5000, density=0.1)
    for cfg in (sparse, dense, dense, sparse):
        t = _t(cfg)
        g = neighbor_graph(t["positions"], t["cell"], t["pbc"], cfg["cutoff"], t["batch_ptr"],
                           shifts=True, algorithm="cell_list", half_list=True)
        torch.cuda.synchronize()
        _check(cfg, g, half_list=True)


def test_graph_vectors_carry_gradients():
    cfg = W.c2(n_structures=8)
    t = _t(cfg)
    pos = t["positions"].double().requires_grad_()
    cell = t["cell"].double().requires_grad_()
    g = neighbor_graph(pos, cell, t["pbc"], cfg["cutoff"], t["batch_ptr"], lengths=True)
    (g.edge_vectors.sum() + g.edge_lengths.sum()).backward()
    gp, gc = pos.grad.clone(), cell.grad.clone()
    pos.grad = None
    cell.grad = None
    P, D, d = neighbor_list("PDd", pos, cell, t["pbc"], cfg["cutoff"], t["batch_ptr"])
    (D.sum() + d.sum()).backward()
    assert torch.allclose(gp, pos.grad, rtol=1e-10, atol=1e-10)
    assert torch.allclose(gc, cell.grad, rtol=1e-10, atol=1e-10)
    assert g.edge_index.shape[1] == P.shape[0] > 0


def test_from_batch_follows_the_readme_example():
    cfg = W.c2(n_structures=16)
    t = _t(cfg)
    batch = SimpleNamespace(pos=t["positions"], cell=t["cell"], pbc=t["pbc"], ptr=t["batch_ptr"])
    g = from_batch(batch, cfg["cutoff"], shifts=True)
    pairs, edge_vectors = neighbor_list("PD", batch.pos, batch.cell, batch.pbc,
                                        cutoff=cfg["cutoff"], batch_ptr=batch.ptr)
    torch.cuda.synchronize()
    assert g.edge_index.shape == pairs.T.shape
    _check(dict(cfg, algorithm="auto"), g)


@pytest.mark.parametrize("block", range(4))
def test_graph_on_random_batches(block):
    # the seeded random batches of tests/test_random_batches.py, each built
    # twice (first and repeated call of the shape), with every option of
    # the search, against the oracle
    from tests.test_random_batches import random_batch
    from tests.test_random_reuse import _usable

    for seed in range(15 * block, 15 * block + 15):
        cfg = random_batch(seed)
        if not _usable(cfg):
            continue
        print(f"[graph] random batch {seed}", flush=True)
        t = _t(cfg)
        options = {k: cfg[k] for k in ("half_list", "include_self", "sorted")}
        for _ in range(2):
            g = neighbor_graph(t["positions"], t["cell"], t["pbc"], cfg["cutoff"],
                               t["batch_ptr"], lengths=True, shifts=True,
                               algorithm=cfg["algorithm"], **options)
            torch.cuda.synchronize()
            _check(cfg, g)
