"""GPU: stencils beyond the emitting pass's staging area.

A bin whose stencil holds more candidates than the emitting pass stages in
LDS (1,280 float64 or 768 float32 records) is emitted from the hit masks
with each hit's candidate record (or, for wrapped atoms, its original
position and wraps) loaded from global memory.  Dense slabs (about 0.9
atoms per cubic Angstrom at an 8 Angstrom cutoff, so stencils of 1,300 to
4,096 candidates) run every pair mode, sorted and unsorted, inside and
outside the cell (wrapped atoms), in float64, and one case in float32.
Every case compares the (i, j, S) multiset with the CPU oracle bit for bit
and D and d with the float64 formula.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests._util import assert_geometry_close, assert_same_keys, keys_of, oracle_call
from tonari_amd import neighbor_list
from tonari_amd import workloads as W

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
MODES = [(False, False), (False, True), (True, False), (True, True)]


def dense_slab(dtype, seed, n=8000, shift=0):
    rng = np.random.Generator(np.random.PCG64(seed))
    cell = W.triclinic_cell((30.0, 30.0, 30.0), (90.0, 90.0, 90.0))
    frac = np.column_stack([rng.uniform(0.0, 1.0, n), rng.uniform(0.0, 1.0, n),
                            rng.uniform(0.0, 10.0 / 30.0, n)])
    if shift:
        frac[:, :2] += rng.integers(-shift, shift + 1, (n, 2))
    return W._pack([frac @ cell], [cell], [np.array([True, True, False])], [n], dtype, 8.0)


def run(cfg, half_list, include_self, sorted_):
    full = dict(cfg, half_list=half_list, include_self=include_self)
    t = [torch.as_tensor(cfg[k]).to(DEV) for k in ("positions", "cell", "pbc")]
    bp = torch.as_tensor(cfg["batch_ptr"]).to(DEV)
    P, S, D, d = neighbor_list("PSDd", *t, cfg["cutoff"], bp, algorithm="cell_list",
                               half_list=half_list, include_self=include_self, sorted=sorted_)
    torch.cuda.synchronize()
    assert_same_keys(keys_of(P, S), keys_of(*oracle_call(full, algorithm="cell_list")))
    assert_geometry_close(P, S, d, D, full)
    if sorted_:
        src = P[:, 0]
        assert bool((src[1:] >= src[:-1]).all())


@pytest.mark.parametrize("half_list,include_self", MODES)
def test_float64_dense_slab(half_list, include_self):
    print(f"[big stencils] float64 half={half_list} self={include_self}", flush=True)
    cfg = dense_slab(np.float64, 70)
    for sorted_ in (False, True):
        run(cfg, half_list, include_self, sorted_)


@pytest.mark.parametrize("half_list,include_self", [(False, False), (True, True)])
def test_float64_wrapped_dense_slab(half_list, include_self):
    print(f"[big stencils] float64 wrapped half={half_list} self={include_self}", flush=True)
    cfg = dense_slab(np.float64, 71, shift=2)
    for sorted_ in (False, True):
        run(cfg, half_list, include_self, sorted_)


def test_float32_dense_slab_gathers():
    print("[big stencils] float32", flush=True)
    run(dense_slab(np.float32, 72), False, False, False)
