"""GPU: the batch set-up taken from the memo of an earlier request.

``k_setup`` keeps each structure's record (batch_ptr checks, pseudo-inverse
of the active rows, image repeats, grid frame) in a memo entry of the
workspace, keyed by every input it depends on and checked by a checksum;
a later request on the same workspace takes the record from the memo when
the key matches and derives it again when any input differs.  These cases
run a batch of skewed crystals and open clusters through the C ABI on one
workspace, repeating it and changing one input at a time (moved atoms, one
structure's cell, the cutoff, a structure's periodicity, an atom moved
from one structure to the next), in both dtypes and with both algorithms,
and compare every result's (i, j, S) multiset with the CPU oracle bit for
bit and D with the float64 formula.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests._util import assert_geometry_close, assert_same_keys, keys_of, oracle_call
from tests.test_gpu_periodic_prologue import search
from tonari_amd import workloads as W
from tonari_amd._extensions import TNR_OK

pytestmark = pytest.mark.gpu


def batch(dtype, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    sizes = [int(x) for x in rng.integers(20, 140, size=24)]
    cells, pos, pbc = [], [], []
    for k, n in enumerate(sizes):
        if k % 5 == 4:
            cells.append(np.zeros((3, 3)))
            pos.append(rng.uniform(0.0, 12.0, (n, 3)))
            pbc.append(np.zeros(3, bool))
        else:
            lengths = rng.uniform(8.0, 14.0, 3)
            angles = rng.uniform(70.0, 110.0, 3)
            cell = W.triclinic_cell(tuple(lengths), tuple(angles))
            cells.append(cell)
            pos.append(rng.uniform(0.0, 1.0, (n, 3)) @ cell)
            pbc.append(np.ones(3, bool))
    return W._pack(pos, cells, pbc, sizes, dtype, 5.0)


def check(cfg, keep, algorithm):
    full = dict(cfg, half_list=False, include_self=False)
    code, msg, plan, P, S, D = search(full, -1, algorithm=algorithm, keep=keep)
    assert code == TNR_OK, msg
    assert_same_keys(keys_of(P, S), keys_of(*oracle_call(full, algorithm=algorithm)))
    assert_geometry_close(P, S, None, D, full)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("algorithm", ["brute_force", "cell_list"])
def test_batch_repeats_on_one_workspace(dtype, algorithm):
    print(f"[setup memo] {np.dtype(dtype).name} {algorithm}", flush=True)
    base = batch(dtype, 60)
    rng = np.random.Generator(np.random.PCG64(61))
    moved = dict(base, positions=(base["positions"]
                                  + rng.normal(0.0, 0.2, base["positions"].shape)).astype(dtype))
    cells = base["cell"].copy()
    cells[3] = (cells[3] * 1.03).astype(dtype)
    recelled = dict(base, cell=cells)
    shorter = dict(base, cutoff=4.5)
    pbc = base["pbc"].copy()
    pbc[2] = [True, False, True]
    reperiod = dict(base, pbc=pbc)
    bp = base["batch_ptr"].copy()
    bp[7] += 1  # the first atom of structure 7 now ends structure 6
    rebatched = dict(base, batch_ptr=bp)
    keep = {}
    for cfg in (base, base, moved, recelled, recelled, shorter, reperiod, rebatched, base):
        check(cfg, keep, algorithm)
