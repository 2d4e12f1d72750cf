"""GPU: brute force on cells that stress the image pruning, against the oracle.

The brute-force kernels visit, per (source, target) pair and row (k0, k1)
of the image box, only the k2 whose translate can fall within the padded
cutoff (a widened closest-approach bound), instead of the whole box.  These
batches make that bound work hard: short and strongly skewed cell vectors
(angles 35-145 degrees, so rows are long and nearly parallel to c2), cutoffs
of several cell lengths (hundreds of images), every periodicity pattern,
unwrapped atoms, both dtypes and every pair mode.  The (i, j, S) multiset
must equal the CPU oracle's bit for bit, with d and D within the stated
tolerance.
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

PBC = [(True, True, True), (True, True, False), (True, False, True), (False, True, True),
       (True, False, False), (False, False, True), (False, False, False)]


def skewed_batch(seed: int, dtype, n_structures: int = 12) -> dict:
    rng = np.random.Generator(np.random.PCG64(seed))
    positions, cells, pbcs, counts = [], [], [], []
    for k in range(n_structures):
        while True:
            lengths = rng.uniform(0.9, 3.5, size=3)
            angles = rng.uniform(35.0, 145.0, size=3)
            try:
                cell = W.triclinic_cell(lengths, angles)
            except (ValueError, FloatingPointError):
                continue
            if np.all(np.isfinite(cell)) and abs(np.linalg.det(cell)) > 0.05 * np.prod(lengths):
                break
        n = int(rng.integers(1, 9))
        frac = rng.random((n, 3)) + rng.integers(-2, 3, size=(n, 3)) * (rng.random((n, 1)) < 0.3)
        positions.append(frac @ cell)
        cells.append(cell)
        pbcs.append(PBC[k % len(PBC)])
        counts.append(n)
    return {
        "positions": np.concatenate(positions).astype(dtype),
        "cell": np.stack(cells).astype(dtype),
        "pbc": np.array(pbcs),
        "batch_ptr": np.concatenate([[0], np.cumsum(counts)]).astype(np.int64),
        "cutoff": float(rng.uniform(2.5, 4.5)),
    }


@pytest.mark.parametrize("seed", [101, 202, 303])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("half_list,include_self", [(False, False), (True, False),
                                                     (False, True), (True, True)])
def test_skewed_cells_match_oracle(seed, dtype, half_list, include_self):
    cfg = skewed_batch(seed, dtype)
    cfg.update(half_list=half_list, include_self=include_self)
    t = lambda x: torch.as_tensor(x).to(DEV)  # noqa: E731
    P, S, d, D = neighbor_list(
        "PSdD", t(cfg["positions"]), t(cfg["cell"]), t(cfg["pbc"]), cfg["cutoff"],
        t(cfg["batch_ptr"]), algorithm="brute_force", half_list=half_list,
        include_self=include_self,
    )
    torch.cuda.synchronize()
    expected = keys_of(*oracle_call(cfg, algorithm="brute_force"))
    assert len(expected) > 0
    assert_same_keys(keys_of(P, S), expected)
    assert_geometry_close(P, S, d, D, cfg)
