"""Seeded random batches of open molecules, searched repeatedly on the GPU.

Each seed draws 1 to 400 non-periodic structures (zero cell, no periodic
axis) of 0 to 200 atoms as Gaussian clouds of random width, now and then
one of 2,100 to 2,600 atoms (beyond the molecule kernel's size, so that
the batch also takes the general brute force or a cell list), a cutoff of
1.5 to 5 Angstrom, either dtype, auto or brute_force (and cell_list for a
few), any pair mode and order.  A batch is searched three times on one
shape: first, repeated (the molecule plan hint and the molecules-only set-up
of batches up to 4,096 structures) and repeated with moved atoms.  Every
result's (i, j, S) multiset must equal the oracle's bit for bit, with d and
D within 1e-5 relative (float32) or 1e-12 (float64) of the float64 formula.
Six of the batches also go through the host provider (CPU suite).
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.test_random_batches import check



def random_molecules(seed: int) -> dict:
    rng = np.random.Generator(np.random.PCG64(12_000 + seed))
    dtype = np.float32 if rng.random() < 0.5 else np.float64
    nb = int(rng.integers(1, 401)) if rng.random() < 0.7 else int(rng.integers(1, 12))
    sizes = [int(x) for x in rng.integers(0, 201, nb)]
    if rng.random() < 0.2:
        sizes[int(rng.integers(0, nb))] = int(rng.integers(2100, 2601))
    pos = [rng.normal(0.0, rng.uniform(1.0, 8.0), (n, 3)) for n in sizes]
    n_total = sum(sizes)
    r = rng.random()
    algorithm = "auto" if r < 0.5 else "brute_force" if r < 0.9 else "cell_list"
    return {
        "positions": (np.concatenate(pos) if n_total else np.zeros((0, 3))).astype(dtype),
        "cell": np.zeros((nb, 3, 3), dtype),
        "pbc": np.zeros((nb, 3), bool),
        "batch_ptr": np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64),
        "cutoff": float(rng.uniform(1.5, 5.0)),
        "algorithm": algorithm,
        "half_list": bool(rng.random() < 0.5),
        "include_self": bool(rng.random() < 0.3),
        "sorted": bool(rng.random() < 0.5),
        "move": rng.normal(0.0, 0.05, (n_total, 3)),
    }


@pytest.mark.gpu
@pytest.mark.parametrize("block", range(6))
def test_random_molecule_batches(block):
    for seed in range(10 * block, 10 * block + 10):
        cfg = random_molecules(seed)
        print(f"[random molecules] seed {seed} {cfg['positions'].dtype} {cfg['algorithm']} "
              f"B={len(cfg['batch_ptr']) - 1} N={len(cfg['positions'])}", flush=True)
        moved = dict(cfg, positions=(cfg["positions"] + cfg["move"]).astype(
            cfg["positions"].dtype))
        for case in (cfg, cfg, moved):
            check(case, "cuda:0")


@pytest.mark.parametrize("seed", range(6))
def test_random_molecule_batches_host_provider(seed):
    check(random_molecules(seed), "cpu")
