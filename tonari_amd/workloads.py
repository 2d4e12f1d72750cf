"""Seeded synthetic inputs for the five benchmark configurations.

Every generator draws with numpy's PCG64 from an explicit seed, builds the
geometry in float64 and casts at the end, so the CPU baseline and the GPU
path see identical arrays.  Each returns a dict with ``positions`` (N, 3),
``cell`` (B, 3, 3), ``pbc`` (B, 3) bool, ``batch_ptr`` (B + 1) int64,
``cutoff`` and the call options of the configuration.

C1  512-atom cubic box, float64, rc 5, 'ijSdD', brute_force and cell_list
C2  256 triclinic crystals (2-64 atoms), float32, rc 6, brute_force, 'PSD'
C3  1024 Gaussian molecules (20-120 atoms), float32, rc 5, half+sorted, 'ijd'
C4  100k-atom periodic box (100 A edge), float32, rc 6, cell_list, 'PD'
C5  64 triclinic slabs (2k-20k atoms), float64, pbc TTF, rc 8,
    include_self+sorted, 'ijSdD'
"""

from __future__ import annotations

import math

import numpy as np


def triclinic_cell(lengths, angles_deg) -> np.ndarray:
    """Rows a, b, c from lengths and (alpha, beta, gamma) in degrees."""
    a, b, c = lengths
    al, be, ga = (math.radians(x) for x in angles_deg)
    ca, cb, cg, sg = math.cos(al), math.cos(be), math.cos(ga), math.sin(ga)
    cy = (ca - cb * cg) / sg
    cz2 = 1.0 - cb * cb - cy * cy
    return np.array(
        [[a, 0.0, 0.0], [b * cg, b * sg, 0.0], [c * cb, c * cy, c * math.sqrt(cz2)]],
        dtype=np.float64,
    )


def _volume_factor(angles_deg) -> float:
    ca, cb, cg = (math.cos(math.radians(x)) for x in angles_deg)
    return 1.0 - ca * ca - cb * cb - cg * cg + 2.0 * ca * cb * cg


def _pack(positions, cells, pbc, counts, dtype, cutoff, **options):
    batch_ptr = np.zeros(len(counts) + 1, dtype=np.int64)
    batch_ptr[1:] = np.cumsum(counts)
    return {
        "positions": np.ascontiguousarray(np.concatenate(positions).astype(dtype)),
        "cell": np.ascontiguousarray(np.stack(cells).astype(dtype)),
        "pbc": np.ascontiguousarray(np.stack(pbc).astype(bool)),
        "batch_ptr": batch_ptr,
        "cutoff": float(cutoff),
        **options,
    }


def c1(seed: int = 1001) -> dict:
    rng = np.random.Generator(np.random.PCG64(seed))
    pos = rng.uniform(0.0, 20.0, size=(512, 3))
    return _pack([pos], [20.0 * np.eye(3)], [np.ones(3, bool)], [512], np.float64, 5.0,
                 quantities="ijSdD", algorithm="brute_force", half_list=False,
                 include_self=False, sorted=False)


def c2(seed: int = 1002, n_structures: int = 256) -> dict:
    rng = np.random.Generator(np.random.PCG64(seed))
    positions, cells, pbcs, counts = [], [], [], []
    for _ in range(n_structures):
        n = int(rng.integers(2, 65))
        while True:
            lengths = rng.uniform(3.0, 12.0, size=3)
            angles = rng.uniform(60.0, 120.0, size=3)
            if _volume_factor(angles) > 1e-3:
                break
        cell = triclinic_cell(lengths, angles)
        frac = rng.uniform(0.0, 1.0, size=(n, 3))
        positions.append(frac @ cell)
        cells.append(cell)
        pbcs.append(np.ones(3, bool))
        counts.append(n)
    return _pack(positions, cells, pbcs, counts, np.float32, 6.0, quantities="PSD",
                 algorithm="brute_force", half_list=False, include_self=False, sorted=False)


def _gaussian_molecule(rng, n: int, sigma: float = 3.0, dmin: float = 1.0) -> np.ndarray:
    atoms = np.empty((n, 3))
    k = 0
    while k < n:
        x = rng.normal(0.0, sigma, size=3)
        if k == 0 or np.min(np.sum((atoms[:k] - x) ** 2, axis=1)) >= dmin * dmin:
            atoms[k] = x
            k += 1
    return atoms


def c3(seed: int = 1003, n_structures: int = 1024) -> dict:
    rng = np.random.Generator(np.random.PCG64(seed))
    positions, cells, pbcs, counts = [], [], [], []
    for _ in range(n_structures):
        n = int(rng.integers(20, 121))
        positions.append(_gaussian_molecule(rng, n))
        cells.append(np.zeros((3, 3)))
        pbcs.append(np.zeros(3, bool))
        counts.append(n)
    return _pack(positions, cells, pbcs, counts, np.float32, 5.0, quantities="ijd",
                 algorithm="auto", half_list=True, include_self=False, sorted=True)


def c4(seed: int = 1004, n_atoms: int = 100_000, density: float = 0.1) -> dict:
    rng = np.random.Generator(np.random.PCG64(seed))
    edge = (n_atoms / density) ** (1.0 / 3.0)
    pos = rng.uniform(0.0, edge, size=(n_atoms, 3))
    return _pack([pos], [edge * np.eye(3)], [np.ones(3, bool)], [n_atoms], np.float32, 6.0,
                 quantities="PD", algorithm="cell_list", half_list=False,
                 include_self=False, sorted=False)


def c5(seed: int = 1005, n_structures: int = 64, n_min: int = 2000, n_max: int = 20000) -> dict:
    rng = np.random.Generator(np.random.PCG64(seed))
    positions, cells, pbcs, counts = [], [], [], []
    for _ in range(n_structures):
        n = int(round(math.exp(rng.uniform(math.log(n_min), math.log(n_max)))))
        while True:
            a, b, slab = rng.uniform(30.0, 60.0, size=3)
            angles = rng.uniform(70.0, 110.0, size=3)
            if _volume_factor(angles) > 1e-3:
                break
        c = slab + 20.0
        cell = triclinic_cell((a, b, c), angles)
        frac = np.column_stack([
            rng.uniform(0.0, 1.0, size=n),
            rng.uniform(0.0, 1.0, size=n),
            rng.uniform(0.0, slab / c, size=n),
        ])
        positions.append(frac @ cell)
        cells.append(cell)
        pbcs.append(np.array([True, True, False]))
        counts.append(n)
    return _pack(positions, cells, pbcs, counts, np.float64, 8.0, quantities="ijSdD",
                 algorithm="auto", half_list=False, include_self=True, sorted=True)


CONFIGS = {"C1": c1, "C2": c2, "C3": c3, "C4": c4, "C5": c5}


def algorithmic_bytes(n_atoms: int, n_pairs: int, quantities: str, itemsize: int) -> int:
    """B_alg = N*3*s + sum over requested quantities of E*w_q (repeats count again).

    w_i = w_j = 8, w_P = 16, w_S = 12, w_d = s, w_D = 3s.
    """
    width = {"i": 8, "j": 8, "P": 16, "S": 12, "d": itemsize, "D": 3 * itemsize}
    return n_atoms * 3 * itemsize + sum(n_pairs * width[q] for q in quantities)
