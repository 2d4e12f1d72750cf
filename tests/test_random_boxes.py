"""Seeded random single boxes against the CPU oracle, searched repeatedly on the GPU.

Each seed draws one structure large enough for a bin grid: a skewed cell
of 22 to 50 Angstrom edges at 70 to 110 degrees, periodic along every axis
or along two, 0.02 to 0.1 atoms per cubic Angstrom (at most 20,000 atoms),
atoms up to 20 % outside the cell along periodic axes, a cutoff of 2.5 to
8 Angstrom, either dtype, cell_list or auto, any pair mode and order.  The
box is searched three times on one shape: a first call, a repeat (the
plan hint, the periodic fast prologue with its grid barrier and set-up
memo, the speculative emit) and a repeat with the atoms moved.  Every
result's (i, j, S) multiset must equal the oracle's bit for bit, with d
and D within 1e-5 relative (float32) or 1e-12 (float64) of the float64
formula.  Eight of the boxes also go through the host provider (CPU suite).
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.test_random_batches import check
from tonari_amd._torch_frontend import _speculation


# plan bit of a fully periodic structure searched with a cell list: its
# repeats take the periodic fast prologue
PLAN_PERIODIC_GRID = 8


def random_box(seed: int) -> dict:
    rng = np.random.Generator(np.random.PCG64(9100 + seed))
    dtype = np.float32 if rng.random() < 0.5 else np.float64
    while True:
        lengths = rng.uniform(22.0, 50.0, 3)
        angles = np.radians(rng.uniform(70.0, 110.0, 3))
        a, b, c = lengths
        al, be, ga = angles
        cx = c * np.cos(be)
        cy = c * (np.cos(al) - np.cos(be) * np.cos(ga)) / np.sin(ga)
        cz2 = c * c - cx * cx - cy * cy
        if cz2 > (0.5 * c) ** 2:
            cell = np.array([[a, 0, 0], [b * np.cos(ga), b * np.sin(ga), 0],
                             [cx, cy, np.sqrt(cz2)]])
            break
    pbc = np.ones(3, bool) if rng.random() < 0.7 else np.array([True, True, False])
    volume = abs(np.linalg.det(cell))
    n = int(min(20_000, rng.uniform(0.02, 0.1) * volume))
    frac = rng.uniform(0.0, 1.0, (n, 3))
    frac[:, pbc] = rng.uniform(-0.2, 1.2, (n, int(pbc.sum())))
    return {
        "positions": (frac @ cell).astype(dtype),
        "cell": cell[None].astype(dtype),
        "pbc": pbc[None],
        "batch_ptr": np.array([0, n], dtype=np.int64),
        "cutoff": float(rng.uniform(2.5, 8.0)),
        "algorithm": "cell_list" if rng.random() < 0.6 else "auto",
        "half_list": bool(rng.random() < 0.4),
        "include_self": bool(rng.random() < 0.3),
        "sorted": bool(rng.random() < 0.4),
        "move": rng.normal(0.0, 0.03, (n, 3)),
    }


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(24))
def test_random_box_repeats(seed):
    cfg = random_box(seed)
    print(f"[random boxes] seed {seed} {cfg['positions'].dtype} N={len(cfg['positions'])} "
          f"rc={cfg['cutoff']:.2f} pbc={cfg['pbc'][0].tolist()} {cfg['algorithm']}", flush=True)
    moved = dict(cfg, positions=(cfg["positions"] + cfg["move"]).astype(cfg["positions"].dtype))
    _speculation().clear()
    for case in (cfg, cfg, moved):
        check(case, "cuda:0")
    (entry,) = _speculation().values()
    if cfg["algorithm"] == "cell_list" and cfg["pbc"].all():
        assert entry[1] & PLAN_PERIODIC_GRID, "the repeats did not take the periodic fast prologue"


@pytest.mark.parametrize("seed", range(8))
def test_random_box_host_provider(seed):
    check(random_box(seed), "cpu")
