"""Seeded random batches against the CPU oracle, on the host provider and on the GPU.

Each seed draws a batch of one to five structures: triclinic cells of 2 to 12
Angstrom edges and 60 to 120 degree angles with a random periodicity per
axis (atoms up to 30 % outside the cell along periodic axes, so that many
are wrapped), or open clusters with a zero cell; 0 to 70 atoms each; a
cutoff of 1 to 7 Angstrom (up to several periodic images per axis); float32
or float64; any algorithm, pair mode and order.  The (i, j, S) multiset must
equal the oracle's for the same algorithm bit for bit, with d and D within
1e-5 relative (float32) or 1e-12 (float64) of the float64 formula; where the
oracle refuses an explicit cell_list request, the call must raise the same
message.  On the GPU every batch is searched twice, the second time with the
atoms moved, so that repeated calls (the speculative emit and the plan
hints) are covered too.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests._util import (
    assert_geometry_close,
    assert_same_keys,
    assert_sorted_by_source,
    keys_of,
    oracle_call,
)
from tonari_amd import neighbor_list

ALGORITHMS = ("auto", "brute_force", "cell_list")


def _cell(rng) -> np.ndarray:
    a, b, c = rng.uniform(2.0, 12.0, 3)
    al, be, ga = np.radians(rng.uniform(60.0, 120.0, 3))
    v1 = np.array([a, 0.0, 0.0])
    v2 = np.array([b * np.cos(ga), b * np.sin(ga), 0.0])
    cx = c * np.cos(be)
    cy = c * (np.cos(al) - np.cos(be) * np.cos(ga)) / np.sin(ga)
    cz2 = c * c - cx * cx - cy * cy
    if cz2 < (0.2 * c) ** 2:  # angles that close no cell: a flatter, valid one
        cz2 = (0.2 * c) ** 2
    return np.array([v1, v2, [cx, cy, np.sqrt(cz2)]])


def random_batch(seed: int) -> dict:
    rng = np.random.Generator(np.random.PCG64(7700 + seed))
    dtype = np.float32 if rng.random() < 0.5 else np.float64
    nb = int(rng.integers(1, 6))
    cells, pbcs, pos, sizes = [], [], [], []
    for _ in range(nb):
        n = int(rng.integers(0, 71))
        if rng.random() < 0.25:
            cell = np.zeros((3, 3))
            pbc = np.zeros(3, bool)
            x = rng.normal(0.0, 3.0, (n, 3))
        else:
            cell = _cell(rng)
            pbc = rng.random(3) < 0.7
            frac = rng.uniform(0.0, 1.0, (n, 3))
            frac[:, pbc] = rng.uniform(-0.3, 1.3, (n, int(pbc.sum())))
            x = frac @ cell
        cells.append(cell)
        pbcs.append(pbc)
        pos.append(x)
        sizes.append(n)
    algorithm = ALGORITHMS[int(rng.integers(0, 3))]
    return {
        "positions": np.concatenate(pos).astype(dtype).reshape(-1, 3),
        "cell": np.stack(cells).astype(dtype),
        "pbc": np.stack(pbcs),
        "batch_ptr": np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64),
        "cutoff": float(rng.uniform(1.0, 7.0)),
        "algorithm": algorithm,
        "half_list": bool(rng.random() < 0.5),
        "include_self": bool(rng.random() < 0.3),
        "sorted": bool(rng.random() < 0.5),
        "move": rng.normal(0.0, 0.05, (sum(sizes), 3)),
    }


def _search(cfg: dict, device: str):
    t = lambda x: torch.as_tensor(x).to(device)  # noqa: E731
    out = neighbor_list(
        "PSdD", t(cfg["positions"]), t(cfg["cell"]), t(cfg["pbc"]), cfg["cutoff"],
        t(cfg["batch_ptr"]), algorithm=cfg["algorithm"], sorted=cfg["sorted"],
        half_list=cfg["half_list"], include_self=cfg["include_self"],
    )
    if device != "cpu":
        torch.cuda.synchronize()
    return out


def check(cfg: dict, device: str) -> None:
    try:
        expected = keys_of(*oracle_call(cfg))
    except oracle.OracleSearchError as refusal:
        with pytest.raises(RuntimeError) as error:
            _search(cfg, device)
        assert str(error.value) == str(refusal)
        return
    P, S, d, D = _search(cfg, device)
    assert_same_keys(keys_of(P, S), expected)
    assert_geometry_close(P, S, d, D, cfg)
    if cfg["sorted"]:
        assert_sorted_by_source(P)


@pytest.mark.parametrize("block", range(20))
def test_random_batches_host_provider(block):
    for seed in range(10 * block, 10 * block + 10):
        check(random_batch(seed), "cpu")


@pytest.mark.gpu
@pytest.mark.parametrize("block", range(40))
def test_random_batches_gpu(block):
    for seed in range(25 * block, 25 * block + 25):
        cfg = random_batch(seed)
        print(f"[random batches] seed {seed} {cfg['positions'].dtype} {cfg['algorithm']} "
              f"B={len(cfg['batch_ptr']) - 1} N={len(cfg['positions'])}", flush=True)
        check(cfg, "cuda:0")
        moved = dict(cfg, positions=(cfg["positions"] + cfg["move"]).astype(
            cfg["positions"].dtype))
        check(moved, "cuda:0")
