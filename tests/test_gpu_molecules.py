"""GPU parity of the molecule form of the brute-force passes.

Brute-force structures without a periodic axis and with at most 2,048 atoms
are counted with hit masks and emitted from them.  These tests run batches
of such structures (sizes on both sides of every chunk, register-pass and
size limit of that form) through ``tonari_amd.neighbor_list`` on ``cuda:0``
and compare the (i, j, S) multiset bit-exactly with the CPU oracle; d and D
within 1e-5 relative (float32) / 1e-12 (float64).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests._util import (
    assert_geometry_close,
    assert_grouped_by_source,
    assert_same_keys,
    assert_sorted_by_source,
    keys_of,
    oracle_call,
)
from tonari_amd import neighbor_list

pytestmark = pytest.mark.gpu

DEV = "cuda:0"

# 64 targets per chunk, 8 chunks per register pass, 32 chunks at most
SIZES = [1, 2, 20, 63, 64, 65, 128, 129, 511, 512, 513, 1000, 2047, 2048, 2049]


def batch(sizes, pbcs, dtype, seed, *, density=0.06, cutoff=4.5, **options):
    rng = np.random.Generator(np.random.PCG64(seed))
    positions, cells = [], []
    for n in sizes:
        edge = (n / density) ** (1.0 / 3.0)
        positions.append(rng.random((n, 3)) * edge + rng.normal(0, 30, size=3))
        cells.append(np.diag([edge, edge, edge]) + 0.2 * np.tril(rng.random((3, 3)), -1))
    cfg = {
        "positions": np.concatenate(positions).astype(dtype),
        "cell": np.stack(cells).astype(dtype),
        "pbc": np.asarray(pbcs, dtype=bool).reshape(len(sizes), 3),
        "batch_ptr": np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64),
        "cutoff": cutoff,
    }
    cfg.update(options)
    return cfg


def gpu(quantities, cfg, **options):
    t = lambda x: torch.as_tensor(x).to(DEV)  # noqa: E731
    kw = dict(
        algorithm=cfg.get("algorithm", "brute_force"),
        sorted=cfg.get("sorted", False),
        half_list=cfg.get("half_list", False),
        include_self=cfg.get("include_self", False),
    )
    kw.update(options)
    out = neighbor_list(
        quantities, t(cfg["positions"]), t(cfg["cell"]), t(cfg["pbc"]), cfg["cutoff"],
        t(cfg["batch_ptr"]), **kw,
    )
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("half_list", [False, True])
@pytest.mark.parametrize("include_self", [False, True])
def test_molecule_sizes_match_oracle(dtype, half_list, include_self):
    cfg = batch(SIZES, [[0, 0, 0]] * len(SIZES), dtype, 4711, half_list=half_list,
                include_self=include_self)
    print(f"molecules {SIZES} {np.dtype(dtype).name} half={half_list} self={include_self}",
          flush=True)
    expected = keys_of(*oracle_call(cfg, algorithm="brute_force"))
    for sorted_ in (False, True):
        pairs, shifts, d, D = gpu("PSdD", cfg, sorted=sorted_)
        assert_same_keys(keys_of(pairs, shifts), expected)
        assert_grouped_by_source(pairs)
        if sorted_:
            assert_sorted_by_source(pairs)
        assert_geometry_close(pairs, shifts, d, D, cfg)
        assert not shifts.any()


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_molecules_mixed_with_periodic_structures(dtype):
    # molecules between periodic and partly periodic brute-force structures
    sizes = [70, 12, 300, 40, 129, 9, 64]
    pbcs = [[0, 0, 0], [1, 1, 1], [0, 0, 0], [1, 0, 1], [0, 0, 0], [1, 1, 1], [0, 0, 0]]
    for mode, (half_list, include_self) in enumerate(
            [(False, False), (False, True), (True, False), (True, True)]):
        cfg = batch(sizes, pbcs, dtype, 811 + mode, half_list=half_list,
                    include_self=include_self)
        print(f"mixed batch {np.dtype(dtype).name} mode {mode}", flush=True)
        expected = keys_of(*oracle_call(cfg, algorithm="brute_force"))
        for algorithm in ("brute_force", "auto"):
            i, j, S, d, D = gpu("ijSdD", cfg, algorithm=algorithm, sorted=True)
            pairs = torch.stack([i, j], dim=1)
            assert_same_keys(keys_of(pairs, S), expected)
            assert_sorted_by_source(pairs)
            assert_geometry_close(pairs, S, d, D, cfg)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_molecule_boundaries_and_coincident_atoms(dtype):
    # pairs exactly at the cutoff (excluded), one ulp inside (kept), coincident
    # atoms (kept, distance zero) and a large common translation, decided by
    # the public predicate itself
    rc = 2.0
    base = np.array([1.0e4, -3.0e3, 7.5e2])
    one = np.nextafter(dtype(rc), dtype(0)) if dtype == np.float32 else np.nextafter(rc, 0.0)
    pts = [
        base,
        base + [rc, 0.0, 0.0],
        base + [0.0, float(one), 0.0],
        base,
        base + [0.0, 0.0, 0.5],
        base + [1.2, 1.6, 0.0],
    ]
    pos = np.asarray(pts, dtype=dtype)
    cfg = {
        "positions": pos,
        "cell": np.zeros((1, 3, 3), dtype=dtype),
        "pbc": np.zeros((1, 3), dtype=bool),
        "batch_ptr": np.array([0, len(pos)], dtype=np.int64),
        "cutoff": rc,
    }
    for half_list in (False, True):
        for include_self in (False, True):
            c = dict(cfg, half_list=half_list, include_self=include_self)
            expected = keys_of(*oracle_call(c, algorithm="brute_force"))
            pairs, shifts, d = gpu("PSd", c)
            assert_same_keys(keys_of(pairs, shifts), expected)
            got = {(int(a), int(b)) for a, b in pairs.cpu().numpy()}
            assert (0, 3) in got and (half_list or (3, 0) in got)
            assert include_self == ((0, 0) in got)


def test_molecule_repeated_calls_with_smaller_batch():
    # the masks and lists left by one call do not leak into the next
    big = batch([700, 300, 90], [[0, 0, 0]] * 3, np.float32, 99)
    small = batch([33, 5], [[0, 0, 0]] * 2, np.float32, 98)
    for cfg in (big, small, big):
        expected = keys_of(*oracle_call(cfg, algorithm="brute_force"))
        pairs, shifts = gpu("PS", cfg)
        assert_same_keys(keys_of(pairs, shifts), expected)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_molecules_beside_cell_list_structures(dtype):
    # with algorithm 'auto', molecules of up to 2,048 atoms take the molecule
    # form and larger ones, and the periodic boxes, a cell list: both store
    # hit masks in one buffer, the molecules in slots counted down from the top
    sizes = [90, 2600, 40, 700, 2500, 120]
    pbcs = [[0, 0, 0], [0, 0, 0], [0, 0, 0], [1, 1, 1], [1, 1, 1], [0, 0, 0]]
    for mode, (half_list, include_self) in enumerate(
            [(False, False), (False, True), (True, False), (True, True)]):
        cfg = batch(sizes, pbcs, dtype, 1201 + mode, half_list=half_list,
                    include_self=include_self)
        print(f"molecules beside cell lists {np.dtype(dtype).name} mode {mode}", flush=True)
        expected = keys_of(*oracle_call(cfg, algorithm="brute_force"))
        for sorted_ in (False, True):
            pairs, shifts, d, D = gpu("PSdD", cfg, algorithm="auto", sorted=sorted_)
            assert_same_keys(keys_of(pairs, shifts), expected)
            assert_grouped_by_source(pairs)
            assert_geometry_close(pairs, shifts, d, D, cfg)
