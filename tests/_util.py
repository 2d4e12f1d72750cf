"""Shared helpers for the test suite (parity checks against the CPU oracle)."""

from __future__ import annotations

import numpy as np

import oracle


def keys_of(pairs, shifts) -> np.ndarray:
    """Canonically sorted (i, j, Sx, Sy, Sz) rows; asserts there are no duplicates."""
    p = pairs.detach().cpu().numpy() if hasattr(pairs, "detach") else np.asarray(pairs)
    s = shifts.detach().cpu().numpy() if hasattr(shifts, "detach") else np.asarray(shifts)
    assert p.dtype == np.int64 and s.dtype == np.int32
    assert p.ndim == 2 and p.shape[1] == 2 and s.shape == (len(p), 3)
    keys = oracle.canonical_keys(p, s)
    if len(keys) > 1:
        dup = np.all(keys[1:] == keys[:-1], axis=1)
        assert not dup.any(), "neighbor list contains duplicate pair identities"
    return keys


def key_set(pairs, shifts) -> set[tuple[int, ...]]:
    return {tuple(int(x) for x in row) for row in keys_of(pairs, shifts)}


def assert_same_keys(actual: np.ndarray, expected: np.ndarray) -> None:
    if actual.shape == expected.shape and np.array_equal(actual, expected):
        return
    a = {tuple(r) for r in actual.tolist()}
    e = {tuple(r) for r in expected.tolist()}
    missing = sorted(e - a)[:10]
    extra = sorted(a - e)[:10]
    raise AssertionError(
        f"pair sets differ: {len(actual)} vs {len(expected)} pairs; "
        f"missing {missing} extra {extra}"
    )


def assert_sorted_by_source(pairs) -> None:
    src = pairs[:, 0]
    if hasattr(src, "detach"):
        assert bool((src[1:] >= src[:-1]).all())
        return
    src = np.asarray(src)
    assert np.all(src[1:] >= src[:-1])


def assert_grouped_by_source(pairs) -> None:
    """The pairs of every source form one contiguous run."""
    src = pairs[:, 0]
    if hasattr(src, "detach"):
        src = src.detach().cpu().numpy()
    src = np.asarray(src)
    if len(src) == 0:
        return
    runs = 1 + int(np.count_nonzero(src[1:] != src[:-1]))
    assert runs == len(np.unique(src)), "pairs of a source are not contiguous"


def oracle_call(cfg: dict, *, algorithm: str | None = None, threads: int = 8, kind: str = "port"):
    return oracle.neighbor_pairs(
        cfg["positions"], cfg["cell"], cfg["pbc"], cfg["cutoff"], cfg["batch_ptr"],
        half_list=cfg.get("half_list", False), include_self=cfg.get("include_self", False),
        algorithm=algorithm or cfg.get("algorithm", "auto"), threads=threads, kind=kind,
    )


def geometry_tolerance(dtype) -> float:
    """d/D agreement bound from the specification: 1e-5 relative (fp32), 1e-12 (fp64)."""
    return 1e-5 if np.dtype(dtype) == np.float32 else 1e-12


def assert_geometry_close(pairs, shifts, d, D, cfg) -> None:
    """Check d and D of each pair against the reference formula D = x[j]-x[i]+S@cell[b].

    Tolerance: |D - D_ref| <= rtol * (|D_ref| + cutoff) componentwise and the same
    for d, with rtol 1e-5 for float32 and 1e-12 for float64; the reference
    formula is evaluated in float64 from the same inputs.
    """
    pos = cfg["positions"].astype(np.float64)
    cell = cfg["cell"].astype(np.float64)
    bp = cfg["batch_ptr"]
    p = pairs.detach().cpu().numpy() if hasattr(pairs, "detach") else pairs
    s = shifts.detach().cpu().numpy() if hasattr(shifts, "detach") else shifts
    b = np.searchsorted(bp[1:], p[:, 0], side="right")
    ref = pos[p[:, 1]] - pos[p[:, 0]] + np.einsum("ei,eij->ej", s.astype(np.float64), cell[b])
    rtol = geometry_tolerance(cfg["positions"].dtype)
    scale = np.abs(ref) + cfg["cutoff"]
    if D is not None:
        Dn = D.detach().cpu().numpy().astype(np.float64)
        bad = np.abs(Dn - ref) > rtol * scale
        assert not bad.any(), f"D differs at {np.argwhere(bad)[:5].tolist()}"
    if d is not None:
        dn = d.detach().cpu().numpy().astype(np.float64)
        dref = np.sqrt(np.sum(ref * ref, axis=1))
        bad = np.abs(dn - dref) > rtol * (dref + cfg["cutoff"])
        assert not bad.any(), f"d differs at {np.argwhere(bad)[:5].tolist()}"


def _signed(k: int) -> int:
    return k - (1 << 64) if k >= (1 << 63) else k


def multiset_hash_torch(pairs, shifts) -> int:
    """``oracle.multiset_hash`` evaluated with torch int64 ops on the tensors' device.

    int64 multiplication, xor and addition wrap modulo 2^64 exactly like the
    uint64 arithmetic of the numpy version; the logical right shift is an
    arithmetic shift masked to the low 64 - k bits.
    """
    import torch

    from oracle import _MIX

    def shr(x, k):
        return (x >> k) & ((1 << (64 - k)) - 1)

    mul1 = _signed(_MIX[1])
    cols = [pairs[:, 0], pairs[:, 1], shifts[:, 0], shifts[:, 1], shifts[:, 2]]
    x = torch.zeros(pairs.shape[0], dtype=torch.int64, device=pairs.device)
    for c, k in zip(cols, _MIX):
        x = (x ^ (c.to(torch.int64) * _signed(k))) * mul1
        x = x ^ shr(x, 31)
    x = x ^ shr(x, 30)
    x = x * mul1
    x = x ^ shr(x, 27)
    x = x * _signed(_MIX[2])
    x = x ^ shr(x, 31)
    return int(x.sum().item()) & ((1 << 64) - 1)


def assert_geometry_close_torch(pairs, shifts, d, D, cfg, chunk: int = 1 << 24) -> None:
    """``assert_geometry_close`` evaluated on the tensors' device, every row.

    The reference formula D = x[j] - x[i] + S @ cell[b] is evaluated in float64
    on the device in chunks of ``chunk`` rows, so full-size outputs (10^8
    rows) are checked without copying them to the host.  Same tolerance:
    |D - D_ref| <= rtol * (|D_ref| + cutoff) componentwise, and the same for
    d, with rtol 1e-5 (float32) or 1e-12 (float64).
    """
    import torch

    dev = pairs.device
    pos = torch.as_tensor(cfg["positions"]).to(dev, torch.float64)
    cell = torch.as_tensor(cfg["cell"]).to(dev, torch.float64)
    bounds = torch.as_tensor(cfg["batch_ptr"][1:]).to(dev)
    rtol = geometry_tolerance(cfg["positions"].dtype)
    rc = cfg["cutoff"]
    for lo in range(0, pairs.shape[0], chunk):
        hi = min(lo + chunk, pairs.shape[0])
        p = pairs[lo:hi]
        b = torch.bucketize(p[:, 0].contiguous(), bounds, right=True)
        ref = pos[p[:, 1]] - pos[p[:, 0]]
        ref += torch.bmm(shifts[lo:hi].to(torch.float64).unsqueeze(1),
                         cell[b].contiguous()).squeeze(1)
        if D is not None:
            err = (D[lo:hi].to(torch.float64) - ref).abs()
            bad = err > rtol * (ref.abs() + rc)
            assert not bool(bad.any()), (
                f"D differs at rows {(torch.nonzero(bad.any(1))[:5, 0] + lo).tolist()}")
        if d is not None:
            dref = torch.linalg.vector_norm(ref, dim=1)
            bad = (d[lo:hi].to(torch.float64) - dref).abs() > rtol * (dref + rc)
            assert not bool(bad.any()), (
                f"d differs at rows {(torch.nonzero(bad)[:5, 0] + lo).tolist()}")
        del p, b, ref


def shifts_from_vectors(pairs, D, cfg):
    """Integer shifts S recovered from D = x[j] - x[i] + S @ cell[b] (rounded).

    For outputs that carry D but not S (C4's 'PD'): S = round((D - (x[j] -
    x[i])) @ inv(cell[b])), exact whenever D is within far less than half a
    cell vector of the formula, which the d/D tolerance check then confirms
    row by row.
    """
    import torch

    dev = pairs.device
    pos = torch.as_tensor(cfg["positions"]).to(dev, torch.float64)
    cell = torch.as_tensor(cfg["cell"]).to(dev, torch.float64)
    inv = torch.linalg.inv(cell.cpu()).to(dev)
    bounds = torch.as_tensor(cfg["batch_ptr"][1:]).to(dev)
    b = torch.bucketize(pairs[:, 0].contiguous(), bounds, right=True)
    frac = D.to(torch.float64) - (pos[pairs[:, 1]] - pos[pairs[:, 0]])
    S = torch.bmm(frac.unsqueeze(1), inv[b].contiguous()).squeeze(1)
    return torch.round(S).to(torch.int32)


def lattice_point_case(seed: int, dtype, pbc, heights: int = 0) -> dict:
    """Atoms on the lattice of a skewed cell, where wraps are decided at the ulp.

    The 125 points i a1 + j a2 + k a3 (i, j, k in -2..2) and 20 points on cell
    faces and half-lattice sites, each rounded in `dtype`: their fractional
    coordinates p . dual lie within rounding of an integer or half-integer,
    so the floor that gives each wrap, and through it the image box a pair
    is taken from, depends on the last bits of the pseudo-inverse.  Cutoff
    0.9 of the largest cell entry; with `heights`, that many heights
    1 / |dual_a| of one periodic axis a instead (computed in double), so that
    the repeat count ceil(rc |dual_a|) is decided at the ulp too.
    """
    import itertools

    rng = np.random.Generator(np.random.PCG64(seed))
    cell = (np.diag(2.0 + 2.0 * rng.random(3)) + 0.6 * (rng.random((3, 3)) - 0.5)).astype(dtype)
    pts = [np.array(ijk, dtype) @ cell for ijk in itertools.product(range(-2, 3), repeat=3)]
    for _ in range(20):
        f = rng.integers(-3, 4, 3).astype(dtype) + rng.choice([0.0, 0.5, 0.25], 3).astype(dtype)
        pts.append(f @ cell)
    pos = np.array(pts, dtype)
    cutoff = float(cell.max()) * 0.9
    if heights:
        act = [a for a in range(3) if pbc[a]]
        dual = np.linalg.pinv(cell.astype(np.float64)[act])  # columns: the active rows' duals
        axis = seed % len(act)
        cutoff = float(heights / np.linalg.norm(dual[:, axis]))
    return {
        "positions": pos,
        "cell": cell[None],
        "pbc": np.array([pbc], dtype=bool),
        "batch_ptr": np.array([0, len(pos)], dtype=np.int64),
        "cutoff": cutoff,
    }
