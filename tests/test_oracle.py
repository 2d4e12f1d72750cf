"""Pins the CPU oracle (no GPU): golden vectors, known answers, closed forms.

The oracle (``oracle/nl_oracle.cpp``) is the checker of every GPU parity test,
so it is pinned here before it is trusted:

* against ``tests/golden/golden.json``: pair counts, canonical SHA-256 and
  multiset checksums written by the reference's own compiled CPU core
  (``neighbor_list_cpu`` of csrc/core/neighbors_cpu.cpp:976-1030) on the
  BASELINE configurations and on the seeded inputs of the reference suite;
* against the literal known answers asserted by the reference's tests;
* against an independent numpy enumeration written from the definitions
  (image box, S = k - wrap_t + wrap_s, public predicate evaluated in the input
  type, identity policy), on small seeded inputs for every pbc pattern, pair
  mode and dtype;
* against invariants of the pair policy (half/self algebra, cell list equals
  brute force);
* against the compiled reference core directly, where it is built.
"""

from __future__ import annotations

import itertools
import json
import os

import numpy as np
import pytest

import oracle
from tests._util import key_set, keys_of, oracle_call
from tests.golden.cases import CASES

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "golden.json")))

# Cases whose oracle run and hashing finish in seconds on 8 host threads.
_SMALL = [name for name, entry in GOLDEN.items() if entry["pairs"] <= 2_000_000]


def _run(name: str, kind: str = "port"):
    make, options = CASES[name]
    cfg = make()
    return oracle.neighbor_pairs(
        cfg["positions"], cfg["cell"], cfg["pbc"], cfg["cutoff"], cfg["batch_ptr"],
        half_list=options.get("half_list", False),
        include_self=options.get("include_self", False),
        algorithm=options.get("algorithm", "auto"), threads=8, kind=kind,
    )


# ------------------------------------------------------------- golden vectors


@pytest.mark.parametrize("name", sorted(_SMALL))
def test_port_matches_golden(name):
    pairs, shifts = _run(name)
    entry = GOLDEN[name]
    assert len(pairs) == entry["pairs"]
    assert f"{oracle.multiset_hash(pairs, shifts):016x}" == entry["multiset"]
    assert oracle.key_hash(pairs, shifts) == entry["sha256"]
    if "keys" in entry:
        assert oracle.canonical_keys(pairs, shifts).tolist() == entry["keys"]


def test_port_matches_golden_c4():
    # 9.05 M pairs: the order-independent checksum (sorting would take ~15 s)
    pairs, shifts = _run("C4")
    assert len(pairs) == GOLDEN["C4"]["pairs"]
    assert f"{oracle.multiset_hash(pairs, shifts):016x}" == GOLDEN["C4"]["multiset"]


def test_golden_hashes_are_sensitive():
    # A plausible slip (one shift component negated, one target swapped)
    # changes both checksums, so the checks above can fail.
    pairs, shifts = _run("ref_forced_cell_1842_f64")
    bad = shifts.copy()
    bad[7, 1] = -bad[7, 1] if bad[7, 1] != 0 else 1
    assert oracle.multiset_hash(pairs, bad) != oracle.multiset_hash(pairs, shifts)
    assert oracle.key_hash(pairs, bad) != oracle.key_hash(pairs, shifts)
    swapped = pairs.copy()
    swapped[3, 1] = (swapped[3, 1] + 1) % 288
    assert oracle.multiset_hash(swapped, shifts) != oracle.multiset_hash(pairs, shifts)


# ------------------------------------------------------ reference known answers


def _single(positions, cell, pbc, cutoff, dtype=np.float64, **options):
    positions = np.asarray(positions, dtype=dtype).reshape(-1, 3)
    cfg = {
        "positions": positions,
        "cell": np.asarray(cell, dtype=dtype).reshape(1, 3, 3),
        "pbc": np.asarray(pbc, dtype=bool).reshape(1, 3),
        "batch_ptr": np.array([0, len(positions)], dtype=np.int64),
        "cutoff": float(cutoff),
    }
    cfg.update(options)
    return cfg


def _keys(cfg, algorithm="auto", kind="port", **options):
    cfg = dict(cfg, **options)
    return key_set(*oracle_call(cfg, algorithm=algorithm, kind=kind))


ALGOS = ("brute_force", "cell_list", "auto")


def test_kat_strict_boundary():
    # tests/backends/test_pair_identity.py:83-104, tests/test_reference.py:10-19
    cfg = _single([[0, 0, 0], [1, 0, 0]], np.zeros((3, 3)), [0, 0, 0], 1.0, np.float32)
    inside = np.nextafter(np.float32(1.0), np.float32(0.0))
    near = _single([[0, 0, 0], [inside, 0, 0]], np.zeros((3, 3)), [0, 0, 0], 1.0, np.float32)
    for algorithm in ALGOS:
        assert _keys(cfg, algorithm) == set()
        assert _keys(near, algorithm) == {(0, 1, 0, 0, 0), (1, 0, 0, 0, 0)}


def test_kat_small_cell_images():
    # tests/backends/test_pair_identity.py:105-117, tests/test_pair_options.py:187-203
    cfg = _single([[0, 0, 0]], np.diag([0.4, 8.0, 8.0]), [1, 0, 0], 1.0, np.float32)
    full = {(0, 0, -2, 0, 0), (0, 0, -1, 0, 0), (0, 0, 1, 0, 0), (0, 0, 2, 0, 0)}
    for algorithm in ALGOS:
        assert _keys(cfg, algorithm) == full
        assert _keys(cfg, algorithm, half_list=True) == {(0, 0, -2, 0, 0), (0, 0, -1, 0, 0)}
        assert _keys(cfg, algorithm, include_self=True) == full | {(0, 0, 0, 0, 0)}


def test_kat_wire():
    # tests/test_reference.py:22-35
    cfg = _single([[0, 0, 0]], np.diag([1.0, 9.0, 9.0]), [1, 0, 0], 2.1)
    for algorithm in ALGOS:
        assert _keys(cfg, algorithm) == {
            (0, 0, -2, 0, 0), (0, 0, -1, 0, 0), (0, 0, 1, 0, 0), (0, 0, 2, 0, 0)}


def test_kat_shift_translates_target():
    # tests/test_api.py:110-120
    cfg = _single([[0.9, 0, 0], [0.1, 0, 0]], np.diag([1.0, 4.0, 4.0]), [1, 0, 0], 0.3,
                  np.float32)
    assert _keys(cfg) == {(0, 1, 1, 0, 0), (1, 0, -1, 0, 0)}


def test_kat_float32_cutoff_rounding():
    # tests/backends/test_cuda_runtime.py:33-53: x = 353.2019f is inside
    # rc = 353.2019167901003 because rc * rc is rounded to float32 first.
    for n in (255, 256):
        pos = np.zeros((n, 3), np.float32)
        pos[1, 0] = np.float32(353.2019)
        pos[2:, 1] = 1000 * np.arange(2, n, dtype=np.float32)
        cfg = _single(pos, np.zeros((3, 3)), [0, 0, 0], 353.2019167901003, np.float32)
        for algorithm in ALGOS:
            assert _keys(cfg, algorithm) == {(0, 1, 0, 0, 0), (1, 0, 0, 0, 0)}


def test_kat_large_common_translation():
    # tests/backends/test_cuda_runtime.py:132-157
    cell = np.array([
        [-0.9499396681785583, 2.3687520027160645, 1.7597240209579468],
        [-3.4348089694976807, -1.8801195621490479, 1.9097744226455688],
        [2.5219004154205322, -1.9322474002838135, 4.843184471130371]], np.float32)
    pos = np.tile(np.array([-2138.380859375, -11887.5810546875, 10318.5625], np.float32), (256, 1))
    pos[52] = [-2135.800048828125, -11886.6826171875, 10317.2880859375]
    pos[40] = [-2141.306396484375, -11885.267578125, 10315.8291015625]
    pos[61] = [-2135.84033203125, -11887.59375, 10317.1181640625]
    cfg = _single(pos, cell, [1, 1, 1], 1.4481067657470703, np.float32)
    for algorithm in ALGOS:
        keys = _keys(cfg, algorithm)
        assert (52, 23, 0, -1, 0) in keys and (23, 52, 0, 1, 0) in keys
        assert (61, 40, -1, -1, 1) not in keys and (40, 61, 1, 1, -1) not in keys


def test_kat_unwrapped_representatives():
    # tests/backends/test_pair_identity.py:312-337
    cell = np.array([
        [-0.7647425305009836, -2.672179555955561, 2.8765648407042885],
        [-1.0423290504477831, -3.665756214439444, -3.2514359787147056],
        [5.609321251949969, -2.2087783511424566, -0.0013679155882546645]])
    pos = np.array([[598110346.0828383, -8096602.288435191, 242913231.3592053],
                    [598110345.1706604, -8096602.339372153, 242913230.9525894]])
    cfg = _single(pos, cell, [1, 1, 1], 1.0)
    for algorithm in ALGOS:
        assert _keys(cfg, algorithm) == {(0, 1, 0, 0, 0), (1, 0, 0, 0, 0)}


def test_kat_zero_shift_self_underflow():
    # tests/test_pair_options.py:229-261
    for dtype, cutoff in ((np.float32, 1e-30), (np.float64, 1e-200)):
        for half in (False, True):
            cfg = _single([[0, 0, 0]], np.zeros((3, 3)), [0, 0, 0], cutoff, dtype)
            assert _keys(cfg, half_list=half, include_self=True) == {(0, 0, 0, 0, 0)}


def test_kat_coincident_atoms_are_not_self():
    # tests/test_pair_options.py:206-226
    for half in (False, True):
        cfg = _single([[0, 0, 0], [0, 0, 0], [1, 0, 0]], np.zeros((3, 3)), [0, 0, 0], 1.0,
                      np.float32)
        expected = {(a, a, 0, 0, 0) for a in range(3)} | {(0, 1, 0, 0, 0)}
        if not half:
            expected.add((1, 0, 0, 0, 0))
        assert _keys(cfg, half_list=half, include_self=True) == expected


def test_kat_mixed_batch_never_crosses():
    # tests/test_reference.py:38-56
    cfg = {
        "positions": np.array([[0, 0, 0], [0.4, 0, 0], [0, 0, 0]], np.float32),
        "cell": np.stack([np.zeros((3, 3)), np.diag([0.5, 8.0, 8.0])]).astype(np.float32),
        "pbc": np.array([[0, 0, 0], [1, 0, 0]], bool),
        "batch_ptr": np.array([0, 2, 3], np.int64),
        "cutoff": 0.6,
    }
    keys = _keys(cfg)
    assert {(0, 1, 0, 0, 0), (1, 0, 0, 0, 0)} <= keys
    assert {(2, 2, -1, 0, 0), (2, 2, 1, 0, 0)} <= keys
    assert all((s < 2 and t < 2) or s == t == 2 for s, t, *_ in keys)


def test_kat_representative_translation_relabels_shift():
    # tests/test_reference.py:59-88: translating one atom by a lattice vector
    # relabels S by that vector and leaves every displacement unchanged.
    rng = np.random.Generator(np.random.PCG64(59))
    cell = np.array([[3.1, 0.2, 0.1], [0.3, 3.4, 0.2], [0.1, 0.4, 3.6]])
    pos = rng.random((12, 3)) @ cell
    moved = pos.copy()
    moved[4] += 2 * cell[0] - cell[2]
    a = _keys(_single(pos, cell, [1, 1, 1], 2.0))
    b = _keys(_single(moved, cell, [1, 1, 1], 2.0))
    relabel = set()
    for s, t, *S in a:
        S = np.array(S)
        if t == 4:
            S = S - np.array([2, 0, -1])
        if s == 4:
            S = S + np.array([2, 0, -1])
        relabel.add((s, t, *S.tolist()))
    assert relabel == b


def test_kat_image_cap_and_empty_structure():
    # tests/test_reference.py:91-111: an empty structure enumerates no
    # images; a 0.001 box with rc 1 needs more than 2^24 images.
    empty = {
        "positions": np.zeros((0, 3)),
        "cell": 0.001 * np.eye(3)[None],
        "pbc": np.ones((1, 3), bool),
        "batch_ptr": np.array([0, 0], np.int64),
        "cutoff": 1.0,
    }
    assert _keys(empty) == set()
    with pytest.raises(oracle.OracleInputError, match="image count.*resource limit"):
        _keys(_single([[0, 0, 0]], 0.001 * np.eye(3), [1, 1, 1], 1.0))


# ---------------------------------------------------------------- error contract


def test_error_contract():
    # tests/backends/test_native_errors.py:11-125, test_algorithms.py:79-107
    def err(exc, match, cfg, **kw):
        with pytest.raises(exc, match=match):
            oracle_call(dict(cfg, **kw))

    z = np.zeros((2, 3))
    batch = lambda bp, nb: {"positions": z, "cell": np.zeros((nb, 3, 3)),  # noqa: E731
                            "pbc": np.zeros((nb, 3), bool), "batch_ptr": np.array(bp),
                            "cutoff": 1.0}
    err(oracle.OracleInputError, "start at zero", batch([1, 1, 2], 2))
    err(oracle.OracleInputError, "end at N_total", batch([0, 1, 1], 2))
    err(oracle.OracleInputError, "nondecreasing", batch([0, 2, 1, 2], 3))
    for value in (np.nan, np.inf):
        pos = np.zeros((2, 3))
        pos[0, 0] = value
        err(oracle.OracleSearchError, "positions must", _single(pos, np.zeros((3, 3)),
                                                                [0, 0, 0], 0.5))
    err(oracle.OracleSearchError, "wraps.*int32",
        _single([[0.1, 0, 0], [2**31 + 0.2, 0, 0]], np.eye(3), [1, 0, 0], 0.5))
    err(oracle.OracleSearchError, "cell shift.*int32",
        _single([[-(2**31) + 0.1, 0, 0], [2**31 - 0.8, 0, 0]], np.eye(3), [1, 0, 0], 0.5))
    err(oracle.OracleInputError, "linearly independent",
        _single([[0, 0, 0]], [[1.0, 0, 0], [2.0, 0, 0], [0, 0, 4.0]], [1, 1, 0], 0.5))
    cell = np.eye(3)
    cell[2, 0] = np.nan
    err(oracle.OracleInputError, "cell must contain only finite values",
        _single([[0, 0, 0]], cell, [1, 1, 0], 0.5))
    pos = np.zeros((256, 3), np.float32)
    pos[:, 0] = np.arange(256) * 10000.0
    sparse = _single(pos, np.zeros((3, 3)), [0, 0, 0], 1.0, np.float32)
    with pytest.raises(oracle.OracleSearchError, match="cell_list cannot safely"):
        oracle_call(sparse, algorithm="cell_list")
    assert key_set(*oracle_call(sparse)) == set()


# ------------------------------------------- independent numpy enumeration


def _active_dual(cell_rows: np.ndarray, active: np.ndarray) -> np.ndarray:
    """(3, 3) matrix whose column a is the dual of active row a, 0 for inactive axes."""
    dual = np.zeros((3, 3))
    idx = np.flatnonzero(active)
    if len(idx):
        dual[:, idx] = np.linalg.pinv(cell_rows[idx].astype(np.float64))
    return dual


def numpy_keys(cfg, half_list=False, include_self=False) -> set[tuple[int, ...]]:
    """Every (s, t, S) with |D(S)|^2 < cutoff^2, written from the definitions.

    For each structure: wraps w = floor(p . dual) of the original positions,
    image repeats R_a = ceil(cutoff * |dual column a|) on periodic axes, and
    for every source s, target t and image k in the box the output shift
    S = k - w_t + w_s.  D = (((p_t - p_s) + S0 c0) + S1 c1) + S2 c2 and
    d2 = (D0^2 + D1^2) + D2^2 are rounded in the input type after every
    operation; the pair is kept when d2 < (T)(cutoff^2).  A zero-shift self
    pair needs include_self; a half list keeps (s, t, S) when it is
    lexicographically below (t, s, -S).
    """
    pos, cells, pbc, bp = cfg["positions"], cfg["cell"], cfg["pbc"], cfg["batch_ptr"]
    T = pos.dtype.type
    cut2 = T(cfg["cutoff"] * cfg["cutoff"])
    out = set()
    for b in range(len(bp) - 1):
        a0, a1 = int(bp[b]), int(bp[b + 1])
        if a1 == a0:
            continue
        p = pos[a0:a1]
        c = cells[b].astype(pos.dtype)
        active = np.asarray(pbc[b], bool)
        dual = _active_dual(c.astype(np.float64), active)
        reps = [int(np.ceil(cfg["cutoff"] * np.linalg.norm(dual[:, a]))) if active[a] else 0
                for a in range(3)]
        w = np.floor(p.astype(np.longdouble) @ dual.astype(pos.dtype).astype(np.longdouble))
        w = w.astype(np.int64)
        n = a1 - a0
        s_idx, t_idx = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
        s_idx, t_idx = s_idx.ravel(), t_idx.ravel()
        base = (p[t_idx] - p[s_idx]).astype(pos.dtype)
        for k in itertools.product(*(range(-r, r + 1) for r in reps)):
            S = np.asarray(k)[None, :] - w[t_idx] + w[s_idx]
            D = base.copy()
            for ax in range(3):
                D = D + S[:, ax : ax + 1].astype(pos.dtype) * c[ax][None, :]
            d2 = D[:, 0] * D[:, 0]
            d2 = d2 + D[:, 1] * D[:, 1]
            d2 = d2 + D[:, 2] * D[:, 2]
            for e in np.flatnonzero(d2 < cut2):
                s, t, sh = int(s_idx[e]), int(t_idx[e]), tuple(int(x) for x in S[e])
                if s == t and sh == (0, 0, 0):
                    if not include_self:
                        continue
                elif half_list and not ((s, t, *sh) < (t, s, *(-x for x in sh))):
                    continue
                out.add((s + a0, t + a0, *sh))
    return out


def _random_cfg(seed, n, pbc, dtype, unwrapped=True):
    rng = np.random.Generator(np.random.PCG64(seed))
    cell = np.diag(1.6 + 2.0 * rng.random(3)) + 0.4 * (rng.random((3, 3)) - 0.5)
    pos = rng.random((n, 3)) @ (cell * 2.5)
    if unwrapped:
        pos[0] += 3 * cell[0] - 2 * cell[2]
        pos[1] -= 4 * cell[1]
    return _single(pos, cell, pbc, 1.3, dtype)


PBC_PATTERNS = [list(p) for p in itertools.product([0, 1], repeat=3)]


@pytest.mark.parametrize("pbc", PBC_PATTERNS)
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_port_matches_numpy_enumeration(pbc, dtype):
    seed = 101 + 8 * int("".join(map(str, pbc)), 2) + (dtype == np.float32)
    cfg = _random_cfg(seed, 70, pbc, dtype)
    for half, self_ in itertools.product([False, True], repeat=2):
        expected = numpy_keys(cfg, half, self_)
        for algorithm in ("brute_force", "cell_list"):
            got = _keys(cfg, algorithm, half_list=half, include_self=self_)
            assert got == expected, (algorithm, half, self_)


def test_numpy_enumeration_is_sensitive():
    # The independent enumeration distinguishes a plausible slip: with the
    # shift applied to the source instead of the target the keys change.
    cfg = _random_cfg(7, 40, [1, 1, 1], np.float64)
    good = numpy_keys(cfg)
    flipped = {(s, t, -a, -b, -c) for s, t, a, b, c in good}
    assert good != flipped
    assert _keys(cfg) == good


def test_batched_structures_match_numpy():
    parts = [_random_cfg(300 + i, 25 + 10 * i, pbc, np.float64)
             for i, pbc in enumerate([[1, 1, 1], [0, 0, 0], [1, 0, 1], [0, 1, 0]])]
    sizes = [len(p["positions"]) for p in parts]
    cfg = {
        "positions": np.concatenate([p["positions"] for p in parts]),
        "cell": np.concatenate([p["cell"] for p in parts]),
        "pbc": np.concatenate([p["pbc"] for p in parts]),
        "batch_ptr": np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64),
        "cutoff": 1.3,
    }
    assert _keys(cfg) == numpy_keys(cfg)


# ---------------------------------------------------------------- invariants


def test_half_and_self_algebra():
    # tests/test_pair_options.py:157-184
    cfg = _random_cfg(4242, 150, [1, 1, 0], np.float64)
    full = _keys(cfg)
    full_self = _keys(cfg, include_self=True)
    half = _keys(cfg, half_list=True)
    half_self = _keys(cfg, half_list=True, include_self=True)
    n = len(cfg["positions"])
    assert full_self - full == {(a, a, 0, 0, 0) for a in range(n)}
    assert half_self - half == {(a, a, 0, 0, 0) for a in range(n)}
    canon = {min((s, t, *S), (t, s, *(-x for x in S))) for s, t, *S in full}
    assert half == canon
    expand = half | {(t, s, *(-x for x in S)) for s, t, *S in half}
    assert expand == full


@pytest.mark.parametrize("seed", range(4))
def test_cell_list_equals_brute_force(seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    pbc = rng.integers(0, 2, 3).tolist()
    cfg = _random_cfg(900 + seed, 400, pbc, np.float32 if seed % 2 else np.float64)
    assert_equal = keys_of(*oracle_call(cfg, algorithm="cell_list"))
    expected = keys_of(*oracle_call(cfg, algorithm="brute_force"))
    assert np.array_equal(assert_equal, expected)


def test_thread_count_invariance():
    # tests/backends/test_cpu_threads.py:56-156
    cfg = CASES["C5_3"][0]()
    one = keys_of(*oracle_call(dict(cfg, include_self=True), threads=1))
    many = keys_of(*oracle_call(dict(cfg, include_self=True), threads=8))
    assert np.array_equal(one, many)


def _quantities(cfg, which="dD"):
    pairs, shifts = oracle_call(cfg)
    return (pairs, shifts) + oracle.quantities(which, cfg["positions"], cfg["cell"],
                                               cfg["batch_ptr"], pairs, shifts)


def test_quantities_known_answer_of_the_reference():
    # tests/test_quantities.py:10-33: two atoms 0.8 apart on a periodic x
    # axis of length 1 and cutoff 0.3; the pairs go through the periodic
    # image, D = -0.2 x (0 -> 1, S = -x) and +0.2 x (1 -> 0, S = +x)
    cfg = _single([[0.1, 0.0, 0.0], [0.9, 0.0, 0.0]], np.diag([1.0, 4.0, 4.0]), [1, 0, 0], 0.3)
    pairs, shifts, d, D = _quantities(cfg)
    got = {(int(i), int(j), tuple(int(x) for x in s_)): (v, dd)
           for (i, j), s_, v, dd in zip(pairs, shifts, D, d)}
    assert set(got) == {(0, 1, (-1, 0, 0)), (1, 0, (1, 0, 0))}
    np.testing.assert_allclose(got[(0, 1, (-1, 0, 0))][0], [-0.2, 0.0, 0.0], atol=1e-15)
    np.testing.assert_allclose(got[(1, 0, (1, 0, 0))][0], [0.2, 0.0, 0.0], atol=1e-15)
    np.testing.assert_allclose(d, [0.2, 0.2], atol=1e-15)


def _half_lattice(rows, shift):
    # the 8 points (i a1 + j a2 + k a3) / 2, i, j, k in {0, 1}, of a periodic
    # cell with rows a1, a2, a3, moved by `shift` (all values binary-exact)
    rows = np.asarray(rows, dtype=np.float64)
    pts = [(i * rows[0] + j * rows[1] + k * rows[2]) / 2 + shift
           for i in (0, 1) for j in (0, 1) for k in (0, 1)]
    return np.array(pts), rows


def test_quantities_of_exact_lattices_in_a_batch():
    # Two periodic cells in one batch: a skewed one whose half-lattice
    # vectors a_c / 2 (lengths 2, 2.06, 2.08) are the only ones within the
    # cutoff 2.2 (the next, (a2 - a1) / 2, is 2.5 long), and a cube of edge
    # 4 (neighbours at +-2 along each axis).  Every atom has exactly six
    # pairs, with D = +-a_c / 2 of its own structure's cell, bit for bit:
    # a transposed cell, a sign slip or another structure's cell changes
    # these vectors.
    skew, rows0 = _half_lattice([[4.0, 0.0, 0.0], [1.0, 4.0, 0.0], [0.5, 1.0, 4.0]], 0.25)
    cube, rows1 = _half_lattice(np.diag([4.0, 4.0, 4.0]), -0.5)
    cfg = {
        "positions": np.concatenate([skew, cube]),
        "cell": np.stack([rows0, rows1]),
        "pbc": np.ones((2, 3), bool),
        "batch_ptr": np.array([0, 8, 16], dtype=np.int64),
        "cutoff": 2.2,
    }
    pairs, shifts, d, D = _quantities(cfg)
    assert len(pairs) == 16 * 6
    for s in range(16):
        rows = rows0 if s < 8 else rows1
        want = sorted(map(tuple, np.concatenate([rows / 2, -rows / 2])))
        mine = pairs[:, 0] == s
        assert sorted(map(tuple, D[mine])) == want, s
        np.testing.assert_allclose(d[mine], np.linalg.norm(D[mine], axis=1), rtol=1e-15)


def test_quantities_invariants():
    # a skewed cell with unwrapped atoms, float64
    cfg = _random_cfg(55, 60, [1, 0, 1], np.float64)
    pairs, shifts, d, D = _quantities(cfg)
    by_key = {(int(i), int(j), tuple(int(x) for x in s_)): v
              for (i, j), s_, v in zip(pairs, shifts, D)}
    np.testing.assert_allclose(d, np.sqrt((D * D).sum(axis=1)), rtol=1e-15)
    assert np.all(d < cfg["cutoff"])
    # the reverse pair (j, i, -S) carries -D, bit for bit
    for (i, j, s_), v in by_key.items():
        assert np.array_equal(by_key[(j, i, tuple(-x for x in s_))], -v)
    # a common translation of every atom leaves every (i, j, S) and D
    moved = dict(cfg, positions=cfg["positions"] + np.array([3.75, -12.125, 0.5]))
    p2, s2, d2, D2 = _quantities(moved)
    moved_key = {(int(i), int(j), tuple(int(x) for x in s_)): v
                 for (i, j), s_, v in zip(p2, s2, D2)}
    assert set(moved_key) == set(by_key)
    for k, v in by_key.items():
        np.testing.assert_allclose(moved_key[k], v, rtol=0, atol=1e-12)
    # atom 7 moved by the first cell vector a0: its pairs keep their D, with
    # S one cell more along a0 as a source and one cell less as a target
    pos = cfg["positions"].copy()
    pos[7] += cfg["cell"][0][0]
    p3, s3, d3, D3 = _quantities(dict(cfg, positions=pos))
    e0 = np.array([1, 0, 0])
    for (i, j), s_, v in zip(p3, s3, D3):
        s_ = np.array(s_)
        old = s_ - (e0 if i == 7 else 0) + (e0 if j == 7 else 0)
        np.testing.assert_allclose(by_key[(int(i), int(j), tuple(int(x) for x in old))], v,
                                   rtol=0, atol=1e-12)
    assert len(p3) == len(pairs)


# ------------------------------------------------ compiled reference core


@pytest.mark.skipif(not oracle.available("reference"),
                    reason="reference core not built (no reference checkout here)")
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("pbc", [[1, 1, 1], [1, 0, 1], [1, 1, 0]])
def test_lattice_point_atoms_match_the_reference_core(dtype, pbc):
    # atoms whose wraps, and cutoffs whose repeat counts, are decided at the
    # ulp (tests/_util.py, lattice_point_case): the long double
    # pseudo-inverse, floor and ceil of the port give the reference core's
    # pairs and shifts
    from tests._util import lattice_point_case

    for seed, heights in [(s_, 0) for s_ in range(12)] + [(s_, 1 + s_ % 2) for s_ in range(8)]:
        cfg = lattice_point_case(seed, dtype, pbc, heights)
        for algorithm in ("brute_force", "cell_list"):
            args = (cfg["positions"], cfg["cell"], cfg["pbc"], cfg["cutoff"], cfg["batch_ptr"])
            port = keys_of(*oracle.neighbor_pairs(*args, algorithm=algorithm, threads=1,
                                                  kind="port"))
            ref = keys_of(*oracle.neighbor_pairs(*args, algorithm=algorithm, threads=1,
                                                 kind="reference"))
            assert np.array_equal(port, ref), (seed, algorithm)


@pytest.mark.skipif(not oracle.available("reference"),
                    reason="reference core not built (no reference checkout here)")
@pytest.mark.parametrize("name", ["C1_brute", "C1_cell", "C3_128", "C5_3",
                                  "ref_unwrapped_1842_f32", "ref_mixed_5801",
                                  "ref_fallback_9041_half_self"])
def test_port_matches_reference_core(name):
    a = keys_of(*_run(name, "port"))
    b = keys_of(*_run(name, "reference"))
    assert np.array_equal(a, b)
