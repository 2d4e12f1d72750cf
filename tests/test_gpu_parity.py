"""GPU parity: the HIP path against the CPU oracle and the reference's known answers.

Every test runs ``tonari_amd.neighbor_list`` on ``cuda:0`` through the C ABI
and compares the (i, j, S) multiset bit-exactly with the oracle on the same
seeded inputs; d and D within 1e-5 relative (float32) / 1e-12 (float64).
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
    key_set,
    keys_of,
    oracle_call,
)
from tonari_amd import neighbor_list
from tonari_amd import workloads as W

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def gpu(quantities, cfg, **options):
    t = lambda x: torch.as_tensor(x).to(DEV)  # noqa: E731
    kw = dict(
        algorithm=cfg.get("algorithm", "auto"),
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


def single(positions, cell, pbc, cutoff, dtype=np.float64, **options):
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


# ------------------------------------------------------------------ KATs
# Expected key sets are the literal answers asserted by the reference suite.


def test_strict_boundary_kat():
    # tests/backends/test_pair_identity.py:83-104
    cfg = single([[0, 0, 0], [1, 0, 0]], np.zeros((3, 3)), [0, 0, 0], 1.0, np.float32)
    assert key_set(*gpu("PS", cfg)) == set()
    inside = np.nextafter(np.float32(1.0), np.float32(0.0))
    cfg = single([[0, 0, 0], [inside, 0, 0]], np.zeros((3, 3)), [0, 0, 0], 1.0, np.float32)
    assert key_set(*gpu("PS", cfg)) == {(0, 1, 0, 0, 0), (1, 0, 0, 0, 0)}


def test_small_cell_images_kat():
    # tests/backends/test_pair_identity.py:105-117, tests/test_pair_options.py:187-203
    cfg = single([[0, 0, 0]], np.diag([0.4, 8.0, 8.0]), [1, 0, 0], 1.0, np.float32)
    full = {(0, 0, -2, 0, 0), (0, 0, -1, 0, 0), (0, 0, 1, 0, 0), (0, 0, 2, 0, 0)}
    for algorithm in ("brute_force", "cell_list", "auto"):
        assert key_set(*gpu("PS", cfg, algorithm=algorithm)) == full
        assert key_set(*gpu("PS", cfg, algorithm=algorithm, half_list=True)) == {
            (0, 0, -2, 0, 0), (0, 0, -1, 0, 0)}
        assert key_set(*gpu("PS", cfg, algorithm=algorithm, include_self=True)) == full | {
            (0, 0, 0, 0, 0)}


def test_wire_kat():
    # tests/test_reference.py:22-35
    cfg = single([[0, 0, 0]], np.diag([1.0, 9.0, 9.0]), [1, 0, 0], 2.1)
    assert key_set(*gpu("PS", cfg)) == {
        (0, 0, -2, 0, 0), (0, 0, -1, 0, 0), (0, 0, 1, 0, 0), (0, 0, 2, 0, 0)}


def test_shift_translates_target_kat():
    # tests/test_api.py:261-271
    cfg = single([[0.9, 0, 0], [0.1, 0, 0]], np.diag([1.0, 4.0, 4.0]), [1, 0, 0], 0.3,
                 np.float32)
    assert key_set(*gpu("PS", cfg)) == {(0, 1, 1, 0, 0), (1, 0, -1, 0, 0)}


def test_float32_cutoff_rounding_kat():
    # tests/backends/test_cuda_runtime.py:33-53
    for n in (255, 256):
        pos = np.zeros((n, 3), np.float32)
        pos[1, 0] = np.float32(353.2019)
        pos[2:, 1] = 1000 * np.arange(2, n, dtype=np.float32)
        cfg = single(pos, np.zeros((3, 3)), [0, 0, 0], 353.2019167901003, np.float32)
        for algorithm in ("brute_force", "cell_list", "auto"):
            assert key_set(*gpu("PS", cfg, algorithm=algorithm)) == {
                (0, 1, 0, 0, 0), (1, 0, 0, 0, 0)}


def test_large_common_translation_kat():
    # tests/backends/test_cuda_runtime.py:306-331
    cell = np.array([
        [-0.9499396681785583, 2.3687520027160645, 1.7597240209579468],
        [-3.4348089694976807, -1.8801195621490479, 1.9097744226455688],
        [2.5219004154205322, -1.9322474002838135, 4.843184471130371]], np.float32)
    pos = np.tile(np.array([-2138.380859375, -11887.5810546875, 10318.5625], np.float32), (256, 1))
    pos[52] = [-2135.800048828125, -11886.6826171875, 10317.2880859375]
    pos[40] = [-2141.306396484375, -11885.267578125, 10315.8291015625]
    pos[61] = [-2135.84033203125, -11887.59375, 10317.1181640625]
    cfg = single(pos, cell, [1, 1, 1], 1.4481067657470703, np.float32)
    expected = keys_of(*oracle_call(cfg))
    for algorithm in ("auto", "brute_force", "cell_list"):
        got = keys_of(*gpu("PS", cfg, algorithm=algorithm))
        keys = {tuple(r) for r in got.tolist()}
        assert (52, 23, 0, -1, 0) in keys and (23, 52, 0, 1, 0) in keys
        assert (61, 40, -1, -1, 1) not in keys and (40, 61, 1, 1, -1) not in keys
        assert_same_keys(got, expected)


def test_unwrapped_representatives_kat():
    # tests/backends/test_pair_identity.py:312-337
    cell = np.array([
        [-0.7647425305009836, -2.672179555955561, 2.8765648407042885],
        [-1.0423290504477831, -3.665756214439444, -3.2514359787147056],
        [5.609321251949969, -2.2087783511424566, -0.0013679155882546645]])
    pos = np.array([[598110346.0828383, -8096602.288435191, 242913231.3592053],
                    [598110345.1706604, -8096602.339372153, 242913230.9525894]])
    cfg = single(pos, cell, [1, 1, 1], 1.0)
    assert key_set(*gpu("PS", cfg)) == {(0, 1, 0, 0, 0), (1, 0, 0, 0, 0)}


def test_zero_shift_self_underflow_kat():
    # tests/test_pair_options.py:229-261
    for dtype, cutoff in ((np.float32, 1e-30), (np.float64, 1e-200)):
        for half in (False, True):
            cfg = single([[0, 0, 0]], np.zeros((3, 3)), [0, 0, 0], cutoff, dtype)
            assert key_set(*gpu("PS", cfg, half_list=half, include_self=True)) == {(0, 0, 0, 0, 0)}


def test_coincident_atoms_are_not_self_kat():
    # tests/test_pair_options.py:206-226
    for half in (False, True):
        cfg = single([[0, 0, 0], [0, 0, 0], [1, 0, 0]], np.zeros((3, 3)), [0, 0, 0], 1.0,
                     np.float32)
        expected = {(a, a, 0, 0, 0) for a in range(3)} | {(0, 1, 0, 0, 0)}
        if not half:
            expected.add((1, 0, 0, 0, 0))
        assert key_set(*gpu("PS", cfg, half_list=half, include_self=True)) == expected


def test_mixed_batch_never_crosses_kat():
    # tests/test_reference.py:38-56, tests/test_api.py:297-304
    cfg = {
        "positions": np.array([[0, 0, 0], [0.4, 0, 0], [0, 0, 0]], np.float32),
        "cell": np.stack([np.zeros((3, 3)), np.diag([0.5, 8.0, 8.0])]).astype(np.float32),
        "pbc": np.array([[0, 0, 0], [1, 0, 0]], bool),
        "batch_ptr": np.array([0, 2, 3], np.int64),
        "cutoff": 0.6,
    }
    keys = key_set(*gpu("PS", cfg))
    assert {(0, 1, 0, 0, 0), (1, 0, 0, 0, 0)} <= keys
    assert (2, 2, -1, 0, 0) in keys and (2, 2, 1, 0, 0) in keys
    assert all((s < 2 and t < 2) or s == t == 2 for s, t, *_ in keys)


def test_empty_structures_and_nondefault_stream():
    # tests/backends/test_cuda_runtime.py:56-69
    positions = torch.tensor([[0.0, 0.0, 0.0], [0.3, 0.0, 0.0]], device=DEV)
    batch_ptr = torch.tensor([0, 0, 2], device=DEV)
    cell = torch.zeros((2, 3, 3), device=DEV)
    pbc = torch.zeros((2, 3), dtype=torch.bool, device=DEV)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        positions = positions + 0.0
        pairs, shifts = neighbor_list("PS", positions, cell, pbc, 0.5, batch_ptr, sorted=True)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    assert key_set(pairs, shifts) == {(0, 1, 0, 0, 0), (1, 0, 0, 0, 0)}
    assert_sorted_by_source(pairs)


def test_empty_inputs():
    out = neighbor_list(
        "ijPSdD", torch.empty((0, 3), dtype=torch.float64, device=DEV),
        (1e-12 * torch.eye(3, dtype=torch.float64, device=DEV))[None],
        torch.ones((1, 3), dtype=torch.bool, device=DEV), 1.0,
        torch.tensor([0, 0], device=DEV))
    assert [tuple(x.shape) for x in out] == [(0,), (0,), (0, 2), (0, 3), (0,), (0, 3)]
    assert neighbor_list("", torch.zeros((1, 3), device=DEV), torch.zeros((3, 3), device=DEV),
                         torch.zeros(3, dtype=torch.bool, device=DEV), 1.0) == ()


# ---------------------------------------------------------- error contract


def _err(exc, match, positions, cell, pbc, cutoff, batch_ptr=None, **kw):
    t = lambda x: None if x is None else torch.as_tensor(x).to(DEV)  # noqa: E731
    with pytest.raises(exc, match=match):
        neighbor_list("PS", t(positions), t(cell), t(pbc), cutoff, t(batch_ptr), **kw)
    torch.cuda.synchronize()


def test_error_contract():
    # tests/backends/test_native_errors.py and test_cuda_runtime.py:334-385
    z = np.zeros((2, 3))
    _err(ValueError, "start at zero", z, np.zeros((2, 3, 3)), np.zeros((2, 3), bool), 1.0,
         np.array([1, 1, 2]))
    _err(ValueError, "end at N_total", z, np.zeros((2, 3, 3)), np.zeros((2, 3), bool), 1.0,
         np.array([0, 1, 1]))
    _err(ValueError, "nondecreasing", z, np.zeros((3, 3, 3)), np.zeros((3, 3), bool), 1.0,
         np.array([0, 2, 1, 2]))
    for value in (np.nan, np.inf):
        pos = np.zeros((2, 3))
        pos[0, 0] = value
        _err(RuntimeError, "positions must", pos, np.zeros((3, 3)), np.zeros(3, bool), 0.5)
    _err(RuntimeError, "wraps.*int32", np.array([[0.1, 0, 0], [2**31 + 0.2, 0, 0]]), np.eye(3),
         np.array([1, 0, 0], bool), 0.5)
    _err(RuntimeError, "cell shift.*int32",
         np.array([[-(2**31) + 0.1, 0, 0], [2**31 - 0.8, 0, 0]]), np.eye(3),
         np.array([1, 0, 0], bool), 0.5)
    _err(ValueError, "linearly independent", np.zeros((1, 3)),
         np.array([[1.0, 0, 0], [2.0, 0, 0], [0, 0, 4.0]]), np.array([1, 1, 0], bool), 0.5)
    cell = np.eye(3)
    cell[2, 0] = np.nan
    _err(ValueError, "cell must contain only finite values", np.zeros((1, 3)), cell,
         np.array([1, 1, 0], bool), 0.5)
    _err(ValueError, "image count.*resource limit", np.zeros((1, 3)), 0.001 * np.eye(3),
         np.ones(3, bool), 1.0)
    pos = np.zeros((256, 3), np.float32)
    pos[:, 0] = np.arange(256) * 10000.0
    _err(RuntimeError, "cell_list cannot safely", pos, np.zeros((3, 3), np.float32),
         np.zeros(3, bool), 1.0, algorithm="cell_list")
    # The automatic path handles the same sparse layout.
    out = neighbor_list("PS", torch.tensor(pos, device=DEV), torch.zeros((3, 3), device=DEV),
                        torch.zeros(3, dtype=torch.bool, device=DEV), 1.0)
    assert key_set(*out) == set()


def test_ill_conditioned_rows_are_accepted():
    # tests/backends/test_native_errors.py:90-112
    cfg = single([[0, 0, 0], [0, 5e-10, 0]], [[1.0, 0, 0], [1.0, 1e-8, 0], [0, 0, 0]], [1, 1, 0],
                 1e-9)
    assert_same_keys(keys_of(*gpu("PS", cfg)), keys_of(*oracle_call(cfg)))


# ------------------------------------------------- seeded differential sets


def _torch_seeded(seed, n, cell, shift_atoms=None):
    g = torch.Generator().manual_seed(seed)
    cell = torch.tensor(cell, dtype=torch.float64)
    pos = torch.rand((n, 3), generator=g, dtype=torch.float64) @ cell
    return pos.numpy(), cell.numpy()


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("algorithm", ["auto", "brute_force", "cell_list"])
@pytest.mark.parametrize("half_list", [False, True])
@pytest.mark.parametrize("include_self", [False, True])
def test_triclinic_modes_match_oracle(dtype, algorithm, half_list, include_self):
    # the structure of tests/backends/test_pair_identity.py:268-289 (seed 1842)
    pos, cell = _torch_seeded(1842, 288, [[8.0, 0.4, 0.1], [0.2, 7.5, 0.5], [0.3, 0.1, 9.0]])
    pos[:5] += 3 * cell[0] - 2 * cell[1]
    cfg = single(pos, cell, [1, 1, 1], 1.2, dtype, half_list=half_list,
                 include_self=include_self)
    expected = keys_of(*oracle_call(cfg, algorithm="brute_force"))
    pairs, shifts, d, D = gpu("PSdD", cfg, algorithm=algorithm, sorted=True)
    assert_same_keys(keys_of(pairs, shifts), expected)
    assert_sorted_by_source(pairs)
    assert_geometry_close(pairs, shifts, d, D, cfg)


@pytest.mark.parametrize("pbc", [[0, 0, 0], [1, 0, 0], [1, 0, 1], [1, 1, 0], [1, 1, 1]])
@pytest.mark.parametrize("algorithm", ["brute_force", "cell_list"])
def test_pbc_patterns_match_oracle(pbc, algorithm):
    # randomized pbc patterns as in tests/backends/test_pair_identity.py:189-223
    rng = np.random.Generator(np.random.PCG64(29381 + sum(pbc)))
    cell = np.diag(1.8 + 2.5 * rng.random(3)) + 0.35 * np.tril(rng.random((3, 3)), -1)
    pos = rng.random((300, 3)) @ (cell * 3)
    pos[0] += 3 * cell[0]
    cfg = single(pos, cell, pbc, 1.1)
    expected = keys_of(*oracle_call(cfg, algorithm="brute_force"))
    assert_same_keys(keys_of(*gpu("PS", cfg, algorithm=algorithm)), expected)


# --------------------------------------------------- benchmark configurations


def test_c1_both_algorithms():
    cfg = W.c1()
    expected = keys_of(*oracle_call(cfg, algorithm="brute_force"))
    for algorithm in ("brute_force", "cell_list"):
        i, j, S, d, D = gpu("ijSdD", cfg, algorithm=algorithm)
        pairs = torch.stack([i, j], dim=1)
        assert_same_keys(keys_of(pairs, S), expected)
        assert_geometry_close(pairs, S, d, D, cfg)


def test_c2_subset():
    cfg = W.c2(n_structures=64)
    expected = keys_of(*oracle_call(cfg))
    P, S, D = gpu("PSD", cfg)
    assert_same_keys(keys_of(P, S), expected)
    assert_geometry_close(P, S, None, D, cfg)


def test_c3_subset():
    cfg = W.c3(n_structures=128)
    expected = keys_of(*oracle_call(cfg))
    i, j, d = gpu("ijd", cfg)
    assert_sorted_by_source(torch.stack([i, j], 1))
    P, S = gpu("PS", cfg)
    assert_same_keys(keys_of(P, S), expected)
    assert torch.equal(P[:, 0], i) and torch.equal(P[:, 1], j)


def test_c4_small():
    cfg = W.c4(n_atoms=20000)
    expected = keys_of(*oracle_call(cfg))
    P, S, D = gpu("PSD", cfg)
    assert_same_keys(keys_of(P, S), expected)
    assert_geometry_close(P, S, None, D, cfg)
    # 'PD' (the benchmark's quantities) returns the same pairs; without
    # `sorted` the order is unspecified, as in the reference.
    P2, D2 = gpu("PD", cfg)
    n = len(cfg["positions"])
    assert torch.equal(torch.sort(P2[:, 0] * n + P2[:, 1]).values,
                       torch.sort(P[:, 0] * n + P[:, 1]).values)
    assert_geometry_close(P2, _shifts_for(P2, P, S), None, D2, cfg)


def test_output_order_sorted_and_unsorted():
    # sorted: sources in increasing index order; unsorted: the same pairs,
    # every source's pairs contiguous (cell-list bin order for a cell-list
    # batch, index order for a batch that also holds brute-force structures)
    cfg = W.c4(n_atoms=20000)
    P1, S1 = gpu("PS", cfg, sorted=True)
    P0, S0 = gpu("PS", cfg, sorted=False)
    assert_sorted_by_source(P1)
    assert_grouped_by_source(P0)
    assert_same_keys(keys_of(P0, S0), keys_of(P1, S1))
    mixed = W.c2()
    mixed["algorithm"] = "auto"
    Pm, Sm = gpu("PS", mixed, sorted=False)
    assert_grouped_by_source(Pm)
    assert_same_keys(keys_of(Pm, Sm), keys_of(*gpu("PS", mixed, sorted=True)))


def _shifts_for(pairs_new, pairs_old, shifts_old):
    """Shifts of pairs_new looked up from a (pairs_old, shifts_old) listing of the same
    pairs, assuming no (i, j) repeats within the listing (true for C4: no small images)."""
    key_old = pairs_old[:, 0] * (1 << 32) + pairs_old[:, 1]
    key_new = pairs_new[:, 0] * (1 << 32) + pairs_new[:, 1]
    order = torch.argsort(key_old)
    pos = torch.searchsorted(key_old[order], key_new)
    assert torch.equal(key_old[order][pos], key_new)
    return shifts_old[order][pos]


def test_c5_subset():
    cfg = W.c5(n_structures=3, n_min=1000, n_max=3000)
    expected = keys_of(*oracle_call(cfg))
    i, j, S, d, D = gpu("ijSdD", cfg)
    pairs = torch.stack([i, j], dim=1)
    assert_same_keys(keys_of(pairs, S), expected)
    assert_sorted_by_source(pairs)
    assert_geometry_close(pairs, S, d, D, cfg)


# ------------------------------------------ full BASELINE sizes vs golden vectors
# The golden fixtures were written by the reference's own compiled CPU core;
# at full size the comparison goes through size-independent checksums.


def _golden():
    import json
    import os

    return json.load(open(os.path.join(os.path.dirname(__file__), "golden", "golden.json")))


@pytest.mark.parametrize("name", ["C2", "C3", "C4", "C5"])
def test_full_size_matches_golden(name):
    """The configuration's own call (its quantities, as the benchmark runs it).

    The (i, j, S) multiset goes through the golden checksum; S comes from the
    output when requested, is zero for a non-periodic batch (C3), and is
    recovered from D for C4's 'PD'.  Every row of d and D is checked against
    the float64 formula on the device.
    """
    from tests._util import (assert_geometry_close_torch, multiset_hash_torch,
                             shifts_from_vectors)
    from tests.golden.cases import CASES

    make, options = CASES[name]
    cfg = dict(make(), **options)
    entry = _golden()[name]
    quantities = cfg["quantities"]
    print(f"[golden] {name}: {len(cfg['positions'])} atoms, '{quantities}', expecting "
          f"{entry['pairs']} pairs", flush=True)
    out = dict(zip(quantities, gpu(quantities, cfg)))
    P = out["P"] if "P" in out else torch.stack([out["i"], out["j"]], 1)
    if "S" in out:
        S = out["S"]
    elif not cfg["pbc"].any():
        S = torch.zeros((P.shape[0], 3), dtype=torch.int32, device=P.device)
    else:
        S = shifts_from_vectors(P, out["D"], cfg)
    assert P.shape[0] == entry["pairs"]
    assert f"{multiset_hash_torch(P, S):016x}" == entry["multiset"]
    if cfg.get("sorted", False):
        assert_sorted_by_source(P)
    else:
        assert_grouped_by_source(P)
    if "sha256" in entry and entry["pairs"] <= 2_000_000:
        import oracle

        assert oracle.key_hash(P.cpu().numpy(), S.cpu().numpy()) == entry["sha256"]
    assert_geometry_close_torch(P, S, out.get("d"), out.get("D"), cfg)
    del P, S, out
    torch.cuda.empty_cache()


def test_float64_vectors_past_32bit_byte_offsets():
    """Float64 D rows (24 bytes) beyond 2^32 / 24 = 178,956,970 rows.

    The emitting fast path stores with 32-bit byte offsets only while every
    row of every requested output fits below 2^32 bytes; the widest row
    decides (D of float64).  A single periodic box at density 0.1 and rc
    7.1 A gives about 150 neighbours per atom (stencils the emit stages in
    LDS) and, with 1.3 M atoms, more than 190 M pairs.  Every D row is
    checked against the float64 formula, so a row written at a wrapped
    offset (or one left unwritten) fails.
    """
    n, density, rc = 1_300_000, 0.1, 7.1
    rng = np.random.Generator(np.random.PCG64(1771))
    edge = (n / density) ** (1.0 / 3.0)
    cfg = single(rng.uniform(0.0, edge, size=(n, 3)), edge * np.eye(3), [1, 1, 1], rc,
                 np.float64)
    print(f"[off32] {n} atoms, float64 'PSD', rc {rc}", flush=True)
    P, S, D = gpu("PSD", cfg, algorithm="cell_list")
    limit = 0xFFFFFFFF // 24
    print(f"[off32] {P.shape[0]} pairs (32-bit limit of D rows {limit})", flush=True)
    assert P.shape[0] > limit + 1_000_000
    from tests._util import assert_geometry_close_torch

    assert_geometry_close_torch(P, S, None, D, cfg)
    del P, S, D
    torch.cuda.empty_cache()


def test_readme_pyg_batch_example():
    """The reference README's PyTorch Geometric example (README.md:81-99), verbatim.

    A PyG batch carries pos, cell, pbc and ptr; the edge list is P.T and the
    edge vectors are D.  The same call through this package must give the
    oracle's pairs and the reference formula's vectors.
    """
    from types import SimpleNamespace

    cfg = W.c2(n_structures=16)
    t = lambda x: torch.as_tensor(x).to("cuda:0")  # noqa: E731
    batch = SimpleNamespace(pos=t(cfg["positions"]), cell=t(cfg["cell"]), pbc=t(cfg["pbc"]),
                            ptr=t(cfg["batch_ptr"]))
    cutoff = cfg["cutoff"]

    pairs, edge_vectors = neighbor_list(
        "PD",
        batch.pos,
        batch.cell,
        batch.pbc,
        cutoff=cutoff,
        batch_ptr=batch.ptr,
    )

    edge_index = pairs.T.contiguous()
    edge_lengths = torch.linalg.vector_norm(edge_vectors, dim=1)
    torch.cuda.synchronize()
    assert edge_index.shape == (2, pairs.shape[0]) and edge_index.is_contiguous()
    assert bool((edge_lengths < cutoff).all())
    P_ref = np.asarray(oracle_call(cfg, algorithm="auto")[0])
    got = pairs.cpu().numpy()
    assert np.array_equal(got[np.lexsort(got.T[::-1])], P_ref[np.lexsort(P_ref.T[::-1])])
