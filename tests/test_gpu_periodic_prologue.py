"""GPU: the periodic fast prologue (plan hint 10: one fully periodic cell-list structure).

A repeated count of one fully periodic structure chooses its bin grid from
the cell and the cutoff before any atom is reduced (``k_periodic_atoms``),
then in one more launch (``k_periodic_place``) finishes the plan in one
workgroup while the others rank the atoms in their bins, meet at a grid
barrier, scan the bin counts (whole in every workgroup up to 8,192 bins, in
slices between two more barriers beyond) and place the atoms.  Every case
here drives the hint through the C ABI and compares the emitted (i, j, S)
multiset with the CPU oracle bit for bit and D with the float64 formula; the
cases cover cubic and triclinic cells, both dtypes, all four pair modes,
wrapped atoms, more bins than one workgroup scans, atoms far enough from the
cell that the stencil reach has to grow, atoms so far that the margin
outgrows the cutoff (planned as brute force), the hint failing (slab,
cluster, small structure under auto) with TNR_RETRY, barrier waits forced
to expire (TNR_PLACE_WAIT_US=0), and repeats on one workspace, where the
set-up is taken from the memo an earlier request with the same inputs left
there and derived again when an input differs.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from tests._util import assert_geometry_close, assert_same_keys, keys_of, oracle_call
from tonari_amd import neighbor_list
from tonari_amd import workloads as W
from tonari_amd._extensions import (
    ALGORITHMS, TNR_OK, TNR_RETRY, Outputs, Request, load_torch_hip,
)
from tonari_amd._torch_frontend import _speculation

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
HINT = 10  # plan bits 1 (cell lists) and 3 (periodic grid)
MODES = [(False, False), (False, True), (True, False), (True, True)]


def search(cfg, hint, *, algorithm="cell_list", half_list=False, include_self=False,
           sorted=False, info=None, keep=None):
    """Count with `hint`, then emit P, S, D; returns (code, message, plan, P, S, D).
    `info`, when given, receives the count's bin total ("bins"); `keep`, when
    given, holds the workspace from one call to the next (filled with garbage
    only when it is first made)."""
    lib = load_torch_hip()
    t = {k: torch.as_tensor(cfg[k]).to(DEV) for k in ("positions", "cell", "pbc", "batch_ptr")}
    pos = t["positions"]
    req = Request(
        dtype=0 if pos.dtype == torch.float32 else 1, algorithm=ALGORITHMS[algorithm],
        n_atoms=pos.shape[0], n_structures=t["batch_ptr"].numel() - 1,
        positions=pos.data_ptr(), batch_ptr=t["batch_ptr"].data_ptr(),
        cell=t["cell"].data_ptr(), pbc=t["pbc"].data_ptr(), cutoff=cfg["cutoff"],
        half_list=int(half_list), include_self=int(include_self), sorted=int(sorted),
        stencil_reach=0,
    )
    ws_bytes = int(lib.tnr_workspace_size(ctypes.byref(req)))
    ws = keep.get("ws") if keep is not None else None
    if ws is None or ws.numel() != ws_bytes:
        # garbage in the workspace: the prologue must not rely on zeroed memory
        ws = torch.full((ws_bytes,), 0xA5, dtype=torch.uint8, device=DEV)
        if keep is not None:
            keep["ws"] = ws
    host = torch.zeros(8, dtype=torch.int64, pin_memory=True)
    err = ctypes.create_string_buffer(512)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.tnr_count_async_hinted(ctypes.byref(req), ws.data_ptr(), ws_bytes, host.data_ptr(),
                                    stream, hint, err, len(err))
    assert rc == TNR_OK, err.value.decode()
    torch.cuda.synchronize()
    n = ctypes.c_int64(-1)
    code = lib.tnr_count_finish(host.data_ptr(), ctypes.byref(n), err, len(err))
    plan = int(host[3])
    if info is not None:
        info["bins"] = int(host[4])
    if code != TNR_OK:
        return code, err.value.decode(), plan, None, None, None
    E = int(n.value)
    P = torch.empty((E, 2), dtype=torch.int64, device=DEV)
    S = torch.empty((E, 3), dtype=torch.int32, device=DEV)
    D = torch.empty((E, 3), dtype=pos.dtype, device=DEV)
    out = Outputs(n_pairs=E, plan=plan, n_tasks=int(host[4]), pairs=P.data_ptr(),
                  shifts=S.data_ptr(), vectors=D.data_ptr())
    if E > 0:
        rc = lib.tnr_emit(ctypes.byref(req), ws.data_ptr(), ws_bytes, ctypes.byref(out), stream,
                          err, len(err))
        assert rc == TNR_OK, err.value.decode()
    torch.cuda.synchronize()
    return code, "", plan, P, S, D


def check(cfg, algorithm="cell_list", expect_plan=HINT, **kw):
    """The hinted search equals the oracle; returns the plan word."""
    full = dict(cfg, half_list=kw.get("half_list", False),
                include_self=kw.get("include_self", False))
    code, msg, plan, P, S, D = search(full, HINT, algorithm=algorithm, **kw)
    assert code == TNR_OK, msg
    assert plan == expect_plan, plan
    assert_same_keys(keys_of(P, S), keys_of(*oracle_call(full, algorithm=algorithm)))
    assert_geometry_close(P, S, None, D, full)
    if kw.get("sorted"):
        src = P[:, 0]
        assert bool((src[1:] >= src[:-1]).all())
    return plan


def box(n, lengths, angles, dtype, cutoff, seed, shift=0):
    """n atoms uniform in a triclinic cell, optionally moved by random
    integer cell vectors in [-shift, shift] (wrapped atoms)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    cell = W.triclinic_cell(lengths, angles)
    frac = rng.uniform(0.0, 1.0, (n, 3))
    if shift:
        frac = frac + rng.integers(-shift, shift + 1, (n, 3))
    pos = frac @ cell
    return W._pack([pos], [cell], [np.ones(3, bool)], [n], dtype, cutoff)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("half_list,include_self", MODES)
def test_cubic_and_triclinic_boxes(dtype, half_list, include_self):
    print(f"[periodic] {np.dtype(dtype).name} half={half_list} self={include_self}", flush=True)
    for sorted_ in (False, True):
        check(box(6000, (40.0, 40.0, 40.0), (90, 90, 90), dtype, 6.0, 31),
              half_list=half_list, include_self=include_self, sorted=sorted_)
        check(box(3000, (30.0, 33.0, 28.0), (75, 100, 65), dtype, 6.0, 32),
              half_list=half_list, include_self=include_self, sorted=sorted_)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_wrapped_atoms(dtype):
    # atoms up to three cells away on each axis: nonzero wraps
    for seed, angles in ((33, (90, 90, 90)), (34, (70, 110, 80))):
        cfg = box(2500, (26.0, 24.0, 27.0), angles, dtype, 5.0, seed, shift=3)
        for half_list, include_self in MODES:
            check(cfg, half_list=half_list, include_self=include_self)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_many_bins_take_the_sliced_scan(dtype):
    # a sparse 90 A box at rc 3: more bins than one workgroup scans whole
    # (8,192), so the bin counts are summed and scanned in slices
    print(f"[periodic] sliced bin scan {np.dtype(dtype).name}", flush=True)
    cfg = box(10000, (90.0, 90.0, 90.0), (90, 90, 90), dtype, 3.0, 44)
    for half_list, include_self in ((False, False), (True, True)):
        info = {}
        check(cfg, half_list=half_list, include_self=include_self, info=info)
        assert info["bins"] > 8192, info
    check(box(9000, (80.0, 85.0, 90.0), (80, 100, 95), dtype, 3.0, 45, shift=1))


def test_expired_barrier_waits_count_again(monkeypatch):
    # a wait bound of zero: workgroups that have to wait at a barrier give up
    # and the count reports that the hint does not hold (the caller counts
    # again without it); a count whose workgroups never wait succeeds.  Either
    # way the frontend's result is the oracle's.
    monkeypatch.setenv("TNR_PLACE_WAIT_US", "0")
    for cfg in (box(40000, (70.0, 70.0, 70.0), (90, 90, 90), np.float32, 6.0, 46),
                box(10000, (90.0, 90.0, 90.0), (90, 90, 90), np.float32, 3.0, 47)):
        print(f"[periodic] wait bound 0, {len(cfg['positions'])} atoms", flush=True)
        full = dict(cfg, half_list=False, include_self=False)
        expected = keys_of(*oracle_call(full, algorithm="cell_list"))
        code, msg, plan, P, S, D = search(full, HINT)
        assert code in (TNR_OK, TNR_RETRY), (code, msg)
        if code == TNR_RETRY:
            assert "plan hint" in msg, msg
        else:
            assert_same_keys(keys_of(P, S), expected)
        t = {k: torch.as_tensor(cfg[k]).to(DEV) for k in ("positions", "cell", "pbc", "batch_ptr")}
        _speculation().clear()
        for call in range(3):
            P, S, D = neighbor_list("PSD", t["positions"], t["cell"], t["pbc"], cfg["cutoff"],
                                    t["batch_ptr"], algorithm="cell_list")
            torch.cuda.synchronize()
            assert_same_keys(keys_of(P, S), expected)
            assert_geometry_close(P, S, None, D, cfg)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_repeats_on_one_workspace(dtype):
    # k_periodic_atoms takes its set-up (record and grid) from the memo an
    # earlier request with the same inputs left in the workspace, and derives
    # it again when any input it depends on differs: a repeat and moved atoms
    # (same cell) take the memo; another cell, cutoff, periodicity, pair mode
    # or algorithm does not.  Every result must be the oracle's.
    print(f"[periodic] one workspace, {np.dtype(dtype).name}", flush=True)
    base = box(6000, (40.0, 40.0, 40.0), (90, 90, 90), dtype, 6.0, 48)
    rng = np.random.Generator(np.random.PCG64(50))
    moved = dict(base, positions=(base["positions"] + rng.normal(0.0, 0.3, (6000, 3))).astype(dtype))
    skewed = dict(base, cell=box(10, (41.0, 40.0, 39.0), (85, 95, 90), dtype, 6.0, 49)["cell"])
    shorter = dict(base, cutoff=5.5)
    slab = dict(base, pbc=np.array([[True, True, False]]))
    keep = {}
    for cfg, kw in ((base, {}), (base, {}), (moved, {}), (skewed, {}), (skewed, {}),
                    (shorter, {}), (slab, {}), (base, {"half_list": True}), (base, {}),
                    (base, {"algorithm": "auto"}), (base, {})):
        algorithm = kw.get("algorithm", "cell_list")
        half = kw.get("half_list", False)
        full = dict(cfg, half_list=half, include_self=False)
        code, msg, plan, P, S, D = search(full, HINT, algorithm=algorithm, half_list=half,
                                          keep=keep)
        if cfg is slab:
            # not fully periodic: the hint does not hold
            assert code == TNR_RETRY and "plan hint" in msg, (code, msg)
            continue
        assert code == TNR_OK, msg
        assert_same_keys(keys_of(P, S), keys_of(*oracle_call(full, algorithm=algorithm)))
        assert_geometry_close(P, S, None, D, full)


def test_c1_auto_and_c4_sizes():
    c1 = W.c1()
    check(c1, algorithm="auto")
    check(c1, algorithm="cell_list", sorted=True)
    check(W.c4(seed=35, n_atoms=20000), algorithm="auto")


def test_reach_grows_with_far_atoms():
    # a 20.01 A box at rc 5 has four bins per axis of 5.0025 A: with atoms
    # two cells away (max |p| 60 A, max |wrap| 2) the float32 margin is
    # 0.0017 A > 0.00125 A, so the finished plan needs a reach of two bins
    # where the grid, chosen for atoms inside the cell, had one
    cfg = box(1200, (20.01, 20.01, 20.01), (90, 90, 90), np.float32, 5.0, 36, shift=2)
    check(cfg)
    check(cfg, algorithm="auto", half_list=True)


def test_margin_beyond_cutoff_is_brute_force():
    # float32 atoms 10^6 A from the cell: the margin outgrows the cutoff, so
    # auto plans brute force (plan 1) and an explicit cell_list is refused
    # with the reference's message, as without the hint
    cfg = box(600, (20.0, 20.0, 20.0), (90, 90, 90), np.float32, 5.0, 37)
    far = dict(cfg, positions=(cfg["positions"] + np.float32(1.0e6)).astype(np.float32))
    lib_msg = "cell_list cannot safely process"
    code, msg, _, _, _, _ = search(far, -1, algorithm="cell_list")
    assert code != TNR_OK and lib_msg in msg
    code, msg, _, _, _, _ = search(far, HINT, algorithm="cell_list")
    assert code != TNR_OK and lib_msg in msg
    code, msg, plan, P, S, D = search(far, HINT, algorithm="auto")
    assert code == TNR_OK and plan == 1, (code, msg, plan)
    assert_same_keys(keys_of(P, S), keys_of(*oracle_call(far, algorithm="auto")))


def test_hint_that_does_not_hold_is_retried():
    # a slab (one open axis), an open cluster, a periodic structure too small
    # for a cell list under auto, and a batch of two boxes
    slab = box(2000, (30.0, 30.0, 30.0), (90, 90, 90), np.float32, 6.0, 38)
    slab["pbc"] = np.array([[True, True, False]])
    cluster = dict(slab, pbc=np.zeros((1, 3), bool), cell=np.zeros((1, 3, 3), np.float32))
    small = box(40, (12.0, 12.0, 12.0), (90, 90, 90), np.float32, 3.0, 39)
    for cfg, algorithm in ((slab, "cell_list"), (cluster, "cell_list"), (small, "auto")):
        code, msg, _, _, _, _ = search(cfg, HINT, algorithm=algorithm)
        assert code == TNR_RETRY and "plan hint" in msg, (code, msg)
        code, msg, plan, P, S, D = search(cfg, -1, algorithm=algorithm)
        assert code == TNR_OK and not plan & 8, (code, msg, plan)
        assert_same_keys(keys_of(P, S), keys_of(*oracle_call(cfg, algorithm=algorithm)))
    # an explicit brute_force request and a batch ignore the hint
    code, msg, plan, P, S, D = search(small, HINT, algorithm="brute_force")
    assert code == TNR_OK and plan == 1
    a = box(1500, (25.0, 25.0, 25.0), (90, 90, 90), np.float32, 6.0, 42)
    b = box(1800, (27.0, 26.0, 25.0), (80, 95, 100), np.float32, 6.0, 43)
    pair = W._pack([a["positions"], b["positions"]], [a["cell"][0], b["cell"][0]],
                   [np.ones(3, bool)] * 2, [1500, 1800], np.float32, 6.0)
    code, msg, plan, P, S, D = search(pair, HINT)
    assert code == TNR_OK and plan == 2, (code, msg, plan)
    assert_same_keys(keys_of(P, S), keys_of(*oracle_call(pair, algorithm="cell_list")))


def test_nonfinite_position_is_reported():
    cfg = box(3000, (30.0, 30.0, 30.0), (90, 90, 90), np.float32, 6.0, 40)
    cfg["positions"][1234, 2] = np.nan
    code, msg, _, _, _, _ = search(cfg, HINT)
    assert code != TNR_OK and "finite" in msg


def test_frontend_repeats_take_the_fast_prologue():
    # the first call reports the plan bit; the repeats run the fast prologue
    cfg = W.c4(seed=41, n_atoms=12000)
    t = {k: torch.as_tensor(cfg[k]).to(DEV) for k in ("positions", "cell", "pbc", "batch_ptr")}
    _speculation().clear()
    expected = keys_of(*oracle_call(cfg, algorithm="cell_list"))
    for call in range(3):
        P, S, D = neighbor_list("PSD", t["positions"], t["cell"], t["pbc"], cfg["cutoff"],
                                t["batch_ptr"], algorithm="cell_list")
        torch.cuda.synchronize()
        assert_same_keys(keys_of(P, S), expected)
        assert_geometry_close(P, S, None, D, cfg)
        plans = {v[1] for v in _speculation().values()}
        assert plans == {HINT}, plans
