"""GPU: Verlet-skin lists (``tonari_amd.verlet``).

Every call of a ``VerletList`` must return what ``neighbor_list`` returns
for the same inputs: the same (i, j, S) set, and d / D equal value for value
(both come from the reference's public predicate, evaluated in the input
dtype).  Checked along random-walk trajectories (the list is reused while
atoms stay within the skin and rebuilt after), for the pair policies and
``sorted``, with float32 coordinates far from the origin (the rounding
margin), with a skin below that margin, for the rebuild triggers (a large
move, a changed cell, pbc or batch_ptr, a new size), with no pairs at all, and
against the CPU oracle directly, all with the filter forced (``mode="filter"``);
the ``"auto"`` and ``"search"`` modes along trajectories too.  Gradients of
d and D equal the public call's.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests._util import (
    assert_grouped_by_source,
    assert_same_keys,
    assert_sorted_by_source,
    keys_of,
    oracle_call,
)
from tonari_amd import neighbor_list
from tonari_amd import workloads as W
from tonari_amd.verlet import VerletList

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _t(cfg, dtype=None):
    t = {k: torch.as_tensor(cfg[k]).to(DEV) for k in ("positions", "cell", "pbc", "batch_ptr")}
    if dtype is not None:
        t["positions"] = t["positions"].to(dtype)
        t["cell"] = t["cell"].to(dtype)
    return t


def _by_key(P, S, *rest):
    """Rows ordered by (i, j, S); returns numpy arrays."""
    P, S = P.cpu().numpy(), S.cpu().numpy()
    order = np.lexsort((S[:, 2], S[:, 1], S[:, 0], P[:, 1], P[:, 0]))
    return (P[order], S[order], *(x.detach().cpu().numpy()[order] for x in rest))


def _assert_equal_to_fresh(vl, t, cutoff, **options):
    P, S, d, D = vl(t["positions"], t["cell"], t["pbc"], t["batch_ptr"])
    Pf, Sf, df, Df = neighbor_list("PSdD", t["positions"], t["cell"], t["pbc"], cutoff,
                                   t["batch_ptr"], **options)
    assert_same_keys(keys_of(P, S), keys_of(Pf, Sf))
    a, b = _by_key(P, S, d, D), _by_key(Pf, Sf, df, Df)
    assert np.array_equal(a[2], b[2]), "d differs from the fresh search"
    assert np.array_equal(a[3], b[3]), "D differs from the fresh search"
    assert_grouped_by_source(P)
    return P


def _walk(t, rng, step, scale=None):
    """Moves every atom by a random vector of length below `step`."""
    n = t["positions"].shape[0]
    v = rng.normal(size=(n, 3))
    v /= np.linalg.norm(v, axis=1, keepdims=True) + 1e-30
    v *= step * rng.uniform(0.0, 1.0, size=(n, 1))
    t = dict(t)
    t["positions"] = t["positions"] + torch.as_tensor(v, dtype=t["positions"].dtype, device=DEV)
    return t


CASES = {
    "C2_f32": lambda: (W.c2(n_structures=32), None),
    "C2_f64": lambda: (W.c2(n_structures=32), torch.float64),
    "C4_f32": lambda: (W.c4(seed=51, n_atoms=20000), None),
    "C5_f64": lambda: (W.c5(n_structures=3, n_min=1500, n_max=3000), None),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_trajectory_equals_fresh_searches(name):
    cfg, dtype = CASES[name]()
    t = _t(cfg, dtype)
    skin = 1.0
    vl = VerletList("PSdD", cfg["cutoff"], skin, mode="filter", algorithm="auto")
    rng = np.random.default_rng(7)
    for step in range(8):
        print(f"[verlet] {name} step {step}", flush=True)
        _assert_equal_to_fresh(vl, t, cfg["cutoff"])
        t = _walk(t, rng, 0.15)
    assert vl.calls == 8
    # steps below 0.15: a build serves at least the three calls after it
    # (displacements below 0.45 < skin / 2 less the rounding margin)
    assert vl.builds <= 2
    builds = vl.builds
    # one atom moved by more than the skin: rebuilt once
    t["positions"] = t["positions"].clone()
    t["positions"][0] += 0.6
    _assert_equal_to_fresh(vl, t, cfg["cutoff"])
    assert vl.builds == builds + 1


@pytest.mark.parametrize("mode", ["auto", "search"])
@pytest.mark.parametrize("name", ["C2_f32", "C4_f32"])
def test_modes_equal_fresh_searches(name, mode):
    # "search" searches afresh at every call; "auto" times one filtered call
    # against a fresh search of the shape and keeps the faster path.  Every
    # call returns the fresh search's pairs, d and D.
    cfg, dtype = CASES[name]()
    t = _t(cfg, dtype)
    vl = VerletList("PSdD", cfg["cutoff"], 1.0, mode=mode)
    rng = np.random.default_rng(8)
    for step in range(6):
        print(f"[verlet] {name} mode={mode} step {step}", flush=True)
        _assert_equal_to_fresh(vl, t, cfg["cutoff"])
        t = _walk(t, rng, 0.05)  # at most 0.25 after five steps: no rebuild
    assert vl.calls == 6
    if mode == "search":
        assert vl.builds == 0 and vl.choice == {}
    else:
        (choice,) = vl.choice.values()
        assert choice in ("filter", "search")
        assert vl.builds == 1


def test_mode_is_checked():
    with pytest.raises(ValueError, match="mode"):
        VerletList("PS", 3.0, 0.5, mode="fast")


def test_small_moves_never_rebuild():
    cfg = W.c4(seed=52, n_atoms=8000)
    t = _t(cfg)
    vl = VerletList("PSdD", cfg["cutoff"], 0.8, mode="filter")
    rng = np.random.default_rng(8)
    base = t
    _assert_equal_to_fresh(vl, base, cfg["cutoff"])  # the build
    for step in range(4):
        t = _walk(base, rng, 0.3)  # each call within 0.3 of the build positions
        _assert_equal_to_fresh(vl, t, cfg["cutoff"])
    assert vl.builds == 1 and vl.calls == 5


@pytest.mark.parametrize("half_list,include_self,sorted_", [
    (True, False, True), (False, True, False), (True, True, False), (False, False, True)])
def test_pair_policies_and_order(half_list, include_self, sorted_):
    cfg = W.c2(n_structures=24)
    t = _t(cfg)
    opts = dict(half_list=half_list, include_self=include_self, sorted=sorted_)
    vl = VerletList("PSdD", cfg["cutoff"], 0.6, mode="filter", **opts)
    rng = np.random.default_rng(9)
    for _ in range(3):
        P = _assert_equal_to_fresh(vl, t, cfg["cutoff"], **opts)
        if sorted_:
            assert_sorted_by_source(P)
        t = _walk(t, rng, 0.1)
    assert vl.builds == 1


def test_quantities_follow_the_public_order():
    cfg = W.c2(n_structures=12)
    t = _t(cfg)
    vl = VerletList("jdiS", cfg["cutoff"], 0.5, mode="filter", sorted=True)
    for _ in range(2):
        j, d, i, S = vl(t["positions"], t["cell"], t["pbc"], t["batch_ptr"])
        P, Sf, df = neighbor_list("PSd", t["positions"], t["cell"], t["pbc"], cfg["cutoff"],
                                  t["batch_ptr"], sorted=True)
        assert i.dtype == j.dtype == torch.int64 and S.dtype == torch.int32
        a = _by_key(torch.stack([i, j], 1), S, d)
        b = _by_key(P, Sf, df)
        assert all(np.array_equal(x, y) for x, y in zip(a, b))


def test_rebuild_triggers():
    cfg = W.c2(n_structures=16)
    t = _t(cfg)
    vl = VerletList("PSdD", cfg["cutoff"], 0.6, mode="filter")
    _assert_equal_to_fresh(vl, t, cfg["cutoff"])
    assert vl.builds == 1
    # one atom moves by more than skin / 2
    moved = dict(t)
    moved["positions"] = t["positions"].clone()
    moved["positions"][5, 0] += 0.31
    _assert_equal_to_fresh(vl, moved, cfg["cutoff"])
    assert vl.builds == 2
    # a changed cell entry
    strained = dict(moved)
    strained["cell"] = moved["cell"].clone()
    strained["cell"][3, 1, 1] *= 1.0001
    _assert_equal_to_fresh(vl, strained, cfg["cutoff"])
    assert vl.builds == 3
    # a changed pbc entry
    slab = dict(strained)
    slab["pbc"] = strained["pbc"].clone()
    slab["pbc"][2, 2] = False
    _assert_equal_to_fresh(vl, slab, cfg["cutoff"])
    assert vl.builds == 4
    # a changed batch_ptr with the same sizes
    split = dict(slab)
    bp = slab["batch_ptr"].clone()
    bp[1] += 1
    split["batch_ptr"] = bp
    _assert_equal_to_fresh(vl, split, cfg["cutoff"])
    assert vl.builds == 5
    # unchanged inputs reuse the list
    _assert_equal_to_fresh(vl, split, cfg["cutoff"])
    assert vl.builds == 5
    # a new size
    small = _t(W.c2(n_structures=8))
    _assert_equal_to_fresh(vl, small, cfg["cutoff"])
    assert vl.builds == 6


def test_far_float32_coordinates_and_a_skin_below_the_margin():
    cfg = W.c4(seed=53, n_atoms=6000)
    t = _t(cfg)
    # unwrapped coordinates several cells away: larger rounding, larger margin
    t["positions"] = t["positions"] + 4.0 * t["cell"][0, 0]
    rng = np.random.default_rng(10)
    vl = VerletList("PSdD", cfg["cutoff"], 1.0, mode="filter")
    for _ in range(3):
        _assert_equal_to_fresh(vl, t, cfg["cutoff"])
        t = _walk(t, rng, 0.1)
    assert vl.builds == 1
    # a skin far below the float32 rounding of these coordinates: every call
    # falls back to a direct search and still equals it
    tiny = VerletList("PSdD", cfg["cutoff"], 1e-6, mode="filter")
    for _ in range(2):
        _assert_equal_to_fresh(tiny, t, cfg["cutoff"])
        t = _walk(t, rng, 0.1)


def test_no_pairs():
    cfg = W.c4(seed=54, n_atoms=500, density=0.001)
    t = _t(cfg)
    vl = VerletList("PSdD", 0.05, 0.01, mode="filter")
    P, S, d, D = vl(t["positions"], t["cell"], t["pbc"], t["batch_ptr"])
    assert P.shape == (0, 2) and S.shape == (0, 3) and d.shape == (0,) and D.shape == (0, 3)
    t = _walk(t, np.random.default_rng(11), 0.001)
    P, S, d, D = vl(t["positions"], t["cell"], t["pbc"], t["batch_ptr"])
    assert P.shape == (0, 2) and vl.builds == 1


def test_matches_the_oracle():
    cfg = W.c2(n_structures=16)
    t = _t(cfg)
    vl = VerletList("PS", cfg["cutoff"], 0.7, mode="filter", half_list=True)
    rng = np.random.default_rng(12)
    for _ in range(3):
        t = _walk(t, rng, 0.1)
        P, S = vl(t["positions"], t["cell"], t["pbc"], t["batch_ptr"])
        now = dict(cfg, positions=t["positions"].cpu().numpy(), half_list=True)
        assert_same_keys(keys_of(P, S), keys_of(*oracle_call(now, algorithm="auto")))
    assert vl.builds == 1


def test_gradients_equal_the_public_call():
    cfg = W.c2(n_structures=8)
    t = _t(cfg, torch.float64)
    vl = VerletList("dD", cfg["cutoff"], 0.5, mode="filter")
    for _ in range(2):
        pos = t["positions"].clone().requires_grad_()
        cell = t["cell"].clone().requires_grad_()
        d, D = vl(pos, cell, t["pbc"], t["batch_ptr"])
        (d.sum() + (D * D).sum()).backward()
        gp, gc = pos.grad.clone(), cell.grad.clone()
        pos.grad = None
        cell.grad = None
        d2, D2 = neighbor_list("dD", pos, cell, t["pbc"], cfg["cutoff"], t["batch_ptr"])
        (d2.sum() + (D2 * D2).sum()).backward()
        assert torch.allclose(gp, pos.grad, rtol=1e-10, atol=1e-10)
        assert torch.allclose(gc, cell.grad, rtol=1e-10, atol=1e-10)
        t = _walk(t, np.random.default_rng(13), 0.05)
    assert vl.builds == 1


def test_shifts_beyond_the_compact_records_fall_back_to_searches():
    # a 0.05 A period along x with a 30 A cutoff: shifts up to about +-600,
    # beyond the stored records' 10-bit fields; every call then equals a
    # direct search
    pos = torch.tensor([[0.01, 0.0, 0.0], [0.02, 1.0, 0.5], [0.03, -0.5, 2.0]],
                       dtype=torch.float64, device=DEV)
    cell = torch.diag(torch.tensor([0.05, 10.0, 10.0], dtype=torch.float64)).to(DEV)
    pbc = torch.tensor([True, False, False], device=DEV)
    bp = torch.tensor([0, 3], device=DEV)
    t = {"positions": pos, "cell": cell[None], "pbc": pbc[None], "batch_ptr": bp}
    vl = VerletList("PSdD", 30.0, 0.5, mode="filter")
    for _ in range(2):
        P = _assert_equal_to_fresh(vl, t, 30.0)
        assert P.shape[0] > 3000
        assert int(neighbor_list("S", pos, cell, pbc, 30.0)[0].abs().max()) > 511
        t = dict(t, positions=t["positions"] + 0.001)


def test_sources_recovered_across_tiles_and_empty_structures():
    # structures of 0 to 300 atoms: runs of every length, tiles that start
    # inside a run, empty structures in batch_ptr
    rng = np.random.default_rng(14)
    counts = [0, 300, 1, 0, 57, 2, 0, 180, 0]
    positions, cells = [], []
    for n in counts:
        L = 9.0
        positions.append(rng.uniform(0, L, size=(n, 3)))
        cells.append(L * np.eye(3))
    cfg = {
        "positions": np.concatenate(positions).astype(np.float32),
        "cell": np.stack(cells).astype(np.float32),
        "pbc": np.ones((len(counts), 3), bool),
        "batch_ptr": np.concatenate([[0], np.cumsum(counts)]).astype(np.int64),
        "cutoff": 4.0,
    }
    t = _t(cfg)
    for sorted_ in (True, False):
        vl = VerletList("PSdD", 4.0, 0.8, mode="filter", sorted=sorted_)
        for _ in range(3):
            P = _assert_equal_to_fresh(vl, t, 4.0, sorted=sorted_)
            assert P.shape[0] > 2 * 2048
            t = _walk(t, rng, 0.1)
        assert vl.builds == 1


def test_filter_in_another_pair_mode_is_refused():
    # a list stored in one pair mode holds other pairs than another mode's:
    # the C ABI records the mode with the list and refuses a filter request
    # whose half_list or include_self differ (the same mode is accepted)
    import ctypes

    from tonari_amd._extensions import (
        ALGORITHMS, TNR_INPUT_ERROR, TNR_OK, Outputs, Request, SkinList, load_torch_hip,
    )

    lib = load_torch_hip()
    cfg = W.c4(seed=91, n_atoms=3000)
    t = _t(cfg)
    P, S = neighbor_list("PS", t["positions"], t["cell"], t["pbc"], cfg["cutoff"] + 0.5,
                         t["batch_ptr"])
    n = P.shape[0]

    def request(half_list, include_self):
        return Request(
            dtype=0, algorithm=ALGORITHMS["auto"], n_atoms=t["positions"].shape[0],
            n_structures=1, positions=t["positions"].data_ptr(),
            batch_ptr=t["batch_ptr"].data_ptr(), cell=t["cell"].data_ptr(),
            pbc=t["pbc"].data_ptr(), cutoff=cfg["cutoff"], half_list=int(half_list),
            include_self=int(include_self), sorted=0, stencil_reach=0,
        )

    req = request(False, False)
    ws_bytes = int(lib.tnr_skin_workspace_size(ctypes.byref(req), n))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    lst = SkinList()
    err = ctypes.create_string_buffer(256)
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.tnr_skin_store(ctypes.byref(req), cfg["cutoff"] + 0.5, P.data_ptr(), S.data_ptr(),
                              n, ws.data_ptr(), ws_bytes, ctypes.byref(lst), stream, err,
                              len(err)) == TNR_OK
    assert lst.pair_mode == 0
    Pout = torch.empty((n, 2), dtype=torch.int64, device=DEV)
    out = Outputs(n_pairs=n, plan=0, n_tasks=0, pairs=Pout.data_ptr())
    host = torch.zeros(8, dtype=torch.int64, pin_memory=True)
    for half_list, include_self in ((True, False), (False, True), (True, True)):
        code = lib.tnr_skin_filter_async(ctypes.byref(request(half_list, include_self)),
                                         ctypes.byref(lst), ws.data_ptr(), ws_bytes,
                                         ctypes.byref(out), host.data_ptr(), stream, err,
                                         len(err))
        assert code == TNR_INPUT_ERROR and b"half_list or include_self" in err.value
    assert lib.tnr_skin_filter_async(ctypes.byref(req), ctypes.byref(lst), ws.data_ptr(),
                                     ws_bytes, ctypes.byref(out), host.data_ptr(), stream, err,
                                     len(err)) == TNR_OK
    torch.cuda.synchronize()
