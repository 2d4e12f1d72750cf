"""GPU: repeated calls of one request shape.

The frontend launches the writing pass of a repeated call before the pair
count is known, into outputs sized from the previous call.  Every case here
compares with the CPU oracle: the plain repeat, and the misses that make the
writing pass run again (more pairs than the outputs hold, more bins than the
launch covered, a plan that switches algorithm).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests._util import assert_geometry_close, assert_same_keys, keys_of, oracle_call
from tonari_amd import neighbor_list
from tonari_amd import workloads as W
from tonari_amd._torch_frontend import _speculation

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def run(quantities, cfg, **kw):
    t = lambda x: torch.as_tensor(x).to(DEV)  # noqa: E731
    out = neighbor_list(
        quantities, t(cfg["positions"]), t(cfg["cell"]), t(cfg["pbc"]), cfg["cutoff"],
        t(cfg["batch_ptr"]), algorithm=kw.pop("algorithm", "auto"), **kw,
    )
    torch.cuda.synchronize()
    return out


def check(cfg, quantities="PSD", **kw):
    P, S, D = run(quantities, cfg, **kw)
    assert_same_keys(keys_of(P, S), keys_of(*oracle_call(cfg, algorithm=kw.get("algorithm"))))
    assert_geometry_close(P, S, None, D, cfg)
    return P


def test_repeated_calls():
    cfg = W.c4(seed=11, n_atoms=20000)
    first = check(cfg)
    for _ in range(3):
        again = check(cfg)
        assert again.shape == first.shape


def test_more_pairs_than_outputs_hold():
    # same atom count, the second box four times denser: the pair count
    # grows far beyond the first call's margin
    sparse = W.c4(seed=12, n_atoms=6000, density=0.025)
    dense = W.c4(seed=13, n_atoms=6000, density=0.1)
    n_sparse = len(check(sparse))
    n_dense = len(check(dense))
    assert n_dense > 2 * n_sparse
    check(dense)
    check(sparse)


def test_more_bins_than_launch_covered():
    # same atom count, a much larger box: more bins than the previous call
    small = W.c4(seed=14, n_atoms=6000, density=0.1)
    large = W.c4(seed=15, n_atoms=6000, density=0.01)
    check(small)
    check(large)
    check(small)


def test_plan_switch():
    # the same atom count searched by brute force (an open cluster of at
    # most 2,048 atoms under auto) and then by a cell list (a periodic box of
    # 300 x 27 atom images)
    rng = np.random.default_rng(16)
    n = 300
    cluster = {
        "positions": rng.uniform(0.0, 8.0, (n, 3)).astype(np.float32),
        "cell": np.zeros((1, 3, 3), np.float32),
        "pbc": np.zeros((1, 3), bool),
        "batch_ptr": np.array([0, n], np.int64),
        "cutoff": 3.0,
    }
    box = W.c4(seed=17, n_atoms=n, density=0.1)
    for cfg in (cluster, box, cluster, box):
        check(cfg)


def _molecules(sizes, seed):
    rng = np.random.default_rng(seed)
    pos = [rng.uniform(0.0, (n / 0.05) ** (1 / 3), (n, 3)) + 40.0 * k for k, n in enumerate(sizes)]
    return {
        "positions": np.concatenate(pos).astype(np.float32),
        "cell": np.zeros((len(sizes), 3, 3), np.float32),
        "pbc": np.zeros((len(sizes), 3), bool),
        "batch_ptr": np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64),
        "cutoff": 4.0,
    }


def test_plan_hint_miss_in_a_batch():
    # batches of one shape: molecules that auto searches by brute force
    # (each at most 2,048 atoms), then the same atom count with one molecule
    # of 2,500 atoms (a cell list), and with a periodic structure (brute
    # force, not a molecule).  A repeat after a molecules-only plan runs the
    # molecule prologue; the device finds the other structure and the count
    # runs again in full.
    brute = _molecules([1200, 1500, 50, 2000], 18)
    mixed = _molecules([2500, 1000, 850, 400], 19)
    periodic = _molecules([1200, 1500, 50, 2000], 20)
    periodic["pbc"][2] = True  # 50 atoms x 27 images: brute force under auto
    periodic["cell"][2] = np.eye(3, dtype=np.float32) * 25.0
    for cfg in (brute, brute, mixed, brute, mixed, mixed, brute, periodic, periodic, brute):
        check(cfg)
    for half_list in (False, True):
        for include_self in (False, True):
            cfg = dict(brute, half_list=half_list, include_self=include_self)
            for _ in range(2):
                check(cfg, half_list=half_list, include_self=include_self)


def test_molecule_plan_guess_with_a_periodic_structure():
    # one shape (4,750 atoms in 4 structures): a cell list and molecules
    # (plan 7), then a cell list, molecules and a small periodic structure
    # searched by brute force (plan 3, not every brute-force structure a
    # molecule).  The repeat's speculative emit, launched with plan 7, takes
    # the molecule kernel, which must write nothing for such a count; the
    # frontend then emits again with the count's plan.
    mixed = _molecules([2500, 1000, 850, 400], 22)
    periodic = _molecules([2500, 1000, 1200, 50], 23)
    periodic["pbc"][3] = True
    periodic["cell"][3] = np.eye(3, dtype=np.float32) * 25.0
    _speculation().clear()
    for cfg in (mixed, periodic, mixed, mixed, periodic, periodic):
        check(cfg)


def test_plan_hint_through_the_abi():
    import ctypes

    from tonari_amd._extensions import (
        ALGORITHMS, TNR_OK, TNR_RETRY, Request, load_torch_hip,
    )

    lib = load_torch_hip()

    def count(cfg, hint):
        t = {k: torch.as_tensor(cfg[k]).to(DEV) for k in ("positions", "cell", "pbc", "batch_ptr")}
        req = Request(
            dtype=0, algorithm=ALGORITHMS["auto"], n_atoms=t["positions"].shape[0],
            n_structures=t["batch_ptr"].numel() - 1, positions=t["positions"].data_ptr(),
            batch_ptr=t["batch_ptr"].data_ptr(), cell=t["cell"].data_ptr(),
            pbc=t["pbc"].data_ptr(), cutoff=cfg["cutoff"], half_list=0, include_self=0,
            sorted=0, stencil_reach=0,
        )
        ws_bytes = int(lib.tnr_workspace_size(ctypes.byref(req)))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
        host = torch.zeros(8, dtype=torch.int64, pin_memory=True)
        err = ctypes.create_string_buffer(256)
        stream = torch.cuda.current_stream().cuda_stream
        assert lib.tnr_count_async_hinted(ctypes.byref(req), ws.data_ptr(), ws_bytes,
                                          host.data_ptr(), stream, hint, err, len(err)) == TNR_OK
        torch.cuda.synchronize()
        n = ctypes.c_int64(-1)
        code = lib.tnr_count_finish(host.data_ptr(), ctypes.byref(n), err, len(err))
        return code, int(n.value), int(host[3]), err.value.decode()

    brute = _molecules([1200, 1500, 50, 2000], 18)
    mixed = _molecules([2500, 1000, 850, 400], 19)
    periodic = _molecules([1200, 1500, 50, 2000], 20)
    periodic["pbc"][2] = True
    periodic["cell"][2] = np.eye(3, dtype=np.float32) * 25.0
    # hint 1: brute force only; hint 5: every structure a molecule
    for cfg, plan in ((brute, 5), (mixed, 3 | 4), (periodic, 1)):
        expected = len(keys_of(*oracle_call(cfg, algorithm="brute_force")))
        code, n, got_plan, _ = count(cfg, -1)
        assert code == TNR_OK and n == expected and got_plan == plan
        for hint in (1, 5):
            code, n, _, msg = count(cfg, hint)
            holds = (plan & 3) == 1 and (hint == 1 or plan & 4)
            if holds:
                assert code == TNR_OK and n == expected, (plan, hint)
            else:
                assert code == TNR_RETRY and "plan hint" in msg, (plan, hint)
    # the molecule prologue skips the atom pass: the molecule count checks
    # the positions
    bad = _molecules([1200, 1500, 50, 2000], 21)
    bad["positions"][1350, 1] = np.nan
    code, _, _, msg = count(bad, 5)
    assert code != TNR_OK and "finite" in msg


def test_cutoff_change_between_calls():
    # one shape at three cutoffs in turn: each call's pairs are its own
    # cutoff's, whether the call follows one at the same cutoff or not
    base = W.c4(seed=14, n_atoms=8000)
    counts = {}
    for rc in (6.0, 4.5, 6.0, 7.0, 4.5):
        cfg = dict(base, cutoff=rc)
        counts.setdefault(rc, set()).add(len(check(cfg)))
    assert all(len(v) == 1 for v in counts.values())
    assert len({next(iter(v)) for v in counts.values()}) == 3
