"""GPU: the width of the hit-mask rows (tnr_request::mask_words).

The counting passes keep one 64-bit hit mask per chunk of 64 candidates in a
row of mask_words words per atom, and report the longest row any source or
brute-force structure wanted (host_result[5]).  A cell-list bin whose stencil
has more chunks than a row holds takes the slow path, which stores no masks,
in both passes; a molecule of more than 64 x mask_words atoms takes the
general brute-force passes; a periodic brute-force structure splits its
sources into at most mask_words k0 slices.  Every case compares the emitted
(i, j, S) multiset with the CPU oracle bit for bit and D with the float64
formula (1e-5 relative for float32, 1e-12 for float64) at widths from one
word through the reported need to the maximum of 64, and checks that the
reported need does not depend on the width and that the workspace shrinks
with the width.
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
    ALGORITHMS, TNR_INPUT_ERROR, TNR_OK, TNR_RETRY, Outputs, Request, load_torch_hip,
)
from tonari_amd._torch_frontend import _speculation

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def search(cfg, mask_words, *, algorithm, hint=-1, half_list=False, include_self=False,
           sorted=False):
    """Count and emit P, S, D through the C ABI with rows of `mask_words`;
    returns (code, message, host_result, workspace bytes, P, S, D)."""
    lib = load_torch_hip()
    t = {k: torch.as_tensor(cfg[k]).to(DEV) for k in ("positions", "cell", "pbc", "batch_ptr")}
    pos = t["positions"]
    req = Request(
        dtype=0 if pos.dtype == torch.float32 else 1, algorithm=ALGORITHMS[algorithm],
        n_atoms=pos.shape[0], n_structures=t["batch_ptr"].numel() - 1,
        positions=pos.data_ptr(), batch_ptr=t["batch_ptr"].data_ptr(),
        cell=t["cell"].data_ptr(), pbc=t["pbc"].data_ptr(), cutoff=cfg["cutoff"],
        half_list=int(half_list), include_self=int(include_self), sorted=int(sorted),
        stencil_reach=0, mask_words=mask_words,
    )
    ws_bytes = int(lib.tnr_workspace_size(ctypes.byref(req)))
    assert ws_bytes > 0
    # garbage in the workspace: no pass may rely on zeroed memory
    ws = torch.full((ws_bytes,), 0x5A, dtype=torch.uint8, device=DEV)
    host = torch.zeros(8, dtype=torch.int64, pin_memory=True)
    err = ctypes.create_string_buffer(512)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.tnr_count_async_hinted(ctypes.byref(req), ws.data_ptr(), ws_bytes, host.data_ptr(),
                                    stream, hint, err, len(err))
    assert rc == TNR_OK, err.value.decode()
    torch.cuda.synchronize()
    n = ctypes.c_int64(-1)
    code = lib.tnr_count_finish(host.data_ptr(), ctypes.byref(n), err, len(err))
    result = [int(x) for x in host]
    if code != TNR_OK:
        return code, err.value.decode(), result, ws_bytes, None, None, None
    E = int(n.value)
    P = torch.empty((E, 2), dtype=torch.int64, device=DEV)
    S = torch.empty((E, 3), dtype=torch.int32, device=DEV)
    D = torch.empty((E, 3), dtype=pos.dtype, device=DEV)
    out = Outputs(n_pairs=E, plan=result[3], n_tasks=result[4], pairs=P.data_ptr(),
                  shifts=S.data_ptr(), vectors=D.data_ptr())
    if E > 0:
        rc = lib.tnr_emit(ctypes.byref(req), ws.data_ptr(), ws_bytes, ctypes.byref(out), stream,
                          err, len(err))
        assert rc == TNR_OK, err.value.decode()
    torch.cuda.synchronize()
    return code, "", result, ws_bytes, P, S, D


def sweep(cfg, algorithm, widths, **kw):
    """Search at the library default, then at every width; returns the
    reported need.  Each run's rows must equal the oracle's."""
    full = dict(cfg, half_list=kw.get("half_list", False),
                include_self=kw.get("include_self", False))
    expected = keys_of(*oracle_call(full, algorithm=algorithm))
    code, msg, host, ws_default, P, S, D = search(full, 0, algorithm=algorithm, **kw)
    assert code == TNR_OK, msg
    need = host[5]
    assert 0 <= need <= 64, need
    assert_same_keys(keys_of(P, S), expected)
    sizes = {}
    for mw in widths(need):
        print(f"[mask_words] {algorithm} width {mw} (need {need})", flush=True)
        code, msg, host, ws_bytes, P, S, D = search(full, mw, algorithm=algorithm, **kw)
        assert code == TNR_OK, msg
        assert host[5] == need, (mw, host[5], need)
        assert_same_keys(keys_of(P, S), expected)
        assert_geometry_close(P, S, None, D, full)
        if kw.get("sorted"):
            src = P[:, 0]
            assert bool((src[1:] >= src[:-1]).all())
        sizes[mw] = ws_bytes
    # the workspace grows with the width, 8 bytes per atom and word
    ordered = [sizes[w] for w in sorted(sizes)]
    assert ordered == sorted(ordered)
    if 64 in sizes:
        assert sizes[64] == ws_default
    return need


def around(need):
    return sorted({1, max(need - 1, 1), max(need, 1), min(need + 1, 64), 32, 64})


def test_cell_list_box():
    # C4's density at 20,000 atoms: stencils of several chunks
    need = sweep(W.c4(seed=61, n_atoms=20_000), "cell_list", around)
    assert need >= 2


@pytest.mark.parametrize("half_list,include_self", [(False, False), (True, True)])
def test_wrapped_slabs_float64(half_list, include_self):
    cfg = W.c5(seed=62, n_structures=3, n_min=400, n_max=1500)
    sweep(cfg, "cell_list", around, half_list=half_list, include_self=include_self, sorted=True)


def test_molecules_wider_than_a_row_take_the_brute_force_passes():
    # C3's molecules (up to a few hundred atoms): at widths below the
    # largest molecule's chunks those molecules run the general passes
    cfg = W.c3(seed=63, n_structures=40)
    need = sweep(cfg, "auto", around, half_list=True, sorted=True)
    largest = int(np.diff(cfg["batch_ptr"]).max())
    assert need == (largest + 63) // 64
    if need > 1:
        # the molecule hint does not hold when a molecule outgrows the row
        full = dict(cfg, half_list=True, include_self=False)
        code, msg, *_ = search(full, need - 1, algorithm="auto", hint=5, half_list=True)
        assert code == TNR_RETRY and "plan hint" in msg, (code, msg)
        code, msg, host, *_ = search(full, need, algorithm="auto", hint=5, half_list=True)
        assert code == TNR_OK and host[3] == 5, (code, msg, host)


def test_periodic_brute_force_slices():
    # one periodic box searched by brute force: 3,000 atoms over K0 = 3
    # planes split into k0 slices, whose counts live in the hit-mask rows
    rng = np.random.Generator(np.random.PCG64(64))
    cell = W.triclinic_cell((30.0, 31.0, 29.0), (85.0, 95.0, 100.0))
    pos = rng.uniform(0.0, 1.0, (3000, 3)) @ cell
    cfg = W._pack([pos], [cell], [np.ones(3, bool)], [3000], np.float32, 6.0)
    need = sweep(cfg, "brute_force", lambda need: sorted({1, 2, max(need, 1), 64}))
    assert need > 1


def test_bad_width_is_rejected():
    cfg = W.c4(seed=65, n_atoms=2000)
    lib = load_torch_hip()
    for mw in (-1, 65):
        req = Request(dtype=0, algorithm=0, n_atoms=2000, n_structures=1, positions=1,
                      batch_ptr=1, cell=1, pbc=1, cutoff=cfg["cutoff"], mask_words=mw)
        assert lib.tnr_workspace_size(ctypes.byref(req)) == 0
        err = ctypes.create_string_buffer(256)
        code = lib.tnr_count_async(ctypes.byref(req), None, 0, None, None, err, len(err))
        assert code == TNR_INPUT_ERROR


def test_frontend_sizes_repeats_from_the_reported_need():
    cfg = W.c4(seed=66, n_atoms=15_000)
    t = {k: torch.as_tensor(cfg[k]).to(DEV) for k in ("positions", "cell", "pbc", "batch_ptr")}
    expected = keys_of(*oracle_call(cfg, algorithm="cell_list"))
    _speculation().clear()
    widths = []
    for call in range(3):
        P, S, D = neighbor_list("PSD", t["positions"], t["cell"], t["pbc"], cfg["cutoff"],
                                t["batch_ptr"], algorithm="cell_list")
        torch.cuda.synchronize()
        assert_same_keys(keys_of(P, S), expected)
        assert_geometry_close(P, S, None, D, cfg)
        widths.append({v[3] for v in _speculation().values()})
    code, msg, host, *_ = search(cfg, 0, algorithm="cell_list")
    assert widths[-1] == {min(host[5] + 1, 64)}, (widths, host[5])
