"""GPU parity of the cell list on structures whose atoms lie outside the cell.

Atoms outside the cell are searched at their wrapped representatives, and
each kept pair's shift is corrected by the two atoms' wraps, S = k - w_t +
w_s, with D formed from the original positions (the reference's
representatives: csrc/core/neighbors_cpu.cpp:98-131, used at 247-261).  The
emitting pass of such a structure takes one of three forms, by the size of a
bin's stencil and the wraps:

- staged: the candidates' original positions, indices and packed k - w_t in
  LDS (every k - w_t within +-511 and a stencil of at most 512 (float32) or
  1,280 (float64) candidates), at most 64 or more than 64 sources per bin;
- loaded: the same values gathered per pair (larger stencils or wraps);
- the slow path beyond 2,048 candidates.

Batches below mix sparse and dense structures, small and large wraps and
partly periodic cells, so that every form runs, and compare the (i, j, S)
multiset bit-exactly with the CPU oracle; d and D within 1e-5 relative
(float32) / 1e-12 (float64).
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
MODES = [(False, False), (True, False), (False, True), (True, True)]


def wrapped_batch(specs, dtype, seed, cutoff):
    """specs: (atoms, cell lengths, largest wrap, pbc) per structure.  Triclinic
    cells; fractional coordinates uniform in the cell, then moved by whole
    cells up to the largest wrap along the periodic axes."""
    rng = np.random.Generator(np.random.PCG64(seed))
    positions, cells, pbcs = [], [], []
    for n, (la, lb, lc), wmax, pbc in specs:
        cell = np.array([[la, 0.0, 0.0], [0.3 * la, lb, 0.0], [-0.2 * la, 0.25 * lb, lc]])
        frac = rng.random((n, 3))
        move = rng.integers(-wmax, wmax + 1, size=(n, 3)) * np.asarray(pbc, dtype=np.int64)
        positions.append((frac + move) @ cell)
        cells.append(cell)
        pbcs.append(pbc)
    return {
        "positions": np.concatenate(positions).astype(dtype),
        "cell": np.stack(cells).astype(dtype),
        "pbc": np.asarray(pbcs, dtype=bool),
        "batch_ptr": np.concatenate([[0], np.cumsum([s[0] for s in specs])]).astype(np.int64),
        "cutoff": cutoff,
    }


def run(cfg, quantities, **options):
    t = lambda x: torch.as_tensor(x).to(DEV)  # noqa: E731
    out = neighbor_list(
        quantities, t(cfg["positions"]), t(cfg["cell"]), t(cfg["pbc"]), cfg["cutoff"],
        t(cfg["batch_ptr"]), **options,
    )
    torch.cuda.synchronize()
    return out


def run_abi(cfg, reach, half_list=False, include_self=False):
    """Count and emit through the C ABI with the stencil reach forced to
    `reach` bins per cutoff; returns P, S, d, D (grouped by source)."""
    import ctypes

    from tonari_amd._extensions import ALGORITHMS, TNR_OK, Outputs, Request, load_torch_hip

    lib = load_torch_hip()
    t = {k: torch.as_tensor(cfg[k]).to(DEV) for k in ("positions", "cell", "pbc", "batch_ptr")}
    pos = t["positions"]
    req = Request(
        dtype=0 if pos.dtype == torch.float32 else 1, algorithm=ALGORITHMS["cell_list"],
        n_atoms=pos.shape[0], n_structures=t["batch_ptr"].numel() - 1,
        positions=pos.data_ptr(), batch_ptr=t["batch_ptr"].data_ptr(),
        cell=t["cell"].data_ptr(), pbc=t["pbc"].data_ptr(), cutoff=cfg["cutoff"],
        half_list=int(half_list), include_self=int(include_self), sorted=0,
        stencil_reach=reach,
    )
    ws_bytes = int(lib.tnr_workspace_size(ctypes.byref(req)))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    host = torch.zeros(8, dtype=torch.int64, pin_memory=True)
    err = ctypes.create_string_buffer(512)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.tnr_count_async(ctypes.byref(req), ws.data_ptr(), ws_bytes, host.data_ptr(),
                             stream, err, len(err))
    assert rc == TNR_OK, err.value.decode()
    torch.cuda.synchronize()
    n = ctypes.c_int64(-1)
    rc = lib.tnr_count_finish(host.data_ptr(), ctypes.byref(n), err, len(err))
    assert rc == TNR_OK, err.value.decode()
    E = int(n.value)
    P = torch.empty((E, 2), dtype=torch.int64, device=DEV)
    S = torch.empty((E, 3), dtype=torch.int32, device=DEV)
    d = torch.empty((E,), dtype=pos.dtype, device=DEV)
    D = torch.empty((E, 3), dtype=pos.dtype, device=DEV)
    out = Outputs(n_pairs=E, plan=int(host[3]), n_tasks=int(host[4]), pairs=P.data_ptr(),
                  shifts=S.data_ptr(), distances=d.data_ptr(), vectors=D.data_ptr())
    rc = lib.tnr_emit(ctypes.byref(req), ws.data_ptr(), ws_bytes, ctypes.byref(out), stream,
                      err, len(err))
    assert rc == TNR_OK, err.value.decode()
    torch.cuda.synchronize()
    return P, S, d, D


def specs(dtype):
    """Sparse (few sources per bin), dense (larger stencils), a slab with one
    open axis, large wraps, and an open middle axis.  Wraps of 600 cells do
    not pack; they are float64 only, since float32 positions 10^4 A from the
    cell round D beyond the float32 tolerance (in the reference too: D is
    formed in the positions' type)."""
    return [
        (900, (28.0, 30.0, 26.0), 2, (True, True, True)),
        (1500, (16.0, 17.0, 15.5), 1, (True, True, True)),
        (1200, (24.0, 24.0, 18.0), 3, (True, True, False)),
        (700, (20.0, 21.0, 19.0), 600 if dtype == np.float64 else 4, (True, True, True)),
        (2500, (30.0, 30.0, 30.0), 1, (True, False, True)),
    ]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("half_list,include_self", MODES)
def test_wrapped_structures_match_oracle(dtype, half_list, include_self):
    cfg = wrapped_batch(specs(dtype), dtype, 5150, cutoff=5.0)
    print(f"[wrapped] {np.dtype(dtype).name} half={half_list} self={include_self}", flush=True)
    cfg = dict(cfg, half_list=half_list, include_self=include_self)
    expected = keys_of(*oracle_call(cfg, algorithm="cell_list"))
    for sorted_ in (False, True):
        P, S, d, D = run(cfg, "PSdD", algorithm="cell_list", half_list=half_list,
                         include_self=include_self, sorted=sorted_)
        assert_same_keys(keys_of(P, S), expected)
        assert_grouped_by_source(P)
        if sorted_:
            assert_sorted_by_source(P)
        assert_geometry_close(P, S, d, D, cfg)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_wrapped_single_structure_separate_rows(dtype):
    # one structure (the single-structure prologue), i and j as separate rows
    cfg = wrapped_batch([(6000, (39.0, 40.0, 38.0), 2, (True, True, True))], dtype, 77,
                        cutoff=5.5)
    expected = keys_of(*oracle_call(cfg, algorithm="cell_list"))
    print(f"[wrapped] single {np.dtype(dtype).name}: {len(expected)} pairs", flush=True)
    i, j, S, d, D = run(cfg, "ijSdD", algorithm="cell_list")
    P = torch.stack([i, j], dim=1)
    assert_same_keys(keys_of(P, S), expected)
    assert_geometry_close(P, S, d, D, cfg)


def test_wrapped_then_unwrapped_calls():
    # the staging of one call's wrapped structures leaves nothing behind for
    # the next call's unwrapped ones, and back
    box = (24.7, 25.0, 24.0)
    wrapped = wrapped_batch([(1500, box, 2, (True, True, True))], np.float64, 3, cutoff=5.0)
    plain = wrapped_batch([(1500, box, 0, (True, True, True))], np.float64, 3, cutoff=5.0)
    for cfg in (wrapped, plain, wrapped):
        expected = keys_of(*oracle_call(cfg, algorithm="cell_list"))
        P, S = run(cfg, "PS", algorithm="cell_list")
        assert_same_keys(keys_of(P, S), expected)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("half_list,include_self", [(False, False), (True, True)])
def test_wrapped_bins_beyond_a_wave_of_sources(dtype, half_list, include_self):
    # Reach 1 on a thin slab (one bin across its open axis: 9-bin stencils)
    # and on a wire (3-bin stencils) puts about 100 sources in a bin under
    # small stencils: the staged decode path with more than 64 sources per
    # bin, float64 on the slab, both types on the wire.  Reach 2 and the
    # automatic choice cover the smaller bins of the same structures.
    cfg = wrapped_batch(
        [(1000, (20.0, 21.0, 4.0), 2, (True, True, False)),
         (600, (30.0, 4.0, 4.0), 3, (True, False, False))],
        dtype, 909, cutoff=5.0)
    expected = keys_of(*oracle_call(dict(cfg, half_list=half_list, include_self=include_self),
                                    algorithm="cell_list"))
    for reach in (1, 2, 0):
        print(f"[wrapped] wide bins {np.dtype(dtype).name} reach={reach} half={half_list} "
              f"self={include_self}", flush=True)
        P, S, d, D = run_abi(cfg, reach, half_list, include_self)
        assert_same_keys(keys_of(P, S), expected)
        assert_grouped_by_source(P)
        assert_geometry_close(P, S, d, D, cfg)
