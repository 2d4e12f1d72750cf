"""Verlet-skin neighbor lists for molecular-dynamics loops.

The reference lists a Verlet skin as unsupported (``docs/design.md:125-127``);
every step of an MD loop then pays a full search.  ``VerletList`` searches
once at ``cutoff + skin`` (the public call, P and S) and stores that list,
8 bytes per pair, with the call's positions, cell, pbc and batch_ptr
(``tnr_skin_store``).  At later steps one pass over the stored pairs
re-decides each with the reference's public predicate at the current
positions and writes the kept ones (``tnr_skin_filter_async``); the same
pass measures the largest displacement since the build and compares cell,
pbc and batch_ptr with the build's, and ``tnr_skin_finish`` accepts the
filtered list only when it provably equals a fresh search at ``cutoff``
(every atom moved less than about skin / 2, less a rounding margin, and
nothing else changed).  Otherwise the list is rebuilt at the current
positions.

Either way a call returns what ``neighbor_list`` returns for the same
arguments: the same (i, j, S) pairs with the same d and D.  The pairs come in
the order of the stored list (a ``sorted`` list stays sorted; the pairs of a
source stay contiguous).  Positions that an MD code wraps back into the cell
move by a cell vector and so force a rebuild; wrap them only at rebuilds, or
not at all.

Filtering pays where a search is costly per kept pair (batches searched by
brute force: C2 0.079 against 0.118 ms); where the search stages its
candidates (a large periodic box under the cell list) it is the faster of
the two.  So by default (``mode="auto"``) the first call of a request shape
that filters without a rebuild also times a fresh search of the same inputs
(wall time, a warm call after a warm-up one) and keeps the faster path for
that shape; ``mode="filter"`` always filters and ``mode="search"`` always
searches.  A search returns the same pairs in its own order.
"""

from __future__ import annotations

import contextlib
import ctypes
import time
from math import isfinite

import torch
from torch import Tensor

from ._extensions import (
    ALGORITHMS,
    HOST_RESULT_SLOTS,
    TNR_OK,
    Outputs,
    Request,
    SkinList,
    check_device,
    load_torch_hip,
)
from ._torch_frontend import (
    _FusedGeometry,
    _allocate,
    _capacity,
    _raise,
    _require_torch_tensors,
    _rows,
    neighbor_list_hip,
    normalize_torch_inputs,
    validate_torch_inputs,
)
from .api import _VALID_QUANTITIES

__all__ = ["VerletList"]


class _Stored:
    """One stored list: its key, the skin workspace that holds it, its ABI record."""

    def __init__(self, key, workspace: Tensor, ws_bytes: int, lst: SkinList):
        self.key = key
        self.workspace, self.ws_bytes, self.list = workspace, ws_bytes, lst


class VerletList:
    """A neighbor list reused across steps while atoms move less than the skin allows.

    ``VerletList(quantities, cutoff, skin)`` takes the options of
    ``neighbor_list`` (``algorithm``, ``sorted``, ``half_list``,
    ``include_self``); calling it with ``(positions, cell, pbc, batch_ptr)``
    returns the requested quantities for those inputs, like
    ``neighbor_list(quantities, positions, cell, pbc, cutoff, batch_ptr, ...)``,
    with autograd on d and D as there.  ``mode`` (``"auto"``, ``"filter"`` or
    ``"search"``) picks between filtering the stored list and a fresh search:
    ``"auto"`` times both once per request shape (device, dtype, atoms,
    structures) and keeps the faster, recorded in ``choice``.  ``builds``
    counts the searches at ``cutoff + skin``; ``calls`` counts the calls.
    ROCm (HIP) tensors only.
    """

    def __init__(self, quantities: str, cutoff: float, skin: float, *, algorithm: str = "auto",
                 sorted: bool = False, half_list: bool = False, include_self: bool = False,
                 mode: str = "auto"):
        if not isinstance(quantities, str) or not quantities:
            raise ValueError("quantities must be a non-empty string")
        if set(quantities) - _VALID_QUANTITIES:
            raise ValueError(f"unsupported quantities: {quantities!r}")
        cutoff, skin = float(cutoff), float(skin)
        if not isfinite(cutoff) or cutoff <= 0:
            raise ValueError("cutoff must be finite and positive")
        if not isfinite(skin) or skin <= 0 or not isfinite(cutoff + skin):
            raise ValueError("skin must be finite and positive")
        if algorithm not in ALGORITHMS:
            raise ValueError("algorithm must be 'auto', 'brute_force', or 'cell_list'")
        if not all(isinstance(o, bool) for o in (sorted, half_list, include_self)):
            raise TypeError("sorted, half_list, and include_self must be bool")
        if mode not in ("auto", "filter", "search"):
            raise ValueError("mode must be 'auto', 'filter', or 'search'")
        self.quantities = quantities
        self.cutoff, self.skin = cutoff, skin
        self.algorithm, self.sorted = algorithm, sorted
        self.half_list, self.include_self = half_list, include_self
        self.mode = mode
        self.builds = 0
        self.calls = 0
        # mode "auto": the faster path per request shape, once timed
        self.choice: dict = {}
        self._stored: _Stored | None = None
        self._capacity: int | None = None
        self._host = None
        self._err = ctypes.create_string_buffer(512)

    def reset(self) -> None:
        """Drop the stored list: the next call rebuilds."""
        self._stored = None
        self._capacity = None

    def __call__(self, positions: Tensor, cell: Tensor, pbc: Tensor,
                 batch_ptr: Tensor | None = None) -> tuple[Tensor, ...]:
        _require_torch_tensors(cell=cell, pbc=pbc, batch_ptr=batch_ptr)
        positions, cell, pbc, batch_ptr = normalize_torch_inputs(positions, cell, pbc, batch_ptr)
        validate_torch_inputs(positions, cell, pbc, self.cutoff, batch_ptr)
        if not positions.is_cuda:
            raise RuntimeError("VerletList runs on ROCm (HIP) devices; move the tensors to a GPU")
        device = positions.device
        try:
            lib = load_torch_hip()
            check_device(device.index if device.index is not None else torch.cuda.current_device())
        except ImportError as error:
            raise RuntimeError(f"the CUDA provider is unavailable: {error}") from error
        self.calls += 1
        grad_positions, grad_cell = positions, cell
        pos = positions.detach().contiguous()
        cel = cell.detach().contiguous()
        pbc, batch_ptr = pbc.contiguous(), batch_ptr.contiguous()
        key = (device, pos.dtype, pos.shape[0], batch_ptr.numel() - 1)
        switch = device.index is not None and device.index != torch.cuda.current_device()
        with torch.cuda.device(device) if switch else contextlib.nullcontext():
            path = self.mode if self.mode != "auto" else self.choice.get(key)
            if path == "search":
                return self._search(pos, cel, pbc, batch_ptr, grad_positions, grad_cell)
            fresh = self._stored is None or self._stored.key != key
            if fresh:
                self._build(lib, key, pos, cel, pbc, batch_ptr)
            timing = self.mode == "auto" and path is None and not fresh
            if timing:
                torch.cuda.synchronize(device)
                t0 = time.perf_counter()
            out = self._filter(lib, pos, cel, pbc, batch_ptr, grad_positions, grad_cell)
            if timing and out is not None:
                torch.cuda.synchronize(device)
                t_filter = time.perf_counter() - t0
                self.choice[key] = (
                    "search" if self._time_search(device, pos, cel, pbc, batch_ptr) < t_filter
                    else "filter"
                )
            if out is None and not fresh:
                self._build(lib, key, pos, cel, pbc, batch_ptr)
                out = self._filter(lib, pos, cel, pbc, batch_ptr, grad_positions, grad_cell)
            if out is None:
                # a skin below the rounding margin of these inputs: search directly
                out = self._search(pos, cel, pbc, batch_ptr, grad_positions, grad_cell)
        return out

    def _search(self, pos: Tensor, cell: Tensor, pbc: Tensor, batch_ptr: Tensor,
                grad_positions, grad_cell) -> tuple[Tensor, ...]:
        """A fresh search of these inputs at the cutoff."""
        return neighbor_list_hip(
            self.quantities, pos, batch_ptr, cell, pbc, self.cutoff,
            half_list=self.half_list, include_self=self.include_self,
            algorithm=self.algorithm, sorted=self.sorted,
            grad_positions=grad_positions, grad_cell=grad_cell,
        )

    def _time_search(self, device, pos: Tensor, cell: Tensor, pbc: Tensor,
                     batch_ptr: Tensor) -> float:
        """Wall time of a warm fresh search of these inputs (after one that
        warms up the search's plan for this shape); its outputs are dropped."""
        with torch.no_grad():
            self._search(pos, cell, pbc, batch_ptr, pos, cell)
            torch.cuda.synchronize(device)
            t0 = time.perf_counter()
            self._search(pos, cell, pbc, batch_ptr, pos, cell)
            torch.cuda.synchronize(device)
        return time.perf_counter() - t0

    def _build(self, lib, key, pos: Tensor, cell: Tensor, pbc: Tensor, batch_ptr: Tensor) -> None:
        build_cutoff = self.cutoff + self.skin
        pairs, shifts = neighbor_list_hip(
            "PS", pos, batch_ptr, cell, pbc, build_cutoff, half_list=self.half_list,
            include_self=self.include_self, algorithm=self.algorithm, sorted=self.sorted,
        )
        pairs, shifts = pairs.contiguous(), shifts.contiguous()
        req = self._request(pos, cell, pbc, batch_ptr)
        n = pairs.shape[0]
        ws_bytes = int(lib.tnr_skin_workspace_size(ctypes.byref(req), n))
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=pos.device)
        lst = SkinList()
        stream = torch.cuda.current_stream(pos.device).cuda_stream
        code = lib.tnr_skin_store(
            ctypes.byref(req), build_cutoff, pairs.data_ptr() if n else None,
            shifts.data_ptr() if n else None, n, workspace.data_ptr(), ws_bytes,
            ctypes.byref(lst), stream, self._err, len(self._err),
        )
        if code != TNR_OK:
            _raise(code, self._err.value.decode())
        # the store runs on the stream: P and S may be released once it is
        # enqueued (later work on the stream reuses their memory after it)
        self._stored = _Stored(key, workspace, ws_bytes, lst)
        self._capacity = None
        self.builds += 1

    def _request(self, pos: Tensor, cell: Tensor, pbc: Tensor, batch_ptr: Tensor) -> Request:
        return Request(
            dtype=0 if pos.dtype == torch.float32 else 1,
            algorithm=ALGORITHMS[self.algorithm],
            n_atoms=pos.shape[0],
            n_structures=batch_ptr.numel() - 1,
            positions=pos.data_ptr() if pos.numel() else None,
            batch_ptr=batch_ptr.data_ptr(),
            cell=cell.data_ptr(),
            pbc=pbc.data_ptr(),
            cutoff=self.cutoff,
            half_list=int(self.half_list),
            include_self=int(self.include_self),
            sorted=int(self.sorted),
            stencil_reach=0,
        )

    def _host_buffer(self):
        if self._host is None:
            host = torch.zeros(HOST_RESULT_SLOTS, dtype=torch.int64, pin_memory=True)
            self._host = (host, torch.cuda.Event())
        return self._host

    def _run(self, lib, req: Request, out: dict, rows: int, stream: int, host) -> None:
        s = self._stored
        ptrs = Outputs(
            n_pairs=rows, plan=0, n_tasks=0,
            pairs=out["P"].data_ptr() if "P" in out else None,
            shifts=out["S"].data_ptr() if "S" in out else None,
            distances=out["d"].data_ptr() if "d" in out else None,
            vectors=out["D"].data_ptr() if "D" in out else None,
            sources=out["i"].data_ptr() if "i" in out else None,
            targets=out["j"].data_ptr() if "j" in out else None,
            edge_index=None,
        )
        code = lib.tnr_skin_filter_async(
            ctypes.byref(req), ctypes.byref(s.list), s.workspace.data_ptr(), s.ws_bytes,
            ctypes.byref(ptrs), host.data_ptr(), stream, self._err, len(self._err),
        )
        if code != TNR_OK:
            _raise(code, self._err.value.decode())

    def _finish(self, lib, req: Request, host) -> int | None:
        n_pairs = ctypes.c_int64(0)
        rebuild = ctypes.c_int32(0)
        code = lib.tnr_skin_finish(ctypes.byref(req), ctypes.byref(self._stored.list),
                                   host.data_ptr(), ctypes.byref(n_pairs), ctypes.byref(rebuild),
                                   self._err, len(self._err))
        if code != TNR_OK:
            _raise(code, self._err.value.decode())
        return None if rebuild.value else int(n_pairs.value)

    def _filter(self, lib, pos: Tensor, cell: Tensor, pbc: Tensor, batch_ptr: Tensor,
                grad_positions: Tensor, grad_cell: Tensor) -> tuple[Tensor, ...] | None:
        """The filtered list, or None when it may differ from a fresh search.

        One pass writes the kept pairs into outputs sized from the previous
        step's count plus a margin (at most the stored count, which always
        suffices); the host waits for the status words only, and filters
        again into outputs of the stored count when E outgrew them.
        """
        stored = self._stored.list.n_pairs
        need_grad = (
            any(q in self.quantities for q in "dD")
            and torch.is_grad_enabled()
            and (grad_positions.requires_grad or grad_cell.requires_grad)
        )
        want = set(self.quantities)
        if need_grad:
            want |= {"P", "S", "D", "d"}
        req = self._request(pos, cell, pbc, batch_ptr)
        torch_stream = torch.cuda.current_stream(pos.device)
        stream = torch_stream.cuda_stream
        host, arrived = self._host_buffer()
        rows = stored if self._capacity is None else min(stored, self._capacity)
        out = _allocate(want, rows, pos.dtype, pos.device)
        self._run(lib, req, out, rows, stream, host)
        arrived.record(torch_stream)
        arrived.synchronize()
        count = self._finish(lib, req, host)
        if count is None:
            return None
        if count > rows:
            rows = stored
            out = _allocate(want, rows, pos.dtype, pos.device)
            self._run(lib, req, out, rows, stream, host)
            arrived.record(torch_stream)
            arrived.synchronize()
            count = self._finish(lib, req, host)
            if count is None:
                return None
        out = _rows(out, count)
        self._capacity = _capacity(count)
        if need_grad:
            out["D"], out["d"] = _FusedGeometry.apply(
                grad_positions, grad_cell, out["P"], out["S"], batch_ptr, out["D"], out["d"]
            )
        return tuple(out[q] for q in self.quantities)
