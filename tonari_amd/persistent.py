"""Repeated neighbor lists of one shape without allocation or host waits.

The public call allocates its outputs once it knows the pair count E, so it
waits for the count (``_torch_frontend.py``).  An MD loop or a captured
graph calls the same shape over and over and can give a capacity instead:
``NeighborListPlan`` allocates the workspace, outputs of ``capacity`` rows and
the status buffer once, and ``run()`` enqueues the count and the writing
pass on the current stream without waiting (the writing pass reads the plan
and the bin count on the device).  ``run()`` can therefore be captured in a
HIP graph (``torch.cuda.graph``) and replayed on new positions copied into the
same input tensors.  This is the persistent-workspace, graph-capturable path
the reference lists as unsupported (``docs/design.md:125-127``).

After the stream has reached the end of ``run()``, ``n_pairs`` (a device
tensor) holds E and rows ``[:E]`` of the outputs are the pairs of the public
call for the same inputs: the same multiset, in the same source grouping.
Rows beyond E are unspecified; E > capacity means the outputs overflowed and
the extra pairs were dropped (``check()`` raises then).  Gradients are not
carried: use the public call for autograd.
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from ._extensions import (
    ALGORITHMS,
    HOST_RESULT_SLOTS,
    TNR_OK,
    Outputs,
    Request,
    check_device,
    load_torch_hip,
)
from ._torch_frontend import (
    _allocate,
    _raise,
    _require_torch_tensors,
    normalize_torch_inputs,
    validate_torch_inputs,
)
from .api import _VALID_QUANTITIES

__all__ = ["NeighborListPlan"]


class NeighborListPlan:
    """A persistent neighbor list of one request shape (see the module docstring).

    The input tensors are kept: ``run()`` reads whatever they hold when the
    stream reaches it, so new positions are written into ``positions`` in
    place (``plan.positions.copy_(...)``) between calls or graph replays.
    """

    def __init__(self, quantities: str, positions: Tensor, cell: Tensor, pbc: Tensor,
                 cutoff: float, batch_ptr: Tensor | None = None, *, capacity: int,
                 algorithm: str = "auto", sorted: bool = False, half_list: bool = False,
                 include_self: bool = False):
        if not isinstance(quantities, str) or not quantities:
            raise ValueError("quantities must be a non-empty string")
        if set(quantities) - _VALID_QUANTITIES:
            raise ValueError(f"unsupported quantities: {quantities!r}")
        _require_torch_tensors(cell=cell, pbc=pbc, batch_ptr=batch_ptr)
        positions, cell, pbc, batch_ptr = normalize_torch_inputs(positions, cell, pbc, batch_ptr)
        cutoff = float(cutoff)
        validate_torch_inputs(positions, cell, pbc, cutoff, batch_ptr)
        if not positions.is_cuda:
            raise RuntimeError("NeighborListPlan runs on ROCm (HIP) devices")
        if algorithm not in ALGORITHMS:
            raise ValueError("algorithm must be 'auto', 'brute_force', or 'cell_list'")
        if capacity < 1:
            raise ValueError("capacity must be positive")
        for name, t in (("positions", positions), ("cell", cell), ("pbc", pbc),
                        ("batch_ptr", batch_ptr)):
            if not t.is_contiguous():
                raise ValueError(f"{name} must be contiguous: run() reads it in place")
        self.quantities = quantities
        self.positions, self.cell, self.pbc, self.batch_ptr = positions, cell, pbc, batch_ptr
        self.capacity = int(capacity)
        try:
            self._lib = load_torch_hip()
            check_device(positions.device.index if positions.device.index is not None
                         else torch.cuda.current_device())
        except ImportError as error:
            raise RuntimeError(f"the CUDA provider is unavailable: {error}") from error
        self._req = Request(
            dtype=0 if positions.dtype == torch.float32 else 1,
            algorithm=ALGORITHMS[algorithm], n_atoms=positions.shape[0],
            n_structures=batch_ptr.numel() - 1, positions=positions.data_ptr(),
            batch_ptr=batch_ptr.data_ptr(), cell=cell.data_ptr(), pbc=pbc.data_ptr(),
            cutoff=cutoff, half_list=int(half_list), include_self=int(include_self),
            sorted=int(sorted), stencil_reach=0,
        )
        device = positions.device
        self._ws_bytes = int(self._lib.tnr_workspace_size(ctypes.byref(self._req)))
        self._workspace = torch.empty(self._ws_bytes, dtype=torch.uint8, device=device)
        self._host = torch.zeros(HOST_RESULT_SLOTS, dtype=torch.int64, pin_memory=True)
        self._out = _allocate(set(quantities), self.capacity, positions.dtype, device)
        ptr = lambda q: self._out[q].data_ptr() if q in self._out else None  # noqa: E731
        self._outputs = Outputs(
            n_pairs=self.capacity, plan=-1, n_tasks=0, pairs=ptr("P"), shifts=ptr("S"),
            distances=ptr("d"), vectors=ptr("D"), sources=ptr("i"), targets=ptr("j"),
        )
        # the pair count E lives in the workspace's status words (slot 1)
        self.n_pairs = self._workspace[8:16].view(torch.int64)
        self._err = ctypes.create_string_buffer(512)

    @property
    def outputs(self) -> tuple[Tensor, ...]:
        """The output tensors in ``quantities`` order, ``capacity`` rows each."""
        return tuple(self._out[q] for q in self.quantities)

    def run(self) -> tuple[Tensor, ...]:
        """Enqueue the count and the writing pass on the current stream; no host wait."""
        stream = torch.cuda.current_stream(self.positions.device).cuda_stream
        lib, err = self._lib, self._err
        code = lib.tnr_count_async(ctypes.byref(self._req), self._workspace.data_ptr(),
                                   self._ws_bytes, self._host.data_ptr(), stream, err, len(err))
        if code != TNR_OK:
            _raise(code, err.value.decode())
        code = lib.tnr_emit(ctypes.byref(self._req), self._workspace.data_ptr(), self._ws_bytes,
                            ctypes.byref(self._outputs), stream, err, len(err))
        if code != TNR_OK:
            _raise(code, err.value.decode())
        return self.outputs

    def check(self) -> int:
        """Wait for the stream, raise the reference's error or an overflow, return E."""
        torch.cuda.current_stream(self.positions.device).synchronize()
        n = ctypes.c_int64(0)
        code = self._lib.tnr_count_finish(self._host.data_ptr(), ctypes.byref(n), self._err,
                                          len(self._err))
        if code != TNR_OK:
            _raise(code, self._err.value.decode())
        if n.value > self.capacity:
            raise RuntimeError(
                f"neighbor list of {n.value} pairs exceeds the plan's capacity of "
                f"{self.capacity} rows"
            )
        return int(n.value)
