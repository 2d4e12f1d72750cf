"""Calls into the host provider (libtonari_cpu.so, include/tonari_cpu.h).

The CPU counterpart of the reference's pybind11 CPU providers
(``csrc/torch/bindings_cpu.cpp:73-122``, ``csrc/numpy/bindings.cpp``): the
search runs in this build's C++ (``tonari_amd/csrc/cpu/nl_cpu.cpp``) on
``threads`` host threads and returns the pairs P (E, 2) int64 and their
shifts S (E, 3) int32, grouped by structure and by source in index order.
The array ecosystem (NumPy or Torch) allocates the outputs.
"""

from __future__ import annotations

import ctypes
from typing import Callable

from ._extensions import ALGORITHMS, TNR_INPUT_ERROR, TNR_OK, load_cpu


def search(
    float64: bool,
    positions: int,
    n_atoms: int,
    batch_ptr: int,
    n_structures: int,
    cell: int,
    pbc: int,
    cutoff: float,
    half_list: bool,
    include_self: bool,
    algorithm: str,
    threads: int,
    allocate: Callable[[int], tuple[object, object, int, int]],
) -> tuple[object, object]:
    """Search on the CPU over contiguous host buffers given by address.

    ``allocate(E)`` returns the P and S arrays of E rows and their
    addresses.  Raises the reference's exception types and messages.
    """
    lib = load_cpu()
    handle = ctypes.c_void_p()
    count = ctypes.c_int64(0)
    err = ctypes.create_string_buffer(512)
    code = lib.tnr_cpu_search(
        1 if float64 else 0, positions, n_atoms, batch_ptr, n_structures, cell, pbc,
        float(cutoff), int(half_list), int(include_self), ALGORITHMS[algorithm], int(threads),
        ctypes.byref(handle), ctypes.byref(count), err, len(err),
    )
    if code != TNR_OK:
        message = err.value.decode()
        raise (ValueError if code == TNR_INPUT_ERROR else RuntimeError)(message)
    try:
        pairs, shifts, pairs_ptr, shifts_ptr = allocate(int(count.value))
        if count.value:
            lib.tnr_cpu_copy(handle, pairs_ptr, shifts_ptr, int(threads))
    finally:
        lib.tnr_cpu_free(handle)
    return pairs, shifts
