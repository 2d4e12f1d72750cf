"""NumPy frontend of ``neighbor_list``: NumPy arrays searched on the CPU.

Restates the reference's NumPy frontend (``src/tonari/_numpy_frontend.py``):
the same type check (``:10-20``), single-structure normalisation
(``:23-46``), validation and messages (``:49-67``), and quantity assembly
(``:70-98``: i and j from P, D = x[j] - x[i] + S @ cell[b] and d = |D| in
NumPy).  The search is this build's host provider (``_cpu_provider``,
``include/tonari_cpu.h``) instead of the reference's pybind11 module
(``:119-130``).  Pairs come grouped by source in index order, as the
reference's CPU path returns them.
"""

from __future__ import annotations

from math import isfinite

import numpy as np

from . import _cpu_provider


def _require_numpy_arrays(*, cell: object, pbc: object, batch_ptr: object | None) -> None:
    for name, value in (("cell", cell), ("pbc", pbc), ("batch_ptr", batch_ptr)):
        if value is None or isinstance(value, np.ndarray):
            continue
        raise TypeError(
            "positions, cell, pbc, and batch_ptr must all be NumPy arrays; "
            f"{name} has type {type(value).__name__}"
        )


def _normalize_numpy_inputs(
    positions: np.ndarray, cell: np.ndarray, pbc: np.ndarray, batch_ptr: np.ndarray | None
) -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    if positions.ndim != 2 or positions.shape[1] != 3:
        raise ValueError("positions must have shape (N_total, 3)")
    if batch_ptr is not None:
        if cell.ndim != 3:
            raise ValueError("batched cell must have shape (B, 3, 3)")
        if pbc.ndim != 2:
            raise ValueError("batched pbc must have shape (B, 3)")
        return positions, cell, pbc, batch_ptr
    # one structure: [0, N] and a leading batch axis
    if cell.ndim != 2 or cell.shape != (3, 3):
        raise ValueError("single-structure cell must have shape (3, 3)")
    if pbc.ndim != 1 or pbc.shape != (3,):
        raise ValueError("single-structure pbc must have shape (3,)")
    return positions, cell[None], pbc[None], np.array([0, len(positions)], dtype=np.int64)


def _validate_numpy_inputs(
    positions: np.ndarray, cell: np.ndarray, pbc: np.ndarray, cutoff: float,
    batch_ptr: np.ndarray,
) -> None:
    n_structures = batch_ptr.size - 1
    checks = (
        (positions.dtype in (np.dtype(np.float32), np.dtype(np.float64)),
         "positions must have dtype float32 or float64"),
        (batch_ptr.ndim == 1 and batch_ptr.size > 0 and batch_ptr.dtype == np.int64,
         "batch_ptr must be int64 with shape (B + 1,)"),
        (cell.shape == (n_structures, 3, 3), "cell must have shape (B, 3, 3)"),
        (cell.dtype == positions.dtype, "cell and positions must have the same dtype"),
        (pbc.shape == (n_structures, 3) and pbc.dtype == np.bool_,
         "pbc must be bool with shape (B, 3)"),
        (isfinite(cutoff) and cutoff > 0, "cutoff must be finite and positive"),
    )
    for ok, message in checks:
        if not ok:
            raise ValueError(message)


def _select_numpy_quantities(
    quantities: str, positions: np.ndarray, cell: np.ndarray, batch_ptr: np.ndarray,
    pairs: np.ndarray, shifts: np.ndarray,
) -> tuple[np.ndarray, ...]:
    source, target = pairs[:, 0], pairs[:, 1]
    out: dict[str, np.ndarray] = {"P": pairs, "S": shifts}
    if "i" in quantities:
        out["i"] = np.ascontiguousarray(source)
    if "j" in quantities:
        out["j"] = np.ascontiguousarray(target)
    if "D" in quantities or "d" in quantities:
        structure = np.searchsorted(batch_ptr[1:], source, side="right")
        translation = np.einsum(
            "ei,eij->ej", shifts.astype(positions.dtype, copy=False), cell[structure]
        )
        out["D"] = positions[target] - positions[source] + translation
        if "d" in quantities:
            out["d"] = np.linalg.norm(out["D"], axis=1)
    return tuple(out[q] for q in quantities)


def neighbor_list_numpy(
    quantities: str,
    positions: np.ndarray,
    cell: np.ndarray,
    pbc: np.ndarray,
    cutoff: float,
    batch_ptr: np.ndarray | None,
    *,
    algorithm: str,
    cpu_threads: int | None,
    sorted: bool,
    half_list: bool,
    include_self: bool,
) -> tuple[np.ndarray, ...]:
    """Neighbor list of NumPy arrays on ``cpu_threads`` host threads (1 by default).

    ``sorted`` is accepted and always holds: the CPU path returns sources in
    index order.
    """
    del sorted  # the CPU path always returns sources in index order
    _require_numpy_arrays(cell=cell, pbc=pbc, batch_ptr=batch_ptr)
    positions, cell, pbc, batch_ptr = _normalize_numpy_inputs(positions, cell, pbc, batch_ptr)
    cutoff = float(cutoff)
    _validate_numpy_inputs(positions, cell, pbc, cutoff, batch_ptr)
    positions = np.ascontiguousarray(positions)
    cell = np.ascontiguousarray(cell)
    batch_ptr = np.ascontiguousarray(batch_ptr)
    pbc_u8 = np.ascontiguousarray(pbc, dtype=np.uint8)

    def allocate(n_pairs: int):
        pairs = np.empty((n_pairs, 2), dtype=np.int64)
        shifts = np.empty((n_pairs, 3), dtype=np.int32)
        return pairs, shifts, pairs.ctypes.data, shifts.ctypes.data

    try:
        pairs, shifts = _cpu_provider.search(
            positions.dtype == np.float64, positions.ctypes.data, len(positions),
            batch_ptr.ctypes.data, batch_ptr.size - 1, cell.ctypes.data, pbc_u8.ctypes.data,
            cutoff, half_list, include_self, algorithm, 1 if cpu_threads is None else cpu_threads,
            allocate,
        )
    except ImportError as error:
        raise RuntimeError(f"the NumPy CPU extension is not built; {error}") from error
    return _select_numpy_quantities(quantities, positions, cell, batch_ptr, pairs, shifts)
