"""Public ``neighbor_list`` entry point.

Same signature, defaults, scalar validation and messages as the reference
(``src/tonari/api.py:18-234``).  PyTorch tensors on a ROCm (HIP) device go to
the MI355X provider; PyTorch CPU tensors and NumPy arrays go to this build's
host provider (``include/tonari_cpu.h``) on ``cpu_threads`` threads.
"""

from __future__ import annotations

import builtins
from typing import TYPE_CHECKING, Literal

if TYPE_CHECKING:
    from torch import Tensor

_VALID_QUANTITIES = frozenset("ijPSdD")
_Algorithm = Literal["auto", "brute_force", "cell_list"]
_VALID_ALGORITHMS = frozenset(("auto", "brute_force", "cell_list"))


def neighbor_list(
    quantities: str,
    positions: Tensor,
    cell: Tensor,
    pbc: Tensor,
    cutoff: float,
    batch_ptr: Tensor | None = None,
    *,
    algorithm: _Algorithm = "auto",
    cpu_threads: int | None = None,
    sorted: bool = False,
    half_list: bool = False,
    include_self: bool = False,
) -> tuple[Tensor, ...]:
    """Build an atomistic neighbor list within a strict distance cutoff.

    ``quantities`` selects the returned arrays in order: ``i`` source and
    ``j`` target indices (int64, (E,)), ``P`` pairs (int64, (E, 2)), ``S``
    integer cell shifts of the target image (int32, (E, 3)), ``d`` distances
    and ``D`` displacement vectors ``positions[j] - positions[i] + S @ cell[b]``
    in the input dtype.  ``positions`` (N_total, 3) float32/float64, ``cell``
    (3, 3) or (B, 3, 3) with rows as cell vectors, ``pbc`` (3,) or (B, 3) bool,
    ``batch_ptr`` optional int64 (B + 1,) structure boundaries.  Pairs have
    squared distance strictly below ``cutoff**2``; ``half_list`` keeps the
    lexicographically smaller of (i, j, S) and (j, i, -S); ``include_self``
    adds the zero-shift self pair of every atom.  The pairs of a source are
    always contiguous.  With ``sorted=True`` sources come in increasing index
    order.  Without it, on the device, sources come in cell-list bin order
    when every structure of the call is searched with a cell list, and in
    index order otherwise; on the CPU they always come in index order.  The
    order of targets within a source is unspecified.
    """
    if not isinstance(quantities, str):
        raise TypeError("quantities must be a string")
    invalid_quantities = set(quantities) - _VALID_QUANTITIES
    if invalid_quantities:
        invalid = "".join(builtins.sorted(invalid_quantities))
        raise ValueError(f"unsupported quantities: {invalid!r}")
    if not isinstance(algorithm, str):
        raise TypeError("algorithm must be a string")
    if algorithm not in _VALID_ALGORITHMS:
        raise ValueError("algorithm must be 'auto', 'brute_force', or 'cell_list'")
    if cpu_threads is not None:
        if isinstance(cpu_threads, bool) or not isinstance(cpu_threads, int):
            raise TypeError("cpu_threads must be an integer or None")
        if cpu_threads < 1:
            raise ValueError("cpu_threads must be positive")
        if cpu_threads > (1 << 63) - 1:
            raise ValueError("cpu_threads is too large")
    if not all(isinstance(option, bool) for option in (sorted, half_list, include_self)):
        raise TypeError("sorted, half_list, and include_self must be bool")
    try:
        import numpy as np
    except ImportError:  # pragma: no cover - numpy ships with torch
        np = None
    if np is not None and isinstance(positions, np.ndarray):
        from ._numpy_frontend import neighbor_list_numpy

        return neighbor_list_numpy(
            quantities,
            positions,
            cell,
            pbc,
            cutoff,
            batch_ptr,
            algorithm=algorithm,
            cpu_threads=cpu_threads,
            sorted=sorted,
            half_list=half_list,
            include_self=include_self,
        )
    try:
        import torch
    except ImportError:
        pass
    else:
        if isinstance(positions, torch.Tensor):
            from ._torch_frontend import neighbor_list_torch

            return neighbor_list_torch(
                quantities,
                positions,
                cell,
                pbc,
                cutoff,
                batch_ptr,
                algorithm=algorithm,
                cpu_threads=cpu_threads,
                sorted=sorted,
                half_list=half_list,
                include_self=include_self,
            )
    raise TypeError("positions must be a PyTorch tensor or NumPy array")
