"""Graph adapter: neighbor lists in the edge-first layout of graph libraries.

The reference keeps its core API edge-last (P is (E, 2), row-aligned with S,
d and D) and leaves the (2, E) graph layout to adapters, which transpose P
into ``edge_index`` and map D to edge vectors at the boundary
(``docs/design.md:61,127``; ``README.md:81-99`` shows
``edge_index = P.T.contiguous()`` for a PyTorch Geometric batch).  This adapter
gives that result without the transpose: the emitting kernels write sources
and targets straight into the two rows of one (2, E) buffer, with E read on
the device (``tnr_outputs::edge_index``).  ``neighbor_list`` itself is
unchanged.
"""

from __future__ import annotations

from typing import NamedTuple

import torch
from torch import Tensor

from ._torch_frontend import (
    EDGE_INDEX,
    _require_torch_tensors,
    neighbor_list_hip,
    normalize_torch_inputs,
    validate_torch_inputs,
)


class Graph(NamedTuple):
    """Edges of a neighbor list; every tensor is row-aligned with edge_index's columns."""

    edge_index: Tensor             # (2, E) int64: row 0 sources i, row 1 targets j
    edge_vectors: Tensor | None    # (E, 3): positions[j] - positions[i] + S @ cell[b] (D)
    edge_lengths: Tensor | None    # (E,): |edge_vectors| (d)
    cell_shifts: Tensor | None     # (E, 3) int32: integer shift of the target image (S)


def neighbor_graph(
    positions: Tensor,
    cell: Tensor,
    pbc: Tensor,
    cutoff: float,
    batch_ptr: Tensor | None = None,
    *,
    vectors: bool = True,
    lengths: bool = False,
    shifts: bool = False,
    algorithm: str = "auto",
    sorted: bool = False,
    half_list: bool = False,
    include_self: bool = False,
) -> Graph:
    """``neighbor_list`` as a graph: ``edge_index`` (2, E) plus the requested edge data.

    The same search, pair set, arguments, validation and errors as
    ``neighbor_list(...)`` on ROCm tensors; ``edge_index`` equals
    ``P.T.contiguous()`` of that call, and ``edge_vectors`` / ``edge_lengths`` /
    ``cell_shifts`` are its D / d / S (differentiable in positions and cell
    like D and d).  Quantities not requested are None.
    """
    if algorithm not in ("auto", "brute_force", "cell_list"):
        raise ValueError("algorithm must be 'auto', 'brute_force', or 'cell_list'")
    if not all(isinstance(x, bool) for x in (vectors, lengths, shifts, sorted, half_list,
                                                include_self)):
        raise TypeError("vectors, lengths, shifts, sorted, half_list, and include_self must be bool")
    if not isinstance(positions, Tensor):
        raise TypeError("positions must be a PyTorch tensor")
    _require_torch_tensors(cell=cell, pbc=pbc, batch_ptr=batch_ptr)
    positions, cell, pbc, batch_ptr = normalize_torch_inputs(positions, cell, pbc, batch_ptr)
    cutoff = float(cutoff)
    validate_torch_inputs(positions, cell, pbc, cutoff, batch_ptr)
    if not positions.is_cuda:
        raise RuntimeError("neighbor_graph runs on ROCm (HIP) devices; move the tensors to a GPU")
    quantities = EDGE_INDEX + ("D" if vectors else "") + ("d" if lengths else "") + (
        "S" if shifts else "")
    out = dict(zip(quantities, neighbor_list_hip(
        quantities,
        positions.detach().contiguous(),
        batch_ptr.contiguous(),
        cell.detach().contiguous(),
        pbc.contiguous(),
        cutoff,
        half_list=half_list,
        include_self=include_self,
        algorithm=algorithm,
        sorted=sorted,
        grad_positions=positions,
        grad_cell=cell,
    )))
    return Graph(out[EDGE_INDEX], out.get("D"), out.get("d"), out.get("S"))


def from_batch(batch, cutoff: float, **options) -> Graph:
    """``neighbor_graph`` of a PyTorch Geometric style batch (``pos``, ``cell``, ``pbc``, ``ptr``)."""
    return neighbor_graph(batch.pos, batch.cell, batch.pbc, cutoff, batch.ptr, **options)


__all__ = ["Graph", "from_batch", "neighbor_graph"]
