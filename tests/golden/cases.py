"""Inputs of the golden fixtures: seeded generators plus call options.

Each case is ``name -> (make_inputs, options)``.  The reference-suite cases
rebuild the seeded inputs of the reference's tests with the same
``torch.Generator`` seeds (file:line in songfeitong/tonari given per case).
"""

from __future__ import annotations

import numpy as np

from tonari_amd import workloads as W


def _single(positions, cell, pbc, cutoff):
    positions = np.ascontiguousarray(positions)
    return {
        "positions": positions,
        "cell": np.ascontiguousarray(np.asarray(cell, dtype=positions.dtype)[None]),
        "pbc": np.asarray(pbc, dtype=bool)[None],
        "batch_ptr": np.array([0, len(positions)], dtype=np.int64),
        "cutoff": float(cutoff),
    }


def _torch_rand(seed, shape, dtype="float64"):
    import torch

    g = torch.Generator().manual_seed(seed)
    return torch.rand(shape, generator=g, dtype=getattr(torch, dtype)).numpy()


def periodic_batch_1945():
    """tests/backends/test_algorithms.py:11-33 (seed 1945, 32 + 288 atoms, pbc TFF)."""
    import torch

    g = torch.Generator().manual_seed(1945)
    counts = (32, 288)
    cell = torch.tensor(
        [[[5.0, 0.0, 0.0], [0.0, 5.5, 0.0], [0.0, 0.0, 6.0]],
         [[8.0, 0.0, 0.0], [0.0, 7.5, 0.0], [0.0, 0.0, 9.0]]], dtype=torch.float64)
    pos = torch.cat([(0.1 + 0.8 * torch.rand((c, 3), generator=g, dtype=torch.float64)) @ cell[i]
                     for i, c in enumerate(counts)])
    return {"positions": pos.numpy(), "cell": cell.numpy(),
            "pbc": np.array([[True, False, False], [True, False, False]]),
            "batch_ptr": np.array([0, 32, 320], dtype=np.int64), "cutoff": 1.2}


def forced_cell_1842(dtype="float64"):
    """tests/backends/test_pair_identity.py:268-289 (seed 1842, 288 atoms, triclinic)."""
    import torch

    g = torch.Generator().manual_seed(1842)
    cell = torch.tensor([[8.0, 0.4, 0.1], [0.2, 7.5, 0.5], [0.3, 0.1, 9.0]],
                        dtype=getattr(torch, dtype))
    pos = torch.rand((288, 3), generator=g, dtype=getattr(torch, dtype)) @ cell
    return _single(pos.numpy(), cell.numpy(), [True] * 3, 1.2)


def unwrapped_1842(dtype="float64"):
    """tests/backends/test_cuda_runtime.py:246-261 (seed 1842, 5 unwrapped atoms)."""
    import torch

    g = torch.Generator().manual_seed(1842)
    cell = torch.tensor([[8.0, 0.4, 0.1], [0.2, 7.5, 0.5], [0.3, 0.1, 9.0]],
                        dtype=getattr(torch, dtype))
    pos = torch.rand((288, 3), generator=g, dtype=getattr(torch, dtype)) @ cell
    pos[:5] += 3 * cell[0] - 2 * cell[1]
    return _single(pos.numpy(), cell.numpy(), [True] * 3, 1.2)


def mixed_5801():
    """tests/backends/test_cuda_runtime.py:264-303 (seed 5801, finite + partial pbc)."""
    import torch

    g = torch.Generator().manual_seed(5801)
    counts = (256, 257)
    cell = torch.tensor([[[0.0] * 3] * 3, [[2.1, 0.3, 0.2], [0.4, 4.0, 0.1], [0.2, 0.5, 5.0]]],
                        dtype=torch.float64)
    pos = torch.cat((torch.rand((counts[0], 3), generator=g, dtype=torch.float64) * 8,
                     torch.rand((counts[1], 3), generator=g, dtype=torch.float64) @ cell[1]))
    pos[-3:] += 4 * cell[1, 0]
    return {"positions": pos.numpy(), "cell": cell.numpy(),
            "pbc": np.array([[False] * 3, [True, False, False]]),
            "batch_ptr": np.array([0, 256, 513], dtype=np.int64), "cutoff": 0.55}


def fallback_9041():
    """tests/test_pair_options.py:362-394 (seed 9041, 256 atoms, one unwrapped)."""
    import torch

    g = torch.Generator().manual_seed(9041)
    cell = torch.tensor([[8.0, 0.2, 0.1], [0.1, 8.5, 0.3], [0.2, 0.1, 9.0]], dtype=torch.float64)
    pos = torch.rand((256, 3), generator=g, dtype=torch.float64) @ cell
    pos[0] += 2 * cell[0] - 3 * cell[2]
    return _single(pos.numpy(), cell.numpy(), [True] * 3, 0.8)


def common_translation_9184():
    """tests/backends/test_algorithms.py:110-128 (seed 9184, 1e8-cell translation)."""
    import torch

    g = torch.Generator().manual_seed(9184)
    cell = torch.tensor([[4.1, 0.3, 0.2], [0.4, 4.7, 0.1], [0.2, 0.5, 5.3]], dtype=torch.float64)
    pos = torch.rand((129, 3), generator=g, dtype=torch.float64) @ cell
    pos += torch.tensor([100000000, -80000000, 60000000], dtype=torch.float64) @ cell
    return _single(pos.numpy(), cell.numpy(), [True] * 3, 1.0)


def float32_grid_1841(n):
    """tests/test_pair_options.py:317-359 (seed 1841 + n, finite float32 box)."""
    import torch

    g = torch.Generator().manual_seed(1841 + n)
    pos = torch.rand((n, 3), generator=g, dtype=torch.float32) * 8
    return _single(pos.numpy(), np.zeros((3, 3), np.float32), [False] * 3, 1.1)


def mixed_boundary_712(dtype="float64"):
    """tests/backends/test_pair_identity.py:13-47 (seed 712, 3 structures)."""
    import torch

    td = getattr(torch, dtype)
    g = torch.Generator().manual_seed(712)
    partial = torch.tensor([[2.1, 0.2, 0.1], [0.0, 2.5, 0.3], [0.0, 0.0, 0.0]], dtype=td)
    periodic = torch.tensor([[1.7, 0.2, 0.0], [0.1, 1.9, 0.3], [0.2, 0.1, 2.2]], dtype=td)
    pos = torch.cat((
        torch.rand((7, 3), generator=g, dtype=td) * 4.0,
        torch.rand((5, 3), generator=g, dtype=td)
        @ torch.tensor([[2.1, 0.2, 0.1], [0.0, 2.5, 0.3], [0.0, 0.0, 8.0]], dtype=td),
        torch.rand((4, 3), generator=g, dtype=td) @ periodic))
    cell = torch.stack((torch.zeros((3, 3), dtype=td), partial, periodic))
    return {"positions": pos.numpy(), "cell": cell.numpy(),
            "pbc": np.array([[False] * 3, [True, True, False], [True] * 3]),
            "batch_ptr": np.array([0, 7, 12, 16], dtype=np.int64), "cutoff": 1.35}


def triclinic_ase():
    """tests/test_pair_options.py:106-116 (3 atoms, partial triclinic, rc 2.4)."""
    return _single(np.array([[0.1, 0.2, 0.3], [0.9, 0.4, 0.8], [1.6, 1.0, 0.5]]),
                   [[1.7, 0.0, 0.0], [0.45, 1.6, 0.0], [0.0, 0.0, 0.0]], [True, True, False], 2.4)


CASES = {
    "C1_brute": (W.c1, {"algorithm": "brute_force"}),
    "C1_cell": (W.c1, {"algorithm": "cell_list"}),
    "C2_64": (lambda: W.c2(n_structures=64), {"algorithm": "brute_force"}),
    "C2": (W.c2, {"algorithm": "brute_force"}),
    "C3_128": (lambda: W.c3(n_structures=128), {"half_list": True}),
    "C3": (W.c3, {"half_list": True}),
    "C4_20k": (lambda: W.c4(n_atoms=20000), {"algorithm": "cell_list"}),
    "C4": (W.c4, {"algorithm": "cell_list"}),
    "C5_3": (lambda: W.c5(n_structures=3, n_min=1000, n_max=3000), {"include_self": True}),
    "C5": (W.c5, {"include_self": True}),
    "ref_periodic_batch_1945_half_self": (periodic_batch_1945,
                                          {"half_list": True, "include_self": True}),
    "ref_forced_cell_1842_f64": (forced_cell_1842, {"algorithm": "cell_list"}),
    "ref_forced_cell_1842_f32": (lambda: forced_cell_1842("float32"), {"algorithm": "cell_list"}),
    "ref_unwrapped_1842_f64": (unwrapped_1842, {}),
    "ref_unwrapped_1842_f32": (lambda: unwrapped_1842("float32"), {}),
    "ref_mixed_5801": (mixed_5801, {}),
    "ref_fallback_9041_full": (fallback_9041, {}),
    "ref_fallback_9041_half_self": (fallback_9041, {"half_list": True, "include_self": True}),
    "ref_common_translation_9184": (common_translation_9184, {"algorithm": "cell_list"}),
    "ref_float32_12_brute": (lambda: float32_grid_1841(12), {"algorithm": "brute_force"}),
    "ref_float32_256_cell_half": (lambda: float32_grid_1841(256),
                                  {"algorithm": "cell_list", "half_list": True}),
    "ref_mixed_boundary_712_f32": (lambda: mixed_boundary_712("float32"), {}),
    "ref_mixed_boundary_712_f64": (mixed_boundary_712, {}),
    "ref_triclinic_ase_full": (triclinic_ase, {}),
    "ref_triclinic_ase_half_self": (triclinic_ase, {"half_list": True, "include_self": True}),
}
