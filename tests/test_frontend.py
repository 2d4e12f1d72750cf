"""Host-side API contract (no GPU): argument validation, messages and types.

Mirrors tests/test_validation.py:35-241 and tests/test_api.py of the
reference for the checks that run before the device call, and checks that
inputs the MI355X provider cannot serve fail loudly instead of falling back to
a CPU search.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import tonari_amd
from tonari_amd import _extensions as ext
from tonari_amd import neighbor_list


def _args(n=4, dtype=torch.float64):
    return (torch.zeros((n, 3), dtype=dtype), torch.eye(3, dtype=dtype),
            torch.tensor([True, False, False]), 1.0)


def test_public_surface():
    assert tonari_amd.neighbor_list is neighbor_list
    import inspect

    sig = inspect.signature(neighbor_list)
    assert list(sig.parameters) == [
        "quantities", "positions", "cell", "pbc", "cutoff", "batch_ptr", "algorithm",
        "cpu_threads", "sorted", "half_list", "include_self"]
    assert sig.parameters["algorithm"].default == "auto"
    for name in ("sorted", "half_list", "include_self"):
        assert sig.parameters[name].default is False


@pytest.mark.parametrize(
    "kwargs, exc, match",
    [
        ({"quantities": "PX"}, ValueError, "unsupported quantities: 'X'"),
        ({"quantities": 3}, TypeError, "quantities must be a string"),
        ({"algorithm": "fast"}, ValueError, "algorithm must be 'auto', 'brute_force', or 'cell_list'"),
        ({"algorithm": 1}, TypeError, "algorithm must be a string"),
        ({"cpu_threads": 0}, ValueError, "cpu_threads must be positive"),
        ({"cpu_threads": True}, TypeError, "cpu_threads must be an integer or None"),
        ({"sorted": 1}, TypeError, "sorted, half_list, and include_self must be bool"),
        ({"half_list": None}, TypeError, "sorted, half_list, and include_self must be bool"),
    ],
)
def test_scalar_validation(kwargs, exc, match):
    q = kwargs.pop("quantities", "PS")
    with pytest.raises(exc, match=match):
        neighbor_list(q, *_args(), **kwargs)


@pytest.mark.parametrize(
    "mutate, match",
    [
        (lambda a: (a[0][:, :2],) + a[1:], "positions must have shape \\(N_total, 3\\)"),
        (lambda a: (a[0], a[1][:2]) + a[2:], "single-structure cell must have shape \\(3, 3\\)"),
        (lambda a: a[:2] + (a[2][:2],) + a[3:], "single-structure pbc must have shape \\(3,\\)"),
        (lambda a: (a[0].int(),) + a[1:], "positions must have dtype float32 or float64"),
        (lambda a: (a[0], a[1].float()) + a[2:], "cell and positions must have the same dtype"),
        (lambda a: a[:3] + (float("nan"),), "cutoff must be finite and positive"),
        (lambda a: a[:3] + (-1.0,), "cutoff must be finite and positive"),
    ],
)
def test_tensor_validation(mutate, match):
    with pytest.raises(ValueError, match=match):
        neighbor_list("PS", *mutate(_args()))


def test_batched_validation():
    pos = torch.zeros((4, 3), dtype=torch.float64)
    cell = torch.zeros((2, 3, 3), dtype=torch.float64)
    pbc = torch.zeros((2, 3), dtype=torch.bool)
    bp = torch.tensor([0, 2, 4])
    with pytest.raises(ValueError, match="batch_ptr must be int64"):
        neighbor_list("PS", pos, cell, pbc, 1.0, bp.int())
    with pytest.raises(ValueError, match="cell must have shape \\(B, 3, 3\\)"):
        neighbor_list("PS", pos, cell[:1], pbc, 1.0, bp)
    with pytest.raises(ValueError, match="pbc must be bool with shape \\(B, 3\\)"):
        neighbor_list("PS", pos, cell, pbc.int(), 1.0, bp)
    with pytest.raises(ValueError, match="batched cell must have shape"):
        neighbor_list("PS", pos, cell[0], pbc, 1.0, bp)
    with pytest.raises(TypeError, match="must all be PyTorch tensors"):
        neighbor_list("PS", pos, cell.numpy(), pbc, 1.0, bp)


def test_cpu_tensors_and_numpy_arrays_take_the_host_provider():
    # CPU tensors and NumPy arrays go to libtonari_cpu.so (tests/test_cpu_provider.py)
    P, S = neighbor_list("PS", np.zeros((2, 3)), np.eye(3), np.array([1, 0, 0], bool), 1.0)
    assert isinstance(P, np.ndarray) and P.shape == (2, 2)
    P, S = neighbor_list("PS", *_args())
    assert isinstance(P, torch.Tensor) and P.device.type == "cpu"


def test_missing_cpu_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(ext, "load_cpu", lambda: ext.open_cpu_library(str(tmp_path / "x.so")))
    import tonari_amd._cpu_provider as provider

    monkeypatch.setattr(provider, "load_cpu", ext.load_cpu)
    with pytest.raises(RuntimeError, match="NumPy CPU extension is not built"):
        neighbor_list("PS", np.zeros((2, 3)), np.eye(3), np.array([1, 0, 0], bool), 1.0)
    with pytest.raises(RuntimeError, match="Torch CPU provider is unavailable"):
        neighbor_list("PS", *_args())


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(ext, "LIBRARY", str(tmp_path / "missing.so"))
    with pytest.raises(ImportError, match="was not built"):
        ext.open_library(ext.LIBRARY)


def test_workloads_are_deterministic():
    from tonari_amd import workloads as W

    a, b = W.c2(n_structures=8), W.c2(n_structures=8)
    assert np.array_equal(a["positions"], b["positions"])
    assert np.array_equal(a["batch_ptr"], b["batch_ptr"])
    c4 = W.c4(n_atoms=1000)
    assert c4["positions"].dtype == np.float32 and c4["positions"].shape == (1000, 3)
    assert W.algorithmic_bytes(100_000, 9_046_552, "PD", 4) == 100_000 * 12 + 9_046_552 * 28


def test_numpy_frontend_does_not_import_torch():
    # tests/packaging/test_import_boundaries.py:21-44: a NumPy caller works in
    # a process where importing torch fails
    import subprocess
    import sys
    import textwrap

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = textwrap.dedent("""
        import importlib.abc
        import sys

        class BlockTorch(importlib.abc.MetaPathFinder):
            def find_spec(self, fullname, path, target=None):
                if fullname == "torch" or fullname.startswith("torch."):
                    raise ModuleNotFoundError("Torch import deliberately blocked")
                return None

        sys.meta_path.insert(0, BlockTorch())
        sys.path.insert(0, %r)
        import numpy as np
        from tonari_amd import neighbor_list

        positions = np.array([[0.0, 0.0, 0.0], [0.8, 0.0, 0.0]])
        cell = np.eye(3) * 4.0
        pbc = np.zeros(3, dtype=np.bool_)
        pair_indices, cell_shifts = neighbor_list("PS", positions, cell, pbc, 1.0)
        assert pair_indices.shape == (2, 2)
        assert cell_shifts.shape == (2, 3)
        assert "torch" not in sys.modules
    """) % root
    subprocess.run([sys.executable, "-c", code], check=True, timeout=120)
