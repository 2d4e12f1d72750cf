"""Loader for the HIP provider ``libtonari_hip.so`` (C ABI, ctypes).

Replaces the reference's provider loader (``src/tonari/_extensions.py:26-66``):
the same lazy, cached load with ``ImportError`` on a missing or incompatible
build, checked against ``torch.version.hip`` instead of ``torch.version.cuda``.
The C ABI is declared in ``include/tonari_hip.h``.
"""

from __future__ import annotations

import ctypes
import os
from functools import lru_cache

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "_lib", "libtonari_hip.so")
ABI_VERSION = 7
HOST_RESULT_SLOTS = 8

TNR_OK, TNR_INPUT_ERROR, TNR_SEARCH_ERROR, TNR_DEVICE_ERROR, TNR_RETRY = 0, 1, 2, 3, 4
ALGORITHMS = {"auto": 0, "brute_force": 1, "cell_list": 2}
EXPORTS = (
    "tnr_abi_version",
    "tnr_device_arch",
    "tnr_hip_version",
    "tnr_workspace_size",
    "tnr_count",
    "tnr_count_async",
    "tnr_count_async_hinted",
    "tnr_count_finish",
    "tnr_geometry_backward",
    "tnr_emit",
    "tnr_search_static",
    "tnr_skin_workspace_size",
    "tnr_skin_store",
    "tnr_skin_filter_async",
    "tnr_skin_finish",
)


class Request(ctypes.Structure):
    """``tnr_request`` of include/tonari_hip.h."""

    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("algorithm", ctypes.c_int32),
        ("n_atoms", ctypes.c_int64),
        ("n_structures", ctypes.c_int64),
        ("positions", ctypes.c_void_p),
        ("batch_ptr", ctypes.c_void_p),
        ("cell", ctypes.c_void_p),
        ("pbc", ctypes.c_void_p),
        ("cutoff", ctypes.c_double),
        ("half_list", ctypes.c_int32),
        ("include_self", ctypes.c_int32),
        ("sorted", ctypes.c_int32),
        ("stencil_reach", ctypes.c_int32),
        ("mask_words", ctypes.c_int32),
    ]


class Outputs(ctypes.Structure):
    """``tnr_outputs`` of include/tonari_hip.h."""

    _fields_ = [
        ("n_pairs", ctypes.c_int64),
        ("plan", ctypes.c_int64),
        ("n_tasks", ctypes.c_int64),
        ("pairs", ctypes.c_void_p),
        ("shifts", ctypes.c_void_p),
        ("distances", ctypes.c_void_p),
        ("vectors", ctypes.c_void_p),
        ("sources", ctypes.c_void_p),
        ("targets", ctypes.c_void_p),
        ("edge_index", ctypes.c_void_p),
    ]


class SkinList(ctypes.Structure):
    """``tnr_skin_list`` of include/tonari_hip.h."""

    _fields_ = [
        ("n_pairs", ctypes.c_int64),
        ("n_atoms", ctypes.c_int64),
        ("n_structures", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("pair_mode", ctypes.c_int32),
        ("build_cutoff", ctypes.c_double),
    ]


def open_library(path: str = LIBRARY) -> ctypes.CDLL:
    """Open the shared library and declare every exported signature."""
    if not os.path.exists(path):
        raise ImportError(
            f"the HIP provider was not built ({path} is missing); "
            "run `python -m tonari_amd.build`"
        )
    lib = ctypes.CDLL(path)
    lib.tnr_abi_version.restype = ctypes.c_int
    lib.tnr_abi_version.argtypes = []
    lib.tnr_device_arch.restype = ctypes.c_char_p
    lib.tnr_device_arch.argtypes = []
    lib.tnr_hip_version.restype = ctypes.c_int
    lib.tnr_hip_version.argtypes = []
    lib.tnr_workspace_size.restype = ctypes.c_size_t
    lib.tnr_workspace_size.argtypes = [ctypes.POINTER(Request)]
    lib.tnr_count.restype = ctypes.c_int
    lib.tnr_count.argtypes = [
        ctypes.POINTER(Request), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64), ctypes.c_char_p, ctypes.c_size_t,
    ]
    lib.tnr_count_async.restype = ctypes.c_int
    lib.tnr_count_async.argtypes = [
        ctypes.POINTER(Request), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t,
    ]
    lib.tnr_count_async_hinted.restype = ctypes.c_int
    lib.tnr_count_async_hinted.argtypes = [
        ctypes.POINTER(Request), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ctypes.c_void_p, ctypes.c_int64, ctypes.c_char_p, ctypes.c_size_t,
    ]
    lib.tnr_count_finish.restype = ctypes.c_int
    lib.tnr_count_finish.argtypes = [
        ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64), ctypes.c_char_p, ctypes.c_size_t,
    ]
    lib.tnr_geometry_backward.restype = ctypes.c_int
    lib.tnr_geometry_backward.argtypes = [
        ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_char_p,
        ctypes.c_size_t,
    ]
    lib.tnr_emit.restype = ctypes.c_int
    lib.tnr_emit.argtypes = [
        ctypes.POINTER(Request), ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(Outputs),
        ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t,
    ]
    lib.tnr_search_static.restype = ctypes.c_int
    lib.tnr_search_static.argtypes = [
        ctypes.POINTER(Request), ctypes.POINTER(Outputs), ctypes.c_void_p, ctypes.c_void_p,
        ctypes.c_char_p, ctypes.c_size_t,
    ]
    lib.tnr_skin_workspace_size.restype = ctypes.c_size_t
    lib.tnr_skin_workspace_size.argtypes = [ctypes.POINTER(Request), ctypes.c_int64]
    lib.tnr_skin_store.restype = ctypes.c_int
    lib.tnr_skin_store.argtypes = [
        ctypes.POINTER(Request), ctypes.c_double, ctypes.c_void_p, ctypes.c_void_p,
        ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(SkinList),
        ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t,
    ]
    lib.tnr_skin_filter_async.restype = ctypes.c_int
    lib.tnr_skin_filter_async.argtypes = [
        ctypes.POINTER(Request), ctypes.POINTER(SkinList), ctypes.c_void_p, ctypes.c_size_t,
        ctypes.POINTER(Outputs), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_char_p,
        ctypes.c_size_t,
    ]
    lib.tnr_skin_finish.restype = ctypes.c_int
    lib.tnr_skin_finish.argtypes = [
        ctypes.POINTER(Request), ctypes.POINTER(SkinList), ctypes.c_void_p,
        ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int32), ctypes.c_char_p,
        ctypes.c_size_t,
    ]
    version = lib.tnr_abi_version()
    if version != ABI_VERSION:
        raise ImportError(
            f"libtonari_hip.so has ABI version {version}, expected {ABI_VERSION}; rebuild it"
        )
    return lib


CPU_LIBRARY = os.path.join(HERE, "_lib", "libtonari_cpu.so")
CPU_ABI_VERSION = 1
CPU_EXPORTS = ("tnr_cpu_abi_version", "tnr_cpu_search", "tnr_cpu_copy", "tnr_cpu_free")


def open_cpu_library(path: str = CPU_LIBRARY) -> ctypes.CDLL:
    """Open the host provider (include/tonari_cpu.h) and declare its signatures."""
    if not os.path.exists(path):
        raise ImportError(
            f"the CPU provider was not built ({path} is missing); "
            "run `python -m tonari_amd.build`"
        )
    lib = ctypes.CDLL(path)
    lib.tnr_cpu_abi_version.restype = ctypes.c_int
    lib.tnr_cpu_abi_version.argtypes = []
    lib.tnr_cpu_search.restype = ctypes.c_int
    lib.tnr_cpu_search.argtypes = [
        ctypes.c_int32, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_double, ctypes.c_int32, ctypes.c_int32,
        ctypes.c_int32, ctypes.c_int64, ctypes.POINTER(ctypes.c_void_p),
        ctypes.POINTER(ctypes.c_int64), ctypes.c_char_p, ctypes.c_size_t,
    ]
    lib.tnr_cpu_copy.restype = None
    lib.tnr_cpu_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    lib.tnr_cpu_free.restype = None
    lib.tnr_cpu_free.argtypes = [ctypes.c_void_p]
    version = lib.tnr_cpu_abi_version()
    if version != CPU_ABI_VERSION:
        raise ImportError(
            f"libtonari_cpu.so has ABI version {version}, expected {CPU_ABI_VERSION}; rebuild it"
        )
    return lib


@lru_cache
def load_cpu() -> ctypes.CDLL:
    """The host provider, loaded once (replaces the reference's load_numpy_cpu /
    load_torch_cpu, src/tonari/_extensions.py:51-59)."""
    return open_cpu_library()


def hip_major_minor(version: str) -> tuple[int, int]:
    """(major, minor) of a HIP version string such as torch.version.hip ("7.0.51831")."""
    parts = version.split(".")
    if len(parts) < 2 or not parts[0].isdigit() or not parts[1].isdigit():
        raise ImportError(f"unrecognised HIP version {version!r}")
    return int(parts[0]), int(parts[1])


def check_runtime(lib: ctypes.CDLL, torch_hip: str | None) -> None:
    """The build checks of the reference loader (``src/tonari/_extensions.py:33-48``).

    The reference compares torch's major.minor and CUDA runtime with its
    build, because its extension links LibTorch and the CUDA runtime.  This
    library links neither LibTorch nor a HIP runtime of its own: it calls the
    C API of the HIP runtime that torch loaded (libamdhip64.so.<major>).  So
    torch must be a ROCm build whose HIP major version equals the one the
    library was compiled with; the minor version may differ (the C API is
    stable within a major version).
    """
    if not torch_hip:
        raise ImportError(
            "tonari_amd requires a ROCm build of PyTorch (torch.version.hip is unset)"
        )
    built = lib.tnr_hip_version()
    runtime = hip_major_minor(torch_hip)
    if runtime[0] != built // 100:
        raise ImportError(
            f"libtonari_hip.so was built with HIP {built // 100}.{built % 100}, but torch uses "
            f"HIP {torch_hip}; rebuild it with a HIP {runtime[0]}.x toolchain"
        )


@lru_cache
def load_torch_hip() -> ctypes.CDLL:
    """Load the provider for PyTorch tensors on ROCm (HIP) devices."""
    import torch

    if not getattr(torch.version, "hip", None):
        raise ImportError(
            "tonari_amd requires a ROCm build of PyTorch (torch.version.hip is unset)"
        )
    lib = open_library()
    check_runtime(lib, torch.version.hip)
    return lib


@lru_cache
def check_device(index: int) -> None:
    """Raise ImportError unless device `index` runs the library's offload target."""
    import torch

    lib = load_torch_hip()
    arch = lib.tnr_device_arch().decode()
    found = torch.cuda.get_device_properties(index).gcnArchName.split(":")[0]
    if found != arch:
        raise ImportError(
            f"libtonari_hip.so holds {arch} code only; device cuda:{index} is {found}"
        )
