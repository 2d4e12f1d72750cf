"""The C ABI of libtonari_hip.so without a GPU.

Checks that the library loads, exports every function ``include/tonari_hip.h``
declares, reports its ABI version and target, sizes workspaces, rejects bad
requests before touching the device, and maps device status words to the
reference's exception types and messages in the reference's priority order
(csrc/torch/bindings_cuda.cpp:69-118, csrc/torch/neighbors_cuda.cu:513-521).
No call here launches a kernel.
"""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from tonari_amd import _extensions as ext

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tonari_hip.h")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(ext.LIBRARY):
        from tonari_amd import build

        build.build()
    return ext.open_library()


def _declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(tnr_\w+)\s*\(", text, flags=re.M)


def _header_define(name: str) -> int:
    m = re.search(rf"#define\s+{name}\s+(\d+)", open(HEADER).read())
    assert m, name
    return int(m.group(1))


def test_header_declares_the_python_exports():
    assert sorted(_declared_functions()) == sorted(ext.EXPORTS)


def test_library_exports_every_declared_function(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), name


def test_version_and_target(lib):
    assert lib.tnr_abi_version() == _header_define("TNR_ABI_VERSION") == ext.ABI_VERSION
    assert lib.tnr_device_arch() == b"gfx950"


def test_struct_layouts_match_header():
    # offsets of tnr_request / tnr_outputs as laid out by the C compiler
    assert ctypes.sizeof(ext.Request) == 88
    assert ext.Request.cutoff.offset == 56 and ext.Request.stencil_reach.offset == 76
    assert ext.Request.mask_words.offset == 80
    assert ctypes.sizeof(ext.Outputs) == 80 and ext.Outputs.targets.offset == 64
    assert ext.Outputs.edge_index.offset == 72
    assert ext.Outputs.n_tasks.offset == 16


def _request(**kw) -> ext.Request:
    base = dict(dtype=0, algorithm=0, n_atoms=10, n_structures=1, positions=1 << 20,
                batch_ptr=1 << 21, cell=1 << 22, pbc=1 << 23, cutoff=1.0, half_list=0,
                include_self=0, sorted=0, stencil_reach=0)
    base.update(kw)
    return ext.Request(**base)


def test_workspace_size(lib):
    sizes = []
    for n in (0, 1, 1000, 100_000):
        for dtype in (0, 1):
            size = lib.tnr_workspace_size(ctypes.byref(_request(n_atoms=n, dtype=dtype)))
            assert size > 0 and size % 256 == 0
            sizes.append(size)
    assert sizes == sorted(sizes) or sizes[-1] > sizes[0]
    # grows with the atom count, and double precision needs more
    r32 = lib.tnr_workspace_size(ctypes.byref(_request(n_atoms=100_000)))
    r64 = lib.tnr_workspace_size(ctypes.byref(_request(n_atoms=100_000, dtype=1)))
    assert r64 > r32 > lib.tnr_workspace_size(ctypes.byref(_request(n_atoms=1000)))
    assert lib.tnr_workspace_size(ctypes.byref(_request(n_atoms=-1))) == 0


def test_workspace_size_follows_mask_words(lib):
    # the hit-mask area is mask_words 8-byte words per atom (plus one row),
    # 64 by default; every other sub-buffer is independent of it
    n = 100_000

    def size(mw):
        return lib.tnr_workspace_size(ctypes.byref(_request(n_atoms=n, mask_words=mw)))

    assert size(0) == size(64)
    for mw in (1, 11, 32, 63):
        grown = size(64) - size(mw)
        exact = 8 * (n + 1) * (64 - mw)
        assert abs(grown - exact) < 256, (mw, grown, exact)
    assert size(-1) == 0 and size(65) == 0


def _count_async(lib, req, ws=1 << 24, ws_bytes=None, host=1 << 25):
    err = ctypes.create_string_buffer(256)
    if ws_bytes is None:
        ws_bytes = lib.tnr_workspace_size(ctypes.byref(req))
    code = lib.tnr_count_async(ctypes.byref(req), ws, ws_bytes, host, None, err, len(err))
    return code, err.value.decode()


@pytest.mark.parametrize(
    "fields, message",
    [
        ({"dtype": 7}, "dtype float32 or float64"),
        ({"algorithm": 5}, "algorithm must be"),
        ({"cutoff": float("nan")}, "cutoff must be finite and positive"),
        ({"cutoff": 0.0}, "cutoff must be finite and positive"),
        ({"cutoff": float("inf")}, "cutoff must be finite and positive"),
        ({"stencil_reach": 9}, "stencil_reach"),
        ({"mask_words": 65}, "mask_words must be in \\[0, 64\\]"),
        ({"mask_words": -2}, "mask_words must be in \\[0, 64\\]"),
        ({"n_atoms": 2**31}, "fewer than 2\\^31 atoms"),
        ({"n_structures": -1}, "invalid sizes"),
    ],
)
def test_bad_requests_are_rejected_on_the_host(lib, fields, message):
    code, text = _count_async(lib, _request(**fields), ws_bytes=1 << 30)
    assert code == ext.TNR_INPUT_ERROR
    assert re.search(message, text), text


def test_workspace_checks(lib):
    req = _request()
    need = lib.tnr_workspace_size(ctypes.byref(req))
    assert _count_async(lib, req, ws_bytes=need - 256)[0] == ext.TNR_INPUT_ERROR
    assert _count_async(lib, req, ws=(1 << 24) + 8)[0] == ext.TNR_INPUT_ERROR
    assert _count_async(lib, req, ws=0)[0] == ext.TNR_INPUT_ERROR
    code, text = _count_async(lib, req, host=0)
    assert code == ext.TNR_INPUT_ERROR and "host_result" in text


def test_emit_with_no_pairs_is_a_no_op(lib):
    req = _request()
    need = lib.tnr_workspace_size(ctypes.byref(req))
    err = ctypes.create_string_buffer(64)
    out = ext.Outputs(n_pairs=0)
    assert lib.tnr_emit(ctypes.byref(req), 1 << 24, need, ctypes.byref(out), None, err,
                        len(err)) == ext.TNR_OK
    assert lib.tnr_emit(ctypes.byref(req), 1 << 24, need, None, None, err,
                        len(err)) == ext.TNR_INPUT_ERROR


# Status bits of the device (tonari_amd/csrc/nl_device.h) and the message
# and exception class each maps to.
STATUS = [
    (0, ext.TNR_INPUT_ERROR, "batch_ptr must start at zero"),
    (1, ext.TNR_INPUT_ERROR, "batch_ptr must end at N_total"),
    (2, ext.TNR_INPUT_ERROR, "batch_ptr must be nondecreasing"),
    (3, ext.TNR_INPUT_ERROR, "cell must contain only finite values"),
    (4, ext.TNR_INPUT_ERROR, "active periodic cell vectors must be linearly independent"),
    (5, ext.TNR_INPUT_ERROR, "active periodic cell dual is outside the float64 range"),
    (6, ext.TNR_INPUT_ERROR, "periodic image range exceeds int32 cell shifts"),
    (7, ext.TNR_INPUT_ERROR, "periodic image count exceeds the 2^24 resource limit"),
    (8, ext.TNR_INPUT_ERROR, "batched periodic image count exceeds the 2^24 resource limit"),
    (9, ext.TNR_SEARCH_ERROR, "positions must contain only finite values"),
    (10, ext.TNR_SEARCH_ERROR, "atom representatives require periodic wraps outside the int32"),
    (12, ext.TNR_SEARCH_ERROR, "cell_list cannot safely process this structure"),
    (11, ext.TNR_SEARCH_ERROR, "a cell shift required by the neighbor list exceeds the int32"),
    (13, ext.TNR_SEARCH_ERROR, "neighbor-list workspace capacity exceeded"),
    (14, ext.TNR_SEARCH_ERROR, "a device-wide scan of the neighbor search did not complete"),
]


def _finish(lib, flags, pairs=0):
    host = (ctypes.c_int64 * 8)(flags, pairs, 0, 0, 0, 0, 0, 0)
    n = ctypes.c_int64(-1)
    err = ctypes.create_string_buffer(256)
    code = lib.tnr_count_finish(host, ctypes.byref(n), err, len(err))
    return code, err.value.decode(), n.value


@pytest.mark.parametrize("bit, code, message", STATUS)
def test_status_words_map_to_reference_errors(lib, bit, code, message):
    got, text, _ = _finish(lib, 1 << bit)
    assert got == code
    assert text.startswith(message)


def test_status_priority_follows_reference_order(lib):
    # Several faults at once report the first in the reference's order.
    for k in range(len(STATUS) - 1):
        bits = sum(1 << b for b, _, _ in STATUS[k:])
        code, text, _ = _finish(lib, bits)
        assert text.startswith(STATUS[k][2]) and code == STATUS[k][1]


def test_finish_reports_pair_count(lib):
    code, text, n = _finish(lib, 0, 12345)
    assert code == ext.TNR_OK and n == 12345


def test_static_search_rejects_requests_beyond_its_scratch(lib):
    # 400,000 float32 atoms need more than the 64 MiB static scratch; the
    # check happens before any device work
    req = _request(n_atoms=400_000)
    assert lib.tnr_workspace_size(ctypes.byref(req)) > 64 << 20
    err = ctypes.create_string_buffer(256)
    code = lib.tnr_search_static(ctypes.byref(req), None, None, None, err, len(err))
    assert code == ext.TNR_INPUT_ERROR
    assert "static scratch holds 67108864 bytes" in err.value.decode()


def test_build_records_its_hip_version(lib):
    version = lib.tnr_hip_version()
    m = re.search(r"#define HIP_VERSION_MAJOR (\d+)\s+#define HIP_VERSION_MINOR (\d+)",
                  open("/opt/rocm/include/hip/hip_version.h").read()) if os.path.exists(
        "/opt/rocm/include/hip/hip_version.h") else None
    assert version >= 700
    if m:
        assert version == int(m.group(1)) * 100 + int(m.group(2))


def test_runtime_check_follows_the_hip_major_version(lib):
    built = lib.tnr_hip_version()
    major, minor = built // 100, built % 100
    # same major: accepted whatever the minor (the C API of libamdhip64.so.<major>)
    ext.check_runtime(lib, f"{major}.{minor}.12345")
    ext.check_runtime(lib, f"{major}.0.51831")
    for bad in (f"{major + 1}.0.1", f"{major - 1}.4.2"):
        with pytest.raises(ImportError, match="rebuild it"):
            ext.check_runtime(lib, bad)
    with pytest.raises(ImportError, match="ROCm build of PyTorch"):
        ext.check_runtime(lib, None)
    with pytest.raises(ImportError, match="unrecognised HIP version"):
        ext.check_runtime(lib, "rocm")


def test_skin_list_layout_and_workspace(lib):
    assert ctypes.sizeof(ext.SkinList) == 40 and ext.SkinList.build_cutoff.offset == 32
    req = _request(n_atoms=1000)
    a = lib.tnr_skin_workspace_size(ctypes.byref(req), 10)
    b = lib.tnr_skin_workspace_size(ctypes.byref(req), 10_000_000)
    # 8 bytes per stored pair, plus per-tile data
    assert 0 < a < b and a % 256 == 0 and b % 256 == 0
    assert 8 * 10_000_000 <= b - a < 9 * 10_000_000
    assert lib.tnr_skin_workspace_size(ctypes.byref(req), -1) == 0
    assert lib.tnr_skin_workspace_size(None, 10) == 0


def _skin_store(lib, req, build_cutoff=1.5, n=5, pairs=1 << 26, shifts=1 << 27, ws=1 << 24,
                ws_bytes=None):
    err = ctypes.create_string_buffer(256)
    if ws_bytes is None:
        ws_bytes = lib.tnr_skin_workspace_size(ctypes.byref(req), max(n, 0))
    lst = ext.SkinList()
    code = lib.tnr_skin_store(ctypes.byref(req), build_cutoff, pairs, shifts, n, ws, ws_bytes,
                              ctypes.byref(lst), None, err, len(err))
    return code, err.value.decode()


def test_skin_requests_are_rejected_on_the_host(lib):
    req = _request(n_atoms=100)
    for kw, message in (
        ({"build_cutoff": 0.5}, "at least the cutoff"),
        ({"build_cutoff": float("nan")}, "at least the cutoff"),
        ({"pairs": None}, "required pointers"),
        ({"n": -1}, "invalid sizes"),
        ({"ws": (1 << 24) + 8}, "256-byte aligned"),
    ):
        code, text = _skin_store(lib, req, **kw)
        assert code == ext.TNR_INPUT_ERROR and message in text, text
    need = lib.tnr_skin_workspace_size(ctypes.byref(req), 5)
    assert _skin_store(lib, req, ws_bytes=need - 256)[0] == ext.TNR_INPUT_ERROR
    code, text = _skin_store(lib, _request(n_atoms=100, cutoff=-1.0))
    assert code == ext.TNR_INPUT_ERROR and "cutoff" in text
    # a filter whose request does not match the stored list
    err = ctypes.create_string_buffer(256)
    lst = ext.SkinList(n_pairs=5, n_atoms=100, n_structures=1, dtype=0, build_cutoff=1.5)
    out = ext.Outputs(n_pairs=5)
    need = lib.tnr_skin_workspace_size(ctypes.byref(req), 5)

    def run(r, o=out, host=1 << 25):
        code = lib.tnr_skin_filter_async(ctypes.byref(r), ctypes.byref(lst), 1 << 24, need,
                                         ctypes.byref(o), host, None, err, len(err))
        return code, err.value.decode()

    code, text = run(_request(n_atoms=101))
    assert code == ext.TNR_INPUT_ERROR and "differ from the stored list" in text
    code, text = run(_request(n_atoms=100, dtype=1))
    assert code == ext.TNR_INPUT_ERROR
    code, text = run(_request(n_atoms=100, cutoff=2.0))
    assert code == ext.TNR_INPUT_ERROR and "at least the cutoff" in text
    code, text = run(req, ext.Outputs(n_pairs=5, edge_index=1 << 28))
    assert code == ext.TNR_INPUT_ERROR and "edge-first" in text
    code, text = run(req, host=0)
    assert code == ext.TNR_INPUT_ERROR and "host_result" in text
