"""CPU oracle for the tonari neighbor-list hot path.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``, and there only as the checker.
The product package ``tonari_amd`` never imports it.

Two interchangeable native builds share one C ABI (``orc_neighbor_list``):

* ``"port"``      - ``oracle/liboracle.so``, a C++20 restatement of the
  reference CPU search (``oracle/nl_oracle.cpp``);
* ``"reference"`` - ``oracle/_ref/libtonari_ref.so``, the reference's own CPU
  core compiled from its sources (``oracle/Makefile``), present only where the
  reference checkout was available at build time.

``quantities()`` restates the reference frontend's assembly of i/j/d/D from
P and S (``src/tonari/_torch_frontend.py:78-105``) in numpy.
"""

from __future__ import annotations

import ctypes
import hashlib
import os
import subprocess
from functools import lru_cache

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PORT_LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libtonari_ref.so")

_ALGORITHMS = {"auto": 0, "brute_force": 1, "cell_list": 2}


class OracleInputError(ValueError):
    """Mirrors the reference's InputError -> ValueError mapping."""


class OracleSearchError(RuntimeError):
    """Mirrors the reference's SearchError -> RuntimeError mapping."""


def build(reference: bool = True) -> None:
    """Compile the restatement (and the reference core when its checkout exists)."""
    targets = ["oracle", "ref"] if reference else ["oracle"]
    subprocess.run(["make", "-s", "-C", HERE, *targets], check=True)


def available(kind: str = "port") -> bool:
    return os.path.exists(PORT_LIB if kind == "port" else REF_LIB)


@lru_cache
def _load(kind: str) -> ctypes.CDLL:
    path = PORT_LIB if kind == "port" else REF_LIB
    if not os.path.exists(path):
        if kind == "port":
            build(reference=False)
        else:
            raise FileNotFoundError(f"{path} is not built")
    lib = ctypes.CDLL(path)
    lib.orc_neighbor_list.restype = ctypes.c_int
    lib.orc_neighbor_list.argtypes = [
        ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_double, ctypes.c_int, ctypes.c_int,
        ctypes.c_int, ctypes.c_int64, ctypes.POINTER(ctypes.c_void_p),
        ctypes.POINTER(ctypes.c_int64), ctypes.c_char_p, ctypes.c_int64,
    ]
    lib.orc_copy.restype = None
    lib.orc_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.orc_free.restype = None
    lib.orc_free.argtypes = [ctypes.c_void_p]
    return lib


def neighbor_pairs(
    positions: np.ndarray,
    cell: np.ndarray,
    pbc: np.ndarray,
    cutoff: float,
    batch_ptr: np.ndarray | None = None,
    *,
    half_list: bool = False,
    include_self: bool = False,
    algorithm: str = "auto",
    threads: int = 1,
    kind: str = "port",
) -> tuple[np.ndarray, np.ndarray]:
    """Return ``(P (E,2) int64, S (E,3) int32)`` in source-major order."""
    positions = np.ascontiguousarray(positions)
    if positions.dtype not in (np.float32, np.float64):
        raise OracleInputError("positions must have dtype float32 or float64")
    if batch_ptr is None:
        batch_ptr = np.array([0, len(positions)], dtype=np.int64)
        cell = np.asarray(cell)[None]
        pbc = np.asarray(pbc)[None]
    cell = np.ascontiguousarray(cell, dtype=positions.dtype)
    pbc = np.ascontiguousarray(pbc, dtype=np.uint8)
    batch_ptr = np.ascontiguousarray(batch_ptr, dtype=np.int64)
    lib = _load(kind)
    handle = ctypes.c_void_p()
    count = ctypes.c_int64()
    err = ctypes.create_string_buffer(512)
    code = lib.orc_neighbor_list(
        0 if positions.dtype == np.float32 else 1,
        positions.ctypes.data, len(positions), batch_ptr.ctypes.data, len(batch_ptr),
        cell.ctypes.data, pbc.ctypes.data, float(cutoff), int(half_list),
        int(include_self), _ALGORITHMS[algorithm], int(threads), ctypes.byref(handle),
        ctypes.byref(count), err, len(err),
    )
    if code == 1:
        raise OracleInputError(err.value.decode())
    if code != 0:
        raise OracleSearchError(err.value.decode())
    try:
        pairs = np.empty((count.value, 2), dtype=np.int64)
        shifts = np.empty((count.value, 3), dtype=np.int32)
        if count.value:
            lib.orc_copy(handle, pairs.ctypes.data, shifts.ctypes.data)
    finally:
        lib.orc_free(handle)
    return pairs, shifts


def quantities(
    which: str,
    positions: np.ndarray,
    cell: np.ndarray,
    batch_ptr: np.ndarray,
    pairs: np.ndarray,
    shifts: np.ndarray,
) -> tuple[np.ndarray, ...]:
    """Assemble i/j/P/S/d/D like the reference frontend (``_torch_frontend.py:78-105``).

    D = positions[j] - positions[i] + S @ cell[b]; d = |D|.
    """
    values: dict[str, np.ndarray] = {"P": pairs, "S": shifts}
    source, target = pairs[:, 0], pairs[:, 1]
    values["i"] = np.ascontiguousarray(source)
    values["j"] = np.ascontiguousarray(target)
    if "d" in which or "D" in which:
        b = np.searchsorted(batch_ptr[1:], source, side="right")
        disp = positions[target] - positions[source] + np.einsum(
            "ei,eij->ej", shifts.astype(positions.dtype), cell[b]
        )
        values["D"] = disp
        values["d"] = np.sqrt(np.sum(disp * disp, axis=1))
    return tuple(values[q] for q in which)


def canonical_keys(pairs: np.ndarray, shifts: np.ndarray) -> np.ndarray:
    """Rows (i, j, Sx, Sy, Sz) as int64, lexicographically sorted."""
    rows = np.concatenate([pairs.astype(np.int64), shifts.astype(np.int64)], axis=1)
    if len(rows) == 0:
        return rows.reshape(0, 5)
    order = np.lexsort(tuple(rows[:, c] for c in range(4, -1, -1)))
    return rows[order]


def key_hash(pairs: np.ndarray, shifts: np.ndarray) -> str:
    """SHA-256 of the canonical key rows as little-endian int64."""
    keys = canonical_keys(pairs, shifts)
    return hashlib.sha256(np.ascontiguousarray(keys, dtype="<i8").tobytes()).hexdigest()


_MIX = (0x9E3779B97F4A7C15, 0xBF58476D1CE4E5B9, 0x94D049BB133111EB, 0xD6E8FEB86659FD93,
        0xA0761D6478BD642F)


def multiset_hash(pairs: np.ndarray, shifts: np.ndarray) -> int:
    """Order-independent 64-bit checksum of the (i, j, Sx, Sy, Sz) multiset.

    Each row is mixed to 64 bits (splitmix64 finaliser over a weighted sum of
    its fields) and the row hashes are added modulo 2^64, so any order of the
    same pairs gives the same value and a changed, missing or extra row
    changes it with probability ~1 - 2^-64.
    """
    cols = [pairs[:, 0], pairs[:, 1], shifts[:, 0], shifts[:, 1], shifts[:, 2]]
    with np.errstate(over="ignore"):
        x = np.zeros(len(pairs), dtype=np.uint64)
        for c, k in zip(cols, _MIX):
            x = (x ^ (c.astype(np.int64).astype(np.uint64) * np.uint64(k))) * np.uint64(_MIX[1])
            x ^= x >> np.uint64(31)
        x ^= x >> np.uint64(30)
        x *= np.uint64(_MIX[1])
        x ^= x >> np.uint64(27)
        x *= np.uint64(_MIX[2])
        x ^= x >> np.uint64(31)
        return int(np.sum(x, dtype=np.uint64))
