"""GPU: an explicit ``cell_list`` request on cells that no bin grid fits.

Where the cutoff spans two or more cell widths on every periodic axis, a
cell list has one bin per axis and needs a stencil of 7^3 periodic pieces,
more than the stencil tables hold.  Such structures are searched with the
brute-force kernels (the same pair set), counted inside the cell-list
counting kernel because an explicit ``cell_list`` request launches no
brute-force counting kernel.  The reference CPU cell list
(``csrc/core/neighbors_cpu.cpp:379-430,675-679``) serves them as long as its
own layout rule holds; where that rule refuses (``"cell_list cannot
safely"``), the GPU must refuse with the same error.  The (i, j, S) multiset
must equal the CPU oracle's bit for bit, with d and D within the stated
tolerance.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests._util import assert_geometry_close, assert_same_keys, keys_of, oracle_call
from tests.test_gpu_brute_stress import skewed_batch
from tonari_amd import neighbor_list

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
MODES = [(False, False), (True, False), (False, True), (True, True)]


def _run(cfg, half_list, include_self, algorithm="cell_list"):
    t = lambda x: torch.as_tensor(x).to(DEV)  # noqa: E731
    out = neighbor_list(
        "PSdD", t(cfg["positions"]), t(cfg["cell"]), t(cfg["pbc"]), cfg["cutoff"],
        t(cfg["batch_ptr"]), algorithm=algorithm, half_list=half_list,
        include_self=include_self,
    )
    torch.cuda.synchronize()
    return out


def _check(cfg, half_list, include_self):
    cfg = dict(cfg, half_list=half_list, include_self=include_self)
    try:
        expected = keys_of(*oracle_call(cfg, algorithm="cell_list"))
    except oracle.OracleSearchError as error:
        with pytest.raises(RuntimeError, match="cell_list cannot safely"):
            _run(cfg, half_list, include_self)
        assert "cell_list cannot safely" in str(error)
        return 0
    P, S, d, D = _run(cfg, half_list, include_self)
    assert_same_keys(keys_of(P, S), expected)
    assert_geometry_close(P, S, d, D, cfg)
    return len(expected)


def small_cube(dtype, edge=3.0, n=10, seed=7):
    rng = np.random.Generator(np.random.PCG64(seed))
    pos = rng.uniform(0.0, edge, size=(n, 3))
    return {
        "positions": pos.astype(dtype),
        "cell": (edge * np.eye(3))[None].astype(dtype),
        "pbc": np.ones((1, 3), bool),
        "batch_ptr": np.array([0, n], np.int64),
        "cutoff": 6.0,
    }


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("half_list,include_self", MODES)
def test_small_cubic_cell(dtype, half_list, include_self):
    # 3 A cube at rc 6: the cutoff spans two cell widths on every axis
    print(f"[fallback] 3 A cube dtype={np.dtype(dtype).name} half={half_list} "
          f"self={include_self}", flush=True)
    n = _check(small_cube(dtype), half_list, include_self)
    assert n > 0


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_small_cubic_cell_matches_other_algorithms(dtype):
    # the three algorithms agree on the tiny cell, and a batch of such cells
    # mixed with an ordinary one keeps every structure's pairs
    cfg = small_cube(dtype, edge=2.0, n=6, seed=11)
    keys = [keys_of(*_run(cfg, False, False, algorithm)[:2])
            for algorithm in ("cell_list", "brute_force", "auto")]
    assert len(keys[0]) > 0
    assert_same_keys(keys[0], keys[1])
    assert_same_keys(keys[0], keys[2])


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_mixed_batch_of_tiny_and_ordinary_cells(dtype):
    tiny = small_cube(dtype, edge=2.5, n=7, seed=3)
    rng = np.random.Generator(np.random.PCG64(5))
    big = rng.uniform(0.0, 14.0, size=(300, 3))
    cfg = {
        "positions": np.concatenate([tiny["positions"], big.astype(dtype)]),
        "cell": np.stack([tiny["cell"][0], 14.0 * np.eye(3)]).astype(dtype),
        "pbc": np.ones((2, 3), bool),
        "batch_ptr": np.array([0, 7, 307], np.int64),
        "cutoff": 6.0,
    }
    for half_list, include_self in MODES:
        print(f"[fallback] mixed batch dtype={np.dtype(dtype).name} half={half_list} "
              f"self={include_self}", flush=True)
        assert _check(cfg, half_list, include_self) > 0


@pytest.mark.parametrize("seed", [101, 202, 303])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("half_list,include_self", MODES)
def test_skewed_cells_with_cell_list(seed, dtype, half_list, include_self):
    print(f"[fallback] skewed seed={seed} dtype={np.dtype(dtype).name} half={half_list} "
          f"self={include_self}", flush=True)
    _check(skewed_batch(seed, dtype), half_list, include_self)
