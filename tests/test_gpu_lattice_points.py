"""GPU: atoms whose wraps are decided at the ulp.

The device computes each structure's pseudo-inverse by float64 Jacobi and
each atom's wrap floor(p . dual) with double-double accumulation, where the
reference uses long double throughout (``csrc/core/geometry.cpp:15-118``,
``neighbors_cpu.cpp:92-133``).  The two can part only where p . dual lies
within about 1e-16 of an integer, and a different wrap moves the image box
a pair is taken from.  ``tests/_util.py``'s ``lattice_point_case`` puts atoms
exactly there: on the lattice points, cell faces and half-lattice sites of
skewed cells, rounded in the input type.  The CPU oracle, checked against
the reference core on the same inputs (``tests/test_oracle.py``), is the
anchor: every case's (i, j, S) multiset must equal the oracle's bit for
bit, with D within the float64 formula's tolerance, for 40 cells, both
dtypes, three periodicity patterns, both algorithms and two pair modes; and
with the cutoff at one cell height, where the repeat count ceil(rc |dual_a|)
is decided at the ulp as well.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests._util import (
    assert_geometry_close, assert_same_keys, keys_of, lattice_point_case, oracle_call,
)
from tonari_amd import neighbor_list

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("pbc", [[1, 1, 1], [1, 0, 1], [1, 1, 0]])
def test_lattice_point_atoms_match_the_oracle(dtype, pbc):
    print(f"[lattice points] {np.dtype(dtype).name} pbc={pbc}", flush=True)
    for seed in range(40):
        cfg = lattice_point_case(seed, dtype, pbc)
        t = [torch.as_tensor(cfg[k]).to(DEV) for k in ("positions", "cell", "pbc")]
        bp = torch.as_tensor(cfg["batch_ptr"]).to(DEV)
        for algorithm in ("brute_force", "cell_list"):
            for half_list, include_self in ((False, False), (True, True)):
                full = dict(cfg, half_list=half_list, include_self=include_self)
                P, S, D = neighbor_list("PSD", *t, cfg["cutoff"], bp, algorithm=algorithm,
                                        half_list=half_list, include_self=include_self)
                torch.cuda.synchronize()
                assert_same_keys(keys_of(P, S), keys_of(*oracle_call(full, algorithm=algorithm)))
                assert_geometry_close(P, S, None, D, full)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("pbc", [[1, 1, 1], [1, 0, 1], [1, 1, 0]])
def test_cutoff_at_a_cell_height_matches_the_oracle(dtype, pbc):
    # the cutoff one height 1 / |dual_a| of a periodic axis (double):
    # rc |dual_a| lies within rounding of 1, so the repeat count R_a = ceil(...)
    # is decided at the ulp
    print(f"[cell heights] {np.dtype(dtype).name} pbc={pbc}", flush=True)
    for seed in range(20):
        cfg = lattice_point_case(seed, dtype, pbc, heights=1)
        t = [torch.as_tensor(cfg[k]).to(DEV) for k in ("positions", "cell", "pbc")]
        bp = torch.as_tensor(cfg["batch_ptr"]).to(DEV)
        for algorithm in ("brute_force", "cell_list"):
            P, S, D = neighbor_list("PSD", *t, cfg["cutoff"], bp, algorithm=algorithm)
            torch.cuda.synchronize()
            assert_same_keys(keys_of(P, S), keys_of(*oracle_call(cfg, algorithm=algorithm)))
            assert_geometry_close(P, S, None, D, cfg)
