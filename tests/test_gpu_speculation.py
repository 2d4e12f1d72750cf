"""GPU: repeated calls of one request shape.

The frontend launches the writing pass of a repeated call before the pair
count is known, into outputs sized from the previous call.  Every case here
compares with the CPU oracle: the plain repeat, and the misses that make the
writing pass run again (more pairs than the outputs hold, more bins than the
launch covered, a plan that switches algorithm).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests._util import assert_geometry_close, assert_same_keys, keys_of, oracle_call
from tonari_amd import neighbor_list
from tonari_amd import workloads as W

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def run(quantities, cfg, **kw):
    t = lambda x: torch.as_tensor(x).to(DEV)  # noqa: E731
    out = neighbor_list(
        quantities, t(cfg["positions"]), t(cfg["cell"]), t(cfg["pbc"]), cfg["cutoff"],
        t(cfg["batch_ptr"]), algorithm=kw.pop("algorithm", "auto"), **kw,
    )
    torch.cuda.synchronize()
    return out


def check(cfg, quantities="PSD", **kw):
    P, S, D = run(quantities, cfg, **kw)
    assert_same_keys(keys_of(P, S), keys_of(*oracle_call(cfg, algorithm=kw.get("algorithm"))))
    assert_geometry_close(P, S, None, D, cfg)
    return P


def test_repeated_calls():
    cfg = W.c4(seed=11, n_atoms=20000)
    first = check(cfg)
    for _ in range(3):
        again = check(cfg)
        assert again.shape == first.shape


def test_more_pairs_than_outputs_hold():
    # same atom count, the second box four times denser: the pair count
    # grows far beyond the first call's margin
    sparse = W.c4(seed=12, n_atoms=6000, density=0.025)
    dense = W.c4(seed=13, n_atoms=6000, density=0.1)
    n_sparse = len(check(sparse))
    n_dense = len(check(dense))
    assert n_dense > 2 * n_sparse
    check(dense)
    check(sparse)


def test_more_bins_than_launch_covered():
    # same atom count, a much larger box: more bins than the previous call
    small = W.c4(seed=14, n_atoms=6000, density=0.1)
    large = W.c4(seed=15, n_atoms=6000, density=0.01)
    check(small)
    check(large)
    check(small)


def test_plan_switch():
    # the same atom count searched by brute force (an open cluster of at
    # most 384 atoms under auto) and then by a cell list (a periodic box of
    # 300 x 27 atom images)
    rng = np.random.default_rng(16)
    n = 300
    cluster = {
        "positions": rng.uniform(0.0, 8.0, (n, 3)).astype(np.float32),
        "cell": np.zeros((1, 3, 3), np.float32),
        "pbc": np.zeros((1, 3), bool),
        "batch_ptr": np.array([0, n], np.int64),
        "cutoff": 3.0,
    }
    box = W.c4(seed=17, n_atoms=n, density=0.1)
    for cfg in (cluster, box, cluster, box):
        check(cfg)
