"""GPU: the molecule prologue without the batch scan (plan hint 5).

A repeated count of a molecules-only batch of at most 4,096 structures runs
k_molecule_setup alone as its prologue: each workgroup of 64 structures
leaves block-local work-unit offsets and a summary (units, images, error
bits), and the molecule counting kernel scans the summaries in every wave,
finds each unit's structure from them, and writes the global offsets for
the emitting pass and the status words.  Every case drives the hint through
the C ABI and compares the emitted (i, j, S) multiset with the CPU oracle
bit for bit and D with the float64 formula (1e-5 relative for float32,
1e-12 for float64): batches spanning several workgroups, with empty
structures and a workgroup holding none but empty ones, all pair modes and
`sorted`, the largest batch of this path (4,096 structures) and the next
(4,097, planned with the batch scan), the frontend's repeats, and the hint
failing.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests._util import assert_geometry_close, assert_same_keys, keys_of, oracle_call
from tests.test_gpu_periodic_prologue import search
from tonari_amd import neighbor_list
from tonari_amd._extensions import TNR_OK, TNR_RETRY

pytestmark = pytest.mark.gpu

HINT = 5  # plan bits 0 (brute force) and 2 (every brute-force structure a molecule)
MODES = [(False, False), (False, True), (True, False), (True, True)]


def molecules(sizes, dtype, seed, cutoff=4.0):
    rng = np.random.Generator(np.random.PCG64(seed))
    pos = [rng.uniform(0.0, max(n / 0.05, 1.0) ** (1 / 3), (n, 3)) + 50.0 * k
           for k, n in enumerate(sizes)]
    return {
        "positions": np.concatenate(pos).astype(dtype) if pos else np.zeros((0, 3), dtype),
        "cell": np.zeros((len(sizes), 3, 3), dtype),
        "pbc": np.zeros((len(sizes), 3), bool),
        "batch_ptr": np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64),
        "cutoff": cutoff,
    }


def check(cfg, algorithm="brute_force", **kw):
    full = dict(cfg, half_list=kw.get("half_list", False),
                include_self=kw.get("include_self", False))
    code, msg, plan, P, S, D = search(full, HINT, algorithm=algorithm, **kw)
    assert code == TNR_OK, msg
    assert plan == HINT, plan
    assert_same_keys(keys_of(P, S), keys_of(*oracle_call(full, algorithm=algorithm)))
    assert_geometry_close(P, S, None, D, full)
    if kw.get("sorted"):
        src = P[:, 0]
        assert bool((src[1:] >= src[:-1]).all())
    return len(P)


def spread(seed):
    # 150 structures in three workgroups of the prologue: the first mixed
    # (empty ones among them), the second all empty, the third mixed
    rng = np.random.Generator(np.random.PCG64(seed))
    first = [int(x) for x in rng.choice([0, 1, 7, 33, 64, 65, 130, 300], size=64)]
    last = [int(x) for x in rng.choice([0, 2, 20, 129, 513], size=22)]
    return first + [0] * 64 + last


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("half_list,include_self", MODES)
def test_batches_across_workgroups(dtype, half_list, include_self):
    print(f"[molecule prologue] {np.dtype(dtype).name} half={half_list} self={include_self}",
          flush=True)
    cfg = molecules(spread(11), dtype, 12)
    for sorted_ in (False, True):
        check(cfg, half_list=half_list, include_self=include_self, sorted=sorted_)
    check(cfg, algorithm="auto", half_list=half_list, include_self=include_self)


def test_largest_local_batch_and_the_next():
    rng = np.random.Generator(np.random.PCG64(13))
    for nb in (4096, 4097):
        sizes = [int(x) for x in rng.integers(0, 13, size=nb)]
        print(f"[molecule prologue] {nb} structures, {sum(sizes)} atoms", flush=True)
        check(molecules(sizes, np.float32, 14 + nb, cutoff=3.0))


def test_frontend_repeats_take_the_hint():
    import torch

    from tonari_amd._torch_frontend import _speculation

    cfg = molecules(spread(15), np.float32, 16)
    t = {k: torch.as_tensor(cfg[k]).to("cuda:0") for k in ("positions", "cell", "pbc", "batch_ptr")}
    expected = keys_of(*oracle_call(cfg, algorithm="brute_force"))
    _speculation().clear()
    for call in range(3):
        P, S, D = neighbor_list("PSD", t["positions"], t["cell"], t["pbc"], cfg["cutoff"],
                                t["batch_ptr"], algorithm="brute_force")
        torch.cuda.synchronize()
        assert_same_keys(keys_of(P, S), expected)
        assert_geometry_close(P, S, None, D, cfg)
    assert {v[1] for v in _speculation().values()} == {HINT}


def test_hint_that_does_not_hold_is_retried():
    # one periodic structure (with atoms) among the molecules: not a molecule
    sizes = spread(17)
    sizes[5] = 40
    cfg = molecules(sizes, np.float32, 18)
    cfg["pbc"][5] = True
    cfg["cell"][5] = np.eye(3, dtype=np.float32) * 40.0
    full = dict(cfg, half_list=False, include_self=False)
    code, msg, plan, P, S, D = search(full, HINT, algorithm="brute_force")
    assert code == TNR_RETRY and "plan hint" in msg, (code, msg)
    code, msg, plan, P, S, D = search(full, -1, algorithm="brute_force")
    assert code == TNR_OK and plan == 1, (code, msg, plan)
    assert_same_keys(keys_of(P, S), keys_of(*oracle_call(full, algorithm="brute_force")))
