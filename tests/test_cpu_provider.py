"""The host provider (libtonari_cpu.so) and its NumPy and Torch CPU frontends.

No GPU.  The CPU path is this build's own C++ (``tonari_amd/csrc/cpu``),
checked like the device path:

* against ``tests/golden/golden.json`` (pair counts, canonical SHA-256 and
  multiset checksums written by the reference's own compiled CPU core) on the
  BASELINE configurations and the reference suite's seeded inputs, with each
  case's own options, through the NumPy frontend;
* against the oracle for every algorithm and pair mode on every
  configuration;
* for the reference's CPU output order (sources in index order, the same
  arrays for any thread count), its error contract (exception types and
  messages, tests/backends/test_native_errors.py:11-125), the quantities
  i/j/d/D, and gradients of d/D through the Torch CPU path.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

import oracle
from tests._util import assert_same_keys, keys_of, oracle_call
from tests.golden.cases import CASES
from tonari_amd import neighbor_list
from tonari_amd import workloads as W

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "golden.json")))
_SMALL = sorted(name for name, entry in GOLDEN.items() if entry["pairs"] <= 2_000_000)


@pytest.fixture(scope="module", autouse=True)
def _built():
    from tonari_amd import _extensions as ext

    if not os.path.exists(ext.CPU_LIBRARY):
        from tonari_amd import build

        build.build_cpu()


def _np_pairs(cfg, threads=8, **options):
    opts = {k: cfg[k] for k in ("algorithm", "half_list", "include_self") if k in cfg}
    opts.update(options)
    return neighbor_list("PS", cfg["positions"], cfg["cell"], cfg["pbc"], cfg["cutoff"],
                         cfg["batch_ptr"], cpu_threads=threads, **opts)


@pytest.mark.parametrize("name", _SMALL)
def test_matches_the_reference_core_golden(name):
    make, options = CASES[name]
    cfg = make()
    P, S = neighbor_list(
        "PS", cfg["positions"], cfg["cell"], cfg["pbc"], cfg["cutoff"], cfg["batch_ptr"],
        algorithm=options.get("algorithm", "auto"), half_list=options.get("half_list", False),
        include_self=options.get("include_self", False), cpu_threads=8,
    )
    entry = GOLDEN[name]
    assert len(P) == entry["pairs"]
    assert f"{oracle.multiset_hash(P, S):016x}" == entry["multiset"]
    assert oracle.key_hash(P, S) == entry["sha256"]


CONFIGS = {
    "C1": lambda: W.c1(),
    "C2": lambda: W.c2(n_structures=24),
    "C3": lambda: W.c3(n_structures=32),
    "C4": lambda: W.c4(seed=61, n_atoms=6000),
    "C5": lambda: W.c5(n_structures=2, n_min=800, n_max=1500),
}


@pytest.mark.parametrize("name", sorted(CONFIGS))
@pytest.mark.parametrize("algorithm", ["auto", "brute_force", "cell_list"])
def test_every_algorithm_and_pair_mode_matches_the_oracle(name, algorithm):
    cfg = CONFIGS[name]()
    for half, self_ in ((False, False), (True, False), (False, True), (True, True)):
        P, S = _np_pairs(cfg, algorithm=algorithm, half_list=half, include_self=self_)
        expected = oracle_call(dict(cfg, half_list=half, include_self=self_), algorithm="auto")
        assert_same_keys(keys_of(P, S), keys_of(*expected))


def test_sources_in_index_order_for_any_thread_count():
    cfg = W.c2(n_structures=16)
    P1, S1 = _np_pairs(cfg, threads=1)
    assert np.all(P1[1:, 0] >= P1[:-1, 0])
    for threads in (2, 3, 8):
        P, S = _np_pairs(cfg, threads=threads)
        assert np.array_equal(P, P1) and np.array_equal(S, S1)
    # sorted=True is honoured as is
    P2, _ = neighbor_list("PS", cfg["positions"], cfg["cell"], cfg["pbc"], cfg["cutoff"],
                          cfg["batch_ptr"], algorithm=cfg["algorithm"], sorted=True)
    assert np.array_equal(P2, P1)


def _single(positions, cell, pbc, cutoff, dtype=np.float64):
    positions = np.asarray(positions, dtype=dtype).reshape(-1, 3)
    return (positions, np.asarray(cell, dtype=dtype).reshape(3, 3),
            np.asarray(pbc, dtype=bool).reshape(3), float(cutoff))


def test_error_contract():
    def err(exc, match, *args, **kw):
        with pytest.raises(exc, match=match):
            neighbor_list("PS", *args, **kw)

    z = np.zeros((2, 3))

    def batch(bp, nb):
        return (z, np.zeros((nb, 3, 3)), np.zeros((nb, 3), bool), 1.0,
                np.array(bp, dtype=np.int64))

    err(ValueError, "start at zero", *batch([1, 1, 2], 2))
    err(ValueError, "end at N_total", *batch([0, 1, 1], 2))
    err(ValueError, "nondecreasing", *batch([0, 2, 1, 2], 3))
    for value in (np.nan, np.inf):
        pos = np.zeros((2, 3))
        pos[0, 0] = value
        err(RuntimeError, "positions must contain only finite values",
            *_single(pos, np.zeros((3, 3)), [0, 0, 0], 0.5))
    err(RuntimeError, "wraps outside the int32 range",
        *_single([[0.1, 0, 0], [2**31 + 0.2, 0, 0]], np.eye(3), [1, 0, 0], 0.5))
    err(RuntimeError, "cell shift.*int32",
        *_single([[-(2**31) + 0.1, 0, 0], [2**31 - 0.8, 0, 0]], np.eye(3), [1, 0, 0], 0.5))
    err(ValueError, "linearly independent",
        *_single([[0, 0, 0]], [[1.0, 0, 0], [2.0, 0, 0], [0, 0, 4.0]], [1, 1, 0], 0.5))
    cell = np.eye(3)
    cell[2, 0] = np.nan
    err(ValueError, "cell must contain only finite values", *_single([[0, 0, 0]], cell, [1, 1, 0], 0.5))
    err(ValueError, "image count exceeds the 2\\^24 resource limit",
        *_single([[0, 0, 0]], 0.001 * np.eye(3), [1, 1, 1], 1.0))
    pos = np.zeros((256, 3), np.float32)
    pos[:, 0] = np.arange(256) * 10000.0
    sparse = _single(pos, np.zeros((3, 3)), [0, 0, 0], 1.0, np.float32)
    err(RuntimeError, "cell_list cannot safely", *sparse, algorithm="cell_list")
    assert len(neighbor_list("P", *sparse)[0]) == 0
    # the frontend's own checks
    err(ValueError, "positions must have dtype", np.zeros((2, 3), np.int64), np.eye(3),
        np.ones(3, bool), 1.0)
    err(ValueError, "cutoff must be finite", *_single(z, np.eye(3), [1, 1, 1], np.nan))
    err(ValueError, "cell and positions must have the same dtype", z, np.eye(3, dtype=np.float32),
        np.ones(3, bool), 1.0)
    err(ValueError, "pbc must be bool", z, np.eye(3)[None], np.ones((1, 3), np.int8), 1.0,
        np.array([0, 2], np.int64))
    err(ValueError, "single-structure cell", z, np.eye(4), np.ones(3, bool), 1.0)
    err(TypeError, "must all be NumPy arrays", z, torch.eye(3), np.ones(3, bool), 1.0)
    err(ValueError, "cpu_threads must be positive", *_single(z, np.eye(3), [1, 1, 1], 1.0),
        cpu_threads=0)


def test_empty_inputs():
    P, S, d = neighbor_list("PSd", np.zeros((0, 3)), np.eye(3), np.ones(3, bool), 1.0)
    assert P.shape == (0, 2) and S.shape == (0, 3) and d.shape == (0,)
    cfg = dict(positions=np.zeros((0, 3)), cell=np.zeros((2, 3, 3)),
               pbc=np.zeros((2, 3), bool), batch_ptr=np.array([0, 0, 0], np.int64))
    P, = neighbor_list("P", cfg["positions"], cfg["cell"], cfg["pbc"], 2.0, cfg["batch_ptr"])
    assert P.shape == (0, 2)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_quantities_follow_the_definitions(dtype):
    cfg = W.c2(n_structures=12)
    pos = cfg["positions"].astype(dtype)
    cell = cfg["cell"].astype(dtype)
    i, j, P, S, d, D = neighbor_list("ijPSdD", pos, cell, cfg["pbc"], cfg["cutoff"],
                                     cfg["batch_ptr"], cpu_threads=4)
    assert i.dtype == j.dtype == np.int64 and S.dtype == np.int32
    assert d.dtype == D.dtype == dtype
    assert np.array_equal(i, P[:, 0]) and np.array_equal(j, P[:, 1])
    b = np.searchsorted(cfg["batch_ptr"][1:], i, side="right")
    ref = (pos[j].astype(np.float64) - pos[i] +
           np.einsum("ei,eij->ej", S.astype(np.float64), cell[b].astype(np.float64)))
    tol = 1e-5 if dtype == np.float32 else 1e-12
    scale = np.abs(ref) + cfg["cutoff"]
    assert np.all(np.abs(D - ref) <= tol * scale)
    assert np.all(np.abs(d - np.linalg.norm(ref, axis=1)) <= tol * (np.linalg.norm(ref, axis=1) + cfg["cutoff"]))
    assert np.all(d < cfg["cutoff"])


def test_torch_cpu_tensors_match_numpy_and_carry_gradients():
    cfg = W.c1()
    t = {k: torch.as_tensor(cfg[k]) for k in ("positions", "cell", "pbc", "batch_ptr")}
    Pn, Sn, dn = neighbor_list("PSd", cfg["positions"], cfg["cell"], cfg["pbc"], cfg["cutoff"],
                               cfg["batch_ptr"], cpu_threads=2)
    pos = t["positions"].clone().requires_grad_()
    cell = t["cell"].clone().requires_grad_()
    P, S, d, D = neighbor_list("PSdD", pos, cell, t["pbc"], cfg["cutoff"], t["batch_ptr"],
                               cpu_threads=2)
    assert P.device.type == "cpu" and P.dtype == torch.int64 and S.dtype == torch.int32
    assert np.array_equal(P.numpy(), Pn) and np.array_equal(S.numpy(), Sn)
    assert np.allclose(d.detach().numpy(), dn, rtol=1e-12, atol=1e-12)
    # gradients: the reference's differentiable Torch expression
    (d.sum() + (D * D).sum()).backward()
    gp, gc = pos.grad.clone(), cell.grad.clone()
    pos2 = t["positions"].clone().requires_grad_()
    cell2 = t["cell"].clone().requires_grad_()
    i, j = P[:, 0], P[:, 1]
    D2 = pos2[j] - pos2[i] + S.to(pos2.dtype) @ cell2[0]
    (torch.linalg.vector_norm(D2, dim=1).sum() + (D2 * D2).sum()).backward()
    assert torch.allclose(gp, pos2.grad, rtol=1e-12, atol=1e-12)
    assert torch.allclose(gc, cell2.grad, rtol=1e-12, atol=1e-9)


def test_torch_cpu_finite_difference_gradient():
    rng = np.random.default_rng(5)
    pos = torch.tensor(rng.uniform(0, 6, size=(12, 3)), dtype=torch.float64, requires_grad=True)
    cell = torch.tensor(6.0 * np.eye(3), dtype=torch.float64)
    pbc = torch.tensor([True, True, False])

    def energy(p):
        d, = neighbor_list("d", p, cell, pbc, 2.5)
        return (d ** 2 * torch.exp(-d)).sum()

    assert torch.autograd.gradcheck(energy, (pos,), eps=1e-6, atol=1e-6)


LAYOUT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "layout_limit.json")))


@pytest.mark.parametrize("case", LAYOUT, ids=lambda c: f"{c['kind']}-{c['dtype']}-{c['L']}")
def test_cell_list_refusal_matches_the_reference_to_the_ulp(case):
    # the reference core's outcome for an explicit cell_list at its bin
    # layout limit (tests/golden/make_layout_golden.py): the last accepted
    # length and three ulps either side
    from tests.golden.make_layout_golden import shape

    cfg = shape(case["kind"], float.fromhex(case["L"]), np.dtype(case["dtype"]))
    args = ("PS", cfg["positions"], cfg["cell"], cfg["pbc"], cfg["cutoff"], cfg["batch_ptr"])
    if case["pairs"] is None:
        with pytest.raises(RuntimeError, match="cell_list cannot safely process this structure"):
            neighbor_list(*args, algorithm="cell_list", cpu_threads=2)
    else:
        P, _ = neighbor_list(*args, algorithm="cell_list", cpu_threads=2)
        assert len(P) == case["pairs"]


def test_shift_range_message_is_the_cpu_paths():
    # neighbors_cpu.cpp:266 words it for the cutoff pairs
    with pytest.raises(RuntimeError, match="^a cell shift required by the cutoff pairs exceeds "
                                           "the int32 output range$"):
        neighbor_list("PS", *_single([[-(2**31) + 0.1, 0, 0], [2**31 - 0.8, 0, 0]], np.eye(3),
                                     [1, 0, 0], 0.5))


def test_worker_pool_survives_thread_start_failure():
    # In a child process whose address space leaves room for only a few
    # thread stacks, a search asking for 64 threads runs on the workers it
    # could start (or reports a clean error), never aborting the process;
    # the same process then searches again.
    import subprocess
    import sys
    import textwrap

    code = textwrap.dedent("""
        import resource, sys
        import numpy as np
        sys.path.insert(0, %r)
        from tonari_amd import neighbor_list
        from tonari_amd import workloads as W
        cfg = W.c4(seed=71, n_atoms=3000)
        args = ("PS", cfg["positions"], cfg["cell"], cfg["pbc"], cfg["cutoff"], cfg["batch_ptr"])
        P1, S1 = neighbor_list(*args, cpu_threads=1)
        with open("/proc/self/statm") as fh:
            vm = int(fh.read().split()[0]) * resource.getpagesize()
        resource.setrlimit(resource.RLIMIT_AS, (vm + (40 << 20), resource.RLIM_INFINITY))
        for attempt in range(2):
            try:
                P, S = neighbor_list(*args, cpu_threads=64)
            except RuntimeError as error:
                print("error:", error)
                continue
            assert np.array_equal(P, P1) and np.array_equal(S, S1)
            print("equal")
    """) % os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    # one malloc arena: a thread that cannot have its own fails to start
    # instead of aborting in the C library
    env = dict(os.environ, MALLOC_ARENA_MAX="1")
    run = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300,
                         env=env)
    assert run.returncode == 0, run.stderr[-2000:]
    lines = run.stdout.split()
    assert "equal" in lines or "error:" in lines, run.stdout
