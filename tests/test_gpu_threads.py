"""GPU: concurrent Python callers on their own streams, and the loader's device check.

The library keeps no mutable state between calls (each call has its own
workspace; the frontend keeps its pinned status buffer and repeated-call
table per thread), and ctypes releases the GIL during each foreign call, so
calls from several threads overlap on the device.  After the reference's
``tests/backends/test_cpu_threads.py:160-215``: every thread's results must
equal the CPU oracle's.
"""

from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import pytest
import torch

from tests._util import assert_same_keys, keys_of, oracle_call
from tonari_amd import neighbor_list
from tonari_amd import workloads as W

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _cases():
    return {
        "batch": dict(W.c2(n_structures=40), algorithm="auto"),
        "box": W.c4(seed=31, n_atoms=12_000),
        "half": dict(W.c3(n_structures=64), sorted=True),
    }


def _call(cfg, t):
    return neighbor_list(
        "PS", t["positions"], t["cell"], t["pbc"], cfg["cutoff"], t["batch_ptr"],
        algorithm=cfg["algorithm"], half_list=cfg.get("half_list", False),
        include_self=cfg.get("include_self", False), sorted=cfg.get("sorted", False),
    )


def test_concurrent_calls_on_separate_streams():
    cases = _cases()
    expected = {name: keys_of(*oracle_call(cfg)) for name, cfg in cases.items()}
    tensors = {name: {k: torch.as_tensor(cfg[k]).to(DEV)
                      for k in ("positions", "cell", "pbc", "batch_ptr")}
               for name, cfg in cases.items()}
    torch.cuda.synchronize()

    def run(job):
        name, rep = job
        stream = torch.cuda.Stream(device=DEV)  # default priority
        # the inputs were written on the default stream, synchronised above
        with torch.cuda.stream(stream):
            results = []
            for _ in range(rep):
                P, S = _call(cases[name], tensors[name])
                results.append((P, S))
            stream.synchronize()
            return name, [keys_of(P, S) for P, S in results]

    jobs = [(name, 3) for name in cases] * 3
    print(f"[threads] {len(jobs)} jobs on 4 threads", flush=True)
    with ThreadPoolExecutor(max_workers=4) as pool:
        outcomes = list(pool.map(run, jobs))
    for name, keys in outcomes:
        for k in keys:
            assert_same_keys(k, expected[name])


def test_device_check_accepts_this_device_and_names_a_mismatch(monkeypatch):
    from tonari_amd import _extensions as ext

    ext.check_device(0)  # the box's device runs the library's target

    class Fake:
        def tnr_device_arch(self):
            return b"gfx942"

    monkeypatch.setattr(ext, "load_torch_hip", lambda: Fake())
    with pytest.raises(ImportError, match="holds gfx942 code only; device cuda:0 is gfx950"):
        ext.check_device.__wrapped__(0)
