"""GPU: the reference's refusal of an explicit cell_list, to the ulp.

The reference's CPU path refuses an explicit cell_list ("cell_list cannot
safely process this structure") when its dense bin layout, built with a
search cutoff padded in long double, would exceed 2^26 bins or 64 bins per
atom image (``csrc/core/neighbors_cpu.cpp:157-218,379-430``).  Every case of
``tests/golden/layout_limit.json``, written from the reference's compiled
core by ``tests/golden/make_layout_golden.py`` (non-periodic lines, a slab
periodic in x and y whose padding comes from wrapped atoms and images, and a
sparse periodic box, each at the last length the reference accepts and three
ulps either side), runs through the device: as one structure (the
single-structure prologue), as a batch of two copies (the batched planner),
and, for the periodic box, under plan hint 10 (the periodic fast prologue)
through the C ABI.  A refused case must raise the reference's message; an
accepted one must give the reference's pair count.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from tests.golden.make_layout_golden import shape
from tests.test_gpu_periodic_prologue import search
from tonari_amd import neighbor_list
from tonari_amd._extensions import TNR_OK, TNR_RETRY

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
LAYOUT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "layout_limit.json")))
MESSAGE = "cell_list cannot safely process this structure"


def tensors(cfg):
    return [torch.as_tensor(cfg[k]).to(DEV) for k in ("positions", "cell", "pbc")] + \
        [cfg["cutoff"], torch.as_tensor(cfg["batch_ptr"]).to(DEV)]


def twice(cfg):
    n = len(cfg["positions"])
    return dict(cfg, positions=np.concatenate([cfg["positions"]] * 2),
                cell=np.concatenate([cfg["cell"]] * 2), pbc=np.concatenate([cfg["pbc"]] * 2),
                batch_ptr=np.array([0, n, 2 * n], dtype=np.int64))


def expect(cfg, pairs):
    args = tensors(cfg)
    if pairs is None:
        with pytest.raises(RuntimeError, match=MESSAGE):
            neighbor_list("PS", *args, algorithm="cell_list")
    else:
        P, _ = neighbor_list("PS", *args, algorithm="cell_list")
        assert len(P) == pairs


@pytest.mark.parametrize("kind", sorted({c["kind"] for c in LAYOUT}))
def test_refusal_matches_the_reference_to_the_ulp(kind):
    for case in (c for c in LAYOUT if c["kind"] == kind):
        L = float.fromhex(case["L"])
        print(f"[layout] {kind} {case['dtype']} L={L!r} reference={case['pairs']}", flush=True)
        cfg = shape(kind, L, np.dtype(case["dtype"]))
        expect(cfg, case["pairs"])
        expect(twice(cfg), None if case["pairs"] is None else 2 * case["pairs"])
        if kind == "box":
            full = dict(cfg, half_list=False, include_self=False)
            code, msg, plan, P, S, D = search(full, 10, algorithm="cell_list")
            assert code != TNR_RETRY, msg
            if case["pairs"] is None:
                assert code != TNR_OK and MESSAGE in msg, (code, msg)
            else:
                assert code == TNR_OK and len(P) == case["pairs"], (code, msg)
