"""GPU: gradients of d and D on seeded random batches.

The batches of ``tests/test_random_batches.py`` (triclinic and open
structures, random periodicity, wrapped atoms, either dtype, any algorithm
and pair mode; explicit cell_list requests the oracle refuses left out) are
searched with positions and cell requiring grad, and the gradient of a
random weighting of D, of d, or of both goes through the fused backward
(``tnr_geometry_backward``).  Each must match autograd of the reference's
expression D = x[j] - x[i] + S @ cell[b] evaluated in float64 on the CPU
over the same pairs: within 1e-10 relative for float64 and 1e-4 for float32
(whose atomics sum in a varying order), as in ``tests/test_gpu_backward.py``.
The pairs themselves are the oracle's (checked by the other sweeps).
"""

from __future__ import annotations

import pytest
import torch

from tests.test_gpu_backward import assert_close, fused_grads
from tests.test_random_reuse import _usable
from tests.test_random_batches import random_batch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("block", range(4))
def test_random_batch_gradients(block):
    for seed in range(20 * block, 20 * block + 20):
        cfg = random_batch(seed)
        if not _usable(cfg):
            continue
        dtype = torch.float32 if cfg["positions"].dtype.itemsize == 4 else torch.float64
        quantities = ("D", "d", "dD")[seed % 3]
        print(f"[random gradients] seed {seed} {dtype} {cfg['algorithm']} {quantities}",
              flush=True)
        (gp, gc), (rp, rc) = fused_grads(
            cfg, quantities, dtype, seed, algorithm=cfg["algorithm"], sorted=cfg["sorted"],
            half_list=cfg["half_list"], include_self=cfg["include_self"])
        assert_close(gp, rp, dtype)
        assert_close(gc, rc, dtype)
