"""CPU: argument checks of the persistent plan (no GPU needed).

NeighborListPlan validates like the public call (the reference's messages)
before it touches a device, and refuses what run() cannot read in place.
"""

from __future__ import annotations

import pytest
import torch

from tonari_amd.persistent import NeighborListPlan


def args(**over):
    a = dict(quantities="PD", positions=torch.zeros(4, 3), cell=torch.eye(3) * 5.0,
             pbc=torch.tensor([True, True, True]), cutoff=2.0, capacity=100)
    a.update(over)
    return a


def make(**over):
    a = args(**over)
    q = a.pop("quantities")
    return NeighborListPlan(q, a.pop("positions"), a.pop("cell"), a.pop("pbc"), a.pop("cutoff"),
                            **a)


def test_rejects_unsupported_quantities():
    with pytest.raises(ValueError, match="unsupported quantities"):
        make(quantities="PX")
    with pytest.raises(ValueError, match="non-empty"):
        make(quantities="")


def test_validates_like_the_public_call():
    with pytest.raises(ValueError, match="positions must have shape"):
        make(positions=torch.zeros(4, 2))
    with pytest.raises(ValueError, match="cutoff must be finite and positive"):
        make(cutoff=-1.0)


def test_cpu_tensors_are_refused():
    with pytest.raises(RuntimeError, match="ROCm"):
        make()
