"""GPU: gradients of d and D through the fused backward kernel.

The reference's d/D are a Torch expression of positions and cell
(src/tonari/_torch_frontend.py:92-104), so autograd reaches both.  Here the
emitting kernel writes d and D, and tnr_geometry_backward computes the
gradient of that same expression.  Each case compares the gradients with
autograd of the expression evaluated in float64 on the CPU over the same
pairs (P, S): within 1e-10 relative for float64 and 1e-4 for float32, whose
float atomics sum in a varying order.  A graph of the gradient
(create_graph) takes the Torch expression, so second derivatives exist.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tonari_amd import neighbor_list
from tonari_amd import workloads as W

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def reference_grads(positions, cell, batch_ptr, P, S, wD, wd):
    """d/dpositions and d/dcell of sum(wD * D) + sum(wd * d), float64 on the CPU."""
    pos = positions.detach().double().cpu().requires_grad_()
    cel = cell.detach().double().cpu().requires_grad_()
    P = P.cpu()
    S = S.cpu()
    b = torch.bucketize(P[:, 0].contiguous(), batch_ptr.cpu()[1:], right=True)
    D = pos[P[:, 1]] - pos[P[:, 0]] + torch.einsum("ei,eij->ej", S.double(), cel[b])
    loss = torch.zeros((), dtype=torch.float64)
    if wD is not None:
        loss = loss + (wD.double().cpu() * D).sum()
    if wd is not None:
        loss = loss + (wd.double().cpu() * torch.linalg.vector_norm(D, dim=1)).sum()
    return torch.autograd.grad(loss, (pos, cel))


def fused_grads(cfg, quantities, dtype, seed, **kw):
    g = torch.Generator().manual_seed(seed)
    positions = torch.as_tensor(cfg["positions"]).to(DEV, dtype).requires_grad_()
    cell = torch.as_tensor(cfg["cell"]).to(DEV, dtype).requires_grad_()
    pbc = torch.as_tensor(cfg["pbc"]).to(DEV)
    batch_ptr = torch.as_tensor(cfg["batch_ptr"]).to(DEV)
    out = neighbor_list(
        "PS" + quantities, positions, cell, pbc, cfg["cutoff"], batch_ptr,
        algorithm=kw.pop("algorithm", "auto"), **kw,
    )
    P, S = out[0], out[1]
    values = dict(zip(quantities, out[2:]))
    E = P.shape[0]
    wD = torch.randn(E, 3, generator=g, dtype=torch.float64).to(DEV, dtype) if "D" in values else None
    wd = torch.randn(E, generator=g, dtype=torch.float64).to(DEV, dtype) if "d" in values else None
    loss = torch.zeros((), dtype=dtype, device=DEV)
    if wD is not None:
        loss = loss + (wD * values["D"]).sum()
    if wd is not None:
        loss = loss + (wd * values["d"]).sum()
    gp, gc = torch.autograd.grad(loss, (positions, cell))
    torch.cuda.synchronize()
    return (gp, gc), reference_grads(positions, cell, batch_ptr, P, S, wD, wd)


def assert_close(actual, expected, dtype):
    tol = 1e-10 if dtype == torch.float64 else 1e-4
    a = actual.detach().double().cpu()
    expected = expected.detach()
    scale = max(1.0, float(expected.abs().max()))
    err = float((a - expected).abs().max())
    assert err <= tol * scale, f"max error {err:.3e} over scale {scale:.3e}"


def small_box(seed=7, n=300, edge=14.0, cutoff=4.5):
    rng = np.random.default_rng(seed)
    cell = W.triclinic_cell((edge, edge * 1.1, edge * 0.9), (80.0, 95.0, 105.0))
    frac = rng.random((n, 3))
    # a few atoms outside the cell, so wraps and shifts are nonzero
    frac[: n // 10] += rng.integers(-2, 3, size=(n // 10, 3))
    return {
        "positions": frac @ cell,
        "cell": cell[None],
        "pbc": np.array([[True, True, True]]),
        "batch_ptr": np.array([0, n], dtype=np.int64),
        "cutoff": cutoff,
    }


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("quantities", ["dD", "D", "d"])
@pytest.mark.parametrize("algorithm", ["cell_list", "brute_force"])
def test_single_structure(dtype, quantities, algorithm):
    cfg = small_box()
    (gp, gc), (rp, rc) = fused_grads(cfg, quantities, dtype, 11, algorithm=algorithm)
    assert_close(gp, rp, dtype)
    assert_close(gc, rc, dtype)


@pytest.mark.parametrize("half_list,include_self", [(False, True), (True, False), (True, True)])
def test_pair_modes(half_list, include_self):
    # include_self adds (i, i, 0) pairs with d = 0, whose d-gradient is 0
    cfg = small_box(seed=3, n=200)
    for dtype in (torch.float64, torch.float32):
        (gp, gc), (rp, rc) = fused_grads(
            cfg, "dD", dtype, 5, half_list=half_list, include_self=include_self
        )
        assert_close(gp, rp, dtype)
        assert_close(gc, rc, dtype)


@pytest.mark.parametrize("sorted_", [False, True])
def test_batches(sorted_):
    # small periodic crystals (brute force) and an unsorted cell-list batch
    for cfg, algorithm in ((W.c2(n_structures=24), "brute_force"),
                           (W.c5(n_structures=3, n_min=600, n_max=900), "cell_list")):
        for dtype in (torch.float64, torch.float32):
            (gp, gc), (rp, rc) = fused_grads(cfg, "dD", dtype, 9, algorithm=algorithm,
                                             sorted=sorted_)
            assert_close(gp, rp, dtype)
            assert_close(gc, rc, dtype)


def test_known_answer_two_atoms():
    # the reference's autograd test (tests/test_quantities.py:97-115): two atoms
    # 0.8 apart in a non-periodic cell; d = 0.8 for both directed pairs, so
    # d(sum d + sum D)/dpositions = (-2, 0, 0) and (2, 0, 0) from d, D cancels
    positions = torch.tensor([[0.0, 0.0, 0.0], [0.8, 0.0, 0.0]], dtype=torch.float64,
                             device=DEV, requires_grad=True)
    cell = (torch.eye(3, dtype=torch.float64, device=DEV) * 4.0).requires_grad_()
    pbc = torch.zeros(3, dtype=torch.bool, device=DEV)
    distances, displacements = neighbor_list("dD", positions, cell, pbc, 1.0)
    (distances.sum() + displacements.sum()).backward()
    expected = torch.tensor([[-2.0, 0.0, 0.0], [2.0, 0.0, 0.0]], dtype=torch.float64)
    assert torch.allclose(positions.grad.cpu(), expected, rtol=0, atol=1e-15)
    assert cell.grad is not None and float(cell.grad.abs().max()) == 0.0


def test_second_derivatives():
    cfg = small_box(seed=13, n=120)
    positions = torch.as_tensor(cfg["positions"]).to(DEV, torch.float64).requires_grad_()
    cell = torch.as_tensor(cfg["cell"]).to(DEV, torch.float64)
    pbc = torch.as_tensor(cfg["pbc"]).to(DEV)
    batch_ptr = torch.as_tensor(cfg["batch_ptr"]).to(DEV)
    P, S, d = neighbor_list("PSd", positions, cell, pbc, cfg["cutoff"], batch_ptr)
    energy = (d ** 2).sum() + torch.cos(d).sum()
    (forces,) = torch.autograd.grad(energy, positions, create_graph=True)
    (hess_vec,) = torch.autograd.grad((forces ** 2).sum(), positions)
    # the same through the Torch expression on the CPU
    pos = positions.detach().cpu().requires_grad_()
    D = pos[P[:, 1].cpu()] - pos[P[:, 0].cpu()] + S.cpu().double() @ cell.cpu()[0]
    dd = torch.linalg.vector_norm(D, dim=1)
    e_ref = (dd ** 2).sum() + torch.cos(dd).sum()
    (f_ref,) = torch.autograd.grad(e_ref, pos, create_graph=True)
    (h_ref,) = torch.autograd.grad((f_ref ** 2).sum(), pos)
    assert_close(forces, f_ref, torch.float64)
    assert_close(hess_vec, h_ref, torch.float64)


def test_edge_cases():
    # no pairs: zero gradients, no kernel work
    positions = torch.tensor([[0.0, 0.0, 0.0], [3.0, 0.0, 0.0]], dtype=torch.float64, device=DEV,
                             requires_grad=True)
    cell = (torch.eye(3, dtype=torch.float64, device=DEV) * 10.0).requires_grad_()
    pbc = torch.zeros(3, dtype=torch.bool, device=DEV)
    d, D = neighbor_list("dD", positions, cell, pbc, 1.0)
    assert d.shape == (0,) and D.shape == (0, 3)
    gp, gc = torch.autograd.grad(d.sum() + D.sum(), (positions, cell))
    assert float(gp.abs().max()) == 0.0 and float(gc.abs().max()) == 0.0

    # only the cell requires grad, positions given as a non-contiguous view
    cfg = small_box(seed=21, n=150)
    base = torch.as_tensor(cfg["positions"].T.copy()).to(DEV, torch.float64)
    positions = base.T  # (N, 3) view with strides (1, N)
    assert not positions.is_contiguous()
    cell = torch.as_tensor(cfg["cell"]).to(DEV, torch.float64).requires_grad_()
    pbc = torch.as_tensor(cfg["pbc"]).to(DEV)
    batch_ptr = torch.as_tensor(cfg["batch_ptr"]).to(DEV)
    P, S, D = neighbor_list("PSD", positions, cell, pbc, cfg["cutoff"], batch_ptr)
    w = torch.randn(D.shape, dtype=torch.float64, generator=torch.Generator().manual_seed(3)).to(DEV)
    (gc,) = torch.autograd.grad((w * D).sum(), cell)
    _, rc = reference_grads(positions, cell, batch_ptr, P, S, w, None)
    assert_close(gc, rc, torch.float64)
