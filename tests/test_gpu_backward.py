"""Gradients of the HIP schedule vs torch autograd through the CPU oracle.

fp32 inputs: against fp64 autograd of the oracle's restatement on the same
values, max|got - ref| / max|ref| < 1e-5 per gradient (the bar stated for
fp32 gradients).  bf16 inputs (the training configuration, positional
assignment): against the reference torch path in bf16 on the same inputs,
norm-relative error < 2e-2, the reference's own tolerance for its fused
backward (tests/test_triton_bwd.py:24-64).
"""
import pytest
import torch

import oracle.schedule as O
from smat_attention_amd import attention as A
from smat_attention_amd.mask import build_mask

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _say(*a):
    print("[case]", *a, flush=True)


def _feats(nb, T, hd, seed, k_scale=1.0):
    Q, K, V = O.seeded_qkv(nb, T, hd, hd, seed=seed, dtype=torch.float32, k_scale=k_scale,
                           q_scale=0.5)
    phi = O.make_phi(hd, hd, dtype=torch.float32, seed=0)
    return O.featurise(Q, K, V, phi)


def _grads_gpu(spec, Phi, Psi, Vb, w, g=None):
    xs = [t.to(DEV).detach().requires_grad_(True) for t in (Phi, Psi, Vb)]
    gd = g.to(DEV).detach().requires_grad_(True) if g is not None else None
    out = A.smat_attention(*xs, spec, g=gd)
    (out * w.to(DEV)).sum().backward()
    gs = [x.grad.detach().cpu() for x in xs]
    if gd is not None:
        gs.append(gd.grad.detach().cpu())
    return out.detach().cpu(), gs


def _grads_ref(spec, Phi, Psi, Vb, w, g=None, dtype=torch.float64):
    xs = [t.to(dtype).detach().requires_grad_(True) for t in (Phi, Psi, Vb)]
    gd = g.to(dtype).detach().requires_grad_(True) if g is not None else None
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    out = O.smat_attention(*xs, spec, g=gd, acc_dtype=acc)
    (out * w.to(out.dtype)).sum().backward()
    gs = [x.grad.detach() for x in xs]
    if gd is not None:
        gs.append(gd.grad.detach())
    return out.detach(), gs


def _rel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-300)).item()


def _nrel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-300)).item()


@pytest.mark.parametrize("T,d,n_P,hd,gate", [(1024, 2, 0, 32, False), (2048, 3, 0, 32, True),
                                             (2048, 3, 16, 32, False), (2000, 3, 0, 16, False),
                                             (1024, 1, 0, 32, False), (4096, 4, 0, 16, True),
                                             (2048, 3, 0, 64, False)])
def test_backward_fp32_vs_fp64_autograd(T, d, n_P, hd, gate):
    _say("backward fp32", T, d, n_P, hd, gate)
    spec = build_mask(T, d, chunk=128, n_P=n_P)
    Phi, Psi, Vb = _feats(2, T, hd, seed=21)
    gen = torch.Generator().manual_seed(22)
    w = torch.randn(2, T, hd, generator=gen)
    g = torch.rand(2, T, generator=gen) + 0.5 if gate else None
    out, gs = _grads_gpu(spec, Phi, Psi, Vb, w, g)
    ref, rs = _grads_ref(spec, Phi, Psi, Vb, w, g)
    assert _rel(out, ref) < 1e-5
    for name, a, b in zip(("dPhi", "dPsi", "dVb", "dg"), gs, rs):
        e = _rel(a, b)
        _say(f"  {name}: rel {e:.2e}")
        assert e < 1e-5, name


@pytest.mark.parametrize("d", [2, 3])
def test_backward_training_shape_bf16(d):
    """B=8, H=12 (nb=96), head_dim 64, T=4096, bf16, dO ~ N(0,1); heads 0-7
    compared against the reference torch path's autograd on the same inputs."""
    _say("backward bf16 training shape", d)
    T, hd, nb = 4096, 64, 96
    spec = build_mask(T, d, chunk=128)
    Phi, Psi, Vb = (x.to(torch.bfloat16) for x in _feats(nb, T, hd, seed=0, k_scale=hd ** -0.5))
    w = torch.randn(nb, T, hd, generator=torch.Generator().manual_seed(1))
    out, gs = _grads_gpu(spec, Phi, Psi, Vb, w)
    assert all(torch.isfinite(x).all() for x in gs)
    h = 8
    ref, rs = _grads_ref(spec, Phi[:h], Psi[:h], Vb[:h], w[:h], dtype=torch.bfloat16)
    assert (out[:h].double() - ref.double()).abs().max().item() < 2e-2
    for name, a, b in zip(("dPhi", "dPsi", "dVb"), gs, rs):
        e = _nrel(a[:h], b)
        _say(f"  {name}: norm-rel {e:.2e}")
        assert e < 2e-2, name
    # and against fp64 autograd of the same bf16 values
    _, r64 = _grads_ref(spec, Phi[:h], Psi[:h], Vb[:h], w[:h])
    for name, a, b in zip(("dPhi", "dPsi", "dVb"), gs, r64):
        assert _nrel(a[:h], b) < 2e-2, name


def test_forward_unchanged_when_grad_is_recorded():
    _say("forward with and without autograd")
    spec = build_mask(2048, 3, chunk=128)
    Phi, Psi, Vb = _feats(2, 2048, 32, seed=23)
    plain = A.smat_attention(Phi.to(DEV), Psi.to(DEV), Vb.to(DEV), spec)
    xs = [t.to(DEV).requires_grad_(True) for t in (Phi, Psi, Vb)]
    tracked = A.smat_attention(*xs, spec)
    assert tracked.requires_grad
    assert (tracked.detach() - plain).abs().max().item() <= 1e-6 * plain.abs().max().item()
