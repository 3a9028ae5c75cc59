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


# ---------------------------------------------------------------------------
# The three kernels as autograd Functions, and patch() (triton_bwd.py:154-346)
# ---------------------------------------------------------------------------

def _fn_grads(fn, inputs, w):
    xs = [t.detach().clone().requires_grad_(True) for t in inputs]
    out = fn(*xs)
    (out * w.to(out.dtype)).sum().backward()
    return out.detach(), [x.grad.detach() for x in xs]


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_chunk_local_function_gradients(dt):
    from smat_attention_amd.kernels import hip_bwd as Bw
    _say("chunk_local autograd Function", dt)
    g = torch.Generator().manual_seed(21)
    nb, nc, C, r, p = 2, 3, 64, 32, 33
    Phi = (torch.rand(nb, nc, C, r, generator=g) + 0.5).to(dt)
    Psi = (torch.rand(nb, nc, C, r, generator=g) + 0.5).to(dt)
    Vb = torch.randn(nb, nc, C, p, generator=g).to(dt)
    Sin = torch.randn(nb, nc, r, p, generator=g)
    w = torch.randn(nb, nc, C, p, generator=g)
    _, got = _fn_grads(Bw.chunk_local, [t.to(DEV) for t in (Phi, Psi, Vb, Sin)], w.to(DEV))
    _, ref = _fn_grads(lambda a, b, c, d: O.chunk_local(a, b, c, d, acc=torch.float64),
                       [t.double() for t in (Phi, Psi, Vb, Sin)], w.double())
    tol = 1e-5 if dt == torch.float32 else 2e-2
    for name, a, b in zip(("dPhi", "dPsi", "dVb", "dSin"), got, ref):
        assert a.dtype == (dt if name != "dSin" else torch.float32)
        err = _rel(a.cpu(), b) if dt == torch.float32 else _nrel(a.cpu(), b)
        assert err < tol, (name, err)


@pytest.mark.parametrize("T,d,n_P", [(2048, 3, 0), (2048, 3, 16), (2000, 2, 0), (4096, 4, 0)])
def test_pool_and_incidence_function_gradients(T, d, n_P):
    from smat_attention_amd.kernels import hip_bwd as Bw
    _say("pool / incidence autograd Functions", T, d, n_P)
    spec = A.to_device(build_mask(T, d, chunk=128, n_P=n_P), DEV)
    g = torch.Generator().manual_seed(22)
    nb, r, p = 2, 32, 33
    Psi = torch.rand(nb, T, r, generator=g) + 0.5
    Vb = torch.randn(nb, T, p, generator=g)
    wF = torch.randn(nb, spec.N0, r, p, generator=g)
    _, got = _fn_grads(lambda a, b: Bw.pool(a, b, spec.n_P, spec.n, spec.N0),
                       [Psi.to(DEV), Vb.to(DEV)], wF.to(DEV))
    _, ref = _fn_grads(lambda a, b: O.pool_profiles(a, b, spec, acc_dtype=torch.float64),
                       [Psi.double(), Vb.double()], wF.double())
    for name, a, b in zip(("dPsi", "dVb"), got, ref):
        assert _rel(a.cpu(), b) < 1e-5, (name, _rel(a.cpu(), b))
    if not spec.uniform_deg:
        return
    F = torch.randn(nb, spec.N0, r, p, generator=g)
    wU = torch.randn(nb, spec.B, r, p, generator=g)
    _, got = _fn_grads(lambda f: Bw.incidence(f, spec.plane_pts_t, spec.B), [F.to(DEV)],
                       wU.to(DEV))
    _, ref = _fn_grads(lambda f: O.apply_incidence(f, spec), [F.double()], wU.double())
    assert _rel(got[0].cpu(), ref[0]) < 1e-6


def test_patch_makes_the_kernel_table_differentiable():
    from smat_attention_amd.kernels import hip_bwd as Bw
    from smat_attention_amd.kernels import hip_fwd as K
    _say("patch()/unpatch() on the kernel table")
    spec = A.to_device(build_mask(1024, 3, chunk=128), DEV)
    Psi = (torch.rand(1, 1024, 16, device=DEV) + 0.5).requires_grad_(True)
    Vb = torch.randn(1, 1024, 17, device=DEV).requires_grad_(True)
    assert not K.pool(Psi, Vb, spec.n_P, spec.n, spec.N0).requires_grad
    Bw.patch()
    try:
        F = K.pool(Psi, Vb, spec.n_P, spec.n, spec.N0)
        assert F.requires_grad
        F.sum().backward()
        assert Psi.grad is not None and torch.isfinite(Psi.grad).all()
    finally:
        Bw.unpatch()
    assert not K.pool(Psi, Vb, spec.n_P, spec.n, spec.N0).requires_grad
