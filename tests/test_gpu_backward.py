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


@pytest.mark.parametrize("T,d,n_P,hd,gate", [(1024, 2, 0, 32, False), (1024, 2, 16, 32, True),
                                             (2048, 3, 0, 32, True),
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


@pytest.mark.parametrize("d,n_P,gate", [(2, 0, False), (2, 16, True), (3, 0, False),
                                          (3, 16, True)])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_backward_head_dim_128(dt, d, n_P, gate):
    """The whole schedule's gradient at head_dim 128 (r = 128, p = 129: a width
    the reference's fused backward refuses, triton_bwd.py:166-167), T = 4096,
    d = 2 and 3, with and without the global channel and the output gate.
    fp32: dPhi, dPsi, dVb and dg within 1e-5 (max-relative) of fp64 autograd
    through the oracle on the same values.  bf16: within the 16-bit bar
    (norm-relative 2e-2) of the reference's torch path's autograd in bf16 on
    the same inputs, and of fp64 autograd on those values."""
    T, hd, nb = 4096, 128, 2
    _say("backward head_dim 128", dt, T, d, n_P, gate)
    spec = build_mask(T, d, chunk=128, n_P=n_P)
    Phi, Psi, Vb = (x.to(dt) for x in _feats(nb, T, hd, seed=31, k_scale=hd ** -0.5))
    gen = torch.Generator().manual_seed(32)
    w = torch.randn(nb, T, hd, generator=gen)
    g = (torch.rand(nb, T, generator=gen) + 0.5) if gate else None
    out, gs = _grads_gpu(spec, Phi, Psi, Vb, w, g)
    names = ("dPhi", "dPsi", "dVb", "dg")
    ref64, r64 = _grads_ref(spec, Phi, Psi, Vb, w, g)
    if dt == torch.float32:
        assert _rel(out, ref64) < 1e-5
        for name, a, b in zip(names, gs, r64):
            e = _rel(a, b)
            _say(f"  {name}: rel vs fp64 {e:.2e}")
            assert e < 1e-5, name
        return
    assert all(torch.isfinite(x).all() for x in gs)
    refbf, rbf = _grads_ref(spec, Phi, Psi, Vb, w, g, dtype=torch.bfloat16)
    assert (out.double() - refbf.double()).abs().max().item() < 2e-2
    for name, a, b, c in zip(names, gs, rbf, r64):
        e, e64 = _nrel(a, b), _nrel(a, c)
        _say(f"  {name}: norm-rel vs bf16 torch path {e:.2e}, vs fp64 {e64:.2e}")
        assert e < 2e-2 and e64 < 2e-2, name


@pytest.mark.parametrize("n_P", [0, 16])
def test_backward_head_dim_128_padded_value_rows(n_P):
    """Vb as the feature map stores it at head_dim 128: rows of 129 values in
    a buffer of 136-element rows, the padding holding NaN.  Every gradient
    equals the one of the same values in dense rows (the pool's and the global
    channel's products must address Vb by its own row stride)."""
    T, hd, nb = 2048, 128, 2
    _say("backward head_dim 128 padded Vb rows", n_P)
    spec = build_mask(T, 3, chunk=128, n_P=n_P)
    Phi, Psi, Vb = (x.to(torch.bfloat16) for x in _feats(nb, T, hd, seed=41, k_scale=hd ** -0.5))
    w = torch.randn(nb, T, hd, generator=torch.Generator().manual_seed(42)).to(DEV)
    buf = torch.full((nb, T, 136), float("nan"), device=DEV, dtype=torch.bfloat16)
    buf[..., :hd + 1] = Vb.to(DEV)
    res = []
    for v in (buf[..., :hd + 1], Vb.to(DEV).contiguous()):
        xs = [Phi.to(DEV).requires_grad_(True), Psi.to(DEV).requires_grad_(True),
              v.detach().requires_grad_(True)]
        (A.smat_attention(*xs, spec) * w).sum().backward()
        res.append([x.grad.float().cpu() for x in xs])
    assert res[0][2].shape == (nb, T, hd + 1)
    for name, a, b in zip(("dPhi", "dPsi", "dVb"), *res):
        assert torch.isfinite(a).all(), name
        assert torch.equal(a, b), name


@pytest.mark.parametrize("T,d,n_P,gate", [(2048, 3, 0, False), (2048, 3, 16, True),
                                          (1024, 2, 0, True)])
def test_parts_and_timer_under_autograd(T, d, n_P, gate):
    """return_parts and timer on a differentiable call (the reference's torch
    path gives both under autograd, attention.py:391-455): the phases run as
    autograd nodes on the HIP kernels, the timer sees lr_pool, lr_incidence,
    lr_query, scan and normalise, the output equals the one-node call's, and the
    gradients of a loss over the output and the parts U and H match fp64
    autograd through the oracle's parts (fp32, 1e-5)."""
    _say("parts and timer under autograd", T, d, n_P, gate)
    spec = build_mask(T, d, chunk=128, n_P=n_P)
    Phi, Psi, Vb = _feats(2, T, 32, seed=41)
    gen = torch.Generator().manual_seed(42)
    w = torch.randn(2, T, 32, generator=gen)
    wH = torch.randn(2, T, 33, generator=gen)
    wU = torch.randn(2, spec.B, 32, 33, generator=gen)
    g = torch.rand(2, T, generator=gen) + 0.5 if gate else None
    seen = []

    class Timer:
        def __init__(self, name):
            seen.append(name)

        def __enter__(self):
            return self

        def __exit__(self, *a):
            return False

    def loss(out, parts, dt):
        return ((out * w.to(out.device, dt)).sum() + (parts["H"] * wH.to(out.device, dt)).sum()
                + (parts["U"] * wU.to(out.device, dt)).sum())

    xs = [t.to(DEV).requires_grad_(True) for t in (Phi, Psi, Vb)]
    gd = g.to(DEV).requires_grad_(True) if gate else None
    out, parts = A.smat_attention(*xs, spec, g=gd, return_parts=True, timer=Timer)
    assert seen == ["lr_pool", "lr_incidence", "lr_query", "scan", "normalise"]
    assert out.requires_grad and parts["H"].requires_grad and parts["U"].requires_grad
    one = A.smat_attention(*xs, spec, g=gd)
    assert _rel(out.detach().cpu(), one.detach().cpu()) < 1e-6
    loss(out, parts, torch.float32).backward()
    got = [x.grad.cpu() for x in xs] + ([gd.grad.cpu()] if gate else [])
    rs = [t.double().requires_grad_(True) for t in (Phi, Psi, Vb)]
    rg = g.double().requires_grad_(True) if gate else None
    ro, rparts = O.smat_attention(*rs, spec, g=rg, acc_dtype=torch.float64, return_parts=True)
    loss(ro, rparts, torch.float64).backward()
    want = [x.grad for x in rs] + ([rg.grad] if gate else [])
    for name, a, b in zip(("dPhi", "dPsi", "dVb", "dg"), got, want):
        e = _rel(a, b)
        _say(f"  {name}: rel vs fp64 {e:.2e}")
        assert e < 1e-5, name


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


def _grel(a, b):
    return ((a.double() - b.double()).abs().max() / b.double().abs().max().clamp_min(1e-30)).item()


@pytest.mark.parametrize("kind", ["elu1", "relu"])
def test_featurise_gradients(kind):
    """featurise on the GPU (HIP forward, the map's derivative backward): every
    gradient -- Q, K, V, the key gate h and W -- against fp64 autograd of the
    oracle's torch map on the same values (the reference differentiates its
    torch featurise, attention.py:82-106)."""
    gen = torch.Generator().manual_seed(31)
    nb, T, dqk, dv, r = 2, 300, 64, 64, 48
    ins = {"Q": torch.randn(nb, T, dqk, generator=gen), "K": torch.randn(nb, T, dqk, generator=gen),
           "V": torch.randn(nb, T, dv, generator=gen),
           "h": torch.rand(nb, T, generator=gen) + 0.5,
           "W": torch.randn(r, dqk, generator=gen) / dqk ** 0.5}
    Rs = [torch.randn(nb, T, r, generator=gen), torch.randn(nb, T, r, generator=gen),
          torch.randn(nb, T, dv + 1, generator=gen)]
    _say("featurise grads", kind)

    def run(dev, dt, feat):
        xs = {k: v.to(dev, dt).requires_grad_(True) for k, v in ins.items()}
        outs = feat(xs)
        sum((o.float() * R_.to(dev)).sum() for o, R_ in zip(outs, Rs)).backward()
        return [o.detach().cpu() for o in outs], {k: v.grad.detach().cpu() for k, v in xs.items()}

    def ref(xs):
        W = xs["W"]
        m = (lambda x: torch.nn.functional.elu(x @ W.T) + 1.0) if kind == "elu1" else \
            (lambda x: torch.nn.functional.relu(x @ W.T) + 1e-3)
        return O.featurise(xs["Q"], xs["K"], xs["V"], m, h=xs["h"])

    def hip(xs):
        return A.featurise(xs["Q"], xs["K"], xs["V"], A.FeatureMap(xs["W"], kind), h=xs["h"])
    o0, g0 = run("cpu", torch.float64, ref)
    o1, g1 = run(DEV, torch.float32, hip)
    for a, b in zip(o1, o0):
        assert _grel(a, b) < 1e-5
    for k in g0:
        assert _grel(g1[k], g0[k]) < 1e-5, (k, _grel(g1[k], g0[k]))
    # the map alone (make_phi's callable) is differentiable too
    xq = ins["Q"].to(DEV).requires_grad_(True)
    A.FeatureMap(ins["W"].to(DEV), kind)(xq).sum().backward()
    assert xq.grad is not None and torch.isfinite(xq.grad).all()


@pytest.mark.parametrize("T,n,C,r,p", [(1024, 512, 128, 16, 17), (1000, 512, 64, 32, 33),
                                       (4096, 2048, 128, 64, 65), (2048, 1024, 256, 16, 17)])
def test_segmented_causal_scan_gradients(T, n, C, r, p):
    """segmented_causal_scan alone as an autograd node (HIP forward and
    backward): dPhi, dPsi, dVb against fp64 autograd of the oracle's scan,
    padded tails and a wide chunk included."""
    gen = torch.Generator().manual_seed(T + C)
    nb = 3
    ins = [torch.rand(nb, T, r, generator=gen) + 0.1, torch.rand(nb, T, r, generator=gen) * 0.1,
           torch.randn(nb, T, p, generator=gen)]
    R_ = torch.randn(nb, T, p, generator=gen)
    _say("scan grads", T, n, C, r, p)

    def run(dev, dt, f):
        xs = [t.to(dev, dt).requires_grad_(True) for t in ins]
        H = f(*xs)
        (H.float() * R_.to(dev)).sum().backward()
        return H.detach().cpu(), [x.grad.detach().cpu() for x in xs]
    h0, g0 = run("cpu", torch.float64, lambda a, b, c: O.segmented_causal_scan(a, b, c, n, C))
    h1, g1 = run(DEV, torch.float32, lambda a, b, c: A.segmented_causal_scan(a, b, c, n, C))
    assert _grel(h1, h0) < 1e-5
    for a, b in zip(g1, g0):
        assert _grel(a, b) < 1e-5


@pytest.mark.parametrize("T,n", [(4096, 2048), (1000, 384), (1024, 1024), (2048, 0)])
def test_fused_chunk_backward(T, n):
    """smat_chunk_backward (bf16 inputs, r = 64, p = 65, C = 128: the training
    shape) against the chain of smat_bgemm products it replaces, and both
    against fp64 autograd of the oracle's scan on the same bf16 values: fp32
    gradients, padded tail chunk and both segment splits included."""
    from smat_attention_amd.kernels import hip_bwd as HB
    C, r, p, nb = 128, 64, 65, 3
    Tp = -(-T // C) * C
    gen = torch.Generator().manual_seed(T + n)
    bf = torch.bfloat16

    def rows(width, make):
        x = torch.zeros(nb, Tp, width)
        x[:, :T] = make((nb, T, width))
        return x
    Ph = rows(r, lambda s: torch.rand(s, generator=gen) + 0.1).to(bf)
    Ps = rows(r, lambda s: torch.rand(s, generator=gen) * 0.1).to(bf)
    Vv = rows(p, lambda s: torch.randn(s, generator=gen)).to(bf)
    dH = rows(p, lambda s: torch.randn(s, generator=gen))
    _say("fused chunk backward", T, n)
    args = [x.to(DEV) for x in (Ph, Ps, Vv, dH)]
    assert HB.fused_chunk_backward_ok(*args[:3], C)
    got = [x.cpu() for x in HB.causal_scan_grad(*args, n, C)]
    try:
        HB.FUSED_CHUNK_BACKWARD = False
        ref = [x.cpu() for x in HB.causal_scan_grad(*args, n, C)]
    finally:
        HB.FUSED_CHUNK_BACKWARD = True
    xs = [x[:, :T].double().requires_grad_(True) for x in (Ph, Ps, Vv)]
    H = O.segmented_causal_scan(*xs, n, C)
    (H * dH[:, :T].double()).sum().backward()
    for name, a, b, x in zip(("dPhi", "dPsi", "dVb"), got, ref, xs):
        e_chain, e_64 = _grel(a, b), _grel(a[:, :T], x.grad)
        _say(f"  {name}: vs bgemm {e_chain:.2e}, vs fp64 {e_64:.2e}")
        assert e_chain < 1e-4 and e_64 < 1e-4, name
        assert torch.isfinite(a).all()
    # gradients stored in bf16 by the kernel: the fp32 ones rounded to nearest
    # even, bit for bit (the same accumulators, only the store differs)
    g16 = [x.cpu() for x in HB.causal_scan_grad(*args, n, C, out_dtype=bf)]
    for name, a, b in zip(("dPhi", "dPsi", "dVb"), g16, got):
        assert a.dtype == bf and torch.equal(a, b.to(bf)), name


@pytest.mark.parametrize("vb_pad", [False, True])
def test_chunk_state_gradients(vb_pad):
    """smat_chunk_dstates: Dr_c = Phi_c^T dH_c for every (sequence, chunk), bf16
    Phi and fp32 dH (contiguous rows of 65 floats, or rows 72 apart), against
    fp64 products of the same values: within 2e-5 of each matrix's largest
    entry (dH enters split hi/lo, about 2^-17 relative)."""
    from smat_attention_amd.kernels.hip_fwd import call, stream_of
    nb, nc, r, p, C = 3, 5, 64, 65, 128
    gen = torch.Generator().manual_seed(93)
    Ph = (torch.rand(nb, nc * C, r, generator=gen) + 0.1).to(torch.bfloat16)
    dH = torch.randn(nb, nc * C, 72 if vb_pad else p, generator=gen)[..., :p]
    Phd, dHd = Ph.to(DEV), dH.to(DEV)
    Dr = torch.empty(nb, nc, r, p, device=DEV)
    call("smat_chunk_dstates", 0, Phd.data_ptr(), dHd.data_ptr(), Dr.data_ptr(), nb, nc, r, p, C,
         Phd.stride(0), Phd.stride(1), dHd.stride(0), dHd.stride(1), stream_of(Dr))
    ref = torch.einsum("bcta,bctv->bcav", Ph.double().reshape(nb, nc, C, r),
                       dH.double().reshape(nb, nc, C, p))
    err = ((Dr.cpu().double() - ref).abs().amax((-1, -2)) / ref.abs().amax((-1, -2))).max()
    _say("chunk state gradients", vb_pad, f"{float(err):.2e}")
    assert float(err) < 2e-5


@pytest.mark.parametrize("T,d,n_P,gate", [(4096, 3, 0, False), (4096, 2, 0, False),
                                          (2048, 3, 16, True), (3000, 3, 0, False)])
def test_fused_attention_backward(T, d, n_P, gate):
    """The whole gradient of smat_attention with bf16 inputs at head_dim 64 --
    the fused chunk backward and the long-range kernels (smat_lr_dphi,
    smat_lr_dfeat, smat_pool_backward) -- against the smat_bgemm products they
    replace (max-relative < 1e-4: the kernels' hi/lo products), and against
    fp64 autograd of the oracle on the same bf16 values at the bf16 bar
    (norm-relative < 2e-2: the forward rounds the within-chunk scores to the
    input dtype, as the reference does, and the fp64 oracle does not).  fp32
    gradients, before the cast to the input dtype."""
    from smat_attention_amd.kernels import hip_bwd as HB
    spec = build_mask(T, d, chunk=128, n_P=n_P)
    nb = 2
    Phi, Psi, Vb = (x.to(torch.bfloat16) for x in _feats(nb, T, 64, seed=5, k_scale=0.125))
    gen = torch.Generator().manual_seed(6)
    w = torch.randn(nb, T, 64, generator=gen)
    g = torch.rand(nb, T, generator=gen) + 0.5 if gate else None
    _say("fused attention backward", T, d, n_P, gate)
    xs = [x.to(DEV) for x in (Phi, Psi, Vb)]
    gd = g.to(DEV) if g is not None else None
    assert HB.long_range_backward_ok(*xs) and HB.fused_chunk_backward_ok(*xs, 128)
    out, parts = A.smat_attention(*xs, spec, g=gd, return_parts=True, _no_grad_fn=True)
    dout = w.to(DEV)

    def grads():
        return [y.cpu() for y in HB.smat_attention_grad(*xs, spec, parts["U"], parts["H"], dout,
                                                        g=gd)[:3]]
    got = grads()
    try:
        HB.FUSED_LONG_RANGE_BACKWARD = HB.FUSED_CHUNK_BACKWARD = False
        ref = grads()
    finally:
        HB.FUSED_LONG_RANGE_BACKWARD = HB.FUSED_CHUNK_BACKWARD = True
    _, r64 = _grads_ref(spec, Phi, Psi, Vb, w, g)
    for name, a, b, c in zip(("dPhi", "dPsi", "dVb"), got, ref, r64):
        e_chain, e_64 = _grel(a, b), _nrel(a, c)
        _say(f"  {name}: vs bgemm {e_chain:.2e}, vs fp64 (norm) {e_64:.2e}")
        assert torch.isfinite(a).all()
        assert e_chain < 1e-4 and e_64 < 2e-2, name
    # gradients in bf16: the long-range terms stored first and added by the
    # chunk backward form the same fp32 sums as the fp32 path, rounded once
    g16 = [y.cpu() for y in HB.smat_attention_grad(*xs, spec, parts["U"], parts["H"], dout,
                                                   g=gd, out_dtype=torch.bfloat16)[:3]]
    for name, a, b in zip(("dPhi", "dPsi", "dVb"), g16, got):
        assert a.dtype == torch.bfloat16 and torch.equal(a, b.to(torch.bfloat16)), name


@pytest.mark.parametrize("d", [2, 3])
def test_fused_cell_backward(d):
    """ContentAssign's hard point read and pool at head_dim 64, bf16: the fused
    backward kernels (smat_cell_read_backward, smat_cell_pool_backward) against
    the list reads and pair sums they replace, same forward.  The hash
    parameters' gradients (through every pair's weight gradient) within 1e-4;
    dQ, dK, dV, cast to bf16 by autograd, within 2e-3 norm-relative."""
    from smat_attention_amd import assign as AS
    B, H, hd, T = 2, 4, 64, 2048
    spec = build_mask(T, d, chunk=128)
    n = spec.n
    gen = torch.Generator().manual_seed(70 + d)
    bf = torch.bfloat16
    Q = torch.randn(B * H, T, hd, generator=gen).to(bf)
    K = (torch.randn(B * H, T, hd, generator=gen) / hd ** 0.5).to(bf)
    V = torch.randn(B * H, T, hd, generator=gen).to(bf)
    dY = torch.randn(B * H, T - n, hd + 1, generator=gen).to(DEV)
    torch.manual_seed(7)
    m = AS.ContentAssign(H, H * hd, spec, mode="point").to(DEV)
    phi = A.make_phi(hd, hd, device=DEV, dtype=bf, seed=0)
    _say("fused cell backward", d, spec.N0)

    def run(fused):
        AS.FUSED_CELL_BACKWARD = fused
        try:
            xs = [t.to(DEV).requires_grad_(True) for t in (Q, K, V)]
            Phi, Psi, Vb = A.featurise(*xs, phi)
            u = xs[1].reshape(B, H, T, hd).transpose(1, 2).reshape(B, T, H * hd).float()
            m.zero_grad()
            Y = m(u, Phi, Psi, Vb, n)
            (Y * dY).sum().backward()
            return ([x.grad.float().cpu() for x in xs]
                    + [getattr(m, k).grad.detach().cpu() for k in ("W", "gamma", "b")])
        finally:
            AS.FUSED_CELL_BACKWARD = True
    g1, g0 = run(True), run(False)
    for name, a, b in zip(("dQ", "dK", "dV", "dW", "dgamma", "db"), g1, g0):
        e = _nrel(a, b) if name in ("dQ", "dK", "dV") else _grel(a, b)
        _say(f"  {name}: {e:.2e}")
        assert torch.isfinite(a).all()
        assert e < (2e-3 if name in ("dQ", "dK", "dV") else 1e-4), name


def test_cell_backward_16bit_outputs_are_rounded_fp32():
    """smat_cell_read_backward and smat_cell_pool_backward with out_dtype bf16
    store the fp32 results rounded to nearest even, bit for bit, into rows of
    larger tensors (the key rows [0, n) and query rows [n, T) of (nb, T, .)
    gradients) and write every row a pair-0 entry names: the buffers start as
    NaN, and the rows outside are left untouched."""
    from smat_attention_amd import assign as AS
    from smat_attention_amd.kernels.hip_fwd import call, stream_of
    nb, T, n, N0, K, r, p = 3, 1500, 700, 37, 4, 64, 65
    gen = torch.Generator().manual_seed(91)
    bf = torch.bfloat16
    X = (torch.rand(nb, T, r, generator=gen) + 0.1).to(bf).to(DEV)      # Phi / Psi
    Vb = torch.randn(nb, T, p, generator=gen).to(bf).to(DEV)
    dY = torch.randn(nb, T - n, p, generator=gen).to(DEV)
    F = torch.randn(nb, N0, r, p, generator=gen).to(DEV)
    idx = torch.randint(0, N0, (nb, T - n, K), generator=gen).to(DEV)
    idk = torch.randint(0, N0, (nb, n, K), generator=gen).to(DEV)

    def read(out_dt):
        ent, eoffs = AS._entry_lists(idx, N0)
        dX = torch.full((nb, T, r), float("nan"), device=DEV, dtype=out_dt)
        dF = torch.empty(nb, N0, r, p, device=DEV)
        dw = torch.empty(nb, T - n, K, device=DEV)
        Xr, dXr = X[:, n:], dX[:, n:]
        call("smat_cell_read_backward", 0, AS._code(dXr, "t"), Xr.data_ptr(), dY.data_ptr(),
             F.data_ptr(), ent.data_ptr(), eoffs.data_ptr(), dXr.data_ptr(), dF.data_ptr(),
             dw.data_ptr(), nb, N0, K, T - n, r, p, Xr.stride(0), Xr.stride(1), dY.stride(0),
             dY.stride(1), F.stride(0), dXr.stride(0), dXr.stride(1), dw.stride(0),
             stream_of(F))
        return dX.cpu(), dF.cpu(), dw.cpu()

    def pool(out_dt):
        ent, eoffs = AS._entry_lists(idk, N0)
        dX = torch.full((nb, T, r), float("nan"), device=DEV, dtype=out_dt)
        dV = torch.full((nb, T, p), float("nan"), device=DEV, dtype=out_dt)
        dw = torch.empty(nb, n, K, device=DEV)
        call("smat_cell_pool_backward", 0, AS._code(dX, "t"), X.data_ptr(), Vb.data_ptr(),
             F.data_ptr(), ent.data_ptr(), eoffs.data_ptr(), dX.data_ptr(), dV.data_ptr(),
             dw.data_ptr(), nb, N0, K, n, r, p, X.stride(0), X.stride(1), Vb.stride(0),
             Vb.stride(1), F.stride(0), dX.stride(0), dX.stride(1), dV.stride(0), dV.stride(1),
             dw.stride(0), stream_of(F))
        return dX.cpu(), dV.cpu(), dw.cpu()
    _say("cell backward 16-bit outputs", nb, T, n, N0, K)
    (a32, f32, w32), (a16, f16_, w16) = read(torch.float32), read(bf)
    assert torch.isfinite(a32[:, n:]).all() and torch.isnan(a32[:, :n]).all()
    assert torch.equal(a16[:, n:], a32[:, n:].to(bf)) and torch.isnan(a16[:, :n].float()).all()
    assert torch.equal(f16_, f32) and torch.equal(w16, w32)
    (p32, v32, w32), (p16, v16, w16) = pool(torch.float32), pool(bf)
    for a, b in ((p16, p32), (v16, v32)):
        assert torch.isfinite(b[:, :n]).all() and torch.isnan(b[:, n:]).all()
        assert torch.equal(a[:, :n], b[:, :n].to(bf)) and torch.isnan(a[:, n:].float()).all()
    assert torch.equal(w16, w32)


def test_fp16_attention_backward_takes_fp32_products():
    """fp16 inputs at the training shape's head_dim 64 take the fp32 smat_bgemm
    products, not the fused kernels (whose bf16 hi/lo operand split needs fp32's
    exponent range).  With normalisers of 1e4-1e5 (T = 4096, elu + 1 features),
    where dH = dout / den is below fp16's normal range, the gradients stay
    finite and within the 16-bit bar (norm-relative 2e-2) of fp64 autograd on
    the same fp16 values."""
    from smat_attention_amd.kernels import hip_bwd as HB
    T, d, nb = 4096, 3, 2
    spec = build_mask(T, d, chunk=128)
    Phi, Psi, Vb = (x.to(torch.float16) for x in _feats(nb, T, 64, seed=8, k_scale=0.125))
    xs = [x.to(DEV) for x in (Phi, Psi, Vb)]
    assert not HB.long_range_backward_ok(*xs) and not HB.fused_chunk_backward_ok(*xs, 128)
    w = torch.randn(nb, T, 64, generator=torch.Generator().manual_seed(9))
    _say("fp16 attention backward", T, d)
    out, parts = A.smat_attention(*xs, spec, return_parts=True)
    den = parts["H"][..., -1].float()
    _say(f"  normaliser range {den.min().item():.3g} .. {den.max().item():.3g}")
    assert den.max().item() > 1e4
    out, gs = _grads_gpu(spec, Phi, Psi, Vb, w)
    _, r64 = _grads_ref(spec, Phi, Psi, Vb, w)
    for name, a, b in zip(("dPhi", "dPsi", "dVb"), gs, r64):
        e = _nrel(a, b)
        _say(f"  {name}: norm-rel vs fp64 {e:.2e}")
        assert torch.isfinite(a).all() and e < 2e-2, name


def test_fp16_cell_backward_matches_fp32_inputs():
    """ContentAssign's hard point read and pool with fp16 Q, K, V at head_dim 64
    take the list reads (fp32 operands), not the fused bf16 cell kernels.  The
    hash sees the same u either way, so the cells are those of the fp32 run on
    the same values; dQ, dK, dV and the hash parameters' gradients within
    norm-relative 2e-2 of that run."""
    from smat_attention_amd import assign as AS
    B, H, hd, T, d = 2, 4, 64, 2048, 3
    spec = build_mask(T, d, chunk=128)
    n = spec.n
    gen = torch.Generator().manual_seed(81)
    h16 = torch.float16
    Q = torch.randn(B * H, T, hd, generator=gen).to(h16)
    K = (torch.randn(B * H, T, hd, generator=gen) / hd ** 0.5).to(h16)
    V = torch.randn(B * H, T, hd, generator=gen).to(h16)
    # dY scaled so dK, whose hash term grows as 1/std of the small keys, stays
    # inside fp16's range (it reaches 3e4 at unit dY)
    dY = (torch.randn(B * H, T - n, hd + 1, generator=gen) / 128).to(DEV)
    torch.manual_seed(7)
    m = AS.ContentAssign(H, H * hd, spec, mode="point").to(DEV)
    _say("fp16 cell backward", d, spec.N0)

    def run(dt):
        phi = A.make_phi(hd, hd, device=DEV, dtype=dt, seed=0)
        xs = [t.to(DEV, dt).requires_grad_(True) for t in (Q, K, V)]
        assert dt != h16 or not AS._cell_backward_ok(xs[0], None)
        Phi, Psi, Vb = A.featurise(*xs, phi)
        u = xs[1].reshape(B, H, T, hd).transpose(1, 2).reshape(B, T, H * hd).float()
        m.zero_grad()
        Y = m(u, Phi, Psi, Vb, n)
        (Y * dY).sum().backward()
        return ([x.grad.float().cpu() for x in xs]
                + [getattr(m, k).grad.detach().cpu() for k in ("W", "gamma", "b")])
    g16, g32 = run(h16), run(torch.float32)
    for name, a, b in zip(("dQ", "dK", "dV", "dW", "dgamma", "db"), g16, g32):
        e = _nrel(a, b)
        _say(f"  {name}: {e:.2e}")
        assert torch.isfinite(a).all() and e < 2e-2, name


@pytest.mark.parametrize("lr,T,d,n_P,gate", [
    ("direct", 2048, 3, 0, False), ("direct", 2048, 3, 16, True),
    ("subtractive", 2048, 3, 0, False), ("subtractive", 4096, 2, 16, True),
    ("endpoint", 256, 0, 0, False), ("endpoint", 300, 0, 0, True), ("endpoint", 1024, 0, 0, False)])
def test_schedule_gradients(lr, T, d, n_P, gate):
    """Gradients through the direct and subtractive long-range schedules and
    the endpoint mask (zeta landmark block, Walsh incidence), fp32, against
    fp64 autograd through the oracle's own schedule (attention.py:333-384,
    430-441, 458-482): dPhi, dPsi, dVb (and dg) within 1e-5 of the largest
    entry (1e-4 for the subtractive schedule, whose forward cancels in the
    normaliser)."""
    nb, hd = 2, 32
    if lr == "endpoint":
        spec, C, lrs = build_mask(T, T.bit_length() - 1, chunk=8), 8, "pooled"
        assert spec.kind == "endpoint"
    else:
        spec, C, lrs = build_mask(T, d, chunk=128, n_P=n_P), 128, lr
    spec_d = A.to_device(spec, DEV, want_direct=lr == "direct")
    _say("schedule gradients", lr, T, d, n_P, gate)
    Phi, Psi, Vb = _feats(nb, T, hd, seed=60 + T)
    gen = torch.Generator().manual_seed(61)
    w = torch.randn(nb, T, hd, generator=gen)
    g = (torch.rand(nb, T, generator=gen) + 0.5) if gate else None
    xs = [t.to(DEV).requires_grad_(True) for t in (Phi, Psi, Vb)]
    gd = g.to(DEV).requires_grad_(True) if g is not None else None
    out = A.smat_attention(*xs, spec_d, chunk=C, g=gd, long_range=lrs)
    (out * w.to(DEV)).sum().backward()
    got = [x.grad.cpu() for x in xs] + ([gd.grad.cpu()] if gd is not None else [])
    ys = [t.double().requires_grad_(True) for t in (Phi, Psi, Vb)]
    g64 = g.double().requires_grad_(True) if g is not None else None
    ref = O.smat_attention(*ys, spec, chunk=C, g=g64, long_range=lrs)
    (ref * w.double()).sum().backward()
    want = [y.grad for y in ys] + ([g64.grad] if g64 is not None else [])
    assert _rel(out.detach().cpu(), ref.detach()) < (1e-4 if lr == "subtractive" else 1e-5)
    tol = 1e-4 if lr == "subtractive" else 1e-5
    for name, a, b in zip(("dPhi", "dPsi", "dVb", "dg"), got, want):
        e = _rel(a, b)
        _say(f"  {name}: {e:.2e}")
        assert torch.isfinite(a).all() and e < tol, name


@pytest.mark.parametrize("T,n,p,with_y,odt", [(300, 128, 65, True, torch.float32),
                                               (256, 0, 65, True, torch.float32),
                                               (256, 256, 129, False, torch.float32),
                                               (1000, 512, 17, True, torch.float32),
                                               (1000, 512, 65, True, torch.bfloat16),
                                               (300, 100, 65, True, torch.float16)])
def test_combine_normalise(T, n, p, with_y, odt):
    """combine_normalise (smat_combine_normalise and its backward) against the
    reference layer's torch ops in fp64 -- ``cat([H[:, :n], H[:, n:] + Y])``
    then ``N[..., :-1] / N[..., -1:].clamp_min(1e-6)`` (model.py:296-300) --
    output and the gradients of H and Y within 1e-6 of the largest entry.  A
    tenth of the rows have a normaliser below the floor (down to 0), where the
    floor divides and passes no gradient to the normaliser.  With a 16-bit
    output (the layer's cast folded in) every output is the fp64 value
    rounded once (within half an ulp, plus 1e-6), and the gradients are those
    of the upstream gradient as the cast's backward delivers it (rounded to the
    output dtype)."""
    gen = torch.Generator().manual_seed(T + n + p)
    nb = 3
    H = torch.randn(nb, T, p, generator=gen)
    H[..., -1] = H[..., -1].abs() + 0.5
    Y = torch.randn(nb, T - n, p, generator=gen) * 0.3 if with_y else None
    if Y is not None:
        Y[..., -1] = Y[..., -1].abs()
    # rows under the floor (their quotients reach 1e6: not for a float16 output)
    small = torch.rand(nb, T, generator=gen) < (0.1 if odt != torch.float16 else 0.0)
    H[..., -1] = torch.where(small, torch.rand(nb, T, generator=gen) * 1e-6, H[..., -1])
    if Y is not None:
        Y[..., -1] = torch.where(small[:, n:], torch.zeros(()), Y[..., -1])
    dO = torch.randn(nb, T, p - 1, generator=gen)

    def ref(h, y):
        N = h if y is None else torch.cat([h[:, :n], h[:, n:] + y], dim=1)
        return N[..., :-1] / N[..., -1:].clamp_min(1e-6)

    dOe = dO.to(odt).double()                        # what reaches the division's backward
    xs0 = [t.double().requires_grad_(True) for t in (H, Y) if t is not None]
    o0 = ref(*(xs0 if with_y else xs0 + [None]))
    (o0 * dOe).sum().backward()
    xs1 = [t.to(DEV).requires_grad_(True) for t in (H, Y) if t is not None]
    o1 = A.combine_normalise(xs1[0], xs1[1] if with_y else None, n, out_dtype=odt)
    (o1.float() * dO.to(DEV)).sum().backward()
    assert o1.dtype == odt and o1.shape == (nb, T, p - 1)
    if odt == torch.float32:
        assert _grel(o1.detach().cpu(), o0.detach()) < 1e-6
    else:
        half_ulp = 2.0 ** -8 if odt == torch.bfloat16 else 2.0 ** -11
        err = (o1.detach().cpu().double() - o0.detach()).abs()
        assert (err <= o0.detach().abs() * half_ulp * (1 + 1e-5) + 1e-6).all()
    for name, a, b in zip(("dH", "dY"), xs1, xs0):
        e = _grel(a.grad.cpu(), b.grad)
        _say(f"  {name}: {e:.2e}")
        assert e < 1e-6, name


@pytest.mark.parametrize("d,plant,nb,L,dm", [(2, False, 2, 300, 96), (2, True, 2, 517, 96),
                                             (3, True, 1, 1000, 768), (3, False, 3, 64, 160),
                                             (4, True, 2, 256, 96), (5, True, 1, 700, 64)])
def test_fused_hash_pairs(d, plant, nb, L, dm):
    """The training path's pairs from smat_hash_pairs and its backward against
    the torch straight-through construction they replace (``_soft_hash`` then
    ``_ste_pairs``, the reference's op order, assign.py:246-317) on the same
    module and fp32 input: cells, pair cells and forward weights equal, the
    load-balance term within 1e-6, and the gradients of u, W, gamma and b for
    a random upstream gradient of every pair weight plus 3 x the load-balance
    term within 1e-5 of the largest entry.  Hash dimension d - 1 = 1..4 (2 to
    16 pairs per token), planted key columns included."""
    from smat_attention_amd.assign import ContentAssign
    H = 3
    spec = build_mask(4096, d, chunk=128)
    gen = torch.Generator().manual_seed(90 + d)
    u0 = torch.randn(nb, L, dm, generator=gen)
    G = torch.randn(nb * H, L, 1 << spec.dim, generator=gen).to(DEV)
    torch.manual_seed(11 + d)
    m = ContentAssign(H, dm, spec, mode="point").to(DEV)
    with torch.no_grad():
        m.gamma.mul_(1.5)
        m.b.normal_(0.0, 0.3)
    _say("fused hash pairs", d, plant, nb, L, dm, spec.q)

    def run(fused):
        m.zero_grad()
        u = u0.to(DEV).requires_grad_(True)
        if fused:
            cells, idx, w, aux = m._hash_pairs(u, plant_at=plant)
        else:
            cells, idx, w, aux = m._ste_pairs(m._soft_hash(u), plant_at=plant)
        ((w * G).sum() + 3.0 * aux).backward()
        return (cells.cpu(), idx.cpu(), w.detach().cpu(), aux.item(),
                [u.grad.cpu()] + [getattr(m, k).grad.detach().cpu() for k in ("W", "gamma", "b")])
    c1, i1, w1, a1, g1 = run(True)
    c0, i0, w0, a0, g0 = run(False)
    assert torch.equal(c1, c0) and torch.equal(i1, i0) and torch.equal(w1, w0)
    assert abs(a1 - a0) < 1e-6 * max(1.0, abs(a0)), (a1, a0)
    for name, a, b in zip(("du", "dW", "dgamma", "db"), g1, g0):
        e = _grel(a, b)
        _say(f"  {name}: {e:.2e}")
        assert torch.isfinite(a).all() and e < 1e-5, name


@pytest.mark.parametrize("d,T,n", [(3, 1024, 512), (2, 700, 256), (4, 512, 384)])
def test_fused_pairs_whole_state(d, T, n):
    """Both sides' pairs from one LayerNorm and projection over the whole
    hidden state (keys: rows before n, planted; queries: the rest) against the
    torch straight-through path on each side's slice: cells, pair cells and
    weights equal, and the gradients of u, W, gamma and b for random upstream
    gradients of every pair weight plus 3 x the load-balance term within 1e-5
    of the largest entry."""
    from smat_attention_amd import assign as AS
    H, dm, nb = 3, 128, 2
    spec = build_mask(4096, d, chunk=128)
    gen = torch.Generator().manual_seed(300 + d)
    u0 = torch.randn(nb, T, dm, generator=gen)
    K = 1 << spec.dim
    Gk = torch.randn(nb * H, n, K, generator=gen).to(DEV)
    Gq = torch.randn(nb * H, T - n, K, generator=gen).to(DEV)
    torch.manual_seed(5)
    m = AS.ContentAssign(H, dm, spec, mode="point").to(DEV)
    _say("fused pairs over the whole state", d, T, n)

    def run(fused):
        AS.FUSED_HASH_PAIRS = fused
        try:
            m.zero_grad()
            u = u0.to(DEV).requires_grad_(True)
            ck, ik, wk, cq, iq, wq = m._pairs_of(u, n, None, None, None, None, False)
            ((wk * Gk).sum() + (wq * Gq).sum() + 3.0 * m.aux).backward()
            return ([t.cpu() for t in (ck, ik, wk.detach(), cq, iq, wq.detach())],
                    [u.grad.cpu()] + [getattr(m, k).grad.detach().cpu() for k in ("W", "gamma", "b")])
        finally:
            AS.FUSED_HASH_PAIRS = True
    f1, g1 = run(True)
    f0, g0 = run(False)
    for a, b in zip(f1, f0):
        assert torch.equal(a, b)
    for name, a, b in zip(("du", "dW", "dgamma", "db"), g1, g0):
        e = _grel(a, b)
        _say(f"  {name}: {e:.2e}")
        assert torch.isfinite(a).all() and e < 1e-5, name


@pytest.mark.parametrize("kind,gate,T", [("elu1", True, 1000), ("relu", True, 2048),
                                         ("elu1", False, 4096)])
def test_fused_featurise_backward(kind, gate, T):
    """The feature map's backward at head_dim 64, bf16 (smat_featurise_backward)
    against the torch products it replaces, same forward and upstream
    gradients: dQ, dK, dh (bf16) within 2e-3 norm-relative, dW (bf16) within
    2e-3, dV equal; a tail tile (T = 1000) and both maps."""
    from smat_attention_amd.kernels import hip_bwd as HB
    nb, hd = 6, 64
    gen = torch.Generator().manual_seed(80 + T)
    bf = torch.bfloat16
    Q, K, V = (torch.randn(nb, T, hd, generator=gen).to(bf) for _ in range(3))
    h = (torch.rand(nb, T, generator=gen) + 0.5).to(bf) if gate else None
    dPhi, dPsi = (torch.randn(nb, T, hd, generator=gen).to(bf) for _ in range(2))
    dVb = torch.randn(nb, T, hd + 1, generator=gen).to(bf)
    _say("fused featurise backward", kind, gate, T)

    def run(fused):
        HB.FUSED_FEATURISE_BACKWARD = fused
        try:
            phi = A.make_phi(hd, hd, kind=kind, device=DEV, dtype=bf, seed=3)
            phi.W.requires_grad_(True)
            xs = [t.to(DEV).requires_grad_(True) for t in (Q, K, V)]
            hd_ = h.to(DEV).requires_grad_(True) if h is not None else None
            Phi, Psi, Vb = A.featurise(*xs, phi, h=hd_)
            torch.autograd.backward([Phi, Psi, Vb], [dPhi.to(DEV), dPsi.to(DEV), dVb.to(DEV)])
            out = [x.grad.float().cpu() for x in xs] + [phi.W.grad.float().cpu()]
            if hd_ is not None:
                out.append(hd_.grad.float().cpu())
            return out
        finally:
            HB.FUSED_FEATURISE_BACKWARD = True
    g1, g0 = run(True), run(False)
    for name, a, b in zip(("dQ", "dK", "dV", "dW", "dh"), g1, g0):
        e = _nrel(a, b)
        _say(f"  {name}: {e:.2e}")
        assert torch.isfinite(a).all()
        assert e < 2e-3, name


@pytest.mark.parametrize("d", [2, 3])
def test_training_step_content_hashed(d):
    """The content-hashed training step at head_dim 64, T = 4096 (4 of the
    configuration's 12 heads, so the fp64 oracle finishes in seconds): the
    feature map, the segmented causal scan plus the content-addressed long-range
    term added to the recent rows, the single division (the reference model's
    layer, model.py:300-311); dQ, dK, dV and the hash input's gradient against
    the same step in fp64 through the oracle, fp32 inputs."""
    from oracle import assign_ref as RA
    from smat_attention_amd.assign import ContentAssign
    H_, T, hd = 4, 4096, 64
    spec = build_mask(T, d, chunk=128)
    n = spec.n
    gen = torch.Generator().manual_seed(40 + d)
    Q = torch.randn(1, H_, T, hd, generator=gen) * 0.5
    K = torch.randn(1, H_, T, hd, generator=gen) / hd ** 0.5
    V = torch.randn(1, H_, T, hd, generator=gen)
    X = torch.randn(1, T, 96, generator=gen)                  # the layer input the hash reads
    dO = torch.randn(H_, T, hd, generator=gen)
    torch.manual_seed(7)
    m = ContentAssign(H_, 96, spec, mode="point")
    W = O.phi_weight(hd, hd, dtype=torch.float64, seed=0)
    pc = torch.tensor([spec.q ** (spec.dim - l) for l in range(1, spec.dim + 1)])
    _say("training step", d, spec.q, spec.N0)

    def step_ref(q, k, v, x, prm):
        phi = lambda z: torch.nn.functional.elu(z @ W.T) + 1.0
        Phi, Psi, Vb = O.featurise(q.reshape(H_, T, hd), k.reshape(H_, T, hd),
                                   v.reshape(H_, T, hd), phi)
        Hs = O.segmented_causal_scan(Phi, Psi, Vb, n, 128)
        Ylr = RA.pairs_branch(x, Phi, Psi, Vb, n, prm["W"], prm["gamma"], prm["b"], spec.q,
                              spec.dim, H_, spec.N0, planted_cols=spec.planted_cols,
                              plant_cells=pc)
        Hs = torch.cat([Hs[:, :n], Hs[:, n:] + Ylr], dim=1)
        return Hs[..., :-1] / Hs[..., -1:].clamp_min(1e-6)

    def step_hip(q, k, v, x, prm):
        phi = A.FeatureMap(W.to(DEV, torch.float32), "elu1")
        Phi, Psi, Vb = A.featurise(q.reshape(H_, T, hd), k.reshape(H_, T, hd),
                                   v.reshape(H_, T, hd), phi)
        Hs = A.segmented_causal_scan(Phi, Psi, Vb, n, 128)
        Ylr = m(x, Phi, Psi, Vb, n)
        Hs = torch.cat([Hs[:, :n], Hs[:, n:] + Ylr], dim=1)
        return Hs[..., :-1] / Hs[..., -1:].clamp_min(1e-6)

    def run(dev, dt, step, prm):
        xs = [t.to(dev, dt).requires_grad_(True) for t in (Q, K, V, X)]
        o = step(*xs, prm)
        (o * dO.to(dev, dt)).sum().backward()
        return o.detach().cpu(), [t.grad.detach().cpu() for t in xs]
    prm64 = {k: getattr(m, k).detach().double().requires_grad_(True) for k in ("W", "gamma", "b")}
    o0, g0 = run("cpu", torch.float64, step_ref, prm64)
    m.to(DEV)
    o1, g1 = run(DEV, torch.float32, step_hip, None)
    # the fp32 hash must give the fp64 cells for the comparison to mean anything
    ck64, _ = RA.cells(X[:, :n].double(), prm64["W"].detach(), prm64["gamma"].detach(),
                       prm64["b"].detach(), spec.q, spec.dim, H_)
    ck64 = RA.plant(ck64, torch.as_tensor(spec.planted_cols, dtype=torch.long), pc)
    assert torch.equal(m.last_hard_k.cpu(), ck64)
    assert _grel(o1, o0) < 1e-5
    for name, a, b in zip(("dQ", "dK", "dV", "dX"), g1, g0):
        assert _grel(a, b) < 1e-5, (name, _grel(a, b))
    for k, pr in prm64.items():
        assert _grel(getattr(m, k).grad.cpu(), pr.grad) < 1e-4, k


def _device_bins(s64, cells, q, dim, margin):
    """Shift that moves each fp64 hash value into the bin the device chose.

    ``s64 (B, L, dim)`` are the oracle's hash values and ``cells (B, L)`` the
    device's cells on the same inputs.  Where they disagree, every coordinate
    whose bin differs must lie within ``margin`` of the edge between the two
    bins (device rounding, not a different hash); the shift puts it just
    inside the device's bin.  Returns (shift, number of coordinates moved)."""
    digits = torch.stack([(cells // q ** (dim - 1 - k)) % q for k in range(dim)], -1)
    lo = s64.floor().long()
    moved = digits != lo
    if moved.any():
        edge = torch.where(digits > lo, digits, digits + 1).double()
        assert (s64[moved] - edge[moved]).abs().max().item() < margin, \
            "a cell differs from the oracle away from a bin edge"
        assert ((digits - lo).abs()[moved] == 1).all()
    target = torch.where(digits > lo, digits.double() + 1e-9, digits.double() + 1 - 1e-9)
    shift = torch.where(moved, target - s64, torch.zeros_like(s64))
    return shift, int(moved.sum())


@pytest.mark.parametrize("d", [2, 3])
def test_training_step_content_hashed_bf16_full_shape(d):
    """The training configuration itself: B=8, H=12, head_dim 64, T=4096, bf16
    q, k, v ~ N(0, 1) (k scaled 1/sqrt(64)), the content hash reading k (u = k
    viewed as (B, T, 768), hashed from its fp32 values as the reference's layer
    hashes x.float(), model.py:265, 313), dO ~ N(0, 1); forward and backward on
    the GPU.  Batch element 0 -- all 12 heads, since each head's hash reads every
    head's k -- against fp64 autograd through the oracle on the same bf16 values:

    * cells equal the oracle's except within 1e-4 of a bin edge (fp32 vs fp64
      rounding of the hash); there the oracle is given the device's bin, which
      changes no gradient formula (the straight-through weights' derivative
      depends on the bin only);
    * O within 2e-2 absolute (the bf16 bar);
    * dQ, dK (through the features and the hash), dV within 2e-2
      norm-relative, the reference's bar for its kernel gradients
      (tests/test_triton_bwd.py:24-64).  dQ is the loosest: it carries the
      bf16 rounding of the feature map's product; the reference's own torch
      path in bf16 (the oracle run on bf16 tensors) is 1.7e-2 from fp64 in dQ
      at this shape (positional, d = 2, 2 heads), this path about 1.5e-2."""
    from oracle import assign_ref as RA
    from smat_attention_amd.assign import ContentAssign
    B, H, hd, T = 8, 12, 64, 4096
    spec = build_mask(T, d, chunk=128)
    n, q, dim = spec.n, spec.q, spec.dim
    _say("training step bf16 full shape", d, q, spec.N0)
    gen = torch.Generator().manual_seed(50 + d)
    bf = torch.bfloat16
    Q = torch.randn(B * H, T, hd, generator=gen).to(bf)
    K = (torch.randn(B * H, T, hd, generator=gen) / hd ** 0.5).to(bf)
    V = torch.randn(B * H, T, hd, generator=gen).to(bf)
    dO = torch.randn(B * H, T, hd, generator=gen)
    torch.manual_seed(7)
    m = ContentAssign(H, H * hd, spec, mode="point")
    pc = torch.tensor([q ** (dim - l) for l in range(1, dim + 1)])

    def as_u(k, nb):
        return k.reshape(nb, H, T, hd).transpose(1, 2).reshape(nb, T, H * hd)

    # ---- the GPU step over the whole batch
    prm = {k: getattr(m, k).detach().double() for k in ("W", "gamma", "b")}
    m.to(DEV)
    phi = A.make_phi(hd, hd, device=DEV, dtype=bf, seed=0)
    xs = [t.to(DEV).requires_grad_(True) for t in (Q, K, V)]
    Phi, Psi, Vb = A.featurise(*xs, phi)
    Hs = A.segmented_causal_scan(Phi, Psi, Vb, n, 128)
    Ylr = m(as_u(xs[1], B).float(), Phi, Psi, Vb, n)
    Hs = torch.cat([Hs[:, :n], Hs[:, n:] + Ylr], dim=1)
    o = Hs[..., :-1] / Hs[..., -1:].clamp_min(1e-6)
    (o * dO.to(DEV)).sum().backward()
    o1 = o.detach()[:H].cpu()
    g1 = [x.grad[:H].cpu() for x in xs]
    ck1, cq1 = m.last_hard_k[:H].cpu(), m.last_hard_q[:H].cpu()

    # ---- batch element 0 in fp64 through the oracle, on the same bf16 values
    W64 = phi.W.double().cpu()
    f64 = lambda z: torch.nn.functional.elu(z @ W64.T) + 1.0
    x0 = [t[:H].double().requires_grad_(True) for t in (Q, K, V)]
    u0 = as_u(x0[1], 1)
    s64 = RA.hash_s(u0.detach(), prm["W"], prm["gamma"], prm["b"], q, H)
    cells64 = torch.zeros(H, T, dtype=torch.long)
    for k in range(dim):
        cells64 += s64[..., k].floor().long() * q ** (dim - 1 - k)
    cols = torch.as_tensor(spec.planted_cols, dtype=torch.long)
    assert torch.equal(RA.plant(cells64[:, :n], cols, pc)[:, cols], ck1[:, cols])
    dev_cells = torch.cat([ck1, cq1], 1)
    dev_cells[:, cols] = cells64[:, cols]           # planted keys carry no hash bin
    shift, moved = _device_bins(s64, dev_cells, q, dim, margin=1e-4)
    _say(f"  coordinates at a bin edge given the device's bin: {moved} of {s64.numel()}")
    Phi0, Psi0, Vb0 = O.featurise(*x0, f64)
    Hs0 = O.segmented_causal_scan(Phi0, Psi0, Vb0, n, 128)
    Y0 = RA.dense_point_ste(u0, Phi0, Psi0, Vb0, n, prm["W"], prm["gamma"], prm["b"], q, dim,
                            H, spec.N0, planted_cols=spec.planted_cols, plant_cells=pc,
                            s_shift=shift)
    Hs0 = torch.cat([Hs0[:, :n], Hs0[:, n:] + Y0], dim=1)
    o0 = Hs0[..., :-1] / Hs0[..., -1:].clamp_min(1e-6)
    (o0 * dO[:H].double()).sum().backward()
    e_o = (o1.double() - o0.detach()).abs().max().item()
    errs = {nm: _nrel(a, b.grad) for nm, a, b in zip(("dQ", "dK", "dV"), g1, x0)}
    _say(f"  O {e_o:.2e} (abs); " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()))
    assert e_o < 2e-2
    for nm, e in errs.items():
        assert e < 2e-2, (nm, e)


# ---------------------------------------------------------------------------
# smat_bgemm itself: every product of the backward runs on it
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("ta,tb", [(torch.float32, torch.float32), (torch.bfloat16, torch.float32),
                                   (torch.float32, torch.bfloat16), (torch.bfloat16, torch.bfloat16),
                                   (torch.float16, torch.float32)])
@pytest.mark.parametrize("a_t,b_t", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("mask,beta", [(0, 0), (1, 0), (2, 1), (0, 1)])
@pytest.mark.parametrize("M,N,K", [(70, 65, 45), (64, 129, 70)])
def test_bgemm_layouts_masks_and_accumulation(ta, tb, a_t, b_t, mask, beta, M, N, K):
    """C[i] (+)= A[i] B[i] over a two-level batch, with each operand stored
    row-major or transposed (swapped strides), ragged M, N, K, the two causal
    masks and beta, against the fp64 product of the same values.  N = 65 and
    129 take the 80-column block, N = 64 products elsewhere the 64-column one."""
    from smat_attention_amd.kernels.hip_bwd import _bgemm
    n1, n2 = 2, 3
    g = torch.Generator().manual_seed(60)
    A64 = torch.randn(n1, n2, M, K, generator=g, dtype=torch.float64)
    B64 = torch.randn(n1, n2, K, N, generator=g, dtype=torch.float64)
    C0 = torch.randn(n1, n2, M, N, generator=g, dtype=torch.float64)
    Aq, Bq = A64.to(ta), B64.to(tb)                  # the values the kernel sees
    # stored layouts: A as (.., M, K) or (.., K, M); B as (.., K, N) or (.., N, K)
    As = (Aq.transpose(-1, -2) if a_t else Aq).contiguous().to(DEV)
    Bs = (Bq.transpose(-1, -2) if b_t else Bq).contiguous().to(DEV)
    a = (n2 * M * K, M * K, 1, M) if a_t else (n2 * M * K, M * K, K, 1)
    b = (n2 * K * N, K * N, 1, K) if b_t else (n2 * K * N, K * N, N, 1)
    C = C0.float().to(DEV)
    _bgemm(As, Bs, C, M=M, N=N, K=K, n1=n1, n2=n2, a=a, b=b,
           c=(n2 * M * N, M * N, N, 1), beta=beta, mask=mask)
    ref = Aq.double() @ Bq.double()
    if mask == 1:
        ref = torch.tril(ref)
    elif mask == 2:
        ref = torch.triu(ref)
    if beta:
        ref = ref + C0.float().double()
    assert (C.double().cpu() - ref).abs().max().item() < 1e-5 * ref.abs().max().item()
