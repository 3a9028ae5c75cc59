"""The forward with the feature map inside the kernels (smat_attention_fused,
smat_forward_fused) against featurise + smat_attention and against the oracle.

The fused kernels form Phi = map(Q W^T), Psi = h map(K W^T) and Vb = [V, 1] in
LDS with the stand-alone featurise kernel's MFMA sequence and rounding, so the
output must equal the unfused HIP path up to fp32 summation order where the
two paths pick different pool kernels (1e-5 of the largest entry), and must
meet the bf16 bar against the reference's torch path on the same bf16
inputs (2e-2 absolute on O, attention.py:82-106 then :391-455).
"""
import pytest
import torch

import oracle.schedule as O
from smat_attention_amd import attention as A
from smat_attention_amd.mask import build_mask

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
BF = torch.bfloat16


def _say(*a):
    print("[case]", *a, flush=True)


def _rel(got, ref):
    got, ref = got.double().cpu(), ref.double().cpu()
    return ((got - ref).abs().max() / ref.abs().max().clamp_min(1e-300)).item()


def _inputs(nb, T, seed, dt=BF, gates=False):
    Q, K, V = O.seeded_qkv(nb, T, 128, 128, seed=seed, dtype=torch.float32,
                           k_scale=128 ** -0.5)
    gen = torch.Generator().manual_seed(seed + 1)
    h = (torch.rand(nb, T, generator=gen) * 0.9 + 0.1).to(dt) if gates else None
    g = (torch.rand(nb, T, generator=gen) + 0.5) if gates else None
    return Q.to(dt), K.to(dt), V.to(dt), h, g


def _run_both(spec, Q, K, V, h, g, kind="elu1", dt=BF):
    W = O.phi_weight(128, 128, dtype=dt, seed=0).to(DEV)
    phi = A.FeatureMap(W, kind)
    Qd, Kd, Vd = (x.to(DEV) for x in (Q, K, V))
    hd = h.to(DEV) if h is not None else None
    gd = g.to(DEV) if g is not None else None
    assert A._fused_ok(Qd, Kd, Vd, phi, spec, min(128, spec.T), hd)
    fused = A.smat_attention_fused(Qd, Kd, Vd, phi, spec, g=gd, h=hd)
    unfused = A.smat_attention(*A.featurise(Qd, Kd, Vd, phi, h=hd), spec, g=gd)
    torch.cuda.synchronize()
    return fused, unfused


@pytest.mark.parametrize("T,d,n_P,gates,kind,nb", [
    (4096, 2, 0, False, "elu1", 6), (4096, 2, 16, True, "relu", 6),
    (8192, 3, 0, True, "elu1", 3), (2048, 3, 16, False, "elu1", 4),
    (4096, 4, 0, False, "elu1", 2), (8192, 2, 0, True, "elu1", 4)])
def test_fused_forward_matches_featurise_then_forward(T, d, n_P, gates, kind, nb):
    """Ragged profiles, the global channel (n_P = 16), the key gate h, the output
    gate g, both feature maps, d = 2..4: the fused forward equals featurise then
    smat_attention within 1e-5 of the largest entry.  d = 2 at T = 8192 (62
    recent rows a type) takes the staged query of the recent rows' Phi."""
    spec = build_mask(T, d, chunk=128, n_P=n_P)
    _say("fused forward", T, d, n_P, gates, kind, nb)
    Q, K, V, h, g = _inputs(nb, T, seed=T + d + n_P, gates=gates)
    fused, unfused = _run_both(spec, Q, K, V, h, g, kind)
    e = _rel(fused, unfused)
    _say(f"  vs featurise + smat_attention: {e:.2e}")
    assert fused.dtype == torch.float32 and fused.shape == (nb, T, 128)
    assert torch.isfinite(fused).all() and e < 1e-5


@pytest.mark.parametrize("T,d,n_P,gates", [(4096, 3, 0, True), (4096, 2, 16, False)])
def test_fused_forward_fp16(T, d, n_P, gates):
    """fp16 q, k, v: the fused kernels' fp16 instantiations (pool, query,
    prepass, scan, with libm's expm1f in the map) equal featurise +
    smat_attention within 1e-5 of the largest entry, and head 0 meets the
    16-bit bar (2e-2 absolute on O) against the oracle's featurise and
    schedule on the same fp16 values."""
    F16 = torch.float16
    spec = build_mask(T, d, chunk=128, n_P=n_P)
    _say("fused forward fp16", T, d, n_P, gates)
    # six sequences: the fused pool needs 256 (sequence, profile) items (N0 = 47 at d = 2)
    Q, K, V, h, g = _inputs(6, T, seed=T + d + 7, dt=F16, gates=gates)
    fused, unfused = _run_both(spec, Q, K, V, h, g, dt=F16)
    e = _rel(fused, unfused)
    W = O.phi_weight(128, 128, dtype=F16, seed=0)
    phi_cpu = lambda x: torch.nn.functional.elu(x.float() @ W.float().T).to(F16) + 1.0
    ref = O.smat_attention(*O.featurise(Q[:1], K[:1], V[:1], phi_cpu,
                                        h=None if h is None else h[:1]),
                           spec, g=None if g is None else g[:1])
    e_o = (fused[:1].double().cpu() - ref.double()).abs().max().item()
    _say(f"  vs unfused {e:.2e}; head 0 vs the torch path on fp16: O {e_o:.2e}")
    assert torch.isfinite(fused).all() and e < 1e-5 and e_o < 2e-2


def test_fused_forward_long_prefill_T32768():
    """The long-prefill configuration at T = 32768 (B=1, H=8, head_dim 128, d=3,
    bf16 q, k, v ~ N(0, 1), k scaled 1/sqrt(128)): all 8 heads against the
    unfused HIP path (1e-5), heads 0-1 against the oracle's featurise and
    schedule run on the same bf16 values (the reference's torch path, 2e-2
    absolute on O), and a repeated call is bit-identical."""
    T = 32768
    spec = build_mask(T, 3, chunk=128)
    _say("fused forward T=32768 d=3 nb=8 hd=128 bf16")
    Q, K, V, _, _ = _inputs(8, T, seed=0)
    fused, unfused = _run_both(spec, Q, K, V, None, None)
    e = _rel(fused, unfused)
    W = O.phi_weight(128, 128, dtype=BF, seed=0)
    phi_cpu = lambda x: torch.nn.functional.elu(x @ W.T) + 1.0
    ref = O.smat_attention(*O.featurise(Q[:2], K[:2], V[:2], phi_cpu), spec)
    e_o = (fused[:2].double().cpu() - ref.double()).abs().max().item()
    _say(f"  vs unfused {e:.2e}; heads 0-1 vs the torch path on bf16: O {e_o:.2e}")
    assert e < 1e-5 and e_o < 2e-2
    phi = A.FeatureMap(W.to(DEV), "elu1")
    again = A.smat_attention_fused(Q.to(DEV), K.to(DEV), V.to(DEV), phi, spec)
    assert torch.equal(again, fused)


def test_fused_forward_long_prefill_T131072():
    """The benchmark shape (B=1, H=8, head_dim 128, d=3, T=131072, bf16 q, k, v
    ~ N(0, 1), k scaled 1/sqrt(128); q = 41, the line-group incidence): all 8
    heads of smat_attention_fused against featurise + smat_attention (1e-5 of
    the largest entry); head 0 against the oracle's featurise and schedule on
    the same bf16 values (the reference's torch path: 2e-2 absolute on O, and
    1e-3 on the log-normaliser, read from the unfused HIP call's parts)."""
    T = 131072
    spec = build_mask(T, 3, chunk=128)
    assert (spec.q, spec.N0, spec.B) == (41, 1681, 1722)
    _say("fused forward T=131072 d=3 nb=8 hd=128 bf16")
    Q, K, V, _, _ = _inputs(8, T, seed=0)
    fused, unfused = _run_both(spec, Q, K, V, None, None)
    e = _rel(fused, unfused)
    _say(f"  all heads vs featurise + smat_attention: {e:.2e}")
    assert torch.isfinite(fused).all() and e < 1e-5
    del unfused
    W = O.phi_weight(128, 128, dtype=BF, seed=0)
    phi_cpu = lambda x: torch.nn.functional.elu(x @ W.T) + 1.0
    feats = O.featurise(Q[:1], K[:1], V[:1], phi_cpu)
    ref, rparts = O.smat_attention(*feats, spec, return_parts=True)
    phi = A.FeatureMap(W.to(DEV), "elu1")
    Pd, Sd, Wd = A.featurise(Q[:1].to(DEV), K[:1].to(DEV), V[:1].to(DEV), phi)
    _, parts = A.smat_attention(Pd, Sd, Wd, spec, return_parts=True)
    lse = torch.log(parts["H"][..., -1].double().cpu())
    lse_ref = torch.log(rparts["H"][..., -1].double())
    e_o = (fused[:1].double().cpu() - ref.double()).abs().max().item()
    e_l = (lse - lse_ref).abs().max().item()
    _say(f"  head 0 vs the torch path on bf16: O {e_o:.2e}, lse {e_l:.2e}")
    assert e_o < 2e-2 and e_l < 1e-3


def test_fused_forward_long_prefill_T524288():
    """T = 524288, d = 3 (q = 67, the row-group incidence; 57-58 recent rows a
    row type, the streaming query's four-tile form), one head: the fused call
    against featurise + smat_attention (1e-5 of the largest entry)."""
    T = 524288
    spec = build_mask(T, 3, chunk=128)
    assert (spec.q, spec.N0, spec.B) == (67, 4489, 4556)
    _say("fused forward T=524288 d=3 nb=1 hd=128 bf16")
    Q, K, V, _, _ = _inputs(1, T, seed=2)
    fused, unfused = _run_both(spec, Q, K, V, None, None)
    e = _rel(fused, unfused)
    _say(f"  vs featurise + smat_attention: {e:.2e}")
    assert torch.isfinite(fused).all() and e < 1e-5


@pytest.mark.parametrize("T,nb,gates", [(4096, 2, False), (8192, 3, True), (131072, 8, False)])
def test_fused_forward_d1_pools_from_the_causal_pass(T, nb, gates):
    """d = 1 (one profile holding every landmark token, the identity incidence):
    the fused forward takes the profile's pool from the causal pass's group
    sums over the tokens [0, n) instead of a pool pass; against featurise +
    smat_attention (1e-5 of the largest entry; the pool sums in another order)."""
    spec = build_mask(T, 1, chunk=128)
    assert (spec.N0, spec.B, spec.n_P) == (1, 1, 0)
    _say(f"fused forward d=1 T={T} nb={nb} gates={gates}")
    Q, K, V, h, g = _inputs(nb, T, seed=11, gates=gates)
    fused, unfused = _run_both(spec, Q, K, V, h, g)
    e = _rel(fused, unfused)
    _say(f"  vs featurise + smat_attention: {e:.2e}")
    assert torch.isfinite(fused).all() and e < 1e-5


def test_fused_forward_falls_back_outside_its_shape_and_under_grad():
    """head_dim 64 (the d=2 single-GPU configuration's width) is not a fused
    shape: smat_attention_fused runs featurise then smat_attention, bitwise the
    same result.  With inputs that require grad the composed path runs too, and
    its gradients are those of the composed call."""
    T = 2048
    spec = build_mask(T, 2, chunk=128)
    gen = torch.Generator().manual_seed(4)
    Q, K, V = (torch.randn(4, T, 64, generator=gen).to(BF).to(DEV) for _ in range(3))
    phi = A.make_phi(64, 64, device=DEV, dtype=BF, seed=0)
    assert not A._fused_ok(Q, K, V, phi, spec, 128, None)
    a = A.smat_attention_fused(Q, K, V, phi, spec)
    b = A.smat_attention(*A.featurise(Q, K, V, phi), spec)
    assert torch.equal(a, b)
    # d = 2 with a global channel and few (sequence, profile) items: the
    # unfused pool's split-K path
    spec1 = build_mask(2048, 2, chunk=128, n_P=16)
    Q1, K1, V1, _, _ = _inputs(1, 2048, seed=3)
    Q1, K1, V1 = Q1.to(DEV), K1.to(DEV), V1.to(DEV)
    phi1 = A.FeatureMap(O.phi_weight(128, 128, dtype=BF, seed=0).to(DEV), "elu1")
    assert spec1.N0 < 256 and not A._fused_ok(Q1, K1, V1, phi1, spec1, 128, None)
    assert torch.equal(A.smat_attention_fused(Q1, K1, V1, phi1, spec1),
                       A.smat_attention(*A.featurise(Q1, K1, V1, phi1), spec1))
    Q2, K2, V2, _, _ = _inputs(2, T, seed=9)
    xs = [x.to(DEV).requires_grad_(True) for x in (Q2, K2, V2)]
    phi2 = A.FeatureMap(O.phi_weight(128, 128, dtype=BF, seed=0).to(DEV), "elu1")
    dO = torch.randn(2, T, 128, generator=gen).to(DEV)
    (A.smat_attention_fused(*xs, phi2, spec) * dO).sum().backward()
    g1 = [x.grad.clone() for x in xs]
    for x in xs:
        x.grad = None
    (A.smat_attention(*A.featurise(*xs, phi2), spec) * dO).sum().backward()
    for a1, b1 in zip(g1, (x.grad for x in xs)):
        assert torch.equal(a1, b1)
