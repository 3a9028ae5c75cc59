"""The oracle's schedule, pinned by what the mathematics fixes.

Ports tests/test_smat.py:212-362 (equivalence with the dense definition,
pooled == direct == subtractive, scan == block-diagonal causal, chunk-width
invariance, butterfly transforms, exact non-influence, decode == prefill,
reduced precision) and adds: d = 1 against plain causal linear attention, the
d = 2 identity incidence, finite-difference gradients, and planted mistakes
that the checks must catch."""
import numpy as np
import pytest
import torch

from oracle import schedule as S
from smat_attention_amd.mask import build_mask, materialise


def _rand(T, nb=2, d_qk=16, d_v=12, r=20, dt=torch.float64, seed=0):
    """test_smat.py:212-220: gated features with the reference's seeding."""
    torch.manual_seed(seed)
    Q = torch.randn(nb, T, d_qk, dtype=dt)
    K = torch.randn(nb, T, d_qk, dtype=dt)
    V = torch.randn(nb, T, d_v, dtype=dt)
    g = torch.rand(nb, T, dtype=dt) + 0.5
    h = torch.rand(nb, T, dtype=dt) + 0.5
    phi = S.make_phi(d_qk, r, dtype=dt)
    return S.featurise(Q, K, V, phi, g=g, h=h), g


def _dense(spec):
    return torch.from_numpy(materialise(spec)).double()


@pytest.mark.parametrize("T,d,nP", [(512, 1, 0), (512, 2, 0), (1024, 2, 0), (1024, 3, 0),
                                    (2048, 3, 0), (2048, 4, 0), (1024, 3, 16), (1024, 10, 0)])
def test_equivalence_with_dense(T, d, nP):
    spec = build_mask(T, d, chunk=64, n_P=nP)
    (Phi, Psi, Vb), g = _rand(T)
    ref = S.dense_masked_kernel_attention(Phi, Psi, Vb, _dense(spec)) * g.unsqueeze(-1)
    got = S.smat_attention(Phi, Psi, Vb, spec, chunk=64, g=g)
    assert (got - ref).abs().max().item() < 1e-10


@pytest.mark.parametrize("T,d", [(1024, 2), (2048, 3), (2048, 4)])
def test_backends_agree(T, d):
    spec = build_mask(T, d, chunk=64)
    (Phi, Psi, Vb), g = _rand(T)
    base = S.smat_attention(Phi, Psi, Vb, spec, chunk=64, g=g)
    for lr in ("direct", "subtractive"):
        got = S.smat_attention(Phi, Psi, Vb, spec, chunk=64, g=g, long_range=lr)
        assert (got - base).abs().max().item() < 1e-10, lr


def test_scan_is_block_diagonal_causal():
    T = 1024
    spec = build_mask(T, 3, chunk=64)
    (Phi, Psi, Vb), _ = _rand(T)
    got = S.segmented_causal_scan(Phi, Psi, Vb, n=spec.n, chunk=64)
    Mseg = np.zeros((T, T))
    Mseg[:spec.n, :spec.n] = np.tril(np.ones((spec.n, spec.n)))
    Mseg[spec.n:, spec.n:] = np.tril(np.ones((spec.T_R, spec.T_R)))
    ref = torch.einsum("nts,nsv->ntv",
                       torch.einsum("nta,nsa->nts", Phi, Psi) * torch.from_numpy(Mseg), Vb)
    assert (got - ref).abs().max().item() < 1e-10


def test_scan_tail_padding():
    """T not a multiple of the chunk: the tail lives in the recent segment."""
    T, C = 1000, 64
    (Phi, Psi, Vb), _ = _rand(T)
    n = 448
    got = S.segmented_causal_scan(Phi, Psi, Vb, n=n, chunk=C)
    Mseg = np.zeros((T, T))
    Mseg[:n, :n] = np.tril(np.ones((n, n)))
    Mseg[n:, n:] = np.tril(np.ones((T - n, T - n)))
    ref = torch.einsum("nts,nsv->ntv",
                       torch.einsum("nta,nsa->nts", Phi, Psi) * torch.from_numpy(Mseg), Vb)
    assert (got - ref).abs().max().item() < 1e-10


def test_chunk_width_invariance():
    (Phi, Psi, Vb), _ = _rand(1024)
    for C in (32, 64, 128, 256):
        s2 = build_mask(1024, 2, chunk=C)
        ref = S.dense_masked_kernel_attention(Phi, Psi, Vb, _dense(s2))
        err = (S.smat_attention(Phi, Psi, Vb, s2, chunk=C) - ref).abs().max().item()
        assert err < 1e-10, C


def test_butterflies_against_dense_matrices():
    nb, N, r, p = 2, 64, 5, 4
    torch.manual_seed(0)
    F = torch.randn(nb, N, r, p, dtype=torch.float64)
    a = np.arange(N)
    Z = torch.from_numpy(((a[:, None] & a[None, :]) == a[None, :]).astype(float))
    assert (S.zeta_transform(F) - torch.einsum("ax,nxrp->narp", Z, F)).abs().max() < 1e-12
    Cw = torch.from_numpy(((np.bitwise_count(a[:, None] & a[None, :]) % 2) == 0).astype(float))
    assert (S.walsh_incidence(F) - torch.einsum("hx,nxrp->nhrp", Cw, F)).abs().max() < 1e-11


@pytest.mark.parametrize("T,d,C", [(1024, 3, 128), (1024, 2, 64), (512, 1, 64)])
def test_exact_noninfluence(T, d, C):
    spec = build_mask(T, d, chunk=C)
    M = materialise(spec).astype(bool)
    (Phi, Psi, Vb), _ = _rand(T)
    base = S.smat_attention(Phi, Psi, Vb, spec, chunk=C)
    rng = np.random.default_rng(0)
    for j in rng.choice(T, size=6, replace=False):
        Psi2, Vb2 = Psi.clone(), Vb.clone()
        Psi2[:, int(j)] = torch.randn_like(Psi2[:, int(j)]).abs()
        Vb2[:, int(j)] = torch.randn_like(Vb2[:, int(j)])
        out = S.smat_attention(Phi, Psi2, Vb2, spec, chunk=C)
        excl = ~M[:, int(j)]
        assert torch.equal(out[:, excl], base[:, excl]), int(j)


@pytest.mark.parametrize("T,d", [(512, 2), (1024, 3), (2048, 4), (512, 1)])
def test_decode_reproduces_prefill(T, d):
    spec = build_mask(T, d, chunk=64)
    (Phi, Psi, Vb), _ = _rand(T)
    full = S.smat_attention(Phi, Psi, Vb, spec, chunk=64)
    n = spec.n
    dec = S.SmatDecoder(Psi[:, :n], Vb[:, :n], spec)
    err = max((dec.step(Phi[:, i], Psi[:, i], Vb[:, i]) - full[:, i]).abs().max().item()
              for i in range(n, T))
    assert err < 1e-11
    assert dec.cache_words() == Psi.shape[0] * (spec.B + 1) * Psi.shape[-1] * Vb.shape[-1]


def test_reduced_precision_close_to_fp64():
    T = 1024
    spec = build_mask(T, 3, chunk=128)
    nb, d_qk, d_v, r = 1, 32, 32, 32
    torch.manual_seed(4)
    Q = torch.randn(nb, T, d_qk, dtype=torch.float64)
    K = torch.randn(nb, T, d_qk, dtype=torch.float64)
    V = torch.randn(nb, T, d_v, dtype=torch.float64)
    ref = S.smat_attention(*S.featurise(Q, K, V, S.make_phi(d_qk, r, dtype=torch.float64)),
                           spec, chunk=128)
    for dt, tol in [(torch.float32, 1e-4), (torch.bfloat16, 6e-2)]:
        Phi, Psi, Vb = S.featurise(Q.to(dt), K.to(dt), V.to(dt), S.make_phi(d_qk, r, dtype=dt))
        got = S.smat_attention(Phi, Psi, Vb, spec, chunk=128, acc_dtype=torch.float32)
        assert (got.double() - ref).abs().max().item() < tol, dt


# --------------------------------------------------------------------------
# textbook special cases
# --------------------------------------------------------------------------

def test_d1_is_plain_causal_linear_attention():
    """M^(1) = L_T: out_t = (Phi_t sum_{s<=t} Psi_s Vb_s^T) normalised, by a running sum."""
    T = 300
    spec = build_mask(T, 1, chunk=32)
    (Phi, Psi, Vb), _ = _rand(T, nb=1)
    got = S.smat_attention(Phi, Psi, Vb, spec, chunk=32)
    state = torch.zeros(Psi.shape[-1], Vb.shape[-1], dtype=torch.float64)
    rows = []
    for t in range(T):
        state = state + torch.outer(Psi[0, t], Vb[0, t])
        o = Phi[0, t] @ state
        rows.append(o[:-1] / o[-1])
    assert (got[0] - torch.stack(rows)).abs().max().item() < 1e-10


def test_d2_incidence_is_identity():
    spec = build_mask(8192, 2, chunk=128)
    np.testing.assert_array_equal(spec.C_indices, np.arange(spec.B))
    torch.manual_seed(1)
    F = torch.randn(2, spec.N0, 3, 4, dtype=torch.float64)
    assert torch.equal(S.apply_incidence(F, spec), F)


def test_pool_is_profile_sum():
    """F_x = sum over the columns j = x (mod N0): brute force on a tiny case."""
    spec = build_mask(2048, 3, chunk=64, n_P=16)
    (_, Psi, Vb), _ = _rand(2048, nb=1, r=3, d_v=2)
    F = S.pool_profiles(Psi, Vb, spec)
    for x in (0, 5, spec.N0 - 1):
        cols = [j for j in range(spec.n_P, spec.n) if (j - spec.n_P) % spec.N0 == x]
        want = sum(torch.outer(Psi[0, j], Vb[0, j]) for j in cols)
        assert (F[0, x] - want).abs().max().item() < 1e-12


def test_query_by_type_rows():
    spec = build_mask(2048, 3, chunk=64)
    torch.manual_seed(2)
    Phi = torch.randn(1, spec.T_R, 4, dtype=torch.float64)
    U = torch.randn(1, spec.B, 4, 5, dtype=torch.float64)
    Y = S.query_by_type(Phi, U, spec)
    for i in (0, 1, spec.B - 1, spec.B, spec.T_R - 1):
        assert (Y[0, i] - Phi[0, i] @ U[0, i % spec.B]).abs().max().item() < 1e-12


# --------------------------------------------------------------------------
# gradients of the oracle: central differences in fp64
# --------------------------------------------------------------------------

def test_oracle_gradients_finite_difference():
    T = 256
    spec = build_mask(T, 3, chunk=32)
    (Phi, Psi, Vb), _ = _rand(T, nb=1, r=4, d_v=3)
    torch.manual_seed(3)
    w = torch.randn(1, T, 3, dtype=torch.float64)
    xs = [t.clone().requires_grad_(True) for t in (Phi, Psi, Vb)]
    (S.smat_attention(*xs, spec, chunk=32) * w).sum().backward()
    rng = np.random.default_rng(0)
    for which in range(3):
        base = [t.detach().clone() for t in xs]
        for _ in range(6):
            idx = tuple(int(rng.integers(0, s)) for s in base[which].shape)
            if which == 2 and idx[-1] == base[2].shape[-1] - 1:
                continue
            eps = 1e-6
            plus = [t.clone() for t in base]
            minus = [t.clone() for t in base]
            plus[which][idx] += eps
            minus[which][idx] -= eps
            fd = ((S.smat_attention(*plus, spec, chunk=32) * w).sum()
                  - (S.smat_attention(*minus, spec, chunk=32) * w).sum()) / (2 * eps)
            assert abs(fd.item() - xs[which].grad[idx].item()) < 1e-6 * max(1, abs(fd.item()))


# --------------------------------------------------------------------------
# planted mistakes: each is a plausible slip, and a check above must catch it
# --------------------------------------------------------------------------

def test_planted_mistakes_are_caught(monkeypatch):
    T, d = 1024, 3
    spec = build_mask(T, d, chunk=64)
    (Phi, Psi, Vb), g = _rand(T)
    ref = S.dense_masked_kernel_attention(Phi, Psi, Vb, _dense(spec))

    def err():
        return (S.smat_attention(Phi, Psi, Vb, spec, chunk=64) - ref).abs().max().item()

    assert err() < 1e-10

    # 1. the scan never resets at n (landmark mass leaks into recent rows)
    orig = S.chunk_states

    def no_reset(Psi_c, Vb_c, n, C, acc):
        return orig(Psi_c, Vb_c, 0, C, acc)
    monkeypatch.setattr(S, "chunk_states", no_reset)
    assert err() > 1e-3
    monkeypatch.setattr(S, "chunk_states", orig)

    # 2. inclusive instead of exclusive prefix (a chunk sees itself twice)
    def inclusive(Psi_c, Vb_c, n, C, acc):
        D, Sin = orig(Psi_c, Vb_c, n, C, acc)
        return D, Sin + D
    monkeypatch.setattr(S, "chunk_states", inclusive)
    assert err() > 1e-3
    monkeypatch.setattr(S, "chunk_states", orig)

    # 3. row type i mod B off by one
    orig_q = S.query_by_type

    def shifted(Phi_rec, U, spec_):
        return orig_q(Phi_rec, torch.roll(U, 1, dims=1), spec_)
    monkeypatch.setattr(S, "query_by_type", shifted)
    assert err() > 1e-3
    monkeypatch.setattr(S, "query_by_type", orig_q)

    # 4. transposed pooled state (r x p read as p x r is shape-invalid unless
    #    r == p; use a square case so the slip type-checks)
    (P2, K2, V2), _ = _rand(T, r=13, d_v=12)
    ref2 = S.dense_masked_kernel_attention(P2, K2, V2, _dense(spec))
    orig_pool = S.pool_profiles

    def transposed(Psi_, Vb_, spec_, acc_dtype=None):
        return orig_pool(Psi_, Vb_, spec_, acc_dtype).transpose(-1, -2).contiguous()
    monkeypatch.setattr(S, "pool_profiles", transposed)
    assert (S.smat_attention(P2, K2, V2, spec, chunk=64) - ref2).abs().max().item() > 1e-3
    monkeypatch.setattr(S, "pool_profiles", orig_pool)

    # 5. causal tile includes the diagonal's upper neighbour (tril offset +1)
    orig_cl = S.chunk_local

    def leaky(Phi_c, Psi_c, Vb_c, Sin, acc=None):
        acc = acc or S.acc_of(Phi_c)
        C = Phi_c.shape[-2]
        tri = torch.ones(C, C, dtype=Phi_c.dtype).tril(1)
        A = (Phi_c @ Psi_c.transpose(-1, -2)) * tri
        return Phi_c.to(acc) @ Sin + A.to(acc) @ Vb_c.to(acc)
    monkeypatch.setattr(S, "chunk_local", leaky)
    assert err() > 1e-3
    monkeypatch.setattr(S, "chunk_local", orig_cl)
    assert err() < 1e-10


@pytest.mark.parametrize("T,n,C", [(48, 24, 8), (50, 20, 8), (37, 16, 16), (64, 0, 16)])
def test_decayed_scan_is_the_recurrence(T, n, C):
    """The chunked decayed scan (model.py:41-82) equals the recurrence run
    token by token, padded tails and a reset inside a chunk (n % C != 0: the
    reference clears the state where chunk n // C begins) included."""
    g = torch.Generator().manual_seed(T + n + C)
    nb, r, p = 2, 3, 4
    Phi, Psi = torch.rand(nb, T, r, generator=g, dtype=torch.float64), \
        torch.rand(nb, T, r, generator=g, dtype=torch.float64)
    Vb = torch.randn(nb, T, p, generator=g, dtype=torch.float64)
    logA = -torch.rand(nb, T, generator=g, dtype=torch.float64) * 2.0
    a = S.decayed_segmented_scan(Phi, Psi, Vb, logA, n, C)
    b = S.decayed_scan_tokens(Phi, Psi, Vb, logA, n, C)
    assert (a - b).abs().max().item() < 1e-12


def test_decayed_scan_without_decay_is_the_plain_scan():
    """logA = 0: every a_t is 1 and the decayed scan is the segmented causal
    scan.  And the recurrence check has teeth: a reset one chunk late, or a
    decay applied at half strength (plausible slips), miss it by far."""
    g = torch.Generator().manual_seed(3)
    nb, T, r, p, n, C = 2, 64, 4, 5, 32, 16
    Phi, Psi = torch.rand(nb, T, r, generator=g, dtype=torch.float64), \
        torch.rand(nb, T, r, generator=g, dtype=torch.float64)
    Vb = torch.randn(nb, T, p, generator=g, dtype=torch.float64)
    zero = torch.zeros(nb, T, dtype=torch.float64)
    assert (S.decayed_segmented_scan(Phi, Psi, Vb, zero, n, C)
            - S.segmented_causal_scan(Phi, Psi, Vb, n, C)).abs().max().item() < 1e-12
    logA = -torch.rand(nb, T, generator=g, dtype=torch.float64)
    ref = S.decayed_scan_tokens(Phi, Psi, Vb, logA, n, C)
    late = S.decayed_segmented_scan(Phi, Psi, Vb, logA, n + C, C)
    half = S.decayed_segmented_scan(Phi, Psi, Vb, logA / 2, n, C)
    assert (late - ref).abs().max().item() > 1e-3
    assert (half - ref).abs().max().item() > 1e-3
