"""The reference's torch path for the SMat schedule, restated on CPU tensors.

Test infrastructure (see ``oracle/__init__.py``): the checker for the HIP
kernels and the CPU baseline that ``bench.py`` times.  Each function follows
the torch branch of the reference function it is named after, in the same op
order and dtype rules, so its bf16/fp32 behaviour is the reference's own
fallback and its fp64 behaviour is the exact schedule.

``spec`` arguments are any object with the attributes of a ``MaskSpec``
(``n, T_R, B, N0, n_P, kind, C_indptr, C_indices, uniform_deg``).
"""
from __future__ import annotations

import math
from typing import Dict

import numpy as np
import torch


def acc_of(x, acc_dtype=None):
    """attention.py:124-127: fp32 accumulation for half inputs, else the input dtype."""
    if acc_dtype is not None:
        return acc_dtype
    return torch.float32 if x.dtype in (torch.float16, torch.bfloat16) else x.dtype


# ---------------------------------------------------------------------------
# features (attention.py:82-106)
# ---------------------------------------------------------------------------

def phi_weight(d_qk: int, r: int, *, dtype=torch.float32, seed: int = 0):
    """``W ~ randn(r, d_qk) / sqrt(d_qk)`` from a seeded CPU generator (attention.py:89-91)."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    W = torch.randn(r, d_qk, generator=gen, dtype=torch.float64) / np.sqrt(d_qk)
    return W.to(dtype=dtype)


def make_phi(d_qk: int, r: int, *, kind: str = "elu1", dtype=torch.float32,
             seed: int = 0):
    W = phi_weight(d_qk, r, dtype=dtype, seed=seed)
    if kind == "elu1":
        return lambda x: torch.nn.functional.elu(x @ W.T) + 1.0
    if kind == "relu":
        return lambda x: torch.nn.functional.relu(x @ W.T) + 1e-3
    raise ValueError(kind)


def featurise(Q, K, V, phi, *, g=None, h=None):
    Phi = phi(Q)
    Psi = phi(K)
    if h is not None:
        Psi = Psi * h.unsqueeze(-1)
    ones = torch.ones(*V.shape[:-1], 1, dtype=V.dtype)
    return Phi, Psi, torch.cat([V, ones], dim=-1)


# ---------------------------------------------------------------------------
# causal pass (attention.py:134-192, torch branch)
# ---------------------------------------------------------------------------

def chunk_states(Psi_c, Vb_c, n: int, C: int, acc):
    """``D_b = Psi_b^T Vb_b`` and the per-segment shifted exclusive scan ``Sin``."""
    nb, nc = Psi_c.shape[:2]
    nc0 = n // C
    D = Psi_c.to(acc).transpose(-1, -2) @ Vb_c.to(acc)
    Sin = torch.zeros_like(D)
    bounds = [(0, nc0), (nc0, nc)] if 0 < nc0 < nc else [(0, nc)]
    for lo, hi in bounds:
        if hi - lo > 1:
            Sin[:, lo + 1:hi] = torch.cumsum(D[:, lo:hi - 1], dim=1)
    return D, Sin


def chunk_local(Phi_c, Psi_c, Vb_c, Sin, acc=None):
    """``Phi_b Sin_b + (tril(Phi_b Psi_b^T)) Vb_b``; the score tile in the input dtype."""
    acc = acc or acc_of(Phi_c)
    C = Phi_c.shape[-2]
    inter = Phi_c.to(acc) @ Sin.to(acc)
    tri = torch.ones(C, C, dtype=Phi_c.dtype).tril()
    A = (Phi_c @ Psi_c.transpose(-1, -2)) * tri
    return inter + A.to(acc) @ Vb_c.to(acc)


def segmented_causal_scan(Phi, Psi, Vb, n: int, chunk: int = 128, acc_dtype=None):
    nb, T, r = Phi.shape
    p = Vb.shape[-1]
    C = min(chunk, T)
    if n % C:
        raise ValueError(f"segment boundary n={n} is not a multiple of chunk={C}")
    acc = acc_of(Phi, acc_dtype)
    pad = (-T) % C
    if pad:
        Phi = torch.nn.functional.pad(Phi, (0, 0, 0, pad))
        Psi = torch.nn.functional.pad(Psi, (0, 0, 0, pad))
        Vb = torch.nn.functional.pad(Vb, (0, 0, 0, pad))
    nc = (T + pad) // C
    Phi_c = Phi.reshape(nb, nc, C, r)
    Psi_c = Psi.reshape(nb, nc, C, r)
    Vb_c = Vb.reshape(nb, nc, C, p)
    _, Sin = chunk_states(Psi_c, Vb_c, n, C, acc)
    out = chunk_local(Phi_c, Psi_c, Vb_c, Sin, acc)
    return out.reshape(nb, T + pad, p)[:, :T]


def decayed_segmented_scan(Phi, Psi, Vb, logA, n: int, chunk: int = 128):
    """model.py:41-82: the chunked decayed scan, fp32 in the reference (here the
    inputs' dtype, so fp64 inputs give the fp64 restatement)."""
    nb, T, r = Phi.shape
    p = Vb.shape[-1]
    C = min(chunk, T)
    pad = (-T) % C
    if pad:
        Phi = torch.nn.functional.pad(Phi, (0, 0, 0, pad))
        Psi = torch.nn.functional.pad(Psi, (0, 0, 0, pad))
        Vb = torch.nn.functional.pad(Vb, (0, 0, 0, pad))
        logA = torch.nn.functional.pad(logA, (0, pad))
    nc = (T + pad) // C
    nc0 = n // C
    Phi_c, Psi_c = Phi.reshape(nb, nc, C, r), Psi.reshape(nb, nc, C, r)
    Vb_c, la = Vb.reshape(nb, nc, C, p), logA.reshape(nb, nc, C)
    L = torch.cumsum(la, dim=-1)
    tri = torch.ones(C, C, dtype=torch.bool).tril()
    diff = (L.unsqueeze(-1) - L.unsqueeze(-2)).masked_fill(~tri, float("-inf"))
    A = (Phi_c @ Psi_c.transpose(-1, -2)) * torch.exp(diff)
    out = A @ Vb_c
    wj = torch.exp(L[..., -1:] - L)
    D = (Psi_c * wj.unsqueeze(-1)).transpose(-1, -2) @ Vb_c
    aC = torch.exp(L[..., -1])
    S = torch.zeros(nb, r, p, dtype=Phi.dtype)
    rows = []
    for b in range(nc):
        if b == nc0:
            S = torch.zeros_like(S)
        rows.append(out[:, b] + (Phi_c[:, b] * torch.exp(L[:, b]).unsqueeze(-1)) @ S)
        S = aC[:, b].view(nb, 1, 1) * S + D[:, b]
    return torch.stack(rows, 1).reshape(nb, nc * C, p)[:, :T]


def decayed_scan_tokens(Phi, Psi, Vb, logA, n: int, chunk: int = 128):
    """The recurrence itself, token by token (for small checks): S_t =
    a_t S_{t-1} + psi_t vb_t^T, y_t = Phi_t S_t, the state cleared where chunk
    n // chunk begins (model.py:75-76 resets at that chunk)."""
    nb, T, r = Phi.shape
    p = Vb.shape[-1]
    C = min(chunk, T)
    reset = (n // C) * C
    S = torch.zeros(nb, r, p, dtype=Phi.dtype)
    ys = []
    for t in range(T):
        if t == reset:
            S = torch.zeros_like(S)
        S = torch.exp(logA[:, t]).view(nb, 1, 1) * S + Psi[:, t].unsqueeze(-1) * Vb[:, t].unsqueeze(1)
        ys.append(torch.einsum("br,brp->bp", Phi[:, t], S))
    return torch.stack(ys, 1)


# ---------------------------------------------------------------------------
# long range (attention.py:199-330, torch branches)
# ---------------------------------------------------------------------------

def pool_profiles(Psi, Vb, spec, acc_dtype=None):
    """``F_x = sum_{prof(j)=x} Psi_j Vb_j^T`` as a batched GEMM (attention.py:223-236)."""
    nb = Psi.shape[0]
    r, p = Psi.shape[-1], Vb.shape[-1]
    acc = acc_of(Psi, acc_dtype)
    n_P, n, N0 = spec.n_P, spec.n, spec.N0
    Ps, Vs = Psi[:, n_P:n], Vb[:, n_P:n]
    g, rem = divmod(n - n_P, N0)
    F = torch.zeros(nb, N0, r, p, dtype=acc)
    if g:
        A = Ps[:, :g * N0].reshape(nb, g, N0, r).permute(0, 2, 3, 1)
        Bm = Vs[:, :g * N0].reshape(nb, g, N0, p).permute(0, 2, 1, 3)
        F = A.to(acc) @ Bm.to(acc)
    if rem:
        F[:, :rem] += (Ps[:, g * N0:].to(acc).unsqueeze(-1)
                       * Vs[:, g * N0:].to(acc).unsqueeze(-2))
    return F


def plane_table(spec):
    """``(B, deg)`` int64 point table when every row of ``C`` has one degree."""
    if not spec.uniform_deg:
        return None
    return torch.from_numpy(spec.C_indices.astype(np.int64)).view(spec.B, spec.uniform_deg)


def apply_incidence(F, spec, gather_chunk: int = 0):
    """``U_h = sum_{x in H_h} F_x`` by a chunked gather (attention.py:267-285)."""
    nb, N0, r, p = F.shape
    B = spec.B
    if spec.kind == "endpoint":
        return walsh_incidence(F)
    plane = plane_table(spec)
    U = torch.zeros(nb, B, r, p, dtype=F.dtype)
    if plane is None:
        ptr = spec.C_indptr
        idx_all = torch.from_numpy(spec.C_indices.astype(np.int64))
        for h in range(B):
            U[:, h] = F[:, idx_all[int(ptr[h]):int(ptr[h + 1])]].sum(1)
        return U
    deg = plane.shape[1]
    step = gather_chunk or max(1, min(deg, (1 << 28) // max(1, nb * B * r * p)))
    for lo in range(0, deg, step):
        idx = plane[:, lo:lo + step].reshape(-1)
        s = idx.numel() // B
        U += F[:, idx].reshape(nb, B, s, r, p).sum(2)
    return U


def apply_incidence_csr(F, spec):
    """The ragged CSR loop of attention.py:268-274, for any mask kind."""
    nb, N0, r, p = F.shape
    U = torch.zeros(nb, spec.B, r, p, dtype=F.dtype)
    ptr = spec.C_indptr
    idx_all = torch.from_numpy(spec.C_indices.astype(np.int64))
    for h in range(spec.B):
        U[:, h] = F[:, idx_all[int(ptr[h]):int(ptr[h + 1])]].sum(1)
    return U


def walsh_incidence(F):
    """``C = (J + H)/2`` applied by a Walsh-Hadamard butterfly (attention.py:288-307)."""
    nb, N, r, p = F.shape
    k = N.bit_length() - 1
    assert 1 << k == N
    tot = F.sum(1, keepdim=True)
    H = F.reshape(nb, N, r * p).clone()
    for j in range(k):
        lo = 1 << j
        H = H.reshape(nb, N // (2 * lo), 2, lo, r * p)
        a, b = H[:, :, 0].clone(), H[:, :, 1].clone()
        H[:, :, 0] = a + b
        H[:, :, 1] = a - b
        H = H.reshape(nb, N, r * p)
    return 0.5 * (tot + H.reshape(nb, N, r, p))


def zeta_transform(F):
    """Subset sums ``(Z_k F)_a = sum_{x subseteq a} F_x`` (attention.py:369-384)."""
    nb, N, r, p = F.shape
    k = N.bit_length() - 1
    assert 1 << k == N
    H = F.reshape(nb, N, r * p).clone()
    for j in range(k):
        lo = 1 << j
        H = H.reshape(nb, N // (2 * lo), 2, lo, r * p)
        H[:, :, 1] += H[:, :, 0]
        H = H.reshape(nb, N, r * p)
    return H.reshape(nb, N, r, p)


def query_by_type(Phi_rec, U, spec):
    """``Y_{R_h} = Phi_{R_h} U_h``, stride-B rows lined up by a reshape (attention.py:310-330)."""
    nb, T_R, r = Phi_rec.shape
    B, p = spec.B, U.shape[-1]
    acc = U.dtype
    out = torch.empty(nb, T_R, p, dtype=acc)
    c = T_R // B
    if c:
        head = Phi_rec[:, :c * B].reshape(nb, c, B, r).transpose(1, 2)
        out[:, :c * B] = (head.to(acc) @ U).transpose(1, 2).reshape(nb, c * B, p)
    rem = T_R - c * B
    if rem:
        tail = Phi_rec[:, c * B:].to(acc).unsqueeze(-2)
        out[:, c * B:] = (tail @ U[:, :rem]).squeeze(-2)
    return out


def type_columns(spec) -> np.ndarray:
    """``(B, kappa)`` landmark columns of each row type, padded with ``n_X`` (attention.py:558-571)."""
    n_X, N0 = spec.n_X, spec.N0
    g = -(-n_X // N0)
    pts = spec.C_indices.reshape(spec.B, -1).astype(np.int64)
    base = pts[:, :, None] + np.arange(g, dtype=np.int64)[None, None, :] * N0
    return np.where(base < n_X, base, n_X).reshape(spec.B, -1).astype(np.int32)


def direct_long_range(Psi, Vb, spec, acc_dtype=None, type_chunk: int = 64):
    """Unpooled ``U_h = sum_{j: prof(j) in H_h} Psi_j Vb_j^T`` (attention.py:333-362)."""
    nb = Psi.shape[0]
    r, p = Psi.shape[-1], Vb.shape[-1]
    acc = acc_of(Psi, acc_dtype)
    cols = torch.from_numpy(type_columns(spec).astype(np.int64))
    B, kap = cols.shape
    Ps = torch.cat([Psi[:, spec.n_P:spec.n], Psi.new_zeros(nb, 1, r)], dim=1)
    Vs = torch.cat([Vb[:, spec.n_P:spec.n], Vb.new_zeros(nb, 1, p)], dim=1)
    U = torch.empty(nb, B, r, p, dtype=acc)
    for lo in range(0, B, type_chunk):
        hi = min(lo + type_chunk, B)
        c = cols[lo:hi].reshape(-1)
        Pk = Ps[:, c].reshape(nb, hi - lo, kap, r)
        Vk = Vs[:, c].reshape(nb, hi - lo, kap, p)
        U[:, lo:hi] = Pk.to(acc).transpose(-1, -2) @ Vk.to(acc)
    return U


# ---------------------------------------------------------------------------
# full forward (attention.py:391-482)
# ---------------------------------------------------------------------------

def smat_attention(Phi, Psi, Vb, spec, *, chunk: int = 128, g=None,
                   acc_dtype=None, long_range: str = "pooled",
                   return_parts: bool = False):
    nb, T, r = Phi.shape
    n = spec.n
    acc = acc_of(Phi, acc_dtype)
    parts: Dict[str, torch.Tensor] = {}
    if long_range == "subtractive":
        F = pool_profiles(Psi, Vb, spec, acc_dtype=acc)
        U = apply_incidence(F, spec)
        Ubar = F.sum(1, keepdim=True) - U
        Y_ex = query_by_type(Phi[:, n:], Ubar, spec)
        H = segmented_causal_scan(Phi, Psi, Vb, n=0, chunk=chunk, acc_dtype=acc)
        H = torch.cat([H[:, :n], H[:, n:] - Y_ex], dim=1)
        out = H[..., :-1] / H[..., -1:]
        if g is not None:
            out = out * g.unsqueeze(-1).to(out.dtype)
        return (out, {"H": H, "Y_ex": Y_ex}) if return_parts else out

    F = pool_profiles(Psi, Vb, spec, acc_dtype=acc)
    if long_range == "direct":
        U = direct_long_range(Psi, Vb, spec, acc_dtype=acc)
    else:
        U = apply_incidence(F, spec)
    if spec.n_P:
        b = Psi[:, :spec.n_P].to(acc).transpose(-1, -2) @ Vb[:, :spec.n_P].to(acc)
        U = U + b.unsqueeze(1)
    Y_lr = query_by_type(Phi[:, n:], U, spec)

    if spec.kind == "endpoint":
        Fz = Psi[:, :n].to(acc).unsqueeze(-1) * Vb[:, :n].to(acc).unsqueeze(-2)
        top = (Phi[:, :n].to(acc).unsqueeze(-2) @ zeta_transform(Fz)).squeeze(-2)
        loc = segmented_causal_scan(Phi[:, n:], Psi[:, n:], Vb[:, n:], n=0,
                                    chunk=chunk, acc_dtype=acc)
        H = torch.cat([top, loc + Y_lr], dim=1)
        parts["zeta"] = top
    else:
        H = segmented_causal_scan(Phi, Psi, Vb, n=n, chunk=chunk, acc_dtype=acc)
        H = torch.cat([H[:, :n], H[:, n:] + Y_lr], dim=1)
    parts.update(U=U, Y_lr=Y_lr, H=H)
    out = H[..., :-1] / H[..., -1:]
    if g is not None:
        out = out * g.unsqueeze(-1).to(out.dtype)
    return (out, parts) if return_parts else out


def dense_masked_kernel_attention(Phi, Psi, Vb, M):
    """The ``O(T^2)`` definition (attention.py:485-489)."""
    A = torch.einsum("nta,nsa->nts", Phi, Psi) * M
    H = torch.einsum("nts,nsv->ntv", A, Vb)
    return H[..., :-1] / H[..., -1:]


def dense_masked_normaliser(Phi, Psi, Vb, M):
    """``H[..., p-1]`` of the definition: the normaliser whose log is compared."""
    A = torch.einsum("nta,nsa->nts", Phi, Psi) * M
    return torch.einsum("nts,ns->nt", A, Vb[..., -1])


# ---------------------------------------------------------------------------
# streaming decode (attention.py:496-535)
# ---------------------------------------------------------------------------

class SmatDecoder:
    def __init__(self, Psi_prefix, Vb_prefix, spec, *, acc_dtype=None):
        self.spec = spec
        acc = acc_of(Psi_prefix, acc_dtype)
        self.acc = acc
        nb, _, r = Psi_prefix.shape
        p = Vb_prefix.shape[-1]
        F = pool_profiles(Psi_prefix, Vb_prefix, spec, acc_dtype=acc)
        self.U = apply_incidence(F, spec)
        if spec.n_P:
            b = (Psi_prefix[:, :spec.n_P].to(acc).transpose(-1, -2)
                 @ Vb_prefix[:, :spec.n_P].to(acc))
            self.U = self.U + b.unsqueeze(1)
        self.S = torch.zeros(nb, r, p, dtype=acc)
        self.i = 0

    def step(self, Phi_t, Psi_t, Vb_t):
        self.S += Psi_t.to(self.acc).unsqueeze(-1) * Vb_t.to(self.acc).unsqueeze(-2)
        H = self.S + self.U[:, self.i % self.spec.B]
        o = (Phi_t.to(self.acc).unsqueeze(-2) @ H).squeeze(-2)
        self.i += 1
        return o[..., :-1] / o[..., -1:]

    def step_H(self, Phi_t, Psi_t, Vb_t):
        """As :meth:`step`, returning the unnormalised ``o`` (numerator and normaliser)."""
        self.S += Psi_t.to(self.acc).unsqueeze(-1) * Vb_t.to(self.acc).unsqueeze(-2)
        H = self.S + self.U[:, self.i % self.spec.B]
        self.i += 1
        return (Phi_t.to(self.acc).unsqueeze(-2) @ H).squeeze(-2)

    def cache_words(self) -> int:
        return int(self.S.numel() + self.U.numel())


# ---------------------------------------------------------------------------
# helpers for the checks
# ---------------------------------------------------------------------------

def log_normaliser(Phi, Psi, Vb, spec, *, chunk: int = 128, acc_dtype=None):
    """``log H[..., p-1]``: the quantity compared at 1e-3 for half-precision runs."""
    _, parts = smat_attention(Phi, Psi, Vb, spec, chunk=chunk, acc_dtype=acc_dtype,
                              return_parts=True)
    return torch.log(parts["H"][..., -1])


def seeded_qkv(nb: int, T: int, d_qk: int, d_v: int, *, seed: int = 0,
               dtype=torch.float32, q_scale: float = 1.0, k_scale: float = 1.0,
               v_scale: float = 1.0):
    """``q, k, v ~ N(0, 1)`` drawn on the CPU from ``seed``, then scaled and cast."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    Q = torch.randn(nb, T, d_qk, generator=gen) * q_scale
    K = torch.randn(nb, T, d_qk, generator=gen) * k_scale
    V = torch.randn(nb, T, d_v, generator=gen) * v_scale
    return Q.to(dtype), K.to(dtype), V.to(dtype)


def rel_err(a, b) -> float:
    """``max|a - b| / max|b|``."""
    return float((a.double() - b.double()).abs().max() / b.double().abs().max().clamp_min(1e-300))


def isfinite_all(*ts) -> bool:
    return all(bool(torch.isfinite(t).all()) for t in ts)


__all__ = [n for n in dir() if not n.startswith("_") and n not in ("math", "np", "torch", "Dict")]
