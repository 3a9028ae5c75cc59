"""The forward kernels behind the ``kernels/`` dispatch, on HIP (gfx950).

Drop-in for ``src/smat/kernels/triton_fwd.py``: the same five names with the
same arguments, shapes and return dtypes --

    available()                          triton_fwd.py:38-39
    chunk_local(Phi_c, Psi_c, Vb_c, Sin) triton_fwd.py:118-152
    incidence(F, plane_pts, B)           triton_fwd.py:191-216
    pool_ok(N0, gmax, P)                 triton_fwd.py:270-278
    pool(Psi, Vb, n_P, n, N0)            triton_fwd.py:281-311

-- plus the schedule stages the reference leaves to torch (chunk summaries,
segmented scan, type-major query, normalisation), the whole forward as one
call, and the decode step.  Inputs are borrowed; outputs are allocated here
with torch's caching allocator and filled by libsmat_hip.so on torch's
current stream.  Every failure raises; nothing falls back.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from ._lib import DTYPE_CODE, HipKernelError, HipUnavailable, call, ptr, stream_of

MAX_R = 128
MAX_P = 144
MAX_C = 256

__all__ = [
    "available", "chunk_local", "incidence", "pool_ok", "pool", "incidence_plane",
    "chunk_states", "segment_scan", "causal_scan", "query", "normalise", "forward",
    "forward_workspace_bytes", "decode_step", "validate_table", "direct", "zeta", "walsh",
    "incidence_complement",
    "HipKernelError", "HipUnavailable", "MAX_R", "MAX_P", "MAX_C",
]


def available() -> bool:
    """True when libsmat_hip.so loads and a GPU is visible."""
    if not torch.cuda.is_available():
        return False
    try:
        _lib.load()
    except HipUnavailable:
        return False
    return True


# ---------------------------------------------------------------------------
# argument plumbing
# ---------------------------------------------------------------------------

def _code(t: torch.Tensor, who: str) -> int:
    try:
        return DTYPE_CODE[t.dtype]
    except KeyError:
        raise TypeError(f"{who}: dtype {t.dtype} is not one of bfloat16, float16, "
                        f"float32") from None


def _on_gpu(who: str, *ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError(f"{who}: tensors must be on the GPU (got {t.device})")


def _shape(who: str, name: str, t: torch.Tensor, want) -> None:
    """Raise ValueError unless ``t.shape`` equals ``want`` (``None`` entries match
    any size).  The kernels trust these sizes: a short buffer would be read past
    its end."""
    got = tuple(t.shape)
    if len(got) != len(want) or any(w is not None and g != w for g, w in zip(got, want)):
        shown = tuple("*" if w is None else w for w in want)
        raise ValueError(f"{who}: {name} has shape {got}, expected {shown}")


def _same_dtype(who: str, ref: torch.Tensor, **ts) -> None:
    for name, t in ts.items():
        if t is not None and t.dtype != ref.dtype:
            raise TypeError(f"{who}: {name} is {t.dtype}, expected {ref.dtype} like the "
                            f"other feature inputs")


def _rows3(t: torch.Tensor):
    """``t`` as a (batch, rows, cols) tensor with unit column stride, plus its
    batch and row strides in elements.  Copies only when no such view exists."""
    if t.stride(-1) != 1:
        t = t.contiguous()
    return t, t.stride(0), t.stride(1)


def _fp32_rows(t: torch.Tensor) -> torch.Tensor:
    t = t if t.dtype == torch.float32 else t.float()
    return t if t.stride(-1) == 1 else t.contiguous()


def validate_table(plane_pts: torch.Tensor, N0: int) -> None:
    """Check once that every point index lies in ``[0, N0)`` (the kernels trust it).

    The check is remembered on the tensor object, so a table staged by
    :func:`smat_attention_amd.attention.to_device` (which checks on the host)
    or already validated costs nothing.
    """
    if getattr(plane_pts, "_smat_checked_N0", None) == N0:
        return
    if plane_pts.numel():
        lo, hi = int(plane_pts.min()), int(plane_pts.max())
        if lo < 0 or hi >= N0:
            raise ValueError(f"incidence table entries must lie in [0, {N0}), got "
                             f"[{lo}, {hi}]")
    plane_pts._smat_checked_N0 = N0


# ---------------------------------------------------------------------------
# the reference's five functions
# ---------------------------------------------------------------------------

_FEATURE_KINDS = {"elu1": 0, "relu": 1}


def featurise(W, kind: str, Q, K=None, V=None, h=None):
    """``Phi = map(Q W^T)``, ``Psi = map(K W^T) * h``, ``Vb = [V, 1]`` in one launch
    (attention.py:82-106).  Returns ``(Phi, Psi, Vb)``, ``None`` for the parts
    not asked for; ``Vb`` is a view of rows padded to 16 bytes."""
    who = "featurise"
    _on_gpu(who, Q, W, K, V, h)
    for t in (W, K, V, h):
        if t is not None and t.dtype != Q.dtype:
            raise TypeError(f"{who}: all inputs must share Q's dtype {Q.dtype}, got {t.dtype}")
    if kind not in _FEATURE_KINDS:
        raise ValueError(f"{who}: unknown feature map {kind!r}")
    code = _code(Q, who)
    nb, T, dqk = Q.shape
    r = W.shape[0]
    if W.shape != (r, dqk):
        raise ValueError(f"{who}: W is {tuple(W.shape)}, expected ({r}, {dqk})")
    Wc = W.contiguous()
    q, q_sb, q_st = _rows3(Q)
    Phi = torch.empty(nb, T, r, device=Q.device, dtype=Q.dtype)
    Psi = k = None
    k_sb = k_st = 0
    if K is not None:
        if K.shape != Q.shape:
            raise ValueError(f"{who}: K is {tuple(K.shape)}, Q is {tuple(Q.shape)}")
        k, k_sb, k_st = _rows3(K)
        Psi = torch.empty_like(Phi)
    Vb = v = None
    v_sb = v_st = vb_sb = vb_st = 0
    d_v = 0
    if V is not None:
        if V.shape[:2] != Q.shape[:2]:
            raise ValueError(f"{who}: V is {tuple(V.shape)}, Q is {tuple(Q.shape)}")
        d_v = V.shape[-1]
        v, v_sb, v_st = _rows3(V)
        pad = -(-(d_v + 1) // 8) * 8
        buf = torch.empty(nb, T, pad, device=V.device, dtype=V.dtype)
        Vb = buf[..., :d_v + 1]
        vb_sb, vb_st = buf.stride(0), buf.stride(1)
    hc = None
    if h is not None:
        if K is None or h.shape != Q.shape[:2]:
            raise ValueError(f"{who}: the key gate h must be ({nb}, {T}) and needs K")
        hc = h.contiguous()
    call("smat_featurise", code, q.data_ptr(), ptr(k), ptr(v), Wc.data_ptr(), ptr(hc),
         Phi.data_ptr(), ptr(Psi), ptr(Vb), nb, T, dqk, r, d_v, _FEATURE_KINDS[kind],
         q_sb, q_st, k_sb, k_st, v_sb, v_st, hc.stride(0) if hc is not None else 0,
         Phi.stride(0), Phi.stride(1), vb_sb, vb_st, stream_of(Q))
    return Phi, Psi, Vb


def chunk_local(Phi_c, Psi_c, Vb_c, Sin):
    """``Phi_b Sin_b + (Phi_b Psi_b^T . L_C) Vb_b`` for every chunk, fused.

    Shapes ``(nb, nc, C, r)``, ``(nb, nc, C, r)``, ``(nb, nc, C, p)``,
    ``(nb, nc, r, p)`` -> fp32 ``(nb, nc, C, p)``.
    """
    who = "chunk_local"
    _on_gpu(who, Phi_c, Psi_c, Vb_c, Sin)
    nb, nc, C, R = Phi_c.shape
    P = Vb_c.shape[-1]
    _same_dtype(who, Phi_c, Psi_c=Psi_c, Vb_c=Vb_c)
    _shape(who, "Psi_c", Psi_c, (nb, nc, C, R))
    _shape(who, "Vb_c", Vb_c, (nb, nc, C, P))
    _shape(who, "Sin", Sin, (nb, nc, R, P))
    code = _code(Phi_c, who)
    q, q_sb, q_st = _rows3(Phi_c.reshape(nb * nc, C, R))
    k, k_sb, k_st = _rows3(Psi_c.reshape(nb * nc, C, R))
    v, v_sb, v_st = _rows3(Vb_c.reshape(nb * nc, C, P))
    s, s_sb, s_sr = _rows3(_fp32_rows(Sin).reshape(nb * nc, R, P))
    out = torch.empty(nb * nc, C, P, device=q.device, dtype=torch.float32)
    call("smat_chunk_local", code, q.data_ptr(), k.data_ptr(), v.data_ptr(), s.data_ptr(),
         out.data_ptr(), nb * nc, C, R, P, q_sb, q_st, k_sb, k_st, v_sb, v_st, s_sb, s_sr,
         out.stride(0), out.stride(1), stream_of(q))
    return out.reshape(nb, nc, C, P)


def chunk_local_decay(Phi_c, Psi_c, Vb_c, Sin, L):
    """``exp(L_m) Phi_m Sin_b + sum_{n <= m} exp(L_m - L_n) (Phi_m . Psi_n) Vb_n`` for
    every chunk (the decayed scan's within-chunk pass, model.py:60-68, 77).

    Shapes as :func:`chunk_local` plus ``L (nb, nc, C)`` fp32, the running sum
    of the log-decays within each chunk -> fp32 ``(nb, nc, C, p)``.
    """
    who = "chunk_local_decay"
    _on_gpu(who, Phi_c, Psi_c, Vb_c, Sin, L)
    nb, nc, C, R = Phi_c.shape
    P = Vb_c.shape[-1]
    _same_dtype(who, Phi_c, Psi_c=Psi_c, Vb_c=Vb_c)
    _shape(who, "Psi_c", Psi_c, (nb, nc, C, R))
    _shape(who, "Vb_c", Vb_c, (nb, nc, C, P))
    _shape(who, "Sin", Sin, (nb, nc, R, P))
    if L.shape != (nb, nc, C):
        raise ValueError(f"{who}: L is {tuple(L.shape)}, expected {(nb, nc, C)}")
    code = _code(Phi_c, who)
    q, q_sb, q_st = _rows3(Phi_c.reshape(nb * nc, C, R))
    k, k_sb, k_st = _rows3(Psi_c.reshape(nb * nc, C, R))
    v, v_sb, v_st = _rows3(Vb_c.reshape(nb * nc, C, P))
    s, s_sb, s_sr = _rows3(_fp32_rows(Sin).reshape(nb * nc, R, P))
    Lc = L.float().contiguous()
    out = torch.empty(nb * nc, C, P, device=q.device, dtype=torch.float32)
    call("smat_chunk_local_decay", code, q.data_ptr(), k.data_ptr(), v.data_ptr(), s.data_ptr(),
         Lc.data_ptr(), out.data_ptr(), nb * nc, C, R, P, q_sb, q_st, k_sb, k_st, v_sb, v_st,
         s_sb, s_sr, out.stride(0), out.stride(1), stream_of(q))
    return out.reshape(nb, nc, C, P)


def decay_scan(D, aC, nc0: int):
    """States entering each chunk of the decayed scan: ``S <- aC[c] S + D[c]``
    with one reset at chunk ``nc0`` (model.py:71-80).  ``D (nb, nc, r, p)``,
    ``aC (nb, nc)`` -> fp32 ``Sin (nb, nc, r, p)``."""
    who = "decay_scan"
    _on_gpu(who, D, aC)
    nb, nc, R, P = D.shape
    if aC.shape != (nb, nc):
        raise ValueError(f"{who}: aC is {tuple(aC.shape)}, expected {(nb, nc)}")
    Dc = D.contiguous().float()
    ac = aC.contiguous().float()
    Sin = torch.empty_like(Dc)
    call("smat_decay_scan", Dc.data_ptr(), ac.data_ptr(), Sin.data_ptr(), nb, nc, nc0, R * P,
         stream_of(Dc))
    return Sin


def incidence_plane(F, plane_code, q: int, *, F_glob=None):
    """``U_h = sum_{x in H_h} F_x`` for d = 3 with the lines generated from
    ``plane_code`` (int32 ``(B,)``, ``e*q + b``) instead of a point table."""
    who = "incidence_plane"
    _on_gpu(who, F, plane_code, F_glob)
    nb, N0, R, P = F.shape
    if plane_code.dim() != 1 or plane_code.dtype != torch.int32:
        raise ValueError(f"{who}: plane_code must be int32 (B,)")
    if q * q != N0:
        raise ValueError(f"{who}: N0={N0} is not q^2 for q={q}")
    if F_glob is not None:
        _shape(who, "F_glob", F_glob, (nb, R, P))
    B = plane_code.shape[0]
    Ff = F.contiguous().float()
    U = torch.empty(nb, B, R, P, device=F.device, dtype=torch.float32)
    call("smat_incidence_plane", Ff.data_ptr(), ptr(F_glob), plane_code.data_ptr(), q,
         U.data_ptr(), nb, N0, B, R * P, stream_of(Ff))
    return U


def incidence(F, plane_pts, B: int):
    """``U_h = sum_{x in H_h} F_x``: ``F (nb, N0, r, p) -> U (nb, B, r, p)`` fp32,
    ``plane_pts (B, deg)`` int64 or int32."""
    who = "incidence"
    _on_gpu(who, F, plane_pts)
    nb, N0, R, P = F.shape
    if plane_pts.dim() != 2 or plane_pts.shape[0] != B:
        raise ValueError(f"{who}: plane_pts must be (B={B}, deg), got {tuple(plane_pts.shape)}")
    if plane_pts.dtype not in (torch.int64, torch.int32):
        raise TypeError(f"{who}: plane_pts must be int64 or int32")
    plane_pts = plane_pts.contiguous()
    validate_table(plane_pts, N0)
    Ff = F.contiguous().float()
    U = torch.empty(nb, B, R, P, device=F.device, dtype=torch.float32)
    call("smat_incidence", Ff.data_ptr(), None, plane_pts.data_ptr(),
         int(plane_pts.dtype == torch.int64), None, int(plane_pts.shape[1]), U.data_ptr(),
         nb, N0, B, R * P, stream_of(Ff))
    return U


def pool_ok(N0: int, gmax: int, P: int) -> bool:
    """Whether the pooling kernel takes this shape.

    The reference gates its kernel to ``N0 >= 64`` because a short grid loses
    to one torch GEMM there; this kernel splits long progressions over several
    workgroups instead, so it runs at every ``N0`` and only ``P`` is bounded.
    """
    return available() and 1 <= P <= MAX_P and N0 >= 1 and gmax >= 0


def pool(Psi, Vb, n_P: int, n: int, N0: int, *, F_glob: Optional[torch.Tensor] = None):
    """``F_x = sum_{prof(j)=x} Psi_j Vb_j^T``: ``(nb, T, r), (nb, T, p) -> (nb, N0, r, p)`` fp32.

    ``F_glob`` (optional, fp32 ``(nb, r, p)``) receives the global-channel
    term ``sum_{j < n_P} Psi_j Vb_j^T`` in the same launch.
    """
    who = "pool"
    _on_gpu(who, Psi, Vb)
    nb, T, R = Psi.shape
    P = Vb.shape[-1]
    _same_dtype(who, Psi, Vb=Vb)
    _shape(who, "Vb", Vb, (nb, T, P))
    if not (0 <= n_P <= n <= T):
        raise ValueError(f"{who}: need 0 <= n_P <= n <= T, got n_P={n_P} n={n} T={T}")
    code = _code(Psi, who)
    k, k_sb, k_st = _rows3(Psi)
    v, v_sb, v_st = _rows3(Vb)
    F = torch.empty(nb, N0, R, P, device=Psi.device, dtype=torch.float32)
    if F_glob is not None:
        if F_glob.shape != (nb, R, P) or F_glob.dtype != torch.float32 or not F_glob.is_contiguous():
            raise ValueError(f"{who}: F_glob must be contiguous fp32 ({nb}, {R}, {P})")
    wsb = _lib.query("smat_pool_workspace_bytes", nb, n_P, n, N0, R, P)
    ws = torch.empty(max(wsb, 1), device=Psi.device, dtype=torch.uint8) if wsb else None
    call("smat_pool", code, k.data_ptr(), v.data_ptr(), F.data_ptr(), ptr(F_glob), nb, n_P, n,
         N0, R, P, k_sb, k_st, v_sb, v_st, ptr(ws), wsb, stream_of(k))
    return F


# ---------------------------------------------------------------------------
# schedule stages the reference runs in torch
# ---------------------------------------------------------------------------

def chunk_states(Psi, Vb, C: int):
    """``D_c = Psi_c^T Vb_c`` for the chunks of width ``C``: fp32 ``(nb, nc, r, p)``."""
    who = "chunk_states"
    _on_gpu(who, Psi, Vb)
    nb, T, R = Psi.shape
    P = Vb.shape[-1]
    _same_dtype(who, Psi, Vb=Vb)
    _shape(who, "Vb", Vb, (nb, T, P))
    code = _code(Psi, who)
    k, k_sb, k_st = _rows3(Psi)
    v, v_sb, v_st = _rows3(Vb)
    nc = -(-T // C)
    D = torch.empty(nb, nc, R, P, device=Psi.device, dtype=torch.float32)
    call("smat_chunk_states", code, k.data_ptr(), v.data_ptr(), D.data_ptr(), nb, T, C, R, P,
         k_sb, k_st, v_sb, v_st, stream_of(k))
    return D


def causal_scan(Phi, Psi, Vb, n: int, chunk: int, *, Y=None, g=None, write_H: bool = False,
                out=None):
    """The fused causal pass (chunk <= 128).  ``write_H``: fp32 ``(nb, T, p)`` H of
    the segmented scan; else the normalised fp32 ``(nb, T, p-1)`` output with
    ``Y`` (``(nb, T-n, p)``) added on recent rows and the gate ``g`` applied."""
    who = "causal_scan"
    _on_gpu(who, Phi, Psi, Vb, Y, g, out)
    nb, T, R = Phi.shape
    P = Vb.shape[-1]
    _same_dtype(who, Phi, Psi=Psi, Vb=Vb)
    _shape(who, "Psi", Psi, (nb, T, R))
    _shape(who, "Vb", Vb, (nb, T, P))
    if Y is not None:
        _shape(who, "Y", Y, (nb, T - n, P))
    if g is not None:
        _shape(who, "g", g, (nb, T))
    if out is not None and (out.shape != (nb, T, P if write_H else P - 1)
                            or out.dtype != torch.float32 or out.stride(-1) != 1):
        raise ValueError(f"{who}: out must be fp32 {(nb, T, P if write_H else P - 1)} with "
                         f"unit column stride")
    code = _code(Phi, who)
    q, q_sb, q_st = _rows3(Phi)
    k, k_sb, k_st = _rows3(Psi)
    v, v_sb, v_st = _rows3(Vb)
    Yc = _fp32_rows(Y) if Y is not None else None
    gc = g.float().contiguous() if g is not None else None
    if out is None:
        out = torch.empty(nb, T, P if write_H else P - 1, device=Phi.device, dtype=torch.float32)
    wsb = _lib.query("smat_causal_scan_workspace_bytes", nb, T, chunk, R, P)
    ws = torch.empty(wsb + 256, device=Phi.device, dtype=torch.uint8)
    base = (ws.data_ptr() + 255) & ~255
    call("smat_causal_scan", code, q.data_ptr(), k.data_ptr(), v.data_ptr(), ptr(Yc), ptr(gc),
         out.data_ptr(), nb, T, n, chunk, R, P, q_sb, q_st, k_sb, k_st, v_sb, v_st,
         Yc.stride(0) if Yc is not None else 0, Yc.stride(1) if Yc is not None else 0,
         out.stride(0), out.stride(1), gc.stride(0) if gc is not None else 0, int(write_H),
         base, wsb, stream_of(q))
    return out


def direct(Psi, Vb, cols, counts, n_P: int):
    """Unpooled ``U_h = sum_{j in cols_h} Psi_{n_P+j}^T Vb_{n_P+j}``: fp32 ``(nb, B, r, p)``.

    ``cols`` (``(B, kappa)`` int32) lists each row type's landmark columns,
    ``counts[h]`` of them first; ``counts`` is ``(B,)`` int32.
    """
    who = "direct"
    _on_gpu(who, Psi, Vb, cols, counts)
    if cols.dtype != torch.int32 or counts.dtype != torch.int32:
        raise TypeError(f"{who}: cols and counts must be int32")
    nb, T, R = Psi.shape
    P = Vb.shape[-1]
    _same_dtype(who, Psi, Vb=Vb)
    _shape(who, "Vb", Vb, (nb, T, P))
    B, kappa = cols.shape
    _shape(who, "counts", counts, (B,))
    code = _code(Psi, who)
    k, k_sb, k_st = _rows3(Psi)
    v, v_sb, v_st = _rows3(Vb)
    cc, cn = cols.contiguous(), counts.contiguous()
    U = torch.empty(nb, B, R, P, device=Psi.device, dtype=torch.float32)
    call("smat_direct", code, k.data_ptr(), v.data_ptr(), cc.data_ptr(), cn.data_ptr(), kappa,
         U.data_ptr(), nb, B, n_P, R, P, k_sb, k_st, v_sb, v_st, stream_of(k))
    return U


def _butterfly(name, F, out):
    _on_gpu(name, F, out)
    nb, N = F.shape[0], F.shape[1]
    Fc = F.contiguous().float()
    rp = Fc[0, 0].numel() if N else 0
    if out is None:
        out = torch.empty_like(Fc)
    elif out.shape != Fc.shape or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError(f"{name}: out must be contiguous fp32 of F's shape")
    call(f"smat_{name}", Fc.data_ptr(), out.data_ptr(), nb, N, rp, stream_of(Fc))
    return out


def zeta(F, *, out=None):
    """Subset sums ``Z_a = sum_{x subset of a} F_x`` over ``N = 2^k`` profiles (fp32)."""
    return _butterfly("zeta", F, out)


def walsh(F, *, out=None):
    """Endpoint incidence ``U = (sum_x F_x + H F) / 2`` over ``N = 2^k`` profiles (fp32)."""
    return _butterfly("walsh", F, out)


def incidence_complement(F, U):
    """In place ``U_h <- U_h - sum_x F_x`` (the negated complement ``-(F_tot - U)``)."""
    who = "incidence_complement"
    _on_gpu(who, F, U)
    if not (F.is_contiguous() and U.is_contiguous()) or F.dtype != torch.float32 or \
            U.dtype != torch.float32:
        raise ValueError(f"{who}: F and U must be contiguous fp32")
    nb, N0, B = F.shape[0], F.shape[1], U.shape[1]
    rp = F[0, 0].numel()
    call("smat_incidence_complement", F.data_ptr(), U.data_ptr(), nb, N0, B, rp, stream_of(F))
    return U


def segment_scan(D, nc0: int):
    """Shifted exclusive scan of ``D (nb, nc, r, p)`` with one reset at chunk ``nc0``."""
    who = "segment_scan"
    _on_gpu(who, D)
    nb, nc, R, P = D.shape
    Dc = D.contiguous().float()
    Sin = torch.empty_like(Dc)
    call("smat_segment_scan", Dc.data_ptr(), Sin.data_ptr(), nb, nc, nc0, R * P, stream_of(Dc))
    return Sin


def query(Phi_rec, U):
    """``Y[i] = Phi_rec[i] U_{i mod B}``: fp32 ``(nb, T_R, p)``.

    The result is a view whose rows are padded to a multiple of 4 floats, so
    the causal pass can read it with 16-byte loads.
    """
    who = "query"
    _on_gpu(who, Phi_rec, U)
    nb, T_R, R = Phi_rec.shape
    B, P = U.shape[1], U.shape[-1]
    _shape(who, "U", U, (nb, B, R, P))
    if B < 1:
        raise ValueError(f"{who}: U has no row types")
    code = _code(Phi_rec, who)
    q, q_sb, q_st = _rows3(Phi_rec)
    Uc = U.contiguous().float()
    Y = torch.empty(nb, T_R, (P + 3) // 4 * 4, device=U.device, dtype=torch.float32)[..., :P]
    call("smat_query", code, q.data_ptr(), Uc.data_ptr(), Y.data_ptr(), nb, T_R, B, R, P,
         q_sb, q_st, Y.stride(0), Y.stride(1), stream_of(Uc))
    return Y


def normalise(H, n: int, Y=None, g=None):
    """``(H + [0; Y])[..., :-1] / (H + [0; Y])[..., -1:]``, times ``g`` when given."""
    who = "normalise"
    _on_gpu(who, H, Y, g)
    nb, T, P = H.shape
    if Y is not None:
        _shape(who, "Y", Y, (nb, T - n, P))
    if g is not None:
        _shape(who, "g", g, (nb, T))
    Hc = _fp32_rows(H)
    Yc = _fp32_rows(Y) if Y is not None else None
    gc = g.float().contiguous() if g is not None else None
    out = torch.empty(nb, T, P - 1, device=H.device, dtype=torch.float32)
    call("smat_normalise", Hc.data_ptr(), ptr(Yc), ptr(gc), out.data_ptr(), nb, T, n, P,
         Hc.stride(0), Hc.stride(1), Yc.stride(0) if Yc is not None else 0,
         Yc.stride(1) if Yc is not None else 0, out.stride(0), out.stride(1),
         gc.stride(0) if gc is not None else 0, stream_of(Hc))
    return out


def forward_workspace_bytes(nb, T, n, N0, B, n_P, C, r, p) -> int:
    return _lib.query("smat_forward_workspace_bytes", nb, T, n, N0, B, n_P, C, r, p)


def forward(Phi, Psi, Vb, idx, deg: int, *, n: int, n_P: int, N0: int, B: int, chunk: int,
            indptr=None, plane_code=None, field_q: int = 0, g=None, out=None, H_out=None,
            workspace=None):
    """The whole forward schedule in one call; returns fp32 ``(nb, T, p-1)``.
    ``idx=None`` (with ``deg=1``, ``B=N0``, ``n_P=0``) declares the incidence the
    identity: the query reads the pooled table directly."""
    who = "forward"
    _on_gpu(who, Phi, Psi, Vb, idx, indptr, g, out, H_out)
    nb, T, R = Phi.shape
    P = Vb.shape[-1]
    _same_dtype(who, Phi, Psi=Psi, Vb=Vb)
    _shape(who, "Psi", Psi, (nb, T, R))
    _shape(who, "Vb", Vb, (nb, T, P))
    if g is not None:
        _shape(who, "g", g, (nb, T))
    code = _code(Phi, who)
    q, q_sb, q_st = _rows3(Phi)
    k, k_sb, k_st = _rows3(Psi)
    v, v_sb, v_st = _rows3(Vb)
    if out is None:
        out = torch.empty(nb, T, P - 1, device=Phi.device, dtype=torch.float32)
    elif out.shape != (nb, T, P - 1) or out.dtype != torch.float32 or out.stride(-1) != 1:
        raise ValueError(f"{who}: out must be fp32 {(nb, T, P - 1)} with unit column stride")
    if H_out is not None and (H_out.shape != (nb, T, P) or not H_out.is_contiguous()
                              or H_out.dtype != torch.float32):
        raise ValueError(f"{who}: H_out must be contiguous fp32 ({nb}, {T}, {P})")
    gc = g.float().contiguous() if g is not None else None
    need = forward_workspace_bytes(nb, T, n, N0, B, n_P, chunk, R, P)

    def _room(ws):
        # bytes left in ``ws`` once its base is rounded up to 256
        if ws is None or ws.device != Phi.device or ws.dtype != torch.uint8:
            return -1
        return ws.numel() - (((ws.data_ptr() + 255) & ~255) - ws.data_ptr())

    if _room(workspace) < need:
        workspace = torch.empty(need + 256, device=Phi.device, dtype=torch.uint8)
    base = workspace.data_ptr()
    aligned = (base + 255) & ~255
    avail = workspace.numel() - (aligned - base)
    call("smat_forward", code, q.data_ptr(), k.data_ptr(), v.data_ptr(), ptr(idx),
         int(idx is not None and idx.dtype == torch.int64), ptr(indptr), deg, ptr(plane_code),
         field_q,
         out.data_ptr(), ptr(H_out), ptr(gc),
         nb, T, n, n_P, N0, B, chunk, R, P, q_sb, q_st, k_sb, k_st, v_sb, v_st,
         out.stride(0), out.stride(1), gc.stride(0) if gc is not None else 0,
         aligned, avail, stream_of(q))
    return out


def forward_fused(W, kind: str, Q, K, V, h, idx, deg: int, *, n: int, n_P: int, N0: int, B: int,
                  chunk: int, indptr=None, plane_code=None, field_q: int = 0, g=None,
                  workspace=None):
    """:func:`forward` from Q, K, V with the feature map inside the kernels
    (``smat_forward_fused``): Phi, Psi and Vb are formed in LDS by the
    consumers and never stored.  Returns fp32 ``(nb, T, d_v)``."""
    who = "forward_fused"
    _on_gpu(who, Q, K, V, W, h, idx, indptr, g)
    nb, T, dqk = Q.shape
    for t in (K, V, W, h):
        if t is not None and t.dtype != Q.dtype:
            raise TypeError(f"{who}: all inputs must share Q's dtype {Q.dtype}, got {t.dtype}")
    if kind not in _FEATURE_KINDS:
        raise ValueError(f"{who}: unknown feature map {kind!r}")
    _shape(who, "K", K, (nb, T, dqk))
    d_v = V.shape[-1]
    _shape(who, "V", V, (nb, T, d_v))
    if h is not None:
        _shape(who, "h", h, (nb, T))
    if g is not None:
        _shape(who, "g", g, (nb, T))
    code = _code(Q, who)
    q, q_sb, q_st = _rows3(Q)
    k, k_sb, k_st = _rows3(K)
    v, v_sb, v_st = _rows3(V)
    Wc = W.contiguous()
    hc = h.contiguous() if h is not None else None
    gc = g.float().contiguous() if g is not None else None
    r, p = W.shape[0], d_v + 1
    out = torch.empty(nb, T, d_v, device=Q.device, dtype=torch.float32)
    need = _lib.query("smat_forward_fused_workspace_bytes", nb, T, n, N0, B, n_P, chunk)
    if (workspace is None or workspace.device != Q.device or workspace.dtype != torch.uint8
            or workspace.numel() < need + 256):
        workspace = torch.empty(need + 256, device=Q.device, dtype=torch.uint8)
    base = workspace.data_ptr()
    aligned = (base + 255) & ~255
    avail = workspace.numel() - (aligned - base)
    call("smat_forward_fused", code, q.data_ptr(), k.data_ptr(), v.data_ptr(), Wc.data_ptr(),
         ptr(hc), _FEATURE_KINDS[kind], ptr(idx),
         int(idx is not None and idx.dtype == torch.int64), ptr(indptr), deg, ptr(plane_code),
         field_q, out.data_ptr(), ptr(gc), nb, T, n, n_P, N0, B, chunk, q_sb, q_st, k_sb, k_st,
         v_sb, v_st, hc.stride(0) if hc is not None else 0, out.stride(0), out.stride(1),
         gc.stride(0) if gc is not None else 0, aligned, avail, stream_of(q))
    return out


def decode_step(Phi_t, Psi_t, Vb_t, S_in, S_out, U, step: int, *, out=None, o_full=None):
    """One decode step for a batch; returns fp32 ``(nb, p-1)`` and writes ``S_out``."""
    who = "decode_step"
    _on_gpu(who, Phi_t, Psi_t, Vb_t, S_in, S_out, U)
    nb, R = Phi_t.shape
    _shape(who, "U", U, (nb, None, R, None))
    B, P = U.shape[1], U.shape[3]
    _shape(who, "Psi_t", Psi_t, (nb, R))
    _shape(who, "Vb_t", Vb_t, (nb, P))
    _shape(who, "S_in", S_in, (nb, R, P))
    _shape(who, "S_out", S_out, (nb, R, P))
    _shape(who, "U", U, (nb, B, R, P))
    if B < 1:
        raise ValueError(f"{who}: U has no row types")
    if S_in.data_ptr() == S_out.data_ptr():
        raise ValueError(f"{who}: S_in and S_out must be distinct buffers")
    if not (Psi_t.dtype == Vb_t.dtype == Phi_t.dtype):
        # the reference takes each input to the accumulation dtype (fp32,
        # attention.py:522-528); mixed inputs do the same here, exactly
        for t in (Phi_t, Psi_t, Vb_t):
            _code(t, who)
        Phi_t, Psi_t, Vb_t = Phi_t.float(), Psi_t.float(), Vb_t.float()
    code = _code(Phi_t, who)
    for t in (Phi_t, Psi_t, Vb_t):
        if t.stride(-1) != 1:
            raise ValueError(f"{who}: feature rows must be contiguous")
    for t in (S_in, S_out, U):
        if not t.is_contiguous() or t.dtype != torch.float32:
            raise ValueError(f"{who}: S and U must be contiguous fp32")
    if out is None:
        out = torch.empty(nb, P - 1, device=Phi_t.device, dtype=torch.float32)
    elif out.shape != (nb, P - 1) or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError(f"{who}: out must be contiguous fp32 {(nb, P - 1)}")
    if o_full is not None and (o_full.shape != (nb, P) or o_full.dtype != torch.float32
                               or not o_full.is_contiguous()):
        raise ValueError(f"{who}: o_full must be contiguous fp32 {(nb, P)}")
    call("smat_decode_step", code, Phi_t.data_ptr(), Psi_t.data_ptr(), Vb_t.data_ptr(),
         S_in.data_ptr(), S_out.data_ptr(), U.data_ptr(), out.data_ptr(), ptr(o_full), nb, B, R,
         P, int(step), Phi_t.stride(0), Psi_t.stride(0), Vb_t.stride(0), stream_of(U))
    return out
