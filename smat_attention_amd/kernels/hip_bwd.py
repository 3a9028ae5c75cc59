"""Gradients of the SMat schedule on HIP (gfx950).

Counterpart of ``src/smat/kernels/triton_bwd.py``.  The reference wraps its
three forward kernels in autograd Functions and patches them into the kernel
table (``patch()``, triton_bwd.py:334-346), leaving the rest of the schedule
(chunk summaries, cumsum, query, normalise) to torch autograd; its fused
backward kernels also stop at ``r, p <= 128`` (triton_bwd.py:166-167).  Here
the whole schedule is one autograd Function whose backward runs on the HIP
kernels for any ``r <= 128, p <= 144``:

    out = H[:, :-1] / H[:, -1] * g,     H = H_causal + [0; Y],
    H_causal  per chunk b:  Phi_b S_b + tril(Phi_b Psi_b^T) Vb_b
    Y_i = Phi_i U_{i mod B},   U_h = sum_{x in H_h} F_x (+ F_glob),
    F_x = sum_{j: prof(j) = x} Psi_j Vb_j^T

    dH            normalise backward
    causal        dA = tril(dH_b Vb_b^T),  A = tril(Phi_b Psi_b^T),
                  Q_b = sum over later chunks of the segment of Phi^T dH,
                  dPhi_b = dH_b S_b^T + dA Psi_b
                  dPsi_b = Vb_b Q_b^T + dA^T Phi_b
                  dVb_b  = Psi_b Q_b + A^T dH_b
    long range    dPhi_i += dY_i U_h^T,  dU_h = sum_{i in R_h} Phi_i^T dY_i,
                  dF = C^T dU (incidence over the transposed table),
                  dPsi_j += dF_x Vb_j,  dVb_j += dF_x^T Psi_j   (j in profile x)

Every product runs on ``smat_bgemm`` (fp32 MFMA, fp32 accumulation), so the
gradients are fp32 products summed in fp32 from the stored inputs; they are
returned in the input dtype, as the reference does.
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from . import _lib
from ._lib import DTYPE_CODE, call, ptr, stream_of
from . import hip_fwd as _hip

__all__ = ["smat_attention_grad", "SmatAttentionFunction", "DecayedScanFunction",
           "transposed_incidence",
           "chunk_local", "pool", "incidence", "patch", "unpatch", "patched"]

# the forward kernels as imported, before patch() swaps the module attributes
_FWD = {"chunk_local": _hip.chunk_local, "pool": _hip.pool, "incidence": _hip.incidence}

def _code(t):
    return DTYPE_CODE[t.dtype]


def _bgemm(A, B, C, *, M, N, K, n1, n2, a, b, c, beta=0, mask=0, a_off=0, b_off=0, c_off=0):
    """C[i] (+)= A[i] B[i] with element strides a = (a1, a2, am, ak), b = (b1, b2, bk, bn),
    c = (c1, c2, cm, cn); *_off are element offsets added to the base pointers."""
    if M <= 0 or N <= 0 or n1 <= 0 or n2 <= 0:
        return
    # host-side bounds check: the last element each operand addresses must lie
    # inside its tensor's storage (all strides here are non-negative)
    for name, t, off, (s1, s2, sr, sc), rows, cols in (
            ("A", A, a_off, a, M, K), ("B", B, b_off, b, K, N), ("C", C, c_off, c, M, N)):
        if rows <= 0 or cols <= 0:
            continue
        last = off + (n1 - 1) * s1 + (n2 - 1) * s2 + (rows - 1) * sr + (cols - 1) * sc
        avail = t.untyped_storage().nbytes() // t.element_size() - t.storage_offset()
        if min(s1, s2, sr, sc, off) < 0 or last >= avail:
            raise ValueError(f"smat_bgemm operand {name}: element {last} addressed, "
                             f"{avail} available")
    ea, eb = A.element_size(), B.element_size()
    call("smat_bgemm", _code(A), _code(B), A.data_ptr() + a_off * ea, B.data_ptr() + b_off * eb,
         C.data_ptr() + c_off * 4, M, N, K, n1, n2, *a, *b, *c, beta, mask, stream_of(C))


def transposed_incidence(spec, device):
    """CSR (indptr, idx) of C^T: for every point x, the row types h whose
    hyperplane contains x (ascending h); cached on the spec."""
    key = ("_smat_CT", str(device))
    hit = getattr(spec, "_smat_CT", None)
    if hit is not None and hit[0] == key:
        return hit[1], hit[2]
    ptr_ = np.asarray(spec.C_indptr, dtype=np.int64)
    ind = np.asarray(spec.C_indices, dtype=np.int64)
    rows = np.repeat(np.arange(spec.B, dtype=np.int64), np.diff(ptr_))
    order = np.lexsort((rows, ind))
    counts = np.bincount(ind, minlength=spec.N0)
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    idx = rows[order].astype(np.int32)
    t_ptr = torch.from_numpy(indptr).to(device)
    t_idx = torch.from_numpy(idx).to(device)
    t_idx._smat_checked_N0 = spec.B
    spec._smat_CT = (key, t_ptr, t_idx)
    return t_ptr, t_idx


def recent_token_lists(spec, device):
    """CSR ``(tptr, tok)`` (int32) of the recent rows feeding each pooled item's
    gradient: for point x < N0, the rows n + h + k*B < T of every row type h
    whose hyperplane contains x (the transposed incidence, each line's rows in
    order); when n_P > 0, item N0 (the global channel) lists every recent row.
    Cached on the spec."""
    key = ("_smat_RT", str(device))
    hit = getattr(spec, "_smat_RT", None)
    if hit is not None and hit[0] == key:
        return hit[1], hit[2]
    n, T_R, B, N0 = spec.n, spec.T_R, spec.B, spec.N0
    ptr_ = np.asarray(spec.C_indptr, dtype=np.int64)
    ind = np.asarray(spec.C_indices, dtype=np.int64)
    lines = np.repeat(np.arange(B, dtype=np.int64), np.diff(ptr_))
    order = np.lexsort((lines, ind))
    pts, lines = ind[order], lines[order]
    h = np.arange(B, dtype=np.int64)
    cnt = np.where(h < T_R, (T_R - h + B - 1) // B, 0)
    per = cnt[lines]
    parts = [n + hh + B * np.arange(c, dtype=np.int64) for hh, c in zip(lines.tolist(), per.tolist())]
    counts = np.bincount(pts, weights=per, minlength=N0).astype(np.int64)
    if spec.n_P:
        parts.append(np.arange(n, n + T_R, dtype=np.int64))
        counts = np.concatenate([counts, [T_R]])
    tok = np.concatenate(parts) if parts else np.zeros(0, np.int64)
    tptr = np.concatenate([[0], np.cumsum(counts)])
    assert tptr[-1] == len(tok) < 2 ** 31
    out = (torch.from_numpy(tptr.astype(np.int32)).to(device),
           torch.from_numpy(tok.astype(np.int32)).to(device))
    spec._smat_RT = (key,) + out
    return out


# The long-range backward kernels (smat_lr_dphi, smat_lr_dfeat,
# smat_pool_backward) serve bf16 inputs at r = 64, p = 65; tests switch them
# off to compare with the smat_bgemm products they replace.  They split fp32
# operands (dH ~ dout / den, U, dF) into bf16 hi/lo pairs, which keeps fp32's
# exponent range; fp16 pairs would overflow above 65504 and lose the lo
# correction below 6e-5, so fp16 inputs take the fp32 smat_bgemm products.
FUSED_LONG_RANGE_BACKWARD = True


def long_range_backward_ok(Ph, Ps, Vv) -> bool:
    return (FUSED_LONG_RANGE_BACKWARD and Ph.dtype == torch.bfloat16
            and Ps.dtype == Ph.dtype and Vv.dtype == Ph.dtype
            and Ph.shape[-1] == 64 and Ps.shape[-1] == 64 and Vv.shape[-1] == 65
            and Ph.stride(-1) == 1 and Ps.stride(-1) == 1 and Vv.stride(-1) == 1
            and Ph.stride(1) % 8 == 0 and Ps.stride(1) % 8 == 0
            and Ph.stride(0) % 8 == 0 and Ps.stride(0) % 8 == 0
            and Ph.data_ptr() % 16 == 0 and Ps.data_ptr() % 16 == 0)


def _incidence_rows(src, idx, indptr, n_out, nb, n_in, rp):
    """out[b, y] = sum_{t in row y} src[b, idx[t]] over (n_in)-row fp32 panels."""
    out = torch.empty(nb, n_out, rp, device=src.device, dtype=torch.float32)
    call("smat_incidence", src.data_ptr(), None, idx.data_ptr(), 0, ptr(indptr), 0,
         out.data_ptr(), nb, n_in, n_out, rp, stream_of(src))
    return out


# The fused chunk backward (smat_chunk_backward) serves bf16 inputs at
# r = 64, p = 65, C = 128 (its hi/lo operand split needs bf16's exponent
# range, as above); tests switch it off to compare it with the chain of
# smat_bgemm products it replaces.
FUSED_CHUNK_BACKWARD = True


def fused_chunk_backward_ok(Ph, Ps, Vv, C: int) -> bool:
    return (FUSED_CHUNK_BACKWARD and Ph.dtype == torch.bfloat16
            and Ps.dtype == Ph.dtype and Vv.dtype == Ph.dtype and C == 128
            and Ph.shape[-1] == 64 and Ps.shape[-1] == 64 and Vv.shape[-1] == 65
            and Ph.stride(-1) == 1 and Ps.stride(-1) == 1 and Vv.stride(-1) == 1
            and Ph.stride(1) % 8 == 0 and Ps.stride(1) % 8 == 0
            and Ph.stride(0) % 8 == 0 and Ps.stride(0) % 8 == 0
            and Ph.data_ptr() % 16 == 0 and Ps.data_ptr() % 16 == 0)


def causal_scan_grad(Ph, Ps, Vv, dH, n: int, C: int, out_dtype=None, add=None):
    """``(dPhi, dPsi, dVb)`` of the segmented causal scan ``H`` (attention.py:134-192)
    given ``dH``: inputs padded to whole chunks of ``C`` rows, ``(nb, Tp, .)``
    gradients (the rows past the input are zero-padding), fp32 -- or, with
    ``out_dtype`` the inputs' 16-bit type and the fused chunk backward serving
    the shape, rounded to that type by the kernel that forms them.  ``add``
    (fused chunk backward only): ``(aPhi, aPsi, aVb, split, end)``, fp32 terms
    the kernel adds before the store -- aPhi's rows [split, end) to dPhi,
    aPsi's and aVb's rows [0, split) to dPsi and dVb (absolute row indices;
    aPsi / aVb may be None).  Chunk states and their per-segment exclusive
    scan, the reverse scan of ``Phi_b^T dH_b``, and the per-chunk products, all
    on smat_bgemm and the segment-scan kernels."""
    nb, Tp, r = Ph.shape
    p = Vv.shape[-1]
    nc = Tp // C
    dev = Ph.device
    fused = fused_chunk_backward_ok(Ph, Ps, Vv, C)
    if add is not None and not fused:
        raise ValueError("causal_scan_grad: added terms need the fused chunk backward")
    gdt = out_dtype if (fused and out_dtype == Ph.dtype) else torch.float32
    dPhi = torch.empty(nb, Tp, r, device=dev, dtype=gdt)
    dPsi = torch.empty(nb, Tp, r, device=dev, dtype=gdt)
    dVb = torch.empty(nb, Tp, p, device=dev, dtype=gdt)
    D = _hip.chunk_states(Ps, Vv, C)                    # (nb, nc, r, p)
    Sin = _hip.segment_scan(D, n // C)
    Dr = torch.empty(nb, nc, r, p, device=dev, dtype=torch.float32)
    rp = r * p
    # Dr_b = Phi_b^T dH_b (rows of Phi and dH at their own strides)
    qb, qt = Ph.stride(0), Ph.stride(1)
    hb, ht = dH.stride(0), dH.stride(1)
    if fused:
        call("smat_chunk_dstates", _code(Ph), Ph.data_ptr(), dH.data_ptr(), Dr.data_ptr(), nb,
             nc, r, p, C, qb, qt, hb, ht, stream_of(Dr))
    else:
        _bgemm(Ph, dH, Dr, M=r, N=p, K=C, n1=nb, n2=nc,
               a=(qb, C * qt, 1, qt), b=(hb, C * ht, ht, 1), c=(nc * rp, rp, p, 1))
    Q = torch.empty_like(Dr)
    call("smat_segment_scan_reverse", Dr.data_ptr(), Q.data_ptr(), nb, nc, n // C, rp,
         stream_of(Q))
    del Dr
    if fused:
        # A and dA stay on chip: one launch for the six products below
        aP, aS, aV, split, end = add if add is not None else (None, None, None, 0, 0)

        def sb(x, i):
            return x.stride(i) if x is not None else 0
        call("smat_chunk_backward", _code(Ph), _code(dPhi), Ph.data_ptr(), Ps.data_ptr(),
             Vv.data_ptr(), dH.data_ptr(), Sin.data_ptr(), Q.data_ptr(), dPhi.data_ptr(),
             dPsi.data_ptr(), dVb.data_ptr(), nb, nc, r, p, C, Ph.stride(0), Ph.stride(1),
             Ps.stride(0), Ps.stride(1), Vv.stride(0), Vv.stride(1), dH.stride(0), dH.stride(1),
             dPhi.stride(0), dPhi.stride(1), dVb.stride(0), dVb.stride(1), ptr(aP), ptr(aS),
             ptr(aV), sb(aP, 0), sb(aP, 1), sb(aS, 0), sb(aS, 1), sb(aV, 0), sb(aV, 1), split, end,
             stream_of(dPhi))
        return dPhi, dPsi, dVb
    # the products below address Phi, Psi, Vb and dH as contiguous rows
    Ph, Ps, Vv, dH = (x.contiguous() for x in (Ph, Ps, Vv, dH))
    A = torch.empty(nb, nc, C, C, device=dev, dtype=torch.float32)
    dA = torch.empty_like(A)
    CC = C * C
    # A = tril(Phi_b Psi_b^T), dA = tril(dH_b Vb_b^T)
    _bgemm(Ph, Ps, A, M=C, N=C, K=r, n1=nb, n2=nc,
           a=(Tp * r, C * r, r, 1), b=(Tp * r, C * r, 1, r), c=(nc * CC, CC, C, 1), mask=1)
    _bgemm(dH, Vv, dA, M=C, N=C, K=p, n1=nb, n2=nc,
           a=(Tp * p, C * p, p, 1), b=(Tp * p, C * p, 1, p), c=(nc * CC, CC, C, 1), mask=1)
    cr, cp_ = (Tp * r, C * r, r, 1), (Tp * p, C * p, p, 1)
    # dPhi = dH S^T + dA Psi
    _bgemm(dH, Sin, dPhi, M=C, N=r, K=p, n1=nb, n2=nc,
           a=cp_, b=(nc * rp, rp, 1, p), c=cr)
    _bgemm(dA, Ps, dPhi, M=C, N=r, K=C, n1=nb, n2=nc,
           a=(nc * CC, CC, C, 1), b=cr, c=cr, beta=1)
    # dPsi = Vb Q^T + dA^T Phi
    _bgemm(Vv, Q, dPsi, M=C, N=r, K=p, n1=nb, n2=nc,
           a=cp_, b=(nc * rp, rp, 1, p), c=cr)
    _bgemm(dA, Ph, dPsi, M=C, N=r, K=C, n1=nb, n2=nc,
           a=(nc * CC, CC, 1, C), b=cr, c=cr, beta=1)
    # dVb = Psi Q + A^T dH
    _bgemm(Ps, Q, dVb, M=C, N=p, K=r, n1=nb, n2=nc,
           a=cr, b=(nc * rp, rp, p, 1), c=cp_)
    _bgemm(A, dH, dVb, M=C, N=p, K=C, n1=nb, n2=nc,
           a=(nc * CC, CC, 1, C), b=cp_, c=cp_, beta=1)
    del A, dA, Sin, Q, D

    return dPhi, dPsi, dVb


def _type_read_grad(Ph, dH, Uc, dPhi, Tp: int, row0: int, nrows: int, B: int):
    """The type-major read's backward (query_by_type, attention.py:310-330): rows
    ``row0 + h + k*B`` (k*B + h < nrows) read table ``U[h]``.  Accumulates
    ``dPhi[row] += dH[row] U[h]^T`` and returns ``dU[h] = sum Phi[row]^T dH[row]``,
    fp32 (nb, B, r, p).  Ph, dH, dPhi are (nb, Tp, .) rows; on smat_bgemm."""
    nb, _, r = Ph.shape
    p = dH.shape[-1]
    rp = r * p
    Brp = B * rp
    dU = torch.empty(nb, B, r, p, device=Ph.device, dtype=torch.float32)
    full, rem = divmod(nrows, B)
    # rows of type h: row0 + h + k*B; first `full` rounds for every type, then
    # one more row for types h < rem
    if full:
        _bgemm(dH, Uc, dPhi, M=full, N=r, K=p, n1=nb, n2=B,
               a=(Tp * p, p, B * p, 1), b=(Brp, rp, 1, p), c=(Tp * r, r, B * r, 1),
               beta=1, a_off=row0 * p, c_off=row0 * r)
        _bgemm(Ph, dH, dU, M=r, N=p, K=full, n1=nb, n2=B,
               a=(Tp * r, r, 1, B * r), b=(Tp * p, p, B * p, 1), c=(Brp, rp, p, 1),
               a_off=row0 * r, b_off=row0 * p)
    else:
        dU.zero_()
    if rem:
        t0 = row0 + full * B
        _bgemm(dH, Uc, dPhi, M=1, N=r, K=p, n1=nb, n2=rem,
               a=(Tp * p, p, 0, 1), b=(Brp, rp, 1, p), c=(Tp * r, r, 0, 1),
               beta=1, a_off=t0 * p, c_off=t0 * r)
        _bgemm(Ph, dH, dU, M=r, N=p, K=1, n1=nb, n2=rem,
               a=(Tp * r, r, 1, 0), b=(Tp * p, p, 0, 1), c=(Brp, rp, p, 1),
               beta=1 if full else 0, a_off=t0 * r, b_off=t0 * p)
        if not full and rem < B:
            dU[:, rem:] = 0
    return dU


def _profile_pool_grad(Ps, Vv, dF, dPsi, dVb, Tp: int, n_P: int, n: int, N0: int):
    """The profile pool's backward (pool_profiles, attention.py:199-236): token
    ``n_P + x + s*N0 < n`` adds ``Psi^T Vb`` to profile x, so
    ``dPsi[tok] += dF[x] Vb[tok]`` and ``dVb[tok] += dF[x]^T Psi[tok]``; on
    smat_bgemm.  dF is (nb, N0, r*p) fp32."""
    nb, _, r = Ps.shape
    p = Vv.shape[-1]
    rp = r * p
    Nrp = N0 * rp
    gq, grem = divmod(n - n_P, N0)
    # pool backward over profile x's tokens n_P + x + s*N0
    for lo, hi, cnt in ((0, grem, gq + 1), (grem, N0, gq)):
        if hi <= lo or cnt <= 0:
            continue
        tok0 = n_P + lo
        _bgemm(Vv, dF, dPsi, M=cnt, N=r, K=p, n1=nb, n2=hi - lo,
               a=(Tp * p, p, N0 * p, 1), b=(Nrp, rp, 1, p), c=(Tp * r, r, N0 * r, 1),
               beta=1, a_off=tok0 * p, b_off=lo * rp, c_off=tok0 * r)
        _bgemm(Ps, dF, dVb, M=cnt, N=p, K=r, n1=nb, n2=hi - lo,
               a=(Tp * r, r, N0 * r, 1), b=(Nrp, rp, p, 1), c=(Tp * p, p, N0 * p, 1),
               beta=1, a_off=tok0 * r, b_off=lo * rp, c_off=tok0 * p)


def smat_attention_grad(Phi, Psi, Vb, spec, U, H, dout, *, chunk: int = 128, g=None,
                        need_dg: bool = False, out_dtype=None):
    """``(dPhi, dPsi, dVb, dg)`` of ``out = smat_attention(Phi, Psi, Vb, spec, g=g)``
    given the forward's ``U`` (nb, B, r, p) and ``H`` (nb, T, p, long-range
    term included), fp32 gradients -- or, with ``out_dtype`` the inputs'
    16-bit type where the fused kernels serve the shape, gradients rounded to
    that type once, by the kernel that adds the last term (dg stays fp32)."""
    nb, T, r = Phi.shape
    p = Vb.shape[-1]
    C = min(chunk, T)
    n, n_P, N0, B = spec.n, spec.n_P, spec.N0, spec.B
    T_R = T - n
    dev = Phi.device
    nc = -(-T // C)
    Tp = nc * C

    # ---- normalise --------------------------------------------------------
    dout = dout.float().contiguous()
    H = H.float().contiguous()
    dH = torch.empty(nb, Tp, p, device=dev, dtype=torch.float32)
    if Tp > T:
        dH[:, T:].zero_()                                              # padding rows
    dg = torch.empty(nb, T, device=dev, dtype=torch.float32) if need_dg else None
    gc = g.float().contiguous() if g is not None else None
    call("smat_normalise_backward", dout.data_ptr(), H.data_ptr(), ptr(gc), dH.data_ptr(),
         ptr(dg), nb, T, p, dout.stride(0), dout.stride(1), H.stride(0), H.stride(1),
         dH.stride(0), dH.stride(1), gc.stride(0) if gc is not None else 0, stream_of(dH))

    # inputs padded to whole chunks (zeros contribute nothing); rows of unit
    # column stride are used where they lie
    def padded(x):
        x = x if x.stride(-1) == 1 else x.contiguous()
        if Tp == T:
            return x
        out = torch.zeros(nb, Tp, x.shape[-1], device=dev, dtype=x.dtype)
        out[:, :T] = x
        return out

    Ph, Ps, Vv = padded(Phi), padded(Psi), padded(Vb)
    rp = r * p

    if (T_R > 0 and long_range_backward_ok(Ph, Ps, Vv) and fused_chunk_backward_ok(Ph, Ps, Vv, C)
            and out_dtype == Ph.dtype):
        # the long-range terms first, stored as fp32 rows (each row has one
        # row type, each landmark row one profile): the chunk backward adds
        # them to the causal terms and rounds each sum once
        st = stream_of(dH)
        Uc = U.float().contiguous()
        code = _code(Ph)
        aPhi = torch.empty(nb, T, r, device=dev, dtype=torch.float32)     # rows [n, T)
        call("smat_lr_dphi", code, dH.data_ptr(), Uc.data_ptr(), aPhi.data_ptr(), nb, T_R, B, n,
             r, p, dH.stride(0), dH.stride(1), Uc.stride(0), aPhi.stride(0), aPhi.stride(1), 0,
             st)
        aPsi = aVb = None
        if n > 0:
            tptr, tok = recent_token_lists(spec, dev)
            nitems = N0 + (1 if n_P else 0)
            dF = torch.empty(nb, nitems, r, p, device=dev, dtype=torch.float32)
            call("smat_lr_dfeat", code, Ph.data_ptr(), dH.data_ptr(), tptr.data_ptr(),
                 tok.data_ptr(), dF.data_ptr(), nb, nitems, r, p, Ph.stride(0), Ph.stride(1),
                 dH.stride(0), dH.stride(1), dF.stride(0), st)
            aPsi = torch.empty(nb, n, r, device=dev, dtype=torch.float32)
            aVb = torch.empty(nb, n, p, device=dev, dtype=torch.float32)
            call("smat_pool_backward", code, Ps.data_ptr(), Vv.data_ptr(), dF.data_ptr(),
                 aPsi.data_ptr(), aVb.data_ptr(), nb, N0, n, n_P, r, p, Ps.stride(0),
                 Ps.stride(1), Vv.stride(0), Vv.stride(1), dF.stride(0), aPsi.stride(0),
                 aPsi.stride(1), aVb.stride(0), aVb.stride(1), 0, st)
            del dF
        dPhi, dPsi, dVb = causal_scan_grad(Ph, Ps, Vv, dH, n, C, out_dtype=out_dtype,
                                           add=(aPhi, aPsi, aVb, n, T))
        return dPhi[:, :T], dPsi[:, :T], dVb[:, :T], dg

    dPhi, dPsi, dVb = causal_scan_grad(Ph, Ps, Vv, dH, n, C)

    # ---- long range --------------------------------------------------------
    if T_R > 0 and long_range_backward_ok(Ph, Ps, Vv):
        # three streaming launches: the query's dPhi, dF = C^T dU straight
        # from the token lists (dU never stored), the pool backward
        st = stream_of(dPhi)
        Uc = U.float().contiguous()
        code = _code(Ph)
        call("smat_lr_dphi", code, dH.data_ptr(), Uc.data_ptr(), dPhi.data_ptr(), nb, T_R, B, n,
             r, p, dH.stride(0), dH.stride(1), Uc.stride(0), dPhi.stride(0), dPhi.stride(1), 1,
             st)
        tptr, tok = recent_token_lists(spec, dev)
        nitems = N0 + (1 if n_P else 0)
        dF = torch.empty(nb, nitems, r, p, device=dev, dtype=torch.float32)
        call("smat_lr_dfeat", code, Ph.data_ptr(), dH.data_ptr(), tptr.data_ptr(),
             tok.data_ptr(), dF.data_ptr(), nb, nitems, r, p, Ph.stride(0), Ph.stride(1),
             dH.stride(0), dH.stride(1), dF.stride(0), st)
        call("smat_pool_backward", code, Ps.data_ptr(), Vv.data_ptr(), dF.data_ptr(),
             dPsi.data_ptr(), dVb.data_ptr(), nb, N0, n, n_P, r, p, Ps.stride(0), Ps.stride(1),
             Vv.stride(0), Vv.stride(1), dF.stride(0), dPsi.stride(0), dPsi.stride(1),
             dVb.stride(0), dVb.stride(1), 1, st)
    elif T_R > 0:
        # the products below address Phi, Psi and Vb as dense rows (the
        # feature map's Vb rows are padded to 8 elements)
        Ph, Ps, Vv = (x.contiguous() for x in (Ph, Ps, Vv))
        Uc = U.float().contiguous()
        dU = _type_read_grad(Ph, dH, Uc, dPhi, Tp, n, T_R, B)
        # dF = C^T dU (and the global channel's sum over all types)
        if getattr(spec, "incidence_identity", False):
            dF = dU.view(nb, N0, rp)                 # C = I: C^T dU = dU
        else:
            t_ptr, t_idx = transposed_incidence(spec, dev)
            dF = _incidence_rows(dU, t_idx, t_ptr, N0, nb, B, rp)
        _profile_pool_grad(Ps, Vv, dF, dPsi, dVb, Tp, n_P, n, N0)
        if n_P:
            allrows = torch.arange(B, device=dev, dtype=torch.int32)
            allrows._smat_checked_N0 = B
            aptr = torch.tensor([0, B], device=dev, dtype=torch.int64)
            dFg = _incidence_rows(dU, allrows, aptr, 1, nb, B, rp)
            _bgemm(Vv, dFg, dPsi, M=n_P, N=r, K=p, n1=nb, n2=1,
                   a=(Tp * p, 0, p, 1), b=(rp, 0, 1, p), c=(Tp * r, 0, r, 1), beta=1)
            _bgemm(Ps, dFg, dVb, M=n_P, N=p, K=r, n1=nb, n2=1,
                   a=(Tp * r, 0, r, 1), b=(rp, 0, p, 1), c=(Tp * p, 0, p, 1), beta=1)
    return dPhi[:, :T], dPsi[:, :T], dVb[:, :T], dg


class SmatAttentionFunction(torch.autograd.Function):
    """``smat_attention`` on a geometric mask with its HIP backward.  The
    direct and subtractive long-range schedules compute the same function as
    the pooled one (the masked attention of attention.py:391-482), so their
    gradient is the pooled schedule's: the forward runs the requested
    schedule, the backward the pooled one on the pooled schedule's tables."""

    @staticmethod
    def forward(ctx, Phi, Psi, Vb, g, spec, chunk, long_range="pooled"):
        from .. import attention as A
        args = (Phi.detach(), Psi.detach(), Vb.detach(), spec)
        gd = None if g is None else g.detach()
        out, parts = A.smat_attention(*args, chunk=chunk, g=gd, long_range=long_range,
                                      return_parts=True, _no_grad_fn=True)
        if "U" not in parts:                 # subtractive: the pooled tables for the backward
            _, parts = A.smat_attention(*args, chunk=chunk, g=gd, return_parts=True,
                                        _no_grad_fn=True)
        ctx.save_for_backward(Phi, Psi, Vb, g, parts["U"], parts["H"])
        ctx.spec, ctx.chunk = spec, chunk
        return out

    @staticmethod
    def backward(ctx, dout):
        Phi, Psi, Vb, g, U, H = ctx.saved_tensors
        need_dg = g is not None and ctx.needs_input_grad[3]
        dPhi, dPsi, dVb, dg = smat_attention_grad(Phi, Psi, Vb, ctx.spec, U, H, dout,
                                                  chunk=ctx.chunk, g=g, need_dg=need_dg,
                                                  out_dtype=Phi.dtype)
        return (dPhi.to(Phi.dtype) if ctx.needs_input_grad[0] else None,
                dPsi.to(Psi.dtype) if ctx.needs_input_grad[1] else None,
                dVb.to(Vb.dtype) if ctx.needs_input_grad[2] else None,
                dg.to(g.dtype) if need_dg else None, None, None, None)


class EndpointAttentionFunction(torch.autograd.Function):
    """``smat_attention`` on the endpoint mask (attention.py:430-441) with its
    gradient: every landmark token is its own profile and every recent row
    its own type (n = N0 = B = 2^k, n_P = 0).  Forward: landmark row t reads
    ``Z_t = sum_{x subset of t} Psi_x^T Vb_x`` (zeta), recent rows run the
    causal scan restarted at n plus the long-range read of ``U = C F`` with
    ``C[h, a] = 1{popcount(h & a) even}``.  Backward: the normalisation's,
    the restarted scan's (causal_scan_grad), the two type reads'
    (``_type_read_grad``: rows n + i read U, landmark rows read Z), then
    ``dF = C dU`` (C is symmetric: the Walsh kernel) plus the superset sums of
    dZ (zeta conjugated by the index complement, ``x -> N0 - 1 - x``), then
    the pool's (``_profile_pool_grad``).  The direct and subtractive long
    range are the same function, so they share this backward."""

    @staticmethod
    def forward(ctx, Phi, Psi, Vb, g, spec, chunk, long_range="pooled"):
        from .. import attention as A
        if spec.n_P or not (spec.n == spec.N0 == spec.B):
            raise NotImplementedError("smat_attention: endpoint gradients need n = N0 = B and "
                                      "n_P = 0")
        args = (Phi.detach(), Psi.detach(), Vb.detach(), spec)
        gd = None if g is None else g.detach()
        out, parts = A.smat_attention(*args, chunk=chunk, g=gd, long_range=long_range,
                                      return_parts=True, _no_grad_fn=True)
        if "U" not in parts:
            _, parts = A.smat_attention(*args, chunk=chunk, g=gd, return_parts=True,
                                        _no_grad_fn=True)
        ctx.save_for_backward(Phi, Psi, Vb, g, parts["U"], parts["H"])
        ctx.spec, ctx.chunk = spec, chunk
        return out

    @staticmethod
    def backward(ctx, dout):
        Phi, Psi, Vb, g, U, H = ctx.saved_tensors
        spec, C = ctx.spec, ctx.chunk
        nb, T, r = Phi.shape
        p = Vb.shape[-1]
        n, N0 = spec.n, spec.N0
        T_R = T - n
        dev = Phi.device
        need_dg = g is not None and ctx.needs_input_grad[3]
        # ---- normalise
        dout = dout.float().contiguous()
        Hc = H.float().contiguous()
        dH = torch.empty(nb, T, p, device=dev, dtype=torch.float32)
        dg = torch.empty(nb, T, device=dev, dtype=torch.float32) if need_dg else None
        gc = g.float().contiguous() if g is not None else None
        call("smat_normalise_backward", dout.data_ptr(), Hc.data_ptr(), ptr(gc), dH.data_ptr(),
             ptr(dg), nb, T, p, dout.stride(0), dout.stride(1), Hc.stride(0), Hc.stride(1),
             dH.stride(0), dH.stride(1), gc.stride(0) if gc is not None else 0, stream_of(dH))
        Ph, Ps, Vv = Phi.contiguous(), Psi.contiguous(), Vb.contiguous()
        dPhi = torch.zeros(nb, T, r, device=dev, dtype=torch.float32)
        dPsi = torch.zeros(nb, T, r, device=dev, dtype=torch.float32)
        dVb = torch.zeros(nb, T, p, device=dev, dtype=torch.float32)
        # ---- the recent block's causal scan, restarted at n (rows padded to whole chunks)
        if T_R:
            Tr = -(-T_R // C) * C

            def padded(x):
                out = torch.zeros(nb, Tr, x.shape[-1], device=dev, dtype=x.dtype)
                out[:, :T_R] = x[:, n:]
                return out
            gP, gS, gV = causal_scan_grad(padded(Ph), padded(Ps), padded(Vv), padded(dH), 0, C)
            dPhi[:, n:] = gP[:, :T_R]
            dPsi[:, n:] = gS[:, :T_R]
            dVb[:, n:] = gV[:, :T_R]
        # ---- the two type reads: recent rows read U, landmark rows read Z
        dF = torch.zeros(nb, N0, r, p, device=dev, dtype=torch.float32)
        if T_R:
            dU = _type_read_grad(Ph, dH, U.float().contiguous(), dPhi, T, n, T_R, spec.B)
            dF += _hip.walsh(dU)                                  # C^T dU = C dU
        if n:
            Z = _hip.zeta(_hip.pool(Ps, Vv, 0, n, N0))
            dZ = _type_read_grad(Ph, dH, Z, dPhi, T, 0, n, N0)
            dF += _hip.zeta(dZ.flip(1).contiguous()).flip(1)    # superset sums
            _profile_pool_grad(Ps, Vv, dF.view(nb, N0, r * p), dPsi, dVb, T, 0, n, N0)
        return (dPhi.to(Phi.dtype) if ctx.needs_input_grad[0] else None,
                dPsi.to(Psi.dtype) if ctx.needs_input_grad[1] else None,
                dVb.to(Vb.dtype) if ctx.needs_input_grad[2] else None,
                dg.to(g.dtype) if need_dg else None, None, None, None)


class CausalScanFunction(torch.autograd.Function):
    """``segmented_causal_scan`` with its HIP backward (:func:`causal_scan_grad`);
    the reference differentiates its torch path (attention.py:134-192)."""

    @staticmethod
    def forward(ctx, Phi, Psi, Vb, n, C, run):
        H = run(Phi.detach(), Psi.detach(), Vb.detach())
        ctx.save_for_backward(Phi, Psi, Vb)
        ctx.n, ctx.C = n, C
        return H

    @staticmethod
    def backward(ctx, dH):
        Phi, Psi, Vb = ctx.saved_tensors
        nb, T, r = Phi.shape
        C = ctx.C
        Tp = -(-T // C) * C

        def padded(x, dt=None):
            x = x if dt is None else x.to(dt)
            x = x if x.stride(-1) == 1 else x.contiguous()
            if Tp == T:
                return x
            out = torch.zeros(nb, Tp, x.shape[-1], device=x.device, dtype=x.dtype)
            out[:, :T] = x
            return out
        dPhi, dPsi, dVb = causal_scan_grad(padded(Phi), padded(Psi), padded(Vb),
                                           padded(dH, torch.float32), ctx.n, C,
                                           out_dtype=Phi.dtype)
        return (dPhi[:, :T].to(Phi.dtype), dPsi[:, :T].to(Psi.dtype), dVb[:, :T].to(Vb.dtype),
                None, None, None)


class DecayedScanFunction(torch.autograd.Function):
    """``decayed_segmented_scan`` (model.py:41-82) with its backward on HIP.

    Per chunk, with ``A = Phi Psi^T``, ``W_ij = exp(L_i - L_j)`` (j <= i),
    ``e_i = exp(L_i)``, ``w_j = exp(L_C - L_j)``, the state ``Sin`` entering
    the chunk and ``dO`` the output gradient::

        dPhi  = e (dO Sin^T) + (dO Vb^T . W) Psi
        dPsi  = (dO Vb^T . W)^T Phi + w (Vb dD^T)
        dVb   = (A . W)^T dO + w (Psi dD)
        dSin  = Phi^T (e dO);   dD by the reverse recurrence (smat_decay_scan_reverse)
        dL_i  = rowsum_i(P) - colsum_i(P) + e_i (Phi_i Sin) . dO_i - w_i (Psi_i dD) . Vb_i
        dL_C += sum_j w_j (Psi_j dD) . Vb_j + exp(L_C) <dD, Sin>,   P = A . W . (dO Vb^T)

    and ``dlogA`` the reverse running sum of ``dL`` inside each chunk.  The
    products run on smat_bgemm (fp32 MFMA), the (C, C) weightings and row
    scales on torch elementwise kernels."""

    @staticmethod
    def forward(ctx, Phi, Psi, Vb, logA, n, C):
        from .. import attention as A
        Ph, Ps, Vv, la = A._decayed_inputs(Phi.detach(), Psi.detach(), Vb.detach(),
                                           logA.detach(), C)
        out, L, Sin = A._decayed_forward(Ph, Ps, Vv, la, n, C)
        ctx.save_for_backward(Ph, Ps, Vv, L, Sin)
        ctx.meta = (n, C, Phi.shape[1], Phi.dtype, Psi.dtype, Vb.dtype, logA.dtype)
        return out[:, :Phi.shape[1]]

    @staticmethod
    def backward(ctx, dout):
        Ph, Ps, Vv, L, Sin = ctx.saved_tensors
        n, C, T, d_phi, d_psi, d_vb, d_la = ctx.meta
        nb, Tp, r = Ph.shape
        p = Vv.shape[-1]
        nc = Tp // C
        dev = Ph.device
        rp, CC = r * p, C * C
        dO = torch.zeros(nb, Tp, p, device=dev, dtype=torch.float32)
        dO[:, :T] = dout.float()
        cr, cp_ = (Tp * r, C * r, r, 1), (Tp * p, C * p, p, 1)
        cc_ = (nc * CC, CC, C, 1)
        e = torch.exp(L)                                            # (nb, nc, C)
        w = torch.exp(L[..., -1:] - L)
        tri = torch.ones(C, C, device=dev, dtype=torch.bool).tril()
        Wd = torch.exp((L.unsqueeze(-1) - L.unsqueeze(-2)).masked_fill(~tri, float("-inf")))
        A = torch.empty(nb, nc, C, C, device=dev, dtype=torch.float32)
        dA = torch.empty_like(A)
        _bgemm(Ph, Ps, A, M=C, N=C, K=r, n1=nb, n2=nc,
               a=(Tp * r, C * r, r, 1), b=(Tp * r, C * r, 1, r), c=cc_, mask=1)
        _bgemm(dO, Vv, dA, M=C, N=C, K=p, n1=nb, n2=nc,
               a=(Tp * p, C * p, p, 1), b=(Tp * p, C * p, 1, p), c=cc_, mask=1)
        AW = A * Wd
        dAW = dA * Wd
        P = AW * dA
        dL = P.sum(-1) - P.sum(-2)
        del A, dA, P, Wd
        # dPhi = e (dO Sin^T) + dAW Psi
        dPhi = torch.empty(nb, Tp, r, device=dev, dtype=torch.float32)
        _bgemm(dO, Sin, dPhi, M=C, N=r, K=p, n1=nb, n2=nc,
               a=cp_, b=(nc * rp, rp, 1, p), c=cr)
        dPhi.view(nb, nc, C, r).mul_(e.unsqueeze(-1))
        _bgemm(dAW, Ps, dPhi, M=C, N=r, K=C, n1=nb, n2=nc, a=cc_, b=cr, c=cr, beta=1)
        # dSin = Phi^T (e dO), then the reverse recurrence
        dOe = (dO.view(nb, nc, C, p) * e.unsqueeze(-1)).reshape(nb, Tp, p)
        dSin = torch.empty(nb, nc, r, p, device=dev, dtype=torch.float32)
        _bgemm(Ph, dOe, dSin, M=r, N=p, K=C, n1=nb, n2=nc,
               a=(Tp * r, C * r, 1, r), b=cp_, c=(nc * rp, rp, p, 1))
        del dOe
        aC = e[..., -1].contiguous()
        dD = torch.empty_like(dSin)
        call("smat_decay_scan_reverse", dSin.data_ptr(), aC.data_ptr(), dD.data_ptr(), nb, nc,
             n // C, rp, stream_of(dD))
        del dSin
        # dPsi = dAW^T Phi + w (Vb dD^T)
        dPsi = torch.empty(nb, Tp, r, device=dev, dtype=torch.float32)
        _bgemm(dAW, Ph, dPsi, M=C, N=r, K=C, n1=nb, n2=nc,
               a=(nc * CC, CC, 1, C), b=cr, c=cr)
        X = torch.empty(nb, Tp, r, device=dev, dtype=torch.float32)
        _bgemm(Vv, dD, X, M=C, N=r, K=p, n1=nb, n2=nc, a=cp_, b=(nc * rp, rp, 1, p), c=cr)
        dPsi.view(nb, nc, C, r).add_(X.view(nb, nc, C, r) * w.unsqueeze(-1))
        del X, dAW
        # dVb = AW^T dO + w (Psi dD); the summaries' weights' gradient from the same product
        dVb = torch.empty(nb, Tp, p, device=dev, dtype=torch.float32)
        _bgemm(AW, dO, dVb, M=C, N=p, K=C, n1=nb, n2=nc,
               a=(nc * CC, CC, 1, C), b=cp_, c=cp_)
        del AW
        Y = torch.empty(nb, Tp, p, device=dev, dtype=torch.float32)
        _bgemm(Ps, dD, Y, M=C, N=p, K=r, n1=nb, n2=nc, a=cr, b=(nc * rp, rp, p, 1), c=cp_)
        Yc = Y.view(nb, nc, C, p)
        dVb.view(nb, nc, C, p).add_(Yc * w.unsqueeze(-1))
        wdw = w * (Yc * Vv.view(nb, nc, C, p)).sum(-1)               # w_j (Psi_j dD) . Vb_j
        dL -= wdw
        dL[..., -1] += wdw.sum(-1) + aC * (dD * Sin).sum((-2, -1))
        # the inter-chunk term's row scale: e_i (Phi_i Sin) . dO_i
        _bgemm(Ph, Sin, Y, M=C, N=p, K=r, n1=nb, n2=nc, a=cr, b=(nc * rp, rp, p, 1), c=cp_)
        dL += e * (Yc * dO.view(nb, nc, C, p)).sum(-1)
        del Y, Yc, dD
        dla = torch.flip(torch.cumsum(torch.flip(dL, [-1]), -1), [-1]).reshape(nb, Tp)
        return (dPhi[:, :T].to(d_phi), dPsi[:, :T].to(d_psi), dVb[:, :T].to(d_vb),
                dla[:, :T].to(d_la), None, None)


class FeaturiseFunction(torch.autograd.Function):
    """``featurise`` / the feature map (attention.py:82-106) with gradients:
    forward the HIP launch; backward, with ``y = x W^T`` and ``m`` the map,
    ``dx = (dPhi * m'(y)) W``, ``dW = sum (dPhi * m'(y))^T x`` for the query
    and gated key maps, ``dh = sum_r dPsi * m(y_k)`` and ``dV = dVb[..., :d_v]``.
    ``m'`` is 1 above 0 and ``e^y`` (elu + 1) or 0 (relu) below; the products
    are plain GEMMs in fp32."""

    @staticmethod
    def forward(ctx, W, kind, Q, K, V, h):
        Phi, Psi, Vb = _hip.featurise(W.detach(), kind, Q.detach(),
                                         None if K is None else K.detach(),
                                         None if V is None else V.detach(),
                                         None if h is None else h.detach())
        ctx.save_for_backward(W, Q, K, h)
        ctx.kind = kind
        ctx.d_v = None if V is None else V.shape[-1]
        ctx.v_dtype = None if V is None else V.dtype
        return Phi, Psi, Vb

    @staticmethod
    def backward(ctx, dPhi, dPsi, dVb):
        W, Q, K, h = ctx.saved_tensors
        if fused_featurise_backward_ok(W, Q, K, h, dPhi, dPsi):
            return _featurise_backward_fused(ctx, W, Q, K, h, dPhi, dPsi, dVb)
        W32 = W.float()

        def dmap(y):
            pos = y > 0
            if ctx.kind == "elu1":
                return torch.where(pos, torch.ones_like(y), torch.exp(torch.clamp(y, max=0.0)))
            return pos.to(y.dtype)

        def fmap(y):
            if ctx.kind == "elu1":
                return torch.nn.functional.elu(y) + 1.0
            return torch.nn.functional.relu(y) + 1e-3
        dW = torch.zeros_like(W32) if ctx.needs_input_grad[0] else None
        dQ = dK = dV = dh = None
        if dPhi is not None:
            x = Q.float()
            y = x @ W32.T
            gq = dPhi.float() * dmap(y)
            dQ = (gq @ W32).to(Q.dtype)
            if dW is not None:
                dW += gq.reshape(-1, gq.shape[-1]).T @ x.reshape(-1, x.shape[-1])
        if K is not None and dPsi is not None:
            x = K.float()
            y = x @ W32.T
            gk = dPsi.float()
            if h is not None:
                dh = (gk * fmap(y)).sum(-1).to(h.dtype)
                gk = gk * h.float().unsqueeze(-1)
            gk = gk * dmap(y)
            dK = (gk @ W32).to(K.dtype)
            if dW is not None:
                dW += gk.reshape(-1, gk.shape[-1]).T @ x.reshape(-1, x.shape[-1])
        if ctx.d_v is not None and dVb is not None:
            dV = dVb[..., :ctx.d_v].to(ctx.v_dtype)
        return (dW.to(W.dtype) if dW is not None else None, None, dQ, dK, dV, dh)


# The fused feature-map backward (smat_featurise_backward) serves 16-bit
# inputs at d_qk = r = 64; tests switch it off to compare with the torch
# products it replaces.
FUSED_FEATURISE_BACKWARD = True


def _rows_ok(t):
    return (t.stride(-1) == 1 and t.stride(1) % 8 == 0 and t.stride(0) % 8 == 0
            and t.data_ptr() % 16 == 0)


def fused_featurise_backward_ok(W, Q, K, h, dPhi, dPsi) -> bool:
    if not FUSED_FEATURISE_BACKWARD or Q.dtype not in (torch.bfloat16, torch.float16):
        return False
    if W.shape != (64, 64) or Q.shape[-1] != 64 or W.dtype != Q.dtype:
        return False
    for t in (K, dPhi, dPsi):
        if t is not None and (t.dtype != Q.dtype or t.shape[-1] != 64 or not _rows_ok(t)):
            return False
    return _rows_ok(Q) and (h is None or h.dtype == Q.dtype)


def _featurise_backward_fused(ctx, W, Q, K, h, dPhi, dPsi, dVb):
    """FeaturiseFunction's backward on smat_featurise_backward: one launch per
    map (recomputed y, the map's derivative, the gate, dx and the partial dW
    sums) and a reduction of dW."""
    dev = Q.device
    nb, T, _ = Q.shape
    Wc = W.contiguous()
    code = _code(Q)
    kind = 0 if ctx.kind == "elu1" else 1
    parts = max(1, int(_lib.query("smat_featurise_backward_parts", nb, T)))
    dWp = torch.empty(parts, 64, 64, device=dev, dtype=torch.float32)
    dW32 = torch.zeros(64, 64, device=dev, dtype=torch.float32)
    beta = 0
    dQ = dK = dV = dh = None
    st = stream_of(Q)
    for X, G, hh, want in ((Q, dPhi, None, True), (K, dPsi, h, K is not None)):
        if not want or G is None:
            continue
        dX = torch.empty(nb, T, 64, device=dev, dtype=X.dtype)
        dhh = torch.empty(nb, T, device=dev, dtype=hh.dtype) if hh is not None else None
        hc = hh.contiguous() if hh is not None else None
        call("smat_featurise_backward", code, X.data_ptr(), G.data_ptr(), Wc.data_ptr(),
             ptr(hc), dX.data_ptr(), dWp.data_ptr(), dW32.data_ptr(), ptr(dhh), nb, T, 64, 64,
             kind, beta, X.stride(0), X.stride(1), G.stride(0), G.stride(1),
             hc.stride(0) if hc is not None else 0, dX.stride(0), dX.stride(1),
             dhh.stride(0) if dhh is not None else 0, st)
        beta = 1
        if X is Q:
            dQ = dX
        else:
            dK, dh = dX, dhh
    if ctx.d_v is not None and dVb is not None:
        dV = dVb[..., :ctx.d_v].to(ctx.v_dtype)
    dW = dW32.to(W.dtype) if ctx.needs_input_grad[0] else None
    return (dW, None, dQ, dK, dV, dh)


# ---------------------------------------------------------------------------
# The three kernels as autograd Functions (triton_bwd.py:154-316).  Products
# run on smat_bgemm (fp32 MFMA, fp32 accumulation) from the stored inputs.
# ---------------------------------------------------------------------------

class _ChunkLocalFn(torch.autograd.Function):
    """``out = Phi_c Sin + tril(Phi_c Psi_c^T) Vb_c`` per chunk (triton_bwd.py:154-197):
    dPhi = dO Sin^T + tril(dO Vb^T) Psi,  dPsi = tril(dO Vb^T)^T Phi,
    dVb = tril(Phi Psi^T)^T dO,  dSin = Phi^T dO."""

    @staticmethod
    def forward(ctx, Phi_c, Psi_c, Vb_c, Sin):
        out = _FWD["chunk_local"](Phi_c, Psi_c, Vb_c, Sin)
        ctx.save_for_backward(Phi_c, Psi_c, Vb_c, Sin)
        return out

    @staticmethod
    def backward(ctx, dOut):
        Phi_c, Psi_c, Vb_c, Sin = ctx.saved_tensors
        nb, nc, C, R = Phi_c.shape
        P = Vb_c.shape[-1]
        dev = Phi_c.device
        q, k, v = Phi_c.contiguous(), Psi_c.contiguous(), Vb_c.contiguous()
        s_ = Sin.float().contiguous()
        do = dOut.float().contiguous()
        CR, CP, RP, CC = C * R, C * P, R * P, C * C
        cr, cp_, cc, rp_ = (nc * CR, CR, R, 1), (nc * CP, CP, P, 1), (nc * CC, CC, C, 1), \
            (nc * RP, RP, P, 1)
        A = torch.empty(nb, nc, C, C, device=dev, dtype=torch.float32)
        dA = torch.empty_like(A)
        _bgemm(q, k, A, M=C, N=C, K=R, n1=nb, n2=nc, a=cr, b=(nc * CR, CR, 1, R), c=cc, mask=1)
        _bgemm(do, v, dA, M=C, N=C, K=P, n1=nb, n2=nc, a=cp_, b=(nc * CP, CP, 1, P), c=cc,
               mask=1)
        dq = torch.empty(nb, nc, C, R, device=dev, dtype=torch.float32)
        dk = torch.empty_like(dq)
        dv = torch.empty(nb, nc, C, P, device=dev, dtype=torch.float32)
        ds = torch.empty(nb, nc, R, P, device=dev, dtype=torch.float32)
        _bgemm(do, s_, dq, M=C, N=R, K=P, n1=nb, n2=nc, a=cp_, b=(nc * RP, RP, 1, P), c=cr)
        _bgemm(dA, k, dq, M=C, N=R, K=C, n1=nb, n2=nc, a=cc, b=cr, c=cr, beta=1)
        _bgemm(dA, q, dk, M=C, N=R, K=C, n1=nb, n2=nc, a=(nc * CC, CC, 1, C), b=cr, c=cr)
        _bgemm(A, do, dv, M=C, N=P, K=C, n1=nb, n2=nc, a=(nc * CC, CC, 1, C), b=cp_, c=cp_)
        _bgemm(q, do, ds, M=R, N=P, K=C, n1=nb, n2=nc, a=(nc * CR, CR, 1, R), b=cp_, c=rp_)
        return (dq.to(Phi_c.dtype), dk.to(Psi_c.dtype), dv.to(Vb_c.dtype), ds.to(Sin.dtype))


class _PoolFn(torch.autograd.Function):
    """``F_x = sum_j Psi_j^T Vb_j`` over landmark tokens j = n_P + x + s*N0
    (triton_bwd.py:240-271): dPsi_j = dF_x Vb_j, dVb_j = dF_x^T Psi_j; tokens
    outside [n_P, n) get zero gradient."""

    @staticmethod
    def forward(ctx, Psi, Vb, n_P, n, N0):
        F = _FWD["pool"](Psi, Vb, n_P, n, N0)
        ctx.save_for_backward(Psi, Vb)
        ctx.dims = (n_P, n, N0)
        return F

    @staticmethod
    def backward(ctx, dF):
        Psi, Vb = ctx.saved_tensors
        n_P, n, N0 = ctx.dims
        nb, T, R = Psi.shape
        P = Vb.shape[-1]
        Ps, Vv = Psi.contiguous(), Vb.contiguous()
        dFc = dF.float().contiguous()
        dPsi = torch.zeros(nb, T, R, device=Psi.device, dtype=torch.float32)
        dVb = torch.zeros(nb, T, P, device=Psi.device, dtype=torch.float32)
        rp = R * P
        gq, grem = divmod(n - n_P, N0)
        for lo, hi, cnt in ((0, grem, gq + 1), (grem, N0, gq)):
            if hi <= lo or cnt <= 0:
                continue
            tok0 = n_P + lo
            _bgemm(Vv, dFc, dPsi, M=cnt, N=R, K=P, n1=nb, n2=hi - lo,
                   a=(T * P, P, N0 * P, 1), b=(N0 * rp, rp, 1, P), c=(T * R, R, N0 * R, 1),
                   a_off=tok0 * P, b_off=lo * rp, c_off=tok0 * R)
            _bgemm(Ps, dFc, dVb, M=cnt, N=P, K=R, n1=nb, n2=hi - lo,
                   a=(T * R, R, N0 * R, 1), b=(N0 * rp, rp, P, 1), c=(T * P, P, N0 * P, 1),
                   a_off=tok0 * R, b_off=lo * rp, c_off=tok0 * P)
        return dPsi.to(Psi.dtype), dVb.to(Vb.dtype), None, None, None


def _adjoint_lists(plane_pts, N0: int):
    """C^T of a ``(B, deg)`` point table as CSR lists, built on the device.

    The table's B*deg entries, read as one sequence of keys (the points), go
    through the counting sort behind every list of this package
    (``smat_csr_lists``): entries grouped by point, each group in table order,
    so entry ``e`` of point x names row type ``e // deg`` and the row types of
    a point come out ascending.  Nothing is read back to the host, nothing is
    cached, and points on any number of hyperplanes (ragged C^T) are allowed.
    Returns ``(rows int32 (B*deg,), offsets int64 (N0 + 1,))``."""
    from ..pool_ops import _class_lists
    B, deg = plane_pts.shape
    order, offs = _class_lists(plane_pts.reshape(1, B * deg), N0, global_index=False)
    return torch.div(order, deg, rounding_mode="floor").to(torch.int32), offs


class _IncidenceFn(torch.autograd.Function):
    """The incidence ``U = C F`` as an autograd node (the reference's is
    triton_bwd.py:300-316).  The map is linear with adjoint C^T, so
    ``dF_x = sum of dU_h over the row types h through x``: the CSR form of
    the incidence kernel over C^T's lists, made from the same table in the
    forward."""

    @staticmethod
    def forward(ctx, F, plane_pts, B):
        U = _FWD["incidence"](F, plane_pts, B)
        rows, offs = _adjoint_lists(plane_pts, F.shape[1])
        ctx.save_for_backward(rows, offs)
        ctx.f_dtype = F.dtype
        return U

    @staticmethod
    def backward(ctx, dU):
        rows, offs = ctx.saved_tensors
        nb, B, R, P = dU.shape
        N0 = offs.numel() - 1
        dF = _incidence_rows(dU.float().contiguous(), rows, offs, N0, nb, B, R * P)
        return dF.view(nb, N0, R, P).to(ctx.f_dtype), None, None


def chunk_local(Phi_c, Psi_c, Vb_c, Sin):
    """Differentiable :func:`hip_fwd.chunk_local` (triton_bwd.py:319-320)."""
    return _ChunkLocalFn.apply(Phi_c, Psi_c, Vb_c, Sin)


def pool(Psi, Vb, n_P, n, N0, *, F_glob=None):
    """Differentiable :func:`hip_fwd.pool` (triton_bwd.py:323-324).  With
    ``F_glob`` the global channel is filled as by the forward kernel; that
    output buffer carries no gradient."""
    if F_glob is not None:
        if torch.is_grad_enabled() and (Psi.requires_grad or Vb.requires_grad):
            raise NotImplementedError("pool: gradients through F_glob are not provided; use "
                                      "smat_attention, whose backward covers the channel")
        return _FWD["pool"](Psi, Vb, n_P, n, N0, F_glob=F_glob)
    return _PoolFn.apply(Psi, Vb, n_P, n, N0)


def incidence(F, plane_pts, B):
    """Differentiable :func:`hip_fwd.incidence` (triton_bwd.py:327-328)."""
    return _IncidenceFn.apply(F, plane_pts, B)


# patch() swaps the differentiable wrappers into the kernel module that the
# schedule dispatches through (and its reference-named alias), as
# triton_bwd.py:334-346 does for its Triton table; unpatch() restores the
# plain kernels.  smat_attention itself is differentiable either way: with an
# input that requires grad it runs as one autograd node (SmatAttentionFunction).
_ORIG = {}


def _kernel_modules():
    from . import triton_fwd as _alias
    return (_hip, _alias)


def patch():
    if _ORIG:
        return
    for mod in _kernel_modules():
        for name, fn in (("chunk_local", chunk_local), ("pool", pool), ("incidence", incidence)):
            _ORIG[(mod.__name__, name)] = (mod, getattr(mod, name))
            setattr(mod, name, fn)


def unpatch():
    for (mod_name, name), (mod, fn) in _ORIG.items():
        setattr(mod, name, fn)
    _ORIG.clear()


def patched() -> bool:
    return bool(_ORIG)


class QueryFunction(torch.autograd.Function):
    """The type-major read ``Y[i] = Phi_rec[i] U[i mod B]`` (query_by_type,
    attention.py:310-330) as an autograd node: :func:`hip_fwd.query` forward;
    backward ``dPhi_rec[i] = dY[i] U^T`` and ``dU[h] = sum Phi_rec[i]^T dY[i]``
    over the rows of type h (:func:`_type_read_grad`, on smat_bgemm)."""

    @staticmethod
    def forward(ctx, Phi_rec, U):
        ctx.save_for_backward(Phi_rec, U)
        return _hip.query(Phi_rec, U)

    @staticmethod
    def backward(ctx, dY):
        Phi_rec, U = ctx.saved_tensors
        nb, T_R, r = Phi_rec.shape
        B = U.shape[1]
        Ph = Phi_rec.contiguous()
        dYc = dY.float().contiguous()
        dPhi = torch.zeros(nb, T_R, r, device=Ph.device, dtype=torch.float32)
        dU = _type_read_grad(Ph, dYc, U.float().contiguous(), dPhi, T_R, 0, T_R, B)
        return dPhi.to(Phi_rec.dtype), dU.to(U.dtype)


class NormaliseFunction(torch.autograd.Function):
    """``N = cat([H[:, :n], H[:, n:] + Y])``, ``out = (N[..., :-1] / N[..., -1:]) g``
    (attention.py:446-453, the division without a floor) as an autograd node:
    :func:`hip_fwd.normalise` forward, ``smat_normalise_backward`` backward
    (dN, whose rows from n on are Y's gradient, and dg)."""

    @staticmethod
    def forward(ctx, H, Y, g, n):
        ctx.save_for_backward(H, Y, g)
        ctx.n = n
        return _hip.normalise(H, n, Y, g)

    @staticmethod
    def backward(ctx, dout):
        H, Y, g = ctx.saved_tensors
        n = ctx.n
        N = H.float().contiguous()
        if Y is not None:
            N = N.clone()
            N[:, n:] += Y.float()
        nb, T, p = N.shape
        d = dout.float().contiguous()
        dN = torch.empty(nb, T, p, device=N.device, dtype=torch.float32)
        need_dg = g is not None and ctx.needs_input_grad[2]
        dg = torch.empty(nb, T, device=N.device, dtype=torch.float32) if need_dg else None
        gc = g.float().contiguous() if g is not None else None
        call("smat_normalise_backward", d.data_ptr(), N.data_ptr(), ptr(gc), dN.data_ptr(),
             ptr(dg), nb, T, p, d.stride(0), d.stride(1), N.stride(0), N.stride(1),
             dN.stride(0), dN.stride(1), gc.stride(0) if gc is not None else 0, stream_of(dN))
        dH = dN.to(H.dtype) if ctx.needs_input_grad[0] else None
        dY = dN[:, n:].to(Y.dtype) if (Y is not None and ctx.needs_input_grad[1]) else None
        return dH, dY, (dg.to(g.dtype) if need_dg else None), None


class CombineNormaliseFunction(torch.autograd.Function):
    """``N = cat([H[:, :n], H[:, n:] + Y])``, ``out = N[..., :-1] /
    N[..., -1:].clamp_min(eps)`` (model.py:296-300) as one autograd node:
    ``smat_combine_normalise`` forward, ``smat_combine_normalise_backward``
    backward, whose dN is H's gradient and, from row n on, Y's."""

    @staticmethod
    def forward(ctx, H, Y, n, eps, out_dtype=torch.float32):
        Hc = _hip._fp32_rows(H)
        Yc = _hip._fp32_rows(Y) if Y is not None else None
        nb, T, P = Hc.shape
        out = torch.empty(nb, T, P - 1, device=Hc.device, dtype=out_dtype)
        call("smat_combine_normalise", DTYPE_CODE[out_dtype], Hc.data_ptr(), ptr(Yc),
             out.data_ptr(), nb, T, n, P, float(eps), Hc.stride(0), Hc.stride(1),
             Yc.stride(0) if Yc is not None else 0, Yc.stride(1) if Yc is not None else 0,
             out.stride(0), out.stride(1), stream_of(Hc))
        ctx.save_for_backward(Hc, Yc)
        ctx.n, ctx.eps = n, float(eps)
        ctx.dtypes = (H.dtype, None if Y is None else Y.dtype)
        return out

    @staticmethod
    def backward(ctx, dout):
        Hc, Yc = ctx.saved_tensors
        n = ctx.n
        nb, T, P = Hc.shape
        d = dout if dout.dtype in DTYPE_CODE else dout.float()
        d = d if d.stride(-1) == 1 else d.contiguous()
        dN = torch.empty(nb, T, P, device=Hc.device, dtype=torch.float32)
        call("smat_combine_normalise_backward", DTYPE_CODE[d.dtype], d.data_ptr(), Hc.data_ptr(),
             ptr(Yc), dN.data_ptr(), nb, T, n, P, ctx.eps, d.stride(0), d.stride(1),
             Hc.stride(0), Hc.stride(1), Yc.stride(0) if Yc is not None else 0,
             Yc.stride(1) if Yc is not None else 0, dN.stride(0), dN.stride(1), stream_of(d))
        dH = dN.to(ctx.dtypes[0]) if ctx.needs_input_grad[0] else None
        dY = dN[:, n:].to(ctx.dtypes[1]) if (Yc is not None and ctx.needs_input_grad[1]) else None
        return dH, dY, None, None, None

