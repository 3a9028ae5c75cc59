"""Weighted pool and read of the content-addressed branch on the HIP list kernels
(the reference's src/smat_lm/smat_pool_ops.py).

Every token carries K (cell, weight) pairs ``idx, w`` of shape (B, L, K) -- the
2^dim corners of the straight-through hash, or one chosen cell::

    pool_segmented(Psi, Vb, idx, w, N0)   F[b, x] = sum_{j,k: idx[b,j,k] = x} w[b,j,k] Psi[b,j] Vb[b,j]^T
    read_gather(Phi, idx, w, F)           y[b, i] = sum_k w[b,i,k] Phi[b,i]^T F[b, idx[b,i,k]]

``pool_sorted`` / ``read_sorted`` are the same two maps (the reference computes
them a second way, through padded sub-rows; the values agree exactly).  Both are
autograd Functions with the gradients of every input but the indices.

GPU work: the pairs of each (sequence, cell) form one list (a stable sort of
the flattened cell index, torch), and every sum over a list is one HIP launch:

* ``smat_gram_lists`` -- ``sum_l A_l^T B_l`` over each list, for F and dF;
* ``smat_query_lists`` -- ``X_l U[cell_l]`` for every list entry, for y, dPhi,
  dPsi, dVb and the weight gradients.

The weights are folded into the rows (``w Psi`` for the pool, ``w Phi`` for dF)
and the K partial reads of a token are summed with torch, so the kernels see
plain lists.  Everything accumulates in fp32; F and y come back in the input
dtype, as the reference returns them.
"""
from __future__ import annotations

import torch

from .kernels import _lib
from .kernels.hip_fwd import _code, _on_gpu, call, stream_of

__all__ = ["pool_segmented", "read_gather", "pool_sorted", "read_sorted"]


# ---------------------------------------------------------------------------
# List helpers
# ---------------------------------------------------------------------------

def _csr(key, nkeys):
    """Stable order of ``key`` (int64, values in [0, nkeys)) and the offsets
    (int64, nkeys + 1) of each key's run in that order: a sort and a binary
    search on the device, nothing read back to the host (a count by
    ``bincount`` reads the largest key back, which stalls the host until the
    device has caught up)."""
    ks, order = torch.sort(key, stable=True)
    offs = torch.searchsorted(ks, torch.arange(nkeys + 1, device=key.device, dtype=key.dtype))
    return order, offs


_CSR_MAX_CLASSES = 8192


def _class_lists(keys, ncls, global_index=True, seq_rows=None, row0=0):
    """Lists of every (sequence, class): keys (nb, L) in [0, ncls) -> order
    (nb*L,) int32, the items of sequence 0's class 0, class 1, ..., then
    sequence 1's, each list in item order (the stable sort of ``b*ncls + key``);
    an item is ``b*seq_rows + row0 + l`` (``global_index``: the row of the item
    in a tensor of sequences ``seq_rows`` rows long, whose rows ``[row0, row0 +
    L)`` the keys label; by default ``b*L + l``) or ``l``.  offs (nb*ncls + 1,)
    int64.  A counting sort on the device (``smat_csr_lists``), nothing read
    back to the host."""
    nb, L = keys.shape
    dev = keys.device
    seq_rows = L if seq_rows is None else int(seq_rows)
    if ncls > _CSR_MAX_CLASSES:
        flat = (torch.arange(nb, device=dev).unsqueeze(1) * ncls + keys).reshape(-1)
        order, offs = _csr(flat, nb * ncls)
        if not global_index:
            order = order % max(L, 1)
        elif seq_rows != L or row0:
            order = order + (order // max(L, 1)) * (seq_rows - L) + row0
        return order.to(torch.int32), offs
    k = keys if (keys.dtype == torch.int64 and keys.is_contiguous()) else \
        keys.to(torch.int64).contiguous()
    order = torch.empty(nb * L, device=dev, dtype=torch.int32)
    offs = torch.empty(nb * ncls + 1, device=dev, dtype=torch.int64)
    ws = torch.empty(max(1, _lib.query("smat_csr_workspace_bytes", nb, L, ncls)), device=dev,
                     dtype=torch.uint8)
    call("smat_csr_lists", k.data_ptr(), order.data_ptr(), offs.data_ptr(), ws.data_ptr(), nb, L,
         ncls, int(global_index), seq_rows, int(row0), stream_of(k))
    return order, offs


def _list_hint(n, ncls):
    """Grid size hint of ``smat_query_lists``: twice the mean list length of n
    rows over ncls classes (longer lists are covered by the same workgroups)."""
    return 2 * -(-n // max(ncls, 1))


def _lists(cls, ncls, seq_rows=None, row0=0):
    """CSR of the rows of each (sequence, class): cls (nb, L) int -> row indices
    (int32, into the flattened rows of sequences ``seq_rows`` rows long whose
    rows ``[row0, row0 + L)`` cls labels -- by default the (nb*L) rows --
    ascending within a class), offsets (int64, nb*ncls + 1) and the
    list-length hint of the query kernel."""
    nb, L = cls.shape
    order, offs = _class_lists(cls, ncls, seq_rows=seq_rows, row0=row0)
    return order, offs, _list_hint(L, ncls)


def _gram_lists(A, B, cls, ncls, lists=None):
    """``G[b, x] = sum_{l: cls[b,l] = x} A[b,l]^T B[b,l]``: A (nb, L, r), B (nb, L, p),
    same dtype, contiguous -> fp32 (nb, ncls, r, p) (smat_gram_lists).  ``lists``:
    the CSR of ``cls`` when the caller already has it."""
    nb, L, r = A.shape
    p = B.shape[-1]
    tok, offs, _ = lists if lists is not None else _lists(cls, ncls)
    G = torch.empty(nb, ncls, r, p, device=A.device, dtype=torch.float32)
    call("smat_gram_lists", _code(A, "pool_ops"), A.data_ptr(), B.data_ptr(),
         tok.data_ptr(), offs.data_ptr(), G.data_ptr(), nb * ncls, r, p, A.stride(1),
         B.stride(1), stream_of(A))
    return G


def _read_lists(X, U, cls, lists=None):
    """``Y[b, l] = X[b, l] U[b, cls[b, l]]``: X (nb, L, c) contiguous, U fp32
    (nb, ncls, c, o) contiguous -> fp32 (nb, L, o) (smat_query_lists).  ``lists``:
    the CSR of ``cls`` when the caller already has it."""
    nb, L, c = X.shape
    ncls, o = U.shape[1], U.shape[-1]
    rows, roffs, maxcnt = lists if lists is not None else _lists(cls, ncls)
    Y = None
    # the kernel contracts at most 128 columns; wider X (c = head_dim + 1) is
    # read in column blocks whose partial products add up
    for c0 in range(0, c, 128):
        c1 = min(c, c0 + 128)
        Xs = X if c1 - c0 == c else X[..., c0:c1].contiguous()
        Us = U if c1 - c0 == c else U[:, :, c0:c1].contiguous()
        Ys = torch.empty(nb, L, o, device=X.device, dtype=torch.float32)
        call("smat_query_lists", _code(Xs, "pool_ops"), Xs.data_ptr(), Us.data_ptr(),
             Ys.data_ptr(), rows.data_ptr(), roffs.data_ptr(), nb * ncls, maxcnt, c1 - c0, o,
             Xs.stride(1), Ys.stride(1), stream_of(Xs))
        Y = Ys if Y is None else Y.add_(Ys)
    return Y


def _f32_rows(x):
    """fp32 copy of ``x`` (nb, L, c) whose rows start 32-byte aligned: a view of
    rows padded to a multiple of 8 floats (the pad is read, never used), so the
    list kernels load X in whole 8-float groups: the last group of a row ends
    at the padded row length, inside the row's own stride."""
    c = x.shape[-1]
    cp = -(-c // 8) * 8
    if cp == c:
        return x.float().contiguous()
    buf = torch.empty(*x.shape[:-1], cp, device=x.device, dtype=torch.float32)
    buf[..., :c] = x
    return buf[..., :c]


def _read_pairs(X, U, idx):
    """``Z[b, l, k] = X[b, l] U[b, idx[b, l, k]]`` for every pair: (nb, L, K, o)."""
    nb, L, c = X.shape
    K = idx.shape[-1]
    return _read_lists(_repeat(X, K), U, idx.reshape(nb, L * K)).view(nb, L, K, -1)


def _repeat(X, K):
    """(nb, L, c) -> (nb, L*K, c): each row K times in a row, contiguous."""
    nb, L, c = X.shape
    if K == 1:
        return X.contiguous()
    return X.unsqueeze(2).expand(nb, L, K, c).reshape(nb, L * K, c)


def _check(who, idx, w, N0, L):
    if idx.dim() != 3 or w.shape != idx.shape or idx.shape[1] != L:
        raise ValueError(f"{who}: idx and w must be (B, L, K) for L = {L} rows "
                         f"(got {tuple(idx.shape)} and {tuple(w.shape)})")
    if idx.dtype not in (torch.int64, torch.int32):
        raise TypeError(f"{who}: idx must be an integer tensor (got {idx.dtype})")
    if idx.numel() and (int(idx.min()) < 0 or int(idx.max()) >= N0):
        raise ValueError(f"{who}: cell indices must lie in [0, {N0})")


# ---------------------------------------------------------------------------
# The two maps
# ---------------------------------------------------------------------------

class _Pool(torch.autograd.Function):
    """``F[b, x] = sum_{j,k: idx = x} w Psi_j Vb_j^T`` (smat_pool_ops.py:17-52)."""

    @staticmethod
    def forward(ctx, Psi, Vb, idx, w, N0):
        B, n, r = Psi.shape
        K = idx.shape[-1]
        P32, V32, w32 = Psi.float(), Vb.float(), w.float()
        A = (P32.unsqueeze(2) * w32.unsqueeze(-1)).reshape(B, n * K, r)    # weight folded in
        F = _gram_lists(A, _repeat(V32, K), idx.reshape(B, n * K), N0)
        ctx.save_for_backward(Psi, Vb, idx, w)
        return F.to(Psi.dtype)

    @staticmethod
    def backward(ctx, Fbar):
        Psi, Vb, idx, w = ctx.saved_tensors
        B, n, r = Psi.shape
        p, K = Vb.shape[-1], idx.shape[-1]
        Fb = Fbar.float().contiguous()
        FbT = Fb.transpose(-1, -2).contiguous()
        P32, V32, w32 = Psi.float(), Vb.float(), w.float()
        GV = _read_pairs(V32, FbT, idx)           # (B, n, K, r): Fbar[idx] Vb_j
        GP = _read_pairs(P32, Fb, idx)            # (B, n, K, p): Fbar[idx]^T Psi_j
        dPsi = (GV * w32.unsqueeze(-1)).sum(2)
        dVb = (GP * w32.unsqueeze(-1)).sum(2)
        dw = (GV * P32.unsqueeze(2)).sum(-1)
        return dPsi.to(Psi.dtype), dVb.to(Vb.dtype), None, dw.to(w.dtype), None


class _Read(torch.autograd.Function):
    """``y[b, i] = sum_k w Phi_i^T F[idx]`` (smat_pool_ops.py:55-91)."""

    @staticmethod
    def forward(ctx, Phi, idx, w, F):
        B, m, r = Phi.shape
        F32 = F.float().contiguous()
        Z = _read_pairs(Phi.float(), F32, idx)    # (B, m, K, p)
        y = (Z * w.float().unsqueeze(-1)).sum(2)
        ctx.save_for_backward(Phi, idx, w, F)
        return y.to(Phi.dtype)

    @staticmethod
    def backward(ctx, ybar):
        Phi, idx, w, F = ctx.saved_tensors
        B, m, r = Phi.shape
        N0, K = F.shape[1], idx.shape[-1]
        y32 = ybar.float().contiguous()
        P32, w32 = Phi.float(), w.float()
        FT = F.float().transpose(-1, -2).contiguous()
        Gy = _read_pairs(y32, FT, idx)            # (B, m, K, r): F[idx] ybar_i
        dPhi = (Gy * w32.unsqueeze(-1)).sum(2)
        dw = (Gy * P32.unsqueeze(2)).sum(-1)
        A = (P32.unsqueeze(2) * w32.unsqueeze(-1)).reshape(B, m * K, r)
        dF = _gram_lists(A, _repeat(y32, K), idx.reshape(B, m * K), N0)
        return dPhi.to(Phi.dtype), None, dw.to(w.dtype), dF.to(F.dtype)


def pool_segmented(Psi, Vb, idx, w, N0):
    """(B, N0, r, p) pool of every pair's outer product ``w Psi_j Vb_j^T`` into
    its cell, in Psi's dtype (fp32 accumulation)."""
    _on_gpu("pool_segmented", Psi, Vb, idx, w)
    _check("pool_segmented", idx, w, int(N0), Psi.shape[1])
    return _Pool.apply(Psi.contiguous(), Vb.contiguous(), idx.contiguous(), w.contiguous(),
                       int(N0))


def read_gather(Phi, idx, w, F):
    """(B, m, p) read ``sum_k w Phi_i^T F[idx_k]``, in Phi's dtype (fp32
    accumulation)."""
    _on_gpu("read_gather", Phi, idx, w, F)
    _check("read_gather", idx, w, F.shape[1], Phi.shape[1])
    return _Read.apply(Phi.contiguous(), idx.contiguous(), w.contiguous(), F.contiguous())


def pool_sorted(Psi, Vb, idx, w, N0):
    """Same map as :func:`pool_segmented` (smat_pool_ops.py:158-170)."""
    return pool_segmented(Psi, Vb, idx, w, N0)


def read_sorted(Phi, idx, w, F):
    """Same map as :func:`read_gather` (smat_pool_ops.py:173-182)."""
    return read_gather(Phi, idx, w, F)
