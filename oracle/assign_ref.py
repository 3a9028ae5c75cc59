"""CPU restatement of the content-addressed assignment.

Test infrastructure (see ``oracle/__init__.py``).  Follows
src/smat/assign.py: the hash of ``_cells`` (:246-276, the ``anneal = 1``
branch :288-295), the planted key columns (:305-317), the dense read
``_dense_read`` (:431-472) with one-hot forward weights, for the point and
plane (linear direction head) modes; with autograd, the straight-through
weights of the dense point read (``dense_point_ste``) and the (cell, weight)
pair branch of the soft phase and the ``sparse_ops`` path (``pairs_branch``:
:257-313, :378-406, with the pool / read maps of
src/smat_lm/smat_pool_ops.py:1-11 written densely).  Pure torch on CPU tensors.
"""
from __future__ import annotations

import torch


def cells(u, W, gamma, b, q: int, dim: int, h: int):
    """assign.py:253-258 + :288-295: hard cell of every token, (nb*h, L) int64,
    and s = clamp(q * Phi_N(z), 0, q - 1e-4), (nb*h, L, dim)."""
    nb, L, dm = u.shape
    Wn = W / W.norm(dim=-1, keepdim=True).clamp_min(1e-6)
    ln = torch.nn.functional.layer_norm(u, (dm,))
    z = torch.einsum("blm,hkm->bhlk", ln, Wn) * gamma[None, :, None, :] + b[None, :, None, :]
    s = torch.special.ndtr(z)
    s = (s * q).clamp(0.0, q - 1e-4)
    s = s.reshape(nb * h, L, dim)
    lo = s.floor().long()
    idx = torch.zeros(nb * h, L, dtype=torch.long)
    for k in range(dim):
        idx = idx + lo[..., k] * q ** (dim - 1 - k)
    return idx, s


def plant(ck, plant_cols, plant_cells):
    """assign.py:305-317: planted key columns get fixed cells."""
    L = ck.shape[1]
    cols = plant_cols[plant_cols < L]
    ck = ck.clone()
    if cols.numel():
        ck[:, cols] = plant_cells[: cols.numel()]
    return ck


def dense_read(Phi, Psi, Vb, n: int, ck, cq, N0: int, *, mode: str = "point", M=None,
               Wd=None, u=None, h: int = 1, dir_override=None):
    """assign.py:431-472 with one-hot forward weights: y (nb*h, T_R, p)."""
    P, V = Psi[:, :n], Vb[:, :n]
    Bsz, r, p = P.shape[0], P.shape[-1], V.shape[-1]
    acc = torch.float64 if Phi.dtype == torch.float64 else torch.float32
    Wk = torch.nn.functional.one_hot(ck, N0).to(acc)                   # (B, n, N0)
    Wq = torch.nn.functional.one_hot(cq, N0).to(acc)                   # (B, T_R, N0)
    PV = torch.einsum("bnr,bnp->bnrp", P.to(acc), V.to(acc)).reshape(Bsz, n, r * p)
    F = torch.bmm(Wk.transpose(1, 2), PV).view(Bsz, N0, r, p)
    Phi_r = Phi[:, n:].to(acc)
    if mode == "point":
        Uq = torch.bmm(Wq, F.reshape(Bsz, N0, r * p)).view(Bsz, -1, r, p)
        return torch.einsum("bir,birp->bip", Phi_r, Uq)
    Mf = M.to(acc)
    U = torch.einsum("eox,bxrp->beorp", Mf, F)
    Z = torch.einsum("bir,beorp->bieop", Phi_r, U)
    D = Mf.shape[0]
    if dir_override is not None:
        e_star = dir_override.reshape(Bsz, -1)
    else:
        dl = torch.einsum("blm,hem->bhle", u[:, n:].to(acc), Wd.to(acc)).reshape(Bsz, -1, D)
        e_star = dl.argmax(-1)
    we = torch.nn.functional.one_hot(e_star, D).to(acc)
    po = torch.einsum("bix,eox->bieo", Wq, Mf)
    wo = torch.nn.functional.one_hot(po.argmax(-1), Mf.shape[1]).to(acc)
    return torch.einsum("bie,bieo,bieop->bip", we, wo, Z)


def hash_s(u, W, gamma, b, q: int, h: int):
    """assign.py:251-256 with autograd: s = clamp(q Phi_N(LN(u) W^ gamma + b), 0, q - 1e-4),
    (nb*h, L, dim)."""
    nb, L, dm = u.shape
    Wn = W / W.norm(dim=-1, keepdim=True).clamp_min(1e-6)
    ln = torch.nn.functional.layer_norm(u, (dm,))
    z = torch.einsum("blm,hkm->bhlk", ln, Wn) * gamma[None, :, None, :] + b[None, :, None, :]
    s = (torch.special.ndtr(z) * q).clamp(0.0, q - 1e-4)
    return s.reshape(nb * h, L, W.shape[1])


def ste_weights(s, q: int, N0: int):
    """assign.py:257-266 and :290-295 at anneal = 1: the dense (B, L, N0) cell
    weights, forward the one-hot of the all-low cell, backward the two-bin
    interpolation of every coordinate."""
    B, L, dim = s.shape
    lo = s.floor()
    frac = s - lo
    lo = lo.long()
    hi = (lo + 1).clamp(max=q - 1)
    idx = torch.zeros(B, L, 1, dtype=torch.long)
    w = torch.ones(B, L, 1, dtype=s.dtype)
    for k in range(dim):
        place = q ** (dim - 1 - k)
        f = frac[..., k:k + 1]
        e_lo = 1.0 + ((1.0 - f) - (1.0 - f).detach())
        e_hi = f - f.detach()
        idx = torch.cat([idx + lo[..., k:k + 1] * place, idx + hi[..., k:k + 1] * place], -1)
        w = torch.cat([w * e_lo, w * e_hi], -1)
    return torch.zeros(B, L, N0, dtype=s.dtype).scatter_add(-1, idx, w)


def dense_point_ste(u, Phi, Psi, Vb, n: int, W, gamma, b, q: int, dim: int, h: int, N0: int,
                    planted_cols=None, plant_cells=None, s_shift=None):
    """The point branch as assign.py:374-446 computes it on its dense path, with
    autograd through Phi, Psi, Vb and the hash (u, W, gamma, b): planted key
    columns get a fixed one-hot row (:305-317), F = Wk^T (Psi (x) Vb) (:436),
    y_i = Phi_i (Wq F)_i (:439-441).  Returns (nb*h, T - n, p).

    ``s_shift`` (optional, (nb*h, T, dim), no gradient) is added to the hash
    values before the cells are taken: a check uses it to move a value that
    lies within rounding of a bin edge into the bin another implementation
    chose; the gradient does not depend on it (the weights' derivative depends
    on the bin, not on the position inside it)."""
    s_all = hash_s(u, W, gamma, b, q, h)
    if s_shift is not None:
        s_all = s_all + s_shift.detach()
    Wk = ste_weights(s_all[:, :n], q, N0)
    if planted_cols is not None and len(planted_cols):
        cols = torch.as_tensor(planted_cols, dtype=torch.long)
        cols = cols[cols < n]
        one = torch.zeros(cols.numel(), N0, dtype=Wk.dtype)
        one[torch.arange(cols.numel()), plant_cells[: cols.numel()]] = 1.0
        Wk = Wk.clone()
        Wk[:, cols] = one
    Wq = ste_weights(s_all[:, n:], q, N0)
    B, _, r = Psi.shape
    p = Vb.shape[-1]
    PV = torch.einsum("bnr,bnp->bnrp", Psi[:, :n], Vb[:, :n]).reshape(B, n, r * p)
    F = torch.bmm(Wk.transpose(1, 2), PV).view(B, N0, r, p)
    Uq = torch.bmm(Wq, F.reshape(B, N0, r * p)).view(B, -1, r, p)
    return torch.einsum("bir,birp->bip", Phi[:, n:], Uq)


def soft_pairs(s, q: int, dim: int, anneal: float = 1.0, single: bool = False):
    """assign.py:257-284: the 2^dim (cell, weight) pairs of every token, weight
    ``(1 - a) s + a e`` per coordinate (``e`` the straight-through form of the
    interpolation weight ``s``); with ``single`` and ``a >= 1`` the chosen cell
    alone (``hard_k1``).  Returns idx, w of shape (B, L, K)."""
    B, L, _ = s.shape
    a = float(anneal)
    lo = s.floor()
    frac = s - lo
    lo = lo.long()
    hi = (lo + 1).clamp(max=q - 1)
    if single and a >= 1.0:
        idx = torch.zeros(B, L, 1, dtype=torch.long)
        w = torch.ones(B, L, 1, dtype=s.dtype)
        for k in range(dim):
            f = frac[..., k:k + 1]
            idx = idx + lo[..., k:k + 1] * q ** (dim - 1 - k)
            w = w * (1.0 + ((1.0 - f) - (1.0 - f).detach()))
        return idx, w
    idx = torch.zeros(B, L, 1, dtype=torch.long)
    w = torch.ones(B, L, 1, dtype=s.dtype)
    for k in range(dim):
        place = q ** (dim - 1 - k)
        f = frac[..., k:k + 1]
        s_lo, s_hi = 1.0 - f, f
        e_lo = 1.0 + (s_lo - s_lo.detach())
        e_hi = s_hi - s_hi.detach()
        idx = torch.cat([idx + lo[..., k:k + 1] * place, idx + hi[..., k:k + 1] * place], -1)
        w = torch.cat([w * ((1 - a) * s_lo + a * e_lo), w * ((1 - a) * s_hi + a * e_hi)], -1)
    return idx, w


def plant_pairs(idx, w, planted_cols, plant_cells):
    """assign.py:305-313: planted key columns get their fixed cell, weight 1 on
    the first pair and 0 on the others, no gradient."""
    cols = torch.as_tensor(planted_cols, dtype=torch.long)
    cols = cols[cols < idx.shape[1]]
    if cols.numel() == 0:
        return idx, w
    idx, w = idx.clone(), w.clone()
    idx[:, cols, :] = plant_cells[: cols.numel()].view(1, -1, 1)
    w[:, cols, :] = 0.0
    w[:, cols, 0] = 1.0
    return idx, w


def pairs_dense(idx, w, N0: int):
    """(B, L, N0) cell weights: every pair's weight added to its cell
    (assign.py:297 ``scatter_add``)."""
    B, L, _ = idx.shape
    return torch.zeros(B, L, N0, dtype=w.dtype).scatter_add(-1, idx, w)


def pairs_branch(u, Phi, Psi, Vb, n: int, W, gamma, b, q: int, dim: int, h: int, N0: int, *,
                 anneal: float = 1.0, single: bool = False, planted_cols=None,
                 plant_cells=None, mode: str = "point", M=None, Wd=None, coset_of=None,
                 dir_soft: bool = False):
    """The long-range term over (cell, weight) pairs with autograd: the dense
    read with the cell weights of any anneal (assign.py:431-472) and, with
    ``single``, the ``sparse_ops`` path (:378-406) -- ``F = Wk^T (Psi (x) Vb)``,
    point ``y = Phi (Wq F)``.  Plane, sparse: ``Fc = M F`` summed to the
    direction cosets, the direction the argmax of ``softmax(u Wd)`` with the
    straight-through factor ``1 + pmax - pmax.detach()``, each query pair read
    at (direction, coset of its cell).  Plane, dense: ``Z = Phi (M F)`` for
    every (direction, offset), mixed by the direction weights ``we`` (the
    straight-through one-hot of the softmax, or the softmax with
    ``dir_soft``) and the straight-through one-hot ``wo`` of the coset
    marginal ``Wq M``.  Returns (nb*h, T - n, p)."""
    planted = planted_cols is not None and any(int(c) < n for c in planted_cols)
    # a planted key side is planted into the full pairs (assign.py:306-310)
    idxk, wk = soft_pairs(hash_s(u[:, :n], W, gamma, b, q, h), q, dim, anneal,
                          single and not planted)
    if planted:
        idxk, wk = plant_pairs(idxk, wk, planted_cols, plant_cells)
    idxq, wq = soft_pairs(hash_s(u[:, n:], W, gamma, b, q, h), q, dim, anneal, single)
    Bs, _, r = Psi.shape
    p = Vb.shape[-1]
    PV = torch.einsum("bnr,bnp->bnrp", Psi[:, :n], Vb[:, :n]).reshape(Bs, n, r * p)
    F = torch.bmm(pairs_dense(idxk, wk, N0).transpose(1, 2), PV).view(Bs, N0, r, p)
    Phi_r = Phi[:, n:]
    if mode == "point":
        Uq = torch.bmm(pairs_dense(idxq, wq, N0), F.reshape(Bs, N0, r * p)).view(Bs, -1, r, p)
        return torch.einsum("bir,birp->bip", Phi_r, Uq)
    D, nc = M.shape[0], M.shape[1]
    T_R = Phi_r.shape[1]
    dl = torch.einsum("blm,hem->bhle", u[:, n:], Wd).reshape(Bs, T_R, D)
    pe = torch.softmax(dl, dim=-1)
    if not single:
        U = torch.einsum("eox,bxrp->beorp", M, F)
        Z = torch.einsum("bir,beorp->bieop", Phi_r, U)
        we = pe if dir_soft else \
            torch.zeros_like(pe).scatter_(-1, pe.argmax(-1, keepdim=True), 1.0) + (pe - pe.detach())
        po = torch.einsum("bix,eox->bieo", pairs_dense(idxq, wq, N0), M)
        wo = torch.zeros_like(po).scatter_(-1, po.argmax(-1, keepdim=True), 1.0) + (po - po.detach())
        return torch.einsum("bie,bieo,bieop->bip", we, wo, Z)
    Fc = torch.einsum("eox,bxrp->beorp", M, F).reshape(Bs, D * nc, r * p)
    e_star = pe.argmax(-1, keepdim=True)
    pmax = pe.gather(-1, e_star)
    ste = 1.0 + (pmax - pmax.detach())
    rows = e_star * nc + coset_of[e_star.expand_as(idxq), idxq]
    Uq = torch.bmm(pairs_dense(rows, wq, D * nc), Fc).view(Bs, T_R, r, p)
    return torch.einsum("bir,birp->bip", Phi_r, Uq) * ste
