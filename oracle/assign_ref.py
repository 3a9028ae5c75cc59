"""CPU restatement of the content-addressed assignment's forward (hard mask).

Test infrastructure (see ``oracle/__init__.py``).  Follows
src/smat/assign.py: the hash of ``_cells`` (:246-276, the ``anneal = 1``
branch :288-295), the planted key columns (:305-317), the dense read
``_dense_read`` (:431-472) with one-hot forward weights, for the point and
plane (linear direction head) modes.  Pure torch on CPU tensors.
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
