"""Content-addressed assignment on the GPU (the reference's src/smat/assign.py).

``ContentAssign`` replaces the positional maps ``prof(j) = (j - n_P) mod N0``
and ``type(i) = i mod B`` with a hash of token content and runs the whole
long-range branch: pool the distant keys by cell, apply the geometry's
cosets for the plane read, contract every recent query with the state of its
type.  It returns the augmented long-range term ``(nb*h, T_R, p)`` that the
causal branch adds before the single division -- where ``query_by_type``
sits in the positional schedule.

GPU work per call:

* ``smat_cell_hash`` (HIP): LayerNorm, the unit-row projection, the normal
  CDF and the floor, one wave per token row (assign.py:246-276);
* a stable sort of tokens by cell (torch, index plumbing);
* ``smat_gram_lists`` (HIP): the pool ``F_x = sum_{cell(j) = x} Psi_j^T Vb_j``
  over each cell's token list (assign.py:431-436);
* plane read: ``smat_incidence`` over the (direction, offset) cosets
  (assign.py:442);
* ``smat_query_lists`` (HIP): ``y_i = Phi_i U_type(i)`` over each type's row
  list (assign.py:437-439, 471-472).

Supported: ``mode`` point/plane and any codimension 1 .. dim (``codim``: the
read sums the coset of a codimension-c subspace through the query's cell),
``src`` hidden/embed/id, ``shift``, ``plant``, ``freeze``, the key convolution
``kconv`` of ``conv_width > 1`` (created for the caller, as the reference
does), the ``linear``, ``mlp``, ``delta`` and ``fixed`` direction heads,
``dir_override``, ``dir_soft``, ``anneal`` in [0, 1], ``sparse_ops`` (with
``hard_k1``), and the analysis methods ``cells_of``, ``oracle_dir``,
``agreement`` and ``key_agreement``.  Parameters are created in the
reference's order, so a module built after ``torch.manual_seed(s)`` holds the
reference's values.  Both reads train, with the reference's gradients: the
hash runs under torch autograd and the pool, the reads and their gradients run
on the list and incidence kernels (see ``_forward_grad``), for the dense read
at any ``anneal`` (the soft phase included), ``dir_soft`` and
``dir_override``, and for the ``sparse_ops`` pair path.  ``delta_updates``
(the reference pools by the gated delta rule of the FLA library,
``chunk_gated_delta_rule``, src/smat_lm/smat_delta_pool.py) raises
``NotImplementedError``.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn as nn

from .kernels.hip_fwd import _code, _on_gpu, _rows3, call, stream_of
from .pool_ops import (_class_lists, _f32_rows, _gram_lists, _list_hint, _lists, _read_lists,
                       _read_pairs, _repeat, pool_sorted, read_sorted)

__all__ = ["ContentAssign", "grouped_planes", "grouped_flats"]


def grouped_planes(q: int, dim: int):
    """(dirs, grouped): normalised directions of F_q^dim and, per (direction,
    offset), the q^(dim-1) points of that affine hyperplane -- the reference's
    enumeration (assign.py:45-60): lex-ordered points, leading nonzero = 1,
    points of a hyperplane in increasing order."""
    idx = np.arange(q ** dim, dtype=np.int64)
    pts = np.stack([(idx // q ** (dim - 1 - k)) % q for k in range(dim)], axis=1)
    nz = pts != 0
    lead = nz.argmax(axis=1)
    is_dir = nz.any(axis=1) & (pts[np.arange(q ** dim), lead] == 1)
    dirs = pts[is_dir]
    inner = (pts @ dirs.T) % q
    order = np.argsort(inner, axis=0, kind="stable")
    grouped = order.T.reshape(dirs.shape[0], q, q ** (dim - 1))
    return dirs, grouped


def grouped_flats(q: int, dim: int, codim: int):
    """(D_c, q^codim, q^(dim-codim)) point indices: every partition of F_q^dim
    into the cosets of a codimension-``codim`` subspace, the reference's
    enumeration (assign.py:63-90).  A full-rank codim x dim matrix A over F_q
    maps point x to the coset A x; the matrices are taken in lexicographic
    order of their entries (row-major), a partition is kept the first time a
    matrix induces it, and its cosets are numbered by their smallest point,
    each listing its points in increasing order.  codim = 1 gives the
    hyperplane partitions of :func:`grouped_planes` (in another order)."""
    N0 = q ** dim
    pts = np.stack([(np.arange(N0) // q ** (dim - 1 - k)) % q for k in range(dim)], 1)
    n_cos, deg = q ** codim, q ** (dim - codim)
    weights = q ** np.arange(codim)
    digits = np.arange(codim * dim)
    seen, parts = set(), []
    for code in range(q ** (codim * dim)):
        A = ((code // q ** (codim * dim - 1 - digits)) % q).reshape(codim, dim)
        key = ((pts @ A.T) % q) @ weights            # the coset of each point, as a number
        _, first, inverse = np.unique(key, return_index=True, return_inverse=True)
        if len(first) != n_cos:
            continue                                 # A is not of full rank
        rank = np.empty(n_cos, dtype=np.int64)
        rank[np.argsort(first)] = np.arange(n_cos)   # cosets by their smallest point
        label = rank[inverse.reshape(-1)]
        sig = label.tobytes()
        if sig in seen:
            continue
        seen.add(sig)
        parts.append(np.argsort(label, kind="stable").reshape(n_cos, deg))
    return np.stack(parts)


def _straight_through(value: float, surrogate):
    """A tensor whose forward value is ``value`` everywhere and whose gradient
    is that of ``surrogate``: value + (surrogate - surrogate.detach())."""
    return value + (surrogate - surrogate.detach())


class ContentAssign(nn.Module):
    """Hash tokens to profiles and queries to types; run the long-range branch.

    Mirrors ``src/smat/assign.py:ContentAssign`` (constructor :136-243,
    ``_cells`` :246-317, ``forward`` :352-406, ``_dense_read`` :431-472).
    """

    def __init__(self, n_heads, d_model, spec, mode="point", plant=True, src="hidden",
                 freeze=False, shift=0, codim=None, vocab=None, conv_width=0,
                 dir_head="linear", dir_hidden=512, dir_window=4, dir_soft=False):
        super().__init__()
        if dir_head not in ("linear", "mlp", "delta", "fixed"):
            raise ValueError(f"ContentAssign: unknown dir_head {dir_head!r}")
        self.codim = None if codim is None else int(codim)
        if self.codim is not None:
            assert 1 <= self.codim <= int(spec.dim), (self.codim, spec.dim)
            mode = "point" if self.codim == int(spec.dim) else "plane"
        assert spec.kind == "geometric" and spec.dim >= 1
        self.h = n_heads
        self.q, self.dim, self.N0 = int(spec.q), int(spec.dim), int(spec.N0)
        self.mode, self.plant = mode, plant
        self.src, self.freeze, self.shift = src, freeze, int(shift)
        self.conv_width = int(conv_width)
        if self.conv_width > 1:
            # the key-side hash input's depthwise causal convolution, uniform over
            # its lags at the start; the caller applies it (key_src), as in the
            # reference, which creates it here (so its draw precedes W's)
            self.kconv = nn.Conv1d(d_model, d_model, self.conv_width, groups=d_model, bias=False)
            with torch.no_grad():
                self.kconv.weight.fill_(1.0 / self.conv_width)
            self.kconv.weight.requires_grad_(not freeze)
        if src == "id":
            assert vocab is not None, "the id hash needs the vocabulary size"
            g = torch.Generator().manual_seed(1234)
            self.register_buffer("id_cell",
                                 torch.randint(0, int(spec.N0), (vocab, n_heads), generator=g))
        if mode == "plane" and self.dim == 1:
            self.mode = "point"
        self.ln = nn.LayerNorm(d_model, elementwise_affine=False)
        self.W = nn.Parameter(torch.randn(n_heads, self.dim, d_model), requires_grad=not freeze)
        self.gamma = nn.Parameter(torch.ones(n_heads, self.dim), requires_grad=not freeze)
        self.b = nn.Parameter(torch.zeros(n_heads, self.dim), requires_grad=not freeze)
        if self.mode == "plane":
            if self.codim in (None, 1):
                grouped = grouped_planes(self.q, self.dim)[1]
            else:
                grouped = grouped_flats(self.q, self.dim, self.codim)
            self.D, self.n_cosets = int(grouped.shape[0]), int(grouped.shape[1])
            self.dir_head = dir_head if self.codim in (None, 1) else "linear"
            self.dir_soft = bool(dir_soft)
            # the linear projection of the direction logits; the sparse read
            # scores directions with it whatever the head (assign.py:201-203)
            self.Wd = nn.Parameter(torch.randn(n_heads, self.D, d_model) * d_model ** -0.5,
                                   requires_grad=not freeze)
            if self.dir_head in ("delta", "fixed"):
                # logits summed over the previous dir_window tokens' cells:
                # Wdelta[head, lag, cell difference, direction] (assign.py:204-233)
                self.win = int(dir_window)
                pts = np.stack([(np.arange(self.N0) // self.q ** (self.dim - 1 - j)) % self.q
                                for j in range(self.dim)], 1)
                place = self.q ** np.arange(self.dim - 1, -1, -1)
                diff = ((pts[:, None, :] - pts[None, :, :]) % self.q) @ place
                self.register_buffer("diff_tab", torch.as_tensor(diff, dtype=torch.long))
                self.Wdelta = nn.Parameter(torch.zeros(n_heads, self.win, self.N0, self.D),
                                           requires_grad=not freeze)
                nn.init.normal_(self.Wdelta, std=0.02)
                if self.dir_head == "fixed":
                    # 1 where direction e annihilates the difference: a fixed map
                    dirs = grouped_planes(self.q, self.dim)[0]
                    ind = torch.as_tensor((pts @ dirs.T) % self.q == 0, dtype=torch.float32)
                    with torch.no_grad():
                        self.Wdelta.copy_(ind.expand(n_heads, self.win, self.N0, self.D))
                    self.Wdelta.requires_grad_(False)
            elif self.dir_head == "mlp":
                self.Wd1 = nn.Parameter(torch.randn(n_heads, dir_hidden, d_model) * d_model ** -0.5,
                                        requires_grad=not freeze)
                self.bd1 = nn.Parameter(torch.zeros(n_heads, dir_hidden), requires_grad=not freeze)
                self.Wd = nn.Parameter(torch.randn(n_heads, self.D, dir_hidden)
                                       * dir_hidden ** -0.5, requires_grad=not freeze)
            else:
                # the reference draws the linear projection a second time
                # (assign.py:236-238); the second draw is the one kept
                self.Wd = nn.Parameter(torch.randn(n_heads, self.D, d_model) * d_model ** -0.5,
                                       requires_grad=not freeze)
            M = np.zeros((self.D, self.n_cosets, self.N0), dtype=np.float32)
            for e in range(self.D):
                for o in range(self.n_cosets):
                    M[e, o, grouped[e, o]] = 1.0
            self.register_buffer("M", torch.from_numpy(M))
            self.register_buffer("coset_of", torch.from_numpy(M.argmax(1)))
            self.register_buffer("coset_pts", torch.from_numpy(
                grouped.reshape(self.D * self.n_cosets, -1).astype(np.int32)))
        cols = spec.planted_cols if spec.planted_cols is not None else np.zeros(0, dtype=np.int64)
        self.register_buffer("plant_cols", torch.as_tensor(np.asarray(cols), dtype=torch.long))
        self.register_buffer("plant_cells",
                             torch.as_tensor([self.q ** (self.dim - l)
                                              for l in range(1, self.dim + 1)], dtype=torch.long))
        self.anneal = 1.0
        self._soft_src = {"q": None, "k": None}
        self.last_hard_k = None
        self.last_hard_q = None
        self.probe = False
        self.last = None
        self.last_occ = None
        self.last_dens = None
        self.aux = None

    # ------------------------------------------------------------------ hash
    def _hash(self, u):
        """(nb, L, d_model) -> cells (nb*h, L) int64 and s (nb*h, L, dim) = q Phi_N(z)."""
        nb, L, dm = u.shape
        uc, u_sb, u_st = _rows3(u)
        Wn = (self.W / self.W.norm(dim=-1, keepdim=True).clamp_min(1e-6)).detach().float()
        Wn = Wn.contiguous()
        gam = self.gamma.detach().float().contiguous()
        bia = self.b.detach().float().contiguous()
        s = torch.empty(nb * self.h, L, self.dim, device=u.device, dtype=torch.float32)
        cells = torch.empty(nb * self.h, L, device=u.device, dtype=torch.int64)
        call("smat_cell_hash", _code(uc, "ContentAssign"), uc.data_ptr(), Wn.data_ptr(),
             gam.data_ptr(), bia.data_ptr(), s.data_ptr(), cells.data_ptr(), nb, L, dm,
             self.h, self.dim, self.q, u_sb, u_st, stream_of(uc))
        return cells, s

    def _cells(self, u, plant_at=False, tok_w=None):
        """Hard cells of every token (nb*h, L) int64, as assign.py:_cells with
        anneal = 1: the hash, the planted columns, and the load-balance term
        (``aux``) from the soft bin occupancy."""
        if self.anneal < 1.0:
            raise NotImplementedError("ContentAssign: the soft read (anneal < 1)")
        cells, s = self._hash(u)
        L = cells.shape[1]
        self.aux = None if self.freeze else self._balance(s, tok_w)
        if plant_at and self.plant and self.plant_cols.numel():
            cols = self.plant_cols[self.plant_cols < L]
            if cols.numel():
                cells[:, cols.to(cells.device)] = self.plant_cells[: cols.numel()].to(cells.device)
        return cells

    def _cells_id(self, ids):
        nb, L = ids.shape
        return self.id_cell[ids].permute(0, 2, 1).reshape(nb * self.h, L)

    # --------------------------------------------------------- soft cells
    def _soft_cells(self, side):
        """The dense soft cell distribution (B, L, N0) of the last forward's
        query (``side`` "q") or key ("k", before planting) tokens: each token
        spreads over the 2^dim cells around its hash with the interpolation
        weights prod_k (1 - f_k or f_k), no straight-through part (the
        reference's ``_soft``, assign.py:266, 291).  Recomputed from the
        recorded hash input, so it carries gradients to the hash parameters
        (and the input) when grad mode is on; for the id hash the one-hot of
        the table cell."""
        rec = self._soft_src.get(side)
        if rec is None:
            return None
        kind, t = rec
        if kind == "cells":
            return torch.nn.functional.one_hot(t, self.N0).float()
        s = self._soft_hash(t)
        B, L, dim = s.shape
        q = self.q
        j = s.detach().floor()
        f = s - j
        lo, hi = j.long(), (j.long() + 1).clamp(max=q - 1)
        out = torch.zeros(B, L, self.N0, device=s.device, dtype=s.dtype)
        for m in range(1 << dim):
            cell, wt = 0, None
            for k in range(dim):
                high = (m >> k) & 1
                cell = cell + (hi if high else lo)[..., k] * q ** (dim - 1 - k)
                ck = f[..., k] if high else 1.0 - f[..., k]
                wt = ck if wt is None else wt * ck
            out = out.scatter_add(-1, cell.unsqueeze(-1), wt.unsqueeze(-1))
        return out

    @property
    def last_soft_q(self):
        """Soft cell distribution (nb*h, T_R, N0) of the last forward's recent
        queries (the reference's ``last_soft_q``); None after a sparse_ops
        forward, as there."""
        return self._soft_cells("q")

    @last_soft_q.setter
    def last_soft_q(self, value):
        self._soft_src["q"] = None if value is None else ("cells", value.argmax(-1))

    @property
    def last_soft_k(self):
        """Soft cell distribution (nb*h, n, N0) of the last forward's distant
        keys, before planting.  The reference reads this attribute in
        ``key_agreement`` but never assigns it (so its method raises); here the
        forward records it like the query side."""
        return self._soft_cells("k")

    @last_soft_k.setter
    def last_soft_k(self, value):
        self._soft_src["k"] = None if value is None else ("cells", value.argmax(-1))

    # ------------------------------------------------------------ analysis
    def cells_of(self, v):
        """``(..., d_model) -> (..., h)`` cell index of every head, for one
        hidden state at a time (assign.py:319-328): the hash of the forward,
        evaluated in the reference's op order (torch, on v's device)."""
        Wn = self.W / self.W.norm(dim=-1, keepdim=True).clamp_min(1e-6)
        z = torch.einsum("...m,hkm->...hk", self.ln(v), Wn) * self.gamma + self.b
        dig = (torch.special.ndtr(z) * self.q).clamp(0.0, self.q - 1e-4).floor().long()
        place = torch.tensor([self.q ** (self.dim - 1 - k) for k in range(self.dim)],
                             device=v.device)
        return (dig * place).sum(-1)

    def oracle_dir(self, cells):
        """cells (B, L, k) -> (B, L): the first direction along which all k cells
        share their offset (the hyperplane of that direction through them), 0 if
        none does (assign.py:330-344)."""
        dirs = grouped_planes(self.q, self.dim)[0]
        pts = np.stack([(np.arange(self.N0) // self.q ** (self.dim - 1 - j)) % self.q
                        for j in range(self.dim)], 1)
        offset = torch.as_tensor((pts @ dirs.T) % self.q, device=cells.device)   # (N0, D)
        per = offset[cells]                                                      # (B, L, k, D)
        common = (per == per[..., :1, :]).all(-2)                                # (B, L, D)
        first = common.int().argmax(-1)
        return torch.where(common.any(-1), first, torch.zeros_like(first))

    def _route_loss(self, soft, src, target_cells, valid):
        """-(mean over valid pairs) of log p(target cell): the cell distribution
        ``soft`` (B, m, N0) of token ``src`` at the cell ``target_cells`` (B, P)
        (the negative log-likelihood of the routing, floored at 1e-9); pairs are
        (nb, P), repeated over the h heads of each sequence."""
        nb = src.shape[0]
        rep = soft.shape[0] // nb
        i = src.repeat_interleave(rep, 0).clamp_min(0)
        tgt = target_cells.clamp_min(0)
        v = valid.repeat_interleave(rep, 0).to(soft.dtype)
        p = soft.gather(1, i.unsqueeze(-1).expand(-1, -1, self.N0))
        lp = p.gather(-1, tgt.unsqueeze(-1)).squeeze(-1).clamp_min(1e-9).log()
        return -(lp * v).sum() / v.sum().clamp_min(1.0)

    def agreement(self, pairs, valid):
        """Routing term of the query side (assign.py:499-515): pairs (nb, P, 2)
        of (recent query i, distant position j) and valid (nb, P); the query's
        soft cell distribution should put its mass on the hard cell of the
        distant key j.  None before a forward that records them."""
        soft = self.last_soft_q
        if soft is None or self.last_hard_k is None:
            return None
        rep = soft.shape[0] // pairs.shape[0]
        j = pairs[..., 1].repeat_interleave(rep, 0).clamp_min(0)
        return self._route_loss(soft, pairs[..., 0], self.last_hard_k.gather(1, j), valid)

    def key_agreement(self, pay_pos, key_cells, valid):
        """Routing term of the key side (assign.py:476-497): a payload at
        distant position pay_pos (nb, P) should be filed under key_cells
        (nb, P, detached targets); valid (nb, P)."""
        soft = self.last_soft_k
        if soft is None:
            return None
        rep = soft.shape[0] // pay_pos.shape[0]
        return self._route_loss(soft, pay_pos, key_cells.repeat_interleave(rep, 0), valid)

    def _dir_logits(self, u, n, ids=None):
        """Direction logits (nb*h, T_R, D) of the recent queries for the dense
        plane read (assign.py:445-458): linear in the layer input, a one-layer
        gelu network (``mlp``), or (``delta`` / ``fixed``) the sum over the
        previous ``dir_window`` tokens of Wdelta[head, lag, cell difference],
        cells from the id table."""
        T_R = u.shape[1] - n
        head = getattr(self, "dir_head", "linear")
        if head in ("delta", "fixed"):
            assert ids is not None, "the delta direction head needs token ids"
            nb = ids.shape[0]
            cq = self.id_cell[ids[:, n:]]                                  # (nb, T_R, h)
            hsel = torch.arange(self.h, device=ids.device)[None, None, :]
            dl = 0.0
            for lag in range(1, self.win + 1):
                cs = self.id_cell[ids[:, n - lag:ids.shape[1] - lag]]
                dl = dl + self.Wdelta[:, lag - 1][hsel, self.diff_tab[cs, cq]]
            return dl.permute(0, 2, 1, 3).reshape(nb * self.h, T_R, self.D)
        if head == "mlp":
            hid = torch.einsum("blm,hkm->bhlk", u[:, n:], self.Wd1) + self.bd1[None, :, None, :]
            dl = torch.einsum("bhlk,hek->bhle", torch.nn.functional.gelu(hid), self.Wd)
        else:
            dl = torch.einsum("blm,hem->bhle", u[:, n:], self.Wd)
        return dl.reshape(u.shape[0] * self.h, T_R, self.D)

    # ------------------------------------------------------------- the branch
    def forward(self, u, Phi, Psi, Vb, n, emb=None, key_src=None, key_w=None,
                dir_override=None, ids=None):
        """u: (nb, T, d_model) layer input; Phi, Psi: (nb*h, T, r); Vb: (nb*h, T, p);
        n: landmark/recent boundary.  Returns fp32 (nb*h, T - n, p)."""
        if getattr(self, "delta_updates", False):
            raise NotImplementedError("ContentAssign: delta_updates (the delta-rule pool)")
        _on_gpu("ContentAssign", u, Phi, Psi, Vb, emb, key_src, key_w, ids)
        soft = self.src != "id" and (self.anneal < 1.0 or getattr(self, "sparse_ops", False))
        # dir_soft mixes the directions in training mode, with or without grad
        soft = soft or (self.mode == "plane" and getattr(self, "dir_soft", False) and self.training
                        and dir_override is None and getattr(self, "dir_ovr", None) is None)
        if soft or (torch.is_grad_enabled() and (
                any(t is not None and t.requires_grad for t in (u, Phi, Psi, Vb, emb, key_src))
                or any(prm.requires_grad for prm in self.parameters()))):
            return self._forward_grad(u, Phi, Psi, Vb, n, emb, key_src, key_w, ids, dir_override)
        if self.src == "id":
            assert ids is not None, "the id hash needs token ids"
            ik = ids if not self.shift else torch.cat(
                [ids.new_zeros(ids.shape[0], self.shift), ids[:, :-self.shift]], dim=1)
            ck, cq = self._cells_id(ik[:, :n]), self._cells_id(ids[:, n:])
            self._soft_src = {"q": ("cells", cq), "k": ("cells", ck)}
            self.aux = None
        else:
            h = u if (self.src == "hidden" or emb is None) else emb
            hk = h if key_src is None else key_src
            if self.shift:
                hk = torch.cat([h.new_zeros(h.shape[0], self.shift, h.shape[2]),
                                h[:, :-self.shift]], dim=1)
            ck = self._cells(hk[:, :n], plant_at=True, tok_w=key_w)
            aux_k = self.aux
            cq = self._cells(h[:, n:])
            self._soft_src = {"q": ("hash", h[:, n:]), "k": ("hash", hk[:, :n])}
            self.aux = None if self.freeze else aux_k + self.aux
        self.last_hard_k = ck.detach()
        self.last_hard_q = cq.detach()
        return self._read(u, Phi, Psi, Vb, n, ck, cq, dir_override, ids)

    # ------------------------------------------------------------ training
    def _soft_hash(self, u):
        """``s = clamp(q Phi_N(LN(u) W^ gamma + b), 0, q - 1e-4)`` with autograd, in
        the reference's op order (assign.py:251-256): the hash of the training
        path, whose floor gives the same cells as the HIP hash."""
        nb, L, _ = u.shape
        Wn = self.W / self.W.norm(dim=-1, keepdim=True).clamp_min(1e-6)
        z = torch.einsum("blm,hkm->bhlk", self.ln(u), Wn) * self.gamma[None, :, None, :] \
            + self.b[None, :, None, :]
        s = torch.special.ndtr(z)
        s = (s * self.q).clamp(0.0, self.q - 1e-4)
        return s.reshape(nb * self.h, L, self.dim)

    def _balance(self, s, tok_w=None):
        """Load-balance term of the hash (the reference's ``aux``,
        assign.py:290-298): a token whose coordinate k sits at s = j + f puts
        mass 1 - f on bin j and f on bin min(j + 1, q - 1), times its gate
        weight ``tok_w``.  Per (sequence, coordinate) the masses over the q bins,
        divided by their total (floored at 1e-6), form the occupancy o, and the
        term is KL(o || uniform) = sum_j o_j log(q max(o_j, 1e-9)), averaged
        over sequences and coordinates.  One index_add over both endpoints of
        every token."""
        B, L, dim = s.shape
        q = self.q
        j = s.detach().floor()
        f = s - j                                    # carries the gradient of s
        ends = torch.stack([j, (j + 1).clamp(max=q - 1)], -1).long()     # (B, L, dim, 2)
        mass = torch.stack([1.0 - f, f], -1)
        if tok_w is not None:
            mass = mass * tok_w.reshape(B, L, 1, 1).to(s.dtype)
        slot = torch.arange(B * dim, device=s.device).view(B, 1, dim, 1) * q + ends
        occ = torch.zeros(B * dim * q, device=s.device, dtype=s.dtype)
        occ = occ.index_add(0, slot.reshape(-1), mass.reshape(-1)).view(B, dim, q)
        occ = occ / occ.sum(-1, keepdim=True).clamp_min(1e-6)
        return (occ * torch.log(q * occ.clamp_min(1e-9))).sum(-1).mean()

    def _ste_pairs(self, s, plant_at=False, tok_w=None, single=False):
        """The 2^dim (cell, weight) pairs of every token (assign.py:257-295).

        Coordinate k of s = j_k + f_k interpolates between its low bin j_k and
        its high bin min(j_k + 1, q - 1).  Pair m takes the high bin in the
        coordinates whose bit is set in m (bit k for coordinate k; pair 0 is the
        chosen cell), cell = sum_k bin_k q^(dim-1-k), and weight
        prod_k c_k with c_k = (1 - a) (1 - f_k) + a lo_k on a low bin and
        (1 - a) f_k + a hi_k on a high one, a the anneal.  lo_k and hi_k are
        straight-through factors: forward 1 and 0, gradients those of 1 - f_k
        and f_k.  With ``single`` and a >= 1 only pair 0 is kept, weight
        prod_k lo_k (the sparse path's ``hard_k1``) -- except on a key side with
        planted columns, which keeps all pairs as the reference does.
        Planted key columns read their fixed cell at weight 1 on pair 0 and 0
        elsewhere, with no gradient (:305-317).  Returns the chosen cells,
        idx (B, L, K), w (B, L, K) and the load-balance term."""
        B, L, dim = s.shape
        q, a = self.q, float(self.anneal)
        j = s.detach().floor()
        f = s - j
        lo_bin = j.long()
        hi_bin = (lo_bin + 1).clamp(max=q - 1)
        st_lo = _straight_through(1.0, 1.0 - f)
        st_hi = _straight_through(0.0, f)
        c_lo = (1 - a) * (1.0 - f) + a * st_lo
        c_hi = (1 - a) * f + a * st_hi
        cols = None
        if plant_at and self.plant and self.plant_cols.numel():
            cols = self.plant_cols[self.plant_cols < L].to(s.device)
            cols = cols if cols.numel() else None
        place = [q ** (dim - 1 - k) for k in range(dim)]
        hard = single and cols is None and a >= 1.0 and getattr(self, "hard_k1", True)
        idx_l, w_l = [], []
        for m in ([0] if hard else range(1 << dim)):
            cell, wt = 0, None
            for k in range(dim):
                high = (m >> k) & 1
                cell = cell + (hi_bin if high else lo_bin)[..., k] * place[k]
                ck = st_lo[..., k] if hard else (c_hi if high else c_lo)[..., k]
                wt = ck if wt is None else wt * ck
            idx_l.append(cell)
            w_l.append(wt)
        idx = torch.stack(idx_l, -1)
        w = torch.stack(w_l, -1)
        aux = None if self.freeze else self._balance(s, tok_w)
        cells = idx[..., 0].clone()
        if cols is not None:
            pc = self.plant_cells[: cols.numel()].to(s.device)
            cells[:, cols] = pc
            planted = torch.zeros(L, dtype=torch.bool, device=s.device)
            planted[cols] = True
            cell_of = torch.zeros(L, dtype=idx.dtype, device=s.device)
            cell_of[cols] = pc
            first = torch.zeros(idx.shape[-1], dtype=w.dtype, device=s.device)
            first[0] = 1.0
            idx = torch.where(planted.view(1, L, 1), cell_of.view(1, L, 1), idx)
            w = torch.where(planted.view(1, L, 1), first.view(1, 1, -1), w)
        return cells, idx, w, aux

    def _pairs_of(self, u, n, emb, key_src, key_w, ids, single):
        """Key and query pairs (assign.py:357-378) for the pair reads."""
        if self.src == "id":
            assert ids is not None, "the id hash needs token ids"
            ik = ids if not self.shift else torch.cat(
                [ids.new_zeros(ids.shape[0], self.shift), ids[:, :-self.shift]], dim=1)
            ck, cq = self._cells_id(ik[:, :n]), self._cells_id(ids[:, n:])
            self._soft_src = {"q": ("cells", cq), "k": ("cells", ck)}
            self.aux = None
            one = lambda c: torch.ones(c.shape + (1,), device=u.device)
            return ck, ck.unsqueeze(-1), one(ck), cq, cq.unsqueeze(-1), one(cq)
        h = u if (self.src == "hidden" or emb is None) else emb
        hk = h if key_src is None else key_src
        if self.shift:
            hk = torch.cat([h.new_zeros(h.shape[0], self.shift, h.shape[2]),
                            h[:, :-self.shift]], dim=1)
        if self._fused_pairs_ok(h, key_w, single):
            if hk is h:
                # one LayerNorm and projection over the whole hidden state
                z = self._hash_z(h)
                ck, idxk, wk, aux_k = self._pairs_from_z(z[:, :n], plant_at=True)
                cq, idxq, wq, aux_q = self._pairs_from_z(z[:, n:])
            else:
                ck, idxk, wk, aux_k = self._pairs_from_z(self._hash_z(hk[:, :n]), plant_at=True)
                cq, idxq, wq, aux_q = self._pairs_from_z(self._hash_z(h[:, n:]))
        else:
            ck, idxk, wk, aux_k = self._ste_pairs(self._soft_hash(hk[:, :n]), plant_at=True,
                                                  tok_w=key_w, single=single)
            cq, idxq, wq, aux_q = self._ste_pairs(self._soft_hash(h[:, n:]), single=single)
        self.aux = None if self.freeze else aux_k + aux_q
        # the sparse read forms no dense soft distribution (assign.py:289-291)
        self._soft_src = ({"q": None, "k": None} if single else
                          {"q": ("hash", h[:, n:]), "k": ("hash", hk[:, :n])})
        return ck, idxk, wk, cq, idxq, wq

    def _fused_pairs_ok(self, h, key_w, single):
        return (FUSED_HASH_PAIRS and self.anneal >= 1.0 and key_w is None and not single
                and h.dtype == torch.float32 and self.dim <= 8 and self.dim * self.q <= 4096
                and self.h * self.dim <= 64)

    def _plant_map(self, L, device):
        """(L,) int64: the planted cell of each key column, -1 elsewhere."""
        key = (L, str(device))
        cache = getattr(self, "_plant_maps", None)
        if cache is None:
            cache = self._plant_maps = {}
        if key not in cache:
            pm = torch.full((L,), -1, dtype=torch.int64)
            if self.plant and self.plant_cols.numel():
                cols = self.plant_cols[self.plant_cols < L].cpu()
                pm[cols] = self.plant_cells[: cols.numel()].cpu()
            cache[key] = pm.to(device)
        return cache[key]

    def _hash_pairs(self, hu, plant_at=False):
        """``_ste_pairs(_soft_hash(hu))`` at ``anneal = 1`` with no token
        weights, in three autograd steps: the projections z (:meth:`_hash_z`),
        then the pairs, the straight-through weights and the occupancy
        (``smat_hash_pairs``, with ``smat_hash_pairs_backward`` for the gradient
        of z), then the load-balance term from the occupancy (torch)."""
        return self._pairs_from_z(self._hash_z(hu), plant_at)

    def _hash_z(self, hu):
        """z = LN(hu) . Wn gamma + b, (nb, L, h*dim), as :meth:`_soft_hash`
        before the CDF; the product's weight gradient is split over the
        tokens (:class:`_Project`)."""
        nb, L, dm = hu.shape
        Wn = self.W / self.W.norm(dim=-1, keepdim=True).clamp_min(1e-6)
        hd = self.h * self.dim
        xh = self.ln(hu).reshape(nb * L, dm)
        z = _Project.apply(xh, Wn.reshape(hd, dm)) * self.gamma.reshape(hd) + self.b.reshape(hd)
        return z.reshape(nb, L, hd)

    def _pairs_from_z(self, z, plant_at=False):
        nb, L, _ = z.shape
        plant = self._plant_map(L, z.device) if (plant_at and self.plant) else None
        cells, idx, w, occ = _HashPairs.apply(z, self.h, self.dim, self.q, plant)
        occ = occ / occ.sum(-1, keepdim=True).clamp_min(1e-6)
        aux = None if self.freeze else (occ * (occ.clamp_min(1e-9) * self.q).log()).sum(-1).mean()
        return cells, idx, w, aux

    def _forward_grad(self, u, Phi, Psi, Vb, n, emb, key_src, key_w, ids, dir_override):
        """The branch with the gradients of the reference's autograd, over the
        (cell, weight) pairs of every token.

        * the dense read (assign.py:431-472): at ``anneal = 1`` the forward
          weights are one-hot, so the pool and the point read run over the
          chosen cells (:class:`_HardPool`, :class:`_HardRead`) and the pairs
          only enter the weight gradients; below, the soft pool and read
          (:func:`pool_sorted` / :func:`read_sorted`); the plane read sums F to
          the direction cosets (incidence kernel) and reads the chosen
          (direction, offset) of each query (:class:`_PlaneRead`);
        * the ``sparse_ops`` path (:378-406): pool and read over the pairs,
          the plane read with the straight-through factor on the direction.

        The hash is torch autograd on the dim values per token; every pool,
        read and their gradients are HIP list kernels.  Returns fp32."""
        if getattr(self, "delta_updates", False):
            raise NotImplementedError("ContentAssign: delta_updates (the delta-rule pool)")
        sparse = bool(getattr(self, "sparse_ops", False)) and self.src != "id"
        ck, idxk, wk, cq, idxq, wq = self._pairs_of(u, n, emb, key_src, key_w, ids, sparse)
        self.last_hard_k = ck.detach()
        self.last_hard_q = cq.detach()
        P, V, Phi_r = Psi[:, :n], Vb[:, :n], Phi[:, n:]
        dt = P.dtype
        dev = Phi.device
        nbh, T_R = Phi_r.shape[0], Phi_r.shape[1]
        nrows = self.D * self.n_cosets if self.mode == "plane" else 0
        if sparse:
            F = pool_sorted(P, V, idxk, wk.to(dt), self.N0)
            if self.mode == "point":
                return read_sorted(Phi_r, idxq, wq.to(dt), F).float()
            from .kernels import hip_bwd
            Fc = hip_bwd.incidence(F, self.coset_pts.to(dev), nrows).to(F.dtype)
            if dir_override is not None:
                e_star = dir_override.reshape(nbh, T_R, 1).long()
                ste = torch.ones(nbh, T_R, 1, device=dev)
            else:
                dl = torch.einsum("blm,hem->bhle", u[:, n:], self.Wd.to(u.dtype)).reshape(
                    nbh, T_R, self.D)
                pe = torch.softmax(dl.float(), dim=-1)
                e_star = pe.argmax(-1, keepdim=True)
                pmax = pe.gather(-1, e_star)
                ste = 1.0 + (pmax - pmax.detach())
            coset = self.coset_of.to(dev)[e_star.expand_as(idxq), idxq]
            y = read_sorted(Phi_r, e_star * self.n_cosets + coset, wq.to(dt), Fc)
            return (y * ste.to(y.dtype)).float()
        hard = self.anneal >= 1.0 or self.src == "id"
        if hard:
            F = _HardPool.apply(Psi, Vb, wk, idxk, ck, self.N0)
        else:
            F = pool_sorted(P, V, idxk, wk.to(dt), self.N0).float()
        if self.mode == "point":
            if hard:
                return _HardRead.apply(Phi, F, wq, idxq, cq)
            return read_sorted(Phi_r, idxq, wq.to(dt), F.to(dt)).float()
        from .kernels import hip_bwd
        U = hip_bwd.incidence(F, self.coset_pts.to(dev), nrows)
        if dir_override is None:
            dir_override = getattr(self, "dir_ovr", None)
        if dir_override is not None:
            # the direction is given, not learned (assign.py:461-462)
            we = torch.zeros(nbh, T_R, self.D, device=dev).scatter_(
                -1, dir_override.reshape(nbh, T_R, 1).long(), 1.0)
        else:
            dl = self._dir_logits(u, n, ids)
            self.last_dir_logits = dl
            pe = torch.softmax(dl, dim=-1)
            if getattr(self, "dir_soft", False) and self.training:
                we = pe
            else:
                we = torch.zeros_like(pe).scatter_(-1, pe.argmax(-1, keepdim=True), 1.0) + \
                    (pe - pe.detach())
        return _PlaneRead.apply(Phi_r, U, we.float(), wq, idxq, self.coset_of.to(dev),
                                self.n_cosets)

    def _read(self, u, Phi, Psi, Vb, n, ck, cq, dir_override, ids=None):
        nbh, T, r = Phi.shape
        p = Vb.shape[-1]
        T_R = T - n
        dev = Phi.device
        N0 = self.N0
        # ---- pool by cell: tokens of each (sequence, cell), in token order
        order, offs = _class_lists(ck, N0)
        order = order.long()
        seq = order // n
        tokens = (seq * T + (order - seq * n)).to(torch.int32)
        Ps = Psi if Psi.stride(0) == T * Psi.stride(1) else Psi.contiguous()
        Vs = Vb if Vb.stride(0) == T * Vb.stride(1) else Vb.contiguous()
        F = torch.empty(nbh, N0, r, p, device=dev, dtype=torch.float32)
        call("smat_gram_lists", _code(Ps, "ContentAssign"), Ps.data_ptr(), Vs.data_ptr(),
             tokens.data_ptr(), offs.data_ptr(), F.data_ptr(), nbh * N0, r, p,
             Ps.stride(1), Vs.stride(1), stream_of(Ps))
        # ---- the read: a type per recent query
        if self.mode == "point":
            U, ntypes, typ = F, N0, cq
        else:
            nrows = self.D * self.n_cosets
            U = torch.empty(nbh, nrows, r, p, device=dev, dtype=torch.float32)
            pts = self.coset_pts.to(dev)
            call("smat_incidence", F.data_ptr(), None, pts.data_ptr(), 0, None, pts.shape[1],
                 U.data_ptr(), nbh, N0, nrows, r * p, stream_of(F))
            if dir_override is None:
                dir_override = getattr(self, "dir_ovr", None)
            if dir_override is not None:
                e_star = dir_override.reshape(nbh, T_R).long()
            else:
                dl = self._dir_logits(u, n, ids)
                self.last_dir_logits = dl
                e_star = dl.argmax(-1)
            typ = e_star * self.n_cosets + self.coset_of.to(dev)[e_star, cq]
            ntypes = nrows
        order, roffs = _class_lists(typ, ntypes)
        order = order.long()
        seq = order // T_R
        rows = (seq * T + n + (order - seq * T_R)).to(torch.int32)
        maxcnt = _list_hint(T_R, ntypes)
        Pr = Phi if Phi.stride(0) == T * Phi.stride(1) else Phi.contiguous()
        Y = torch.empty(nbh, T, p, device=dev, dtype=torch.float32)
        call("smat_query_lists", _code(Pr, "ContentAssign"), Pr.data_ptr(), U.data_ptr(),
             Y.data_ptr(), rows.data_ptr(), roffs.data_ptr(), nbh * ntypes, maxcnt, r, p,
             Pr.stride(1), Y.stride(1), stream_of(Pr))
        return Y[:, n:]


# ---------------------------------------------------------------------------
# The hard point branch with its gradients (HIP)
# ---------------------------------------------------------------------------

# The fused backward kernels of the hard read and pool (smat_cell_read_backward,
# smat_cell_pool_backward) serve bf16 inputs at r = 64, p = 65; tests switch
# them off to compare with the list reads they replace.  They split fp32
# operands (F, dF, dY) into bf16 hi/lo pairs, which keeps fp32's exponent
# range; fp16 inputs take the list reads, which widen every operand to fp32.
FUSED_CELL_BACKWARD = True


def _cell_backward_ok(X, Y, r_ok=64, p_ok=65):
    return (FUSED_CELL_BACKWARD and X.dtype == torch.bfloat16
            and X.shape[-1] == r_ok and (Y is None or (Y.dtype == X.dtype
                                                       and Y.shape[-1] == p_ok))
            and X.stride(-1) == 1 and X.stride(1) % 8 == 0 and X.stride(0) % 8 == 0
            and X.data_ptr() % 16 == 0)


def _entry_lists(idx, N0):
    """CSR of the (token, pair) entries of every (sequence, cell): idx (nb, L, K)
    -> entry ids pair*L + token (int32, ascending within a cell, so a cell's
    pair-0 entries come first) and offsets (int64, nb*N0 + 1)."""
    nb, L, K = idx.shape
    return _class_lists(idx.transpose(1, 2).reshape(nb, K * L), N0, global_index=False)


# The pairs of the training path from one kernel (smat_hash_pairs) and its
# backward; tests switch it off to compare with the torch straight-through path.
FUSED_HASH_PAIRS = True


class _Project(torch.autograd.Function):
    """``x @ W^T`` for many token rows x (R, dm) and few output rows W (k, dm).
    The weight gradient ``dy^T x`` has a long contraction (R) and a small
    output (k x dm); it is taken as a batched product over 16-32 slices of the
    rows and a sum of the slices, which spreads it over many workgroups."""

    @staticmethod
    def forward(ctx, x, W):
        ctx.save_for_backward(x, W)
        return x @ W.t()

    @staticmethod
    def backward(ctx, dy):
        x, W = ctx.saved_tensors
        dx = dy @ W if ctx.needs_input_grad[0] else None
        dW = None
        if ctx.needs_input_grad[1]:
            R, k = dy.shape
            S = 32
            while S > 1 and (R % S or R // S < 256):
                S //= 2
            if S > 1:
                dyT = dy.reshape(S, R // S, k).transpose(1, 2).contiguous()
                dW = torch.bmm(dyT, x.reshape(S, R // S, x.shape[1]).contiguous()).sum(0)
            else:
                dW = dy.t().contiguous() @ x
        return dx, dW


class _HashPairs(torch.autograd.Function):
    """z (nb, L, h*dim) -> cells (nb*h, L), idx (nb*h, L, 2^dim), the one-hot
    forward weights w (nb*h, L, 2^dim) and the soft occupancy (nb*h, dim, q):
    the straight-through pairs of assign.py:257-317 at ``anneal = 1``.  The
    gradients of w and of the occupancy come back to z through
    ``smat_hash_pairs_backward``."""

    @staticmethod
    def forward(ctx, z, nh, dim, q, plant):
        nb, L, _ = z.shape
        B, K = nb * nh, 1 << dim
        z = z.contiguous()
        s = torch.empty(B, L, dim, device=z.device, dtype=torch.float32)
        cells = torch.empty(B, L, device=z.device, dtype=torch.int64)
        idx = torch.empty(B, L, K, device=z.device, dtype=torch.int64)
        occ = torch.empty(B, dim, q, device=z.device, dtype=torch.float32)
        if L:
            call("smat_hash_pairs", z.data_ptr(), None if plant is None else plant.data_ptr(),
                 s.data_ptr(), cells.data_ptr(), idx.data_ptr(), occ.data_ptr(), nb, L, nh, dim,
                 q, stream_of(z))
        else:
            occ.zero_()
        w = torch.zeros(B, L, K, device=z.device, dtype=torch.float32)
        w[..., 0] = 1.0
        ctx.save_for_backward(z, s)
        ctx.plant, ctx.shape = plant, (nb, L, nh, dim, q)
        ctx.mark_non_differentiable(cells, idx)
        ctx.set_materialize_grads(False)
        return cells, idx, w, occ

    @staticmethod
    def backward(ctx, dcells, didx, dw, docc):
        z, s = ctx.saved_tensors
        nb, L, nh, dim, q = ctx.shape
        if (dw is None and docc is None) or not L:
            return None, None, None, None, None
        dw = None if dw is None else dw.float().contiguous()
        docc = None if docc is None else docc.float().contiguous()
        dz = torch.empty_like(z)
        plant = ctx.plant
        call("smat_hash_pairs_backward", z.data_ptr(), s.data_ptr(),
             None if plant is None else plant.data_ptr(),
             None if dw is None else dw.data_ptr(), None if docc is None else docc.data_ptr(),
             dz.data_ptr(), nb, L, nh, dim, q, stream_of(z))
        return dz, None, None, None, None


def _one_hot_first(w):
    """Whether the forward weights put 1 on each row's first pair and 0 elsewhere."""
    return bool((w[..., 0] == 1).all()) and bool((w[..., 1:] == 0).all())


def _whole_rows(*xs):
    """Whether every (nb, T, .) tensor stores each sequence's T rows one after
    another (batch stride = T * row stride), so that flat row ids ``b*T + t``
    address them from the first element."""
    return all(x.stride(-1) == 1 and x.stride(0) == x.shape[1] * x.stride(1) for x in xs)


def _grad_rows(x, lo, hi, dtype):
    """A gradient for ``x`` (nb, T, c) whose rows ``[lo, hi)`` a kernel writes:
    the rows outside are zero.  Rows of c elements, 16-byte aligned."""
    g = torch.empty(x.shape, device=x.device, dtype=dtype)
    if lo > 0:
        g[:, :lo].zero_()
    if hi < x.shape[1]:
        g[:, hi:].zero_()
    return g


def _slice_grad(x, g, lo):
    """(nb, T, c) gradient of ``x`` from the gradient ``g`` of rows ``[lo, lo + L)``."""
    out = torch.zeros(x.shape, device=x.device, dtype=x.dtype)
    out[:, lo:lo + g.shape[1]] = g
    return out


class _HardPool(torch.autograd.Function):
    """The dense pool with one-hot forward weights (assign.py:431-436 at
    ``anneal = 1``): ``F_x = sum_{ck_j = x} Psi_j^T Vb_j`` over the first ``n``
    rows of Psi and Vb (``n = ck.shape[1]``); backward ``dPsi_j = dF[ck_j]
    Vb_j``, ``dVb_j = dF[ck_j]^T Psi_j`` and, for every pair, ``dw_jk = Psi_j .
    (dF[idx_jk] Vb_j)`` -- for the first pair (the chosen cell, ``idx_j0 =
    ck_j``) that is ``Psi_j . dPsi_j``.  Psi and Vb are the layer's whole
    (nb, T, .) tensors: the kernels read the key rows in place, and the
    gradients are whole tensors of Psi's and Vb's dtypes with zero rows from
    ``n`` on, so no slice is copied either way.  fp32 F."""

    @staticmethod
    def forward(ctx, Psi, Vb, wk, idxk, ck, N0):
        r, p = Psi.shape[-1], Vb.shape[-1]
        if r > 128 or p > 144:
            raise NotImplementedError("ContentAssign gradients: r <= 128, p <= 144")
        n = ck.shape[1]
        if _whole_rows(Psi, Vb):
            lists = _lists(ck, N0, seq_rows=Psi.shape[1])
            F = _gram_lists(Psi, Vb, ck, N0, lists)
        else:
            F = _gram_lists(Psi[:, :n].contiguous(), Vb[:, :n].contiguous(), ck, N0)
        ctx.save_for_backward(Psi, Vb, idxk, ck)
        ctx.n = n
        ctx.w_dtype = wk.dtype
        return F

    @staticmethod
    def backward(ctx, dF):
        Psi, Vb, idxk, ck = ctx.saved_tensors
        n = ctx.n
        dF = dF.float().contiguous()
        if _cell_backward_ok(Psi, Vb):
            # one launch per (sequence, cell): dPsi, dVb and every pair's dw,
            # rounded to the inputs' type as they are stored
            nb, _, r = Psi.shape
            p, N0, K = Vb.shape[-1], dF.shape[1], idxk.shape[-1]
            ent, eoffs = _entry_lists(idxk, N0)
            dPsi = _grad_rows(Psi, 0, n, Psi.dtype)
            dVb = _grad_rows(Vb, 0, n, Vb.dtype)
            dwk = torch.empty(nb, n, K, device=Psi.device, dtype=torch.float32)
            call("smat_cell_pool_backward", _code(Psi, "ContentAssign"), _code(dPsi, "ContentAssign"),
                 Psi.data_ptr(), Vb.data_ptr(), dF.data_ptr(), ent.data_ptr(), eoffs.data_ptr(),
                 dPsi.data_ptr(), dVb.data_ptr(), dwk.data_ptr(), nb, N0, K, n, r, p, Psi.stride(0),
                 Psi.stride(1), Vb.stride(0), Vb.stride(1), dF.stride(0), dPsi.stride(0),
                 dPsi.stride(1), dVb.stride(0), dVb.stride(1), dwk.stride(0), stream_of(dF))
            return dPsi, dVb, dwk.to(ctx.w_dtype), None, None, None
        Pk, Vk = Psi[:, :n].contiguous(), Vb[:, :n].contiguous()
        lists = _lists(ck, dF.shape[1])
        dFT = dF.transpose(-1, -2).contiguous()
        P32, V32 = Pk.float(), _f32_rows(Vk)         # Vb rows of p floats, 16-byte aligned
        dPsi = _read_lists(V32, dFT, ck, lists)
        dVb = _read_lists(P32, dF, ck, lists)
        dwk = _pair_dw(P32, dPsi, V32, dFT, idxk)
        return (_slice_grad(Psi, dPsi, 0), _slice_grad(Vb, dVb, 0), dwk.to(ctx.w_dtype), None,
                None, None)


def _pair_dw(X, G0, Y, UT, idx):
    """``dw[b, l, k] = X_l . (U[idx_lk] Y_l)`` for every pair, given
    ``G0 = U[idx_l0] Y_l`` of the first pair (already computed as a gradient):
    the other pairs are one list read over the flattened (row, pair) lists."""
    dw0 = (X * G0).sum(-1, keepdim=True)
    if idx.shape[-1] == 1:
        return dw0
    rest = (_read_pairs(Y, UT, idx[..., 1:].contiguous()) * X.unsqueeze(2)).sum(-1)
    return torch.cat([dw0, rest], -1)


class _HardRead(torch.autograd.Function):
    """The dense point read with one-hot forward weights (assign.py:437-441 at
    ``anneal = 1``): ``y_i = Phi_i F[cq_i]`` for the last ``T_R = cq.shape[1]``
    rows of Phi; backward ``dPhi_i = F[cq_i] dy_i``, ``dF_x = sum_{cq_i = x}
    Phi_i^T dy_i`` and ``dw_ik = Phi_i . (F[idx_ik] dy_i)`` (``Phi_i . dPhi_i``
    for the first pair).  Phi is the layer's whole (nb, T, r) tensor, read in
    place; its gradient is a whole tensor of Phi's dtype, zero before the
    recent rows.  y: fp32 (nb, T_R, p), rows of sequences T rows apart (a view
    of a (nb, T, p) buffer whose first T_R rows of each sequence it holds)."""

    @staticmethod
    def forward(ctx, Phi, F, wq, idxq, cq):
        nb, T, r = Phi.shape
        T_R = cq.shape[1]
        n = T - T_R
        N0, p = F.shape[1], F.shape[-1]
        Fc = F.contiguous()
        if _whole_rows(Phi) and r <= 128:
            # row ids b*T + l address Phi from row n and the output from row 0
            rows, roffs, hint = _lists(cq, N0, seq_rows=T)
            Yw = torch.empty(nb, T, p, device=Phi.device, dtype=torch.float32)
            Xr = Phi[:, n:]
            call("smat_query_lists", _code(Xr, "ContentAssign"), Xr.data_ptr(), Fc.data_ptr(),
                 Yw.data_ptr(), rows.data_ptr(), roffs.data_ptr(), nb * N0, hint, r, p,
                 Xr.stride(1), Yw.stride(1), stream_of(Xr))
            Y = Yw[:, :T_R]
        else:
            Y = _read_lists(Phi[:, n:].contiguous(), Fc, cq)
        ctx.save_for_backward(Phi, F, idxq, cq)
        ctx.w_dtype = wq.dtype
        return Y

    @staticmethod
    def backward(ctx, dY):
        Phi, F, idxq, cq = ctx.saved_tensors
        nb, T, r = Phi.shape
        T_R = cq.shape[1]
        n = T - T_R
        Phr = Phi[:, n:]
        if _cell_backward_ok(Phr, None) and F.shape[-1] == 65 and F.shape[-2] == 64:
            # one launch per (sequence, cell): dPhi, dF and every pair's dw
            dYc = dY.float()
            dYc = dYc if dYc.stride(-1) == 1 else dYc.contiguous()
            Fc = F.float().contiguous()
            N0, p, K = Fc.shape[1], Fc.shape[-1], idxq.shape[-1]
            ent, eoffs = _entry_lists(idxq, N0)
            dPhi = _grad_rows(Phi, n, T, Phi.dtype)
            dPr = dPhi[:, n:]
            dF = torch.empty(nb, N0, r, p, device=Phi.device, dtype=torch.float32)
            dwq = torch.empty(nb, T_R, K, device=Phi.device, dtype=torch.float32)
            call("smat_cell_read_backward", _code(Phr, "ContentAssign"),
                 _code(dPr, "ContentAssign"), Phr.data_ptr(), dYc.data_ptr(), Fc.data_ptr(),
                 ent.data_ptr(), eoffs.data_ptr(), dPr.data_ptr(), dF.data_ptr(), dwq.data_ptr(),
                 nb, N0, K, T_R, r, p, Phr.stride(0), Phr.stride(1), dYc.stride(0), dYc.stride(1),
                 Fc.stride(0), dPr.stride(0), dPr.stride(1), dwq.stride(0), stream_of(Fc))
            return dPhi, dF, dwq.to(ctx.w_dtype), None, None
        Phr = Phr.contiguous()
        lists = _lists(cq, F.shape[1])
        dY = _f32_rows(dY)                            # rows of p floats, 16-byte aligned
        Ph32 = Phr.float()
        FT = F.transpose(-1, -2).contiguous()
        dPhi = _read_lists(dY, FT, cq, lists)
        dF = _gram_lists(Ph32, dY, cq, F.shape[1], lists)
        dwq = _pair_dw(Ph32, dPhi, dY, FT, idxq)
        return _slice_grad(Phi, dPhi, n), dF, dwq.to(ctx.w_dtype), None, None


def _offset_rows(idxq, wq, coset_of, nc):
    """(B, T_R, D) row ``e*nc + o*`` of every direction: o* the argmax over
    offsets of the query's coset marginal ``po[e, o] = sum_k wq_k [coset(e,
    idx_k) = o]`` (assign.py:466)."""
    D = coset_of.shape[0]
    base = torch.arange(D, device=idxq.device) * nc
    if _one_hot_first(wq):
        return base + coset_of[:, idxq[..., 0]].permute(1, 2, 0)
    B, T_R, _ = idxq.shape
    rows = torch.empty(B, T_R, D, dtype=torch.long, device=idxq.device)
    for e in range(D):
        po = torch.zeros(B, T_R, nc, device=idxq.device, dtype=wq.dtype)
        po.scatter_add_(-1, coset_of[e][idxq], wq)
        rows[..., e] = e * nc + po.argmax(-1)
    return rows


class _PlaneRead(torch.autograd.Function):
    """The dense plane read (assign.py:443-472) under the reference's autograd:
    ``y_i = sum_{e,o} we[i,e] wo[i,e,o] Phi_i U[e,o]`` with ``wo`` the
    straight-through one-hot of the coset marginal ``po = Wq M`` and ``we``
    the direction weights (straight-through one-hot of the softmax, the softmax
    itself, or a given direction).  Forward reads the chosen offset of each
    direction that carries weight; backward::

        dPhi_i  = sum_e we[i,e] U[e,o*] dy_i     dU[e,o*] += we[i,e] Phi_i^T dy_i
        dwe[i,e] = Phi_i U[e,o*(i,e)] dy_i      (every direction)
        dwq_ik  = sum_e we[i,e] Phi_i U[e, coset(e, idx_ik)] dy_i

    (the last is ``dpo`` through ``M`` back to the query's pair weights).
    U: fp32 (B, D*nc, r, p) from the incidence kernel over the cosets."""

    @staticmethod
    def forward(ctx, Phr, U, we, wq, idxq, coset_of, nc):
        P32 = Phr.float().contiguous()
        U = U.contiguous()
        we_f, wq_f = we.detach(), wq.detach()
        rows = _offset_rows(idxq, wq_f, coset_of, nc)
        onehot = bool(((we_f == 0) | (we_f == 1)).all()) and bool((we_f.sum(-1) == 1).all())
        if onehot:
            e_star = we_f.argmax(-1, keepdim=True)
            y = _read_lists(P32, U, rows.gather(-1, e_star).squeeze(-1))
        else:
            y = (_read_pairs(P32, U, rows) * we_f.unsqueeze(-1)).sum(2)
        ctx.save_for_backward(P32, U, we_f, idxq, rows, coset_of)
        ctx.meta = (onehot, nc, Phr.dtype, we.dtype, wq.dtype)
        return y

    @staticmethod
    def backward(ctx, dy):
        P32, U, we_f, idxq, rows, coset_of = ctx.saved_tensors
        onehot, nc, d_phi, d_we, d_wq = ctx.meta
        B, T_R, D = we_f.shape
        K = idxq.shape[-1]
        dy = dy.float().contiguous()
        UT = U.transpose(-1, -2).contiguous()
        Gy = _read_pairs(dy, UT, rows)                        # (B, T_R, D, r)
        dwe = (Gy * P32.unsqueeze(2)).sum(-1)
        dPhi = (Gy * we_f.unsqueeze(-1)).sum(2)
        if onehot:
            e_star = we_f.argmax(-1, keepdim=True)
            dU = _gram_lists(P32, dy, rows.gather(-1, e_star).squeeze(-1), D * nc)
            rk = e_star * nc + coset_of[e_star.expand_as(idxq), idxq]
            dwq = (_read_pairs(dy, UT, rk) * P32.unsqueeze(2)).sum(-1)
        else:
            A = (P32.unsqueeze(2) * we_f.unsqueeze(-1)).reshape(B, T_R * D, -1)
            dU = _gram_lists(A, _repeat(dy, D), rows.reshape(B, T_R * D), D * nc)
            e = torch.arange(D, device=idxq.device).view(1, 1, D, 1)
            rk = (e * nc + coset_of[e.expand(B, T_R, D, K), idxq.unsqueeze(2).expand(B, T_R, D, K)])
            Z = (_read_pairs(dy, UT, rk.reshape(B, T_R, D * K)) * P32.unsqueeze(2)).sum(-1)
            dwq = (Z.view(B, T_R, D, K) * we_f.unsqueeze(-1)).sum(2)
        return dPhi.to(d_phi), dU, dwe.to(d_we), dwq.to(d_wq), None, None, None
