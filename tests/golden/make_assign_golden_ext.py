#!/usr/bin/env python3
"""Fixtures for ContentAssign's options beyond the point / plane reads of
``make_assign_golden.py``: the learned key convolution (``conv_width``), the
``mlp``, ``delta`` and ``fixed`` direction heads, a codimension between 1 and
dim, and the analysis methods ``cells_of``, ``oracle_dir`` and ``agreement``.

Like ``make_assign_golden.py`` it imports the reference's own ``assign.py``
and ``mask.py`` (in the build container only), builds the module after a fixed
seed, runs it on seeded inputs and stores inputs, parameters, outputs and
gradients as data:

    assign_golden_ext.npz   per case: the inputs (u, Phi, Psi, Vb, and ids for
                            the id hash), every parameter and buffer the case
                            adds (kconv, Wd1 / bd1 / Wd, Wdelta, id_cell, M),
                            the output y of the hard read, R and the gradients
                            of (y * R).sum() (every case draws the same u, Phi,
                            Psi, Vb: stored once under inputs/); for the
                            analysis case, cells_of
                            of random hidden states, oracle_dir of random cell
                            sets, and agreement's value with its gradients

Run from the repository root (needs /root/reference, numpy and torch):

    python tests/golden/make_assign_golden_ext.py
"""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np
import torch

REF = "/root/reference/src/smat"
REF_LM = "/root/reference/src/smat_lm"
HERE = os.path.dirname(os.path.abspath(__file__))

# (name, T, d, module options)
CASES = [
    ("T512_d3_point_conv4", 512, 3, dict(mode="point", conv_width=4)),
    ("T512_d3_plane_mlp", 512, 3, dict(mode="plane", dir_head="mlp", dir_hidden=32)),
    ("T512_d3_plane_delta", 512, 3, dict(mode="plane", src="id", vocab=64, dir_head="delta",
                                         dir_window=4)),
    ("T512_d3_plane_fixed", 512, 3, dict(mode="plane", src="id", vocab=64, dir_head="fixed",
                                         dir_window=3)),
    ("T512_d4_codim2", 512, 4, dict(codim=2)),
    ("T512_d4_codim3", 512, 4, dict(codim=3)),
]
H, DM, NB, R_FEAT = 2, 32, 1, 16


def _load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def _inputs(T, h, r, vocab=None):
    g = torch.Generator().manual_seed(2000)
    u = torch.randn(NB, T, DM, generator=g)
    Phi = torch.rand(NB * h, T, r, generator=g) + 0.5
    Psi = torch.rand(NB * h, T, r, generator=g) * 0.1 + 0.05
    Vb = torch.cat([torch.randn(NB * h, T, r, generator=g), torch.ones(NB * h, T, 1)], -1)
    ids = torch.randint(0, vocab, (NB, T), generator=g) if vocab else None
    return u, Phi, Psi, Vb, ids


def main():
    sys.path.insert(0, REF_LM)
    mask = _load("_ref_smat_mask", os.path.join(REF, "mask.py"))
    assign = _load("_ref_smat_assign", os.path.join(REF, "assign.py"))
    out = {}
    for name, T, d, opts in CASES:
        spec = mask.build_mask(T, d, chunk=64)
        n = spec.n
        torch.manual_seed(1000)
        m = assign.ContentAssign(H, DM, spec, **opts)
        m.eval()
        u, Phi, Psi, Vb, ids = _inputs(T, H, R_FEAT, opts.get("vocab"))
        kw = {} if ids is None else {"ids": ids}
        with torch.no_grad():
            y = m(u, Phi, Psi, Vb, n, **kw)
        # every case draws the same u, Phi, Psi, Vb (the generator's first draws):
        # stored once, under inputs/
        for key, t in (("u", u), ("Phi", Phi), ("Psi", Psi), ("Vb", Vb)):
            if f"inputs/{key}" in out:
                assert np.array_equal(out[f"inputs/{key}"], t.numpy())
            out[f"inputs/{key}"] = t.numpy()
        out[f"{name}/y"] = y.numpy()
        if ids is not None:
            out[f"{name}/ids"] = ids.numpy()
        params = {k: v.detach() for k, v in m.named_parameters()}
        params.update({k: v for k, v in m.named_buffers() if k in ("id_cell", "M")})
        for k, v in params.items():
            out[f"{name}/param.{k}"] = v.numpy()
        out[f"{name}/meta"] = np.array([T, d, n])
        R = torch.randn(y.shape, generator=torch.Generator().manual_seed(3000))
        xs = [t.detach().clone().requires_grad_(True) for t in (u, Phi, Psi, Vb)]
        m.zero_grad()
        yg = m(*xs, n, **kw)
        (yg * R).sum().backward()
        out[f"{name}/R"] = R.numpy()
        for key, t in zip(("u", "Phi", "Psi", "Vb"), xs):
            if t.grad is not None:
                out[f"{name}/grad.{key}"] = t.grad.numpy()
        for k, v in m.named_parameters():
            if v.grad is not None:
                out[f"{name}/grad.{k}"] = v.grad.numpy()

    # analysis methods on the d = 3 plane read of the hidden-state hash
    name, T = "T512_d3_analysis", 512
    spec = mask.build_mask(T, 3, chunk=64)
    n = spec.n
    torch.manual_seed(1000)
    m = assign.ContentAssign(H, DM, spec, mode="plane")
    m.eval()
    u, Phi, Psi, Vb, _ = _inputs(T, H, R_FEAT)
    g = torch.Generator().manual_seed(4000)
    v = torch.randn(3, 5, DM, generator=g)
    with torch.no_grad():
        out[f"{name}/cells_v"] = v.numpy()
        out[f"{name}/cells_of"] = m.cells_of(v).numpy()
    for k in (1, 2, 3):
        cells = torch.randint(0, spec.N0, (4, 6, k), generator=g)
        out[f"{name}/oracle_cells{k}"] = cells.numpy()
        out[f"{name}/oracle_dir{k}"] = m.oracle_dir(cells).numpy()
    xs = [t.detach().clone() for t in (u, Phi, Psi, Vb)]
    m.zero_grad()
    m(*xs, n)
    # pairs (recent query i, distant key j): j holds head 0's hard cell of the
    # query where one does, so the query's soft mass reaches its target and the
    # term has gradients
    P = 7
    hq = m.cells_of(u[:, n:])                                   # (nb, T_R, h)
    hk = m.last_hard_k                                          # (nb*h, n)
    qi = torch.randint(0, T - n, (NB, P), generator=g)
    kj = torch.randint(0, n, (NB, P), generator=g)
    for bb in range(NB):
        for pp in range(P):
            hit = torch.nonzero(hk[bb * H] == hq[bb, qi[bb, pp], 0]).flatten()
            if hit.numel():
                kj[bb, pp] = hit[0]
    pairs = torch.stack([qi, kj], -1)
    valid = torch.rand(NB, P, generator=g) < 0.8
    a = m.agreement(pairs, valid)
    a.backward()
    a = a.detach()
    out[f"{name}/pairs"] = pairs.numpy()
    out[f"{name}/valid"] = valid.numpy()
    out[f"{name}/agreement"] = np.array(float(a))
    out[f"{name}/hard_k"] = m.last_hard_k.numpy()
    for k in ("W", "gamma", "b"):
        out[f"{name}/grad.{k}"] = getattr(m, k).grad.numpy()
    np.savez_compressed(os.path.join(HERE, "assign_golden_ext.npz"), **out)
    print("wrote", len(CASES) + 1, "cases")


if __name__ == "__main__":
    main()
