#!/usr/bin/env python3
"""Write the content-assignment fixtures that only the reference itself pins.

The hash of ``ContentAssign._cells`` (src/smat/assign.py:246-317) is float
arithmetic whose bins decide every token's cell, and the module's parameters
come from the global RNG in constructor order (:136-243); no closed form fixes
either.  This script imports the reference's own ``assign.py`` and
``mask.py`` (in the build container), builds the module after a fixed seed,
runs its forward on seeded inputs and stores inputs, parameters, cells and
outputs as data:

    assign_golden.npz   per case: u, Phi, Psi, Vb, W, gamma, b, [Wd], the key
                        cells (last_hard_k), the query cells (cells_of), the
                        load-balance term aux and the forward output y; every
                        case also R and the gradients of
                        (y * R).sum(): du, dPhi, dPsi, dVb, dW, dgamma, db
                        (and dWd for the plane read); an input equal to an
                        earlier case's is stored once, the later case holding
                        ``<key>.base``, the first holder's name, in its place

Run from the repository root (needs /root/reference, numpy and torch):

    python tests/golden/make_assign_golden.py
"""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np
import torch

REF = "/root/reference/src/smat"
REF_LM = "/root/reference/src/smat_lm"     # smat_pool_ops, imported by the sparse_ops path
HERE = os.path.dirname(os.path.abspath(__file__))

# (name, T, d, mode, heads, d_model, nb, anneal, sparse_ops): point and plane
# reads, d = 2 and 3; the soft phase (anneal < 1) of the dense read and the
# sparse_ops pair path (one chosen cell at anneal 1, all 2^dim pairs below)
CASES = [
    ("T512_d3_point", 512, 3, "point", 2, 64, 2, 1.0, False),
    ("T512_d3_plane", 512, 3, "plane", 2, 64, 2, 1.0, False),
    ("T512_d2_point", 512, 2, "point", 2, 64, 2, 1.0, False),
    ("T512_d3_point_soft", 512, 3, "point", 2, 64, 2, 0.5, False),
    ("T512_d3_point_sparse", 512, 3, "point", 2, 64, 2, 1.0, True),
    ("T512_d3_point_sparse_soft", 512, 3, "point", 2, 64, 2, 0.5, True),
    ("T512_d3_plane_sparse", 512, 3, "plane", 2, 64, 2, 1.0, True),
    ("T512_d3_plane_soft", 512, 3, "plane", 2, 64, 2, 0.5, False),
    ("T512_d3_plane_dirsoft", 512, 3, "plane", 2, 64, 2, 1.0, False),
]
DIR_SOFT = {"T512_d3_plane_dirsoft"}      # dir_soft mixes the directions in training mode
SHARED = ("u", "Phi", "Psi", "Vb", "W", "gamma", "b", "Wd", "R")


def _load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def main():
    sys.path.insert(0, REF_LM)
    mask = _load("_ref_smat_mask", os.path.join(REF, "mask.py"))
    assign = _load("_ref_smat_assign", os.path.join(REF, "assign.py"))
    out = {}
    for name, T, d, mode, h, dm, nb, anneal, sparse in CASES:
        spec = mask.build_mask(T, d, chunk=64)
        n, r = spec.n, 16
        torch.manual_seed(1000)
        m = assign.ContentAssign(h, dm, spec, mode=mode)
        m.eval()
        m.anneal = anneal
        m.sparse_ops = sparse
        if name in DIR_SOFT:
            m.dir_soft = True
            m.train()
        g = torch.Generator().manual_seed(2000)
        u = torch.randn(nb, T, dm, generator=g)
        Phi = torch.rand(nb * h, T, r, generator=g) + 0.5
        Psi = torch.rand(nb * h, T, r, generator=g) * 0.1 + 0.05
        Vb = torch.cat([torch.randn(nb * h, T, r, generator=g), torch.ones(nb * h, T, 1)], -1)
        with torch.no_grad():
            y = m(u, Phi, Psi, Vb, n)
            cq = m.cells_of(u[:, n:]).permute(0, 2, 1).reshape(nb * h, T - n)
        out[f"{name}/u"] = u.numpy()
        out[f"{name}/Phi"] = Phi.numpy()
        out[f"{name}/Psi"] = Psi.numpy()
        out[f"{name}/Vb"] = Vb.numpy()
        out[f"{name}/W"] = m.W.detach().numpy()
        out[f"{name}/gamma"] = m.gamma.detach().numpy()
        out[f"{name}/b"] = m.b.detach().numpy()
        if mode == "plane":
            out[f"{name}/Wd"] = m.Wd.detach().numpy()
        out[f"{name}/ck"] = m.last_hard_k.numpy()
        out[f"{name}/cq"] = cq.numpy()
        out[f"{name}/aux"] = np.array(float(m.aux))
        out[f"{name}/y"] = y.numpy()
        out[f"{name}/meta"] = np.array([T, d, h, dm, nb, n, r, 1 if mode == "plane" else 0])
        out[f"{name}/opts"] = np.array([anneal, 1.0 if sparse else 0.0,
                                        1.0 if name in DIR_SOFT else 0.0])
        # gradients of (y * R).sum() through the module's straight-through path
        R = torch.randn(y.shape, generator=torch.Generator().manual_seed(3000))
        xs = [t.detach().clone().requires_grad_(True) for t in (u, Phi, Psi, Vb)]
        m.zero_grad()
        yg = m(xs[0], xs[1], xs[2], xs[3], n)
        (yg * R).sum().backward()
        out[f"{name}/R"] = R.numpy()
        for key, t in zip(("du", "dPhi", "dPsi", "dVb"), xs):
            out[f"{name}/{key}"] = t.grad.numpy()
        out[f"{name}/dW"] = m.W.grad.numpy()
        out[f"{name}/dgamma"] = m.gamma.grad.numpy()
        out[f"{name}/db"] = m.b.grad.numpy()
        if mode == "plane":
            out[f"{name}/dWd"] = m.Wd.grad.numpy()
    # cases built from the same seeds share their inputs: keep each once and
    # point later cases at the first holder (``<case>/<key>.base``)
    first = {}
    for name, *_ in CASES:
        for key in SHARED:
            k = f"{name}/{key}"
            if k not in out:
                continue
            hit = next((b for b in first.get(key, []) if np.array_equal(out[f"{b}/{key}"], out[k])),
                       None)
            if hit is None:
                first.setdefault(key, []).append(name)
            else:
                del out[k]
                out[f"{name}/{key}.base"] = np.array(hit)
    np.savez_compressed(os.path.join(HERE, "assign_golden.npz"), **out)
    print("wrote", len(CASES), "cases")


if __name__ == "__main__":
    main()
