#!/usr/bin/env python3
"""Write the mask fixtures that only the reference implementation itself pins.

The invariants of the incidence (uniform degree, sorted distinct rows, every
member on its hyperplane, the planted identity, G == R C S^T) fix the SET of
hyperplanes but not their ORDER, and the order decides which hyperplane row
type ``i mod B`` reads.  So the exact ``C_indices`` permutation and
``planted_cols`` are taken from the reference's own ``build_mask``
(src/smat/mask.py:244-389) by importing it here, in the build container, and
stored as data:

    mask_golden.json    per (T, d, chunk, n_P): scalars, planted_cols and the
                        sha256 of C_indptr (int64) / C_indices (int32)
    mask_indices.npz    the full C_indices arrays for every case with
                        nnz(C) <= 100000

Run from the repository root (needs /root/reference, numpy only):

    python tests/golden/make_mask_golden.py
"""
from __future__ import annotations

import hashlib
import importlib.util
import json
import os
import sys

import numpy as np

REF_MASK = "/root/reference/src/smat/mask.py"
HERE = os.path.dirname(os.path.abspath(__file__))

# (T, d, chunk, n_P): every case the parity tests, the benchmark workloads and
# the reference's own tests build.
CASES = sorted(set([
    # test_smat.py structure / block layout / planted / equivalence / decode
    (256, 1, 64, 0), (512, 1, 64, 0), (1000, 1, 64, 0), (512, 2, 64, 0),
    (1024, 2, 64, 0), (1024, 3, 64, 0), (2048, 3, 64, 0), (2048, 4, 64, 0),
    (2048, 3, 64, 16), (1024, 3, 64, 16), (4096, 4, 64, 0), (16384, 5, 64, 0),
    (1024, 10, 64, 0), (128, 7, 8, 0), (256, 8, 8, 0), (300, 8, 8, 0),
    # chunk-width invariance
    (1024, 2, 32, 0), (1024, 2, 128, 0), (1024, 2, 256, 0),
    # incidence counting
    (4096, 2, 128, 0), (16384, 2, 128, 0), (4096, 3, 128, 0),
    (16384, 3, 128, 0), (65536, 3, 128, 0), (16384, 4, 128, 0),
    (65536, 4, 128, 0), (1024, 3, 128, 0), (1024, 2, 128, 0),
    # GPU parity shapes
    (2048, 3, 128, 0), (4096, 1, 128, 0), (8192, 3, 128, 0), (8192, 4, 128, 0),
    (2048, 1, 128, 0), (2048, 2, 128, 0), (8192, 2, 128, 0),
    # the workloads: CPU plumbing, single-GPU d=2, long prefill d=3 and its
    # d=1 control, training d=2/3, cached decode d=3
    (1024, 2, 128, 0), (8192, 2, 128, 0), (32768, 3, 128, 0),
    (131072, 3, 128, 0), (524288, 3, 128, 0), (32768, 1, 128, 0),
    (131072, 1, 128, 0), (524288, 1, 128, 0), (4096, 3, 128, 0),
    (65536, 3, 128, 0), (69632, 3, 128, 0),
]))


def _load_reference_mask():
    spec = importlib.util.spec_from_file_location("_ref_smat_mask", REF_MASK)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod          # dataclasses resolve the module
    spec.loader.exec_module(mod)
    return mod


def _sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main() -> int:
    ref = _load_reference_mask()
    rows, arrays = [], {}
    for T, d, chunk, n_P in CASES:
        s = ref.build_mask(T, d, chunk=chunk, n_P=n_P)
        key = f"T{T}_d{d}_c{chunk}_p{n_P}"
        ind = s.C_indices.astype(np.int32)
        ptr = s.C_indptr.astype(np.int64)
        rows.append(dict(
            key=key, T=T, d=d, chunk=chunk, n_P=n_P, kind=s.kind, n=s.n,
            T_R=s.T_R, q=s.q, dim=s.dim, N0=s.N0, n_dirs=s.n_dirs, B=s.B,
            n_planted=s.n_planted, k=s.k, uniform_deg=s.uniform_deg,
            nnz=int(ind.size), I_tok=int(s.I_tok),
            planted_cols=[int(x) for x in s.planted_cols],
            warnings=len(s.warnings),
            C_indptr_sha256=_sha(ptr), C_indices_sha256=_sha(ind)))
        if ind.size <= 100_000:
            arrays[key] = ind
        print(f"{key}: q={s.q} N0={s.N0} B={s.B} nnz={ind.size}")
    with open(os.path.join(HERE, "mask_golden.json"), "w") as f:
        json.dump({"source": "src/smat/mask.py:244-425 (build_mask)",
                   "cases": rows}, f, indent=1)
    np.savez_compressed(os.path.join(HERE, "mask_indices.npz"), **arrays)
    return 0


if __name__ == "__main__":
    sys.exit(main())
