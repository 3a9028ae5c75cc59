"""The SMat incidence and dense mask rebuilt from their definitions, with loops.

Test infrastructure (see ``oracle/__init__.py``).  Written for small cases and
kept deliberately naive so it shares no code path with the product's
vectorised ``smat_attention_amd.mask``: points are enumerated one by one,
hyperplane membership is tested point by point, and every mask entry is
evaluated from ``M^(d)``'s definition.

Follows src/smat/mask.py:91-126 (points, planted normals), :294-389 (the
geometric construction and its ordering) and :392-425 (endpoint), :557-577
(materialise).
"""
from __future__ import annotations

import math
from typing import List, Tuple


def is_prime(x: int) -> bool:
    return x >= 2 and all(x % f for f in range(2, int(math.isqrt(x)) + 1))


def field_size(n: int, d: int) -> int:
    """``nextprime(ceil(n ** (1/d)))`` in double precision (mask.py:296)."""
    x = max(2, int(math.ceil(float(n) ** (1.0 / d))))
    while not is_prime(x):
        x += 1
    return x


def point(idx: int, q: int, dim: int) -> Tuple[int, ...]:
    """Coordinates of point ``idx``, coordinate 0 most significant (mask.py:91-100)."""
    return tuple((idx // q ** (dim - 1 - k)) % q for k in range(dim))


def index_of(x, q: int) -> int:
    v = 0
    for c in x:
        v = v * q + int(c)
    return v


def directions(q: int, dim: int) -> List[Tuple[int, ...]]:
    """Nonzero points whose first nonzero coordinate is 1, in point order."""
    out = []
    for idx in range(q ** dim):
        x = point(idx, q, dim)
        nz = [c for c in x if c != 0]
        if nz and nz[0] == 1:
            out.append(x)
    return out


def planted(d: int) -> List[Tuple[Tuple[int, ...], int]]:
    """``(a_R, b_R)`` for bitmask ``R`` (mask.py:103-126)."""
    dim = d - 1
    out = []
    for R in range(1 << dim):
        if R == (1 << dim) - 1:
            out.append((tuple([1] * dim), 1))
        else:
            out.append((tuple(0 if (R >> k) & 1 else 1 for k in range(dim)), 0))
    return out


def geometry(T: int, d: int, chunk: int = 1, n_P: int = 0):
    """``dict(n, T_R, q, N0, B, deg, rows, planted_cols)`` for a geometric mask.

    ``rows[h]`` is the ascending list of points on the hyperplane of row type
    ``h``: planted hyperplanes first (bitmask order), then all others by flat
    index ``e*q + b`` (mask.py:347-373).
    """
    c = max(1, chunk)
    n = c * (T // (2 * c))
    T_R = T - n
    if d == 1:
        return dict(n=n, T_R=T_R, q=0, N0=1, B=1, deg=1, rows=[[0]],
                    planted_cols=[], n_P=0)
    dim = d - 1
    q = field_size(n, d)
    N0 = q ** dim
    dirs = directions(q, dim)
    flat = []                                   # flat index e*q + b
    for a in dirs:
        for b in range(q):
            flat.append([idx for idx in range(N0)
                         if sum(ai * xi for ai, xi in zip(a, point(idx, q, dim))) % q == b])
    plant = [dirs.index(a) * q + b for a, b in planted(d)]
    order = plant + [h for h in range(len(flat)) if h not in plant]
    B = len(flat)
    rows = [flat[h] for h in order[:B]]
    planted_cols = [n_P + q ** (dim - l) for l in range(1, dim + 1)]
    return dict(n=n, T_R=T_R, q=q, N0=N0, B=B, deg=q ** (dim - 1), rows=rows,
                planted_cols=planted_cols, n_P=n_P)


def endpoint_geometry(T: int, d: int):
    """``d = floor(log2 T)``: ``C[h, a] = 1{popcount(h & a) even}`` (mask.py:392-425)."""
    k = d - 1
    n = 1 << k
    rows = [[a for a in range(n) if bin(h & a).count("1") % 2 == 0] for h in range(n)]
    return dict(n=n, T_R=T - n, q=2, N0=n, B=n, deg=0, rows=rows, k=k, n_P=0)


def dense_mask(T: int, geo, endpoint: bool = False):
    """Every entry of ``M^(d)`` from its definition, as a list of lists of 0/1.

    Landmark block: ``L_n`` (geometric) or the zeta mask ``x subseteq a``
    (endpoint).  Recent-recent: causal.  Recent-landmark: the global channel
    ``j < n_P`` always, otherwise ``prof(j) in H_{i mod B}`` with
    ``prof(j) = (j - n_P) mod N0`` (identity for the endpoint).
    """
    n, B, N0, n_P = geo["n"], geo["B"], geo["N0"], geo["n_P"]
    member = [set(r) for r in geo["rows"]]
    M = [[0] * T for _ in range(T)]
    for i in range(T):
        for j in range(i + 1):
            if i < n:
                if endpoint:
                    M[i][j] = int((i & j) == j)
                else:
                    M[i][j] = 1
            elif j >= n:
                M[i][j] = 1
            elif j < n_P:
                M[i][j] = 1
            else:
                prof = (j - n_P) if endpoint else (j - n_P) % N0
                M[i][j] = int(prof in member[(i - n) % B])
    return M
