"""Host-side geometry of the SMat masks ``M^(d)``: parameters, incidence, audit.

Interface follows the reference's ``src/smat/mask.py`` (``__all__`` at
mask.py:51-61) so callers switch by changing the import.  Everything here is
integer numpy work on the host; :func:`smat_attention_amd.attention.to_device`
stages the incidence on the GPU.

The mask, with ``n`` landmark positions and ``T_R = T - n`` recent ones::

    M^(d) = [ L_n  0       ]        G[i, j] = 1{ prof(j) in H_{i mod B} }
            [ G    L_{T_R} ]        prof(j) = (j - n_P) mod N0

``C in {0,1}^{B x N0}`` is the incidence between ``B`` affine hyperplanes of
``F_q^{d-1}`` and its ``N0 = q^{d-1}`` points; ``G = R C S^T``.

Ordering contract (bit-exact with mask.py:347-389):

* points of ``F_q^dim`` are numbered in lexicographic order, coordinate 0 most
  significant;
* normalised directions are the nonzero points whose first nonzero coordinate
  is 1, in point order; hyperplane ``(e, b)`` is ``{x : <a_e, x> = b mod q}``
  and gets flat index ``e * q + b``;
* each hyperplane lists its points in ascending point index;
* the ``2^{d-1}`` planted hyperplanes (:func:`planted_hyperplane_normals`) take
  row types ``0 .. 2^{d-1}-1`` in bitmask order, followed by every other
  hyperplane in ascending flat index, truncated to ``B``.
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np

__all__ = [
    "MaskSpec",
    "build_mask",
    "incidence_audit",
    "materialise",
    "estimate_cost",
    "next_prime",
    "d_max_geometric",
    "planted_hyperplane_normals",
    "shatter_witness",
]


# ---------------------------------------------------------------------------
# number theory (mask.py:68-88)
# ---------------------------------------------------------------------------

def _is_prime(x: int) -> bool:
    if x < 2:
        return False
    if x % 2 == 0:
        return x == 2
    f = 3
    while f * f <= x:
        if x % f == 0:
            return False
        f += 2
    return True


def next_prime(x: int) -> int:
    """Smallest prime ``>= max(2, x)`` (mask.py:83-88)."""
    p = max(2, int(x))
    while not _is_prime(p):
        p += 1
    return p


def _field_size(n: int, d: int) -> int:
    """``q = nextprime(ceil(n^(1/d)))`` with the reference's float pow.

    mask.py:296 evaluates ``n ** (1.0 / d)`` in double precision, so e.g.
    ``32768 ** (1/3) = 31.999...`` rounds up to 32, not to 33; the same
    expression is used here so ``q`` agrees at every ``(n, d)``.
    """
    return next_prime(int(math.ceil(float(n) ** (1.0 / d))))


def _lex_points(q: int, dim: int) -> np.ndarray:
    """``(q^dim, dim)`` coordinates of every point of ``F_q^dim`` (mask.py:91-100).

    Point ``idx`` has ``x_k = (idx // q^(dim-1-k)) mod q``; the basis vector
    ``e_l`` (1-based) is therefore point ``q^(dim-l)``.
    """
    if dim == 0:
        return np.zeros((1, 0), dtype=np.int64)
    idx = np.arange(q ** dim, dtype=np.int64)
    place = q ** np.arange(dim - 1, -1, -1, dtype=np.int64)
    return (idx[:, None] // place[None, :]) % q


def planted_hyperplane_normals(d: int) -> List[Tuple[np.ndarray, int]]:
    """The ``2^{d-1}`` planted ``(a_R, b_R)``, ``R`` a bitmask over ``[d-1]``.

    mask.py:103-126: for a proper subset ``R``, ``a_R`` is 0 on ``R`` and 1
    elsewhere with ``b_R = 0``; for ``R = [d-1]``, ``a_R = 1`` and ``b_R = 1``.
    Then ``e_i in H_R`` exactly when ``i in R``.
    """
    dim = d - 1
    full = (1 << dim) - 1
    out: List[Tuple[np.ndarray, int]] = []
    for R in range(1 << dim):
        bits = np.array([(R >> k) & 1 for k in range(dim)], dtype=np.int64)
        if R == full:
            out.append((np.ones(dim, dtype=np.int64), 1))
        else:
            out.append((1 - bits, 0))
    return out


def d_max_geometric(T: int, *, chunk: int = 1, n_P: int = 0) -> int:
    """Largest ``d`` whose geometric mask exists at this ``T`` (mask.py:129-143)."""
    d = 1
    while True:
        try:
            build_mask(T, d + 1, chunk=chunk, n_P=n_P, _probe=True)
        except (ValueError, NotImplementedError):
            return d
        d += 1


# ---------------------------------------------------------------------------
# the spec (mask.py:150-237)
# ---------------------------------------------------------------------------

@dataclass
class MaskSpec:
    """A precompiled ``M^(d)``; arrays are numpy, ``to_device`` adds GPU views."""

    T: int
    d: int
    kind: str                 # "geometric" | "endpoint"
    n: int                    # landmark positions [0, n)
    T_R: int                  # recent positions [n, T)
    chunk_align: int = 1

    q: int = 0
    dim: int = 0
    N0: int = 1
    n_dirs: int = 0
    B: int = 1
    n_planted: int = 0
    planted_cols: Optional[np.ndarray] = None

    k: int = 0                # endpoint: n = 2^k

    n_P: int = 0              # optional global channel: columns [0, n_P)

    C_indptr: Optional[np.ndarray] = None       # (B+1,) int64
    C_indices: Optional[np.ndarray] = None      # (nnz,) int32
    uniform_deg: int = 0                        # row degree if uniform, else 0

    build_times: Dict[str, float] = field(default_factory=dict)
    warnings: List[str] = field(default_factory=list)

    # device views, filled by attention.to_device
    C_indptr_t: object = None
    C_indices_t: object = None
    plane_pts_t: object = None                  # (B, uniform_deg) int64
    type_cols_t: object = None                  # (B, kappa) int32
    point_planes_t: object = None               # (N0, D) int32, transpose of C

    @property
    def n_X(self) -> int:
        return self.n - self.n_P

    @property
    def I_prof(self) -> int:
        return int(self.C_indices.size)

    @property
    def profile_degree(self) -> np.ndarray:
        return np.bincount(self.C_indices, minlength=self.N0).astype(np.int64)

    @property
    def I_tok(self) -> int:
        """``sum_j nu(prof(j))``: what an unpooled per-column scatter pays."""
        return int(self.profile_degree[self.prof_of_column()].sum())

    def prof_of_column(self) -> np.ndarray:
        cols = np.arange(self.n_X, dtype=np.int64)
        return cols if self.kind == "endpoint" else cols % self.N0

    def row_type(self, i):
        return i % self.B

    def dense_C(self) -> np.ndarray:
        C = np.zeros((self.B, self.N0), dtype=np.int8)
        rows = np.repeat(np.arange(self.B), np.diff(self.C_indptr))
        C[rows, self.C_indices] = 1
        return C

    def summary(self) -> str:
        if self.kind == "endpoint":
            return (f"M^({self.d}) endpoint T={self.T}: k={self.k} n={self.n} "
                    f"B={self.B} nnz(C)={self.I_prof:,}")
        return (f"M^({self.d}) T={self.T}: q={self.q} N0={self.N0} B={self.B} "
                f"deg={self.uniform_deg} n={self.n} T_R={self.T_R} "
                f"I_prof={self.I_prof:,} I_tok={self.I_tok:,}")


# ---------------------------------------------------------------------------
# construction (mask.py:244-425)
# ---------------------------------------------------------------------------

def build_mask(T: int, d: int, *, chunk: int = 1, n_P: int = 0,
               B_frac: float = 1.0, max_I_prof: Optional[int] = None,
               _probe: bool = False) -> MaskSpec:
    """Build ``M^(d)`` for context length ``T`` (mask.py:244-389).

    ``n = c * floor(T / 2c)`` with ``c = chunk``, so the landmark/recent
    boundary falls on a scan-chunk boundary.  ``d = floor(log2 T)`` (d >= 2)
    gives the endpoint mask; ``d = 1`` gives ``M^(1) = L_T`` with
    ``B = N0 = 1``.
    """
    if T < 8:
        raise ValueError(f"T must be >= 8, got {T}")
    d_ceiling = T.bit_length() - 1
    if not (1 <= d <= d_ceiling):
        raise ValueError(f"need 1 <= d <= floor(log2 T) = {d_ceiling}, got d={d}")
    c = max(1, int(chunk))
    n = c * (T // (2 * c))
    if n <= 0:
        raise ValueError(f"chunk={c} too large for T={T}")
    T_R = T - n
    t0 = time.perf_counter()

    if d == d_ceiling and d >= 2:
        return _build_endpoint(T, d, c, t0, _probe=_probe)

    if d == 1:
        spec = MaskSpec(T=T, d=1, kind="geometric", n=n, T_R=T_R, chunk_align=c,
                        q=0, dim=0, N0=1, n_dirs=0, B=1, n_planted=0,
                        planted_cols=np.zeros(0, dtype=np.int64), n_P=0,
                        C_indptr=np.array([0, 1], dtype=np.int64),
                        C_indices=np.zeros(1, dtype=np.int32), uniform_deg=1)
        spec.build_times["total"] = time.perf_counter() - t0
        return spec

    times: Dict[str, float] = {}
    warns: List[str] = []
    t = time.perf_counter()
    dim = d - 1
    q = _field_size(n, d)
    N0 = q ** dim
    times["prime"] = time.perf_counter() - t
    if n_P < 0 or n_P >= n:
        raise ValueError(f"n_P={n_P} out of range for n={n}")
    if N0 > n - n_P:
        raise ValueError(
            f"T={T}, d={d}: ambient |F_q^{dim}| = {N0} exceeds the {n - n_P} "
            f"profiled landmark columns; T is too small for this d")

    # normalised directions: nonzero points whose leading coordinate is 1
    t = time.perf_counter()
    pts = _lex_points(q, dim)
    nonzero = pts != 0
    has_nz = nonzero.any(axis=1)
    lead_val = pts[np.arange(N0), nonzero.argmax(axis=1)]
    dir_pts = np.flatnonzero(has_nz & (lead_val == 1))          # point indices
    D = int(dir_pts.size)
    if D != (q ** dim - 1) // (q - 1):
        raise AssertionError((D, q, dim))
    dir_of_point = np.full(N0, -1, dtype=np.int64)
    dir_of_point[dir_pts] = np.arange(D)
    B_max = D * q
    times["directions"] = time.perf_counter() - t

    n_planted = 1 << dim
    B = max(n_planted, min(int(round(B_frac * B_max)), B_max))
    if T_R < 2 * B:
        msg = (f"T={T}, d={d}: recent block T_R={T_R} < 2B={2 * B}; the type map "
               f"does not complete two cycles, so the VC lower bound does not apply")
        if _probe:
            raise ValueError(msg)
        warns.append(msg)
    deg = q ** (dim - 1)
    if max_I_prof is not None and B * deg > max_I_prof:
        raise MemoryError(f"T={T}, d={d}: nnz(C)={B * deg:,} exceeds "
                          f"max_I_prof={max_I_prof:,}")
    if _probe:
        return MaskSpec(T=T, d=d, kind="geometric", n=n, T_R=T_R, chunk_align=c,
                        q=q, dim=dim, N0=N0, n_dirs=D, B=B, n_planted=n_planted,
                        n_P=n_P, uniform_deg=deg)

    # every hyperplane's points: group the points of each direction by their
    # offset b = <a_e, x> mod q, ascending point index inside a group.  The
    # composite key b*N0 + idx is unique, so any sort gives that order.
    t = time.perf_counter()
    offs = (pts @ pts[dir_pts].T) % q                            # (N0, D)
    key = offs * N0 + np.arange(N0, dtype=np.int64)[:, None]
    members = np.argsort(key, axis=0).T.reshape(B_max, deg)      # row e*q+b
    times["incidence"] = time.perf_counter() - t

    # planted hyperplanes first, then the rest in flat order
    t = time.perf_counter()
    weights = q ** np.arange(dim - 1, -1, -1, dtype=np.int64)
    planted = []
    for a, b in planted_hyperplane_normals(d):
        e = int(dir_of_point[int(a @ weights)])
        if e < 0:
            raise AssertionError(f"planted normal {a} is not a normalised direction")
        planted.append(e * q + b)
    if len(set(planted)) != n_planted:
        raise AssertionError("planted hyperplanes are not distinct")
    keep = np.ones(B_max, dtype=bool)
    keep[planted] = False
    order = np.concatenate([np.asarray(planted, dtype=np.int64),
                            np.flatnonzero(keep)])[:B]
    plane_pts = members[order].astype(np.int32)
    times["reorder"] = time.perf_counter() - t

    planted_cols = n_P + q ** np.arange(dim - 1, -1, -1, dtype=np.int64)
    if planted_cols.size and planted_cols.max() >= n:
        raise AssertionError("planted column outside the landmark block")
    times["total"] = time.perf_counter() - t0
    return MaskSpec(T=T, d=d, kind="geometric", n=n, T_R=T_R, chunk_align=c,
                    q=q, dim=dim, N0=N0, n_dirs=D, B=B, n_planted=n_planted,
                    planted_cols=planted_cols, n_P=n_P,
                    C_indptr=np.arange(B + 1, dtype=np.int64) * deg,
                    C_indices=plane_pts.reshape(-1), uniform_deg=deg,
                    build_times=times, warnings=warns)


def _build_endpoint(T: int, d: int, c: int, t0: float, *,
                    _probe: bool = False) -> MaskSpec:
    """``d = floor(log2 T)`` (mask.py:392-425): zeta landmarks, Walsh rows.

    ``C[h, a] = 1{popcount(h & a) even}`` over ``n = B = 2^(d-1)``; row 0 is
    the whole space, so the rows are ragged.
    """
    k = d - 1
    n = 1 << k
    T_R = T - n
    B = n
    warns: List[str] = []
    if T_R < B:
        warns.append(f"T={T}: recent block T_R={T_R} < B={B}; fewer than one full "
                     f"Walsh cycle, so not every row type occurs and the lower "
                     f"bound fails.")
    if _probe:
        raise NotImplementedError("endpoint is not part of the geometric family")
    a = np.arange(n, dtype=np.int64)
    even = (np.bitwise_count(a[:, None] & a[None, :]) & 1) == 0      # (B, n)
    indptr = np.concatenate([[0], np.cumsum(even.sum(1))]).astype(np.int64)
    indices = np.nonzero(even)[1].astype(np.int32)
    spec = MaskSpec(T=T, d=d, kind="endpoint", n=n, T_R=T_R, chunk_align=c,
                    q=2, dim=k, N0=n, n_dirs=B, B=B, n_planted=0,
                    planted_cols=(1 << np.arange(k, dtype=np.int64)),
                    k=k, n_P=0, C_indptr=indptr, C_indices=indices,
                    uniform_deg=0, warnings=warns)
    spec.build_times["total"] = time.perf_counter() - t0
    return spec


# ---------------------------------------------------------------------------
# audit (mask.py:432-482)
# ---------------------------------------------------------------------------

def incidence_audit(spec: MaskSpec) -> Dict[str, object]:
    """Counting identities behind the cost bounds, checked on the built ``C``."""
    nu = spec.profile_degree
    row_deg = np.diff(spec.C_indptr)
    sampled = range(0, spec.B, max(1, spec.B // 32))
    out: Dict[str, object] = {
        "kind": spec.kind, "d": spec.d, "T": spec.T,
        "q": spec.q, "N0": spec.N0, "B": spec.B,
        "I_prof": spec.I_prof, "I_tok": spec.I_tok,
        "pool_gain": spec.I_tok / max(1, spec.I_prof),
        "row_deg_min": int(row_deg.min()), "row_deg_max": int(row_deg.max()),
        "col_deg_min": int(nu.min()), "col_deg_max": int(nu.max()),
        "nnz_eq_sum_nu": bool(spec.I_prof == int(nu.sum())),
        "rows_distinct_cols": bool(all(
            np.unique(spec.C_indices[spec.C_indptr[h]:spec.C_indptr[h + 1]]).size
            == row_deg[h] for h in sampled)),
    }
    if spec.kind == "geometric" and spec.d >= 2:
        q, dim = spec.q, spec.dim
        out["deg_is_q_pow_d_minus_2"] = bool(
            row_deg.min() == row_deg.max() == q ** (dim - 1))
        full = spec.B == spec.n_dirs * q
        out["full_hyperplane_family"] = bool(full)
        if full:
            out["nu_is_D"] = bool(nu.min() == nu.max() == spec.n_dirs)
        C = spec.dense_C()
        pcols = spec.planted_cols - spec.n_P
        ok = all(bool(C[R, pcols[l]]) == bool((R >> l) & 1)
                 for R in range(spec.n_planted) for l in range(dim))
        out["planted_identity"] = bool(ok)
        out["B_ge_2_pow_d_minus_1"] = bool(spec.B >= (1 << dim))
        out["T_R_ge_2B"] = bool(spec.T_R >= 2 * spec.B)
    if spec.kind == "endpoint":
        out["T_R_ge_B"] = bool(spec.T_R >= spec.B)
    out["exact"] = bool(out["nnz_eq_sum_nu"] and out["rows_distinct_cols"]
                        and out.get("planted_identity", True)
                        and out.get("deg_is_q_pow_d_minus_2", True))
    return out


# ---------------------------------------------------------------------------
# the constructive lower-bound witness (mask.py:489-550)
# ---------------------------------------------------------------------------

def shatter_witness(spec: MaskSpec):
    """``(cols, ok, rows)``: the ``d`` shattered columns, checked from the definition."""
    C = spec.dense_C()
    if spec.kind == "endpoint":
        k, n = spec.k, spec.n
        cols = [1 << j for j in range(k)] + [n]
        ok, rows = True, {}
        for pat in range(1 << (k + 1)):
            want = [bool((pat >> b) & 1) for b in range(k + 1)]
            found = None
            if not want[-1]:
                a = sum(cols[b] for b in range(k) if want[b])
                got = [((c & a) == c) if c < n else False for c in cols]
                found = ("zeta", a) if got == want else None
            else:
                for i in range(min(spec.T_R, spec.B)):
                    got = [bool(C[i % spec.B, c]) if c < n else (i >= c - n)
                           for c in cols]
                    if got == want:
                        found = ("recent", i)
                        break
            ok &= found is not None
            rows[pat] = found
        return cols, bool(ok), rows

    dim, n = spec.dim, spec.n
    cols = [int(c) for c in spec.planted_cols] + [n + spec.B]
    prof = spec.prof_of_column()

    def entry(i, j):
        if j < spec.n_P:
            return True
        if j < n:
            return bool(C[i % spec.B, prof[j - spec.n_P]])
        return i >= j - n

    ok, rows = True, {}
    for R in range(1 << dim):
        for bit in (0, 1):
            i = R + (spec.B if bit else 0)
            want = [bool((R >> l) & 1) for l in range(dim)] + [bool(bit)]
            ok &= (i < spec.T_R) and ([entry(i, c) for c in cols] == want)
            rows[(R, bit)] = i
    return cols, bool(ok), rows


# ---------------------------------------------------------------------------
# dense materialisation, O(T^2): verification only (mask.py:557-577)
# ---------------------------------------------------------------------------

def materialise(spec: MaskSpec, dtype=np.float64) -> np.ndarray:
    T, n, T_R = spec.T, spec.n, spec.T_R
    M = np.zeros((T, T), dtype=dtype)
    if spec.kind == "endpoint":
        a = np.arange(n, dtype=np.int64)
        M[:n, :n] = ((a[:, None] & a[None, :]) == a[None, :])
    else:
        M[:n, :n] = np.tri(n, dtype=dtype)
    M[n:, n:] = np.tri(T_R, dtype=dtype)
    if spec.n_P:
        M[n:, :spec.n_P] = 1
    C = spec.dense_C()
    rho = np.arange(T_R, dtype=np.int64) % spec.B
    M[n:, spec.n_P:n] = C[np.ix_(rho, spec.prof_of_column())]
    return M


# ---------------------------------------------------------------------------
# cost prediction (mask.py:584-614)
# ---------------------------------------------------------------------------

def estimate_cost(T: int, d: int, r: int, d_v: int, *, chunk: int = 128,
                  n_P: int = 0) -> Dict[str, float]:
    try:
        s = build_mask(T, d, chunk=chunk, n_P=n_P, _probe=True)
    except NotImplementedError:
        s = None
    except ValueError as e:
        return {"feasible": False, "reason": str(e)}
    p = d_v + 1
    if s is None or s.kind == "endpoint":
        k = d - 1
        B = N0 = 1 << k
        I_prof = B * (1 << max(0, k - 1))
        q = 2
    else:
        B, N0, q = s.B, s.N0, s.q
        I_prof = B * (s.uniform_deg if d >= 2 else 1)
    macs = (2 * T * r * d_v + T * chunk * (r + p) + 3 * T * r * p
            + I_prof * r * p)
    return {
        "feasible": True, "q": q, "B": B, "N0": N0, "I_prof": I_prof,
        "macs": float(macs),
        "table_bytes_fp32": 4.0 * (B + N0) * r * p,
        "dense_mask_bytes_fp32": 4.0 * T * T,
        "flash_macs": float(T) * T * (r + d_v),
    }
