"""Host-side geometry of the SMat masks ``M^(d)``: parameters, incidence, audit.

The public names are those of the reference's ``src/smat/mask.py``
(``__all__`` at mask.py:51-61), so callers switch by changing the import.  All
of it is integer numpy work on the host; ``attention.to_device`` stages the
tables on the GPU.

With ``n`` landmark positions and ``T_R = T - n`` recent ones::

    M^(d) = [ L_n  0       ]        G[i, j] = 1{ prof(j) in H_{i mod B} }
            [ G    L_{T_R} ]        prof(j) = (j - n_P) mod N0

and ``C in {0,1}^{B x N0}`` the incidence between ``B`` affine hyperplanes of
``F_q^dim`` (``dim = d - 1``) and its ``N0 = q^dim`` points, so
``G = R C S^T``.

How the tables are produced here
--------------------------------
* :class:`_Plan` fixes every scalar of a mask (``n, q, N0, B, deg`` ...) and
  runs every admissibility check once; :func:`build_mask`, the probe,
  :func:`d_max_geometric` and :func:`estimate_cost` all start from it.
* :func:`_hyperplane_table` lists the points of all ``D*q`` hyperplanes at once
  from one integer matrix of inner products.
* :func:`_row_type_order` puts the planted hyperplanes first.
* The endpoint rows come from a Sylvester doubling of the Walsh sign matrix.

The order of ``C_indices`` must be the reference's, bit for bit, because it
decides which hyperplane each row type ``i mod B`` reads (mask.py:347-389):

* points of ``F_q^dim`` in lexicographic order, coordinate 0 most significant;
* directions: the nonzero points whose first nonzero coordinate is 1, in point
  order; hyperplane ``(e, b) = {x : <a_e, x> = b mod q}`` has flat index
  ``e*q + b``, and lists its points in ascending index;
* the ``2^dim`` planted hyperplanes (:func:`planted_hyperplane_normals`) come
  first, in bitmask order, then every other hyperplane by flat index,
  truncated to ``B``.
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
# integers (mask.py:68-100)
# ---------------------------------------------------------------------------

def next_prime(x: int) -> int:
    """The least prime ``p >= max(2, x)`` (mask.py:83-88), by trial division
    over 2 and the odd numbers up to ``sqrt(p)``."""
    p = max(2, int(x))
    while True:
        if p == 2 or (p % 2 and all(p % f for f in range(3, math.isqrt(p) + 1, 2))):
            return p
        p += 1


def _field_size(n: int, d: int) -> int:
    """``q = nextprime(ceil(n^(1/d)))``, evaluated as the reference does it.

    mask.py:296 takes the root in double precision, so ``32768 ** (1/3)`` is
    ``31.999...`` and ``q = nextprime(32) = 37`` rather than 33's successor;
    the same float expression keeps ``q`` equal at every ``(n, d)``.
    """
    return next_prime(int(math.ceil(float(n) ** (1.0 / d))))


def _digits(q: int, dim: int) -> np.ndarray:
    """Base-``q`` digits of ``0 .. q^dim - 1``, most significant first:
    row ``idx`` is the point of ``F_q^dim`` numbered ``idx`` (mask.py:91-100)."""
    out = np.zeros((q ** dim, dim), dtype=np.int64)
    rest = np.arange(q ** dim, dtype=np.int64)
    for k in range(dim - 1, -1, -1):
        rest, out[:, k] = np.divmod(rest, q)
    return out


def planted_hyperplane_normals(d: int) -> List[Tuple[np.ndarray, int]]:
    """The ``2^(d-1)`` planted hyperplanes ``(a_R, b_R)``, ``R`` a bitmask over
    the ``d-1`` coordinates (mask.py:103-126).

    The basis point ``e_i`` must lie on ``H_R`` exactly when bit ``i`` of
    ``R`` is set.  For ``R`` short of all bits, the normal is the complement
    indicator of ``R`` with offset 0 (``<a_R, e_i> = 0`` iff ``i in R``); the
    full mask uses the all-ones normal with offset 1 (every ``<1, e_i> = 1``).
    """
    dim = d - 1
    full = (1 << dim) - 1
    bits = (np.arange(1 << dim)[:, None] >> np.arange(dim)[None, :]) & 1
    normals = [(1 - bits[R]).astype(np.int64) for R in range(full)]
    normals.append(np.ones(dim, dtype=np.int64))
    return [(a, int(R == full)) for R, a in enumerate(normals)]


# ---------------------------------------------------------------------------
# the spec (mask.py:150-237)
# ---------------------------------------------------------------------------

@dataclass
class MaskSpec:
    """A built ``M^(d)``: scalars, the incidence ``C`` in CSR, and (after
    ``attention.to_device``) its device views.  Field names are the
    reference's; ``plane_ids`` is added here."""

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

    # flat hyperplane index e*q + b of each row type (geometric d >= 2)
    plane_ids: Optional[np.ndarray] = None

    @property
    def n_X(self) -> int:
        """Landmark columns that carry a profile."""
        return self.n - self.n_P

    @property
    def I_prof(self) -> int:
        """``nnz(C)``: the pooled long-range work."""
        return int(len(self.C_indices))

    @property
    def profile_degree(self) -> np.ndarray:
        """``nu(x)``, the number of row types whose hyperplane holds profile ``x``."""
        return np.bincount(self.C_indices, minlength=self.N0).astype(np.int64)

    @property
    def I_tok(self) -> int:
        """``sum_j nu(prof(j))``, what an unpooled per-column scatter pays:
        the profile degrees weighted by how many columns carry each profile."""
        uses = np.bincount(self.prof_of_column(), minlength=self.N0)
        return int(self.profile_degree @ uses)

    def prof_of_column(self) -> np.ndarray:
        """Profile of each profiled landmark column ``n_P + j``: ``j`` itself for
        the endpoint mask, round-robin ``j mod N0`` otherwise."""
        j = np.arange(self.n_X, dtype=np.int64)
        return j if self.kind == "endpoint" else np.remainder(j, self.N0)

    def row_type(self, i):
        """Type of recent row ``i`` (0-based inside the recent block)."""
        return i % self.B

    def dense_C(self) -> np.ndarray:
        """``C`` as a dense ``(B, N0)`` int8 0/1 matrix."""
        C = np.zeros((self.B, self.N0), dtype=np.int8)
        owner = np.repeat(np.arange(self.B), np.diff(self.C_indptr))
        C[owner, self.C_indices] = 1
        return C

    def summary(self) -> str:
        """One line naming the mask and its sizes."""
        size = f"nnz(C)={self.I_prof:,}" if self.C_indices is not None else "not built"
        if self.kind == "endpoint":
            return (f"endpoint M^({self.d}), T={self.T}: n=2^{self.k}={self.n}, "
                    f"B={self.B} Walsh row types, {size}")
        shape = (f"F_{self.q}^{self.dim}, N0={self.N0}, B={self.B} hyperplanes of "
                 f"{self.uniform_deg} points" if self.d >= 2 else "B=N0=1 (causal)")
        return (f"geometric M^({self.d}), T={self.T}: n={self.n} landmarks + "
                f"T_R={self.T_R} recent; {shape}; {size}"
                + (f", I_tok={self.I_tok:,}" if self.C_indices is not None else ""))


# ---------------------------------------------------------------------------
# planning: every scalar and every admissibility check (mask.py:244-340)
# ---------------------------------------------------------------------------

@dataclass
class _Plan:
    """The scalars of ``M^(d)`` at length ``T``, before any table is built."""

    T: int
    d: int
    chunk: int
    kind: str
    n: int
    T_R: int
    n_P: int = 0
    q: int = 0
    dim: int = 0
    N0: int = 1
    D: int = 0
    B: int = 1
    deg: int = 1
    n_planted: int = 0
    short_recent: str = ""        # why T_R is below the bound, when it is

    @staticmethod
    def of(T: int, d: int, chunk: int = 1, n_P: int = 0, B_frac: float = 1.0) -> "_Plan":
        """Plan ``M^(d)``; raises ValueError when no mask of this family exists."""
        if T < 8:
            raise ValueError(f"build_mask: the context must hold at least 8 tokens (T={T})")
        top = T.bit_length() - 1                      # floor(log2 T)
        if not 1 <= d <= top:
            raise ValueError(f"build_mask: d={d} is outside 1..floor(log2 T)={top} "
                             f"for T={T}")
        c = max(1, int(chunk))
        n = (T // (2 * c)) * c                        # the boundary on a chunk edge
        if n < 1:
            raise ValueError(f"build_mask: chunk={c} leaves no landmark block at T={T}")
        if d >= 2 and d == top:
            k = d - 1
            p = _Plan(T, d, c, "endpoint", 1 << k, T - (1 << k), q=2, dim=k, N0=1 << k,
                      D=1 << k, B=1 << k, deg=0)
            if p.T_R < p.B:
                p.short_recent = (f"T={T}: only {p.T_R} recent rows for the {p.B} Walsh "
                                  f"row types; some types never occur, and the "
                                  f"shattering bound of the endpoint mask is lost")
            return p
        if d == 1:                                    # M^(1) = L_T, one type, one profile
            return _Plan(T, 1, c, "geometric", n, T - n, deg=1)
        if not 0 <= n_P < n:
            raise ValueError(f"build_mask: the global channel n_P={n_P} must lie in "
                             f"[0, n={n})")
        dim = d - 1
        q = _field_size(n, d)
        N0 = q ** dim
        if N0 > n - n_P:
            raise ValueError(f"build_mask: T={T} is too short for d={d}: the {N0} points "
                             f"of F_{q}^{dim} need as many profiled landmark columns, "
                             f"and there are {n - n_P}")
        D = (N0 - 1) // (q - 1)
        n_planted = 1 << dim
        B = max(n_planted, min(int(round(B_frac * D * q)), D * q))
        p = _Plan(T, d, c, "geometric", n, T - n, n_P, q, dim, N0, D, B, q ** (dim - 1),
                  n_planted)
        if p.T_R < 2 * B:
            p.short_recent = (f"T={T}, d={d}: {p.T_R} recent rows cover fewer than two "
                              f"periods of the B={B} row types, which the VC lower "
                              f"bound needs")
        return p

    @property
    def nnz(self) -> int:
        if self.kind == "endpoint":
            # row 0 holds every point, each other Walsh row half of them
            return self.N0 + (self.B - 1) * (self.N0 // 2)
        return self.B * self.deg

    def spec(self, **arrays) -> MaskSpec:
        return MaskSpec(T=self.T, d=self.d, kind=self.kind, n=self.n, T_R=self.T_R,
                        chunk_align=self.chunk, q=self.q, dim=self.dim, N0=self.N0,
                        n_dirs=self.D, B=self.B, n_planted=self.n_planted,
                        k=self.dim if self.kind == "endpoint" else 0, n_P=self.n_P,
                        uniform_deg=self.deg, **arrays)


def d_max_geometric(T: int, *, chunk: int = 1, n_P: int = 0) -> int:
    """The largest ``d`` such that every geometric ``M^(2) .. M^(d)`` exists at
    this ``T`` with two full type periods in the recent block (mask.py:129-143)."""
    d = 1
    while True:
        try:
            p = _Plan.of(T, d + 1, chunk, n_P)
        except ValueError:
            return d
        if p.kind != "geometric" or p.short_recent:
            return d
        d += 1


# ---------------------------------------------------------------------------
# construction (mask.py:244-425)
# ---------------------------------------------------------------------------

def _hyperplane_table(q: int, dim: int) -> Tuple[np.ndarray, np.ndarray]:
    """Points of every affine hyperplane of ``F_q^dim``, and the directions.

    Returns ``members (D*q, q^(dim-1))``, row ``e*q + b`` listing the points
    ``x`` with ``<a_e, x> = b`` in ascending index, and ``dir_pts (D,)``, the
    point index of each direction ``a_e``.  One matrix of inner products
    ``(N0, D)`` holds all offsets; sorting each column by ``offset * N0 + x``
    lists direction ``e``'s ``q`` parallel hyperplanes one after the other,
    each in point order (the key is unique, so the sort needs no stability).
    """
    pts = _digits(q, dim)
    N0 = q ** dim
    first = np.argmax(pts != 0, axis=1)
    lead = pts[np.arange(N0), first]
    dir_pts = np.flatnonzero(lead == 1)               # the zero point has lead 0
    offsets = (pts @ pts[dir_pts].T) % q
    key = offsets * N0 + np.arange(N0, dtype=np.int64)[:, None]
    members = np.sort(key, axis=0).T % N0             # (D, N0), per direction
    return members.reshape(len(dir_pts) * q, N0 // q), dir_pts


def _row_type_order(q: int, dim: int, dir_pts: np.ndarray, B: int) -> np.ndarray:
    """Flat hyperplane index of each row type: the planted hyperplanes first
    (type ``R`` is ``H_R``), then the others by flat index, ``B`` in all."""
    dir_index = np.full(q ** dim, -1, dtype=np.int64)
    dir_index[dir_pts] = np.arange(len(dir_pts))
    place = q ** np.arange(dim - 1, -1, -1, dtype=np.int64)
    planted = np.array([dir_index[int(a @ place)] * q + b
                        for a, b in planted_hyperplane_normals(dim + 1)], dtype=np.int64)
    if planted.min() < 0 or len(np.unique(planted)) != len(planted):
        raise AssertionError("the planted normals must be distinct normalised directions")
    others = np.ones(len(dir_pts) * q, dtype=bool)
    others[planted] = False
    return np.concatenate([planted, np.flatnonzero(others)])[:B]


def _walsh_rows(k: int) -> Tuple[np.ndarray, np.ndarray]:
    """CSR of ``C[h, a] = 1{popcount(h & a) even}`` on ``2^k`` points: the +1
    entries of the Sylvester-Hadamard matrix ``H_k = [[H, H], [H, -H]]``."""
    H = np.ones((1, 1), dtype=np.int8)
    for _ in range(k):
        H = np.block([[H, H], [H, -H]])
    plus = H > 0
    indptr = np.zeros(len(H) + 1, dtype=np.int64)
    np.cumsum(plus.sum(axis=1), out=indptr[1:])
    return indptr, np.nonzero(plus)[1].astype(np.int32)


def build_mask(T: int, d: int, *, chunk: int = 1, n_P: int = 0,
               B_frac: float = 1.0, max_I_prof: Optional[int] = None,
               _probe: bool = False) -> MaskSpec:
    """``M^(d)`` at context length ``T`` (mask.py:244-425).

    The landmark block ends on a chunk edge, ``n = chunk * floor(T / 2 chunk)``.
    ``d = 1`` is the causal triangle with one profile and one row type;
    ``d = floor(log2 T)`` (>= 2) is the endpoint mask; every ``d`` between is
    the geometric mask over ``F_q^(d-1)``.  ``B_frac`` keeps that fraction of
    the ``D*q`` hyperplanes (the planted ones always).  ``n_P > 0`` reserves
    the first ``n_P`` landmark columns as a global channel every recent row
    sees.  A recent block shorter than two type periods is allowed with a
    warning; ``_probe`` (used by :func:`d_max_geometric`) refuses it instead,
    refuses the endpoint mask with NotImplementedError, and returns the
    scalars without tables.  ``max_I_prof`` bounds ``nnz(C)`` before anything
    is allocated (MemoryError).
    """
    t_start = time.perf_counter()
    plan = _Plan.of(T, d, chunk, n_P, B_frac)
    times: Dict[str, float] = {"plan": time.perf_counter() - t_start}
    warns = [plan.short_recent] if plan.short_recent else []

    if plan.kind == "endpoint":
        if _probe:
            raise NotImplementedError("build_mask: the endpoint mask (d = floor(log2 T)) "
                                      "is not a member of the geometric family")
        t = time.perf_counter()
        indptr, indices = _walsh_rows(plan.dim)
        times["walsh"] = time.perf_counter() - t
        spec = plan.spec(C_indptr=indptr, C_indices=indices,
                         planted_cols=np.left_shift(1, np.arange(plan.dim, dtype=np.int64)),
                         build_times=times, warnings=warns)
        spec.build_times["total"] = time.perf_counter() - t_start
        return spec

    if plan.d == 1:
        spec = plan.spec(C_indptr=np.array([0, 1], dtype=np.int64),
                         C_indices=np.zeros(1, dtype=np.int32),
                         planted_cols=np.zeros(0, dtype=np.int64))
        spec.build_times["total"] = time.perf_counter() - t_start
        return spec

    if _probe and plan.short_recent:
        raise ValueError(plan.short_recent)
    if max_I_prof is not None and plan.nnz > max_I_prof:
        raise MemoryError(f"build_mask: T={T}, d={d} has nnz(C) = {plan.nnz:,}, over "
                          f"max_I_prof = {max_I_prof:,}")
    if _probe:
        return plan.spec()

    t = time.perf_counter()
    members, dir_pts = _hyperplane_table(plan.q, plan.dim)
    times["hyperplanes"] = time.perf_counter() - t
    t = time.perf_counter()
    order = _row_type_order(plan.q, plan.dim, dir_pts, plan.B)
    rows = members[order].astype(np.int32)
    times["row_types"] = time.perf_counter() - t

    # profile of the basis point e_l (1-based l) is q^(dim-l): that column
    # carries e_l, so the planted rows see exactly the columns of their mask
    planted_cols = plan.n_P + plan.q ** np.arange(plan.dim - 1, -1, -1, dtype=np.int64)
    if planted_cols.max() >= plan.n:
        raise AssertionError("a planted column falls outside the landmark block")
    times["total"] = time.perf_counter() - t_start
    return plan.spec(C_indptr=np.arange(0, plan.B * plan.deg + 1, plan.deg, dtype=np.int64),
                     C_indices=rows.reshape(-1), planted_cols=planted_cols,
                     plane_ids=order, build_times=times, warnings=warns)


# ---------------------------------------------------------------------------
# audit (mask.py:432-482)
# ---------------------------------------------------------------------------

def _rows_strictly_increasing(spec: MaskSpec) -> bool:
    """Every row of ``C`` lists distinct points in ascending order (all rows)."""
    idx = spec.C_indices.astype(np.int64)
    step = np.diff(idx)
    inside = np.ones(len(step), dtype=bool)
    ends = spec.C_indptr[1:-1] - 1                    # last entry of each row but the last
    inside[ends[(ends >= 0) & (ends < len(step))]] = False
    return bool(np.all(step[inside] > 0))


def _rows_on_their_hyperplanes(spec: MaskSpec) -> bool:
    """Each row type's points satisfy ``<a_e, x> = b`` for its ``plane_ids``
    entry ``e*q + b``, and there are exactly ``q^(dim-1)`` of them."""
    q, dim = spec.q, spec.dim
    pts = _digits(q, dim)
    dirs = pts[np.flatnonzero(pts[np.arange(spec.N0), np.argmax(pts != 0, axis=1)] == 1)]
    e, b = np.divmod(spec.plane_ids, q)
    rows = spec.C_indices.reshape(spec.B, -1).astype(np.int64)
    lhs = np.einsum("hkj,hj->hk", pts[rows], dirs[e]) % q
    return bool(np.all(lhs == b[:, None]) and rows.shape[1] == q ** (dim - 1))


def incidence_audit(spec: MaskSpec) -> Dict[str, object]:
    """Check the incidence against the identities the cost model relies on.

    Facts: ``kind, d, T, q, N0, B, I_prof, I_tok, pool_gain`` (``I_tok /
    I_prof``) and the row / column degree ranges.  Checks, each a bool:

    * ``nnz_eq_sum_nu``: ``nnz(C)`` equals the sum of profile degrees;
    * ``rows_distinct_cols``: every row lists distinct points, ascending;
    * geometric ``d >= 2``: ``deg_is_q_pow_d_minus_2`` (uniform degree
      ``q^(d-2)``), ``full_hyperplane_family`` (``B = D q``) and then
      ``nu_is_D`` (every point on ``D`` rows), ``rows_on_hyperplanes`` (every
      row satisfies its hyperplane's equation), ``planted_identity``
      (``e_l in H_R`` iff bit ``l`` of ``R``), ``B_ge_2_pow_d_minus_1`` and
      ``T_R_ge_2B``;
    * endpoint: ``walsh_rows`` (``C`` is the even-parity matrix) and
      ``T_R_ge_B``.

    ``exact`` is the conjunction of the structural checks (not of the two
    length conditions, which only the lower bound needs).
    """
    nu = spec.profile_degree
    row_deg = np.diff(spec.C_indptr)
    facts: Dict[str, object] = {
        "kind": spec.kind, "d": spec.d, "T": spec.T, "q": spec.q, "N0": spec.N0,
        "B": spec.B, "I_prof": spec.I_prof, "I_tok": spec.I_tok,
        "pool_gain": spec.I_tok / max(1, spec.I_prof),
        "row_deg_min": int(row_deg.min()), "row_deg_max": int(row_deg.max()),
        "col_deg_min": int(nu.min()), "col_deg_max": int(nu.max()),
    }
    structural: Dict[str, bool] = {
        "nnz_eq_sum_nu": int(nu.sum()) == spec.I_prof,
        "rows_distinct_cols": _rows_strictly_increasing(spec),
    }
    lengths: Dict[str, bool] = {}
    if spec.kind == "geometric" and spec.d >= 2:
        q, dim = spec.q, spec.dim
        structural["deg_is_q_pow_d_minus_2"] = bool(np.all(row_deg == q ** (dim - 1)))
        full = spec.B == spec.n_dirs * q
        facts["full_hyperplane_family"] = full
        if full:
            structural["nu_is_D"] = bool(np.all(nu == spec.n_dirs))
        if spec.plane_ids is not None:
            structural["rows_on_hyperplanes"] = _rows_on_their_hyperplanes(spec)
        planted = spec.C_indices.reshape(spec.B, -1)[:spec.n_planted]
        profiles = np.asarray(spec.planted_cols) - spec.n_P
        seen = (planted[:, :, None] == profiles[None, None, :]).any(axis=1)   # (R, l)
        wanted = (np.arange(spec.n_planted)[:, None] >> np.arange(dim)[None, :]) & 1
        structural["planted_identity"] = bool(np.array_equal(seen, wanted.astype(bool)))
        lengths["B_ge_2_pow_d_minus_1"] = spec.B >= 1 << dim
        lengths["T_R_ge_2B"] = spec.T_R >= 2 * spec.B
    elif spec.kind == "endpoint":
        indptr, indices = _walsh_rows(spec.k)
        structural["walsh_rows"] = bool(np.array_equal(indptr, spec.C_indptr)
                                        and np.array_equal(indices, spec.C_indices))
        lengths["T_R_ge_B"] = spec.T_R >= spec.B
    out = dict(facts)
    out.update({k: bool(v) for k, v in structural.items()})
    out.update({k: bool(v) for k, v in lengths.items()})
    out["exact"] = all(structural.values())
    return out


# ---------------------------------------------------------------------------
# the constructive lower-bound witness (mask.py:489-550)
# ---------------------------------------------------------------------------

def _entry(spec: MaskSpec, i: int, j: int, C: np.ndarray) -> bool:
    """``M[n + i, j]`` for recent row ``i``, from the definition of the blocks."""
    if j >= spec.n:
        return i >= j - spec.n                        # L_{T_R}
    if j < spec.n_P:
        return True                                   # the global channel
    x = j - spec.n_P
    prof = x if spec.kind == "endpoint" else x % spec.N0
    return bool(C[i % spec.B, prof])


def shatter_witness(spec: MaskSpec):
    """``(cols, ok, rows)``: ``d`` columns every 0/1 pattern of which some row
    of ``M`` realises, each pattern's row named in ``rows`` and every entry
    read back from the block definitions.

    Geometric: the planted columns (profile ``e_l``) and recent column ``B``.
    Pattern ``(R, bit)`` is realised by recent row ``R + bit * B``: its type
    is ``R``, whose planted hyperplane holds ``e_l`` iff bit ``l`` of ``R``,
    and it lies at or past column ``B`` iff ``bit``.

    Endpoint: the columns ``2^j`` and the first recent column ``n``.  A pattern
    without the recent bit is the zeta row ``a`` = the union of its columns
    (``2^j`` is a subset of ``a`` iff bit ``j`` is set); one with it is recent
    row ``h < B`` of Walsh type ``h`` = the complement of the pattern's low
    bits (column ``2^j`` is in row ``h`` iff bit ``j`` of ``h`` is clear).
    """
    C = spec.dense_C()
    rows: Dict[object, object] = {}
    ok = True
    if spec.kind == "endpoint":
        k, n = spec.k, spec.n
        cols = [1 << j for j in range(k)] + [n]
        for pat in range(1 << (k + 1)):
            want = [bool((pat >> j) & 1) for j in range(k + 1)]
            low = pat & (n - 1)
            if not want[k]:
                got = [(c & low) == c for c in cols[:k]] + [False]
                rows[pat] = ("zeta", low) if got == want else None
            else:
                h = (n - 1) & ~low
                good = h < spec.T_R and [_entry(spec, h, c, C) for c in cols] == want
                rows[pat] = ("recent", h) if good else None
            ok &= rows[pat] is not None
        return cols, bool(ok), rows

    cols = [int(c) for c in spec.planted_cols] + [spec.n + spec.B]
    for R in range(1 << spec.dim):
        for bit in (0, 1):
            i = R + bit * spec.B
            want = [bool((R >> l) & 1) for l in range(spec.dim)] + [bool(bit)]
            ok &= i < spec.T_R and [_entry(spec, i, c, C) for c in cols] == want
            rows[(R, bit)] = i
    return cols, bool(ok), rows


# ---------------------------------------------------------------------------
# dense materialisation, O(T^2): verification only (mask.py:557-577)
# ---------------------------------------------------------------------------

def materialise(spec: MaskSpec, dtype=np.float64) -> np.ndarray:
    """The dense ``T x T`` 0/1 matrix ``M^(d)``, for checks at small ``T``.

    The recent rows' landmark block is periodic in the row with period ``B``
    (row ``i`` reads type ``i mod B``), so it is one period ``C[:, prof]``
    tiled down the recent block.
    """
    T, n, T_R = spec.T, spec.n, spec.T_R
    M = np.zeros((T, T), dtype=dtype)
    causal = np.tril(np.ones((max(n, T_R),) * 2, dtype=dtype))
    if spec.kind == "endpoint":
        a = np.arange(n, dtype=np.int64)
        M[:n, :n] = (a[:, None] | a[None, :]) == a[:, None]     # column a subset of row
    else:
        M[:n, :n] = causal[:n, :n]
    M[n:, n:] = causal[:T_R, :T_R]
    M[n:, :spec.n_P] = 1
    period = spec.dense_C()[:, spec.prof_of_column()]          # (B, n_X)
    reps = -(-T_R // spec.B)
    M[n:, spec.n_P:n] = np.tile(period, (reps, 1))[:T_R]
    return M


# ---------------------------------------------------------------------------
# cost model (mask.py:584-614)
# ---------------------------------------------------------------------------

def estimate_cost(T: int, d: int, r: int, d_v: int, *, chunk: int = 128,
                  n_P: int = 0) -> Dict[str, float]:
    """Work and memory of one forward pass of one sequence, without building
    ``C``.  Infeasible configurations give ``{"feasible": False, "reason": ...}``.

    MACs are those of the chunkwise schedule at feature rank ``r`` and
    ``p = d_v + 1`` value columns, counted as useful work:

    * ``intra``: the causal half of each chunk's score tile and its product
      with ``[V, 1]``, ``T (C + 1) / 2 (r + p)``;
    * ``states``: ``Phi . S_in`` and the chunk summaries, ``2 T r p``;
    * ``pool``: ``(n - n_P) r p``; ``query``: ``T_R r p``;
    * ``feature_map``: ``2 T r d_v`` when the maps are computed with the
      schedule (``d_qk`` taken equal to ``d_v``), reported apart.

    ``incidence_adds = nnz(C) r p`` is fp32 vector work, not MACs.  Bytes:
    ``inputs_bf16`` (Phi, Psi, Vb), ``output_fp32``, and the fp32 pooled tables
    ``F`` and ``U`` (``table_bytes_fp32``) when they cross memory.
    """
    try:
        plan = _Plan.of(T, d, chunk, n_P)
    except ValueError as e:
        return {"feasible": False, "reason": str(e)}
    if plan.kind == "geometric" and plan.d >= 2 and plan.short_recent:
        return {"feasible": False, "reason": plan.short_recent}
    p = d_v + 1
    C = min(chunk, T)
    rp = r * p
    macs = {
        "intra": T * (C + 1) / 2 * (r + p),
        "states": 2.0 * T * rp,
        "pool": float(plan.n - plan.n_P) * rp,
        "query": float(plan.T_R) * rp,
    }
    total = sum(macs.values())
    return {
        "feasible": True, "kind": plan.kind, "q": plan.q, "B": plan.B, "N0": plan.N0,
        "n": plan.n, "T_R": plan.T_R, "I_prof": plan.nnz,
        "macs": total, "mfma_flops": 2.0 * total,
        **{f"macs_{k}": v for k, v in macs.items()},
        "feature_map_macs": 2.0 * T * r * d_v,
        "incidence_adds": float(plan.nnz) * rp,
        "inputs_bf16": 2.0 * T * (2 * r + p),
        "output_fp32": 4.0 * T * d_v,
        "table_bytes_fp32": 4.0 * (plan.B + plan.N0) * rp,
        "dense_mask_bytes_fp32": 4.0 * T * T,
    }
