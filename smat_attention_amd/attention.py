"""SMat attention's chunkwise schedule on MI355X: the Python surface.

Mirrors ``src/smat/attention.py`` (``__all__`` at attention.py:42-48), so a
caller switches by changing the import.  Everything runs on the GPU through
the HIP kernels of :mod:`smat_attention_amd.kernels.hip_fwd`; there is no
torch fallback, and a call that the kernels cannot serve raises.

Everything operates on kernel features ``Phi = phi(Q)``, ``Psi = h phi(K)``,
``Vb = [V, 1]`` (``p = d_v + 1`` columns), and the output is
``H[..., :-1] / H[..., -1:]`` with

    H = [[L_n, 0], [G, L_{T_R}]] Phi Psi^T Vb,      G = R C S^T,

computed as two passes summed before the single division:

  long range   F = S^T (Psi (x) Vb)   pool by profile      (pool)
               U = C F                 incidence            (incidence)
               Y = R (Phi_rec U)       type-major query     (query)
  causal       one chunked scan over all T with a single reset at n.

Reference differences, all deliberate:
  * ``backend="torch"`` / ``"walsh"`` select torch code in the reference; here
    they raise -- this package has one implementation, the kernels.
  * fp64 inputs raise (the reference keeps fp64 on torch, attention.py:109-121,
    so the kernels never see it there either).
  * ``featurise`` returns ``Vb`` as a view with 16-byte aligned rows (same
    values, padded row stride), the layout the kernels load fastest.
"""
from __future__ import annotations

from contextlib import nullcontext
from typing import Callable, Dict, Optional

import numpy as np
import torch

from .kernels import hip_fwd as _hip
from .mask import MaskSpec

__all__ = [
    "make_phi", "featurise", "to_device",
    "segmented_causal_scan", "decayed_segmented_scan", "combine_normalise", "pool_profiles",
    "apply_incidence",
    "query_by_type", "zeta_transform", "walsh_incidence", "direct_long_range",
    "smat_attention", "smat_attention_fused", "dense_masked_kernel_attention", "SmatDecoder",
    "have_triton", "have_hip",
]

_KERNEL_BACKENDS = ("auto", "hip", "triton")
# apply_incidence realisations (attention.py:239-285): "torch" is the gather
# (here the gather-reduce kernel), "walsh" the endpoint butterfly
_INCIDENCE_BACKENDS = _KERNEL_BACKENDS + ("torch", "walsh")


def have_hip() -> bool:
    """True when the HIP library is built and a GPU is visible."""
    return _hip.available()


def have_triton() -> bool:
    """Name kept from the reference (attention.py:54-55); means :func:`have_hip`."""
    return have_hip()


def _backend(name: str, who: str) -> None:
    if name not in _KERNEL_BACKENDS:
        raise ValueError(f"{who}: backend {name!r} is not available; this package runs "
                         f"only its HIP kernels ({', '.join(_KERNEL_BACKENDS)})")


def _acc(x: torch.Tensor, acc_dtype, who: str) -> torch.dtype:
    """The kernels accumulate and return fp32 (attention.py:109-127)."""
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"{who}: inputs must be bfloat16, float16 or float32, got {x.dtype}")
    if acc_dtype not in (None, torch.float32):
        raise TypeError(f"{who}: the kernels accumulate in float32, got acc_dtype={acc_dtype}")
    if not x.is_cuda:
        raise ValueError(f"{who}: inputs must be on the GPU, got {x.device}")
    return torch.float32


# ---------------------------------------------------------------------------
# feature map (attention.py:82-106)
# ---------------------------------------------------------------------------

def _wants_grad(*ts) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts)


class FeatureMap:
    """The map ``x -> elu(x W^T) + 1`` (or ``relu(x W^T) + 1e-3``) that
    :func:`make_phi` returns: callable like the reference's closure
    (attention.py:82-96), with ``W`` and ``kind`` exposed so :func:`featurise`
    can run it as one HIP launch.  GPU tensors only: there is no host path."""

    def __init__(self, W: torch.Tensor, kind: str):
        self.W, self.kind = W, kind

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if not x.is_cuda:
            raise TypeError("FeatureMap runs on the GPU only (the HIP featurise kernel); "
                            f"got a {x.device} tensor")
        if _wants_grad(x, self.W):
            from .kernels.hip_bwd import FeaturiseFunction
            return FeaturiseFunction.apply(self.W, self.kind, x, None, None, None)[0]
        return _hip.featurise(self.W, self.kind, x)[0]


def make_phi(d_qk: int, r: int, *, kind: str = "elu1", device="cpu",
             dtype=torch.float32, seed: int = 0) -> FeatureMap:
    """A positive rank-``r`` feature map with ``W ~ randn(r, d_qk)/sqrt(d_qk)``.

    ``W`` comes from a seeded CPU generator in float64 and is then cast, as in
    attention.py:82-96, so the same seed gives the same map on any device.
    """
    gen = torch.Generator(device="cpu").manual_seed(seed)
    W = (torch.randn(r, d_qk, generator=gen, dtype=torch.float64)
         / np.sqrt(d_qk)).to(device=device, dtype=dtype)
    if kind not in ("elu1", "relu"):
        raise ValueError(f"unknown feature map {kind!r}")
    return FeatureMap(W, kind)


def featurise(Q, K, V, phi, *, g=None, h=None):
    """``(Q, K, V) -> (Phi, Psi, Vb)`` with the key gate folded into ``Psi``.

    With a :class:`FeatureMap` on GPU tensors this is one HIP launch (both
    maps, the gate and ``[V, 1]``).  ``g`` is accepted and unused, as in the
    reference (the output gate is applied by :func:`smat_attention`).  Any
    other callable is the caller's own map and is called as given.  ``Vb`` is
    returned as a view whose rows start on 16-byte boundaries (row stride
    rounded up to 8 elements).  Gradients reach Q, K, V, h and W as in the
    reference (an autograd node around the launch).
    """
    if isinstance(phi, FeatureMap):
        if not Q.is_cuda:
            raise TypeError("featurise with a FeatureMap runs on the GPU only (the HIP "
                            f"featurise kernel); got {Q.device} tensors")
        if _wants_grad(Q, K, V, h, phi.W):
            # the HIP launch forward, the map's derivative backward
            from .kernels.hip_bwd import FeaturiseFunction
            return FeaturiseFunction.apply(phi.W, phi.kind, Q, K, V, h)
        return _hip.featurise(phi.W, phi.kind, Q, K, V, h)
    Phi = phi(Q)
    Psi = phi(K)
    if h is not None:
        Psi = Psi * h.unsqueeze(-1)
    d_v = V.shape[-1]
    p = d_v + 1
    pad = -(-p // 8) * 8
    buf = torch.empty(*V.shape[:-1], pad, device=V.device, dtype=V.dtype)
    buf[..., :d_v] = V
    buf[..., d_v:] = 1
    return Phi, Psi, buf[..., :p]


# ---------------------------------------------------------------------------
# device staging (attention.py:542-571)
# ---------------------------------------------------------------------------

def to_device(spec: MaskSpec, device, *, want_direct: bool = False) -> MaskSpec:
    """Stage the incidence on ``device``.

    Same attributes as the reference (``C_indptr_t``, ``C_indices_t`` int64,
    ``plane_pts_t`` the ``(B, deg)`` view when the degree is uniform), plus the
    int32 copies the kernels read.  Every index is range-checked on the host
    here, so the kernels can trust the tables.
    """
    ind = np.asarray(spec.C_indices)
    ptr_ = np.asarray(spec.C_indptr)
    if ind.size and (ind.min() < 0 or ind.max() >= spec.N0):
        raise ValueError("C_indices out of range [0, N0)")
    if ptr_[0] != 0 or ptr_[-1] != ind.size or np.any(np.diff(ptr_) < 0):
        raise ValueError("C_indptr is not a valid CSR row pointer")
    spec.C_indptr_t = torch.from_numpy(ptr_.astype(np.int64)).to(device)
    spec.C_indices_t = torch.from_numpy(ind.astype(np.int64)).to(device)
    spec.C_indices_i32_t = torch.from_numpy(ind.astype(np.int32)).to(device)
    spec.C_indices_par_t = (torch.from_numpy(parity_interleaved_table(spec)).to(device)
                            if spec.uniform_deg else spec.C_indices_i32_t)
    codes = plane_line_codes(spec)
    spec.plane_code_t = torch.from_numpy(codes).to(device) if codes is not None else None
    for t in (spec.C_indices_t, spec.C_indices_i32_t, spec.C_indices_par_t):
        t._smat_checked_N0 = spec.N0
    # C = I (every d = 2 geometric mask: row h is [h]): U = F exactly
    spec.incidence_identity = bool(spec.uniform_deg == 1 and spec.B == spec.N0
                                   and np.array_equal(ind, np.arange(spec.N0)))
    if spec.uniform_deg:
        spec.plane_pts_t = spec.C_indices_t.view(spec.B, spec.uniform_deg)
        spec.plane_pts_t._smat_checked_N0 = spec.N0
    else:
        spec.plane_pts_t = None
    if want_direct:
        if not spec.uniform_deg:
            raise ValueError("the direct backend needs a uniform row degree; "
                             "the endpoint mask is ragged")
        cols = _type_columns(spec)
        spec.type_cols_t = torch.from_numpy(cols).to(device)
        # the same lists with the n_X padding moved to the end of each row
        valid = cols < spec.n_X
        order = np.argsort(~valid, axis=1, kind="stable")
        spec.type_cols_c_t = torch.from_numpy(
            np.take_along_axis(cols, order, axis=1).astype(np.int32)).to(device)
        spec.type_counts_t = torch.from_numpy(valid.sum(1).astype(np.int32)).to(device)
    spec._smat_device = torch.device(device)
    return spec


def plane_line_codes(spec: MaskSpec) -> Optional[np.ndarray]:
    """``(B,)`` int32 codes ``e*q + b`` naming each row type's line of ``F_q^2``
    (d = 3), for the incidence kernel that generates the points itself; None for
    other masks.  Line ``e = 0`` is ``x1 = b``; line ``e >= 1`` is
    ``x0 + (e-1) x1 = b (mod q)``, with point ``x = x0*q + x1``.  Every code is
    checked here: the generated point set must equal the row of ``C``."""
    if spec.kind != "geometric" or spec.d != 3 or not spec.uniform_deg:
        return None
    q, B = spec.q, spec.B
    rows = np.sort(np.asarray(spec.C_indices, dtype=np.int64).reshape(B, q), axis=1)
    ids = getattr(spec, "plane_ids", None)
    if ids is not None and len(ids) == B:
        # build_mask recorded each row's line: regenerate and compare below
        e, b = np.divmod(np.asarray(ids, dtype=np.int64), q)
        vertical = e == 0
        return _checked_codes(q, rows, e, b, vertical)
    # a spec from elsewhere: recover each line from two of its points
    x0, x1 = rows // q, rows % q
    vertical = np.all(x1 == x1[:, :1], axis=1)          # e = 0: constant x1
    # e >= 1: x0 + m x1 = b with m from two points of the row (x1 distinct there)
    dx0 = (x0[:, 1] - x0[:, 0]) % q
    dx1 = (x1[:, 0] - x1[:, 1]) % q
    inv = np.array([pow(int(v), q - 2, q) if v else 0 for v in dx1], dtype=np.int64)
    m = (dx0 * inv) % q
    b = (x0[:, 0] + m * x1[:, 0]) % q
    e = np.where(vertical, 0, m + 1)
    b = np.where(vertical, x1[:, 0], b)
    return _checked_codes(q, rows, e, b, vertical)


def _checked_codes(q, rows, e, b, vertical):
    """``e*q + b`` as int32 if every generated line equals its (sorted) row of C."""
    t = np.arange(q, dtype=np.int64)[None, :]
    gen_vert = t * q + b[:, None]
    gen_sl = ((b[:, None] - (e[:, None] - 1) * t) % q) * q + t
    gen = np.sort(np.where(vertical[:, None], gen_vert, gen_sl), axis=1)
    if not np.array_equal(gen, rows):
        return None
    return (e * q + b).astype(np.int32)


def parity_interleaved_table(spec: MaskSpec) -> np.ndarray:
    """The ``(B*deg,)`` int32 point table with each row's points reordered for the
    LDS incidence kernel: even point indices first on even rows, odd first on odd
    rows (ascending within a parity).  The kernel reads the rows of two adjacent
    hyperplanes in one LDS cycle; opposite parities put them in opposite bank
    halves.  The same points per row, so the same U up to fp32 summation order."""
    deg = spec.uniform_deg
    pts = np.asarray(spec.C_indices, dtype=np.int64).reshape(spec.B, deg)
    odd = (pts & 1).astype(np.int64)
    first = (np.arange(spec.B) & 1)[:, None]                  # parity taken first
    key = (odd != first).astype(np.int64) * (2 * spec.N0) + pts
    order = np.argsort(key, axis=1, kind="stable")
    return np.take_along_axis(pts, order, axis=1).reshape(-1).astype(np.int32)


def _type_columns(spec: MaskSpec) -> np.ndarray:
    """``(B, kappa)`` landmark columns per row type, padded with ``n_X``.

    Profile ``x`` owns the columns ``x, x + N0, ...`` of the landmark block, so
    a row type's columns are those progressions for its ``deg`` points.
    """
    n_X, N0 = spec.n_X, spec.N0
    g = -(-n_X // N0)
    pts = spec.C_indices.reshape(spec.B, -1).astype(np.int64)
    cols = pts[:, :, None] + np.arange(g, dtype=np.int64)[None, None, :] * N0
    return np.where(cols < n_X, cols, n_X).reshape(spec.B, -1).astype(np.int32)


def _staged(spec: MaskSpec, device) -> MaskSpec:
    dev = torch.device(device)
    have = getattr(spec, "_smat_device", None)
    if getattr(spec, "C_indices_i32_t", None) is None or have is None or have != dev:
        to_device(spec, dev)
    return spec


def _incidence_args(spec: MaskSpec):
    """``(idx, indptr, deg)`` for the incidence kernel: the uniform ``(B, deg)``
    table (rows parity-interleaved) when there is one, else CSR."""
    if spec.uniform_deg:
        return spec.C_indices_par_t, None, int(spec.uniform_deg)
    return spec.C_indices_i32_t, spec.C_indptr_t, 0


# ---------------------------------------------------------------------------
# the stages (attention.py:134-330)
# ---------------------------------------------------------------------------

def segmented_causal_scan(Phi, Psi, Vb, n: int, chunk: int = 128,
                          acc_dtype=None, backend: str = "auto"):
    """``[[L_n, 0], [0, L_{T_R}]] Phi Psi^T Vb`` as one chunked scan with one reset.

    Chunks of up to 128 rows go through the fused scan kernel (state carried in
    registers across chunks, seeded per group of chunks by a shifted exclusive
    scan, never cumsum-minus-self, attention.py:163-179); wider chunks run the
    chunk summaries, the per-segment scan and the chunk-local pass as separate
    kernels.  Returns fp32 ``(nb, T, p)``.
    """
    who = "segmented_causal_scan"
    _backend(backend, who)
    _acc(Phi, acc_dtype, who)
    T = Phi.shape[1]
    C = min(chunk, T)
    if n % C:
        raise ValueError(f"segment boundary n={n} is not a multiple of chunk={C}")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (Phi, Psi, Vb)):
        # the reference differentiates its torch path; here one autograd node
        # with the HIP backward
        from .kernels.hip_bwd import CausalScanFunction
        return CausalScanFunction.apply(Phi, Psi, Vb, n, C,
                                        lambda P, S, V: _causal_scan(P, S, V, n, C))
    return _causal_scan(Phi, Psi, Vb, n, C)


def combine_normalise(H, Y, n: int, eps: float = 1e-6, out_dtype=torch.float32):
    """The layer's last step over the causal term ``H`` (nb, T, p) and the
    long-range term ``Y`` (nb, T - n, p) of the recent rows, in one kernel each
    way: ``N = cat([H[:, :n], H[:, n:] + Y], 1)``, then
    ``N[..., :-1] / N[..., -1:].clamp_min(eps)`` (model.py:296-300, 311-316),
    computed in fp32 and stored as ``out_dtype`` (fp32, or the layer's
    ``.to(x.dtype)`` cast of model.py:317 folded in: bf16 / fp16, rounded to
    nearest even).  ``Y`` may be None (no long-range rows).  Returns
    (nb, T, p - 1); differentiable in H and Y."""
    who = "combine_normalise"
    _hip._on_gpu(who, H, Y)
    nb, T, P = H.shape
    if not 0 <= n <= T or P < 2:
        raise ValueError(f"{who}: need 0 <= n <= T and p >= 2 (n={n}, T={T}, p={P})")
    if Y is not None and tuple(Y.shape) != (nb, T - n, P):
        raise ValueError(f"{who}: Y must be {(nb, T - n, P)}, got {tuple(Y.shape)}")
    if eps < 0:
        raise ValueError(f"{who}: eps must be >= 0")
    if out_dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise ValueError(f"{who}: out_dtype must be float32, bfloat16 or float16")
    from .kernels.hip_bwd import CombineNormaliseFunction
    return CombineNormaliseFunction.apply(H, Y, n, eps, out_dtype)


def _causal_scan(Phi, Psi, Vb, n: int, C: int):
    nb, T, r = Phi.shape
    p = Vb.shape[-1]
    if C <= 128:
        return _hip.causal_scan(Phi, Psi, Vb, n, C, write_H=True)
    # wide chunks: summaries, scan and chunk-local pass as separate kernels
    nc = -(-T // C)
    D = _hip.chunk_states(Psi, Vb, C)
    Sin = _hip.segment_scan(D, n // C)
    pad = nc * C - T
    if pad:
        Phi = torch.nn.functional.pad(Phi, (0, 0, 0, pad))
        Psi = torch.nn.functional.pad(Psi, (0, 0, 0, pad))
        Vb = torch.nn.functional.pad(Vb, (0, 0, 0, pad))
    out = _hip.chunk_local(Phi.reshape(nb, nc, C, r), Psi.reshape(nb, nc, C, r),
                           Vb.reshape(nb, nc, C, p), Sin)
    return out.reshape(nb, nc * C, p)[:, :T]


def decayed_segmented_scan(Phi, Psi, Vb, logA, n: int, chunk: int = 128):
    """The causal term with a selective decay (src/smat/model.py:41-82)::

        S_t = a_t S_{t-1} + psi_t vb_t^T,   y_t = Phi_t S_t,   a_t = exp(logA_t)

    with one reset at chunk ``n // chunk``, chunked, fp32, as the reference
    computes it: the within-chunk weights ``exp(L_i - L_j)`` (``L`` the running
    sum of ``logA`` inside a chunk, formed only for ``j <= i``), the chunk
    summaries ``sum_j exp(L_C - L_j) psi_j vb_j^T`` and the states carried
    across chunks with the total decay ``exp(L_C)``.  ``Phi, Psi (nb, T, r)``,
    ``Vb (nb, T, p)``, ``logA (nb, T)`` -> fp32 ``(nb, T, p)``.

    GPU work: the chunk summaries on the chunk-state kernel (over the
    decay-weighted Psi), the state recurrence ``smat_decay_scan`` and the
    within-chunk pass ``smat_chunk_local_decay``; the reference upcasts to
    fp32 first, and so does this (the fp32 MFMA path).  Gradients reach Phi,
    Psi, Vb and logA (an autograd node whose backward runs on smat_bgemm and
    ``smat_decay_scan_reverse``).
    """
    who = "decayed_segmented_scan"
    for t in (Phi, Psi, Vb, logA):
        if not t.is_cuda:
            raise ValueError(f"{who}: tensors must be on the GPU (got {t.device})")
    nb, T, r = Phi.shape
    if logA.shape != (nb, T):
        raise ValueError(f"{who}: logA is {tuple(logA.shape)}, expected {(nb, T)}")
    C = min(chunk, T)
    if torch.is_grad_enabled() and any(t.requires_grad for t in (Phi, Psi, Vb, logA)):
        from .kernels.hip_bwd import DecayedScanFunction
        return DecayedScanFunction.apply(Phi, Psi, Vb, logA, n, C)
    return _decayed_forward(*_decayed_inputs(Phi, Psi, Vb, logA, C), n, C)[0][:, :T]


def _decayed_inputs(Phi, Psi, Vb, logA, C: int):
    """fp32 copies padded to whole chunks (zero rows, zero log-decay)."""
    T = Phi.shape[1]
    pad = (-T) % C
    Ph, Ps, Vv, la = Phi.float(), Psi.float(), Vb.float(), logA.float()
    if pad:
        Ph = torch.nn.functional.pad(Ph, (0, 0, 0, pad))
        Ps = torch.nn.functional.pad(Ps, (0, 0, 0, pad))
        Vv = torch.nn.functional.pad(Vv, (0, 0, 0, pad))
        la = torch.nn.functional.pad(la, (0, pad))
    return Ph.contiguous(), Ps.contiguous(), Vv.contiguous(), la.contiguous()


def _decayed_forward(Ph, Ps, Vv, la, n: int, C: int):
    """(out (nb, Tp, p), L (nb, nc, C), Sin (nb, nc, r, p)) of the decayed scan
    over padded fp32 inputs."""
    nb, Tp, r = Ph.shape
    p = Vv.shape[-1]
    nc = Tp // C
    L = torch.cumsum(la.reshape(nb, nc, C), dim=-1)
    wj = torch.exp(L[..., -1:] - L)                               # decay to the chunk end, <= 1
    Psw = (Ps.reshape(nb, nc, C, r) * wj.unsqueeze(-1)).reshape(nb, Tp, r)
    D = _hip.chunk_states(Psw, Vv, C)
    Sin = _hip.decay_scan(D, torch.exp(L[..., -1]), n // C)
    out = _hip.chunk_local_decay(Ph.reshape(nb, nc, C, r), Ps.reshape(nb, nc, C, r),
                                 Vv.reshape(nb, nc, C, p), Sin, L)
    return out.reshape(nb, Tp, p), L, Sin


def pool_profiles(Psi, Vb, spec: MaskSpec, acc_dtype=None, backend: str = "auto"):
    """``F_x = sum_{prof(j)=x} Psi_j Vb_j^T``: fp32 ``(nb, N0, r, p)``."""
    who = "pool_profiles"
    _backend(backend, who)
    _acc(Psi, acc_dtype, who)
    return _hip.pool(Psi, Vb, spec.n_P, spec.n, spec.N0)


def apply_incidence(F, spec: MaskSpec, *, backend: str = "auto", gather_chunk: int = 0):
    """``U_h = sum_{x in H_h} F_x``: fp32 ``(nb, B, r, p)`` (attention.py:239-285).

    As in the reference, the endpoint mask takes the Walsh butterfly under
    ``"auto"``/``"walsh"``; every other case is the gather-reduce kernel
    (``"triton"`` requires a uniform degree, as the reference's kernel does).
    ``gather_chunk`` tuned the reference's torch gather and is ignored.
    """
    who = "apply_incidence"
    if backend not in _INCIDENCE_BACKENDS:
        raise ValueError(f"{who}: unknown backend {backend!r}")
    if not F.is_cuda:
        raise ValueError(f"{who}: F must be on the GPU")
    if spec.kind == "endpoint" and backend in ("auto", "walsh"):
        return walsh_incidence(F)
    if backend == "triton" and not spec.uniform_deg:
        raise ValueError("the triton incidence kernel needs a uniform row degree; this mask "
                         "is ragged (use walsh or torch)")
    _staged(spec, F.device)
    return _incidence(F, spec, None)


def _incidence(F, spec: MaskSpec, F_glob):
    """``C F`` (+ the global channel) through the fastest kernel the mask allows."""
    nb, N0, r, p = F.shape
    Ff = F.contiguous().float()
    if getattr(spec, "incidence_identity", False) and F_glob is None:
        return Ff                                    # C = I: U = F exactly
    U = torch.empty(nb, spec.B, r, p, device=F.device, dtype=torch.float32)
    profiled = spec.n > spec.n_P
    if profiled and getattr(spec, "plane_code_t", None) is not None and _plane_ok(spec, r * p):
        _hip.call("smat_incidence_plane", Ff.data_ptr(), _hip.ptr(F_glob),
                  spec.plane_code_t.data_ptr(), spec.q, U.data_ptr(), nb, N0, spec.B, r * p,
                  _hip.stream_of(Ff))
        return U
    idx, indptr, deg = _incidence_args(spec)
    _hip.call("smat_incidence", Ff.data_ptr(), _hip.ptr(F_glob), idx.data_ptr(), 0,
              _hip.ptr(indptr) if profiled else None, deg if profiled else 0,
              U.data_ptr(), nb, N0, spec.B, r * p, _hip.stream_of(Ff))
    return U


def _plane_ok(spec: MaskSpec, rp: int) -> bool:
    """The generated-line kernel needs rp % 4 == 0 and an N0 x 4 float panel on chip."""
    return rp % 4 == 0 and spec.N0 * 16 <= 150 * 1024


def query_by_type(Phi_rec, U, spec: MaskSpec):
    """``Y_{R_h} = Phi_{R_h} U_h``, ``rho(i) = i mod B``: fp32 ``(nb, T_R, p)``."""
    if U.shape[1] != spec.B:
        raise ValueError(f"query_by_type: U has {U.shape[1]} types, spec.B = {spec.B}")
    return _hip.query(Phi_rec, U)


def zeta_transform(F):
    """``(Z_k F)_a = sum_{x subset of a} F_x`` over ``N = 2^k`` profiles
    (attention.py:369-384): a k-stage butterfly in LDS, fp32 out of place."""
    nb, N = F.shape[0], F.shape[1]
    if N & (N - 1):
        raise AssertionError("zeta needs a power-of-two profile count")
    return _hip.zeta(F)


def walsh_incidence(F):
    """``C = (J + H)/2`` applied by a Walsh butterfly (attention.py:288-307):
    the endpoint mask's ``C[h, a] = 1{popcount(h & a) even}``, fp32."""
    nb, N = F.shape[0], F.shape[1]
    if N & (N - 1):
        raise AssertionError("Walsh route needs a power-of-two profile count")
    return _hip.walsh(F)


def direct_long_range(Psi, Vb, spec: MaskSpec, acc_dtype=None, type_chunk: int = 64):
    """The unpooled backend (attention.py:333-362): ``U_h`` summed straight from
    the landmark columns of row type ``h``, one Gram sum per type on the GPU.
    Needs ``to_device(spec, ..., want_direct=True)`` like the reference;
    ``type_chunk`` bounded the reference's gather and is ignored."""
    who = "direct_long_range"
    _acc(Psi, acc_dtype, who)
    if getattr(spec, "type_cols_c_t", None) is None:
        raise ValueError("the direct backend needs to_device(..., want_direct=True)")
    return _hip.direct(Psi, Vb, spec.type_cols_c_t, spec.type_counts_t, spec.n_P)


# ---------------------------------------------------------------------------
# full forward (attention.py:391-455)
# ---------------------------------------------------------------------------

def smat_attention(Phi, Psi, Vb, spec: MaskSpec, *, chunk: int = 128, g=None,
                   acc_dtype=None, timer=None, long_range: str = "pooled",
                   scan_backend: str = "auto", incidence_backend: str = "auto",
                   return_parts: bool = False, workspace: Optional[torch.Tensor] = None,
                   _no_grad_fn: bool = False):
    """Algorithm 1 of the reference (attention.py:391-455) on the GPU.

    Long range (pool by profile, incidence, type-major query) and the causal
    segmented scan are summed before the single division.  ``long_range`` is
    ``"pooled"``, ``"direct"`` (the unpooled comparison) or ``"subtractive"``
    (one unbroken scan minus the excluded mass, attention.py:458-482); the
    endpoint mask's landmark block goes through the zeta transform.  Returns
    fp32 ``(nb, T, d_v)``; with ``return_parts`` also the reference's parts.
    ``timer(name)`` (a context-manager factory) brackets the phases
    ``lr_pool``, ``lr_incidence``, ``lr_query``, ``zeta``, ``scan`` and
    ``normalise``.  The pooled schedule of a geometric mask without a timer or
    parts is one library call; ``workspace`` (uint8, on the device) may be
    passed to reuse its scratch.  When an input requires grad (and grad mode
    is on) that schedule is recorded as one autograd node whose backward runs
    on the HIP kernels
    (:class:`smat_attention_amd.kernels.hip_bwd.SmatAttentionFunction`).
    """
    who = "smat_attention"
    _backend(scan_backend, who)
    if incidence_backend not in _INCIDENCE_BACKENDS:
        raise ValueError(f"{who}: unknown incidence_backend {incidence_backend!r}")
    if long_range not in ("pooled", "direct", "subtractive"):
        raise ValueError(f"{who}: long_range must be pooled, direct or subtractive, "
                         f"got {long_range!r}")
    _acc(Phi, acc_dtype, who)
    if Psi.dtype != Phi.dtype or Vb.dtype != Phi.dtype:
        raise TypeError(f"{who}: Phi, Psi and Vb must share a dtype")
    nb, T, r = Phi.shape
    if T != spec.T:
        raise ValueError(f"{who}: T={T} but the mask was built for T={spec.T}")
    C = min(chunk, T)
    n = spec.n
    endpoint = spec.kind == "endpoint"
    segmented = long_range != "subtractive" and not endpoint
    if segmented and n % C:
        raise ValueError(f"segment boundary n={n} is not a multiple of chunk={C}")
    _staged(spec, Phi.device)
    plain = long_range == "pooled" and not endpoint

    wants_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (Phi, Psi, Vb, g))
    if wants_grad and not _no_grad_fn:
        if return_parts or timer is not None:
            if not plain or spec.plane_pts_t is None:
                raise NotImplementedError(
                    f"{who}: return_parts/timer under autograd are provided for the pooled "
                    f"schedule of a geometric mask; the {long_range} schedule"
                    f"{' of the endpoint mask' if endpoint else ''} records them under "
                    f"torch.no_grad() or on detached inputs")
            return _staged_with_grad(Phi, Psi, Vb, spec, C, g,
                                     timer or (lambda name: nullcontext()), return_parts)
        if endpoint:
            from .kernels.hip_bwd import EndpointAttentionFunction
            return EndpointAttentionFunction.apply(Phi, Psi, Vb, g, spec, C, long_range)
        from .kernels.hip_bwd import SmatAttentionFunction
        return SmatAttentionFunction.apply(Phi, Psi, Vb, g, spec, C, long_range)

    if plain and timer is None and not return_parts:
        idx, indptr, deg = _incidence_args(spec)
        pc = spec.plane_code_t if _plane_ok(spec, r * Vb.shape[-1]) else None
        if getattr(spec, "incidence_identity", False) and spec.n_P == 0:
            idx, pc = None, None                     # the query reads F as U
        return _hip.forward(Phi, Psi, Vb, idx, deg, n=n, n_P=spec.n_P, N0=spec.N0, B=spec.B,
                            chunk=C, indptr=indptr, plane_code=pc, field_q=spec.q, g=g,
                            workspace=workspace)

    tm = timer or (lambda name: nullcontext())
    if long_range == "subtractive":
        return _subtractive(Phi, Psi, Vb, spec, C, g, tm, return_parts, incidence_backend)
    parts: Dict[str, torch.Tensor] = {}
    p = Vb.shape[-1]
    F = None
    with tm("lr_pool"):
        F_glob = (torch.empty(nb, r, p, device=Phi.device, dtype=torch.float32)
                  if spec.n_P else None)
        if long_range == "pooled" or endpoint:
            F = _hip.pool(Psi, Vb, spec.n_P, n, spec.N0, F_glob=F_glob)
        elif F_glob is not None:        # direct: only the global channel's rank-one term
            _hip.pool(Psi, Vb, spec.n_P, spec.n_P, 1, F_glob=F_glob)
    with tm("lr_incidence"):
        if long_range == "direct":
            U = direct_long_range(Psi, Vb, spec)
            if F_glob is not None:
                U += F_glob.unsqueeze(1)
        elif endpoint and incidence_backend in ("auto", "walsh"):
            U = walsh_incidence(F)
        else:
            U = _incidence(F, spec, F_glob)
    with tm("lr_query"):
        Y_lr = _hip.query(Phi[:, n:], U)
    if endpoint:
        with tm("zeta"):
            if F is None:
                F = _hip.pool(Psi, Vb, 0, n, spec.N0)
            top = _hip.query(Phi[:, :n], _hip.zeta(F, out=F))   # row t reads Z_t
        with tm("scan"):
            loc = segmented_causal_scan(Phi[:, n:], Psi[:, n:], Vb[:, n:], n=0, chunk=C)
        H = torch.cat([top, loc], dim=1)
        parts["zeta"] = top
    else:
        with tm("scan"):
            H = segmented_causal_scan(Phi, Psi, Vb, n=n, chunk=C)
    if return_parts:
        # H is this call's own buffer: the long-range term goes into it in
        # place, and the parts' H is the sum the division reads
        with tm("normalise"):
            H[:, n:] += Y_lr
            out = _hip.normalise(H, n, None, g)
        parts.update(U=U, Y_lr=Y_lr, H=H)
        return out, parts
    with tm("normalise"):
        out = _hip.normalise(H, n, Y_lr, g)
    return out


def _staged_with_grad(Phi, Psi, Vb, spec, C, g, tm, return_parts):
    """The pooled schedule phase by phase, each phase an autograd node on the
    HIP kernels, for a differentiable call that asks for its parts or times its
    phases (the reference's torch path does both under autograd,
    attention.py:391-455): the pool (and the global channel's rank-one term,
    a pool of the first n_P tokens into one profile), the incidence, the
    type-major query, the segmented causal scan and the division.  The parts
    are part of the graph, as the reference's are."""
    from .kernels import hip_bwd as HB
    n, n_P, N0, B = spec.n, spec.n_P, spec.N0, spec.B
    with tm("lr_pool"):
        F = HB.pool(Psi, Vb, n_P, n, N0)
        F_glob = HB.pool(Psi, Vb, 0, n_P, 1)[:, 0] if n_P else None
    with tm("lr_incidence"):
        U = HB.incidence(F, spec.plane_pts_t, B)
        if F_glob is not None:
            U = U + F_glob.unsqueeze(1)
    with tm("lr_query"):
        Y_lr = HB.QueryFunction.apply(Phi[:, n:], U) if Phi.shape[1] > n else None
    with tm("scan"):
        H = segmented_causal_scan(Phi, Psi, Vb, n=n, chunk=C)
    with tm("normalise"):
        out = HB.NormaliseFunction.apply(H, Y_lr, g, n)
    if not return_parts:
        return out
    Hfull = H if Y_lr is None else torch.cat([H[:, :n], H[:, n:] + Y_lr], dim=1)
    return out, {"U": U, "Y_lr": Y_lr, "H": Hfull}


def _fused_ok(Q, K, V, phi, spec, C, h) -> bool:
    """Whether :func:`smat_attention_fused` runs the fused kernels for these inputs."""
    if not (isinstance(phi, FeatureMap) and Q.is_cuda
            and Q.dtype in (torch.bfloat16, torch.float16)):
        return False
    if spec.kind == "endpoint" or tuple(phi.W.shape) != (128, 128) or phi.W.dtype != Q.dtype:
        return False
    nb, T, dqk = Q.shape
    if dqk != 128 or K.shape != Q.shape or V.shape != Q.shape or K.dtype != Q.dtype \
            or V.dtype != Q.dtype or (h is not None and h.dtype != Q.dtype):
        return False
    if C not in (64, 128) or T % 64 or spec.n % C:
        return False
    # the fused pool runs one workgroup per (sequence, profile): with fewer than
    # 256 of them the unfused pool's split-K reduction is the faster path --
    # except for one profile holding every landmark token (d = 1, no global
    # channel), whose pool the fused forward takes from the causal pass's
    # group sums
    one_profile = spec.N0 == 1 and spec.B == 1 and spec.n_P == 0
    if T > spec.n and spec.n > spec.n_P and nb * spec.N0 < 256 and not one_profile:
        return False
    for t in (Q, K, V):
        if t.stride(-1) != 1 or t.stride(1) % 8 or t.stride(0) % 8 or t.data_ptr() % 16:
            return False
    return phi.W.is_contiguous() and phi.W.data_ptr() % 16 == 0


def smat_attention_fused(Q, K, V, phi, spec: MaskSpec, *, g=None, h=None, chunk: int = 128,
                         workspace: Optional[torch.Tensor] = None):
    """``smat_attention(*featurise(Q, K, V, phi, h=h), spec, g=g)`` with the
    feature map computed inside the schedule's kernels (the reference's
    featurise, attention.py:82-106, then Algorithm 1, :391-455).

    For 16-bit inputs at d_qk = d_v = r = 128 (the streaming shape: T, n and the
    chunk multiples of 64) the pool, the
    query, the prepass and the scan form ``Phi = map(Q W^T)``, ``Psi = h
    map(K W^T)`` and ``Vb = [V, 1]`` in LDS from the Q, K, V tiles they stream
    (``smat_forward_fused``), bitwise the features :func:`featurise` writes,
    so the output equals the unfused path's while Phi, Psi and Vb never reach
    memory (where a row type has more than 64 recent rows, the recent rows'
    Phi alone is featurised for the general query kernel; d = 1's single
    profile is pooled from the causal pass's group sums).  Other inputs --
    other widths and dtypes, fewer than 256 (sequence, profile) pools with
    more than one profile or a global channel -- and inputs that require grad
    run :func:`featurise` then :func:`smat_attention`.  Returns fp32 (nb, T, d_v).
    """
    who = "smat_attention_fused"
    _hip._on_gpu(who, Q, K, V, g, h)
    T = Q.shape[1]
    if T != spec.T:
        raise ValueError(f"{who}: T={T} but the mask was built for T={spec.T}")
    C = min(chunk, T)
    if _wants_grad(Q, K, V, g, h, phi.W if isinstance(phi, FeatureMap) else None) \
            or not _fused_ok(Q, K, V, phi, spec, C, h):
        Phi, Psi, Vb = featurise(Q, K, V, phi, h=h)
        return smat_attention(Phi, Psi, Vb, spec, chunk=chunk, g=g, workspace=workspace)
    _staged(spec, Q.device)
    idx, indptr, deg = _incidence_args(spec)
    pc = spec.plane_code_t if _plane_ok(spec, 128 * 129) else None
    if getattr(spec, "incidence_identity", False) and spec.n_P == 0:
        idx, pc = None, None                         # the query reads F as U
    return _hip.forward_fused(phi.W, phi.kind, Q, K, V, h, idx, deg, n=spec.n, n_P=spec.n_P,
                              N0=spec.N0, B=spec.B, chunk=C, indptr=indptr, plane_code=pc,
                              field_q=spec.q, g=g, workspace=workspace)


def _subtractive(Phi, Psi, Vb, spec, C, g, tm, return_parts, incidence_backend):
    """Remark 3.10 (attention.py:458-482): one unbroken causal scan minus the
    excluded long-range mass ``Ybar = R (F_tot - U)``.  The complement kernel
    forms ``U - F_tot`` in place, so the query returns ``-Y_ex`` and the
    normalisation adds it."""
    n = spec.n
    with tm("lr_pool"):
        F = _hip.pool(Psi, Vb, spec.n_P, n, spec.N0)
    with tm("lr_incidence"):
        if spec.kind == "endpoint" and incidence_backend in ("auto", "walsh"):
            U = walsh_incidence(F)
        else:
            U = _incidence(F, spec, None)
        _hip.incidence_complement(F, U)
    with tm("lr_query"):
        Y_neg = _hip.query(Phi[:, n:], U)
    with tm("scan"):
        H = segmented_causal_scan(Phi, Psi, Vb, n=0, chunk=C)
    with tm("normalise"):
        out = _hip.normalise(H, n, Y_neg, g)
    if return_parts:
        Hfull = H.clone()
        Hfull[:, n:] += Y_neg
        return out, {"H": Hfull, "Y_ex": -Y_neg}
    return out


def dense_masked_kernel_attention(Phi, Psi, Vb, M):
    """``O(T^2)`` definition (attention.py:485-489).  Verification only: it is
    not a kernel path and computes with plain (non-batched-view) products."""
    A = (Phi @ Psi.transpose(-1, -2).contiguous()) * M
    H = A @ Vb
    return H[..., :-1] / H[..., -1:]


# ---------------------------------------------------------------------------
# streaming decode (attention.py:496-535)
# ---------------------------------------------------------------------------

class SmatDecoder:
    """Exact autoregressive decoding at ``O(rp)`` per token, flat in ``T``.

    Every landmark key precedes every recent query, so the type table
    ``U = C S^T (Psi (x) Vb)`` over the prefix is fixed after prefill (built
    here by the pool and incidence kernels); each step adds ``psi vb^T`` to the
    running state ``S`` and reads ``U[i mod B]`` (attention.py:496-528).  The
    state is double-buffered on the device; :attr:`S` is the current one.
    """

    def __init__(self, Psi_prefix, Vb_prefix, spec: MaskSpec, *, acc_dtype=None,
                 incidence_backend: str = "auto"):
        who = "SmatDecoder"
        if incidence_backend not in _INCIDENCE_BACKENDS:
            raise ValueError(f"{who}: unknown incidence_backend {incidence_backend!r}")
        _acc(Psi_prefix, acc_dtype, who)
        self.spec = spec
        self.acc = torch.float32
        nb, _, r = Psi_prefix.shape
        p = Vb_prefix.shape[-1]
        self.nb, self.r, self.p = nb, r, p
        dev = Psi_prefix.device
        _staged(spec, dev)
        F_glob = torch.empty(nb, r, p, device=dev, dtype=torch.float32) if spec.n_P else None
        Vp = Vb_prefix
        if (Vp.dtype in (torch.bfloat16, torch.float16) and Vp.dim() == 3
                and (Vp.stride(-1) != 1 or Vp.stride(1) % 8 or Vp.stride(0) % 8)):
            # 16-byte aligned rows (a view of rows padded to 8 elements) let the
            # pool use its vector-load kernels; one copy of the prefix pays for
            # itself several times over at long T
            pad = -(-p // 8) * 8
            buf = torch.empty(*Vp.shape[:-1], pad, device=Vp.device, dtype=Vp.dtype)
            buf[..., :p] = Vp
            Vp = buf[..., :p]
        F = _hip.pool(Psi_prefix, Vp, spec.n_P, spec.n, spec.N0, F_glob=F_glob)
        if spec.kind == "endpoint" and incidence_backend in ("auto", "walsh"):
            self.U = walsh_incidence(F)
        else:
            self.U = _incidence(F, spec, F_glob)
        del F
        self._S = [torch.zeros(nb, r, p, device=dev, dtype=torch.float32),
                   torch.empty(nb, r, p, device=dev, dtype=torch.float32)]
        self._cur = 0
        self.i = 0

    @property
    def S(self) -> torch.Tensor:
        return self._S[self._cur]

    def advance(self, Psi_block, Vb_block) -> None:
        """Take the next ``L`` recent tokens into the running state at once:
        ``S += sum_t psi_t vb_t^T`` over the block (one Gram launch) and the
        step counter moves by ``L``, as ``L`` calls of :meth:`step` would leave
        them.  For resuming decode after a chunked prefill of those tokens
        (the reference steps through them one by one, attention.py:522-528).
        ``Psi_block (nb, L, r)``, ``Vb_block (nb, L, p)``."""
        who = "SmatDecoder.advance"
        nb, L, r = Psi_block.shape
        if (nb, r) != (self.nb, self.r) or Vb_block.shape != (nb, L, self.p):
            raise ValueError(f"{who}: blocks must be ({self.nb}, L, {self.r}) and "
                             f"({self.nb}, L, {self.p}), got {tuple(Psi_block.shape)} and "
                             f"{tuple(Vb_block.shape)}")
        if L == 0:
            return
        G = _hip.pool(Psi_block, Vb_block, 0, L, 1)            # one profile: the whole block
        self._S[self._cur].add_(G[:, 0])
        self.i += L

    def step(self, Phi_t, Psi_t, Vb_t, *, out=None):
        """One token.  ``Phi_t, Psi_t: (nb, r)``, ``Vb_t: (nb, p)``; returns fp32 ``(nb, p-1)``."""
        S_in, S_out = self._S[self._cur], self._S[1 - self._cur]
        o = _hip.decode_step(Phi_t, Psi_t, Vb_t, S_in, S_out, self.U, self.i, out=out)
        self._cur = 1 - self._cur
        self.i += 1
        return o

    def cache_words(self) -> int:
        return int(self.S.numel() + self.U.numel())

    @staticmethod
    def kv_cache_words(nb: int, T: int, d_v: int) -> int:
        return int(nb * 2 * T * d_v)
