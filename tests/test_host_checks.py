"""Host-side argument checks of the kernel wrappers and of the C ABI, CPU only.

The kernels trust the sizes and dtypes they are given (a short buffer would be
read past its end), so every wrapper validates them before it calls into the
library.  These tests run the wrappers on CPU tensors with the device check
switched off and the library call replaced by a recorder: a bad argument must
raise before anything is launched.
"""
import pytest
import torch

from smat_attention_amd.kernels import _lib
from smat_attention_amd.kernels import hip_fwd as K


@pytest.fixture
def no_device(monkeypatch):
    """Skip the GPU-residency check and record library calls instead of making them."""
    calls = []
    monkeypatch.setattr(K, "_on_gpu", lambda who, *ts: None)
    monkeypatch.setattr(K, "call", lambda name, *args: calls.append((name, args)) or 0)
    monkeypatch.setattr(K, "stream_of", lambda t: 0)
    return calls


def _decode_args(nb=4, r=8, p=9, B=3, dt=torch.float32):
    return dict(Phi_t=torch.rand(nb, r, dtype=dt), Psi_t=torch.rand(nb, r, dtype=dt),
                Vb_t=torch.rand(nb, p, dtype=dt), S_in=torch.zeros(nb, r, p),
                S_out=torch.zeros(nb, r, p), U=torch.zeros(nb, B, r, p), step=0)


def test_decode_step_checks_shapes(no_device):
    a = _decode_args()
    K.decode_step(**a)
    assert no_device and no_device[-1][0] == "smat_decode_step"
    for name, bad in (("Psi_t", torch.rand(4, 7)), ("Vb_t", torch.rand(4, 10)),
                      ("S_in", torch.zeros(4, 8, 8)), ("U", torch.zeros(3, 3, 8, 9)),
                      ("S_out", torch.zeros(4, 9, 9))):
        b = dict(a, **{name: bad})
        with pytest.raises(ValueError, match=name):
            K.decode_step(**b)
    with pytest.raises(ValueError, match="distinct"):
        K.decode_step(**dict(a, S_out=a["S_in"]))


def test_decode_step_mixed_dtypes_compute_in_fp32(no_device):
    """Mixed feature dtypes are taken to fp32 as the reference takes every input
    to its accumulation dtype; the kernel is then told fp32 and reads fp32 rows."""
    a = _decode_args()
    a["Psi_t"] = a["Psi_t"].bfloat16()
    a["Vb_t"] = a["Vb_t"].half()
    K.decode_step(**a)
    name, args = no_device[-1]
    assert name == "smat_decode_step" and args[0] == _lib.SMAT_F32


def test_wrappers_reject_mismatched_dtypes_and_shapes(no_device):
    Psi = torch.rand(2, 256, 8, dtype=torch.bfloat16)
    Vb = torch.rand(2, 256, 9, dtype=torch.bfloat16)
    with pytest.raises(TypeError, match="Vb"):
        K.chunk_states(Psi, Vb.float(), 128)
    with pytest.raises(ValueError, match="Vb"):
        K.chunk_states(Psi, Vb[:, :128], 128)
    with pytest.raises(TypeError, match="Vb"):
        K.pool(Psi, Vb.half(), 0, 128, 4)
    K.chunk_states(Psi, Vb, 128)
    # the query's U must match Phi_rec's batch and rank
    Phi = torch.rand(2, 100, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="U"):
        K.query(Phi, torch.zeros(2, 5, 7, 9))
    with pytest.raises(ValueError, match="U"):
        K.query(Phi, torch.zeros(3, 5, 8, 9))
    K.query(Phi, torch.zeros(2, 5, 8, 9))
    with pytest.raises(ValueError, match="Y"):
        K.causal_scan(Phi, Phi, torch.rand(2, 100, 9, dtype=torch.bfloat16), 64, 64,
                      Y=torch.zeros(2, 30, 9))
    with pytest.raises(ValueError, match="Sin"):
        K.chunk_local(torch.rand(1, 2, 64, 8), torch.rand(1, 2, 64, 8), torch.rand(1, 2, 64, 9),
                      torch.zeros(1, 2, 8, 8))


def test_forward_reuses_an_unaligned_workspace_only_if_it_fits(no_device, monkeypatch):
    """A workspace of exactly the queried size whose base is not 256-byte aligned
    has less room after alignment: forward() allocates instead of passing a
    short region to the library."""
    need = 4096
    monkeypatch.setattr(K, "forward_workspace_bytes", lambda *a: need)
    Phi = torch.rand(1, 256, 8, dtype=torch.bfloat16)
    Vb = torch.rand(1, 256, 9, dtype=torch.bfloat16)
    big = torch.empty(need + 512, dtype=torch.uint8)
    off = (-big.data_ptr()) % 256 + 16            # a base 16 bytes past a 256-byte boundary
    exact = big[off:off + need]
    assert exact.data_ptr() % 256 == 16
    K.forward(Phi, Phi, Vb, None, 1, n=128, n_P=0, N0=4, B=4, chunk=128, workspace=exact)
    args = no_device[-1][1]
    base, avail = args[-3], args[-2]
    assert avail >= need and base % 256 == 0
    assert not (exact.data_ptr() <= base < exact.data_ptr() + need)   # a fresh buffer
    roomy = big[off:]
    K.forward(Phi, Phi, Vb, None, 1, n=128, n_P=0, N0=4, B=4, chunk=128, workspace=roomy)
    base, avail = no_device[-1][1][-3], no_device[-1][1][-2]
    assert roomy.data_ptr() <= base < roomy.data_ptr() + roomy.numel() and avail >= need


def test_variant_hook_is_explicit_and_restored():
    """Kernel variants are chosen through smat_set_variant only (no environment
    variable is read); the context manager restores the previous choice."""
    lib = _lib.load()
    assert lib.smat_set_variant(0, 0) == 0
    with _lib.general_kernel("scan"):
        assert lib.smat_set_variant(0, 1) == 1
    assert lib.smat_set_variant(0, 0) == 0
    assert lib.smat_set_variant(99, 1) == -1          # SMAT_EINVAL
    assert lib.smat_set_variant(1, 7) == -1
    assert lib.smat_set_variant(1, 0) == 0            # a good call clears the message
    assert lib.smat_last_error() == b""


# ---------------------------------------------------------------------------
# the bound of the 8-element tile loaders (smat_common.hpp tile8_load)
# ---------------------------------------------------------------------------

def _tile8_reads(ncols, stride, elem, rows):
    """Byte ranges a VEC tile loader reads for a matrix of ``rows`` rows: every
    8-element group starting at a multiple of 8 below ``ncols`` is read whole
    (one 8*elem-byte load at row * stride + c0)."""
    for row in range(rows):
        for c0 in range(0, ncols, 8):
            start = (row * stride + c0) * elem
            yield start, start + 8 * elem


def _vec8_ok(stride, batch_stride):
    """The dispatch predicate the kernels use (rows_vec8_ok, 16-byte aligned base)."""
    return stride % 8 == 0 and batch_stride % 8 == 0


@pytest.mark.parametrize("elem", [2, 4])
@pytest.mark.parametrize("ncols", [33, 65, 129, 64, 128, 17])
def test_vector_tile_reads_stay_in_the_allocation(elem, ncols):
    """Every stride the list operands and feature rows use (packed, padded to 4
    and to 8 elements): when the dispatch takes the vector path, no read ends
    past rows * stride elements, the extent of the matrix."""
    rows = 5
    for stride in sorted({ncols, -(-ncols // 4) * 4, -(-ncols // 8) * 8}):
        if _vec8_ok(stride, stride * rows):
            extent = rows * stride * elem
            assert max(end for _, end in _tile8_reads(ncols, stride, elem, rows)) <= extent


@pytest.mark.parametrize("ncols,stride", [(33, 36), (65, 68), (129, 132)])
def test_fp32_rows_padded_to_4_floats_take_the_element_path(ncols, stride):
    """fp32 rows padded to 4 floats are 16-byte aligned, which the former
    predicate (16-byte groups) accepted, yet the last 8-float group of the
    last row reads 16 bytes past the matrix.  The 8-element predicate turns
    them away."""
    rows = 5
    over = max(end for _, end in _tile8_reads(ncols, stride, 4, rows)) - rows * stride * 4
    assert over == 16
    assert stride % 4 == 0 and not _vec8_ok(stride, stride * rows)


# ---------------------------------------------------------------------------
# the line-group incidence kernel's LDS addresses (incidence.hip, d = 3)
# ---------------------------------------------------------------------------
# The functions below restate the kernel's own integer arithmetic step by step
# (LgDiv, LgSlot, LgGroup, the row parts ot[] and the lane parts vb), so a
# change to that arithmetic must be mirrored here to keep the checks honest.

_KCW, _KPLANE, _KPF, _KTHREADS, _KPLANES, _KWAVES = 56, 2304, 7, 1024, 4, 16
_WAVE_Q = (2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37, 41)
_U32 = 1 << 32


def _lgdiv(q, xmax):
    """(M, S) of LgDiv<q, xmax>: the smallest S with M = ceil(2^S / q) exact on
    [0, xmax), and x M below 2^32 there (the 24-bit multiply where below 2^24)."""
    S = 1
    while True:
        M = ((1 << S) + q - 1) // q
        if all((x * M) >> S == x // q for x in range(xmax)):
            assert xmax * M < _U32
            return M, S
        S += 1


def _wave_staging(q):
    """Entries the staging writes, {entry index: point}: slot
    ps = 16 (wave + 16 u) + (tid & 15) of plane kx = (tid >> 4) & 3, x1 = ps / q
    by LgSlot's multiply-shift, copies at x0 + c q below q + 15; and every F
    byte offset a prefetch reads, in units of 16 bytes at rp = 4."""
    N0 = q * q
    M, S = _lgdiv(q, 16 * _KWAVES * _KPF)
    panel = {}
    for tid in range(_KTHREADS):
        kx = (tid >> 4) & 3
        for u in range(_KPF):
            ps = 16 * ((tid >> 6) + 16 * u) + (tid & 15)
            x1 = (ps * M) >> S
            x0 = ps - q * x1
            if ps >= N0:
                continue
            assert (x1, x0) == divmod(ps, q)
            for c in range((q + 15 + q - 1) // q):
                if x0 + c * q < q + 15:
                    e = kx * _KPLANE + _KCW * x1 + x0 + c * q
                    assert e not in panel
                    panel[e] = x0 * q + x1
    return panel


def _group(q, g, P=None):
    """LgGroup<q, P>(g): (b0, s0, qm, d16, lcb, nvalid, sloped)."""
    P = (q + 15) // 16 if P is None else P
    G = (q + 1) * P
    d = g // P
    b0 = (g - d * P) * 16
    sloped = d < q
    s0 = b0 if sloped else 0
    qm = q - d if sloped else 0
    return b0, s0, qm, (16 * qm) % q, ((d + 1) * q + b0) if sloped else b0, \
        (min(16, q - b0) if g < G else 0), sloped


def _wave_plan(q):
    """(P, G, NTG, R, NOL) of incidence_wave_kernel<q>: groups a direction, groups,
    group tasks (two groups each), and, past 16 lines a direction with fewer
    than ten after its last full group, those R lines a direction taken one a
    lane over all four planes (NOL of them)."""
    R = q % 16
    own = q > 16 and 0 < R < 10
    P = q // 16 if own else (q + 15) // 16
    G = (q + 1) * P
    return P, G, (G + 1) // 2, R, ((q + 1) * R if own else 0)


def _own_lane_reads(q, cw, P, R, NOL, plane_entries):
    """Yield (("own", li), 0, plane, t, entry, line code) for the lines of their
    own: own_lane's LrLane walk (entry c1 N + s_N, s advancing by qm modulo m,
    32-bit unsigned), m and c1 rebuilt from qm (zero only for vertical lines)
    as the kernel does; the lanes of the last task past NOL included."""
    for li in range(((NOL + 63) // 64) * 64):
        valid = li < NOL
        d = li // R if valid else 0
        b = 16 * P + (li - d * R if valid else 0)
        sl = d < q
        s16 = 16 * (b if sl else cw * b)
        qm16 = 16 * (q - d) if sl else 0
        m16 = 16 * q if qm16 else 0x80000000
        c16 = 16 * cw if qm16 else 16
        code = ((d + 1) * q + b if sl else b) if valid else None
        for t in range(q):
            addr = c16 * t + s16
            assert addr % 16 == 0 and c16 * t < (1 << 24)
            for plane in range(len(plane_entries)):
                yield ("own", li), 0, plane, t, addr // 16 + plane_entries[plane], code
            c = (s16 + qm16) % _U32
            s16 = min(c, (c - m16) % _U32)


def _wave_reads(q):
    """Yield (group, lane j, plane, pp, step, entry, line code) for every read the
    kernel makes, by its own arithmetic: rows 0, 1 of a wave task take group
    2 task (plane pairs (0, 1), (2, 3)), rows 2, 3 group 2 task + 1; a row's lane
    l computes ot[run] for step 16 run + l, and step t takes lane t % 16's value
    of its own row.  The lines of their own (_own_lane_reads) come first, with
    pp = None."""
    P, G, NTG, R, NOL = _wave_plan(q)
    NR = (q + 15) // 16
    M, S = _lgdiv(q, 16 * ((q + 15) // 16) + 16 * q)
    planes = [k * _KPLANE for k in range(_KPLANES)]
    for grp, j, plane, t, e, lc in _own_lane_reads(q, _KCW, P, R, NOL, planes):
        yield grp, j, plane, None, t, e, lc
    for task in range(NTG):
        for gsel in range(2):
            grp = 2 * task + gsel
            b0, s0, qm, d16, lcb, nvalid, sloped = _group(q, grp, P)
            ot = {}
            for l in range(16):
                x = s0 + qm * l
                s = x - q * ((x * M) >> S)
                assert s == x % q
                for r in range(NR):
                    ot[r, l] = (256 * _KCW * r + 16 * _KCW * l if sloped else 256 * r + 16 * l) \
                        + 16 * s
                    c = (s + d16) % _U32
                    s = min(c, (c - q) % _U32)
            for pp in range(2):
                for j in range(16):
                    valid = j < nvalid
                    bl = b0 + j
                    col = bl if valid else (bl - 16 if bl >= 16 else 0)
                    vb = 16 * 2 * pp * _KPLANE + 16 * j + (0 if sloped else 16 * _KCW * col)
                    lc = min(lcb + j, q * (q + 1) - 1)
                    for t in range(q):
                        addr = vb + ot[t // 16, t % 16]
                        assert addr % 16 == 0
                        for half in range(2):
                            yield (grp, j, 2 * pp + half, pp, t,
                                   (addr + half * 16 * _KPLANE) // 16, lc if valid else None)


@pytest.mark.parametrize("q", _WAVE_Q)
def test_line_group_incidence_reads_each_line_once_in_bounds(q):
    """Emulates the line-group kernel for every field size it is compiled for:
    every read lands on a staged entry inside the four planes (the line table
    starts at 4 kPlane entries), each stored line reads exactly its q points
    once per plane -- the sloped line (m, b) the points (b - m t mod q, t), the
    vertical line b the column x1 = b -- and stores under its own line code."""
    panel = _wave_staging(q)
    assert max(panel) < _KPLANES * _KPLANE
    P, G, NTG, R, NOL = _wave_plan(q)
    # the lines of their own sit in one task slot of the waves (kOwnK)
    NT = NTG + (NOL + 63) // 64
    assert NOL == 0 or (NT - 1) // _KWAVES == NTG // _KWAVES
    got, codes = {}, {}
    for grp, j, plane, pp, t, e, lc in _wave_reads(q):
        assert 0 <= e < _KPLANES * _KPLANE and e in panel
        assert e // _KPLANE == plane
        got.setdefault((grp, j, plane), []).append(panel[e])
        codes[grp, j] = lc

    def want(dirn, b):
        if dirn < q:                                            # e = m + 1
            return sorted(((b - dirn * t) % q) * q + t for t in range(q)), (dirn + 1) * q + b
        return sorted(x0 * q + b for x0 in range(q)), b        # e = 0

    stored = {}
    for grp in range(G):
        dirn, part = divmod(grp, P)
        for j in range(16):
            b = part * 16 + j
            if b >= q:
                assert codes[grp, j] is None
                continue
            pts, code = want(dirn, b)
            assert codes[grp, j] == code
            for plane in range(_KPLANES):
                assert sorted(got[grp, j, plane]) == pts
            stored[code] = stored.get(code, 0) + 1
    for li in range(((NOL + 63) // 64) * 64):
        if li >= NOL:
            assert codes[("own", li), 0] is None
            continue
        dirn, k = divmod(li, R)
        pts, code = want(dirn, 16 * P + k)
        assert codes[("own", li), 0] == code
        for plane in range(_KPLANES):
            assert sorted(got[("own", li), 0, plane]) == pts
        stored[code] = stored.get(code, 0) + 1
    # every line of the plane stored exactly once
    assert sorted(stored) == list(range(q * (q + 1))) and set(stored.values()) == {1}


@pytest.mark.parametrize("q", [17, 29, 37, 41])
def test_line_group_incidence_rows_read_one_bank_phase_each(q):
    """At every step the sixteen lanes of a row read sixteen distinct 16-byte
    phases (entry mod 16): consecutive entries for sloped lines, an odd stride
    for vertical ones; and the two rows of a 32-lane half (the plane pairs of one
    group) read at the same phases, the pattern ds_read_b128 serves at full rate."""
    rows = {}
    for grp, j, plane, pp, t, e, lc in _wave_reads(q):
        if pp is None:                                   # lines of their own
            continue
        rows.setdefault((grp, plane - 2 * pp, pp, t), {})[j] = e
    for (grp, half, pp, t), lanes in rows.items():
        assert sorted(e % 16 for e in lanes.values()) == list(range(16))
        other = rows[grp, half, 1 - pp, t]
        assert all((lanes[j] - other[j]) % 16 == 0 for j in range(16))


def test_line_group_incidence_half_exchange_stores_whole_lines():
    """After the exchange of 32-lane halves (v_permlane32_swap of (a0, a1) and of
    the line index) the first register holds group A's planes in rows 0-3 and
    the second group B's, each row at the plane it stores (splane = 0, 2, 1, 3):
    a line's four planes leave in one store instruction."""
    a0 = [("A", 0), ("A", 2), ("B", 0), ("B", 2)]        # (group, plane) by row
    a1 = [("A", 1), ("A", 3), ("B", 1), ("B", 3)]
    x = a0[:2] + a1[:2]                                  # (x_lo, y_lo)
    y = a0[2:] + a1[2:]                                  # (x_hi, y_hi)
    splane = [((row & 1) << 1) | (row >> 1) for row in range(4)]
    assert [p for _, p in x] == splane and [p for _, p in y] == splane
    assert {g for g, _ in x} == {"A"} and {g for g, _ in y} == {"B"}


# ---------------------------------------------------------------------------
# the row-group incidence kernel's LDS addresses (incidence.hip, d = 3, q > 41)
# ---------------------------------------------------------------------------
# Restates ir::Shape, LrSlot and the task loop of incidence_row_kernel: one
# plane an item, each row of a wave its own group (group 4 task + row).

_ROW_Q = (43, 47, 53, 59, 61, 67, 71, 73, 79, 83)


def _row_shape(q):
    """(kCW, kEntries, kLdsBytes) of ir::Shape<q>."""
    cw = (q + 15 + 1) // 2 * 2
    entries = (cw * q + 15) // 16 * 16
    return cw, entries, entries * 16 + ((q * (q + 1) * 2 + 15) // 16) * 16


def _row_staging(q):
    """{entry: point} the staging writes: slot ps = tid + 1024 u, x1 = ps / q by
    LrSlot's multiply-shift, copies at x0 + c q below q + 15."""
    cw, _, _ = _row_shape(q)
    M, S = _lgdiv(q, 64 * _KWAVES * _KPF)
    panel = {}
    for tid in range(_KTHREADS):
        for u in range(_KPF):
            ps = tid + 1024 * u
            x1 = ((ps * M) % _U32) >> S
            x0 = ps - q * x1
            if ps >= q * q:
                continue
            assert (x1, x0) == divmod(ps, q)
            for c in range((q + 15 + q - 1) // q):
                if x0 + c * q < q + 15:
                    e = cw * x1 + x0 + c * q
                    assert e not in panel
                    panel[e] = x0 * q + x1
    return panel


def _row_plan(q):
    """(P, G, NTG, R, NOL) of incidence_row_kernel<q>: groups a direction, groups,
    group tasks, and, when fewer than ten lines follow a direction's last full
    group, those R lines a direction taken one a lane (NOL of them)."""
    R = q % 16
    own = 0 < R < 10
    P = q // 16 if own else (q + 15) // 16
    G = (q + 1) * P
    return P, G, (G + 3) // 4, R, ((q + 1) * R if own else 0)


def _row_reads(q):
    """Yield (group, lane j, step, entry, line code) for every read of the
    row-group kernel: row k of group task n takes group 4 n + k; the lines of
    their own are yielded as group ("own", line index), lane 0."""
    cw, _, _ = _row_shape(q)
    P, G, NTG, R, NOL = _row_plan(q)
    NR = (q + 15) // 16
    M, S = _lgdiv(q, 16 * ((q + 15) // 16) + 16 * q)
    for grp, j, _, t, e, lc in _own_lane_reads(q, cw, P, R, NOL, [0]):
        yield grp, j, t, e, lc
    for task in range(NTG):
        for row in range(4):
            grp = 4 * task + row
            b0, s0, qm, d16, lcb, nvalid, sloped = _group(q, grp, P)
            ot = {}
            for l in range(16):
                x = s0 + qm * l
                s = x - q * ((x * M) >> S)
                assert s == x % q
                for r in range(NR):
                    ot[r, l] = (256 * cw * r + 16 * cw * l if sloped else 256 * r + 16 * l) \
                        + 16 * s
                    c = (s + d16) % _U32
                    s = min(c, (c - q) % _U32)
            for j in range(16):
                valid = j < nvalid
                bl = b0 + j
                col = bl if valid else (bl - 16 if bl >= 16 else 0)
                vb = 16 * j + (0 if sloped else 16 * cw * col)
                lc = min(lcb + j, q * (q + 1) - 1)
                for t in range(q):
                    addr = vb + ot[t // 16, t % 16]
                    assert addr % 16 == 0
                    yield grp, j, t, addr // 16, (lc if valid else None)


@pytest.mark.parametrize("q", _ROW_Q)
def test_row_group_incidence_reads_each_line_once_in_bounds(q):
    """Emulates the row-group kernel for every field size it is compiled for:
    the panel and line table fit the 160 KB LDS, every read lands on a staged
    entry below the line table, each stored line reads exactly its q points once
    and stores under its own line code."""
    cw, entries, lds = _row_shape(q)
    assert lds <= 160 * 1024 and q * q <= _KPF * _KTHREADS
    panel = _row_staging(q)
    assert len(panel) == q * (q + 15) and max(panel) < entries
    P, G, NTG, R, NOL = _row_plan(q)
    got, codes, phases = {}, {}, {}
    for grp, j, t, e, lc in _row_reads(q):
        assert 0 <= e < entries and e in panel
        got.setdefault((grp, j), []).append(panel[e])
        codes[grp, j] = lc
        if not isinstance(grp, tuple):
            phases.setdefault((grp, t), set()).add(e % 16)
    assert all(len(v) == 16 for v in phases.values())   # one bank phase a group row

    def want(dirn, b):
        if dirn < q:
            return sorted(((b - dirn * t) % q) * q + t for t in range(q)), (dirn + 1) * q + b
        return sorted(x0 * q + b for x0 in range(q)), b

    stored = {}
    for grp in range(G):
        dirn, part = divmod(grp, P)
        for j in range(16):
            b = part * 16 + j
            if b >= q:
                assert codes[grp, j] is None
                continue
            pts, code = want(dirn, b)
            assert codes[grp, j] == code and sorted(got[grp, j]) == pts
            stored[code] = stored.get(code, 0) + 1
    for li in range(((NOL + 63) // 64) * 64):
        if li >= NOL:
            assert codes[("own", li), 0] is None
            continue
        dirn, k = divmod(li, R)
        pts, code = want(dirn, 16 * P + k)
        assert codes[("own", li), 0] == code and sorted(got[("own", li), 0]) == pts
        stored[code] = stored.get(code, 0) + 1
    # every line of the plane stored exactly once
    assert sorted(stored) == list(range(q * (q + 1))) and set(stored.values()) == {1}
