"""Host geometry: the product's build_mask against the reference's own outputs,
the closed forms, and a loop-based rebuild from the definitions.

Ports tests/test_smat.py:43-173 (structure, block layout, planted identity,
counting) and adds the bit-exact index checks the reference's tests do not
make (golden C_indices from the reference's build_mask)."""
import hashlib

import numpy as np
import pytest

from oracle import mask_ref
from smat_attention_amd.mask import (build_mask, d_max_geometric, estimate_cost,
                                     incidence_audit, materialise, next_prime,
                                     planted_hyperplane_normals, shatter_witness)


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# --------------------------------------------------------------------------
# bit-exact against the reference's build_mask
# --------------------------------------------------------------------------

def test_golden_indices_bit_exact(golden, golden_arrays):
    for c in golden:
        s = build_mask(c["T"], c["d"], chunk=c["chunk"], n_P=c["n_P"])
        assert s.kind == c["kind"], c["key"]
        for k in ("n", "T_R", "q", "dim", "N0", "n_dirs", "B", "n_planted", "k",
                  "uniform_deg", "nnz", "I_tok"):
            got = s.I_prof if k == "nnz" else getattr(s, k)
            assert got == c[k], (c["key"], k, got, c[k])
        assert [int(x) for x in s.planted_cols] == c["planted_cols"], c["key"]
        assert _sha(s.C_indices.astype(np.int32)) == c["C_indices_sha256"], c["key"]
        assert _sha(s.C_indptr.astype(np.int64)) == c["C_indptr_sha256"], c["key"]
        if c["key"] in golden_arrays:
            np.testing.assert_array_equal(s.C_indices, golden_arrays[c["key"]])


def test_published_rows_scalars(ref_tables):
    """Every (T, d) row of the published sweeps and the counting table."""
    for table in ("prefill_h200", "prefill_a100", "theory_counting"):
        for row in ref_tables[table]:
            try:
                s = build_mask(row["T"], row["d"], chunk=row["chunk"], _probe=True)
            except ValueError:
                # the probe refuses T_R < 2B (those rows were built with a
                # warning); check the oracle's closed forms instead
                n = row["chunk"] * (row["T"] // (2 * row["chunk"]))
                q = mask_ref.field_size(n, row["d"])
                dim = row["d"] - 1
                assert q == row["q"] and q ** dim == row["N0"], row
                assert row["B"] == q * (q ** dim - 1) // (q - 1), row
                assert row["deg"] == q ** (dim - 1) and row["I_prof"] == row["B"] * row["deg"]
                continue
            assert s.q == row["q"] and s.B == row["B"] and s.N0 == row["N0"], row
            assert s.uniform_deg == row["deg"], row
            assert s.B * s.uniform_deg == row["I_prof"], row
            if "n" in row:
                assert s.n == row["n"] and s.T_R == row["T_R"], row
            # I_tok = sum_j nu(prof(j)) = n_X * D for the full family (closed form)
            D = (s.q ** s.dim - 1) // (s.q - 1) if s.d >= 2 else 1
            assert (s.n - s.n_P) * D == row["I_tok"], row


def test_theory_structure_checksums(ref_tables):
    """nnz and density of the materialised mask (results/theory_structure.csv)."""
    for row in ref_tables["theory_structure"]:
        s = build_mask(row["T"], row["d"], chunk=row["chunk"])
        M = materialise(s, np.int8)
        assert (s.n, s.T_R, s.q, s.B, s.N0) == (row["n"], row["T_R"], row["q"],
                                                row["B"], row["N0"]), row
        assert int(M.sum(dtype=np.int64)) == row["nnz"], row
        assert abs(M.sum(dtype=np.int64) / row["T"] ** 2 - row["density"]) < 1e-12


# --------------------------------------------------------------------------
# against the loop-based rebuild from the definitions
# --------------------------------------------------------------------------

@pytest.mark.parametrize("T,d,chunk,n_P", [
    (512, 2, 64, 0), (1024, 3, 64, 0), (2048, 3, 64, 16), (2048, 4, 64, 0),
    (1024, 2, 128, 0), (4096, 3, 128, 0), (8192, 4, 128, 0)])
def test_incidence_matches_definition(T, d, chunk, n_P):
    s = build_mask(T, d, chunk=chunk, n_P=n_P)
    geo = mask_ref.geometry(T, d, chunk=chunk, n_P=n_P)
    assert (s.q, s.N0, s.B, s.uniform_deg) == (geo["q"], geo["N0"], geo["B"], geo["deg"])
    rows = s.C_indices.reshape(s.B, s.uniform_deg)
    assert [list(map(int, r)) for r in rows] == geo["rows"]
    assert list(map(int, s.planted_cols)) == geo["planted_cols"]


@pytest.mark.parametrize("T,d,chunk,n_P,endpoint", [
    (256, 1, 64, 0, False), (512, 2, 64, 0, False), (512, 3, 64, 0, False),
    (640, 3, 64, 16, False), (256, 8, 8, 0, True), (300, 8, 8, 0, True)])
def test_dense_mask_matches_definition(T, d, chunk, n_P, endpoint):
    s = build_mask(T, d, chunk=chunk, n_P=n_P)
    geo = (mask_ref.endpoint_geometry(T, d) if endpoint
           else mask_ref.geometry(T, d, chunk=chunk, n_P=n_P))
    if endpoint:
        assert s.kind == "endpoint"
        assert [list(map(int, s.C_indices[s.C_indptr[h]:s.C_indptr[h + 1]]))
                for h in range(s.B)] == geo["rows"]
    M = materialise(s, np.int8)
    ref = np.array(mask_ref.dense_mask(T, geo, endpoint=endpoint), dtype=np.int8)
    np.testing.assert_array_equal(M, ref)


# --------------------------------------------------------------------------
# structure (test_smat.py:43-89)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("T,d", [(256, 1), (512, 2), (1024, 2), (1024, 3),
                                 (2048, 3), (2048, 4)])
def test_structure(T, d):
    s = build_mask(T, d, chunk=64)
    M = materialise(s)
    L = np.tril(np.ones((T, T)))
    assert np.all(np.triu(M, 1) == 0)
    assert np.all(np.diag(M) == 1)
    assert np.all((M == 0) | (M == 1))
    assert np.all(M <= L)
    floor = (s.n * (s.n + 1) + s.T_R * (s.T_R + 1)) / 2
    assert M.sum() >= floor


@pytest.mark.parametrize("T", [256, 512, 1000])
def test_d1_is_causal_triangle(T):
    s = build_mask(T, 1, chunk=64)
    np.testing.assert_array_equal(materialise(s), np.tril(np.ones((T, T))))


def test_landmark_rows_see_their_prefix():
    s = build_mask(1024, 3, chunk=64)
    M = materialise(s)
    np.testing.assert_array_equal(M[:s.n, :s.n].sum(1), np.arange(1, s.n + 1))


def test_range_checks():
    with pytest.raises(ValueError):
        build_mask(1024, 11, chunk=64)
    with pytest.raises(ValueError):
        build_mask(4, 1)
    assert build_mask(1024, 10, chunk=64).kind == "endpoint"
    for T in (4096, 65536):
        assert d_max_geometric(T, chunk=128) < T.bit_length() - 1
    with pytest.raises(MemoryError):
        build_mask(65536, 4, chunk=128, max_I_prof=1000)


def test_q_uses_double_precision_pow():
    # 32768 ** (1/3) = 31.999999999999996 in IEEE double; ceil gives 32
    assert float(32768) ** (1.0 / 3) < 32
    s = build_mask(65536, 3, chunk=128)          # n = 32768
    assert s.q == 37 and next_prime(32) == 37
    # n = 29^3: a prime cube root must give q = 29 itself
    assert build_mask(2 * 24389, 3, chunk=1, _probe=True).q == 29


# --------------------------------------------------------------------------
# block layout, planted identity, counting (test_smat.py:92-173)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("T,d,nP", [(1024, 2, 0), (2048, 3, 0), (2048, 4, 0), (2048, 3, 16)])
def test_block_layout(T, d, nP):
    s = build_mask(T, d, chunk=64, n_P=nP)
    M = materialise(s)
    n, T_R = s.n, s.T_R
    np.testing.assert_array_equal(M[:n, :n], np.tril(np.ones((n, n))))
    assert np.all(M[:n, n:] == 0)
    np.testing.assert_array_equal(M[n:, n:], np.tril(np.ones((T_R, T_R))))
    if nP:
        assert np.all(M[n:, :nP] == 1)
    C = s.dense_C()
    prof = s.prof_of_column()
    R = np.zeros((T_R, s.B))
    R[np.arange(T_R), np.arange(T_R) % s.B] = 1
    S = np.zeros((s.n_X, s.N0))
    S[np.arange(s.n_X), prof] = 1
    np.testing.assert_array_equal(M[n:, s.n_P:n], R @ C @ S.T)


@pytest.mark.parametrize("T,d", [(1024, 2), (2048, 3), (4096, 4), (16384, 5)])
def test_planted(T, d):
    s = build_mask(T, d, chunk=64)
    a = incidence_audit(s)
    assert a["planted_identity"] and a["B_ge_2_pow_d_minus_1"]
    hs = planted_hyperplane_normals(d)
    assert all(np.any(a_ != 0) for a_, _ in hs)
    assert len({(tuple(a_), b) for a_, b in hs}) == len(hs)
    cols, ok, _ = shatter_witness(s)
    assert ok and len(cols) == d


@pytest.mark.parametrize("T,d", [(4096, 2), (16384, 2), (4096, 3), (16384, 3),
                                 (65536, 3), (16384, 4), (65536, 4)])
def test_incidence_audit(T, d):
    s = build_mask(T, d, chunk=128)
    a = incidence_audit(s)
    assert a["exact"] and a["nu_is_D"] and a["full_hyperplane_family"]
    # every member satisfies its hyperplane equation: rebuild <a_e, x> = b from
    # the planted normals for the first 2^(d-1) rows
    q, dim = s.q, s.dim
    rows = s.C_indices.reshape(s.B, -1)
    for R, (avec, b) in enumerate(planted_hyperplane_normals(d)):
        pts = np.array([mask_ref.point(int(x), q, dim) for x in rows[R]])
        assert np.all((pts @ avec) % q == b)


@pytest.mark.parametrize("d", [2, 3, 4, 5])
def test_closed_forms(d):
    for T in [2 ** k for k in range(14, 20)]:
        s = build_mask(T, d, chunk=128, _probe=True)
        q = s.q
        assert s.B * s.uniform_deg == q ** (d - 1) * (q ** (d - 1) - 1) // (q - 1)
        assert s.B == q * (q ** (d - 1) - 1) // (q - 1)
        assert s.N0 == q ** (d - 1)


def test_endpoint_walsh_rows():
    s = build_mask(1024, 10, chunk=64)
    a = np.arange(s.N0)
    Cw = (np.bitwise_count(a[:, None] & a[None, :]) % 2) == 0
    np.testing.assert_array_equal(s.dense_C().astype(bool), Cw)
    assert s.uniform_deg == 0 and incidence_audit(s)["exact"]


def test_estimate_cost():
    e = estimate_cost(131072, 3, 128, 128)
    assert e["feasible"] and e["I_prof"] == 70602 and e["B"] == 1722
    assert not estimate_cost(64, 5, 8, 8)["feasible"]


def test_parity_interleaved_table_keeps_rows_and_alternates():
    """The kernel-side table reorders points within each row only, even-first on
    even rows and odd-first on odd rows."""
    from smat_attention_amd.attention import parity_interleaved_table
    spec = build_mask(131072, 3, chunk=128)
    par = parity_interleaved_table(spec).reshape(spec.B, spec.uniform_deg)
    ref = spec.C_indices.reshape(spec.B, spec.uniform_deg)
    assert np.array_equal(np.sort(par, axis=1), np.sort(ref, axis=1))
    for h in (0, 1, 2, 3, 1721):
        row = par[h]
        first = h & 1
        par_bits = row & 1
        n_first = int((par_bits == first).sum())
        assert np.all(par_bits[:n_first] == first) and np.all(par_bits[n_first:] != first)
        assert np.all(np.diff(row[:n_first]) > 0) and np.all(np.diff(row[n_first:]) > 0)


@pytest.mark.parametrize("T", [2048, 4096, 32768, 131072, 524288, 69632])
def test_plane_line_codes_regenerate_every_row(T):
    """d = 3: each row of C is the line named by its code (checked set-wise
    inside plane_line_codes; here also against the loop-built oracle rows)."""
    from smat_attention_amd.attention import plane_line_codes
    spec = build_mask(T, 3, chunk=128)
    code = plane_line_codes(spec)
    assert code is not None and code.shape == (spec.B,)
    q = spec.q
    e, b = code // q, code % q
    if T <= 4096:
        geo = mask_ref.geometry(T, 3, chunk=128)
        for h in range(spec.B):
            if e[h] == 0:
                pts = {x0 * q + int(b[h]) for x0 in range(q)}
            else:
                m = int(e[h]) - 1
                pts = {((int(b[h]) - m * x1) % q) * q + x1 for x1 in range(q)}
            assert pts == set(geo["rows"][h])


def test_plane_line_codes_absent_for_other_masks():
    from smat_attention_amd.attention import plane_line_codes
    assert plane_line_codes(build_mask(4096, 2, chunk=128)) is None
    assert plane_line_codes(build_mask(8192, 4, chunk=128)) is None


# --------------------------------------------------------------------------
# the audit's own checks catch planted mistakes; witness and cost model
# --------------------------------------------------------------------------

@pytest.mark.parametrize("T,d", [(4096, 3), (16384, 4)])
def test_audit_catches_a_moved_point(T, d):
    """Each row must satisfy its hyperplane's equation: moving one point of one
    row (a plausible off-by-one in the table) fails ``rows_on_hyperplanes``
    and ``exact`` even though degrees and counts are unchanged."""
    s = build_mask(T, d, chunk=128)
    a = incidence_audit(s)
    assert a["rows_on_hyperplanes"] and a["exact"] and a["planted_identity"]
    rows = s.C_indices.reshape(s.B, -1).copy()
    h = s.B // 2
    row = set(int(x) for x in rows[h])
    outsider = next(x for x in range(s.N0) if x not in row)
    rows[h, -1] = outsider
    rows[h] = np.sort(rows[h])
    bad = build_mask(T, d, chunk=128)
    bad.C_indices = rows.reshape(-1)
    b = incidence_audit(bad)
    assert not b["rows_on_hyperplanes"] and not b["exact"]


def test_audit_catches_a_wrong_planted_order():
    s = build_mask(4096, 3, chunk=128)
    rows = s.C_indices.reshape(s.B, -1).copy()
    rows[[0, 1]] = rows[[1, 0]]                  # swap the first two row types
    s.C_indices = rows.reshape(-1)
    s.plane_ids = s.plane_ids[[1, 0] + list(range(2, s.B))]
    a = incidence_audit(s)
    assert a["rows_on_hyperplanes"] and not a["planted_identity"] and not a["exact"]


@pytest.mark.parametrize("T", [512, 1024, 1000])
def test_endpoint_audit_and_witness(T):
    """Endpoint masks: the Walsh rows, and the witness at T = 2^m where the
    recent block holds exactly B rows (the first recent column suffices)."""
    s = build_mask(T, T.bit_length() - 1, chunk=8)
    a = incidence_audit(s)
    assert s.kind == "endpoint" and a["walsh_rows"] and a["exact"]
    cols, ok, rows = shatter_witness(s)
    assert ok and len(cols) == s.d
    M = materialise(s, np.int8)
    for pat, found in rows.items():
        kind, i = found
        r = i if kind == "zeta" else s.n + i
        assert [bool(M[r, c]) for c in cols] == [bool((pat >> j) & 1) for j in range(len(cols))]


@pytest.mark.parametrize("T,d", [(2048, 3), (4096, 4), (2048, 2)])
def test_geometric_witness_rows_realise_their_patterns(T, d):
    s = build_mask(T, d, chunk=64)
    cols, ok, rows = shatter_witness(s)
    assert ok
    M = materialise(s, np.int8)
    for (R, bit), i in rows.items():
        got = [bool(M[s.n + i, c]) for c in cols]
        assert got == [bool((R >> l) & 1) for l in range(s.dim)] + [bool(bit)]


def test_cost_model_counts():
    """Useful MFMA work of the long prefill at T = 131072, d = 3, r = p - 1 = 128:
    1.386e11 FLOP over 8 heads; the incidence's adds are nnz(C) r p; the
    endpoint nnz counts row 0 whole and every other Walsh row half."""
    e = estimate_cost(131072, 3, 128, 128)
    assert abs(8 * e["mfma_flops"] - 1.3865e11) / 1.3865e11 < 1e-3
    assert e["incidence_adds"] == 70602 * 128 * 129
    assert e["macs"] == sum(e[k] for k in ("macs_intra", "macs_states", "macs_pool",
                                           "macs_query"))
    s = build_mask(1024, 10, chunk=64)
    assert estimate_cost(1024, 10, 8, 8)["I_prof"] == s.I_prof
    assert estimate_cost(4096, 3, 8, 8)["I_prof"] == build_mask(4096, 3, chunk=128).I_prof


def test_plane_ids_name_the_row_types():
    """plane_ids[h] = e*q + b of row type h: the planted ones first."""
    s = build_mask(131072, 3, chunk=128)
    assert s.plane_ids.shape == (s.B,)
    assert len(np.unique(s.plane_ids)) == s.B
    rest = s.plane_ids[s.n_planted:]
    assert np.all(np.diff(rest) > 0)


@pytest.mark.parametrize("T", [4096, 131072])
def test_line_codes_recorded_equal_recovered(T):
    """The line codes taken from build_mask's plane_ids equal those recovered
    from the rows alone (the path a mask built elsewhere takes)."""
    from smat_attention_amd.attention import plane_line_codes
    spec = build_mask(T, 3, chunk=128)
    recorded = plane_line_codes(spec)
    spec.plane_ids = None
    recovered = plane_line_codes(spec)
    assert recorded is not None and np.array_equal(recorded, recovered)
