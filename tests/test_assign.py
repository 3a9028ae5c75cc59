"""Content-addressed assignment (src/smat/assign.py): the oracle against the
reference's own fixtures, the module's parameters, and (on the GPU) the HIP
path against both."""
import os

import numpy as np
import pytest
import torch

from oracle import assign_ref as R
from smat_attention_amd.mask import build_mask

GOLD = os.path.join(os.path.dirname(__file__), "golden", "assign_golden.npz")
# hard dense reads (anneal 1) and the pair reads: the soft phase of the dense
# read, the sparse_ops path at anneal 1 (one cell per token) and below (2^dim)
HARD_CASES = ["T512_d3_point", "T512_d3_plane", "T512_d2_point"]
PAIR_CASES = ["T512_d3_point_soft", "T512_d3_point_sparse", "T512_d3_point_sparse_soft",
              "T512_d3_plane_sparse", "T512_d3_plane_soft", "T512_d3_plane_dirsoft"]
CASES = HARD_CASES + PAIR_CASES


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


def _case(gold, name):
    g = {}
    for k in gold.files:
        if k.startswith(name + "/"):
            key = k.split("/", 1)[1]
            if key.endswith(".base"):      # an input stored once, under an earlier case
                key = key[:-5]
                g[key] = torch.from_numpy(gold[f"{gold[k]}/{key}"])
            else:
                g[key] = torch.from_numpy(gold[k])
    T, d, h, dm, nb, n, r, plane = [int(x) for x in g["meta"]]
    anneal, sparse, dir_soft = (float(x) for x in g["opts"])
    return g, dict(T=T, d=d, h=h, dm=dm, nb=nb, n=n, r=r, mode="plane" if plane else "point",
                   anneal=anneal, sparse=bool(sparse), dir_soft=bool(dir_soft))


def _module(meta, device="cpu"):
    from smat_attention_amd.assign import ContentAssign
    spec = build_mask(meta["T"], meta["d"], chunk=64)
    torch.manual_seed(1000)
    m = ContentAssign(meta["h"], meta["dm"], spec, mode=meta["mode"])
    m.anneal = meta["anneal"]
    m.sparse_ops = meta["sparse"]
    if meta["dir_soft"]:
        m.dir_soft = True
        m.train()
    return m.to(device), spec


def _plane_tables(spec):
    from smat_attention_amd.assign import grouped_planes
    _, grouped = grouped_planes(spec.q, spec.dim)
    M = torch.zeros(grouped.shape[0], grouped.shape[1], spec.N0)
    for e in range(grouped.shape[0]):
        for o in range(grouped.shape[1]):
            M[e, o, grouped[e, o]] = 1.0
    return M, M.argmax(1)


@pytest.mark.parametrize("name", HARD_CASES)
def test_oracle_reproduces_reference_fixtures(gold, name):
    g, meta = _case(gold, name)
    spec = build_mask(meta["T"], meta["d"], chunk=64)
    n, h = meta["n"], meta["h"]
    ck, sk = R.cells(g["u"][:, :n], g["W"], g["gamma"], g["b"], spec.q, spec.dim, h)
    ck = R.plant(ck, torch.as_tensor(spec.planted_cols, dtype=torch.long),
                 torch.tensor([spec.q ** (spec.dim - l) for l in range(1, spec.dim + 1)]))
    cq, _ = R.cells(g["u"][:, n:], g["W"], g["gamma"], g["b"], spec.q, spec.dim, h)
    assert torch.equal(ck, g["ck"]) and torch.equal(cq, g["cq"])
    M = _plane_tables(spec)[0] if meta["mode"] == "plane" else None
    y = R.dense_read(g["Phi"], g["Psi"], g["Vb"], n, ck, cq, spec.N0, mode=meta["mode"], M=M,
                     Wd=g.get("Wd"), u=g["u"], h=h)
    rel = (y - g["y"]).abs().max() / g["y"].abs().max()
    assert rel < 1e-5


@pytest.mark.parametrize("name", CASES)
def test_module_parameters_match_reference_init(gold, name):
    """Constructed after the same seed, the module holds the reference's values."""
    g, meta = _case(gold, name)
    m, _ = _module(meta)
    assert torch.equal(m.W.detach(), g["W"])
    assert torch.equal(m.gamma.detach(), g["gamma"]) and torch.equal(m.b.detach(), g["b"])
    if meta["mode"] == "plane":
        assert torch.equal(m.Wd.detach(), g["Wd"])


@pytest.mark.parametrize("name", CASES)
def test_pairs_and_balance_term_on_the_host(gold, name):
    """The module's straight-through pairs and load-balance term, run on host
    tensors of the hash that the reference module saw (the oracle's hash_s
    of the fixture's inputs and parameters): pairs equal to the oracle's
    (assign.py:257-317 restated; cells exact, weights and their gradients
    through s within 1e-6) at anneal 1 and 0.5, all pairs and the single
    chosen cell, planted key columns included; the balance term of both sides
    equal to the reference module's ``aux`` within 1e-5."""
    g, meta = _case(gold, name)
    m, spec = _module(meta)
    n, h = meta["n"], meta["h"]
    gen = torch.Generator().manual_seed(5)
    aux = 0.0
    for u, plant in ((g["u"][:, :n], True), (g["u"][:, n:], False)):
        s0 = R.hash_s(u, g["W"], g["gamma"], g["b"], spec.q, h).detach()
        cols = torch.as_tensor(spec.planted_cols, dtype=torch.long)
        planted = plant and bool((cols < s0.shape[1]).any())
        for anneal in (1.0, 0.5):
            for single in (False, True):
                m.anneal = anneal
                s = s0.clone().requires_grad_(True)
                cells, idx, w, a = m._ste_pairs(s, plant_at=plant, single=single)
                sr = s0.clone().requires_grad_(True)
                idx_r, w_r = R.soft_pairs(sr, spec.q, spec.dim, anneal,
                                          single=single and not planted)
                if plant:
                    idx_r, w_r = R.plant_pairs(idx_r, w_r, spec.planted_cols, m.plant_cells)
                assert torch.equal(idx, idx_r) and torch.equal(cells, idx_r[..., 0])
                assert (w - w_r).abs().max().item() < 1e-6
                wt = torch.randn(w.shape, generator=gen, dtype=w.dtype)
                (w * wt).sum().backward()
                (w_r * wt).sum().backward()
                assert (s.grad - sr.grad).abs().max().item() < 1e-6
        aux = aux + float(m._balance(s0))
    if "aux" in g:
        assert abs(aux - float(g["aux"])) < 1e-5


def test_grouped_planes_are_the_hyperplanes():
    """Every (direction, offset) row is the solution set of <a_e, x> = o."""
    from smat_attention_amd.assign import grouped_planes
    for q, dim in [(5, 2), (3, 3), (7, 1)]:
        dirs, grouped = grouped_planes(q, dim)
        idx = np.arange(q ** dim)
        pts = np.stack([(idx // q ** (dim - 1 - k)) % q for k in range(dim)], axis=1)
        assert grouped.shape == (dirs.shape[0], q, q ** (dim - 1))
        for e in range(dirs.shape[0]):
            for o in range(q):
                sel = np.flatnonzero((pts @ dirs[e]) % q == o)
                assert np.array_equal(np.sort(grouped[e, o]), sel)


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_content_assign_on_gpu(gold, name):
    """HIP hash + sorted pool + list read against the reference's fixtures."""
    g, meta = _case(gold, name)
    dev = torch.device("cuda:0")
    m, spec = _module(meta, dev)
    n = meta["n"]
    with torch.no_grad():
        y = m(g["u"].to(dev), g["Phi"].to(dev), g["Psi"].to(dev), g["Vb"].to(dev), n)
        ck = m.last_hard_k.cpu()
        cq, s = m._hash(g["u"][:, n:].to(dev))
    torch.cuda.synchronize()
    # cells: identical except a token whose q*Phi(z) sits within float noise of a bin edge
    _, sk_ref = R.cells(g["u"][:, :n], g["W"], g["gamma"], g["b"], spec.q, spec.dim, meta["h"])
    near = ((sk_ref - sk_ref.round()).abs() < 1e-4).any(-1)
    bad = (ck != g["ck"]) & ~near
    assert int(bad.sum()) == 0
    assert torch.equal(cq.cpu(), g["cq"]) or int((cq.cpu() != g["cq"]).sum()) <= 2
    if int((ck != g["ck"]).sum()) == 0:
        rel = (y.cpu() - g["y"]).abs().max() / g["y"].abs().max()
        assert rel < 1e-5
    assert abs(float(m.aux.detach()) - float(g["aux"])) < 1e-5


GRAD_CASES = ["T512_d3_point", "T512_d2_point", "T512_d3_plane"] + PAIR_CASES
GRAD_KEYS = ("du", "dPhi", "dPsi", "dVb", "dW", "dgamma", "db")


def _grad_keys(meta):
    return GRAD_KEYS + (("dWd",) if meta["mode"] == "plane" else ())


def _grads(fn, g, meta, params):
    xs = {k: g[k].clone().requires_grad_(True) for k in ("u", "Phi", "Psi", "Vb")}
    y = fn(xs, params)
    (y * g["R"].to(y.dtype).to(y.device)).sum().backward()
    out = {"d" + k: xs[k].grad.detach().cpu() for k in ("u", "Phi", "Psi", "Vb")}
    out.update({"d" + k: params[k].grad.detach().cpu() for k in params})
    return y.detach().cpu(), out


def _grel(a, b):
    return ((a.double() - b.double()).abs().max() / b.double().abs().max().clamp_min(1e-30)).item()


@pytest.mark.parametrize("name", ["T512_d3_point", "T512_d2_point"])
def test_oracle_gradients_match_reference_fixtures(gold, name):
    """The oracle's dense straight-through restatement, under autograd, gives the
    reference module's gradients (fixtures of assign.py's own backward)."""
    g, meta = _case(gold, name)
    spec = build_mask(meta["T"], meta["d"], chunk=64)
    prm = {k: g[k].clone().requires_grad_(True) for k in ("W", "gamma", "b")}
    pc = torch.tensor([spec.q ** (spec.dim - l) for l in range(1, spec.dim + 1)])

    def fn(xs, p_):
        return R.dense_point_ste(xs["u"], xs["Phi"], xs["Psi"], xs["Vb"], meta["n"], p_["W"],
                                 p_["gamma"], p_["b"], spec.q, spec.dim, meta["h"], spec.N0,
                                 spec.planted_cols, pc)
    y, gr = _grads(fn, g, meta, prm)
    assert _grel(y, g["y"]) < 1e-5
    for k in GRAD_KEYS:
        assert _grel(gr[k], g[k]) < 1e-4, (k, _grel(gr[k], g[k]))


@pytest.mark.gpu
@pytest.mark.parametrize("name", GRAD_CASES)
def test_content_assign_gradients_on_gpu(gold, name):
    """The HIP training path (point read): gradients of the module's inputs and
    parameters against the reference's own backward (fixtures)."""
    g, meta = _case(gold, name)
    dev = torch.device("cuda:0")
    m, spec = _module(meta, dev)
    with torch.no_grad():
        for k in ("W", "gamma", "b"):
            getattr(m, k).copy_(g[k].to(dev))
    gd = {k: v.to(dev) if k in ("u", "Phi", "Psi", "Vb", "R") else v for k, v in g.items()}

    def fn(xs, p_):
        return m(xs["u"], xs["Phi"], xs["Psi"], xs["Vb"], meta["n"])
    prm = {"W": m.W, "gamma": m.gamma, "b": m.b}
    if meta["mode"] == "plane":
        with torch.no_grad():
            m.Wd.copy_(g["Wd"].to(dev))
        prm["Wd"] = m.Wd
    y, gr = _grads(fn, gd, meta, prm)
    assert _grel(y, g["y"]) < 1e-5
    assert abs(float(m.aux.detach()) - float(g["aux"])) < 1e-5
    assert torch.equal(m.last_hard_k.cpu(), g["ck"].long())
    for k in _grad_keys(meta):
        assert _grel(gr[k], g[k]) < 1e-4, (k, _grel(gr[k], g[k]))


def test_content_assign_refuses_cpu_tensors_and_unbuilt_options():
    """The module runs on the GPU only and says so before any kernel; the
    delta-rule pool (an option outside the port) raises."""
    from smat_attention_amd.assign import ContentAssign
    spec = build_mask(512, 3, chunk=64)
    m = ContentAssign(2, 32, spec, mode="plane")
    u = torch.randn(1, 512, 32)
    Phi = torch.rand(2, 512, 8)
    Vb = torch.rand(2, 512, 9)
    with pytest.raises(ValueError, match="GPU"):
        m(u, Phi, Phi, Vb, 256)
    m.delta_updates = True
    with pytest.raises(NotImplementedError, match="delta"):
        m(u, Phi, Phi, Vb, 256)
    with pytest.raises(ValueError, match="dir_head"):
        ContentAssign(2, 32, spec, mode="plane", dir_head="attention")


@pytest.mark.gpu
def test_content_assign_gradients_head_dim_128():
    """Head size 128 (r = 128, p = 129: the reads over p run in two column
    blocks), T = 1024, two sequences, two heads: every gradient of the HIP
    training path against the oracle's dense straight-through path under CPU
    autograd, fp32 both, to 1e-4 of each gradient's largest entry."""
    from smat_attention_amd.assign import ContentAssign
    T, d, h, dm, nb, r = 1024, 3, 2, 64, 2, 128
    spec = build_mask(T, d, chunk=64)
    n = T // 2
    torch.manual_seed(77)
    m = ContentAssign(h, dm, spec, mode="point")
    gen = torch.Generator().manual_seed(78)
    u = torch.randn(nb, T, dm, generator=gen)
    Phi = torch.rand(nb * h, T, r, generator=gen) + 0.1
    Psi = torch.rand(nb * h, T, r, generator=gen) + 0.1
    Vb = torch.cat([torch.randn(nb * h, T, r, generator=gen), torch.ones(nb * h, T, 1)], -1)
    R_ = torch.randn(nb * h, T - n, r + 1, generator=gen)
    pc = torch.tensor([spec.q ** (spec.dim - l) for l in range(1, spec.dim + 1)])
    g = {"u": u, "Phi": Phi, "Psi": Psi, "Vb": Vb, "R": R_}
    prm = {k: getattr(m, k).detach().clone().requires_grad_(True) for k in ("W", "gamma", "b")}

    def ref(xs, p_):
        return R.dense_point_ste(xs["u"], xs["Phi"], xs["Psi"], xs["Vb"], n, p_["W"],
                                 p_["gamma"], p_["b"], spec.q, spec.dim, h, spec.N0,
                                 spec.planted_cols, pc)
    y0, g0 = _grads(ref, g, None, prm)

    dev = torch.device("cuda:0")
    m = m.to(dev)
    gd = {k: v.to(dev) for k, v in g.items()}

    def hip(xs, p_):
        return m(xs["u"], xs["Phi"], xs["Psi"], xs["Vb"], n)
    y1, g1 = _grads(hip, gd, None, {"W": m.W, "gamma": m.gamma, "b": m.b})
    assert _grel(y1, y0) < 1e-5
    for k in GRAD_KEYS:
        assert _grel(g1[k], g0[k]) < 1e-4, (k, _grel(g1[k], g0[k]))


@pytest.mark.parametrize("name", GRAD_CASES)
def test_oracle_pair_branch_matches_reference_fixtures(gold, name):
    """The oracle's pair branch (soft weights, one-cell sparse pairs, coset
    read) under CPU autograd gives the reference module's forward and
    gradients, for every case the fixtures hold gradients of."""
    g, meta = _case(gold, name)
    spec = build_mask(meta["T"], meta["d"], chunk=64)
    pc = torch.tensor([spec.q ** (spec.dim - l) for l in range(1, spec.dim + 1)])
    keys = ("W", "gamma", "b") + (("Wd",) if meta["mode"] == "plane" else ())
    prm = {k: g[k].clone().requires_grad_(True) for k in keys}
    M, coset_of = _plane_tables(spec) if meta["mode"] == "plane" else (None, None)

    def fn(xs, p_):
        return R.pairs_branch(xs["u"], xs["Phi"], xs["Psi"], xs["Vb"], meta["n"], p_["W"],
                              p_["gamma"], p_["b"], spec.q, spec.dim, meta["h"], spec.N0,
                              anneal=meta["anneal"], single=meta["sparse"],
                              planted_cols=spec.planted_cols, plant_cells=pc, mode=meta["mode"],
                              M=M, Wd=p_.get("Wd"), coset_of=coset_of,
                              dir_soft=meta["dir_soft"])
    y, gr = _grads(fn, g, meta, prm)
    assert _grel(y, g["y"]) < 1e-5
    for k in _grad_keys(meta):
        assert _grel(gr[k], g[k]) < 1e-4, (k, _grel(gr[k], g[k]))


def test_oracle_pair_maps_brute_force():
    """The dense form of the pair maps against explicit loops:
    F[b, x] = sum_{j,k: idx = x} w Psi_j Vb_j^T, y_i = sum_k w Phi_i F[idx_ik],
    duplicates within a token included."""
    gen = torch.Generator().manual_seed(5)
    Bs, L, m, K, N0, r, p = 2, 6, 5, 3, 4, 2, 3
    Psi, Vb, Phi = (torch.randn(Bs, L, r, generator=gen), torch.randn(Bs, L, p, generator=gen),
                    torch.randn(Bs, m, r, generator=gen))
    idk = torch.randint(0, N0, (Bs, L, K), generator=gen)
    idk[0, 0, 1] = idk[0, 0, 0]
    idq = torch.randint(0, N0, (Bs, m, K), generator=gen)
    wk, wq = torch.randn(Bs, L, K, generator=gen), torch.randn(Bs, m, K, generator=gen)
    F = torch.bmm(R.pairs_dense(idk, wk, N0).transpose(1, 2),
                  torch.einsum("bnr,bnp->bnrp", Psi, Vb).reshape(Bs, L, r * p)).view(Bs, N0, r, p)
    y = torch.einsum("bir,birp->bip", Phi,
                     torch.bmm(R.pairs_dense(idq, wq, N0), F.reshape(Bs, N0, r * p)).view(Bs, m, r, p))
    Fl = torch.zeros(Bs, N0, r, p)
    for b in range(Bs):
        for j in range(L):
            for k in range(K):
                Fl[b, idk[b, j, k]] += wk[b, j, k] * torch.outer(Psi[b, j], Vb[b, j])
    yl = torch.zeros(Bs, m, p)
    for b in range(Bs):
        for i in range(m):
            for k in range(K):
                yl[b, i] += wq[b, i, k] * (Phi[b, i] @ Fl[b, idq[b, i, k]])
    assert torch.allclose(F, Fl, atol=1e-5) and torch.allclose(y, yl, atol=1e-5)


def test_pool_ops_refuse_cpu_tensors_and_bad_cells():
    from smat_attention_amd import pool_ops
    Psi = torch.rand(1, 4, 2)
    idx = torch.zeros(1, 4, 1, dtype=torch.long)
    with pytest.raises(ValueError, match="GPU"):
        pool_ops.pool_segmented(Psi, Psi, idx, torch.ones(1, 4, 1), 3)
    with pytest.raises(ValueError, match="cell indices"):
        pool_ops._check("pool_segmented", idx + 3, torch.ones(1, 4, 1), 3, 4)


def test_csr_offsets_match_counts():
    """The device CSR builder (a stable sort and a binary search, no read-back)
    against bincount and a stable argsort, empty keys and an empty input
    included."""
    from smat_attention_amd.pool_ops import _csr
    gen = torch.Generator().manual_seed(3)
    for n, nkeys in ((1000, 37), (5, 40), (0, 4), (300, 1)):
        key = torch.randint(0, nkeys, (n,), generator=gen)
        if n:
            key[key == nkeys // 2] = 0                  # some keys with no entries
        order, offs = _csr(key, nkeys)
        counts = torch.bincount(key, minlength=nkeys)
        assert torch.equal(offs[1:] - offs[:-1], counts) and offs[0] == 0 and offs[-1] == n
        assert torch.equal(order, torch.argsort(key, stable=True))


@pytest.mark.gpu
@pytest.mark.parametrize("nb,L,ncls", [(3, 300, 7), (2, 5000, 169), (1, 2048, 1), (4, 64, 300),
                                       (2, 0, 5), (96, 8192, 169), (1, 4100, 8192),
                                       (0, 100, 5), (1, 600_000, 8192)])
def test_class_lists_match_stable_sort(nb, L, ncls):
    """smat_csr_lists (the counting sort behind every cell and type list)
    against torch's stable argsort and bincount of ``b*ncls + key`` on the CPU:
    the same order (as global, as in-sequence and as rows of longer sequences
    from a row offset) and offsets.  Ragged tiles (L not a multiple of the
    512-item tile), one class, empty classes, empty sequences, the largest
    class count and a sequence long enough that the tile doubles (600 000
    items, 8192 classes: 2048-item tiles) included."""
    from smat_attention_amd.pool_ops import _class_lists
    gen = torch.Generator().manual_seed(nb * 7 + L + ncls)
    keys = torch.randint(0, ncls, (nb, L), generator=gen)
    if L and ncls > 2:
        keys[keys == ncls // 2] = 0                     # an empty class in every sequence
    flat = (torch.arange(nb).unsqueeze(1) * ncls + keys).reshape(-1)
    ref = torch.argsort(flat, stable=True)
    cnt = torch.bincount(flat, minlength=nb * ncls)
    dev = torch.device("cuda:0")
    for glob in (True, False):
        order, offs = _class_lists(keys.to(dev), ncls, global_index=glob)
        assert order.dtype == torch.int32 and offs.dtype == torch.int64
        want = ref if glob else ref % max(L, 1)
        assert torch.equal(order.cpu().long(), want)
        offs = offs.cpu()
        assert offs[0] == 0 and offs[-1] == nb * L
        assert torch.equal(offs[1:] - offs[:-1], cnt)
    if L:
        # rows [11, 11 + L) of sequences L + 37 rows long: item b*(L+37) + 11 + l
        order, offs = _class_lists(keys.to(dev), ncls, seq_rows=L + 37, row0=11)
        want = (ref // L) * (L + 37) + 11 + ref % L
        assert torch.equal(order.cpu().long(), want)
        assert torch.equal(offs.cpu()[1:] - offs.cpu()[:-1], cnt)
    if nb == 0:
        # the one offset of an empty batch is written, not left as it was
        from smat_attention_amd.kernels._lib import call, stream_of
        offs = torch.full((1,), 7, device=dev, dtype=torch.int64)
        call("smat_csr_lists", None, None, offs.data_ptr(), None, 0, L, ncls, 1, L, 0,
             stream_of(offs))
        assert offs.item() == 0


@pytest.mark.gpu
@pytest.mark.parametrize("hint", [0, 1, 64, None])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_list_read_covers_lists_longer_than_the_grid(hint, dt):
    """smat_query_lists sized by a hint below the longest list (80 % of the
    rows in one class, up to 560 rows against a 64-row workgroup): every row is
    still read, y_l = X_l U[cls_l] against the fp64 product (1e-5 for fp32, the
    bf16 inputs' own values for bf16)."""
    from smat_attention_amd import pool_ops
    gen = torch.Generator().manual_seed(17)
    nb, L, ncls, r, p = 2, 700, 5, 64, 65
    cls = torch.where(torch.rand(nb, L, generator=gen) < 0.8, 0,
                      torch.randint(1, ncls, (nb, L), generator=gen))
    X = torch.randn(nb, L, r, generator=gen).to(dt)
    U = torch.randn(nb, ncls, r, p, generator=gen)
    dev = torch.device("cuda:0")
    rows, offs, h = pool_ops._lists(cls.to(dev), ncls)
    Y = pool_ops._read_lists(X.to(dev), U.to(dev), cls.to(dev),
                             (rows, offs, h if hint is None else hint))
    Ug = U.double()[torch.arange(nb).unsqueeze(1), cls]
    ref = (X.double().unsqueeze(-1) * Ug).sum(-2)
    assert _grel(Y.cpu(), ref) < (1e-5 if dt == torch.float32 else 1e-4)


@pytest.mark.gpu
@pytest.mark.parametrize("K,r,p", [(1, 16, 17), (4, 16, 17), (8, 128, 129)])
def test_pool_ops_match_dense_maps(K, r, p):
    """pool_segmented / read_gather (HIP list kernels, fp32) and every gradient
    against the dense maps under fp64 CPU autograd (the reference's own
    exactness check, smat_pool_ops.py:94-117), repeated cells included."""
    from smat_attention_amd import pool_ops
    gen = torch.Generator().manual_seed(10 + K)
    Bs, n, m, N0 = 3, 300, 200, 7
    Psi, Vb, Phi = (torch.randn(Bs, n, r, generator=gen), torch.randn(Bs, n, p, generator=gen),
                    torch.randn(Bs, m, r, generator=gen))
    idk, idq = (torch.randint(0, N0, (Bs, n, K), generator=gen),
                torch.randint(0, N0, (Bs, m, K), generator=gen))
    wk, wq = torch.rand(Bs, n, K, generator=gen), torch.rand(Bs, m, K, generator=gen)
    R_ = torch.randn(Bs, m, p, generator=gen)
    ins = {"Psi": Psi, "Vb": Vb, "Phi": Phi, "wk": wk, "wq": wq}

    def run(dev, dt, pool, read):
        xs = {k: v.to(dev, dt).requires_grad_(True) for k, v in ins.items()}
        F = pool(xs["Psi"], xs["Vb"], idk.to(dev), xs["wk"], N0)
        y = read(xs["Phi"], idq.to(dev), xs["wq"], F)
        (y * R_.to(dev, dt)).sum().backward()
        return y.detach().cpu(), {k: v.grad.detach().cpu() for k, v in xs.items()}

    def dpool(Ps, V, idx, w, N0_):
        return torch.bmm(R.pairs_dense(idx, w, N0_).transpose(1, 2),
                         torch.einsum("bnr,bnp->bnrp", Ps, V).reshape(Bs, n, r * p)).view(Bs, N0_, r, p)

    def dread(Ph, idx, w, F):
        U = torch.bmm(R.pairs_dense(idx, w, F.shape[1]), F.reshape(Bs, F.shape[1], r * p))
        return torch.einsum("bir,birp->bip", Ph, U.view(Bs, m, r, p))
    y0, g0 = run("cpu", torch.float64, dpool, dread)
    y1, g1 = run(torch.device("cuda:0"), torch.float32, pool_ops.pool_segmented,
                 pool_ops.read_gather)
    assert _grel(y1, y0) < 1e-5
    for k in g0:
        assert _grel(g1[k], g0[k]) < 1e-5, (k, _grel(g1[k], g0[k]))


@pytest.mark.gpu
@pytest.mark.parametrize("T,d", [(128, 2), (128, 3), (512, 2), (512, 3)])
@pytest.mark.parametrize("mode", ["point", "plane"])
def test_branch_is_masked_attention_under_its_own_hash(T, d, mode):
    """The HIP branch equals dense masked kernel attention under the mask its
    own hash induces (the reference's exactness check,
    tests/test_content_addr.py:11-42): G[i, j] = 1 when key j's cell is query
    i's cell (point), or lies on query i's chosen hyperplane (plane)."""
    from smat_attention_amd.assign import ContentAssign
    spec = build_mask(T, d, chunk=32)
    n, m_ = spec.n, spec.T_R
    nb, h, dh, r, p = 3, 2, 8, 5, 4
    torch.manual_seed(0)
    dev = torch.device("cuda:0")
    ca = ContentAssign(h, dh, spec, mode=mode).to(dev)
    B = nb * h
    g = torch.Generator().manual_seed(T + d)
    u = torch.randn(nb, T, dh, generator=g)
    Phi, Psi = torch.rand(B, T, r, generator=g), torch.rand(B, T, r, generator=g)
    Vb = torch.randn(B, T, p, generator=g)
    with torch.no_grad():
        got = ca(u.to(dev), Phi.to(dev), Psi.to(dev), Vb.to(dev), n).cpu().double()
        kc = ca.last_hard_k.cpu()
        qc, _ = ca._hash(u[:, n:].to(dev))
        qc = qc.cpu()
    if ca.mode == "point":
        G = (qc.unsqueeze(2) == kc.unsqueeze(1)).double()
    else:
        dl = torch.einsum("blm,hem->bhle", u[:, n:], ca.Wd.detach().cpu())
        e = dl.reshape(B, m_, ca.D).argmax(-1)
        o = ca.coset_of.cpu()[e, qc]
        Mi = ca.M.cpu().double()[e, o]
        G = Mi.gather(2, kc.unsqueeze(1).expand(B, m_, n))
    Sc = torch.einsum("bir,bjr->bij", Phi[:, n:].double(), Psi[:, :n].double())
    ref = (Sc * G) @ Vb[:, :n].double()
    assert G.mean().item() > 0, "the mask is empty: the check would be vacuous"
    assert _grel(got, ref) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["point", "plane"])
def test_straight_through_gradient_reaches_the_hash(mode):
    """A nonzero gradient reaches the hash projection W (the reference's
    tests/test_content_addr.py:45-55), through the HIP training path."""
    from smat_attention_amd.assign import ContentAssign
    spec = build_mask(512, 3, chunk=32)
    dev = torch.device("cuda:0")
    torch.manual_seed(1)
    ca = ContentAssign(2, 8, spec, mode=mode).to(dev)
    g = torch.Generator().manual_seed(2)
    u = torch.randn(3, 512, 8, generator=g).to(dev)
    Phi, Psi = torch.rand(6, 512, 5, generator=g).to(dev), torch.rand(6, 512, 5, generator=g).to(dev)
    ca(u, Phi, Psi, torch.randn(6, 512, 4, generator=g).to(dev), spec.n).sum().backward()
    assert ca.W.grad.abs().max().item() > 0


# ---------------------------------------------------------------------------
# options beyond the point / plane reads: key convolution, direction heads,
# codimension, analysis methods (tests/golden/make_assign_golden_ext.py)
# ---------------------------------------------------------------------------

GOLD_EXT = os.path.join(os.path.dirname(__file__), "golden", "assign_golden_ext.npz")
EXT_CASES = {
    "T512_d3_point_conv4": (512, 3, dict(mode="point", conv_width=4)),
    "T512_d3_plane_mlp": (512, 3, dict(mode="plane", dir_head="mlp", dir_hidden=32)),
    "T512_d3_plane_delta": (512, 3, dict(mode="plane", src="id", vocab=64, dir_head="delta",
                                         dir_window=4)),
    "T512_d3_plane_fixed": (512, 3, dict(mode="plane", src="id", vocab=64, dir_head="fixed",
                                         dir_window=3)),
    "T512_d4_codim2": (512, 4, dict(codim=2)),
    "T512_d4_codim3": (512, 4, dict(codim=3)),
}
EXT_H, EXT_DM = 2, 32


@pytest.fixture(scope="module")
def gold_ext():
    return np.load(GOLD_EXT)


def _ext(gold_ext, name):
    return {k.split("/", 1)[1]: torch.from_numpy(gold_ext[k]) for k in gold_ext.files
            if k.startswith(name + "/")}


def _ext_module(name, device="cpu"):
    from smat_attention_amd.assign import ContentAssign
    T, d, opts = EXT_CASES[name]
    spec = build_mask(T, d, chunk=64)
    torch.manual_seed(1000)
    m = ContentAssign(EXT_H, EXT_DM, spec, **opts)
    m.eval()
    return m.to(device), spec


@pytest.mark.parametrize("name", sorted(EXT_CASES))
def test_option_parameters_match_reference_init(gold_ext, name):
    """Built after the same seed, every parameter and table the option adds
    (the key convolution, the mlp head's layers, Wdelta and the fixed
    indicator, the id table, the coset matrix M of a codimension-2 read over
    F_5^3) equals the reference module's."""
    g = _ext(gold_ext, name)
    m, _ = _ext_module(name)
    params = dict(m.named_parameters())
    params.update(dict(m.named_buffers()))
    want = {k[len("param."):]: v for k, v in g.items() if k.startswith("param.")}
    assert set(want) <= set(params), set(want) - set(params)
    for k, v in want.items():
        assert torch.equal(params[k].detach().to(v.dtype), v), k


def test_grouped_flats_are_coset_partitions():
    """Every partition of grouped_flats(5, 3, 2) is the set of cosets of a
    1-dimensional subspace of F_5^3 (the line through 0 in the direction of the
    difference of two points of a coset): 31 distinct partitions, one per
    line through the origin, of 25 cosets of 5 points each; codim 1 gives the
    hyperplane partitions of grouped_planes."""
    from smat_attention_amd.assign import grouped_flats, grouped_planes
    q, dim = 5, 3
    g = grouped_flats(q, dim, 2)
    assert g.shape == (31, 25, 5)
    pts = np.stack([(np.arange(q ** dim) // q ** (dim - 1 - k)) % q for k in range(dim)], 1)
    seen = set()
    for part in g:
        assert sorted(part.reshape(-1).tolist()) == list(range(q ** dim))
        d0 = (pts[part[0, 1]] - pts[part[0, 0]]) % q
        for coset in part:
            diffs = (pts[coset] - pts[coset[0]]) % q
            # every point of the coset is the first plus a multiple of d0
            assert all(any(np.array_equal(x, (t * d0) % q) for t in range(q)) for x in diffs)
        seen.add(frozenset(frozenset(c.tolist()) for c in part))
    assert len(seen) == 31
    hp = {frozenset(frozenset(c.tolist()) for c in part) for part in grouped_planes(q, dim)[1]}
    assert {frozenset(frozenset(c.tolist()) for c in part)
            for part in grouped_flats(q, dim, 1)} == hp


def test_cells_of_and_oracle_dir_match_reference(gold_ext):
    """cells_of (the hash of one hidden state per head) and oracle_dir (the
    first direction whose offsets agree over a set of cells) equal the
    reference module's on the fixture's inputs, for sets of 1, 2 and 3 cells."""
    from smat_attention_amd.assign import ContentAssign
    g = _ext(gold_ext, "T512_d3_analysis")
    spec = build_mask(512, 3, chunk=64)
    torch.manual_seed(1000)
    m = ContentAssign(EXT_H, EXT_DM, spec, mode="plane")
    assert torch.equal(m.cells_of(g["cells_v"]), g["cells_of"])
    for k in (1, 2, 3):
        assert torch.equal(m.oracle_dir(g[f"oracle_cells{k}"]), g[f"oracle_dir{k}"]), k


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(EXT_CASES))
def test_options_forward_and_gradients_on_gpu(gold_ext, name):
    """The hard read with each option on the GPU against the reference
    module's output (1e-5 relative) and the gradients of (y * R).sum() with
    respect to Phi, Psi, Vb, the layer input and every trained parameter
    (1e-4 relative): the mlp and delta direction heads (the fixed head's
    frozen indicator), the codimension-2 coset read and the point read of
    codimension dim, and a module with the key convolution."""
    dev = torch.device("cuda:0")
    g = _ext(gold_ext, name)
    gin = _ext(gold_ext, "inputs")
    m, spec = _ext_module(name, dev)
    n = spec.n
    kw = {"ids": g["ids"].to(dev)} if "ids" in g else {}
    xs = [gin[k].to(dev) for k in ("u", "Phi", "Psi", "Vb")]
    with torch.no_grad():
        y = m(*xs, n, **kw).cpu()
    rel = lambda a, b: ((a.double() - b.double()).abs().max() / b.abs().max()).item()
    assert rel(y, g["y"]) < 1e-5
    xs = [x.clone().requires_grad_(True) for x in xs]
    m.zero_grad()
    yg = m(*xs, n, **kw)
    assert rel(yg.detach().cpu(), g["y"]) < 1e-5
    (yg * g["R"].to(dev)).sum().backward()
    for key, x in zip(("u", "Phi", "Psi", "Vb"), xs):
        if f"grad.{key}" in g:
            assert rel(x.grad.cpu(), g[f"grad.{key}"]) < 1e-4, key
    params = dict(m.named_parameters())
    for k, v in g.items():
        if k.startswith("grad.") and k[5:] in params:
            assert rel(params[k[5:]].grad.cpu(), v) < 1e-4, k


@pytest.mark.gpu
def test_agreement_terms_on_gpu(gold_ext):
    """agreement (the query side's routing term) after a forward of the d = 3
    plane read: value within 1e-5 and its gradients to W, gamma and b within
    1e-4 of the reference module's.  key_agreement reads the key side's soft
    distribution, which the reference never records: with the recent half of
    the layer input equal to the distant half, the two sides' distributions
    are equal, and key_agreement at payload positions J filed under their
    hard cells equals agreement over the pairs (J, J)."""
    from smat_attention_amd.assign import ContentAssign
    dev = torch.device("cuda:0")
    g = _ext(gold_ext, "T512_d3_analysis")
    gin = _ext(gold_ext, "inputs")
    spec = build_mask(512, 3, chunk=64)
    n = spec.n
    torch.manual_seed(1000)
    m = ContentAssign(EXT_H, EXT_DM, spec, mode="plane").to(dev)
    m.eval()
    xs = [gin[k].to(dev) for k in ("u", "Phi", "Psi", "Vb")]
    m(*xs, n)
    assert torch.equal(m.last_hard_k.cpu(), g["hard_k"])
    a = m.agreement(g["pairs"].to(dev), g["valid"].to(dev))
    assert abs(a.item() - g["agreement"].item()) < 1e-5 * max(1.0, abs(g["agreement"].item()))
    a.backward()
    for k in ("W", "gamma", "b"):
        want = g[f"grad.{k}"]
        got = getattr(m, k).grad.cpu()
        assert ((got - want).abs().max() / want.abs().max()).item() < 1e-4, k
    # the key side, pinned through the query side
    torch.manual_seed(5)
    m1 = ContentAssign(1, EXT_DM, spec, mode="plane").to(dev)
    m1.eval()
    u = xs[0][:, :n].repeat(1, 2, 1)                       # recent half == distant half
    Phi, Psi, Vb = (x[:1] for x in xs[1:])
    with torch.no_grad():
        m1(u, Phi, Psi, Vb, n)
        assert torch.equal(m1.last_soft_k, m1.last_soft_q)
        J = torch.randint(0, n, (1, 9), generator=torch.Generator().manual_seed(6)).to(dev)
        valid = torch.ones(1, 9, dtype=torch.bool, device=dev)
        C = m1.last_hard_k.gather(1, J)
        ka = m1.key_agreement(J, C, valid)
        qa = m1.agreement(torch.stack([J, J], -1), valid)
    assert torch.isfinite(ka) and ka.item() == qa.item()
