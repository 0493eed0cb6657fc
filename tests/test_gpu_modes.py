"""GPU parity of the other operand-load modes and of cfg2 at its full size.

* The > 4 GiB load mode (queries through an item-based buffer, candidates through
  64-bit row pointers) forced at small sizes with UNG_HIP_FORCE_WIDE=1, bit-exact
  against the oracle.
* The exact rescan of flagged rows (one or several ranges per row), forced for every
  row with UNG_HIP_EPS_SCALE (a certification bound widened 1e30-fold), bit-exact
  against the oracle.
* cfg2 at its full size (1M x 128): every cross-edge row (2.06e10 pairs) and every mid
  group compared bit-exactly with the reference's own compiled distance + queue
  (oracle/_ref, else the plain-C oracle), plus size-independent properties of every
  row (sorted by (dist, id), ids inside the row's minimum-superset union, sizes) and
  the additional edges.
"""
import os

import numpy as np
import pytest

import filtervectorcode_refactor_amd as F
from filtervectorcode_refactor_amd import datasets as D
from test_gpu_parity import _assert_rows_equal, _two_level_problem

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def wide_ctx():
    old = os.environ.get("UNG_HIP_FORCE_WIDE")
    os.environ["UNG_HIP_FORCE_WIDE"] = "1"
    try:
        c = F.HipContext(0)
    finally:
        if old is None:
            del os.environ["UNG_HIP_FORCE_WIDE"]
        else:
            os.environ["UNG_HIP_FORCE_WIDE"] = old
    yield c
    c.close()


def _ctx_with_env(name, value):
    old = os.environ.get(name)
    os.environ[name] = value
    try:
        return F.HipContext(0)
    finally:
        if old is None:
            del os.environ[name]
        else:
            os.environ[name] = old


@pytest.fixture(scope="module")
def rescan_ctx():
    c = _ctx_with_env("UNG_HIP_EPS_SCALE", "1e30")
    yield c
    c.close()


@pytest.mark.parametrize("dim,k,seed,targets", [(20, 6, 31, [9000, 5000, 300]), (128, 20, 32, [9000, 5000, 300]),
                                                 (8, 6, 33, [140000, 5000, 3])])
def test_rescan_cross(rescan_ctx, oracle, dim, k, seed, targets):
    """Unions of up to 145,003 candidates: up to 70 rescan ranges per flagged row (more
    ranges than merge lanes in the last case)."""
    print(f"rescan cross dim={dim} k={k} targets={targets}", flush=True)
    rng = np.random.default_rng(seed)
    children = [5, 130, 1, 40]
    X, gb, op, oi = _two_level_problem(rng, children, targets, dim, dup=True)
    t0 = len(children) + 1
    rows = [[t0, t0 + 1, t0 + 2], [t0, t0 + 1, t0 + 2], [t0, t0 + 1, t0 + 2], [t0, t0 + 2]]
    op[:] = 0
    for c, r in enumerate(rows, start=1):
        op[c + 1] = op[c] + len(r)
    op[len(rows) + 2:] = op[len(rows) + 1]
    oi = np.array([v for r in rows for v in r], np.uint32)
    rescan_ctx.prepare_vectors(X)
    ids, dist, size, stats = rescan_ctx.cross_topk(gb, op, oi, k)
    assert stats["fallback_rows"] == sum(children)
    ip, ii = F.in_neighbors(op, oi)
    o_ids, o_d, o_s = oracle.cross_exact(X, gb, ip, ii, k)
    _assert_rows_equal(ids, dist, size, o_ids, o_d, o_s, f"rescan dim={dim} k={k}")


@pytest.mark.parametrize("n,list_k,dim", [(700, 32, 20), (9000, 32, 16)])
def test_rescan_intra(rescan_ctx, oracle, n, list_k, dim):
    print(f"rescan intra n={n} k={list_k} dim={dim}", flush=True)
    rng = np.random.default_rng(n + dim)
    X = rng.standard_normal((n + 7, dim)).astype(np.float32)
    X[5] = X[3]
    rescan_ctx.prepare_vectors(X)
    ids, dist, stats = rescan_ctx.group_knn([3], [n], list_k)
    assert stats["fallback_rows"] == n
    oi, od = oracle.intra_exact(X, 3, n, list_k)
    _assert_rows_equal(ids, dist, None, oi, od, None, f"rescan intra n={n}")


@pytest.mark.parametrize("dim,k,seed", [(128, 6, 21), (12, 6, 22), (768, 20, 23), (36, 1, 24)])
def test_wide_cross(wide_ctx, oracle, dim, k, seed):
    print(f"wide cross dim={dim} k={k}", flush=True)
    rng = np.random.default_rng(seed)
    X, gb, op, oi = _two_level_problem(rng, [1, 3, 130, 300, 7], [4, 200, 2, 129, 5], dim, dup=True)
    wide_ctx.prepare_vectors(X)
    ids, dist, size, _ = wide_ctx.cross_topk(gb, op, oi, k)
    ip, ii = F.in_neighbors(op, oi)
    o_ids, o_d, o_s = oracle.cross_exact(X, gb, ip, ii, k)
    _assert_rows_equal(ids, dist, size, o_ids, o_d, o_s, f"wide dim={dim} k={k}")


@pytest.mark.parametrize("n,list_k,dim", [(129, 32, 128), (700, 32, 384), (300, 8, 20), (300, 6, 128)])
def test_wide_intra(wide_ctx, oracle, n, list_k, dim):
    print(f"wide intra n={n} k={list_k} dim={dim}", flush=True)
    rng = np.random.default_rng(n + dim)
    X = rng.standard_normal((n + 7, dim)).astype(np.float32)
    X[5] = X[3]
    wide_ctx.prepare_vectors(X)
    ids, dist, _ = wide_ctx.group_knn([3], [n], list_k)
    oi, od = oracle.intra_exact(X, 3, n, list_k)
    _assert_rows_equal(ids, dist, None, oi, od, None, f"wide intra n={n}")


@pytest.fixture(scope="module")
def panel_ctx():
    c = _ctx_with_env("UNG_HIP_NO_QREG", "1")
    yield c
    c.close()


@pytest.mark.parametrize("dim,k,seed", [(128, 6, 41), (128, 8, 42)])
def test_panel_layout_cross(panel_ctx, oracle, dim, k, seed):
    """dp = 128 with the query panel restaged every step (the layout every other dp uses)."""
    print(f"panel cross dim={dim} k={k}", flush=True)
    rng = np.random.default_rng(seed)
    X, gb, op, oi = _two_level_problem(rng, [1, 3, 130, 300, 7], [4, 200, 2, 129, 5], dim, dup=True)
    panel_ctx.prepare_vectors(X)
    ids, dist, size, _ = panel_ctx.cross_topk(gb, op, oi, k)
    ip, ii = F.in_neighbors(op, oi)
    o_ids, o_d, o_s = oracle.cross_exact(X, gb, ip, ii, k)
    _assert_rows_equal(ids, dist, size, o_ids, o_d, o_s, f"panel dim={dim} k={k}")


@pytest.mark.parametrize("n,list_k", [(300, 6), (1000, 8)])
def test_panel_layout_intra(panel_ctx, oracle, n, list_k):
    print(f"panel intra n={n} k={list_k}", flush=True)
    rng = np.random.default_rng(n + 128)
    X = rng.standard_normal((n + 7, 128)).astype(np.float32)
    X[5] = X[3]
    panel_ctx.prepare_vectors(X)
    ids, dist, _ = panel_ctx.group_knn([3], [n], list_k)
    oi, od = oracle.intra_exact(X, 3, n, list_k)
    _assert_rows_equal(ids, dist, None, oi, od, None, f"panel intra n={n}")


def _checker(oracle):
    from oracle import RefOracle, ref_available
    return RefOracle() if ref_available() else oracle


def test_cfg2_full_size(oracle):
    cfg = D.CONFIGS["cfg2"]
    print("cfg2 full: generate", flush=True)
    X, lp, li = D.generate(cfg)
    st = F.UngBuildStage(num_cross_edges=6, max_degree=32)
    st.prepare_inputs(X, lp, li)
    del X
    ctx = st.ctx
    ctx.prepare_vectors(st.base)
    print("cfg2 full: cross", flush=True)
    ids, dist, size, stats = ctx.cross_topk(st.group_begin, st.out_ptr, st.out_idx, 6)
    N = st.base.shape[0]
    # the certified bound leaves only rare rows to the exact rescan
    assert stats["fallback_rows"] <= N // 10000
    sizes = np.diff(st.group_begin.astype(np.int64))[1:]
    out_cnt = np.diff(st.out_ptr.astype(np.int64))[1:]
    union = np.zeros(st.num_groups + 1, np.int64)
    for c in np.nonzero(out_cnt)[0] + 1:
        xs = st.out_idx[st.out_ptr[c]: st.out_ptr[c + 1]].astype(np.int64)
        union[c] = int(sizes[xs - 1].sum())
    pg = st.new_vec_id_to_group_id
    # sizes and padding, every row
    assert np.array_equal(size, np.minimum(6, union[pg]).astype(np.int32))
    valid = np.arange(6)[None, :] < size[:, None]
    assert ((ids == 0xFFFFFFFF) == ~valid).all()
    # (dist, id) order, every row
    d0, d1 = dist[:, :-1], dist[:, 1:]
    i0, i1 = ids[:, :-1], ids[:, 1:]
    both = valid[:, 1:]
    assert ((d0 < d1) | ((d0 == d1) & (i0 < i1)) | ~both).all()
    # ids inside the union of the row's minimum supersets, every row
    gid = np.where(valid, pg[np.minimum(ids, N - 1)], 0)
    for c in np.nonzero(out_cnt)[0] + 1:
        rows = slice(int(st.group_begin[c]), int(st.group_begin[c + 1]))
        allowed = np.zeros(st.num_groups + 1, bool)
        allowed[st.out_idx[st.out_ptr[c]: st.out_ptr[c + 1]]] = True
        g = gid[rows][valid[rows]]
        assert allowed[g].all(), f"group {c}: id outside its union"
    # bit-exact against the reference: every row with a non-empty union (2.06e10 pairs)
    chk = _checker(oracle)
    q = np.nonzero(union[pg] > 0)[0].astype(np.uint32)
    print(f"cfg2 full: reference check of all {q.size} rows", flush=True)
    res = chk.cross_exact_points(st.base, st.group_begin, pg, st.out_ptr, st.out_idx, q, 6)
    _assert_rows_equal(ids[q], dist[q], None, res[0], res[1], None, "cfg2 full cross rows")
    # intra: every mid group, bit-exact
    gids = st.mid_groups()
    pick = gids
    begins = st.group_begin[gids]
    gsz = st.group_begin[gids + 1] - begins
    print(f"cfg2 full: intra {len(gids)} groups", flush=True)
    kids, kdist, kstats = ctx.group_knn(begins, gsz, 32)
    assert kstats["fallback_rows"] <= N // 10000
    starts = np.zeros(len(gids), np.int64)
    starts[1:] = np.cumsum(gsz.astype(np.int64))[:-1]
    row_of = dict(zip(gids.tolist(), starts.tolist()))
    for g in pick:
        b, n = int(st.group_begin[g]), int(st.group_begin[g + 1] - st.group_begin[g])
        o_i, o_d = chk.intra_exact(st.base, b, n, 32)
        r0 = row_of[int(g)]
        _assert_rows_equal(kids[r0: r0 + n], kdist[r0: r0 + n], None, o_i, o_d, None, f"cfg2 full intra {g}")
    # additional edges from the same (resident) cross rows, against the oracle fed those rows
    ctx.cross_topk_device(st.group_begin, st.out_ptr, st.out_idx, 6)
    got = ctx.additional_edges(st.group_begin, st.out_ptr, st.out_idx, 6)
    print(f"cfg2 full: {got[1].size} additional edges, stats {got[3]}", flush=True)
    want = oracle.additional_edges(st.base, st.group_begin, st.out_ptr, st.out_idx, ids, 6)
    for a, b in zip(got[:3], want):
        assert np.array_equal(a, b)
    st.close()
