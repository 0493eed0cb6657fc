"""GPU parity of the HIP path against the CPU oracle (run on an MI355X).

Bar: ids bit-exact and fp32 distances bit-exact (the exact re-rank reproduces
the reference's summation order), sizes exact.  Every call goes through the C ABI
(libung_hip.so via ctypes).
"""
import numpy as np
import pytest

import filtervectorcode_refactor_amd as F
from filtervectorcode_refactor_amd import datasets as D

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = F.HipContext(0)
    yield c
    c.close()


def _say(msg):
    print(msg, flush=True)


def _assert_rows_equal(ids_g, dist_g, size_g, ids_o, dist_o, size_o, what):
    assert ids_g.shape == ids_o.shape, what
    bad = np.nonzero((ids_g != ids_o).any(axis=1))[0]
    assert bad.size == 0, f"{what}: {bad.size} rows differ in ids, first {bad[:5]}: gpu {ids_g[bad[0]]} oracle {ids_o[bad[0]]} d_gpu {dist_g[bad[0]]} d_or {dist_o[bad[0]]}"
    assert np.array_equal(dist_g.view(np.uint32), dist_o.view(np.uint32)), f"{what}: distances not bit-exact"
    if size_g is not None:
        assert np.array_equal(size_g, size_o), f"{what}: sizes differ"


def test_mfma_layout(ctx):
    _say("test_mfma_layout")
    assert ctx.selftest_mfma() == 0.0


def test_cross_cfg1_bitexact(ctx, cfg1_stage, oracle):
    st = cfg1_stage
    _say("cross cfg1: prepare")
    ctx.prepare_vectors(st.base)
    ids, dist, size, stats = ctx.cross_topk(st.group_begin, st.out_ptr, st.out_idx, 6)
    _say(f"cross cfg1 stats {stats}")
    oi, od, os_ = oracle.cross_exact(st.base, st.group_begin, st.in_ptr, st.in_idx, 6)
    _assert_rows_equal(ids, dist, size, oi, od, os_, "cfg1 cross k=6")
    assert stats["pairs"] == F.count_pairs(st.group_begin, st.out_ptr, st.out_idx)[0]


@pytest.mark.parametrize("k", [6, 1, 40])
def test_cross_tiny_and_tiled_jobs(ctx, oracle, k):
    """Groups of 1-130 vectors with 0-4 random out-groups: jobs of a few queries and small
    unions take the exact per-job scan, the others the select and the merge (q = 9 with
    U <= 64 is just past the tiny bound); unions smaller than k leave rows part-empty;
    a duplicated vector gives distance ties."""
    rng = np.random.default_rng(50 + k)
    sizes = rng.choice([1, 2, 3, 5, 8, 9, 17, 40, 70, 130], size=60)
    G, d = sizes.size, 40
    N = int(sizes.sum())
    X = rng.standard_normal((N, d)).astype(np.float32)
    X[5] = X[6]
    gb = np.concatenate([[0, 0], np.cumsum(sizes)]).astype(np.uint32)
    rows = [[] for _ in range(G + 1)]
    for g in range(1, G + 1):
        cand = [x for x in range(1, G + 1) if x != g]
        rows[g] = sorted(rng.choice(cand, size=int(rng.integers(0, 5)), replace=False).tolist())
    op = np.zeros(G + 2, np.uint32)
    op[2:] = np.cumsum([len(rows[g]) for g in range(1, G + 1)])
    oi = np.array([x for g in range(1, G + 1) for x in rows[g]], np.uint32)
    ctx.prepare_vectors(X)
    ids, dist, size, st = ctx.cross_topk(gb, op, oi, k)
    _say(f"tiny/tiled k={k}: {st['work_items']} select items, {st['rows']} rows")
    pg = np.repeat(np.arange(1, G + 1, dtype=np.uint32), sizes)
    o = oracle.cross_exact_points(X, gb, pg, op, oi, np.arange(N, dtype=np.uint32), k)
    _assert_rows_equal(ids, dist, None, o[0], o[1], None, f"tiny/tiled k={k}")
    assert np.array_equal(size, (ids != 0xFFFFFFFF).sum(axis=1)), "row sizes"


def test_intra_cfg1_bitexact(ctx, cfg1_stage, oracle):
    st = cfg1_stage
    ctx.prepare_vectors(st.base)
    gids = st.mid_groups()
    assert len(gids) > 0
    begins = st.group_begin[gids]
    sizes = st.group_begin[gids + 1] - begins
    _say(f"intra cfg1: {len(gids)} groups, sizes {sizes.min()}..{sizes.max()}")
    ids, dist, stats = ctx.group_knn(begins, sizes, 32)
    _say(f"intra cfg1 stats {stats}")
    row = 0
    for b, n in zip(begins, sizes):
        oi, od = oracle.intra_exact(st.base, int(b), int(n), 32)
        _assert_rows_equal(ids[row: row + n], dist[row: row + n], None, oi, od, None, f"intra group@{b} n={n}")
        row += n


def test_pack_cfg1_matches_oracle(ctx, cfg1_stage, oracle):
    st = cfg1_stage
    ctx.prepare_vectors(st.base)
    gids = st.mid_groups()
    begins = st.group_begin[gids]
    sizes = st.group_begin[gids + 1] - begins
    for list_k, anchor_tail in ((32, 1), (63, 0)):
        ids, dist, _ = ctx.group_knn(begins, sizes, list_k)
        graph, entries, _ = ctx.pack_anchor_rows(ids.shape[0], len(gids), 64, 32, 24, anchor_tail, 0, 0)
        row = 0
        for b, n in zip(begins, sizes):
            cand = min(64, 63, int(n) - 1)
            for j in range(int(n)):
                ref = oracle.pack_anchor_row(ids[row + j][:cand] if cand <= list_k else ids[row + j], cand, int(n), j,
                                             32, 24, anchor_tail, 0, 0, 33)
                assert np.array_equal(graph[row + j], ref), (list_k, anchor_tail, b, j)
            row += n
        assert (entries == 0).all()


def _two_level_problem(rng, sizes_children, sizes_targets, dim, dup=False):
    """Children 1..C, targets C+1..C+T; every child points to a random subset of
    targets (possibly none).  Returns X (group-contiguous), group_begin, out CSR."""
    C = len(sizes_children)
    sizes = list(sizes_children) + list(sizes_targets)
    G = len(sizes)
    gb = np.zeros(G + 2, np.uint32)
    gb[2:] = np.cumsum(sizes)
    N = int(gb[-1])
    X = rng.standard_normal((N, dim)).astype(np.float32)
    if dup:
        # exact duplicates across groups -> equal distances, ties broken by id
        X[gb[C + 1]: gb[C + 1] + 3] = X[gb[1]: gb[1] + 3]
        X[gb[G]: gb[G] + 2] = X[gb[C + 1]: gb[C + 1] + 2]
    out_ptr = np.zeros(G + 2, np.uint32)
    rows = []
    for c in range(1, G + 1):
        if c <= C:
            m = rng.integers(0, len(sizes_targets) + 1)
            row = sorted(rng.choice(np.arange(C + 1, G + 1), size=m, replace=False).tolist())
        else:
            row = []
        rows.append(row)
        out_ptr[c + 1] = out_ptr[c] + len(row)
    out_idx = np.array([v for r in rows for v in r], np.uint32)
    return X, gb, out_ptr, out_idx


@pytest.mark.parametrize("dim,k,seed", [(128, 6, 1), (37, 6, 2), (12, 1, 3), (64, 64, 4), (128, 20, 5),
                                        (768, 6, 6), (5, 6, 7), (128, 12, 8), (40, 16, 9), (128, 8, 10)])
def test_cross_edge_cases(ctx, oracle, dim, k, seed):
    rng = np.random.default_rng(seed)
    _say(f"cross edge case dim={dim} k={k}")
    X, gb, op, oi = _two_level_problem(rng, [1, 2, 3, 130, 300, 7, 1], [1, 4, 200, 2, 129, 5], dim, dup=(seed == 1))
    ctx.prepare_vectors(X)
    ids, dist, size, stats = ctx.cross_topk(gb, op, oi, k)
    ip, ii = F.in_neighbors(op, oi)
    o_ids, o_d, o_s = oracle.cross_exact(X, gb, ip, ii, k)
    _assert_rows_equal(ids, dist, size, o_ids, o_d, o_s, f"edge dim={dim} k={k}")


def test_cross_multi_split(ctx, oracle):
    """Unions above one work item's candidate split (32768) are merged on device."""
    rng = np.random.default_rng(11)
    X, gb, op, oi = _two_level_problem(rng, [300, 5], [20000, 15000, 3], 128)
    op = np.array([0, 0, 3, 6, 6, 6, 6], np.uint32)
    oi = np.array([3, 4, 5, 3, 4, 5], np.uint32)
    ctx.prepare_vectors(X)
    ids, dist, size, stats = ctx.cross_topk(gb, op, oi, 6)
    _say(f"multi split stats {stats}")
    assert stats["work_items"] > 4  # 4 query blocks, each over more than one split
    ip, ii = F.in_neighbors(op, oi)
    o_ids, o_d, o_s = oracle.cross_exact(X, gb, ip, ii, 6)
    _assert_rows_equal(ids, dist, size, o_ids, o_d, o_s, "multi split")


@pytest.mark.parametrize("n,list_k,dim", [(2, 32, 128), (3, 1, 16), (129, 32, 128), (200, 64, 40), (700, 32, 384),
                                          (20000, 8, 64), (300, 6, 128), (1000, 8, 128), (500, 16, 128),
                                          (600, 12, 72)])
def test_intra_edge_cases(ctx, oracle, n, list_k, dim):
    rng = np.random.default_rng(n)
    _say(f"intra edge case n={n} k={list_k} dim={dim}")
    X = rng.standard_normal((n + 10, dim)).astype(np.float32)
    if n > 5:
        X[6] = X[2]  # duplicate inside the group: equal distances, (dist, id) order
    ctx.prepare_vectors(X)
    ids, dist, stats = ctx.group_knn([5], [n], list_k)
    oi, od = oracle.intra_exact(X, 5, n, list_k)
    _assert_rows_equal(ids, dist, None, oi, od, None, f"intra n={n}")


@pytest.mark.parametrize("dim,k", [(128, 6), (24, 16)])
def test_cross_integer_ties(ctx, oracle, dim, k):
    """Coordinates in {0, 1, 2}: many candidates share the k-th distance exactly, so the
    (dist, id) order decides and no candidate at the k-th distance may be left out of
    the exact re-score."""
    rng = np.random.default_rng(dim + k)
    _say(f"cross integer ties dim={dim} k={k}")
    _, gb, op, oi = _two_level_problem(rng, [40, 130, 7], [300, 2, 129, 50], dim)
    X = rng.integers(0, 3, size=(int(gb[-1]), dim)).astype(np.float32)
    ctx.prepare_vectors(X)
    ids, dist, size, stats = ctx.cross_topk(gb, op, oi, k)
    ip, ii = F.in_neighbors(op, oi)
    o_ids, o_d, o_s = oracle.cross_exact(X, gb, ip, ii, k)
    _assert_rows_equal(ids, dist, size, o_ids, o_d, o_s, f"integer ties dim={dim} k={k}")


@pytest.mark.parametrize("n,list_k,dim", [(300, 32, 128), (150, 8, 16)])
def test_intra_integer_ties(ctx, oracle, n, list_k, dim):
    rng = np.random.default_rng(n + dim)
    _say(f"intra integer ties n={n} k={list_k} dim={dim}")
    X = rng.integers(0, 3, size=(n + 10, dim)).astype(np.float32)
    ctx.prepare_vectors(X)
    ids, dist, stats = ctx.group_knn([5], [n], list_k)
    oi, od = oracle.intra_exact(X, 5, n, list_k)
    _assert_rows_equal(ids, dist, None, oi, od, None, f"intra integer ties n={n}")


def test_cross_many_lists(ctx, oracle):
    """An LNG with more than 2^18 out-list entries, groups without points among the
    targets, and an out-of-range entry rejected."""
    rng = np.random.default_rng(77)
    G = 4000
    sizes = rng.integers(0, 4, size=G)  # some groups without points
    gb = np.zeros(G + 2, np.uint32)
    gb[2:] = np.cumsum(sizes)
    rows = [np.sort(rng.choice(np.setdiff1d(np.arange(1, G + 1), [c]), size=70, replace=False))
            for c in range(1, G + 1)]
    op = np.zeros(G + 2, np.uint32)
    op[2:] = np.cumsum([len(r) for r in rows])
    oi = np.concatenate(rows).astype(np.uint32)
    assert len(oi) >= (1 << 18)
    X = rng.standard_normal((int(gb[-1]), 16)).astype(np.float32)
    _say(f"cross many lists G={G} entries={len(oi)}")
    ctx.prepare_vectors(X)
    ids, dist, size, stats = ctx.cross_topk(gb, op, oi, 6)
    ip, ii = F.in_neighbors(op, oi)
    o_ids, o_d, o_s = oracle.cross_exact(X, gb, ip, ii, 6)
    _assert_rows_equal(ids, dist, size, o_ids, o_d, o_s, "many lists")
    with pytest.raises(F.UngHipError):
        bad = oi.copy()
        c = int(np.nonzero(sizes)[0][-1]) + 1  # the last group with points reads its list
        bad[int(op[c]) + 3] = G + 1
        ctx.cross_topk(gb, op, bad, 6)


def test_errors(ctx):
    X = np.zeros((10, 8), np.float32)
    ctx.prepare_vectors(X)
    gb = np.array([0, 0, 5, 10], np.uint32)
    op = np.array([0, 0, 1, 1], np.uint32)
    oi = np.array([2], np.uint32)
    with pytest.raises(F.UngHipError) as e:
        ctx.cross_topk(gb, op, oi, 0)
    assert e.value.code == -1
    with pytest.raises(F.UngHipError):
        ctx.cross_topk(gb, op, oi, 65)
    with pytest.raises(F.UngHipError):
        ctx.cross_topk(np.array([0, 0, 5, 9], np.uint32), op, oi, 6)  # N mismatch
    with pytest.raises(F.UngHipError):
        ctx.group_knn([8], [5], 4)  # out of range
    ctx.release_vectors()
    with pytest.raises(F.UngHipError) as e:
        ctx.cross_topk(gb, op, oi, 6)
    assert e.value.code == -3


def test_cfg2_scaled_parity(ctx, oracle):
    """cfg2's generator at 60k points: cross + intra, bit-exact."""
    cfg = D.scaled(D.CONFIGS["cfg2"], 60_000)
    X, lp, li = D.generate(cfg)
    st = F.UngBuildStage()
    st.prepare_inputs(X, lp, li)
    ctx.prepare_vectors(st.base)
    _say("cfg2@60k cross")
    ids, dist, size, stats = ctx.cross_topk(st.group_begin, st.out_ptr, st.out_idx, 6)
    _say(f"stats {stats}")
    oi, od, os_ = oracle.cross_exact(st.base, st.group_begin, st.in_ptr, st.in_idx, 6)
    _assert_rows_equal(ids, dist, size, oi, od, os_, "cfg2@60k cross")
    gids = st.mid_groups()
    begins = st.group_begin[gids]
    sizes = st.group_begin[gids + 1] - begins
    _say(f"cfg2@60k intra {len(gids)} groups")
    ids, dist, stats = ctx.group_knn(begins, sizes, 32)
    row = 0
    for b, n in zip(begins, sizes):
        o_i, o_d = oracle.intra_exact(st.base, int(b), int(n), 32)
        _assert_rows_equal(ids[row: row + n], dist[row: row + n], None, o_i, o_d, None, f"cfg2@60k intra {b}")
        row += n


# ---------------------------------------------------------------- additional edges
def _assert_edges_equal(got, want, what):
    for name, a, b in zip(("edge_ptr", "edge_from", "edge_to"), got[:3], want):
        assert np.array_equal(a, b), f"{what}: {name} differs"


def test_additional_edges_cfg1(ctx, cfg1_stage, oracle):
    st = cfg1_stage
    ctx.prepare_vectors(st.base)
    ids, _, _, _ = ctx.cross_topk(st.group_begin, st.out_ptr, st.out_idx, 6)
    got = ctx.additional_edges(st.group_begin, st.out_ptr, st.out_idx, 6)
    _say(f"additional cfg1: {got[1].size} edges, stats {got[3]}")
    want = oracle.additional_edges(st.base, st.group_begin, st.out_ptr, st.out_idx, ids, 6)
    assert got[1].size > 0
    _assert_edges_equal(got, want, "cfg1 additional")


@pytest.mark.parametrize("k", [6, 7, 2, 1])
def test_additional_edges_closed_form_problem(ctx, oracle, k):
    from test_oracle import _addl_problem
    X, gb, op, oi = _addl_problem(np.random.default_rng(3))
    ctx.prepare_vectors(X)
    ids, _, _, _ = ctx.cross_topk(gb, op, oi, k)
    got = ctx.additional_edges(gb, op, oi, k)
    want = oracle.additional_edges(X, gb, op, oi, ids, k)
    _assert_edges_equal(got, want, f"closed-form problem k={k}")
    assert (got[1].size == 0) == (k < 2)


@pytest.mark.parametrize("nx", [7, 8, 5, 1])
def test_additional_edges_small_target_k64(ctx, oracle, nx):
    """k = 64 and a target group of nx <= 8 vectors that no cross edge reaches: the entry
    scores m * nx = ceil(64 / nx) * nx (up to 70) (query row, vector) pairs in one wave,
    the most the small-target kernel takes."""
    rng = np.random.default_rng(40 + nx)
    nc, n1, d = 70, 100, 16
    X = np.concatenate([rng.standard_normal((nc + n1, d)) * 0.1,
                        rng.standard_normal((nx, d)) * 0.1 + 50.0]).astype(np.float32)
    gb = np.array([0, 0, nc, nc + n1, nc + n1 + nx], np.uint32)
    op = np.array([0, 0, 2, 2, 2], np.uint32)
    oi = np.array([2, 3], np.uint32)  # C -> (the near group, the far small group)
    ctx.prepare_vectors(X)
    ids, _, _, _ = ctx.cross_topk(gb, op, oi, 64)
    got = ctx.additional_edges(gb, op, oi, 64)
    want = oracle.additional_edges(X, gb, op, oi, ids, 64)
    m = min(nc, -(-64 // nx))
    _say(f"small target nx={nx}: {got[1].size} edges ({m} query rows)")
    assert got[1].size == m * nx
    _assert_edges_equal(got, want, f"small target nx={nx} k=64")


def test_additional_edges_errors(ctx):
    X = np.zeros((10, 8), np.float32)
    ctx.prepare_vectors(X)
    gb = np.array([0, 0, 5, 10], np.uint32)
    op = np.array([0, 0, 1, 1], np.uint32)
    oi = np.array([2], np.uint32)
    with pytest.raises(F.UngHipError) as e:
        ctx.additional_edges(gb, op, oi, 6)  # no cross edges computed for these vectors
    assert e.value.code == -3
    ctx.cross_topk(gb, op, oi, 4)
    with pytest.raises(F.UngHipError) as e:
        ctx.additional_edges(gb, op, oi, 5)  # more than the k of the cross call
    assert e.value.code == -1


def test_additional_edges_cfg2_scaled(ctx, oracle):
    cfg = D.scaled(D.CONFIGS["cfg2"], 60_000)
    X, lp, li = D.generate(cfg)
    st = F.UngBuildStage()
    st.prepare_inputs(X, lp, li)
    ctx.prepare_vectors(st.base)
    ids, _, _, _ = ctx.cross_topk(st.group_begin, st.out_ptr, st.out_idx, 6)
    got = ctx.additional_edges(st.group_begin, st.out_ptr, st.out_idx, 6)
    want = oracle.additional_edges(st.base, st.group_begin, st.out_ptr, st.out_idx, ids, 6)
    _say(f"additional cfg2@60k: {got[1].size} edges")
    _assert_edges_equal(got, want, "cfg2@60k additional")


def test_pipeline_graph_cfg1(cfg1_stage, oracle, tmp_path):
    """The stage end to end on cfg1: cross edges, additional edges and the exact-anchor
    batch on the GPU, assembled into the final CSR and saved as Graph::save text; the
    same graph from the oracle's cross and additional edges (intra rows: the packed rows,
    checked against the oracle by test_pack_cfg1_matches_oracle)."""
    import copy
    st = copy.copy(cfg1_stage)
    st._ctx = None
    st.gpu_prepare_all_vectors_on_device()
    st.gpu_cross_groups_search_all_batched()
    st.build_cross_edges_generate_additional()
    batch = st.build_fast_exact_batch()
    N = int(st.group_begin[-1])
    gids = st.mid_groups()
    deg = np.zeros(N, np.int64)
    rows = {}
    r = 0
    for g in gids:
        b, n = int(st.group_begin[g]), int(st.group_begin[g + 1] - st.group_begin[g])
        for j in range(n):
            row = batch.packed_graph[r + j]
            rows[b + j] = row[1: 1 + row[0]]
            deg[b + j] = row[0]
        r += n
    ip = np.zeros(N + 1, np.uint64)
    ip[1:] = np.cumsum(deg)
    ii = np.concatenate([rows[i] for i in sorted(rows)]).astype(np.uint32)
    rp, ci = st.build_csr_adjacency(ip, ii)
    cross, _, _ = oracle.cross_exact(st.base, st.group_begin, st.in_ptr, st.in_idx, 6)
    add = oracle.additional_edges(st.base, st.group_begin, st.out_ptr, st.out_idx, cross, 6)
    wrp, wci = oracle.assemble_graph(N, st.group_begin, ip, ii, False, cross, 6, *add)
    assert np.array_equal(rp, wrp) and np.array_equal(ci, wci)
    st.save_graph(tmp_path / "graph")
    assert (tmp_path / "graph").read_bytes().count(b"\n") == N
    st.close()


def test_pipeline_equality_scenario_cfg1(oracle):
    """The "equality" scenario end to end on cfg1 (src/uni_nav_graph.cpp:95-99): the
    cross-edge call returns padding rows only, there are no additional edges, and the graph
    holds the intra rows with add_offset only."""
    from filtervectorcode_refactor_amd import datasets as D
    X, lp, li = D.generate(D.CONFIGS["cfg1"])
    st = F.UngBuildStage(scenario="equality")
    st.prepare_inputs(X, lp, li)
    st.gpu_prepare_all_vectors_on_device()
    ids, dist, size = st.gpu_cross_groups_search_all_batched()
    assert (ids == 0xFFFFFFFF).all() and np.isinf(dist).all() and not size.any()
    ptr_, ef, et = st.build_cross_edges_generate_additional()
    assert ef.size == 0 and et.size == 0 and not ptr_.any()
    batch = st.build_fast_exact_batch()
    N = int(st.group_begin[-1])
    deg = np.zeros(N, np.int64)
    rows = {}
    r = 0
    for g in st.mid_groups():
        b, n = int(st.group_begin[g]), int(st.group_begin[g + 1] - st.group_begin[g])
        for j in range(n):
            row = batch.packed_graph[r + j]
            rows[b + j] = row[1: 1 + row[0]]
            deg[b + j] = row[0]
        r += n
    ip = np.zeros(N + 1, np.uint64)
    ip[1:] = np.cumsum(deg)
    ii = np.concatenate([rows[i] for i in sorted(rows)]).astype(np.uint32)
    rp, ci = st.build_csr_adjacency(ip, ii)
    wrp, wci = oracle.assemble_graph(N, st.group_begin, ip, ii, False, None, 0, None, None, None)
    assert np.array_equal(rp, wrp) and np.array_equal(ci, wci)
    st.close()


def test_cross_intra_overlapped_equals_sequential(ctx, oracle):
    """ung_hip_cross_intra_begin / ung_hip_intra_end (cross edges and the mid groups' kNN
    on two streams, additional edges in between) give the rows of the sequential calls,
    and calls that would touch the running group call are refused until it ends."""
    cfg = D.scaled(D.CONFIGS["cfg2"], 60_000)
    X, lp, li = D.generate(cfg)
    st = F.UngBuildStage()
    st.prepare_inputs(X, lp, li)
    ctx.prepare_vectors(st.base)
    gids = st.mid_groups().astype(np.int64)
    b = st.group_begin[gids].astype(np.uint32)
    n = (st.group_begin[gids + 1] - st.group_begin[gids]).astype(np.uint32)
    _say(f"overlapped cross + intra: {len(gids)} mid groups")
    c_ids, c_dist, c_size, _ = ctx.cross_topk(st.group_begin, st.out_ptr, st.out_idx, 6)
    want_add = ctx.additional_edges(st.group_begin, st.out_ptr, st.out_idx, 6)
    g_ids, g_dist, _ = ctx.group_knn(b, n, 32)
    for rep in range(2):
        ctx.cross_intra_begin(st.group_begin, st.out_ptr, st.out_idx, 6, b, n, 32)
        with pytest.raises(F.UngHipError):
            ctx.prepare_vectors(st.base)
        with pytest.raises(F.UngHipError):
            ctx.group_knn(b[:1], n[:1], 32)
        got_add = ctx.additional_edges(st.group_begin, st.out_ptr, st.out_idx, 6)
        ids, dist, size, _ = ctx.download_cross(st.base.shape[0], 6)
        stats = ctx.intra_end()
        assert stats["rows"] == int(n.sum())
        with pytest.raises(F.UngHipError):
            ctx.intra_end()
        check_ids, check_dist, _ = ctx.download_group(g_ids.shape[0], 32)
        assert np.array_equal(ids, c_ids) and np.array_equal(dist, c_dist) and np.array_equal(size, c_size)
        for a, w in zip(got_add[:3], want_add[:3]):
            assert np.array_equal(a, w)
        assert np.array_equal(check_ids, g_ids) and np.array_equal(check_dist, g_dist)
    # an invalid group list or list_k is refused by the host checks before anything is
    # enqueued (no call is left in flight); the next overlapped call gives the same rows
    bad_n = n.copy()
    bad_n[0] = 0
    for bad_sizes, bad_k in ((bad_n, 32), (n, 0), (n, 65)):
        with pytest.raises(F.UngHipError) as e:
            ctx.cross_intra_begin(st.group_begin, st.out_ptr, st.out_idx, 6, b, bad_sizes, bad_k)
        assert e.value.code == -1
        with pytest.raises(F.UngHipError) as e:
            ctx.intra_end()
        assert e.value.code == -3
    # the resident cross rows of the last complete call are still there
    ids, dist, size, _ = ctx.download_cross(st.base.shape[0], 6)
    assert np.array_equal(ids, c_ids) and np.array_equal(dist, c_dist) and np.array_equal(size, c_size)
    ctx.cross_intra_begin(st.group_begin, st.out_ptr, st.out_idx, 6, b, n, 32)
    ids, dist, size, _ = ctx.download_cross(st.base.shape[0], 6)
    ctx.intra_end()
    check_ids, check_dist, _ = ctx.download_group(g_ids.shape[0], 32)
    assert np.array_equal(ids, c_ids) and np.array_equal(dist, c_dist) and np.array_equal(size, c_size)
    assert np.array_equal(check_ids, g_ids) and np.array_equal(check_dist, g_dist)
    # the cross rows also equal the oracle's on a sample (the sequential call is pinned elsewhere)
    pg = st.new_vec_id_to_group_id
    q = np.arange(0, st.base.shape[0], 97, dtype=np.uint32)
    res = oracle.cross_exact_points(st.base, st.group_begin, pg, st.out_ptr, st.out_idx, q, 6)
    _assert_rows_equal(ids[q], dist[q], None, res[0], res[1], None, "overlapped cross sample")
