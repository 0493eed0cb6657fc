"""GPU tests of the filter-and-buffer group kNN select (ung_knn_select_kernel), the path
of every group kNN call with d <= 128 whose partial rows hold fewer than 64 entries
(list_k <= 50) and whose items scan fewer than 65,536 candidates:
  * the same lists as the register-queue select (UNG_HIP_NO_KNN=1 at context creation)
    and as the CPU oracle, on cfg2's generator and on single groups of many sizes;
  * the paths that leave a row to the certificate and the exact rescan: a bin of the
    refresh histogram holding more values than a buffer keeps (96 candidates at one
    distance), a group of exact duplicates, and candidates in decreasing distance,
    which overflow the buffer (values dropped, the threshold capped below them).
Every call goes through the C ABI."""
import os

import numpy as np
import pytest

import filtervectorcode_refactor_amd as F
from filtervectorcode_refactor_amd import datasets as D
from test_gpu_parity import _assert_rows_equal

pytestmark = pytest.mark.gpu


def _ctx(env=None):
    old = {}
    for k, v in (env or {}).items():
        old[k] = os.environ.get(k)
        os.environ[k] = v
    try:
        return F.HipContext(0)
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


@pytest.fixture(scope="module")
def knn_ctx():
    c = _ctx()
    yield c
    c.close()


@pytest.fixture(scope="module")
def queue_ctx():
    c = _ctx({"UNG_HIP_NO_KNN": "1"})
    yield c
    c.close()


def _say(msg):
    print(msg, flush=True)


def test_cfg2_mid_groups_match_register_queue_select(knn_ctx, queue_ctx, oracle):
    cfg = D.scaled(D.CONFIGS["cfg2"], 120_000)
    X, lp, li = D.generate(cfg)
    st = F.UngBuildStage()
    st.prepare_inputs(X, lp, li)
    gids = st.mid_groups().astype(np.int64)
    b = st.group_begin[gids].astype(np.uint32)
    n = (st.group_begin[gids + 1] - st.group_begin[gids]).astype(np.uint32)
    _say(f"cfg2@120k: {len(gids)} mid groups, n {n.min()}..{n.max()}")
    knn_ctx.prepare_vectors(st.base)
    queue_ctx.prepare_vectors(st.base)
    for list_k in (32, 8, 48):
        i1, d1, s1 = knn_ctx.group_knn(b, n, list_k)
        i2, d2, s2 = queue_ctx.group_knn(b, n, list_k)
        _say(f"list_k={list_k}: filter-and-buffer select {s1['select_ms']:.3f} ms ({s1['fallback_rows']} rescanned), "
             f"register queues {s2['select_ms']:.3f} ms ({s2['fallback_rows']} rescanned)")
        _assert_rows_equal(i1, d1, None, i2, d2, None, f"cfg2@120k list_k={list_k}")
    # and against the oracle on a few groups
    rng = np.random.default_rng(9)
    starts = np.concatenate([[0], np.cumsum(n.astype(np.int64))])
    i1, d1, _ = knn_ctx.group_knn(b, n, 32)
    for gi in rng.choice(len(gids), size=min(6, len(gids)), replace=False):
        oi, od = oracle.intra_exact(st.base, int(b[gi]), int(n[gi]), 32)
        r0 = int(starts[gi])
        _assert_rows_equal(i1[r0: r0 + n[gi]], d1[r0: r0 + n[gi]], None, oi, od, None, f"cfg2@120k group {gi}")


@pytest.mark.parametrize("n,list_k,dim,seed", [(129, 32, 128, 1), (300, 32, 384, 2), (1000, 16, 64, 3),
                                                (4096, 32, 128, 4), (20000, 32, 32, 5), (64, 32, 128, 6),
                                                (700, 50, 24, 7), (2, 6, 8, 8)])
def test_single_groups(knn_ctx, oracle, n, list_k, dim, seed):
    _say(f"group n={n} list_k={list_k} dim={dim}")
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n + 9, dim)).astype(np.float32)
    X[7] = X[4]  # an exact duplicate inside the group
    knn_ctx.prepare_vectors(X)
    ids, dist, _ = knn_ctx.group_knn([5], [n], list_k)
    oi, od = oracle.intra_exact(X, 5, n, list_k)
    _assert_rows_equal(ids, dist, None, oi, od, None, f"n={n} list_k={list_k}")


def test_dense_bin_overflow(knn_ctx, oracle):
    """Query 0 at the origin, 96 candidates at exactly the same distance (+-2 e_i, squared
    distance 4 in every precision) and the rest farther: the refresh histogram puts all
    96 in the bin of the query's 41st value, more than a buffer keeps, so only the bins
    below it stay (none), the bound falls to 4, the certificate fails and the exact rescan
    computes the row (ties by id)."""
    rng = np.random.default_rng(11)
    dim, n = 48, 300
    X = np.zeros((n, dim), dtype=np.float32)
    for i in range(dim):
        X[1 + 2 * i, i] = 2.0
        X[2 + 2 * i, i] = -2.0
    far = rng.standard_normal((n - 97, dim))
    far *= (5.0 + rng.random((n - 97, 1))) / np.linalg.norm(far, axis=1, keepdims=True)
    X[97:] = far.astype(np.float32)
    knn_ctx.prepare_vectors(X)
    ids, dist, st = knn_ctx.group_knn([0], [n], 32)
    _say(f"dense bin: {st['fallback_rows']} rows rescanned")
    assert st["fallback_rows"] >= 1
    assert 0 in knn_ctx.rescanned_rows(1)
    oi, od = oracle.intra_exact(X, 0, n, 32)
    _assert_rows_equal(ids, dist, None, oi, od, None, "dense bin")


def test_decreasing_order_overflow(knn_ctx, oracle):
    """Query 0 at the origin and candidate j at radius 20 - j/64: every tile's values lie
    below every earlier one, so all 128 pass the filter and the buffer overflows; the
    dropped values cap the threshold, and the row is still exact (directly or through
    the rescan)."""
    rng = np.random.default_rng(13)
    dim, n = 32, 700
    dirs = rng.standard_normal((n, dim))
    dirs /= np.linalg.norm(dirs, axis=1, keepdims=True)
    radius = 20.0 - np.arange(n) / 64.0
    X = (dirs * radius[:, None]).astype(np.float32)
    X[0] = 0.0
    knn_ctx.prepare_vectors(X)
    ids, dist, st = knn_ctx.group_knn([0], [n], 32)
    _say(f"decreasing order: {st['fallback_rows']} rows rescanned")
    oi, od = oracle.intra_exact(X, 0, n, 32)
    _assert_rows_equal(ids, dist, None, oi, od, None, "decreasing order")


def test_duplicates_lowest_bin(knn_ctx, oracle):
    """100 exact copies of one vector among 300 others: every copy's 41st value lies in the
    lowest bin (distance 0) with more than 64 values, so nothing is taken below the
    threshold and the rescan computes those rows (ties broken by id)."""
    rng = np.random.default_rng(12)
    dim = 32
    X = rng.standard_normal((400, dim)).astype(np.float32)
    X[50:150] = X[50]
    knn_ctx.prepare_vectors(X)
    ids, dist, st = knn_ctx.group_knn([0], [400], 32)
    _say(f"duplicates: {st['fallback_rows']} rows rescanned")
    assert st["fallback_rows"] >= 100
    oi, od = oracle.intra_exact(X, 0, 400, 32)
    _assert_rows_equal(ids, dist, None, oi, od, None, "duplicates")
