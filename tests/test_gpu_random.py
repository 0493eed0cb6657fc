"""Randomised GPU parity: small random problems across the shapes the kernels branch on,
every row compared bit for bit with the CPU oracle (which is pinned against the
reference's compiled code by test_oracle.py).

  * cross edges: dimensions 3..768 (one to twenty-four 32-dimension chunks: the
    register-query layout at 128, the restaged panels elsewhere), k from 1 to 64 (queue
    lengths 8, 16 and 32), groups of 1..700 vectors with 0..5 random out-groups (jobs
    from the exact per-job scan to several candidate splits);
  * group kNN: groups of 2..1500 vectors, K from 1 to 50 (filter-and-buffer select at
    d <= 128, register queues above, and the merge's rank paths; at d >= 256 the merge
    re-scores two candidates per lane group, checked with dimension tails of 4 to 7);
  * integer coordinates in some cases, so that exact distance ties occur.
Every call goes through the C ABI."""
import numpy as np
import pytest

import filtervectorcode_refactor_amd as F
from test_gpu_parity import _assert_rows_equal

pytestmark = pytest.mark.gpu

NONE = 0xFFFFFFFF


@pytest.fixture(scope="module")
def ctx():
    c = F.HipContext(0)
    yield c
    c.close()


def _say(msg):
    print(msg, flush=True)


def _vectors(rng, n, d, integer):
    if integer:
        return rng.integers(-3, 4, size=(n, d)).astype(np.float32)
    X = rng.standard_normal((n, d)).astype(np.float32)
    X *= np.float32(rng.choice([0.01, 1.0, 30.0]))
    return X


def _cases(n, dims, ks, seed):
    """n random (seed, d, k, integer) cases, the same on every run."""
    rng = np.random.default_rng(seed)
    return [(i + 1, int(rng.choice(dims)), int(rng.choice(ks)), bool(i % 4 == 3)) for i in range(n)]


CROSS_CASES = [  # (seed, d, k, integer coordinates)
    (1, 3, 6, False), (2, 17, 1, False), (3, 64, 16, False), (4, 128, 6, False), (5, 128, 33, True),
    (6, 130, 6, False), (7, 200, 10, True), (8, 384, 64, False), (9, 520, 6, False), (10, 96, 2, True),
] + [(s + 10, d, k, i) for s, d, k, i in
     _cases(20, [5, 24, 32, 48, 64, 127, 128, 129, 256, 300, 384, 768], [1, 3, 6, 8, 9, 16, 17, 32, 40, 64], 77)]


@pytest.mark.parametrize("seed,d,k,integer", CROSS_CASES)
def test_random_cross(ctx, oracle, seed, d, k, integer):
    rng = np.random.default_rng(1000 + seed)
    G = int(rng.integers(20, 60))
    sizes = rng.choice([1, 2, 3, 7, 16, 40, 129, 300, 700], size=G, p=[.15, .1, .1, .15, .15, .15, .1, .06, .04])
    N = int(sizes.sum())
    X = _vectors(rng, N, d, integer)
    gb = np.concatenate([[0, 0], np.cumsum(sizes)]).astype(np.uint32)
    rows = []
    for g in range(1, G + 1):
        cand = [x for x in range(1, G + 1) if x != g]
        rows.append(sorted(rng.choice(cand, size=int(rng.integers(0, 6)), replace=False).tolist()))
    op = np.zeros(G + 2, np.uint32)
    op[2:] = np.cumsum([len(r) for r in rows])
    oi = np.array([x for r in rows for x in r], np.uint32)
    _say(f"random cross seed={seed}: N={N} d={d} k={k} groups={G} lng={oi.size}")
    ctx.prepare_vectors(X)
    ids, dist, size, st = ctx.cross_topk(gb, op, oi, k)
    pg = np.repeat(np.arange(1, G + 1, dtype=np.uint32), sizes)
    o = oracle.cross_exact_points(X, gb, pg, op, oi, np.arange(N, dtype=np.uint32), k)
    _assert_rows_equal(ids, dist, None, o[0], o[1], None, f"random cross seed={seed}")
    assert np.array_equal(size, (ids != NONE).sum(axis=1)), "row sizes"


INTRA_CASES = [  # (seed, d, K, integer coordinates)
    (1, 8, 1, False), (2, 32, 8, False), (3, 100, 32, True), (4, 128, 32, False), (5, 128, 50, False),
    (6, 160, 32, False), (7, 384, 16, True), (8, 64, 50, True),
] + [(s + 8, d, k, i) for s, d, k, i in _cases(12, [7, 16, 40, 96, 128, 192, 384], [1, 2, 6, 10, 20, 32, 45, 50], 78)] + [
    # d >= 256 (two candidates per re-score pass) with 5, 4 and 7 dimensions past the last
    # block of eight; 519: the wider partial-row margin and the XCD-contiguous merge
    (21, 261, 32, False), (22, 300, 20, True), (23, 519, 32, False)]


@pytest.mark.parametrize("seed,d,K,integer", INTRA_CASES)
def test_random_group_knn(ctx, oracle, seed, d, K, integer):
    rng = np.random.default_rng(2000 + seed)
    ng = int(rng.integers(2, 7))
    n = rng.choice([2, 40, 129, 300, 900, 1500], size=ng)
    gap = rng.integers(0, 50, size=ng)  # vectors between the groups
    begins = np.cumsum(np.concatenate([[0], (n + gap)[:-1]])) + gap[0]
    N = int(begins[-1] + n[-1] + 5)
    X = _vectors(rng, N, d, integer)
    _say(f"random group kNN seed={seed}: groups {n.tolist()} d={d} K={K}")
    ctx.prepare_vectors(X)
    ids, dist, _ = ctx.group_knn(begins.astype(np.uint32), n.astype(np.uint32), K)
    r0 = 0
    for b, m in zip(begins.tolist(), n.tolist()):
        oi, od = oracle.intra_exact(X, int(b), int(m), K)
        _assert_rows_equal(ids[r0: r0 + m], dist[r0: r0 + m], None, oi, od, None,
                           f"random group kNN seed={seed} group at {b} (n={m})")
        r0 += m
