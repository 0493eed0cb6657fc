"""GPU parity of the large-group graph (exact candidate lists + the FastGrnnd prune,
ung_hip_prune_group_graph) against the plain-C restatement ungo_large_group_graph,
bit-exact row by row: random and integer-valued data (many equal distances, exact
duplicates), several groups per call, the reference's default caps (63 forward, 32
reverse, degree 32) and a group above 32,768 points (candidates not split)."""
import numpy as np
import pytest

import filtervectorcode_refactor_amd as F

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = F.HipContext(0)
    yield c
    c.close()


def _say(msg):
    print(msg, flush=True)


def _check(ctx, oracle, X, groups, knn_k, fcap, rcap, fd, alpha, label):
    ctx.prepare_vectors(X)
    begins = np.array([b for b, _ in groups], np.uint32)
    sizes = np.array([n for _, n in groups], np.uint32)
    ctx.group_knn_device(begins, sizes, knn_k)
    rows, entries, st = ctx.prune_group_graph(int(sizes.sum()), len(groups), fcap, rcap, fd, alpha)
    assert (entries == 0).all()
    r0 = 0
    for b, n in groups:
        want = oracle.large_group_graph(X, b, n, knn_k, fcap, rcap, fd, alpha)
        got = rows[r0:r0 + n]
        bad = np.nonzero((got != want).any(1))[0]
        assert bad.size == 0, f"{label}: group ({b},{n}) row {bad[:5]}: got {got[bad[0]][:8]} want {want[bad[0]][:8]}"
        r0 += n
    return rows, st


@pytest.mark.parametrize("dim,knn_k,fcap,rcap,fd,alpha,seed", [(16, 20, 20, 8, 12, 1.2, 1), (128, 63, 63, 32, 32, 1.2, 2),
                                                               (5, 40, 30, 16, 24, 1.0, 3), (37, 63, 63, 32, 32, 1.5, 4)])
def test_prune_random(ctx, oracle, dim, knn_k, fcap, rcap, fd, alpha, seed):
    _say(f"large-group prune dim={dim} k={knn_k} caps={fcap}/{rcap} fd={fd} alpha={alpha}")
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((7000, dim)).astype(np.float32)
    X[11] = X[40]  # exact duplicate inside the first group
    _check(ctx, oracle, X, [(3, 700), (900, 4500), (5500, 300)], knn_k, fcap, rcap, fd, alpha, "random")


@pytest.mark.parametrize("dim,seed", [(768, 5), (1100, 6)])
def test_prune_large_dim(ctx, oracle, dim, seed):
    # d = 768: the candidate's row staged in LDS; d = 1100: above the staging size, every
    # distance reads both rows from memory
    _say(f"large-group prune dim={dim}")
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((1700, dim)).astype(np.float32)
    _check(ctx, oracle, X, [(3, 700), (800, 900)], 63, 63, 32, 32, 1.2, f"dim {dim}")


def test_prune_integer_ties(ctx, oracle):
    _say("large-group prune, integer data (ties)")
    rng = np.random.default_rng(11)
    X = rng.integers(-3, 4, size=(2500, 6)).astype(np.float32)
    _check(ctx, oracle, X, [(0, 2000), (2000, 500)], 63, 63, 32, 32, 1.2, "integer")


def test_prune_unsplit_big_group(ctx, oracle):
    _say("large-group prune, one group of 33,000 points (candidates not split)")
    rng = np.random.default_rng(12)
    X = rng.standard_normal((33010, 8)).astype(np.float32)
    _check(ctx, oracle, X, [(5, 33000)], 63, 63, 32, 32, 1.2, "big")


def test_prune_errors(ctx):
    rng = np.random.default_rng(13)
    X = rng.standard_normal((600, 8)).astype(np.float32)
    ctx.prepare_vectors(X)
    ctx.group_knn_device(np.array([0], np.uint32), np.array([500], np.uint32), 20)
    for args in [(21, 8, 12, 1.2), (20, 33, 12, 1.2), (20, 8, 65, 1.2), (20, 8, 0, 1.2), (0, 8, 12, 1.2),
                 (20, 8, 12, -1.0)]:
        with pytest.raises(F.UngHipError):
            ctx.prune_group_graph(500, 1, *args)


def test_stage_large_groups_cfg2_scaled(oracle):
    """UngBuildStage.build_large_group_graph on cfg2's generator at 60k points: the large
    groups' rows equal the restatement."""
    from filtervectorcode_refactor_amd import datasets as D
    _say("stage large groups cfg2 scaled")
    X, lp, li = D.generate(D.scaled(D.CONFIGS["cfg2"], 60000))
    st = F.UngBuildStage(exact_max_nx=1024)
    st.prepare_inputs(X, lp, li)
    st.ctx.prepare_vectors(st.base)
    gids = st.large_groups()
    assert len(gids) > 0
    res = st.build_large_group_graph()
    for i, g in enumerate(gids[:4]):
        b, e = int(st.group_begin[g]), int(st.group_begin[g + 1])
        want = oracle.large_group_graph(st.base, b, e - b, 63, 63, 32, 32, 1.2)
        got = res.packed_graph[res.packed_offsets[i]:res.packed_offsets[i + 1]]
        assert np.array_equal(got, want), f"group {g}"
    st.close()


def _prune_ctx(var):
    """A context with one of the prune test hooks set: UNG_HIP_PRUNE_EXACT=1 scores every
    alpha test exactly, UNG_HIP_PRUNE_GRAM=1 takes the certified Gram kernel at any d."""
    import os
    old = os.environ.get(var)
    os.environ[var] = "1"
    try:
        return F.HipContext(0)
    finally:
        if old is None:
            del os.environ[var]
        else:
            os.environ[var] = old


@pytest.mark.parametrize("kind,dim", [("far", 128), ("far", 768), ("mixed", 64), ("int", 9), ("far", 300)])
def test_prune_gram_matches_exact_scan(oracle, kind, dim):
    """The certified Gram pre-decision against the exact scan of every alpha test, row for
    row, on data that leaves many pairs undecided (tight clusters far from the origin:
    distances far below the bound's error term; coordinates of mixed magnitudes; integer
    data with exact ties at alpha * d == d), for alpha 1.2, 0, 1e30 and +inf (inf * 0 is NaN:
    a pair at distance 0 stays undecided and is scored exactly), with groups of 40 and 10
    points (rows with fewer candidates than one 32-row block of the Gram matrix), and
    against the restatement."""
    _say(f"prune gram vs exact scan: {kind} d={dim}")
    rng = np.random.default_rng(40 + dim)
    N = 3000
    if kind == "far":
        centres = rng.standard_normal((3, dim))
        centres *= 100.0 / np.linalg.norm(centres, axis=1, keepdims=True)
        X = (centres[rng.integers(0, 3, size=N)] + 0.05 * rng.standard_normal((N, dim))).astype(np.float32)
    elif kind == "mixed":
        X = (rng.standard_normal((N, dim)) * 10.0 ** rng.uniform(-3, 3, size=dim)).astype(np.float32)
    else:
        X = rng.integers(-2, 3, size=(N, dim)).astype(np.float32)
    X[2000] = X[1900]  # an exact duplicate: d(kept, candidate) = 0
    groups = [(0, 1800), (1800, 1150), (2950, 40), (2990, 10)]
    begins = np.array([b for b, _ in groups], np.uint32)
    sizes = np.array([n for _, n in groups], np.uint32)
    ex, gr = _prune_ctx("UNG_HIP_PRUNE_EXACT"), _prune_ctx("UNG_HIP_PRUNE_GRAM")
    try:
        ex.prepare_vectors(X)
        gr.prepare_vectors(X)
        for alpha in (1.2, 0.0, 1e30, np.inf):
            got = []
            for c in (gr, ex):
                c.group_knn_device(begins, sizes, 63)
                rows, _, _ = c.prune_group_graph(N, len(groups), 63, 32, 32, alpha)
                got.append(rows)
            bad = np.nonzero((got[0] != got[1]).any(1))[0]
            assert bad.size == 0, f"{kind} d={dim} alpha={alpha}: rows {bad[:5]} differ"
            if alpha == 1.2:
                want = oracle.large_group_graph(X, 0, 1800, 63, 63, 32, 32, 1.2)
                assert np.array_equal(got[0][:1800], want), f"{kind} d={dim}: restatement"
                want = oracle.large_group_graph(X, 2950, 40, 63, 63, 32, 32, 1.2)
                assert np.array_equal(got[0][2950:2990], want), f"{kind} d={dim}: restatement, 40 points"
    finally:
        ex.close()
        gr.close()
