"""The certificate's error model checked on the hardware: every candidate a select kernel
kept in a partial row carries its approximate squared distance a (split-bf16 MFMA,
expansion form |q|^2 + |x|^2 - 2<q,x>), and the merge certifies rows with
|a - D| <= eps_coef * (|q| + R)^2 for the exact squared distance D.  Here a comes back
through ung_hip_debug_partial_rows and D is computed in fp64 from the fp32 inputs, for
every entry, on data chosen for cancellation (tight clusters far from the origin), mixed
coordinate magnitudes, integer ties and three dimensions (the register-query layout at
d = 128 and the restaged panels at 384 and 768).

The group kNN calls' selects are checked the same way, and so is the other half of the
partial-row contract: every candidate of a row's split that the row does not hold has
a >= the row's bound (ung_hip_debug_partial_bounds), so its exact distance is at least
bound - eps.  That is the filter-and-buffer select's pre-filter and threshold at
d <= 128 (ung_knn_select_kernel) and the register-queue select with self-exclusion at
d = 384."""
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


def _random_lng(rng, sizes):
    """group_begin / out_ptr / out_idx of groups of the given sizes, each with 1..5
    random out-groups."""
    G = len(sizes)
    gb = np.concatenate([[0, 0], np.cumsum(sizes)]).astype(np.uint32)
    rows = [sorted(rng.choice([x for x in range(1, G + 1) if x != g], size=int(rng.integers(1, 6)),
                              replace=False).tolist()) for g in range(1, G + 1)]
    op = np.zeros(G + 2, np.uint32)
    op[2:] = np.cumsum([len(r) for r in rows])
    oi = np.array([x for r in rows for x in r], np.uint32)
    return gb, op, oi


def _check_bound(ctx, X, gb, op, oi, label):
    ctx.prepare_vectors(X)
    _, _, _, st = ctx.cross_topk(gb, op, oi, 6)
    q, c, a, eps_coef, rmax = ctx.debug_partial_rows()
    assert q.size > 0, f"{label}: no partial-row entries"
    Xd = X.astype(np.float64)
    # the kernel's per-query term: |q| from the cached fp32 |q|^2 (fp64 sum rounded once)
    qn32 = (Xd * Xd).sum(axis=1).astype(np.float32).astype(np.float64)
    assert rmax >= np.sqrt((Xd * Xd).sum(axis=1)).max() * (1 - 1e-7), f"{label}: R below the largest norm"
    worst, worst_i = 0.0, -1
    ratios = []
    for s in range(0, q.size, 200_000):
        qs, cs = q[s:s + 200_000].astype(np.int64), c[s:s + 200_000].astype(np.int64)
        dexact = ((Xd[qs] - Xd[cs]) ** 2).sum(axis=1)
        eps = eps_coef * (np.sqrt(qn32[qs] * (1.0 + 1e-6)) + rmax) ** 2
        r = np.abs(a[s:s + 200_000].astype(np.float64) - dexact) / eps
        ratios.append(r)
        i = int(np.argmax(r))
        if r[i] > worst:
            worst, worst_i = float(r[i]), s + i
    ratios = np.concatenate(ratios)
    _say(f"{label}: {q.size} entries, rescanned rows {st['fallback_rows']}, |a - D| / eps max {worst:.3g}, "
         f"99.9 % {np.quantile(ratios, 0.999):.3g}, median {np.median(ratios):.3g}")
    assert worst <= 1.0, (f"{label}: entry {worst_i} (query {q[worst_i]}, candidate {c[worst_i]}) has "
                          f"|a - D| = {worst:.3g} eps")
    return ratios


def test_bound_cfg2_slice(ctx):
    X, lp, li = D.generate(D.scaled(D.CONFIGS["cfg2"], 40_000))
    st = F.UngBuildStage()
    st.prepare_inputs(X, lp, li)
    _check_bound(ctx, st.base, st.group_begin, st.out_ptr, st.out_idx, "cfg2 slice (d=128)")


@pytest.mark.parametrize("d", [128, 384, 768])
def test_bound_far_clusters(ctx, d):
    """Tight clusters (spread 0.05) around centres of norm 100: distances of order 1
    against norms of order 10^4, the expansion form's worst cancellation."""
    rng = np.random.default_rng(100 + d)
    sizes = rng.choice([3, 40, 200, 700], size=30)
    gb, op, oi = _random_lng(rng, sizes)
    N = int(gb[-1])
    centres = rng.standard_normal((4, d))
    centres *= 100.0 / np.linalg.norm(centres, axis=1, keepdims=True)
    X = (centres[rng.integers(0, 4, size=N)] + 0.05 * rng.standard_normal((N, d))).astype(np.float32)
    _check_bound(ctx, X, gb, op, oi, f"far clusters d={d}")


def test_bound_mixed_magnitudes(ctx):
    """Coordinates of very different scales within a vector (1e3 to 1e-3)."""
    rng = np.random.default_rng(7)
    d = 128
    sizes = rng.choice([5, 60, 300, 900], size=25)
    gb, op, oi = _random_lng(rng, sizes)
    N = int(gb[-1])
    scale = 10.0 ** rng.uniform(-3, 3, size=d)
    X = (rng.standard_normal((N, d)) * scale).astype(np.float32)
    _check_bound(ctx, X, gb, op, oi, "mixed magnitudes")


def test_bound_integer_ties(ctx):
    rng = np.random.default_rng(8)
    sizes = rng.choice([4, 50, 400], size=30)
    gb, op, oi = _random_lng(rng, sizes)
    X = rng.integers(-4, 5, size=(int(gb[-1]), 96)).astype(np.float32)
    _check_bound(ctx, X, gb, op, oi, "integer data")


def _check_left_out(ctx, X, label, eps_coef, rmax, q, c):
    """Every candidate of a partial row's split that the row does not hold (the query
    itself aside) has an exact distance >= bound - eps: exact distances of whole groups
    from fp64 Gram matrices.  Rows of multi-range unions are skipped."""
    qb, b0, b1, bd = ctx.debug_partial_bounds()
    assert qb.size > 0, f"{label}: no partial rows"
    one = b0 != 0xFFFFFFFF
    Xd = X.astype(np.float64)
    qn32 = (Xd * Xd).sum(axis=1).astype(np.float32).astype(np.float64)
    held = {}
    for qq, cc in zip(q.tolist(), c.tolist()):
        held.setdefault(qq, []).append(cc)
    checked, worst = 0, -np.inf
    ranges = np.unique(np.stack([b0[one], b1[one]], axis=1), axis=0)
    for lo, hi in ranges.tolist():
        rows = np.nonzero(one & (b0 == lo) & (b1 == hi))[0]
        Y = Xd[lo:hi]
        yn = (Y * Y).sum(axis=1)
        for s in range(0, rows.size, 512):
            rs = rows[s:s + 512]
            Q = Xd[qb[rs].astype(np.int64)]
            D = (Q * Q).sum(axis=1)[:, None] + yn[None, :] - 2.0 * (Q @ Y.T)
            for j, r in enumerate(rs.tolist()):
                mask = np.ones(hi - lo, bool)
                qq = int(qb[r])
                if lo <= qq < hi:
                    mask[qq - lo] = False
                for cc in held.get(qq, []):
                    if lo <= cc < hi:
                        mask[cc - lo] = False
                if not mask.any() or not np.isfinite(bd[r]):
                    continue
                eps = eps_coef * (np.sqrt(qn32[qq] * (1.0 + 1e-6)) + rmax) ** 2
                # (bound - D) / eps must stay below 1 (D from a Gram matrix: fp64
                # cancellation far below eps)
                v = float((float(bd[r]) - D[j][mask].min()) / eps)
                worst = max(worst, v)
                checked += 1
                assert v <= 1.0, (f"{label}: query {qq}, split [{lo}, {hi}): a left-out candidate has exact "
                                  f"distance {D[j][mask].min():.9g} < bound {bd[r]:.9g} - eps")
    _say(f"{label}: {checked} rows' left-out candidates checked, (bound - min D) / eps max {worst:.3g}")
    return checked


def _check_group(ctx, X, begins, sizes, K, label):
    ctx.prepare_vectors(X)
    st = ctx.group_knn_device(begins, sizes, K)
    q, c, a, eps_coef, rmax = ctx.debug_partial_rows()
    assert q.size > 0, f"{label}: no partial-row entries"
    Xd = X.astype(np.float64)
    qn32 = (Xd * Xd).sum(axis=1).astype(np.float32).astype(np.float64)
    dexact = ((Xd[q.astype(np.int64)] - Xd[c.astype(np.int64)]) ** 2).sum(axis=1)
    eps = eps_coef * (np.sqrt(qn32[q.astype(np.int64)] * (1.0 + 1e-6)) + rmax) ** 2
    r = np.abs(a.astype(np.float64) - dexact) / eps
    # group jobs hold the query's own group only, without the query itself
    grp = np.searchsorted(begins.astype(np.int64), q.astype(np.int64), side="right") - 1
    assert (c.astype(np.int64) >= begins[grp]).all() and (c.astype(np.int64) < begins[grp] + sizes[grp]).all()
    assert not (q == c).any(), f"{label}: a partial row holds its own query"
    _say(f"{label}: {q.size} entries, rescanned rows {st['fallback_rows']}, |a - D| / eps max {r.max():.3g}")
    assert r.max() <= 1.0, f"{label}: |a - D| = {r.max():.3g} eps"
    assert _check_left_out(ctx, X, label, eps_coef, rmax, q, c) > 0


def test_group_bound_cfg2_mid_groups(ctx):
    """cfg2's generator: a random sample of its mid groups (the largest included) through
    the filter-and-buffer select at K = 32."""
    X, lp, li = D.generate(D.CONFIGS["cfg2"])
    st = F.UngBuildStage()
    st.prepare_inputs(X, lp, li)
    del X
    gids = st.mid_groups().astype(np.int64)
    sizes_all = (st.group_begin[gids + 1] - st.group_begin[gids]).astype(np.int64)
    rng = np.random.default_rng(11)
    pick = np.union1d(rng.choice(gids.size, size=min(60, gids.size), replace=False), [int(np.argmax(sizes_all))])
    pick = np.sort(pick)
    # the groups' points only: ids stay group-local to this smaller base set
    parts = [st.base[st.group_begin[g]: st.group_begin[g + 1]] for g in gids[pick]]
    sizes = np.array([p.shape[0] for p in parts], np.uint32)
    begins = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.uint32)
    _check_group(ctx, np.ascontiguousarray(np.concatenate(parts)), begins, sizes, 32,
                 f"cfg2 mid groups ({len(parts)} of {gids.size}, largest {int(sizes.max())})")


@pytest.mark.parametrize("d", [128, 384])
def test_group_bound_far_clusters(ctx, d):
    """Tight clusters (spread 0.05) around centres of norm 100, groups of 2 to 4096
    points, K = 32 and 6."""
    rng = np.random.default_rng(200 + d)
    sizes = np.array([2, 40, 130, 300, 1000, 2500, 4096], np.uint32)
    begins = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.uint32)
    N = int(sizes.sum())
    centres = rng.standard_normal((4, d))
    centres *= 100.0 / np.linalg.norm(centres, axis=1, keepdims=True)
    X = (centres[rng.integers(0, 4, size=N)] + 0.05 * rng.standard_normal((N, d))).astype(np.float32)
    for K in (32, 6):
        _check_group(ctx, X, begins, sizes, K, f"group far clusters d={d} K={K}")


@pytest.mark.parametrize("d", [128, 384])
def test_cross_left_out_single_targets(ctx, d):
    """The cross select's bound, checked over unions of one target group each (one
    candidate range: 150 to 70,000 candidates, the largest in three splits), on tight
    clusters far from the origin."""
    rng = np.random.default_rng(300 + d)
    sizes = [300, 900, 2000, 5000, 70000, 150, 600]
    gb = np.concatenate([[0, 0], np.cumsum(sizes)]).astype(np.uint32)
    target = {1: 5, 2: 4, 3: 5, 4: 2, 6: 5, 7: 3}           # child group -> its one out-group
    op = np.zeros(len(sizes) + 2, np.uint32)
    op[2:] = np.cumsum([1 if g in target else 0 for g in range(1, len(sizes) + 1)])
    oi = np.array([target[g] for g in range(1, len(sizes) + 1) if g in target], np.uint32)
    N = int(gb[-1])
    centres = rng.standard_normal((6, d))
    centres *= 100.0 / np.linalg.norm(centres, axis=1, keepdims=True)
    X = (centres[rng.integers(0, 6, size=N)] + 0.05 * rng.standard_normal((N, d))).astype(np.float32)
    ctx.prepare_vectors(X)
    st = ctx.cross_topk_device(gb, op, oi, 6)
    q, c, _, eps_coef, rmax = ctx.debug_partial_rows()
    _say(f"single targets d={d}: rescanned rows {st['fallback_rows']}")
    assert _check_left_out(ctx, X, f"single targets d={d}", eps_coef, rmax, q, c) >= 2450 * 3


def test_debug_rows_refused_without_partial_rows(ctx):
    """After prepare_vectors (no call yet) and after a no-allocation call (its partial
    rows live in the scratch array) the diagnostics refuse."""
    import ctypes as C
    X = np.random.default_rng(9).standard_normal((300, 16)).astype(np.float32)
    ctx.prepare_vectors(X)
    with pytest.raises(F.UngHipError):
        ctx.debug_partial_rows()
    with pytest.raises(F.UngHipError):
        ctx.debug_partial_bounds()
    ctx.group_knn_device(np.array([0], np.uint32), np.array([300], np.uint32), 8)
    q, _, _, _, _ = ctx.debug_partial_rows()
    assert q.size == 300 * 12  # list_k = 8: 12 entries a row, every one a real candidate
    hip = C.CDLL("libamdhip64.so")
    ptrs = []
    try:
        for nbytes in (300 * 6 * 4, 300 * 6 * 4, 300 * 4):
            p = C.c_void_p()
            assert hip.hipMalloc(C.byref(p), C.c_size_t(nbytes)) == 0
            ptrs.append(p)
        gb = np.array([0, 0, 100, 300], np.uint32)
        op = np.array([0, 0, 1, 1], np.uint32)
        oi = np.array([2], np.uint32)
        ctx.cross_topk_noalloc(gb, op, oi, 6, *[p.value for p in ptrs])
        with pytest.raises(F.UngHipError):
            ctx.debug_partial_rows()
        with pytest.raises(F.UngHipError):
            ctx.debug_partial_bounds()
    finally:
        for p in ptrs:
            hip.hipFree(p)
