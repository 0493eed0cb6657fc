"""The certificate's error model checked on the hardware: every candidate the cross
select kept in a partial row carries its approximate squared distance a (split-bf16
MFMA, expansion form |q|^2 + |x|^2 - 2<q,x>), and the merge certifies rows with
|a - D| <= eps_coef * (|q| + R)^2 for the exact squared distance D.  Here a comes back
through ung_hip_debug_partial_rows and D is computed in fp64 from the fp32 inputs, for
every entry, on data chosen for cancellation (tight clusters far from the origin), mixed
coordinate magnitudes, integer ties and three dimensions (the register-query layout at
d = 128 and the restaged panels at 384 and 768)."""
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


def test_debug_rows_need_a_cross_call(ctx):
    X = np.random.default_rng(9).standard_normal((300, 16)).astype(np.float32)
    ctx.prepare_vectors(X)
    ctx.group_knn_device(np.array([0], np.uint32), np.array([300], np.uint32), 8)
    with pytest.raises(F.UngHipError):
        ctx.debug_partial_rows()
