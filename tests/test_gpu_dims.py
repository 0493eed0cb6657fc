"""GPU parity at dimensions around the merge's LDS staging limit (query rows of group-kNN
merges staged in LDS up to d = 1024, read from global memory above) and far above it,
bit-exact against the oracle: group kNN lists (K = 32 and 64, rows of several re-score
passes) and cross edges (k = 6 and 64)."""
import numpy as np
import pytest

import filtervectorcode_refactor_amd as F
from test_gpu_parity import _assert_rows_equal, _two_level_problem

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = F.HipContext(0)
    yield c
    c.close()


@pytest.mark.parametrize("n,list_k,dim,seed", [(300, 32, 1024, 81), (300, 32, 1025, 82), (700, 32, 1100, 83),
                                               (200, 64, 2000, 84), (150, 64, 1024, 85)])
def test_group_knn_dims(ctx, oracle, n, list_k, dim, seed):
    print(f"group knn n={n} k={list_k} dim={dim}", flush=True)
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n + 9, dim)).astype(np.float32)
    X[7] = X[5]  # an exact duplicate inside the group: equal distances, ties by id
    ctx.prepare_vectors(X)
    ids, dist, stats = ctx.group_knn([4], [n], list_k)
    o_i, o_d = oracle.intra_exact(X, 4, n, list_k)
    _assert_rows_equal(ids, dist, None, o_i, o_d, None, f"group knn dim={dim}")


@pytest.mark.parametrize("dim,k,seed", [(1024, 6, 86), (1100, 6, 87), (1100, 64, 88), (2000, 20, 89)])
def test_cross_dims(ctx, oracle, dim, k, seed):
    print(f"cross dim={dim} k={k}", flush=True)
    rng = np.random.default_rng(seed)
    X, gb, op, oi = _two_level_problem(rng, [1, 3, 130, 40, 7], [4, 200, 2, 129, 70], dim, dup=True)
    ctx.prepare_vectors(X)
    ids, dist, size, _ = ctx.cross_topk(gb, op, oi, k)
    ip, ii = F.in_neighbors(op, oi)
    o_ids, o_d, o_s = oracle.cross_exact(X, gb, ip, ii, k)
    _assert_rows_equal(ids, dist, size, o_ids, o_d, o_s, f"cross dim={dim} k={k}")
