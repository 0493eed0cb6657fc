"""GPU test of ung_hip_cross_topk_noalloc, the cross-edge entry point that allocates
nothing (its work lists, partial rows and flags live in a file-scope device array of
UNG_HIP_NOALLOC_SCRATCH_BYTES per GPU).  Every call goes through the C ABI; the rows are
compared bit for bit with those of the allocating entry point ung_hip_cross_topk_device on
the same inputs: a call, then a call with a smaller input (fewer jobs: the array keeps the
first call's contents), then the first input again; plus the host-side refusals (a plan
larger than the array, host memory as output) that run no kernel."""
import ctypes as C

import numpy as np
import pytest

import filtervectorcode_refactor_amd as F
from filtervectorcode_refactor_amd import datasets as D

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20


class DeviceRows:
    """Caller-owned device buffers for N rows of k (hipMalloc through ctypes)."""

    def __init__(self, hip, N, k):
        self.hip, self.N, self.k = hip, N, k
        self.ptrs = []
        for nbytes in (N * k * 4, N * k * 4, N * 4):
            p = C.c_void_p()
            assert hip.hipMalloc(C.byref(p), C.c_size_t(max(nbytes, 4))) == 0
            self.ptrs.append(p)

    def addrs(self):
        return [p.value for p in self.ptrs]

    def download(self):
        ids = np.empty((self.N, self.k), np.uint32)
        dist = np.empty((self.N, self.k), np.float32)
        size = np.empty(self.N, np.int32)
        for host, dev in zip((ids, dist, size), self.ptrs):
            assert self.hip.hipMemcpy(host.ctypes.data_as(C.c_void_p), dev, C.c_size_t(host.nbytes), 2) == 0
        return ids, dist, size

    def free(self):
        for p in self.ptrs:
            self.hip.hipFree(p)
        self.ptrs = []


def _say(msg):
    print(msg, flush=True)


def _restricted(out_ptr, out_idx, keep_every):
    """The LNG with only every keep_every-th group's row (fewer jobs, same base set)."""
    G = out_ptr.shape[0] - 2
    rows = [out_idx[out_ptr[c]: out_ptr[c + 1]] if c % keep_every == 0 else out_idx[:0] for c in range(1, G + 1)]
    op = np.zeros(G + 2, np.uint32)
    op[2:] = np.cumsum([len(r) for r in rows])
    return op, (np.concatenate(rows) if op[-1] else np.zeros(0, np.uint32)).astype(np.uint32)


def _expect(ctx, gb, op, oi, k):
    ctx.cross_topk_device(gb, op, oi, k)
    ids, dist, size, _ = ctx.download_cross()
    return ids, dist, size


def _check(got, want, what):
    ids, dist, size = got
    wids, wdist, wsize = want
    bad = np.nonzero((ids != wids).any(axis=1))[0]
    assert bad.size == 0, f"{what}: {bad.size} rows differ, first {bad[:3]}"
    assert np.array_equal(dist.view(np.uint32), wdist.view(np.uint32)), f"{what}: distances"
    assert np.array_equal(size, wsize), f"{what}: sizes"


def test_noalloc_matches_allocating_entry_point():
    hip = C.CDLL("libamdhip64.so")
    X, lp, li = D.generate(D.scaled(D.CONFIGS["cfg2"], 60_000))
    st = F.UngBuildStage()
    st.prepare_inputs(X, lp, li)
    N, k = st.base.shape[0], 6
    gb, op, oi = st.group_begin, st.out_ptr, st.out_idx
    op2, oi2 = _restricted(op, oi, 3)
    with F.HipContext(0) as ctx:
        ctx.prepare_vectors(st.base)  # set-up (allocates)
        want1 = _expect(ctx, gb, op, oi, k)
        want2 = _expect(ctx, gb, op2, oi2, k)
        rows = DeviceRows(hip, N, k)
        try:
            _say(f"noalloc call 1: {len(oi)} LNG entries")
            s1 = ctx.cross_topk_noalloc(gb, op, oi, k, *rows.addrs())
            _check(rows.download(), want1, "noalloc call 1")
            _say(f"noalloc call 2 (smaller): {len(oi2)} LNG entries")
            s2 = ctx.cross_topk_noalloc(gb, op2, oi2, k, *rows.addrs())
            assert s2["rows"] < s1["rows"] and s2["pairs"] < s1["pairs"]
            _check(rows.download(), want2, "noalloc call 2")
            _say("noalloc call 3 (first input again)")
            ctx.cross_topk_noalloc(gb, op, oi, k, *rows.addrs())
            _check(rows.download(), want1, "noalloc call 3")
        finally:
            rows.free()


def test_noalloc_wide_rows():
    """d = 520: partial rows keep the wider margin past k (16 entries for k = 6), so the
    scratch array holds longer rows; two calls, the second on a smaller LNG."""
    hip = C.CDLL("libamdhip64.so")
    rng = np.random.default_rng(5)
    sizes = [300, 40, 2000, 900, 7]
    gb = np.zeros(len(sizes) + 2, np.uint32)
    gb[2:] = np.cumsum(sizes)
    op = np.array([0, 0, 2, 4, 5, 5, 5], np.uint32)   # 1 -> {3, 4}, 2 -> {3, 5}, 3 -> {5}
    oi = np.array([3, 4, 3, 5, 5], np.uint32)
    op2 = np.array([0, 0, 1, 1, 1, 1, 1], np.uint32)  # 1 -> {3}
    oi2 = np.array([3], np.uint32)
    X = rng.standard_normal((int(gb[-1]), 520)).astype(np.float32)
    k = 6
    with F.HipContext(0) as ctx:
        ctx.prepare_vectors(X)
        want1 = _expect(ctx, gb, op, oi, k)
        want2 = _expect(ctx, gb, op2, oi2, k)
        rows = DeviceRows(hip, X.shape[0], k)
        try:
            _say("noalloc d=520 call 1")
            s1 = ctx.cross_topk_noalloc(gb, op, oi, k, *rows.addrs())
            _check(rows.download(), want1, "noalloc d=520 call 1")
            _say("noalloc d=520 call 2 (smaller)")
            s2 = ctx.cross_topk_noalloc(gb, op2, oi2, k, *rows.addrs())
            assert s2["pairs"] < s1["pairs"]
            _check(rows.download(), want2, "noalloc d=520 call 2")
        finally:
            rows.free()


def test_noalloc_rescan_and_k64():
    """Every row through the exact rescan (a certification bound widened 1e30-fold) with
    unions of several ranges, and k = 64 (the longest partial rows)."""
    import os
    hip = C.CDLL("libamdhip64.so")
    rng = np.random.default_rng(3)
    sizes = [300, 40, 70000, 900]           # children 1, 2; targets 3, 4
    gb = np.zeros(len(sizes) + 2, np.uint32)
    gb[2:] = np.cumsum(sizes)
    op = np.array([0, 0, 2, 3, 3, 3], np.uint32)
    oi = np.array([3, 4, 4], np.uint32)
    X = rng.standard_normal((int(gb[-1]), 24)).astype(np.float32)
    X[gb[3]: gb[3] + 5] = X[0:5]            # exact duplicates across groups: ties by id
    old = os.environ.get("UNG_HIP_EPS_SCALE")
    os.environ["UNG_HIP_EPS_SCALE"] = "1e30"
    try:
        ctx = F.HipContext(0)
    finally:
        if old is None:
            del os.environ["UNG_HIP_EPS_SCALE"]
        else:
            os.environ["UNG_HIP_EPS_SCALE"] = old
    try:
        ctx.prepare_vectors(X)
        for k in (6, 64):
            want = _expect(ctx, gb, op, oi, k)
            rows = DeviceRows(hip, X.shape[0], k)
            try:
                s = ctx.cross_topk_noalloc(gb, op, oi, k, *rows.addrs())
                assert s["fallback_rows"] == 340
                _check(rows.download(), want, f"noalloc rescan k={k}")
            finally:
                rows.free()
    finally:
        ctx.close()


def test_noalloc_refusals():
    """Host-side refusals: a plan larger than the scratch array, host memory as output;
    nothing is launched, and a valid call afterwards still gives the right rows."""
    hip = C.CDLL("libamdhip64.so")
    rng = np.random.default_rng(4)
    sizes = [120_000, 2000]                 # k = 64: 120k partial rows of 80 entries > 64 MiB
    gb = np.zeros(4, np.uint32)
    gb[2:] = np.cumsum(sizes)
    op = np.array([0, 0, 1, 1], np.uint32)
    oi = np.array([2], np.uint32)
    X = rng.standard_normal((int(gb[-1]), 8)).astype(np.float32)
    with F.HipContext(0) as ctx:
        ctx.prepare_vectors(X)
        rows = DeviceRows(hip, X.shape[0], 64)
        try:
            with pytest.raises(F.UngHipError) as e:
                ctx.cross_topk_noalloc(gb, op, oi, 64, *rows.addrs())
            assert e.value.code == -1 and "scratch" in str(e.value)
            host = np.zeros((X.shape[0], 64), np.uint32)
            a = rows.addrs()
            with pytest.raises(F.UngHipError) as e:
                ctx.cross_topk_noalloc(gb, op, oi, 6, host.ctypes.data, a[1], a[2])
            assert e.value.code == -1
            # a fitting call on the same context (k = 6: 10 entries a partial row)
            want = _expect(ctx, gb, op, oi, 6)
            rows6 = DeviceRows(hip, X.shape[0], 6)
            try:
                ctx.cross_topk_noalloc(gb, op, oi, 6, *rows6.addrs())
                _check(rows6.download(), want, "noalloc after refusals")
            finally:
                rows6.free()
        finally:
            rows.free()
