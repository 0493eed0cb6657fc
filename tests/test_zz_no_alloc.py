"""GPU test of ung_hip_cross_topk_noalloc, the cross-edge entry point that allocates
nothing (its work lists, partial rows and flags live in a file-scope device array of
UNG_HIP_NOALLOC_SCRATCH_BYTES per GPU).  Every call goes through the C ABI; the rows are
compared bit for bit with those of the allocating entry point ung_hip_cross_topk_device on
the same inputs: a call, then a call with a smaller input (fewer jobs: the array keeps the
first call's contents), then the first input again; a fresh context whose first call is
a no-allocation one; two host threads calling at once; plus the host-side refusals (a
plan larger than the array, host memory or a short buffer as output) that run no kernel.
Every no-allocation call must report ung_hip_stats::allocations == 0."""
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


def _noalloc(ctx, *args):
    """A no-allocation call whose stats must report no allocation."""
    s = ctx.cross_topk_noalloc(*args)
    assert s["allocations"] == 0, f"the no-allocation call allocated {s['allocations']} buffers"
    return s


def test_noalloc_fresh_context_first():
    """The first cross-edge call of a fresh context (nothing grown yet) is a no-allocation
    call; its rows are compared with an allocating call on a second context, which does
    allocate (the counter is live)."""
    hip = C.CDLL("libamdhip64.so")
    X, lp, li = D.generate(D.scaled(D.CONFIGS["cfg2"], 30_000))
    st = F.UngBuildStage()
    st.prepare_inputs(X, lp, li)
    N, k = st.base.shape[0], 6
    gb, op, oi = st.group_begin, st.out_ptr, st.out_idx
    rows = DeviceRows(hip, N, k)
    try:
        with F.HipContext(0) as ctx:
            up = ctx.prepare_vectors(st.base)  # set-up (allocates)
            assert up["allocations"] > 0
            _say("noalloc on a fresh context")
            s = _noalloc(ctx, gb, op, oi, k, *rows.addrs())
            assert s["rows"] > 0
            got = rows.download()
            _say("second noalloc call on the fresh context")
            _noalloc(ctx, gb, op, oi, k, *rows.addrs())
            _check(rows.download(), got, "fresh context, second call")
        with F.HipContext(0) as ref:
            ref.prepare_vectors(st.base)
            s_ref = ref.cross_topk_device(gb, op, oi, k)
            assert s_ref["allocations"] > 0  # the allocating entry point grows its buffers
            ids, dist, size, _ = ref.download_cross()
        _check(got, (ids, dist, size), "fresh context")
    finally:
        rows.free()


def test_noalloc_two_threads():
    """Two host threads, each with its own context on the same GPU, call the
    no-allocation entry point at the same time (the scratch array is per GPU: the calls
    run one after the other); both results equal the allocating entry point's."""
    import threading
    hip = C.CDLL("libamdhip64.so")
    X, lp, li = D.generate(D.scaled(D.CONFIGS["cfg2"], 40_000))
    st = F.UngBuildStage()
    st.prepare_inputs(X, lp, li)
    N, k = st.base.shape[0], 6
    inputs = [(st.group_begin, st.out_ptr, st.out_idx),
              (st.group_begin,) + _restricted(st.out_ptr, st.out_idx, 2)]
    ctxs = [F.HipContext(0), F.HipContext(0)]
    rows = [DeviceRows(hip, N, k), DeviceRows(hip, N, k)]
    try:
        wants = []
        for c, (gb, op, oi) in zip(ctxs, inputs):
            c.prepare_vectors(st.base)
            wants.append(_expect(c, gb, op, oi, k))
        errors = [None, None]
        start = threading.Barrier(2)

        def run(t):
            try:
                start.wait()
                for _ in range(3):
                    _noalloc(ctxs[t], *inputs[t], k, *rows[t].addrs())
            except Exception as e:  # reported by the main thread
                errors[t] = e

        _say("noalloc from two threads")
        th = [threading.Thread(target=run, args=(t,)) for t in range(2)]
        for t in th:
            t.start()
        for t in th:
            t.join()
        for t in range(2):
            assert errors[t] is None, f"thread {t}: {errors[t]}"
            _check(rows[t].download(), wants[t], f"thread {t}")
    finally:
        for r in rows:
            r.free()
        for c in ctxs:
            c.close()


def test_noalloc_leaves_no_cross_result():
    """After a no-allocation call the entry points that read the last cross-edge call's
    rows refuse (UNG_HIP_ESTATE) instead of reading an older call's rows; the next
    allocating call restores them."""
    hip = C.CDLL("libamdhip64.so")
    rng = np.random.default_rng(6)
    gb = np.array([0, 0, 200, 700], np.uint32)
    op = np.array([0, 0, 1, 1], np.uint32)
    oi = np.array([2], np.uint32)
    X = rng.standard_normal((700, 32)).astype(np.float32)
    with F.HipContext(0) as ctx:
        ctx.prepare_vectors(X)
        ctx.cross_topk_device(gb, op, oi, 6)
        ctx.download_cross()
        rows = DeviceRows(hip, 700, 6)
        try:
            _noalloc(ctx, gb, op, oi, 6, *rows.addrs())
            for call in (lambda: ctx.download_cross(700, 6), lambda: ctx.result_shape(0),
                         lambda: ctx.rescanned_rows(0), lambda: ctx.additional_edges(gb, op, oi, 6)):
                with pytest.raises(F.UngHipError) as e:
                    call()
                assert e.value.code == -3
            ctx.cross_topk_device(gb, op, oi, 6)
            assert ctx.result_shape(0)[0] == 700
        finally:
            rows.free()


def test_noalloc_short_output_buffer_refused():
    """Output buffers shorter than the rows the call writes are refused before anything
    runs."""
    hip = C.CDLL("libamdhip64.so")
    rng = np.random.default_rng(12)
    gb = np.array([0, 0, 200, 700], np.uint32)
    op = np.array([0, 0, 1, 1], np.uint32)
    oi = np.array([2], np.uint32)
    X = rng.standard_normal((700, 32)).astype(np.float32)
    with F.HipContext(0) as ctx:
        ctx.prepare_vectors(X)
        small = DeviceRows(hip, 699, 6)  # one row short
        rows = DeviceRows(hip, 700, 6)
        try:
            for addrs in (small.addrs(), [small.addrs()[0]] + rows.addrs()[1:],
                          rows.addrs()[:2] + [small.addrs()[2]],
                          [rows.addrs()[0] + 8] + rows.addrs()[1:]):  # 8 bytes into the buffer
                with pytest.raises(F.UngHipError) as e:
                    ctx.cross_topk_noalloc(gb, op, oi, 6, *addrs)
                assert e.value.code == -1 and "bytes" in str(e.value)
            want = _expect(ctx, gb, op, oi, 6)
            _noalloc(ctx, gb, op, oi, 6, *rows.addrs())
            _check(rows.download(), want, "after refusals")
        finally:
            small.free()
            rows.free()


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
            s1 = _noalloc(ctx, gb, op, oi, k, *rows.addrs())
            _check(rows.download(), want1, "noalloc call 1")
            _say(f"noalloc call 2 (smaller): {len(oi2)} LNG entries")
            s2 = _noalloc(ctx, gb, op2, oi2, k, *rows.addrs())
            assert s2["rows"] < s1["rows"] and s2["pairs"] < s1["pairs"]
            _check(rows.download(), want2, "noalloc call 2")
            _say("noalloc call 3 (first input again)")
            _noalloc(ctx, gb, op, oi, k, *rows.addrs())
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
            s1 = _noalloc(ctx, gb, op, oi, k, *rows.addrs())
            _check(rows.download(), want1, "noalloc d=520 call 1")
            _say("noalloc d=520 call 2 (smaller)")
            s2 = _noalloc(ctx, gb, op2, oi2, k, *rows.addrs())
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
                s = _noalloc(ctx, gb, op, oi, k, *rows.addrs())
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
