// ung_runtime.hip -- host side of the gfx950 UNG cross-edge / mid-group kNN build
// stage: the context (resident base set, two workspaces with their streams), the host
// work-list planning, kernel launches, the certified rescan and the C ABI of
// include/ung_hip.h.  The kernels are in ung_kernels.hip, included here (one
// translation unit).
#include "ung_kernels.hip"

#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include "ung_hip.h"
#include "ung_internal.h"

using ung::clear_error;
using ung::set_error;

namespace {

#define HIPCHECK(expr)                                                                     \
    do {                                                                                   \
        hipError_t _e = (expr);                                                            \
        if (_e != hipSuccess) {                                                            \
            set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e), __FILE__, __LINE__); \
            return UNG_HIP_EDEVICE;                                                        \
        }                                                                                  \
    } while (0)

using clk = std::chrono::steady_clock;
static double ms_since(clk::time_point t0)
{
    return std::chrono::duration<double, std::milli>(clk::now() - t0).count();
}

// Device (hipMalloc) and pinned host (hipHostMalloc) allocations made by the calling
// thread; ung_hip_stats::allocations reports the ones made during a call.
thread_local uint64_t t_alloc_calls = 0;

// Adds the allocations made while it lives to st->allocations (st may be null).
struct AllocCount {
    ung_hip_stats *st;
    uint64_t before;
    explicit AllocCount(ung_hip_stats *s) : st(s), before(t_alloc_calls) {}
    ~AllocCount()
    {
        if (st)
            st->allocations += t_alloc_calls - before;
    }
    AllocCount(const AllocCount &) = delete;
    AllocCount &operator=(const AllocCount &) = delete;
};

hipError_t counted_malloc(void **p, size_t bytes)
{
    ++t_alloc_calls;
    return hipMalloc(p, bytes);
}

template <class T>
struct DevBuf {
    T *p = nullptr;
    size_t cap = 0; // elements
    int ensure(size_t n)
    {
        if (n <= cap)
            return UNG_HIP_OK;
        if (p)
            (void)hipFree(p);
        p = nullptr;
        cap = 0;
        size_t want = n + n / 4 + 64;
        hipError_t e = counted_malloc((void **)&p, want * sizeof(T));
        if (e != hipSuccess) {
            p = nullptr;
            set_error("hipMalloc(%zu bytes) failed: %s", want * sizeof(T), hipGetErrorString(e));
            return UNG_HIP_EDEVICE;
        }
        cap = want;
        return UNG_HIP_OK;
    }
    void release()
    {
        if (p)
            (void)hipFree(p);
        p = nullptr;
        cap = 0;
    }
};

// Pinned host memory (hipHostMalloc), grown on demand.
struct HostBuf {
    void *p = nullptr;
    size_t cap = 0; // bytes
    int ensure(size_t n)
    {
        if (n <= cap)
            return UNG_HIP_OK;
        if (p)
            (void)hipHostFree(p);
        p = nullptr;
        cap = 0;
        const size_t want = n + n / 4 + 4096;
        ++t_alloc_calls;
        hipError_t e = hipHostMalloc(&p, want, hipHostMallocDefault);
        if (e != hipSuccess) {
            p = nullptr;
            set_error("hipHostMalloc(%zu bytes) failed: %s", want, hipGetErrorString(e));
            return UNG_HIP_EDEVICE;
        }
        cap = want;
        return UNG_HIP_OK;
    }
    void release()
    {
        if (p)
            (void)hipHostFree(p);
        p = nullptr;
        cap = 0;
    }
};

struct Plan {
    ung::RawVector<Job> jobs;
    ung::RawVector<Item> items;
    uint64_t n_mitems = 0;         // merge: MERGE_ROWS rows per block (written at launch)
    std::vector<MergeItem> pitems; // packing: MERGE_Q rows per block (group plans)
    ung::RawVector<uint32_t> seg_start, seg_vend;
    uint64_t part_rows = 0;
    uint64_t pairs = 0;
    uint64_t padded = 0;
    uint64_t rows = 0;
    uint64_t max_item_cand = 0;    // largest candidate range of an item
    // jobs of a few queries and a small union (tiny_job), scanned exactly without the
    // select and the merge (n_split = 0): [0].x = n_tiny, then (job, 0) for each
    ung::RawVector<uint2> tiny;
    uint64_t n_tiny = 0;
    // entries per partial row of the cross call whose partial rows are still in the
    // first workspace (set when such a call succeeds; 0: none)
    uint32_t part_lp = 0;
};


struct ResultBufs {
    DevBuf<uint32_t> ids;
    DevBuf<float> dist;
    DevBuf<int32_t> size;
    uint64_t rows = 0;
    uint32_t k = 0;
    bool valid = false;
    std::vector<uint32_t> rescanned; // output rows of the last call that took the exact rescan
    void release()
    {
        ids.release();
        dist.release();
        size.release();
        rows = 0;
        valid = false;
        rescanned.clear();
    }
};

} // namespace

namespace {
// Host staging of a plan's uploads: jobs | items (sorted) | seg_start | seg_vend | merge
// items (written after the select kernel is enqueued, so building and uploading them
// overlaps it); 256-byte aligned parts.
struct StageLayout {
    size_t bj, bi, bs, bt, bm;     // bytes of jobs, items, each segment array, tiny rows, merge items
    size_t oj, oi, os, ov, ot, om; // offsets
    size_t total;
};

StageLayout stage_layout(const Plan &pl)
{
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    StageLayout L{};
    L.bj = pl.jobs.size() * sizeof(Job);
    L.bi = pl.items.size() * sizeof(Item);
    L.bs = pl.seg_start.size() * sizeof(uint32_t);
    L.bt = pl.n_tiny ? (pl.n_tiny + 1) * sizeof(uint2) : 0;
    L.bm = pl.n_mitems * sizeof(MergeItem);
    L.oj = 0;
    L.oi = al(L.bj);
    L.os = L.oi + al(L.bi);
    L.ov = L.os + al(L.bs);
    L.ot = L.ov + al(L.bs);
    L.om = L.ot + al(L.bt);
    L.total = L.om + al(L.bm);
    return L;
}

// Where a planned call reads its work lists, keeps its partial rows and flags, and
// writes its result rows.
struct PlanMem {
    Job *jobs = nullptr;
    Item *items = nullptr;
    MergeItem *mitems = nullptr;
    uint32_t *seg_start = nullptr, *seg_vend = nullptr;
    uint32_t *part_ids = nullptr;
    float *part_dist = nullptr, *part_bound = nullptr;
    uint32_t *flag_count = nullptr; // [0]: rows flagged for the rescan, [1]: select item counter
    uint2 *flagged = nullptr;
    uint2 *tiny = nullptr;          // Plan::tiny
    uint32_t *out_ids = nullptr;    // result rows
    float *out_dist = nullptr;
    int32_t *out_size = nullptr;
    std::vector<uint32_t> *rescanned = nullptr; // output rows that took the exact rescan
    char *stage = nullptr;          // host staging (stage_layout), stable until the call ends
    // rescan range partials: grown in the workspace on demand, or a fixed region
    bool fb_grow = true;
    uint32_t *fb_ids = nullptr;
    float *fb_dist = nullptr;
    uint64_t fb_cap = 0;            // entries of fb_ids / fb_dist when !fb_grow
};

// Work lists, partial rows, flags and timing events of one planned call, with the stream
// it runs on.  A context has two, so a group kNN call can run on the second stream while
// the cross-edge call and the additional edges use the first.
struct Workspace {
    hipStream_t stream = nullptr;
    hipStream_t upload = nullptr; // merge-item uploads, beside the select kernel
    hipEvent_t ev[5] = {};        // select start, select end, merge end, rescan end, merge start
    hipEvent_t ev_up = nullptr;   // merge items uploaded
    DevBuf<Job> jobs;
    DevBuf<Item> items;
    DevBuf<MergeItem> mitems;
    DevBuf<uint32_t> seg_start, seg_vend;
    DevBuf<uint32_t> part_ids;
    DevBuf<float> part_dist;
    DevBuf<float> part_bound;
    DevBuf<uint32_t> flag_count; // [0]: rows flagged for the rescan, [1]: select item counter
    DevBuf<uint2> flagged;
    DevBuf<uint2> tiny;
    DevBuf<uint32_t> fb_ids; // rescan range results
    DevBuf<float> fb_dist;
    HostBuf stage;           // pinned staging of the work-list uploads
    void release()
    {
        stage.release();
        jobs.release();
        items.release();
        mitems.release();
        seg_start.release();
        seg_vend.release();
        part_ids.release();
        part_dist.release();
        part_bound.release();
        flag_count.release();
        flagged.release();
        tiny.release();
        fb_ids.release();
        fb_dist.release();
    }
};
} // namespace

struct ung_hip_ctx {
    int device = 0;
    hipStream_t stream = nullptr; // the first workspace's stream
    hipEvent_t ev[8] = {};
    // resident base set
    float *X = nullptr;
    uint32_t *XS = nullptr; // split base set (bf16 hi/lo pairs) for the MFMA pre-selection
    uint32_t dp = 0;        // its row pitch in words
    float *xn = nullptr;
    unsigned int *maxbits = nullptr;
    uint64_t N = 0;
    uint32_t d = 0;
    double rmax = 0.0;
    // work lists / scratch: [0] cross edges, additional edges and synchronous group calls,
    // [1] the group call started by ung_hip_cross_intra_begin
    Workspace ws[2];
    // a group call in flight on ws[1] (ung_hip_cross_intra_begin .. ung_hip_intra_end)
    bool intra_pending = false;
    // work lists of the calls on ws[0] (one at a time), kept between calls so their
    // storage is reused instead of allocated and first touched again every call
    Plan plan0;
    Plan intra_plan;
    PlanMem intra_mem; // memory of the group call in flight on ws[1]
    // ung_hip_cross_topk_noalloc: this device's address of the file-scope scratch array
    // (resolved once per device at ung_hip_create), host staging and rescanned rows
    unsigned char *scratch_dev = nullptr;
    std::vector<char> noalloc_stage;
    std::vector<uint32_t> noalloc_rescanned;
    uint32_t intra_list_k = 0;
    ung_hip_stats intra_stats{};
    std::chrono::steady_clock::time_point intra_t0;
    // results
    ResultBufs cross;
    ResultBufs group;
    // last group plan (for packing)
    std::vector<Job> group_jobs;
    std::vector<MergeItem> group_pitems;
    DevBuf<Job> gjobs;
    DevBuf<MergeItem> gmitems;
    uint32_t group_list_k = 0;
    DevBuf<uint32_t> graph;
    // large-group prune: reverse-edge counts/offsets, fill positions, lists, scan scratch
    DevBuf<uint32_t> rv_cnt, rv_fill, rv_src;
    DevBuf<float> rv_dist;
    DevBuf<unsigned char> rv_tmp;
    // additional edges: group ranges, LNG rows, point groups, reached flags, entry groups,
    // per-entry row/edge counts (scanned in place), group offsets, edge lists, counters
    DevBuf<uint32_t> a_gb, a_op, a_oi, a_pg, a_reached, a_eg, a_rows, a_edges, a_ptr, a_from, a_to;
    DevBuf<uint32_t> a_items, a_ientry, a_pid; // additional-edge scan items and their partial lists
    DevBuf<float> a_pdist;
    DevBuf<unsigned long long> a_cnt;
    DevBuf<unsigned char> a_tmp;
    HostBuf a_stage;
    // result downloads to host memory: DL_SLOTS pinned staging slots of DL_PIECE bytes and
    // an event per slot (see download_regions)
    HostBuf dl_stage;
    std::vector<hipEvent_t> dl_ev; // one per piece of the largest download so far
    // host threads of the work-list planning and staging (persistent, created at create)
    std::unique_ptr<ung::WorkerPool> pool;
    // test hook: UNG_HIP_FORCE_WIDE=1 at create selects the > 4 GiB load mode for any size
    bool force_wide = false;
    // UNG_HIP_NO_KNN=1 at create sends every group kNN call through ung_select_kernel (the
    // register-queue select) instead of the filter-and-buffer ung_knn_select_kernel
    bool knn = true;
    // test hook: UNG_HIP_NO_QREG=1 at create keeps the select kernel's restaged query panel
    // where the register-query layout would apply
    bool qreg = true;
    // test hook: UNG_HIP_EPS_SCALE=s (s >= 1) at create widens the certification error
    // bound by s, which sends more rows (all, for a huge s) through the exact rescan
    double eps_scale = 1.0;
    // large-group prune: the certified Gram pre-decision (ung_prune_gram_kernel) from
    // dp >= 256, where the exact alpha tests' row loads dominate (cfg4, d = 768: 272 -> 76
    // ms; cfg3, d = 384: 21.8 -> 9.4 ms), every alpha test scored exactly (ung_prune_kernel)
    // below (cfg2, d = 128: 12.7 against 19.8 ms).  Test hooks at create:
    // UNG_HIP_PRUNE_EXACT=1 takes the exact scan, UNG_HIP_PRUNE_GRAM=1 the Gram kernel, at
    // any d.
    int prune_mode = 0; // 0: by dp, 1: exact, 2: Gram
};

namespace {

int set_device(ung_hip_ctx *ctx)
{
    HIPCHECK(hipSetDevice(ctx->device));
    return UNG_HIP_OK;
}

// Candidates per split of a union of u candidates: SPLIT_V, raised (in whole tiles)
// so that a job never has more than MAX_SPLITS splits.
uint32_t split_size(uint64_t u)
{
    uint64_t s = (u + MAX_SPLITS - 1) / MAX_SPLITS;
    s = (s + BC - 1) / BC * BC;
    return (uint32_t)std::max<uint64_t>(SPLIT_V, s);
}

// Empties a plan, keeping the capacity of its lists.
void plan_reset(Plan &pl)
{
    pl.jobs.clear();
    pl.items.clear();
    pl.pitems.clear();
    pl.seg_start.clear();
    pl.seg_vend.clear();
    pl.n_mitems = 0;
    pl.max_item_cand = 0;
    pl.tiny.clear();
    pl.n_tiny = 0;
    pl.part_lp = 0;
    pl.part_rows = 0;
    pl.pairs = 0;
    pl.padded = 0;
    pl.rows = 0;
}

void add_items_for_job(Plan &pl, uint32_t job_index)
{
    const Job &jb = pl.jobs[job_index];
    // split-major: consecutive items are query blocks streaming the same candidates
    for (uint32_t s = 0; s < jb.n_split; ++s) {
        for (uint32_t qo = 0; qo < jb.q_count; qo += BQ) {
            const uint32_t qc = std::min<uint32_t>(BQ, jb.q_count - qo);
            Item it{};
            it.job = job_index;
            it.q_off = qo;
            it.q_cnt = qc;
            it.v_begin = s * jb.split_v;
            it.v_end = (uint32_t)std::min<uint64_t>(jb.n_cand, (uint64_t)(s + 1) * jb.split_v);
            it.split = s;
            pl.items.push_back(it);
            pl.padded += (uint64_t)BQ * (uint64_t)(((it.v_end - it.v_begin) + BC - 1) / BC * BC);
        }
    }
    pl.n_mitems += (jb.q_count + MERGE_ROWS - 1) / MERGE_ROWS;
}

// Merge items (MERGE_ROWS result rows of one job each) of a plan, written to `out`
// (pl.n_mitems entries).
void write_merge_items(const Plan &pl, MergeItem *out)
{
    size_t n = 0;
    for (uint32_t j = 0; j < (uint32_t)pl.jobs.size(); ++j) {
        const uint32_t qc = pl.jobs[j].q_count;
        if (pl.jobs[j].n_split == 0)
            continue; // scanned exactly (Plan::tiny)
        for (uint32_t qo = 0; qo < qc; qo += MERGE_ROWS)
            out[n++] = MergeItem{j, qo, std::min<uint32_t>(MERGE_ROWS, qc - qo), 0u};
    }
}

// Packing items (MERGE_Q rows of one job each) of a group plan.
void add_pack_items(Plan &pl)
{
    for (uint32_t j = 0; j < (uint32_t)pl.jobs.size(); ++j) {
        const uint32_t qc = pl.jobs[j].q_count;
        for (uint32_t qo = 0; qo < qc; qo += MERGE_Q)
            pl.pitems.push_back(MergeItem{j, qo, std::min<uint32_t>(MERGE_Q, qc - qo), 0u});
    }
}

// Entries per partial row: the k results plus a margin, at most two per merge lane
// and at most the 4 queues' entries.  The certified error bound grows with d; from
// d = 512 a margin of 10 keeps the first value left out far enough above the k-th
// that few rows need the exact rescan (cfg4: 133 rescanned cross rows, 4.5 ms, with a
// margin of 4), while at d = 128 the longer rows cost more than the rescans they save.
uint32_t pick_lp(uint32_t k, int lt, uint32_t d)
{
    const uint32_t margin = std::max<uint32_t>(d >= 512u ? 10u : 4u, k / 4);
    return std::min<uint32_t>(std::min<uint32_t>(128u, 4u * (uint32_t)lt), k + margin);
}

// Queue length: k <= LT lets the 4 queues of a query share thresholds.
int pick_lt(uint32_t k)
{
    if (k <= 8)
        return 8;
    if (k <= 16)
        return 16;
    return 32;
}

template <int LT>
int launch_select_t(ung_hip_ctx *ctx, hipStream_t stream, const SelectParams &P, uint32_t n_items, bool excl)
{
    // 32-bit buffer offsets need a split base set below 4 GiB
    const uint64_t x_bytes = (uint64_t)ctx->N * ctx->dp * sizeof(uint32_t);
    const int mode = (x_bytes < (1ull << 32) && !ctx->force_wide) ? LOAD_BUF32 : LOAD_WIDE;
    // grid dimension x is limited to 2^31-1; chunk the item list
    const uint32_t max_grid = 1u << 30;
    for (uint32_t off = 0; off < n_items; off += max_grid) {
        SelectParams Q = P;
        Q.items = P.items + off;
        Q.x_bytes = mode == LOAD_BUF32 ? (uint32_t)x_bytes : 0u;
        const uint32_t n = std::min(max_grid, n_items - off);
        Q.n_items = n;
        if (off > 0) { // the counter was zeroed for the first chunk by the caller
            hipLaunchKernelGGL(ung_zero_u32_kernel, dim3(1), dim3(64), 0, stream, P.item_ctr, 1u);
            HIPCHECK(hipGetLastError());
        }
        // queues longer than 8 take the one-column-per-lane layout (two waves per SIMD)
        constexpr int NB = LT <= 8 ? 2 : 1;
        const dim3 g(n), b(select_threads<NB>());
        // two columns per lane and dp = 128: the register-query layout
        const bool qr = NB == 2 && ctx->dp == (uint32_t)(QR_NK * KC) && ctx->qreg;
        if constexpr (NB == 2) {
            if (qr && mode == LOAD_BUF32 && excl)
                hipLaunchKernelGGL((ung_select_kernel<LT, LOAD_BUF32, true, NB, true>), g, b, 0, stream, Q);
            else if (qr && mode == LOAD_BUF32)
                hipLaunchKernelGGL((ung_select_kernel<LT, LOAD_BUF32, false, NB, true>), g, b, 0, stream, Q);
            else if (qr && excl)
                hipLaunchKernelGGL((ung_select_kernel<LT, LOAD_WIDE, true, NB, true>), g, b, 0, stream, Q);
            else if (qr)
                hipLaunchKernelGGL((ung_select_kernel<LT, LOAD_WIDE, false, NB, true>), g, b, 0, stream, Q);
        }
        if (qr)
            ; // launched above
        else if (mode == LOAD_BUF32 && excl)
            hipLaunchKernelGGL((ung_select_kernel<LT, LOAD_BUF32, true, NB, false>), g, b, 0, stream, Q);
        else if (mode == LOAD_BUF32)
            hipLaunchKernelGGL((ung_select_kernel<LT, LOAD_BUF32, false, NB, false>), g, b, 0, stream, Q);
        else if (excl)
            hipLaunchKernelGGL((ung_select_kernel<LT, LOAD_WIDE, true, NB, false>), g, b, 0, stream, Q);
        else
            hipLaunchKernelGGL((ung_select_kernel<LT, LOAD_WIDE, false, NB, false>), g, b, 0, stream, Q);
        HIPCHECK(hipGetLastError());
    }
    return UNG_HIP_OK;
}

// Filter-and-buffer select of a group plan (ung_knn_select_kernel, dp <= 128), grid
// chunked like launch_select_t.
template <int NK>
int launch_knn_select_t(ung_hip_ctx *ctx, hipStream_t stream, const SelectParams &P, uint32_t n_items)
{
    const uint64_t x_bytes = (uint64_t)ctx->N * ctx->dp * sizeof(uint32_t);
    const int mode = (x_bytes < (1ull << 32) && !ctx->force_wide) ? LOAD_BUF32 : LOAD_WIDE;
    const uint32_t max_grid = 1u << 30;
    for (uint32_t off = 0; off < n_items; off += max_grid) {
        SelectParams Q = P;
        Q.items = P.items + off;
        Q.x_bytes = mode == LOAD_BUF32 ? (uint32_t)x_bytes : 0u;
        const uint32_t n = std::min(max_grid, n_items - off);
        Q.n_items = n;
        if (off > 0) {
            hipLaunchKernelGGL(ung_zero_u32_kernel, dim3(1), dim3(64), 0, stream, P.item_ctr, 1u);
            HIPCHECK(hipGetLastError());
        }
        if (mode == LOAD_BUF32)
            hipLaunchKernelGGL((ung_knn_select_kernel<LOAD_BUF32, NK>), dim3(n), dim3(KNN_THREADS), 0, stream, Q);
        else
            hipLaunchKernelGGL((ung_knn_select_kernel<LOAD_WIDE, NK>), dim3(n), dim3(KNN_THREADS), 0, stream, Q);
        HIPCHECK(hipGetLastError());
    }
    return UNG_HIP_OK;
}

int launch_knn_select(ung_hip_ctx *ctx, hipStream_t stream, const SelectParams &P, uint32_t n_items)
{
    switch (ctx->dp / KC) {
    case 1:
        return launch_knn_select_t<1>(ctx, stream, P, n_items);
    case 2:
        return launch_knn_select_t<2>(ctx, stream, P, n_items);
    case 3:
        return launch_knn_select_t<3>(ctx, stream, P, n_items);
    case 4:
        return launch_knn_select_t<4>(ctx, stream, P, n_items);
    default:
        set_error("filter-and-buffer select: dp=%u above %d", ctx->dp, KNN_MAX_NK * KC);
        return UNG_HIP_EINVAL;
    }
}

// Error factor of the expansion-form value a = fl(|q|^2 - 2*acc) of the select kernel:
// |a - D| <= eps_coef * (|q| + R)^2 with D the exact squared distance, u = 2^-24.
//  * norm caches fl(|x|^2), fl(|q|^2): fp64 sums rounded once, <= u relative each
//                                                                     -> u (|q|+R)^2
//  * split operands: each product x_i q_i is replaced by hi*hi + hi*lo + lo*hi, exact in
//    fp32 (8-bit significands); the dropped terms are <= 3.01 * 2^-18 |x_i q_i|, so <=
//    192.6 u |x||q| in s and 385.2 u |x||q| <= 96.3 u (|q|+R)^2 in a
//  * accumulation of the 3d products from 0 (sum of |products| <= 1.0079 |x||q|): with
//    round-to-nearest additions in any order <= 3d*u*1.0079 |x||q|; a fused adder that
//    truncates each of its 17 operands by at most one ulp of the largest and rounds once
//    gives <= 17u per MFMA over 3d/16 MFMAs, 3.19 d*u*1.0079 |x||q|.  In a: <= 1.61 d*u
//    (|q|+R)^2
//  * adding -fl(|x|^2)/2 and the pre-filter bound cb (|cb| <= (|q|+R)^2: a threshold
//    distance at most (|q|+R)^2, halved, plus |q|^2/2) by one more MFMA whose six bf16
//    products sum exactly to those two fp32 values: at most 7 operand truncations and one
//    rounding in the fused-adder model above, <= 7.5 u max(|acc|, |x|^2/2, |cb|) <=
//    7.5 u (|q|+R)^2, then -s read back as fl(acc - cb): <= 2 u (|q|+R)^2, so in a:
//    <= 19 u (|q|+R)^2; the final fma: <= 1.01 u (|q|+R)^2
// Sum <= (1.61 d + 117.4) u (|q|+R)^2; the factor below keeps a margin.  Flushed bf16 or
// fp32 subnormals add at most ~6d * 2^-126 absolute, covered by the 1e-30 term of
// lower_bound_ea.
double eps_coef_for(uint32_t d)
{
    return (1.75 * (double)d + 132.0) * std::ldexp(1.0, -24);
}

// PlanMem in the workspace's own buffers, grown to the plan (hipMalloc / hipHostMalloc
// when a buffer is too small); rows into `res`.
int workspace_mem(Workspace &ws, const Plan &pl, uint32_t lp, ResultBufs &res, PlanMem &m)
{
    int rc;
    if ((rc = ws.jobs.ensure(pl.jobs.size())) || (rc = ws.items.ensure(pl.items.size())) ||
        (rc = ws.mitems.ensure(pl.n_mitems)) || (rc = ws.seg_start.ensure(pl.seg_start.size())) ||
        (rc = ws.seg_vend.ensure(pl.seg_vend.size())) ||
        (rc = ws.part_ids.ensure(pl.part_rows * lp)) || (rc = ws.part_dist.ensure(pl.part_rows * lp)) ||
        (rc = ws.part_bound.ensure(pl.part_rows)) || (rc = ws.flag_count.ensure(2)) ||
        (rc = ws.flagged.ensure(std::max<uint64_t>(pl.rows, 1))) || (rc = ws.tiny.ensure(pl.n_tiny + 1)))
        return rc;
    if (!pl.jobs.empty()) {
        // the previous call's uploads from the staging buffer have completed (its merge
        // launch event follows them on the stream)
        HIPCHECK(hipEventSynchronize(ws.ev[2]));
        if ((rc = ws.stage.ensure(stage_layout(pl).total)))
            return rc;
    }
    m.jobs = ws.jobs.p;
    m.items = ws.items.p;
    m.mitems = ws.mitems.p;
    m.seg_start = ws.seg_start.p;
    m.seg_vend = ws.seg_vend.p;
    m.part_ids = ws.part_ids.p;
    m.part_dist = ws.part_dist.p;
    m.part_bound = ws.part_bound.p;
    m.flag_count = ws.flag_count.p;
    m.flagged = ws.flagged.p;
    m.tiny = ws.tiny.p;
    m.out_ids = res.ids.p;
    m.out_dist = res.dist.p;
    m.out_size = res.size.p;
    m.rescanned = &res.rescanned;
    m.stage = static_cast<char *>(ws.stage.p);
    m.fb_grow = true;
    return UNG_HIP_OK;
}

// Copies a plan's jobs and segments into the staging buffer, and its items in order of
// decreasing cost (candidate tiles): a stable counting sort by tile count (the query
// blocks of one split stay next to each other).  Large plans run on the worker pool:
// per-chunk histograms, a prefix over (bucket, chunk), a scatter.
void stage_plan(ung_hip_ctx *ctx, const Plan &pl, const StageLayout &L, char *hs)
{
    auto tiles = [](const Item &it) { return (it.v_end - it.v_begin + BC - 1) / BC; };
    const uint64_t n = pl.items.size();
    const int T = ctx->pool ? ctx->pool->size() : 1;
    Item *sorted = reinterpret_cast<Item *>(hs + L.oi);
    if (L.bt)
        std::memcpy(hs + L.ot, pl.tiny.data(), L.bt);
    uint32_t max_t = 0;
    if (n < 65536 || T == 1) {
        std::memcpy(hs + L.oj, pl.jobs.data(), L.bj);
        std::memcpy(hs + L.os, pl.seg_start.data(), L.bs);
        std::memcpy(hs + L.ov, pl.seg_vend.data(), L.bs);
        for (const Item &it : pl.items)
            max_t = std::max(max_t, tiles(it));
        std::vector<uint64_t> start(max_t + 2, 0);
        for (const Item &it : pl.items)
            ++start[max_t - tiles(it) + 1];
        for (uint32_t t = 0; t <= max_t; ++t)
            start[t + 1] += start[t];
        for (const Item &it : pl.items)
            sorted[start[max_t - tiles(it)]++] = it;
        return;
    }
    const uint32_t nch = (uint32_t)std::min<uint64_t>(4ull * (uint64_t)T, (n + 4095) / 4096);
    auto chunk_begin = [&](uint32_t c) { return n * c / nch; };
    std::vector<uint32_t> cmax(nch, 0);
    ctx->pool->run(nch, [&](int64_t c) {
        uint32_t m = 0;
        for (uint64_t i = chunk_begin((uint32_t)c); i < chunk_begin((uint32_t)c + 1); ++i)
            m = std::max(m, tiles(pl.items[i]));
        cmax[c] = m;
    });
    for (uint32_t m : cmax)
        max_t = std::max(max_t, m);
    const uint32_t nb = max_t + 1; // bucket max_t - tiles: decreasing cost first
    std::vector<uint64_t> hist((size_t)nch * nb, 0);
    // histograms, and the job / segment copies in pieces beside them
    const uint32_t ncopy = (uint32_t)T;
    ctx->pool->run(nch + 3 * ncopy, [&](int64_t task) {
        if (task < (int64_t)nch) {
            uint64_t *h = hist.data() + (size_t)task * nb;
            for (uint64_t i = chunk_begin((uint32_t)task); i < chunk_begin((uint32_t)task + 1); ++i)
                ++h[max_t - tiles(pl.items[i])];
            return;
        }
        const uint32_t which = (uint32_t)(task - nch) / ncopy, piece = (uint32_t)(task - nch) % ncopy;
        const char *src = which == 0 ? reinterpret_cast<const char *>(pl.jobs.data())
                        : which == 1 ? reinterpret_cast<const char *>(pl.seg_start.data())
                                     : reinterpret_cast<const char *>(pl.seg_vend.data());
        char *dst = hs + (which == 0 ? L.oj : which == 1 ? L.os : L.ov);
        const size_t bytes = which == 0 ? L.bj : L.bs;
        const size_t b0 = bytes * piece / ncopy, b1 = bytes * (piece + 1) / ncopy;
        std::memcpy(dst + b0, src + b0, b1 - b0);
    });
    uint64_t pos = 0;
    for (uint32_t b = 0; b < nb; ++b)
        for (uint32_t c = 0; c < nch; ++c) {
            const uint64_t cnt = hist[(size_t)c * nb + b];
            hist[(size_t)c * nb + b] = pos;
            pos += cnt;
        }
    ctx->pool->run(nch, [&](int64_t c) {
        uint64_t *h = hist.data() + (size_t)c * nb;
        for (uint64_t i = chunk_begin((uint32_t)c); i < chunk_begin((uint32_t)c + 1); ++i) {
            const Item &it = pl.items[i];
            sorted[h[max_t - tiles(it)]++] = it;
        }
    });
}

// Dynamic LDS of a merge launch: the query row of each of its waves when d allows.
size_t merge_qlds_bytes(uint32_t d)
{
    return d <= MERGE_QLDS ? (size_t)MERGE_ROWS * d * sizeof(float) : 0;
}

// Runs a planned job list on workspace `ws` (its stream and events) with the memory of
// `m`; result rows already initialised by the caller when some rows have no job.
// plan_launch uploads the work lists and enqueues the select and merge kernels;
// plan_finish reads the flagged-row count back, rescans those rows and collects the
// statistics.
int plan_launch_merge(ung_hip_ctx *ctx, Workspace &ws, const Plan &pl, uint32_t k, PlanMem &m, ung_hip_stats *st);

int plan_launch(ung_hip_ctx *ctx, Workspace &ws, const Plan &pl, uint32_t k, PlanMem &m, ung_hip_stats *st,
                hipEvent_t start_after = nullptr)
{
    int rc;
    const int lt = pick_lt(k);
    const uint32_t lp = pick_lp(k, lt, ctx->d);
    const auto t_h2d = clk::now();
    const StageLayout L = stage_layout(pl);
    char *hs = m.stage;
    if (!pl.jobs.empty()) {
        stage_plan(ctx, pl, L, hs);
        HIPCHECK(hipMemcpyAsync(m.jobs, hs + L.oj, L.bj, hipMemcpyHostToDevice, ws.stream));
        HIPCHECK(hipMemcpyAsync(m.items, hs + L.oi, L.bi, hipMemcpyHostToDevice, ws.stream));
        HIPCHECK(hipMemcpyAsync(m.seg_start, hs + L.os, L.bs, hipMemcpyHostToDevice, ws.stream));
        HIPCHECK(hipMemcpyAsync(m.seg_vend, hs + L.ov, L.bs, hipMemcpyHostToDevice, ws.stream));
        if (L.bt)
            HIPCHECK(hipMemcpyAsync(m.tiny, hs + L.ot, L.bt, hipMemcpyHostToDevice, ws.stream));
    }
    if (st)
        st->h2d_ms += ms_since(t_h2d);
    if (pl.jobs.empty())
        return UNG_HIP_OK;

    // kernels of this plan start after `start_after` (another stream's event), if given
    if (start_after)
        HIPCHECK(hipStreamWaitEvent(ws.stream, start_after, 0));
    hipLaunchKernelGGL(ung_zero_u32_kernel, dim3(1), dim3(64), 0, ws.stream, m.flag_count, 2u);
    HIPCHECK(hipGetLastError());
    HIPCHECK(hipEventRecord(ws.ev[0], ws.stream));

    SelectParams P{};
    P.xs = ctx->XS;
    P.xn = ctx->xn;
    P.dp = ctx->dp;
    P.k = k;
    P.jobs = m.jobs;
    P.items = m.items;
    P.seg_start = m.seg_start;
    P.seg_vend = m.seg_vend;
    P.part_ids = m.part_ids;
    P.part_dist = m.part_dist;
    P.part_bound = m.part_bound;
    P.eps_coef = eps_coef_for(ctx->d) * ctx->eps_scale;
    P.shrink = ((double)ctx->d / 8.0 + 8.0) * std::ldexp(1.0, -24);
    P.rmax = ctx->rmax;
    P.item_ctr = m.flag_count + 1;
    P.lp = lp;
    const uint32_t n_items = (uint32_t)pl.items.size();
    const bool excl = (pl.jobs[0].flags & 1u) != 0; // one kind of job per plan
    // group kNN lists with partial rows below 64 entries, splits below 65,536 candidates
    // and d <= 128 (the mid-group batch of the exact kNN stage): the filter-and-buffer select
    const bool knn = ctx->knn && excl && lp + 1u <= KNN_OUT && pl.max_item_cand <= KNN_MAX_SPLIT &&
                     ctx->dp <= (uint32_t)(KNN_MAX_NK * KC);
    if (knn)
        rc = launch_knn_select(ctx, ws.stream, P, n_items);
    else if (lt == 8)
        rc = launch_select_t<8>(ctx, ws.stream, P, n_items, excl);
    else if (lt == 16)
        rc = launch_select_t<16>(ctx, ws.stream, P, n_items, excl);
    else
        rc = launch_select_t<32>(ctx, ws.stream, P, n_items, excl);
    if (rc)
        return rc;
    HIPCHECK(hipEventRecord(ws.ev[1], ws.stream));
    if (pl.n_tiny > 0) {
        // the jobs left out of the select (tiny_job), one wave each, exact
        FallbackParams F{};
        F.X = ctx->X;
        F.d = ctx->d;
        F.k = k;
        F.jobs = m.jobs;
        F.seg_start = m.seg_start;
        F.seg_vend = m.seg_vend;
        F.flag_count = reinterpret_cast<const uint32_t *>(m.tiny);
        F.flagged = m.tiny + 1;
        F.splits = 1;
        F.out_ids = m.out_ids;
        F.out_dist = m.out_dist;
        F.out_size = m.out_size;
        const uint64_t blocks = (pl.n_tiny + TINY_WAVES - 1) / TINY_WAVES;
        hipLaunchKernelGGL(ung_tiny_jobs_kernel, dim3((unsigned)std::min<uint64_t>(blocks, 1u << 20)),
                           dim3(64 * TINY_WAVES), 0, ws.stream, F);
        HIPCHECK(hipGetLastError());
    }
    return plan_launch_merge(ctx, ws, pl, k, m, st);
}

// The merge of a launched plan, after its select kernel on ws.stream.
int plan_launch_merge(ung_hip_ctx *ctx, Workspace &ws, const Plan &pl, uint32_t k, PlanMem &m, ung_hip_stats *st)
{
    if (pl.jobs.empty())
        return UNG_HIP_OK;
    const uint32_t lp = pick_lp(k, pick_lt(k), ctx->d);
    const StageLayout L = stage_layout(pl);
    char *hs = m.stage;
    // merge items, built and uploaded (on the upload stream) while the select kernel runs
    const auto t_mi = clk::now();
    write_merge_items(pl, reinterpret_cast<MergeItem *>(hs + L.om));
    HIPCHECK(hipMemcpyAsync(m.mitems, hs + L.om, L.bm, hipMemcpyHostToDevice, ws.upload));
    HIPCHECK(hipEventRecord(ws.ev_up, ws.upload));
    HIPCHECK(hipStreamWaitEvent(ws.stream, ws.ev_up, 0));
    HIPCHECK(hipEventRecord(ws.ev[4], ws.stream));
    if (st)
        st->h2d_ms += ms_since(t_mi);

    MergeParams M{};
    M.X = ctx->X;
    M.xn = ctx->xn;
    M.d = ctx->d;
    M.jobs = m.jobs;
    M.mitems = m.mitems;
    M.part_ids = m.part_ids;
    M.part_dist = m.part_dist;
    M.part_bound = m.part_bound;
    M.lp = lp;
    M.k = k;
    M.eps_coef = eps_coef_for(ctx->d) * ctx->eps_scale;
    M.shrink = ((double)ctx->d / 8.0 + 8.0) * std::ldexp(1.0, -24);
    M.rmax = ctx->rmax;
    M.out_ids = m.out_ids;
    M.out_dist = m.out_dist;
    M.out_size = m.out_size;
    M.flag_count = m.flag_count;
    M.flagged = m.flagged;
    // group kNN plans (exclusive jobs: a group against itself) of long rows spread their
    // items over the XCDs in contiguous ranges (d = 768: intra merge 11.3 -> 8.5 ms; at
    // d = 128 and 384 it measured the same or 2 % slower)
    const bool group_plan = (pl.jobs[0].flags & 1u) != 0;
    M.xcd_spread = group_plan && ctx->d >= 512 ? 1u : 0u;
    // two candidates per re-score pass for group kNN rows of d >= 256 (cfg3 intra merge
    // 1.28 -> 1.14 ms, cfg4 8.58 -> 7.71 ms; at d = 128 and in the cross merge slower)
    const bool pair = group_plan && ctx->d >= 256;
    // group kNN rows (~33 re-scored candidates) read the query row from LDS; the cross
    // merge's short rows do not (the copy costs them more than it saves)
    const size_t qlds = group_plan ? merge_qlds_bytes(ctx->d) : 0;
    M.qlds = qlds ? 1u : 0u;
    const uint32_t n_m = (uint32_t)pl.n_mitems;
    for (uint32_t off = 0; off < n_m; off += (1u << 30)) {
        MergeParams Mc = M;
        Mc.mitems = M.mitems + off;
        const uint32_t n = std::min<uint32_t>(1u << 30, n_m - off);
        Mc.n_mitems = n;
        const uint32_t grid = M.xcd_spread ? NUM_XCD * ((n + NUM_XCD - 1u) / NUM_XCD) : n;
        if (pair)
            hipLaunchKernelGGL(ung_merge_kernel<true>, dim3(grid), dim3(64 * MERGE_ROWS), qlds, ws.stream, Mc);
        else
            hipLaunchKernelGGL(ung_merge_kernel<false>, dim3(grid), dim3(64 * MERGE_ROWS), qlds, ws.stream, Mc);
        HIPCHECK(hipGetLastError());
    }
    HIPCHECK(hipEventRecord(ws.ev[2], ws.stream));
    return UNG_HIP_OK;
}

// Exact rescan of flagged rows: a row's union is cut into ranges of at least
// FALLBACK_RANGE candidates, at most MAX_FALLBACK_SPLITS of them, one wave each (a few
// rows with small unions still spread over a few hundred waves).
constexpr uint32_t FALLBACK_RANGE = 256;
constexpr uint32_t MAX_FALLBACK_SPLITS = 1024;

int plan_finish(ung_hip_ctx *ctx, Workspace &ws, const Plan &pl, uint32_t k, PlanMem &m, ung_hip_stats *st)
{
    int rc;
    if (pl.jobs.empty())
        return UNG_HIP_OK;
    uint32_t nflag = 0;
    HIPCHECK(hipMemcpyAsync(&nflag, m.flag_count, sizeof(uint32_t), hipMemcpyDeviceToHost, ws.stream));
    HIPCHECK(hipStreamSynchronize(ws.stream));
    if (nflag > 0) {
        // a flagged row's union is cut into ranges of >= FALLBACK_RANGE candidates
        uint64_t max_cand = 0;
        for (const Job &jb : pl.jobs)
            max_cand = std::max<uint64_t>(max_cand, jb.n_cand);
        uint32_t S =
            (uint32_t)std::min<uint64_t>(MAX_FALLBACK_SPLITS, std::max<uint64_t>(1, max_cand / FALLBACK_RANGE));
        if (!m.fb_grow) // the fixed region bounds the ranges (one range writes the row itself)
            S = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(S, m.fb_cap / ((uint64_t)nflag * k)));
        FallbackParams F{};
        F.X = ctx->X;
        F.d = ctx->d;
        F.k = k;
        F.jobs = m.jobs;
        F.seg_start = m.seg_start;
        F.seg_vend = m.seg_vend;
        F.flag_count = m.flag_count;
        F.flagged = m.flagged;
        F.splits = S;
        F.out_ids = m.out_ids;
        F.out_dist = m.out_dist;
        F.out_size = m.out_size;
        if (S > 1) {
            if (m.fb_grow) {
                if ((rc = ws.fb_ids.ensure((uint64_t)nflag * S * k)) ||
                    (rc = ws.fb_dist.ensure((uint64_t)nflag * S * k)))
                    return rc;
                m.fb_ids = ws.fb_ids.p;
                m.fb_dist = ws.fb_dist.p;
            }
            F.part_ids = m.fb_ids;
            F.part_dist = m.fb_dist;
        }
        const uint64_t items = (uint64_t)nflag * S;
        hipLaunchKernelGGL(ung_fallback_kernel, dim3((unsigned)std::min<uint64_t>(items, 1u << 20)), dim3(64), 0,
                           ws.stream, F);
        HIPCHECK(hipGetLastError());
        if (S > 1) {
            hipLaunchKernelGGL(ung_fallback_merge_kernel, dim3(std::min<uint32_t>(nflag, 8192u)), dim3(64), 0,
                               ws.stream, F);
            HIPCHECK(hipGetLastError());
        }
    }
    std::vector<uint2> flagged_host(nflag);
    if (nflag > 0)
        HIPCHECK(hipMemcpyAsync(flagged_host.data(), m.flagged, nflag * sizeof(uint2), hipMemcpyDeviceToHost,
                                ws.stream));
    HIPCHECK(hipEventRecord(ws.ev[3], ws.stream));
    HIPCHECK(hipEventSynchronize(ws.ev[3]));
    if (m.rescanned) {
        for (const uint2 &f : flagged_host)
            m.rescanned->push_back(pl.jobs[f.x].out_row + f.y);
        std::sort(m.rescanned->begin(), m.rescanned->end());
    }
    if (st) {
        float a = 0, b = 0, c = 0;
        HIPCHECK(hipEventElapsedTime(&a, ws.ev[0], ws.ev[1]));
        HIPCHECK(hipEventElapsedTime(&b, ws.ev[4], ws.ev[2]));
        HIPCHECK(hipEventElapsedTime(&c, ws.ev[2], ws.ev[3]));
        st->select_ms += a;
        st->merge_ms += b;
        st->fallback_ms += c;
        st->kernel_ms += a + b + c;
        st->fallback_rows += nflag;
        st->pairs += pl.pairs;
        st->padded_pairs += pl.padded;
        uint64_t rows_streamed = 0;
        for (const Item &it : pl.items)
            rows_streamed += (uint64_t)it.q_cnt + (it.v_end - it.v_begin);
        st->select_bytes += rows_streamed * ctx->dp * sizeof(uint32_t);
        st->rows += pl.rows;
        st->work_items += pl.items.size();
        st->select_launches += 1;
    }
    return UNG_HIP_OK;
}

// Launch + finish in the workspace's own (growable) memory, rows into `res`.
int run_plan(ung_hip_ctx *ctx, Workspace &ws, const Plan &pl, uint32_t k, ResultBufs &res, ung_hip_stats *st)
{
    int rc;
    PlanMem m;
    if ((rc = workspace_mem(ws, pl, pick_lp(k, pick_lt(k), ctx->d), res, m)) || (rc = plan_launch(ctx, ws, pl, k, m, st)))
        return rc;
    return plan_finish(ctx, ws, pl, k, m, st);
}

int check_ready(ung_hip_ctx *ctx)
{
    if (!ctx) {
        set_error("null context");
        return UNG_HIP_EINVAL;
    }
    if (!ctx->X) {
        set_error("base vectors not prepared (call ung_hip_prepare_vectors first)");
        return UNG_HIP_ESTATE;
    }
    return UNG_HIP_OK;
}

// One chunk of groups of a cross plan: pass 1 counts its jobs, segments and items and
// validates its groups; after a prefix over the chunks pass 2 writes them at its offsets.
struct PlanChunk {
    uint32_t g_begin = 0, g_end = 0; // groups [g_begin, g_end)
    uint64_t jobs = 0, segs = 0, items = 0, mitems = 0, part_rows = 0, pairs = 0, padded = 0, rows = 0, tiny = 0;
    int rc = UNG_HIP_OK;
    char msg[192] = {};
};

// Cross plan: one job per group C with a non-empty union of its out-groups, its segments
// (the out-groups' ranges in LNG row order), and its items (query blocks x splits,
// split-major).  Two passes over chunks of groups on the context's worker pool.
int build_cross_plan(ung_hip_ctx *ctx, uint32_t G, const uint32_t *group_begin, const uint32_t *out_ptr,
                     const uint32_t *out_idx, Plan &pl)
{
    if (!group_begin || !out_ptr || (out_ptr[G + 1] > 0 && !out_idx)) {
        set_error("ung_hip_cross_topk: null group_begin/out_ptr/out_idx");
        return UNG_HIP_EINVAL;
    }
    if ((uint64_t)group_begin[G + 1] != ctx->N) {
        set_error("ung_hip_cross_topk: group_begin[G+1]=%u but %llu vectors are prepared", group_begin[G + 1],
                  (unsigned long long)ctx->N);
        return UNG_HIP_EINVAL;
    }
    // chunks of about equal groups + LNG entries (G small: one chunk, no thread hand-off)
    const int T = ctx->pool ? ctx->pool->size() : 1;
    const uint32_t nch = G < 4096 || T == 1 ? 1u : (uint32_t)std::min<uint64_t>(G, 8ull * (uint64_t)T);
    std::vector<PlanChunk> ch(nch);
    {
        const uint64_t E = out_ptr[G + 1];
        uint32_t prev = 1;
        for (uint32_t t = 0; t < nch; ++t) {
            ch[t].g_begin = prev;
            uint32_t end = G + 1;
            if (t + 1 < nch) {
                // first group c with (c - 1) + out_ptr[c] >= the chunk's share
                const uint64_t want = (uint64_t)(t + 1) * ((uint64_t)G + E) / nch;
                uint32_t lo = prev, hi = G + 1;
                while (lo < hi) {
                    const uint32_t mid = lo + (hi - lo) / 2;
                    if ((uint64_t)(mid - 1) + out_ptr[mid] >= want)
                        hi = mid;
                    else
                        lo = mid + 1;
                }
                end = std::max(prev, lo);
            }
            ch[t].g_end = end;
            prev = end;
        }
    }
#define PLAN_FAIL(c, ...)                                                                  \
    do {                                                                                   \
        (c).rc = UNG_HIP_EINVAL;                                                           \
        std::snprintf((c).msg, sizeof((c).msg), __VA_ARGS__);                              \
        return;                                                                            \
    } while (0)
    auto pass1 = [&](int64_t t) {
        PlanChunk &c = ch[t];
        for (uint32_t g = c.g_begin; g < c.g_end; ++g) {
            if (group_begin[g + 1] < group_begin[g])
                PLAN_FAIL(c, "ung_hip_cross_topk: group_begin not monotone at group %u", g);
            if (out_ptr[g + 1] < out_ptr[g])
                PLAN_FAIL(c, "ung_hip_cross_topk: out_ptr not monotone at group %u", g);
            const uint32_t qn = group_begin[g + 1] - group_begin[g];
            if (qn == 0 || out_ptr[g + 1] == out_ptr[g])
                continue;
            uint64_t u = 0, segs = 0;
            for (uint32_t e = out_ptr[g]; e < out_ptr[g + 1]; ++e) {
                const uint32_t x = out_idx[e];
                if (x < 1 || x > G)
                    PLAN_FAIL(c, "ung_hip_cross_topk: out_idx entry %u out of range 1..%u", x, G);
                const uint32_t nx = group_begin[x + 1] - group_begin[x];
                if (nx == 0)
                    continue;
                u += nx;
                ++segs;
                if (u >= 0xFFFFFFFFull)
                    PLAN_FAIL(c, "ung_hip_cross_topk: candidate union of group %u exceeds 2^32", g);
            }
            if (u == 0)
                continue;
            c.jobs += 1;
            c.segs += segs;
            c.pairs += (uint64_t)qn * u;
            c.rows += qn;
            if (tiny_job(qn, u)) {
                c.tiny += 1;
                continue;
            }
            const uint64_t sv = split_size(u), ns = (u + sv - 1) / sv, qb = (qn + BQ - 1) / BQ;
            c.items += ns * qb;
            c.mitems += (qn + MERGE_ROWS - 1) / MERGE_ROWS;
            c.part_rows += (uint64_t)qn * ns;
            const uint64_t last = u - (ns - 1) * sv;
            c.padded += (uint64_t)BQ * qb * ((ns - 1) * sv + (last + BC - 1) / BC * BC);
        }
    };
#undef PLAN_FAIL
    if (nch == 1)
        pass1(0);
    else
        ctx->pool->run(nch, pass1);
    uint64_t n_jobs = 0, n_segs = 0, n_items = 0;
    std::vector<uint64_t> o_job(nch), o_seg(nch), o_item(nch), o_part(nch), o_tiny(nch);
    for (uint32_t t = 0; t < nch; ++t) {
        if (ch[t].rc) {
            set_error("%s", ch[t].msg);
            return ch[t].rc;
        }
        o_job[t] = n_jobs;
        o_seg[t] = n_segs;
        o_item[t] = n_items;
        o_part[t] = pl.part_rows;
        o_tiny[t] = pl.n_tiny;
        pl.n_tiny += ch[t].tiny;
        n_jobs += ch[t].jobs;
        n_segs += ch[t].segs;
        n_items += ch[t].items;
        pl.part_rows += ch[t].part_rows;
        pl.n_mitems += ch[t].mitems;
        pl.pairs += ch[t].pairs;
        pl.padded += ch[t].padded;
        pl.rows += ch[t].rows;
    }
    if (pl.part_rows >= 0xFFFFFFFFull || n_segs >= 0xFFFFFFFFull) {
        set_error("ung_hip_cross_topk: partial rows exceed 2^32");
        return UNG_HIP_EINVAL;
    }
    pl.jobs.resize(n_jobs);
    pl.items.resize(n_items);
    pl.seg_start.resize(n_segs);
    pl.seg_vend.resize(n_segs);
    if (pl.n_tiny) {
        pl.tiny.resize(pl.n_tiny + 1);
        pl.tiny[0] = make_uint2((uint32_t)pl.n_tiny, 0u);
    }
    auto pass2 = [&](int64_t t) {
        uint64_t j = o_job[t], sg = o_seg[t], itn = o_item[t], part = o_part[t], tn = 1 + o_tiny[t];
        for (uint32_t g = ch[t].g_begin; g < ch[t].g_end; ++g) {
            const uint32_t qn = group_begin[g + 1] - group_begin[g];
            if (qn == 0 || out_ptr[g + 1] == out_ptr[g])
                continue;
            const uint64_t seg0 = sg;
            uint64_t u = 0;
            for (uint32_t e = out_ptr[g]; e < out_ptr[g + 1]; ++e) {
                const uint32_t x = out_idx[e];
                const uint32_t nx = group_begin[x + 1] - group_begin[x];
                if (nx == 0)
                    continue;
                u += nx;
                pl.seg_start[sg] = group_begin[x];
                pl.seg_vend[sg] = (uint32_t)u;
                ++sg;
            }
            if (u == 0)
                continue;
            Job jb{};
            jb.q_begin = group_begin[g];
            jb.q_count = qn;
            jb.seg_begin = (uint32_t)seg0;
            jb.seg_count = (uint32_t)(sg - seg0);
            jb.n_cand = (uint32_t)u;
            jb.out_row = group_begin[g];
            jb.id_base = 0;
            jb.flags = 0;
            if (tiny_job(qn, u)) {
                pl.jobs[j] = jb; // n_split = 0: no items, partial rows or merge
                pl.tiny[tn++] = make_uint2((uint32_t)j, 0u);
                ++j;
                continue;
            }
            jb.split_v = split_size(u);
            jb.n_split = (uint32_t)((u + jb.split_v - 1) / jb.split_v);
            jb.part_base = (uint32_t)part;
            part += (uint64_t)qn * jb.n_split;
            pl.jobs[j] = jb;
            // split-major: consecutive items are query blocks streaming the same candidates
            for (uint32_t s = 0; s < jb.n_split; ++s)
                for (uint32_t qo = 0; qo < qn; qo += BQ) {
                    Item it{};
                    it.job = (uint32_t)j;
                    it.q_off = qo;
                    it.q_cnt = std::min<uint32_t>(BQ, qn - qo);
                    it.v_begin = s * jb.split_v;
                    it.v_end = (uint32_t)std::min<uint64_t>(u, (uint64_t)(s + 1) * jb.split_v);
                    it.split = s;
                    pl.items[itn++] = it;
                }
            ++j;
        }
    };
    if (nch == 1)
        pass2(0);
    else
        ctx->pool->run(nch, pass2);
    return UNG_HIP_OK;
}

int build_group_plan(ung_hip_ctx *ctx, uint32_t n_groups, const uint32_t *grp_begin, const uint32_t *grp_size,
                     uint32_t list_k, Plan &pl);
int group_prepare_result(ung_hip_ctx *ctx, const Plan &pl, uint32_t list_k);
int group_complete(ung_hip_ctx *ctx, Workspace &ws, const Plan &pl, uint32_t list_k);
int check_not_pending(ung_hip_ctx *ctx, const char *who);

// After a failed call: waits for whatever the workspaces still have in flight, so no
// buffer is reused or freed under a running kernel.  The failed call's result stays
// invalid (cross_prepare_result / group_prepare_result cleared its flag before anything
// was enqueued).  Errors of the waits are ignored: the call's own error is reported.
void drain_after_failure(ung_hip_ctx *ctx)
{
    for (Workspace &w : ctx->ws) {
        if (w.stream)
            (void)hipStreamSynchronize(w.stream);
        if (w.upload)
            (void)hipStreamSynchronize(w.upload);
    }
}

// Result rows of a cross call, initialised (padding) on the first workspace's stream.
int cross_prepare_result(ung_hip_ctx *ctx, uint32_t k)
{
    int rc;
    ResultBufs &res = ctx->cross;
    res.valid = false;
    res.rescanned.clear();
    if ((rc = res.ids.ensure(ctx->N * k)) || (rc = res.dist.ensure(ctx->N * k)) || (rc = res.size.ensure(ctx->N)))
        return rc;
    res.rows = ctx->N;
    res.k = k;
    const uint64_t tot = ctx->N * k;
    if (tot > 0) {
        hipLaunchKernelGGL(ung_fill_rows_kernel, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, ctx->ws[0].stream,
                           res.ids.p, res.dist.p, res.size.p, ctx->N, k);
        HIPCHECK(hipGetLastError());
    }
    return UNG_HIP_OK;
}

int cross_device(ung_hip_ctx *ctx, uint32_t G, const uint32_t *group_begin, const uint32_t *out_ptr,
                 const uint32_t *out_idx, uint32_t k, ung_hip_stats *st)
{
    int rc;
    if ((rc = check_ready(ctx)))
        return rc;
    if (k < 1 || k > 64) {
        set_error("k=%u outside 1..64", k);
        return UNG_HIP_EINVAL;
    }
    if ((rc = set_device(ctx)))
        return rc;
    const auto t0 = clk::now();
    Plan &pl = ctx->plan0;
    plan_reset(pl);
    if ((rc = build_cross_plan(ctx, G, group_begin, out_ptr, out_idx, pl)))
        return rc;
    if (st)
        st->plan_ms += ms_since(t0);
    if ((rc = cross_prepare_result(ctx, k)) || (rc = run_plan(ctx, ctx->ws[0], pl, k, ctx->cross, st))) {
        drain_after_failure(ctx);
        return rc;
    }
    HIPCHECK(hipStreamSynchronize(ctx->ws[0].stream));
    ctx->cross.valid = true;
    pl.part_lp = pick_lp(k, pick_lt(k), ctx->d);
    if (st)
        st->wall_ms += ms_since(t0);
    return UNG_HIP_OK;
}

// Cross edges on the first workspace and a group kNN call on the second, overlapped: the
// group call's kernels start when the cross select ends and run beside the cross merge,
// rescan and whatever the caller does next (additional edges).
int cross_intra_begin(ung_hip_ctx *ctx, uint32_t G, const uint32_t *group_begin, const uint32_t *out_ptr,
                      const uint32_t *out_idx, uint32_t k, uint32_t n_groups, const uint32_t *grp_begin,
                      const uint32_t *grp_size, uint32_t list_k, ung_hip_stats *st)
{
    int rc;
    if ((rc = check_ready(ctx)) || (rc = check_not_pending(ctx, "ung_hip_cross_intra_begin")))
        return rc;
    if (k < 1 || k > 64) {
        set_error("k=%u outside 1..64", k);
        return UNG_HIP_EINVAL;
    }
    if ((rc = set_device(ctx)))
        return rc;
    const auto t0 = clk::now();
    Plan &pl = ctx->plan0;
    plan_reset(pl);
    if ((rc = build_cross_plan(ctx, G, group_begin, out_ptr, out_idx, pl)))
        return rc;
    if (st)
        st->plan_ms += ms_since(t0);
    // both calls are planned and validated before anything is enqueued, so an invalid
    // group list leaves no cross work in flight
    ctx->intra_stats = ung_hip_stats{};
    ctx->intra_t0 = clk::now();
    plan_reset(ctx->intra_plan);
    if ((rc = build_group_plan(ctx, n_groups, grp_begin, grp_size, list_k, ctx->intra_plan)))
        return rc;
    ctx->intra_stats.plan_ms += ms_since(ctx->intra_t0);
    // the group call's kernels start when the cross select ends: they share the chip with
    // the cross merge (bound by its re-score loads), the rescan and the caller's additional
    // edges, whose different bounds fill each other's gaps (cfg2: 17.7 ms a step, against
    // 18.0 ms with the group select alone between the cross merge and the additional edges)
    PlanMem m0;
    if ((rc = cross_prepare_result(ctx, k)) ||
        (rc = workspace_mem(ctx->ws[0], pl, pick_lp(k, pick_lt(k), ctx->d), ctx->cross, m0)) ||
        (rc = plan_launch(ctx, ctx->ws[0], pl, k, m0, st)) ||
        (rc = group_prepare_result(ctx, ctx->intra_plan, list_k)) ||
        (rc = workspace_mem(ctx->ws[1], ctx->intra_plan, pick_lp(list_k, pick_lt(list_k), ctx->d), ctx->group,
                            ctx->intra_mem)) ||
        (rc = plan_launch(ctx, ctx->ws[1], ctx->intra_plan, list_k, ctx->intra_mem, &ctx->intra_stats,
                          ctx->ws[0].ev[1]))) {
        drain_after_failure(ctx);
        return rc;
    }
    // from here the group call is in flight on the second workspace until intra_end
    ctx->intra_list_k = list_k;
    ctx->intra_pending = true;
    rc = plan_finish(ctx, ctx->ws[0], pl, k, m0, st);
    if (rc == UNG_HIP_OK && hipStreamSynchronize(ctx->ws[0].stream) != hipSuccess) {
        set_error("ung_hip_cross_intra_begin: stream synchronisation failed");
        rc = UNG_HIP_EDEVICE;
    }
    if (rc) { // the group call is abandoned with the cross call (its lists stay invalid)
        drain_after_failure(ctx);
        ctx->intra_pending = false;
        return rc;
    }
    ctx->cross.valid = true;
    pl.part_lp = pick_lp(k, pick_lt(k), ctx->d);
    if (st)
        st->wall_ms += ms_since(t0);
    return UNG_HIP_OK;
}

int intra_end(ung_hip_ctx *ctx, ung_hip_stats *st)
{
    int rc;
    if (!ctx || !ctx->intra_pending) {
        set_error("ung_hip_intra_end: no group kNN call in flight");
        return UNG_HIP_ESTATE;
    }
    if ((rc = set_device(ctx)))
        return rc;
    ctx->intra_pending = false;
    const uint32_t list_k = ctx->intra_list_k;
    if ((rc = plan_finish(ctx, ctx->ws[1], ctx->intra_plan, list_k, ctx->intra_mem, &ctx->intra_stats)) ||
        (rc = group_complete(ctx, ctx->ws[1], ctx->intra_plan, list_k))) {
        drain_after_failure(ctx);
        return rc;
    }
    ctx->intra_stats.wall_ms += ms_since(ctx->intra_t0);
    if (st) {
        st->wall_ms += ctx->intra_stats.wall_ms;
        st->plan_ms += ctx->intra_stats.plan_ms;
        st->h2d_ms += ctx->intra_stats.h2d_ms;
        st->kernel_ms += ctx->intra_stats.kernel_ms;
        st->select_ms += ctx->intra_stats.select_ms;
        st->merge_ms += ctx->intra_stats.merge_ms;
        st->fallback_ms += ctx->intra_stats.fallback_ms;
        st->d2h_ms += ctx->intra_stats.d2h_ms;
        st->pairs += ctx->intra_stats.pairs;
        st->rows += ctx->intra_stats.rows;
        st->work_items += ctx->intra_stats.work_items;
        st->select_launches += ctx->intra_stats.select_launches;
        st->fallback_rows += ctx->intra_stats.fallback_rows;
        st->padded_pairs += ctx->intra_stats.padded_pairs;
        st->select_bytes += ctx->intra_stats.select_bytes;
    }
    return UNG_HIP_OK;
}

// Validated job list of a group kNN call: one job per group, its own range as candidates.
int build_group_plan(ung_hip_ctx *ctx, uint32_t n_groups, const uint32_t *grp_begin, const uint32_t *grp_size,
                     uint32_t list_k, Plan &pl)
{
    if (list_k < 1 || list_k > 64) {
        set_error("list_k=%u outside 1..64", list_k);
        return UNG_HIP_EINVAL;
    }
    if (n_groups > 0 && (!grp_begin || !grp_size)) {
        set_error("ung_hip_group_knn: null grp_begin/grp_size");
        return UNG_HIP_EINVAL;
    }
    uint64_t row = 0;
    for (uint32_t g = 0; g < n_groups; ++g) {
        const uint32_t n = grp_size[g];
        if (n == 0 || (uint64_t)grp_begin[g] + n > ctx->N) {
            set_error("ung_hip_group_knn: group %u (begin %u, size %u) invalid for N=%llu (need n>=1)", g,
                      grp_begin[g], n, (unsigned long long)ctx->N);
            return UNG_HIP_EINVAL;
        }
        Job jb{};
        jb.q_begin = grp_begin[g];
        jb.q_count = n;
        jb.seg_begin = (uint32_t)pl.seg_start.size();
        jb.seg_count = 1;
        pl.seg_start.push_back(grp_begin[g]);
        pl.seg_vend.push_back(n);
        jb.n_cand = n;
        // a group with many query blocks keeps its candidates whole: the blocks already
        // spread it over the chip, and splits would multiply its partial rows
        jb.split_v = (n + BQ - 1) / BQ >= 256 ? n : split_size(n);
        jb.n_split = (n + jb.split_v - 1) / jb.split_v;
        pl.max_item_cand = std::max<uint64_t>(pl.max_item_cand, std::min(jb.split_v, n));
        jb.part_base = (uint32_t)pl.part_rows;
        jb.out_row = (uint32_t)row;
        jb.id_base = grp_begin[g];
        jb.flags = 1u;
        pl.part_rows += (uint64_t)n * jb.n_split;
        pl.pairs += (uint64_t)n * (n - 1);
        pl.rows += n;
        row += n;
        if (row >= 0xFFFFFFFFull || pl.part_rows >= 0xFFFFFFFFull) {
            set_error("ung_hip_group_knn: more than 2^32 rows");
            return UNG_HIP_EINVAL;
        }
        pl.jobs.push_back(jb);
        add_items_for_job(pl, (uint32_t)pl.jobs.size() - 1);
    }
    add_pack_items(pl);
    return UNG_HIP_OK;
}

int group_prepare_result(ung_hip_ctx *ctx, const Plan &pl, uint32_t list_k)
{
    int rc;
    ResultBufs &res = ctx->group;
    res.valid = false;
    res.rescanned.clear();
    if ((rc = res.ids.ensure(std::max<uint64_t>(pl.rows * list_k, 1))) ||
        (rc = res.dist.ensure(std::max<uint64_t>(pl.rows * list_k, 1))) ||
        (rc = res.size.ensure(std::max<uint64_t>(pl.rows, 1))))
        return rc;
    res.rows = pl.rows;
    res.k = list_k;
    return UNG_HIP_OK;
}

// Keeps the job table for packing and pruning, marks the lists valid.
int group_complete(ung_hip_ctx *ctx, Workspace &ws, const Plan &pl, uint32_t list_k)
{
    int rc;
    ctx->group_jobs.assign(pl.jobs.begin(), pl.jobs.end());
    ctx->group_pitems = pl.pitems;
    ctx->group_list_k = list_k;
    if (!pl.jobs.empty()) {
        if ((rc = ctx->gjobs.ensure(pl.jobs.size())) || (rc = ctx->gmitems.ensure(pl.pitems.size())))
            return rc;
        HIPCHECK(hipMemcpyAsync(ctx->gjobs.p, pl.jobs.data(), pl.jobs.size() * sizeof(Job), hipMemcpyHostToDevice, ws.stream));
        HIPCHECK(hipMemcpyAsync(ctx->gmitems.p, pl.pitems.data(), pl.pitems.size() * sizeof(MergeItem), hipMemcpyHostToDevice, ws.stream));
    }
    HIPCHECK(hipStreamSynchronize(ws.stream));
    ctx->group.valid = true;
    return UNG_HIP_OK;
}

int check_not_pending(ung_hip_ctx *ctx, const char *who)
{
    if (ctx->intra_pending) {
        set_error("%s: a group kNN call started by ung_hip_cross_intra_begin is in flight (call ung_hip_intra_end first)",
                  who);
        return UNG_HIP_ESTATE;
    }
    return UNG_HIP_OK;
}

int group_device(ung_hip_ctx *ctx, uint32_t n_groups, const uint32_t *grp_begin, const uint32_t *grp_size,
                 uint32_t list_k, ung_hip_stats *st)
{
    int rc;
    if ((rc = check_ready(ctx)) || (rc = check_not_pending(ctx, "ung_hip_group_knn")))
        return rc;
    if ((rc = set_device(ctx)))
        return rc;
    const auto t0 = clk::now();
    Plan &pl = ctx->plan0;
    plan_reset(pl);
    if ((rc = build_group_plan(ctx, n_groups, grp_begin, grp_size, list_k, pl)))
        return rc;
    if (st)
        st->plan_ms += ms_since(t0);
    if ((rc = group_prepare_result(ctx, pl, list_k)) || (rc = run_plan(ctx, ctx->ws[0], pl, list_k, ctx->group, st)) ||
        (rc = group_complete(ctx, ctx->ws[0], pl, list_k))) {
        drain_after_failure(ctx);
        return rc;
    }
    pl.part_lp = pick_lp(list_k, pick_lt(list_k), ctx->d); // partial rows kept for the diagnostics
    if (st)
        st->wall_ms += ms_since(t0);
    return UNG_HIP_OK;
}

// Additional edges (src/uni_nav_graph_cross_edges.cpp:442-596, exact branch :543-562)
// from the resident cross-edge rows, planned and scored on the device: reached out-groups
// are marked, every missing (C, X) entry counts its query rows (C's first m vectors, m
// vectors of min(|X|, num_cross/2) edges each until num_cross are reached) and edges, two
// exclusive scans give each row its place in the per-group edge lists, and one wave per
// row writes its exact nearest members of X there.  The host reads back three totals and
// the finished lists.
int additional_device(ung_hip_ctx *ctx, uint32_t G, const uint32_t *group_begin, const uint32_t *out_ptr,
                      const uint32_t *out_idx, uint32_t num_cross, uint32_t *edge_ptr, uint32_t *edge_from,
                      uint32_t *edge_to, uint64_t capacity, uint64_t *n_edges, ung_hip_stats *st)
{
    int rc;
    if ((rc = check_ready(ctx)))
        return rc;
    if (!ctx->cross.valid) {
        set_error("ung_hip_additional_edges: no cross-edge result on the device (run ung_hip_cross_topk first)");
        return UNG_HIP_ESTATE;
    }
    if (num_cross < 1 || num_cross > ctx->cross.k) {
        set_error("ung_hip_additional_edges: num_cross=%u outside 1..%u (the k of the cross-edge call)", num_cross,
                  ctx->cross.k);
        return UNG_HIP_EINVAL;
    }
    if (!group_begin || !out_ptr || !edge_ptr || !n_edges || (out_ptr[G + 1] > 0 && !out_idx)) {
        set_error("ung_hip_additional_edges: null argument");
        return UNG_HIP_EINVAL;
    }
    if ((uint64_t)group_begin[G + 1] != ctx->N || group_begin[1] != 0) {
        set_error("ung_hip_additional_edges: group_begin[1]=%u, group_begin[G+1]=%u but %llu vectors are prepared",
                  group_begin[1], group_begin[G + 1], (unsigned long long)ctx->N);
        return UNG_HIP_EINVAL;
    }
    for (uint32_t g = 1; g <= G; ++g)
        if (group_begin[g + 1] < group_begin[g] || out_ptr[g + 1] < out_ptr[g]) {
            set_error("ung_hip_additional_edges: group_begin/out_ptr not monotone at group %u", g);
            return UNG_HIP_EINVAL;
        }
    const uint32_t E = out_ptr[G + 1];
    for (uint32_t p = 0; p < E; ++p)
        if (out_idx[p] < 1 || out_idx[p] > G) {
            set_error("ung_hip_additional_edges: out_idx entry %u out of range 1..%u", out_idx[p], G);
            return UNG_HIP_EINVAL;
        }
    // an entry adds at most num_cross query rows and fewer than 3 * num_cross / 2 edges:
    // both running totals stay 32-bit
    if ((uint64_t)E * 2u * num_cross >= 0xFFFFFFFFull) {
        set_error("ung_hip_additional_edges: %u LNG entries x num_cross=%u exceed 32-bit edge offsets", E, num_cross);
        return UNG_HIP_EINVAL;
    }
    if ((rc = set_device(ctx)))
        return rc;
    const auto t0 = clk::now();
    const uint64_t N = ctx->N;
    hipStream_t sm0 = ctx->stream;
    // inputs through pinned staging
    if ((rc = ctx->a_gb.ensure(G + 2)) || (rc = ctx->a_op.ensure(G + 2)) || (rc = ctx->a_oi.ensure(E + 1)) ||
        (rc = ctx->a_pg.ensure(N)) || (rc = ctx->a_reached.ensure(E + 1)) || (rc = ctx->a_eg.ensure(E + 1)) ||
        (rc = ctx->a_rows.ensure(E + 1)) || (rc = ctx->a_edges.ensure(E + 1)) || (rc = ctx->a_items.ensure(E + 1)) ||
        (rc = ctx->a_ptr.ensure(G + 2)) ||
        (rc = ctx->a_cnt.ensure(2)) || (rc = ctx->a_stage.ensure(((size_t)2 * (G + 2) + E + 4) * sizeof(uint32_t))))
        return rc;
    uint32_t *hs = static_cast<uint32_t *>(ctx->a_stage.p);
    std::memcpy(hs, group_begin, (G + 2) * sizeof(uint32_t));
    std::memcpy(hs + (G + 2), out_ptr, (G + 2) * sizeof(uint32_t));
    if (E)
        std::memcpy(hs + 2 * (G + 2), out_idx, E * sizeof(uint32_t));
    HIPCHECK(hipMemcpyAsync(ctx->a_gb.p, hs, (G + 2) * sizeof(uint32_t), hipMemcpyHostToDevice, sm0));
    HIPCHECK(hipMemcpyAsync(ctx->a_op.p, hs + (G + 2), (G + 2) * sizeof(uint32_t), hipMemcpyHostToDevice, sm0));
    if (E)
        HIPCHECK(hipMemcpyAsync(ctx->a_oi.p, hs + 2 * (G + 2), E * sizeof(uint32_t), hipMemcpyHostToDevice, sm0));
    HIPCHECK(hipEventRecord(ctx->ev[0], sm0));
    // step 1: reached entries; step 2: rows and edges per entry, their scans
    const unsigned eb = (unsigned)std::min<uint64_t>((E + 256) / 256, 65535);
    hipLaunchKernelGGL(ung_zero_u32_kernel, dim3(eb), dim3(256), 0, sm0, ctx->a_reached.p, E + 1);
    hipLaunchKernelGGL(ung_zero_u32_kernel, dim3(eb), dim3(256), 0, sm0, ctx->a_eg.p, E + 1);
    hipLaunchKernelGGL(ung_zero_u32_kernel, dim3(1), dim3(64), 0, sm0, reinterpret_cast<uint32_t *>(ctx->a_cnt.p), 4u);
    hipLaunchKernelGGL(ung_point_group_kernel, dim3(std::max<uint32_t>(1u, std::min<uint32_t>(G, 65535u))), dim3(256),
                       0, sm0, ctx->a_gb.p, G, ctx->a_pg.p);
    hipLaunchKernelGGL(ung_point_group_kernel, dim3(std::max<uint32_t>(1u, std::min<uint32_t>(G, 65535u))), dim3(256),
                       0, sm0, ctx->a_op.p, G, ctx->a_eg.p);
    HIPCHECK(hipGetLastError());
    if (E > 0 && num_cross / 2 > 0) {
        hipLaunchKernelGGL(ung_addl_mark_kernel, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, sm0,
                           ctx->cross.ids.p, ctx->cross.k, num_cross, ctx->a_pg.p, N, ctx->a_op.p, ctx->a_oi.p,
                           ctx->a_reached.p);
        HIPCHECK(hipGetLastError());
    }
    hipLaunchKernelGGL(ung_addl_count_kernel, dim3(eb), dim3(256), 0, sm0, ctx->a_gb.p, ctx->a_oi.p, ctx->a_eg.p,
                       ctx->a_reached.p, E, num_cross, ctx->a_rows.p, ctx->a_edges.p, ctx->a_items.p, ctx->a_cnt.p);
    HIPCHECK(hipGetLastError());
    hipLaunchKernelGGL(ung_zero_u32_kernel, dim3(1), dim3(64), 0, sm0, ctx->a_rows.p + E, 1u);
    hipLaunchKernelGGL(ung_zero_u32_kernel, dim3(1), dim3(64), 0, sm0, ctx->a_edges.p + E, 1u);
    hipLaunchKernelGGL(ung_zero_u32_kernel, dim3(1), dim3(64), 0, sm0, ctx->a_items.p + E, 1u);
    size_t tmp = 0, tmp2 = 0;
    HIPCHECK(hipcub::DeviceScan::ExclusiveSum(nullptr, tmp, ctx->a_rows.p, ctx->a_rows.p, (int)(E + 1), sm0));
    HIPCHECK(hipcub::DeviceScan::ExclusiveSum(nullptr, tmp2, ctx->a_edges.p, ctx->a_edges.p, (int)(E + 1), sm0));
    if ((rc = ctx->a_tmp.ensure(std::max(tmp, tmp2) + 1)))
        return rc;
    HIPCHECK(hipcub::DeviceScan::ExclusiveSum(ctx->a_tmp.p, tmp, ctx->a_rows.p, ctx->a_rows.p, (int)(E + 1), sm0));
    HIPCHECK(hipcub::DeviceScan::ExclusiveSum(ctx->a_tmp.p, tmp2, ctx->a_edges.p, ctx->a_edges.p, (int)(E + 1), sm0));
    HIPCHECK(hipcub::DeviceScan::ExclusiveSum(ctx->a_tmp.p, tmp2, ctx->a_items.p, ctx->a_items.p, (int)(E + 1), sm0));
    uint32_t totals[3] = {0, 0, 0};
    unsigned long long cnt[2] = {0, 0};
    HIPCHECK(hipMemcpyAsync(&totals[0], ctx->a_rows.p + E, sizeof(uint32_t), hipMemcpyDeviceToHost, sm0));
    HIPCHECK(hipMemcpyAsync(&totals[1], ctx->a_edges.p + E, sizeof(uint32_t), hipMemcpyDeviceToHost, sm0));
    HIPCHECK(hipMemcpyAsync(&totals[2], ctx->a_items.p + E, sizeof(uint32_t), hipMemcpyDeviceToHost, sm0));
    HIPCHECK(hipMemcpyAsync(cnt, ctx->a_cnt.p, sizeof(cnt), hipMemcpyDeviceToHost, sm0));
    HIPCHECK(hipStreamSynchronize(sm0));
    const uint32_t R = totals[0], I = totals[2];
    // the scan items (at most R + pairs / ADDL_RANGE) were counted in 32 bits
    if ((uint64_t)R + cnt[0] / ADDL_RANGE >= 0xFFFFFFFFull) {
        set_error("ung_hip_additional_edges: %llu target vectors to scan exceed 32-bit item counts",
                  (unsigned long long)cnt[0]);
        return UNG_HIP_EINVAL;
    }
    const uint64_t total_edges = totals[1];
    *n_edges = total_edges;
    if (st)
        st->plan_ms += ms_since(t0);
    if (total_edges > capacity || (total_edges > 0 && (!edge_from || !edge_to))) {
        set_error("ung_hip_additional_edges: %llu edges need capacity (got %llu)", (unsigned long long)total_edges,
                  (unsigned long long)capacity);
        return UNG_HIP_EINVAL;
    }
    // step 3: the scans, written in place; per-group offsets
    const uint32_t per_max = num_cross / 2;
    if ((rc = ctx->a_from.ensure(total_edges + 1)) || (rc = ctx->a_to.ensure(total_edges + 1)) ||
        (rc = ctx->a_ientry.ensure((uint64_t)I + 1)) || (rc = ctx->a_pid.ensure((uint64_t)I * per_max + 1)) ||
        (rc = ctx->a_pdist.ensure((uint64_t)I * per_max + 1)))
        return rc;
    HIPCHECK(hipEventRecord(ctx->ev[1], sm0));
    if (R > 0) {
        AddlParams A{};
        A.X = ctx->X;
        A.d = ctx->d;
        A.gb = ctx->a_gb.p;
        A.oi = ctx->a_oi.p;
        A.eg = ctx->a_eg.p;
        A.row_off = ctx->a_rows.p;
        A.edge_off = ctx->a_edges.p;
        A.item_off = ctx->a_items.p;
        A.item_entry = ctx->a_ientry.p;
        A.E = E;
        A.I = I;
        A.per_max = per_max;
        A.part_ids = ctx->a_pid.p;
        A.part_dist = ctx->a_pdist.p;
        A.from = ctx->a_from.p;
        A.to = ctx->a_to.p;
        hipLaunchKernelGGL(ung_addl_small_kernel, dim3((E + 3) / 4), dim3(256), 0, sm0, A);
        HIPCHECK(hipGetLastError());
        if (I > 0) {
            hipLaunchKernelGGL(ung_addl_expand_kernel, dim3(std::min<uint32_t>((E + 255) / 256, 65535u)), dim3(256), 0,
                               sm0, ctx->a_items.p, E, ctx->a_ientry.p);
            hipLaunchKernelGGL(ung_addl_scan_kernel, dim3(std::min<uint32_t>(I, 262144u)), dim3(64), 0, sm0, A);
            hipLaunchKernelGGL(ung_addl_merge_kernel, dim3(std::min<uint32_t>(I, 65536u)), dim3(64), 0, sm0, A);
            HIPCHECK(hipGetLastError());
        }
    }
    hipLaunchKernelGGL(ung_addl_ptr_kernel, dim3((G + 2 + 255) / 256), dim3(256), 0, sm0, ctx->a_op.p, ctx->a_edges.p,
                       G, ctx->a_ptr.p);
    HIPCHECK(hipGetLastError());
    HIPCHECK(hipEventRecord(ctx->ev[2], sm0));
    const auto t1 = clk::now();
    HIPCHECK(hipMemcpyAsync(edge_ptr, ctx->a_ptr.p, (G + 2) * sizeof(uint32_t), hipMemcpyDeviceToHost, sm0));
    if (total_edges) {
        HIPCHECK(hipMemcpyAsync(edge_from, ctx->a_from.p, total_edges * sizeof(uint32_t), hipMemcpyDeviceToHost, sm0));
        HIPCHECK(hipMemcpyAsync(edge_to, ctx->a_to.p, total_edges * sizeof(uint32_t), hipMemcpyDeviceToHost, sm0));
    }
    HIPCHECK(hipStreamSynchronize(sm0));
    if (st) {
        float k1 = 0, k2 = 0;
        HIPCHECK(hipEventElapsedTime(&k1, ctx->ev[0], ctx->ev[1]));
        HIPCHECK(hipEventElapsedTime(&k2, ctx->ev[1], ctx->ev[2]));
        st->fallback_ms += k2;
        st->kernel_ms += k1 + k2;
        st->d2h_ms += ms_since(t1);
        st->rows += R;
        st->pairs += cnt[0];
        st->work_items += cnt[1];
        st->wall_ms += ms_since(t0);
    }
    return UNG_HIP_OK;
}

// Device-to-host copy of result regions into the caller's (pageable) memory through the
// context's pinned staging: the regions are cut into pieces of DL_PIECE bytes that cycle
// through DL_SLOTS pinned slots.  One run of the worker pool does all host copies: worker
// t copies part t of every piece in order (waiting for the piece's DMA event), and the
// worker that finishes a piece's last part enqueues the DMA of the piece that reuses its
// slot.  So the DMA engine fills the next slots while the host threads copy the finished
// piece into the caller's memory (first-touch page faults of a fresh destination
// included), and the transfer runs near the link's pinned rate instead of the runtime's
// single-threaded pageable path.  Small copies go straight through.
constexpr size_t DL_PIECE = 8u << 20;
constexpr int DL_SLOTS = 4;
constexpr size_t DL_DIRECT = 1u << 20; // below this, one plain copy

struct DlRegion {
    void *dst;
    const void *src;
    size_t bytes;
};

int download_regions(ung_hip_ctx *ctx, hipStream_t stream, const DlRegion *reg, int nreg)
{
    size_t total = 0;
    for (int r = 0; r < nreg; ++r)
        total += reg[r].dst ? reg[r].bytes : 0;
    if (total < DL_DIRECT || !ctx->pool || ctx->pool->size() < 2) {
        for (int r = 0; r < nreg; ++r)
            if (reg[r].dst && reg[r].bytes)
                HIPCHECK(hipMemcpyAsync(reg[r].dst, reg[r].src, reg[r].bytes, hipMemcpyDeviceToHost, stream));
        HIPCHECK(hipStreamSynchronize(stream));
        return UNG_HIP_OK;
    }
    int rc;
    if ((rc = ctx->dl_stage.ensure(DL_PIECE * DL_SLOTS)))
        return rc;
    struct Piece {
        char *dst;
        const char *src;
        size_t bytes;
    };
    std::vector<Piece> pieces;
    for (int r = 0; r < nreg; ++r) {
        if (!reg[r].dst)
            continue;
        for (size_t o = 0; o < reg[r].bytes; o += DL_PIECE)
            pieces.push_back(Piece{static_cast<char *>(reg[r].dst) + o, static_cast<const char *>(reg[r].src) + o,
                                   std::min(DL_PIECE, reg[r].bytes - o)});
    }
    const size_t np = pieces.size();
    while (ctx->dl_ev.size() < np) {
        hipEvent_t ev = nullptr;
        HIPCHECK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
        ctx->dl_ev.push_back(ev);
    }
    char *stage = static_cast<char *>(ctx->dl_stage.p);
    // enqueue[i]: DMA of piece i into its slot and its event (the event is recorded before
    // the flag is raised, so a worker that sees the flag waits on this piece's DMA)
    std::unique_ptr<std::atomic<int>[]> queued(new std::atomic<int>[np]);
    std::unique_ptr<std::atomic<int>[]> done(new std::atomic<int>[np]);
    for (size_t i = 0; i < np; ++i) {
        queued[i].store(0, std::memory_order_relaxed);
        done[i].store(0, std::memory_order_relaxed);
    }
    std::atomic<int> failed{0};
    auto enqueue = [&](size_t i) -> int {
        const size_t slot = i % DL_SLOTS;
        if (hipMemcpyAsync(stage + slot * DL_PIECE, pieces[i].src, pieces[i].bytes, hipMemcpyDeviceToHost, stream) !=
                hipSuccess ||
            hipEventRecord(ctx->dl_ev[i], stream) != hipSuccess)
            return UNG_HIP_EDEVICE;
        queued[i].store(1, std::memory_order_release);
        return UNG_HIP_OK;
    };
    for (size_t i = 0; i < np && i < (size_t)DL_SLOTS; ++i)
        if (enqueue(i) != UNG_HIP_OK) {
            (void)hipStreamSynchronize(stream);
            set_error("download: device-to-host copy failed");
            return UNG_HIP_EDEVICE;
        }
    const int T = ctx->pool->size();
    const int device = ctx->device;
    ctx->pool->run(T, [&](int64_t t) {
        (void)hipSetDevice(device);
        for (size_t i = 0; i < np; ++i) {
            while (!queued[i].load(std::memory_order_acquire)) {
                if (failed.load(std::memory_order_relaxed))
                    return;
                std::this_thread::yield();
            }
            if (hipEventSynchronize(ctx->dl_ev[i]) != hipSuccess) {
                failed.store(1);
                return;
            }
            const Piece &pc = pieces[i];
            const size_t b0 = pc.bytes * (size_t)t / (size_t)T, b1 = pc.bytes * (size_t)(t + 1) / (size_t)T;
            std::memcpy(pc.dst + b0, stage + (i % DL_SLOTS) * DL_PIECE + b0, b1 - b0);
            // the last part of piece i frees its slot for piece i + DL_SLOTS
            if (done[i].fetch_add(1, std::memory_order_acq_rel) == T - 1 && i + DL_SLOTS < np &&
                enqueue(i + DL_SLOTS) != UNG_HIP_OK)
                failed.store(1);
        }
    });
    if (failed.load()) {
        (void)hipStreamSynchronize(stream);
        set_error("download: device-to-host copy failed");
        return UNG_HIP_EDEVICE;
    }
    return UNG_HIP_OK;
}

int download(ung_hip_ctx *ctx, ResultBufs &res, uint32_t *ids, float *dist, int32_t *size, ung_hip_stats *st)
{
    if (!res.valid) {
        set_error("no result to download (run the corresponding *_device call first)");
        return UNG_HIP_ESTATE;
    }
    if (!ids) {
        set_error("null output ids");
        return UNG_HIP_EINVAL;
    }
    const auto t0 = clk::now();
    const size_t n = (size_t)res.rows * res.k;
    const DlRegion reg[3] = {{ids, res.ids.p, n * sizeof(uint32_t)},
                             {dist, res.dist.p, n * sizeof(float)},
                             {size, res.size.p, (size_t)res.rows * sizeof(int32_t)}};
    int rc;
    if ((rc = download_regions(ctx, ctx->stream, reg, 3)))
        return rc;
    if (st)
        st->d2h_ms += ms_since(t0);
    return UNG_HIP_OK;
}

int prepare_common(ung_hip_ctx *ctx, const float *src, bool src_device, uint64_t N, uint32_t dim, ung_hip_stats *st)
{
    if (!ctx || !src || dim == 0 || N == 0 || N >= 0xFFFFFFFFull) {
        set_error("ung_hip_prepare_vectors: bad arguments (N=%llu dim=%u)", (unsigned long long)N, dim);
        return UNG_HIP_EINVAL;
    }
    int rc;
    if ((rc = check_not_pending(ctx, "ung_hip_prepare_vectors")) || (rc = set_device(ctx)))
        return rc;
    ung_hip_release_vectors(ctx);
    const auto t0 = clk::now();
    const uint32_t dp = (dim + KC - 1) / KC * KC;
    HIPCHECK(counted_malloc((void **)&ctx->X, N * dim * sizeof(float)));
    HIPCHECK(counted_malloc((void **)&ctx->XS, N * dp * sizeof(uint32_t)));
    HIPCHECK(counted_malloc((void **)&ctx->xn, N * sizeof(float)));
    HIPCHECK(counted_malloc((void **)&ctx->maxbits, sizeof(unsigned int)));
    HIPCHECK(hipMemcpyAsync(ctx->X, src, N * dim * sizeof(float),
                            src_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, ctx->stream));
    hipLaunchKernelGGL(ung_zero_u32_kernel, dim3(1), dim3(64), 0, ctx->stream, (uint32_t *)ctx->maxbits, 1u);
    HIPCHECK(hipGetLastError());
    HIPCHECK(hipStreamSynchronize(ctx->stream));
    const double h2d = ms_since(t0);
    HIPCHECK(hipEventRecord(ctx->ev[4], ctx->stream));
    const uint64_t norm_blocks = std::min<uint64_t>((N + 3) / 4, 8192);
    hipLaunchKernelGGL(ung_norm_kernel, dim3((unsigned)norm_blocks), dim3(256), 0, ctx->stream, ctx->X, N, dim,
                       ctx->xn, ctx->maxbits);
    HIPCHECK(hipGetLastError());
    const uint64_t split_blocks = std::min<uint64_t>((N * (dp / 2) + 255) / 256, 16384);
    hipLaunchKernelGGL(ung_split_kernel, dim3((unsigned)split_blocks), dim3(256), 0, ctx->stream, ctx->X, N, dim, dp,
                       ctx->XS);
    HIPCHECK(hipGetLastError());
    HIPCHECK(hipEventRecord(ctx->ev[5], ctx->stream));
    unsigned int mb = 0;
    HIPCHECK(hipMemcpyAsync(&mb, ctx->maxbits, sizeof(mb), hipMemcpyDeviceToHost, ctx->stream));
    HIPCHECK(hipStreamSynchronize(ctx->stream));
    float mxf;
    std::memcpy(&mxf, &mb, sizeof(mxf));
    // the pinned staging of result downloads, once per context at set-up (not in the
    // first download's time)
    if ((rc = ctx->dl_stage.ensure(DL_PIECE * DL_SLOTS)))
        return rc;
    ctx->N = N;
    ctx->d = dim;
    ctx->dp = dp;
    // max norm, inflated for the rounding of the norm cache
    ctx->rmax = std::sqrt((double)mxf * (1.0 + 1e-5)) * (1.0 + 1e-6);
    ctx->cross.valid = false;
    ctx->group.valid = false;
    if (st) {
        float kms = 0;
        HIPCHECK(hipEventElapsedTime(&kms, ctx->ev[4], ctx->ev[5]));
        st->h2d_ms += h2d;
        st->kernel_ms += kms;
        st->wall_ms += ms_since(t0);
    }
    return UNG_HIP_OK;
}

} // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// Scratch of ung_hip_cross_topk_noalloc: one file-scope device array per GPU, held until
// the process ends.  In host code `scratch` only names the symbol: kernels get the
// device address resolved by hipGetSymbolAddress (per device, at ung_hip_create).
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[UNG_HIP_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int MAX_SCRATCH_DEVICES = 64;
std::mutex g_scratch_mu;
unsigned char *g_scratch_addr[MAX_SCRATCH_DEVICES] = {};
// Held by a no-allocation call for as long as it uses its device's scratch array, so that
// calls on one GPU from several host threads or contexts run one after the other.
std::mutex g_scratch_call_mu[MAX_SCRATCH_DEVICES];

// The device address of `scratch` on `device` (current), resolved once per device.
int resolve_scratch(int device, unsigned char **addr)
{
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device < 0 || device >= MAX_SCRATCH_DEVICES) {
        set_error("no scratch address table entry for device %d", device);
        return UNG_HIP_EINVAL;
    }
    if (!g_scratch_addr[device]) {
        void *ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", device, hipGetErrorString(e));
            return UNG_HIP_EDEVICE;
        }
        g_scratch_addr[device] = static_cast<unsigned char *>(ptr);
    }
    *addr = g_scratch_addr[device];
    return UNG_HIP_OK;
}

// Carves a planned cross call's memory out of the scratch array: work lists, partial rows
// and flags first, the rest for the rescan's range partials.  UNG_HIP_EINVAL when the plan
// does not fit.
int scratch_mem(ung_hip_ctx *ctx, const Plan &pl, uint32_t lp, PlanMem &m)
{
    auto al = [](uint64_t b) { return (b + 255) & ~(uint64_t)255; };
    uint64_t off = 0;
    auto take = [&](uint64_t bytes) {
        const uint64_t at = off;
        off += al(bytes);
        return at;
    };
    const uint64_t o_jobs = take(pl.jobs.size() * sizeof(Job));
    const uint64_t o_items = take(pl.items.size() * sizeof(Item));
    const uint64_t o_mitems = take(pl.n_mitems * sizeof(MergeItem));
    const uint64_t o_ss = take(pl.seg_start.size() * sizeof(uint32_t));
    const uint64_t o_sv = take(pl.seg_vend.size() * sizeof(uint32_t));
    const uint64_t o_pid = take(pl.part_rows * lp * sizeof(uint32_t));
    const uint64_t o_pd = take(pl.part_rows * lp * sizeof(float));
    const uint64_t o_pb = take(pl.part_rows * sizeof(float));
    const uint64_t o_fc = take(2 * sizeof(uint32_t));
    const uint64_t o_fl = take(std::max<uint64_t>(pl.rows, 1) * sizeof(uint2));
    const uint64_t o_tiny = take((pl.n_tiny + 1) * sizeof(uint2));
    if (off > UNG_HIP_NOALLOC_SCRATCH_BYTES) {
        set_error("ung_hip_cross_topk_noalloc: the call needs %llu bytes of scratch, the maximum is %llu "
                  "(use ung_hip_cross_topk_device)",
                  (unsigned long long)off, (unsigned long long)UNG_HIP_NOALLOC_SCRATCH_BYTES);
        return UNG_HIP_EINVAL;
    }
    unsigned char *b = ctx->scratch_dev;
    m.jobs = reinterpret_cast<Job *>(b + o_jobs);
    m.items = reinterpret_cast<Item *>(b + o_items);
    m.mitems = reinterpret_cast<MergeItem *>(b + o_mitems);
    m.seg_start = reinterpret_cast<uint32_t *>(b + o_ss);
    m.seg_vend = reinterpret_cast<uint32_t *>(b + o_sv);
    m.part_ids = reinterpret_cast<uint32_t *>(b + o_pid);
    m.part_dist = reinterpret_cast<float *>(b + o_pd);
    m.part_bound = reinterpret_cast<float *>(b + o_pb);
    m.flag_count = reinterpret_cast<uint32_t *>(b + o_fc);
    m.flagged = reinterpret_cast<uint2 *>(b + o_fl);
    m.tiny = reinterpret_cast<uint2 *>(b + o_tiny);
    const uint64_t rest = UNG_HIP_NOALLOC_SCRATCH_BYTES - off;
    m.fb_grow = false;
    m.fb_cap = rest / (sizeof(uint32_t) + sizeof(float)) / 64 * 64;
    m.fb_ids = reinterpret_cast<uint32_t *>(b + off);
    m.fb_dist = reinterpret_cast<float *>(b + off + al(m.fb_cap * sizeof(uint32_t)));
    if (off + al(m.fb_cap * sizeof(uint32_t)) + m.fb_cap * sizeof(float) > UNG_HIP_NOALLOC_SCRATCH_BYTES)
        m.fb_cap = 0; // (alignment left too little room: one range per rescanned row)
    return UNG_HIP_OK;
}

// p must be device memory of `device` with at least `bytes` bytes from p to the end of
// its allocation (hipMemGetAddressRange), so the kernels' writes stay inside it.
int check_device_ptr(const void *p, uint64_t bytes, int device, const char *what)
{
    hipPointerAttribute_t a{};
    if (!p || hipPointerGetAttributes(&a, p) != hipSuccess || a.type != hipMemoryTypeDevice || a.device != device) {
        (void)hipGetLastError();
        set_error("ung_hip_cross_topk_noalloc: %s is not device memory of device %d", what, device);
        return UNG_HIP_EINVAL;
    }
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p) != hipSuccess || !base) {
        (void)hipGetLastError();
        set_error("ung_hip_cross_topk_noalloc: the allocation holding %s was not found", what);
        return UNG_HIP_EINVAL;
    }
    const uint64_t off = (uint64_t)((const char *)p - (const char *)base);
    if (off > size || size - off < bytes) {
        set_error("ung_hip_cross_topk_noalloc: %s has %llu bytes to the end of its allocation, the call writes %llu",
                  what, (unsigned long long)(off > size ? 0 : size - off), (unsigned long long)bytes);
        return UNG_HIP_EINVAL;
    }
    return UNG_HIP_OK;
}

int cross_noalloc(ung_hip_ctx *ctx, uint32_t G, const uint32_t *group_begin, const uint32_t *out_ptr,
                  const uint32_t *out_idx, uint32_t k, uint32_t *ids, float *dist, int32_t *size, ung_hip_stats *st)
{
    int rc;
    if ((rc = check_ready(ctx)))
        return rc;
    if (k < 1 || k > 64) {
        set_error("k=%u outside 1..64", k);
        return UNG_HIP_EINVAL;
    }
    if (!ctx->scratch_dev) {
        set_error("ung_hip_cross_topk_noalloc: the scratch array of device %d was not resolved", ctx->device);
        return UNG_HIP_ESTATE;
    }
    if (ctx->device < 0 || ctx->device >= MAX_SCRATCH_DEVICES) {
        set_error("ung_hip_cross_topk_noalloc: device %d has no scratch array", ctx->device);
        return UNG_HIP_EINVAL;
    }
    const uint64_t row_bytes = ctx->N * k * 4u;
    if ((rc = set_device(ctx)) || (rc = check_device_ptr(ids, row_bytes, ctx->device, "out_ids_dev")) ||
        (rc = check_device_ptr(dist, row_bytes, ctx->device, "out_dist_dev")) ||
        (rc = check_device_ptr(size, ctx->N * 4u, ctx->device, "out_size_dev")))
        return rc;
    const auto t0 = clk::now();
    // the rows of the context's last allocating cross call are not this call's: the entry
    // points that describe "the last cross-edge call" refuse until the next such call
    ctx->cross.valid = false;
    ctx->cross.rescanned.clear();
    Plan &pl = ctx->plan0;
    plan_reset(pl);
    if ((rc = build_cross_plan(ctx, G, group_begin, out_ptr, out_idx, pl)))
        return rc;
    if (st)
        st->plan_ms += ms_since(t0);
    // this device's scratch array is this call's until its last kernel has finished
    std::lock_guard<std::mutex> scratch_lock(g_scratch_call_mu[ctx->device]);
    PlanMem m;
    if ((rc = scratch_mem(ctx, pl, pick_lp(k, pick_lt(k), ctx->d), m)))
        return rc;
    const size_t stage_bytes = stage_layout(pl).total;
    if (ctx->noalloc_stage.size() < stage_bytes) // host memory, reused by later calls
        ctx->noalloc_stage.resize(stage_bytes);
    m.stage = ctx->noalloc_stage.data();
    ctx->noalloc_rescanned.clear();
    m.rescanned = &ctx->noalloc_rescanned;
    m.out_ids = ids;
    m.out_dist = dist;
    m.out_size = size;
    Workspace &ws = ctx->ws[0];
    const uint64_t tot = ctx->N * k;
    if (tot > 0) { // padding of the rows no job writes
        hipLaunchKernelGGL(ung_fill_rows_kernel, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, ws.stream, ids,
                           dist, size, ctx->N, k);
        rc = hipGetLastError() == hipSuccess ? UNG_HIP_OK : UNG_HIP_EDEVICE;
        if (rc)
            set_error("ung_fill_rows_kernel launch failed");
    }
    if (rc || (rc = plan_launch(ctx, ws, pl, k, m, st)) || (rc = plan_finish(ctx, ws, pl, k, m, st))) {
        drain_after_failure(ctx);
        return rc;
    }
    HIPCHECK(hipStreamSynchronize(ws.stream));
    if (st)
        st->wall_ms += ms_since(t0);
    return UNG_HIP_OK;
}

} // namespace

extern "C" {

const char *ung_hip_version(void) { return "ung_hip 0.2 (gfx950, split-bf16 MFMA pre-select + exact fp32 re-rank)"; }

int ung_hip_create(int device, ung_hip_ctx **out)
{
    clear_error();
    if (!out) {
        set_error("ung_hip_create: null out");
        return UNG_HIP_EINVAL;
    }
    *out = nullptr;
    int ndev = 0;
    HIPCHECK(hipGetDeviceCount(&ndev));
    if (device < 0 || device >= ndev) {
        set_error("ung_hip_create: device %d not present (%d devices)", device, ndev);
        return UNG_HIP_EINVAL;
    }
    HIPCHECK(hipSetDevice(device));
    ung_hip_ctx *ctx = new ung_hip_ctx();
    ctx->device = device;
    if (const char *s = std::getenv("UNG_HIP_FORCE_WIDE"))
        ctx->force_wide = s[0] == '1';
    if (const char *s = std::getenv("UNG_HIP_NO_QREG"))
        ctx->qreg = s[0] != '1';
    if (const char *s = std::getenv("UNG_HIP_NO_KNN"))
        ctx->knn = s[0] != '1';
    if (const char *s = std::getenv("UNG_HIP_PRUNE_EXACT"); s && s[0] == '1')
        ctx->prune_mode = 1;
    if (const char *s = std::getenv("UNG_HIP_PRUNE_GRAM"); s && s[0] == '1')
        ctx->prune_mode = 2;
    if (const char *s = std::getenv("UNG_HIP_EPS_SCALE")) {
        const double v = std::atof(s);
        ctx->eps_scale = v >= 1.0 ? v : 1.0; // a smaller bound would not be an error bound
    }
    hipError_t e = hipSuccess;
    for (auto &w : ctx->ws) { // all streams at the default priority
        e = hipStreamCreateWithFlags(&w.stream, hipStreamNonBlocking);
        if (e == hipSuccess)
            e = hipStreamCreateWithFlags(&w.upload, hipStreamNonBlocking);
        if (e == hipSuccess)
            e = hipEventCreateWithFlags(&w.ev_up, hipEventDisableTiming);
        for (auto &ev : w.ev)
            if (e == hipSuccess)
                e = hipEventCreate(&ev);
        if (e != hipSuccess)
            break;
    }
    ctx->stream = ctx->ws[0].stream;
    for (auto &ev : ctx->ev)
        if (e == hipSuccess)
            e = hipEventCreate(&ev);
    if (e != hipSuccess) {
        set_error("stream/event creation failed: %s", hipGetErrorString(e));
        ung_hip_destroy(ctx);
        return UNG_HIP_EDEVICE;
    }
    {
        // host threads for planning: UNG_HIP_HOST_THREADS, else OMP_NUM_THREADS, else the
        // hardware's (at most 16)
        int nt = 0;
        if (const char *v = std::getenv("UNG_HIP_HOST_THREADS"))
            nt = std::atoi(v);
        else if (const char *v2 = std::getenv("OMP_NUM_THREADS"))
            nt = std::atoi(v2);
        if (nt <= 0)
            nt = std::min(16, ung::resolve_threads(0));
        ctx->pool = std::make_unique<ung::WorkerPool>(std::min(nt, 64));
    }
    int rc = resolve_scratch(device, &ctx->scratch_dev);
    if (rc) {
        ung_hip_destroy(ctx);
        return rc;
    }
    *out = ctx;
    return UNG_HIP_OK;
}

int ung_hip_release_vectors(ung_hip_ctx *ctx)
{
    clear_error();
    if (!ctx) {
        set_error("null context");
        return UNG_HIP_EINVAL;
    }
    int rc;
    if ((rc = check_not_pending(ctx, "ung_hip_release_vectors")))
        return rc;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream)
        (void)hipStreamSynchronize(ctx->stream);
    if (ctx->X)
        (void)hipFree(ctx->X);
    if (ctx->XS)
        (void)hipFree(ctx->XS);
    if (ctx->xn)
        (void)hipFree(ctx->xn);
    if (ctx->maxbits)
        (void)hipFree(ctx->maxbits);
    ctx->X = nullptr;
    ctx->XS = nullptr;
    ctx->dp = 0;
    ctx->xn = nullptr;
    ctx->maxbits = nullptr;
    ctx->N = 0;
    ctx->d = 0;
    ctx->cross.valid = false;
    ctx->group.valid = false;
    ctx->plan0.part_lp = 0; // partial rows of the released base set
    return UNG_HIP_OK;
}

int ung_hip_destroy(ung_hip_ctx *ctx)
{
    clear_error();
    if (!ctx)
        return UNG_HIP_OK;
    (void)hipSetDevice(ctx->device);
    for (auto &w : ctx->ws)
        if (w.stream)
            (void)hipStreamSynchronize(w.stream);
    ctx->intra_pending = false;
    ung_hip_release_vectors(ctx);
    for (auto &w : ctx->ws)
        w.release();
    ctx->cross.release();
    ctx->group.release();
    ctx->gjobs.release();
    ctx->gmitems.release();
    ctx->graph.release();
    ctx->rv_cnt.release();
    ctx->rv_fill.release();
    ctx->rv_src.release();
    ctx->rv_dist.release();
    ctx->rv_tmp.release();
    ctx->a_gb.release();
    ctx->a_op.release();
    ctx->a_oi.release();
    ctx->a_pg.release();
    ctx->a_reached.release();
    ctx->a_eg.release();
    ctx->a_rows.release();
    ctx->a_edges.release();
    ctx->a_ptr.release();
    ctx->a_from.release();
    ctx->a_to.release();
    ctx->a_cnt.release();
    ctx->a_tmp.release();
    ctx->a_stage.release();
    ctx->dl_stage.release();
    for (hipEvent_t ev : ctx->dl_ev)
        if (ev)
            (void)hipEventDestroy(ev);
    ctx->dl_ev.clear();
    for (auto &ev : ctx->ev)
        if (ev)
            (void)hipEventDestroy(ev);
    for (auto &w : ctx->ws) {
        for (auto &ev : w.ev)
            if (ev)
                (void)hipEventDestroy(ev);
        if (w.ev_up)
            (void)hipEventDestroy(w.ev_up);
        if (w.upload)
            (void)hipStreamDestroy(w.upload);
        if (w.stream)
            (void)hipStreamDestroy(w.stream);
    }
    delete ctx;
    return UNG_HIP_OK;
}

int ung_hip_prepare_vectors(ung_hip_ctx *ctx, const float *X, uint64_t N, uint32_t dim, ung_hip_stats *st)
{
    clear_error();
    AllocCount alloc_count(st);
    return prepare_common(ctx, X, false, N, dim, st);
}

int ung_hip_prepare_vectors_device(ung_hip_ctx *ctx, const float *X_dev, uint64_t N, uint32_t dim,
                                   ung_hip_stats *st)
{
    clear_error();
    AllocCount alloc_count(st);
    return prepare_common(ctx, X_dev, true, N, dim, st);
}

int ung_hip_cross_topk_device(ung_hip_ctx *ctx, uint32_t G, const uint32_t *group_begin, const uint32_t *out_ptr,
                              const uint32_t *out_idx, uint32_t k, ung_hip_stats *st)
{
    clear_error();
    AllocCount alloc_count(st);
    return cross_device(ctx, G, group_begin, out_ptr, out_idx, k, st);
}

int ung_hip_cross_topk(ung_hip_ctx *ctx, uint32_t G, const uint32_t *group_begin, const uint32_t *out_ptr,
                       const uint32_t *out_idx, uint32_t k, uint32_t *out_ids, float *out_dist,
                       int32_t *out_size, ung_hip_stats *st)
{
    clear_error();
    AllocCount alloc_count(st);
    if (!out_ids) {
        set_error("ung_hip_cross_topk: null out_ids");
        return UNG_HIP_EINVAL;
    }
    const auto t0 = clk::now();
    int rc = cross_device(ctx, G, group_begin, out_ptr, out_idx, k, st);
    if (rc)
        return rc;
    rc = download(ctx, ctx->cross, out_ids, out_dist, out_size, st);
    if (st)
        st->wall_ms = ms_since(t0);
    return rc;
}

int ung_hip_cross_topk_noalloc(ung_hip_ctx *ctx, uint32_t G, const uint32_t *group_begin, const uint32_t *out_ptr,
                               const uint32_t *out_idx, uint32_t k, uint32_t *out_ids_dev, float *out_dist_dev,
                               int32_t *out_size_dev, ung_hip_stats *st)
{
    clear_error();
    AllocCount alloc_count(st);
    return cross_noalloc(ctx, G, group_begin, out_ptr, out_idx, k, out_ids_dev, out_dist_dev, out_size_dev, st);
}

int ung_hip_cross_result_device(ung_hip_ctx *ctx, uint32_t **ids_dev, float **dist_dev)
{
    clear_error();
    if (!ctx || !ctx->cross.valid) {
        set_error("no cross-edge result on the device");
        return UNG_HIP_ESTATE;
    }
    if (ids_dev)
        *ids_dev = ctx->cross.ids.p;
    if (dist_dev)
        *dist_dev = ctx->cross.dist.p;
    return UNG_HIP_OK;
}

int ung_hip_download_cross(ung_hip_ctx *ctx, uint32_t *out_ids, float *out_dist, int32_t *out_size,
                           ung_hip_stats *st)
{
    clear_error();
    AllocCount alloc_count(st);
    if (!ctx) {
        set_error("null context");
        return UNG_HIP_EINVAL;
    }
    return download(ctx, ctx->cross, out_ids, out_dist, out_size, st);
}

int ung_hip_additional_edges(ung_hip_ctx *ctx, uint32_t G, const uint32_t *group_begin, const uint32_t *out_ptr,
                             const uint32_t *out_idx, uint32_t num_cross, uint32_t *edge_ptr, uint32_t *edge_from,
                             uint32_t *edge_to, uint64_t capacity, uint64_t *n_edges, ung_hip_stats *st)
{
    clear_error();
    AllocCount alloc_count(st);
    return additional_device(ctx, G, group_begin, out_ptr, out_idx, num_cross, edge_ptr, edge_from, edge_to, capacity,
                             n_edges, st);
}

int ung_hip_group_knn_device(ung_hip_ctx *ctx, uint32_t n_groups, const uint32_t *grp_begin,
                             const uint32_t *grp_size, uint32_t list_k, ung_hip_stats *st)
{
    clear_error();
    AllocCount alloc_count(st);
    return group_device(ctx, n_groups, grp_begin, grp_size, list_k, st);
}

int ung_hip_group_knn(ung_hip_ctx *ctx, uint32_t n_groups, const uint32_t *grp_begin, const uint32_t *grp_size,
                      uint32_t list_k, uint32_t *out_ids, float *out_dist, ung_hip_stats *st)
{
    clear_error();
    AllocCount alloc_count(st);
    if (!out_ids) {
        set_error("ung_hip_group_knn: null out_ids");
        return UNG_HIP_EINVAL;
    }
    const auto t0 = clk::now();
    int rc = group_device(ctx, n_groups, grp_begin, grp_size, list_k, st);
    if (rc)
        return rc;
    rc = download(ctx, ctx->group, out_ids, out_dist, nullptr, st);
    if (st)
        st->wall_ms = ms_since(t0);
    return rc;
}

int ung_hip_cross_intra_begin(ung_hip_ctx *ctx, uint32_t G, const uint32_t *group_begin, const uint32_t *out_ptr,
                              const uint32_t *out_idx, uint32_t k, uint32_t n_groups, const uint32_t *grp_begin,
                              const uint32_t *grp_size, uint32_t list_k, ung_hip_stats *st)
{
    clear_error();
    AllocCount alloc_count(st);
    return cross_intra_begin(ctx, G, group_begin, out_ptr, out_idx, k, n_groups, grp_begin, grp_size, list_k, st);
}

int ung_hip_intra_end(ung_hip_ctx *ctx, ung_hip_stats *st)
{
    clear_error();
    AllocCount alloc_count(st);
    return intra_end(ctx, st);
}

int ung_hip_group_result_device(ung_hip_ctx *ctx, uint32_t **ids_dev, float **dist_dev, uint64_t *rows)
{
    clear_error();
    if (!ctx || !ctx->group.valid) {
        set_error("no group kNN result on the device");
        return UNG_HIP_ESTATE;
    }
    if (ids_dev)
        *ids_dev = ctx->group.ids.p;
    if (dist_dev)
        *dist_dev = ctx->group.dist.p;
    if (rows)
        *rows = ctx->group.rows;
    return UNG_HIP_OK;
}

int ung_hip_result_shape(ung_hip_ctx *ctx, int which, uint64_t *rows, uint32_t *k, uint32_t *n_groups)
{
    clear_error();
    if (!ctx || (which != 0 && which != 1)) {
        set_error("ung_hip_result_shape: null context or which not 0/1");
        return UNG_HIP_EINVAL;
    }
    const ResultBufs &res = which == 0 ? ctx->cross : ctx->group;
    if (!res.valid) {
        set_error("ung_hip_result_shape: no %s result on the device", which == 0 ? "cross-edge" : "group kNN");
        return UNG_HIP_ESTATE;
    }
    if (rows)
        *rows = res.rows;
    if (k)
        *k = res.k;
    if (n_groups)
        *n_groups = which == 0 ? 0u : (uint32_t)ctx->group_jobs.size();
    return UNG_HIP_OK;
}

int ung_hip_rescanned_rows(ung_hip_ctx *ctx, int which, uint32_t *rows, uint64_t capacity, uint64_t *n_rows)
{
    clear_error();
    if (!ctx || (which != 0 && which != 1) || !n_rows) {
        set_error("ung_hip_rescanned_rows: null context/n_rows or which not 0/1");
        return UNG_HIP_EINVAL;
    }
    const ResultBufs &res = which == 0 ? ctx->cross : ctx->group;
    if (!res.valid) {
        set_error("ung_hip_rescanned_rows: no %s result on the device", which == 0 ? "cross-edge" : "group kNN");
        return UNG_HIP_ESTATE;
    }
    *n_rows = res.rescanned.size();
    if (res.rescanned.size() > capacity || (!rows && !res.rescanned.empty())) {
        set_error("ung_hip_rescanned_rows: capacity %llu < %zu rows", (unsigned long long)capacity,
                  res.rescanned.size());
        return UNG_HIP_EINVAL;
    }
    if (!res.rescanned.empty())
        std::memcpy(rows, res.rescanned.data(), res.rescanned.size() * sizeof(uint32_t));
    return UNG_HIP_OK;
}

int ung_hip_download_group(ung_hip_ctx *ctx, uint32_t *out_ids, float *out_dist, ung_hip_stats *st)
{
    clear_error();
    AllocCount alloc_count(st);
    if (!ctx) {
        set_error("null context");
        return UNG_HIP_EINVAL;
    }
    return download(ctx, ctx->group, out_ids, out_dist, nullptr, st);
}

int ung_hip_pack_anchor_rows(ung_hip_ctx *ctx, uint32_t tagore_k, uint32_t final_degree, uint32_t head_keep,
                             uint32_t anchor_tail, uint32_t anchor_slots, uint32_t bidir_anchor,
                             uint32_t *out_graph, uint32_t *entry_points, ung_hip_stats *st)
{
    clear_error();
    AllocCount alloc_count(st);
    if (!ctx || !ctx->group.valid) {
        set_error("ung_hip_pack_anchor_rows: run ung_hip_group_knn(_device) first");
        return UNG_HIP_ESTATE;
    }
    if (!out_graph || final_degree == 0 || tagore_k == 0) {
        set_error("ung_hip_pack_anchor_rows: null out_graph or zero final_degree/tagore_k");
        return UNG_HIP_EINVAL;
    }
    // the reference raises k to final_degree+1 (tagore_graph_builder.cu:1788-1789)
    if (tagore_k <= final_degree)
        tagore_k = final_degree + 1;
    const uint32_t list_k = ctx->group_list_k;
    uint32_t need = std::min<uint32_t>(64u, tagore_k - 1);
    if (anchor_tail && anchor_slots == 0)
        need = std::min(need, std::min(head_keep, final_degree));
    for (const Job &jb : ctx->group_jobs) {
        const uint32_t cd = std::min(need, jb.q_count - 1);
        if (cd > list_k) {
            set_error("ung_hip_pack_anchor_rows: packing reads %u list entries but the kNN lists hold %u", cd, list_k);
            return UNG_HIP_EINVAL;
        }
    }
    int rc;
    if ((rc = set_device(ctx)))
        return rc;
    const auto t0 = clk::now();
    const uint32_t stride = final_degree + 1;
    const uint64_t rows = ctx->group.rows;
    if ((rc = ctx->graph.ensure(std::max<uint64_t>(rows * stride, 1))))
        return rc;
    if (!ctx->group_pitems.empty()) {
        PackParams K{};
        K.jobs = ctx->gjobs.p;
        K.mitems = ctx->gmitems.p;
        K.list_ids = ctx->group.ids.p;
        K.list_k = list_k;
        K.tagore_k = tagore_k;
        K.final_degree = final_degree;
        K.head_keep = head_keep;
        K.anchor_tail = anchor_tail;
        K.anchor_slots = anchor_slots;
        K.bidir_anchor = bidir_anchor;
        K.graph_stride = stride;
        K.graph = ctx->graph.p;
        HIPCHECK(hipEventRecord(ctx->ev[6], ctx->stream));
        hipLaunchKernelGGL(ung_pack_kernel, dim3((unsigned)ctx->group_pitems.size()), dim3(MERGE_Q), 0, ctx->stream, K);
        HIPCHECK(hipGetLastError());
        HIPCHECK(hipEventRecord(ctx->ev[7], ctx->stream));
    }
    const auto t1 = clk::now();
    const DlRegion reg{out_graph, ctx->graph.p, (size_t)rows * stride * sizeof(uint32_t)};
    if ((rc = download_regions(ctx, ctx->stream, &reg, 1)))
        return rc;
    if (entry_points)
        std::memset(entry_points, 0, ctx->group_jobs.size() * sizeof(uint32_t));
    if (st) {
        float kms = 0;
        if (!ctx->group_pitems.empty())
            HIPCHECK(hipEventElapsedTime(&kms, ctx->ev[6], ctx->ev[7]));
        st->kernel_ms += kms;
        st->d2h_ms += ms_since(t1);
        st->wall_ms += ms_since(t0);
    }
    return UNG_HIP_OK;
}

int ung_hip_prune_group_graph(ung_hip_ctx *ctx, uint32_t forward_cap, uint32_t reverse_cap, uint32_t final_degree,
                              float alpha, uint32_t *out_graph, uint32_t *entry_points, ung_hip_stats *st)
{
    clear_error();
    AllocCount alloc_count(st);
    if (!ctx || !ctx->group.valid) {
        set_error("ung_hip_prune_group_graph: run ung_hip_group_knn(_device) first");
        return UNG_HIP_ESTATE;
    }
    const uint32_t list_k = ctx->group_list_k;
    if (!out_graph || final_degree == 0 || final_degree > 64 || reverse_cap > 32 || forward_cap == 0 ||
        forward_cap > list_k || !(alpha >= 0.0f)) {
        set_error("ung_hip_prune_group_graph: need out_graph, 1<=final_degree<=64, reverse_cap<=32, "
                  "1<=forward_cap<=%u (the kNN list length), alpha>=0", list_k);
        return UNG_HIP_EINVAL;
    }
    int rc;
    if ((rc = set_device(ctx)))
        return rc;
    const auto t0 = clk::now();
    const uint32_t stride = final_degree + 1;
    const uint64_t rows = ctx->group.rows;
    const uint32_t n_jobs = (uint32_t)ctx->group_jobs.size();
    if (rows == 0 || n_jobs == 0)
        return UNG_HIP_OK;
    if (rows >= (1ull << 31)) {
        set_error("ung_hip_prune_group_graph: %llu rows (at most 2^31-1)", (unsigned long long)rows);
        return UNG_HIP_EINVAL;
    }
    if ((rc = ctx->graph.ensure(rows * stride)) || (rc = ctx->rv_cnt.ensure(rows + 1)) ||
        (rc = ctx->rv_fill.ensure(rows)))
        return rc;
    PruneParams K{};
    K.X = ctx->X;
    K.d = ctx->d;
    K.jobs = ctx->gjobs.p;
    K.n_jobs = n_jobs;
    K.ids = ctx->group.ids.p;
    K.dist = ctx->group.dist.p;
    K.size = ctx->group.size.p;
    K.list_k = list_k;
    K.forward_cap = forward_cap;
    K.reverse_cap = reverse_cap;
    K.final_degree = final_degree;
    K.alpha = alpha;
    K.rows = rows;
    K.rev_cnt = ctx->rv_cnt.p;
    K.rev_fill = ctx->rv_fill.p;
    K.graph = ctx->graph.p;
    K.xs = ctx->XS;
    K.xn = ctx->xn;
    K.dp = ctx->dp;
    K.eps_coef = eps_coef_for(ctx->d) * ctx->eps_scale;
    K.shrink = ((double)ctx->d / 8.0 + 8.0) * std::ldexp(1.0, -24);
    HIPCHECK(hipEventRecord(ctx->ev[6], ctx->stream));
    const unsigned zb = (unsigned)std::min<uint64_t>((rows + 256) / 256, 65535);
    hipLaunchKernelGGL(ung_zero_u32_kernel, dim3(zb), dim3(256), 0, ctx->stream, ctx->rv_cnt.p, (uint32_t)(rows + 1));
    hipLaunchKernelGGL(ung_zero_u32_kernel, dim3(zb), dim3(256), 0, ctx->stream, ctx->rv_fill.p, (uint32_t)rows);
    HIPCHECK(hipGetLastError());
    const unsigned rb = (unsigned)std::min<uint64_t>((rows + 255) / 256, 16384);
    hipLaunchKernelGGL(ung_reverse_kernel<false>, dim3(rb), dim3(256), 0, ctx->stream, K);
    HIPCHECK(hipGetLastError());
    // counts -> offsets (exclusive scan over rows + 1 entries, in place)
    size_t tmp_bytes = 0;
    HIPCHECK(hipcub::DeviceScan::ExclusiveSum(nullptr, tmp_bytes, ctx->rv_cnt.p, ctx->rv_cnt.p, (int)(rows + 1),
                                              ctx->stream));
    if ((rc = ctx->rv_tmp.ensure(tmp_bytes + 1)))
        return rc;
    HIPCHECK(hipcub::DeviceScan::ExclusiveSum(ctx->rv_tmp.p, tmp_bytes, ctx->rv_cnt.p, ctx->rv_cnt.p, (int)(rows + 1),
                                              ctx->stream));
    uint32_t total = 0;
    HIPCHECK(hipMemcpyAsync(&total, ctx->rv_cnt.p + rows, sizeof(uint32_t), hipMemcpyDeviceToHost, ctx->stream));
    HIPCHECK(hipStreamSynchronize(ctx->stream));
    if ((rc = ctx->rv_src.ensure((uint64_t)total + 1)) || (rc = ctx->rv_dist.ensure((uint64_t)total + 1)))
        return rc;
    K.rev_src = ctx->rv_src.p;
    K.rev_dist = ctx->rv_dist.p;
    hipLaunchKernelGGL(ung_reverse_kernel<true>, dim3(rb), dim3(256), 0, ctx->stream, K);
    HIPCHECK(hipGetLastError());
    if (ctx->prune_mode == 2 || (ctx->prune_mode == 0 && ctx->dp >= 256u))
        hipLaunchKernelGGL(ung_prune_gram_kernel, dim3((unsigned)rows), dim3(64), 0, ctx->stream, K);
    else
        hipLaunchKernelGGL(ung_prune_kernel, dim3((unsigned)rows), dim3(64), 0, ctx->stream, K);
    HIPCHECK(hipGetLastError());
    HIPCHECK(hipEventRecord(ctx->ev[7], ctx->stream));
    const auto t1 = clk::now();
    const DlRegion reg{out_graph, ctx->graph.p, (size_t)rows * stride * sizeof(uint32_t)};
    if ((rc = download_regions(ctx, ctx->stream, &reg, 1)))
        return rc;
    // FastGrnnd's entry point is the group's first point (ep_dev cleared, :2036)
    if (entry_points)
        std::memset(entry_points, 0, n_jobs * sizeof(uint32_t));
    if (st) {
        float kms = 0;
        HIPCHECK(hipEventElapsedTime(&kms, ctx->ev[6], ctx->ev[7]));
        st->kernel_ms += kms;
        st->d2h_ms += ms_since(t1);
        st->wall_ms += ms_since(t0);
        st->rows += rows;
    }
    return UNG_HIP_OK;
}

int ung_hip_synchronize(ung_hip_ctx *ctx)
{
    clear_error();
    if (!ctx) {
        set_error("null context");
        return UNG_HIP_EINVAL;
    }
    HIPCHECK(hipStreamSynchronize(ctx->stream));
    return UNG_HIP_OK;
}

int ung_hip_selftest_mfma(ung_hip_ctx *ctx, double *max_abs_err)
{
    clear_error();
    if (!ctx || !max_abs_err) {
        set_error("null argument");
        return UNG_HIP_EINVAL;
    }
    int rc;
    if ((rc = set_device(ctx)))
        return rc;
    float *d_out = nullptr;
    HIPCHECK(counted_malloc((void **)&d_out, 32 * 32 * sizeof(float)));
    hipLaunchKernelGGL(ung_mfma_probe_kernel, dim3(1), dim3(64), 0, ctx->stream, d_out);
    hipError_t e = hipGetLastError();
    float host[32 * 32];
    if (e == hipSuccess)
        e = hipMemcpyAsync(host, d_out, sizeof(host), hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess)
        e = hipStreamSynchronize(ctx->stream);
    (void)hipFree(d_out);
    if (e != hipSuccess) {
        set_error("mfma self test failed: %s", hipGetErrorString(e));
        return UNG_HIP_EDEVICE;
    }
    double mx = 0;
    for (int m = 0; m < 32; ++m)
        for (int n = 0; n < 32; ++n) {
            double ref = 0;
            for (int kk = 0; kk < 16; ++kk)
                ref += ((double)(m - 16) + 0.25 * (kk % 8)) * ((double)(kk % 4 + 1) * (double)(n - 7));
            mx = std::max(mx, std::fabs(ref - (double)host[m * 32 + n]));
        }
    *max_abs_err = mx;
    return UNG_HIP_OK;
}

int ung_hip_debug_partial_rows(ung_hip_ctx *ctx, uint64_t capacity, uint32_t *query, uint32_t *cand, float *approx,
                               uint64_t *n_entries, double *eps_coef, double *rmax)
{
    clear_error();
    if (!ctx || !n_entries) {
        set_error("ung_hip_debug_partial_rows: null context/n_entries");
        return UNG_HIP_EINVAL;
    }
    const Plan &pl = ctx->plan0;
    if (pl.part_lp == 0) {
        set_error("ung_hip_debug_partial_rows: no partial rows of a cross or synchronous group call on the device");
        return UNG_HIP_ESTATE;
    }
    int rc;
    if ((rc = set_device(ctx)))
        return rc;
    const uint32_t lp = pl.part_lp;
    const uint64_t n = pl.part_rows * lp;
    std::vector<uint32_t> ids(n);
    std::vector<float> dist(n);
    if (n) {
        HIPCHECK(hipMemcpyAsync(ids.data(), ctx->ws[0].part_ids.p, n * sizeof(uint32_t), hipMemcpyDeviceToHost,
                                ctx->ws[0].stream));
        HIPCHECK(hipMemcpyAsync(dist.data(), ctx->ws[0].part_dist.p, n * sizeof(float), hipMemcpyDeviceToHost,
                                ctx->ws[0].stream));
    }
    HIPCHECK(hipStreamSynchronize(ctx->ws[0].stream));
    // every entry of every job's partial rows: split s, query j at row part_base + s*q_count + j
    uint64_t cnt = 0;
    for (int pass = 0; pass < 2; ++pass) {
        cnt = 0;
        for (const Job &jb : pl.jobs)
            for (uint32_t sp = 0; sp < jb.n_split; ++sp)
                for (uint32_t qj = 0; qj < jb.q_count; ++qj) {
                    const uint64_t prow = (uint64_t)jb.part_base + (uint64_t)sp * jb.q_count + qj;
                    for (uint32_t e = 0; e < lp; ++e) {
                        const uint32_t id = ids[prow * lp + e];
                        if (id == NONE)
                            continue;
                        if (pass == 1) {
                            query[cnt] = jb.q_begin + qj;
                            cand[cnt] = id;
                            approx[cnt] = dist[prow * lp + e];
                        }
                        ++cnt;
                    }
                }
        if (pass == 0) {
            *n_entries = cnt;
            if (eps_coef)
                *eps_coef = eps_coef_for(ctx->d) * ctx->eps_scale;
            if (rmax)
                *rmax = ctx->rmax;
            if (cnt > capacity || (cnt > 0 && (!query || !cand || !approx))) {
                set_error("ung_hip_debug_partial_rows: capacity %llu < %llu entries", (unsigned long long)capacity,
                          (unsigned long long)cnt);
                return UNG_HIP_EINVAL;
            }
        }
    }
    return UNG_HIP_OK;
}

int ung_hip_debug_partial_bounds(ung_hip_ctx *ctx, uint64_t capacity, uint32_t *query, uint32_t *cand_begin,
                                 uint32_t *cand_end, float *bound, uint64_t *n_rows)
{
    clear_error();
    if (!ctx || !n_rows) {
        set_error("ung_hip_debug_partial_bounds: null context/n_rows");
        return UNG_HIP_EINVAL;
    }
    const Plan &pl = ctx->plan0;
    if (pl.part_lp == 0) {
        set_error("ung_hip_debug_partial_bounds: no partial rows of a cross or synchronous group call on the device");
        return UNG_HIP_ESTATE;
    }
    // rows of the jobs that went through the select (tiny cross jobs have none)
    uint64_t n = 0;
    for (const Job &jb : pl.jobs)
        n += (uint64_t)jb.n_split * jb.q_count;
    *n_rows = n;
    if (n > capacity || (n > 0 && (!query || !cand_begin || !cand_end || !bound))) {
        set_error("ung_hip_debug_partial_bounds: capacity %llu < %llu rows", (unsigned long long)capacity,
                  (unsigned long long)n);
        return UNG_HIP_EINVAL;
    }
    int rc;
    if ((rc = set_device(ctx)))
        return rc;
    std::vector<float> b(pl.part_rows);
    if (pl.part_rows)
        HIPCHECK(hipMemcpyAsync(b.data(), ctx->ws[0].part_bound.p, pl.part_rows * sizeof(float), hipMemcpyDeviceToHost,
                                ctx->ws[0].stream));
    HIPCHECK(hipStreamSynchronize(ctx->ws[0].stream));
    uint64_t r = 0;
    for (const Job &jb : pl.jobs)
        for (uint32_t sp = 0; sp < jb.n_split; ++sp) {
            const uint32_t v0 = sp * jb.split_v;
            const uint32_t v1 = (uint32_t)std::min<uint64_t>(jb.n_cand, (uint64_t)(sp + 1) * jb.split_v);
            const bool one = jb.seg_count == 1;
            const uint32_t s0 = one ? pl.seg_start[jb.seg_begin] : 0u;
            for (uint32_t qj = 0; qj < jb.q_count; ++qj, ++r) {
                query[r] = jb.q_begin + qj;
                cand_begin[r] = one ? s0 + v0 : NONE;
                cand_end[r] = one ? s0 + v1 : NONE;
                bound[r] = b[(uint64_t)jb.part_base + (uint64_t)sp * jb.q_count + qj];
            }
        }
    return UNG_HIP_OK;
}

} // extern "C"
