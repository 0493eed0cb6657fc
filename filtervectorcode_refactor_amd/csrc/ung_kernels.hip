// ung_kernels.hip -- gfx950 (MI355X) device code of the UNG cross-edge / mid-group
// kNN build stage: the kernels and the work-list structures they read.  The host side
// (context, planning, launches, C ABI) is ung_runtime.hip, which includes this file;
// the two form one translation unit.
//
// Path (one call = one "job list"):
//   select  : fused distance tiles on the bf16 matrix cores -- every fp32 coordinate
//             is split into bf16 hi + lo and each product is taken as hi*hi + hi*lo +
//             lo*hi by three v_mfma_f32_32x32x16_bf16 passes (LDS-staged candidate
//             panels, query rows held in registers and LDS at dp = 128) -- with
//             per-row register queues in the epilogue: no distance matrix ever reaches
//             HBM.  At the end of a work item the approximate (expansion-form) top-Lp
//             of every query is written as a partial row with a bound that every
//             candidate left out satisfies.
//   merge   : per result row, merges the partial rows of its candidate splits,
//             re-scores the best EXACTLY in the reference's fp32 summation order and
//             certifies, from a proven bound on the pre-selection's error, that no
//             candidate left out can enter the top-k.
//   fallback: rows whose bound does not certify the result are rescanned exactly
//             (rare; counted in ung_hip_stats::fallback_rows).
//   tiny    : cross jobs of a few queries and a small union skip the select and the
//             merge: one wave scores all their (query, candidate) pairs exactly.
//
// Reference semantics reproduced: src/uni_nav_graph_cross_edges.cpp:32-57,154-220
// (cross edges), src/uni_nav_graph_special_blocks.cpp:70-111 (intra exact kNN),
// src/distance.cpp:34-91 (distance rounding), src/search_queue.cpp:26-53
// ((dist,id) order), src/tagore_graph_builder.cu:727-794 (anchor packing).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

namespace {

constexpr int BQ = 128;          // queries per work item (columns of the MFMA tiles)
constexpr int BC = 128;          // candidates per tile (rows of the MFMA tiles)
constexpr int KC = 32;           // k-chunk staged in LDS (dimensions)
constexpr int LDSW = KC + 4;     // padded LDS row stride (32-bit words; a chunk row is 32 words)
constexpr int NTHREADS = 256;    // 4 waves: 2 (candidate halves) x 2 (query halves)
constexpr uint32_t SPLIT_V = 32768; // candidates per work item (raised so a job has <= 64 splits)
constexpr uint32_t MAX_SPLITS = 64; // one wave lane per split in the merge
constexpr uint32_t MERGE_ROWS = 4;  // result rows (one wave each) per merge block
constexpr uint32_t MERGE_QLDS = 1024; // largest d whose query rows the merge stages in LDS
constexpr uint32_t MERGE_Q = 256;   // rows per packing block
constexpr uint32_t NONE = 0xFFFFFFFFu;

struct Job {
    uint32_t q_begin, q_count;     // queries: global ids [q_begin, q_begin+q_count)
    uint32_t seg_begin, seg_count; // candidate segments (seg_start/seg_vend)
    uint32_t n_cand, n_split;      // virtual candidate count U, number of splits S
    uint32_t part_base;            // partial row of (split s, query j) = part_base + s*q_count + j
    uint32_t out_row;              // result row of query 0
    uint32_t id_base;              // subtracted from result ids (group begin for local ids)
    uint32_t flags;                // bit 0: exclude the query itself
    uint32_t split_v;              // candidates per split
};

struct Item {
    uint32_t job, q_off, q_cnt, v_begin, v_end, split, pad0, pad1;
};

struct MergeItem {
    uint32_t job, q_off, q_cnt, pad;
};

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct SelectParams {
    const uint32_t *xs; // split base set: [N][dp] words, see ung_split_kernel
    const float *xn;
    uint32_t dp;        // words per split row = d rounded up to a multiple of KC
    uint32_t k;
    const Job *jobs;
    const Item *items;
    const uint32_t *seg_start;
    const uint32_t *seg_vend;
    uint32_t *part_ids;
    float *part_dist;
    float *part_bound;
    double eps_coef;  // (7d/4+112)*2^-24 : expansion-form error factor on (|q|+R)^2
    double shrink;    // (d/8+8)*2^-24 : relative error of the reference summation
    double rmax;      // max candidate norm (slightly inflated)
    uint32_t n_items; // items of this launch
    uint32_t *item_ctr; // next item to take (zeroed before the launch)
    uint32_t lp;      // entries per partial row (approximate top-Lp)
    uint32_t x_bytes; // bytes of the split base set (buffer range of the 32-bit-offset kernels)
};

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t cand_id(const uint32_t *__restrict__ seg_start,
                                            const uint32_t *__restrict__ seg_vend, uint32_t sb,
                                            uint32_t sc, uint32_t v)
{
    uint32_t lo = 0, hi = sc;
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (seg_vend[sb + mid] > v)
            hi = mid;
        else
            lo = mid + 1;
    }
    const uint32_t vstart = lo ? seg_vend[sb + lo - 1] : 0u;
    return seg_start[sb + lo] + (v - vstart);
}

__device__ __forceinline__ bool cand_less(float da, uint32_t ia, float db, uint32_t ib)
{
    // bitwise, not short-circuit: lane masks combine without branches
    return (da < db) | ((da == db) & (ia < ib));
}

// Squared L2 with the rounding of the reference's release build of
// FloatL2DistanceHandler::compute (src/distance.cpp:34-91: 8 lane accumulators
// with fused multiply-add per 8-float block, upper+lower lane fold, fused 4- and
// <4-float tails, then (s0+s1)+(s2+s3)).  Cooperative: the 8 lanes of an aligned
// group each own one accumulator; all 8 must call; the result is valid in sub 0.
#pragma clang fp contract(off)
__device__ __forceinline__ float l2_ref_8lane(const float *__restrict__ a,
                                              const float *__restrict__ b, uint32_t d, int sub)
{
    float acc = 0.0f;
    const uint32_t nb8 = d >> 3;
    uint32_t blk = 0;
    // 8 blocks of loads in flight before their fused multiply-adds (same order)
    for (; blk + 8 <= nb8; blk += 8) {
        float ta[8], tb[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            ta[u] = a[8 * (blk + u) + sub];
            tb[u] = b[8 * (blk + u) + sub];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const float t = ta[u] - tb[u];
            acc = __builtin_fmaf(t, t, acc);
        }
    }
    for (; blk < nb8; ++blk) {
        const float t = a[8 * blk + sub] - b[8 * blk + sub];
        acc = __builtin_fmaf(t, t, acc);
    }
    const float hi = __shfl_xor(acc, 4, 8);
    float s = hi + acc;
    uint32_t p = nb8 * 8, rem = d - p;
    if (rem >= 4) {
        if (sub < 4) {
            const float t = a[p + sub] - b[p + sub];
            s = __builtin_fmaf(t, t, s);
        }
        p += 4;
        rem -= 4;
    }
    if ((uint32_t)sub < rem) {
        const float t = a[p + sub] - b[p + sub];
        s = __builtin_fmaf(t, t, s);
    }
    const float s_odd = __shfl_xor(s, 1, 8);
    const float pair = s + s_odd;            // sub 0: s0+s1, sub 2: s2+s3
    const float pair_hi = __shfl_xor(pair, 2, 8);
    return pair + pair_hi;                   // sub 0: (s0+s1)+(s2+s3)
}

// l2_ref_8lane for two rows b0, b1 against one row a at once: each value is computed
// by exactly the operations of l2_ref_8lane (bit-identical), with a's loads shared and
// twice the loads in flight per block of eight.
__device__ __forceinline__ void l2_ref_8lane2(const float *__restrict__ a, const float *__restrict__ b0,
                                              const float *__restrict__ b1, uint32_t d, int sub, float &v0,
                                              float &v1)
{
    float acc0 = 0.0f, acc1 = 0.0f;
    const uint32_t nb8 = d >> 3;
    uint32_t blk = 0;
    for (; blk + 8 <= nb8; blk += 8) {
        float ta[8], t0[8], t1[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            ta[u] = a[8 * (blk + u) + sub];
            t0[u] = b0[8 * (blk + u) + sub];
            t1[u] = b1[8 * (blk + u) + sub];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const float x0 = ta[u] - t0[u], x1 = ta[u] - t1[u];
            acc0 = __builtin_fmaf(x0, x0, acc0);
            acc1 = __builtin_fmaf(x1, x1, acc1);
        }
    }
    for (; blk < nb8; ++blk) {
        const float av = a[8 * blk + sub];
        const float x0 = av - b0[8 * blk + sub], x1 = av - b1[8 * blk + sub];
        acc0 = __builtin_fmaf(x0, x0, acc0);
        acc1 = __builtin_fmaf(x1, x1, acc1);
    }
    float s0 = __shfl_xor(acc0, 4, 8) + acc0;
    float s1 = __shfl_xor(acc1, 4, 8) + acc1;
    uint32_t p = nb8 * 8, rem = d - p;
    if (rem >= 4) {
        if (sub < 4) {
            const float av = a[p + sub];
            const float x0 = av - b0[p + sub], x1 = av - b1[p + sub];
            s0 = __builtin_fmaf(x0, x0, s0);
            s1 = __builtin_fmaf(x1, x1, s1);
        }
        p += 4;
        rem -= 4;
    }
    if ((uint32_t)sub < rem) {
        const float av = a[p + sub];
        const float x0 = av - b0[p + sub], x1 = av - b1[p + sub];
        s0 = __builtin_fmaf(x0, x0, s0);
        s1 = __builtin_fmaf(x1, x1, s1);
    }
    const float pr0 = s0 + __shfl_xor(s0, 1, 8), pr1 = s1 + __shfl_xor(s1, 1, 8);
    v0 = pr0 + __shfl_xor(pr0, 2, 8);
    v1 = pr1 + __shfl_xor(pr1, 2, 8);
}

// Same value computed by one lane alone.  Rows 16-byte aligned (d % 4 == 0) are read
// with float4 loads; the accumulation order is the same either way.
__device__ __forceinline__ float l2_ref_lane(const float *__restrict__ a,
                                             const float *__restrict__ b, uint32_t d)
{
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint32_t p = 0;
    if ((d & 3u) == 0) {
        const float4 *a4 = reinterpret_cast<const float4 *>(a);
        const float4 *b4 = reinterpret_cast<const float4 *>(b);
        // four 8-float blocks of loads in flight before their fused multiply-adds
        for (; p + 32 <= d; p += 32) {
            float4 x[8], y[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                x[u] = a4[(p >> 2) + u];
                y[u] = b4[(p >> 2) + u];
            }
#pragma unroll
            for (int u = 0; u < 8; u += 2) {
                const float t[8] = {x[u].x - y[u].x, x[u].y - y[u].y, x[u].z - y[u].z, x[u].w - y[u].w,
                                    x[u + 1].x - y[u + 1].x, x[u + 1].y - y[u + 1].y, x[u + 1].z - y[u + 1].z,
                                    x[u + 1].w - y[u + 1].w};
#pragma unroll
                for (int l = 0; l < 8; ++l)
                    acc[l] = __builtin_fmaf(t[l], t[l], acc[l]);
            }
        }
        for (; p + 8 <= d; p += 8) {
            const float4 x0 = a4[p >> 2], x1 = a4[(p >> 2) + 1];
            const float4 y0 = b4[p >> 2], y1 = b4[(p >> 2) + 1];
            const float t[8] = {x0.x - y0.x, x0.y - y0.y, x0.z - y0.z, x0.w - y0.w,
                                x1.x - y1.x, x1.y - y1.y, x1.z - y1.z, x1.w - y1.w};
#pragma unroll
            for (int l = 0; l < 8; ++l)
                acc[l] = __builtin_fmaf(t[l], t[l], acc[l]);
        }
    }
    for (; p + 8 <= d; p += 8) {
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const float t = a[p + l] - b[p + l];
            acc[l] = __builtin_fmaf(t, t, acc[l]);
        }
    }
    float s[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        s[i] = acc[i + 4] + acc[i];
    uint32_t rem = d - p;
    if (rem >= 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float t = a[p + i] - b[p + i];
            s[i] = __builtin_fmaf(t, t, s[i]);
        }
        p += 4;
        rem -= 4;
    }
    for (uint32_t i = 0; i < rem; ++i) {
        const float t = a[p + i] - b[p + i];
        s[i] = __builtin_fmaf(t, t, s[i]);
    }
    return (s[0] + s[1]) + (s[2] + s[3]);
}
#pragma clang fp contract(on)

// Sorted insert of (nd, ni) into an ascending register queue (ties keep the older
// entry first; nd = +inf changes nothing).  Runs from the tail so every entry is
// updated in place from the old values of itself and its predecessor.  The new
// distance at j is the median of (old j-1, nd, old j) -- one v_med3_f32, which returns
// one of its inputs exactly; the id follows the same choice by the two comparisons.
template <int LT>
__device__ __forceinline__ void list_insert(float (&ld)[LT], uint32_t (&li)[LT], float nd,
                                            uint32_t ni)
{
    bool c_hi = nd < ld[LT - 1];
#pragma unroll
    for (int j = LT - 1; j > 0; --j) {
        const bool c_lo = nd < ld[j - 1];
        ld[j] = __builtin_amdgcn_fmed3f(ld[j - 1], nd, ld[j]);
        li[j] = c_hi ? (c_lo ? li[j - 1] : ni) : li[j];
        c_hi = c_lo;
    }
    ld[0] = c_hi ? nd : ld[0];
    li[0] = c_hi ? ni : li[0];
}

// Error term of one query, computed once per row: ea = eps_coef * (|q| + R)^2 (|q| from
// the cached |q|^2, rounded up), with
//   |a - D| <= eps_coef * (|q| + R)^2   (norm cache, MFMA dot, epilogue roundings)
//   e >= D * (1 - shrink), e <= D * (1 + shrink)   (reference summation)
// for the expansion-form MFMA value a, the exact squared distance D and the reference's
// rounded value e.
__device__ __forceinline__ double bound_ea(float qn, double eps_coef, double rmax)
{
    const double r = sqrt((double)fmaxf(qn, 0.0f) * (1.0 + 1e-6)) + rmax;
    return eps_coef * r * r;
}

// Lower bound on the exact (reference-rounded) distance of any candidate whose
// expansion-form MFMA distance is >= A, rounded toward -inf when narrowed to fp32.
__device__ __forceinline__ float lower_bound_ea(float A, double ea, double shrink)
{
    if (!(A < INFINITY))
        return INFINITY;
    double b = ((double)A - ea);
    b = b > 0.0 ? b * (1.0 - shrink) : b * (1.0 + shrink);
    b -= 1e-30;
    return __double2float_rd(b);
}

// Upper bound on the exact (reference-rounded) distance of a candidate whose
// expansion-form MFMA distance is A (the same two error terms, the other way; the
// exact distance is >= 0), rounded toward +inf.
__device__ __forceinline__ float upper_bound_ea(float A, double ea, double shrink)
{
    if (!(A < INFINITY))
        return INFINITY;
    const double b = fmax((double)A + ea, 0.0) * (1.0 + shrink) + 1e-30;
    return __double2float_ru(b);
}

// (dist, id) ascending sort of one value per lane over the wave (bitonic network, 21
// exchange stages): lane t ends with the t-th smallest.
__device__ __forceinline__ void wave_sort64(float &d, uint32_t &id, int lane)
{
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1)
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const float od = __shfl_xor(d, j);
            const uint32_t oi = __shfl_xor(id, j);
            const bool up = (lane & k) == 0;
            const bool lower = (lane & j) == 0;
            const bool take = (lower == up) ? cand_less(od, oi, d, id) : cand_less(d, id, od, oi);
            d = take ? od : d;
            id = take ? oi : id;
        }
}

// (dist, id) argmin across the wave; every lane ends with the minimum.
__device__ __forceinline__ void wave_argmin(float &d, uint32_t &i)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float od = __shfl_xor(d, off);
        const uint32_t oi = __shfl_xor(i, off);
        if (cand_less(od, oi, d, i)) {
            d = od;
            i = oi;
        }
    }
}

// bf16 bits of x rounded to nearest, ties to even (finite x; -inf gives the bf16 -inf).
__device__ __forceinline__ uint32_t bf16_rne(float x)
{
    const uint32_t u = __float_as_uint(x);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// ---------------------------------------------------------------------------
// select kernel
// ---------------------------------------------------------------------------
// End-of-item reduction area: the queues of 64 queries.
struct SelectRed {
    float ed[64][129];   // entry distances (approx, then exact); stride padded
    uint32_t ei[64][129];
    float alist[64][4];  // per queue: bound on every candidate it did not keep
    float drop[64];      // smallest queued value not written to the partial row
};

struct alignas(16) SelectSmem {
    union {
        struct {
            // float4-typed so every panel access is a 16-byte ds_read/ds_write_b128
            float4 qs[2][BQ][LDSW / 4];
            float4 xs[2][BC][LDSW / 4];
        } p;
        SelectRed r;
    } u;
    uint32_t rowid[3][BC]; // candidate ids of tiles t%3 (ring: built one tile ahead; NONE = padding)
    // their -|x|^2/2 as the A words of the bias MFMA: bf16 terms hi | mid << 16, lo (padding
    // rows: -inf, 0, 0)
    uint2 nhx[3][BC];
    float qn[BQ];
    float tau[2][2][BQ];   // [tile parity][candidate wave][query]: a wave's queue threshold
};
static_assert(BQ == BC, "the epilogue staging addresses assume square panels");

// Register-query layout (dp = 128, two query columns per lane): a lane keeps the high
// bf16 words of its query columns for all 8 k-blocks in registers for the whole item,
// and the low words of the item's queries stay resident in LDS; per step only the
// candidate chunk is loaded and staged.  LDS traffic per step and wave: 8 KB of
// candidate operands + 4 KB of query low words + 4 KB of staging writes, against 16 +
// 8 KB when both panels are restaged every step.
constexpr int QR_NK = 4;              // chunks of 32 dimensions (dp = 128)
constexpr int QLO_W = QR_NK * 16 + 4; // words per resident low-word query row (padded)
struct alignas(16) SelectSmemQ {
    union {
        struct {
            float4 xs[2][BC][LDSW / 4];
            float4 qlo[BQ][QLO_W / 4];
        } p;
        SelectRed r;
    } u;
    uint32_t rowid[3][BC];
    uint2 nhx[3][BC];
    float qn[BQ];
    float tau[2][2][BQ];
};
// flat float offsets inside SelectSmem::u.p
constexpr int PANEL_X = 2 * BQ * LDSW; // start of xs relative to qs
constexpr int ROW32 = 32 * LDSW;       // 32 panel rows

// Work item of a block, taken from a launch-wide counter when the block starts.  The
// hardware deals blocks to the 8 XCDs and to their shader engines round-robin by
// block index, a fixed share each; with item costs from 1 to 256 tiles a fixed share
// leaves engines idle while others still work.  Taking the next item (items sorted
// by decreasing cost) when a block actually starts balances the engines.  The grid
// has exactly n_items blocks, so every block gets one distinct item.
__device__ __forceinline__ uint32_t take_item(uint32_t *ctr, uint32_t *slot)
{
    if (threadIdx.x == 0)
        *slot = atomicAdd(ctr, 1u);
    __syncthreads();
    return *slot;
}

// Pre-filter bound in s-space: s = |x|^2/2 - <x,q> and a = fl(2s + |q|^2).  Returns c
// with  s >= c  =>  a >= thr  (the margin covers the rounding of 2s + |q|^2), so a
// candidate failing s < c can never pass the exact test a < thr.
__device__ __forceinline__ float s_bound(float thr, float qn)
{
    if (!(thr < INFINITY))
        return INFINITY;
    return 0.5f * (thr - qn) + 0x1p-20f * (fabsf(thr) + fabsf(qn));
}

// Position of a row thread in the job's segment list.  The thread's virtual index only
// grows (tile after tile), so the segment is found by a forward step: no memory access
// inside the current segment, one load on entering the next one, a binary search over
// the rest only when a tile skips whole segments.
struct RowCursor {
    uint32_t seg = 0xFFFFFFFFu; // current segment (none yet)
    uint32_t vend = 0;          // its virtual end
    uint32_t base = 0;          // global id = base + v inside it (mod 2^32)
};

// Global id of virtual candidate v (v < the job's union size, v >= any earlier v).
__device__ __forceinline__ uint32_t cursor_id(RowCursor &c, const SelectParams &P, const Job &jb, uint32_t v)
{
    if (v >= c.vend) {
        const uint32_t *__restrict__ ve = P.seg_vend + jb.seg_begin;
        uint32_t lo = c.seg + 1u, vstart = c.vend;
        uint32_t e = ve[lo];
        if (e <= v) {
            // first segment in [lo+1, seg_count) ending after v; the last one ends at
            // the union size > v
            uint32_t hi = jb.seg_count - 1u;
            ++lo;
            while (lo < hi) {
                const uint32_t mid = (lo + hi) >> 1;
                if (ve[mid] > v)
                    hi = mid;
                else
                    lo = mid + 1u;
            }
            vstart = ve[lo - 1u];
            e = ve[lo];
        }
        c.seg = lo;
        c.vend = e;
        c.base = P.seg_start[jb.seg_begin + lo] - vstart;
    }
    return c.base + v;
}

// Row ids of the candidate tile starting at virtual index v0 into ring slot `slot`;
// returns the row's |x|^2 (+inf for padding rows), a load the caller consumes later
// (finish_rowids), so its latency overlaps other work.
template <class Smem>
__device__ __forceinline__ float start_rowids(Smem &sm, int slot, RowCursor &cur, const SelectParams &P,
                                              const Job &jb, uint32_t v0, uint32_t v_end, int tid)
{
    float nx = INFINITY;
    if (tid < BC) {
        const uint32_t v = v0 + (uint32_t)tid;
        uint32_t g = NONE;
        if (v < v_end) {
            g = cursor_id(cur, P, jb, v);
            nx = P.xn[g];
        }
        sm.rowid[slot][tid] = g;
    }
    return nx;
}

template <class Smem>
__device__ __forceinline__ void finish_rowids(Smem &sm, int slot, float nx, int tid)
{
    if (tid < BC) {
        // -|x|^2/2 (exact scaling) split exactly into three bf16 terms
        const float v = -0.5f * nx;
        const uint32_t hi = bf16_rne(v);
        const float r1 = v - __uint_as_float(hi << 16);
        const uint32_t mid = bf16_rne(r1);
        const uint32_t lo = bf16_rne(r1 - __uint_as_float(mid << 16));
        const bool fin = v > -INFINITY;
        sm.nhx[slot][tid] = make_uint2(hi | (fin ? mid << 16 : 0u), fin ? lo : 0u);
    }
}

// Tile row (0..127) of a lane's j-th value of one query column, j = 16*mb + i of
// acc[mb][nb][i]:  wm*64 + mb*32 + 8*(i/4) + 4*h + i%4.
__device__ __forceinline__ uint32_t tile_row(int wm, int h, uint32_t j)
{
    return (uint32_t)(wm * 64 + 4 * h) + ((j & 28u) << 1) + (j & 3u);
}

// Index j of tile row offset o = row - (wm*64 + 4*h) when the row belongs to the lane
// (0 <= o < 64 and bit 2 of o clear), else 32.
__device__ __forceinline__ uint32_t lane_index_of(int o)
{
    return (o >= 0 && o < 64 && (o & 4) == 0) ? (((uint32_t)o >> 1) & 28u) | ((uint32_t)o & 3u) : 32u;
}

// Compare-exchange of entries a < b of a register queue (ascending by distance): one
// comparison and four selects (equal entries, two +inf included, stay in place).

template <int N>
__device__ __forceinline__ void cas(float (&d)[N], uint32_t (&id)[N], int a, int b)
{
    const float da = d[a], db = d[b];
    const bool sw = db < da;
    d[a] = sw ? db : da;
    d[b] = sw ? da : db;
    const uint32_t ia = id[a], ib = id[b];
    id[a] = sw ? ib : ia;
    id[b] = sw ? ia : ib;
}

// Ascending bitonic sort of the 8 entries at base..base+7 (24 compare-exchanges).
template <int N>
__device__ __forceinline__ void sort8(float (&d)[N], uint32_t (&id)[N], int base)
{
#pragma unroll
    for (int k = 2; k <= 8; k <<= 1)
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int l = i ^ j;
                if (l > i) {
                    if ((i & k) == 0)
                        cas(d, id, base + i, base + l);
                    else
                        cas(d, id, base + l, base + i);
                }
            }
}

// The 8 smallest of two ascending 8-runs at a and b, ascending, into the run at a
// (half cleaner on a[i] vs b[7-i], then a bitonic merge of the 8 kept).
template <int N>
__device__ __forceinline__ void merge8_keep(float (&d)[N], uint32_t (&id)[N], int a, int b)
{
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int l = b + 7 - i;
        const bool t = d[l] < d[a + i];
        d[a + i] = t ? d[l] : d[a + i];
        id[a + i] = t ? id[l] : id[a + i];
    }
#pragma unroll
    for (int j = 4; j > 0; j >>= 1)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int l = i ^ j;
            if (l > i)
                cas(d, id, a + i, a + l);
        }
}

// Ascending queue of the LT smallest of 32 (dist, id) entries: the first tile of an
// item fills its empty queues with a sorting network instead of 32 insertions.
template <int LT>
__device__ __forceinline__ void best_of_32(float (&d)[32], uint32_t (&id)[32], float (&ld)[LT], uint32_t (&li)[LT])
{
    if constexpr (LT == 8) {
#pragma unroll
        for (int g = 0; g < 4; ++g)
            sort8(d, id, 8 * g);
        merge8_keep(d, id, 0, 8);
        merge8_keep(d, id, 16, 24);
        merge8_keep(d, id, 0, 16);
    } else {
#pragma unroll
        for (int k = 2; k <= 32; k <<= 1)
#pragma unroll
            for (int j = k >> 1; j > 0; j >>= 1)
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    const int l = i ^ j;
                    if (l > i) {
                        if ((i & k) == 0)
                            cas(d, id, i, l);
                        else
                            cas(d, id, l, i);
                    }
                }
    }
#pragma unroll
    for (int j = 0; j < LT; ++j) {
        ld[j] = d[j];
        li[j] = id[j];
    }
}

// Ascending bitonic sort of 32 (dist, id) entries (240 compare-exchanges).
__device__ __forceinline__ void sort32(float (&d)[32], uint32_t (&id)[32])
{
#pragma unroll
    for (int k = 2; k <= 32; k <<= 1)
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1)
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                const int l = i ^ j;
                if (l > i) {
                    if ((i & k) == 0)
                        cas(d, id, i, l);
                    else
                        cas(d, id, l, i);
                }
            }
}

// The 32 smallest of an ascending queue of 32 and 32 new entries, ascending, into the
// queue: the new entries sorted, a half cleaner (queue[i] vs new[31-i]) leaves the 32
// smallest as a bitonic run, a bitonic merge sorts it (352 compare-exchanges in all,
// whatever the number of entries that enter).
__device__ __forceinline__ void merge_into_queue32(float (&d)[32], uint32_t (&id)[32], float (&ld)[32],
                                                   uint32_t (&li)[32])
{
    sort32(d, id);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const bool t = d[31 - i] < ld[i];
        ld[i] = t ? d[31 - i] : ld[i];
        li[i] = t ? id[31 - i] : li[i];
    }
#pragma unroll
    for (int j = 16; j > 0; j >>= 1)
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const int l = i ^ j;
            if (l > i)
                cas(ld, li, i, l);
        }
}

// Operand loads from the split base set (rows of dp words, every chunk whole):
//   LOAD_BUF32 : split set smaller than 4 GiB -- candidate rows by buffer loads with
//                32-bit byte offsets; the k-chunk advances a scalar offset, so the main
//                loop spends no vector ALU work on addresses;
//   LOAD_WIDE  : larger -- candidate rows through 64-bit row pointers (one add per load).
// In both the item's query rows are read through a buffer of exactly those rows.
enum : int { LOAD_BUF32 = 1, LOAD_WIDE = 2 };

// Staging area of the NB = 1 layout: each thread's 32 values of its list (row stride 36
// words spreads the 16-byte stores over the banks).
struct alignas(16) SelectStage {
    float v[2 * NTHREADS][36];
};
struct NoStage {};

// NB query columns per lane: NB = 2 -- 4 waves, each a 64x64 block (2x2 accumulators),
// two blocks per CU; NB = 1 -- 8 waves, each a 64x32 block, one block per CU, half the
// queue registers per lane (long queues at two waves per SIMD).
template <int NB>
constexpr int select_threads()
{
    return NB == 2 ? NTHREADS : 2 * NTHREADS;
}

template <int LT, int MODE, bool EXCL, int NB, bool QR>
__global__ __launch_bounds__(select_threads<NB>(), (LT <= 8 ? 2 : 1)) void ung_select_kernel(SelectParams P)
{
    static_assert(NB == 1 || NB == 2, "one or two query columns per lane");
    static_assert(!QR || (NB == 2 && LT == 8), "register-query layout: NB = 2, LT = 8");
    constexpr int NTH = select_threads<NB>();
    constexpr int WN = 4 / NB;         // query waves
    constexpr int QW = 32 * NB;        // query columns per wave
    constexpr int RSTEP = NTH / 8;     // loader row step
    constexpr int LM = BQ / RSTEP;     // rows per thread and panel
    __shared__ typename std::conditional<QR, SelectSmemQ, SelectSmem>::type sm;
    __shared__ typename std::conditional<NB == 1, SelectStage, NoStage>::type stage;
    // long queues: [tile parity][candidate wave][query] the larger m4-th entry of a wave's
    // two queues of the query
    struct Tau4 {
        float v[2][2][BQ];
    };
    __shared__ typename std::conditional<(LT >= 16), Tau4, NoStage>::type tau4;
    __shared__ uint32_t item_slot;
    const uint32_t logical = take_item(P.item_ctr, &item_slot);
    if (logical >= P.n_items)
        return;
    const Item it = P.items[logical];
    const Job jb = P.jobs[it.job];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave / WN, wn = wave % WN;
    const int r = lane & 31, h = lane >> 5;
    // block-uniform values loaded with vector loads: readfirstlane keeps the query
    // buffer descriptor of the wide mode in scalar registers
    const uint32_t q0 = __builtin_amdgcn_readfirstlane(jb.q_begin + it.q_off);
    const uint32_t qcnt = __builtin_amdgcn_readfirstlane(it.q_cnt);
    const uint32_t dp = QR ? (uint32_t)(QR_NK * KC) : P.dp;
    const uint32_t *__restrict__ XS = P.xs;

    if (tid < BQ)
        sm.qn[tid] = (uint32_t)tid < qcnt ? P.xn[q0 + tid] : 0.0f;
    RowCursor cur;
    finish_rowids(sm, 0, start_rowids(sm, 0, cur, P, jb, it.v_begin, it.v_end, tid), tid);

    float ld[NB][LT];
    uint32_t li[NB][LT];
    float tfin[NB]; // lowest threshold a queue has applied so far
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
        tfin[nb] = INFINITY;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int j = 0; j < LT; ++j) {
            ld[nb][j] = INFINITY;
            li[nb][j] = NONE;
        }
    // thresholds may be shared between a query's queues only when one queue's LT
    // entries already cover the k results
    const bool share = P.k <= (uint32_t)LT;
    // counting bound: 4*m4 >= Lp+1 (Lp = P.lp < 4*LT)
    const uint32_t m4 = (P.lp + 4u) / 4u;
    // LT = 8: the counting bound replaces the other wave's share bound in sm.tau (it is
    // the tighter one once the queues hold m4 entries); pm4o: this wave's value of the
    // query after its latest tile
    constexpr bool CNT8 = LT == 8;
    [[maybe_unused]] float pm4o[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
        pm4o[nb] = INFINITY;

    // loader mapping: rows lr = (tid>>3) + RSTEP*m, columns c4 .. c4+3 of the chunk
    const int lr0 = tid >> 3;
    const int c4 = (tid & 7) * 4;
    [[maybe_unused]] __amdgpu_buffer_rsrc_t qres, xres;
    [[maybe_unused]] uint32_t xoff[LM];
    [[maybe_unused]] const uint32_t *xrow[LM];
    if constexpr (MODE == LOAD_BUF32)
        xres = __builtin_amdgcn_make_buffer_rsrc((void *)XS, (short)0, (int)P.x_bytes, 0x00020000);
    // the item's query rows: a buffer of exactly qcnt rows, so that rows past them
    // (padding columns, whose results are never read) read zeros without touching memory
    qres = __builtin_amdgcn_make_buffer_rsrc((void *)(XS + (size_t)q0 * dp), (short)0, (int)(qcnt * dp * 4u),
                                             0x00020000);
    // query rows lr0 + RSTEP*m: one vector offset, the row steps as scalar offsets
    const uint32_t qrow_step = (uint32_t)RSTEP * dp * 4u;
    const uint32_t qoff = ((uint32_t)lr0 * dp + (uint32_t)c4) * 4u;

    // register-query layout: the high words of this lane's query columns (k-block kb:
    // chunk kb/2, float4 column 2*(kb%2) + h of the chunk row) and the low words of all
    // the item's queries (float4 column 4*chunk + c of row q) into LDS
    [[maybe_unused]] bf16x8 bhr[2 * QR_NK][NB];
    if constexpr (QR) {
        // rows of the item's queries (row 0 of qres is query q0; zeros past its qcnt rows)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const uint32_t row = (uint32_t)(wn * QW + 32 * nb + r);
#pragma unroll
            for (int kb = 0; kb < 2 * QR_NK; ++kb)
                bhr[kb][nb] = __builtin_bit_cast(
                    bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                qres, (row * dp + (uint32_t)((kb >> 1) * KC + (2 * (kb & 1) + h) * 4)) * 4u, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < BQ * QR_NK * 4 / NTH; ++i) {
            const int idx = tid + NTH * i;
            const int q = idx >> 4, f = idx & 15; // f = 4*chunk + float4 column of the low words
            const uint32_t off = ((uint32_t)q * dp + (uint32_t)((f >> 2) * KC + 16 + (f & 3) * 4)) * 4u;
            sm.u.p.qlo[q][f] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(qres, off, 0, 0));
        }
    }

    __syncthreads();
    float qnv[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
        qnv[nb] = sm.qn[wn * QW + nb * 32 + r];

    // One flat software pipeline over (candidate tile, k-chunk) steps: the panels are
    // double-buffered in LDS and each step prefetches the next step's chunk (also
    // across tile boundaries) into registers; the row-id table of tile t+1 is built
    // in ring slot (t+1)%3 while tile t computes.
    const uint32_t ntiles = (it.v_end - it.v_begin + BC - 1) / BC;
    const uint32_t nk = dp / KC;
    const uint32_t total = ntiles * nk;

    auto set_xrows = [&](int slot) {
#pragma unroll
        for (int m = 0; m < LM; ++m) {
            uint32_t g = sm.rowid[slot][lr0 + RSTEP * m];
            g = (g == NONE) ? 0u : g; // padding rows load row 0 (their -|x|^2/2 is -inf)
            if constexpr (MODE == LOAD_BUF32)
                xoff[m] = (g * dp + (uint32_t)c4) * 4u;
            else
                xrow[m] = XS + (size_t)g * dp + c4;
        }
    };
    [[maybe_unused]] float4 rq[LM];
    float4 rx[LM]; // raw split words (bf16 pairs), typed for 16-byte moves
    auto load_chunk = [&](uint32_t kc) {
#pragma unroll
        for (int m = 0; m < LM; ++m) {
            if constexpr (MODE == LOAD_BUF32) {
                if constexpr (!QR)
                    rq[m] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(qres, qoff, kc * 4u + m * qrow_step, 0));
                rx[m] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xres, xoff[m], kc * 4u, 0));
            } else {
                if constexpr (!QR)
                    rq[m] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(qres, qoff, kc * 4u + m * qrow_step, 0));
                rx[m] = __builtin_bit_cast(float4, *reinterpret_cast<const u32x4 *>(xrow[m] + kc));
            }
        }
    };

    // accumulators start at 0 (the first chunk's MFMAs take C = 0) and hold <x,q> after
    // the k-loop; the epilogue adds the row's -|x|^2/2 once, so acc = -s with
    // s = |x|^2/2 - <x,q>  (padding rows: -inf).  Adding the norm term last keeps the
    // running sums at the size of the products, which halves the accumulation error of
    // the certified bound.
    floatx16 acc[2][NB];

    __syncthreads(); // ring slot 0 and qn visible
    set_xrows(0);
    load_chunk(0);

    uint32_t tile = 0, kc_state = 0;
    int slot = 0;
    float pend_nx = INFINITY;
    // one step; kcv: the chunk index, a compile-time constant in the register-query layout
    auto step = [&](uint32_t s, auto kcv) __attribute__((always_inline)) {
        const uint32_t kc = (uint32_t)kcv;
        const int buf = (int)(s & 1u);
        const int next_slot = slot == 2 ? 0 : slot + 1;
#pragma unroll
        for (int m = 0; m < LM; ++m) {
            if constexpr (!QR)
                sm.u.p.qs[buf][lr0 + RSTEP * m][c4 >> 2] = rq[m];
            sm.u.p.xs[buf][lr0 + RSTEP * m][c4 >> 2] = rx[m];
        }
        if (nk == 1 && tile + 1 < ntiles)
            finish_rowids(sm, next_slot,
                          start_rowids(sm, next_slot, cur, P, jb, it.v_begin + (tile + 1) * BC, it.v_end, tid), tid);
        // |x|^2 of the next tile's rows, loaded during the previous step
        if (nk > 1 && kc == 1 && tile + 1 < ntiles)
            finish_rowids(sm, next_slot, pend_nx, tid);
        __syncthreads();
        if (s + 1 < total) {
            if (kc + 1 == nk) {
                set_xrows(next_slot);
                load_chunk(0);
            } else {
                load_chunk((kc + 1) * KC);
            }
        }
        // The chunk's 32 dimensions as two k-blocks of 16; a panel row holds the bf16 high
        // parts of the 32 dimensions (words 0..15) then the low parts (words 16..31).
        // Lane half h feeds dimensions 16*kb + 8h .. +7 of block kb (8 bf16 = one float4),
        // the same k order for the candidate (A) and query (B) operands.  Three passes per
        // block: hi*hi, hi*lo, lo*hi (the dropped lo*lo term is within the error bound);
        // pass-major order keeps four independent accumulators between dependent MFMAs.
        // A tile's first MFMA of each accumulator takes C = 0 (no zeroing instructions).
        auto mfma_chunk = [&](auto first_chunk) {
            constexpr bool FIRST = decltype(first_chunk)::value;
            const floatx16 zero = {};
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int ch = 2 * kb + h; // float4 column of the high parts; +4: low parts
                bf16x8 ah[2], al[2], bh[NB], bl[NB];
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    ah[mb] = __builtin_bit_cast(bf16x8, sm.u.p.xs[buf][wm * 64 + 32 * mb + r][ch]);
                    al[mb] = __builtin_bit_cast(bf16x8, sm.u.p.xs[buf][wm * 64 + 32 * mb + r][ch + 4]);
                }
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    if constexpr (QR) {
                        constexpr int KCI = decltype(kcv)::value;
                        bh[nb] = bhr[2 * KCI + kb][nb];
                        bl[nb] = __builtin_bit_cast(bf16x8, sm.u.p.qlo[wn * QW + 32 * nb + r][4 * KCI + ch]);
                    } else {
                        bh[nb] = __builtin_bit_cast(bf16x8, sm.u.p.qs[buf][wn * QW + 32 * nb + r][ch]);
                        bl[nb] = __builtin_bit_cast(bf16x8, sm.u.p.qs[buf][wn * QW + 32 * nb + r][ch + 4]);
                    }
                }
                const bool z = FIRST && kb == 0;
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb)
                        acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[mb], bh[nb], z ? zero : acc[mb][nb], 0, 0, 0);
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb)
                        acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[mb], bl[nb], acc[mb][nb], 0, 0, 0);
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb)
                        acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[mb], bh[nb], acc[mb][nb], 0, 0, 0);
            }
        };
        // the MFMA block at raised wave priority: the SIMD's other wave (in its epilogue's
        // VALU work) yields issue slots to it, which keeps the matrix core fed.  In the
        // register-query layout the priority also grows with the chunk (1, 2, 3, 3): of
        // two waves in their MFMA steps, the one nearer its epilogue issues first, so it
        // reaches the epilogue while the other still has matrix work.  Their phases drift
        // apart instead of locking (cfg2 cross select -1.5 to 2 %).  With restaged query
        // panels (12 to 24 chunks a tile) a graded priority measured slower, so those
        // steps stay at 1.
        if constexpr (QR) {
            constexpr uint32_t KCP = decltype(kcv)::value + 1u;
            __builtin_amdgcn_s_setprio(KCP > 3u ? 3 : (int16_t)KCP);
        } else {
            __builtin_amdgcn_s_setprio(1);
        }
        if (kc == 0)
            mfma_chunk(std::true_type{});
        else
            mfma_chunk(std::false_type{});
        __builtin_amdgcn_s_setprio(0);
        // next tile's row ids: issued after this step's MFMAs, visible after the next
        // step's barrier, consumed by the prefetch of the tile's first chunk (at step
        // nk-1 >= 1); the |x|^2 values are stored at the top of step 1
        if (nk > 1 && kc == 0 && tile + 1 < ntiles)
            pend_nx = start_rowids(sm, next_slot, cur, P, jb, it.v_begin + (tile + 1) * BC, it.v_end, tid);

        if (kc + 1 == nk) {
            // epilogue: acc[mb][nb][i] = -s for row tile_row(wm, h, 16*mb + i) and query
            // col = wn*QW+nb*32+r, s = |x|^2/2 - <x,q>; the expansion-form distance is
            // a = fl(2s + |q|^2) = fma(-2, acc, |q|^2) (padding rows: acc = -inf).
            //
            // The four queues of a query (lane halves h, candidate waves wm) share a
            // threshold: a candidate is queued only if a < min(own LT-th, partner lane's,
            // other wave's of the previous tile).  Any candidate with a >= that value can
            // not be among the query's LT best (one queue already holds LT better ones),
            // and thresholds only decrease, so a stale value is safe.
            //
            // Queues of LT = 8 and LT >= 16 also apply a counting bound, valid for any k:
            // the query's four queues hold m4 entries each at or below the largest of their
            // m4-th entries (4*m4 >= Lp+1 entries in all), so a candidate at or above that
            // value is not among the query's Lp+1 best.  The other wave's value is from the
            // previous tile: entries only decrease, so it bounds the current one.  (For
            // k = 6, Lp = 10: the larger of the four queues' 3rd entries, near the query's
            // 16th best, against about its 26th for the smallest of their 8th entries.)
            float tsh[NB], ncth[NB];
            [[maybe_unused]] float pm4[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const int col = wn * QW + nb * 32 + r;
                const float own = ld[nb][LT - 1];
                const float partner = __shfl_xor(own, 32);
                float t = fminf(own, tfin[nb]);
                if (share) {
                    t = fminf(t, partner);
                    if (!CNT8 && tile > 0)
                        t = fminf(t, sm.tau[(tile - 1) & 1][wm ^ 1][col]);
                }
                if constexpr (CNT8)
                    if (tile > 0)
                        t = fminf(t, fmaxf(pm4o[nb], sm.tau[(tile - 1) & 1][wm ^ 1][col]));
                if constexpr (LT >= 16) {
                    float o4 = INFINITY;
#pragma unroll
                    for (int j = 0; j < LT; ++j)
                        o4 = (uint32_t)j + 1u == m4 ? ld[nb][j] : o4;
                    pm4[nb] = fmaxf(o4, __shfl_xor(o4, 32));
                    if (tile > 0)
                        t = fminf(t, fmaxf(pm4[nb], tau4.v[(tile - 1) & 1][wm ^ 1][col]));
                }
                tsh[nb] = t;
                ncth[nb] = -s_bound(t, qnv[nb]);
            }
            // The row's -|x|^2/2 and the pre-filter bound are added by one more MFMA per
            // accumulator: the A row carries -|x|^2/2 split exactly into three bf16 terms
            // (k = 0..2, lane half 0; a padding row's -inf in the first term alone) and 1 at
            // k = 3..5; B is 1 at k = 0..2 and carries the query column's bound cb split
            // exactly into three bf16 terms (truncations: hi + mid + lo = cb) at k = 3..5.
            // So acc = -s + cb and a candidate is pending iff acc > 0 (s < cb; the sign
            // bit, a padding row's -inf included, rejects it), and the round reads
            // -s = acc - cb.  cb (s-space, with slack: a superset of a < tsh) is the larger
            // of the column's two lanes' bounds; it is 0 on the first tile and whenever
            // some lane of the wave has no finite bound yet (then the pending test is
            // -cb' - acc < 0 with the lane's own bound cb', as before the fold).
            float cb[NB];
            bool fold = tile > 0;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                cb[nb] = fmaxf(-ncth[nb], -__shfl_xor(ncth[nb], 32));
                fold = fold && cb[nb] < INFINITY;
            }
            fold = __ballot(!fold) == 0;
            {
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    cb[nb] = fold ? cb[nb] : 0.0f;
                bf16x8 bcol[NB];
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const uint32_t u0 = __float_as_uint(cb[nb]) & 0xFFFF0000u;
                    const float r1 = cb[nb] - __uint_as_float(u0);
                    const uint32_t u1 = __float_as_uint(r1) & 0xFFFF0000u;
                    const uint32_t u2 = __float_as_uint(r1 - __uint_as_float(u1)) & 0xFFFF0000u;
                    // k = 0..7 (lane half 1 meets zeros in A): 1, 1, 1, hi, mid, lo, 0, 0
                    bcol[nb] = __builtin_bit_cast(bf16x8, make_uint4(0x3F803F80u, 0x3F80u | u0, (u1 >> 16) | u2, 0u));
                }
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    const uint2 w = sm.nhx[slot][wm * 64 + 32 * mb + r];
                    const bf16x8 abias = __builtin_bit_cast(
                        bf16x8, make_uint4(h == 0 ? w.x : 0u, h == 0 ? (w.y | 0x3F800000u) : 0u, h == 0 ? 0x3F803F80u : 0u, 0u));
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb)
                        acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(abias, bcol[nb], acc[mb][nb], 0, 0, 0);
                }
            }
            // branch-free pass: per list a lane mask whose bit (31 - j) marks element j
            // under the pre-filter bound (folded: the sign bit of acc, inverted; otherwise
            // s < c  <=>  the sign bit of -c - acc, where a NaN from -inf - -inf only marks a
            // padding row, which the round rejects)
            uint32_t pend[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                pend[nb] = 0u;
            if (fold) {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int i = 0; i < 16; ++i)
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb)
                            pend[nb] = (pend[nb] << 1) | (__float_as_uint(acc[mb][nb][i]) >> 31);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    pend[nb] = ~pend[nb];
            } else {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int i = 0; i < 16; ++i)
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb)
                            pend[nb] = (pend[nb] << 1) | (__float_as_uint(ncth[nb] - acc[mb][nb][i]) >> 31);
            }
            // self exclusion (candidate space = query space): clear the query's own bit
            uint32_t self_j[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                self_j[nb] = 32u;
            if constexpr (EXCL) {
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const int o = (int)(it.q_off + (uint32_t)(wn * QW + nb * 32 + r)) -
                                  (int)(it.v_begin + tile * BC) - (wm * 64 + 4 * h);
                    self_j[nb] = lane_index_of(o);
                    pend[nb] &= self_j[nb] < 32u ? ~(0x80000000u >> self_j[nb]) : 0xFFFFFFFFu;
                }
            }
            // rounds: each lane inserts at most one pending element of mask m per round; the
            // body is branch-free (an idle lane inserts +inf, which changes nothing) and the
            // round count is the wave's largest pending count (binary search on ballots:
            // wave-uniform, no cross-lane data movement).  staged(j) is element j's value.
            auto round_count = [&](uint32_t m) __attribute__((always_inline)) -> uint32_t {
                const uint32_t np = (uint32_t)__popc(m);
                uint32_t nr = 0;
#pragma unroll
                for (int b = 5; b >= 0; --b) {
                    const uint32_t c = nr | (1u << b);
                    if (__ballot(np >= c))
                        nr = c;
                }
                return nr;
            };
            auto rounds = [&](int nb, uint32_t m, uint32_t nr, auto &&staged) __attribute__((always_inline)) {
                for (uint32_t rr = 0; rr < nr; ++rr) {
                    const uint32_t j = (uint32_t)__builtin_clz(m | 1u);
                    const bool act = m != 0u;
                    m &= ~(0x80000000u >> j);
                    const float av = staged(j) - cb[nb];
                    const uint32_t rid = sm.rowid[slot][tile_row(wm, h, j)];
                    float dd = __builtin_fmaf(-2.0f, av, qnv[nb]);
                    dd = (act && dd < ld[nb][LT - 1] && dd < tsh[nb]) ? dd : INFINITY;
                    list_insert<LT>(ld[nb], li[nb], dd, rid);
                }
            };
            // (dist, id) of element j of list nb for the first tile's sorting network
            auto entry = [&](int nb, int j, uint32_t idg, float &dd, uint32_t &id) __attribute__((always_inline)) {
                dd = __builtin_fmaf(-2.0f, acc[j >> 4][nb][j & 15] - cb[nb], qnv[nb]);
                if constexpr (EXCL)
                    dd = (uint32_t)j == self_j[nb] ? INFINITY : dd;
                id = dd < INFINITY ? idg : NONE;
            };
            if constexpr (!QR) {
                // One list's 32 values are staged in LDS, so a round reads its element with
                // one LDS load instead of a register select tree.  NB = 2: each thread owns
                // the 8 panel slots it fills at the next step (buffer buf^1, read by no wave
                // before the next barrier), slot g holding values 4g..4g+3; NB = 1: its row
                // of the staging area.
                float *const pnl = reinterpret_cast<float *>(&sm.u.p);
                [[maybe_unused]] const int own0 = ((buf ^ 1) * BQ + lr0) * LDSW + c4;
                auto staged = [&](uint32_t j) -> float & {
                    if constexpr (NB == 1)
                        return stage.v[tid][j];
                    else
                        return pnl[own0 + (int)(j >> 4) * PANEL_X + (int)((j >> 2) & 3u) * ROW32 + (int)(j & 3u)];
                };
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
                    for (int g = 0; g < 8; ++g) {
                        const int mb = g >> 2, g4 = g & 3;
                        const float4 v = make_float4(acc[mb][nb][4 * g4], acc[mb][nb][4 * g4 + 1],
                                                     acc[mb][nb][4 * g4 + 2], acc[mb][nb][4 * g4 + 3]);
                        *reinterpret_cast<float4 *>(&staged(4u * (uint32_t)g)) = v;
                    }
                    if (tile == 0) {
                        // first tile: the queues are empty; a sorting network keeps the LT
                        // best of the tile's 32 candidates instead of up to 32 insertion rounds
                        float dv[32];
                        uint32_t iv[32];
#pragma unroll
                        for (int g = 0; g < 8; ++g) {
                            const uint4 ids = *reinterpret_cast<const uint4 *>(&sm.rowid[slot][tile_row(wm, h, 4u * g)]);
                            const uint32_t idg[4] = {ids.x, ids.y, ids.z, ids.w};
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                entry(nb, 4 * g + e, idg[e], dv[4 * g + e], iv[4 * g + e]);
                        }
                        best_of_32<LT>(dv, iv, ld[nb], li[nb]);
                    } else {
                        const uint32_t nr = round_count(pend[nb]);
                        bool merged = false;
                        if constexpr (LT == 32) {
                            // an early tile of a long queue: more than ~13 rounds (about 142
                            // instructions each) cost more than merging the tile's 32 entries
                            // with a sorting network (about 1,900)
                            if (nr > 13u) {
                                float dv[32];
                                uint32_t iv[32];
#pragma unroll
                                for (int g = 0; g < 8; ++g) {
                                    const uint4 ids =
                                        *reinterpret_cast<const uint4 *>(&sm.rowid[slot][tile_row(wm, h, 4u * g)]);
                                    const uint32_t idg[4] = {ids.x, ids.y, ids.z, ids.w};
#pragma unroll
                                    for (int e = 0; e < 4; ++e)
                                        entry(nb, 4 * g + e, idg[e], dv[4 * g + e], iv[4 * g + e]);
                                }
                                merge_into_queue32(dv, iv, ld[nb], li[nb]);
                                merged = true;
                            }
                        }
                        if (!merged)
                            rounds(nb, pend[nb], nr, staged);
                    }
                }
            } else {
                // register-query layout: no LDS room to stage a list, a round reads its
                // element from the accumulators through a select tree
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    if (tile == 0) {
                        // first tile: best 8 of each half by a sorting network, then the
                        // best 8 of both
                        float dv[16];
                        uint32_t iv[16];
#pragma unroll
                        for (int hv = 0; hv < 2; ++hv) {
#pragma unroll
                            for (int g = 0; g < 4; ++g) {
                                const uint4 ids =
                                    *reinterpret_cast<const uint4 *>(&sm.rowid[slot][tile_row(wm, h, 16u * hv + 4u * g)]);
                                const uint32_t idg[4] = {ids.x, ids.y, ids.z, ids.w};
#pragma unroll
                                for (int e = 0; e < 4; ++e)
                                    entry(nb, 16 * hv + 4 * g + e, idg[e], dv[4 * g + e], iv[4 * g + e]);
                            }
                            sort8(dv, iv, 0);
                            sort8(dv, iv, 8);
                            merge8_keep(dv, iv, 0, 8);
                            if (hv == 1) {
#pragma unroll
                                for (int j = 0; j < 8; ++j) {
                                    dv[8 + j] = ld[nb][j];
                                    iv[8 + j] = li[nb][j];
                                }
                                merge8_keep(dv, iv, 0, 8);
                            }
#pragma unroll
                            for (int j = 0; j < 8; ++j) {
                                ld[nb][j] = dv[j];
                                li[nb][j] = iv[j];
                            }
                        }
                    } else {
                        // element j of the list through a select tree over its 32
                        // accumulator values (bit 4 of j: the half, bits 3..0: the entry)
                        // (each level's bit of j sign-extended to a lane mask by one
                        // bit-field extract; each select one bit-select instruction)
                        auto pick = [&](uint32_t j) -> float {
                            auto sel = [](uint32_t m, float a, float b) {
                                return __uint_as_float((__float_as_uint(a) & m) | (__float_as_uint(b) & ~m));
                            };
                            // (the empty asm keeps the compiler from turning the masks
                            // back into compares and lane-mask selects)
                            float v[16];
                            uint32_t m = (uint32_t)__builtin_amdgcn_sbfe((int)j, 4, 1);
                            asm("" : "+v"(m));
#pragma unroll
                            for (int i = 0; i < 16; ++i)
                                v[i] = sel(m, acc[1][nb][i], acc[0][nb][i]);
#pragma unroll
                            for (int w = 8, b = 3; w >= 1; w >>= 1, --b) {
                                m = (uint32_t)__builtin_amdgcn_sbfe((int)j, b, 1);
                                asm("" : "+v"(m));
#pragma unroll
                                for (int i = 0; i < w; ++i)
                                    v[i] = sel(m, v[i + w], v[i]);
                            }
                            return v[0];
                        };
                        rounds(nb, pend[nb], round_count(pend[nb]), pick);
                    }
                }
            }
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                // publish this wave's threshold of the query for the other wave
                const float t = fminf(tsh[nb], ld[nb][LT - 1]);
                tfin[nb] = t;
                if constexpr (CNT8) {
                    float o4 = INFINITY;
#pragma unroll
                    for (int j = 0; j < LT; ++j)
                        o4 = (uint32_t)j + 1u == m4 ? ld[nb][j] : o4;
                    pm4o[nb] = fmaxf(o4, __shfl_xor(o4, 32));
                    if (h == 0)
                        sm.tau[tile & 1][wm][wn * QW + nb * 32 + r] = pm4o[nb];
                } else {
                    const float pair_t = fminf(t, __shfl_xor(t, 32));
                    if (share && h == 0)
                        sm.tau[tile & 1][wm][wn * QW + nb * 32 + r] = pair_t;
                }
                if constexpr (LT >= 16)
                    if (h == 0)
                        tau4.v[tile & 1][wm][wn * QW + nb * 32 + r] = pm4[nb];
            }
            ++tile;
            kc_state = 0;
            slot = next_slot;
        } else {
            ++kc_state;
        }
    };
    if constexpr (QR) {
        for (uint32_t s = 0; s < total; s += QR_NK) {
            step(s, std::integral_constant<uint32_t, 0>{});
            step(s + 1, std::integral_constant<uint32_t, 1>{});
            step(s + 2, std::integral_constant<uint32_t, 2>{});
            step(s + 3, std::integral_constant<uint32_t, 3>{});
        }
    } else {
        for (uint32_t s = 0; s < total; ++s)
            step(s, kc_state);
    }

    // ---- per query: the Lp best queued candidates by approximate distance, and a
    // bound every other candidate of this split satisfies (two passes of 64 queries) ----
    constexpr int E = 4 * LT;
    const uint32_t Lp = P.lp;
    const int npass = qcnt > 64 ? 2 : 1;
    for (int pass = 0; pass < npass; ++pass) {
        const int rows_here = (int)min(64u, qcnt - (uint32_t)pass * 64u);
        __syncthreads();
        // the waves whose query columns lie in this pass's 64 queries
        if ((wn * QW) / 64 == pass) {
            const int lid = wm * 2 + h;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const int jl = (wn * QW) % 64 + nb * 32 + r;
#pragma unroll
                for (int j = 0; j < LT; ++j) {
                    sm.u.r.ed[jl][lid * LT + j] = ld[nb][j];
                    sm.u.r.ei[jl][lid * LT + j] = li[nb][j];
                }
                // every candidate this queue never kept has a >= this value
                sm.u.r.alist[jl][lid] = fminf(ld[nb][LT - 1], tfin[nb]);
            }
        }
        __syncthreads();
        // one thread per query: 4-way merge of the sorted queues -> approximate top-Lp;
        // the first value left out joins the bound
        if (tid < rows_here) {
            const int jl = tid;
            const uint32_t ql = (uint32_t)(pass * 64 + jl);
            const size_t prow = (size_t)jb.part_base + (size_t)it.split * jb.q_count + it.q_off + ql;
            int hp[4] = {0, 0, 0, 0};
            float drop = INFINITY;
            for (uint32_t t = 0; t <= Lp; ++t) {
                float bd = INFINITY;
                uint32_t bi = NONE;
                int bl = -1;
#pragma unroll
                for (int l = 0; l < 4; ++l) {
                    if (hp[l] < LT) {
                        const float dl = sm.u.r.ed[jl][l * LT + hp[l]];
                        const uint32_t il = sm.u.r.ei[jl][l * LT + hp[l]];
                        if (il != NONE && cand_less(dl, il, bd, bi)) {
                            bd = dl;
                            bi = il;
                            bl = l;
                        }
                    }
                }
                if (t == Lp) {
                    drop = bd;
                    break;
                }
                P.part_ids[prow * Lp + t] = bi;
                P.part_dist[prow * Lp + t] = bd;
                if (bl >= 0)
                    ++hp[bl];
            }
            float A = drop;
#pragma unroll
            for (int l = 0; l < 4; ++l)
                A = fminf(A, sm.u.r.alist[jl][l]);
            P.part_bound[prow] = A; // approximate-distance space
        }
    }
}

// ---------------------------------------------------------------------------
// filter-and-buffer select (group kNN lists)
// ---------------------------------------------------------------------------
// For group kNN calls with d <= 128 whose splits hold fewer than 65,536 candidates (the
// mid-group batch of the exact kNN stage: K = 32, Lp = 40).  ung_select_kernel needs
// queues of LT >= K entries for such lists, and their sorted insertions (about 4.4
// instructions per queue entry, for the wave's largest survivor count) dominate it;
// here a survivor costs one LDS append:
//   * each query has a buffer of up to KNN_CAP (value, candidate) entries in LDS and a
//     threshold tau: every candidate of the split whose value is below tau is in the
//     buffer, so no candidate at or above tau is needed again;
//   * per tile, a lane's values that pass a branch-free pre-filter (in s-space, a
//     superset of a < tau) are appended behind one LDS atomic per lane; the first tile
//     (tau = +inf) appends every candidate;
//   * when a buffer holds more than KNN_TRIG entries (KNN_TRIG_LATE from the third tile
//     on, when far fewer values pass) the block refreshes all buffers: a 64-bin
//     histogram of a query's live entries (below tau) over [min, max], counted in
//     registers (refined into 8 parts when the bin alone would pass the limit), gives
//     the bin of its (Lp+1)-th value; the buffer keeps the bins up to it (only those
//     below it when that would be more than the limit) and tau drops to the smallest
//     value left out (every kept value is below it: the bin is monotone in the value);
//   * a buffer that would overflow drops the values and records the smallest, which
//     caps tau at the next refresh, so the first point holds again;
//   * after the last tile a final refresh keeps at most KNN_OUT entries; four threads
//     per query sort them by value (bitonic, 16 each) and write the partial row: its Lp
//     smallest entries and the bound min(tau, the (Lp+1)-th).
// Every candidate left out of the row then has a value at or above the bound: the
// partial-row contract of ung_select_kernel, whose merge, certificate and rescan follow.
// The query operands stay in registers for the whole item (16 words per 32-dimension
// chunk and lane), so a step loads and stages only the candidate chunk.
constexpr int KNN_CAP = 128;              // buffer entries per query
constexpr int KNN_VROW = KNN_CAP + 4;     // value row stride in floats (16-byte rows; bank rotation)
constexpr int KNN_IROW = KNN_CAP + 8;     // candidate row stride in u16
constexpr uint32_t KNN_TRIG = 80;         // a buffer above this many entries asks for a refresh (tiles 0, 1)
constexpr uint32_t KNN_TRIG_LATE = 100;   // from tile 2 on (fewer values pass a tile)
constexpr uint32_t KNN_KEEP = 80;         // most entries a refresh keeps
constexpr uint32_t KNN_OUT = 64;          // most entries the final refresh keeps (4 threads x 16)
constexpr int KNN_THREADS = 512;          // 8 waves: 2 (candidate halves) x 4 (query quarters)
constexpr uint32_t KNN_MAX_SPLIT = 65535; // candidates per item (16-bit candidate index)
constexpr int KNN_MAX_NK = 4;             // dp <= 128

struct alignas(16) KnnSmem {
    float4 xs[2][BC][LDSW / 4];     // candidate chunks, double-buffered
    float bval[BQ][KNN_VROW];       // buffer values (expansion-form distances)
    uint16_t bidx[BQ][KNN_IROW];    // their candidates (index in the item's split)
    uint32_t rowid[3][BC];
    uint2 nhx[3][BC];
    float qn[BQ];
    float tau[BQ];
    uint32_t lost[BQ];  // order key of the smallest value a full buffer dropped
    uint32_t fill[BQ];
    uint32_t need[2];   // by tile parity: some buffer passed its refresh trigger
};
static_assert(KNN_THREADS == 4 * BQ, "four threads per query in the refresh and the sort");

// Unsigned key with the order of the float (negative values included).
__device__ __forceinline__ uint32_t ord_key(float f)
{
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ord_val(uint32_t k)
{
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Value of lane (lane ^ X) within each group of four lanes (DPP quad permutation).
template <int X>
__device__ __forceinline__ uint32_t quad_xor(uint32_t v)
{
    static_assert(X == 1 || X == 2, "partner within the quad");
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, X == 1 ? 0xB1 : 0x4E, 0xF, 0xF, false);
}
template <int X>
__device__ __forceinline__ float quad_xor(float v)
{
    return __uint_as_float(quad_xor<X>(__float_as_uint(v)));
}
__device__ __forceinline__ uint32_t quad_sum(uint32_t v)
{
    v += quad_xor<1>(v);
    return v + quad_xor<2>(v);
}
__device__ __forceinline__ float quad_min(float v)
{
    v = fminf(v, quad_xor<1>(v));
    return fminf(v, quad_xor<2>(v));
}
__device__ __forceinline__ float quad_max(float v)
{
    v = fmaxf(v, quad_xor<1>(v));
    return fmaxf(v, quad_xor<2>(v));
}
// Inclusive prefix sum over the quad (lane order p = lane & 3): add lane p-1's value
// (quad_perm [0,0,1,2]), then lane p-2's partial sum (lanes 2, 3 read lanes 0, 1).
__device__ __forceinline__ uint32_t quad_incl(uint32_t v, int p)
{
    const uint32_t a = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x90, 0xF, 0xF, false);
    v += p >= 1 ? a : 0u;
    const uint32_t b = quad_xor<2>(v);
    return v + (p >= 2 ? b : 0u);
}

template <int MODE, int NK>
__global__ __launch_bounds__(KNN_THREADS, 1) void ung_knn_select_kernel(SelectParams P)
{
    constexpr int NTH = KNN_THREADS;
    constexpr int RSTEP = NTH / 8;  // loader row step
    constexpr int LM = BC / RSTEP;  // candidate rows per thread and chunk
    constexpr uint32_t DP = (uint32_t)NK * KC;
    __shared__ KnnSmem sm;
    __shared__ uint32_t item_slot;
    const uint32_t logical = take_item(P.item_ctr, &item_slot);
    if (logical >= P.n_items)
        return;
    const Item it = P.items[logical];
    const Job jb = P.jobs[it.job];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave / 4, wn = wave % 4;
    const int r = lane & 31, h = lane >> 5;
    const int col = wn * 32 + r; // this lane's query column
    const uint32_t q0 = __builtin_amdgcn_readfirstlane(jb.q_begin + it.q_off);
    const uint32_t qcnt = __builtin_amdgcn_readfirstlane(it.q_cnt);
    const uint32_t ncand = it.v_end - it.v_begin;
    const uint32_t Lp = P.lp;
    const uint32_t *__restrict__ XS = P.xs;

    if (tid < BQ) {
        sm.qn[tid] = (uint32_t)tid < qcnt ? P.xn[q0 + tid] : 0.0f;
        sm.tau[tid] = INFINITY;
        sm.lost[tid] = ord_key(INFINITY);
        sm.fill[tid] = 0u;
    }
    if (tid < 2)
        sm.need[tid] = 0u;
    // every buffer slot starts at +inf (thread t: slots 32(t%4) .. +31 of query t/4)
#pragma unroll
    for (int i4 = 0; i4 < 8; ++i4)
        *reinterpret_cast<float4 *>(&sm.bval[tid >> 2][32 * (tid & 3) + 4 * i4]) =
            make_float4(INFINITY, INFINITY, INFINITY, INFINITY);

    const int lr0 = tid >> 3;
    const int c4 = (tid & 7) * 4;
    [[maybe_unused]] __amdgpu_buffer_rsrc_t qres, xres;
    [[maybe_unused]] uint32_t xoff[LM];
    [[maybe_unused]] const uint32_t *xrow[LM];
    if constexpr (MODE == LOAD_BUF32)
        xres = __builtin_amdgcn_make_buffer_rsrc((void *)XS, (short)0, (int)P.x_bytes, 0x00020000);
    qres = __builtin_amdgcn_make_buffer_rsrc((void *)(XS + (size_t)q0 * DP), (short)0, (int)(qcnt * DP * 4u),
                                             0x00020000);
    // this lane's query column for the whole item: the high and low words of every
    // k-block (chunk kc, block kb: float4 column 2*kb + h of the chunk row, +4 for the
    // low words); columns past the item's queries load zeros
    bf16x8 qh[NK][2], ql[NK][2];
#pragma unroll
    for (int kc = 0; kc < NK; ++kc)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const uint32_t off = ((uint32_t)col * DP + (uint32_t)(kc * KC + (2 * kb + h) * 4)) * 4u;
            qh[kc][kb] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(qres, off, 0, 0));
            ql[kc][kb] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(qres, off + 64u, 0, 0));
        }
    auto set_xrows = [&](int slot) {
#pragma unroll
        for (int m = 0; m < LM; ++m) {
            uint32_t g = sm.rowid[slot][lr0 + RSTEP * m];
            g = (g == NONE) ? 0u : g; // padding rows load row 0 (their -|x|^2/2 is -inf)
            if constexpr (MODE == LOAD_BUF32)
                xoff[m] = (g * DP + (uint32_t)c4) * 4u;
            else
                xrow[m] = XS + (size_t)g * DP + c4;
        }
    };
    float4 rx[LM];
    auto load_chunk = [&](uint32_t kc) {
#pragma unroll
        for (int m = 0; m < LM; ++m) {
            if constexpr (MODE == LOAD_BUF32)
                rx[m] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xres, xoff[m], kc * 4u, 0));
            else
                rx[m] = __builtin_bit_cast(float4, *reinterpret_cast<const u32x4 *>(xrow[m] + kc));
        }
    };

    const uint32_t ntiles = (ncand + BC - 1) / BC;
    __syncthreads(); // qn and the buffer state
    const float qnv = sm.qn[col];
    const bool qok = (uint32_t)col < qcnt;
    // the query's own virtual candidate index (group jobs: candidates = the queries' group)
    const uint32_t self_v = (jb.flags & 1u) ? it.q_off + (uint32_t)col : NONE;

    // Refresh of every query's buffer (block-uniform call; four threads per query, one
    // quad of a wave, read and write its row, so no block barrier is needed; thread p
    // holds slots 32p .. 32p+31).  Slots at or past a buffer's fill hold +inf (set at the
    // item's start and rewritten by every compaction), so the live entries are the values
    // below T0 = min(tau, lost).  fin: the final one (at most KNN_OUT kept).  The
    // (Lp+1)-th live value is located on the scale t = (v - min) * sc, sc = 64 (1 - 2^-16)
    // / (top - min), monotone in v and below 64 for every live value: byte counters of
    // the 8 bins floor(t / 8) in one 64-bit register per thread, summed over the quad;
    // then those of the 8 sub-bins floor(t) of the bin that holds it; and, when that
    // sub-bin alone would take the buffer past its limit, those of its 8 parts floor(8t)
    // (8t is exactly 8 times t, so the three levels nest).  The buffer keeps the parts up
    // to the one that holds the (Lp+1)-th value (only those below it when that would be
    // more than the limit) and tau drops to the smallest live value left out.
    auto refresh = [&](bool fin) __attribute__((always_inline)) {
        const int q = tid >> 2, p = tid & 3;
        const uint32_t f = min(sm.fill[q], (uint32_t)KNN_CAP);
        const float tq = sm.tau[q];
        const float T0 = fminf(tq, ord_val(sm.lost[q]));
        float v[32];
        uint32_t ip[16];
#pragma unroll
        for (int i4 = 0; i4 < 8; ++i4) {
            const float4 x = *reinterpret_cast<const float4 *>(&sm.bval[q][32 * p + 4 * i4]);
            v[4 * i4] = x.x;
            v[4 * i4 + 1] = x.y;
            v[4 * i4 + 2] = x.z;
            v[4 * i4 + 3] = x.w;
        }
#pragma unroll
        for (int i8 = 0; i8 < 4; ++i8) {
            const uint4 w = *reinterpret_cast<const uint4 *>(&sm.bidx[q][32 * p + 8 * i8]);
            ip[4 * i8] = w.x;
            ip[4 * i8 + 1] = w.y;
            ip[4 * i8 + 2] = w.z;
            ip[4 * i8 + 3] = w.w;
        }
        // live entries: below T0 (the others become +inf)
        uint32_t n_own = 0u;
        float mn = INFINITY;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            v[i] = v[i] < T0 ? v[i] : INFINITY;
            n_own += v[i] < INFINITY ? 1u : 0u;
            mn = fminf(mn, v[i]);
        }
        const uint32_t n_live = quad_sum(n_own);
        mn = quad_min(mn);
        // the window's top: T0 bounds every live entry once it is finite (the first
        // refresh of an item takes the largest live entry)
        float mx = T0;
        if (!(T0 < INFINITY)) {
            mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 32; ++i)
                mx = (v[i] < INFINITY && v[i] > mx) ? v[i] : mx;
            mx = quad_max(mx);
        }
        const uint32_t target = Lp + 1u;
        const uint32_t limit = fin ? KNN_OUT : KNN_KEEP;
        const bool hist = fin ? n_live > KNN_OUT : n_live > target;
        // a row is rewritten when it is cut, holds dead slots below its fill, or a dropped
        // value lowers its threshold; a wave with none of these leaves its rows as they are
        if (__ballot(hist || n_live < f || T0 < tq) == 0)
            return;
        // keys floor(t) (dead slots: 127), four bytes a word
        const float sc = mx > mn ? (64.0f * (1.0f - 0x1p-16f)) / (mx - mn) : 0.0f;
        uint32_t kw[8];
#pragma unroll
        for (int w = 0; w < 8; ++w)
            kw[w] = 0u;
#pragma unroll
        for (int i = 0; i < 32; ++i)
            kw[i >> 2] |= (uint32_t)fminf((v[i] - mn) * sc, 127.0f) << ((i & 3) << 3);
        auto key = [&](int i) { return (kw[i >> 2] >> ((i & 3) << 3)) & 0xFFu; };
        // the first of 8 counts (bytes of w0, w1) whose running sum from `below` reaches
        // the target: its index, the running sum before it and the count itself
        auto find_bin = [&](uint32_t w0, uint32_t w1, uint32_t below, uint32_t &bin, uint32_t &lt,
                            uint32_t &cnt) __attribute__((always_inline)) {
            uint32_t cum = below;
            bool found = false;
            bin = 0u;
            lt = below;
            cnt = 0u;
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const uint32_t c = ((b < 4 ? w0 : w1) >> ((b & 3) << 3)) & 0xFFu;
                const bool hit = !found && cum + c >= target;
                bin = hit ? (uint32_t)b : bin;
                lt = hit ? cum : lt;
                cnt = hit ? c : cnt;
                found = found || hit;
                cum += c;
            }
        };
        // kept: the keys below kkey (every live entry without a cut: live keys are <= 63);
        // kkey: past the part that holds the target-th value, or that part itself when
        // keeping it would be more than the limit
        uint32_t kkey = 127u;
        bool deep = false; // the target's sub-bin is crowded: the third level decides
        uint32_t base3 = 0u, c_lt2 = 0u, c_le = 0u;
        if (hist) {
            // byte b of the 64-bit counter: entries with floor(t / 8) = b (at most 128: no
            // carries); bin 7 also took the dead slots
            uint64_t c8 = 0u;
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                c8 += (uint64_t)1u << (key(i) & 0x38u);
                asm("" : "+v"(c8)); // one running sum (no tree of 64-bit partial sums)
            }
            const uint32_t cw0 = quad_sum((uint32_t)c8);
            const uint32_t cw1 = quad_sum((uint32_t)(c8 >> 32)) - ((128u - n_live) << 24);
            uint32_t b1, c_lt, c_in;
            find_bin(cw0, cw1, 0u, b1, c_lt, c_in);
            // sub-bins floor(t) - 8 b1: entries below the bin count in sub-bin 0, those above
            // it (and the dead slots) in sub-bin 7, taken out after the sums
            uint64_t d8 = 0u;
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                const int sb = min(max((int)key(i) - (int)(8u * b1), 0), 7);
                d8 += (uint64_t)1u << ((uint32_t)sb << 3);
                asm("" : "+v"(d8));
            }
            const uint32_t dw0 = quad_sum((uint32_t)d8) - c_lt;
            const uint32_t dw1 = quad_sum((uint32_t)(d8 >> 32)) - ((128u - c_lt - c_in) << 24);
            uint32_t b2, c_in2;
            find_bin(dw0, dw1, c_lt, b2, c_lt2, c_in2);
            c_le = c_lt2 + c_in2;
            kkey = 8u * b1 + b2 + (c_le <= limit ? 1u : 0u);
            deep = c_le > limit;
            base3 = 8u * (8u * b1 + b2);
        }
        if (__ballot(deep)) {
            if (deep) {
                // the 8 parts floor(8t) - base3 of the crowded sub-bin (8t is exactly 8 times
                // t, so floor(8t) / 8 = floor(t)); the keys become 0 below it, 1 + the part
                // inside it and 9 above it (dead slots stay 127)
                const float sc8 = sc * 8.0f;
                uint64_t e8 = 0u;
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    const int r3 = (int)(uint32_t)fminf((v[i] - mn) * sc8, 1023.0f) - (int)base3;
                    e8 += (uint64_t)1u << ((uint32_t)min(max(r3, 0), 7) << 3);
                    asm("" : "+v"(e8));
                    const uint32_t k3 = key(i) == 127u ? 127u : (uint32_t)min(max(r3 + 1, 0), 9);
                    const int sh = (i & 3) << 3;
                    kw[i >> 2] = (kw[i >> 2] & ~(0xFFu << sh)) | (k3 << sh);
                }
                const uint32_t ew0 = quad_sum((uint32_t)e8) - c_lt2;
                const uint32_t ew1 = quad_sum((uint32_t)(e8 >> 32)) - ((128u - c_le) << 24);
                uint32_t b3, c_lt3, c_in3;
                find_bin(ew0, ew1, c_lt2, b3, c_lt3, c_in3);
                kkey = 1u + b3 + (c_lt3 + c_in3 <= limit ? 1u : 0u);
            }
        }
        // compaction to the front of the row (the entries are all in registers); tau
        // drops to the smallest live value left out (every kept value is below it)
        uint32_t nk_ = 0u;
        float tmin = INFINITY;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const bool kp = key(i) < kkey;
            nk_ += kp ? 1u : 0u;
            tmin = kp ? tmin : fminf(tmin, v[i]);
        }
        const float tnew = hist ? fminf(T0, quad_min(tmin)) : T0;
        const uint32_t kincl = quad_incl(nk_, p);
        uint32_t pos = kincl - nk_;
        // the row's slots become +inf, then the kept entries go to its front (the quad's
        // LDS accesses execute in program order)
#pragma unroll
        for (int i4 = 0; i4 < 8; ++i4)
            *reinterpret_cast<float4 *>(&sm.bval[q][32 * p + 4 * i4]) =
                make_float4(INFINITY, INFINITY, INFINITY, INFINITY);
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const bool kp = key(i) < kkey;
            if (kp) {
                sm.bval[q][pos] = v[i];
                sm.bidx[q][pos] = (uint16_t)(ip[i >> 1] >> ((i & 1) << 4));
            }
            pos += kp ? 1u : 0u;
        }
        if (p == 3) {
            sm.fill[q] = kincl;
            sm.tau[q] = tnew;
            sm.lost[q] = ord_key(INFINITY);
        }
    };

    RowCursor cur;
    finish_rowids(sm, 0, start_rowids(sm, 0, cur, P, jb, it.v_begin, it.v_end, tid), tid);
    __syncthreads();
    set_xrows(0);
    load_chunk(0);
    floatx16 acc[2];
    int slot = 0;
    uint32_t s = 0; // steps done
    for (uint32_t tile = 0; tile < ntiles; ++tile) {
        const int next_slot = slot == 2 ? 0 : slot + 1;
        const bool more = tile + 1 < ntiles;
        float pend_nx = INFINITY;
        // the tile's chunks: panels double-buffered in LDS, the next chunk (also the next
        // tile's first) prefetched into registers, the next tile's row ids built in ring
        // slot (tile+1)%3 meanwhile
#pragma unroll
        for (int kc = 0; kc < NK; ++kc) {
            const int buf = (int)((s + (uint32_t)kc) & 1u);
#pragma unroll
            for (int m = 0; m < LM; ++m)
                sm.xs[buf][lr0 + RSTEP * m][c4 >> 2] = rx[m];
            if (NK == 1 && more)
                finish_rowids(sm, next_slot,
                              start_rowids(sm, next_slot, cur, P, jb, it.v_begin + (tile + 1) * BC, it.v_end, tid), tid);
            if (NK > 1 && kc == 1 && more)
                finish_rowids(sm, next_slot, pend_nx, tid);
            __syncthreads();
            if (kc + 1 < NK) {
                load_chunk((uint32_t)(kc + 1) * KC);
            } else if (more) {
                set_xrows(next_slot);
                load_chunk(0);
            }
            // three bf16 passes per 16-dimension block (hi*hi, hi*lo, lo*hi); the tile's
            // first MFMA of each accumulator takes C = 0
            __builtin_amdgcn_s_setprio(1);
            const floatx16 zero = {};
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int ch = 2 * kb + h;
                bf16x8 ah[2], al[2];
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    ah[mb] = __builtin_bit_cast(bf16x8, sm.xs[buf][wm * 64 + 32 * mb + r][ch]);
                    al[mb] = __builtin_bit_cast(bf16x8, sm.xs[buf][wm * 64 + 32 * mb + r][ch + 4]);
                }
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
                    acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[mb], qh[kc][kb],
                                                                      (kc == 0 && kb == 0) ? zero : acc[mb], 0, 0, 0);
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
                    acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[mb], ql[kc][kb], acc[mb], 0, 0, 0);
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
                    acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[mb], qh[kc][kb], acc[mb], 0, 0, 0);
            }
            __builtin_amdgcn_s_setprio(0);
            if (NK > 1 && kc == 0 && more)
                pend_nx = start_rowids(sm, next_slot, cur, P, jb, it.v_begin + (tile + 1) * BC, it.v_end, tid);
        }
        s += (uint32_t)NK;
        // -|x|^2/2 of the candidate row by one more MFMA (three exact bf16 terms against
        // ones): acc = -s, s = |x|^2/2 - <x,q>  (padding rows: -inf)
        {
            const bf16x8 bone = __builtin_bit_cast(
                bf16x8, make_uint4(h == 0 ? 0x3F803F80u : 0u, h == 0 ? 0x00003F80u : 0u, 0u, 0u));
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
                const uint2 w = sm.nhx[slot][wm * 64 + 32 * mb + r];
                const bf16x8 abias = __builtin_bit_cast(bf16x8, make_uint4(h == 0 ? w.x : 0u, h == 0 ? w.y : 0u, 0u, 0u));
                acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(abias, bone, acc[mb], 0, 0, 0);
            }
        }
        // the lane's values below tau into its query's buffer.  Bit 31-j of the masks is
        // value j (row tile_row(wm, h, j)); rows past the split and the query itself are
        // never candidates.
        {
            const uint32_t base_row = (uint32_t)(wm * 64 + 4 * h);
            const uint32_t tile_v = tile * BC;
            const int dv = (int)min(ncand - tile_v, (uint32_t)BC) - (int)base_row;
            const uint32_t nv = dv <= 0 ? 0u : min(32u, 4u * ((uint32_t)dv >> 3) + min((uint32_t)dv & 7u, 4u));
            uint32_t valid = nv == 0u ? 0u : (0xFFFFFFFFu << (32u - nv));
            const int o = (int)(self_v - it.v_begin - tile_v) - (int)base_row;
            const uint32_t sj = self_v != NONE ? lane_index_of(o) : 32u;
            valid &= sj < 32u ? ~(0x80000000u >> sj) : 0xFFFFFFFFu;
            valid = qok ? valid : 0u;
            // s < c  <=>  the sign bit of -c - acc  (c = +inf: every finite value); tau as
            // the latest refresh left it (visible after this tile's step barriers)
            const float ncth = -s_bound(sm.tau[col], qnv);
            uint32_t mask = 0u;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    mask = (mask << 1) | (__float_as_uint(ncth - acc[mb][i]) >> 31);
            mask &= valid;
            if (__ballot(mask != 0u)) {
                const uint32_t cnt = (uint32_t)__popc(mask);
                const uint32_t base = cnt ? atomicAdd(&sm.fill[col], cnt) : 0u;
                if (base + cnt > (tile < 2u ? KNN_TRIG : KNN_TRIG_LATE))
                    sm.need[tile & 1u] = 1u;
                float *const vrow = &sm.bval[col][0];
                uint16_t *const irow = &sm.bidx[col][0];
                const uint32_t vbase = tile_v + base_row;
                if (__ballot(base + cnt > (uint32_t)KNN_CAP) == 0) {
#pragma unroll
                    for (int j = 0; j < 32; ++j) {
                        if ((int)(mask << j) < 0) {
                            const uint32_t pos = base + (uint32_t)__popc(mask & ~(0xFFFFFFFFu >> j));
                            vrow[pos] = __builtin_fmaf(-2.0f, acc[j >> 4][j & 15], qnv);
                            irow[pos] = (uint16_t)(vbase + (((uint32_t)j & 28u) << 1) + ((uint32_t)j & 3u));
                        }
                    }
                } else {
                    // a full buffer: the values past its capacity are dropped, the
                    // smallest of them caps tau at the next refresh
                    uint32_t lk = ord_key(INFINITY);
#pragma unroll
                    for (int j = 0; j < 32; ++j) {
                        if ((int)(mask << j) < 0) {
                            const uint32_t pos = base + (uint32_t)__popc(mask & ~(0xFFFFFFFFu >> j));
                            const float a = __builtin_fmaf(-2.0f, acc[j >> 4][j & 15], qnv);
                            if (pos < (uint32_t)KNN_CAP) {
                                vrow[pos] = a;
                                irow[pos] = (uint16_t)(vbase + (((uint32_t)j & 28u) << 1) + ((uint32_t)j & 3u));
                            } else {
                                lk = min(lk, ord_key(a));
                            }
                        }
                    }
                    if (lk != ord_key(INFINITY))
                        atomicMin(&sm.lost[col], lk);
                }
            }
        }
        __syncthreads(); // appends done
        // the next tile's flag is cleared here: it is set only after the next tile's step
        // barriers, and read only after its append barrier
        const bool do_refresh = sm.need[tile & 1u] != 0u || !more;
        if (tid == 0)
            sm.need[(tile + 1u) & 1u] = 0u;
        if (do_refresh)
            refresh(!more);
        slot = next_slot;
    }

    // per query (four threads): bitonic sort of its <= KNN_OUT entries by value over
    // elements e = 16p + i, then the partial row and its bound
    __syncthreads();
    {
        const int q = tid >> 2, p = tid & 3;
        const uint32_t f = sm.fill[q];
        float d[16];
        uint32_t id[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t e = (uint32_t)(16 * p + i);
            const bool in = e < f;
            d[i] = in ? sm.bval[q][e] : INFINITY;
            id[i] = in ? (uint32_t)sm.bidx[q][e] : NONE;
        }
#pragma unroll
        for (int k = 2; k <= 64; k <<= 1)
#pragma unroll
            for (int j = k >> 1; j > 0; j >>= 1) {
                if (j >= 16) {
                    // partner element e ^ j: same slot of quad lane p ^ (j/16)
                    const bool asc = ((16 * p) & k) == 0;
                    const bool lower = ((16 * p) & j) == 0;
                    const bool keep_min = lower == asc;
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const float pd = j == 16 ? quad_xor<1>(d[i]) : quad_xor<2>(d[i]);
                        const uint32_t pi = j == 16 ? quad_xor<1>(id[i]) : quad_xor<2>(id[i]);
                        const bool take = keep_min ? pd < d[i] : pd > d[i];
                        d[i] = take ? pd : d[i];
                        id[i] = take ? pi : id[i];
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int l = i ^ j;
                        if (l > i) {
                            // ascending pairs put the smaller value first
                            const bool asc = k < 16 ? (i & k) == 0 : ((16 * p) & k) == 0;
                            const bool sw = asc ? d[l] < d[i] : d[i] < d[l];
                            const float di = d[i], dl = d[l];
                            const uint32_t ii = id[i], il = id[l];
                            d[i] = sw ? dl : di;
                            d[l] = sw ? di : dl;
                            id[i] = sw ? il : ii;
                            id[l] = sw ? ii : il;
                        }
                    }
                }
            }
        float next = INFINITY; // the (Lp+1)-th entry (Lp < KNN_OUT)
#pragma unroll
        for (int i = 0; i < 16; ++i)
            next = (uint32_t)(16 * p + i) == Lp ? d[i] : next;
        next = quad_min(next);
        if ((uint32_t)q < qcnt) {
            const size_t prow = (size_t)jb.part_base + (size_t)it.split * jb.q_count + it.q_off + (uint32_t)q;
            const uint32_t id0 = P.seg_start[jb.seg_begin] + it.v_begin; // group jobs: one segment
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t e = (uint32_t)(16 * p + i);
                if (e < Lp) {
                    P.part_ids[prow * Lp + e] = d[i] < INFINITY ? id0 + id[i] : NONE;
                    P.part_dist[prow * Lp + e] = d[i];
                }
            }
            if (p == 0)
                P.part_bound[prow] = fminf(sm.tau[q], next);
        }
    }
}

// ---------------------------------------------------------------------------
// merge + certification
// ---------------------------------------------------------------------------
struct MergeParams {
    const float *X;
    const float *xn;
    uint32_t d;
    const Job *jobs;
    const MergeItem *mitems; // q_cnt <= MERGE_ROWS: one wave per result row
    const uint32_t *part_ids;
    const float *part_dist;
    const float *part_bound;
    uint32_t lp;
    uint32_t k;
    double eps_coef, shrink, rmax;
    uint32_t *out_ids;
    float *out_dist;
    int32_t *out_size;
    uint32_t *flag_count;
    uint2 *flagged;
    uint32_t n_mitems;   // items of this launch
    uint32_t xcd_spread; // 1: consecutive items to one XCD (see ung_merge_kernel)
    uint32_t qlds;       // 1: the launch gave MERGE_ROWS * d floats of LDS for query rows
};

// The MI355X's XCDs; the dispatcher hands a launch's workgroups to them round-robin.
constexpr uint32_t NUM_XCD = 8;

// One wave per result row: k-way merge of the row's S partial rows (S <= 64, each
// sorted by approximate distance) to its Lp best approximate candidates, exact
// re-score of those in the reference's summation order, (dist, id) ranking, and the
// certificate  T_k < lower bound of every candidate left out.  PAIR: each eight-lane
// group re-scores two candidates per pass (long rows of large d: group kNN lists at
// d >= 256, 10 % faster there; more registers, which cost the short cross rows and
// d = 128 more than the shared loads gain).
template <bool PAIR>
__global__ __launch_bounds__(64 * MERGE_ROWS) void ung_merge_kernel(MergeParams M)
{
    __shared__ uint32_t mrank[MERGE_ROWS][128]; // a wave's candidates in rank order
    __shared__ float mrankd[MERGE_ROWS][128];   // and their approximate distances
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    // group kNN rows of large d (all re-scored against their own group's vectors):
    // consecutive items run on one XCD, so a group's vectors are read into one L2 instead
    // of eight (cfg4, d = 768: 11.3 -> 8.5 ms; the cross merge ran slower so)
    uint32_t li = blockIdx.x;
    if (M.xcd_spread) {
        const uint32_t per = (M.n_mitems + NUM_XCD - 1u) / NUM_XCD;
        li = (blockIdx.x % NUM_XCD) * per + blockIdx.x / NUM_XCD;
        if (li >= M.n_mitems)
            return; // whole block; no block barrier in this kernel
    }
    const MergeItem mi = M.mitems[li];
    if ((uint32_t)w >= mi.q_cnt)
        return; // whole wave; no block barrier below
    const Job jb = M.jobs[mi.job];
    const uint32_t ql = mi.q_off + (uint32_t)w;
    const uint32_t q = jb.q_begin + ql;
    const uint32_t S = jb.n_split, Lp = M.lp, k = M.k;

    // slot h of lane t holds the (64h + t)-th smallest approximate candidate (Lp <= 128)
    // and its approximate distance
    uint32_t ci[2] = {NONE, NONE};
    float ca[2] = {INFINITY, INFINITY};
    float B; // approximate-space bound of every candidate left out
    if (S == 1) {
        // one split: its partial row is already the approximate top-Lp
        const size_t prow = (size_t)jb.part_base + ql;
#pragma unroll
        for (int h = 0; h < 2; ++h)
            if ((uint32_t)(64 * h + lane) < Lp) {
                ci[h] = M.part_ids[prow * Lp + 64 * h + lane];
                ca[h] = M.part_dist[prow * Lp + 64 * h + lane];
            }
        B = M.part_bound[prow];
    } else if (S * Lp <= 64u) {
        // all S*Lp entries in the wave (one per lane; splits are disjoint, so the ids of the
        // entries are distinct, NONE aside): a wave sort by (dist, id) puts the entry of
        // rank t in lane t, the one of rank Lp is the first left out
        const uint32_t n = S * Lp;
        float ed = INFINITY;
        uint32_t eid = NONE;
        if ((uint32_t)lane < n) {
            const uint32_t sp = (uint32_t)lane / Lp, pos = (uint32_t)lane - sp * Lp;
            const size_t prow = (size_t)jb.part_base + (size_t)sp * jb.q_count + ql;
            ed = M.part_dist[prow * Lp + pos];
            eid = M.part_ids[prow * Lp + pos];
        }
        float bnd = (uint32_t)lane < S ? M.part_bound[(size_t)jb.part_base + (size_t)lane * jb.q_count + ql] : INFINITY;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
            bnd = fminf(bnd, __shfl_xor(bnd, off));
        wave_sort64(ed, eid, lane);
        if ((uint32_t)lane < Lp) {
            ci[0] = eid;
            ca[0] = ed;
        }
        const float a_next = __shfl(ed, (int)Lp); // Lp < 64 here
        B = fminf(bnd, a_next);
    } else if (S * Lp <= 128u) {
        // all S*Lp entries in the wave (two per lane): each entry's rank under (dist, id,
        // entry index) by comparing with every other one, no dependent loads; the entry of
        // rank t goes to lane t % 64, slot t / 64, the one of rank Lp is the first left out
        const uint32_t n = S * Lp;
        float ed[2];
        uint32_t eid[2];
        float bnd = INFINITY;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t e = 64u * (uint32_t)h + (uint32_t)lane;
            ed[h] = INFINITY;
            eid[h] = NONE;
            if (e < n) {
                const uint32_t sp = e / Lp, pos = e - sp * Lp;
                const size_t prow = (size_t)jb.part_base + (size_t)sp * jb.q_count + ql;
                ed[h] = M.part_dist[prow * Lp + pos];
                eid[h] = M.part_ids[prow * Lp + pos];
            }
        }
        if ((uint32_t)lane < S)
            bnd = M.part_bound[(size_t)jb.part_base + (size_t)lane * jb.q_count + ql];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
            bnd = fminf(bnd, __shfl_xor(bnd, off));
        uint32_t rk[2] = {0u, 0u};
        if (n <= 64u) {
            for (uint32_t f = 0; f < n; ++f) {
                const float df = __shfl(ed[0], (int)f);
                const uint32_t idf = __shfl(eid[0], (int)f);
                rk[0] += ((df < ed[0]) | ((df == ed[0]) & ((idf < eid[0]) | ((idf == eid[0]) & (f < (uint32_t)lane))))) ? 1u : 0u;
            }
        } else {
            for (uint32_t f = 0; f < n; ++f) {
                const int src = (int)(f & 63u);
                const float df = f < 64u ? __shfl(ed[0], src) : __shfl(ed[1], src);
                const uint32_t idf = f < 64u ? __shfl(eid[0], src) : __shfl(eid[1], src);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t me = 64u * (uint32_t)h + (uint32_t)lane;
                    rk[h] += ((df < ed[h]) | ((df == ed[h]) & ((idf < eid[h]) | ((idf == eid[h]) & (f < me))))) ? 1u : 0u;
                }
            }
        }
        // scatter through this wave's LDS row: every rank below n is held by one entry
        float a_next = INFINITY;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const bool in = 64u * (uint32_t)h + (uint32_t)lane < n;
            if (in && rk[h] < Lp) {
                mrank[w][rk[h]] = eid[h];
                mrankd[w][rk[h]] = ed[h];
            }
            if (in && rk[h] == Lp)
                a_next = ed[h];
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int h = 0; h < 2; ++h)
            if (64u * (uint32_t)h + (uint32_t)lane < Lp) {
                ci[h] = mrank[w][64 * h + lane];
                ca[h] = mrankd[w][64 * h + lane];
            }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
            a_next = fminf(a_next, __shfl_xor(a_next, off));
        B = fminf(bnd, a_next);
    } else {
        size_t prow = 0;
        uint32_t pos = 0;
        float hd = INFINITY, bnd = INFINITY;
        uint32_t hi = NONE;
        if ((uint32_t)lane < S) {
            prow = (size_t)jb.part_base + (size_t)lane * jb.q_count + ql;
            bnd = M.part_bound[prow];
            hd = M.part_dist[prow * Lp];
            hi = M.part_ids[prow * Lp];
        }
        float bmin = bnd;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
            bmin = fminf(bmin, __shfl_xor(bmin, off));
        float a_next = INFINITY;
        for (uint32_t t = 0; t <= Lp; ++t) {
            float bd = hd;
            uint32_t bi = hi;
            wave_argmin(bd, bi);
            if (bi == NONE)
                break; // every head is exhausted (uniform)
            if (t == Lp) {
                a_next = bd;
                break;
            }
            if ((uint32_t)lane == (t & 63u)) {
                if (t < 64) {
                    ci[0] = bi;
                    ca[0] = bd;
                } else {
                    ci[1] = bi;
                    ca[1] = bd;
                }
            }
            if (hi == bi) {
                ++pos;
                if (pos < Lp) {
                    hd = M.part_dist[prow * Lp + pos];
                    hi = M.part_ids[prow * Lp + pos];
                } else {
                    hd = INFINITY;
                    hi = NONE;
                }
            }
        }
        B = fminf(bmin, a_next);
    }

    // Only candidates that can be among the k best are re-scored: the k best by
    // approximate distance all have exact distances <= U = upper_bound_ea(a_{k-1}), so
    // the k-th exact distance T <= U, and a candidate whose lower bound exceeds U has an
    // exact distance > T (it is neither a result nor needed by the certificate).  The
    // candidates are in ascending approximate order, so the re-scored ones are a prefix.
    const float xq = M.xn[q];
    const double ea = bound_ea(xq, M.eps_coef, M.rmax);
    uint32_t m_need = Lp;
    if (k <= Lp) {
        const int src = (int)((k - 1u) & 63u);
        const float ak = k - 1u < 64u ? __shfl(ca[0], src) : __shfl(ca[1], src);
        const float U = upper_bound_ea(ak, ea, M.shrink);
        if (U < INFINITY) {
            uint32_t cnt_need = 0;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (64u * (uint32_t)h < Lp) {
                    const bool in = (uint32_t)(64 * h + lane) < Lp;
                    const bool need = in && !(lower_bound_ea(ca[h], ea, M.shrink) > U);
                    cnt_need += (uint32_t)__popcll(__ballot(need));
                }
            }
            m_need = cnt_need;
        }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
        if ((uint32_t)(64 * h + lane) >= m_need)
            ci[h] = NONE; // left out (exact distance > T): not a result

    // exact re-score: 8 lanes per candidate (one per accumulator of the reference's
    // summation), 8 candidates per pass (PAIR: 16); candidate t's value goes to lane
    // t % 64, slot t / 64.  Rows of more than two passes read the query row from a copy
    // in this wave's LDS slice when the launch gave one (group kNN merges, d <=
    // MERGE_QLDS), so that every pass loads only the candidates' rows from memory (~33
    // candidates: cfg4 7.8 -> 6.2 ms, cfg2 0.71 -> 0.67 ms).  The arithmetic is the same
    // either way.
    float ex[2] = {INFINITY, INFINITY};
    auto rescore = [&](const float *qv) __attribute__((always_inline)) {
        if constexpr (PAIR) {
            // group g scores candidates 16p + g and 16p + 8 + g (t < 128: Lp <= 128); lane L
            // takes candidate 8 (2p + e) + L % 8 from group L % 8, e = 0, 1
            const int g = lane >> 3, sub = lane & 7;
            const uint32_t npass = (m_need + 15u) / 16u;
            for (uint32_t p = 0; p < npass; ++p) {
                const uint32_t t0 = 16u * p + (uint32_t)g, t1 = t0 + 8u;
                const uint32_t c0 = t0 < 64u ? __shfl(ci[0], (int)(t0 & 63u)) : __shfl(ci[1], (int)(t0 & 63u));
                const uint32_t c1 = t1 < 64u ? __shfl(ci[0], (int)(t1 & 63u)) : __shfl(ci[1], (int)(t1 & 63u));
                const bool ok0 = t0 < Lp && c0 != NONE, ok1 = t1 < Lp && c1 != NONE;
                float v0, v1 = INFINITY;
                if (16u * p + 8u < m_need) // wave-uniform: the pass's second half holds candidates
                    l2_ref_8lane2(qv, M.X + (size_t)(ok0 ? c0 : q) * M.d, M.X + (size_t)(ok1 ? c1 : q) * M.d, M.d,
                                  sub, v0, v1);
                else
                    v0 = l2_ref_8lane(qv, M.X + (size_t)(ok0 ? c0 : q) * M.d, M.d, sub);
                const float got0 = __shfl(v0, 8 * (lane & 7)), got1 = __shfl(v1, 8 * (lane & 7));
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const uint32_t pp = 2u * p + (uint32_t)e; // candidates 8pp .. 8pp + 7
                    if ((uint32_t)g == (pp & 7u)) {
                        const float got = e == 0 ? got0 : got1;
                        if (pp < 8u)
                            ex[0] = ci[0] != NONE ? got : INFINITY;
                        else
                            ex[1] = ci[1] != NONE ? got : INFINITY;
                    }
                }
            }
        } else {
            const int g = lane >> 3, sub = lane & 7;
            const uint32_t npass = (m_need + 7u) / 8u;
            for (uint32_t p = 0; p < npass; ++p) {
                const uint32_t t = 8u * p + (uint32_t)g;
                const int src = (int)(t & 63u);
                const uint32_t c = t < 64u ? __shfl(ci[0], src) : __shfl(ci[1], src);
                const bool ok = t < Lp && c != NONE;
                const float v = l2_ref_8lane(qv, M.X + (size_t)(ok ? c : q) * M.d, M.d, sub);
                const float got = __shfl(v, 8 * (lane & 7)); // candidate 8p + (lane % 8)
                const uint32_t pl = p & 7u;
                if ((uint32_t)g == pl) {
                    if (p < 8u)
                        ex[0] = ci[0] != NONE ? got : INFINITY;
                    else
                        ex[1] = ci[1] != NONE ? got : INFINITY;
                }
            }
        }
    };
    if (M.qlds && m_need > 16u) { // (m_need is wave-uniform)
        extern __shared__ float mq[]; // [MERGE_ROWS][d], sized by the launch
        float *const qs = mq + (size_t)w * M.d;
        const float *const qg = M.X + (size_t)q * M.d;
        for (uint32_t i = (uint32_t)lane; i < M.d; i += 64u)
            qs[i] = qg[i];
        __builtin_amdgcn_wave_barrier(); // (a wave's LDS accesses execute in order)
        rescore(qs);
    } else {
        rescore(M.X + (size_t)q * M.d);
    }
    const size_t orow = (size_t)jb.out_row + ql;
    const float Bx = lower_bound_ea(B, ea, M.shrink);
    if (m_need <= 64u && m_need > 16u) {
        // one candidate per lane: a wave sort by (exact, id) puts rank t in lane t (the
        // re-scored ids are distinct; left-out lanes hold (+inf, NONE) and sort last).
        // Its 21 exchange stages cost less than the rank loop below from about 16
        // candidates on.
        const bool real = (uint32_t)lane < m_need && ci[0] != NONE;
        float d = real ? ex[0] : INFINITY;
        uint32_t id = real ? ci[0] : NONE;
        wave_sort64(d, id, lane);
        const float T = __shfl(d, (int)(k - 1u)); // k <= 64
        const uint32_t cnt = (uint32_t)__popcll(__ballot((uint32_t)lane < k && id != NONE));
        const bool certified = (cnt < k) ? !(B < INFINITY) : (T < Bx);
        if (!certified) {
            if (lane == 0) {
                const uint32_t slot = atomicAdd(M.flag_count, 1u);
                M.flagged[slot] = make_uint2(mi.job, ql);
            }
            return;
        }
        if ((uint32_t)lane < k) {
            M.out_ids[orow * k + lane] = id != NONE ? id - jb.id_base : NONE;
            if (M.out_dist)
                M.out_dist[orow * k + lane] = id != NONE ? d : INFINITY;
        }
        if (lane == 0 && M.out_size)
            M.out_size[orow] = (int32_t)cnt;
        return;
    }
    // rank under (exact, id, position); a left-out candidate (exact distance > T) ranks
    // after every re-scored one and takes no place in the row
    uint32_t rank[2] = {0u, 0u};
    for (uint32_t f = 0; f < m_need; ++f) {
        const int src = (int)(f & 63u);
        const float df = f < 64 ? __shfl(ex[0], src) : __shfl(ex[1], src);
        const uint32_t idf = f < 64 ? __shfl(ci[0], src) : __shfl(ci[1], src);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t me = 64u * (uint32_t)h + (uint32_t)lane;
            rank[h] += ((df < ex[h]) | ((df == ex[h]) & ((idf < ci[h]) | ((idf == ci[h]) & (f < me))))) ? 1u : 0u;
        }
    }
    bool mine[2], real[2];
    float T = INFINITY;
    uint32_t cnt = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        mine[h] = (uint32_t)(64 * h + lane) < m_need;
        real[h] = mine[h] && ci[h] != NONE;
        T = (mine[h] && rank[h] == k - 1) ? ex[h] : T;
        cnt += (uint32_t)__popcll(__ballot(real[h] && rank[h] < k));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        T = fminf(T, __shfl_xor(T, off));
    const bool certified = (cnt < k) ? !(B < INFINITY) : (T < Bx);
    if (!certified) {
        if (lane == 0) {
            const uint32_t slot = atomicAdd(M.flag_count, 1u);
            M.flagged[slot] = make_uint2(mi.job, ql);
        }
        return;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
        if (mine[h] && rank[h] < k) {
            M.out_ids[orow * k + rank[h]] = real[h] ? ci[h] - jb.id_base : NONE;
            if (M.out_dist)
                M.out_dist[orow * k + rank[h]] = real[h] ? ex[h] : INFINITY;
        }
    if (lane == 0 && M.out_size)
        M.out_size[orow] = (int32_t)cnt;
}

// ---------------------------------------------------------------------------
// exact fallback: every flagged row's union is cut into `splits` ranges; one wave scans
// one (row, range) item (persistent over the items) and keeps its k best by (dist, id).
// With one range the wave writes the result row; otherwise it writes a partial row and
// ung_fallback_merge_kernel merges a row's ranges.
// ---------------------------------------------------------------------------
struct FallbackParams {
    const float *X;
    uint32_t d;
    uint32_t k;
    const Job *jobs;
    const uint32_t *seg_start;
    const uint32_t *seg_vend;
    const uint32_t *flag_count;
    const uint2 *flagged;
    uint32_t splits;     // ranges per flagged row (at least 1)
    uint32_t *part_ids;  // [flagged x splits x k] global ids (splits > 1)
    float *part_dist;
    uint32_t *out_ids;
    float *out_dist;
    int32_t *out_size;
};

__global__ __launch_bounds__(64) void ung_fallback_kernel(FallbackParams F)
{
    __shared__ float sd[64][65];
    __shared__ uint32_t si[64][65];
    const int lane = threadIdx.x;
    const uint32_t S = F.splits;
    const uint64_t total = (uint64_t)*F.flag_count * S;
    const uint32_t k = F.k;
    for (uint64_t w = blockIdx.x; w < total; w += gridDim.x) {
        const uint32_t f = (uint32_t)(w / S);
        const uint32_t sp = (uint32_t)(w - (uint64_t)f * S);
        const uint2 fl = F.flagged[f];
        const Job jb = F.jobs[fl.x];
        const uint32_t q = jb.q_begin + fl.y;
        const bool excl = (jb.flags & 1u) != 0;
        const float *qv = F.X + (size_t)q * F.d;
        const uint32_t v0 = (uint32_t)((uint64_t)jb.n_cand * sp / S);
        const uint32_t v1 = (uint32_t)((uint64_t)jb.n_cand * (sp + 1) / S);
        int32_t size = 0;
        for (uint32_t v = v0 + (uint32_t)lane; v < v1; v += 64) {
            const uint32_t g = cand_id(F.seg_start, F.seg_vend, jb.seg_begin, jb.seg_count, v);
            if (excl && g == q)
                continue;
            const float dist = l2_ref_lane(qv, F.X + (size_t)g * F.d, F.d);
            // bounded sorted insert (search_queue.cpp:26-53 order; ids are unique here)
            if (size == (int32_t)k && !cand_less(dist, g, sd[lane][size - 1], si[lane][size - 1]))
                continue;
            int32_t pos = size < (int32_t)k ? size : (int32_t)k - 1;
            while (pos > 0 && cand_less(dist, g, sd[lane][pos - 1], si[lane][pos - 1])) {
                sd[lane][pos] = sd[lane][pos - 1];
                si[lane][pos] = si[lane][pos - 1];
                --pos;
            }
            sd[lane][pos] = dist;
            si[lane][pos] = g;
            if (size < (int32_t)k)
                ++size;
        }
        // wave merge: k rounds of (dist,id) argmin over the lane heads
        int head = 0;
        const size_t orow = (size_t)jb.out_row + fl.y;
        uint32_t count = 0;
        for (uint32_t t = 0; t < k; ++t) {
            float hd = head < size ? sd[lane][head] : INFINITY;
            uint32_t hi = head < size ? si[lane][head] : NONE;
            float bd = hd;
            uint32_t bi = hi;
            for (int off = 32; off > 0; off >>= 1) {
                const float od = __shfl_xor(bd, off);
                const uint32_t oi = __shfl_xor(bi, off);
                if (cand_less(od, oi, bd, bi)) {
                    bd = od;
                    bi = oi;
                }
            }
            if (bi != NONE && hi == bi)
                ++head;
            if (lane == 0) {
                if (S == 1) {
                    F.out_ids[orow * k + t] = bi != NONE ? bi - jb.id_base : NONE;
                    if (F.out_dist)
                        F.out_dist[orow * k + t] = bi != NONE ? bd : INFINITY;
                } else {
                    F.part_ids[w * k + t] = bi;
                    F.part_dist[w * k + t] = bi != NONE ? bd : INFINITY;
                }
            }
            count += bi != NONE ? 1u : 0u;
        }
        if (S == 1 && lane == 0 && F.out_size)
            F.out_size[orow] = (int32_t)count;
        __syncthreads();
    }
}

// Cross jobs whose q query rows times ceil(U / 64) candidate rounds stay within
// TINY_ROUNDS (U <= TINY_U) are scanned exactly, one wave per job
// (ung_tiny_jobs_kernel), instead of by the select and the merge: their 128 x 128 tiles
// are mostly padding (cfg3: most jobs have 1-4 queries and a few dozen candidates), and
// their exact scan costs less than their tiles.
constexpr uint32_t TINY_U = 1024;
constexpr uint32_t TINY_ROUNDS = 8;
constexpr uint32_t TINY_PAIRS = 64 * TINY_ROUNDS; // q * U <= q * 64 * ceil(U / 64)
constexpr int TINY_WAVES = 4;                      // jobs (waves) per block
__host__ __device__ inline bool tiny_job(uint32_t q, uint64_t u)
{
    return u <= TINY_U && (uint64_t)q * ((u + 63) / 64) <= TINY_ROUNDS;
}

// Those jobs (F.flagged[0 .. *F.flag_count).x, splits = 1): a wave scores the job's
// q x U (query row, candidate) pairs, one per lane (the reference's summation order),
// into its LDS slots [row * U + v], then for each row k rounds of a (dist, id) argmin
// over the lanes' best slots of the row, the winning lane rescanning its slots.
__global__ __launch_bounds__(64 * TINY_WAVES) void ung_tiny_jobs_kernel(FallbackParams F)
{
    __shared__ float td[TINY_WAVES][TINY_PAIRS];
    __shared__ uint32_t ti[TINY_WAVES][TINY_PAIRS];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t njobs = *F.flag_count, k = F.k;
    for (uint32_t jt = blockIdx.x * TINY_WAVES + (uint32_t)w; jt < njobs; jt += gridDim.x * TINY_WAVES) {
        const Job jb = F.jobs[F.flagged[jt].x];
        const bool excl = (jb.flags & 1u) != 0;
        const uint32_t U = jb.n_cand;
        // the planner keeps q * U within TINY_PAIRS (tiny_job); the bound keeps the slots safe
        const uint32_t Q = U ? min(jb.q_count, TINY_PAIRS / U) : 0u, P = Q * U;
        for (uint32_t p = (uint32_t)lane; p < P; p += 64) {
            const uint32_t r = p / U, v = p - r * U;
            const uint32_t q = jb.q_begin + r;
            const uint32_t g = cand_id(F.seg_start, F.seg_vend, jb.seg_begin, jb.seg_count, v);
            const bool ok = !(excl && g == q);
            td[w][p] = ok ? l2_ref_lane(F.X + (size_t)q * F.d, F.X + (size_t)g * F.d, F.d) : INFINITY;
            ti[w][p] = ok ? g : NONE;
        }
        // the slots of a row were written by other lanes of the wave
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        for (uint32_t r = 0; r < Q; ++r) {
            float bd = INFINITY;
            uint32_t bi = NONE, bp = 0;
            for (uint32_t v = (uint32_t)lane; v < U; v += 64)
                if (cand_less(td[w][r * U + v], ti[w][r * U + v], bd, bi)) {
                    bd = td[w][r * U + v];
                    bi = ti[w][r * U + v];
                    bp = r * U + v;
                }
            const size_t orow = (size_t)jb.out_row + r;
            uint32_t count = 0;
            for (uint32_t t = 0; t < k; ++t) {
                float md = bd;
                uint32_t mi = bi;
                wave_argmin(md, mi);
                if (mi == NONE)
                    break; // no candidate left (wave-uniform); the row's rest keeps its fill
                if (lane == 0) {
                    F.out_ids[orow * k + t] = mi - jb.id_base;
                    if (F.out_dist)
                        F.out_dist[orow * k + t] = md;
                }
                ++count;
                if (bi == mi) { // the winning lane (ids are unique) takes its next best
                    td[w][bp] = INFINITY;
                    ti[w][bp] = NONE;
                    bd = INFINITY;
                    bi = NONE;
                    for (uint32_t v = (uint32_t)lane; v < U; v += 64)
                        if (cand_less(td[w][r * U + v], ti[w][r * U + v], bd, bi)) {
                            bd = td[w][r * U + v];
                            bi = ti[w][r * U + v];
                            bp = r * U + v;
                        }
                }
            }
            if (lane == 0 && F.out_size)
                F.out_size[orow] = (int32_t)count;
        }
        // the next job rewrites the slots other lanes read above
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

// Merge of a flagged row's range results (ranges are disjoint, so ids are unique):
// lane l first keeps the k best entries of ranges l, l+64, ... in its LDS queue, then
// k rounds of a (dist, id) argmin over the lane heads.
__global__ __launch_bounds__(64) void ung_fallback_merge_kernel(FallbackParams F)
{
    __shared__ float sd[64][65];
    __shared__ uint32_t si[64][65];
    const int lane = threadIdx.x;
    const uint32_t S = F.splits, k = F.k;
    const uint32_t total = *F.flag_count;
    for (uint32_t f = blockIdx.x; f < total; f += gridDim.x) {
        const uint2 fl = F.flagged[f];
        const Job jb = F.jobs[fl.x];
        const size_t orow = (size_t)jb.out_row + fl.y;
        int32_t size = 0;
        for (uint32_t sp = (uint32_t)lane; sp < S; sp += 64) {
            const size_t base = ((size_t)f * S + sp) * k;
            for (uint32_t t = 0; t < k; ++t) {
                const uint32_t g = F.part_ids[base + t];
                if (g == NONE)
                    break; // a range's list is sorted, NONE entries come last
                const float dist = F.part_dist[base + t];
                if (size == (int32_t)k && !cand_less(dist, g, sd[lane][size - 1], si[lane][size - 1]))
                    break; // the rest of this sorted list can not enter either
                int32_t pos = size < (int32_t)k ? size : (int32_t)k - 1;
                while (pos > 0 && cand_less(dist, g, sd[lane][pos - 1], si[lane][pos - 1])) {
                    sd[lane][pos] = sd[lane][pos - 1];
                    si[lane][pos] = si[lane][pos - 1];
                    --pos;
                }
                sd[lane][pos] = dist;
                si[lane][pos] = g;
                if (size < (int32_t)k)
                    ++size;
            }
        }
        int head = 0;
        uint32_t count = 0;
        for (uint32_t t = 0; t < k; ++t) {
            const float hd = head < size ? sd[lane][head] : INFINITY;
            const uint32_t hi = head < size ? si[lane][head] : NONE;
            float bd = hd;
            uint32_t bi = hi;
            for (int off = 32; off > 0; off >>= 1) {
                const float od = __shfl_xor(bd, off);
                const uint32_t oi = __shfl_xor(bi, off);
                if (cand_less(od, oi, bd, bi)) {
                    bd = od;
                    bi = oi;
                }
            }
            if (bi != NONE && hi == bi)
                ++head;
            if (lane == 0) {
                F.out_ids[orow * k + t] = bi != NONE ? bi - jb.id_base : NONE;
                if (F.out_dist)
                    F.out_dist[orow * k + t] = bi != NONE ? bd : INFINITY;
            }
            count += bi != NONE ? 1u : 0u;
        }
        if (lane == 0 && F.out_size)
            F.out_size[orow] = (int32_t)count;
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// small kernels
// ---------------------------------------------------------------------------

// Split base set for the MFMA pre-selection: x = hi + lo + r with hi = bf16(x) and
// lo = bf16(x - hi) (x - hi is exact: both lie within a factor 2 of each other), so
// |r| <= 2^-18 |x|.  Row n holds dp words (dp = d rounded up to a multiple of KC); its
// chunk c (dimensions 32c .. 32c+31) is 16 words of hi pairs then 16 words of lo pairs,
// dimension 32c+2j in the low half of word j.  Dimensions >= d are zero.
__global__ __launch_bounds__(256) void ung_split_kernel(const float *__restrict__ X, uint64_t N, uint32_t d,
                                                        uint32_t dp, uint32_t *__restrict__ XS)
{
    const uint64_t per_row = dp / 2; // one (hi word, lo word) pair per thread
    const uint64_t total = N * per_row;
    for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t n = t / per_row;
        const uint32_t w = (uint32_t)(t - n * per_row); // pair index within the row
        const uint32_t c = w >> 4, j = w & 15u;
        const uint32_t dim = 32u * c + 2u * j;
        const float *x = X + n * d;
        const float x0 = dim < d ? x[dim] : 0.0f;
        const float x1 = dim + 1 < d ? x[dim + 1] : 0.0f;
        const uint32_t h0 = bf16_rne(x0), h1 = bf16_rne(x1);
        const uint32_t l0 = bf16_rne(x0 - __uint_as_float(h0 << 16));
        const uint32_t l1 = bf16_rne(x1 - __uint_as_float(h1 << 16));
        uint32_t *row = XS + n * dp + 32u * c;
        row[j] = h0 | (h1 << 16);
        row[16 + j] = l0 | (l1 << 16);
    }
}

// Squared norms (one wave per row, grid-stride over rows; lanes stride the row) and the
// largest of them: a block-wide maximum, then one atomic per block.  Accumulated in fp64
// and rounded once, so each cached norm is within 2^-24 (relative) of |x|^2.
__global__ __launch_bounds__(256) void ung_norm_kernel(const float *__restrict__ X, uint64_t N, uint32_t d,
                                                       float *__restrict__ xn, unsigned int *__restrict__ maxbits)
{
    __shared__ unsigned int wmax[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t nwaves = (uint64_t)gridDim.x * 4u;
    unsigned int mx = 0u; // non-negative floats order as their bit patterns
    for (uint64_t row = (uint64_t)blockIdx.x * 4u + (uint64_t)wave; row < N; row += nwaves) {
        const float *x = X + row * d;
        double sd = 0.0;
        for (uint32_t t = lane; t < d; t += 64)
            sd = __builtin_fma((double)x[t], (double)x[t], sd);
        for (int off = 32; off > 0; off >>= 1)
            sd += __shfl_xor(sd, off);
        const float s = (float)sd;
        if (lane == 0)
            xn[row] = s;
        mx = max(mx, __float_as_uint(s));
    }
    if (lane == 0)
        wmax[wave] = mx;
    __syncthreads();
    if (threadIdx.x == 0)
        atomicMax(maxbits, max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3])));
}

__global__ void ung_fill_rows_kernel(uint32_t *ids, float *dist, int32_t *size, uint64_t rows,
                                     uint32_t k)
{
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < rows * k) {
        ids[i] = NONE;
        if (dist)
            dist[i] = INFINITY;
    }
    if (size && i < rows)
        size[i] = 0;
}

__global__ void ung_zero_u32_kernel(uint32_t *p, uint32_t n)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        p[i] = 0;
}

// Group id (1..G) of every point, from the group-contiguous ranges.
__global__ void ung_point_group_kernel(const uint32_t *__restrict__ group_begin, uint32_t G,
                                       uint32_t *__restrict__ pg)
{
    for (uint32_t g = blockIdx.x + 1; g <= G; g += gridDim.x)
        for (uint32_t i = group_begin[g] + threadIdx.x; i < group_begin[g + 1]; i += blockDim.x)
            pg[i] = g;
}

// Additional edges, step 1 (src/uni_nav_graph_cross_edges.cpp:489-531): marks every entry
// p of the LNG row of C = group(i) whose group is reached by one of the first `use` cross
// edges of point i.  One thread per point; entries only ever go 0 -> 1.
__global__ void ung_addl_mark_kernel(const uint32_t *__restrict__ ids, uint32_t stride, uint32_t use,
                                     const uint32_t *__restrict__ pg, uint64_t N,
                                     const uint32_t *__restrict__ out_ptr, const uint32_t *__restrict__ out_idx,
                                     uint32_t *__restrict__ reached)
{
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N)
        return;
    const uint32_t c = pg[i];
    const uint32_t b = out_ptr[c], e = out_ptr[c + 1];
    for (uint32_t t = 0; t < use && b < e; ++t) {
        const uint32_t nb = ids[i * stride + t];
        if (nb == NONE)
            continue;
        const uint32_t x = pg[nb];
        for (uint32_t p = b; p < e; ++p)
            if (out_idx[p] == x) {
                reached[p] = 1u;
                break;
            }
    }
}

// Additional edges, step 2: per LNG entry p = (C, X) left unreached, the query rows
// m = min(|C|, ceil(num_cross / per)) and edges m * per it adds, per = min(|X|, num_cross/2)
// (src/uni_nav_graph_cross_edges.cpp:543-562: vectors of C in order, per edges each, until
// num_cross are appended); 0 for reached entries and for entries of no group (eg = 0).
// cnt[0] += scored (query, candidate) pairs, cnt[1] += entries that add edges.
// Additional edges: a target group of more than ADDL_SMALL vectors is scanned in ranges of
// ADDL_RANGE, one wave each (a query row of a large group spreads over many waves).
constexpr uint32_t ADDL_SMALL = 8;     // target groups up to this size: one thread per entry
constexpr uint32_t ADDL_RANGE = 1024;  // candidates per scan item

__global__ void ung_addl_count_kernel(const uint32_t *__restrict__ gb, const uint32_t *__restrict__ oi,
                                      const uint32_t *__restrict__ eg, const uint32_t *__restrict__ reached,
                                      uint32_t E, uint32_t num_cross, uint32_t *__restrict__ rows,
                                      uint32_t *__restrict__ edges, uint32_t *__restrict__ items,
                                      unsigned long long *__restrict__ cnt)
{
    unsigned long long my_pairs = 0, my_entries = 0;
    for (uint32_t p = blockIdx.x * blockDim.x + threadIdx.x; p < E; p += gridDim.x * blockDim.x) {
        uint32_t m = 0, per = 0, nx = 0;
        const uint32_t c = eg[p];
        if (!reached[p] && c != 0) {
            const uint32_t x = oi[p];
            const uint32_t nc = gb[c + 1] - gb[c];
            nx = gb[x + 1] - gb[x];
            per = min(nx, num_cross / 2u);
            if (per > 0 && nc > 0)
                m = min(nc, (num_cross + per - 1) / per);
            my_pairs += (unsigned long long)m * nx;
            my_entries += m > 0;
        }
        rows[p] = m;
        edges[p] = m * per;
        items[p] = nx > ADDL_SMALL ? m * ((nx + ADDL_RANGE - 1) / ADDL_RANGE) : 0u;
    }
    // one atomic per wave and counter (same-address atomics serialise in the L2)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        my_pairs += __shfl_xor(my_pairs, o);
        my_entries += __shfl_xor(my_entries, o);
    }
    if ((threadIdx.x & 63u) == 0 && my_pairs)
        atomicAdd(&cnt[0], my_pairs);
    if ((threadIdx.x & 63u) == 0 && my_entries)
        atomicAdd(&cnt[1], my_entries);
}

// Additional edges, step 3: scan items (an entry p = (C, X) with a target group of more
// than ADDL_SMALL vectors has m query rows, vectors 0..m-1 of C, times ceil(|X| /
// ADDL_RANGE) ranges of X): one wave per item scans its range in the reference's summation
// order and keeps the first `per` by (dist, id).  A row of one range writes its results to
// their final place in the per-group edge lists (entries in LNG order, vectors, ranks);
// the ranges of a larger row write partial lists that ung_addl_merge_kernel merges.
struct AddlParams {
    const float *X;
    uint32_t d;
    const uint32_t *gb, *oi, *eg;
    const uint32_t *row_off, *edge_off; // [E+1] exclusive scans
    const uint32_t *item_off;           // [E+1] exclusive scan of the scan items
    const uint32_t *item_entry;         // [I] entry of each scan item
    uint32_t E, I;
    uint32_t per_max;
    uint32_t *part_ids; // [I x per_max] partial lists of the rows of several ranges
    float *part_dist;
    uint32_t *from, *to;
};

// The entry of each scan item (one thread per entry).
__global__ void ung_addl_expand_kernel(const uint32_t *__restrict__ item_off, uint32_t E,
                                       uint32_t *__restrict__ item_entry)
{
    for (uint32_t p = blockIdx.x * blockDim.x + threadIdx.x; p < E; p += gridDim.x * blockDim.x)
        for (uint32_t w = item_off[p]; w < item_off[p + 1]; ++w)
            item_entry[w] = p;
}

// Where scan item w sits: its entry, target range, query row and ranges per row.
struct AddlItem {
    uint32_t p, q, x0, nx, nr, j, r, per;
};
__device__ __forceinline__ AddlItem addl_item(const AddlParams &A, uint32_t w)
{
    AddlItem t;
    t.p = A.item_entry[w];
    const uint32_t c = A.eg[t.p], x = A.oi[t.p];
    t.x0 = A.gb[x];
    t.nx = A.gb[x + 1] - t.x0;
    t.nr = (t.nx + ADDL_RANGE - 1) / ADDL_RANGE;
    const uint32_t loc = w - A.item_off[t.p];
    t.j = loc / t.nr;
    t.r = loc - t.j * t.nr;
    t.q = A.gb[c] + t.j;
    t.per = min(t.nx, A.per_max);
    return t;
}

__global__ __launch_bounds__(64) void ung_addl_scan_kernel(AddlParams A)
{
    __shared__ float sd[64][33];
    __shared__ uint32_t si[64][33];
    const int lane = threadIdx.x;
    for (uint32_t w = blockIdx.x; w < A.I; w += gridDim.x) {
        const AddlItem t = addl_item(A, w);
        const float *qv = A.X + (size_t)t.q * A.d;
        const uint32_t v0 = t.x0 + t.r * ADDL_RANGE, v1 = min(t.x0 + t.nx, v0 + ADDL_RANGE);
        const uint32_t per = t.per;
        int32_t size = 0;
        for (uint32_t g = v0 + (uint32_t)lane; g < v1; g += 64) {
            const float dist = l2_ref_lane(qv, A.X + (size_t)g * A.d, A.d);
            if (size == (int32_t)per && !cand_less(dist, g, sd[lane][size - 1], si[lane][size - 1]))
                continue;
            int32_t pos = size < (int32_t)per ? size : (int32_t)per - 1;
            while (pos > 0 && cand_less(dist, g, sd[lane][pos - 1], si[lane][pos - 1])) {
                sd[lane][pos] = sd[lane][pos - 1];
                si[lane][pos] = si[lane][pos - 1];
                --pos;
            }
            sd[lane][pos] = dist;
            si[lane][pos] = g;
            if (size < (int32_t)per)
                ++size;
        }
        // per rounds of a (dist, id) argmin over the lane heads
        int head = 0;
        const size_t o = (size_t)A.edge_off[t.p] + (size_t)t.j * per;
        for (uint32_t k = 0; k < per; ++k) {
            const float hd = head < size ? sd[lane][head] : INFINITY;
            const uint32_t hi2 = head < size ? si[lane][head] : NONE;
            float bd = hd;
            uint32_t bi = hi2;
            for (int off = 32; off > 0; off >>= 1) {
                const float od = __shfl_xor(bd, off);
                const uint32_t oi2 = __shfl_xor(bi, off);
                if (cand_less(od, oi2, bd, bi)) {
                    bd = od;
                    bi = oi2;
                }
            }
            if (bi != NONE && hi2 == bi)
                ++head;
            if (lane == 0) {
                if (t.nr == 1) {
                    A.from[o + k] = t.q;
                    A.to[o + k] = bi;
                } else {
                    A.part_ids[(size_t)w * A.per_max + k] = bi;
                    A.part_dist[(size_t)w * A.per_max + k] = bd;
                }
            }
        }
        __syncthreads();
    }
}

// The rows of several ranges (the item of range 0 stands for the row): lane l first keeps
// the per best entries of ranges l, l+64, ... (each list sorted, ranges disjoint) in its
// LDS queue, then per rounds of a (dist, id) argmin over the lane heads.
__global__ __launch_bounds__(64) void ung_addl_merge_kernel(AddlParams A)
{
    __shared__ float sd[64][33];
    __shared__ uint32_t si[64][33];
    const int lane = threadIdx.x;
    for (uint32_t w = blockIdx.x; w < A.I; w += gridDim.x) {
        const AddlItem t = addl_item(A, w);
        if (t.nr == 1 || t.r != 0)
            continue; // uniform: one wave per block
        const uint32_t per = t.per;
        int32_t size = 0;
        for (uint32_t rr = (uint32_t)lane; rr < t.nr; rr += 64) {
            const size_t base = (size_t)(w + rr) * A.per_max;
            for (uint32_t k = 0; k < per; ++k) {
                const uint32_t g = A.part_ids[base + k];
                if (g == NONE)
                    break; // a range's list is sorted, NONE entries come last
                const float dist = A.part_dist[base + k];
                if (size == (int32_t)per && !cand_less(dist, g, sd[lane][size - 1], si[lane][size - 1]))
                    break; // the rest of this sorted list can not enter either
                int32_t pos = size < (int32_t)per ? size : (int32_t)per - 1;
                while (pos > 0 && cand_less(dist, g, sd[lane][pos - 1], si[lane][pos - 1])) {
                    sd[lane][pos] = sd[lane][pos - 1];
                    si[lane][pos] = si[lane][pos - 1];
                    --pos;
                }
                sd[lane][pos] = dist;
                si[lane][pos] = g;
                if (size < (int32_t)per)
                    ++size;
            }
        }
        int head = 0;
        const size_t o = (size_t)A.edge_off[t.p] + (size_t)t.j * per;
        for (uint32_t k = 0; k < per; ++k) {
            const float hd = head < size ? sd[lane][head] : INFINITY;
            const uint32_t hi2 = head < size ? si[lane][head] : NONE;
            float bd = hd;
            uint32_t bi = hi2;
            for (int off = 32; off > 0; off >>= 1) {
                const float od = __shfl_xor(bd, off);
                const uint32_t oi2 = __shfl_xor(bi, off);
                if (cand_less(od, oi2, bd, bi)) {
                    bd = od;
                    bi = oi2;
                }
            }
            if (bi != NONE && hi2 == bi)
                ++head;
            if (lane == 0) {
                A.from[o + k] = t.q;
                A.to[o + k] = bi;
            }
        }
        __syncthreads();
    }
}

// Additional edges, step 3 for target groups of at most ADDL_SMALL vectors: one wave per
// LNG entry.  Its m x nx (query row, target vector) pairs are scored by groups of 8 lanes
// in the reference's summation order (coalesced 32-byte row segments), then lane j < m
// orders row j's nx candidates by (dist, id) with an insertion network and writes the
// first `per`; the wave kernel above skips these rows.  m x nx <= num_cross + ADDL_SMALL
// - 1 (per = nx when nx <= num_cross / 2, else m <= 3), below ADDL_SMALL_PAIRS for
// num_cross <= 64.
constexpr uint32_t ADDL_SMALL_PAIRS = 72;

__global__ __launch_bounds__(256) void ung_addl_small_kernel(AddlParams A)
{
    __shared__ float sd[4][ADDL_SMALL_PAIRS];
    const int w = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63u);
    const int sg = lane >> 3, sub = lane & 7;
    const uint32_t p = blockIdx.x * 4u + (uint32_t)w;
    uint32_t m = 0, nx = 0, x0 = 0, q0 = 0;
    if (p < A.E) {
        m = A.row_off[p + 1] - A.row_off[p];
        const uint32_t x = A.oi[p];
        x0 = A.gb[x];
        nx = A.gb[x + 1] - x0;
        if (nx > ADDL_SMALL)
            m = 0;
        if (m > 0)
            q0 = A.gb[A.eg[p]];
    }
    const uint32_t np = m * nx;
    for (uint32_t i = (uint32_t)sg; i < np; i += 8u) {
        const uint32_t j = i / nx, t = i - j * nx;
        const float v = l2_ref_8lane(A.X + (size_t)(q0 + j) * A.d, A.X + (size_t)(x0 + t) * A.d, A.d, sub);
        if (sub == 0)
            sd[w][i] = v;
    }
    __syncthreads();
    if ((uint32_t)lane >= m)
        return;
    const uint32_t j = (uint32_t)lane;
    float dv[ADDL_SMALL];
    uint32_t iv[ADDL_SMALL];
#pragma unroll
    for (uint32_t t = 0; t < ADDL_SMALL; ++t) {
        dv[t] = t < nx ? sd[w][j * nx + t] : INFINITY;
        iv[t] = t < nx ? x0 + t : NONE;
    }
    // insertion network under (dist, id): candidates arrive in id order
#pragma unroll
    for (int t = 1; t < (int)ADDL_SMALL; ++t)
#pragma unroll
        for (int u = t; u > 0; --u)
            if (cand_less(dv[u], iv[u], dv[u - 1], iv[u - 1])) {
                const float td = dv[u];
                dv[u] = dv[u - 1];
                dv[u - 1] = td;
                const uint32_t ti = iv[u];
                iv[u] = iv[u - 1];
                iv[u - 1] = ti;
            }
    const uint32_t per = min(nx, A.per_max);
    const size_t o = (size_t)A.edge_off[p] + (size_t)j * per;
#pragma unroll
    for (uint32_t t = 0; t < ADDL_SMALL; ++t)
        if (t < per) {
            A.from[o + t] = q0 + j;
            A.to[o + t] = iv[t];
        }
}

// edge_ptr[c] = first edge of group c: the edge offset of its first LNG entry.
__global__ void ung_addl_ptr_kernel(const uint32_t *__restrict__ op, const uint32_t *__restrict__ edge_off,
                                    uint32_t G, uint32_t *__restrict__ edge_ptr)
{
    for (uint32_t c = blockIdx.x * blockDim.x + threadIdx.x; c <= G + 1; c += gridDim.x * blockDim.x)
        edge_ptr[c] = c == 0 ? 0u : edge_off[op[c]];
}

// Exact-anchor row packing (src/tagore_graph_builder.cu:727-794), one thread per row.
struct PackParams {
    const Job *jobs;
    const MergeItem *mitems;
    const uint32_t *list_ids; // [rows x list_k] local ids
    uint32_t list_k;
    uint32_t tagore_k, final_degree, head_keep, anchor_tail, anchor_slots, bidir_anchor;
    uint32_t graph_stride;
    uint32_t *graph;
};

__device__ __forceinline__ bool row_has(const uint32_t *row, uint32_t write, uint32_t v)
{
    for (uint32_t p = 0; p < write; ++p)
        if (row[1 + p] == v)
            return true;
    return false;
}

__global__ __launch_bounds__(MERGE_Q) void ung_pack_kernel(PackParams K)
{
    const MergeItem mi = K.mitems[blockIdx.x];
    if (threadIdx.x >= mi.q_cnt)
        return;
    const Job jb = K.jobs[mi.job];
    const uint32_t local_src = mi.q_off + threadIdx.x;
    const uint32_t n = jb.q_count;
    const size_t orow = (size_t)jb.out_row + local_src;
    const uint32_t *top = K.list_ids + orow * K.list_k;
    uint32_t *row = K.graph + orow * K.graph_stride;
    const uint32_t kcap = K.tagore_k > 0 ? K.tagore_k - 1 : 0;
    uint32_t cand_degree = 64u < kcap ? 64u : kcap;
    cand_degree = cand_degree < (n > 0 ? n - 1 : 0) ? cand_degree : (n > 0 ? n - 1 : 0);
    const uint32_t fd = K.final_degree;
    const uint32_t out_degree = fd < cand_degree ? fd : cand_degree;
    row[0] = out_degree;
    if (out_degree > 0) {
        uint32_t near_limit = K.head_keep < fd ? K.head_keep : fd;
        near_limit = out_degree < near_limit ? out_degree : near_limit;
        uint32_t write = 0;
        for (; write < near_limit; ++write)
            row[1 + write] = top[write];
        const uint32_t remaining = fd > write ? fd - write : 0;
        uint32_t anchor_limit = 0;
        if (K.anchor_tail)
            anchor_limit = K.anchor_slots == 0 ? remaining : (K.anchor_slots < remaining ? K.anchor_slots : remaining);
        if (anchor_limit > 0 && n > 1) {
            for (uint32_t t = 0; t < anchor_limit && write < out_degree; ++t) {
                uint32_t hop = ((t + 1) * n) / (anchor_limit + 1);
                hop = hop < 1 ? 1 : hop;
                const bool backward = K.bidir_anchor && (t & 1u);
                uint32_t cand = backward ? (local_src + n - (hop % n)) % n : (local_src + hop) % n;
                for (uint32_t retry = 0; retry < n && write < out_degree; ++retry) {
                    if (cand != local_src && !row_has(row, write, cand)) {
                        row[1 + write++] = cand;
                        break;
                    }
                    cand = backward ? (cand + n - 1) % n : (cand + 1) % n;
                }
            }
        }
        const uint32_t tail_start = near_limit;
        const uint32_t tail_count = cand_degree > tail_start ? cand_degree - tail_start : 0;
        const uint32_t step = (tail_count > remaining && remaining > 0) ? (tail_count + remaining - 1) / remaining : 1;
        for (uint32_t s = tail_start; s < cand_degree && write < out_degree; s += step)
            row[1 + write++] = top[s];
        for (uint32_t s = tail_start; s < cand_degree && write < out_degree; ++s)
            if (!row_has(row, write, top[s]))
                row[1 + write++] = top[s];
    }
    for (uint32_t j = out_degree; j + 1 < K.graph_stride; ++j)
        row[1 + j] = local_src;
}

// ---------------------------------------------------------------------------
// large-group graph: the FastGrnnd prune (tagore_graph_builder.cu:1463-1568, kernels
// build_sampled_reverse_kernel :141-163 and fast_grnnd_prune_kernel :279-387) over the
// resident exact kNN lists of ung_hip_group_knn.  Rows are local ids.
// ---------------------------------------------------------------------------
struct PruneParams {
    const float *X;
    uint32_t d;
    const Job *jobs;
    uint32_t n_jobs;
    const uint32_t *ids;  // [rows x list_k] local ids, by (dist, id)
    const float *dist;
    const int32_t *size;
    uint32_t list_k;
    uint32_t forward_cap, reverse_cap, final_degree;
    float alpha;
    uint64_t rows;
    uint32_t *rev_cnt;    // [rows + 1]: reverse counts, then (scanned) offsets
    uint32_t *rev_fill;   // [rows] fill positions
    uint32_t *rev_src;    // [total] source local ids
    float *rev_dist;
    uint32_t *graph;      // [rows x (final_degree + 1)]
    // the certified Gram pre-decision (ung_prune_gram_kernel)
    const uint32_t *xs;   // split base set, [N][dp] words
    const float *xn;      // squared norms
    uint32_t dp;
    double eps_coef;      // expansion-form error factor (as the select's), on (|a| + |b|)^2
    double shrink;        // relative error of the reference summation
};

// Job (group) of a result row: the last job whose first row is <= r.
__device__ __forceinline__ uint32_t job_of_row(const Job *__restrict__ jobs, uint32_t n_jobs, uint32_t r)
{
    uint32_t lo = 0, hi = n_jobs - 1;
    while (lo < hi) {
        const uint32_t mid = (lo + hi + 1) >> 1;
        if (jobs[mid].out_row <= r)
            lo = mid;
        else
            hi = mid - 1;
    }
    return lo;
}

// Reverse edges: source row r adds itself to the list of each of its first forward_cap
// candidates (counting pass, then, after a scan, the filling pass; the order inside a
// list is fixed later by sorting).
template <bool FILL>
__global__ __launch_bounds__(256) void ung_reverse_kernel(PruneParams K)
{
    for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < K.rows;
         r += (uint64_t)gridDim.x * blockDim.x) {
        const Job jb = K.jobs[job_of_row(K.jobs, K.n_jobs, (uint32_t)r)];
        const uint32_t src = (uint32_t)r - jb.out_row;
        const uint32_t cnt = min((uint32_t)K.size[r], K.forward_cap);
        for (uint32_t t = 0; t < cnt; ++t) {
            const uint32_t dst = jb.out_row + K.ids[r * K.list_k + t];
            if constexpr (!FILL) {
                atomicAdd(&K.rev_cnt[dst], 1u);
            } else {
                const uint32_t at = K.rev_cnt[dst] + atomicAdd(&K.rev_fill[dst], 1u);
                K.rev_src[at] = src;
                K.rev_dist[at] = K.dist[r * K.list_k + t]; // d(src, dst) == d(dst, src) bit for bit
            }
        }
    }
}

constexpr uint32_t PRUNE_LDS_D = 1024;

// One wave (block) per row: forward candidates + the reverse_cap nearest reverse edges,
// merged by (dist, id) without duplicates, then the greedy alpha scan.
__global__ __launch_bounds__(64) void ung_prune_kernel(PruneParams K)
{
    __shared__ float cd[128];
    __shared__ uint32_t ci[128];
    __shared__ float rd[32];
    __shared__ uint32_t ri[32];
    __shared__ uint32_t kept[64];
    __shared__ uint32_t ncand;
    // the candidate's row, staged once per candidate and read by every pivot's distance
    // (rows of up to PRUNE_LDS_D floats; larger ones are read from memory each time)
    __shared__ __align__(16) float trow[PRUNE_LDS_D];
    const int lane = threadIdx.x;
    const uint64_t r = blockIdx.x;
    if (r >= K.rows)
        return;
    const Job jb = K.jobs[job_of_row(K.jobs, K.n_jobs, (uint32_t)r)];
    const uint32_t s = (uint32_t)r - jb.out_row;
    const uint32_t cnt_f = min((uint32_t)K.size[r], K.forward_cap);
    // the reverse_cap nearest reverse edges: 32 best kept in lanes 0..31 while chunks of
    // 32 pass through lanes 32..63
    const uint32_t r0 = K.rev_cnt[r], r1 = K.rev_cnt[r + 1];
    float bd = INFINITY;
    uint32_t bi = NONE;
    for (uint32_t c0 = r0; c0 < r1; c0 += 32) {
        if (lane >= 32) {
            const uint32_t at = c0 + (uint32_t)(lane - 32);
            bd = at < r1 ? K.rev_dist[at] : INFINITY;
            bi = at < r1 ? K.rev_src[at] : NONE;
        }
        wave_sort64(bd, bi, lane);
    }
    const uint32_t cnt_r = min(K.reverse_cap, r1 - r0);
    if ((uint32_t)lane < cnt_r) {
        rd[lane] = bd;
        ri[lane] = bi;
    }
    __syncthreads();
    if (lane == 0) {
        const float *fdp = K.dist + r * K.list_k;
        const uint32_t *fip = K.ids + r * K.list_k;
        uint32_t i = 0, j = 0, nc = 0;
        while (i < cnt_f || j < cnt_r) {
            const bool take_f = j == cnt_r || (i < cnt_f && !cand_less(rd[j], ri[j], fdp[i], fip[i]));
            const float dv = take_f ? fdp[i] : rd[j];
            const uint32_t iv = take_f ? fip[i] : ri[j];
            i += take_f ? 1u : 0u;
            j += take_f ? 0u : 1u;
            if (nc > 0 && ci[nc - 1] == iv)
                continue; // the same id twice carries the same distance: adjacent
            cd[nc] = dv;
            ci[nc] = iv;
            ++nc;
        }
        ncand = nc;
    }
    __syncthreads();
    const uint32_t nc = ncand;
    const float *__restrict__ X = K.X + (size_t)jb.q_begin * K.d;
    const int g = lane >> 3, sub = lane & 7;
    // float4 staging: rows 16-byte aligned (d % 4 == 0) that fit
    const bool stage_t = (K.d & 3u) == 0u && K.d <= (uint32_t)PRUNE_LDS_D;
    uint32_t na = 0;
    for (uint32_t c = 0; c < nc && na < K.final_degree; ++c) {
        const uint32_t t = ci[c];
        const float dc = cd[c];
        if (t == s)
            continue;
        bool reject = false;
        if (na > 0 && stage_t) {
            // one wave per block: the barrier orders the previous candidate's reads of
            // trow before these writes, and these writes before the reads below
            __syncthreads();
            const float4 *src = reinterpret_cast<const float4 *>(X + (size_t)t * K.d);
            for (uint32_t i = (uint32_t)lane; i < (K.d >> 2); i += 64u)
                reinterpret_cast<float4 *>(trow)[i] = src[i];
            __syncthreads();
        }
        for (uint32_t p0 = 0; p0 < na && !reject; p0 += 8) {
            const uint32_t p = p0 + (uint32_t)g;
            const bool valid = p < na;
            const uint32_t piv = valid ? kept[p] : t;
            const float dij = stage_t ? l2_ref_8lane(X + (size_t)piv * K.d, trow, K.d, sub)
                                      : l2_ref_8lane(X + (size_t)piv * K.d, X + (size_t)t * K.d, K.d, sub);
            reject = __ballot(valid && sub == 0 && K.alpha * dij < dc) != 0;
        }
        if (!reject) {
            if (lane == 0)
                kept[na] = t;
            ++na;
            __syncthreads();
        }
    }
    uint32_t *row = K.graph + r * (K.final_degree + 1);
    if (lane == 0)
        row[0] = na;
    for (uint32_t j = (uint32_t)lane; j < K.final_degree; j += 64)
        row[1 + j] = j < na ? kept[j] : s;
}

// ---------------------------------------------------------------------------
// The same prune with its alpha tests decided from a certified Gram matrix: the row's
// candidates (at most 96: forward_cap <= 64 plus reverse_cap <= 32) go through the split-bf16
// MFMA passes of the select kernel as a 96 x 96 Gram matrix (upper triangle: six 32 x 32
// blocks), so an approximate distance of every pair of candidates costs no row loads of its
// own.  The alpha test `alpha * d(kept, cand) < d(row, cand)` of the exact scan
// (fp32 distances in the reference's summation order) is then decided from bounds: with
// D~ = |a|^2 + |b|^2 - 2 G(a, b) and |D~ - D| <= eps_coef (|a| + |b|)^2 (the select's error
// model: split operands, accumulation from 0, norm caches and the final fma), the
// reference's distance lies in [L, U] = lower_bound_ea / upper_bound_ea of D~; fp32
// multiplication by alpha is monotone, so fl(alpha U) < d(row, cand) proves a rejection and
// fl(alpha L) >= d(row, cand) proves a pass.  Only pairs left undecided (near the
// boundary, or exact ties) are scored exactly, as in ung_prune_kernel.  The kept lists are
// therefore identical to ung_prune_kernel's.  One wave per row.
// ---------------------------------------------------------------------------
constexpr int PG_N = 96;             // candidates of a row (padded)
constexpr int PG_W = KC + 4;         // staged chunk row stride (words)

// Block (bi, bj), bi <= bj, of the upper triangle of 32 x 32 blocks: 0 1 2 / 3 4 / 5.
__device__ __forceinline__ int pg_block(int bi, int bj)
{
    return bj + (bi == 0 ? 0 : bi + 1);
}

struct alignas(16) PruneGramSmem {
    union {
        float4 xs[2][PG_N][PG_W / 4]; // a chunk (32 dimensions) of every candidate row, two
                                      // buffers
        float g[6][32][33];           // the Gram blocks after the last chunk (pg_block order)
    } u;
    float cd[128];
    uint32_t ci[128];
    float cn[PG_N];                  // candidates' squared norms
    float cr[PG_N];                  // and norms (rounded up)
    float rd[32];
    uint32_t ri[32];
    uint32_t kept[64];               // kept candidates (local ids)
    uint32_t kpos[64];               // and their positions in the candidate list
    uint32_t ncand;
};

__global__ __launch_bounds__(64) void ung_prune_gram_kernel(PruneParams K)
{
    __shared__ PruneGramSmem sm;
    const int lane = threadIdx.x;
    const uint64_t r = blockIdx.x;
    if (r >= K.rows)
        return;
    const Job jb = K.jobs[job_of_row(K.jobs, K.n_jobs, (uint32_t)r)];
    const uint32_t s = (uint32_t)r - jb.out_row;
    const uint32_t cnt_f = min((uint32_t)K.size[r], K.forward_cap);
    // the reverse_cap nearest reverse edges (as ung_prune_kernel)
    const uint32_t r0 = K.rev_cnt[r], r1 = K.rev_cnt[r + 1];
    float bd = INFINITY;
    uint32_t bi = NONE;
    for (uint32_t c0 = r0; c0 < r1; c0 += 32) {
        if (lane >= 32) {
            const uint32_t at = c0 + (uint32_t)(lane - 32);
            bd = at < r1 ? K.rev_dist[at] : INFINITY;
            bi = at < r1 ? K.rev_src[at] : NONE;
        }
        wave_sort64(bd, bi, lane);
    }
    const uint32_t cnt_r = min(K.reverse_cap, r1 - r0);
    if ((uint32_t)lane < cnt_r) {
        sm.rd[lane] = bd;
        sm.ri[lane] = bi;
    }
    __syncthreads();
    if (lane == 0) {
        const float *fdp = K.dist + r * K.list_k;
        const uint32_t *fip = K.ids + r * K.list_k;
        uint32_t i = 0, j = 0, nc = 0;
        while (i < cnt_f || j < cnt_r) {
            const bool take_f = j == cnt_r || (i < cnt_f && !cand_less(sm.rd[j], sm.ri[j], fdp[i], fip[i]));
            const float dv = take_f ? fdp[i] : sm.rd[j];
            const uint32_t iv = take_f ? fip[i] : sm.ri[j];
            i += take_f ? 1u : 0u;
            j += take_f ? 0u : 1u;
            if (nc > 0 && sm.ci[nc - 1] == iv)
                continue; // the same id twice carries the same distance: adjacent
            sm.cd[nc] = dv;
            sm.ci[nc] = iv;
            ++nc;
        }
        sm.ncand = nc;
    }
    __syncthreads();
    const uint32_t nc = sm.ncand; // <= cnt_f + cnt_r <= 96
    const float *__restrict__ X = K.X + (size_t)jb.q_begin * K.d;
    const uint32_t *__restrict__ XS = K.xs + (size_t)jb.q_begin * K.dp;
    // padding positions (>= nc) repeat the row's own point: their Gram entries are never read
    for (uint32_t i = (uint32_t)lane; i < (uint32_t)PG_N; i += 64u) {
        const float x2 = i < nc ? K.xn[jb.q_begin + sm.ci[i]] : 0.0f;
        sm.cn[i] = x2;
        sm.cr[i] = __double2float_ru(sqrt((double)fmaxf(x2, 0.0f) * (1.0 + 1e-6)));
    }

    // Gram of the candidates: chunk by chunk (32 dimensions = two k-blocks of 16) through
    // LDS; lane (r32, h) feeds row/column r32 of a 32-block, dimensions 16 kb + 8 h .. + 7;
    // three passes per k-block (hi*hi, hi*lo, lo*hi), blocks (bi, bj) with bi <= bj
    const int r32 = lane & 31, h = lane >> 5;
    floatx16 acc[6];
    const floatx16 zero = {};
    // loader: row lr = lane / 8 + 8 m (m = 0..11), float4 column c4 = lane % 8 of the chunk
    const int lc = lane & 7, lr0 = lane >> 3;
    const uint32_t nk = K.dp / KC;
    // the lane's rows (local ids)
    uint32_t rid[PG_N / 8];
#pragma unroll
    for (int m = 0; m < PG_N / 8; ++m) {
        const uint32_t row = (uint32_t)(lr0 + 8 * m);
        rid[m] = row < nc ? sm.ci[row] : s;
    }
    const uint32_t *__restrict__ XSl = XS + 4u * (uint32_t)lc;
    // chunk kc + 1 is loaded into registers while chunk kc is multiplied from LDS, and
    // staged into the other LDS buffer after it
    u32x4 pre[PG_N / 8];
    auto load_chunk = [&](uint32_t kc) __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < PG_N / 8; ++m)
            pre[m] = *reinterpret_cast<const u32x4 *>(XSl + (size_t)rid[m] * K.dp + kc * KC);
    };
    auto stage_chunk = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < PG_N / 8; ++m)
            *reinterpret_cast<u32x4 *>(&sm.u.xs[buf][lr0 + 8 * m][lc]) = pre[m];
    };
    load_chunk(0);
    stage_chunk(0);
    __syncthreads();
    if (nk > 1)
        load_chunk(1);
    for (uint32_t kc = 0; kc < nk; ++kc) {
        const int buf = (int)(kc & 1u);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int ch = 2 * kb + h;
            bf16x8 hi[3], lo[3];
#pragma unroll
            for (int b = 0; b < 3; ++b) {
                hi[b] = __builtin_bit_cast(bf16x8, sm.u.xs[buf][32 * b + r32][ch]);
                lo[b] = __builtin_bit_cast(bf16x8, sm.u.xs[buf][32 * b + r32][ch + 4]);
            }
            // pass-major: six independent accumulators between dependent MFMAs
            const bool z = kc == 0 && kb == 0;
            constexpr int BI[6] = {0, 0, 0, 1, 1, 2}, BJ[6] = {0, 1, 2, 1, 2, 2}; // pg_block order
#pragma unroll
            for (int t = 0; t < 6; ++t)
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(hi[BI[t]], hi[BJ[t]], z ? zero : acc[t], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 6; ++t)
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(hi[BI[t]], lo[BJ[t]], acc[t], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 6; ++t)
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lo[BI[t]], hi[BJ[t]], acc[t], 0, 0, 0);
        }
        if (kc + 1 < nk)
            stage_chunk(buf ^ 1); // its previous reads (chunk kc - 1) ended at the last barrier
        __syncthreads();
        if (kc + 2 < nk)
            load_chunk(kc + 2);
    }
    // (the loop's last barrier ended the last chunk's operand reads: the Gram takes their
    // place)
    {
        int t = 0;
#pragma unroll
        for (int bi2 = 0; bi2 < 3; ++bi2)
#pragma unroll
            for (int bj = bi2; bj < 3; ++bj, ++t)
#pragma unroll
                for (int q = 0; q < 16; ++q)
                    sm.u.g[t][8 * (q >> 2) + 4 * h + (q & 3)][r32] = acc[t][q];
    }
    __syncthreads();

    // greedy scan: lane l < na holds kept point l; a candidate is decided from the bounds
    // of its Gram distances, undecided pairs are scored exactly (eight lanes a pair)
    const int g8 = lane >> 3, sub = lane & 7;
    uint32_t na = 0;
    for (uint32_t c = 0; c < nc && na < K.final_degree; ++c) {
        const uint32_t t = sm.ci[c];
        const float dc = sm.cd[c];
        if (t == s)
            continue;
        bool sure_rej = false, unsure = false;
        if ((uint32_t)lane < na) {
            const uint32_t kp = sm.kpos[lane]; // kp < c
            const float xa = sm.cn[kp], xb = sm.cn[c];
            const float gv = sm.u.g[pg_block((int)(kp >> 5), (int)(c >> 5))][kp & 31u][c & 31u];
            const float dt = __builtin_fmaf(-2.0f, gv, xa + xb);
            const double nab = (double)sm.cr[kp] + (double)sm.cr[c];
            const double ea = K.eps_coef * nab * nab;
            const float lo_b = fmaxf(lower_bound_ea(dt, ea, K.shrink), 0.0f);
            const float up_b = upper_bound_ea(dt, ea, K.shrink);
            sure_rej = K.alpha * up_b < dc;
            unsure = !sure_rej && !(K.alpha * lo_b >= dc);
        }
        bool reject = __ballot(sure_rej) != 0;
        uint64_t um = __ballot(unsure);
        // undecided kept points, eight per pass (a uniform loop)
        while (!reject && um) {
            uint32_t pick = NONE;
            uint64_t mm = um;
            for (int q = 0; q <= g8 && mm; ++q) {
                const uint32_t f = (uint32_t)__builtin_ctzll(mm);
                mm &= mm - 1;
                if (q == g8)
                    pick = f;
            }
            for (int q = 0; q < 8 && um; ++q)
                um &= um - 1;
            const bool valid = pick != NONE;
            const uint32_t piv = valid ? sm.kept[pick] : t;
            const float dij = l2_ref_8lane(X + (size_t)piv * K.d, X + (size_t)t * K.d, K.d, sub);
            reject = __ballot(valid && sub == 0 && K.alpha * dij < dc) != 0;
        }
        if (!reject) {
            if (lane == 0) {
                sm.kept[na] = t;
                sm.kpos[na] = c;
            }
            ++na;
            __syncthreads();
        }
    }
    uint32_t *row = K.graph + r * (K.final_degree + 1);
    if (lane == 0)
        row[0] = na;
    for (uint32_t j = (uint32_t)lane; j < K.final_degree; j += 64)
        row[1 + j] = j < na ? sm.kept[j] : s;
}

// MFMA fragment layout probe: D = A(32x2) * B(2x32) for a known A, B.
__global__ void ung_mfma_probe_kernel(float *out)
{
    const int lane = threadIdx.x;
    const int r = lane & 31, h = lane >> 5;
    // A[m][k] = (m - 16) + (k % 8) / 4 ; B[k][n] = (k % 4 + 1) * (n - 7): exact in bf16,
    // products and sums exact in fp32.  Lane (r, h) feeds k = 8h + j of row/column r.
    bf16x8 a, b;
    for (int j = 0; j < 8; ++j) {
        const int kk = 8 * h + j;
        a[j] = (__bf16)((float)(r - 16) + 0.25f * (float)(kk % 8));
        b[j] = (__bf16)((float)(kk % 4 + 1) * (float)(r - 7));
    }
    floatx16 acc;
    for (int i = 0; i < 16; ++i)
        acc[i] = 0.0f;
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
    for (int i = 0; i < 16; ++i) {
        const int row = 8 * (i >> 2) + 4 * h + (i & 3);
        out[row * 32 + r] = acc[i];
    }
}

} // namespace
