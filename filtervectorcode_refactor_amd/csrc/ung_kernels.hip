// ung_kernels.hip -- gfx950 (MI355X) kernels and device-side C ABI of the UNG
// cross-edge / mid-group kNN build stage.
//
// Path (one call = one "job list"):
//   select  : fused fp32 MFMA distance tiles (v_mfma_f32_32x32x2f32, LDS-staged
//             query/candidate panels) with a per-row register top-LT queue in the
//             epilogue -- no distance matrix ever reaches HBM.  At the end of a
//             work item the queued candidates are re-scored EXACTLY in the
//             reference's summation order and the k best are written as a partial
//             row together with a certified lower bound on every candidate that
//             was not queued.
//   merge   : per result row, merges the partial rows of its candidate splits and
//             certifies that no unqueued candidate can enter the top-k.
//   fallback: rows whose bound does not certify the result are rescanned exactly
//             (rare; counted in ung_hip_stats::fallback_rows).
//
// Reference semantics reproduced: src/uni_nav_graph_cross_edges.cpp:32-57,154-220
// (cross edges), src/uni_nav_graph_special_blocks.cpp:70-111 (intra exact kNN),
// src/distance.cpp:34-91 (distance rounding), src/search_queue.cpp:26-53
// ((dist,id) order), src/tagore_graph_builder.cu:727-794 (anchor packing).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "ung_hip.h"
#include "ung_internal.h"

using ung::set_error;
using ung::clear_error;

namespace {

constexpr int BQ = 128;          // queries per work item (columns of the MFMA tiles)
constexpr int BC = 128;          // candidates per tile (rows of the MFMA tiles)
constexpr int KC = 32;           // k-chunk staged in LDS
constexpr int LDSW = KC + 4;     // padded LDS row stride (floats)
constexpr int NTHREADS = 256;    // 4 waves: 2 (candidate halves) x 2 (query halves)
constexpr uint32_t SPLIT_V = 16384; // max candidates per work item (load balance)
constexpr uint32_t MERGE_Q = 256;   // rows per merge block
constexpr uint32_t NONE = 0xFFFFFFFFu;

struct Job {
    uint32_t q_begin, q_count;     // queries: global ids [q_begin, q_begin+q_count)
    uint32_t seg_begin, seg_count; // candidate segments (seg_start/seg_vend)
    uint32_t n_cand, n_split;      // virtual candidate count U, number of splits S
    uint32_t part_base;            // partial row of (split s, query j) = part_base + s*q_count + j
    uint32_t out_row;              // result row of query 0
    uint32_t id_base;              // subtracted from result ids (group begin for local ids)
    uint32_t flags;                // bit 0: exclude the query itself
};

struct Item {
    uint32_t job, q_off, q_cnt, v_begin, v_end, split, pad0, pad1;
};

struct MergeItem {
    uint32_t job, q_off, q_cnt, pad;
};

typedef float floatx16 __attribute__((ext_vector_type(16)));

struct SelectParams {
    const float *X;
    const float *xn;
    uint32_t d;
    uint32_t k;
    const Job *jobs;
    const Item *items;
    const uint32_t *seg_start;
    const uint32_t *seg_vend;
    uint32_t *part_ids;
    float *part_dist;
    float *part_bound;
    double eps_coef;  // 2*(d+4)*2^-24 : expansion-form error factor on (|q|+R)^2
    double shrink;    // (d/8+8)*2^-24 : relative error of the reference summation
    double rmax;      // max candidate norm (slightly inflated)
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
    return da < db || (da == db && ia < ib);
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
    for (uint32_t blk = 0; blk < nb8; ++blk) {
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

// Same value computed by one lane alone (fallback path).
__device__ __forceinline__ float l2_ref_lane(const float *__restrict__ a,
                                             const float *__restrict__ b, uint32_t d)
{
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint32_t p = 0;
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

template <int LT>
__device__ __forceinline__ void list_insert(float (&ld)[LT], uint32_t (&li)[LT], float nd,
                                            uint32_t ni)
{
#pragma unroll
    for (int j = 0; j < LT; ++j) {
        const bool sw = nd < ld[j];
        const float td = ld[j];
        const uint32_t ti = li[j];
        ld[j] = sw ? nd : td;
        li[j] = sw ? ni : ti;
        nd = sw ? td : nd;
        ni = sw ? ti : ni;
    }
}

// Lower bound on the exact (reference-rounded) distance of any candidate whose
// expansion-form MFMA distance is >= A:
//   |a - D| <= eps_coef * (|q| + R)^2   (norm cache, MFMA dot, epilogue roundings)
//   e >= D * (1 - shrink)               (reference summation)
// Rounded toward -inf when narrowed to fp32.
__device__ __forceinline__ float lower_bound_exact(float A, float qn, const SelectParams &P)
{
    if (!(A < INFINITY))
        return INFINITY;
    const double qnorm = sqrt((double)fmaxf(qn, 0.0f) * (1.0 + 1e-6));
    const double r = qnorm + P.rmax;
    const double ea = P.eps_coef * r * r;
    double b = ((double)A - ea);
    b = b > 0.0 ? b * (1.0 - P.shrink) : b * (1.0 + P.shrink);
    b -= 1e-30;
    return __double2float_rd(b);
}

// ---------------------------------------------------------------------------
// select kernel
// ---------------------------------------------------------------------------
struct SelectSmem {
    union {
        struct {
            float qs[2][BQ][LDSW];
            float xs[2][BC][LDSW];
        } p;
        struct {
            float ed[64][129];   // entry distances (approx, then exact); stride padded
            uint32_t ei[64][129];
            float alist[64][4];  // LT-th approx of each queue (+inf when not full)
        } r;
    } u;
    uint32_t rowid[BC];
    float xnr[BC];
    float qn[BQ];
};

template <int LT, bool VEC4>
__global__ __launch_bounds__(NTHREADS, (LT <= 16 ? 2 : 1)) void ung_select_kernel(SelectParams P)
{
    __shared__ SelectSmem sm;
    const Item it = P.items[blockIdx.x];
    const Job jb = P.jobs[it.job];
    const uint32_t d = P.d;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int r = lane & 31, h = lane >> 5;
    const uint32_t q0 = jb.q_begin + it.q_off;
    const uint32_t qcnt = it.q_cnt;
    const bool excl = (jb.flags & 1u) != 0;
    const float *__restrict__ X = P.X;

    if (tid < BQ)
        sm.qn[tid] = (uint32_t)tid < qcnt ? P.xn[q0 + tid] : 0.0f;

    float ld[2][LT];
    uint32_t li[2][LT];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int j = 0; j < LT; ++j) {
            ld[nb][j] = INFINITY;
            li[nb][j] = NONE;
        }

    // loader mapping: rows lr = (tid>>3) + 32m, columns c4 .. c4+3 of the chunk
    const int lr0 = tid >> 3;
    const int c4 = (tid & 7) * 4;
    const float *qrow[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        uint32_t ql = (uint32_t)(lr0 + 32 * m);
        ql = ql < qcnt ? ql : qcnt - 1;
        qrow[m] = X + (size_t)(q0 + ql) * d;
    }

    __syncthreads();
    uint32_t qid[2];
    float qnv[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const int ql = wn * 64 + nb * 32 + r;
        qid[nb] = q0 + (uint32_t)ql;
        qnv[nb] = sm.qn[ql];
    }

    for (uint32_t v0 = it.v_begin; v0 < it.v_end; v0 += BC) {
        __syncthreads(); // previous epilogue done with rowid / panels
        if (tid < BC) {
            const uint32_t v = v0 + (uint32_t)tid;
            uint32_t g = NONE;
            float nx = 0.0f;
            if (v < it.v_end) {
                g = cand_id(P.seg_start, P.seg_vend, jb.seg_begin, jb.seg_count, v);
                nx = P.xn[g];
            }
            sm.rowid[tid] = g;
            sm.xnr[tid] = nx;
        }
        __syncthreads();
        const float *xrow[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            uint32_t g = sm.rowid[lr0 + 32 * m];
            g = (g == NONE) ? sm.rowid[0] : g;
            xrow[m] = X + (size_t)g * d;
        }

        floatx16 acc[2][2];
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    acc[a][b][i] = 0.0f;

        float4 rq[4], rx[4];
        auto load_chunk = [&](uint32_t kc) {
            const uint32_t col = kc + (uint32_t)c4;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                if (VEC4) {
                    if (col < d) {
                        rq[m] = *reinterpret_cast<const float4 *>(qrow[m] + col);
                        rx[m] = *reinterpret_cast<const float4 *>(xrow[m] + col);
                    } else {
                        rq[m] = make_float4(0.f, 0.f, 0.f, 0.f);
                        rx[m] = make_float4(0.f, 0.f, 0.f, 0.f);
                    }
                } else {
                    float tq[4], tx[4];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const bool ok = col + t < d;
                        tq[t] = ok ? qrow[m][col + t] : 0.0f;
                        tx[t] = ok ? xrow[m][col + t] : 0.0f;
                    }
                    rq[m] = make_float4(tq[0], tq[1], tq[2], tq[3]);
                    rx[m] = make_float4(tx[0], tx[1], tx[2], tx[3]);
                }
            }
        };

        load_chunk(0);
        int buf = 0;
        for (uint32_t kc = 0; kc < d; kc += KC, buf ^= 1) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                *reinterpret_cast<float4 *>(&sm.u.p.qs[buf][lr0 + 32 * m][c4]) = rq[m];
                *reinterpret_cast<float4 *>(&sm.u.p.xs[buf][lr0 + 32 * m][c4]) = rx[m];
            }
            __syncthreads();
            if (kc + KC < d)
                load_chunk(kc + KC);
            // 16 MFMA k-steps: step t covers dims kc+t (lanes h=0) and kc+16+t (h=1)
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const int kk = h * 16 + s4 * 4;
                const float4 a0 = *reinterpret_cast<const float4 *>(&sm.u.p.xs[buf][wm * 64 + r][kk]);
                const float4 a1 = *reinterpret_cast<const float4 *>(&sm.u.p.xs[buf][wm * 64 + 32 + r][kk]);
                const float4 b0 = *reinterpret_cast<const float4 *>(&sm.u.p.qs[buf][wn * 64 + r][kk]);
                const float4 b1 = *reinterpret_cast<const float4 *>(&sm.u.p.qs[buf][wn * 64 + 32 + r][kk]);
                const float av0[4] = {a0.x, a0.y, a0.z, a0.w};
                const float av1[4] = {a1.x, a1.y, a1.z, a1.w};
                const float bv0[4] = {b0.x, b0.y, b0.z, b0.w};
                const float bv1[4] = {b1.x, b1.y, b1.z, b1.w};
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(av0[c], bv0[c], acc[0][0], 0, 0, 0);
                    acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(av0[c], bv1[c], acc[0][1], 0, 0, 0);
                    acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(av1[c], bv0[c], acc[1][0], 0, 0, 0);
                    acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(av1[c], bv1[c], acc[1][1], 0, 0, 0);
                }
            }
        }

        // epilogue: acc[mb][nb][i] = <x_row, q_col>, row = wm*64+mb*32+8*(i/4)+4*h+(i%4),
        // col = wn*64+nb*32+r
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int row = wm * 64 + mb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
                    const uint32_t g = sm.rowid[row];
                    float dd = __builtin_fmaf(-2.0f, acc[mb][nb][i], qnv[nb] + sm.xnr[row]);
                    const bool valid = (g != NONE) && !(excl && g == qid[nb]);
                    dd = valid ? dd : INFINITY;
                    const bool p = dd < ld[nb][LT - 1];
                    if (__ballot(p)) {
                        if (p)
                            list_insert<LT>(ld[nb], li[nb], dd, g);
                    }
                }
            }
        }
    }

    // ---- exact re-score of the queued candidates, two passes of 64 queries ----
    constexpr int E = 4 * LT;
    const int sub = tid & 7;
    const int grp = tid >> 3; // 32 groups of 8 lanes
    for (int pass = 0; pass < 2; ++pass) {
        __syncthreads();
        if (wn == pass) {
            const int lid = wm * 2 + h;
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                const int jl = nb * 32 + r;
#pragma unroll
                for (int j = 0; j < LT; ++j) {
                    sm.u.r.ed[jl][lid * LT + j] = ld[nb][j];
                    sm.u.r.ei[jl][lid * LT + j] = li[nb][j];
                }
                sm.u.r.alist[jl][lid] = ld[nb][LT - 1];
            }
        }
        __syncthreads();
        for (int p = grp; p < 64 * E; p += 32) {
            const int jl = p / E, e = p % E;
            const uint32_t ql = (uint32_t)(pass * 64 + jl);
            const uint32_t id = sm.u.r.ei[jl][e];
            const bool ok = id != NONE && ql < qcnt;
            const float *a = X + (size_t)(q0 + (ql < qcnt ? ql : 0u)) * d;
            const float *b = X + (size_t)(ok ? id : q0) * d;
            const float ex = l2_ref_8lane(a, b, d, sub);
            if (sub == 0)
                sm.u.r.ed[jl][e] = ok ? ex : INFINITY;
        }
        __syncthreads();
        // rank of every entry under (exact, id, slot); the k best go to the partial row
        for (int p = tid; p < 64 * E; p += NTHREADS) {
            const int jl = p / E, e = p % E;
            const uint32_t ql = (uint32_t)(pass * 64 + jl);
            if (ql >= qcnt)
                continue;
            const float de = sm.u.r.ed[jl][e];
            const uint32_t ie = sm.u.r.ei[jl][e];
            int rank = 0;
            for (int f = 0; f < E; ++f) {
                const float df = sm.u.r.ed[jl][f];
                const uint32_t idf = sm.u.r.ei[jl][f];
                rank += (df < de || (df == de && (idf < ie || (idf == ie && f < e)))) ? 1 : 0;
            }
            const uint32_t prow = jb.part_base + it.split * jb.q_count + it.q_off + ql;
            if ((uint32_t)rank < P.k) {
                const bool real = ie != NONE && de < INFINITY;
                P.part_ids[(size_t)prow * P.k + rank] = real ? ie : NONE;
                P.part_dist[(size_t)prow * P.k + rank] = real ? de : INFINITY;
            }
            if (e == 0) {
                float A = sm.u.r.alist[jl][0];
#pragma unroll
                for (int l = 1; l < 4; ++l)
                    A = fminf(A, sm.u.r.alist[jl][l]);
                P.part_bound[prow] = lower_bound_exact(A, sm.qn[ql], P);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// merge + certification
// ---------------------------------------------------------------------------
struct MergeParams {
    const Job *jobs;
    const MergeItem *mitems;
    const uint32_t *part_ids;
    const float *part_dist;
    const float *part_bound;
    uint32_t k;
    uint32_t *out_ids;
    float *out_dist;
    int32_t *out_size;
    uint32_t *flag_count;
    uint2 *flagged;
};

template <int KM>
__global__ __launch_bounds__(MERGE_Q) void ung_merge_kernel(MergeParams M)
{
    const MergeItem mi = M.mitems[blockIdx.x];
    if (threadIdx.x >= mi.q_cnt)
        return;
    const Job jb = M.jobs[mi.job];
    const uint32_t ql = mi.q_off + threadIdx.x;
    const uint32_t k = M.k;
    float bd[KM];
    uint32_t bi[KM];
#pragma unroll
    for (int j = 0; j < KM; ++j) {
        bd[j] = INFINITY;
        bi[j] = NONE;
    }
    float bmin = INFINITY;
    for (uint32_t s = 0; s < jb.n_split; ++s) {
        const size_t prow = (size_t)jb.part_base + (size_t)s * jb.q_count + ql;
        bmin = fminf(bmin, M.part_bound[prow]);
        for (uint32_t j = 0; j < k; ++j) {
            const uint32_t id = M.part_ids[prow * k + j];
            if (id == NONE)
                break;
            float nd = M.part_dist[prow * k + j];
            uint32_t ni = id;
            // (dist,id)-ordered insertion into the running top-KM
#pragma unroll
            for (int t = 0; t < KM; ++t) {
                const bool sw = cand_less(nd, ni, bd[t], bi[t]);
                const float td = bd[t];
                const uint32_t ti = bi[t];
                bd[t] = sw ? nd : td;
                bi[t] = sw ? ni : ti;
                nd = sw ? td : nd;
                ni = sw ? ti : ni;
            }
        }
    }
    uint32_t count = 0;
#pragma unroll
    for (int t = 0; t < KM; ++t)
        count += ((uint32_t)t < k && bi[t] != NONE) ? 1u : 0u;
    float T = INFINITY;
#pragma unroll
    for (int t = 0; t < KM; ++t)
        if ((uint32_t)t == k - 1)
            T = bd[t];
    const bool certified = (count < k) ? !(bmin < INFINITY) : (T < bmin);
    const size_t orow = (size_t)jb.out_row + ql;
    if (!certified) {
        const uint32_t slot = atomicAdd(M.flag_count, 1u);
        M.flagged[slot] = make_uint2(mi.job, ql);
        return;
    }
#pragma unroll
    for (int t = 0; t < KM; ++t) {
        if ((uint32_t)t < k) {
            const bool ok = bi[t] != NONE;
            M.out_ids[orow * k + t] = ok ? bi[t] - jb.id_base : NONE;
            if (M.out_dist)
                M.out_dist[orow * k + t] = ok ? bd[t] : INFINITY;
        }
    }
    if (M.out_size)
        M.out_size[orow] = (int32_t)count;
}

// ---------------------------------------------------------------------------
// exact fallback: one wave per flagged row, persistent over the flagged list
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
    uint32_t *out_ids;
    float *out_dist;
    int32_t *out_size;
};

__global__ __launch_bounds__(64) void ung_fallback_kernel(FallbackParams F)
{
    __shared__ float sd[64][65];
    __shared__ uint32_t si[64][65];
    const int lane = threadIdx.x;
    const uint32_t total = *F.flag_count;
    const uint32_t k = F.k;
    for (uint32_t f = blockIdx.x; f < total; f += gridDim.x) {
        const uint2 fl = F.flagged[f];
        const Job jb = F.jobs[fl.x];
        const uint32_t q = jb.q_begin + fl.y;
        const bool excl = (jb.flags & 1u) != 0;
        const float *qv = F.X + (size_t)q * F.d;
        int32_t size = 0;
        for (uint32_t v = lane; v < jb.n_cand; v += 64) {
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
__global__ void ung_norm_kernel(const float *__restrict__ X, uint64_t N, uint32_t d,
                                float *__restrict__ xn, unsigned int *__restrict__ maxbits)
{
    // one wave per row; lanes stride the row
    const uint64_t row = (uint64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= N)
        return;
    const float *x = X + row * d;
    float s = 0.0f;
    for (uint32_t t = lane; t < d; t += 64)
        s = __builtin_fmaf(x[t], x[t], s);
    for (int off = 32; off > 0; off >>= 1)
        s += __shfl_xor(s, off);
    if (lane == 0) {
        xn[row] = s;
        atomicMax(maxbits, __float_as_uint(s)); // non-negative floats order as uints
    }
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

// MFMA fragment layout probe: D = A(32x2) * B(2x32) for a known A, B.
__global__ void ung_mfma_probe_kernel(float *out)
{
    const int lane = threadIdx.x;
    const int r = lane & 31, h = lane >> 5;
    // A[m][k] = m + 0.5*k ; B[k][n] = (k+1) * (n - 7)
    const float a = (float)r + 0.5f * (float)h;
    const float b = (float)(h + 1) * (float)(r - 7);
    floatx16 acc;
    for (int i = 0; i < 16; ++i)
        acc[i] = 0.0f;
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
    for (int i = 0; i < 16; ++i) {
        const int row = 8 * (i >> 2) + 4 * h + (i & 3);
        out[row * 32 + r] = acc[i];
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
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
        hipError_t e = hipMalloc((void **)&p, want * sizeof(T));
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

struct Plan {
    std::vector<Job> jobs;
    std::vector<Item> items;
    std::vector<MergeItem> mitems;
    std::vector<uint32_t> seg_start, seg_vend;
    uint64_t part_rows = 0;
    uint64_t pairs = 0;
    uint64_t padded = 0;
    uint64_t rows = 0;
};

struct ResultBufs {
    DevBuf<uint32_t> ids;
    DevBuf<float> dist;
    DevBuf<int32_t> size;
    uint64_t rows = 0;
    uint32_t k = 0;
    bool valid = false;
    void release()
    {
        ids.release();
        dist.release();
        size.release();
        rows = 0;
        valid = false;
    }
};

} // namespace

struct ung_hip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev[8] = {};
    // resident base set
    float *X = nullptr;
    float *xn = nullptr;
    unsigned int *maxbits = nullptr;
    uint64_t N = 0;
    uint32_t d = 0;
    double rmax = 0.0;
    // work lists / scratch
    DevBuf<Job> jobs;
    DevBuf<Item> items;
    DevBuf<MergeItem> mitems;
    DevBuf<uint32_t> seg_start, seg_vend;
    DevBuf<uint32_t> part_ids;
    DevBuf<float> part_dist;
    DevBuf<float> part_bound;
    DevBuf<uint32_t> flag_count;
    DevBuf<uint2> flagged;
    // results
    ResultBufs cross;
    ResultBufs group;
    // last group plan (for packing)
    std::vector<Job> group_jobs;
    std::vector<MergeItem> group_mitems;
    DevBuf<Job> gjobs;
    DevBuf<MergeItem> gmitems;
    uint32_t group_list_k = 0;
    DevBuf<uint32_t> graph;
};

namespace {

int set_device(ung_hip_ctx *ctx)
{
    HIPCHECK(hipSetDevice(ctx->device));
    return UNG_HIP_OK;
}

void add_items_for_job(Plan &pl, uint32_t job_index)
{
    const Job &jb = pl.jobs[job_index];
    for (uint32_t qo = 0; qo < jb.q_count; qo += BQ) {
        const uint32_t qc = std::min<uint32_t>(BQ, jb.q_count - qo);
        for (uint32_t s = 0; s < jb.n_split; ++s) {
            Item it{};
            it.job = job_index;
            it.q_off = qo;
            it.q_cnt = qc;
            it.v_begin = s * SPLIT_V;
            it.v_end = std::min<uint32_t>(jb.n_cand, (s + 1) * SPLIT_V);
            it.split = s;
            pl.items.push_back(it);
            pl.padded += (uint64_t)BQ * (uint64_t)(((it.v_end - it.v_begin) + BC - 1) / BC * BC);
        }
    }
    for (uint32_t qo = 0; qo < jb.q_count; qo += MERGE_Q) {
        MergeItem mi{};
        mi.job = job_index;
        mi.q_off = qo;
        mi.q_cnt = std::min<uint32_t>(MERGE_Q, jb.q_count - qo);
        pl.mitems.push_back(mi);
    }
}

int pick_lt(uint32_t k)
{
    if (k <= 16)
        return 8;
    if (k <= 32)
        return 16;
    return 32;
}

template <int LT>
int launch_select_t(ung_hip_ctx *ctx, const SelectParams &P, uint32_t n_items)
{
    const bool vec4 = (ctx->d % 4) == 0;
    // grid dimension x is limited to 2^31-1; chunk the item list
    const uint32_t max_grid = 1u << 30;
    for (uint32_t off = 0; off < n_items; off += max_grid) {
        SelectParams Q = P;
        Q.items = P.items + off;
        const uint32_t n = std::min(max_grid, n_items - off);
        if (vec4)
            hipLaunchKernelGGL((ung_select_kernel<LT, true>), dim3(n), dim3(NTHREADS), 0, ctx->stream, Q);
        else
            hipLaunchKernelGGL((ung_select_kernel<LT, false>), dim3(n), dim3(NTHREADS), 0, ctx->stream, Q);
        HIPCHECK(hipGetLastError());
    }
    return UNG_HIP_OK;
}

template <int KM>
int launch_merge_t(ung_hip_ctx *ctx, const MergeParams &M, uint32_t n)
{
    hipLaunchKernelGGL((ung_merge_kernel<KM>), dim3(n), dim3(MERGE_Q), 0, ctx->stream, M);
    HIPCHECK(hipGetLastError());
    return UNG_HIP_OK;
}

// Runs a planned job list; results into `res` (rows x k), rows of res already
// initialised by the caller when some rows have no job.
int run_plan(ung_hip_ctx *ctx, const Plan &pl, uint32_t k, ResultBufs &res, ung_hip_stats *st)
{
    int rc;
    const auto t_h2d = clk::now();
    if ((rc = ctx->jobs.ensure(pl.jobs.size())) || (rc = ctx->items.ensure(pl.items.size())) ||
        (rc = ctx->mitems.ensure(pl.mitems.size())) || (rc = ctx->seg_start.ensure(pl.seg_start.size())) ||
        (rc = ctx->seg_vend.ensure(pl.seg_vend.size())) ||
        (rc = ctx->part_ids.ensure(pl.part_rows * k)) || (rc = ctx->part_dist.ensure(pl.part_rows * k)) ||
        (rc = ctx->part_bound.ensure(pl.part_rows)) || (rc = ctx->flag_count.ensure(1)) ||
        (rc = ctx->flagged.ensure(std::max<uint64_t>(pl.rows, 1))))
        return rc;
    if (!pl.jobs.empty()) {
        HIPCHECK(hipMemcpyAsync(ctx->jobs.p, pl.jobs.data(), pl.jobs.size() * sizeof(Job), hipMemcpyHostToDevice, ctx->stream));
        HIPCHECK(hipMemcpyAsync(ctx->items.p, pl.items.data(), pl.items.size() * sizeof(Item), hipMemcpyHostToDevice, ctx->stream));
        HIPCHECK(hipMemcpyAsync(ctx->mitems.p, pl.mitems.data(), pl.mitems.size() * sizeof(MergeItem), hipMemcpyHostToDevice, ctx->stream));
        HIPCHECK(hipMemcpyAsync(ctx->seg_start.p, pl.seg_start.data(), pl.seg_start.size() * sizeof(uint32_t), hipMemcpyHostToDevice, ctx->stream));
        HIPCHECK(hipMemcpyAsync(ctx->seg_vend.p, pl.seg_vend.data(), pl.seg_vend.size() * sizeof(uint32_t), hipMemcpyHostToDevice, ctx->stream));
    }
    HIPCHECK(hipStreamSynchronize(ctx->stream));
    if (st)
        st->h2d_ms += ms_since(t_h2d);
    if (pl.jobs.empty())
        return UNG_HIP_OK;

    hipLaunchKernelGGL(ung_zero_u32_kernel, dim3(1), dim3(64), 0, ctx->stream, ctx->flag_count.p, 1u);
    HIPCHECK(hipGetLastError());
    HIPCHECK(hipEventRecord(ctx->ev[0], ctx->stream));

    SelectParams P{};
    P.X = ctx->X;
    P.xn = ctx->xn;
    P.d = ctx->d;
    P.k = k;
    P.jobs = ctx->jobs.p;
    P.items = ctx->items.p;
    P.seg_start = ctx->seg_start.p;
    P.seg_vend = ctx->seg_vend.p;
    P.part_ids = ctx->part_ids.p;
    P.part_dist = ctx->part_dist.p;
    P.part_bound = ctx->part_bound.p;
    P.eps_coef = 2.0 * ((double)ctx->d + 4.0) * std::ldexp(1.0, -24);
    P.shrink = ((double)ctx->d / 8.0 + 8.0) * std::ldexp(1.0, -24);
    P.rmax = ctx->rmax;
    const int lt = pick_lt(k);
    const uint32_t n_items = (uint32_t)pl.items.size();
    if (lt == 8)
        rc = launch_select_t<8>(ctx, P, n_items);
    else if (lt == 16)
        rc = launch_select_t<16>(ctx, P, n_items);
    else
        rc = launch_select_t<32>(ctx, P, n_items);
    if (rc)
        return rc;
    HIPCHECK(hipEventRecord(ctx->ev[1], ctx->stream));

    MergeParams M{};
    M.jobs = ctx->jobs.p;
    M.mitems = ctx->mitems.p;
    M.part_ids = ctx->part_ids.p;
    M.part_dist = ctx->part_dist.p;
    M.part_bound = ctx->part_bound.p;
    M.k = k;
    M.out_ids = res.ids.p;
    M.out_dist = res.dist.p;
    M.out_size = res.size.p;
    M.flag_count = ctx->flag_count.p;
    M.flagged = ctx->flagged.p;
    const uint32_t n_m = (uint32_t)pl.mitems.size();
    if (k <= 8)
        rc = launch_merge_t<8>(ctx, M, n_m);
    else if (k <= 16)
        rc = launch_merge_t<16>(ctx, M, n_m);
    else if (k <= 32)
        rc = launch_merge_t<32>(ctx, M, n_m);
    else
        rc = launch_merge_t<64>(ctx, M, n_m);
    if (rc)
        return rc;
    HIPCHECK(hipEventRecord(ctx->ev[2], ctx->stream));

    FallbackParams F{};
    F.X = ctx->X;
    F.d = ctx->d;
    F.k = k;
    F.jobs = ctx->jobs.p;
    F.seg_start = ctx->seg_start.p;
    F.seg_vend = ctx->seg_vend.p;
    F.flag_count = ctx->flag_count.p;
    F.flagged = ctx->flagged.p;
    F.out_ids = res.ids.p;
    F.out_dist = res.dist.p;
    F.out_size = res.size.p;
    hipLaunchKernelGGL(ung_fallback_kernel, dim3(512), dim3(64), 0, ctx->stream, F);
    HIPCHECK(hipGetLastError());
    HIPCHECK(hipEventRecord(ctx->ev[3], ctx->stream));
    HIPCHECK(hipEventSynchronize(ctx->ev[3]));

    uint32_t nflag = 0;
    HIPCHECK(hipMemcpy(&nflag, ctx->flag_count.p, sizeof(uint32_t), hipMemcpyDeviceToHost));
    if (st) {
        float a = 0, b = 0, c = 0;
        HIPCHECK(hipEventElapsedTime(&a, ctx->ev[0], ctx->ev[1]));
        HIPCHECK(hipEventElapsedTime(&b, ctx->ev[1], ctx->ev[2]));
        HIPCHECK(hipEventElapsedTime(&c, ctx->ev[2], ctx->ev[3]));
        st->select_ms += a;
        st->merge_ms += b;
        st->fallback_ms += c;
        st->kernel_ms += a + b + c;
        st->fallback_rows += nflag;
        st->pairs += pl.pairs;
        st->padded_pairs += pl.padded;
        st->rows += pl.rows;
        st->work_items += pl.items.size();
        st->select_launches += 1;
    }
    return UNG_HIP_OK;
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
    for (uint32_t g = 1; g <= G; ++g) {
        if (group_begin[g + 1] < group_begin[g]) {
            set_error("ung_hip_cross_topk: group_begin not monotone at group %u", g);
            return UNG_HIP_EINVAL;
        }
        if (out_ptr[g + 1] < out_ptr[g]) {
            set_error("ung_hip_cross_topk: out_ptr not monotone at group %u", g);
            return UNG_HIP_EINVAL;
        }
    }
    for (uint32_t c = 1; c <= G; ++c) {
        const uint32_t qn = group_begin[c + 1] - group_begin[c];
        if (qn == 0 || out_ptr[c + 1] == out_ptr[c])
            continue;
        Job jb{};
        jb.q_begin = group_begin[c];
        jb.q_count = qn;
        jb.seg_begin = (uint32_t)pl.seg_start.size();
        uint64_t u = 0;
        for (uint32_t e = out_ptr[c]; e < out_ptr[c + 1]; ++e) {
            const uint32_t x = out_idx[e];
            if (x < 1 || x > G) {
                set_error("ung_hip_cross_topk: out_idx entry %u out of range 1..%u", x, G);
                return UNG_HIP_EINVAL;
            }
            const uint32_t nx = group_begin[x + 1] - group_begin[x];
            if (nx == 0)
                continue;
            u += nx;
            if (u >= 0xFFFFFFFFull) {
                set_error("ung_hip_cross_topk: candidate union of group %u exceeds 2^32", c);
                return UNG_HIP_EINVAL;
            }
            pl.seg_start.push_back(group_begin[x]);
            pl.seg_vend.push_back((uint32_t)u);
        }
        if (u == 0)
            continue;
        jb.seg_count = (uint32_t)pl.seg_start.size() - jb.seg_begin;
        jb.n_cand = (uint32_t)u;
        jb.n_split = (uint32_t)((u + SPLIT_V - 1) / SPLIT_V);
        jb.part_base = (uint32_t)pl.part_rows;
        jb.out_row = group_begin[c];
        jb.id_base = 0;
        jb.flags = 0;
        pl.part_rows += (uint64_t)qn * jb.n_split;
        if (pl.part_rows >= 0xFFFFFFFFull) {
            set_error("ung_hip_cross_topk: partial rows exceed 2^32");
            return UNG_HIP_EINVAL;
        }
        pl.pairs += (uint64_t)qn * u;
        pl.rows += qn;
        pl.jobs.push_back(jb);
        add_items_for_job(pl, (uint32_t)pl.jobs.size() - 1);
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
    Plan pl;
    if ((rc = build_cross_plan(ctx, G, group_begin, out_ptr, out_idx, pl)))
        return rc;
    if (st)
        st->plan_ms += ms_since(t0);
    ResultBufs &res = ctx->cross;
    res.valid = false;
    if ((rc = res.ids.ensure(ctx->N * k)) || (rc = res.dist.ensure(ctx->N * k)) || (rc = res.size.ensure(ctx->N)))
        return rc;
    res.rows = ctx->N;
    res.k = k;
    const uint64_t tot = ctx->N * k;
    if (tot > 0) {
        hipLaunchKernelGGL(ung_fill_rows_kernel, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, ctx->stream,
                           res.ids.p, res.dist.p, res.size.p, ctx->N, k);
        HIPCHECK(hipGetLastError());
    }
    if ((rc = run_plan(ctx, pl, k, res, st)))
        return rc;
    HIPCHECK(hipStreamSynchronize(ctx->stream));
    res.valid = true;
    if (st)
        st->wall_ms += ms_since(t0);
    return UNG_HIP_OK;
}

int group_device(ung_hip_ctx *ctx, uint32_t n_groups, const uint32_t *grp_begin, const uint32_t *grp_size,
                 uint32_t list_k, ung_hip_stats *st)
{
    int rc;
    if ((rc = check_ready(ctx)))
        return rc;
    if (list_k < 1 || list_k > 64) {
        set_error("list_k=%u outside 1..64", list_k);
        return UNG_HIP_EINVAL;
    }
    if (n_groups > 0 && (!grp_begin || !grp_size)) {
        set_error("ung_hip_group_knn: null grp_begin/grp_size");
        return UNG_HIP_EINVAL;
    }
    if ((rc = set_device(ctx)))
        return rc;
    const auto t0 = clk::now();
    Plan pl;
    uint64_t row = 0;
    for (uint32_t g = 0; g < n_groups; ++g) {
        const uint32_t n = grp_size[g];
        if (n == 0 || n > 65536 || (uint64_t)grp_begin[g] + n > ctx->N) {
            set_error("ung_hip_group_knn: group %u (begin %u, size %u) invalid for N=%llu (need 1<=n<=65536)", g,
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
        jb.n_split = (n + SPLIT_V - 1) / SPLIT_V;
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
    if (st)
        st->plan_ms += ms_since(t0);
    ResultBufs &res = ctx->group;
    res.valid = false;
    if ((rc = res.ids.ensure(std::max<uint64_t>(row * list_k, 1))) ||
        (rc = res.dist.ensure(std::max<uint64_t>(row * list_k, 1))) || (rc = res.size.ensure(std::max<uint64_t>(row, 1))))
        return rc;
    res.rows = row;
    res.k = list_k;
    if ((rc = run_plan(ctx, pl, list_k, res, st)))
        return rc;
    // keep the job table for packing
    ctx->group_jobs = pl.jobs;
    ctx->group_mitems = pl.mitems;
    ctx->group_list_k = list_k;
    if (!pl.jobs.empty()) {
        if ((rc = ctx->gjobs.ensure(pl.jobs.size())) || (rc = ctx->gmitems.ensure(pl.mitems.size())))
            return rc;
        HIPCHECK(hipMemcpyAsync(ctx->gjobs.p, pl.jobs.data(), pl.jobs.size() * sizeof(Job), hipMemcpyHostToDevice, ctx->stream));
        HIPCHECK(hipMemcpyAsync(ctx->gmitems.p, pl.mitems.data(), pl.mitems.size() * sizeof(MergeItem), hipMemcpyHostToDevice, ctx->stream));
    }
    HIPCHECK(hipStreamSynchronize(ctx->stream));
    res.valid = true;
    if (st)
        st->wall_ms += ms_since(t0);
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
    if (n) {
        HIPCHECK(hipMemcpyAsync(ids, res.ids.p, n * sizeof(uint32_t), hipMemcpyDeviceToHost, ctx->stream));
        if (dist)
            HIPCHECK(hipMemcpyAsync(dist, res.dist.p, n * sizeof(float), hipMemcpyDeviceToHost, ctx->stream));
        if (size)
            HIPCHECK(hipMemcpyAsync(size, res.size.p, res.rows * sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
    }
    HIPCHECK(hipStreamSynchronize(ctx->stream));
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
    if ((rc = set_device(ctx)))
        return rc;
    ung_hip_release_vectors(ctx);
    const auto t0 = clk::now();
    HIPCHECK(hipMalloc((void **)&ctx->X, N * dim * sizeof(float)));
    HIPCHECK(hipMalloc((void **)&ctx->xn, N * sizeof(float)));
    HIPCHECK(hipMalloc((void **)&ctx->maxbits, sizeof(unsigned int)));
    HIPCHECK(hipMemcpyAsync(ctx->X, src, N * dim * sizeof(float),
                            src_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, ctx->stream));
    hipLaunchKernelGGL(ung_zero_u32_kernel, dim3(1), dim3(64), 0, ctx->stream, (uint32_t *)ctx->maxbits, 1u);
    HIPCHECK(hipGetLastError());
    HIPCHECK(hipStreamSynchronize(ctx->stream));
    const double h2d = ms_since(t0);
    HIPCHECK(hipEventRecord(ctx->ev[4], ctx->stream));
    const uint32_t rows_per_block = 4;
    hipLaunchKernelGGL(ung_norm_kernel, dim3((unsigned)((N + rows_per_block - 1) / rows_per_block)), dim3(64 * rows_per_block),
                       0, ctx->stream, ctx->X, N, dim, ctx->xn, ctx->maxbits);
    HIPCHECK(hipGetLastError());
    HIPCHECK(hipEventRecord(ctx->ev[5], ctx->stream));
    unsigned int mb = 0;
    HIPCHECK(hipMemcpyAsync(&mb, ctx->maxbits, sizeof(mb), hipMemcpyDeviceToHost, ctx->stream));
    HIPCHECK(hipStreamSynchronize(ctx->stream));
    float mxf;
    std::memcpy(&mxf, &mb, sizeof(mxf));
    ctx->N = N;
    ctx->d = dim;
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
extern "C" {

const char *ung_hip_version(void) { return "ung_hip 0.1 (gfx950, fp32 MFMA select + exact re-rank)"; }

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
    hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        set_error("hipStreamCreateWithFlags failed: %s", hipGetErrorString(e));
        delete ctx;
        return UNG_HIP_EDEVICE;
    }
    for (auto &ev : ctx->ev) {
        e = hipEventCreate(&ev);
        if (e != hipSuccess) {
            set_error("hipEventCreate failed: %s", hipGetErrorString(e));
            ung_hip_destroy(ctx);
            return UNG_HIP_EDEVICE;
        }
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
    (void)hipSetDevice(ctx->device);
    if (ctx->stream)
        (void)hipStreamSynchronize(ctx->stream);
    if (ctx->X)
        (void)hipFree(ctx->X);
    if (ctx->xn)
        (void)hipFree(ctx->xn);
    if (ctx->maxbits)
        (void)hipFree(ctx->maxbits);
    ctx->X = nullptr;
    ctx->xn = nullptr;
    ctx->maxbits = nullptr;
    ctx->N = 0;
    ctx->d = 0;
    ctx->cross.valid = false;
    ctx->group.valid = false;
    return UNG_HIP_OK;
}

int ung_hip_destroy(ung_hip_ctx *ctx)
{
    clear_error();
    if (!ctx)
        return UNG_HIP_OK;
    ung_hip_release_vectors(ctx);
    ctx->jobs.release();
    ctx->items.release();
    ctx->mitems.release();
    ctx->seg_start.release();
    ctx->seg_vend.release();
    ctx->part_ids.release();
    ctx->part_dist.release();
    ctx->part_bound.release();
    ctx->flag_count.release();
    ctx->flagged.release();
    ctx->cross.release();
    ctx->group.release();
    ctx->gjobs.release();
    ctx->gmitems.release();
    ctx->graph.release();
    for (auto &ev : ctx->ev)
        if (ev)
            (void)hipEventDestroy(ev);
    if (ctx->stream)
        (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return UNG_HIP_OK;
}

int ung_hip_prepare_vectors(ung_hip_ctx *ctx, const float *X, uint64_t N, uint32_t dim, ung_hip_stats *st)
{
    clear_error();
    return prepare_common(ctx, X, false, N, dim, st);
}

int ung_hip_prepare_vectors_device(ung_hip_ctx *ctx, const float *X_dev, uint64_t N, uint32_t dim,
                                   ung_hip_stats *st)
{
    clear_error();
    return prepare_common(ctx, X_dev, true, N, dim, st);
}

int ung_hip_cross_topk_device(ung_hip_ctx *ctx, uint32_t G, const uint32_t *group_begin, const uint32_t *out_ptr,
                              const uint32_t *out_idx, uint32_t k, ung_hip_stats *st)
{
    clear_error();
    return cross_device(ctx, G, group_begin, out_ptr, out_idx, k, st);
}

int ung_hip_cross_topk(ung_hip_ctx *ctx, uint32_t G, const uint32_t *group_begin, const uint32_t *out_ptr,
                       const uint32_t *out_idx, uint32_t k, uint32_t *out_ids, float *out_dist,
                       int32_t *out_size, ung_hip_stats *st)
{
    clear_error();
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
    if (!ctx) {
        set_error("null context");
        return UNG_HIP_EINVAL;
    }
    return download(ctx, ctx->cross, out_ids, out_dist, out_size, st);
}

int ung_hip_group_knn_device(ung_hip_ctx *ctx, uint32_t n_groups, const uint32_t *grp_begin,
                             const uint32_t *grp_size, uint32_t list_k, ung_hip_stats *st)
{
    clear_error();
    return group_device(ctx, n_groups, grp_begin, grp_size, list_k, st);
}

int ung_hip_group_knn(ung_hip_ctx *ctx, uint32_t n_groups, const uint32_t *grp_begin, const uint32_t *grp_size,
                      uint32_t list_k, uint32_t *out_ids, float *out_dist, ung_hip_stats *st)
{
    clear_error();
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

int ung_hip_download_group(ung_hip_ctx *ctx, uint32_t *out_ids, float *out_dist, ung_hip_stats *st)
{
    clear_error();
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
    if (!ctx->group_mitems.empty()) {
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
        hipLaunchKernelGGL(ung_pack_kernel, dim3((unsigned)ctx->group_mitems.size()), dim3(MERGE_Q), 0, ctx->stream, K);
        HIPCHECK(hipGetLastError());
        HIPCHECK(hipEventRecord(ctx->ev[7], ctx->stream));
    }
    const auto t1 = clk::now();
    if (rows)
        HIPCHECK(hipMemcpyAsync(out_graph, ctx->graph.p, rows * stride * sizeof(uint32_t), hipMemcpyDeviceToHost, ctx->stream));
    HIPCHECK(hipStreamSynchronize(ctx->stream));
    if (entry_points)
        std::memset(entry_points, 0, ctx->group_jobs.size() * sizeof(uint32_t));
    if (st) {
        float kms = 0;
        if (!ctx->group_mitems.empty())
            HIPCHECK(hipEventElapsedTime(&kms, ctx->ev[6], ctx->ev[7]));
        st->kernel_ms += kms;
        st->d2h_ms += ms_since(t1);
        st->wall_ms += ms_since(t0);
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
    HIPCHECK(hipMalloc((void **)&d_out, 32 * 32 * sizeof(float)));
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
            for (int kk = 0; kk < 2; ++kk)
                ref += ((double)m + 0.5 * kk) * ((double)(kk + 1) * (double)(n - 7));
            mx = std::max(mx, std::fabs(ref - (double)host[m * 32 + n]));
        }
    *max_abs_err = mx;
    return UNG_HIP_OK;
}

} // extern "C"
