/*
 * ung_oracle.c -- CPU oracle for the UNG cross-edge / mid-group kNN build stage.
 *
 * TEST INFRASTRUCTURE ONLY (see ung_oracle.h): loaded by tests/, by
 * __graft_entry__.smoke() and by the cpu_baseline leg of bench.py, never by the
 * product.  Plain C restatement of the reference's CPU semantics; every
 * function names the reference file:line it follows (paths under UNG/codes/).
 *
 * Build: oracle/Makefile (gcc -O3 -fopenmp -ffp-contract=off; fmaf() is the
 * only fused operation, written out where the reference's release build fuses).
 *
 * Parity pins (tests/test_oracle.py):
 *   ungo_l2            bit-exact vs the reference's own distance.cpp compiled
 *                      under oracle/_ref with its release flags, and within
 *                      fp32 error bounds of a float64 brute force;
 *   ungo_queue_insert  element-wise vs the reference's compiled SearchQueue
 *                      (oracle/_ref) on random insert streams, and vs sorting;
 *   ungo_cross_exact   vs committed golden fixtures made by oracle/_ref and
 *                      vs a float64 brute-force top-k outside the tie band;
 *   ungo_intra_exact   vs oracle/_ref fixtures and a float64 brute force;
 *   ungo_divide_groups vs a Python dict-based first-appearance grouping;
 *   ungo_min_supersets vs a Python itertools enumeration of the definition;
 *   ungo_pack_anchor_row  vs hand-worked rows (small n) and invariants;
 *   ungo_additional_edges vs golden fixtures and the restatement around the
 *                      reference's own SearchQueue/distance (oracle/_ref), and vs
 *                      closed-form edge counts;
 *   ungo_assemble_graph vs the reference's own Graph/NeighborList filled by the
 *                      reference's loops (oracle/_ref) and a hand-worked case.
 */
#include "ung_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* src/distance.cpp:34-91 (release build: the _mm256_add_ps(acc, _mm256_mul_ps(d,d))
 * pair is contracted to one vfmadd231ps; verified against the compiled reference). */
float ungo_l2(const float *a, const float *b, uint32_t dim)
{
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint32_t p = 0;
    while (dim - p >= 8) {
        for (int l = 0; l < 8; ++l) {
            const float d = a[p + l] - b[p + l];
            acc[l] = fmaf(d, d, acc[l]);
        }
        p += 8;
    }
    float s[4];
    for (int i = 0; i < 4; ++i)
        s[i] = acc[i + 4] + acc[i];
    uint32_t rem = dim - p;
    if (rem >= 4) {
        for (int i = 0; i < 4; ++i) {
            const float d = a[p + i] - b[p + i];
            s[i] = fmaf(d, d, s[i]);
        }
        p += 4;
        rem -= 4;
    }
    for (uint32_t i = 0; i < rem; ++i) {
        const float d = a[p + i] - b[p + i];
        s[i] = fmaf(d, d, s[i]);
    }
    return (s[0] + s[1]) + (s[2] + s[3]);
}

void ungo_l2_pairs(const float *X, uint32_t dim, const uint32_t *a, const uint32_t *b, uint64_t n, float *out)
{
#pragma omp parallel for schedule(static, 4096)
    for (int64_t i = 0; i < (int64_t)n; ++i)
        out[i] = b[i] == 0xFFFFFFFFu ? INFINITY
                                     : ungo_l2(X + (size_t)a[i] * dim, X + (size_t)b[i] * dim, dim);
}

double ungo_l2_f64(const float *a, const float *b, uint32_t dim)
{
    double s = 0.0;
    for (uint32_t i = 0; i < dim; ++i) {
        const double d = (double)a[i] - (double)b[i];
        s += d * d;
    }
    return s;
}

static inline int cand_less(float da, uint32_t ia, float db, uint32_t ib)
{
    return da < db || (da == db && ia < ib);
}

/* src/search_queue.cpp:26-53 */
int ungo_queue_insert(uint32_t *ids, float *dists, int32_t *size, int32_t cap,
                      uint32_t id, float dist)
{
    int32_t n = *size;
    if (cap <= 0)
        return -1;
    if (n == cap && cand_less(dists[n - 1], ids[n - 1], dist, id))
        return -1;
    int32_t lo = 0, hi = n;
    while (lo < hi) {
        const int32_t mid = (lo + hi) >> 1;
        if (cand_less(dist, id, dists[mid], ids[mid]))
            hi = mid;
        else if (ids[mid] == id)
            return -1;
        else
            lo = mid + 1;
    }
    /* the reference keeps capacity+1 slots and lets the tail fall off */
    int32_t last = (n < cap) ? n : cap - 1;
    for (int32_t j = last; j > lo; --j) {
        ids[j] = ids[j - 1];
        dists[j] = dists[j - 1];
    }
    if (lo < cap) {
        ids[lo] = id;
        dists[lo] = dist;
    }
    if (n < cap)
        *size = n + 1;
    return lo < cap ? lo : -1;
}

/* ---- group division (label_graph.cpp:21-43, trie.cpp:23-55, uni_nav_graph.cpp:148-166) ---- */

typedef struct {
    const uint32_t *lab_ptr;
    const uint32_t *lab_idx;
} label_ctx;

static const label_ctx *g_sort_ctx;

static int cmp_label_rows(uint32_t a, uint32_t b, const label_ctx *c)
{
    uint32_t la = c->lab_ptr[a + 1] - c->lab_ptr[a];
    uint32_t lb = c->lab_ptr[b + 1] - c->lab_ptr[b];
    const uint32_t *pa = c->lab_idx + c->lab_ptr[a];
    const uint32_t *pb = c->lab_idx + c->lab_ptr[b];
    uint32_t m = la < lb ? la : lb;
    for (uint32_t i = 0; i < m; ++i) {
        if (pa[i] != pb[i])
            return pa[i] < pb[i] ? -1 : 1;
    }
    if (la != lb)
        return la < lb ? -1 : 1;
    return 0;
}

static int cmp_points(const void *x, const void *y)
{
    uint32_t a = *(const uint32_t *)x, b = *(const uint32_t *)y;
    int c = cmp_label_rows(a, b, g_sort_ctx);
    if (c)
        return c;
    return a < b ? -1 : (a > b);
}

typedef struct {
    uint32_t first_point;
    uint32_t rank; /* index into the sorted distinct list */
} first_seen;

static int cmp_first(const void *x, const void *y)
{
    const first_seen *a = (const first_seen *)x, *b = (const first_seen *)y;
    return a->first_point < b->first_point ? -1 : (a->first_point > b->first_point);
}

uint32_t ungo_divide_groups(uint32_t n, const uint32_t *lab_ptr, const uint32_t *lab_idx,
                            uint32_t *point_group, uint32_t *group_begin, uint32_t *new_to_old)
{
    if (n == 0) {
        group_begin[0] = 0;
        group_begin[1] = 0;
        return 0;
    }
    label_ctx ctx = {lab_ptr, lab_idx};
    uint32_t *order = (uint32_t *)malloc(sizeof(uint32_t) * n);
    for (uint32_t i = 0; i < n; ++i)
        order[i] = i;
    g_sort_ctx = &ctx;
    qsort(order, n, sizeof(uint32_t), cmp_points);
    /* distinct label sets; within one set `order` is ascending point id, so the
     * first element is the first appearance */
    first_seen *fs = (first_seen *)malloc(sizeof(first_seen) * n);
    uint32_t *rank_of_sorted = (uint32_t *)malloc(sizeof(uint32_t) * n);
    uint32_t nd = 0;
    for (uint32_t i = 0; i < n; ++i) {
        if (i == 0 || cmp_label_rows(order[i - 1], order[i], &ctx) != 0) {
            fs[nd].first_point = order[i];
            fs[nd].rank = nd;
            ++nd;
        }
        rank_of_sorted[i] = nd - 1;
    }
    qsort(fs, nd, sizeof(first_seen), cmp_first);
    uint32_t *gid_of_rank = (uint32_t *)malloc(sizeof(uint32_t) * nd);
    for (uint32_t g = 0; g < nd; ++g)
        gid_of_rank[fs[g].rank] = g + 1; /* group ids 1..G in first-appearance order */
    for (uint32_t i = 0; i < n; ++i)
        point_group[order[i]] = gid_of_rank[rank_of_sorted[i]];
    /* reorder: groups 1..G, original ascending order inside a group */
    uint32_t *count = (uint32_t *)calloc(nd + 2, sizeof(uint32_t));
    for (uint32_t i = 0; i < n; ++i)
        count[point_group[i]]++;
    group_begin[0] = 0;
    group_begin[1] = 0;
    for (uint32_t g = 1; g <= nd; ++g)
        group_begin[g + 1] = group_begin[g] + count[g];
    uint32_t *fill = (uint32_t *)calloc(nd + 2, sizeof(uint32_t));
    for (uint32_t i = 0; i < n; ++i) {
        uint32_t g = point_group[i];
        new_to_old[group_begin[g] + fill[g]++] = i;
    }
    free(fill);
    free(count);
    free(gid_of_rank);
    free(rank_of_sorted);
    free(fs);
    free(order);
    return nd;
}

/* ---- minimum proper supersets by definition ---- */

static int is_subset(const uint32_t *a, uint32_t la, const uint32_t *b, uint32_t lb)
{
    /* a subset-of b, both sorted ascending (std::includes semantics) */
    uint32_t i = 0, j = 0;
    while (i < la) {
        while (j < lb && b[j] < a[i])
            ++j;
        if (j == lb || b[j] != a[i])
            return 0;
        ++i;
        ++j;
    }
    return 1;
}

int64_t ungo_min_supersets(uint32_t G, const uint32_t *set_ptr, const uint32_t *set_idx,
                           uint32_t *out_ptr, uint32_t *out_idx, int64_t out_cap)
{
    int64_t total = 0;
    uint32_t *sup = (uint32_t *)malloc(sizeof(uint32_t) * (G + 1));
    out_ptr[0] = 0;
    out_ptr[1] = 0;
    for (uint32_t c = 1; c <= G; ++c) {
        const uint32_t *sc = set_idx + set_ptr[c];
        const uint32_t lc = set_ptr[c + 1] - set_ptr[c];
        uint32_t ns = 0;
        for (uint32_t x = 1; x <= G; ++x) {
            const uint32_t lx = set_ptr[x + 1] - set_ptr[x];
            if (x == c || lx <= lc)
                continue;
            if (is_subset(sc, lc, set_idx + set_ptr[x], lx))
                sup[ns++] = x;
        }
        for (uint32_t i = 0; i < ns; ++i) {
            const uint32_t x = sup[i];
            const uint32_t lx = set_ptr[x + 1] - set_ptr[x];
            int minimal = 1;
            for (uint32_t j = 0; j < ns && minimal; ++j) {
                const uint32_t y = sup[j];
                const uint32_t ly = set_ptr[y + 1] - set_ptr[y];
                if (y != x && ly < lx && is_subset(set_idx + set_ptr[y], ly, set_idx + set_ptr[x], lx))
                    minimal = 0;
            }
            if (minimal) {
                if (total >= out_cap) {
                    free(sup);
                    return -1;
                }
                out_idx[total++] = x;
            }
        }
        out_ptr[c + 1] = (uint32_t)total;
    }
    free(sup);
    return total;
}

/* ---- cross edges: uni_nav_graph_cross_edges.cpp:154-220 and :32-57 ---- */

static void local_topk_over_range(const float *X, uint32_t dim, uint32_t q, uint32_t first,
                                  uint32_t second, uint32_t k, uint32_t *lids, float *ldists,
                                  uint32_t *qids, float *qdists, int32_t *qsize)
{
    int32_t lsize = 0;
    const float *qv = X + (size_t)q * dim;
    for (uint32_t t = first; t < second; ++t) {
        const float d = ungo_l2(qv, X + (size_t)t * dim, dim);
        ungo_queue_insert(lids, ldists, &lsize, (int32_t)k, t, d);
    }
    for (int32_t j = 0; j < lsize; ++j)
        ungo_queue_insert(qids, qdists, qsize, (int32_t)k, lids[j], ldists[j]);
}

void ungo_cross_exact(const float *X, uint32_t N, uint32_t dim, uint32_t G,
                      const uint32_t *group_begin, const uint32_t *in_ptr, const uint32_t *in_idx,
                      uint32_t k, uint32_t *out_ids, float *out_dists, int32_t *out_size,
                      int nthreads)
{
    for (size_t i = 0; i < (size_t)N * k; ++i) {
        out_ids[i] = UINT32_MAX;
        out_dists[i] = INFINITY;
    }
    for (uint32_t i = 0; i < N; ++i)
        out_size[i] = 0;
#ifdef _OPENMP
    if (nthreads > 0)
        omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
    for (uint32_t x = 1; x <= G; ++x) {
        if (in_ptr[x + 1] == in_ptr[x])
            continue;
        const uint32_t xf = group_begin[x], xs = group_begin[x + 1];
        if (xs == xf)
            continue;
        for (uint32_t e = in_ptr[x]; e < in_ptr[x + 1]; ++e) {
            const uint32_t c = in_idx[e];
            const int64_t qf = group_begin[c], qs = group_begin[c + 1];
#pragma omp parallel
            {
                uint32_t *lids = (uint32_t *)malloc(sizeof(uint32_t) * (k + 1));
                float *ld = (float *)malloc(sizeof(float) * (k + 1));
#pragma omp for schedule(dynamic, 1)
                for (int64_t q = qf; q < qs; ++q)
                    local_topk_over_range(X, dim, (uint32_t)q, xf, xs, k, lids, ld,
                                          out_ids + (size_t)q * k, out_dists + (size_t)q * k,
                                          out_size + q);
                free(lids);
                free(ld);
            }
        }
    }
}

void ungo_cross_exact_points(const float *X, uint32_t N, uint32_t dim, uint32_t G,
                             const uint32_t *group_begin, const uint32_t *point_group,
                             const uint32_t *out_ptr, const uint32_t *out_idx,
                             const uint32_t *q_list, uint32_t n_q, uint32_t k,
                             uint32_t *out_ids, float *out_dists, int32_t *out_size,
                             int nthreads)
{
    (void)N;
    (void)G;
#ifdef _OPENMP
    if (nthreads > 0)
        omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
#pragma omp parallel
    {
        uint32_t *lids = (uint32_t *)malloc(sizeof(uint32_t) * (k + 1));
        float *ld = (float *)malloc(sizeof(float) * (k + 1));
#pragma omp for schedule(dynamic, 1)
        for (int64_t i = 0; i < (int64_t)n_q; ++i) {
            const uint32_t q = q_list[i];
            uint32_t *qi = out_ids + (size_t)i * k;
            float *qd = out_dists + (size_t)i * k;
            for (uint32_t j = 0; j < k; ++j) {
                qi[j] = UINT32_MAX;
                qd[j] = INFINITY;
            }
            out_size[i] = 0;
            const uint32_t c = point_group[q];
            for (uint32_t e = out_ptr[c]; e < out_ptr[c + 1]; ++e) {
                const uint32_t x = out_idx[e];
                local_topk_over_range(X, dim, q, group_begin[x], group_begin[x + 1], k, lids, ld,
                                      qi, qd, out_size + i);
            }
        }
        free(lids);
        free(ld);
    }
}

/* ---- additional edges: uni_nav_graph_cross_edges.cpp:442-596 (exact branch :543-562) ---- */

int64_t ungo_additional_edges(const float *X, uint32_t N, uint32_t dim, uint32_t G,
                              const uint32_t *group_begin, const uint32_t *out_ptr,
                              const uint32_t *out_idx, const uint32_t *cross_ids, uint32_t stride,
                              uint32_t num_cross, uint32_t *edge_ptr, uint32_t *edge_from,
                              uint32_t *edge_to, int64_t cap, int64_t *needed)
{
    uint32_t *pg = (uint32_t *)malloc(sizeof(uint32_t) * (N ? N : 1));
    uint32_t *mark = (uint32_t *)calloc((size_t)G + 1, sizeof(uint32_t));
    uint32_t *qi = (uint32_t *)malloc(sizeof(uint32_t) * (num_cross + 1));
    float *qd = (float *)malloc(sizeof(float) * (num_cross + 1));
    for (uint32_t g = 1; g <= G; ++g)
        for (uint32_t i = group_begin[g]; i < group_begin[g + 1]; ++i)
            pg[i] = g;
    const uint32_t use = num_cross < stride ? num_cross : stride;
    int64_t n = 0;
    edge_ptr[0] = edge_ptr[1] = 0;
    for (uint32_t c = 1; c <= G; ++c) {
        const uint32_t s = group_begin[c], e = group_begin[c + 1];
        for (uint32_t i = s; i < e; ++i)
            for (uint32_t t = 0; t < use; ++t) {
                const uint32_t nb = cross_ids[(size_t)i * stride + t];
                if (nb != UINT32_MAX)
                    mark[pg[nb]] = c; /* epoch = C */
            }
        for (uint32_t p = out_ptr[c]; p < out_ptr[c + 1]; ++p) {
            const uint32_t x = out_idx[p];
            if (mark[x] == c)
                continue;
            uint32_t cnt = 0;
            for (uint32_t v = s; v < e && cnt < num_cross; ++v) {
                int32_t size = 0;
                const float *qv = X + (size_t)v * dim;
                for (uint32_t t = group_begin[x]; t < group_begin[x + 1]; ++t)
                    ungo_queue_insert(qi, qd, &size, (int32_t)num_cross, t, ungo_l2(qv, X + (size_t)t * dim, dim));
                for (int32_t j = 0; j < size && j < (int32_t)(num_cross / 2); ++j) {
                    if (n < cap) {
                        edge_from[n] = v;
                        edge_to[n] = qi[j];
                    }
                    ++n;
                    ++cnt;
                }
            }
        }
        edge_ptr[c + 1] = (uint32_t)n;
    }
    free(pg);
    free(mark);
    free(qi);
    free(qd);
    if (needed)
        *needed = n;
    return n <= cap ? n : -1;
}

/* ---- final adjacency: uni_nav_graph.cpp:285-297, uni_nav_graph_cross_edges.cpp:849-868 ---- */

typedef struct {
    uint32_t *v;
    uint64_t n, cap;
} u32list;

static void list_push(u32list *l, uint32_t x)
{
    if (l->n == l->cap) {
        l->cap = l->cap ? 2 * l->cap : 8;
        l->v = (uint32_t *)realloc(l->v, sizeof(uint32_t) * l->cap);
    }
    l->v[l->n++] = x;
}

int64_t ungo_assemble_graph(uint64_t N, uint32_t G, const uint32_t *group_begin, const uint64_t *intra_ptr,
                            const uint32_t *intra_idx, int intra_global, const uint32_t *cross_ids,
                            uint32_t cross_stride, uint32_t num_cross, const uint32_t *add_ptr,
                            const uint32_t *add_from, const uint32_t *add_to, uint64_t *row_ptr,
                            uint32_t *col_idx, int64_t cap)
{
    u32list *nb = (u32list *)calloc(N ? N : 1, sizeof(u32list));
    for (uint32_t c = 1; c <= G; ++c)
        for (uint64_t i = group_begin[c]; i < group_begin[c + 1]; ++i) {
            if (intra_ptr) /* intra graph of the group (local ids), then add_offset */
                for (uint64_t p = intra_ptr[i]; p < intra_ptr[i + 1]; ++p)
                    list_push(&nb[i], intra_idx[p] + (intra_global ? 0u : group_begin[c]));
        }
    if (cross_ids)
        for (uint64_t i = 0; i < N; ++i)
            for (uint32_t t = 0; t < num_cross; ++t) {
                const uint32_t x = cross_ids[i * cross_stride + t];
                if (x != UINT32_MAX)
                    list_push(&nb[i], x);
            }
    if (add_ptr)
        for (uint32_t c = 1; c <= G; ++c)
            for (uint32_t e = add_ptr[c]; e < add_ptr[c + 1]; ++e)
                list_push(&nb[add_from[e]], add_to[e]);
    int64_t n = 0;
    row_ptr[0] = 0;
    for (uint64_t i = 0; i < N; ++i) {
        for (uint64_t j = 0; j < nb[i].n; ++j) {
            if (n < cap)
                col_idx[n] = nb[i].v[j];
            ++n;
        }
        row_ptr[i + 1] = (uint64_t)n;
        free(nb[i].v);
    }
    free(nb);
    return n <= cap ? n : -1;
}

/* ---- intra-group exact top-K: uni_nav_graph_special_blocks.cpp:70-111 ---- */

void ungo_intra_exact(const float *X, uint32_t dim, uint32_t begin, uint32_t n, uint32_t K,
                      uint32_t *out_ids, float *out_dists, int nthreads)
{
#ifdef _OPENMP
    if (nthreads > 0)
        omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
    const uint32_t degree = (n > 0) ? (K < n - 1 ? K : n - 1) : 0;
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t i = 0; i < (int64_t)n; ++i) {
        uint32_t *ids = out_ids + (size_t)i * K;
        float *ds = out_dists + (size_t)i * K;
        for (uint32_t j = 0; j < K; ++j) {
            ids[j] = UINT32_MAX;
            ds[j] = INFINITY;
        }
        if (degree == 0)
            continue;
        int32_t size = 0;
        const float *src = X + ((size_t)begin + (size_t)i) * dim;
        /* (dist, local j) is a total order over distinct j, so keeping the
         * `degree` smallest while scanning equals nth_element + sort */
        for (uint32_t j = 0; j < n; ++j) {
            if (j == (uint32_t)i)
                continue;
            const float d = ungo_l2(src, X + ((size_t)begin + j) * dim, dim);
            ungo_queue_insert(ids, ds, &size, (int32_t)degree, j, d);
        }
    }
}

/* ---- exact-anchor packing: tagore_graph_builder.cu:727-794 ---- */

static int row_has(const uint32_t *row, uint32_t write, uint32_t v)
{
    for (uint32_t p = 0; p < write; ++p)
        if (row[1 + p] == v)
            return 1;
    return 0;
}

void ungo_pack_anchor_row(const uint32_t *top_idx, uint32_t cand_degree, uint32_t n,
                          uint32_t local_src, uint32_t final_degree, uint32_t head_keep,
                          uint32_t anchor_tail, uint32_t anchor_slots, uint32_t bidir_anchor,
                          uint32_t graph_stride, uint32_t *row)
{
    const uint32_t out_degree = final_degree < cand_degree ? final_degree : cand_degree;
    row[0] = out_degree;
    if (out_degree > 0) {
        uint32_t near_limit = head_keep < final_degree ? head_keep : final_degree;
        if (out_degree < near_limit)
            near_limit = out_degree;
        uint32_t write = 0;
        for (; write < near_limit; ++write)
            row[1 + write] = top_idx[write];
        const uint32_t remaining = final_degree > write ? final_degree - write : 0;
        uint32_t anchor_limit = 0;
        if (anchor_tail)
            anchor_limit = (anchor_slots == 0) ? remaining : (anchor_slots < remaining ? anchor_slots : remaining);
        if (anchor_limit > 0 && n > 1) {
            for (uint32_t t = 0; t < anchor_limit && write < out_degree; ++t) {
                uint32_t hop = ((t + 1) * n) / (anchor_limit + 1);
                if (hop < 1)
                    hop = 1;
                const int backward = bidir_anchor && (t & 1u);
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
        const uint32_t step = (tail_count > remaining && remaining > 0)
                                  ? (tail_count + remaining - 1) / remaining
                                  : 1;
        for (uint32_t s = tail_start; s < cand_degree && write < out_degree; s += step)
            row[1 + write++] = top_idx[s];
        for (uint32_t s = tail_start; s < cand_degree && write < out_degree; ++s)
            if (!row_has(row, write, top_idx[s]))
                row[1 + write++] = top_idx[s];
    }
    for (uint32_t j = out_degree; j + 1 < graph_stride; ++j)
        row[1 + j] = local_src;
}

/* ---- large-group graph: exact candidate lists + the FastGrnnd prune ----
 * tagore_graph_builder.cu:1777-2159 (batch driver: candidate graph, then
 * launch_fast_grnnd_prune_impl :1463-1568), build_sampled_reverse_kernel :141-163,
 * fast_grnnd_prune_kernel :279-387, configuration tagore_cuda_config.cpp:45-68. */

typedef struct {
    float d;
    uint32_t id;
} dist_id;

static int cmp_dist_id(const void *x, const void *y)
{
    const dist_id *a = (const dist_id *)x, *b = (const dist_id *)y;
    if (cand_less(a->d, a->id, b->d, b->id))
        return -1;
    if (cand_less(b->d, b->id, a->d, a->id))
        return 1;
    return 0;
}

void ungo_large_group_graph(const float *X, uint32_t dim, uint32_t begin, uint32_t n, uint32_t knn_k,
                            uint32_t forward_cap, uint32_t reverse_cap, uint32_t final_degree, float alpha,
                            uint32_t *rows)
{
    const uint32_t stride = final_degree + 1;
    uint32_t *ids = (uint32_t *)malloc((size_t)n * knn_k * sizeof(uint32_t));
    float *ds = (float *)malloc((size_t)n * knn_k * sizeof(float));
    ungo_intra_exact(X, dim, begin, n, knn_k, ids, ds, 0);
    const uint32_t deg = n > 0 ? (knn_k < n - 1 ? knn_k : n - 1) : 0;
    const uint32_t fwd = deg < forward_cap ? deg : forward_cap;
    /* reverse lists: every source whose first `fwd` candidates hold the point */
    uint32_t *rcnt = (uint32_t *)calloc((size_t)n + 1, sizeof(uint32_t));
    for (uint32_t s = 0; s < n; ++s)
        for (uint32_t j = 0; j < fwd; ++j)
            rcnt[ids[(size_t)s * knn_k + j] + 1]++;
    for (uint32_t i = 0; i < n; ++i)
        rcnt[i + 1] += rcnt[i];
    dist_id *rev = (dist_id *)malloc(((size_t)rcnt[n] + 1) * sizeof(dist_id));
    uint32_t *pos = (uint32_t *)malloc(((size_t)n + 1) * sizeof(uint32_t));
    memcpy(pos, rcnt, ((size_t)n + 1) * sizeof(uint32_t));
    for (uint32_t s = 0; s < n; ++s)
        for (uint32_t j = 0; j < fwd; ++j) {
            const uint32_t t = ids[(size_t)s * knn_k + j];
            rev[pos[t]].d = ds[(size_t)s * knn_k + j]; /* dist(s, t) == dist(t, s) bit for bit */
            rev[pos[t]].id = s;
            pos[t]++;
        }
#pragma omp parallel
    {
        dist_id *cand = (dist_id *)malloc(((size_t)fwd + reverse_cap + 1) * sizeof(dist_id));
        uint32_t *acc = (uint32_t *)malloc(((size_t)final_degree + 1) * sizeof(uint32_t));
#pragma omp for schedule(dynamic, 16)
        for (int64_t si = 0; si < (int64_t)n; ++si) {
            const uint32_t s = (uint32_t)si;
            uint32_t nc = 0;
            for (uint32_t j = 0; j < fwd; ++j) {
                cand[nc].d = ds[(size_t)s * knn_k + j];
                cand[nc].id = ids[(size_t)s * knn_k + j];
                nc++;
            }
            /* sampled reverse edges: the reverse_cap nearest by (dist, source id) */
            const uint32_t r0 = rcnt[s], r1 = rcnt[s + 1];
            qsort(rev + r0, r1 - r0, sizeof(dist_id), cmp_dist_id);
            for (uint32_t j = r0; j < r1 && j - r0 < reverse_cap; ++j)
                cand[nc++] = rev[j];
            qsort(cand, nc, sizeof(dist_id), cmp_dist_id);
            /* equal ids carry equal distances, so duplicates are adjacent */
            uint32_t w = 0;
            for (uint32_t j = 0; j < nc; ++j)
                if (w == 0 || cand[j].id != cand[w - 1].id)
                    cand[w++] = cand[j];
            nc = w;
            uint32_t na = 0;
            for (uint32_t j = 0; j < nc && na < final_degree; ++j) {
                const uint32_t t = cand[j].id;
                if (t == s)
                    continue;
                int reject = 0;
                for (uint32_t p = 0; p < na && !reject; ++p) {
                    const float dij = ungo_l2(X + ((size_t)begin + acc[p]) * dim, X + ((size_t)begin + t) * dim, dim);
                    if (alpha * dij < cand[j].d)
                        reject = 1;
                }
                if (!reject)
                    acc[na++] = t;
            }
            uint32_t *row = rows + (size_t)s * stride;
            row[0] = na;
            for (uint32_t j = 0; j < final_degree; ++j)
                row[1 + j] = j < na ? acc[j] : s;
        }
        free(cand);
        free(acc);
    }
    free(ids);
    free(ds);
    free(rcnt);
    free(rev);
    free(pos);
}
