// ref_driver.cpp -- thin C entry points around the reference's OWN compiled
// FloatL2DistanceHandler (UNG/codes/src/distance.cpp), SearchQueue
// (UNG/codes/src/search_queue.cpp) and TrieIndex (UNG/codes/src/trie.cpp), built into
// oracle/_ref/libungref.so by oracle/Makefile directly from /root/reference (nothing
// copied into this repo).
//
// TEST INFRASTRUCTURE ONLY: used to pin the plain-C oracle (oracle/ung_oracle.c),
// to write tests/golden fixtures, and as the "reference" CPU baseline in bench.py.
//
// The two loops below restate the reference's CPU exact builders around those
// compiled objects:
//   ungref_cross_exact  -> UniNavGraph::build_cross_edges_generate_cpu_exact_scan
//                          + append_cross_edges_from_target_range
//                          (src/uni_nav_graph_cross_edges.cpp:154-220, :32-57)
//   ungref_intra_exact  -> build_exact_topk_graph_for_points
//                          (src/uni_nav_graph_special_blocks.cpp:70-111)
//   ungref_additional_edges -> build_cross_edges_generate_additional, exact branch
//                          (src/uni_nav_graph_cross_edges.cpp:442-596)
//   ungref_trie_lng     -> build_trie_and_divide_groups + LNG phase 1 with
//                          get_min_super_sets_optimized_bucket around the compiled
//                          TrieIndex (src/uni_nav_graph_label_graph.cpp:21-43,103-206,851-890)
//   ungref_assemble_graph / ungref_graph_save -> the reference's own Graph/NeighborList
//                          (include/graph.h) filled as add_offset_for_uni_nav_graph,
//                          merge_cross_edges_to_graph and merge_additional_edges_to_graph
//                          fill it, and its Graph::save
// (their host file needs Boost and cannot be compiled here).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <limits>
#include <memory>
#include <utility>
#include <vector>
#include <omp.h>

#include "distance.h"
#include "graph.h"
#include "search_queue.h"
#include "trie.h"

using ANNS::FloatL2DistanceHandler;
using ANNS::SearchQueue;

extern "C" {

float ungref_l2(const float *a, const float *b, uint32_t dim)
{
    static const FloatL2DistanceHandler h;
    return h.compute(reinterpret_cast<const char *>(a), reinterpret_cast<const char *>(b), dim);
}

// Feed a stream of (id, dist) into one SearchQueue of capacity cap and return
// its final content (size returned).
int32_t ungref_queue_stream(const uint32_t *ids, const float *dists, uint32_t n, int32_t cap,
                            uint32_t *out_ids, float *out_dists)
{
    SearchQueue q;
    q.reserve(cap);
    for (uint32_t i = 0; i < n; ++i)
        q.insert(ids[i], dists[i]);
    for (int32_t j = 0; j < q.size(); ++j) {
        out_ids[j] = q[j].id;
        out_dists[j] = q[j].distance;
    }
    return q.size();
}

void ungref_cross_exact(const float *X, uint32_t N, uint32_t dim, uint32_t G,
                        const uint32_t *group_begin, const uint32_t *in_ptr, const uint32_t *in_idx,
                        uint32_t k, uint32_t *out_ids, float *out_dists, int32_t *out_size,
                        int nthreads)
{
    const FloatL2DistanceHandler h;
    std::vector<SearchQueue> queues(N);
    for (uint32_t i = 0; i < N; ++i)
        queues[i].reserve((int32_t)k);
    if (nthreads > 0)
        omp_set_num_threads(nthreads);
    for (uint32_t x = 1; x <= G; ++x) {
        if (in_ptr[x + 1] == in_ptr[x])
            continue;
        const uint32_t xf = group_begin[x], xs = group_begin[x + 1];
        if (xs == xf)
            continue;
        for (uint32_t e = in_ptr[x]; e < in_ptr[x + 1]; ++e) {
            const uint32_t c = in_idx[e];
            const int64_t qf = group_begin[c], qs = group_begin[c + 1];
#pragma omp parallel for schedule(dynamic, 1)
            for (int64_t q = qf; q < qs; ++q) {
                SearchQueue local;
                local.reserve((int32_t)k);
                const char *qv = reinterpret_cast<const char *>(X + (size_t)q * dim);
                for (uint32_t t = xf; t < xs; ++t)
                    local.insert(t, h.compute(qv, reinterpret_cast<const char *>(X + (size_t)t * dim), dim));
                for (int j = 0; j < local.size(); ++j)
                    queues[q].insert(local[j].id, local[j].distance);
            }
        }
    }
    for (uint32_t i = 0; i < N; ++i) {
        out_size[i] = queues[i].size();
        for (uint32_t j = 0; j < k; ++j) {
            const bool has = (int32_t)j < queues[i].size();
            out_ids[(size_t)i * k + j] = has ? queues[i][j].id : UINT32_MAX;
            out_dists[(size_t)i * k + j] = has ? queues[i][j].distance : INFINITY;
        }
    }
}

// Bounded sample of the cross-edge exact scan for listed query points (used for
// the timed CPU baseline): same per-(target, query) local queue + merge, with
// the targets of a point's group given as an out-neighbour CSR.
void ungref_cross_exact_points(const float *X, uint32_t dim, const uint32_t *group_begin,
                               const uint32_t *point_group, const uint32_t *out_ptr,
                               const uint32_t *out_idx, const uint32_t *q_list, uint32_t n_q,
                               uint32_t k, uint32_t *out_ids, float *out_dists, int nthreads)
{
    const FloatL2DistanceHandler h;
    if (nthreads > 0)
        omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t i = 0; i < (int64_t)n_q; ++i) {
        const uint32_t q = q_list[i];
        SearchQueue acc;
        acc.reserve((int32_t)k);
        const char *qv = reinterpret_cast<const char *>(X + (size_t)q * dim);
        const uint32_t c = point_group[q];
        for (uint32_t e = out_ptr[c]; e < out_ptr[c + 1]; ++e) {
            const uint32_t x = out_idx[e];
            SearchQueue local;
            local.reserve((int32_t)k);
            for (uint32_t t = group_begin[x]; t < group_begin[x + 1]; ++t)
                local.insert(t, h.compute(qv, reinterpret_cast<const char *>(X + (size_t)t * dim), dim));
            for (int j = 0; j < local.size(); ++j)
                acc.insert(local[j].id, local[j].distance);
        }
        for (uint32_t j = 0; j < k; ++j) {
            const bool has = (int32_t)j < acc.size();
            out_ids[(size_t)i * k + j] = has ? acc[j].id : UINT32_MAX;
            out_dists[(size_t)i * k + j] = has ? acc[j].distance : INFINITY;
        }
    }
}

void ungref_intra_exact(const float *X, uint32_t dim, uint32_t begin, uint32_t n, uint32_t K,
                        uint32_t *out_ids, float *out_dists, int nthreads)
{
    const FloatL2DistanceHandler h;
    if (nthreads > 0)
        omp_set_num_threads(nthreads);
    const uint32_t degree = n > 0 ? std::min<uint32_t>(K, n - 1) : 0;
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t i = 0; i < (int64_t)n; ++i) {
        uint32_t *ids = out_ids + (size_t)i * K;
        float *ds = out_dists + (size_t)i * K;
        for (uint32_t j = 0; j < K; ++j) {
            ids[j] = UINT32_MAX;
            ds[j] = INFINITY;
        }
        if (n <= 1)
            continue;
        std::vector<std::pair<float, uint32_t>> cand;
        cand.reserve(n - 1);
        const char *src = reinterpret_cast<const char *>(X + ((size_t)begin + i) * dim);
        for (uint32_t j = 0; j < n; ++j) {
            if (j == (uint32_t)i)
                continue;
            cand.emplace_back(h.compute(src, reinterpret_cast<const char *>(X + ((size_t)begin + j) * dim), dim), j);
        }
        auto less = [](const std::pair<float, uint32_t> &a, const std::pair<float, uint32_t> &b) {
            return a.first < b.first || (a.first == b.first && a.second < b.second);
        };
        if (cand.size() > degree) {
            std::nth_element(cand.begin(), cand.begin() + degree, cand.end(), less);
            cand.resize(degree);
        }
        std::sort(cand.begin(), cand.end(), less);
        for (size_t j = 0; j < cand.size(); ++j) {
            ids[j] = cand[j].second;
            ds[j] = cand[j].first;
        }
    }
}

// Additional edges, CPU exact variant (UniNavGraph::build_cross_edges_generate_additional,
// src/uni_nav_graph_cross_edges.cpp:442-596, CpuExactScan branch :543-562, special
// blocks off), with the reference's own SearchQueue and distance.  Same contract as
// ungo_additional_edges in oracle/ung_oracle.h.
int64_t ungref_additional_edges(const float *X, uint32_t N, uint32_t dim, uint32_t G,
                                const uint32_t *group_begin, const uint32_t *out_ptr,
                                const uint32_t *out_idx, const uint32_t *cross_ids, uint32_t stride,
                                uint32_t num_cross, uint32_t *edge_ptr, uint32_t *edge_from,
                                uint32_t *edge_to, int64_t cap, int64_t *needed)
{
    const FloatL2DistanceHandler h;
    std::vector<uint32_t> pg(N);
    for (uint32_t g = 1; g <= G; ++g)
        for (uint32_t i = group_begin[g]; i < group_begin[g + 1]; ++i)
            pg[i] = g;
    std::vector<uint32_t> connected_epoch((size_t)G + 1, 0);
    const uint32_t use = std::min(num_cross, stride);
    int64_t n = 0;
    edge_ptr[0] = edge_ptr[1] = 0;
    for (uint32_t c = 1; c <= G; ++c) {
        for (uint32_t i = group_begin[c]; i < group_begin[c + 1]; ++i)
            for (uint32_t t = 0; t < use; ++t) {
                const uint32_t nb = cross_ids[(size_t)i * stride + t];
                if (nb != UINT32_MAX)
                    connected_epoch[pg[nb]] = c;
            }
        for (uint32_t p = out_ptr[c]; p < out_ptr[c + 1]; ++p) {
            const uint32_t x = out_idx[p];
            if (connected_epoch[x] == c)
                continue;
            uint32_t cnt = 0;
            for (uint32_t v = group_begin[c]; v < group_begin[c + 1] && cnt < num_cross; ++v) {
                SearchQueue local_topk;
                local_topk.reserve((int32_t)num_cross);
                const char *qv = reinterpret_cast<const char *>(X + (size_t)v * dim);
                for (uint32_t t = group_begin[x]; t < group_begin[x + 1]; ++t)
                    local_topk.insert(t, h.compute(qv, reinterpret_cast<const char *>(X + (size_t)t * dim), dim));
                for (int k = 0; k < local_topk.size() && k < (int)(num_cross / 2); ++k) {
                    if (n < cap) {
                        edge_from[n] = v;
                        edge_to[n] = local_topk[k].id;
                    }
                    ++n;
                    ++cnt;
                }
            }
        }
        edge_ptr[c + 1] = (uint32_t)n;
    }
    if (needed)
        *needed = n;
    return n <= cap ? n : -1;
}

// The final adjacency in the reference's own container: intra edges as the group
// graph builders leave them (local ids), add_offset_for_uni_nav_graph
// (src/uni_nav_graph.cpp:285-297), then the writer's cross-edge append
// (src/ung_cross_edge_output_writer.cpp:68-95, FlatId rows) and the additional-edge
// merge (:30-42).  Exported as CSR; same contract as ung_assemble_graph_csr.
int64_t ungref_assemble_graph(uint64_t N, uint32_t G, const uint32_t *group_begin, const uint64_t *intra_ptr,
                              const uint32_t *intra_idx, int intra_global, const uint32_t *cross_ids,
                              uint32_t cross_stride, uint32_t num_cross, const uint32_t *add_ptr,
                              const uint32_t *add_from, const uint32_t *add_to, uint64_t *row_ptr,
                              uint32_t *col_idx, int64_t cap)
{
    ANNS::Graph g((ANNS::IdxType)N);
    std::vector<uint32_t> group_of(N);
    for (uint32_t c = 1; c <= G; ++c)
        for (uint32_t i = group_begin[c]; i < group_begin[c + 1]; ++i)
            group_of[i] = c;
    if (intra_ptr)
        for (uint64_t i = 0; i < N; ++i)
            for (uint64_t p = intra_ptr[i]; p < intra_ptr[i + 1]; ++p)
                g.neighbors[i].emplace_back(intra_idx[p]);
    if (!intra_global)
        for (uint64_t i = 0; i < N; ++i)
            for (auto &neighbor : g.neighbors[i])
                neighbor += group_begin[group_of[i]];
    if (cross_ids)
        for (uint64_t i = 0; i < N; ++i)
            for (uint32_t k = 0; k < num_cross; ++k) {
                const uint32_t nb = cross_ids[i * cross_stride + k];
                if (nb != std::numeric_limits<uint32_t>::max())
                    g.neighbors[i].emplace_back(nb);
            }
    if (add_ptr)
        for (uint32_t c = 1; c <= G; ++c)
            for (uint32_t e = add_ptr[c]; e < add_ptr[c + 1]; ++e)
                g.neighbors[add_from[e]].emplace_back(add_to[e]);
    int64_t n = 0;
    row_ptr[0] = 0;
    for (uint64_t i = 0; i < N; ++i) {
        for (auto nb : g.neighbors[i]) {
            if (n < cap)
                col_idx[n] = nb;
            ++n;
        }
        row_ptr[i + 1] = (uint64_t)n;
    }
    return n <= cap ? n : -1;
}

// Group division and label navigating graph with the reference's OWN TrieIndex
// (src/trie.cpp, compiled into this library):
//   * build_trie_and_divide_groups (src/uni_nav_graph_label_graph.cpp:21-43): every
//     vector's label set inserted in vector order; point_group[i] = its group id;
//   * phase 1 of build_label_nav_graph_optimized_phase1 (:851-890): per group, in id
//     order, get_min_super_sets(label set, ids, avoid_self = true) with the default
//     OptimizedBucket implementation (include/ung_build_config.h:83), restated from
//     get_min_super_sets_optimized_bucket (:103-206) around the reference's
//     TrieIndex::get_super_set_entrances (need_containment = true, the default of
//     include/uni_nav_graph.h:284-285).
// out_ptr needs G+2 entries (at most N+2); out_idx is written when out_cap is large
// enough.  Returns the number of LNG edges (the caller retries with a larger out_cap
// when it exceeds out_cap).
int64_t ungref_trie_lng(uint64_t N, const uint32_t *lab_ptr, const uint32_t *lab_idx,
                        uint32_t *point_group, uint32_t *G_out, uint32_t *out_ptr, uint32_t *out_idx,
                        int64_t out_cap)
{
    using ANNS::IdxType;
    using ANNS::LabelType;
    using ANNS::TrieNode;
    ANNS::TrieIndex trie;
    IdxType new_group_id = 1;
    std::vector<std::vector<LabelType>> set_of(1);
    for (uint64_t i = 0; i < N; ++i) {
        std::vector<LabelType> ls(lab_idx + lab_ptr[i], lab_idx + lab_ptr[i + 1]);
        const IdxType g = trie.insert(ls, new_group_id);
        if (g + 1 > set_of.size()) {
            set_of.resize(g + 1);
            set_of[g] = ls;
        }
        point_group[i] = g;
    }
    const uint32_t G = new_group_id - 1;
    *G_out = G;

    int64_t total = 0;
    out_ptr[0] = out_ptr[1] = 0;
    std::vector<std::shared_ptr<TrieNode>> candidates;
    std::vector<TrieNode *> nodes;
    std::vector<const std::vector<LabelType> *> min_sets;
    std::vector<IdxType> row;
    std::vector<std::vector<TrieNode *>> buckets;
    for (uint32_t c = 1; c <= G; ++c) {
        row.clear();
        trie.get_super_set_entrances(set_of[c], candidates, true, true);
        if (candidates.size() == 1) {
            row.push_back(candidates[0]->group_id);
        } else if (candidates.size() > 1) {
            nodes.clear();
            LabelType lo = candidates[0]->label_set_size, hi = lo;
            for (const auto &sp : candidates) {
                nodes.push_back(sp.get());
                lo = std::min(lo, sp->label_set_size);
                hi = std::max(hi, sp->label_set_size);
            }
            min_sets.clear();
            auto consider = [&](const TrieNode *cand) {
                const auto &ls = set_of[cand->group_id];
                bool minimal = true;
                if (cand->label_set_size > lo)
                    for (const auto *m : min_sets)
                        if (std::includes(ls.begin(), ls.end(), m->begin(), m->end())) {
                            minimal = false;
                            break;
                        }
                if (minimal) {
                    row.push_back(cand->group_id);
                    min_sets.push_back(&ls);
                }
            };
            if (hi - lo <= 256) { // size buckets, each in entrance (BFS) order
                buckets.assign(hi - lo + 1, {});
                for (TrieNode *nd : nodes)
                    buckets[nd->label_set_size - lo].push_back(nd);
                for (const auto &b : buckets)
                    for (const TrieNode *nd : b)
                        consider(nd);
            } else {
                std::sort(nodes.begin(), nodes.end(), [](const TrieNode *a, const TrieNode *b) {
                    return a->label_set_size < b->label_set_size;
                });
                for (const TrieNode *nd : nodes)
                    consider(nd);
            }
        }
        for (IdxType x : row) {
            if (total < out_cap)
                out_idx[total] = x;
            ++total;
        }
        out_ptr[c + 1] = (uint32_t)total;
    }
    return total;
}

// Graph::save of the reference (include/graph.h:207-216) on a CSR adjacency.
void ungref_graph_save(const char *path, uint64_t N, const uint64_t *row_ptr, const uint32_t *col_idx)
{
    ANNS::Graph g((ANNS::IdxType)N);
    for (uint64_t i = 0; i < N; ++i)
        for (uint64_t p = row_ptr[i]; p < row_ptr[i + 1]; ++p)
            g.neighbors[i].emplace_back(col_idx[p]);
    std::string name(path);
    g.save(name);
}

} // extern "C"
