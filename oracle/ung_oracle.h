/*
 * ung_oracle.h -- CPU oracle for the UNG cross-edge / mid-group kNN build stage.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or the timed CPU baseline.  The product (filtervectorcode_refactor_amd) never
 * links, loads or calls it.
 *
 * Each function restates one piece of the reference's CPU semantics in plain C;
 * the reference file:line it follows is given on every declaration (paths are
 * relative to UNG/codes/ in panjd123/FilterVectorCode_refactor).
 */
#ifndef UNG_ORACLE_H
#define UNG_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Squared L2 in the summation order of the reference's release build of
 * FloatL2DistanceHandler::compute (src/distance.cpp:34-91, compiled with
 * -Ofast -mfma, CMakeLists.txt:47-49): 8 lane accumulators updated with a
 * fused multiply-add per 8-float block, fold of the upper 4 lanes onto the
 * lower 4, a 4-float tail and a masked <4 tail (both fused), then two
 * horizontal adds: (s0+s1)+(s2+s3). */
float ungo_l2(const float *a, const float *b, uint32_t dim);

/* ungo_l2 of n row pairs of X [* x dim]: out[i] = ungo_l2(X[a[i]], X[b[i]]) (OpenMP);
 * pairs with b[i] == UINT32_MAX give +inf.  Used by tests to check every reported
 * distance of a large result bit for bit. */
void ungo_l2_pairs(const float *X, uint32_t dim, const uint32_t *a, const uint32_t *b, uint64_t n, float *out);

/* Double-precision squared L2 (no relation to the reference; used by tests as
 * an independent brute-force check of ungo_l2). */
double ungo_l2_f64(const float *a, const float *b, uint32_t dim);

/* Bounded sorted queue insert with the semantics of SearchQueue::insert
 * (src/search_queue.cpp:26-53; order (distance, id) from search_queue.h:20-22):
 * ids/dists hold *size entries sorted ascending, capacity cap.  Returns the
 * position written or -1 when the candidate was rejected. */
int ungo_queue_insert(uint32_t *ids, float *dists, int32_t *size, int32_t cap,
                      uint32_t id, float dist);

/* Group division in first-appearance order of exact label sets
 * (src/uni_nav_graph_label_graph.cpp:21-43 with TrieIndex::insert,
 * src/trie.cpp:23-55) and the group-contiguous reorder
 * (src/uni_nav_graph.cpp:148-166).
 * in : labels as CSR (lab_ptr[N+1], lab_idx), each row sorted ascending
 *      (src/storage.cpp:137-145).
 * out: point_group[N] (1-based group id of each ORIGINAL point),
 *      group_begin[G+2] (new-id range of group g is [group_begin[g], group_begin[g+1]), g=1..G;
 *      group_begin[0]=0), new_to_old[N].  Returns G. */
uint32_t ungo_divide_groups(uint32_t n, const uint32_t *lab_ptr, const uint32_t *lab_idx,
                            uint32_t *point_group, uint32_t *group_begin, uint32_t *new_to_old);

/* Minimum proper supersets by definition (brute force O(G^2 * L)): for each
 * group C, out(C) = { X != C : labels(C) strict-subset labels(X), and no Y with
 * labels(C) < labels(Y) < labels(X) }.  This is the set the reference's
 * trie search + minimality filter returns (src/uni_nav_graph_label_graph.cpp:45-206,
 * src/trie.cpp:78-143); order inside a row is ascending group id.
 * in : group label sets as CSR over groups 1..G (set_ptr[G+2], set_idx).
 * out: out_ptr[G+2] CSR offsets, out_idx (capacity out_cap). Returns total
 *      edges or -1 when out_cap is too small. */
int64_t ungo_min_supersets(uint32_t G, const uint32_t *set_ptr, const uint32_t *set_idx,
                           uint32_t *out_ptr, uint32_t *out_idx, int64_t out_cap);

/* CPU exact cross-edge generation, restating
 * build_cross_edges_generate_cpu_exact_scan (src/uni_nav_graph_cross_edges.cpp:154-220)
 * and append_cross_edges_from_target_range (same file :32-57):
 *   for target X=1..G with in(X) non-empty, for C in in(X), for q in C:
 *     local SearchQueue(k) over X's range, then insert into q's SearchQueue(k).
 * X is the group-contiguous (reordered) base set [N x dim].
 * in_ptr/in_idx: in-neighbour CSR over groups 1..G (in_ptr[G+2]).
 * out_ids/out_dists: [N x k]; out_size[N] = queue size per point; unused
 * slots are set to UINT32_MAX / +inf.  Parallel over q with OpenMP
 * (schedule(dynamic,1) as in the reference), nthreads<=0 -> default. */
void ungo_cross_exact(const float *X, uint32_t N, uint32_t dim, uint32_t G,
                      const uint32_t *group_begin, const uint32_t *in_ptr, const uint32_t *in_idx,
                      uint32_t k, uint32_t *out_ids, float *out_dists, int32_t *out_size,
                      int nthreads);

/* Same as ungo_cross_exact for a subset of query points only (q_list, n_q),
 * used for bounded CPU-baseline samples.  Writes rows for the listed points
 * into out_ids/out_dists[n_q x k]. point_group[N] maps new id -> group. */
void ungo_cross_exact_points(const float *X, uint32_t N, uint32_t dim, uint32_t G,
                             const uint32_t *group_begin, const uint32_t *point_group,
                             const uint32_t *out_ptr, const uint32_t *out_idx,
                             const uint32_t *q_list, uint32_t n_q, uint32_t k,
                             uint32_t *out_ids, float *out_dists, int32_t *out_size,
                             int nthreads);

/* Additional edges, CPU exact variant, restating
 * UniNavGraph::build_cross_edges_generate_additional (src/uni_nav_graph_cross_edges.cpp:
 * 442-596, CpuExactScan branch :543-562; special blocks off):
 *   for C = 1..G: the groups reached by the first num_cross entries of the cross-edge
 *   rows of C's members (cross_ids[N x stride], UINT32_MAX = none) are connected; for
 *   every X of out(C) (row order) that is not, vectors v = s_C, s_C+1, ... while fewer
 *   than num_cross edges were appended for this X get the first num_cross/2 entries of an
 *   exact SearchQueue(num_cross) over X's range (ids ascending).
 * out: edge_ptr[G+2] CSR over groups 1..G, edge_from/edge_to (global new ids) in that
 * order.  Returns the edge count; -1 when cap is too small (*needed = the count). */
int64_t ungo_additional_edges(const float *X, uint32_t N, uint32_t dim, uint32_t G,
                              const uint32_t *group_begin, const uint32_t *out_ptr,
                              const uint32_t *out_idx, const uint32_t *cross_ids, uint32_t stride,
                              uint32_t num_cross, uint32_t *edge_ptr, uint32_t *edge_from,
                              uint32_t *edge_to, int64_t cap, int64_t *needed);

/* Final adjacency, restating add_offset_for_uni_nav_graph (src/uni_nav_graph.cpp:285-297)
 * followed by merge_cross_edges_to_graph / merge_additional_edges_to_graph
 * (src/uni_nav_graph_cross_edges.cpp:849-868; writer src/ung_cross_edge_output_writer.cpp:
 * 30-42, 68-95): row i = intra edges (+ the group's first id unless intra_global), the
 * first num_cross FlatId entries of i (UINT32_MAX skipped), then i's additional edges in
 * the order of the per-group lists.  Same contract as ung_assemble_graph_csr; returns
 * the entry count or -1 when cap is too small. */
int64_t ungo_assemble_graph(uint64_t N, uint32_t G, const uint32_t *group_begin, const uint64_t *intra_ptr,
                            const uint32_t *intra_idx, int intra_global, const uint32_t *cross_ids,
                            uint32_t cross_stride, uint32_t num_cross, const uint32_t *add_ptr,
                            const uint32_t *add_from, const uint32_t *add_to, uint64_t *row_ptr,
                            uint32_t *col_idx, int64_t cap);

/* Exact intra-group top-K, restating build_exact_topk_graph_for_points
 * (src/uni_nav_graph_special_blocks.cpp:70-111): for every point i of the
 * group [begin, begin+n) the first min(K, n-1) local ids j != i ordered by
 * (dist, j).  out_ids/out_dists: [n x K] local ids, padding UINT32_MAX/+inf.
 * Parallel over points with OpenMP. */
void ungo_intra_exact(const float *X, uint32_t dim, uint32_t begin, uint32_t n, uint32_t K,
                      uint32_t *out_ids, float *out_dists, int nthreads);

/* Exact-anchor row packing of batched_exact_knn_graph_kernel
 * (src/tagore_graph_builder.cu:727-794): from a point's exact candidate list
 * top_idx[cand_degree] (local ids by (dist,id)), writes row[0]=out_degree and
 * row[1..graph_stride-1] (head, anchors, strided tail, dedup tail, then
 * local_src padding). */
void ungo_pack_anchor_row(const uint32_t *top_idx, uint32_t cand_degree, uint32_t n,
                          uint32_t local_src, uint32_t final_degree, uint32_t head_keep,
                          uint32_t anchor_tail, uint32_t anchor_slots, uint32_t bidir_anchor,
                          uint32_t graph_stride, uint32_t *row);

/* Graph of a large group (n above the exact batch), restating the FastGrnnd batch path
 * (tagore_graph_builder.cu:1777-2159) with exact candidate lists in place of its
 * un-vendored NN-descent, and the in-tree prune:
 *  1. candidates: the exact top-knn_k of every point by (dist, local id)
 *     (special_blocks.cpp:70-111 order);
 *  2. build_sampled_reverse_kernel (:141-163): source s joins the reverse list of every
 *     point among its first forward_cap candidates; the reference keeps the first
 *     reverse_cap arrivals of an atomic counter (run-dependent), here the reverse_cap
 *     nearest by (dist, source id);
 *  3. fast_grnnd_prune_kernel (:279-387): forward (first forward_cap) + reverse
 *     candidates sorted by (dist, id), duplicates dropped, then a greedy scan keeps a
 *     candidate unless alpha * d(kept, candidate) < d(point, candidate) for a kept one,
 *     up to final_degree; distances in fp32 (ungo_l2) where the reference uses fp16.
 * rows: [n x (final_degree+1)]: row[0] = kept count, row[1..] kept local ids, padded
 * with the point's own local id (:385-387).  Parity with the reference itself is
 * unpinned (NN-descent source absent, reverse sampling run-dependent); this function
 * is the specification the device path is checked against. */
void ungo_large_group_graph(const float *X, uint32_t dim, uint32_t begin, uint32_t n, uint32_t knn_k,
                            uint32_t forward_cap, uint32_t reverse_cap, uint32_t final_degree, float alpha,
                            uint32_t *rows);

#ifdef __cplusplus
}
#endif

#endif
