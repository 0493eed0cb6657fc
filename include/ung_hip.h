/*
 * ung_hip.h -- C ABI of the MI355X (gfx950) UNG cross-edge / mid-group kNN build stage.
 *
 * This is the drop-in boundary.  Every entry point is plain C: pointers, sizes,
 * integer error codes, no C++ or torch types.  Paths in citations are relative to
 * UNG/codes/ in panjd123/FilterVectorCode_refactor.
 *
 * Conventions shared by all entry points
 *   - Ids are uint32 "new ids" (group-contiguous order after the reorder of
 *     src/uni_nav_graph.cpp:148-181).  Groups are numbered 1..G.
 *   - group_begin has G+2 entries: group g occupies [group_begin[g], group_begin[g+1]);
 *     group_begin[0] = group_begin[1] = 0 (same role as _group_id_to_range,
 *     include/uni_nav_graph.h).
 *   - out_ptr/out_idx: LNG out-neighbour CSR over groups (out_ptr has G+2 entries,
 *     out(C) = out_idx[out_ptr[C] .. out_ptr[C+1])), i.e. _label_nav_graph->out_neighbors
 *     (src/uni_nav_graph_label_graph.cpp:851-911).
 *   - Distances are fp32 squared L2 with the exact rounding of the reference's
 *     release-build FloatL2DistanceHandler::compute (src/distance.cpp:34-91).
 *   - Result rows are ordered by (distance, id) ascending (search_queue.h:20-22);
 *     missing entries are UINT32_MAX / +inf (the FlatId sentinel of
 *     src/gpu_cross_edge_output.cuh:87-103).
 *   - Return 0 on success, a negative UNG_HIP_E* code on failure; nothing throws
 *     across the ABI.  ung_hip_last_error() gives the message of the calling
 *     thread's last failure.
 *   - A context is bound to one device and is not reentrant (one call at a time),
 *     as the reference's file-static device buffers (src/gpu_cross_edge_buffers.cuh).
 */
#ifndef UNG_HIP_H
#define UNG_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UNG_HIP_OK 0
#define UNG_HIP_EINVAL -1   /* bad argument (sizes, null pointers, k out of range) */
#define UNG_HIP_EDEVICE -2  /* HIP runtime error (allocation, launch, copy) */
#define UNG_HIP_ESTATE -3   /* call order error (e.g. vectors not prepared) */

typedef struct ung_hip_ctx ung_hip_ctx;

/* Timing / work report filled by the entry points that take it (may be NULL).
 * Times are milliseconds; kernel times come from HIP events on the context's
 * stream. */
typedef struct ung_hip_stats {
    double wall_ms;          /* whole call, host clock */
    double plan_ms;          /* host work-list packing */
    double h2d_ms;           /* host->device copies made by this call */
    double kernel_ms;        /* all kernels of the call (events) */
    double select_ms;        /* fused MFMA distance + top-k selection kernel(s) */
    double merge_ms;         /* per-row merge + certification kernel */
    double fallback_ms;      /* exact rescan of uncertified rows */
    double d2h_ms;           /* device->host copies */
    uint64_t pairs;          /* algorithmic distance evaluations P (no padding) */
    uint64_t rows;           /* result rows produced */
    uint64_t work_items;     /* select work items launched */
    uint64_t select_launches;/* select kernel launches */
    uint64_t fallback_rows;  /* rows whose MFMA pre-selection could not be certified
                                and were rescanned exactly */
    uint64_t padded_pairs;   /* pairs computed by the MFMA tiles incl. padding */
    uint64_t select_bytes;   /* operand bytes the select kernel(s) stream: per work item,
                                its query rows and its candidate rows of the split base
                                set (4 * dp bytes a row, dp = dim rounded up to 32) */
    uint64_t allocations;    /* device (hipMalloc) and pinned host (hipHostMalloc)
                                allocations the call made (buffers grown on demand) */
} ung_hip_stats;

/* Message of the calling thread's last failure ("" if none). */
const char *ung_hip_last_error(void);

/* Library version string. */
const char *ung_hip_version(void);

/* Create / destroy a context on HIP device `device`.  No counterpart in the
 * reference (its device state is file-static, src/gpu_cross_edge_buffers.cuh:11-48). */
int ung_hip_create(int device, ung_hip_ctx **out);
int ung_hip_destroy(ung_hip_ctx *ctx);

/* Upload the group-contiguous base set X [N x dim] fp32 (row-major host memory)
 * and compute the squared-norm cache.  Replaces
 * UniNavGraph::gpu_prepare_all_vectors_on_device (include/uni_nav_graph.h:430-432,
 * src/gpu_cross_edge_resident_vectors.cuh:10-215, l2_norm_sq_kernel
 * src/gpu_cross_edge_update_kernels.cuh:7-34).  The whole set stays resident. */
int ung_hip_prepare_vectors(ung_hip_ctx *ctx, const float *X, uint64_t N, uint32_t dim,
                            ung_hip_stats *st);

/* Same, from a device pointer already holding X (copied device-to-device). */
int ung_hip_prepare_vectors_device(ung_hip_ctx *ctx, const float *X_dev, uint64_t N, uint32_t dim,
                                   ung_hip_stats *st);

/* Free the resident base set.  Replaces UniNavGraph::gpu_release_all_vectors_on_device
 * (include/uni_nav_graph.h:433). */
int ung_hip_release_vectors(ung_hip_ctx *ctx);

/* Cross-group edges.  Replaces UniNavGraph::gpu_cross_groups_search_all_batched
 * (include/uni_nav_graph.h:436-444, src/gpu_gemm_topk.cu:377-970) with the
 * semantics of the CPU exact builder build_cross_edges_generate_cpu_exact_scan
 * (src/uni_nav_graph_cross_edges.cpp:154-220, :32-57): for every point q of every
 * group C with out(C) non-empty, the top-k of the union of the ranges of out(C)
 * by (distance, id).  Points of groups with empty out(C) get an empty row.
 * Output (host memory): out_ids [N x k] global new ids, out_dist [N x k]
 * (nullable), out_size [N] (nullable) = number of valid entries per row.
 * 1 <= k <= 64. */
int ung_hip_cross_topk(ung_hip_ctx *ctx, uint32_t G, const uint32_t *group_begin,
                       const uint32_t *out_ptr, const uint32_t *out_idx, uint32_t k,
                       uint32_t *out_ids, float *out_dist, int32_t *out_size,
                       ung_hip_stats *st);

/* Device-resident variant of ung_hip_cross_topk: results stay in context-owned
 * device buffers (read them with ung_hip_cross_result_device or
 * ung_hip_download_cross).  Used when the caller keeps the graph on the GPU. */
int ung_hip_cross_topk_device(ung_hip_ctx *ctx, uint32_t G, const uint32_t *group_begin,
                              const uint32_t *out_ptr, const uint32_t *out_idx, uint32_t k,
                              ung_hip_stats *st);
int ung_hip_cross_result_device(ung_hip_ctx *ctx, uint32_t **ids_dev, float **dist_dev);

/* Bytes of the per-GPU scratch array of ung_hip_cross_topk_noalloc. */
#define UNG_HIP_NOALLOC_SCRATCH_BYTES (64ull << 20)

/* Cross-group edges that allocate nothing.  No counterpart in the reference: this is for
 * callers that must not allocate device or pinned memory during the call -- tight serving
 * loops, harnesses that forbid hipMalloc.  It cannot be captured into a HIP graph: it
 * plans on the host, uploads from host memory and waits for its own stream.  Same rows as
 * ung_hip_cross_topk_device, written to the caller's device buffers out_ids_dev
 * [N x k], out_dist_dev [N x k] and out_size_dev [N] (all required, device memory of the
 * context's device with that many bytes to the end of their allocations; checked with
 * hipPointerGetAttributes and hipMemGetAddressRange).  The call's work lists, partial rows
 * and flags live in a file-scope device array of UNG_HIP_NOALLOC_SCRATCH_BYTES (64 MiB)
 * per GPU, held until the process ends; a call whose plan needs more returns
 * UNG_HIP_EINVAL (the message gives the bytes needed) -- roughly 600k result rows with
 * single-split unions at k = 6 and d < 512.  The call makes no hipMalloc, hipHostMalloc
 * or hipFree (ung_hip_stats::allocations stays 0); its host work lists reuse the
 * context's storage.  It needs the base set prepared beforehand (ung_hip_prepare_vectors,
 * which allocates, at set-up).  Calls on one GPU share that GPU's array: a per-device
 * lock held from the plan's upload to the end of its last kernel makes calls from
 * several host threads or contexts run one after the other.  The rows are not kept in
 * the context: afterwards the entry points that read the last cross-edge call's rows
 * (ung_hip_download_cross, ung_hip_cross_result_device, ung_hip_result_shape(0),
 * ung_hip_rescanned_rows(0), ung_hip_additional_edges, the diagnostics) return
 * UNG_HIP_ESTATE until the next allocating cross-edge call. */
int ung_hip_cross_topk_noalloc(ung_hip_ctx *ctx, uint32_t G, const uint32_t *group_begin,
                               const uint32_t *out_ptr, const uint32_t *out_idx, uint32_t k,
                               uint32_t *out_ids_dev, float *out_dist_dev, int32_t *out_size_dev,
                               ung_hip_stats *st);
int ung_hip_download_cross(ung_hip_ctx *ctx, uint32_t *out_ids, float *out_dist,
                           int32_t *out_size, ung_hip_stats *st);

/* Additional edges, exact variant.  Replaces
 * UniNavGraph::build_cross_edges_generate_additional (src/uni_nav_graph_cross_edges.cpp:
 * 442-596, UngAdditionalEdgesImpl::CpuExactScan branch :543-562; special blocks off):
 * for every group C the out-groups X (LNG row order) that no cross edge of C's members
 * reaches get edges from C's first vectors -- each vector the first num_cross/2 entries
 * of an exact (distance, id) SearchQueue(num_cross) over X -- until at least num_cross
 * edges were added for X or C has no more vectors.
 * Uses the cross-edge rows left in HBM by the last ung_hip_cross_topk(_device) call (same
 * G, group_begin, out_ptr, out_idx; num_cross <= that call's k; its first num_cross
 * entries per row are read, as the reference reads its FlatId rows, :500-512).
 * Output (host memory): edge_ptr[G+2] CSR over groups 1..G (the materialized per-group
 * lists of the reference, edges of C in [edge_ptr[C], edge_ptr[C+1])), edge_from /
 * edge_to global new ids, in the reference's append order.  capacity = entries of
 * edge_from/edge_to; *n_edges receives the count; UNG_HIP_EINVAL (nothing written) when
 * capacity is too small.  group_begin[1] must be 0 and out_ptr[G+1] * 2 * num_cross must
 * stay below 2^32 (32-bit edge offsets); UNG_HIP_EINVAL otherwise. */
int ung_hip_additional_edges(ung_hip_ctx *ctx, uint32_t G, const uint32_t *group_begin,
                             const uint32_t *out_ptr, const uint32_t *out_idx, uint32_t num_cross,
                             uint32_t *edge_ptr, uint32_t *edge_from, uint32_t *edge_to,
                             uint64_t capacity, uint64_t *n_edges, ung_hip_stats *st);

/* Exact intra-group kNN for a batch of groups.  Replaces the exact list computed by
 * batched_exact_knn_graph_kernel (src/tagore_graph_builder.cu:650-728, host driver
 * build_fast_exact_cuda_batch :1058-1429) with the semantics of the CPU builder
 * build_exact_topk_graph_for_points (src/uni_nav_graph_special_blocks.cpp:70-111):
 * for every point i of group [grp_begin[g], grp_begin[g]+grp_size[g]) the first
 * min(list_k, n-1) LOCAL ids j != i ordered by (distance, j).
 * Rows are packed group after group (row offset of group g = sum of earlier sizes,
 * the packed_offsets of TagoreBatchBuildResult, include/tagore_graph_builder.h:80-88).
 * Output (host memory): out_ids [sum n x list_k] local ids, out_dist (nullable).
 * 1 <= list_k <= 64; n >= 1 per group. */
int ung_hip_group_knn(ung_hip_ctx *ctx, uint32_t n_groups, const uint32_t *grp_begin,
                      const uint32_t *grp_size, uint32_t list_k, uint32_t *out_ids,
                      float *out_dist, ung_hip_stats *st);

/* The cross-edge call (ung_hip_cross_topk_device) and a group kNN call
 * (ung_hip_group_knn_device) overlapped on the context's two streams.  No counterpart in
 * the reference, which runs build_cross_edges_generate_gpu_optimized
 * (src/uni_nav_graph_cross_edges.cpp:334-440) and the exact group batch
 * (src/uni_nav_graph_group_graph.cpp:643-738) one after the other; the results are those
 * of the two calls.  Returns when the cross-edge rows are complete (as
 * ung_hip_cross_topk_device); the group call keeps running until ung_hip_intra_end, and
 * meanwhile calls that read the group lists or replace the base set return
 * UNG_HIP_ESTATE.  Cross-edge calls and ung_hip_additional_edges may run in between. */
int ung_hip_cross_intra_begin(ung_hip_ctx *ctx, uint32_t G, const uint32_t *group_begin,
                              const uint32_t *out_ptr, const uint32_t *out_idx, uint32_t k,
                              uint32_t n_groups, const uint32_t *grp_begin, const uint32_t *grp_size,
                              uint32_t list_k, ung_hip_stats *st_cross);
/* Completes the group call of ung_hip_cross_intra_begin (its statistics into st). */
int ung_hip_intra_end(ung_hip_ctx *ctx, ung_hip_stats *st);

/* Device-resident variant of ung_hip_group_knn (results in context buffers). */
int ung_hip_group_knn_device(ung_hip_ctx *ctx, uint32_t n_groups, const uint32_t *grp_begin,
                             const uint32_t *grp_size, uint32_t list_k, ung_hip_stats *st);
int ung_hip_group_result_device(ung_hip_ctx *ctx, uint32_t **ids_dev, float **dist_dev,
                                uint64_t *rows);
int ung_hip_download_group(ung_hip_ctx *ctx, uint32_t *out_ids, float *out_dist,
                           ung_hip_stats *st);

/* Shape of a resident result, for sizing the host buffers of the downloads, the packed
 * rows and the pruned rows: which = 0 the cross-edge rows (rows = N, k = the call's k,
 * n_groups = 0), which = 1 the group kNN lists of the last group call (rows = sum n,
 * k = list_k, n_groups = its group count).  Output pointers may be NULL.
 * UNG_HIP_ESTATE when there is no such result.  No counterpart in the reference, whose
 * results are std::vectors that carry their sizes. */
int ung_hip_result_shape(ung_hip_ctx *ctx, int which, uint64_t *rows, uint32_t *k, uint32_t *n_groups);

/* Output rows of the last cross-edge call (which = 0: point ids) or group kNN call
 * (which = 1: packed row indices) whose MFMA pre-selection could not be certified and
 * that were rescanned exactly (ung_hip_stats::fallback_rows of that call), ascending.
 * *n_rows receives the count; UNG_HIP_EINVAL (nothing written) when capacity is smaller.
 * Diagnostic for parity checks; the reference's sampled verifier
 * (src/gpu_cross_edge_verify.cuh:38-203) has no such list. */
int ung_hip_rescanned_rows(ung_hip_ctx *ctx, int which, uint32_t *rows, uint64_t capacity, uint64_t *n_rows);

/* Exact-anchor row packing of the last ung_hip_group_knn(_device) result, on the
 * device.  Same rows as batched_exact_knn_graph_kernel's epilogue
 * (src/tagore_graph_builder.cu:727-794) with its defaults from
 * make_fast_exact_batch_config (src/tagore_cuda_config.cpp:23-48):
 * row = [out_degree, ids...] with graph_stride = final_degree + 1 entries,
 * cand_degree = min(64, tagore_k - 1, n - 1), out_degree = min(final_degree, cand_degree).
 * The packer reads list positions < cand_degree; the last kNN call must have
 * produced list_k >= cand_degree, except when anchor_tail=1 and anchor_slots=0,
 * where only positions < min(head_keep, final_degree) are read (the anchors always
 * fill the row) and list_k >= that is enough.
 * out_graph (host): [sum n x graph_stride] uint32; entry_points (nullable):
 * [n_groups] (always 0, as the reference's kernel writes). */
int ung_hip_pack_anchor_rows(ung_hip_ctx *ctx, uint32_t tagore_k, uint32_t final_degree,
                             uint32_t head_keep, uint32_t anchor_tail, uint32_t anchor_slots,
                             uint32_t bidir_anchor, uint32_t *out_graph, uint32_t *entry_points,
                             ung_hip_stats *st);

/* Graph of groups too large for the exact batch (n above exact_max_nx), from the last
 * ung_hip_group_knn(_device) result (exact lists, list_k = min(64, tagore_k - 1)).  Replaces
 * build_tagore_vamana_cuda_batch's FastGrnnd path (src/tagore_graph_builder.cu:1777-2159):
 * its candidate graph comes from the un-vendored NN-descent (here: the exact lists), and its
 * prune launch_fast_grnnd_prune_impl (:1463-1568) is restated:
 *  - reverse edges (build_sampled_reverse_kernel :141-163): source s is a reverse candidate
 *    of each of its first forward_cap list entries; of those, each point keeps the
 *    reverse_cap nearest by (dist, source id) (the reference keeps the first reverse_cap
 *    arrivals of an atomic counter, which depend on the run);
 *  - fast_grnnd_prune_kernel (:279-387): forward (first forward_cap entries) and reverse
 *    candidates by (dist, id) without duplicates, then a greedy scan keeps a candidate unless
 *    alpha * d(kept, candidate) < d(point, candidate) for a kept one, up to final_degree
 *    (distances in the reference's fp32 summation order; the reference prunes on fp16
 *    copies).
 * Defaults of make_fast_grnnd_prune_config (src/tagore_cuda_config.cpp:45-68) for tagore_k =
 * 64, final_degree = 32: forward_cap = 63, reverse_cap = 32.
 * out_graph (host): [sum n x (final_degree + 1)]: [count, local ids..., padded with the
 * point's own id]; entry_points (nullable): [n_groups], 0 (the reference clears ep_dev,
 * :2036).  1 <= final_degree <= 64, reverse_cap <= 32, 1 <= forward_cap <= list_k. */
int ung_hip_prune_group_graph(ung_hip_ctx *ctx, uint32_t forward_cap, uint32_t reverse_cap,
                              uint32_t final_degree, float alpha, uint32_t *out_graph,
                              uint32_t *entry_points, ung_hip_stats *st);

/* Synchronise the context's stream (for callers timing the device variants). */
int ung_hip_synchronize(ung_hip_ctx *ctx);

/* Device-side self test of the bf16 MFMA fragment layout the kernels rely on
 * (v_mfma_f32_32x32x16_bf16; diagnostic, no counterpart in the reference).  *max_abs_err receives the
 * largest deviation from a host-computed product; returns 0 when it ran. */
int ung_hip_selftest_mfma(ung_hip_ctx *ctx, double *max_abs_err);

/* Diagnostic, no counterpart in the reference: the approximate (split-bf16 MFMA,
 * expansion-form) distances behind the context's last cross-edge call or synchronous
 * group kNN call (ung_hip_group_knn, ung_hip_group_knn_device), for checking the
 * certified error bound against exact distances.  Writes one entry per partial-row
 * candidate -- query id, candidate id (global ids), approximate squared distance a --
 * and the bound's constants: |a - D| <= eps_coef * (|q| + rmax)^2 for the exact squared
 * distance D.  Tiny jobs (scanned exactly) have no entries.  *n_entries receives the
 * count; a capacity below it returns UNG_HIP_EINVAL (query/cand/approx may be NULL to
 * ask for the count).  UNG_HIP_ESTATE when the last call on the context's first
 * workspace was neither of those (ung_hip_cross_topk, ung_hip_cross_topk_device,
 * ung_hip_cross_intra_begin, ung_hip_group_knn, ung_hip_group_knn_device). */
int ung_hip_debug_partial_rows(ung_hip_ctx *ctx, uint64_t capacity, uint32_t *query, uint32_t *cand, float *approx,
                               uint64_t *n_entries, double *eps_coef, double *rmax);

/* Diagnostic, no counterpart in the reference: the bound of every partial row of the same
 * call (the select's contract: every candidate of the row's split that the row does not
 * hold has an approximate distance a >= bound, so an exact distance D >= bound -
 * eps_coef * (|q| + rmax)^2).  One row per (query, split): query id, the split's
 * candidates as the global id range [cand_begin, cand_end) when the job's union is one
 * range (every group kNN job; UINT32_MAX for multi-range cross unions), and the bound
 * (+inf: the split holds no candidate past the row).  *n_rows receives the count; a
 * capacity below it returns UNG_HIP_EINVAL.  UNG_HIP_ESTATE as above. */
int ung_hip_debug_partial_bounds(ung_hip_ctx *ctx, uint64_t capacity, uint32_t *query, uint32_t *cand_begin,
                                 uint32_t *cand_end, float *bound, uint64_t *n_rows);

/* ---------------------------------------------------------------------------
 * Output boundary (CPU, multi-threaded C++).
 * ------------------------------------------------------------------------- */

/* The final adjacency as CSR: replaces the per-point NeighborList fill of
 * add_offset_for_uni_nav_graph (src/uni_nav_graph.cpp:285-297),
 * merge_cross_edges_to_graph + merge_additional_edges_to_graph
 * (src/uni_nav_graph_cross_edges.cpp:849-868) and the writer's build_csr_adjacency
 * (src/ung_cross_edge_output_writer.cpp:44-66, :104-147).  Row i = the intra-group
 * edges of i (intra_ptr[N+1] / intra_idx, group-local ids plus the group's first id
 * unless intra_global), then the first num_cross entries of its FlatId cross row
 * (cross_ids [N x cross_stride], UINT32_MAX skipped; cross_ids may be NULL), then its
 * additional edges in list order (add_ptr[G+2] CSR over groups as written by
 * ung_hip_additional_edges; each group's list holds edges from its own points; may be
 * NULL).  Output: row_ptr[N+1], col_idx (capacity entries); *n_entries = entries needed;
 * UNG_HIP_EINVAL when capacity is too small. */
int ung_assemble_graph_csr(uint64_t N, uint32_t G, const uint32_t *group_begin, const uint64_t *intra_ptr,
                           const uint32_t *intra_idx, int intra_global, const uint32_t *cross_ids,
                           uint32_t cross_stride, uint32_t num_cross, const uint32_t *add_ptr,
                           const uint32_t *add_from, const uint32_t *add_to, uint64_t *row_ptr,
                           uint32_t *col_idx, uint64_t capacity, uint64_t *n_entries, int nthreads);

/* Graph::save text format (include/graph.h:207-216): one line per point,
 * "i n1 n2 ... \n" with a space after every number, rows from a CSR. */
int ung_graph_save_text(const char *path, uint64_t N, const uint64_t *row_ptr, const uint32_t *col_idx,
                        int nthreads);

/* ---------------------------------------------------------------------------
 * Host-side inputs of the path (CPU, multi-threaded C++).
 * ------------------------------------------------------------------------- */

/* Group division by exact label set in first-appearance order + reorder.
 * Replaces UniNavGraph::build_trie_and_divide_groups
 * (src/uni_nav_graph_label_graph.cpp:21-43) and the id bookkeeping of
 * prepare_group_storages_graphs (src/uni_nav_graph.cpp:148-166).
 * in : lab_ptr[N+1], lab_idx: per-point label lists, each sorted ascending
 *      (src/storage.cpp:137-145).
 * out: point_group[N] (group of each ORIGINAL point), group_begin[N+2] (first G+2
 *      used), new_to_old[N]; *G_out = number of groups.
 * Group label sets (CSR over groups, needed by ung_lng_build) are returned by
 * ung_group_label_sets. */
int ung_divide_groups(uint64_t N, const uint32_t *lab_ptr, const uint32_t *lab_idx,
                      uint32_t *point_group, uint32_t *group_begin, uint32_t *new_to_old,
                      uint32_t *G_out);

/* Label set of each group as CSR over groups 1..G: set_ptr[G+2], set_idx[cap]. */
int ung_group_label_sets(uint64_t N, const uint32_t *lab_ptr, const uint32_t *lab_idx,
                         const uint32_t *group_begin, const uint32_t *new_to_old, uint32_t G,
                         uint32_t *set_ptr, uint32_t *set_idx, uint64_t set_cap);

/* Label navigating graph: out(C) = minimum proper supersets among the groups.
 * Replaces build_label_nav_graph phase 1 (src/uni_nav_graph_label_graph.cpp:851-911,
 * get_min_super_sets :45-206 with TrieIndex::get_super_set_entrances
 * src/trie.cpp:78-143).  out_ptr[G+2]; out_idx capacity out_cap.  Each row is in the
 * reference's order: by label-set size, and within one size in the discovery order of
 * the reference's trie walk (get_min_super_sets_optimized_bucket,
 * src/uni_nav_graph_label_graph.cpp:103-206, whose groups are inserted in first-appearance
 * order); rows whose candidate label-set sizes span more than 256 are sorted by the
 * reference with an unstable std::sort and keep the walk order here.  *n_edges receives
 * the edge count; returns UNG_HIP_EINVAL with *n_edges set to the needed capacity when
 * out_cap is too small. */
int ung_lng_build(uint32_t G, const uint32_t *set_ptr, const uint32_t *set_idx,
                  uint32_t *out_ptr, uint32_t *out_idx, uint64_t out_cap, uint64_t *n_edges,
                  int nthreads);

/* Reorder rows: dst[i] = src[new_to_old[i]] (storage.cpp:206-228). */
int ung_reorder_rows(const float *src, uint64_t N, uint32_t dim, const uint32_t *new_to_old,
                     float *dst, int nthreads);

/* Algorithmic work of the path (distance pairs, no padding):
 *   P_cross = sum_{C: out(C) non-empty} |C| * sum_{X in out(C)} |X|
 *   P_intra = sum over groups with lo <= n <= hi of n*(n-1). */
int ung_count_pairs(uint32_t G, const uint32_t *group_begin, const uint32_t *out_ptr,
                    const uint32_t *out_idx, uint32_t intra_lo, uint32_t intra_hi,
                    uint64_t *p_cross, uint64_t *p_intra);

/* Seeded synthetic inputs (deterministic on any host; no libm transcendental
 * calls).  Vectors: centroids c_j ~ N(0, centroid_scale^2 I) (n_centroids of them,
 * seed_c), x_i = c_{u_i} + sigma * N(0, I) with u_i uniform (seed_x); n_centroids = 0
 * gives i.i.d. N(0, 1) rows from seed_x; normalize != 0 scales rows to unit L2.
 * Labels (seed_l): mode 0 = each point draws m ~ U{m_min..m_max} labels from
 * 1..vocab without replacement with P(r) ~ r^-zipf_s; mode 1 = hierarchical: one
 * parent label 1+p, p ~ U{0..9}, plus c ~ U{0..3} child labels drawn uniformly
 * without replacement from 11+9p..19+9p.  Rows sorted ascending.
 * lab_idx capacity must be N*m_max (mode 0) or N*4 (mode 1). */
int ung_synth_vectors(uint64_t N, uint32_t dim, uint32_t n_centroids, float centroid_scale,
                      float sigma, int normalize, uint64_t seed_c, uint64_t seed_x, float *X,
                      int nthreads);
int ung_synth_labels(uint64_t N, int mode, uint32_t vocab, uint32_t m_min, uint32_t m_max,
                     double zipf_s, uint64_t seed_l, uint32_t *lab_ptr, uint32_t *lab_idx,
                     int nthreads);

#ifdef __cplusplus
}
#endif

#endif /* UNG_HIP_H */
