// ung_hip_adapter.hpp -- header-only C++ adapter over the C ABI (ung_hip.h) that
// keeps the shapes of the reference's C++ call sites of this stage, so the
// reference's UniNavGraph can call it with its own containers.  Errors throw
// std::runtime_error, as the reference's GPU route does
// (src/gpu_cross_edge_buffers.cuh:86-100; caught in
// src/uni_nav_graph_cross_edges.cpp:394-420 for the CPU fallback).
//
// Paths are relative to UNG/codes/ of panjd123/FilterVectorCode_refactor.
#pragma once

#include <algorithm>
#include <cstdint>
#include <exception>
#include <limits>
#include <stdexcept>
#include <string>
#include <thread>
#include <utility>
#include <vector>

#include "ung_hip.h"

namespace ung_hip {

inline void throw_if(int rc, const char *what)
{
    if (rc != UNG_HIP_OK)
        throw std::runtime_error(std::string(what) + ": " + ung_hip_last_error());
}

// Group ranges indexed by group id (entry 0 unused), as UniNavGraph::_group_id_to_range.
using GroupRanges = std::vector<std::pair<uint32_t, uint32_t>>;
// LNG rows indexed by group id, as LabelNavGraph::out_neighbors.
using GroupRows = std::vector<std::vector<uint32_t>>;

struct ExactBatchResult {
    // Mirrors TagoreBatchBuildResult (include/tagore_graph_builder.h:80-88).
    std::vector<uint32_t> packed_graph;   // [sum n x packed_graph_stride]
    std::vector<uint32_t> packed_offsets; // [n_groups + 1]
    uint32_t packed_graph_stride = 0;
    std::vector<uint32_t> entry_points;   // [n_groups]
    std::vector<uint32_t> exact_ids;      // [sum n x list_k] local ids, (dist,id) order
    std::vector<float> exact_dists;
    uint32_t list_k = 0;
    ung_hip_stats stats{};
};

class Backend {
  public:
    explicit Backend(int device = 0) { throw_if(ung_hip_create(device, &ctx_), "ung_hip_create"); }
    ~Backend() { ung_hip_destroy(ctx_); }
    Backend(const Backend &) = delete;
    Backend &operator=(const Backend &) = delete;

    // UniNavGraph::gpu_prepare_all_vectors_on_device (include/uni_nav_graph.h:430-432):
    // the reordered base set, [N x dim] row-major fp32.
    void prepare_all_vectors_on_device(const float *X, uint64_t N, uint32_t dim)
    {
        throw_if(ung_hip_prepare_vectors(ctx_, X, N, dim, &last_), "prepare_all_vectors_on_device");
        N_ = N;
    }

    // UniNavGraph::gpu_release_all_vectors_on_device (include/uni_nav_graph.h:433).
    void release_all_vectors_on_device() { throw_if(ung_hip_release_vectors(ctx_), "release_all_vectors_on_device"); }

    // UniNavGraph::gpu_cross_groups_search_all_batched (include/uni_nav_graph.h:436-444).
    // target_group_ids: the targets X to scan (the reference passes every group with
    // in-neighbours); out_neighbors: LNG out rows.  Results go to whichever outputs
    // are non-null: flat_ids ([N x topk], UINT32_MAX padding: the FlatId writeback),
    // id_vectors (IdVector writeback), flat_dists (fp32 distances).  For SearchQueue
    // writeback call for_each_cross_edge() afterwards.
    void cross_groups_search_all_batched(const std::vector<uint32_t> &target_group_ids, int topk,
                                         const GroupRanges &group_id_to_range, const GroupRows &out_neighbors,
                                         std::vector<uint32_t> *flat_ids, std::vector<float> *flat_dists,
                                         std::vector<std::vector<uint32_t>> *id_vectors)
    {
        const uint32_t G = (uint32_t)group_id_to_range.size() - 1;
        std::vector<uint32_t> group_begin(G + 2, 0);
        for (uint32_t g = 1; g <= G; ++g) {
            if (group_id_to_range[g].first != group_begin[g])
                throw std::runtime_error("cross_groups_search_all_batched: groups must be contiguous in id order");
            group_begin[g + 1] = group_id_to_range[g].second;
        }
        std::vector<char> is_target(G + 2, 0);
        for (uint32_t x : target_group_ids)
            if (x >= 1 && x <= G)
                is_target[x] = 1;
        std::vector<uint32_t> out_ptr(G + 2, 0), out_idx;
        for (uint32_t c = 1; c <= G; ++c) {
            if (c < out_neighbors.size())
                for (uint32_t x : out_neighbors[c])
                    if (x <= G && is_target[x])
                        out_idx.push_back(x);
            out_ptr[c + 1] = (uint32_t)out_idx.size();
        }
        const uint64_t N = group_begin[G + 1];
        k_ = (uint32_t)topk;
        last_ = ung_hip_stats{};
        throw_if(ung_hip_cross_topk_device(ctx_, G, group_begin.data(), out_ptr.data(),
                                           out_idx.empty() ? nullptr : out_idx.data(), k_, &last_),
                 "cross_groups_search_all_batched");
        // the rows go straight into the caller's vectors (no second host copy): ids into
        // flat_ids when given (else the adapter's own buffer), distances into flat_dists;
        // for_each_cross_edge fetches ids and distances again when it needs them
        have_rows_ = false;
        sizes_.resize(N);
        std::vector<uint32_t> *ids = flat_ids ? flat_ids : &ids_;
        ids->resize(N * k_);
        if (flat_dists)
            flat_dists->resize(N * k_);
        throw_if(ung_hip_download_cross(ctx_, ids->data(), flat_dists ? flat_dists->data() : nullptr, sizes_.data(),
                                        &last_),
                 "cross_groups_search_all_batched (download)");
        if (id_vectors) {
            // IdVector writeback, rows filled in parallel (part 0 on this thread; an
            // exception of any part is rethrown here after every thread has joined)
            id_vectors->assign(N, {});
            const uint32_t *src = ids->data();
            const unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
            std::vector<std::exception_ptr> err(nt);
            auto fill = [&](unsigned t) {
                try {
                    for (uint64_t p = N * t / nt; p < N * (t + 1) / nt; ++p)
                        (*id_vectors)[p].assign(src + p * k_, src + p * k_ + sizes_[p]);
                } catch (...) {
                    err[t] = std::current_exception();
                }
            };
            std::vector<std::thread> pool;
            pool.reserve(nt);
            for (unsigned t = 1; t < nt; ++t) {
                try {
                    pool.emplace_back(fill, t);
                } catch (...) {
                    fill(t); // no thread to spare: this part runs here
                }
            }
            fill(0);
            for (auto &th : pool)
                th.join();
            for (const auto &e : err)
                if (e)
                    std::rethrow_exception(e);
        }
    }

    // SearchQueue writeback: sink(point, id, dist) for every cross edge, in
    // (dist, id) order per point -- e.g. [&](auto p, auto id, auto d){ queues[p].insert(id, d); }.
    // Reads the rows of the last cross_groups_search_all_batched call from the device.
    template <class Sink>
    void for_each_cross_edge(Sink &&sink)
    {
        if (!have_rows_) {
            ids_.resize(sizes_.size() * k_);
            dists_.resize(sizes_.size() * k_);
            throw_if(ung_hip_download_cross(ctx_, ids_.data(), dists_.data(), nullptr, &last_), "for_each_cross_edge");
            have_rows_ = true;
        }
        for (uint64_t p = 0; p < sizes_.size(); ++p)
            for (int32_t j = 0; j < sizes_[p]; ++j)
                sink((uint32_t)p, ids_[p * k_ + j], dists_[p * k_ + j]);
    }

    // UniNavGraph::build_cross_edges_generate_additional, exact variant
    // (src/uni_nav_graph_cross_edges.cpp:442-596) after cross_groups_search_all_batched:
    // materialized[C] = the (from, to) pairs appended for group C, in the reference's
    // order (materialized has G+1 entries; entry 0 is unused).
    void cross_edges_generate_additional(const GroupRanges &group_id_to_range, const GroupRows &out_neighbors,
                                         uint32_t num_cross_edges,
                                         std::vector<std::vector<std::pair<uint32_t, uint32_t>>> &materialized)
    {
        const uint32_t G = (uint32_t)group_id_to_range.size() - 1;
        std::vector<uint32_t> group_begin(G + 2, 0), out_ptr(G + 2, 0), out_idx;
        for (uint32_t g = 1; g <= G; ++g)
            group_begin[g + 1] = group_id_to_range[g].second;
        for (uint32_t c = 1; c <= G; ++c) {
            if (c < out_neighbors.size())
                out_idx.insert(out_idx.end(), out_neighbors[c].begin(), out_neighbors[c].end());
            out_ptr[c + 1] = (uint32_t)out_idx.size();
        }
        std::vector<uint32_t> edge_ptr(G + 2, 0), from, to;
        uint64_t n = 0, cap = group_begin[G + 1] / 8 + 1024;
        for (;;) {
            from.resize(cap);
            to.resize(cap);
            const int rc = ung_hip_additional_edges(ctx_, G, group_begin.data(), out_ptr.data(),
                                                    out_idx.empty() ? nullptr : out_idx.data(), num_cross_edges,
                                                    edge_ptr.data(), from.data(), to.data(), cap, &n, &last_);
            if (rc == UNG_HIP_EINVAL && n > cap) {
                cap = n;
                continue;
            }
            throw_if(rc, "cross_edges_generate_additional");
            break;
        }
        materialized.assign(G + 1, {});
        for (uint32_t c = 1; c <= G; ++c)
            for (uint32_t e = edge_ptr[c]; e < edge_ptr[c + 1]; ++e)
                materialized[c].emplace_back(from[e], to[e]);
    }

    // build_fast_exact_cuda_batch (src/tagore_graph_builder.cu:1058-1429) for groups
    // that are contiguous id ranges of the resident base set: exact top lists +
    // anchor-packed rows [deg, ids...] with stride final_degree+1.
    ExactBatchResult build_fast_exact_batch(const std::vector<std::pair<uint32_t, uint32_t>> &groups /*begin, n*/,
                                            uint32_t k, uint32_t final_degree, uint32_t head_keep,
                                            uint32_t anchor_tail = 1, uint32_t anchor_slots = 0,
                                            uint32_t bidir_anchor = 0)
    {
        ExactBatchResult r;
        if (k <= final_degree)
            k = final_degree + 1;
        std::vector<uint32_t> begin(groups.size()), size(groups.size());
        r.packed_offsets.assign(groups.size() + 1, 0);
        for (size_t i = 0; i < groups.size(); ++i) {
            begin[i] = groups[i].first;
            size[i] = groups[i].second;
            r.packed_offsets[i + 1] = r.packed_offsets[i] + size[i];
        }
        const uint64_t rows = r.packed_offsets.back();
        uint32_t list_k = (anchor_tail && anchor_slots == 0) ? final_degree : std::min<uint32_t>(64, k - 1);
        if (list_k > 64)
            list_k = 64;
        r.list_k = list_k;
        r.exact_ids.assign(rows * list_k, 0);
        r.exact_dists.assign(rows * list_k, 0.0f);
        throw_if(ung_hip_group_knn(ctx_, (uint32_t)groups.size(), begin.data(), size.data(), list_k,
                                   r.exact_ids.data(), r.exact_dists.data(), &r.stats),
                 "build_fast_exact_batch (kNN)");
        r.packed_graph_stride = final_degree + 1;
        r.packed_graph.assign(rows * r.packed_graph_stride, 0);
        r.entry_points.assign(groups.size(), 0);
        throw_if(ung_hip_pack_anchor_rows(ctx_, k, final_degree, head_keep, anchor_tail, anchor_slots, bidir_anchor,
                                          r.packed_graph.data(), r.entry_points.data(), &r.stats),
                 "build_fast_exact_batch (pack)");
        return r;
    }

    // The FastGrnnd batch of build_tagore_vamana_cuda_batch (src/tagore_graph_builder.cu:
    // 1777-2159) for groups above the exact batch: exact candidate lists of length
    // min(64, k-1) (in place of NN-descent) and the FastGrnnd prune with the caps of
    // make_fast_grnnd_prune_config (src/tagore_cuda_config.cpp:45-68).  Rows [count, local
    // ids...] with stride final_degree+1, entry points 0.
    ExactBatchResult build_large_group_batch(const std::vector<std::pair<uint32_t, uint32_t>> &groups /*begin, n*/,
                                             uint32_t k, uint32_t final_degree, float alpha)
    {
        ExactBatchResult r;
        if (k <= final_degree)
            k = final_degree + 1;
        std::vector<uint32_t> begin(groups.size()), size(groups.size());
        r.packed_offsets.assign(groups.size() + 1, 0);
        for (size_t i = 0; i < groups.size(); ++i) {
            begin[i] = groups[i].first;
            size[i] = groups[i].second;
            r.packed_offsets[i + 1] = r.packed_offsets[i] + size[i];
        }
        const uint64_t rows = r.packed_offsets.back();
        const uint32_t list_k = std::min<uint32_t>(64, k - 1);
        const uint32_t forward_cap = std::min(list_k, std::max(final_degree, 2 * final_degree));
        const uint32_t reverse_cap = std::min<uint32_t>(32, std::max<uint32_t>(1, final_degree));
        r.list_k = list_k;
        throw_if(ung_hip_group_knn_device(ctx_, (uint32_t)groups.size(), begin.data(), size.data(), list_k, &r.stats),
                 "build_large_group_batch (kNN)");
        r.packed_graph_stride = final_degree + 1;
        r.packed_graph.assign(rows * r.packed_graph_stride, 0);
        r.entry_points.assign(groups.size(), 0);
        throw_if(ung_hip_prune_group_graph(ctx_, forward_cap, reverse_cap, final_degree, alpha, r.packed_graph.data(),
                                           r.entry_points.data(), &r.stats),
                 "build_large_group_batch (prune)");
        return r;
    }

    const ung_hip_stats &last_stats() const { return last_; }
    ung_hip_ctx *handle() const { return ctx_; }

  private:
    ung_hip_ctx *ctx_ = nullptr;
    ung_hip_stats last_{};
    uint64_t N_ = 0;
    uint32_t k_ = 0;
    std::vector<uint32_t> ids_;
    std::vector<float> dists_;
    std::vector<int32_t> sizes_;
    bool have_rows_ = false; // ids_/dists_ hold the last search's rows
};

} // namespace ung_hip
