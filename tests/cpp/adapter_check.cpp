// adapter_check.cpp -- runs the header-only C++ adapter (include/ung_hip_adapter.hpp)
// against libung_hip.so the way the reference's call sites would
// (src/uni_nav_graph_cross_edges.cpp:380-392, src/uni_nav_graph_group_graph.cpp:643-738):
// the reference's containers in, its output shapes out.  Test infrastructure: the GPU test
// tests/test_gpu_adapter.py writes the inputs, runs this program and checks every output
// against the CPU oracle.
//
// usage: adapter_check <dir>
//   in : meta.txt ("N dim G topk final_degree tagore_k head_keep alpha n_mid n_large"),
//        X.f32 [N x dim], group_begin.u32 [G+2], out_ptr.u32 [G+2], out_idx.u32,
//        mid.u32 / large.u32 ([n x 2]: begin, size of each group of the batch)
//   out: flat_ids.u32, flat_dists.f32 (FlatId writeback), idvec_ptr.u64 + idvec.u32
//        (IdVector writeback), sink.bin ((point, id, dist) triples in SearchQueue-sink
//        order), addl_ptr.u32 + addl.u32 (materialized (from, to) pairs per group),
//        exact_ids.u32, exact_dists.f32, packed.u32, packed_offsets.u32, entry.u32 (exact
//        batch), large_packed.u32, large_entry.u32 (large-group batch)
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <string>
#include <vector>

#include "ung_hip_adapter.hpp"

namespace {

template <class T>
std::vector<T> read_vec(const std::string &path)
{
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f)
        throw std::runtime_error("cannot open " + path);
    const std::streamsize bytes = f.tellg();
    f.seekg(0);
    std::vector<T> v((size_t)bytes / sizeof(T));
    if (bytes > 0 && !f.read(reinterpret_cast<char *>(v.data()), bytes))
        throw std::runtime_error("cannot read " + path);
    return v;
}

template <class T>
void write_vec(const std::string &path, const std::vector<T> &v)
{
    std::ofstream f(path, std::ios::binary);
    if (!f || (!v.empty() && !f.write(reinterpret_cast<const char *>(v.data()), (std::streamsize)(v.size() * sizeof(T)))))
        throw std::runtime_error("cannot write " + path);
}

std::vector<std::pair<uint32_t, uint32_t>> read_batch(const std::string &path)
{
    const auto raw = read_vec<uint32_t>(path);
    std::vector<std::pair<uint32_t, uint32_t>> out;
    for (size_t i = 0; i + 1 < raw.size(); i += 2)
        out.emplace_back(raw[i], raw[i + 1]);
    return out;
}

} // namespace

int main(int argc, char **argv)
{
    if (argc != 2) {
        std::cerr << "usage: adapter_check <dir>\n";
        return 2;
    }
    const std::string dir = std::string(argv[1]) + "/";
    try {
        uint64_t N = 0;
        uint32_t dim = 0, G = 0, topk = 0, final_degree = 0, tagore_k = 0, head_keep = 0, n_mid = 0, n_large = 0;
        float alpha = 0.0f;
        {
            std::ifstream m(dir + "meta.txt");
            if (!(m >> N >> dim >> G >> topk >> final_degree >> tagore_k >> head_keep >> alpha >> n_mid >> n_large))
                throw std::runtime_error("bad meta.txt");
        }
        const auto X = read_vec<float>(dir + "X.f32");
        const auto group_begin = read_vec<uint32_t>(dir + "group_begin.u32");
        const auto out_ptr = read_vec<uint32_t>(dir + "out_ptr.u32");
        const auto out_idx = read_vec<uint32_t>(dir + "out_idx.u32");
        if (X.size() != N * dim || group_begin.size() != G + 2 || out_ptr.size() != G + 2)
            throw std::runtime_error("input sizes do not match meta.txt");

        // the reference's containers: _group_id_to_range and _label_nav_graph->out_neighbors
        ung_hip::GroupRanges ranges(G + 1);
        ung_hip::GroupRows out_neighbors(G + 1);
        std::vector<uint32_t> targets;
        std::vector<char> has_in(G + 2, 0);
        for (uint32_t g = 1; g <= G; ++g) {
            ranges[g] = {group_begin[g], group_begin[g + 1]};
            out_neighbors[g].assign(out_idx.begin() + out_ptr[g], out_idx.begin() + out_ptr[g + 1]);
            for (uint32_t x : out_neighbors[g])
                has_in[x] = 1;
        }
        for (uint32_t g = 1; g <= G; ++g) // the reference passes the groups with in-neighbours
            if (has_in[g])
                targets.push_back(g);

        ung_hip::Backend backend(0);
        backend.prepare_all_vectors_on_device(X.data(), N, dim);

        std::vector<uint32_t> flat_ids;
        std::vector<float> flat_dists;
        std::vector<std::vector<uint32_t>> id_vectors;
        backend.cross_groups_search_all_batched(targets, (int)topk, ranges, out_neighbors, &flat_ids, &flat_dists,
                                                &id_vectors);
        write_vec(dir + "flat_ids.u32", flat_ids);
        write_vec(dir + "flat_dists.f32", flat_dists);
        std::vector<uint64_t> idvec_ptr(N + 1, 0);
        std::vector<uint32_t> idvec;
        for (uint64_t p = 0; p < N; ++p) {
            idvec.insert(idvec.end(), id_vectors[p].begin(), id_vectors[p].end());
            idvec_ptr[p + 1] = idvec.size();
        }
        write_vec(dir + "idvec_ptr.u64", idvec_ptr);
        write_vec(dir + "idvec.u32", idvec);

        // SearchQueue writeback: the sink sees each point's edges in (dist, id) order
        std::vector<uint32_t> sink;
        backend.for_each_cross_edge([&](uint32_t p, uint32_t id, float d) {
            uint32_t bits;
            std::memcpy(&bits, &d, sizeof(bits));
            sink.push_back(p);
            sink.push_back(id);
            sink.push_back(bits);
        });
        write_vec(dir + "sink.bin", sink);

        std::vector<std::vector<std::pair<uint32_t, uint32_t>>> materialized;
        backend.cross_edges_generate_additional(ranges, out_neighbors, topk, materialized);
        std::vector<uint32_t> addl_ptr(G + 2, 0), addl;
        for (uint32_t c = 1; c <= G; ++c) {
            for (const auto &e : materialized[c]) {
                addl.push_back(e.first);
                addl.push_back(e.second);
            }
            addl_ptr[c + 1] = (uint32_t)(addl.size() / 2);
        }
        write_vec(dir + "addl_ptr.u32", addl_ptr);
        write_vec(dir + "addl.u32", addl);

        const auto mid = read_batch(dir + "mid.u32");
        const auto large = read_batch(dir + "large.u32");
        if (mid.size() != n_mid || large.size() != n_large)
            throw std::runtime_error("batch sizes do not match meta.txt");
        const auto ex = backend.build_fast_exact_batch(mid, tagore_k, final_degree, head_keep);
        write_vec(dir + "exact_ids.u32", ex.exact_ids);
        write_vec(dir + "exact_dists.f32", ex.exact_dists);
        write_vec(dir + "packed.u32", ex.packed_graph);
        write_vec(dir + "packed_offsets.u32", ex.packed_offsets);
        write_vec(dir + "entry.u32", ex.entry_points);
        const auto lg = backend.build_large_group_batch(large, tagore_k, final_degree, alpha);
        write_vec(dir + "large_packed.u32", lg.packed_graph);
        write_vec(dir + "large_entry.u32", lg.entry_points);
        std::cout << "adapter_check ok: " << N << " points, " << flat_ids.size() / (topk ? topk : 1) << " cross rows, "
                  << addl.size() / 2 << " additional edges, " << ex.packed_offsets.back() << " exact-batch rows, "
                  << lg.packed_graph.size() / (final_degree + 1) << " large-batch rows" << std::endl;
    } catch (const std::exception &e) {
        std::cerr << "adapter_check failed: " << e.what() << std::endl;
        return 1;
    }
    return 0;
}
