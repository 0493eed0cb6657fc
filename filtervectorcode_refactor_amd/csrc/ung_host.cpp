// ung_host.cpp -- CPU half of libung_hip.so: the inputs of the cross-edge /
// group-kNN path (synthetic data, group division, label navigating graph,
// reorder, work counting) and the error-message plumbing of the C ABI.
//
// Compiled with -ffp-contract=off so the synthetic generator is bit-reproducible
// on any x86-64 host (it uses only IEEE +,-,*,/ and sqrt).
#include "ung_hip.h"
#include "ung_internal.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>

#pragma STDC FP_CONTRACT OFF

namespace ung {

static thread_local std::string g_last_error;

void set_error(const char *fmt, ...)
{
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

// ---------------------------------------------------------------------------
// Deterministic random numbers: splitmix64 streams keyed by (seed, index), a
// log/exp built from IEEE arithmetic only, Marsaglia's polar method for normals.
// ---------------------------------------------------------------------------
static inline uint64_t splitmix64_next(uint64_t &s)
{
    uint64_t z = (s += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

static double det_log(double x)
{
    // x > 0.  x = m * 2^e with m in [sqrt(1/2), sqrt(2)); ln m = 2 atanh(z), z=(m-1)/(m+1)
    int e = 0;
    double m = std::frexp(x, &e); // m in [0.5, 1)
    if (m < 0.70710678118654752440) {
        m *= 2.0;
        e -= 1;
    }
    const double z = (m - 1.0) / (m + 1.0);
    const double z2 = z * z;
    double term = z, sum = 0.0;
    for (int n = 1; n < 60; n += 2) {
        const double add = term / (double)n;
        sum += add;
        if (std::fabs(add) < 1e-20)
            break;
        term *= z2;
    }
    return 2.0 * sum + (double)e * 0.69314718055994530942;
}

static double det_exp(double x)
{
    const double ln2 = 0.69314718055994530942;
    const double kf = std::floor(x / ln2 + 0.5);
    const double r = x - kf * ln2;
    double term = 1.0, sum = 1.0;
    for (int n = 1; n < 40; ++n) {
        term *= r / (double)n;
        sum += term;
        if (std::fabs(term) < 1e-20)
            break;
    }
    return std::ldexp(sum, (int)kf);
}

struct Rng {
    uint64_t s;
    bool has_spare = false;
    double spare = 0.0;
    Rng(uint64_t seed, uint64_t stream)
    {
        s = seed * 0xD1B54A32D192ED03ULL ^ (stream + 0x8CB92BA72F3D8DD7ULL) * 0x9E3779B97F4A7C15ULL;
        splitmix64_next(s);
    }
    uint64_t next() { return splitmix64_next(s); }
    double uniform() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); } // [0,1)
    uint32_t below(uint32_t n)
    {
        // multiply-shift on 32 random bits (n small, bias negligible and deterministic)
        return (uint32_t)(((next() >> 32) * (uint64_t)n) >> 32);
    }
    double normal()
    {
        if (has_spare) {
            has_spare = false;
            return spare;
        }
        for (;;) {
            const double u = 2.0 * uniform() - 1.0;
            const double v = 2.0 * uniform() - 1.0;
            const double s2 = u * u + v * v;
            if (s2 <= 0.0 || s2 >= 1.0)
                continue;
            const double f = std::sqrt(-2.0 * det_log(s2) / s2);
            spare = v * f;
            has_spare = true;
            return u * f;
        }
    }
};

} // namespace ung

using namespace ung;

extern "C" int ung_synth_vectors(uint64_t N, uint32_t dim, uint32_t n_centroids,
                                 float centroid_scale, float sigma, int normalize, uint64_t seed_c,
                                 uint64_t seed_x, float *X, int nthreads)
{
    clear_error();
    if (!X || dim == 0) {
        set_error("ung_synth_vectors: null X or dim == 0");
        return UNG_HIP_EINVAL;
    }
    std::vector<float> cent((size_t)n_centroids * dim);
    for (uint32_t j = 0; j < n_centroids; ++j) {
        Rng r(seed_c, j);
        for (uint32_t t = 0; t < dim; ++t)
            cent[(size_t)j * dim + t] = (float)((double)centroid_scale * r.normal());
    }
    parallel_for((int64_t)N, nthreads, 4096, [&](int64_t b, int64_t e) {
        std::vector<double> row(dim);
        for (int64_t i = b; i < e; ++i) {
            Rng r(seed_x, (uint64_t)i);
            if (n_centroids > 0) {
                const uint32_t u = r.below(n_centroids);
                const float *c = cent.data() + (size_t)u * dim;
                for (uint32_t t = 0; t < dim; ++t)
                    row[t] = (double)c[t] + (double)sigma * r.normal();
            } else {
                for (uint32_t t = 0; t < dim; ++t)
                    row[t] = r.normal();
            }
            float *out = X + (size_t)i * dim;
            if (normalize) {
                double ss = 0.0;
                for (uint32_t t = 0; t < dim; ++t)
                    ss += row[t] * row[t];
                const double inv = ss > 0.0 ? 1.0 / std::sqrt(ss) : 0.0;
                for (uint32_t t = 0; t < dim; ++t)
                    out[t] = (float)(row[t] * inv);
            } else {
                for (uint32_t t = 0; t < dim; ++t)
                    out[t] = (float)row[t];
            }
        }
    });
    return UNG_HIP_OK;
}

extern "C" int ung_synth_labels(uint64_t N, int mode, uint32_t vocab, uint32_t m_min,
                                uint32_t m_max, double zipf_s, uint64_t seed_l, uint32_t *lab_ptr,
                                uint32_t *lab_idx, int nthreads)
{
    clear_error();
    if (!lab_ptr || !lab_idx) {
        set_error("ung_synth_labels: null output");
        return UNG_HIP_EINVAL;
    }
    uint32_t width = 0;
    std::vector<double> cdf;
    if (mode == 0) {
        if (vocab == 0 || m_min == 0 || m_min > m_max || m_max > vocab) {
            set_error("ung_synth_labels: need 1 <= m_min <= m_max <= vocab");
            return UNG_HIP_EINVAL;
        }
        width = m_max;
        cdf.resize(vocab);
        double acc = 0.0;
        for (uint32_t r = 1; r <= vocab; ++r) {
            acc += det_exp(-zipf_s * det_log((double)r));
            cdf[r - 1] = acc;
        }
        for (auto &c : cdf)
            c /= acc;
    } else if (mode == 1) {
        width = 4;
    } else {
        set_error("ung_synth_labels: unknown mode %d", mode);
        return UNG_HIP_EINVAL;
    }
    // fixed-width staging, compacted afterwards
    std::vector<uint32_t> cnt(N);
    std::vector<uint32_t> tmp((size_t)N * width);
    parallel_for((int64_t)N, nthreads, 8192, [&](int64_t b, int64_t e) {
        for (int64_t i = b; i < e; ++i) {
            Rng r(seed_l, (uint64_t)i);
            uint32_t *row = tmp.data() + (size_t)i * width;
            uint32_t m = 0;
            if (mode == 0) {
                const uint32_t want = m_min + r.below(m_max - m_min + 1);
                while (m < want) {
                    const double u = r.uniform();
                    uint32_t lab = (uint32_t)(std::upper_bound(cdf.begin(), cdf.end(), u) - cdf.begin()) + 1;
                    if (lab > vocab)
                        lab = vocab;
                    bool dup = false;
                    for (uint32_t t = 0; t < m; ++t)
                        dup |= (row[t] == lab);
                    if (!dup)
                        row[m++] = lab;
                }
            } else {
                const uint32_t p = r.below(10);
                row[m++] = 1 + p;
                const uint32_t c = r.below(4);
                uint32_t taken = 0;
                while (m < 1 + c) {
                    const uint32_t j = r.below(9);
                    if (taken & (1u << j))
                        continue;
                    taken |= 1u << j;
                    row[m++] = 11 + 9 * p + j;
                }
            }
            std::sort(row, row + m);
            cnt[i] = m;
        }
    });
    lab_ptr[0] = 0;
    for (uint64_t i = 0; i < N; ++i)
        lab_ptr[i + 1] = lab_ptr[i] + cnt[i];
    parallel_for((int64_t)N, nthreads, 65536, [&](int64_t b, int64_t e) {
        for (int64_t i = b; i < e; ++i)
            std::memcpy(lab_idx + lab_ptr[i], tmp.data() + (size_t)i * width, cnt[i] * sizeof(uint32_t));
    });
    return UNG_HIP_OK;
}

// ---------------------------------------------------------------------------
// Group division (first-appearance order of exact label sets) + reorder ids.
// ---------------------------------------------------------------------------
namespace {

struct SetKeyHash {
    size_t operator()(const std::pair<const uint32_t *, uint32_t> &k) const
    {
        uint64_t h = 1469598103934665603ULL ^ k.second;
        for (uint32_t i = 0; i < k.second; ++i) {
            h ^= k.first[i];
            h *= 1099511628211ULL;
            h ^= h >> 29;
        }
        return (size_t)h;
    }
};
struct SetKeyEq {
    bool operator()(const std::pair<const uint32_t *, uint32_t> &a,
                    const std::pair<const uint32_t *, uint32_t> &b) const
    {
        return a.second == b.second && std::equal(a.first, a.first + a.second, b.first);
    }
};

} // namespace

extern "C" int ung_divide_groups(uint64_t N, const uint32_t *lab_ptr, const uint32_t *lab_idx,
                                 uint32_t *point_group, uint32_t *group_begin,
                                 uint32_t *new_to_old, uint32_t *G_out)
{
    clear_error();
    if (!lab_ptr || !point_group || !group_begin || !new_to_old || !G_out || N >= 0xFFFFFFFFull) {
        set_error("ung_divide_groups: bad arguments");
        return UNG_HIP_EINVAL;
    }
    std::unordered_map<std::pair<const uint32_t *, uint32_t>, uint32_t, SetKeyHash, SetKeyEq> ids;
    ids.reserve(1024);
    uint32_t G = 0;
    for (uint64_t i = 0; i < N; ++i) {
        const uint32_t len = lab_ptr[i + 1] - lab_ptr[i];
        auto key = std::make_pair(lab_idx + lab_ptr[i], len);
        auto it = ids.find(key);
        if (it == ids.end()) {
            ++G;
            ids.emplace(key, G);
            point_group[i] = G;
        } else {
            point_group[i] = it->second;
        }
    }
    std::vector<uint32_t> count(G + 2, 0);
    for (uint64_t i = 0; i < N; ++i)
        count[point_group[i]]++;
    group_begin[0] = 0;
    group_begin[1] = 0;
    for (uint32_t g = 1; g <= G; ++g)
        group_begin[g + 1] = group_begin[g] + count[g];
    std::vector<uint32_t> fill(G + 2, 0);
    for (uint64_t i = 0; i < N; ++i) {
        const uint32_t g = point_group[i];
        new_to_old[group_begin[g] + fill[g]++] = (uint32_t)i;
    }
    *G_out = G;
    return UNG_HIP_OK;
}

extern "C" int ung_group_label_sets(uint64_t N, const uint32_t *lab_ptr, const uint32_t *lab_idx,
                                    const uint32_t *group_begin, const uint32_t *new_to_old,
                                    uint32_t G, uint32_t *set_ptr, uint32_t *set_idx,
                                    uint64_t set_cap)
{
    clear_error();
    (void)N;
    set_ptr[0] = 0;
    set_ptr[1] = 0;
    uint64_t total = 0;
    for (uint32_t g = 1; g <= G; ++g) {
        if (group_begin[g + 1] == group_begin[g]) {
            set_error("ung_group_label_sets: group %u is empty", g);
            return UNG_HIP_EINVAL;
        }
        const uint32_t p = new_to_old[group_begin[g]];
        const uint32_t len = lab_ptr[p + 1] - lab_ptr[p];
        if (total + len > set_cap) {
            set_error("ung_group_label_sets: set_idx capacity %llu too small", (unsigned long long)set_cap);
            return UNG_HIP_EINVAL;
        }
        std::memcpy(set_idx + total, lab_idx + lab_ptr[p], len * sizeof(uint32_t));
        total += len;
        set_ptr[g + 1] = (uint32_t)total;
    }
    return UNG_HIP_OK;
}

// ---------------------------------------------------------------------------
// Row order of the label navigating graph.
//
// The reference lists out(C) as the minimal supersets in label-set-size order, and
// within one size in the order its trie walk discovers them
// (get_min_super_sets_optimized_bucket, src/uni_nav_graph_label_graph.cpp:103-206,
// over TrieIndex::get_super_set_entrances, src/trie.cpp:78-143).  The walk is a
// breadth-first search that starts from the trie nodes carrying C's largest label L
// whose path holds all of C (in the order those nodes were created) and visits each
// node's children in the iteration order of its std::unordered_map.  Breadth-first
// order over that forest is lexicographic order of
//   (levels below the start node, creation index of the start node,
//    child rank at each level from the start node down),
// so the rows are sorted by (set size, that key).  The trie is rebuilt here from
// the group label sets in group id order (first appearance, which creates the nodes
// in the reference's order) with an std::unordered_map per node filled by the same
// sequence of insertions, which reproduces its iteration order.  An empty C starts
// from the root's children (the root's own rank path).
// ---------------------------------------------------------------------------
namespace {

struct LabelTrie {
    std::vector<uint32_t> parent, label, depth, rank, created; // per node (0 = root)
    std::vector<uint32_t> group_node;                          // per group id

    LabelTrie(uint32_t G, const uint32_t *set_ptr, const uint32_t *set_idx)
    {
        std::vector<std::unordered_map<uint32_t, uint32_t>> kids(1);
        std::unordered_map<uint32_t, uint32_t> made_with_label;
        parent.push_back(0);
        label.push_back(0);
        depth.push_back(0);
        created.push_back(0);
        group_node.assign((size_t)G + 1, 0);
        for (uint32_t g = 1; g <= G; ++g) {
            uint32_t cur = 0;
            for (uint32_t i = set_ptr[g]; i < set_ptr[g + 1]; ++i) {
                const uint32_t l = set_idx[i];
                auto it = kids[cur].find(l);
                if (it == kids[cur].end()) {
                    const uint32_t nd = (uint32_t)parent.size();
                    parent.push_back(cur);
                    label.push_back(l);
                    depth.push_back(depth[cur] + 1);
                    created.push_back(made_with_label[l]++);
                    kids[cur].emplace(l, nd);
                    kids.emplace_back();
                    cur = nd;
                } else {
                    cur = it->second;
                }
            }
            group_node[g] = cur;
        }
        rank.assign(parent.size(), 0);
        for (auto &m : kids) {
            uint32_t r = 0;
            for (const auto &kv : m)
                rank[kv.second] = r++;
        }
    }

    // key of group x in the row of a group whose largest label is L (has_L false: empty
    // label set): [depth(x), levels below the start node, start node's creation index,
    // child ranks from the start node down]
    void key(uint32_t x, bool has_L, uint32_t L, std::vector<uint32_t> &out) const
    {
        out.clear();
        uint32_t nd = group_node[x];
        const uint32_t dx = depth[nd];
        std::vector<uint32_t> &path = out; // ranks bottom-up, reversed below
        while (nd != 0 && !(has_L && label[nd] == L)) {
            path.push_back(rank[nd]);
            nd = parent[nd];
        }
        const uint32_t levels = (uint32_t)path.size();
        const uint32_t start = has_L ? created[nd] : 0;
        std::reverse(path.begin(), path.end());
        path.insert(path.begin(), {dx, levels, start});
    }
};

} // namespace

// ---------------------------------------------------------------------------
// Label navigating graph: minimum proper supersets.
// Candidates of C are found by intersecting label posting lists (every superset
// of C contains each of C's labels); they are scanned by increasing set size and
// a candidate is kept unless it contains an already-kept one, which yields
// exactly the minimal elements (a non-minimal superset contains a minimal one of
// smaller size).  Each row is then put in the reference's order (LabelTrie).
// ---------------------------------------------------------------------------
extern "C" int ung_lng_build(uint32_t G, const uint32_t *set_ptr, const uint32_t *set_idx,
                             uint32_t *out_ptr, uint32_t *out_idx, uint64_t out_cap,
                             uint64_t *n_edges, int nthreads)
{
    clear_error();
    if (!set_ptr || !out_ptr || !n_edges) {
        set_error("ung_lng_build: null argument");
        return UNG_HIP_EINVAL;
    }
    uint32_t max_label = 0;
    for (uint64_t i = 0; i < set_ptr[G + 1]; ++i)
        max_label = std::max(max_label, set_idx[i]);
    const bool use_bits = max_label < 4096;
    const uint32_t W = use_bits ? (max_label / 64 + 1) : 0;
    std::vector<uint64_t> bits(use_bits ? (size_t)(G + 1) * W : 0, 0);
    if (use_bits)
        for (uint32_t g = 1; g <= G; ++g)
            for (uint32_t i = set_ptr[g]; i < set_ptr[g + 1]; ++i)
                bits[(size_t)g * W + set_idx[i] / 64] |= 1ull << (set_idx[i] % 64);
    auto len_of = [&](uint32_t g) { return set_ptr[g + 1] - set_ptr[g]; };
    auto subset = [&](uint32_t a, uint32_t b) -> bool { // labels(a) subset-of labels(b)
        if (use_bits) {
            const uint64_t *pa = bits.data() + (size_t)a * W, *pb = bits.data() + (size_t)b * W;
            for (uint32_t w = 0; w < W; ++w)
                if (pa[w] & ~pb[w])
                    return false;
            return true;
        }
        return std::includes(set_idx + set_ptr[b], set_idx + set_ptr[b + 1], set_idx + set_ptr[a],
                             set_idx + set_ptr[a + 1]);
    };
    // postings: label -> groups containing it (ascending group id)
    std::unordered_map<uint32_t, std::vector<uint32_t>> post;
    for (uint32_t g = 1; g <= G; ++g)
        for (uint32_t i = set_ptr[g]; i < set_ptr[g + 1]; ++i)
            post[set_idx[i]].push_back(g);
    std::vector<uint32_t> all_groups(G);
    for (uint32_t g = 1; g <= G; ++g)
        all_groups[g - 1] = g;

    const LabelTrie trie(G, set_ptr, set_idx);
    std::vector<std::vector<uint32_t>> rows(G + 1);
    parallel_for((int64_t)G, nthreads, 64, [&](int64_t b, int64_t e) {
        std::vector<uint32_t> cand, kept;
        std::vector<std::pair<std::vector<uint32_t>, uint32_t>> keyed;
        for (int64_t gi = b; gi < e; ++gi) {
            const uint32_t c = (uint32_t)gi + 1;
            const uint32_t lc = len_of(c);
            const std::vector<uint32_t> *base = &all_groups;
            for (uint32_t i = set_ptr[c]; i < set_ptr[c + 1]; ++i) {
                auto it = post.find(set_idx[i]);
                if (it->second.size() < base->size())
                    base = &it->second;
            }
            cand.clear();
            for (uint32_t x : *base)
                if (x != c && len_of(x) > lc && subset(c, x))
                    cand.push_back(x);
            std::stable_sort(cand.begin(), cand.end(),
                             [&](uint32_t a, uint32_t bb) { return len_of(a) < len_of(bb); });
            kept.clear();
            for (uint32_t x : cand) {
                bool minimal = true;
                for (uint32_t y : kept)
                    if (len_of(y) < len_of(x) && subset(y, x)) {
                        minimal = false;
                        break;
                    }
                if (minimal)
                    kept.push_back(x);
            }
            if (kept.size() > 1) {
                const bool has_L = lc > 0;
                const uint32_t L = has_L ? set_idx[set_ptr[c + 1] - 1] : 0;
                keyed.resize(kept.size());
                for (size_t i = 0; i < kept.size(); ++i) {
                    trie.key(kept[i], has_L, L, keyed[i].first);
                    keyed[i].second = kept[i];
                }
                std::sort(keyed.begin(), keyed.end());
                for (size_t i = 0; i < kept.size(); ++i)
                    kept[i] = keyed[i].second;
            }
            rows[c] = kept;
        }
    });
    uint64_t total = 0;
    for (uint32_t g = 1; g <= G; ++g)
        total += rows[g].size();
    *n_edges = total;
    if (total > out_cap || (total > 0 && !out_idx)) {
        set_error("ung_lng_build: out_idx capacity %llu < %llu edges", (unsigned long long)out_cap,
                  (unsigned long long)total);
        return UNG_HIP_EINVAL;
    }
    out_ptr[0] = 0;
    out_ptr[1] = 0;
    uint64_t pos = 0;
    for (uint32_t g = 1; g <= G; ++g) {
        std::copy(rows[g].begin(), rows[g].end(), out_idx + pos);
        pos += rows[g].size();
        out_ptr[g + 1] = (uint32_t)pos;
    }
    return UNG_HIP_OK;
}

extern "C" int ung_reorder_rows(const float *src, uint64_t N, uint32_t dim,
                                const uint32_t *new_to_old, float *dst, int nthreads)
{
    clear_error();
    if (!src || !dst || !new_to_old) {
        set_error("ung_reorder_rows: null argument");
        return UNG_HIP_EINVAL;
    }
    parallel_for((int64_t)N, nthreads, 16384, [&](int64_t b, int64_t e) {
        for (int64_t i = b; i < e; ++i)
            std::memcpy(dst + (size_t)i * dim, src + (size_t)new_to_old[i] * dim, dim * sizeof(float));
    });
    return UNG_HIP_OK;
}

extern "C" int ung_count_pairs(uint32_t G, const uint32_t *group_begin, const uint32_t *out_ptr,
                               const uint32_t *out_idx, uint32_t intra_lo, uint32_t intra_hi,
                               uint64_t *p_cross, uint64_t *p_intra)
{
    clear_error();
    uint64_t pc = 0, pi = 0;
    for (uint32_t c = 1; c <= G; ++c) {
        const uint64_t nc = group_begin[c + 1] - group_begin[c];
        uint64_t u = 0;
        if (out_ptr)
            for (uint32_t e = out_ptr[c]; e < out_ptr[c + 1]; ++e)
                u += group_begin[out_idx[e] + 1] - group_begin[out_idx[e]];
        pc += nc * u;
        if (nc >= intra_lo && nc <= intra_hi && nc > 0)
            pi += nc * (nc - 1);
    }
    if (p_cross)
        *p_cross = pc;
    if (p_intra)
        *p_intra = pi;
    return UNG_HIP_OK;
}

// ---------------------------------------------------------------------------
// Output boundary: the final adjacency as CSR and the Graph::save text format
// ---------------------------------------------------------------------------
extern "C" int ung_assemble_graph_csr(uint64_t N, uint32_t G, const uint32_t *group_begin, const uint64_t *intra_ptr,
                                      const uint32_t *intra_idx, int intra_global, const uint32_t *cross_ids,
                                      uint32_t cross_stride, uint32_t num_cross, const uint32_t *add_ptr,
                                      const uint32_t *add_from, const uint32_t *add_to, uint64_t *row_ptr,
                                      uint32_t *col_idx, uint64_t capacity, uint64_t *n_entries, int nthreads)
{
    clear_error();
    if (!group_begin || !row_ptr || !n_entries || (intra_ptr && !intra_idx && intra_ptr[N] > 0) ||
        (cross_ids && num_cross > cross_stride) || (add_ptr && (!add_from || !add_to) && add_ptr[G + 1] > 0)) {
        set_error("ung_assemble_graph_csr: null or inconsistent argument");
        return UNG_HIP_EINVAL;
    }
    if ((uint64_t)group_begin[G + 1] != N) {
        set_error("ung_assemble_graph_csr: group_begin[G+1]=%u != N=%llu", group_begin[G + 1], (unsigned long long)N);
        return UNG_HIP_EINVAL;
    }
    const uint32_t use = cross_ids ? num_cross : 0u;
    // point -> first id of its group (add_offset_for_uni_nav_graph) and per-point counts
    std::vector<uint32_t> base(N);
    std::vector<uint64_t> cnt(N + 1, 0);
    for (uint32_t g = 1; g <= G; ++g) {
        if (group_begin[g + 1] < group_begin[g]) {
            set_error("ung_assemble_graph_csr: group_begin not monotone at group %u", g);
            return UNG_HIP_EINVAL;
        }
        for (uint64_t i = group_begin[g]; i < group_begin[g + 1]; ++i)
            base[i] = group_begin[g];
    }
    parallel_for((int64_t)N, nthreads, 65536, [&](int64_t b, int64_t e) {
        for (int64_t i = b; i < e; ++i) {
            uint64_t c = intra_ptr ? intra_ptr[i + 1] - intra_ptr[i] : 0;
            for (uint32_t t = 0; t < use; ++t)
                c += cross_ids[(uint64_t)i * cross_stride + t] != 0xFFFFFFFFu;
            cnt[i + 1] = c;
        }
    });
    if (add_ptr)
        for (uint32_t g = 1; g <= G; ++g)
            for (uint64_t e = add_ptr[g]; e < add_ptr[g + 1]; ++e) {
                // a group's list holds edges from its own points only (one writer per row)
                if (add_from[e] < group_begin[g] || add_from[e] >= group_begin[g + 1]) {
                    set_error("ung_assemble_graph_csr: additional edge %llu of group %u starts at %u, outside the group",
                              (unsigned long long)e, g, add_from[e]);
                    return UNG_HIP_EINVAL;
                }
                ++cnt[add_from[e] + 1];
            }
    for (uint64_t i = 0; i < N; ++i)
        cnt[i + 1] += cnt[i];
    *n_entries = cnt[N];
    if (cnt[N] > capacity || (cnt[N] > 0 && !col_idx)) {
        set_error("ung_assemble_graph_csr: %llu entries need capacity (got %llu)", (unsigned long long)cnt[N],
                  (unsigned long long)capacity);
        return UNG_HIP_EINVAL;
    }
    std::memcpy(row_ptr, cnt.data(), (N + 1) * sizeof(uint64_t));
    // intra (+ group offset) then cross edges; cursors left at the end of each row's cross part
    std::vector<uint64_t> cur(N);
    parallel_for((int64_t)N, nthreads, 65536, [&](int64_t b, int64_t e) {
        for (int64_t i = b; i < e; ++i) {
            uint64_t w = row_ptr[i];
            if (intra_ptr)
                for (uint64_t p = intra_ptr[i]; p < intra_ptr[i + 1]; ++p)
                    col_idx[w++] = intra_idx[p] + (intra_global ? 0u : base[i]);
            for (uint32_t t = 0; t < use; ++t) {
                const uint32_t nb = cross_ids[(uint64_t)i * cross_stride + t];
                if (nb != 0xFFFFFFFFu)
                    col_idx[w++] = nb;
            }
            cur[i] = w;
        }
    });
    // additional edges, group list by group list (a group's lists only hold its own points)
    if (add_ptr)
        parallel_for((int64_t)G, nthreads, 256, [&](int64_t b, int64_t e) {
            for (int64_t g = b + 1; g <= e; ++g)
                for (uint64_t p = add_ptr[g]; p < add_ptr[g + 1]; ++p)
                    col_idx[cur[add_from[p]]++] = add_to[p];
        });
    return UNG_HIP_OK;
}

extern "C" int ung_graph_save_text(const char *path, uint64_t N, const uint64_t *row_ptr, const uint32_t *col_idx,
                                   int nthreads)
{
    clear_error();
    if (!path || !row_ptr || (row_ptr[N] > 0 && !col_idx)) {
        set_error("ung_graph_save_text: null argument");
        return UNG_HIP_EINVAL;
    }
    FILE *f = std::fopen(path, "wb");
    if (!f) {
        set_error("ung_graph_save_text: cannot open %s", path);
        return UNG_HIP_EINVAL;
    }
    // format blocks of points in parallel, write them in order: "i n1 n2 ... \n"
    const int64_t block = 1 << 16;
    const int64_t nblocks = ((int64_t)N + block - 1) / block;
    const int wave = std::max(1, resolve_threads(nthreads)) * 2;
    std::vector<std::string> text;
    auto put = [](std::string &s, uint64_t v) {
        char tmp[24];
        int n = 0;
        do {
            tmp[n++] = (char)('0' + v % 10);
            v /= 10;
        } while (v);
        while (n)
            s.push_back(tmp[--n]);
        s.push_back(' ');
    };
    bool ok = true;
    for (int64_t b0 = 0; b0 < nblocks && ok; b0 += wave) {
        const int64_t nb = std::min<int64_t>(wave, nblocks - b0);
        text.assign((size_t)nb, std::string());
        parallel_for(nb, nthreads, 1, [&](int64_t b, int64_t e) {
            for (int64_t j = b; j < e; ++j) {
                std::string &s = text[(size_t)j];
                const uint64_t lo = (uint64_t)(b0 + j) * block, hi = std::min<uint64_t>(N, lo + block);
                s.reserve((size_t)(hi - lo) * 16 + (size_t)(row_ptr[hi] - row_ptr[lo]) * 8);
                for (uint64_t i = lo; i < hi; ++i) {
                    put(s, i);
                    for (uint64_t p = row_ptr[i]; p < row_ptr[i + 1]; ++p)
                        put(s, col_idx[p]);
                    s.push_back('\n');
                }
            }
        });
        for (const std::string &s : text)
            if (std::fwrite(s.data(), 1, s.size(), f) != s.size()) {
                ok = false;
                break;
            }
    }
    if (std::fclose(f) != 0 || !ok) {
        set_error("ung_graph_save_text: write to %s failed", path);
        return UNG_HIP_EINVAL;
    }
    return UNG_HIP_OK;
}

extern "C" const char *ung_hip_last_error(void) { return ung::g_last_error.c_str(); }
