"""Host-side mirror of the reference's UNG build stage around the HIP path.

``UngBuildStage`` keeps the names, argument meaning and error behaviour of the
reference's ``UniNavGraph`` steps that feed and consume the cross-edge and
mid-group kNN stage (paths under UNG/codes/ of panjd123/FilterVectorCode_refactor):

  build_trie_and_divide_groups      src/uni_nav_graph_label_graph.cpp:21-43
  prepare_group_storages_graphs     src/uni_nav_graph.cpp:148-181 (reorder)
  build_label_nav_graph             src/uni_nav_graph_label_graph.cpp:851-911
  gpu_prepare_all_vectors_on_device include/uni_nav_graph.h:430-432
  gpu_cross_groups_search_all_batched include/uni_nav_graph.h:436-444
  gpu_release_all_vectors_on_device include/uni_nav_graph.h:433
  build_fast_exact_batch            src/tagore_graph_builder.cu:1058-1429 (exact-anchor
                                    batch; exact lists as build_exact_topk_graph_for_points,
                                    src/uni_nav_graph_special_blocks.cpp:70-111)
  build_cross_edges_generate_additional src/uni_nav_graph_cross_edges.cpp:442-596 (exact)
  merge_cross_edges_to_graph        src/ung_cross_edge_output_writer.cpp:68-95
  add_offset_for_uni_nav_graph      src/uni_nav_graph.cpp:285-297
  build_csr_adjacency / Graph::save src/ung_cross_edge_output_writer.cpp:44-66,
                                    include/graph.h:207-216

Every device computation goes through libung_hip.so; failures raise
``RuntimeError`` (``UngHipError``), as the reference's GPU route throws
``std::runtime_error``.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from ._lib import Stats, UngHipError, check, f32, ptr, u32

NONE_ID = 0xFFFFFFFF


@dataclass
class TagoreBatchBuildResult:
    """Mirror of TagoreBatchBuildResult (include/tagore_graph_builder.h:80-88)."""
    packed_graph: np.ndarray            # [sum n, packed_graph_stride] uint32
    packed_offsets: np.ndarray          # [n_groups + 1] uint32
    packed_graph_stride: int
    entry_points: np.ndarray            # [n_groups] uint32 (0, as the reference kernel)
    exact_ids: np.ndarray               # [sum n, list_k] local ids, (dist,id) order
    exact_dists: np.ndarray             # [sum n, list_k] float32
    stats: dict = field(default_factory=dict)


class HipContext:
    """RAII wrapper of an ung_hip_ctx (one device, one stream)."""

    def __init__(self, device: int = 0):
        self.lib = _lib.load()
        h = C.c_void_p()
        check(self.lib.ung_hip_create(device, C.byref(h)))
        self.h = h
        self.device = device

    def close(self):
        if getattr(self, "h", None) is not None and self.h.value:
            self.lib.ung_hip_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- thin wrappers ------------------------------------------------------
    def prepare_vectors(self, X: np.ndarray) -> dict:
        X = f32(X)
        st = Stats()
        check(self.lib.ung_hip_prepare_vectors(self.h, ptr(X), X.shape[0], X.shape[1], C.byref(st)))
        return st.as_dict()

    def release_vectors(self):
        check(self.lib.ung_hip_release_vectors(self.h))

    def cross_topk(self, group_begin, out_ptr, out_idx, k: int, with_dist=True, with_size=True):
        """Cross edges with host output (ung_hip_cross_topk): ids [N x k] (the FlatId rows),
        distances and row sizes when asked for (None otherwise), stats."""
        group_begin, out_ptr = u32(group_begin), u32(out_ptr)
        out_idx = u32(out_idx) if len(out_idx) else np.zeros(1, np.uint32)
        G = group_begin.shape[0] - 2
        N = int(group_begin[-1])
        ids = np.empty((N, k), np.uint32)
        dist = np.empty((N, k), np.float32) if with_dist else None
        size = np.empty(N, np.int32) if with_size else None
        st = Stats()
        check(self.lib.ung_hip_cross_topk(self.h, G, ptr(group_begin), ptr(out_ptr), ptr(out_idx), k,
                                          ptr(ids), ptr(dist), ptr(size), C.byref(st)))
        return ids, dist, size, st.as_dict()

    def cross_topk_device(self, group_begin, out_ptr, out_idx, k: int) -> dict:
        group_begin, out_ptr = u32(group_begin), u32(out_ptr)
        out_idx = u32(out_idx) if len(out_idx) else np.zeros(1, np.uint32)
        G = group_begin.shape[0] - 2
        st = Stats()
        check(self.lib.ung_hip_cross_topk_device(self.h, G, ptr(group_begin), ptr(out_ptr), ptr(out_idx), k,
                                                 C.byref(st)))
        return st.as_dict()

    def cross_topk_noalloc(self, group_begin, out_ptr, out_idx, k: int, ids_dev: int, dist_dev: int,
                           size_dev: int) -> dict:
        """Cross edges into caller-owned device buffers (addresses of [N x k] uint32, [N x k]
        float32, [N] int32), with no allocation in the call (ung_hip_cross_topk_noalloc)."""
        group_begin, out_ptr = u32(group_begin), u32(out_ptr)
        out_idx = u32(out_idx) if len(out_idx) else np.zeros(1, np.uint32)
        G = group_begin.shape[0] - 2
        st = Stats()
        check(self.lib.ung_hip_cross_topk_noalloc(self.h, G, ptr(group_begin), ptr(out_ptr), ptr(out_idx), k,
                                                  ids_dev, dist_dev, size_dev, C.byref(st)))
        return st.as_dict()

    def cross_intra_begin(self, group_begin, out_ptr, out_idx, k: int, grp_begin, grp_size, list_k: int) -> dict:
        """Cross edges (device-resident, complete on return) and a group kNN call left running
        on the second stream until intra_end (ung_hip_cross_intra_begin)."""
        group_begin, out_ptr = u32(group_begin), u32(out_ptr)
        out_idx = u32(out_idx) if len(out_idx) else np.zeros(1, np.uint32)
        grp_begin, grp_size = u32(grp_begin), u32(grp_size)
        G = group_begin.shape[0] - 2
        st = Stats()
        check(self.lib.ung_hip_cross_intra_begin(self.h, G, ptr(group_begin), ptr(out_ptr), ptr(out_idx), k,
                                                 grp_begin.shape[0], ptr(grp_begin) if len(grp_begin) else None,
                                                 ptr(grp_size) if len(grp_size) else None, list_k, C.byref(st)))
        self._keep = (grp_begin, grp_size)
        return st.as_dict()

    def intra_end(self) -> dict:
        st = Stats()
        check(self.lib.ung_hip_intra_end(self.h, C.byref(st)))
        self._keep = None
        return st.as_dict()

    def result_shape(self, which: int):
        """(rows, k, n_groups) of the resident cross rows (which=0) or group lists (which=1)
        (ung_hip_result_shape); raises when there is none."""
        rows, k, ng = C.c_uint64(), C.c_uint32(), C.c_uint32()
        check(self.lib.ung_hip_result_shape(self.h, which, C.byref(rows), C.byref(k), C.byref(ng)))
        return int(rows.value), int(k.value), int(ng.value)

    def rescanned_rows(self, which: int) -> np.ndarray:
        """Output rows of the last cross (which=0) or group (which=1) call that took the exact
        rescan, ascending (ung_hip_rescanned_rows)."""
        n = C.c_uint64(0)
        rc = self.lib.ung_hip_rescanned_rows(self.h, which, None, 0, C.byref(n))
        if rc == _lib.UNG_HIP_OK:
            return np.zeros(0, np.uint32)
        if rc != _lib.UNG_HIP_EINVAL or n.value == 0:
            check(rc)
        rows = np.empty(int(n.value), np.uint32)
        check(self.lib.ung_hip_rescanned_rows(self.h, which, ptr(rows), rows.shape[0], C.byref(n)))
        return rows

    def _checked_shape(self, which, rows=None, k=None, n_groups=None):
        """The resident shape; a caller-given size that differs from it raises ValueError
        (the library writes the resident shape, not the caller's)."""
        r, kk, ng = self.result_shape(which)
        for name, want, got in (("rows", rows, r), ("k", k, kk), ("n_groups", n_groups, ng)):
            if want is not None and int(want) != got:
                raise ValueError(f"{name}={want} does not match the resident result ({name}={got})")
        return r, kk, ng

    def download_cross(self, N: int | None = None, k: int | None = None):
        N, k, _ = self._checked_shape(0, N, k)
        ids = np.empty((N, k), np.uint32)
        dist = np.empty((N, k), np.float32)
        size = np.empty(N, np.int32)
        st = Stats()
        check(self.lib.ung_hip_download_cross(self.h, ptr(ids), ptr(dist), ptr(size), C.byref(st)))
        return ids, dist, size, st.as_dict()

    def download_group(self, rows: int | None = None, list_k: int | None = None):
        """The resident lists of the last group kNN call (ung_hip_download_group)."""
        rows, list_k, _ = self._checked_shape(1, rows, list_k)
        ids = np.empty((rows, list_k), np.uint32)
        dist = np.empty((rows, list_k), np.float32)
        st = Stats()
        check(self.lib.ung_hip_download_group(self.h, ptr(ids), ptr(dist), C.byref(st)))
        return ids, dist, st.as_dict()

    def additional_edges(self, group_begin, out_ptr, out_idx, num_cross: int):
        """Additional edges (exact variant) from the resident cross-edge rows of the last
        cross_topk(_device) call: (edge_ptr[G+2], edge_from, edge_to, stats); the edges of
        group C are [edge_ptr[C], edge_ptr[C+1]).  stats["fallback_ms"] is the exact-scan
        kernel time, stats["rows"] the query rows scanned."""
        group_begin, out_ptr = u32(group_begin), u32(out_ptr)
        out_idx = u32(out_idx) if len(out_idx) else np.zeros(1, np.uint32)
        G = group_begin.shape[0] - 2
        edge_ptr = np.zeros(G + 2, np.uint32)
        n = C.c_uint64(0)
        # the capacity the last call needed (a retry repeats the host planning)
        cap = max(1024, int(group_begin[-1]) // 2, getattr(self, "_addl_cap", 0))
        while True:
            ef = np.empty(cap, np.uint32)
            et = np.empty(cap, np.uint32)
            st = Stats()
            rc = self.lib.ung_hip_additional_edges(self.h, G, ptr(group_begin), ptr(out_ptr), ptr(out_idx), num_cross,
                                                   ptr(edge_ptr), ptr(ef), ptr(et), cap, C.byref(n), C.byref(st))
            if rc == _lib.UNG_HIP_EINVAL and n.value > cap:
                cap = int(n.value)
                self._addl_cap = cap
                continue
            check(rc)
            return edge_ptr, ef[: n.value].copy(), et[: n.value].copy(), st.as_dict()

    def group_knn(self, grp_begin, grp_size, list_k: int):
        grp_begin, grp_size = u32(grp_begin), u32(grp_size)
        rows = int(grp_size.astype(np.uint64).sum())
        ids = np.empty((rows, list_k), np.uint32)
        dist = np.empty((rows, list_k), np.float32)
        st = Stats()
        check(self.lib.ung_hip_group_knn(self.h, grp_begin.shape[0], ptr(grp_begin) if rows else None,
                                         ptr(grp_size) if rows else None, list_k, ptr(ids), ptr(dist),
                                         C.byref(st)))
        return ids, dist, st.as_dict()

    def group_knn_device(self, grp_begin, grp_size, list_k: int) -> dict:
        grp_begin, grp_size = u32(grp_begin), u32(grp_size)
        st = Stats()
        check(self.lib.ung_hip_group_knn_device(self.h, grp_begin.shape[0], ptr(grp_begin), ptr(grp_size),
                                                list_k, C.byref(st)))
        return st.as_dict()

    def pack_anchor_rows(self, rows: int | None, n_groups: int | None, tagore_k: int, final_degree: int,
                         head_keep: int, anchor_tail: int = 1, anchor_slots: int = 0,
                         bidir_anchor: int = 0):
        rows, _, n_groups = self._checked_shape(1, rows, None, n_groups)
        stride = final_degree + 1
        graph = np.empty((rows, stride), np.uint32)
        entries = np.empty(max(n_groups, 1), np.uint32)
        st = Stats()
        check(self.lib.ung_hip_pack_anchor_rows(self.h, tagore_k, final_degree, head_keep, anchor_tail,
                                                anchor_slots, bidir_anchor, ptr(graph), ptr(entries),
                                                C.byref(st)))
        return graph, entries[:n_groups], st.as_dict()

    def prune_group_graph(self, rows: int | None, n_groups: int | None, forward_cap: int, reverse_cap: int,
                          final_degree: int, alpha: float):
        """FastGrnnd-style prune of the last group_knn(_device) lists (ung_hip_prune_group_graph):
        rows [rows x (final_degree+1)] = [count, local ids, padding], entry points, stats."""
        rows, _, n_groups = self._checked_shape(1, rows, None, n_groups)
        stride = final_degree + 1
        graph = np.empty((rows, stride), np.uint32)
        entries = np.empty(max(n_groups, 1), np.uint32)
        st = Stats()
        check(self.lib.ung_hip_prune_group_graph(self.h, forward_cap, reverse_cap, final_degree, alpha, ptr(graph),
                                                 ptr(entries), C.byref(st)))
        return graph, entries[:n_groups], st.as_dict()

    def synchronize(self):
        check(self.lib.ung_hip_synchronize(self.h))

    def selftest_mfma(self) -> float:
        err = C.c_double()
        check(self.lib.ung_hip_selftest_mfma(self.h, C.byref(err)))
        return err.value

    def debug_partial_rows(self):
        """(query ids, candidate ids, approximate squared distances, eps_coef, rmax) of the
        last cross-edge call's partial rows (ung_hip_debug_partial_rows; diagnostic)."""
        n = C.c_uint64(0)
        ec, rm = C.c_double(), C.c_double()
        rc = self.lib.ung_hip_debug_partial_rows(self.h, 0, None, None, None, C.byref(n), C.byref(ec), C.byref(rm))
        if rc != 0 and n.value == 0:
            check(rc)
        q = np.empty(n.value, np.uint32)
        c = np.empty(n.value, np.uint32)
        a = np.empty(n.value, np.float32)
        check(self.lib.ung_hip_debug_partial_rows(self.h, n.value, ptr(q), ptr(c), ptr(a), C.byref(n),
                                                  C.byref(ec), C.byref(rm)))
        return q, c, a, ec.value, rm.value

    def debug_partial_bounds(self):
        """(query ids, split candidate ranges [begin, end) as global ids, bounds) of the same
        call's partial rows (ung_hip_debug_partial_bounds; diagnostic)."""
        n = C.c_uint64(0)
        rc = self.lib.ung_hip_debug_partial_bounds(self.h, 0, None, None, None, None, C.byref(n))
        if rc != 0 and n.value == 0:
            check(rc)
        q = np.empty(n.value, np.uint32)
        b0 = np.empty(n.value, np.uint32)
        b1 = np.empty(n.value, np.uint32)
        bd = np.empty(n.value, np.float32)
        check(self.lib.ung_hip_debug_partial_bounds(self.h, n.value, ptr(q), ptr(b0), ptr(b1), ptr(bd), C.byref(n)))
        return q, b0, b1, bd


# ---------------------------------------------------------------------------
# host-side inputs (C++ in libung_hip.so)
# ---------------------------------------------------------------------------
def divide_groups(lab_ptr, lab_idx):
    """Groups by exact label set in first-appearance order; returns
    (G, point_group[N] for original ids, group_begin[G+2], new_to_old[N])."""
    lib = _lib.load()
    lab_ptr = u32(lab_ptr)
    lab_idx = u32(lab_idx) if len(lab_idx) else np.zeros(1, np.uint32)
    N = lab_ptr.shape[0] - 1
    pg = np.empty(max(N, 1), np.uint32)
    gb = np.empty(N + 2, np.uint32)
    n2o = np.empty(max(N, 1), np.uint32)
    G = C.c_uint32()
    check(lib.ung_divide_groups(N, ptr(lab_ptr), ptr(lab_idx), ptr(pg), ptr(gb), ptr(n2o), C.byref(G)))
    G = G.value
    return G, pg[:N], gb[: G + 2].copy(), n2o[:N]


def group_label_sets(lab_ptr, lab_idx, group_begin, new_to_old, G):
    lib = _lib.load()
    lab_ptr, group_begin, new_to_old = u32(lab_ptr), u32(group_begin), u32(new_to_old)
    lab_idx = u32(lab_idx) if len(lab_idx) else np.zeros(1, np.uint32)
    N = lab_ptr.shape[0] - 1
    set_ptr = np.empty(G + 2, np.uint32)
    cap = max(int(lab_ptr[-1]), 1)
    set_idx = np.empty(cap, np.uint32)
    check(lib.ung_group_label_sets(N, ptr(lab_ptr), ptr(lab_idx), ptr(group_begin), ptr(new_to_old), G,
                                   ptr(set_ptr), ptr(set_idx), cap))
    return set_ptr, set_idx[: set_ptr[-1]].copy()


def lng_build(set_ptr, set_idx, nthreads: int = 0):
    """Minimum-superset out-neighbour CSR (out_ptr[G+2], out_idx)."""
    lib = _lib.load()
    set_ptr = u32(set_ptr)
    set_idx = u32(set_idx) if len(set_idx) else np.zeros(1, np.uint32)
    G = set_ptr.shape[0] - 2
    out_ptr = np.empty(G + 2, np.uint32)
    n_edges = C.c_uint64()
    rc = lib.ung_lng_build(G, ptr(set_ptr), ptr(set_idx), ptr(out_ptr), None, 0, C.byref(n_edges), nthreads)
    if rc not in (_lib.UNG_HIP_OK, _lib.UNG_HIP_EINVAL):
        check(rc)
    cap = max(int(n_edges.value), 1)
    out_idx = np.empty(cap, np.uint32)
    check(lib.ung_lng_build(G, ptr(set_ptr), ptr(set_idx), ptr(out_ptr), ptr(out_idx), cap, C.byref(n_edges),
                            nthreads))
    return out_ptr, out_idx[: n_edges.value].copy()


def in_neighbors(out_ptr, out_idx):
    """Transpose of the LNG: in(X) = {C : X in out(C)} ascending (phase 2 of
    build_label_nav_graph, src/uni_nav_graph_label_graph.cpp:893-908)."""
    out_ptr = np.asarray(out_ptr, np.int64)
    G = out_ptr.shape[0] - 2
    src = np.repeat(np.arange(G + 2, dtype=np.int64), np.diff(np.concatenate([out_ptr, out_ptr[-1:]])))
    src = src[: len(out_idx)]
    order = np.lexsort((src, np.asarray(out_idx, np.int64)))
    dst_sorted = np.asarray(out_idx, np.int64)[order]
    in_idx = src[order].astype(np.uint32)
    counts = np.bincount(dst_sorted, minlength=G + 2)[: G + 2]
    in_ptr = np.zeros(G + 2, np.uint32)
    in_ptr[2:] = np.cumsum(counts[1: G + 1])
    return in_ptr, in_idx


def reorder_rows(X, new_to_old, nthreads: int = 0):
    lib = _lib.load()
    X = f32(X)
    new_to_old = u32(new_to_old)
    out = np.empty_like(X)
    check(lib.ung_reorder_rows(ptr(X), X.shape[0], X.shape[1], ptr(new_to_old), ptr(out), nthreads))
    return out


def count_pairs(group_begin, out_ptr, out_idx, intra_lo=128, intra_hi=4096):
    lib = _lib.load()
    group_begin, out_ptr = u32(group_begin), u32(out_ptr)
    out_idx = u32(out_idx) if len(out_idx) else np.zeros(1, np.uint32)
    G = group_begin.shape[0] - 2
    pc, pi = C.c_uint64(), C.c_uint64()
    check(lib.ung_count_pairs(G, ptr(group_begin), ptr(out_ptr), ptr(out_idx), intra_lo, intra_hi,
                              C.byref(pc), C.byref(pi)))
    return pc.value, pi.value


def assemble_graph_csr(N, group_begin, intra_ptr=None, intra_idx=None, intra_global=False, cross_ids=None,
                       num_cross=None, add_ptr=None, add_from=None, add_to=None, nthreads: int = 0):
    """Final adjacency as CSR (row_ptr[N+1] uint64, col_idx uint32): per point its intra
    edges (group-local ids + the group's first id unless intra_global), the first
    num_cross entries of its FlatId cross row, then its additional edges -- the
    NeighborList the reference builds with add_offset_for_uni_nav_graph and the
    cross/additional merges (src/uni_nav_graph.cpp:285-297,
    src/uni_nav_graph_cross_edges.cpp:849-868)."""
    lib = _lib.load()
    group_begin = u32(group_begin)
    G = group_begin.shape[0] - 2
    ip = None if intra_ptr is None else np.ascontiguousarray(intra_ptr, np.uint64)
    ii = None if intra_idx is None else (u32(intra_idx) if len(intra_idx) else np.zeros(1, np.uint32))
    cr = None if cross_ids is None else u32(cross_ids)
    stride = 0 if cr is None else (cr.shape[1] if cr.ndim == 2 else 1)
    nc = stride if num_cross is None else int(num_cross)
    ap = None if add_ptr is None else u32(add_ptr)
    af = None if add_from is None else (u32(add_from) if len(add_from) else np.zeros(1, np.uint32))
    at = None if add_to is None else (u32(add_to) if len(add_to) else np.zeros(1, np.uint32))
    row_ptr = np.zeros(N + 1, np.uint64)
    n = C.c_uint64(0)
    rc = lib.ung_assemble_graph_csr(N, G, ptr(group_begin), ptr(ip), ptr(ii), int(intra_global), ptr(cr), stride, nc,
                                    ptr(ap), ptr(af), ptr(at), ptr(row_ptr), None, 0, C.byref(n), nthreads)
    if rc != _lib.UNG_HIP_EINVAL or n.value == 0:
        check(rc)
    col = np.empty(max(int(n.value), 1), np.uint32)
    check(lib.ung_assemble_graph_csr(N, G, ptr(group_begin), ptr(ip), ptr(ii), int(intra_global), ptr(cr), stride,
                                     nc, ptr(ap), ptr(af), ptr(at), ptr(row_ptr), ptr(col), col.shape[0],
                                     C.byref(n), nthreads))
    return row_ptr, col[: n.value]


def graph_save_text(path, row_ptr, col_idx, nthreads: int = 0):
    """Graph::save text format (include/graph.h:207-216): "i n1 n2 ... \\n" per point."""
    lib = _lib.load()
    row_ptr = np.ascontiguousarray(row_ptr, np.uint64)
    col = u32(col_idx) if len(col_idx) else np.zeros(1, np.uint32)
    check(lib.ung_graph_save_text(str(path).encode(), row_ptr.shape[0] - 1, ptr(row_ptr), ptr(col), nthreads))


# ---------------------------------------------------------------------------
# the stage object
# ---------------------------------------------------------------------------
class UngBuildStage:
    """The cross-edge + mid-group kNN stage of UniNavGraph::build, MI355X path.

    Parameters mirror the reference CLI/config: ``num_cross_edges`` (k, default 6,
    include/config.h:51), ``max_degree`` (include/config.h:41; 32 in the target
    configs), ``tagore_k`` (UNG_TAGORE_K, default 64, src/ung_build_config.cpp:341),
    ``tagore_min_group_size`` / ``exact_max_nx`` (mid-group range 128..4096,
    src/ung_build_config.cpp:339, src/ung_build_settings.cpp:246-252), ``alpha`` (the
    prune factor, include/config.h), ``scenario`` (the build's --scenario,
    apps/build_UNG_index.cpp:52, default "general"; "equality" builds no label navigating
    graph and no cross edges, src/uni_nav_graph.cpp:95-99)."""

    def __init__(self, num_cross_edges: int = 6, max_degree: int = 32, tagore_k: int = 64,
                 tagore_min_group_size: int = 128, exact_max_nx: int = 4096, device: int = 0,
                 num_threads: int = 0, alpha: float = 1.2, scenario: str = "general"):
        self.scenario = str(scenario)
        self.num_cross_edges = int(num_cross_edges)
        self.max_degree = int(max_degree)
        self.alpha = float(alpha)
        self.tagore_k = int(tagore_k)
        self.tagore_min_group_size = int(tagore_min_group_size)
        self.exact_max_nx = int(exact_max_nx)
        self.num_threads = int(num_threads)
        self.device = device
        self._ctx: HipContext | None = None
        self.base = None
        self.lab_ptr = None
        self.lab_idx = None

    # ---- inputs -------------------------------------------------------------
    def load_arrays(self, X: np.ndarray, lab_ptr, lab_idx):
        """Storage::load_from_file equivalent for in-memory arrays (src/storage.cpp:102-169)."""
        self.base = f32(X)
        self.lab_ptr = u32(lab_ptr)
        self.lab_idx = u32(lab_idx)
        if self.lab_ptr.shape[0] != self.base.shape[0] + 1:
            raise ValueError("label CSR does not match the number of vectors")

    def build_trie_and_divide_groups(self):
        G, pg, gb, n2o = divide_groups(self.lab_ptr, self.lab_idx)
        self.num_groups = G
        self._point_group_old = pg
        self.group_begin = gb
        self.new_to_old = n2o

    def prepare_group_storages_graphs(self):
        self.base = reorder_rows(self.base, self.new_to_old, self.num_threads)
        sizes = np.diff(self.group_begin.astype(np.int64))[1:]
        self.new_vec_id_to_group_id = np.repeat(np.arange(1, self.num_groups + 1, dtype=np.uint32), sizes)

    def build_label_nav_graph(self):
        set_ptr, set_idx = group_label_sets(self.lab_ptr, self.lab_idx, self.group_begin, self.new_to_old,
                                            self.num_groups)
        self.group_set_ptr, self.group_set_idx = set_ptr, set_idx
        self.out_ptr, self.out_idx = lng_build(set_ptr, set_idx, self.num_threads)
        self.in_ptr, self.in_idx = in_neighbors(self.out_ptr, self.out_idx)

    def skip_label_nav_graph(self):
        """The "equality" scenario (src/uni_nav_graph.cpp:95-99): no label navigating graph,
        so every group's LNG row is empty -- the cross-edge call then returns padding rows
        only, the additional edges are empty, and the assembled graph holds the intra edges
        with add_offset_for_uni_nav_graph, as the reference's build does."""
        G = self.num_groups
        self.out_ptr = np.zeros(G + 2, np.uint32)
        self.out_idx = np.zeros(0, np.uint32)
        self.in_ptr = np.zeros(G + 2, np.uint32)
        self.in_idx = np.zeros(0, np.uint32)

    def prepare_inputs(self, X, lab_ptr, lab_idx):
        """Steps 2, 3 and 7 of UniNavGraph::build (src/uni_nav_graph.cpp:54-146)."""
        self.load_arrays(X, lab_ptr, lab_idx)
        self.build_trie_and_divide_groups()
        self.prepare_group_storages_graphs()
        if self.scenario == "equality":
            self.skip_label_nav_graph()
        else:
            self.build_label_nav_graph()

    # ---- device -------------------------------------------------------------
    @property
    def ctx(self) -> HipContext:
        if self._ctx is None:
            self._ctx = HipContext(self.device)
        return self._ctx

    def gpu_prepare_all_vectors_on_device(self) -> dict:
        return self.ctx.prepare_vectors(self.base)

    def gpu_release_all_vectors_on_device(self):
        if self._ctx is not None:
            self._ctx.release_vectors()

    def close(self):
        if self._ctx is not None:
            self._ctx.close()
            self._ctx = None

    def _restricted_out(self, target_group_ids):
        if target_group_ids is None:
            return self.out_ptr, self.out_idx
        keep = np.zeros(self.num_groups + 2, bool)
        keep[np.asarray(target_group_ids, np.int64)] = True
        sel = keep[self.out_idx.astype(np.int64)]
        src = np.repeat(np.arange(self.num_groups + 2), np.diff(np.concatenate([self.out_ptr, self.out_ptr[-1:]])))
        src = src[: len(self.out_idx)][sel]
        out_idx = self.out_idx[sel]
        cnt = np.bincount(src, minlength=self.num_groups + 2)[: self.num_groups + 2]
        out_ptr = np.zeros(self.num_groups + 2, np.uint32)
        out_ptr[2:] = np.cumsum(cnt[1: self.num_groups + 1])
        return out_ptr, out_idx

    def gpu_cross_groups_search_all_batched(self, target_group_ids=None, topk: int | None = None):
        """Cross edges of every point: FlatId layout [N x k] (UINT32_MAX padding),
        plus fp32 distances and row sizes.  ``target_group_ids`` restricts the
        targets X (the reference passes the groups with in-neighbours; None = all)."""
        k = self.num_cross_edges if topk is None else int(topk)
        out_ptr, out_idx = self._restricted_out(target_group_ids)
        ids, dist, size, st = self.ctx.cross_topk(self.group_begin, out_ptr, out_idx, k)
        self.cross_flat_ids, self.cross_dists, self.cross_sizes = ids, dist, size
        self.cross_stats = st
        return ids, dist, size

    def build_cross_edges_generate_additional(self):
        """Additional edges, exact variant (build_cross_edges_generate_additional,
        src/uni_nav_graph_cross_edges.cpp:442-596): per group C, the out-groups that no
        cross edge of C's members reaches get num_cross/2 exact nearest targets from each of
        C's first vectors until num_cross edges were added.  Needs the cross edges of
        gpu_cross_groups_search_all_batched on the device.  Returns the per-group CSR
        (edge_ptr[G+2], edge_from, edge_to) -- the reference's materialized lists."""
        ptr_, ef, et, st = self.ctx.additional_edges(self.group_begin, self.out_ptr, self.out_idx,
                                                     self.num_cross_edges)
        self.additional_edges = (ptr_, ef, et)
        self.additional_stats = st
        return ptr_, ef, et

    def build_csr_adjacency(self, intra_ptr=None, intra_idx=None, intra_global=False):
        """The final graph as CSR (row_ptr[N+1], col_idx): intra edges (the group graphs'
        local lists as CSR over points, offset by add_offset_for_uni_nav_graph unless
        intra_global), the cross edges of gpu_cross_groups_search_all_batched, then the
        additional edges of build_cross_edges_generate_additional when they were built."""
        N = int(self.group_begin[-1])
        add = getattr(self, "additional_edges", None)
        cross = getattr(self, "cross_flat_ids", None)
        self.graph_csr = assemble_graph_csr(N, self.group_begin, intra_ptr, intra_idx, intra_global, cross,
                                            self.num_cross_edges if cross is not None else None,
                                            *(add if add is not None else (None, None, None)))
        return self.graph_csr

    def save_graph(self, path):
        """Graph::save of the assembled graph (include/graph.h:207-216)."""
        graph_save_text(path, *self.graph_csr)

    def mid_groups(self):
        """Groups routed to the exact batch (partition_tagore_groups +
        build_tagore_batch_artifacts: complete_threshold < n, tagore_min_group_size <= n
        <= exact_max_nx; src/uni_nav_graph_group_graph.cpp:617-677)."""
        sizes = np.diff(self.group_begin.astype(np.int64))[1:]
        complete_threshold = max(self.max_degree, 64)
        gids = np.nonzero((sizes > complete_threshold) & (sizes >= self.tagore_min_group_size) &
                          (sizes <= self.exact_max_nx))[0] + 1
        return gids.astype(np.uint32)

    def large_groups(self):
        """Groups above the exact batch that the reference gives to the FastGrnnd batch
        (partition_tagore_groups + build_tagore_batch_artifacts: n > exact_max_nx;
        src/uni_nav_graph_group_graph.cpp:617-738)."""
        sizes = np.diff(self.group_begin.astype(np.int64))[1:]
        complete_threshold = max(self.max_degree, 64)
        gids = np.nonzero((sizes > complete_threshold) & (sizes >= self.tagore_min_group_size) &
                          (sizes > self.exact_max_nx))[0] + 1
        return gids.astype(np.uint32)

    def build_large_group_graph(self, group_ids=None, forward_cap: int | None = None,
                                reverse_cap: int | None = None) -> TagoreBatchBuildResult:
        """Graph rows of the large groups: exact candidate lists (list_k = min(64, tagore_k-1))
        and the FastGrnnd prune (ung_hip_prune_group_graph), with the defaults of
        make_fast_grnnd_prune_config (src/tagore_cuda_config.cpp:45-68)."""
        if group_ids is None:
            group_ids = self.large_groups()
        group_ids = np.asarray(group_ids, np.int64)
        begins = self.group_begin[group_ids].astype(np.uint32)
        sizes = (self.group_begin[group_ids + 1] - self.group_begin[group_ids]).astype(np.uint32)
        fd = self.max_degree
        tk = self.tagore_k if self.tagore_k > fd else fd + 1
        list_k = min(64, tk - 1)
        if forward_cap is None:
            forward_cap = min(tk - 1, max(fd, 2 * fd), list_k)
        if reverse_cap is None:
            reverse_cap = min(32, max(1, fd))
        st = self.ctx.group_knn_device(begins, sizes, list_k)
        graph, entries, st2 = self.ctx.prune_group_graph(int(sizes.astype(np.int64).sum()), len(group_ids),
                                                         forward_cap, reverse_cap, fd, self.alpha)
        offsets = np.zeros(len(group_ids) + 1, np.uint32)
        offsets[1:] = np.cumsum(sizes)
        st["prune_kernel_ms"] = st2["kernel_ms"]
        st["prune_wall_ms"] = st2["wall_ms"]
        return TagoreBatchBuildResult(graph, offsets, fd + 1, entries, None, None, st)

    def build_fast_exact_batch(self, group_ids=None, list_k: int | None = None,
                               head_keep: int | None = None, anchor_tail: int = 1,
                               anchor_slots: int = 0, bidir_anchor: int = 0) -> TagoreBatchBuildResult:
        """Exact intra-group kNN lists + anchor-packed rows for the mid groups."""
        if group_ids is None:
            group_ids = self.mid_groups()
        group_ids = np.asarray(group_ids, np.int64)
        begins = self.group_begin[group_ids].astype(np.uint32)
        sizes = (self.group_begin[group_ids + 1] - self.group_begin[group_ids]).astype(np.uint32)
        fd = self.max_degree
        tk = self.tagore_k if self.tagore_k > fd else fd + 1
        if head_keep is None:
            head_keep = fd - 8 if fd > 8 else fd
        if list_k is None:
            list_k = fd if (anchor_tail and anchor_slots == 0) else min(64, tk - 1)
        ids, dist, st = self.ctx.group_knn(begins, sizes, list_k)
        graph, entries, st2 = self.ctx.pack_anchor_rows(ids.shape[0], len(group_ids), tk, fd, head_keep,
                                                        anchor_tail, anchor_slots, bidir_anchor)
        offsets = np.zeros(len(group_ids) + 1, np.uint32)
        offsets[1:] = np.cumsum(sizes)
        st["pack_kernel_ms"] = st2["kernel_ms"]
        return TagoreBatchBuildResult(graph, offsets, fd + 1, entries, ids, dist, st)

    # ---- output boundary ------------------------------------------------------
    def merge_cross_edges_to_graph(self, neighbors: list):
        """Append each point's cross edges (FlatId rows, sentinel skipped) to its
        neighbour list, as CrossEdgeGraphMaterializationWriter::append_cross_edges."""
        ids = self.cross_flat_ids
        for p in range(ids.shape[0]):
            row = ids[p]
            neighbors[p].extend(int(v) for v in row if v != NONE_ID)
        return neighbors
