"""ctypes bindings for the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker / timed CPU
baseline.  The product package never imports it.

``Oracle`` wraps oracle/liboracle.so (plain-C restatement, ung_oracle.c);
``RefOracle`` wraps oracle/_ref/libungref.so (the reference's own
distance.cpp + search_queue.cpp compiled from /root/reference, see
oracle/Makefile), when that library has been built.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libungref.so")

_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")


def _u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


_ADDL_ARGS = [_f32p, C.c_uint32, C.c_uint32, C.c_uint32, _u32p, _u32p, _u32p, _u32p, C.c_uint32,
              C.c_uint32, _u32p, _u32p, _u32p, C.c_int64, C.POINTER(C.c_int64)]


def _additional_edges(fn, X, group_begin, out_ptr, out_idx, cross_ids, num_cross):
    """Shared driver of the two additional-edge restatements: returns
    (edge_ptr[G+2], edge_from, edge_to)."""
    X = _f32(X)
    N, d = X.shape
    G = group_begin.shape[0] - 2
    cross_ids = _u32(cross_ids)
    stride = cross_ids.shape[1] if cross_ids.ndim == 2 else 1
    out_idx = _u32(out_idx) if len(out_idx) else np.zeros(1, np.uint32)
    ptr = np.zeros(G + 2, np.uint32)
    need = C.c_int64(0)
    cap = 1 << 16
    while True:
        ef = np.zeros(cap, np.uint32)
        et = np.zeros(cap, np.uint32)
        n = fn(X, N, d, G, _u32(group_begin), _u32(out_ptr), out_idx, cross_ids.reshape(-1), stride,
               num_cross, ptr, ef, et, cap, C.byref(need))
        if n >= 0:
            return ptr, ef[:n].copy(), et[:n].copy()
        cap = int(need.value)


_ASM_ARGS = [C.c_uint64, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_uint32,
             C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64]


def _opt(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


def _assemble(fn, N, group_begin, intra_ptr, intra_idx, intra_global, cross_ids, num_cross,
              add_ptr, add_from, add_to):
    """Shared driver of the two final-adjacency restatements: (row_ptr[N+1], col_idx)."""
    G = group_begin.shape[0] - 2
    ip, ii = _opt(intra_ptr, np.uint64), _opt(intra_idx, np.uint32)
    cr = _opt(cross_ids, np.uint32)
    stride = 0 if cr is None else (cr.shape[1] if cr.ndim == 2 else 1)
    ap, af, at = _opt(add_ptr, np.uint32), _opt(add_from, np.uint32), _opt(add_to, np.uint32)
    if ii is not None and ii.size == 0:
        ii = np.zeros(1, np.uint32)
    if af is not None and af.size == 0:
        af, at = np.zeros(1, np.uint32), np.zeros(1, np.uint32)
    row_ptr = np.zeros(N + 1, np.uint64)
    p = lambda a: None if a is None else a.ctypes.data
    gb = _u32(group_begin)
    cap = 1 << 20
    while True:
        col = np.zeros(cap, np.uint32)
        n = fn(N, G, p(gb), p(ip), p(ii), int(intra_global), p(None if cr is None else cr.reshape(-1)), stride,
               num_cross, p(ap), p(af), p(at), p(row_ptr), p(col), cap)
        if n >= 0:
            return row_ptr, col[:n].copy()
        cap *= 4


class Oracle:
    """Plain-C restatement of the reference CPU semantics."""

    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (run `make -C oracle`)")
        L = C.CDLL(path)
        L.ungo_l2.restype = C.c_float
        L.ungo_l2.argtypes = [_f32p, _f32p, C.c_uint32]
        L.ungo_l2_pairs.restype = None
        L.ungo_l2_pairs.argtypes = [_f32p, C.c_uint32, _u32p, _u32p, C.c_uint64, _f32p]
        L.ungo_l2_f64.restype = C.c_double
        L.ungo_l2_f64.argtypes = [_f32p, _f32p, C.c_uint32]
        L.ungo_queue_insert.restype = C.c_int
        L.ungo_queue_insert.argtypes = [_u32p, _f32p, C.POINTER(C.c_int32), C.c_int32,
                                        C.c_uint32, C.c_float]
        L.ungo_divide_groups.restype = C.c_uint32
        L.ungo_divide_groups.argtypes = [C.c_uint32, _u32p, _u32p, _u32p, _u32p, _u32p]
        L.ungo_min_supersets.restype = C.c_int64
        L.ungo_min_supersets.argtypes = [C.c_uint32, _u32p, _u32p, _u32p, _u32p, C.c_int64]
        L.ungo_cross_exact.restype = None
        L.ungo_cross_exact.argtypes = [_f32p, C.c_uint32, C.c_uint32, C.c_uint32, _u32p, _u32p,
                                       _u32p, C.c_uint32, _u32p, _f32p, _i32p, C.c_int]
        L.ungo_cross_exact_points.restype = None
        L.ungo_cross_exact_points.argtypes = [_f32p, C.c_uint32, C.c_uint32, C.c_uint32, _u32p,
                                              _u32p, _u32p, _u32p, _u32p, C.c_uint32, C.c_uint32,
                                              _u32p, _f32p, _i32p, C.c_int]
        L.ungo_intra_exact.restype = None
        L.ungo_intra_exact.argtypes = [_f32p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                       _u32p, _f32p, C.c_int]
        L.ungo_additional_edges.restype = C.c_int64
        L.ungo_additional_edges.argtypes = _ADDL_ARGS
        L.ungo_assemble_graph.restype = C.c_int64
        L.ungo_assemble_graph.argtypes = _ASM_ARGS
        L.ungo_large_group_graph.restype = None
        L.ungo_large_group_graph.argtypes = [_f32p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                             C.c_uint32, C.c_uint32, C.c_float, _u32p]
        L.ungo_pack_anchor_row.restype = None
        L.ungo_pack_anchor_row.argtypes = [_u32p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                           C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                           C.c_uint32, _u32p]
        self.lib = L

    # -- distances -------------------------------------------------------
    def l2(self, a, b) -> float:
        a, b = _f32(a), _f32(b)
        return float(self.lib.ungo_l2(a, b, a.shape[0]))

    def l2_pairs(self, X, a, b):
        """ungo_l2 of the row pairs (X[a[i]], X[b[i]]); +inf where b[i] is UINT32_MAX."""
        X = _f32(X)
        a, b = _u32(a).reshape(-1), _u32(b).reshape(-1)
        out = np.empty(a.shape[0], np.float32)
        self.lib.ungo_l2_pairs(X, X.shape[1], a, b, a.shape[0], out)
        return out

    def l2_f64(self, a, b) -> float:
        a, b = _f32(a), _f32(b)
        return float(self.lib.ungo_l2_f64(a, b, a.shape[0]))

    # -- queue -----------------------------------------------------------
    def queue_stream(self, ids, dists, cap):
        qi = np.zeros(cap + 1, np.uint32)
        qd = np.zeros(cap + 1, np.float32)
        size = C.c_int32(0)
        for i, d in zip(np.asarray(ids, np.uint32), np.asarray(dists, np.float32)):
            self.lib.ungo_queue_insert(qi, qd, C.byref(size), cap, int(i), float(d))
        return qi[: size.value].copy(), qd[: size.value].copy()

    # -- groups / LNG -----------------------------------------------------
    def divide_groups(self, lab_ptr, lab_idx):
        lab_ptr, lab_idx = _u32(lab_ptr), _u32(lab_idx)
        n = lab_ptr.shape[0] - 1
        pg = np.zeros(max(n, 1), np.uint32)
        gb = np.zeros(n + 2, np.uint32)
        n2o = np.zeros(max(n, 1), np.uint32)
        G = self.lib.ungo_divide_groups(n, lab_ptr, lab_idx if lab_idx.size else np.zeros(1, np.uint32), pg, gb, n2o)
        return int(G), pg[:n], gb[: G + 2], n2o[:n]

    def min_supersets(self, set_ptr, set_idx):
        set_ptr, set_idx = _u32(set_ptr), _u32(set_idx)
        G = set_ptr.shape[0] - 2
        cap = max(16, G * 64)
        while True:
            out_ptr = np.zeros(G + 2, np.uint32)
            out_idx = np.zeros(cap, np.uint32)
            tot = self.lib.ungo_min_supersets(G, set_ptr, set_idx if set_idx.size else np.zeros(1, np.uint32),
                                              out_ptr, out_idx, cap)
            if tot >= 0:
                return out_ptr, out_idx[:tot].copy()
            cap *= 4

    # -- builders ----------------------------------------------------------
    def cross_exact(self, X, group_begin, in_ptr, in_idx, k, nthreads=0):
        X = _f32(X)
        N, d = X.shape
        G = group_begin.shape[0] - 2
        ids = np.zeros((N, k), np.uint32)
        dists = np.zeros((N, k), np.float32)
        size = np.zeros(N, np.int32)
        in_idx = _u32(in_idx) if len(in_idx) else np.zeros(1, np.uint32)
        self.lib.ungo_cross_exact(X, N, d, G, _u32(group_begin), _u32(in_ptr), in_idx,
                                  k, ids, dists, size, nthreads)
        return ids, dists, size

    def cross_exact_points(self, X, group_begin, point_group, out_ptr, out_idx, q_list, k, nthreads=0):
        X = _f32(X)
        N, d = X.shape
        G = group_begin.shape[0] - 2
        q_list = _u32(q_list)
        nq = q_list.shape[0]
        ids = np.zeros((nq, k), np.uint32)
        dists = np.zeros((nq, k), np.float32)
        size = np.zeros(nq, np.int32)
        out_idx = _u32(out_idx) if len(out_idx) else np.zeros(1, np.uint32)
        self.lib.ungo_cross_exact_points(X, N, d, G, _u32(group_begin), _u32(point_group),
                                         _u32(out_ptr), out_idx, q_list, nq, k, ids, dists, size,
                                         nthreads)
        return ids, dists, size

    def intra_exact(self, X, begin, n, K, nthreads=0):
        X = _f32(X)
        ids = np.zeros((n, K), np.uint32)
        dists = np.zeros((n, K), np.float32)
        self.lib.ungo_intra_exact(X, X.shape[1], begin, n, K, ids, dists, nthreads)
        return ids, dists

    def large_group_graph(self, X, begin, n, knn_k=63, forward_cap=63, reverse_cap=32, final_degree=32,
                          alpha=1.2):
        """Rows [n x (final_degree+1)] of ungo_large_group_graph (count, local ids, padding)."""
        X = _f32(X)
        rows = np.zeros((n, final_degree + 1), np.uint32)
        self.lib.ungo_large_group_graph(X, X.shape[1], begin, n, knn_k, forward_cap, reverse_cap, final_degree,
                                        alpha, rows)
        return rows

    def additional_edges(self, X, group_begin, out_ptr, out_idx, cross_ids, num_cross):
        return _additional_edges(self.lib.ungo_additional_edges, X, group_begin, out_ptr, out_idx,
                                 cross_ids, num_cross)

    def assemble_graph(self, N, group_begin, intra_ptr, intra_idx, intra_global, cross_ids, num_cross,
                       add_ptr, add_from, add_to):
        return _assemble(self.lib.ungo_assemble_graph, N, group_begin, intra_ptr, intra_idx, intra_global,
                         cross_ids, num_cross, add_ptr, add_from, add_to)

    def pack_anchor_row(self, top_idx, cand_degree, n, local_src, final_degree, head_keep,
                        anchor_tail=1, anchor_slots=0, bidir_anchor=0, graph_stride=None):
        if graph_stride is None:
            graph_stride = final_degree + 1
        top = _u32(top_idx) if len(top_idx) else np.zeros(1, np.uint32)
        row = np.zeros(graph_stride, np.uint32)
        self.lib.ungo_pack_anchor_row(top, cand_degree, n, local_src, final_degree, head_keep,
                                      anchor_tail, anchor_slots, bidir_anchor, graph_stride, row)
        return row


class RefOracle:
    """The reference's own compiled distance + SearchQueue (oracle/_ref)."""

    def __init__(self, path: str = REF_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (needs /root/reference; `make -C oracle ref`)")
        L = C.CDLL(path)
        L.ungref_l2.restype = C.c_float
        L.ungref_l2.argtypes = [_f32p, _f32p, C.c_uint32]
        L.ungref_queue_stream.restype = C.c_int32
        L.ungref_queue_stream.argtypes = [_u32p, _f32p, C.c_uint32, C.c_int32, _u32p, _f32p]
        L.ungref_cross_exact.restype = None
        L.ungref_cross_exact.argtypes = [_f32p, C.c_uint32, C.c_uint32, C.c_uint32, _u32p, _u32p,
                                         _u32p, C.c_uint32, _u32p, _f32p, _i32p, C.c_int]
        L.ungref_cross_exact_points.restype = None
        L.ungref_cross_exact_points.argtypes = [_f32p, C.c_uint32, _u32p, _u32p, _u32p, _u32p,
                                                _u32p, C.c_uint32, C.c_uint32, _u32p, _f32p, C.c_int]
        L.ungref_intra_exact.restype = None
        L.ungref_intra_exact.argtypes = [_f32p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                         _u32p, _f32p, C.c_int]
        L.ungref_additional_edges.restype = C.c_int64
        L.ungref_additional_edges.argtypes = _ADDL_ARGS
        L.ungref_assemble_graph.restype = C.c_int64
        L.ungref_assemble_graph.argtypes = _ASM_ARGS
        L.ungref_graph_save.restype = None
        L.ungref_graph_save.argtypes = [C.c_char_p, C.c_uint64, C.POINTER(C.c_uint64), _u32p]
        L.ungref_trie_lng.restype = C.c_int64
        L.ungref_trie_lng.argtypes = [C.c_uint64, _u32p, _u32p, _u32p, C.POINTER(C.c_uint32), _u32p, _u32p,
                                      C.c_int64]
        self.lib = L

    def trie_lng(self, lab_ptr, lab_idx):
        """Groups and LNG with the reference's own TrieIndex (ungref_trie_lng):
        (G, point_group[N], out_ptr[G+2], out_idx) -- rows in the reference's order."""
        lab_ptr = _u32(lab_ptr)
        lab_idx = _u32(lab_idx) if len(lab_idx) else np.zeros(1, np.uint32)
        N = lab_ptr.shape[0] - 1
        pg = np.zeros(max(N, 1), np.uint32)
        G = C.c_uint32(0)
        out_ptr = np.zeros(N + 2, np.uint32)
        cap = max(4 * N, 16)
        while True:
            out_idx = np.zeros(cap, np.uint32)
            n = self.lib.ungref_trie_lng(N, lab_ptr, lab_idx, pg, C.byref(G), out_ptr, out_idx, cap)
            if n <= cap:
                break
            cap = int(n)
        g = G.value
        return g, pg[:N].copy(), out_ptr[: g + 2].copy(), out_idx[:n].copy()

    def l2(self, a, b) -> float:
        a, b = _f32(a), _f32(b)
        return float(self.lib.ungref_l2(a, b, a.shape[0]))

    def queue_stream(self, ids, dists, cap):
        ids, dists = _u32(ids), _f32(dists)
        oi = np.zeros(max(cap, 1), np.uint32)
        od = np.zeros(max(cap, 1), np.float32)
        n = self.lib.ungref_queue_stream(ids, dists, ids.shape[0], cap, oi, od)
        return oi[:n].copy(), od[:n].copy()

    def cross_exact(self, X, group_begin, in_ptr, in_idx, k, nthreads=0):
        X = _f32(X)
        N, d = X.shape
        G = group_begin.shape[0] - 2
        ids = np.zeros((N, k), np.uint32)
        dists = np.zeros((N, k), np.float32)
        size = np.zeros(N, np.int32)
        in_idx = _u32(in_idx) if len(in_idx) else np.zeros(1, np.uint32)
        self.lib.ungref_cross_exact(X, N, d, G, _u32(group_begin), _u32(in_ptr), in_idx,
                                    k, ids, dists, size, nthreads)
        return ids, dists, size

    def cross_exact_points(self, X, group_begin, point_group, out_ptr, out_idx, q_list, k, nthreads=0):
        X = _f32(X)
        q_list = _u32(q_list)
        nq = q_list.shape[0]
        ids = np.zeros((nq, k), np.uint32)
        dists = np.zeros((nq, k), np.float32)
        out_idx = _u32(out_idx) if len(out_idx) else np.zeros(1, np.uint32)
        self.lib.ungref_cross_exact_points(X, X.shape[1], _u32(group_begin), _u32(point_group),
                                           _u32(out_ptr), out_idx, q_list, nq, k, ids, dists,
                                           nthreads)
        return ids, dists

    def intra_exact(self, X, begin, n, K, nthreads=0):
        X = _f32(X)
        ids = np.zeros((n, K), np.uint32)
        dists = np.zeros((n, K), np.float32)
        self.lib.ungref_intra_exact(X, X.shape[1], begin, n, K, ids, dists, nthreads)
        return ids, dists

    def additional_edges(self, X, group_begin, out_ptr, out_idx, cross_ids, num_cross):
        return _additional_edges(self.lib.ungref_additional_edges, X, group_begin, out_ptr, out_idx,
                                 cross_ids, num_cross)

    def assemble_graph(self, N, group_begin, intra_ptr, intra_idx, intra_global, cross_ids, num_cross,
                       add_ptr, add_from, add_to):
        return _assemble(self.lib.ungref_assemble_graph, N, group_begin, intra_ptr, intra_idx, intra_global,
                         cross_ids, num_cross, add_ptr, add_from, add_to)

    def graph_save(self, path, row_ptr, col_idx):
        row_ptr = np.ascontiguousarray(row_ptr, np.uint64)
        col = _u32(col_idx) if len(col_idx) else np.zeros(1, np.uint32)
        self.lib.ungref_graph_save(str(path).encode(), row_ptr.shape[0] - 1,
                                   row_ptr.ctypes.data_as(C.POINTER(C.c_uint64)), col)


def ref_available() -> bool:
    return os.path.exists(REF_PATH)
