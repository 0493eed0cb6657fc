#!/usr/bin/env python3
"""Writes the golden fixtures of tests/golden/ from the reference's OWN compiled
code: oracle/_ref/libungref.so = UNG/codes/src/distance.cpp + search_queue.cpp +
trie.cpp built from /root/reference by oracle/Makefile, driven by
oracle/ref_driver.cpp (restating build_trie_and_divide_groups + the LNG phase 1
with get_min_super_sets_optimized_bucket, build_cross_edges_generate_cpu_exact_scan,
build_cross_edges_generate_additional (exact branch) and
build_exact_topk_graph_for_points around those objects).

Inputs come from the product's seeded generator (cfg1 and a d=384 normalised
variant); their SHA-256 digests are stored so a test can tell input drift from
result drift.  Fixtures are data only (inputs' digests, expected outputs).

Run in the build container (needs /root/reference):  python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import filtervectorcode_refactor_amd as F  # noqa: E402
from filtervectorcode_refactor_amd import datasets as D  # noqa: E402
from oracle import RefOracle  # noqa: E402


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def make(cfg, name, k_cross=6, k_intra=32, intra_row_stride=1):
    ref = RefOracle()
    X, lp, li = D.generate(cfg)
    st = F.UngBuildStage()
    st.prepare_inputs(X, lp, li)
    # groups and LNG rows from the reference's own TrieIndex (oracle/_ref); the product's
    # reorder is only used to lay out the vectors group by group
    G, pg, out_ptr, out_idx = ref.trie_lng(lp, li)
    assert G == st.num_groups and np.array_equal(pg, st._point_group_old)
    in_ptr, in_idx = F.in_neighbors(out_ptr, out_idx)
    ids, dists, size = ref.cross_exact(st.base, st.group_begin, in_ptr, in_idx, k_cross)
    addl_ptr, addl_from, addl_to = ref.additional_edges(st.base, st.group_begin, out_ptr, out_idx,
                                                        ids, k_cross)
    gids = st.mid_groups()
    rows_i, rows_d, grp_of_row, local_row = [], [], [], []
    for g in gids:
        b, e = int(st.group_begin[g]), int(st.group_begin[g + 1])
        oi, od = ref.intra_exact(st.base, b, e - b, k_intra)
        rows_i.append(oi)
        rows_d.append(od)
        grp_of_row.append(np.full(e - b, g, np.uint32))
        local_row.append(np.arange(e - b, dtype=np.uint32))
    intra_ids = np.concatenate(rows_i) if rows_i else np.zeros((0, k_intra), np.uint32)
    intra_d = np.concatenate(rows_d) if rows_d else np.zeros((0, k_intra), np.float32)
    keep = np.arange(0, intra_ids.shape[0], intra_row_stride)
    out = dict(
        x_sha256=np.array(sha(X)), labels_sha256=np.array(sha(lp, li)),
        group_begin=st.group_begin, out_ptr=out_ptr, out_idx=out_idx,
        cross_ids=ids, cross_dists=dists, cross_size=size,
        cross_sha256=np.array(sha(ids, dists, size)),
        addl_ptr=addl_ptr, addl_from=addl_from, addl_to=addl_to,
        intra_groups=gids, intra_k=np.array(k_intra),
        intra_sha256=np.array(sha(intra_ids, intra_d)),
        intra_rows=keep.astype(np.uint32),
        intra_row_group=np.concatenate(grp_of_row)[keep] if grp_of_row else np.zeros(0, np.uint32),
        intra_row_local=np.concatenate(local_row)[keep] if local_row else np.zeros(0, np.uint32),
        intra_ids=intra_ids[keep].astype(np.uint16), intra_dists=intra_d[keep],
    )
    path = os.path.join(HERE, name)
    np.savez_compressed(path, **out)
    print(f"wrote {path}: N={X.shape[0]} d={X.shape[1]} groups={st.num_groups} "
          f"mid={len(gids)} intra_rows={intra_ids.shape[0]} stored={len(keep)} "
          f"size={os.path.getsize(path)} B")


def make_tiny():
    """Hand-sized problems with known structure: ties from duplicated vectors,
    unions smaller than k, a group with no supersets, dim not a multiple of 8."""
    ref = RefOracle()
    rng = np.random.default_rng(5)
    cases = {}
    # groups: 1={1}, 2={1,2}, 3={1,3}, 4={1,2,3}, 5={4}
    sizes = [6, 3, 2, 4, 5]
    gb = np.zeros(len(sizes) + 2, np.uint32)
    gb[2:] = np.cumsum(sizes)
    out_ptr = np.array([0, 0, 2, 3, 4, 4, 4], np.uint32)
    out_idx = np.array([2, 3, 4, 4], np.uint32)
    in_ptr, in_idx = F.in_neighbors(out_ptr, out_idx)
    for dim in (3, 7, 12):
        X = rng.integers(-3, 4, size=(int(gb[-1]), dim)).astype(np.float32)  # small ints: many exact ties
        X[7] = X[0]
        for k in (1, 2, 6):
            ids, dists, size = ref.cross_exact(X, gb, in_ptr, in_idx, k)
            cases[f"d{dim}_k{k}_X"] = X
            cases[f"d{dim}_k{k}_ids"] = ids
            cases[f"d{dim}_k{k}_dists"] = dists
            cases[f"d{dim}_k{k}_size"] = size
        ii, idd = ref.intra_exact(X, 0, 6, 4)
        cases[f"d{dim}_intra_ids"] = ii
        cases[f"d{dim}_intra_dists"] = idd
    cases["group_begin"] = gb
    cases["out_ptr"] = out_ptr
    cases["out_idx"] = out_idx
    path = os.path.join(HERE, "tiny_cases.npz")
    np.savez_compressed(path, **cases)
    print(f"wrote {path} ({os.path.getsize(path)} B)")


if __name__ == "__main__":
    make(D.CONFIGS["cfg1"], "cfg1_ref.npz", intra_row_stride=4)
    make(D.scaled(D.CONFIGS["cfg3"], 6000), "cfg3_6k_ref.npz", intra_row_stride=8)
    make_tiny()
