#!/usr/bin/env python3
"""Benchmark of the UNG cross-edge + mid-group kNN build stage on one MI355X.

Workload "cfg2" (the headline configuration): 1M x 128 fp32 vectors from a
1000-centroid Gaussian mixture, 40 labels (1-4 per vector, Zipf 1.2), k=6 cross
edges per vector and exact K=32 intra-group kNN for every mid-size group
(128 <= n <= 4096).  Synthetic, seeded data (no network).

A step = the whole device job with the base set already resident in HBM:
host work-list packing + descriptor upload + MFMA select + merge + exact
fallback for the cross edges, the additional edges of the groups whose
out-groups no cross edge reaches (edge lists returned to the host, as the
reference's materialized lists), and the intra-group kNN -- by default started on
the library's second stream with the cross edges (ung_hip_cross_intra_begin) and
collected after the additional edges (ung_hip_intra_end); --sequential runs the three
one after the other.  Cross and intra results stay in HBM.  value = (P_cross +
P_intra) / step time (distance evaluations/s, algorithmic pairs only).

Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense
MFMA_FP32_PEAK_TFLOPS = 157.3
HBM_PEAK_GBS = 8000.0
METRIC = "cross-edge build wall time + distance evals/s (MFMA util %), 1M×128 fp32, 1 GPU"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_select_cross_cfg2.txt")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def read_traffic(config_name):
    """HBM bytes per launch of the cross select kernel on cfg2, measured offline with
    rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE) and calibrated on a copy kernel; None for
    other workloads (not measured)."""
    if config_name != "cfg2" or not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                try:
                    return float(line.split(":", 1)[1].strip())
                except ValueError:
                    return None
    return None


def calib_copy(nbytes):
    """One device-to-device hipMemcpy of nbytes (the runtime's blit kernel): the
    reference reading for FETCH_SIZE / WRITE_SIZE in a rocprofv3 --pmc pass."""
    hip = C.CDLL("libamdhip64.so")
    src, dst = C.c_void_p(), C.c_void_p()
    for p in (src, dst):
        if hip.hipMalloc(C.byref(p), C.c_size_t(nbytes)) != 0:
            raise RuntimeError("hipMalloc failed in calib_copy")
    try:
        if hip.hipMemcpy(dst, src, C.c_size_t(nbytes), 3) != 0 or hip.hipDeviceSynchronize() != 0:
            raise RuntimeError("hipMemcpy failed in calib_copy")
    finally:
        hip.hipFree(src)
        hip.hipFree(dst)
    log(f"calibration copy {nbytes} bytes done")


def cpu_baseline(st, k, seconds=12.0, threads=None):
    """The reference's own compiled distance + SearchQueue (oracle/_ref) when built,
    else the plain-C oracle, on a bounded random sample of cross-edge queries."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Oracle, RefOracle, ref_available
    threads = threads or int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    kind = "reference" if ref_available() else "port"
    lib = RefOracle() if kind == "reference" else Oracle()
    sizes = np.diff(st.group_begin.astype(np.int64))[1:]
    out_cnt = np.diff(st.out_ptr.astype(np.int64))[1:]
    union = np.zeros(st.num_groups + 1, np.int64)
    for c in np.nonzero(out_cnt)[0] + 1:
        xs = st.out_idx[st.out_ptr[c]: st.out_ptr[c + 1]].astype(np.int64)
        union[c] = int(sizes[xs - 1].sum())
    point_group = st.new_vec_id_to_group_id
    eligible = np.nonzero(union[point_group] > 0)[0].astype(np.uint32)
    rng = np.random.default_rng(7)
    rng.shuffle(eligible)

    def run(nq):
        q = eligible[:nq]
        t0 = time.perf_counter()
        if kind == "reference":
            lib.cross_exact_points(st.base, st.group_begin, point_group, st.out_ptr, st.out_idx, q, k, threads)
        else:
            lib.cross_exact_points(st.base, st.group_begin, point_group, st.out_ptr, st.out_idx, q, k, threads)
        dt = time.perf_counter() - t0
        return int(union[point_group[q]].sum()), dt

    nq = min(len(eligible), 64)
    pairs, dt = run(nq)
    while dt < seconds / 8 and nq < len(eligible):
        nq = min(len(eligible), nq * 4)
        pairs, dt = run(nq)
    if dt < seconds / 2 and nq < len(eligible):
        nq = min(len(eligible), int(nq * (seconds / max(dt, 1e-3))))
        pairs, dt = run(nq)
    return {"value": pairs / dt, "unit": "distance evals/s", "cores": threads, "kind": kind,
            "sample": f"{nq} random cross-edge query points of cfg2 (exact scan of each point's "
                      f"minimum-superset union, {pairs} pairs, {dt:.1f} s, {threads} OpenMP threads)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--config", default="cfg2")
    ap.add_argument("--n", type=int, default=0, help="override point count (smaller runs)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--sequential", action="store_true",
                    help="cross edges, additional edges and the mid groups' kNN one after the other "
                         "(default: the kNN overlapped on the second stream)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--calib-copy", action="store_true",
                    help="end with a 1 GiB device-to-device copy (counter calibration for --pmc runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU (one-GPU boxes); "
                                   "multi-GPU sharding is not built", "n_gpus": args.gpus}))
        sys.exit(2)

    import filtervectorcode_refactor_amd as F
    from filtervectorcode_refactor_amd import datasets as D

    cfg = D.CONFIGS[args.config]
    if args.n:
        cfg = D.scaled(cfg, args.n)
    t0 = time.perf_counter()
    X, lp, li = D.generate(cfg)
    log(f"generated {cfg.name} in {time.perf_counter() - t0:.1f}s")
    st = F.UngBuildStage(num_cross_edges=cfg.k_cross, max_degree=cfg.k_intra)
    t0 = time.perf_counter()
    st.prepare_inputs(X, lp, li)
    del X
    lng_s = time.perf_counter() - t0
    gids = st.mid_groups()
    begins = st.group_begin[gids].astype(np.uint32)
    sizes = (st.group_begin[gids + 1] - st.group_begin[gids]).astype(np.uint32)
    p_cross, _ = F.count_pairs(st.group_begin, st.out_ptr, st.out_idx)
    p_intra = int((sizes.astype(np.int64) * (sizes.astype(np.int64) - 1)).sum())
    log(f"groups={st.num_groups} lng_edges={len(st.out_idx)} mid_groups={len(gids)} "
        f"P_cross={p_cross:.3e} P_intra={p_intra:.3e} inputs {lng_s:.1f}s")

    ctx = st.ctx
    up = ctx.prepare_vectors(st.base)
    log(f"resident upload {up['h2d_ms']:.1f} ms ({st.base.nbytes / up['h2d_ms'] / 1e6:.1f} GB/s incl. PCIe)")

    def step():
        if args.sequential:
            s1 = ctx.cross_topk_device(st.group_begin, st.out_ptr, st.out_idx, cfg.k_cross)
        else:  # the mid groups' kNN runs on the second stream beside the cross tail
            s1 = ctx.cross_intra_begin(st.group_begin, st.out_ptr, st.out_idx, cfg.k_cross, begins, sizes,
                                       cfg.k_intra)
        t0 = time.perf_counter()
        _, ef, _, s3 = ctx.additional_edges(st.group_begin, st.out_ptr, st.out_idx, cfg.k_cross)
        s3["wall_ms"] = (time.perf_counter() - t0) * 1e3
        s3["edges"] = int(ef.size)
        s2 = ctx.group_knn_device(begins, sizes, cfg.k_intra) if args.sequential else ctx.intra_end()
        return s1, s2, s3

    for _ in range(args.warmup):
        step()
    ctx.synchronize()
    cross_stats, intra_stats, addl_stats = [], [], []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        s1, s2, s3 = step()
        cross_stats.append(s1)
        intra_stats.append(s2)
        addl_stats.append(s3)
    ctx.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps

    def avg(lst, key):
        return float(np.mean([s[key] for s in lst]))

    sel_cross_ms = avg(cross_stats, "select_ms")
    sel_intra_ms = avg(intra_stats, "select_ms")
    d = cfg.dim
    dp = (d + 31) // 32 * 32
    # The cross select kernel's two floors: its MFMA work (three bf16 products per fp32
    # product: 3 * 2 * dp flops per algorithmic pair, against the dense bf16 peak) and its
    # HBM traffic (measured, against 8 TB/s).  The larger floor is the roofline that
    # bounds it; achieved = algorithmic bytes (query + candidate rows each work item
    # streams) or flops per launch / the launch's average duration.
    sel_s = sel_cross_ms * 1e-3
    flops_cross = 2.0 * d * p_cross
    mfma_flops = 3.0 * 2.0 * dp * p_cross
    alg_bytes = float(cross_stats[-1]["select_bytes"])
    traffic = read_traffic(cfg.name) if not args.n else None
    mfma_floor_ms = mfma_flops / (MFMA_BF16_PEAK_TFLOPS * 1e12) * 1e3
    hbm_floor_ms = (traffic if traffic else alg_bytes) / (HBM_PEAK_GBS * 1e9) * 1e3
    mfma_tflops = mfma_flops / sel_s / 1e12
    hbm_gbs = alg_bytes / sel_s / 1e9
    if hbm_floor_ms >= mfma_floor_ms:
        roofline = {"bound": "hbm", "achieved": round(hbm_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(hbm_gbs / HBM_PEAK_GBS, 4), "traffic": traffic}
    else:
        roofline = {"bound": "mfma", "achieved": round(mfma_tflops, 3), "peak": MFMA_BF16_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(mfma_tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": traffic}
    roofline.update({
        "kernel": ("ung_select_kernel<8,1,false,2,true> (cross edges, register-query layout, one launch per step)"
                   if dp == 128 else "ung_select_kernel<8,1,false,2,false> (cross edges, one launch per step)"),
        "avg_launch_ms": round(sel_cross_ms, 4),
        "alg_bytes_per_launch": alg_bytes, "hbm_floor_ms": round(hbm_floor_ms, 3),
        "mfma_bf16_flops_per_launch": mfma_flops, "mfma_floor_ms": round(mfma_floor_ms, 3),
        "mfma_bf16_tflops": round(mfma_tflops, 2), "mfma_bf16_frac": round(mfma_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        "measured_hbm_gbs": round(traffic / sel_s / 1e9, 1) if traffic else None,
        "fp32_equiv_tflops": round(flops_cross / sel_s / 1e12, 2),
    })
    value = (p_cross + p_intra) / (ms_per_step * 1e-3)
    result = {
        "metric": METRIC, "value": value, "unit": "distance evals/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32 (3xbf16 MFMA pre-select, exact f32 re-score)",
        "data": "synthetic",
        "config": {"workload": f"{cfg.name}: {cfg.n}x{cfg.dim} fp32 Gaussian mixture "
                               f"({cfg.n_centroids} centroids, sigma {cfg.sigma}), vocab {cfg.vocab}, "
                               f"{cfg.m_min}-{cfg.m_max} labels Zipf({cfg.zipf_s}); cross k={cfg.k_cross} + "
                               f"intra exact K={cfg.k_intra} for 128<=n<=4096",
                   "groups": st.num_groups, "lng_edges": int(len(st.out_idx)), "mid_groups": int(len(gids)),
                   "P_cross": int(p_cross), "P_intra": int(p_intra),
                   "intra_overlapped": not args.sequential},
        "roofline": roofline,
        "breakdown": {
            "cross_wall_ms": round(avg(cross_stats, "wall_ms"), 3),
            "cross_plan_ms": round(avg(cross_stats, "plan_ms"), 3),
            "cross_h2d_ms": round(avg(cross_stats, "h2d_ms"), 3),
            "cross_select_ms": round(sel_cross_ms, 3),
            "cross_merge_ms": round(avg(cross_stats, "merge_ms"), 3),
            "cross_fallback_ms": round(avg(cross_stats, "fallback_ms"), 3),
            "cross_fallback_rows": int(cross_stats[-1]["fallback_rows"]),
            "cross_padded_pairs": int(cross_stats[-1]["padded_pairs"]),
            "additional_wall_ms": round(avg(addl_stats, "wall_ms"), 3),
            "additional_kernel_ms": round(avg(addl_stats, "kernel_ms"), 3),
            "additional_edges": int(addl_stats[-1]["edges"]),
            "additional_query_rows": int(addl_stats[-1]["rows"]),
            "intra_wall_ms": round(avg(intra_stats, "wall_ms"), 3),
            "intra_select_ms": round(sel_intra_ms, 3),
            "intra_merge_ms": round(avg(intra_stats, "merge_ms"), 3),
            "intra_fallback_rows": int(intra_stats[-1]["fallback_rows"]),
            "intra_select_tflops": round(2.0 * d * p_intra / (sel_intra_ms * 1e-3) / 1e12, 3) if p_intra else None,
            "cross_evals_per_s": p_cross / (avg(cross_stats, "wall_ms") * 1e-3),
            "resident_upload_ms": round(up["h2d_ms"], 3),
        },
    }
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(st, cfg.k_cross, seconds=args.cpu_seconds)
    st.close()
    if args.calib_copy:
        calib_copy(1 << 30)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
