"""Seeded synthetic workloads of the benchmark configurations, and the
reference's on-disk formats.

Configurations (vectors / labels; seeds fixed here):
  cfg1  10k x 128, i.i.d. N(0,1); vocab 20, 1-3 labels, Zipf(1.2)           (plumbing)
  cfg2  1M x 128, 1000-centroid mixture (scale 1.0, sigma 0.3);
        vocab 40, 1-4 labels, Zipf(1.2); k=6 cross edges, K=32 intra kNN     (headline)
  cfg3  1M x 384, mixture then L2-normalised; vocab 40, 1-6 labels, Zipf(1.0)
  cfg4  2M x 768, normalised mixture; hierarchical labels (1 of 10 parents +
        0-3 children from that parent's block of 9)
  cfg5  10M x 128, 10k-centroid mixture; labels as cfg2
"Labels per vector" is read as a uniform count m in [m_min, m_max] whose label
identities are drawn by Zipf rank without replacement.

Formats: vectors ``.bin`` = uint32 n, uint32 dim, float32[n*dim]
(src/storage.cpp:114-120); labels = one line per vector, comma-separated
(src/storage.cpp:133-147).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import check, ptr


@dataclass(frozen=True)
class Config:
    name: str
    n: int
    dim: int
    n_centroids: int
    centroid_scale: float
    sigma: float
    normalize: bool
    label_mode: int  # 0 zipf, 1 hierarchical
    vocab: int
    m_min: int
    m_max: int
    zipf_s: float
    seed_c: int
    seed_x: int
    seed_l: int
    k_cross: int = 6
    k_intra: int = 32


CONFIGS = {
    "cfg1": Config("cfg1", 10_000, 128, 0, 1.0, 1.0, False, 0, 20, 1, 3, 1.2,
                   20261200, 20261201, 20261202),
    "cfg2": Config("cfg2", 1_000_000, 128, 1000, 1.0, 0.3, False, 0, 40, 1, 4, 1.2,
                   20261211, 20261212, 20261213),
    "cfg3": Config("cfg3", 1_000_000, 384, 1000, 1.0, 0.3, True, 0, 40, 1, 6, 1.0,
                   20261221, 20261222, 20261223),
    "cfg4": Config("cfg4", 2_000_000, 768, 1000, 1.0, 0.3, True, 1, 100, 1, 4, 0.0,
                   20261231, 20261232, 20261233),
    "cfg5": Config("cfg5", 10_000_000, 128, 10000, 1.0, 0.3, False, 0, 40, 1, 4, 1.2,
                   20261241, 20261242, 20261243),
}


def scaled(cfg: Config, n: int) -> Config:
    """The same generator at another size (tests use small n)."""
    d = dict(cfg.__dict__)
    d["n"] = int(n)
    d["name"] = f"{cfg.name}@{n}"
    return Config(**d)


def synth_vectors(cfg: Config, nthreads: int = 0) -> np.ndarray:
    lib = _lib.load()
    X = np.empty((cfg.n, cfg.dim), np.float32)
    check(lib.ung_synth_vectors(cfg.n, cfg.dim, cfg.n_centroids, cfg.centroid_scale, cfg.sigma,
                                int(cfg.normalize), cfg.seed_c, cfg.seed_x, ptr(X), nthreads))
    return X


def synth_labels(cfg: Config, nthreads: int = 0):
    lib = _lib.load()
    width = cfg.m_max if cfg.label_mode == 0 else 4
    lab_ptr = np.empty(cfg.n + 1, np.uint32)
    lab_idx = np.empty(cfg.n * width, np.uint32)
    check(lib.ung_synth_labels(cfg.n, cfg.label_mode, cfg.vocab, cfg.m_min, cfg.m_max, cfg.zipf_s,
                               cfg.seed_l, ptr(lab_ptr), ptr(lab_idx), nthreads))
    return lab_ptr, lab_idx[: lab_ptr[-1]].copy()


def generate(cfg: Config, nthreads: int = 0):
    """(X [n x dim] float32, lab_ptr [n+1], lab_idx) in ORIGINAL point order."""
    return synth_vectors(cfg, nthreads), *synth_labels(cfg, nthreads)


def write_bin(path: str, X: np.ndarray) -> None:
    X = np.ascontiguousarray(X, np.float32)
    with open(path, "wb") as f:
        np.array([X.shape[0], X.shape[1]], np.uint32).tofile(f)
        X.tofile(f)


def read_bin(path: str) -> np.ndarray:
    with open(path, "rb") as f:
        n, d = np.fromfile(f, np.uint32, 2)
        return np.fromfile(f, np.float32, int(n) * int(d)).reshape(int(n), int(d))


def write_labels(path: str, lab_ptr, lab_idx) -> None:
    with open(path, "w") as f:
        for i in range(len(lab_ptr) - 1):
            row = lab_idx[lab_ptr[i]: lab_ptr[i + 1]]
            f.write(",".join(str(int(v)) for v in row) + "\n")


def read_labels(path: str, n: int):
    """Parse like Storage::load_from_file: ints split on ',', sorted per row; a
    missing file gives every vector the label set {1} (src/storage.cpp:133-158)."""
    import os
    rows = []
    if os.path.exists(path):
        with open(path) as f:
            for i, line in zip(range(n), f):
                line = line.rstrip("\n")
                rows.append(sorted(int(t) for t in line.split(",") if t.strip() != "") if line else [])
        rows += [[] for _ in range(n - len(rows))]
    else:
        rows = [[1] for _ in range(n)]
    lab_ptr = np.zeros(n + 1, np.uint32)
    lab_ptr[1:] = np.cumsum([len(r) for r in rows])
    lab_idx = np.array([v for r in rows for v in r], np.uint32)
    return lab_ptr, lab_idx
