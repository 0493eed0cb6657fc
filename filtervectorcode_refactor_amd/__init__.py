"""MI355X-native UNG cross-edge / mid-group kNN build stage.

The product is libung_hip.so (C ABI in include/ung_hip.h: gfx950 kernels plus the
host-side inputs of the path).  This package binds it with ctypes and mirrors the
reference's UniNavGraph build-stage interface (``UngBuildStage``).
"""
from ._lib import LIB_PATH, Stats, UngHipError, load  # noqa: F401
from .ung import (HipContext, TagoreBatchBuildResult, UngBuildStage, assemble_graph_csr,  # noqa: F401
                  count_pairs, divide_groups, graph_save_text, group_label_sets, in_neighbors, lng_build,
                  reorder_rows)
from . import datasets  # noqa: F401

__all__ = [
    "LIB_PATH", "Stats", "UngHipError", "load", "HipContext", "TagoreBatchBuildResult",
    "UngBuildStage", "assemble_graph_csr", "count_pairs", "divide_groups", "graph_save_text",
    "group_label_sets", "in_neighbors", "lng_build", "reorder_rows", "datasets",
]
