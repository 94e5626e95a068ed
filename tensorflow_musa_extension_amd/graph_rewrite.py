"""Host side of the graph rewrite: serialized GraphDef in, serialized GraphDef out.

Mirrors what the reference's Grappler optimizer does for the hot path
(musa_ext/mu/optimizer/musa_graph_optimizer.cc:5480-5994: fusion patterns in
priority groups to a fixed point, then grouping of optimizer updates,
:2014-2120) through the C entry point TFMA_OptimizeGraph.  The
``disabled_patterns`` names are the reference's ``disabled_fusion_patterns``
parameter (:5448-5475) for the patterns this pass has.
"""
import ctypes

from . import _lib
from .errors import raise_for_status

PATTERNS = ("MusaBiasAddRelu", "MusaAddV2Relu", "MusaShiftedAffineMap",
            "MusaResourceApplyAdamMixed", "MusaGroupedResourceApplyAdam",
            # the reference's names for two of them
            "MusaShiftedAffineMapFusion", "MusaAdamMixedFusion")


def optimize_graph_def(graph_def: bytes, fetch=(), device_filter=None, disabled_patterns=()):
    """Rewrites a serialized tensorflow.GraphDef.

    fetch: node names (or "name:port") that must survive the rewrite.
    device_filter: only nodes whose device contains this substring are
      rewritten (the reference uses "MUSA"); None rewrites every node.
    disabled_patterns: pattern names from PATTERNS to skip.
    Returns (serialized GraphDef, stats dict with the number of fused nodes per
    pattern, grouped Adam nodes created, Adam nodes grouped and Casts folded
    into MusaResourceApplyAdamMixed).
    """
    lib = _lib.load()
    data = bytes(graph_def)
    fetch = [f.encode() for f in fetch]
    fetch_arr = (ctypes.c_char_p * max(len(fetch), 1))(*fetch)
    unknown = [p for p in disabled_patterns if p not in PATTERNS]
    if unknown:
        raise ValueError(f"unknown fusion pattern(s) {unknown}; known: {PATTERNS}")
    out = ctypes.c_void_p()
    out_n = ctypes.c_size_t()
    stats = _lib.TFMA_GraphRewriteStats()
    st = _lib.TFMA_Status()
    buf = ctypes.create_string_buffer(data, len(data))
    lib.TFMA_OptimizeGraph(ctypes.cast(buf, ctypes.c_void_p), len(data), fetch_arr, len(fetch),
                           device_filter.encode() if device_filter else None,
                           ",".join(disabled_patterns).encode(), ctypes.byref(out),
                           ctypes.byref(out_n), ctypes.byref(stats), ctypes.byref(st))
    raise_for_status(st)
    try:
        result = ctypes.string_at(out.value, out_n.value) if out_n.value else b""
    finally:
        lib.TFMA_FreeBuffer(out)
    return result, {k: getattr(stats, k) for k, _ in stats._fields_}
