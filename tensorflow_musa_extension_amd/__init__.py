"""MI355X (gfx950) fused data-parallel kernels behind the op interface of
MooreThreads/tensorflow_musa_extension's hot path.

    import tensorflow_musa_extension_amd as tfma
    out = tfma.raw_ops.FusedBatchNormV3(x, scale, offset, mean, var, ...)

torch is imported first so that the HIP runtime it bundles is the one
libtfma.so binds to (both carry the soname libamdhip64.so.7).
"""
import torch  # noqa: F401  (loads the process's HIP runtime)

from . import _lib, errors, graph_rewrite, raw_ops, stream_executor, tf_plugin  # noqa: F401
from .errors import (FailedPreconditionError, InternalError,  # noqa: F401
                     InvalidArgumentError, OpError, UnimplementedError)

__all__ = ["raw_ops", "errors", "graph_rewrite", "stream_executor", "load_library", "device_count",
           "LIB_PATH"]

LIB_PATH = _lib.LIB_PATH


def load_library():
    """Loads libtfma.so (raises ImportError if it is not built)."""
    return _lib.load()


def device_count():
    """Visible devices as the plugin would report them (0 without a driver)."""
    import ctypes
    lib = _lib.load()
    n = ctypes.c_int(0)
    st = _lib.TFMA_Status()
    lib.TFMA_GetDeviceCount(ctypes.byref(n), ctypes.byref(st))
    errors.raise_for_status(st)
    return n.value
