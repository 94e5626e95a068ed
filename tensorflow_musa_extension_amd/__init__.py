"""MI355X (gfx950) fused data-parallel kernels behind the op interface of
MooreThreads/tensorflow_musa_extension's hot path.

    import tensorflow_musa_extension_amd as tfma
    tfma.tf_plugin.load_plugin()        # TensorFlow: device "AMDGPU" + kernels
    out = tfma.raw_ops.FusedBatchNormV3(x, scale, offset, mean, var, ...)  # torch tensors

Importing the package (and its TensorFlow loader, `tf_plugin`) needs neither
torch nor TensorFlow, as the reference's loader needs only TensorFlow
(python/__init__.py:66-75).  `raw_ops` and `stream_executor`, which take
torch tensors as device buffers, import torch when first used; libtfma.so is
loaded (after torch, when torch is installed, so that both bind the same HIP
runtime) on the first call into it.
"""
import importlib

from . import _lib, errors, graph_rewrite, tf_plugin  # noqa: F401
from .errors import (FailedPreconditionError, InternalError,  # noqa: F401
                     InvalidArgumentError, OpError, UnimplementedError)

__all__ = ["raw_ops", "errors", "graph_rewrite", "stream_executor", "tf_plugin",
           "load_library", "device_count", "LIB_PATH"]

LIB_PATH = _lib.LIB_PATH
_LAZY = ("raw_ops", "stream_executor")


def __getattr__(name):
    if name in _LAZY:
        return importlib.import_module(f".{name}", __name__)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")


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
