"""Host data path of the stream executor: the calls a PluggableDevice's
SP_StreamExecutor copy / dependency / callback slots forward to
(reference: musa_ext/mu/musa_se_plugin.cc - memcpy_htod and
sync_memcpy_htod with the pinned bounce :127-211, :621-747; memcpy_dtoh
:599-619, :712-728; create_stream_dependency :365-432; host_callback
:808-835).  Device memory and streams are torch's here; host buffers are
numpy arrays or CPU tensors (pageable or pinned).
"""
import ctypes

import numpy as np
import torch

from . import _lib
from .errors import raise_for_status

HOST_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p)


def _host_ptr(a):
    if isinstance(a, np.ndarray):
        if not a.flags["C_CONTIGUOUS"]:
            raise ValueError("host array must be contiguous")
        return a.ctypes.data, a.nbytes
    if isinstance(a, torch.Tensor):
        if not a.is_contiguous():
            raise ValueError("host tensor must be contiguous")
        return a.data_ptr(), a.numel() * a.element_size()
    raise TypeError("host buffer must be a numpy array or a torch tensor")


def _stream(s):
    if s is None:
        s = torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def memcpy_htod(dst, src, size=None, stream=None, sync=False):
    """Copies host buffer `src` (numpy array or CPU tensor, pageable or
    pinned; or a device tensor) into device tensor `dst`.  Returns once
    `src` may be reused; with sync=True once the copy is done."""
    sp, nbytes = _host_ptr(src)
    size = nbytes if size is None else size
    if size > nbytes or size > dst.numel() * dst.element_size():
        raise ValueError("size exceeds a buffer")
    st = _lib.TFMA_Status()
    _lib.load().TFMA_MemcpyHtoD(_stream(stream), ctypes.c_void_p(dst.data_ptr()),
                                ctypes.c_void_p(sp), size, 1 if sync else 0, ctypes.byref(st))
    raise_for_status(st)


def memcpy_dtoh(dst, src, size=None, stream=None, sync=True):
    """Copies device tensor `src` into host buffer `dst`."""
    dp, nbytes = _host_ptr(dst)
    size = nbytes if size is None else size
    if size > nbytes or size > src.numel() * src.element_size():
        raise ValueError("size exceeds a buffer")
    st = _lib.TFMA_Status()
    _lib.load().TFMA_MemcpyDtoH(_stream(stream), ctypes.c_void_p(dp),
                                ctypes.c_void_p(src.data_ptr()), size, 1 if sync else 0,
                                ctypes.byref(st))
    raise_for_status(st)


def create_stream_dependency(dependent, other):
    """Work enqueued on `dependent` from now on waits for what `other` has
    enqueued so far (torch streams)."""
    st = _lib.TFMA_Status()
    _lib.load().TFMA_CreateStreamDependency(_stream(dependent), _stream(other), ctypes.byref(st))
    raise_for_status(st)


_callbacks = {}


def host_callback(stream, fn):
    """Runs fn() on a host thread after the work enqueued on `stream`."""
    key = object()

    def trampoline(_):
        try:
            fn()
        finally:
            _callbacks.pop(key, None)

    cb = HOST_FN(trampoline)
    _callbacks[key] = cb  # keep the ctypes thunk alive until it has run
    st = _lib.TFMA_Status()
    _lib.load().TFMA_HostCallback(_stream(stream), ctypes.cast(cb, ctypes.c_void_p), None,
                                  ctypes.byref(st))
    if st.code != 0:
        _callbacks.pop(key, None)
    raise_for_status(st)


def staging_pool_stats():
    """(blocks, host_allocs, reuses, pending) of the current device's pool."""
    vals = [ctypes.c_uint64(0) for _ in range(4)]
    st = _lib.TFMA_Status()
    _lib.load().TFMA_StagingPoolStats(*[ctypes.byref(v) for v in vals], ctypes.byref(st))
    raise_for_status(st)
    return tuple(v.value for v in vals)
