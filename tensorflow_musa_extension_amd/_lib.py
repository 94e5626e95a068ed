"""ctypes binding of libtfma.so (the C ABI declared in include/tfma.h).

The library is looked up next to this file.  There is no fallback: if it is
missing or fails to load, every op raises, so a missing build can never be
mistaken for a working GPU path.
"""
import ctypes
import os

MAX_DIMS = 8

# TF_Code values.
OK = 0
CANCELLED = 1
UNKNOWN = 2
INVALID_ARGUMENT = 3
NOT_FOUND = 5
RESOURCE_EXHAUSTED = 8
FAILED_PRECONDITION = 9
OUT_OF_RANGE = 11
UNIMPLEMENTED = 12
INTERNAL = 13
UNAVAILABLE = 14

# TF_DataType values.
DT_FLOAT = 1
DT_DOUBLE = 2
DT_INT32 = 3
DT_UINT8 = 4
DT_INT64 = 9
DT_BFLOAT16 = 14
DT_HALF = 19


class TFMA_Tensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndims", ctypes.c_int32),
        ("dims", ctypes.c_int64 * MAX_DIMS),
    ]


class TFMA_Status(ctypes.Structure):
    _fields_ = [("code", ctypes.c_int32), ("message", ctypes.c_char * 500)]


class TFMA_GraphRewriteStats(ctypes.Structure):
    _fields_ = [("bias_add_relu", ctypes.c_int32), ("add_v2_relu", ctypes.c_int32),
                ("mul_add", ctypes.c_int32), ("adam_groups", ctypes.c_int32),
                ("adam_grouped_nodes", ctypes.c_int32), ("adam_mixed", ctypes.c_int32)]


class TFMA_FusedBatchNormPlan(ctypes.Structure):
    _fields_ = [("fused", ctypes.c_int32), ("workgroups", ctypes.c_int32),
                ("row_groups", ctypes.c_int64), ("channel_tiles", ctypes.c_int32),
                ("dynamic_rows", ctypes.c_int32), ("dynamic_chunk", ctypes.c_int32),
                ("register_rows", ctypes.c_int32), ("lds_rows", ctypes.c_int32),
                ("slices", ctypes.c_int32)]


LIB_NAME = "libtfma.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

# Every exported entry point with its argument types (all return int codes
# unless listed in _RESTYPES).
_T = ctypes.POINTER(TFMA_Tensor)
_S = ctypes.POINTER(TFMA_Status)
_vp = ctypes.c_void_p
_f = ctypes.c_float
_i = ctypes.c_int
_cs = ctypes.c_char_p
_sz = ctypes.c_size_t

SIGNATURES = {
    "TFMA_Version": [],
    "TFMA_GetDeviceCount": [ctypes.POINTER(ctypes.c_int), _S],
    "TFMA_FusedBatchNormWorkspaceBytes": [_T, _cs, ctypes.POINTER(_sz), _S],
    "TFMA_FusedBatchNormV3": [_vp, _T, _T, _T, _T, _T, _f, _f, _cs, _i, _T, _T, _T, _T, _T,
                              _T, _vp, _sz, _S],
    "TFMA_FusedBatchNormGradV3": [_vp, _T, _T, _T, _T, _T, _T, _f, _cs, _i, _T, _T, _T, _T,
                                  _T, _vp, _sz, _S],
    "TFMA_ResourceApplyAdam": [_vp, _T, _T, _T, _T, _T, _T, _T, _T, _T, _T, _i, _i, _S],
    "TFMA_MusaResourceApplyAdamMixed": [_vp, _T, _T, _T, _T, _T, _T, _T, _T, _T, _T, _i, _i,
                                        _S],
    "TFMA_GroupedApplyAdamWorkspaceBytes": [_i, _T, ctypes.POINTER(_sz), _S],
    "TFMA_GroupedResourceApplyAdam": [_vp, _i, _T, _T, _T, _T, _T, _T, _T, _T, _T, _T, _i, _i,
                                      _vp, _sz, _S],
    "TFMA_BiasAdd": [_vp, _T, _T, _cs, _T, _S],
    "TFMA_Relu": [_vp, _T, _T, _S],
    "TFMA_AddV2": [_vp, _T, _T, _T, _S],
    "TFMA_Mul": [_vp, _T, _T, _T, _S],
    "TFMA_ReluGrad": [_vp, _T, _T, _T, _S],
    "TFMA_BiasAddGradWorkspaceBytes": [_T, _cs, ctypes.POINTER(_sz), _S],
    "TFMA_BiasAddGrad": [_vp, _T, _cs, _T, _vp, _sz, _S],
    "TFMA_BiasAddGradNoAlloc": [_vp, _T, _cs, _T, _S],
    "TFMA_MusaBiasAddRelu": [_vp, _T, _T, _cs, _T, _S],
    "TFMA_MusaAddV2Relu": [_vp, _T, _T, _T, _S],
    "TFMA_MusaShiftedAffineMap": [_vp, _T, _T, _T, _T, _S],
    "TFMA_OptimizeGraph": [_vp, _sz, ctypes.POINTER(_cs), _i, _cs, _cs, ctypes.POINTER(_vp),
                           ctypes.POINTER(_sz), ctypes.POINTER(TFMA_GraphRewriteStats), _S],
    "TFMA_FreeBuffer": [_vp],
    "TFMA_TraceEnable": [_cs, _S],
    "TFMA_TraceRead": [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64), _S],
    "TFMA_StreamCopy": [_vp, _vp, _vp, ctypes.c_uint64, _S],
    "TFMA_LastKernelName": [],
    "TFMA_FusedBatchNormBarrierTimedOut": [ctypes.POINTER(ctypes.c_int32), ctypes.c_int32, _S],
    "TFMA_FusedBatchNormLastPlan": [ctypes.POINTER(TFMA_FusedBatchNormPlan), _S],
    "TFMA_MemcpyHtoD": [_vp, _vp, _vp, ctypes.c_uint64, ctypes.c_int32, _S],
    "TFMA_MemcpyDtoH": [_vp, _vp, _vp, ctypes.c_uint64, ctypes.c_int32, _S],
    "TFMA_CreateStreamDependency": [_vp, _vp, _S],
    "TFMA_HostCallback": [_vp, _vp, _vp, _S],
    "TFMA_StagingPoolStats": [ctypes.POINTER(ctypes.c_uint64)] * 4 + [_S],
    "TFMA_SetTuningOverride": [_cs, ctypes.c_int32, _S],
    "TFMA_FusedBatchNormStamps": [ctypes.POINTER(ctypes.c_uint64), ctypes.c_uint64, _S],
}
_RESTYPES = {"TFMA_Version": ctypes.c_char_p, "TFMA_LastKernelName": ctypes.c_char_p,
             "TFMA_FreeBuffer": None}

_lib = None
_load_error = None


def load():
    """Returns the loaded library, raising ImportError if it is unavailable."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if _load_error is not None:
        raise ImportError(_load_error)
    if not os.path.exists(LIB_PATH):
        _load_error = (f"{LIB_PATH} is not built; run "
                       "`python -c 'import __graft_entry__ as g; g.build()'`")
        raise ImportError(_load_error)
    # torch bundles its own HIP runtime with the same soname
    # (libamdhip64.so.7): when torch is installed it is loaded first, so that
    # libtfma.so binds that one rather than a second copy.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    try:
        lib = ctypes.CDLL(LIB_PATH)
    except OSError as e:  # pragma: no cover - depends on the machine
        _load_error = f"failed to load {LIB_PATH}: {e}"
        raise ImportError(_load_error) from e
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
    _lib = lib
    return lib


def make_tensor(ptr, dtype, shape):
    """Builds a TFMA_Tensor from a raw pointer, TF dtype code and shape."""
    t = TFMA_Tensor()
    t.data = ptr
    t.dtype = dtype
    shape = tuple(int(s) for s in shape)
    if len(shape) > MAX_DIMS:
        raise ValueError(f"rank {len(shape)} exceeds {MAX_DIMS}")
    t.ndims = len(shape)
    for i, s in enumerate(shape):
        t.dims[i] = s
    return t
