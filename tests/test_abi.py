"""CPU tests of the C ABI: the library loads, exports every entry point that
include/tfma.h declares, and its host-side validation returns TF's codes and
the reference's messages without touching a device (the pointers below are
never dereferenced: each call fails validation first)."""
import ctypes
import os
import re
import threading

import pytest

from tensorflow_musa_extension_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAKE = 0x1000  # a non-null device address that validation never touches


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "tfma.h")).read()
    return sorted(set(re.findall(r"\b(TFMA_[A-Za-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_version_and_device_count():
    lib = _lib.load()
    assert lib.TFMA_Version().decode().startswith("tfma")
    n = ctypes.c_int(-1)
    st = _lib.TFMA_Status()
    assert lib.TFMA_GetDeviceCount(ctypes.byref(n), ctypes.byref(st)) == _lib.OK
    assert n.value >= 0  # 0 on a host without a GPU driver, as the plugin reports


def T(shape, dtype=_lib.DT_FLOAT, ptr=FAKE):
    return _lib.make_tensor(ptr, dtype, shape)


def call(name, *args):
    st = _lib.TFMA_Status()
    code = getattr(_lib.load(), name)(*args, ctypes.byref(st))
    assert code == st.code
    return code, st.message.decode()


def ref(t):
    return ctypes.byref(t) if t is not None else None


def bn_fwd(x, scale, offset, mean, var, factor=1.0, fmt=b"NHWC", training=1, c=None):
    c = c if c is not None else scale.dims[0]
    outs = [T((c,)) for _ in range(4)] + [T(())]
    y = T(tuple(x.dims[:x.ndims]), x.dtype)
    return call("TFMA_FusedBatchNormV3", None, ref(x), ref(scale), ref(offset), ref(mean),
                ref(var), 1e-3, factor, fmt, training, ref(y), *[ref(o) for o in outs],
                ctypes.c_void_p(FAKE), 1 << 30)


def test_bn_validation():
    x = T((2, 3, 3, 4))
    ok4 = T((4,))
    e = T((0,), ptr=None)
    code, msg = bn_fwd(x, T((5,)), ok4, e, e, c=4)
    assert code == _lib.INVALID_ARGUMENT and "scale must have the same number" in msg
    code, msg = bn_fwd(x, ok4, T((3,)), e, e)
    assert code == _lib.INVALID_ARGUMENT and "offset must have the same number" in msg
    code, msg = bn_fwd(x, ok4, ok4, e, e, training=0)
    assert code == _lib.INVALID_ARGUMENT and msg.startswith("When is_training=false, mean")
    code, msg = bn_fwd(x, ok4, ok4, e, e, factor=0.5)
    assert msg.startswith("When exponential_avg_factor != 1, mean")
    code, msg = bn_fwd(T((2, 3, 4)), ok4, ok4, e, e)
    assert code == _lib.INVALID_ARGUMENT and "4 or 5-dimensional" in msg
    code, msg = bn_fwd(x, ok4, ok4, e, e, fmt=b"NHCW")
    assert code == _lib.INVALID_ARGUMENT and msg == "Invalid data format"
    code, msg = bn_fwd(T((2, 3, 3, 4), _lib.DT_INT32), ok4, ok4, e, e)
    assert code == _lib.UNIMPLEMENTED
    # NCHW: channels are dim 1.
    code, msg = bn_fwd(T((2, 4, 3, 3)), T((3,)), T((3,)), e, e, fmt=b"NCHW", c=3)
    assert "scale must have the same number of elements as the channels of x, got 3 and 4" in msg


def test_bn_workspace_query():
    st = _lib.TFMA_Status()
    nbytes = ctypes.c_size_t(0)
    x = T((256, 56, 56, 256), _lib.DT_HALF)
    assert _lib.load().TFMA_FusedBatchNormWorkspaceBytes(ctypes.byref(x), b"NHWC",
                                                         ctypes.byref(nbytes),
                                                         ctypes.byref(st)) == _lib.OK
    # Partials + coefficients stay a small fraction of x (411 MB).
    assert 256 * 16 <= nbytes.value < 16 << 20


def test_bn_grad_validation():
    x = T((2, 3, 3, 4))
    c4 = T((4,))
    outs = [T((2, 3, 3, 4)), T((4,)), T((4,)), T((4,)), T((4,))]
    code, msg = call("TFMA_FusedBatchNormGradV3", None, ref(T((2, 3, 3, 5))), ref(x), ref(c4),
                     ref(c4), ref(c4), ref(T(())), 1e-3, b"NHWC", 1, *[ref(o) for o in outs],
                     ctypes.c_void_p(FAKE), 1 << 30)
    assert code == _lib.INVALID_ARGUMENT
    assert msg.startswith("x and y_backprop must have same shape, but x has shape [2,3,3,4]")
    code, msg = call("TFMA_FusedBatchNormGradV3", None, ref(x), ref(x), ref(c4), ref(T((3,))),
                     ref(c4), ref(T(())), 1e-3, b"NHWC", 1, *[ref(o) for o in outs],
                     ctypes.c_void_p(FAKE), 1 << 30)
    assert "reserve_space_1 must have the same number of elements" in msg


def scalars(dtype=_lib.DT_FLOAT, values=(0.9, 0.999, 1e-3, 0.9, 0.999, 1e-7)):
    bufs = [(ctypes.c_float * 1)(v) for v in values]
    descs = [_lib.make_tensor(ctypes.addressof(b), dtype, ()) for b in bufs]
    return bufs, descs


def adam(var, m, v, grad, descs, locking=0):
    return call("TFMA_ResourceApplyAdam", None, ref(var), ref(m), ref(v),
                *[ref(d) for d in descs], ref(grad), locking, 0)


def test_adam_validation():
    bufs, descs = scalars()
    a, b = T((4, 3)), T((4, 2))
    code, msg = adam(a, b, a, a, descs)
    assert code == _lib.INVALID_ARGUMENT
    assert msg == "var and m must have the same shape. var: [4,3] m: [4,2]"
    code, msg = adam(a, a, b, a, descs)
    assert msg == "var and v must have the same shape. var: [4,3] v: [4,2]"
    code, msg = adam(a, a, a, b, descs)
    assert msg == "var and grad must have the same shape. var: [4,3] grad: [4,2]"
    code, msg = adam(T((4, 3), ptr=None), a, a, a, descs)
    assert code == _lib.FAILED_PRECONDITION and msg == "Adam variables (var/m/v) not initialized."
    bad = list(descs)
    bad[2] = _lib.make_tensor(ctypes.addressof(bufs[2]), _lib.DT_FLOAT, (1,))
    code, msg = adam(a, a, a, a, bad)
    assert code == _lib.INVALID_ARGUMENT and msg == "lr is not a scalar: [1]"
    # int32 / int64 state (the reference registers both): the scalars must be
    # of the state's type; an empty update succeeds without a device.
    i32 = lambda shape=(4, 3): T(shape, _lib.DT_INT32)
    code, msg = adam(i32(), i32(), i32(), i32(), descs)
    assert code == _lib.INVALID_ARGUMENT and msg == "beta1_power has dtype float, expected int32"
    ibufs = [(ctypes.c_int32 * 1)(v) for v in (1, 1, 3, 0, 0, 1)]
    idescs = [_lib.make_tensor(ctypes.addressof(b), _lib.DT_INT32, ()) for b in ibufs]
    code, msg = adam(i32((0, 3)), i32((0, 3)), i32((0, 3)), i32((0, 3)), idescs)
    assert code == _lib.OK, msg
    code, msg = adam(i32(), i32(), i32(), T((4, 3), _lib.DT_INT64), idescs)
    assert code == _lib.INVALID_ARGUMENT


def test_adam_mixed_validation():
    """MusaResourceApplyAdamMixed's checks and messages
    (musa_applyadam_mixed_op.cc:160-207); nothing reaches the device."""
    _, descs = scalars()
    mixed = lambda var, m, v, g: call("TFMA_MusaResourceApplyAdamMixed", None, ref(var), ref(m),
                                      ref(v), *[ref(d) for d in descs], ref(g), 0, 0)
    f, h = T((4, 3)), T((4, 3), _lib.DT_HALF)
    code, msg = mixed(T((4, 3), ptr=None), f, f, h)
    assert code == _lib.FAILED_PRECONDITION
    assert msg == "Mixed-precision Adam variables (var/m/v) not initialized."
    code, msg = mixed(h, f, f, h)
    assert code == _lib.INVALID_ARGUMENT and msg == "MusaResourceApplyAdamMixed requires fp32 var, got half"
    code, msg = mixed(f, T((4, 3), _lib.DT_BFLOAT16), f, h)
    assert msg == "MusaResourceApplyAdamMixed requires fp32 m, got bfloat16"
    code, msg = mixed(f, f, T((4, 3), _lib.DT_DOUBLE), h)
    assert msg == "MusaResourceApplyAdamMixed requires fp32 v, got double"
    code, msg = mixed(f, f, f, T((4, 2), _lib.DT_HALF))
    assert msg == "var and grad must have the same shape. var: [4,3] grad: [4,2]"
    code, msg = mixed(f, f, f, T((4, 3), _lib.DT_INT32))
    assert code == _lib.INVALID_ARGUMENT and "grad dtype int32" in msg
    hd = scalars(dtype=_lib.DT_HALF)[1]
    code, msg = call("TFMA_MusaResourceApplyAdamMixed", None, ref(f), ref(f), ref(f),
                     *[ref(d) for d in hd], ref(h), 0, 0)
    assert code == _lib.INVALID_ARGUMENT and msg == "beta1_power has dtype half, expected float"


def test_relu_grad_and_bias_add_grad_validation():
    code, msg = call("TFMA_ReluGrad", None, ref(T((4, 3))), ref(T((3, 4))), ref(T((4, 3))))
    assert code == _lib.INVALID_ARGUMENT
    assert msg == "Inputs to ReluGrad must have the same shape. gradients: [4,3], features: [3,4]"
    n = ctypes.c_size_t(0)
    code, msg = call("TFMA_BiasAddGradWorkspaceBytes", ref(T((2, 3))), b"NCDHW", ctypes.byref(n))
    assert code == _lib.INVALID_ARGUMENT and msg == "Invalid data format"
    code, msg = call("TFMA_BiasAddGradWorkspaceBytes", ref(T(())), b"NHWC", ctypes.byref(n))
    assert msg == "Input tensor must be at least 1D: []"
    code, msg = call("TFMA_BiasAddGradWorkspaceBytes", ref(T((64, 7, 9))), b"NCHW", ctypes.byref(n))
    assert code == _lib.OK and n.value > 0
    code, msg = call("TFMA_BiasAddGrad", None, ref(T((64, 7, 9))), b"NCHW", ref(T((9,))),
                     ctypes.c_void_p(FAKE), 1 << 20)
    assert code == _lib.INVALID_ARGUMENT and "output shape [9], expected [7]" in msg
    code, msg = call("TFMA_BiasAddGrad", None, ref(T((64, 7, 9))), b"NCHW", ref(T((7,))),
                     ctypes.c_void_p(FAKE), 1)
    assert code == _lib.INVALID_ARGUMENT and "workspace of" in msg


def test_adam_locking_is_deadlock_free():
    """Concurrent use_locking calls over overlapping var/m/v sets in every
    order complete (locks are taken in address order).  Empty tensors make
    each call return after locking, before any device work."""
    bufs, descs = scalars()
    ptrs = [0x10000 * (i + 1) for i in range(3)]
    orders = [(0, 1, 2), (2, 1, 0), (1, 0, 2), (2, 0, 1)]
    errors = []

    def worker(order):
        try:
            for _ in range(2000):
                ts = [T((0,), ptr=ptrs[k]) for k in order]
                code, _ = adam(ts[0], ts[1], ts[2], T((0,)), descs, locking=1)
                assert code == _lib.OK
        except Exception as e:  # pragma: no cover
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(o,)) for o in orders]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads), "deadlock"
    assert not errors


def test_grouped_adam_validation():
    bufs, descs = scalars()
    n = 2
    arr = lambda shapes: (_lib.TFMA_Tensor * n)(*[T(s) for s in shapes])
    vs = arr([(4,), (5,)])
    ms = arr([(4,), (6,)])
    code, msg = call("TFMA_GroupedResourceApplyAdam", None, n, vs, ms, arr([(4,), (5,)]),
                     arr([(4,), (5,)]), *[ref(d) for d in descs], 0, 0,
                     ctypes.c_void_p(FAKE), 4096)
    assert code == _lib.INVALID_ARGUMENT
    assert msg == "tensor 1: var and m must have the same shape. var: [5] m: [6]"
    code, msg = call("TFMA_GroupedResourceApplyAdam", None, n, vs, arr([(4,), (5,)]),
                     arr([(4,), (5,)]), arr([(4,), (5,)]), *[ref(d) for d in descs], 0, 0,
                     None, 0)
    assert code == _lib.INVALID_ARGUMENT and "workspace" in msg


def test_elementwise_validation():
    x = T((4, 5))
    code, msg = call("TFMA_BiasAdd", None, ref(x), ref(T((4,))), b"NHWC", ref(T((4, 5))))
    assert code == _lib.INVALID_ARGUMENT and msg == "Dimension mismatch in BiasAdd"
    code, msg = call("TFMA_BiasAdd", None, ref(T((5,))), ref(T((5,))), b"NHWC", ref(T((5,))))
    assert msg == "Input tensor must be at least 2D: [5]"
    code, msg = call("TFMA_BiasAdd", None, ref(x), ref(T((1, 5))), b"NHWC", ref(T((4, 5))))
    assert msg == "Biases must be 1D: [1,5]"
    code, msg = call("TFMA_AddV2", None, ref(x), ref(T((3,))), ref(T((4, 5))))
    assert code == _lib.INVALID_ARGUMENT and msg == "Incompatible shapes for Add: [4,5] and [3]"
    code, msg = call("TFMA_Mul", None, ref(x), ref(T((4, 1))), ref(T((4, 4))))
    assert "does not match broadcast shape [4,5]" in msg
    code, msg = call("TFMA_MusaShiftedAffineMap", None, ref(x), ref(T((5,))),
                     ref(T((2, 1, 5))), ref(T((4, 5))))
    assert "does not match broadcast shape [2,4,5]" in msg
    code, msg = call("TFMA_AddV2", None, ref(x), ref(T((4, 5), _lib.DT_HALF)), ref(T((4, 5))))
    assert code == _lib.INVALID_ARGUMENT and "dtype" in msg
    # Empty outputs succeed without device work.
    code, _ = call("TFMA_Relu", None, ref(T((0, 5))), ref(T((0, 5))))
    assert code == _lib.OK


def test_bias_add_empty_bias_is_a_dimension_mismatch():
    """An empty bias against a non-empty channel dimension is TF's dimension
    error, not a silent success (the channel check runs before any shortcut
    for empty tensors); an empty value with a matching bias is OK."""
    code, msg = call("TFMA_BiasAdd", None, ref(T((2, 3))), ref(T((0,))), b"NHWC",
                     ref(T((2, 3))))
    assert code == _lib.INVALID_ARGUMENT and msg == "Dimension mismatch in BiasAdd"
    code, msg = call("TFMA_MusaBiasAddRelu", None, ref(T((2, 3))), ref(T((0,))), b"NHWC",
                     ref(T((2, 3))))
    assert code == _lib.INVALID_ARGUMENT and msg == "Dimension mismatch in BiasAdd"
    code, _ = call("TFMA_BiasAdd", None, ref(T((0, 3))), ref(T((3,))), b"NHWC", ref(T((0, 3))))
    assert code == _lib.OK


def test_invalid_input_with_null_status_returns_the_code():
    """Every entry point accepts a NULL status: invalid input then returns
    the error code instead of dereferencing the status."""
    lib = _lib.load()
    bufs, descs = scalars()
    a, b = T((4, 3)), T((4, 2))
    assert lib.TFMA_ResourceApplyAdam(None, ref(a), ref(b), ref(a), *[ref(d) for d in descs],
                                      ref(a), 0, 0, None) == _lib.INVALID_ARGUMENT
    assert lib.TFMA_ResourceApplyAdam(None, ref(T((4, 3), ptr=None)), ref(a), ref(a),
                                      *[ref(d) for d in descs], ref(a), 0, 0,
                                      None) == _lib.FAILED_PRECONDITION
    bad = list(descs)
    bad[2] = _lib.make_tensor(ctypes.addressof(bufs[2]), _lib.DT_FLOAT, (1,))
    assert lib.TFMA_ResourceApplyAdam(None, ref(a), ref(a), ref(a), *[ref(d) for d in bad],
                                      ref(a), 0, 0, None) == _lib.INVALID_ARGUMENT
    n = 2
    arr = lambda shapes: (_lib.TFMA_Tensor * n)(*[T(s) for s in shapes])
    assert lib.TFMA_GroupedResourceApplyAdam(
        None, n, arr([(4,), (5,)]), arr([(4,), (6,)]), arr([(4,), (5,)]), arr([(4,), (5,)]),
        *[ref(d) for d in descs], 0, 0, ctypes.c_void_p(FAKE), 4096,
        None) == _lib.INVALID_ARGUMENT
    assert lib.TFMA_GroupedResourceApplyAdam(
        None, n, arr([(4,), (5,)]), arr([(4,), (5,)]), arr([(4,), (5,)]), arr([(4,), (5,)]),
        *[ref(d) for d in bad], 0, 0, ctypes.c_void_p(FAKE), 4096,
        None) == _lib.INVALID_ARGUMENT
    sz = ctypes.c_size_t(0)
    assert lib.TFMA_BiasAddGradWorkspaceBytes(ref(T(())), b"NHWC", ctypes.byref(sz),
                                              None) == _lib.INVALID_ARGUMENT
    assert lib.TFMA_BiasAddGrad(None, ref(T((64, 7, 9))), b"NCDHW", ref(T((7,))),
                                ctypes.c_void_p(FAKE), 1 << 20, None) == _lib.INVALID_ARGUMENT


def test_fused_batch_norm_plan_query_without_device():
    lib = _lib.load()
    st = _lib.TFMA_Status()
    plan = _lib.TFMA_FusedBatchNormPlan()
    assert lib.TFMA_FusedBatchNormLastPlan(ctypes.byref(plan), ctypes.byref(st)) == _lib.OK
    assert plan.fused == 0 and plan.workgroups == 0
    assert lib.TFMA_FusedBatchNormLastPlan(None, ctypes.byref(st)) == _lib.INVALID_ARGUMENT


def test_trace_api_without_device():
    st = _lib.TFMA_Status()
    lib = _lib.load()
    assert lib.TFMA_TraceEnable(b"tfma_bn", ctypes.byref(st)) == _lib.OK
    ms = ctypes.c_double(-1)
    n = ctypes.c_int64(-1)
    assert lib.TFMA_TraceRead(ctypes.byref(ms), ctypes.byref(n), ctypes.byref(st)) == _lib.OK
    assert ms.value == 0 and n.value == 0
    assert lib.TFMA_TraceEnable(None, ctypes.byref(st)) == _lib.OK


def test_host_path_validation_without_device():
    """The host data path's argument checks (musa_se_plugin.cc:103-111,
    365-371, 808-812): zero-size copies succeed, null pointers and streams
    are InvalidArgument - all before any device call."""
    lib = _lib.load()
    st = _lib.TFMA_Status()
    buf = ctypes.create_string_buffer(16)
    assert lib.TFMA_MemcpyHtoD(None, None, None, 0, 0, ctypes.byref(st)) == _lib.OK
    assert lib.TFMA_MemcpyDtoH(None, None, None, 0, 1, ctypes.byref(st)) == _lib.OK
    assert lib.TFMA_MemcpyHtoD(None, ctypes.cast(buf, ctypes.c_void_p), None, 16, 0,
                               ctypes.byref(st)) == _lib.INVALID_ARGUMENT
    assert b"null host pointer for src in memcpy_htod" in st.message
    assert lib.TFMA_MemcpyHtoD(None, None, ctypes.cast(buf, ctypes.c_void_p), 16, 0,
                               ctypes.byref(st)) == _lib.INVALID_ARGUMENT
    assert lib.TFMA_MemcpyDtoH(None, None, ctypes.cast(buf, ctypes.c_void_p), 16, 1,
                               ctypes.byref(st)) == _lib.INVALID_ARGUMENT
    assert b"null host pointer for dst in memcpy_dtoh" in st.message
    assert lib.TFMA_CreateStreamDependency(None, ctypes.c_void_p(1),
                                           ctypes.byref(st)) == _lib.INVALID_ARGUMENT
    assert b"null stream in create_stream_dependency" in st.message
    assert lib.TFMA_HostCallback(ctypes.c_void_p(1), None, None,
                                 ctypes.byref(st)) == _lib.INVALID_ARGUMENT


def test_elementwise_integer_dtype_validation():
    """The integer dtypes each stock op takes (uint8: Add only; the fused
    ops, Relu and ReluGrad none), checked before any device access."""
    u8, i32 = _lib.DT_UINT8, _lib.DT_INT32
    # uint8 Mul and BiasAdd, int32 Relu / fused ops: not registered
    code, msg = call("TFMA_Mul", None, ref(T((4,), u8)), ref(T((4,), u8)), ref(T((4,), u8)))
    assert code == _lib.UNIMPLEMENTED and "uint8" in msg
    code, _ = call("TFMA_BiasAdd", None, ref(T((2, 4), u8)), ref(T((4,), u8)), b"NHWC",
                   ref(T((2, 4), u8)))
    assert code == _lib.UNIMPLEMENTED
    code, _ = call("TFMA_MusaAddV2Relu", None, ref(T((4,), i32)), ref(T((4,), i32)),
                   ref(T((4,), i32)))
    assert code == _lib.UNIMPLEMENTED
    code, _ = call("TFMA_Relu", None, ref(T((4,), i32)), ref(T((4,), i32)))
    assert code == _lib.UNIMPLEMENTED
    # mixed integer dtypes and bad shapes are still INVALID_ARGUMENT
    code, msg = call("TFMA_AddV2", None, ref(T((4,), i32)), ref(T((4,), _lib.DT_INT64)),
                     ref(T((4,), i32)))
    assert code == _lib.INVALID_ARGUMENT and "int64" in msg
    code, msg = call("TFMA_AddV2", None, ref(T((4, 5), u8)), ref(T((3,), u8)),
                     ref(T((4, 5), u8)))
    assert msg == "Incompatible shapes for Add: [4,5] and [3]"
    # empty integer outputs succeed without a launch
    for dt in (u8, i32, _lib.DT_INT64):
        code, _ = call("TFMA_AddV2", None, ref(T((0, 4), dt, None)), ref(T((4,), dt)),
                       ref(T((0, 4), dt, None)))
        assert code == _lib.OK


def test_tuning_overrides():
    """TFMA_SetTuningOverride takes the documented names (-1 restores the
    default) and rejects others; host only."""
    for name in (b"ew_nt", b"bn_slice_tw", b"bn_sliced_overlap", b"bn_nchw_owned",
                 b"bag_fused"):
        assert call("TFMA_SetTuningOverride", name, 0)[0] == _lib.OK
        assert call("TFMA_SetTuningOverride", name, -1)[0] == _lib.OK
    code, msg = call("TFMA_SetTuningOverride", b"bn_slices", 4)
    assert code == _lib.INVALID_ARGUMENT and "bn_slices" in msg
    assert call("TFMA_SetTuningOverride", None, 4)[0] == _lib.INVALID_ARGUMENT


def test_package_and_tf_loader_import_without_torch():
    """Importing the package and its TensorFlow loader needs neither torch
    nor TensorFlow (the reference's loader needs only TensorFlow,
    python/__init__.py:66-75); raw_ops, which takes torch tensors, does."""
    import subprocess
    import sys
    code = ("import sys; sys.modules['torch'] = None\n"
            "import tensorflow_musa_extension_amd as tfma\n"
            "from tensorflow_musa_extension_amd import tf_plugin\n"
            "assert tf_plugin.find_plugin_library().endswith('libtfma_tf.so')\n"
            "assert 'torch' not in [m for m in sys.modules if sys.modules[m] is not None]\n"
            "try:\n"
            "    tfma.raw_ops\n"
            "except ImportError:\n"
            "    print('raw_ops needs torch')\n")
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "raw_ops needs torch"
