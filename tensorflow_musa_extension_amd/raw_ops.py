"""Host-side mirror of the reference's op interface for the hot path.

Each function has the op name, argument names, defaults and output order of
the TensorFlow op the reference registers (tf.raw_ops.<Name>), takes device
tensors (torch CUDA/HIP tensors stand in for TF's device buffers: memory and
streams only) and calls libtfma.so through its C ABI on the current stream.
Errors come back as the tf.errors-style exceptions of `errors.py`.

Reference ops mirrored:
  FusedBatchNormV3 / FusedBatchNormGradV3
      musa_ext/kernels/nn/musa_fused_batchnorm_op.cc:42-182, 206-295, 303-325
  ResourceApplyAdam    musa_ext/kernels/training/musa_applyadam_op.cc:130-416
  MusaGroupedResourceApplyAdam  (grouped optimizer pattern of
      musa_ext/kernels/training/musa_applygradientdescent_op.cc:305-448)
  BiasAdd              musa_ext/kernels/nn/musa_biasadd_op.cc:10-82
  Relu                 musa_ext/kernels/nn/musa_relu_op.cc:10-60
  AddV2, Add           musa_ext/kernels/math/musa_add_op.cc:379-470
  BiasAddV1            musa_ext/kernels/nn/musa_biasadd_op.cc:71-73
  Mul                  musa_ext/kernels/math/musa_multiply_op.cc:248-324
  MusaShiftedAffineMap musa_ext/kernels/fusion/musa_shifted_affine_map_op.cc:108-262
  MusaBiasAddRelu, MusaAddV2Relu: fused chains with no reference op.
"""
import collections
import ctypes

import numpy as np
import torch

from . import _lib
from .errors import raise_for_status

_TORCH_TO_TF = {
    torch.float32: _lib.DT_FLOAT,
    torch.float16: _lib.DT_HALF,
    torch.bfloat16: _lib.DT_BFLOAT16,
    torch.float64: _lib.DT_DOUBLE,
    torch.int32: _lib.DT_INT32,
    torch.int64: _lib.DT_INT64,
    torch.uint8: _lib.DT_UINT8,
}

FusedBatchNormV3Result = collections.namedtuple(
    "FusedBatchNormV3",
    ["y", "batch_mean", "batch_variance", "reserve_space_1", "reserve_space_2",
     "reserve_space_3"])
FusedBatchNormGradV3Result = collections.namedtuple(
    "FusedBatchNormGradV3",
    ["x_backprop", "scale_backprop", "offset_backprop", "reserve_space_4",
     "reserve_space_5"])


def _check_device(t, name):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a device tensor, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.dtype not in _TORCH_TO_TF:
        raise TypeError(f"{name}: unsupported dtype {t.dtype}")


def _desc(t, name="tensor"):
    _check_device(t, name)
    ptr = t.data_ptr() if t.numel() > 0 else None
    return _lib.make_tensor(ptr, _TORCH_TO_TF[t.dtype], t.shape)


def _ref(x):
    return ctypes.byref(x)


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


_BIND = False  # set while building a Bound call instead of running it


class Bound:
    """A prepared op call: descriptors and host scalars are built once, so
    each call costs one ctypes dispatch (the analogue of a kernel that TF
    has already constructed).  The tensors it was built from must stay
    alive and keep their shapes."""

    def __init__(self, fn, args, keepalive, result):
        self._fn = fn
        self._args = args
        self._status = _lib.TFMA_Status()
        self._keep = keepalive
        self.result = result

    def __call__(self):
        self._fn(*self._args, ctypes.byref(self._status))
        if self._status.code:
            raise_for_status(self._status)
        return self.result


_bound = None


def _call(fn_name, *args, keep=()):
    """Runs lib.fn_name(*args, &status); `keep` lists objects the raw
    pointers in args refer to (workspaces, host scalars), which a Bound call
    must keep alive."""
    global _bound
    lib = _lib.load()
    if _BIND:
        _bound = (getattr(lib, fn_name), args, keep)
        return
    status = _lib.TFMA_Status()
    getattr(lib, fn_name)(*args, ctypes.byref(status))
    raise_for_status(status)


def bind(op, *args, **kwargs):
    """Prepares op(*args, **kwargs) and returns a Bound callable that runs
    it (e.g. bind(FusedBatchNormV3, x, scale, ...)).  Every op writes into
    the same output tensors on each call."""
    global _BIND, _bound
    _BIND = True
    _bound = None
    try:
        result = op(*args, **kwargs)
        fn, cargs, keep = _bound
    finally:
        _BIND = False
    return Bound(fn, cargs, (args, kwargs, keep), result)


def _fmt(data_format):
    if isinstance(data_format, str):
        data_format = data_format.encode()
    return data_format


# ---------------------------------------------------------------------------
# FusedBatchNormV3 / FusedBatchNormGradV3
# ---------------------------------------------------------------------------
def fused_batch_norm_workspace_bytes(x, data_format="NHWC"):
    lib = _lib.load()
    status = _lib.TFMA_Status()
    nbytes = ctypes.c_size_t(0)
    d = _lib.make_tensor(None, _TORCH_TO_TF[x.dtype], x.shape)
    lib.TFMA_FusedBatchNormWorkspaceBytes(_ref(d), _fmt(data_format), ctypes.byref(nbytes),
                                          ctypes.byref(status))
    raise_for_status(status)
    return nbytes.value


def _workspace(x, data_format, workspace):
    need = fused_batch_norm_workspace_bytes(x, data_format)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    return workspace, workspace.numel()


def FusedBatchNormV3(x, scale, offset, mean, variance, epsilon=0.0001,
                     exponential_avg_factor=1.0, data_format="NHWC", is_training=True,
                     workspace=None, out=None):
    """tf.raw_ops.FusedBatchNormV3.  `out` may hold preallocated outputs
    (a FusedBatchNormV3Result) to reuse; `workspace` a uint8 scratch tensor."""
    c = scale.shape[0] if scale.dim() == 1 else 0
    if out is None:
        f32 = dict(dtype=torch.float32, device=x.device)
        out = FusedBatchNormV3Result(
            torch.empty_like(x), torch.empty(c, **f32), torch.empty(c, **f32),
            torch.empty(c, **f32), torch.empty(c, **f32), torch.empty((), **f32))
    ws, ws_bytes = _workspace(x, data_format, workspace)
    dx, ds, do = _desc(x, "x"), _desc(scale, "scale"), _desc(offset, "offset")
    dm = _desc(mean, "mean")
    dv = _desc(variance, "variance")
    outs = [_desc(t, n) for t, n in zip(out, FusedBatchNormV3Result._fields)]
    _call("TFMA_FusedBatchNormV3", _stream(x), _ref(dx), _ref(ds), _ref(do), _ref(dm),
          _ref(dv), float(epsilon), float(exponential_avg_factor), _fmt(data_format),
          int(bool(is_training)), *[_ref(o) for o in outs], ctypes.c_void_p(ws.data_ptr()),
          ws_bytes, keep=(ws,))
    return out


def FusedBatchNormGradV3(y_backprop, x, scale, reserve_space_1, reserve_space_2,
                         reserve_space_3, epsilon=0.0001, data_format="NHWC",
                         is_training=True, workspace=None, out=None):
    """tf.raw_ops.FusedBatchNormGradV3.  reserve_space_4/5 are returned as
    zero-filled [C] tensors, as the reference allocates them."""
    c = scale.shape[0] if scale.dim() == 1 else 0
    if out is None:
        f32 = dict(dtype=torch.float32, device=x.device)
        out = FusedBatchNormGradV3Result(
            torch.empty_like(x), torch.empty(c, **f32), torch.empty(c, **f32),
            torch.empty(c, **f32), torch.empty(c, **f32))
    ws, ws_bytes = _workspace(x, data_format, workspace)
    d_in = [_desc(y_backprop, "y_backprop"), _desc(x, "x"), _desc(scale, "scale"),
            _desc(reserve_space_1, "reserve_space_1"), _desc(reserve_space_2, "reserve_space_2"),
            _desc(reserve_space_3, "reserve_space_3")]
    outs = [_desc(t, n) for t, n in zip(out, FusedBatchNormGradV3Result._fields)]
    _call("TFMA_FusedBatchNormGradV3", _stream(x), *[_ref(d) for d in d_in], float(epsilon),
          _fmt(data_format), int(bool(is_training)), *[_ref(o) for o in outs],
          ctypes.c_void_p(ws.data_ptr()), ws_bytes, keep=(ws,))
    return out


# ---------------------------------------------------------------------------
# Adam
# ---------------------------------------------------------------------------
_SCALAR_NAMES = ["beta1_power", "beta2_power", "lr", "beta1", "beta2", "epsilon"]


def host_scalar(value, dtype):
    """A 0-d host tensor of `dtype` (TF HostMemory scalar) kept alive by the
    returned pair (buffer, descriptor)."""
    if isinstance(value, torch.Tensor):
        value = value.detach().cpu().reshape(()).item()
    if not dtype.is_floating_point:
        value = int(value)
    buf = torch.tensor([value], dtype=dtype)
    desc = _lib.make_tensor(buf.data_ptr(), _TORCH_TO_TF[dtype], ())
    return buf, desc


def ResourceApplyAdam(var, m, v, beta1_power, beta2_power, lr, beta1, beta2, epsilon, grad,
                      use_locking=False, use_nesterov=False):
    """tf.raw_ops.ResourceApplyAdam on device tensors var/m/v (in place).
    Scalars are Python numbers or tensors, passed as host scalars of var's
    dtype."""
    scal = [host_scalar(s, var.dtype) for s in
            (beta1_power, beta2_power, lr, beta1, beta2, epsilon)]
    dvar, dm, dv, dg = _desc(var, "var"), _desc(m, "m"), _desc(v, "v"), _desc(grad, "grad")
    _call("TFMA_ResourceApplyAdam", _stream(var), _ref(dvar), _ref(dm), _ref(dv),
          *[_ref(s[1]) for s in scal], _ref(dg), int(bool(use_locking)),
          int(bool(use_nesterov)), keep=(scal,))


def MusaResourceApplyAdamMixed(var, m, v, beta1_power, beta2_power, lr, beta1, beta2, epsilon,
                               grad, use_locking=False, use_nesterov=False):
    """The reference's MusaResourceApplyAdamMixed: fp32 var/m/v updated in
    place from a float, half or bfloat16 grad; float host scalars."""
    scal = [host_scalar(s, torch.float32) for s in
            (beta1_power, beta2_power, lr, beta1, beta2, epsilon)]
    dvar, dm, dv, dg = _desc(var, "var"), _desc(m, "m"), _desc(v, "v"), _desc(grad, "grad")
    _call("TFMA_MusaResourceApplyAdamMixed", _stream(var), _ref(dvar), _ref(dm), _ref(dv),
          *[_ref(s[1]) for s in scal], _ref(dg), int(bool(use_locking)),
          int(bool(use_nesterov)), keep=(scal,))


def _tensor_array(ts, name):
    arr = (_lib.TFMA_Tensor * len(ts))()
    for i, t in enumerate(ts):
        arr[i] = _desc(t, f"{name}[{i}]")
    return arr


def MusaGroupedResourceApplyAdam(vars, ms, vs, grads, beta1_power, beta2_power, lr, beta1,
                                 beta2, epsilon, use_locking=False, use_nesterov=False,
                                 workspace=None):
    """N ResourceApplyAdam updates with shared scalars in one launch
    (inputs vars/ms/vs/grads: N tensors each).  With float32 vars the grads
    may all be float16 or bfloat16 (mixed precision)."""
    n = len(vars)
    if not (len(ms) == len(vs) == len(grads) == n) or n < 1:
        raise ValueError("vars, ms, vs, grads must be non-empty lists of equal length")
    av, am, avv, ag = (_tensor_array(vars, "vars"), _tensor_array(ms, "ms"),
                       _tensor_array(vs, "vs"), _tensor_array(grads, "grads"))
    lib = _lib.load()
    status = _lib.TFMA_Status()
    need = ctypes.c_size_t(0)
    lib.TFMA_GroupedApplyAdamWorkspaceBytes(n, av, ctypes.byref(need), ctypes.byref(status))
    raise_for_status(status)
    if workspace is None:
        workspace = torch.empty(need.value, dtype=torch.uint8, device=vars[0].device)
    scal = [host_scalar(s, vars[0].dtype) for s in
            (beta1_power, beta2_power, lr, beta1, beta2, epsilon)]
    _call("TFMA_GroupedResourceApplyAdam", _stream(vars[0]), n, av, am, avv, ag,
          *[_ref(s[1]) for s in scal], int(bool(use_locking)), int(bool(use_nesterov)),
          ctypes.c_void_p(workspace.data_ptr()), workspace.numel(),
          keep=(scal, workspace, av, am, avv, ag))


# ---------------------------------------------------------------------------
# Elementwise
# ---------------------------------------------------------------------------
def broadcast_shape(*shapes):
    """TF BCast output shape (numpy rules); raises InvalidArgument-style
    ValueError through the library when incompatible."""
    try:
        return tuple(np.broadcast_shapes(*[tuple(s) for s in shapes]))
    except ValueError:
        return None


def _binary(fn_name, x, y, out):
    if out is None:
        shape = broadcast_shape(x.shape, y.shape)
        # An incompatible pair still goes to the library, which reports it.
        out = torch.empty(shape if shape is not None else x.shape, dtype=x.dtype,
                          device=x.device)
    dx, dy, dz = _desc(x, "x"), _desc(y, "y"), _desc(out, "z")
    _call(fn_name, _stream(x), _ref(dx), _ref(dy), _ref(dz))
    return out


def BiasAdd(value, bias, data_format="NHWC", out=None):
    out = torch.empty_like(value) if out is None else out
    dv, db, do = _desc(value, "value"), _desc(bias, "bias"), _desc(out, "output")
    _call("TFMA_BiasAdd", _stream(value), _ref(dv), _ref(db), _fmt(data_format), _ref(do))
    return out


def BiasAddV1(value, bias, out=None):
    """tf.raw_ops.BiasAddV1: BiasAdd over the last dimension (no data_format
    attr; the reference registers it with BiasAdd's compute,
    musa_biasadd_op.cc:71-73)."""
    return BiasAdd(value, bias, "NHWC", out)


def MusaBiasAddRelu(value, bias, data_format="NHWC", out=None):
    out = torch.empty_like(value) if out is None else out
    dv, db, do = _desc(value, "value"), _desc(bias, "bias"), _desc(out, "output")
    _call("TFMA_MusaBiasAddRelu", _stream(value), _ref(dv), _ref(db), _fmt(data_format),
          _ref(do))
    return out


def Relu(features, out=None):
    out = torch.empty_like(features) if out is None else out
    df, do = _desc(features, "features"), _desc(out, "activations")
    _call("TFMA_Relu", _stream(features), _ref(df), _ref(do))
    return out


def ReluGrad(gradients, features, out=None):
    """tf.raw_ops.ReluGrad: gradients * (features > 0)."""
    out = torch.empty_like(gradients) if out is None else out
    dg, df, do = _desc(gradients, "gradients"), _desc(features, "features"), _desc(out, "backprops")
    _call("TFMA_ReluGrad", _stream(gradients), _ref(dg), _ref(df), _ref(do))
    return out


def bias_add_grad_workspace_bytes(out_backprop, data_format="NHWC"):
    lib = _lib.load()
    status = _lib.TFMA_Status()
    nbytes = ctypes.c_size_t(0)
    d = _lib.make_tensor(None, _TORCH_TO_TF[out_backprop.dtype], out_backprop.shape)
    lib.TFMA_BiasAddGradWorkspaceBytes(_ref(d), _fmt(data_format), ctypes.byref(nbytes),
                                       ctypes.byref(status))
    raise_for_status(status)
    return nbytes.value


def BiasAddGrad(out_backprop, data_format="NHWC", out=None, workspace=None):
    """tf.raw_ops.BiasAddGrad: per-channel sum over every other dimension
    (channel = last dim for NHWC, dim 1 for NCHW)."""
    nd = out_backprop.dim()
    cd = 1 if (str(data_format).upper().startswith("NC") and nd > 1) else nd - 1
    c = out_backprop.shape[cd] if nd >= 1 else 0
    out = torch.empty(c, dtype=out_backprop.dtype, device=out_backprop.device) if out is None else out
    if workspace is None:
        need = bias_add_grad_workspace_bytes(out_backprop, data_format) if nd >= 1 else 0
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=out_backprop.device)
    dx, do = _desc(out_backprop, "out_backprop"), _desc(out, "output")
    _call("TFMA_BiasAddGrad", _stream(out_backprop), _ref(dx), _fmt(data_format), _ref(do),
          ctypes.c_void_p(workspace.data_ptr()), workspace.numel(), keep=(workspace,))
    return out


def bias_add_grad_no_alloc(out_backprop, out, data_format="NHWC"):
    """BiasAddGrad through the allocation-free entry point
    (TFMA_BiasAddGradNoAlloc): the caller passes the output; the library's
    static per-GPU scratch holds the partials, so nothing is allocated."""
    dx, do = _desc(out_backprop, "out_backprop"), _desc(out, "output")
    _call("TFMA_BiasAddGradNoAlloc", _stream(out_backprop), _ref(dx), _fmt(data_format),
          _ref(do))
    return out


def AddV2(x, y, out=None):
    return _binary("TFMA_AddV2", x, y, out)


def Add(x, y, out=None):
    """tf.raw_ops.Add: the legacy name, AddV2's compute (the reference
    registers both on MusaAddOp, musa_add_op.cc:455-460)."""
    return _binary("TFMA_AddV2", x, y, out)


def Mul(x, y, out=None):
    return _binary("TFMA_Mul", x, y, out)


def MusaAddV2Relu(x, y, out=None):
    return _binary("TFMA_MusaAddV2Relu", x, y, out)


def MusaShiftedAffineMap(data_left, mask, sliced_var_right, out=None):
    """mask * data_left + sliced_var_right with broadcasting (Mul+Add)."""
    if out is None:
        shape = broadcast_shape(data_left.shape, mask.shape, sliced_var_right.shape)
        out = torch.empty(shape if shape is not None else data_left.shape,
                          dtype=data_left.dtype, device=data_left.device)
    d = [_desc(data_left, "data_left"), _desc(mask, "mask"),
         _desc(sliced_var_right, "sliced_var_right"), _desc(out, "output")]
    _call("TFMA_MusaShiftedAffineMap", _stream(data_left), *[_ref(x) for x in d])
    return out


# ---------------------------------------------------------------------------
# Tracing
# ---------------------------------------------------------------------------
def stream_copy(dst, src):
    """dst <- src (same byte count, a multiple of 16, 16-byte aligned) through
    the library's streaming-copy kernel (TFMA_StreamCopy): the measuring stick
    for the stream-copy ceiling, not an op."""
    nbytes = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != nbytes:
        raise ValueError("stream_copy: dst and src differ in size")
    _call("TFMA_StreamCopy", _stream(src), ctypes.c_void_p(dst.data_ptr()),
          ctypes.c_void_p(src.data_ptr()), nbytes)
    return dst


def trace_enable(name_substr):
    lib = _lib.load()
    status = _lib.TFMA_Status()
    lib.TFMA_TraceEnable(name_substr.encode() if name_substr else None, ctypes.byref(status))
    raise_for_status(status)


def trace_read():
    lib = _lib.load()
    status = _lib.TFMA_Status()
    ms = ctypes.c_double(0)
    n = ctypes.c_int64(0)
    lib.TFMA_TraceRead(ctypes.byref(ms), ctypes.byref(n), ctypes.byref(status))
    raise_for_status(status)
    return ms.value, n.value


def fused_batch_norm_last_plan():
    """Launch plan of this thread's last FusedBatchNormV3 / GradV3 call, as a
    dict: fused (persistent kernel ran), workgroups, row_groups,
    channel_tiles, dynamic_rows / dynamic_chunk (phase-3 rows per thread
    handed out in chunks), register_rows, lds_rows."""
    lib = _lib.load()
    status = _lib.TFMA_Status()
    plan = _lib.TFMA_FusedBatchNormPlan()
    lib.TFMA_FusedBatchNormLastPlan(ctypes.byref(plan), ctypes.byref(status))
    raise_for_status(status)
    return {name: getattr(plan, name) for name, _ in plan._fields_}


def fused_batch_norm_barrier_timed_out(reset=False):
    """True if a fused BatchNorm launch on the current device gave up a
    grid-wide wait for other workgroups' values since the last reset (its
    outputs for the channels concerned are NaN, and the next BatchNorm call
    raised InternalError); synchronizes the device."""
    lib = _lib.load()
    status = _lib.TFMA_Status()
    flag = ctypes.c_int32(0)
    lib.TFMA_FusedBatchNormBarrierTimedOut(ctypes.byref(flag), 1 if reset else 0,
                                           ctypes.byref(status))
    raise_for_status(status)
    return bool(flag.value)


def set_tuning_override(name, value):
    """Plan / cache-mode override (TFMA_SetTuningOverride): "ew_nt",
    "bn_slice_tw", "bn_sliced_overlap", "bn_nchw_owned" or "bag_fused"; value None or -1
    restores the library's own choice.  For tests and measurements."""
    st = _lib.TFMA_Status()
    _lib.load().TFMA_SetTuningOverride(name.encode(), -1 if value is None else int(value),
                                       ctypes.byref(st))
    raise_for_status(st)


def last_kernel_name():
    return _lib.load().TFMA_LastKernelName().decode()
