"""ctypes front end of the C oracle (tfcpu_oracle.c).

TEST INFRASTRUCTURE ONLY: the TF-CPU restatement that the parity tests,
__graft_entry__.smoke() and bench.py's cpu_baseline leg use as the checker.
The product (tensorflow_musa_extension_amd) never imports this module.

Arrays are numpy; bfloat16 data is carried as uint16 bit patterns with
dtype="bfloat16" passed explicitly.

adam_int (integer ResourceApplyAdam, numpy) restates the reference's generic
op chain; its integer square root and division are closed muDNN operations
in the reference, so for those two steps parity with the reference is
unpinned (the oracle fixes one definition, pinned against an independent
big-integer restatement and a closed form in tests/test_oracle.py).
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
DT = {"float32": 1, "float64": 2, "bfloat16": 14, "float16": 19, "int32": 3, "uint8": 4,
      "int64": 9}
EW_OPS = {"add": 0, "add_relu": 1, "mul": 2, "mul_add": 3, "relu": 4, "relu_grad": 5}

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    vp, i64, f, i, d = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int, ctypes.c_double
    lib.oracle_bn_fwd.argtypes = [i, i, vp, i64, i64, i64, vp, vp, vp, vp, f, f, i, vp, vp, vp,
                                  vp, vp]
    lib.oracle_bn_grad.argtypes = [i, i, vp, vp, i64, i64, i64, vp, vp, vp, f, i, vp, vp, vp]
    lib.oracle_adam.argtypes = [i, vp, vp, vp, vp, i64, d, d, d, d, d, d, i]
    lib.oracle_eltwise.argtypes = [i, i, i, vp, vp, vp, i, vp, vp]
    lib.oracle_bias_add_grad.argtypes = [i, vp, i64, i64, i64, vp]
    lib.oracle_baseline_rows.argtypes = [i, i, vp, vp, i, vp, i, i64, i64, vp]
    lib.oracle_baseline_adam_f32.argtypes = [vp, vp, vp, vp, i64, d, d, d, d, d, d]
    lib.oracle_baseline_bn_fwd.argtypes = [i, vp, i64, i64, vp, vp, f, vp, vp, vp]
    lib.oracle_baseline_bn_grad.argtypes = [i, vp, vp, i64, i64, vp, vp, vp, f, vp, vp, vp]
    lib.oracle_set_threads.argtypes = [i]
    lib.oracle_get_threads.restype = i
    lib.oracle_f32_to_f16.argtypes = [f]
    lib.oracle_f32_to_f16.restype = ctypes.c_uint16
    lib.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.oracle_f16_to_f32.restype = f
    lib.oracle_f32_to_bf16.argtypes = [f]
    lib.oracle_f32_to_bf16.restype = ctypes.c_uint16
    lib.oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
    lib.oracle_bf16_to_f32.restype = f
    for fn in ("oracle_bn_fwd", "oracle_bn_grad", "oracle_adam", "oracle_eltwise",
               "oracle_bias_add_grad", "oracle_baseline_rows", "oracle_baseline_bn_fwd",
               "oracle_baseline_bn_grad", "oracle_baseline_adam_f32",
               "oracle_set_threads"):
        getattr(lib, fn).restype = None
    _lib = lib
    return lib


def set_threads(n):
    load().oracle_set_threads(int(n))


def get_threads():
    return load().oracle_get_threads()


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _c(a, dtype=None):
    return np.ascontiguousarray(a if dtype is None else a.astype(dtype))


# ---------------------------------------------------------------------------
# dtype helpers (bfloat16 as uint16 bits)
# ---------------------------------------------------------------------------
def storage_dtype(dtype):
    return {"float32": np.float32, "float16": np.float16, "bfloat16": np.uint16,
            "float64": np.float64}[dtype]


def f32_to_bf16_bits(a):
    """Round float32 values to bfloat16 (nearest even), returned as uint16."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    qnan = np.where((u & 0x80000000) != 0, 0xFFC0, 0x7FC0).astype(np.uint16)
    return np.where(nan, qnan, r).astype(np.uint16)


def bf16_bits_to_f32(b):
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_storage(a_f64, dtype):
    """Rounds float64 data to the storage dtype (bfloat16 -> uint16 bits)."""
    if dtype == "bfloat16":
        return f32_to_bf16_bits(np.asarray(a_f64, dtype=np.float32))
    return np.asarray(a_f64).astype(storage_dtype(dtype))


def to_f32(a, dtype):
    if dtype == "bfloat16":
        return bf16_bits_to_f32(a)
    return np.asarray(a).astype(np.float32)


# ---------------------------------------------------------------------------
# Ops
# ---------------------------------------------------------------------------
def _bn_dims(x, data_format):
    if x.ndim < 4:
        raise ValueError("x must be rank 4 or 5")
    if data_format in ("NHWC", "NDHWC"):
        return x.shape[0], x.shape[-1], int(np.prod(x.shape[1:-1])), 1
    return x.shape[0], x.shape[1], int(np.prod(x.shape[2:])), 0


def bn_fwd(x, scale, offset, mean=None, variance=None, epsilon=1e-4,
           exponential_avg_factor=1.0, data_format="NHWC", is_training=True,
           dtype="float32"):
    """TF-CPU FusedBatchNormV3; returns (y, batch_mean, batch_var, saved_mean,
    saved_var) with y in the storage dtype."""
    lib = load()
    x = _c(x)
    n, c, s, nhwc = _bn_dims(x, data_format)
    scale = _c(scale, np.float32)
    offset = _c(offset, np.float32)
    mean = _c(mean, np.float32) if mean is not None else np.zeros(c, np.float32)
    variance = _c(variance, np.float32) if variance is not None else np.ones(c, np.float32)
    y = np.empty_like(x)
    outs = [np.empty(c, np.float32) for _ in range(4)]
    lib.oracle_bn_fwd(DT[dtype], nhwc, _p(x), n, c, s, _p(scale), _p(offset), _p(mean),
                      _p(variance), float(epsilon), float(exponential_avg_factor),
                      int(bool(is_training)), _p(y), *[_p(o) for o in outs])
    return (y, *outs)


def bn_grad(dy, x, scale, mean, variance, epsilon=1e-4, data_format="NHWC",
            is_training=True, dtype="float32"):
    """TF-CPU FusedBatchNormGradV3 (mean/variance = reserve_space_1/2);
    returns (dx, scale_backprop, offset_backprop)."""
    lib = load()
    x = _c(x)
    dy = _c(dy)
    n, c, s, nhwc = _bn_dims(x, data_format)
    scale = _c(scale, np.float32)
    mean = _c(mean, np.float32)
    variance = _c(variance, np.float32)
    dx = np.empty_like(x)
    sb = np.empty(c, np.float32)
    ob = np.empty(c, np.float32)
    lib.oracle_bn_grad(DT[dtype], nhwc, _p(dy), _p(x), n, c, s, _p(scale), _p(mean),
                       _p(variance), float(epsilon), int(bool(is_training)), _p(dx), _p(sb),
                       _p(ob))
    return dx, sb, ob


def adam(var, m, v, grad, beta1_power, beta2_power, lr, beta1, beta2, epsilon,
         use_nesterov=False, dtype="float32"):
    """TF-CPU ResourceApplyAdam, in place on the (contiguous) var/m/v arrays.
    Scalars must already be representable in T."""
    lib = load()
    for a in (var, m, v, grad):
        if not a.flags["C_CONTIGUOUS"]:
            raise ValueError("arrays must be contiguous")
    lib.oracle_adam(DT[dtype], _p(var), _p(m), _p(v), _p(grad), var.size, float(beta1_power),
                    float(beta2_power), float(lr), float(beta1), float(beta2), float(epsilon),
                    int(bool(use_nesterov)))


def baseline_adam_f32(var, m, v, grad, beta1_power, beta2_power, lr, beta1, beta2, epsilon):
    """CPU baseline of float32 ResourceApplyAdam (bench.py's cpu_baseline
    leg, not the checker): in place, the checker's bits, 8-wide."""
    for a in (var, m, v, grad):
        if not a.flags["C_CONTIGUOUS"] or a.dtype != np.float32:
            raise ValueError("arrays must be contiguous float32")
    load().oracle_baseline_adam_f32(_p(var), _p(m), _p(v), _p(grad), var.size,
                                    float(beta1_power), float(beta2_power), float(lr),
                                    float(beta1), float(beta2), float(epsilon))


def adam_mixed(var, m, v, grad, beta1_power, beta2_power, lr, beta1, beta2, epsilon,
               use_nesterov=False, grad_dtype="float16"):
    """MusaResourceApplyAdamMixed as the TF-CPU pair it replaces
    (reference: musa_ext/graph/fusion/adam_mixed_fusion.cc:93-216 folds
    Cast(grad, float) -> ResourceApplyAdam<float>): widen the half/bfloat16
    grad to float32 (exact) and run the float32 ResourceApplyAdam on the
    float32 var/m/v."""
    g32 = np.ascontiguousarray(to_f32(grad, grad_dtype), dtype=np.float32)
    adam(var, m, v, g32, beta1_power, beta2_power, lr, beta1, beta2, epsilon,
         use_nesterov=use_nesterov, dtype="float32")


def _int_alpha(beta1_power, beta2_power, lr, dtype):
    """The reference's alpha for integer T: computed in double from the T
    scalars, lr when beta1_power is within 1e-10 of 1
    (musa_ext/kernels/training/musa_applyadam_op.cc:231-246), then
    static_cast<T> as its x86-64 host converts: truncation toward zero, T's
    minimum for NaN or out-of-range values."""
    import math
    b1p, b2p, lrd = float(int(beta1_power)), float(int(beta2_power)), float(int(lr))
    omb1p = 1.0 - b1p
    if abs(omb1p) < 1e-10:
        a = lrd
    else:
        r = 1.0 - b2p
        a = lrd * math.sqrt(r) / omb1p if r >= 0 else float("nan")
    info = np.iinfo(dtype)
    if not (a == a) or not (-2.0 ** (info.bits - 1) <= math.trunc(a) < 2.0 ** (info.bits - 1)):
        return int(info.min)
    return int(math.trunc(a))


def adam_int(var, m, v, grad, beta1_power, beta2_power, lr, beta1, beta2, epsilon):
    """ResourceApplyAdam for int32 / int64 var, m, v, grad (in place): the
    reference's generic op chain (musa_ext/kernels/training/
    musa_applyadam_op.cc:300-408), each step in T with two's-complement
    wrap: m = m*beta1 + grad*(1-beta1); v = v*beta2 + (grad*grad)*(1-beta2);
    var -= (m / (sqrt(v) + epsilon)) * alpha.  The square root and the
    division are closed muDNN integer ops in the reference; here sqrt is the
    exact integer square root (0 for v <= 0) and the division truncates
    toward zero, 0 for a zero divisor, MIN / -1 = MIN (the definition the
    library implements; parity with muDNN unpinned)."""
    dt = var.dtype
    if dt not in (np.int32, np.int64):
        raise ValueError("int32 or int64 arrays")
    t = lambda x: np.array(int(x), dtype=np.int64).astype(dt)  # wraps like static_cast<T>
    b1, b2, eps = t(beta1), t(beta2), t(epsilon)
    one = np.array(1, dtype=dt)
    with np.errstate(over="ignore"):
        omb1, omb2 = one - b1, one - b2
        alpha = np.array(_int_alpha(beta1_power, beta2_power, lr, dt), dtype=dt)
        g = grad.astype(dt, copy=False)
        mn = m * b1 + g * omb1
        vn = v * b2 + (g * g) * omb2
        # exact integer square root
        pos = vn > 0
        u = np.where(pos, vn, 0).astype(np.uint64)
        r = np.floor(np.sqrt(u.astype(np.float64))).astype(np.uint64)
        for _ in range(4):
            r = np.where(r * r > u, r - np.uint64(1), r)
            r = np.where((r + np.uint64(1)) * (r + np.uint64(1)) <= u, r + np.uint64(1), r)
        root = r.astype(dt)
        d = root + eps
        # truncating division; 0 for d == 0, -a for d == -1 (MIN / -1 wraps)
        safe = np.where((d == 0) | (d == -1), one, d)
        rem = np.fmod(mn, safe)
        q = (mn - rem) // safe
        q = np.where(d == 0, np.zeros_like(q), np.where(d == -1, np.zeros_like(mn) - mn, q))
        var -= q * alpha
    m[...] = mn
    v[...] = vn


def bias_add_grad(x, data_format="NHWC", dtype="float32"):
    """TF-CPU BiasAddGrad: sum over every dimension but the channel one (last
    for NHWC, 1 for NCHW); floating types in double, rounded once to T;
    int32/int64 wrap.  A rank-1 input is returned as is (the reference's
    identity case, musa_biasadd_grad_op.cc:52-58)."""
    x = np.ascontiguousarray(x)
    if x.ndim == 1:
        return x.copy()
    cd = 1 if data_format.startswith("NC") else x.ndim - 1
    c = x.shape[cd]
    outer = int(np.prod(x.shape[:cd]))
    inner = int(np.prod(x.shape[cd + 1:]))
    out = np.zeros(c, dtype=x.dtype)
    codes = dict(DT, int32=3, int64=9)
    load().oracle_bias_add_grad(codes[dtype], _p(x), outer, c, inner, _p(out))
    return out


def eltwise(op, inputs, dtype="float32"):
    """TF-CPU elementwise op with broadcasting: add, add_relu, mul, mul_add
    (inputs[0]*inputs[1] rounded, + inputs[2]), relu, or relu_grad
    (inputs[0] = gradients, inputs[1] = features).  int32 / int64 / uint8
    take add and mul, wrapping modulo 2^bits."""
    if dtype in ("int32", "int64", "uint8") and op not in ("add", "mul"):
        raise ValueError(f"{op} is not defined for {dtype}")
    lib = load()
    ins = [_c(a) for a in inputs]
    out_shape = np.broadcast_shapes(*[a.shape for a in ins])
    out = np.empty(out_shape, dtype=ins[0].dtype)
    nin = len(ins)
    ptrs = (ctypes.c_void_p * nin)(*[a.ctypes.data for a in ins])
    dims = np.zeros(8 * nin, np.int64)
    nd = np.zeros(nin, np.int32)
    for k, a in enumerate(ins):
        nd[k] = a.ndim
        dims[8 * k:8 * k + a.ndim] = a.shape
    od = np.array(out_shape, np.int64)
    lib.oracle_eltwise(DT[dtype], EW_OPS[op], nin, ptrs, _p(dims), _p(nd), len(out_shape),
                       _p(od) if len(out_shape) else None, _p(out))
    return out


def baseline_rows(op, x, b, c=None, dtype="float32"):
    """CPU baseline of the cfg4 chains (bench.py's cpu_baseline leg, not the
    checker): x [rows, cols] contiguous; b and c full [rows, cols] or a
    [cols] row; op "add", "add_relu" or "mul_add" (x*b rounded, + c)."""
    codes = {"add": 0, "add_relu": 1, "mul_add": 3}
    x = np.ascontiguousarray(x)
    rows, cols = x.shape
    b = np.ascontiguousarray(b)
    c = None if c is None else np.ascontiguousarray(c)
    out = np.empty_like(x)
    lib = load()
    lib.oracle_baseline_rows(DT[dtype], codes[op], _p(x), _p(b), int(b.ndim == 1), _p(c),
                             int(c is not None and c.ndim == 1), rows, cols, _p(out))
    return out


def baseline_bn_fwd(x, scale, offset, epsilon, dtype="float32"):
    """CPU baseline of the NHWC training forward (bench.py's cpu_baseline leg,
    not the checker): x [..., C] contiguous; returns y and the population
    mean and variance."""
    x = np.ascontiguousarray(x)
    c = x.shape[-1]
    rows = x.size // c if c else 0
    y = np.empty_like(x)
    mean, var = np.zeros(c, np.float32), np.zeros(c, np.float32)
    load().oracle_baseline_bn_fwd(DT[dtype], _p(x), rows, c, _p(_c(scale, np.float32)),
                                  _p(_c(offset, np.float32)), float(epsilon), _p(y), _p(mean),
                                  _p(var))
    return y, mean, var


def baseline_bn_grad(dy, x, scale, mean, var, epsilon, dtype="float32"):
    """CPU baseline of the NHWC training gradient (bench.py's cpu_baseline
    leg): returns x_backprop, scale_backprop, offset_backprop."""
    x = np.ascontiguousarray(x)
    dy = np.ascontiguousarray(dy)
    c = x.shape[-1]
    rows = x.size // c if c else 0
    dx = np.empty_like(x)
    sbp, obp = np.zeros(c, np.float32), np.zeros(c, np.float32)
    load().oracle_baseline_bn_grad(DT[dtype], _p(dy), _p(x), rows, c, _p(_c(scale, np.float32)),
                                   _p(_c(mean, np.float32)), _p(_c(var, np.float32)),
                                   float(epsilon), _p(dx), _p(sbp), _p(obp))
    return dx, sbp, obp


def bias_add(value, bias, data_format="NHWC", relu=False, dtype="float32"):
    """BiasAdd (and Relu(BiasAdd)) as the TF-CPU add with the bias broadcast
    over the channel dimension (last for NHWC, 1 for NCHW)."""
    if data_format == "NCHW" and value.ndim > 2:
        b = bias.reshape((bias.shape[0],) + (1,) * (value.ndim - 2))
    else:
        b = bias
    return eltwise("add_relu" if relu else "add", [value, b], dtype)
