"""Seeded random sweeps on the GPU against the oracle: FusedBatchNormV3 +
GradV3 over shapes, layouts, dtypes, modes and forced launch plans, and the
elementwise ops over random broadcast patterns.  Each case is drawn from its
own seed (printed in its id), so a failure names the exact case.

Bars: BN float32 activations 1e-5 and float16/bfloat16 activations 1e-2 of
max|ref|, as in the per-op tests; statistics 1e-5 of the larger of max|ref|
and the scale of the values they sum (per channel, the maximum over channels
of mean|x| for means, of sum|dy| for offset_backprop and of sum|dy*x_hat| for
scale_backprop), because with one or a few channels a mean or a gradient sum
can cancel to near zero and its rounding error is set by its summands, not by
its value; elementwise bitwise.
"""
import numpy as np
import pytest
import torch

import tensorflow_musa_extension_amd as tfma
from oracle import oracle
from tests.helpers import assert_bitwise, assert_close, gen, max_rel_err, to_dev, to_np
from tests.test_gpu_bn import _run_fwd_grad

pytestmark = pytest.mark.gpu
ops = tfma.raw_ops

ACT_TOL = {"float32": 1e-5, "float16": 1e-2, "bfloat16": 1e-2}
STAT_TOL = 1e-5
CHANNELS = [1, 3, 8, 16, 24, 33, 64, 100, 128, 256, 300, 512, 520, 1024]


def _channels_last(a, dtype, fmt):
    """Storage array -> float64 (rows, C)."""
    f = oracle.to_f32(a, dtype).astype(np.float64)
    if fmt == "NCHW":
        f = np.moveaxis(f, 1, -1)
    return f.reshape(-1, f.shape[-1])


def _stat_close(got, ref, floor, name):
    err = max_rel_err(got, ref, "float32", floor=floor)
    assert err <= STAT_TOL, f"{name}: max error {err:.3e} (relative to {floor:.3e}) > {STAT_TOL}"


def _bn_case(seed):
    rng = np.random.default_rng(seed)
    dtype = ["float32", "float16", "bfloat16"][rng.integers(3)]
    fmt = "NHWC" if rng.random() < 0.7 else "NCHW"
    if rng.random() < 0.25:  # enough rows per channel for register, LDS and streamed rows
        c = int(rng.choice([16, 64, 128, 256]))
        n, h, w = (int(v) for v in rng.integers([8, 20, 20], [33, 57, 57]))
    else:
        c = int(rng.choice(CHANNELS))
        n, h, w = (int(v) for v in rng.integers(1, [9, 21, 21]))
    shape = (n, h, w, c) if fmt == "NHWC" else (n, c, h, w)
    training = bool(rng.random() < 0.8)
    factor = 1.0 if rng.random() < 0.7 else 0.3
    loc = float(rng.choice([0.0, 3.0]))
    env = {}
    if fmt == "NHWC":
        tw = rng.choice(["", "8", "16", "32"], p=[0.55, 0.15, 0.15, 0.15])
        if tw:
            env["bn_slice_tw"] = int(tw)
            if rng.random() < 0.5:
                env["bn_sliced_overlap"] = 0
    return dict(dtype=dtype, fmt=fmt, shape=shape, training=training, factor=factor, loc=loc,
                env=env, rng=rng)


@pytest.mark.parametrize("seed", range(100, 160))
def test_bn_sweep(dev, tune, seed):
    k = _bn_case(seed)
    for name, value in k["env"].items():
        tune(name, value)
    rng, dtype, fmt, shape = k["rng"], k["dtype"], k["fmt"], k["shape"]
    print(f"seed {seed}: {shape} {dtype} {fmt} training={k['training']} "
          f"factor={k['factor']} loc={k['loc']} env={k['env']}", flush=True)
    c = shape[-1] if fmt == "NHWC" else shape[1]
    eps = 1e-3
    x = gen(rng, shape, dtype, loc=k["loc"])
    dy = gen(rng, shape, dtype)
    scale = rng.uniform(0.5, 1.5, c).astype(np.float32)
    offset = (0.1 * rng.standard_normal(c)).astype(np.float32)
    mean_in = (0.1 * rng.standard_normal(c)).astype(np.float32)
    var_in = rng.uniform(0.5, 2.0, c).astype(np.float32)
    training, factor = k["training"], k["factor"]
    use_running = (not training) or factor != 1.0
    mean = mean_in if use_running else None
    var = var_in if use_running else None
    # Every output starts as NaN, so each must be written.
    fwd, grad = _run_fwd_grad(dev, x, scale, offset, dy, dtype, fmt, eps, mean=mean, var=var,
                              factor=factor, is_training=training)
    ry, rbm, rbv, rsm, rsv = oracle.bn_fwd(x, scale, offset, mean, var, epsilon=eps,
                                          exponential_avg_factor=factor, data_format=fmt,
                                          is_training=training, dtype=dtype)
    assert_close(to_np(fwd.y, dtype), ry, dtype, ACT_TOL[dtype], "y")
    xf = _channels_last(x, dtype, fmt)
    mean_floor = float(np.abs(xf).mean(axis=0).max())
    for name, got, ref, floor in (("batch_mean", fwd.batch_mean, rbm, mean_floor),
                                  ("batch_variance", fwd.batch_variance, rbv, None),
                                  ("reserve_space_1", fwd.reserve_space_1, rsm, mean_floor),
                                  ("reserve_space_2", fwd.reserve_space_2, rsv, None)):
        _stat_close(got.cpu().numpy(), ref, floor or 0.0, name)
    sm, sv = fwd.reserve_space_1, fwd.reserve_space_2
    rdx, rsb, rob = oracle.bn_grad(dy, x, scale, sm.cpu().numpy(), sv.cpu().numpy(), epsilon=eps,
                                   data_format=fmt, is_training=training, dtype=dtype)
    assert_close(to_np(grad.x_backprop, dtype), rdx, dtype, ACT_TOL[dtype], "x_backprop")
    dyf = _channels_last(dy, dtype, fmt)
    xhat = (xf - sm.cpu().numpy()) / np.sqrt(sv.cpu().numpy().astype(np.float64) + eps)
    _stat_close(grad.scale_backprop.cpu().numpy(), rsb,
                float(np.abs(dyf * xhat).sum(axis=0).max()), "scale_backprop")
    _stat_close(grad.offset_backprop.cpu().numpy(), rob, float(np.abs(dyf).sum(axis=0).max()),
                "offset_backprop")


def _bcast_shape(rng, out):
    """A shape that broadcasts to `out` (TF rules): a random suffix of it,
    with random dimensions set to 1."""
    k = int(rng.integers(0, len(out) + 1))
    s = list(out[len(out) - k:])
    for i in range(len(s)):
        if rng.random() < 0.35:
            s[i] = 1
    return tuple(s)


@pytest.mark.parametrize("seed", range(200, 260))
def test_eltwise_sweep(dev, seed):
    rng = np.random.default_rng(seed)
    dtype = ["float32", "float16", "bfloat16"][rng.integers(3)]
    rank = int(rng.integers(1, 5))
    out = tuple(int(v) for v in rng.integers(1, 40, rank))
    if rng.random() < 0.3:  # a long last dimension, odd or aligned
        out = out[:-1] + (int(rng.choice([4095, 4096, 1021, 2048, 8191])),)
    while int(np.prod(out)) > 1 << 22:  # at most 4M elements: the oracle stays quick
        i = int(np.argmax(out[:-1]))
        out = out[:i] + (max(1, out[i] // 2),) + out[i + 1:]
    op = ["add", "add_relu", "mul", "mul_add", "relu", "relu_grad", "bias_add"][rng.integers(7)]
    print(f"seed {seed}: {op} out={out} {dtype}", flush=True)
    x = gen(rng, out, dtype)
    if op == "relu":
        got = ops.Relu(to_dev(x, dtype, dev))
        ref = oracle.eltwise("relu", [x], dtype)
    elif op == "relu_grad":
        feat = gen(rng, out, dtype)
        got = ops.ReluGrad(to_dev(x, dtype, dev), to_dev(feat, dtype, dev))
        ref = oracle.eltwise("relu_grad", [x, feat], dtype)
    elif op == "bias_add":
        b = gen(rng, out[-1:], dtype)
        relu = bool(rng.random() < 0.5)
        fn = ops.MusaBiasAddRelu if relu else ops.BiasAdd
        if x.ndim < 2:  # TF's BiasAdd rejects these
            with pytest.raises(tfma.errors.InvalidArgumentError, match="at least 2D"):
                fn(to_dev(x, dtype, dev), to_dev(b, dtype, dev))
            return
        got = fn(to_dev(x, dtype, dev), to_dev(b, dtype, dev))
        ref = oracle.bias_add(x, b, relu=relu, dtype=dtype)
    elif op == "mul_add":
        a = gen(rng, _bcast_shape(rng, out), dtype)
        b = gen(rng, _bcast_shape(rng, out), dtype)
        got = ops.MusaShiftedAffineMap(to_dev(x, dtype, dev), to_dev(a, dtype, dev),
                                       to_dev(b, dtype, dev))
        ref = oracle.eltwise("mul_add", [x, a, b], dtype)
    else:
        y = gen(rng, _bcast_shape(rng, out), dtype)
        first, second = (x, y) if rng.random() < 0.75 else (y, x)
        fn = {"add": ops.AddV2, "add_relu": ops.MusaAddV2Relu, "mul": ops.Mul}[op]
        got = fn(to_dev(first, dtype, dev), to_dev(second, dtype, dev))
        ref = oracle.eltwise(op, [first, second], dtype)
    torch.cuda.synchronize()
    assert_bitwise(to_np(got, dtype), ref, op)
