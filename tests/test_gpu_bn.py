"""FusedBatchNormV3 / FusedBatchNormGradV3 on the GPU vs the TF-CPU oracle.

Tolerances (written per check): float32 outputs and all float32 statistics
1e-5, float16/bfloat16 activations 1e-2, each as max|got-ref| / max|ref| over
the output (the reference's own tests use np.allclose with rtol=atol=1e-4 at
[2,2,2,4], test/ops/fused_batchnorm_op_test.py:25-55).
"""
import zlib

import numpy as np
import pytest
import torch

import tensorflow_musa_extension_amd as tfma
from oracle import oracle
from tests.helpers import (assert_close, bn_fwd_ref32, bn_grad_ref32, bn_max_ulp,
                           bn_scale_backprop_ref64, gen, max_ulp_vs, to_dev, to_np)

pytestmark = pytest.mark.gpu
ops = tfma.raw_ops

ACT_TOL = {"float32": 1e-5, "float16": 1e-2, "bfloat16": 1e-2}
STAT_TOL = 1e-5


def _inputs(rng, shape, dtype, data_format, loc=0.0):
    c = shape[-1] if data_format == "NHWC" else shape[1]
    x = gen(rng, shape, dtype, loc=loc)
    scale = rng.uniform(0.5, 1.5, c).astype(np.float32)
    offset = (0.1 * rng.standard_normal(c)).astype(np.float32)
    dy = gen(rng, shape, dtype)
    return x, scale, offset, dy


def _run_fwd_grad(dev, x, scale, offset, dy, dtype, data_format, eps, poison=True,
                  mean=None, var=None, factor=1.0, is_training=True):
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    tx = to_dev(x, dtype, dev)
    c = scale.shape[0]
    f32 = dict(dtype=torch.float32, device=dev)
    out = ops.FusedBatchNormV3Result(
        torch.empty_like(tx), torch.empty(c, **f32), torch.empty(c, **f32),
        torch.empty(c, **f32), torch.empty(c, **f32), torch.empty((), **f32))
    if poison:  # every output must be overwritten
        for o in out:
            o.fill_(float("nan"))
    tm = f(mean) if mean is not None else torch.empty(0, **f32)
    tv = f(var) if var is not None else torch.empty(0, **f32)
    fwd = ops.FusedBatchNormV3(tx, f(scale), f(offset), tm, tv, epsilon=eps,
                               exponential_avg_factor=factor, data_format=data_format,
                               is_training=is_training, out=out)
    tdy = to_dev(dy, dtype, dev)
    gout = ops.FusedBatchNormGradV3Result(
        torch.empty_like(tx), torch.empty(c, **f32), torch.empty(c, **f32),
        torch.empty(c, **f32), torch.empty(c, **f32))
    if poison:
        for o in gout:
            o.fill_(float("nan"))
    grad = ops.FusedBatchNormGradV3(tdy, tx, f(scale), fwd.reserve_space_1,
                                    fwd.reserve_space_2, fwd.reserve_space_3, epsilon=eps,
                                    data_format=data_format, is_training=is_training, out=gout)
    torch.cuda.synchronize()
    return fwd, grad


CASES = [
    # (shape, dtype, data_format)
    ((2, 2, 2, 4), "float32", "NHWC"),       # reference test shape
    ((2, 4, 5, 3), "float32", "NHWC"),       # C % 4 != 0: scalar path
    ((4, 7, 9, 64), "float32", "NHWC"),
    ((32, 56, 56, 64), "float32", "NHWC"),   # cfg1
    ((8, 14, 14, 256), "float16", "NHWC"),
    ((8, 14, 14, 256), "bfloat16", "NHWC"),
    ((3, 5, 5, 2048), "float16", "NHWC"),
    ((16, 7, 7, 33), "float16", "NHWC"),     # odd C: scalar path
    ((5, 3, 3, 520), "bfloat16", "NHWC"),    # C % 256 != 0: partial channel tile
    ((2, 3, 5, 5), "float32", "NCHW"),
    # The reference's regression shapes (test/ops/fused_batchnorm_op_test.py):
    # Keras' 2-D BatchNormalization as [N,1,1,C] (:97-141), the NCHW grad
    # (:178-216) and the NCHW batch / saved variance values (:407-).
    ((512, 1, 1, 64), "float32", "NHWC"),
    ((4, 8, 6, 6), "float32", "NCHW"),
    ((2, 3, 4, 5), "float32", "NCHW"),
    ((4, 16, 7, 7), "float16", "NCHW"),
    ((2, 8, 28, 28), "bfloat16", "NCHW"),
    ((3, 6, 8, 8), "float32", "NCHW"),
    # test/ops/fused_batchnorm_hcnw_op_test.py:86-105
    ((2, 32, 1, 1), "float32", "NCHW"),
    ((2, 1, 1, 32), "float32", "NHWC"),
    ((4, 16, 8, 8), "float16", "NCHW"),
    ((1, 64, 32, 32), "float32", "NCHW"),
    ((8, 128, 16, 16), "float32", "NCHW"),
    ((2, 3, 224, 224), "float32", "NCHW"),
]


@pytest.mark.parametrize("shape,dtype,data_format", CASES)
def test_fwd_grad_matches_oracle(dev, shape, dtype, data_format):
    rng = np.random.default_rng(zlib.crc32(repr((shape, dtype, data_format)).encode()))
    eps = 1e-3
    x, scale, offset, dy = _inputs(rng, shape, dtype, data_format)
    fwd, grad = _run_fwd_grad(dev, x, scale, offset, dy, dtype, data_format, eps)
    ry, rbm, rbv, rsm, rsv = oracle.bn_fwd(x, scale, offset, epsilon=eps,
                                          data_format=data_format, dtype=dtype)
    assert_close(to_np(fwd.y, dtype), ry, dtype, ACT_TOL[dtype], "y")
    for name, got, ref in (("batch_mean", fwd.batch_mean, rbm),
                           ("batch_variance", fwd.batch_variance, rbv),
                           ("reserve_space_1", fwd.reserve_space_1, rsm),
                           ("reserve_space_2", fwd.reserve_space_2, rsv)):
        assert_close(got.cpu().numpy(), ref, "float32", STAT_TOL, name)
    assert float(fwd.reserve_space_3.cpu()) == 0.0
    # Grad consumes the forward's reserve spaces, as in a training step.
    rdx, rsb, rob = oracle.bn_grad(dy, x, scale, fwd.reserve_space_1.cpu().numpy(),
                                   fwd.reserve_space_2.cpu().numpy(), epsilon=eps,
                                   data_format=data_format, dtype=dtype)
    assert_close(to_np(grad.x_backprop, dtype), rdx, dtype, ACT_TOL[dtype], "x_backprop")
    assert_close(grad.scale_backprop.cpu().numpy(), rsb, "float32", STAT_TOL, "scale_backprop")
    assert_close(grad.offset_backprop.cpu().numpy(), rob, "float32", STAT_TOL, "offset_backprop")
    assert torch.all(grad.reserve_space_4 == 0) and torch.all(grad.reserve_space_5 == 0)


def test_dense_weight_grad_through_batch_norm(dev):
    """The reference's testFusedBatchNormGradDX2DWeightGrad
    (test/ops/fused_batchnorm_op_test.py:143-176): h = x @ w of [4096,128] x
    [128,256], BatchNormalization over the 256 features as the [N,1,1,C] op
    Keras runs, loss = sum(y), and the dense layer's weight gradient
    dW = x^T @ dh compared with the same product of the oracle's dh (float64
    products, rtol 1e-3 and atol 1e-3 as there)."""
    rng = np.random.default_rng(61)
    xin = rng.standard_normal((4096, 128)).astype(np.float32)
    w = rng.standard_normal((128, 256)).astype(np.float32)
    h = (xin @ w).astype(np.float32).reshape(4096, 1, 1, 256)
    scale = np.ones(256, np.float32)
    offset = np.zeros(256, np.float32)
    dy = np.ones_like(h)  # d sum(y) / dy
    eps = 1e-5
    fwd, grad = _run_fwd_grad(dev, h, scale, offset, dy, "float32", "NHWC", eps)
    rdx, _, _ = oracle.bn_grad(dy, h, scale, fwd.reserve_space_1.cpu().numpy(),
                               fwd.reserve_space_2.cpu().numpy(), epsilon=eps)
    dx = grad.x_backprop.cpu().numpy().reshape(4096, 256).astype(np.float64)
    dw = xin.astype(np.float64).T @ dx
    rdw = xin.astype(np.float64).T @ rdx.reshape(4096, 256).astype(np.float64)
    np.testing.assert_allclose(dw, rdw, rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_layer_norm_grad_large_variance(dev, dtype):
    """The reference's testLayerNormGradNCHWLargeVariance
    (test/ops/fused_batchnorm_op_test.py:218-256): Keras' LayerNormalization
    of [128,1536] runs FusedBatchNormV3 / GradV3 on NCHW [1,128,1536,1]
    (128 channels of 1536 elements), x = 10 N(0,1) (variance 100), dy =
    1e-3 N(0,1), epsilon 1e-3; the grad must use the population variance
    from reserve_space_2 (the reference's bug: a variance passed where the
    reciprocal standard deviation was expected inflated dx by orders of
    magnitude).  Against the oracle at this file's bars."""
    rng = np.random.default_rng(42)
    x = gen(rng, (1, 128, 1536, 1), dtype, scale=10.0)
    dy = gen(rng, (1, 128, 1536, 1), dtype, scale=1e-3)
    scale = np.ones(128, np.float32)
    offset = np.zeros(128, np.float32)
    eps = 1e-3
    fwd, grad = _run_fwd_grad(dev, x, scale, offset, dy, dtype, "NCHW", eps)
    ry, _, _, rsm, rsv = oracle.bn_fwd(x, scale, offset, epsilon=eps, data_format="NCHW",
                                       dtype=dtype)
    assert_close(to_np(fwd.y, dtype), ry, dtype, ACT_TOL[dtype], "y")
    assert_close(fwd.reserve_space_2.cpu().numpy(), rsv, "float32", STAT_TOL, "reserve_space_2")
    rdx, rsb, rob = oracle.bn_grad(dy, x, scale, fwd.reserve_space_1.cpu().numpy(),
                                   fwd.reserve_space_2.cpu().numpy(), epsilon=eps,
                                   data_format="NCHW", dtype=dtype)
    assert_close(to_np(grad.x_backprop, dtype), rdx, dtype, ACT_TOL[dtype], "x_backprop")
    assert_close(grad.scale_backprop.cpu().numpy(), rsb, "float32", STAT_TOL, "scale_backprop")
    # dx stays at the scale of dy / std (1e-4), not inflated
    assert float(grad.x_backprop.float().abs().max()) < 1e-2


SLICED_CASES = [
    ((4, 9, 11, 256), "float16"),
    ((4, 9, 11, 256), "bfloat16"),
    ((3, 7, 13, 128), "float32"),
    ((6, 5, 7, 200), "float16"),   # 25 vectors: a last tile with one active vector
    ((2, 3, 3, 512), "bfloat16"),  # fewer rows than a workgroup pass: empty groups
]


@pytest.mark.parametrize("tw", [4, 8, 16, 32])
@pytest.mark.parametrize("is_training", [True, False])
@pytest.mark.parametrize("shape,dtype", SLICED_CASES)
def test_sliced_grad_matches_oracle(dev, tune, shape, dtype, tw, is_training):
    """The sliced fused gradient (each workgroup runs the whole two-phase pass
    once per channel tile of tw vectors), forced at small shapes, against the
    oracle; the plan query shows how many slices ran."""
    tune("bn_slice_tw", tw)
    rng = np.random.default_rng(zlib.crc32(repr((shape, dtype, tw)).encode()))
    eps = 1e-3
    c = shape[-1]
    x, scale, offset, dy = _inputs(rng, shape, dtype, "NHWC")
    mean = (0.1 * rng.standard_normal(c)).astype(np.float32)
    var = rng.uniform(0.5, 2.0, c).astype(np.float32)
    fwd, grad = _run_fwd_grad(dev, x, scale, offset, dy, dtype, "NHWC", eps, mean=mean,
                              var=var, is_training=is_training)
    plan = ops.fused_batch_norm_last_plan()
    vec = 4 if dtype == "float32" else 8
    tiles = -(-(c // vec) // tw)
    assert plan["fused"] == 1
    if 2 <= tiles <= 8:  # forced plans run at most 8 slices
        assert plan["slices"] == tiles and plan["channel_tiles"] == tiles, plan
    else:
        assert plan["slices"] == 1, plan
    sm = fwd.reserve_space_1.cpu().numpy() if is_training else mean
    sv = fwd.reserve_space_2.cpu().numpy() if is_training else var
    rdx, rsb, rob = oracle.bn_grad(dy, x, scale, sm, sv, epsilon=eps, dtype=dtype,
                                   is_training=is_training)
    assert_close(to_np(grad.x_backprop, dtype), rdx, dtype, ACT_TOL[dtype], "x_backprop")
    assert_close(grad.scale_backprop.cpu().numpy(), rsb, "float32", STAT_TOL, "scale_backprop")
    assert_close(grad.offset_backprop.cpu().numpy(), rob, "float32", STAT_TOL, "offset_backprop")
    assert torch.all(grad.reserve_space_4 == 0) and torch.all(grad.reserve_space_5 == 0)


@pytest.mark.parametrize("shape,dtype,tw", [((64, 56, 56, 256), "float16", 8),
                                            ((64, 56, 56, 256), "bfloat16", 8),
                                            ((64, 56, 56, 256), "float16", 4),
                                            ((32, 28, 28, 128), "float32", 8),
                                            ((6, 5, 7, 200), "float16", 8),
                                            ((64, 28, 28, 512), "bfloat16", 32),
                                            ((16, 28, 28, 512), "float32", 16)])
def test_sliced_overlap_equals_plain_sliced(dev, tune, shape, dtype, tw):
    """The sliced gradient that reads the next slice's streamed rows while a
    slice's coefficients are pending, against the plain sliced pass
    (override bn_sliced_overlap 0), both forced to tw-vector tiles: the same
    slices, so scale_backprop and offset_backprop within 1e-5 of their
    largest value (the streamed rows' sums are added in a different order)
    and x_backprop within one ulp of its largest value; both against the
    oracle as well."""
    tune("bn_slice_tw", tw)
    rng = np.random.default_rng(zlib.crc32(repr((shape, dtype, tw, "overlap")).encode()))
    eps = 1e-3
    x, scale, offset, dy = _inputs(rng, shape, dtype, "NHWC", loc=0.5)
    outs = {}
    for mode in ("1", "0"):
        tune("bn_sliced_overlap", int(mode))
        fwd, grad = _run_fwd_grad(dev, x, scale, offset, dy, dtype, "NHWC", eps)
        plan = ops.fused_batch_norm_last_plan()
        vec = 4 if dtype == "float32" else 8
        assert plan["slices"] == -(-(shape[-1] // vec) // tw), plan
        outs[mode] = (fwd, grad)
    (fa, ga), (fb, gb) = outs["1"], outs["0"]
    for name in ("scale_backprop", "offset_backprop"):
        a, b = getattr(ga, name).cpu().numpy(), getattr(gb, name).cpu().numpy()
        assert np.max(np.abs(a - b)) <= 1e-5 * np.max(np.abs(b)), name
    da, db = to_np(ga.x_backprop, dtype).astype(np.float64), to_np(gb.x_backprop, dtype).astype(np.float64)
    big = np.max(np.abs(db))
    ulp = {"float32": 2.0 ** -23, "float16": 2.0 ** -10, "bfloat16": 2.0 ** -7}[dtype]
    assert np.max(np.abs(da - db)) <= ulp * 2.0 ** np.ceil(np.log2(big)), "x_backprop"
    rdx, rsb, rob = oracle.bn_grad(dy, x, scale, fa.reserve_space_1.cpu().numpy(),
                                   fa.reserve_space_2.cpu().numpy(), epsilon=eps, dtype=dtype)
    assert_close(to_np(ga.x_backprop, dtype), rdx, dtype, ACT_TOL[dtype], "x_backprop")
    assert_close(ga.scale_backprop.cpu().numpy(), rsb, "float32", STAT_TOL, "scale_backprop")
    assert_close(ga.offset_backprop.cpu().numpy(), rob, "float32", STAT_TOL, "offset_backprop")


OWNED_CASES = [
    ((4, 256, 7, 8), "float16"),      # 28 vectors per channel: most threads idle
    ((64, 256, 28, 28), "bfloat16"),  # every row on chip
    ((32, 512, 14, 14), "float32"),   # two channels per CU
    ((8, 300, 12, 12), "float16"),    # C not a multiple of the CU count
    ((2, 256, 64, 72), "float16"),    # a plane of 576 vectors: rows step within planes
    ((64, 256, 32, 56), "bfloat16"),  # grad rows past registers + LDS: streamed
    ((256, 256, 28, 28), "float16"),  # forward rows streamed too
]


@pytest.mark.parametrize("shape,dtype", OWNED_CASES)
def test_nchw_owned_matches_oracle(dev, shape, dtype):
    """NCHW training with at least one channel per CU runs the
    channel-per-workgroup kernel (plan fused = 2) forward and backward;
    against the oracle like the split path."""
    if shape[1] < torch.cuda.get_device_properties(dev).multi_processor_count:
        pytest.skip("fewer channels than CUs: split path")
    rng = np.random.default_rng(zlib.crc32(repr((shape, dtype, "owned")).encode()))
    eps = 1e-3
    x, scale, offset, dy = _inputs(rng, shape, dtype, "NCHW", loc=0.5)
    fwd, grad = _run_fwd_grad(dev, x, scale, offset, dy, dtype, "NCHW", eps)
    plan = ops.fused_batch_norm_last_plan()
    assert plan["fused"] == 2 and plan["workgroups"] == shape[1], plan
    ry, rbm, rbv, rsm, rsv = oracle.bn_fwd(x, scale, offset, epsilon=eps, data_format="NCHW",
                                          dtype=dtype)
    assert_close(to_np(fwd.y, dtype), ry, dtype, ACT_TOL[dtype], "y")
    for name, got, ref in (("batch_mean", fwd.batch_mean, rbm),
                           ("batch_variance", fwd.batch_variance, rbv),
                           ("reserve_space_1", fwd.reserve_space_1, rsm),
                           ("reserve_space_2", fwd.reserve_space_2, rsv)):
        assert_close(got.cpu().numpy(), ref, "float32", STAT_TOL, name)
    rdx, rsb, rob = oracle.bn_grad(dy, x, scale, fwd.reserve_space_1.cpu().numpy(),
                                   fwd.reserve_space_2.cpu().numpy(), epsilon=eps,
                                   data_format="NCHW", dtype=dtype)
    assert_close(to_np(grad.x_backprop, dtype), rdx, dtype, ACT_TOL[dtype], "x_backprop")
    assert_close(grad.scale_backprop.cpu().numpy(), rsb, "float32", STAT_TOL, "scale_backprop")
    assert_close(grad.offset_backprop.cpu().numpy(), rob, "float32", STAT_TOL, "offset_backprop")
    assert torch.all(grad.reserve_space_4 == 0) and torch.all(grad.reserve_space_5 == 0)


def test_nchw_owned_equals_split_path(dev, tune):
    """The channel-per-workgroup kernel and the split path (forced with
    override bn_nchw_owned 0) agree: statistics to 1e-5 of their largest value
    (the float32 partial sums of the two are taken in different orders, and
    sums such as offset_backprop cancel), outputs within one ulp of their
    largest value."""
    rng = np.random.default_rng(5)
    shape, dtype = (32, 256, 28, 28), "float16"
    x, scale, offset, dy = _inputs(rng, shape, dtype, "NCHW")
    f1, g1 = _run_fwd_grad(dev, x, scale, offset, dy, dtype, "NCHW", 1e-3)
    assert ops.fused_batch_norm_last_plan()["fused"] == 2
    tune("bn_nchw_owned", 0)
    f2, g2 = _run_fwd_grad(dev, x, scale, offset, dy, dtype, "NCHW", 1e-3)
    assert ops.fused_batch_norm_last_plan()["fused"] == 0
    for name, a, b in (("mean", f1.reserve_space_1, f2.reserve_space_1),
                       ("variance", f1.reserve_space_2, f2.reserve_space_2),
                       ("scale_backprop", g1.scale_backprop, g2.scale_backprop),
                       ("offset_backprop", g1.offset_backprop, g2.offset_backprop)):
        assert_close(a.cpu().numpy(), b.cpu().numpy(), "float32", STAT_TOL, name)
    for a, b in ((f1.y, f2.y), (g1.x_backprop, g2.x_backprop)):
        assert (a.float() - b.float()).abs().max().item() <= 2 ** -9 * max(1.0, b.float().abs().max().item())


def test_large_mean_statistics(dev):
    """|mean| >> std: the shifted sums must not cancel (variance to 1e-5)."""
    rng = np.random.default_rng(7)
    shape = (16, 28, 28, 64)
    x, scale, offset, dy = _inputs(rng, shape, "float32", "NHWC", loc=1000.0)
    fwd, _ = _run_fwd_grad(dev, x, scale, offset, dy, "float32", "NHWC", 1e-3)
    _, rbm, rbv, rsm, rsv = oracle.bn_fwd(x, scale, offset, epsilon=1e-3)
    assert_close(fwd.reserve_space_1.cpu().numpy(), rsm, "float32", STAT_TOL, "mean")
    assert_close(fwd.reserve_space_2.cpu().numpy(), rsv, "float32", 1e-5, "variance")


@pytest.mark.parametrize("shape,data_format", [((64, 28, 28, 64), "NHWC"),
                                               ((16, 64, 28, 28), "NCHW"),
                                               ((256, 14, 14, 1024), "NHWC")])
def test_outlier_first_element_statistics(dev, shape, data_format):
    """A channel whose first element is a large outlier (1e3 against N(0,1)
    data, and -5e2 in a second channel): the statistics must still match
    TF-CPU's two-pass computation to 1e-5, i.e. the kernels' sums must not
    be taken around that element."""
    rng = np.random.default_rng(17)
    x, scale, offset, dy = _inputs(rng, shape, "float32", data_format)
    first = (0, 0, 0, slice(None)) if data_format == "NHWC" else (0, slice(None), 0, 0)
    row0 = x[first].copy()
    row0[3] = 1e3
    row0[5] = -5e2
    x[first] = row0
    fwd, _ = _run_fwd_grad(dev, x, scale, offset, dy, "float32", data_format, 1e-3)
    _, rbm, rbv, rsm, rsv = oracle.bn_fwd(x, scale, offset, epsilon=1e-3,
                                          data_format=data_format)
    assert_close(fwd.reserve_space_1.cpu().numpy(), rsm, "float32", STAT_TOL, "mean")
    assert_close(fwd.reserve_space_2.cpu().numpy(), rsv, "float32", 1e-5, "variance")
    assert_close(fwd.batch_variance.cpu().numpy(), rbv, "float32", 1e-5, "Bessel variance")


def test_exponential_avg_factor_and_inference(dev):
    rng = np.random.default_rng(11)
    shape = (4, 6, 6, 32)
    x, scale, offset, dy = _inputs(rng, shape, "float32", "NHWC")
    run_mean = rng.standard_normal(32).astype(np.float32)
    run_var = rng.uniform(0.5, 2.0, 32).astype(np.float32)
    fwd, _ = _run_fwd_grad(dev, x, scale, offset, dy, "float32", "NHWC", 1e-3,
                           mean=run_mean, var=run_var, factor=0.3)
    ry, rbm, rbv, rsm, rsv = oracle.bn_fwd(x, scale, offset, run_mean, run_var, epsilon=1e-3,
                                          exponential_avg_factor=0.3)
    assert_close(fwd.batch_mean.cpu().numpy(), rbm, "float32", STAT_TOL, "blended mean")
    assert_close(fwd.batch_variance.cpu().numpy(), rbv, "float32", STAT_TOL, "blended var")
    assert_close(to_np(fwd.y, "float32"), ry, "float32", 1e-5, "y")
    # Inference: y from the running statistics; grad with is_training=False.
    fwd, grad = _run_fwd_grad(dev, x, scale, offset, dy, "float32", "NHWC", 1e-3,
                              mean=run_mean, var=run_var, is_training=False)
    ry, rbm, rbv, _, _ = oracle.bn_fwd(x, scale, offset, run_mean, run_var, epsilon=1e-3,
                                      is_training=False)
    assert_close(to_np(fwd.y, "float32"), ry, "float32", 1e-5, "inference y")
    np.testing.assert_array_equal(fwd.batch_mean.cpu().numpy(), run_mean)
    rdx, rsb, rob = oracle.bn_grad(dy, x, scale, run_mean, run_var, epsilon=1e-3,
                                   is_training=False)
    assert_close(to_np(grad.x_backprop, "float32"), rdx, "float32", 1e-5, "inference dx")
    assert_close(grad.scale_backprop.cpu().numpy(), rsb, "float32", STAT_TOL, "inference dscale")


def test_empty_batch(dev):
    f32 = dict(dtype=torch.float32, device=dev)
    x = torch.empty((0, 4, 4, 8), **f32)
    scale = torch.ones(8, **f32)
    offset = torch.zeros(8, **f32)
    e = torch.empty(0, **f32)
    fwd = ops.FusedBatchNormV3(x, scale, offset, e, e)
    torch.cuda.synchronize()
    assert fwd.y.shape == x.shape
    assert torch.isnan(fwd.batch_mean).all() and torch.isnan(fwd.batch_variance).all()
    grad = ops.FusedBatchNormGradV3(x, x, scale, fwd.reserve_space_1, fwd.reserve_space_2,
                                    fwd.reserve_space_3)
    torch.cuda.synchronize()
    assert torch.all(grad.scale_backprop == 0) and torch.all(grad.offset_backprop == 0)


def test_constant_channel(dev):
    """sigma^2 = 0: y = offset exactly, batch_variance = 0."""
    f32 = dict(dtype=torch.float32, device=dev)
    x = torch.full((4, 5, 5, 16), 3.25, **f32)
    scale = torch.linspace(0.5, 1.5, 16, **f32)
    offset = torch.linspace(-1, 1, 16, **f32)
    e = torch.empty(0, **f32)
    fwd = ops.FusedBatchNormV3(x, scale, offset, e, e, epsilon=1e-3)
    torch.cuda.synchronize()
    assert torch.equal(fwd.y, offset.expand_as(fwd.y))
    assert torch.all(fwd.batch_variance == 0)
    assert torch.all(fwd.batch_mean == 3.25)


CFG2_SHAPES = [(256, 56, 56, 256), (256, 28, 28, 512), (256, 14, 14, 1024), (256, 7, 7, 2048)]


@pytest.mark.parametrize("shape", CFG2_SHAPES)
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_cfg2_full_size(dev, shape, dtype):
    """BASELINE cfg2 at full size, every shape in both dtypes, against the
    oracle (eps=1.001e-5): y and x_backprop to 1e-2 normwise and within 1
    ulp at every element (BN16_ATOL floor), every statistic
    (batch_mean, batch_variance, reserve spaces, scale_backprop,
    offset_backprop) to 1e-5 - the outputs the reference's own test checks,
    test/ops/fused_batchnorm_op_test.py:358-448.  The 56x56 gradient runs
    in 4 slices of 64 channels and the 28x28 gradient in 2 of 256 (both
    hiding their slices' hand-offs); the 56x56 forward hands part of phase 3
    out dynamically; the plan query shows that these paths are the ones
    compared here."""
    rng = np.random.default_rng(zlib.crc32(repr((shape, dtype)).encode()))
    eps = 1.001e-5
    x, scale, offset, dy = _inputs(rng, shape, dtype, "NHWC")
    print(f"cfg2 {shape} {dtype}: inputs ready", flush=True)
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    tx, tdy = to_dev(x, dtype, dev), to_dev(dy, dtype, dev)
    e = torch.empty(0, device=dev)
    fwd = ops.FusedBatchNormV3(tx, f(scale), f(offset), e, e, epsilon=eps)
    fplan = ops.fused_batch_norm_last_plan()
    grad = ops.FusedBatchNormGradV3(tdy, tx, f(scale), fwd.reserve_space_1,
                                    fwd.reserve_space_2, fwd.reserve_space_3, epsilon=eps)
    gplan = ops.fused_batch_norm_last_plan()
    torch.cuda.synchronize()
    assert fplan["fused"] == 1 and gplan["fused"] == 1
    if shape[1] == 56:
        assert gplan["slices"] == 4 and gplan["dynamic_rows"] == 0, gplan
        assert fplan["dynamic_rows"] > 0, fplan
    elif shape[1] == 28:
        assert gplan["slices"] == 2 and gplan["dynamic_rows"] == 0, gplan
    else:
        assert gplan["slices"] == 1, gplan
    del tx, tdy
    ry, rbm, rbv, rsm, rsv = oracle.bn_fwd(x, scale, offset, epsilon=eps, dtype=dtype)
    assert_close(to_np(fwd.y, dtype), ry, dtype, 1e-2, "y")
    # Element by element: every y within 1 ulp of the oracle's (or BN16_ATOL
    # where the float32 terms cancel to near zero).
    uy = max_ulp_vs(fwd.y, ry, dtype)
    assert uy <= 1, f"y: {uy} ulp from the oracle"
    del ry
    for name, got, want in (("batch_mean", fwd.batch_mean, rbm),
                            ("batch_variance", fwd.batch_variance, rbv),
                            ("reserve_space_1", fwd.reserve_space_1, rsm),
                            ("reserve_space_2", fwd.reserve_space_2, rsv)):
        assert_close(got.cpu().numpy(), want, "float32", STAT_TOL, name)
    # The oracle's grad from its own statistics: the kernel's dx and
    # scale_backprop are checked against values that share nothing with it.
    rdx, rsb, rob = oracle.bn_grad(dy, x, scale, rsm, rsv, epsilon=eps, dtype=dtype)
    assert_close(to_np(grad.x_backprop, dtype), rdx, dtype, 1e-2, "x_backprop")
    udx = max_ulp_vs(grad.x_backprop, rdx, dtype)
    assert udx <= 1, f"x_backprop: {udx} ulp from the oracle"
    assert_close(grad.scale_backprop.cpu().numpy(), rsb, "float32", STAT_TOL, "scale_backprop")
    assert_close(grad.offset_backprop.cpu().numpy(), rob, "float32", STAT_TOL, "offset_backprop")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_largest_shape_invariants(dev, dtype):
    """[256,56,56,256] (cfg2's largest) in f16 and bf16: size-independent
    properties.  Per channel: mean(y) = offset and var(y) = scale^2
    var/(var+eps) (both measured in float64 on the device); offset_backprop =
    sum(dy) and scale_backprop = rsqrt(var+eps) * sum(dy*(x-mean)) against
    float64 sums of the inputs; y and dx elementwise within 1 ulp of the
    float32 closed form (or 1e-6: the float32 precision of its terms)."""
    torch.manual_seed(0)
    shape = (256, 56, 56, 256)
    x = torch.randn(shape, device=dev).to(dtype)
    dy = torch.randn(shape, device=dev).to(dtype)
    scale = torch.rand(256, device=dev) + 0.5
    offset = 0.1 * torch.randn(256, device=dev)
    e = torch.empty(0, device=dev)
    eps = 1.001e-5
    fwd = ops.FusedBatchNormV3(x, scale, offset, e, e, epsilon=eps)
    xd = x.double().reshape(-1, 256)
    mean_ref = xd.mean(0)
    var_ref = xd.var(0, unbiased=False)
    assert torch.allclose(fwd.reserve_space_1.double(), mean_ref, rtol=0, atol=1e-5)
    assert torch.allclose(fwd.reserve_space_2.double(), var_ref, rtol=1e-5, atol=0)
    yd = fwd.y.double().reshape(-1, 256)
    assert torch.allclose(yd.mean(0), offset.double(), atol=2e-3)
    want_var = scale.double() ** 2 * var_ref / (var_ref + eps)
    assert torch.allclose(yd.var(0, unbiased=False), want_var, rtol=2e-3)
    del yd
    grad = ops.FusedBatchNormGradV3(dy, x, scale, fwd.reserve_space_1, fwd.reserve_space_2,
                                    fwd.reserve_space_3, epsilon=eps)
    assert ops.fused_batch_norm_last_plan()["slices"] == 4
    dyd = dy.double().reshape(-1, 256)
    assert torch.allclose(grad.offset_backprop.double(), dyd.sum(0), rtol=1e-5, atol=1e-2)
    del dyd
    rows = xd.shape[0]
    sbp = bn_scale_backprop_ref64(dy, x, fwd.reserve_space_1, fwd.reserve_space_2, eps, rows,
                                  256)
    assert torch.allclose(grad.scale_backprop.double(), sbp, rtol=1e-5, atol=1e-2)
    # Every element of y and dx within 1 ulp of the float32 closed form from
    # the kernel's own statistics, in its operation order.  (sum(dx) = 0 is
    # not a usable check for 16-bit dx: where scale*k is near a short binary
    # fraction, scale*k*dy falls on or halfway between f16 values and the
    # small mean terms bias every rounding the same way - TF-CPU's f16 output
    # does this too, with |sum(dx)| in the hundreds at this size.)
    mu, sig = fwd.reserve_space_1, fwd.reserve_space_2
    assert bn_max_ulp(fwd.y, bn_fwd_ref32(x, mu, sig, scale, offset, eps, rows, 256), rows,
                      256) <= 1
    ref = bn_grad_ref32(dy, x, scale, mu, sig, grad.offset_backprop, grad.scale_backprop, eps,
                        rows, 256)
    assert bn_max_ulp(grad.x_backprop, ref, rows, 256) <= 1
    torch.cuda.synchronize()


def test_fused_launches_alternate_streams(dev):
    """Fused (persistent) launches issued on two streams in turn.  The library
    chains each launch to the previous one's end event, so only one grid is
    resident at a time: every output must equal the single-stream result bit
    for bit and no grid-barrier wait may have given up, with tracing off and
    on (a traced launch's end event is a trace event)."""
    torch.manual_seed(3)
    eps = 1.001e-5
    cases = []
    for shape, dt in (((16, 14, 14, 256), torch.float16), ((8, 7, 7, 512), torch.bfloat16)):
        c = shape[-1]
        cases.append((torch.randn(shape, device=dev).to(dt), torch.randn(shape, device=dev).to(dt),
                      torch.rand(c, device=dev) + 0.5, 0.1 * torch.randn(c, device=dev)))
    e = torch.empty(0, device=dev)

    def step(x, dy, scale, offset):
        f = ops.FusedBatchNormV3(x, scale, offset, e, e, epsilon=eps)
        g = ops.FusedBatchNormGradV3(dy, x, scale, f.reserve_space_1, f.reserve_space_2,
                                     f.reserve_space_3, epsilon=eps)
        assert ops.last_kernel_name() == "tfma_bn_grad_fused"
        return [f.y, f.batch_mean, f.batch_variance, g.x_backprop, g.scale_backprop,
                g.offset_backprop]

    ops.fused_batch_norm_barrier_timed_out(reset=True)
    want = [[t.clone() for t in step(*c)] for c in cases]
    torch.cuda.synchronize()
    streams = (torch.cuda.Stream(), torch.cuda.Stream())
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    for trace in (None, "tfma_bn_grad_fused"):
        ops.trace_enable(trace)
        got = []
        for i in range(12):
            with torch.cuda.stream(streams[i % 2]):
                got.append((i % len(cases), step(*cases[i % len(cases)])))
        torch.cuda.synchronize()
        ms, n = ops.trace_read()
        ops.trace_enable(None)
        assert n == (12 if trace else 0)
        assert not ops.fused_batch_norm_barrier_timed_out()
        for k, outs in got:
            for w, g in zip(want[k], outs):
                assert torch.equal(w, g)


def test_shape_errors(dev):
    f32 = dict(dtype=torch.float32, device=dev)
    x = torch.zeros((2, 3, 3, 4), **f32)
    e = torch.empty(0, **f32)
    with pytest.raises(tfma.InvalidArgumentError, match="scale must have the same number"):
        ops.FusedBatchNormV3(x, torch.ones(5, **f32), torch.zeros(4, **f32), e, e)
    with pytest.raises(tfma.InvalidArgumentError, match="When is_training=false, mean"):
        ops.FusedBatchNormV3(x, torch.ones(4, **f32), torch.zeros(4, **f32), e, e,
                             is_training=False)
    with pytest.raises(tfma.InvalidArgumentError, match="x and y_backprop must have same shape"):
        ops.FusedBatchNormGradV3(torch.zeros((2, 3, 3, 5), **f32), x, torch.ones(4, **f32),
                                 torch.zeros(4, **f32), torch.ones(4, **f32),
                                 torch.zeros((), **f32))


def test_fused_epochs_fresh_values(dev):
    """Fused launches publish their partials and coefficients tagged with the
    launch's epoch, in library-owned slots that later launches reuse.  Back-to-
    back launches with no synchronization between them - same shape with other
    data, and shapes whose (group, channel) slots and channel words overlap
    differently - must each equal the same launch run alone, bit for bit, and
    no poll may give up (a stale value taken for a fresh one would show as a
    mismatch here)."""
    torch.manual_seed(5)
    eps = 1.001e-5
    e = torch.empty(0, device=dev)
    cases = []
    for shape, dt in (((32, 14, 14, 256), torch.float16), ((32, 14, 14, 256), torch.float16),
                      ((16, 7, 7, 512), torch.bfloat16), ((64, 28, 28, 64), torch.float32),
                      ((8, 7, 7, 2048), torch.float16)):
        c = shape[-1]
        cases.append((torch.randn(shape, device=dev).to(dt), torch.randn(shape, device=dev).to(dt),
                      torch.rand(c, device=dev) + 0.5, 0.1 * torch.randn(c, device=dev)))

    def step(x, dy, scale, offset):
        f = ops.FusedBatchNormV3(x, scale, offset, e, e, epsilon=eps)
        g = ops.FusedBatchNormGradV3(dy, x, scale, f.reserve_space_1, f.reserve_space_2,
                                     f.reserve_space_3, epsilon=eps)
        assert ops.last_kernel_name() == "tfma_bn_grad_fused"
        return [f.y, f.batch_mean, f.batch_variance, g.x_backprop, g.scale_backprop,
                g.offset_backprop]

    ops.fused_batch_norm_barrier_timed_out(reset=True)
    want = []
    for cs in cases:
        want.append([t.clone() for t in step(*cs)])
        torch.cuda.synchronize()
    order = [0, 1, 0, 2, 3, 1, 4, 4, 0, 2, 1, 3]
    got = [(k, step(*cases[k])) for k in order]
    torch.cuda.synchronize()
    assert not ops.fused_batch_norm_barrier_timed_out()
    for k, outs in got:
        for w, g in zip(want[k], outs):
            assert torch.equal(w, g)


_WRAP_SCRIPT = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
import tensorflow_musa_extension_amd as tfma
ops = tfma.raw_ops
dev = torch.device("cuda:0")
torch.manual_seed(6)
x = torch.randn(16, 14, 14, 256, device=dev).half()
dy = torch.randn_like(x)
scale = torch.rand(256, device=dev) + 0.5
offset = 0.1 * torch.randn(256, device=dev)
e = torch.empty(0, device=dev)
outs = []
for i in range(6):
    f = ops.FusedBatchNormV3(x, scale, offset, e, e, epsilon=1e-3)
    g = ops.FusedBatchNormGradV3(dy, x, scale, f.reserve_space_1, f.reserve_space_2,
                                 f.reserve_space_3, epsilon=1e-3)
    assert ops.last_kernel_name() == "tfma_bn_grad_fused"
    outs.append([t.clone() for t in (f.y, f.batch_mean, f.batch_variance, g.x_backprop,
                                     g.scale_backprop, g.offset_backprop)])
torch.cuda.synchronize()
assert not ops.fused_batch_norm_barrier_timed_out()
for o in outs[1:]:
    for a, b in zip(outs[0], o):
        assert torch.equal(a, b)
print("wrap ok")
"""


def test_fused_epoch_wrap(tmp_path):
    """The eager epoch counter wraps below 2^31: the library zeroes its
    epoch-tagged regions and starts again at 1.  A fresh process whose counter
    starts 3 below the wrap (TFMA_BN_EPOCH_START) runs 12 fused launches across
    it; every forward and grad must equal the first bit for bit."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    script = tmp_path / "wrap.py"
    script.write_text(_WRAP_SCRIPT)
    env = dict(os.environ, TFMA_BN_EPOCH_START=str(2**31 - 4))
    r = subprocess.run([sys.executable, str(script), root], env=env, capture_output=True,
                       text=True, timeout=240)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "wrap ok" in r.stdout


_GIVE_UP_SCRIPT = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
import tensorflow_musa_extension_amd as tfma
ops = tfma.raw_ops
dev = torch.device("cuda:0")
torch.manual_seed(8)
x = torch.randn(16, 14, 14, 256, device=dev).half()
dy = torch.randn_like(x)
scale = torch.rand(256, device=dev) + 0.5
offset = 0.1 * torch.randn(256, device=dev)
e = torch.empty(0, device=dev)

def fwd():
    return ops.FusedBatchNormV3(x, scale, offset, e, e, epsilon=1e-3)

def expect_internal(fn, what):
    try:
        fn()
    except tfma.InternalError as err:
        assert "gave up waiting" in str(err), str(err)
        print(what, "InternalError:", str(err)[:80], flush=True)
        return
    raise AssertionError(what + ": no InternalError")

f = fwd()
assert ops.last_kernel_name() == "tfma_bn_fwd_fused"
torch.cuda.synchronize()
assert torch.isnan(f.y.float()).all() and torch.isnan(f.batch_mean).all()
assert torch.isnan(f.batch_variance).all()
# The launch that gave up is reported once, by the next call, which does not launch.
expect_internal(fwd, "forward after forward")
f2 = fwd()  # reported already: this one launches (and gives up again)
torch.cuda.synchronize()
assert ops.fused_batch_norm_barrier_timed_out()
expect_internal(lambda: ops.FusedBatchNormGradV3(dy, x, scale, f2.reserve_space_1,
                                                  f2.reserve_space_2, f2.reserve_space_3,
                                                  epsilon=1e-3), "grad after forward")
assert ops.fused_batch_norm_barrier_timed_out(reset=True)
assert not ops.fused_batch_norm_barrier_timed_out()
g = ops.FusedBatchNormGradV3(dy, x, scale, f.reserve_space_1, f.reserve_space_2,
                             f.reserve_space_3, epsilon=1e-3)
assert ops.last_kernel_name() == "tfma_bn_grad_fused"
torch.cuda.synchronize()
assert torch.isnan(g.x_backprop.float()).all() and torch.isnan(g.scale_backprop).all()
expect_internal(fwd, "forward after grad")
# A sliced gradient (forced: 4 slices of 64 channels, two waits per slice)
# gives up the same way.
ops.set_tuning_override("bn_slice_tw", 8)
gs = ops.FusedBatchNormGradV3(dy, x, scale, f.reserve_space_1, f.reserve_space_2,
                              f.reserve_space_3, epsilon=1e-3)
assert ops.fused_batch_norm_last_plan()["slices"] == 4
torch.cuda.synchronize()
assert torch.isnan(gs.x_backprop.float()).all() and torch.isnan(gs.scale_backprop).all()
expect_internal(fwd, "forward after sliced grad")
print("give-up ok", flush=True)
"""


def test_fused_give_up_is_an_error(tmp_path):
    """A fused launch whose grid-wide wait gives up (forced from the host:
    TFMA_BN_FORCE_GIVE_UP makes every eager fused launch wait, with a short
    spin limit, for an epoch no launch publishes - every kernel still exits
    normally) writes NaN statistics and outputs, and the next FusedBatchNorm
    call on the device raises InternalError without launching, once per such
    launch; the diagnostic reports it until reset.  Fresh process, since the
    hook is read once."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    script = tmp_path / "give_up.py"
    script.write_text(_GIVE_UP_SCRIPT)
    env = dict(os.environ, TFMA_BN_FORCE_GIVE_UP="1")
    r = subprocess.run([sys.executable, str(script), root], env=env, capture_output=True,
                       text=True, timeout=240)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "give-up ok" in r.stdout
