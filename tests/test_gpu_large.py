"""Maximum sizes: every op on tensors of more than 2^31 elements, where a
32-bit flat index would wrap.  The outputs are checked at sampled positions -
the first and last rows, both sides of every internal 2^31-element chunk
boundary, and random windows - against the oracle (elementwise ops and Adam are
per element, so a sample is a complete input for them), and through
size-independent properties where the op reduces over the whole tensor
(BatchNorm statistics against float64 sums taken on the device in chunks;
BiasAddGrad against the oracle on the full tensor).  Each test needs 9-35 GB
of device memory (and the BiasAddGrad check 4.3 GB of host memory) and
skips when the device has less free.
"""
import numpy as np
import pytest
import torch

import tensorflow_musa_extension_amd as tfma
from oracle import oracle
from tests.helpers import (assert_bitwise, assert_close, bn_fwd_ref32, bn_grad_ref32,
                           bn_max_ulp, bn_scale_backprop_ref64, to_np)

pytestmark = pytest.mark.gpu
ops = tfma.raw_ops
BIG = 2**31


def _need(gb):
    free, _ = torch.cuda.mem_get_info()
    if free < gb * 2**30:
        pytest.skip(f"needs {gb} GiB of free device memory, {free / 2**30:.0f} GiB free")


@pytest.fixture(autouse=True)
def _release():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _window_starts(total, width, boundaries, rng, n_random):
    """Starts of `width`-long windows: both ends, centred on each boundary,
    and n_random random ones."""
    starts = {0, total - width}
    starts.update(b - width // 2 for b in boundaries)
    starts.update(int(r) for r in rng.integers(0, total - width, n_random))
    return sorted(min(max(st, 0), total - width) for st in starts)


def _take(t, starts, width, dtype):
    """The windows t[s:s+width] along dim 0, copied to the host one slice at
    a time (contiguous copies; torch's gather kernel computes 32-bit offsets
    and faults on tensors of more than 2^31 elements)."""
    return np.concatenate([to_np(t[st:st + width], dtype) for st in starts])


def test_bias_add_relu_f16_over_2_31(dev):
    """[524291, 4096] f16 = 2,147,495,936 elements: the flat launches run in
    chunks of 524287 rows (the largest multiple of the 4096-element bias
    period below 2^31), so rows 524286-524288 straddle a chunk start."""
    _need(10)
    rows, c = 524291, 4096
    assert rows * c > BIG
    torch.manual_seed(11)
    x = torch.randn(rows, c, device=dev, dtype=torch.float16)
    b = torch.randn(c, device=dev, dtype=torch.float16)
    y = ops.MusaBiasAddRelu(x, b)
    assert ops.last_kernel_name() == "tfma_ew_add_relu"  # the flat path, not the strided one
    rng = np.random.default_rng(1)
    starts = _window_starts(rows, 4, [(BIG - 1) // c], rng, 32)
    got = _take(y, starts, 4, "float16")
    ref = oracle.bias_add(_take(x, starts, 4, "float16"), to_np(b, "float16"),
                          relu=True, dtype="float16")
    assert_bitwise(got, ref, "MusaBiasAddRelu f16 > 2^31")


def test_mul_add_full_f16_over_2_31(dev):
    """x*a+b with three full 1-D operands of 2^31 + 67 elements (chunks of
    2^31 - 16, then an 83-element tail that is not a whole number of
    vectors)."""
    _need(18)
    n = BIG + 67
    torch.manual_seed(12)
    x = torch.randn(n, device=dev, dtype=torch.float16)
    a = torch.randn(n, device=dev, dtype=torch.float16)
    b = torch.randn(n, device=dev, dtype=torch.float16)
    y = ops.MusaShiftedAffineMap(x, a, b)
    assert ops.last_kernel_name() == "tfma_ew_mul_add"
    rng = np.random.default_rng(2)
    chunk = (BIG - 1) // 16 * 16
    starts = _window_starts(n, 1024, [chunk], rng, 16)
    pick = lambda t: _take(t, starts, 1024, "float16")
    ref = oracle.eltwise("mul_add", [pick(x), pick(a), pick(b)], "float16")
    assert_bitwise(pick(y), ref, "MusaShiftedAffineMap f16 > 2^31")


def test_adam_f32_over_2_31(dev):
    """ResourceApplyAdam over 2^31 + 4099 float32 elements (262145 chunks of
    8192 plus a partial one): sampled elements bit-identical to the oracle."""
    _need(36)
    n = BIG + 4099
    torch.manual_seed(13)
    var = torch.randn(n, device=dev).mul_(0.02)
    m = torch.zeros(n, device=dev)
    v = torch.zeros(n, device=dev)
    g = torch.randn(n, device=dev).mul_(1e-3)
    rng = np.random.default_rng(3)
    starts = _window_starts(n, 8192, [BIG, n - 4099], rng, 16)
    pick = lambda t: _take(t, starts, 8192, "float32")
    v0, m0, vv0, g0 = pick(var), pick(m), pick(v), pick(g)
    scal = dict(beta1_power=0.9, beta2_power=0.999, lr=1e-3, beta1=0.9, beta2=0.999,
                epsilon=1e-7)
    ops.ResourceApplyAdam(var, m, v, grad=g, **scal)
    oracle.adam(v0, m0, vv0, g0, 0.9, 0.999, 1e-3, 0.9, 0.999, 1e-7)
    assert_bitwise(pick(var), v0, "var")
    assert_bitwise(pick(m), m0, "m")
    assert_bitwise(pick(v), vv0, "v")


def _chunked_sums(t, c, fn, rows_per=1 << 20):
    acc = torch.zeros(c, dtype=torch.float64, device=t.device)
    flat = t.view(-1, c)
    for r in range(0, flat.shape[0], rows_per):
        acc += fn(flat[r:r + rows_per].double()).sum(0)
    return acc


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_batch_norm_over_2_31(dev, dtype):
    """FusedBatchNormV3 + GradV3 on [1, 8388640, 1, 256] f16 and bf16
    (2,147,491,840 elements; the forward's fused kernel has 2048 rows per
    thread, the gradient runs in 4 slices of 64 channels with 512 rows per
    thread per slice, and both hand phase-3 rows out dynamically).  Statistics against float64 sums
    taken on the device in chunks (mean 1e-5 absolute; variance 5e-5
    relative - each thread sums 2048 rows in float32 before the float64
    combine; sum(dy) and rsqrt(var+eps) * sum(dy*(x-mean)) 1e-5 relative +
    5e-2).  Every element of y and dx within 1 ulp of the float32 closed form
    evaluated from the kernel's own statistics in the kernel's operation
    order (the coefficients can differ in their last float32 bit, which moves
    a rounding tie by one ulp; differences within 1e-6, the float32 precision
    of the terms whose difference forms y and dx, are not counted)."""
    _need(24)
    c, rows = 256, 8388640
    shape = (1, rows, 1, c)
    assert rows * c > BIG
    torch.manual_seed(14)
    x = torch.randn(shape, device=dev, dtype=dtype).add_(0.5)
    dy = torch.randn(shape, device=dev, dtype=dtype)
    scale = torch.rand(c, device=dev) + 0.5
    offset = 0.1 * torch.randn(c, device=dev)
    e = torch.empty(0, device=dev)
    eps = 1.001e-5
    f = ops.FusedBatchNormV3(x, scale, offset, e, e, epsilon=eps)
    assert ops.last_kernel_name() == "tfma_bn_fwd_fused"
    s1 = _chunked_sums(x, c, lambda a: a)
    s2 = _chunked_sums(x, c, lambda a: a * a)
    mean = s1 / rows
    var = s2 / rows - mean * mean
    assert torch.allclose(f.reserve_space_1.double(), mean, rtol=0, atol=1e-5)
    assert torch.allclose(f.reserve_space_2.double(), var, rtol=5e-5, atol=0)
    assert torch.allclose(f.batch_variance.double(), var * rows / (rows - 1), rtol=5e-5, atol=0)
    mu, sig = f.reserve_space_1, f.reserve_space_2
    assert bn_max_ulp(f.y, bn_fwd_ref32(x, mu, sig, scale, offset, eps, rows, c), rows, c) <= 1

    g = ops.FusedBatchNormGradV3(dy, x, scale, mu, sig, f.reserve_space_3, epsilon=eps)
    assert ops.last_kernel_name() == "tfma_bn_grad_fused"
    plan = ops.fused_batch_norm_last_plan()
    assert plan["slices"] == 4 and plan["dynamic_rows"] > 0, plan
    sdy = _chunked_sums(dy, c, lambda a: a)
    assert torch.allclose(g.offset_backprop.double(), sdy, rtol=1e-5, atol=5e-2)
    sbp = bn_scale_backprop_ref64(dy, x, mu, sig, eps, rows, c)
    assert torch.allclose(g.scale_backprop.double(), sbp, rtol=1e-5, atol=5e-2)
    ref = bn_grad_ref32(dy, x, scale, mu, sig, g.offset_backprop, g.scale_backprop, eps, rows, c)
    assert bn_max_ulp(g.x_backprop, ref, rows, c) <= 1


def test_bias_add_grad_f16_over_2_31(dev):
    """BiasAddGrad over [524291, 4096] f16 against the oracle's float64 sums
    of the whole tensor (f16 bar 1e-2 of max|ref|)."""
    _need(10)
    rows, c = 524291, 4096
    torch.manual_seed(15)
    x = torch.randn(rows, c, device=dev, dtype=torch.float16)
    out = ops.BiasAddGrad(x)
    got = to_np(out, "float16")
    ref = oracle.bias_add_grad(to_np(x, "float16"), "NHWC", "float16")
    assert_close(got, ref, "float16", 1e-2, "BiasAddGrad f16 > 2^31")


@pytest.mark.parametrize("rows,kernel", [(15000, "fused"), (16384, "apply")])
def test_batch_norm_wide_channels_group_span(dev, rows, kernel):
    """FusedBatchNormV3 + GradV3 on [1, rows, 1, 65536] f16: 256 channel
    tiles, so one row group of all rows per tile.  The fused kernel reads a
    workgroup's rows through a buffer resource with 32-bit byte offsets; at
    15000 rows the largest offset is ~2.0e9 (just below 2^31) and the fused
    path runs, at 16384 rows the group's span reaches 2^31 bytes and the op
    must take the split path instead.  Both: statistics against float64 sums
    and every element of y and dx within 1 ulp (or 1e-6) of the float32 closed
    form from the kernel's own statistics (tolerances as in the 2^31-element
    test)."""
    _need(16)
    c = 65536
    shape = (1, rows, 1, c)
    torch.manual_seed(15)
    x = torch.randn(shape, device=dev, dtype=torch.float16).add_(0.5)
    dy = torch.randn(shape, device=dev, dtype=torch.float16)
    scale = torch.rand(c, device=dev) + 0.5
    offset = 0.1 * torch.randn(c, device=dev)
    e = torch.empty(0, device=dev)
    eps = 1.001e-5
    f = ops.FusedBatchNormV3(x, scale, offset, e, e, epsilon=eps)
    assert ops.last_kernel_name() == f"tfma_bn_fwd_{kernel}"
    s1 = _chunked_sums(x, c, lambda a: a, rows_per=1024)
    s2 = _chunked_sums(x, c, lambda a: a * a, rows_per=1024)
    mean = s1 / rows
    var = s2 / rows - mean * mean
    assert torch.allclose(f.reserve_space_1.double(), mean, rtol=0, atol=1e-5)
    assert torch.allclose(f.reserve_space_2.double(), var, rtol=5e-5, atol=0)
    mu, sig = f.reserve_space_1, f.reserve_space_2
    assert bn_max_ulp(f.y, bn_fwd_ref32(x, mu, sig, scale, offset, eps, rows, c), rows, c,
                      rows_per=2048) <= 1
    g = ops.FusedBatchNormGradV3(dy, x, scale, mu, sig, f.reserve_space_3, epsilon=eps)
    assert ops.last_kernel_name() == f"tfma_bn_grad_{kernel}"
    sdy = _chunked_sums(dy, c, lambda a: a, rows_per=1024)
    assert torch.allclose(g.offset_backprop.double(), sdy, rtol=1e-5, atol=5e-2)
    sbp = bn_scale_backprop_ref64(dy, x, mu, sig, eps, rows, c, rows_per=1024)
    assert torch.allclose(g.scale_backprop.double(), sbp, rtol=1e-5, atol=5e-2)
    ref = bn_grad_ref32(dy, x, scale, mu, sig, g.offset_backprop, g.scale_backprop, eps, rows, c)
    assert bn_max_ulp(g.x_backprop, ref, rows, c, rows_per=2048) <= 1
