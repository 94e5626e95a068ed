"""BiasAddGrad on the GPU vs the TF-CPU oracle (float64 sums rounded once).
Bars: float32 1e-5 and float16/bfloat16 1e-2 of max|ref| (the BN bars; TF
itself sums in float in Eigen's order), float64 1e-12, integers exact
(wrapping).  Shapes: the reference's own test cases
(test/ops/biasadd_grad_op_test.py:16-127: [2,8,8,32] NHWC, [2,32,8,8] NCHW,
empty inputs), the cfg4 shape, odd widths and the rank-1 identity."""
import numpy as np
import pytest
import torch

import tensorflow_musa_extension_amd as tfma
from oracle import oracle
from tests.helpers import assert_bitwise, assert_close, gen, to_dev, to_np

pytestmark = pytest.mark.gpu
ops = tfma.raw_ops
TOL = {"float32": 1e-5, "float16": 1e-2, "bfloat16": 1e-2}

CASES = [((2, 8, 8, 32), "NHWC"), ((2, 32, 8, 8), "NCHW"), ((8192, 4096), "NHWC"),
         ((8191, 4095), "NHWC"), ((256, 7, 7, 2048), "NHWC"), ((4, 16, 7, 7), "NCHW"),
         ((3, 5, 2, 3, 4), "NCHW"), ((1, 3), "NHWC"), ((100000, 3), "NHWC"), ((64, 2, 1000), "NCHW"),
         # very wide channel dimensions (4.2M channels of rows; 20000 NCHW planes)
         ((2, 4200000), "NHWC"), ((2, 20000, 3), "NCHW")]


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("shape,fmt", CASES)
def test_bias_add_grad(dev, dtype, shape, fmt):
    rng = np.random.default_rng(hash((shape, fmt)) % 2**32)
    x = gen(rng, shape, dtype)
    out = ops.BiasAddGrad(to_dev(x, dtype, dev), data_format=fmt)
    torch.cuda.synchronize()
    ref = oracle.bias_add_grad(x, fmt, dtype)
    assert_close(to_np(out, dtype), ref, dtype, TOL[dtype], f"{dtype} {shape} {fmt}")


def test_bias_add_grad_deterministic(dev):
    x = torch.randn(4096, 1024, device=dev)
    a = ops.BiasAddGrad(x)
    b = ops.BiasAddGrad(x)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_bias_add_grad_float64_and_integers(dev):
    rng = np.random.default_rng(8)
    x = rng.standard_normal((513, 77))
    out = ops.BiasAddGrad(torch.from_numpy(x).to(dev))
    torch.cuda.synchronize()
    assert np.max(np.abs(out.cpu().numpy() - oracle.bias_add_grad(x, "NHWC", "float64"))) < 1e-12 * 513
    xi = rng.integers(-2**31, 2**31, size=(1000, 33), dtype=np.int64).astype(np.int32)
    oi = ops.BiasAddGrad(torch.from_numpy(xi).to(dev))
    x64 = rng.integers(-2**62, 2**62, size=(20, 5, 9), dtype=np.int64)
    o64 = ops.BiasAddGrad(torch.from_numpy(x64).to(dev), data_format="NCHW")
    torch.cuda.synchronize()
    assert_bitwise(oi.cpu().numpy(), oracle.bias_add_grad(xi, "NHWC", "int32"), "int32")
    assert_bitwise(o64.cpu().numpy(), oracle.bias_add_grad(x64, "NCHW", "int64"), "int64")


@pytest.mark.parametrize("shape", [(4096, 0, 512), (0, 16), (3, 0, 4)])
def test_bias_add_grad_empty_gives_zeros(dev, shape):
    """The reference's empty-input case (biasadd_grad_op_test.py:88-127)."""
    for dt in (torch.float32, torch.float16, torch.bfloat16):
        out = ops.BiasAddGrad(torch.zeros(shape, dtype=dt, device=dev))
        out2 = torch.full_like(out, 7)
        ops.BiasAddGrad(torch.zeros(shape, dtype=dt, device=dev), out=out2)
        torch.cuda.synchronize()
        assert out2.shape == (shape[-1],) and not out2.float().abs().sum().item()


def test_bias_add_grad_rank1_is_identity(dev):
    x = torch.randn(37, device=dev)
    out = ops.BiasAddGrad(x)
    torch.cuda.synchronize()
    assert torch.equal(out, x)


def test_bias_add_grad_unaligned_view(dev):
    base = torch.randn(1000 * 64 + 1, device=dev)
    x = base[1:].view(1000, 64)  # not 16-byte aligned: scalar path
    out = ops.BiasAddGrad(x)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), oracle.bias_add_grad(x.cpu().numpy(), "NHWC", "float32"),
                 "float32", 1e-5, "unaligned")


def test_bias_add_grad_two_streams(dev):
    """Forty calls alternating between two streams, each with its own input
    and workspace: every result matches its run on one stream bit for bit."""
    xs = [torch.randn(2048 + 64 * k, 1024, device=dev).half() for k in range(40)]
    want = [ops.BiasAddGrad(x) for x in xs]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)
    for s in (s1, s2):
        s.wait_stream(torch.cuda.current_stream(dev))
    got = []
    for k, x in enumerate(xs):
        with torch.cuda.stream(s1 if k % 2 else s2):
            got.append(ops.BiasAddGrad(x))
    torch.cuda.synchronize()
    for k, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), k


def test_bias_add_grad_captured_equals_eager(dev):
    """Recorded into a graph (stream capture), BiasAddGrad's replays give the
    eager bits, with eager calls between the replays."""
    x = torch.randn(4096, 2048, device=dev).half()
    eager = ops.BiasAddGrad(x)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ops.BiasAddGrad(x)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16))
        again = ops.BiasAddGrad(x)
        torch.cuda.synchronize()
        assert torch.equal(again.view(torch.int16), eager.view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape,fmt", CASES)
def test_one_launch_equals_two_kernels(dev, tune, dtype, shape, fmt):
    """The one-launch form (tagged partials, finalizing workgroups at the end
    of the same grid) against the two-kernel form (override bag_fused 0):
    same plan, partials and summation order, so the same bits - including
    the shapes whose partials exceed the tagged slots and fall back."""
    gen_ = torch.Generator(device=dev)
    gen_.manual_seed(31)
    x = torch.randn(shape, generator=gen_, device=dev).to(dtype)
    one = ops.BiasAddGrad(x, data_format=fmt)
    name_one = ops.last_kernel_name()
    tune("bag_fused", 0)
    two = ops.BiasAddGrad(x, data_format=fmt)
    assert ops.last_kernel_name() == "tfma_bias_add_grad_finalize"
    torch.cuda.synchronize()
    assert name_one in ("tfma_bias_add_grad_fused", "tfma_bias_add_grad_finalize")
    if shape == (8192, 4096):
        assert name_one == "tfma_bias_add_grad_fused"
    assert torch.equal(one.view(torch.int16 if dtype != torch.float32 else torch.int32),
                       two.view(torch.int16 if dtype != torch.float32 else torch.int32))


def test_one_launch_calls_on_two_streams(dev):
    """One-launch calls alternating between two streams with no
    synchronization between them share the library's tagged slots: each is
    chained to the previous one, so every result equals the same call run
    alone, bit for bit."""
    gen_ = torch.Generator(device=dev)
    gen_.manual_seed(32)
    shapes = [(8192, 4096), (96, 40), (2048, 1024), (33, 7, 7, 64)] * 3
    xs = [torch.randn(s, generator=gen_, device=dev).half() for s in shapes]
    wants = [ops.BiasAddGrad(x) for x in xs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = []
    for i, x in enumerate(xs):
        with torch.cuda.stream(streams[i % 2]):
            outs.append(ops.BiasAddGrad(x))
    torch.cuda.synchronize()
    for i, (o, w) in enumerate(zip(outs, wants)):
        assert torch.equal(o.view(torch.int16), w.view(torch.int16)), f"call {i} {shapes[i]}"
