"""Elementwise ops and fused chains on the GPU vs the TF-CPU oracle.  Bar:
bitwise equality (each fused chain rounds exactly where the unfused TF ops
do)."""
import numpy as np
import pytest
import torch

import tensorflow_musa_extension_amd as tfma
from oracle import oracle
from tests.helpers import assert_bitwise, gen, to_dev, to_np

pytestmark = pytest.mark.gpu
ops = tfma.raw_ops
DTYPES = ["float32", "float16", "bfloat16"]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(8192, 4096), (8191, 4095), (3, 5), (1, 1), (7, 9, 33),
                                   # the reference's shapes (test/ops/biasadd_op_test.py:74-116)
                                   (10, 5), (2, 3, 4, 5), (2, 3, 4), (100, 50)])
@pytest.mark.parametrize("relu", [False, True])
def test_bias_add_nhwc(dev, dtype, shape, relu):
    rng = np.random.default_rng(1)
    x = gen(rng, shape, dtype)
    b = gen(rng, shape[-1:], dtype)
    fn = ops.MusaBiasAddRelu if relu else ops.BiasAdd
    out = fn(to_dev(x, dtype, dev), to_dev(b, dtype, dev))
    torch.cuda.synchronize()
    assert_bitwise(to_np(out, dtype), oracle.bias_add(x, b, relu=relu, dtype=dtype), "bias_add")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(4, 16, 7, 7), (2, 3, 5, 8), (2, 5, 3),
                                   (2, 5, 3, 4)])   # biasadd_op_test.py:88-91
@pytest.mark.parametrize("relu", [False, True])
def test_bias_add_nchw(dev, dtype, shape, relu):
    rng = np.random.default_rng(2)
    x = gen(rng, shape, dtype)
    b = gen(rng, shape[1:2], dtype)
    fn = ops.MusaBiasAddRelu if relu else ops.BiasAdd
    out = fn(to_dev(x, dtype, dev), to_dev(b, dtype, dev), data_format="NCHW")
    torch.cuda.synchronize()
    ref = oracle.bias_add(x, b, data_format="NCHW", relu=relu, dtype=dtype)
    assert_bitwise(to_np(out, dtype), ref, "bias_add nchw")


BCAST = [
    ((8192, 4096), (4096,)),        # cfg4 row broadcast
    ((8191, 4095), (4095,)),        # odd tail
    ((8192, 4096), (8192, 4096)),   # full
    ((4096,), (8192, 4096)),        # broadcast operand first
    ((64, 33), ()),                 # scalar
    ((64, 33), (64, 1)),            # column broadcast (inner > 1)
    ((37, 3), (3,)),                # period shorter than a vector: wraps inside it
    ((9, 7, 11), (7, 1)),           # inner 11, period 7: incremental walk
    ((5, 1021), (1021,)),           # odd period, wrap in a few vectors
    ((3, 8191), (8191,)),           # odd period longer than the staged copies hold: global walk
    ((3, 9001), (9001,)),           # longer odd period, few vectors: global walk
    ((2048, 33), (33,)),            # short odd period, staged shifted copies
    ((221, 37), (37,)),             # f32: 2044 vectors, just below the staging minimum
    ((222, 37), (37,)),             # f32: 2053 vectors, staged by a single workgroup
    ((8192, 3), (3,)),              # period shorter than a vector, staged
    ((9000, 3), (9000, 1)),         # inner 3, long period: global walk
    ((64, 37, 33), (37, 1)),        # inner 33, period 37: staged walk
    ((4, 1, 5), (1, 3, 1)),         # neither operand full: strided path
    ((2, 3, 4, 8), (3, 1, 8)),      # two broadcast runs: strided path
    ((0, 4), (4,)),                 # empty
    # the reference's hot shapes (test/ops/add_op_test.py:80-107,
    # multiply_op_test.py:114-126)
    ((7, 48), (48,)),
    ((5, 64), (64,)),
    ((3, 768), (1, 768)),
    ((2, 8, 160), (160,)),
    ((), (64,)),
    ((1024, 1024), (1024, 1024)),
    ((1024, 1024), ()),
    ((1024, 1024), (1024,)),
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("xs,ys", BCAST)
@pytest.mark.parametrize("op", ["add", "add_relu", "mul"])
def test_binary_broadcast(dev, dtype, xs, ys, op):
    rng = np.random.default_rng(3)
    x = gen(rng, xs, dtype)
    y = gen(rng, ys, dtype)
    fn = {"add": ops.AddV2, "add_relu": ops.MusaAddV2Relu, "mul": ops.Mul}[op]
    out = fn(to_dev(x, dtype, dev), to_dev(y, dtype, dev))
    torch.cuda.synchronize()
    assert_bitwise(to_np(out, dtype), oracle.eltwise(op, [x, y], dtype), op)


INT_DTYPES = ["int32", "int64", "uint8"]
# cfg4's shapes, and a broadcast case of every operand kind per dtype (row,
# odd row period staged in LDS, inner-extent walk, scalar, strided).
INT_BCAST = [
    ((8192, 4096), (4096,)),
    ((8192, 4096), (8192, 4096)),
    ((8191, 4095), (4095,)),
    ((8191, 4095), (8191, 4095)),
    ((2048, 33), (33,)),
    ((64, 37, 33), (37, 1)),
    ((64, 33), ()),
    ((4, 1, 5), (1, 3, 1)),
    ((3, 9001), (9001,)),
    ((0, 4), (4,)),
    ((1024, 1024), ()),             # the reference's Mul hot shapes with int32 / int64
    ((1024, 1024), (1024,)),
]


@pytest.mark.parametrize("dtype", INT_DTYPES)
@pytest.mark.parametrize("xs,ys", INT_BCAST)
def test_integer_add_mul(dev, dtype, xs, ys):
    """The reference's integer registrations of AddV2 / Add (int32, int64,
    uint8) and Mul (int32, int64): wrapping arithmetic, bitwise against the
    oracle over the types' whole range."""
    rng = np.random.default_rng(8)
    x, y = gen(rng, xs, dtype), gen(rng, ys, dtype)
    xd, yd = to_dev(x, dtype, dev), to_dev(y, dtype, dev)
    for name, fn, op in (("AddV2", ops.AddV2, "add"), ("Add", ops.Add, "add"),
                         ("Mul", ops.Mul, "mul")):
        if op == "mul" and dtype == "uint8":
            with pytest.raises(tfma.UnimplementedError):
                ops.Mul(xd, yd)
            continue
        out = fn(xd, yd)
        torch.cuda.synchronize()
        assert_bitwise(to_np(out, dtype), oracle.eltwise(op, [x, y], dtype), name)


@pytest.mark.parametrize("dtype", ["int32", "int64"])
@pytest.mark.parametrize("shape,fmt", [((8192, 4096), "NHWC"), ((8191, 4095), "NHWC"),
                                       ((4, 16, 7, 7), "NCHW"), ((2, 5, 3), "NCHW"),
                                       ((5, 3), "NHWC")])   # biasadd_op_test.py:98-111
def test_integer_bias_add(dev, dtype, shape, fmt):
    """BiasAdd / BiasAddV1 for int32 and int64 (musa_biasadd_op.cc:67-79)."""
    rng = np.random.default_rng(9)
    x = gen(rng, shape, dtype)
    b = gen(rng, shape[1:2] if fmt == "NCHW" else shape[-1:], dtype)
    xd, bd = to_dev(x, dtype, dev), to_dev(b, dtype, dev)
    out = ops.BiasAdd(xd, bd, data_format=fmt)
    torch.cuda.synchronize()
    ref = oracle.bias_add(x, b, data_format=fmt, dtype=dtype)
    assert_bitwise(to_np(out, dtype), ref, "BiasAdd")
    if fmt == "NHWC":
        assert_bitwise(to_np(ops.BiasAddV1(xd, bd), dtype), ref, "BiasAddV1")
    with pytest.raises(tfma.UnimplementedError):
        ops.MusaBiasAddRelu(xd, bd, data_format=fmt)


def test_uint8_bias_add_is_unregistered(dev):
    x = torch.zeros(4, 8, dtype=torch.uint8, device=dev)
    with pytest.raises(tfma.UnimplementedError):
        ops.BiasAdd(x, torch.zeros(8, dtype=torch.uint8, device=dev))


MULADD = [
    ((8192, 4096), (8192, 4096), (8192, 4096)),   # a, b full
    ((8192, 4096), (4096,), (4096,)),             # a, b row broadcast
    ((8191, 4095), (8191, 4095), (8191, 4095)),
    ((8191, 4095), (4095,), (4095,)),
    ((5, 7), (5, 7), ()),
    ((5, 1, 7), (1, 3, 1), (3, 7)),               # strided path
    ((1024, 1021), (1021,), (1021,)),             # two staged odd-period operands
    # the reference's cases (test/ops/shifted_affine_map_op_test.py:53-152)
    ((2, 4, 8), (2, 4, 8), (8,)),
    ((2, 1, 4, 8), (2, 3, 1, 8), (1, 3, 4, 1)),   # rank expansion, multi-axis broadcast
    ((0, 8), (0, 8), (8,)),                       # empty
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("xs,as_,bs", MULADD)
def test_mul_add(dev, dtype, xs, as_, bs):
    rng = np.random.default_rng(4)
    x, a, b = gen(rng, xs, dtype), gen(rng, as_, dtype), gen(rng, bs, dtype)
    out = ops.MusaShiftedAffineMap(to_dev(x, dtype, dev), to_dev(a, dtype, dev),
                                   to_dev(b, dtype, dev))
    torch.cuda.synchronize()
    assert_bitwise(to_np(out, dtype), oracle.eltwise("mul_add", [x, a, b], dtype), "mul_add")


def test_relu_known_answers(dev):
    """The reference's Relu literal (test/ops/relu_op_test.py:45-96) plus
    -0 and NaN, which keep their bits as with Eigen's max."""
    x = torch.tensor([-2.0, -1.0, 0.0, 1.0, 2.0, -0.0, float("nan"), float("-inf")], device=dev)
    y = ops.Relu(x).cpu()
    want = torch.tensor([0.0, 0.0, 0.0, 1.0, 2.0, -0.0, float("nan"), 0.0])
    assert torch.equal(y[:6], want[:6])
    assert torch.signbit(y[5]) and torch.isnan(y[6]) and y[7] == 0


@pytest.mark.parametrize("dtype", DTYPES)
def test_relu_large(dev, dtype):
    rng = np.random.default_rng(5)
    x = gen(rng, (4097, 1031), dtype)
    out = ops.Relu(to_dev(x, dtype, dev))
    torch.cuda.synchronize()
    assert_bitwise(to_np(out, dtype), oracle.eltwise("relu", [x], dtype), "relu")


def test_vector_path_is_taken(dev):
    x = torch.randn(8192, 4096, device=dev)
    b = torch.randn(4096, device=dev)
    ops.MusaBiasAddRelu(x, b)
    assert ops.last_kernel_name() == "tfma_ew_add_relu"


def test_errors(dev):
    x = torch.zeros(4, 5, device=dev)
    with pytest.raises(tfma.InvalidArgumentError, match="Dimension mismatch in BiasAdd"):
        ops.BiasAdd(x, torch.zeros(4, device=dev))
    with pytest.raises(tfma.InvalidArgumentError, match="Incompatible shapes for Add"):
        ops.AddV2(x, torch.zeros(3, device=dev))


def _assert_bitwise_nan_aware(got, want, dtype, name):
    """Bitwise, except that NaN payloads may differ (the device's bf16
    conversion keeps payload bits Eigen canonicalises)."""
    nan_w = np.isnan(oracle.to_f32(want, dtype))
    assert np.array_equal(np.isnan(oracle.to_f32(got, dtype)), nan_w), name
    assert_bitwise(got[~nan_w], want[~nan_w], name)


@pytest.mark.parametrize("dtype", DTYPES + ["float64"])
@pytest.mark.parametrize("shape", [(8192, 4096), (8191, 4095), (3, 5), (1,), (0, 7)])
def test_relu_grad(dev, dtype, shape):
    rng = np.random.default_rng(21)
    g = rng.standard_normal(shape)
    f = rng.standard_normal(shape)
    if g.size >= 6:  # NaN / inf gradients, signed zeros, features at 0
        g.ravel()[:6] = [np.nan, np.inf, -np.inf, -2.0, 0.0, -0.0]
        f.ravel()[:6] = [-1.0, 0.0, 1.0, -3.0, 0.0, 5.0]
    if dtype == "float64":
        out = ops.ReluGrad(torch.from_numpy(g).to(dev), torch.from_numpy(f).to(dev))
        torch.cuda.synchronize()
        assert_bitwise(out.cpu().numpy(), g * (f > 0).astype(np.float64), "float64")
        return
    gs, fs = oracle.to_storage(g, dtype), oracle.to_storage(f, dtype)
    out = ops.ReluGrad(to_dev(gs, dtype, dev), to_dev(fs, dtype, dev))
    torch.cuda.synchronize()
    _assert_bitwise_nan_aware(to_np(out, dtype), oracle.eltwise("relu_grad", [gs, fs], dtype),
                              dtype, f"relu_grad {dtype} {shape}")


def test_relu_grad_shape_mismatch(dev):
    a = torch.zeros(4, 3, device=dev)
    with pytest.raises(tfma.InvalidArgumentError,
                       match=r"Inputs to ReluGrad must have the same shape. gradients: \[4,3\], "
                             r"features: \[3,4\]"):
        ops.ReluGrad(a, torch.zeros(3, 4, device=dev))


@pytest.mark.parametrize("dtype", DTYPES)
def test_signed_zero_products(dev, dtype):
    """Products that are -0 stay -0 (TF rounds the float product to T), in the
    vector body and in the tail: Mul, Mul+Add with a -0 addend, ReluGrad."""
    n = 8 * 5 + 5  # vectors and a tail for every dtype's vector width
    x = np.tile([-2.0, 2.0, -0.0, 0.0, -1.5], n // 5)
    y = np.tile([0.0, -0.0, 3.0, -3.0, -0.0], n // 5)
    z = np.full(n, -0.0)
    xs, ys, zs = (oracle.to_storage(a, dtype) for a in (x, y, z))
    dx, dy_, dz = (to_dev(a, dtype, dev) for a in (xs, ys, zs))
    outs = {"mul": ops.Mul(dx, dy_), "mul_add": ops.MusaShiftedAffineMap(dx, dy_, dz),
            "relu_grad": ops.ReluGrad(dx, dy_)}
    torch.cuda.synchronize()
    want = {"mul": oracle.eltwise("mul", [xs, ys], dtype),
            "mul_add": oracle.eltwise("mul_add", [xs, ys, zs], dtype),
            "relu_grad": oracle.eltwise("relu_grad", [xs, ys], dtype)}
    for k, t in outs.items():
        w = want[k]
        assert np.all(np.signbit(oracle.to_f32(w, dtype)[:4]) == [True, True, True, True]) or \
            k == "relu_grad"
        assert_bitwise(to_np(t, dtype), w, f"{dtype} {k}")


def test_multiply_zero_values_and_float64(dev):
    """The reference's testMultiplyZeroValues and testMultiplyFloat64StaysOnMusa
    (test/ops/multiply_op_test.py:99-112, 128-140): literal operands and
    results, the float64 product on the device."""
    x = torch.tensor([[0.0, 1.0], [2.0, 0.0]], device=dev)
    y = torch.tensor([[1.0, 0.0], [0.0, 3.0]], device=dev)
    out = ops.Mul(x, y)
    assert out.device.type == "cuda"
    assert torch.equal(out.cpu(), torch.zeros(2, 2))
    d = ops.Mul(torch.tensor([2.0], dtype=torch.float64, device=dev),
                torch.tensor([3.0], dtype=torch.float64, device=dev))
    assert d.dtype == torch.float64 and d.device.type == "cuda"
    assert float(d.cpu()[0]) == 6.0


F64_CASES = [
    ((2, 3, 4), (2, 1, 4), (4,)),       # shifted_affine_map_op_test.py:121-136
    ((8191, 4095), (4095,), (4095,)),
    ((64, 37, 33), (37, 1), (33,)),
    ((4, 1, 5), (1, 3, 1), (3, 5)),     # strided path
    ((0, 4), (4,), (4,)),
]


@pytest.mark.parametrize("xs,ys,zs", F64_CASES)
def test_float64_binary_and_mul_add(dev, xs, ys, zs):
    """The float64 registrations (AddV2, Mul, MusaAddV2Relu,
    MusaShiftedAffineMap) against numpy's IEEE double arithmetic: every op
    rounds once per TF op (mul_add rounds the product, then the sum), so the
    bar is bitwise."""
    rng = np.random.default_rng(12)
    x, y, z = (rng.standard_normal(s) for s in (xs, ys, zs))
    xd, yd, zd = (torch.from_numpy(a).to(dev) for a in (x, y, z))
    s = x + y
    for name, got, ref in (
            ("AddV2", ops.AddV2(xd, yd), s),
            ("Mul", ops.Mul(xd, yd), x * y),
            ("MusaAddV2Relu", ops.MusaAddV2Relu(xd, yd), np.where(s < 0, 0.0, s)),
            ("MusaShiftedAffineMap", ops.MusaShiftedAffineMap(xd, yd, zd), y * x + z)):
        assert got.dtype == torch.float64
        assert_bitwise(got.cpu().numpy(), ref, name)
