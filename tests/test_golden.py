"""Golden fixtures (tests/golden/golden.npz, written by make_golden.py).

CPU: the oracle reproduces every stored output bit for bit (guards the
checker against regressions).  GPU: the HIP path against the stored outputs,
to the bars of the other parity tests (BN f32 1e-5, f16/bf16 1e-2; Adam and
elementwise bitwise)."""
import os

import numpy as np
import pytest

from oracle import oracle
from tests.helpers import assert_bitwise, assert_close

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")
BN = {"bn_nhwc_f32": ("float32", "NHWC"), "bn_nhwc_f32_c3": ("float32", "NHWC"),
      "bn_nhwc_f16": ("float16", "NHWC"), "bn_nhwc_bf16": ("bfloat16", "NHWC"),
      "bn_nchw_f32": ("float32", "NCHW")}
DTYPES = ("float32", "float16", "bfloat16")


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("name", sorted(BN))
def test_oracle_reproduces_bn(g, name):
    dt, fmt = BN[name]
    p = lambda k: g[f"{name}/{k}"]
    y, bm, bv, sm, sv = oracle.bn_fwd(p("x"), p("scale"), p("offset"), epsilon=1e-3,
                                      data_format=fmt, dtype=dt)
    dx, dsc, dof = oracle.bn_grad(p("dy"), p("x"), p("scale"), sm, sv, epsilon=1e-3,
                                  data_format=fmt, dtype=dt)
    for k, v in dict(y=y, batch_mean=bm, batch_variance=bv, reserve_space_1=sm,
                     reserve_space_2=sv, dx=dx, scale_backprop=dsc, offset_backprop=dof).items():
        assert_bitwise(v, p(k), f"{name}/{k}")


@pytest.mark.parametrize("dt", DTYPES)
def test_oracle_reproduces_adam_and_eltwise(g, dt):
    var = g[f"adam_{dt}/var0"].copy()
    n = var.size
    m = oracle.to_storage(np.zeros(n), dt)
    v = oracle.to_storage(np.zeros(n), dt)
    oracle.adam(var, m, v, g[f"adam_{dt}/grad"], *g[f"adam_{dt}/scalars"], dtype=dt)
    for k, arr in (("var", var), ("m", m), ("v", v)):
        assert_bitwise(arr, g[f"adam_{dt}/{k}"], f"adam {dt} {k}")
    x, bias, a, b = (g[f"ew_{dt}/{k}"] for k in ("x", "bias", "a", "b"))
    assert_bitwise(oracle.bias_add(x, bias, relu=True, dtype=dt), g[f"ew_{dt}/bias_add_relu"])
    assert_bitwise(oracle.eltwise("add_relu", [x, bias], dt), g[f"ew_{dt}/add_v2_relu"])
    assert_bitwise(oracle.eltwise("mul_add", [x, a, b], dt), g[f"ew_{dt}/mul_add"])
    assert_bitwise(oracle.eltwise("relu", [x], dt), g[f"ew_{dt}/relu"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(BN))
def test_gpu_bn_matches_golden(g, dev, name):
    import torch
    import tensorflow_musa_extension_amd as tfma
    from tests.helpers import to_dev, to_np
    ops = tfma.raw_ops
    dt, fmt = BN[name]
    p = lambda k: g[f"{name}/{k}"]
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    e = torch.empty(0, device=dev)
    x = to_dev(p("x"), dt, dev)
    fwd = ops.FusedBatchNormV3(x, f(p("scale")), f(p("offset")), e, e, epsilon=1e-3,
                               data_format=fmt)
    grad = ops.FusedBatchNormGradV3(to_dev(p("dy"), dt, dev), x, f(p("scale")),
                                    fwd.reserve_space_1, fwd.reserve_space_2,
                                    fwd.reserve_space_3, epsilon=1e-3, data_format=fmt)
    torch.cuda.synchronize()
    act = 1e-5 if dt == "float32" else 1e-2
    assert_close(to_np(fwd.y, dt), p("y"), dt, act, "y")
    assert_close(to_np(grad.x_backprop, dt), p("dx"), dt, act, "dx")
    for k, t in (("batch_mean", fwd.batch_mean), ("batch_variance", fwd.batch_variance),
                 ("scale_backprop", grad.scale_backprop),
                 ("offset_backprop", grad.offset_backprop)):
        assert_close(t.cpu().numpy(), p(k), "float32", 1e-5, k)


@pytest.mark.gpu
@pytest.mark.parametrize("dt", DTYPES)
def test_gpu_adam_and_eltwise_match_golden(g, dev, dt):
    import torch
    import tensorflow_musa_extension_amd as tfma
    from tests.helpers import to_dev, to_np
    ops = tfma.raw_ops
    n = g[f"adam_{dt}/var0"].size
    var = to_dev(g[f"adam_{dt}/var0"], dt, dev)
    m = to_dev(oracle.to_storage(np.zeros(n), dt), dt, dev)
    v = to_dev(oracle.to_storage(np.zeros(n), dt), dt, dev)
    ops.ResourceApplyAdam(var, m, v, *g[f"adam_{dt}/scalars"][:6],
                          to_dev(g[f"adam_{dt}/grad"], dt, dev))
    x, bias, a, b = (to_dev(g[f"ew_{dt}/{k}"], dt, dev) for k in ("x", "bias", "a", "b"))
    outs = {"bias_add_relu": ops.MusaBiasAddRelu(x, bias),
            "add_v2_relu": ops.MusaAddV2Relu(x, bias),
            "mul_add": ops.MusaShiftedAffineMap(x, a, b), "relu": ops.Relu(x)}
    torch.cuda.synchronize()
    for k, arr in (("var", var), ("m", m), ("v", v)):
        assert_bitwise(to_np(arr, dt), g[f"adam_{dt}/{k}"], f"adam {dt} {k}")
    for k, t in outs.items():
        assert_bitwise(to_np(t, dt), g[f"ew_{dt}/{k}"], f"{dt} {k}")


def _nan_aware_bitwise(got, want, dtype, name):
    nan_w = np.isnan(oracle.to_f32(want, dtype))
    assert np.array_equal(np.isnan(oracle.to_f32(got, dtype)), nan_w), name
    assert_bitwise(got[~nan_w], want[~nan_w], name)


@pytest.mark.parametrize("dt", DTYPES)
def test_oracle_reproduces_backward_ops(g, dt):
    _nan_aware_bitwise(oracle.eltwise("relu_grad", [g[f"relu_grad_{dt}/g"], g[f"relu_grad_{dt}/f"]],
                                      dt), g[f"relu_grad_{dt}/out"], dt, "relu_grad")
    for fmt in ("NHWC", "NCHW"):
        assert_bitwise(oracle.bias_add_grad(g[f"bias_add_grad_{dt}_{fmt}/x"], fmt, dt),
                       g[f"bias_add_grad_{dt}_{fmt}/out"], f"bias_add_grad {fmt}")


@pytest.mark.parametrize("gdt", ["float16", "bfloat16"])
def test_oracle_reproduces_adam_mixed(g, gdt):
    var = g[f"adam_mixed_{gdt}/var0"].copy()
    m, v = np.zeros_like(var), np.zeros_like(var)
    oracle.adam_mixed(var, m, v, g[f"adam_mixed_{gdt}/grad"], *g[f"adam_mixed_{gdt}/scalars"],
                      grad_dtype=gdt)
    for k, arr in (("var", var), ("m", m), ("v", v)):
        assert_bitwise(arr, g[f"adam_mixed_{gdt}/{k}"], f"adam_mixed {gdt} {k}")


@pytest.mark.gpu
@pytest.mark.parametrize("dt", DTYPES)
def test_gpu_backward_ops_match_golden(g, dev, dt):
    import torch
    import tensorflow_musa_extension_amd as tfma
    from tests.helpers import to_dev, to_np
    ops = tfma.raw_ops
    rg = ops.ReluGrad(to_dev(g[f"relu_grad_{dt}/g"], dt, dev), to_dev(g[f"relu_grad_{dt}/f"], dt, dev))
    outs = {fmt: ops.BiasAddGrad(to_dev(g[f"bias_add_grad_{dt}_{fmt}/x"], dt, dev), data_format=fmt)
            for fmt in ("NHWC", "NCHW")}
    torch.cuda.synchronize()
    _nan_aware_bitwise(to_np(rg, dt), g[f"relu_grad_{dt}/out"], dt, "relu_grad")
    tol = 1e-5 if dt == "float32" else 1e-2
    for fmt, t in outs.items():
        assert_close(to_np(t, dt), g[f"bias_add_grad_{dt}_{fmt}/out"], dt, tol, f"bias_add_grad {fmt}")


@pytest.mark.gpu
@pytest.mark.parametrize("gdt", ["float16", "bfloat16"])
def test_gpu_adam_mixed_matches_golden(g, dev, gdt):
    import torch
    import tensorflow_musa_extension_amd as tfma
    from tests.helpers import to_dev, to_np
    ops = tfma.raw_ops
    var = torch.from_numpy(g[f"adam_mixed_{gdt}/var0"].copy()).to(dev)
    m, v = torch.zeros_like(var), torch.zeros_like(var)
    ops.MusaResourceApplyAdamMixed(var, m, v, *g[f"adam_mixed_{gdt}/scalars"],
                                   to_dev(g[f"adam_mixed_{gdt}/grad"], gdt, dev))
    torch.cuda.synchronize()
    for k, t in (("var", var), ("m", m), ("v", v)):
        assert_bitwise(t.cpu().numpy(), g[f"adam_mixed_{gdt}/{k}"], f"adam_mixed {gdt} {k}")
