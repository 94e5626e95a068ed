"""ResourceApplyAdam and the grouped (multi-tensor) Adam on the GPU vs the
TF-CPU oracle.  Bar: bitwise equality for every dtype (the north-star
tolerance for fp32 is 2 ulp; the kernel rounds exactly where TF-CPU does, so
0 ulp is what is checked)."""
import numpy as np
import pytest
import torch

import tensorflow_musa_extension_amd as tfma
from oracle import oracle
from bench import resnet50_shapes
from tests.helpers import assert_bitwise, gen, to_dev, to_np

pytestmark = pytest.mark.gpu
ops = tfma.raw_ops

LR, B1, B2, EPS = 1e-3, 0.9, 0.999, 1e-7


def _t_scalar(v, dtype):
    """The value of v as the host scalar of dtype T holds it."""
    return float(torch.tensor([v], dtype={"float32": torch.float32, "float16": torch.float16,
                                          "bfloat16": torch.bfloat16,
                                          "float64": torch.float64}[dtype]).double())


def _run_steps(dev, n, dtype, steps, nesterov=False, offset=0, seed=0, m_v_zero=True):
    rng = np.random.default_rng(seed)
    var = gen(rng, n + offset, dtype, scale=0.02)
    if m_v_zero:
        m = oracle.to_storage(np.zeros(n + offset), dtype)
        v = oracle.to_storage(np.zeros(n + offset), dtype)
    else:
        m = oracle.to_storage(np.abs(1e-4 * rng.standard_normal(n + offset)), dtype)
        v = oracle.to_storage(np.abs(1e-4 * rng.standard_normal(n + offset)), dtype)
    tv, tm, tvv = to_dev(var, dtype, dev), to_dev(m, dtype, dev), to_dev(v, dtype, dev)
    # Views starting `offset` elements in test the unaligned path.
    gv, gm, gvv = tv[offset:], tm[offset:], tvv[offset:]
    rv, rm, rvv = var[offset:].copy(), m[offset:].copy(), v[offset:].copy()
    b1p, b2p = 1.0, 1.0
    for _ in range(steps):
        b1p = _t_scalar(b1p * B1, dtype) if dtype != "float64" else b1p * B1
        b2p = _t_scalar(b2p * B2, dtype) if dtype != "float64" else b2p * B2
        g = gen(rng, n, dtype, scale=1e-3)
        ops.ResourceApplyAdam(gv, gm, gvv, b1p, b2p, LR, B1, B2, EPS, to_dev(g, dtype, dev),
                              use_nesterov=nesterov)
        oracle.adam(rv, rm, rvv, g, b1p, b2p, _t_scalar(LR, dtype), _t_scalar(B1, dtype),
                    _t_scalar(B2, dtype), _t_scalar(EPS, dtype), use_nesterov=nesterov,
                    dtype=dtype)
    torch.cuda.synchronize()
    return (to_np(gv, dtype), to_np(gm, dtype), to_np(gvv, dtype)), (rv, rm, rvv)


@pytest.mark.parametrize("n", [1, 3, 4, 5, 1000, 100003, 1 << 20])
def test_adam_f32_bitwise(dev, n):
    got, ref = _run_steps(dev, n, "float32", steps=3)
    for name, g, r in zip(("var", "m", "v"), got, ref):
        assert_bitwise(g, r, name)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float64"])
@pytest.mark.parametrize("nesterov", [False, True])
def test_adam_dtypes_bitwise(dev, dtype, nesterov):
    got, ref = _run_steps(dev, 65537, dtype, steps=4, nesterov=nesterov, m_v_zero=False)
    for name, g, r in zip(("var", "m", "v"), got, ref):
        assert_bitwise(g, r, f"{dtype} {name}")


def test_adam_nesterov_f32(dev):
    got, ref = _run_steps(dev, 40001, "float32", steps=3, nesterov=True)
    for name, g, r in zip(("var", "m", "v"), got, ref):
        assert_bitwise(g, r, name)


def test_adam_unaligned_views(dev):
    got, ref = _run_steps(dev, 10007, "float32", steps=2, offset=1)
    for name, g, r in zip(("var", "m", "v"), got, ref):
        assert_bitwise(g, r, name)
    assert "scalar" in ops.last_kernel_name()


def test_adam_cfg3_full(dev):
    """cfg3: 25.6M fp32, m = v = 0, ten steps t = 1..10, fresh grads."""
    got, ref = _run_steps(dev, 25_600_000, "float32", steps=10)
    for name, g, r in zip(("var", "m", "v"), got, ref):
        assert_bitwise(g, r, name)


def test_resnet50_shapes_count():
    shapes = resnet50_shapes()
    assert len(shapes) == 161
    assert sum(int(np.prod(s)) for s in shapes) == 25_557_032


@pytest.mark.parametrize("nesterov", [False, True])
def test_grouped_equals_single_and_oracle(dev, nesterov):
    rng = np.random.default_rng(3)
    shapes = resnet50_shapes() + [(0,), (7,), (8193,)]
    vars_, ms, vs, grads = [], [], [], []
    for s in shapes:
        vars_.append(to_dev(gen(rng, s, "float32", scale=0.02), "float32", dev))
        ms.append(to_dev(oracle.to_storage(np.abs(1e-4 * rng.standard_normal(s)), "float32"), "float32", dev))
        vs.append(to_dev(oracle.to_storage(np.abs(1e-4 * rng.standard_normal(s)), "float32"), "float32", dev))
        grads.append(to_dev(gen(rng, s, "float32", scale=1e-3), "float32", dev))
    single = [(v.clone(), m.clone(), w.clone()) for v, m, w in zip(vars_, ms, vs)]
    refs = [(to_np(v, "float32"), to_np(m, "float32"), to_np(w, "float32"))
            for v, m, w in zip(vars_, ms, vs)]
    b1p, b2p = _t_scalar(B1 ** 3, "float32"), _t_scalar(B2 ** 3, "float32")
    ops.MusaGroupedResourceApplyAdam(vars_, ms, vs, grads, b1p, b2p, LR, B1, B2, EPS,
                                     use_nesterov=nesterov)
    for (v, m, w), g in zip(single, grads):
        ops.ResourceApplyAdam(v, m, w, b1p, b2p, LR, B1, B2, EPS, g, use_nesterov=nesterov)
    torch.cuda.synchronize()
    for i, ((v, m, w), (sv, sm, sw), (rv, rm, rw), g) in enumerate(zip(
            zip(vars_, ms, vs), single, refs, grads)):
        oracle.adam(rv, rm, rw, to_np(g, "float32"), b1p, b2p, _t_scalar(LR, "float32"),
                    _t_scalar(B1, "float32"), _t_scalar(B2, "float32"),
                    _t_scalar(EPS, "float32"), use_nesterov=nesterov)
        for name, a, b, r in (("var", v, sv, rv), ("m", m, sm, rm), ("v", w, sw, rw)):
            assert_bitwise(to_np(a, "float32"), to_np(b, "float32"), f"tensor {i} {name} vs single")
            assert_bitwise(to_np(a, "float32"), r, f"tensor {i} {name} vs oracle")


def test_grouped_repeated_calls_reuse_staging(dev):
    """More calls than staging slots, each with a different table."""
    rng = np.random.default_rng(5)
    n_calls = 40
    ts = []
    for k in range(n_calls):
        n = 1000 + 37 * k
        var = gen(rng, n, "float32", scale=0.02)
        m = gen(rng, n, "float32", scale=1e-4)
        v = np.abs(gen(rng, n, "float32", scale=1e-4))  # second moment >= 0
        g = gen(rng, n, "float32", scale=1e-3)
        ts.append([to_dev(a, "float32", dev) for a in (var, m, v, g)])
    refs = [[to_np(t, "float32").copy() for t in group] for group in ts]
    for group in ts:
        var, m, v, g = group
        ops.MusaGroupedResourceApplyAdam([var], [m], [v], [g], 0.9, 0.999, LR, B1, B2, EPS)
    torch.cuda.synchronize()
    for group, ref in zip(ts, refs):
        rv, rm, rw, rg = ref
        oracle.adam(rv, rm, rw, rg, _t_scalar(0.9, "float32"), _t_scalar(0.999, "float32"),
                    _t_scalar(LR, "float32"), _t_scalar(B1, "float32"),
                    _t_scalar(B2, "float32"), _t_scalar(EPS, "float32"))
        assert_bitwise(to_np(group[0], "float32"), rv, "var")
        assert_bitwise(to_np(group[1], "float32"), rm, "m")
        assert_bitwise(to_np(group[2], "float32"), rw, "v")


def test_adam_errors(dev):
    f32 = dict(dtype=torch.float32, device=dev)
    a, b = torch.zeros(4, **f32), torch.zeros(5, **f32)
    with pytest.raises(tfma.InvalidArgumentError, match="var and m must have the same shape"):
        ops.ResourceApplyAdam(a, b, a.clone(), 0.9, 0.999, LR, B1, B2, EPS, a.clone())
    with pytest.raises(tfma.InvalidArgumentError, match="var and grad must have the same shape"):
        ops.ResourceApplyAdam(a, a.clone(), a.clone(), 0.9, 0.999, LR, B1, B2, EPS, b)
