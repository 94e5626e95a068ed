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


# ---------------------------------------------------------------------------
# Mixed precision: fp32 var/m/v, half / bfloat16 / float grad
# ---------------------------------------------------------------------------
def _mixed_case(dev, rng, n, gdt, offset=0):
    var = gen(rng, n + offset, "float32", scale=0.02)
    m = oracle.to_storage(np.abs(1e-4 * rng.standard_normal(n + offset)), "float32")
    v = oracle.to_storage(np.abs(1e-4 * rng.standard_normal(n + offset)), "float32")
    dev_t = [to_dev(a, "float32", dev)[offset:] for a in (var, m, v)]
    return dev_t, [var[offset:].copy(), m[offset:].copy(), v[offset:].copy()]


@pytest.mark.parametrize("gdt", ["float16", "bfloat16", "float32"])
@pytest.mark.parametrize("nesterov", [False, True])
@pytest.mark.parametrize("n,offset", [(1, 0), (5, 0), (65537, 0), (10007, 1), (1 << 20, 0)])
def test_adam_mixed_bitwise(dev, gdt, nesterov, n, offset):
    rng = np.random.default_rng(n + offset)
    (tv, tm, tw), (rv, rm, rw) = _mixed_case(dev, rng, n, gdt, offset)
    b1p, b2p = 1.0, 1.0
    for _ in range(3):
        b1p, b2p = _t_scalar(b1p * B1, "float32"), _t_scalar(b2p * B2, "float32")
        g = gen(rng, n + offset, gdt, scale=1e-3)[offset:]
        gd = to_dev(g, gdt, dev)
        ops.MusaResourceApplyAdamMixed(tv, tm, tw, b1p, b2p, LR, B1, B2, EPS, gd,
                                       use_nesterov=nesterov)
        oracle.adam_mixed(rv, rm, rw, np.ascontiguousarray(g), b1p, b2p, _t_scalar(LR, "float32"),
                          _t_scalar(B1, "float32"), _t_scalar(B2, "float32"),
                          _t_scalar(EPS, "float32"), use_nesterov=nesterov, grad_dtype=gdt)
    torch.cuda.synchronize()
    for name, t, r in (("var", tv, rv), ("m", tm, rm), ("v", tw, rw)):
        assert_bitwise(to_np(t, "float32"), r, f"mixed {gdt} {name}")


def test_adam_mixed_equals_cast_then_fp32_adam(dev):
    """The mixed op is exactly Cast(grad, float) followed by fp32 Adam."""
    rng = np.random.default_rng(9)
    n = 300001
    (tv, tm, tw), _ = _mixed_case(dev, rng, n, "bfloat16")
    cv, cm, cw = tv.clone(), tm.clone(), tw.clone()
    g = to_dev(gen(rng, n, "bfloat16", scale=1e-3), "bfloat16", dev)
    ops.MusaResourceApplyAdamMixed(tv, tm, tw, 0.81, 0.998, LR, B1, B2, EPS, g)
    ops.ResourceApplyAdam(cv, cm, cw, 0.81, 0.998, LR, B1, B2, EPS, g.float())
    torch.cuda.synchronize()
    for a, b in ((tv, cv), (tm, cm), (tw, cw)):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))


@pytest.mark.parametrize("gdt", ["float16", "bfloat16"])
def test_grouped_mixed_equals_single_mixed_and_oracle(dev, gdt):
    rng = np.random.default_rng(4)
    shapes = [(64,), (3, 3, 64, 64), (1000, 2048), (7,), (0,), (8193,)]
    vars_, ms, vs, grads, refs = [], [], [], [], []
    for s in shapes:
        n = int(np.prod(s))
        (tv, tm, tw), ref = _mixed_case(dev, rng, n, gdt)
        vars_.append(tv)
        ms.append(tm)
        vs.append(tw)
        refs.append(ref)
        grads.append(to_dev(gen(rng, n, gdt, scale=1e-3), gdt, dev))
    single = [(v.clone(), m.clone(), w.clone()) for v, m, w in zip(vars_, ms, vs)]
    ops.MusaGroupedResourceApplyAdam(vars_, ms, vs, grads, 0.729, 0.997, LR, B1, B2, EPS)
    for (v, m, w), g in zip(single, grads):
        ops.MusaResourceApplyAdamMixed(v, m, w, 0.729, 0.997, LR, B1, B2, EPS, g)
    torch.cuda.synchronize()
    for i, (v, m, w) in enumerate(zip(vars_, ms, vs)):
        rv, rm, rw = refs[i]
        oracle.adam_mixed(rv, rm, rw, to_np(grads[i], gdt), _t_scalar(0.729, "float32"),
                          _t_scalar(0.997, "float32"), _t_scalar(LR, "float32"),
                          _t_scalar(B1, "float32"), _t_scalar(B2, "float32"),
                          _t_scalar(EPS, "float32"), grad_dtype=gdt)
        for name, a, b, r in (("var", v, single[i][0], rv), ("m", m, single[i][1], rm),
                              ("v", w, single[i][2], rw)):
            assert_bitwise(to_np(a, "float32"), to_np(b, "float32"), f"tensor {i} {name} vs single")
            assert_bitwise(to_np(a, "float32"), r, f"tensor {i} {name} vs oracle")


def test_grouped_mixed_rejects_mixed_grad_dtypes(dev):
    f32 = dict(dtype=torch.float32, device=dev)
    vs = [torch.zeros(8, **f32) for _ in range(2)]
    grads = [torch.zeros(8, dtype=torch.float16, device=dev),
             torch.zeros(8, dtype=torch.bfloat16, device=dev)]
    with pytest.raises(tfma.InvalidArgumentError, match="grad dtype bfloat16, expected half"):
        ops.MusaGroupedResourceApplyAdam(vs, [v.clone() for v in vs], [v.clone() for v in vs],
                                         grads, 0.9, 0.999, LR, B1, B2, EPS)


def test_grouped_adam_cfg5_sampled(dev):
    """cfg5: 145 fp32 tensors, 1.31B parameters (21 GB of state), one grouped
    step.  Every 1009th element of every tensor, and the whole of one
    [2048,2048] tensor, is checked bitwise against the oracle on the same
    inputs (copied to the host before the step)."""
    from bench import cfg5_shapes
    shapes = cfg5_shapes()
    assert len(shapes) == 145 and sum(int(np.prod(s)) for s in shapes) == 1_310_982_144
    gen_ = torch.Generator(device=dev)
    gen_.manual_seed(5)
    tv = [0.02 * torch.randn(s, generator=gen_, device=dev) for s in shapes]
    tm = [(1e-4 * torch.randn(s, generator=gen_, device=dev)).abs_() for s in shapes]
    tw = [(1e-4 * torch.randn(s, generator=gen_, device=dev)).abs_() for s in shapes]
    tg = [1e-3 * torch.randn(s, generator=gen_, device=dev) for s in shapes]
    k, whole = 1009, 7

    def sample(ts, i):
        return ts[i].reshape(-1).cpu().numpy().copy() if i == whole else \
            ts[i].reshape(-1)[::k].cpu().numpy().copy()

    before = [[sample(ts, i) for ts in (tv, tm, tw, tg)] for i in range(len(shapes))]
    b1p, b2p = _t_scalar(B1 ** 4, "float32"), _t_scalar(B2 ** 4, "float32")
    ops.MusaGroupedResourceApplyAdam(tv, tm, tw, tg, b1p, b2p, LR, B1, B2, EPS)
    torch.cuda.synchronize()
    for i in range(len(shapes)):
        rv, rm, rw, rg = before[i]
        oracle.adam(rv, rm, rw, rg, b1p, b2p, _t_scalar(LR, "float32"), _t_scalar(B1, "float32"),
                    _t_scalar(B2, "float32"), _t_scalar(EPS, "float32"))
        for name, ts, r in (("var", tv, rv), ("m", tm, rm), ("v", tw, rw)):
            assert_bitwise(sample(ts, i), r, f"cfg5 tensor {i} {name}")
    del tv, tm, tw, tg
    torch.cuda.empty_cache()


def test_grouped_tables_over_one_staging_slot(dev):
    """24000 tiny tensors give a device table of about 1.2 MB, more than one
    1 MiB pinned staging slot, so each call's table is copied in two pieces
    through consecutive slots.  Nine calls, each with a different split of the
    same buffers (so no call reuses a cached table), wrap the 16-slot ring;
    every call must still match the oracle bit for bit."""
    rng = np.random.default_rng(21)
    n_tensors, n_calls = 24000, 9
    sizes = [rng.integers(1, 65, n_tensors) for _ in range(n_calls)]
    total = int(max(int(s.sum()) for s in sizes))
    var = gen(rng, total, "float32", scale=0.02)
    m = gen(rng, total, "float32", scale=1e-4)
    v = np.abs(gen(rng, total, "float32", scale=1e-4))
    tv, tm, tw = (to_dev(a, "float32", dev) for a in (var, m, v))
    rv, rm, rw = var.copy(), m.copy(), v.copy()
    for k in range(n_calls):
        g = gen(rng, total, "float32", scale=1e-3)
        tg = to_dev(g, "float32", dev)
        cut = [int(s) for s in sizes[k]]
        used = sum(cut)
        parts = [list(torch.split(t[:used], cut)) for t in (tv, tm, tw, tg)]
        ops.MusaGroupedResourceApplyAdam(*parts, 0.9, 0.999, LR, B1, B2, EPS)
        oracle.adam(rv[:used], rm[:used], rw[:used], g[:used], _t_scalar(0.9, "float32"),
                    _t_scalar(0.999, "float32"), _t_scalar(LR, "float32"),
                    _t_scalar(B1, "float32"), _t_scalar(B2, "float32"),
                    _t_scalar(EPS, "float32"))
    torch.cuda.synchronize()
    assert_bitwise(to_np(tv, "float32"), rv, "var")
    assert_bitwise(to_np(tm, "float32"), rm, "m")
    assert_bitwise(to_np(tw, "float32"), rw, "v")


def test_grouped_repeated_steps_use_cached_table(dev):
    """The same tensors every step (as in training): the second and later
    calls run on the library's cached device table - on the caller's stream
    and on a second stream - and still match the oracle bit for bit."""
    rng = np.random.default_rng(12)
    shapes = [(64,), (3, 3, 64, 64), (1000, 2048), (7,)]
    vars_ = [to_dev(gen(rng, s, "float32", scale=0.02), "float32", dev) for s in shapes]
    ms = [torch.zeros(s, device=dev) for s in shapes]
    vs = [torch.zeros(s, device=dev) for s in shapes]
    grads = [to_dev(gen(rng, s, "float32", scale=1e-3), "float32", dev) for s in shapes]
    refs = [[to_np(v, "float32").copy(), np.zeros(int(np.prod(s)), np.float32).reshape(s),
             np.zeros(int(np.prod(s)), np.float32).reshape(s)] for v, s in zip(vars_, shapes)]
    side = torch.cuda.Stream(device=dev)
    b1p = b2p = 1.0
    for step in range(4):
        b1p, b2p = _t_scalar(b1p * B1, "float32"), _t_scalar(b2p * B2, "float32")
        if step == 2:
            side.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(side):
                ops.MusaGroupedResourceApplyAdam(vars_, ms, vs, grads, b1p, b2p, LR, B1, B2, EPS)
            torch.cuda.current_stream(dev).wait_stream(side)
        else:
            ops.MusaGroupedResourceApplyAdam(vars_, ms, vs, grads, b1p, b2p, LR, B1, B2, EPS)
        for (rv, rm, rw), gt in zip(refs, grads):
            oracle.adam(rv, rm, rw, to_np(gt, "float32"), b1p, b2p, _t_scalar(LR, "float32"),
                        _t_scalar(B1, "float32"), _t_scalar(B2, "float32"),
                        _t_scalar(EPS, "float32"))
    torch.cuda.synchronize()
    for i, (v, m, w) in enumerate(zip(vars_, ms, vs)):
        for name, t, r in (("var", v, refs[i][0]), ("m", m, refs[i][1]), ("v", w, refs[i][2])):
            assert_bitwise(to_np(t, "float32"), r, f"tensor {i} {name}")


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_adam_int_matches_oracle(dev, dtype):
    """int32 / int64 ResourceApplyAdam (the reference's integer registrations,
    musa_applyadam_op.cc:645-676, which run its generic op chain in T)
    bitwise against the oracle's integer chain: three steps under every
    alpha regime (beta1_power 1 -> lr, a NaN alpha -> T's minimum, one out of
    T's range), with products that wrap, v <= 0, zero divisors and MIN / -1.
    The integer square root and division are this build's definition (the
    reference's are closed muDNN ops)."""
    npdt = np.int32 if dtype == torch.int32 else np.int64
    info = np.iinfo(npdt)
    rng = np.random.default_rng(info.bits + 7)
    n = 100003
    full = lambda: rng.integers(info.min, info.max, n, dtype=npdt, endpoint=True)
    var0, m0, v0 = full(), full(), full()
    half = n // 2
    for a in (var0, m0, v0):
        a[:half] = rng.integers(-5000, 5000, half)
    v0[:64] = np.arange(-32, 32)
    m0[64:96] = info.min
    scalars = [(3, 1, 9, 2, 3, 1), (1, 0, 11, 1, 1, -1), (2, 5, 7, 0, 1, 0),
               (2, -3, info.max, 3, 2, 2), (0, 0, 3, 0, 0, -1), (-3, -8, -6, 7, -2, 5)]
    for sc in scalars:
        tv, tm, tvv = (torch.from_numpy(a.copy()).to(dev) for a in (var0, m0, v0))
        rv, rm, rvv = var0.copy(), m0.copy(), v0.copy()
        for step in range(3):
            g = full()
            g[:half] = rng.integers(-300, 300, half)
            ops.ResourceApplyAdam(tv, tm, tvv, *sc, torch.from_numpy(g).to(dev))
            assert ops.last_kernel_name() == "tfma_adam_int"
            oracle.adam_int(rv, rm, rvv, g, *sc)
        torch.cuda.synchronize()
        for name, got, want in (("var", tv, rv), ("m", tm, rm), ("v", tvv, rvv)):
            np.testing.assert_array_equal(got.cpu().numpy(), want, err_msg=f"{name} {sc}")


def test_resource_apply_adam_reference_setup(dev):
    """The setup of the reference's ResourceApplyAdam test
    (test/ops/apply_resource_op_test.py:12-55): float32 variables, one update
    with beta1_power 0.9, beta2_power 0.999, lr 0.01, beta1 0.9, beta2 0.999,
    epsilon 1e-8, use_nesterov False.  Checked bitwise against the oracle and,
    from m = v = 0, against the closed form of the first step:
    var - 0.01 * sqrt(0.001) * g / (sqrt(0.001) * |g| + 1e-8)."""
    rng = np.random.default_rng(21)
    n = 4099
    var = rng.standard_normal(n).astype(np.float32)
    g = (rng.standard_normal(n) * 10.0 ** rng.integers(-6, 2, n)).astype(np.float32)
    zeros = np.zeros(n, np.float32)
    tv, tm, tvv = (torch.from_numpy(a.copy()).to(dev) for a in (var, zeros, zeros))
    ops.ResourceApplyAdam(tv, tm, tvv, 0.9, 0.999, 0.01, 0.9, 0.999, 1e-8,
                          torch.from_numpy(g).to(dev), use_nesterov=False)
    torch.cuda.synchronize()
    rv, rm, rvv = var.copy(), zeros.copy(), zeros.copy()
    oracle.adam(rv, rm, rvv, g, _t_scalar(0.9, "float32"), _t_scalar(0.999, "float32"),
                _t_scalar(0.01, "float32"), _t_scalar(0.9, "float32"),
                _t_scalar(0.999, "float32"), _t_scalar(1e-8, "float32"), dtype="float32")
    for name, got, ref in (("var", tv, rv), ("m", tm, rm), ("v", tvv, rvv)):
        assert_bitwise(got.cpu().numpy(), ref, name)
    g64 = g.astype(np.float64)
    step = 0.01 * np.sqrt(0.001) * g64 / (np.sqrt(0.001) * np.abs(g64) + 1e-8)
    got_step = var.astype(np.float64) - tv.cpu().numpy().astype(np.float64)
    # f32 rounding of var (|var| < 6) and of the update: a few float ulps.
    assert np.max(np.abs(got_step - step)) < 4e-6
    # 1 - beta is taken in float32: 1 - f32(0.9) is 0.1 within 2.4e-7 and
    # 1 - f32(0.999) is 0.001 within 1.3e-5, relative.
    np.testing.assert_allclose(tm.cpu().numpy(), 0.1 * g64, rtol=5e-7, atol=0)
    np.testing.assert_allclose(tvv.cpu().numpy(), 0.001 * g64 * g64, rtol=2e-5, atol=0)
