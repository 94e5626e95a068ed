"""Pins for the CPU oracle (oracle/tfcpu_oracle.c).

Each check is independent of the oracle's code: library routines (numpy's
IEEE float32/float16 arithmetic, torch's bfloat16 rounding, torch's float64
batch_norm and its autograd, torch.optim.Adam), closed forms in float64,
invariants, finite differences, and the reference's own known answers.
Each is chosen so that a plausible mistake (a dropped term, a wrong sign,
Bessel applied to the wrong output, a transposed layout, a missing rounding
step) fails it.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle
from tests.helpers import assert_bitwise, ulp_diff_f32

rng_global = np.random.default_rng(1234)


# ---------------------------------------------------------------------------
# Rounding helpers
# ---------------------------------------------------------------------------
def _edge_f32():
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6, 6.1e-5, 6e-8,
            5.96e-8, 2.98e-8, 2.9802322e-08, 1e-10, np.inf, -np.inf, 3.0e38]
    # every half-way point between consecutive float16 values in [1, 2) and in
    # the subnormal range
    h = np.arange(0x3C00, 0x4000, dtype=np.uint16).view(np.float16).astype(np.float32)
    mids = ((h[:-1].astype(np.float64) + h[1:]) / 2).astype(np.float32)
    s = np.arange(1, 0x400, dtype=np.uint16).view(np.float16).astype(np.float64)
    smids = ((s[:-1] + s[1:]) / 2).astype(np.float32)
    return np.concatenate([np.array(vals, np.float32), mids, smids])


def test_f16_rounding_matches_numpy():
    lib = oracle.load()
    x = np.concatenate([
        _edge_f32(),
        (rng_global.standard_normal(20000) * 10.0 ** rng_global.integers(-9, 5, 20000)
         ).astype(np.float32)])
    got = np.array([lib.oracle_f32_to_f16(float(v)) for v in x], np.uint16)
    want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)
    back = np.array([lib.oracle_f16_to_f32(int(b)) for b in want], np.float32)
    np.testing.assert_array_equal(back, want.view(np.float16).astype(np.float32))


def test_bf16_rounding_matches_torch():
    lib = oracle.load()
    x = np.concatenate([_edge_f32(), (rng_global.standard_normal(20000) * 10.0 **
                                      rng_global.integers(-30, 30, 20000)).astype(np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([lib.oracle_f32_to_bf16(float(v)) for v in x], np.uint16)
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(oracle.f32_to_bf16_bits(x), want)
    np.testing.assert_array_equal(oracle.bf16_bits_to_f32(want),
                                  torch.from_numpy(want.view(np.int16)).view(torch.bfloat16)
                                  .float().numpy())


# ---------------------------------------------------------------------------
# FusedBatchNormV3
# ---------------------------------------------------------------------------
def _bn_case(shape, dtype="float32", seed=0, loc=0.0):
    rng = np.random.default_rng(seed)
    x = oracle.to_storage(loc + rng.standard_normal(shape), dtype)
    c = shape[-1]
    scale = rng.uniform(0.5, 1.5, c).astype(np.float32)
    offset = (0.1 * rng.standard_normal(c)).astype(np.float32)
    return x, scale, offset


def _torch_bn_f64(x_nhwc, scale, offset, eps):
    """torch.nn.functional.batch_norm in float64 (training statistics)."""
    x = torch.from_numpy(np.asarray(x_nhwc, np.float64)).permute(0, 3, 1, 2).contiguous()
    x.requires_grad_(True)
    w = torch.from_numpy(scale.astype(np.float64)).requires_grad_(True)
    b = torch.from_numpy(offset.astype(np.float64)).requires_grad_(True)
    y = torch.nn.functional.batch_norm(x, None, None, w, b, training=True, eps=eps)
    return x, w, b, y


@pytest.mark.parametrize("shape", [(2, 2, 2, 4), (2, 4, 5, 3), (4, 7, 9, 64), (32, 9, 9, 16)])
def test_bn_fwd_vs_torch_f64(shape):
    eps = 1e-3
    x, scale, offset = _bn_case(shape)
    y, bm, bv, sm, sv = oracle.bn_fwd(x, scale, offset, epsilon=eps)
    xt, _, _, yt = _torch_bn_f64(x, scale, offset, eps)
    y_ref = yt.detach().permute(0, 2, 3, 1).numpy()
    xd = x.astype(np.float64).reshape(-1, shape[-1])
    tol = lambda a, b: np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30)
    assert tol(y, y_ref) < 1e-6
    assert tol(sm, xd.mean(0)) < 1e-6
    assert tol(sv, xd.var(0, ddof=0)) < 1e-6          # reserve_space_2: population
    assert tol(bv, xd.var(0, ddof=1)) < 1e-6          # batch_variance: Bessel
    np.testing.assert_array_equal(bm, sm)


def test_bn_reference_shape_brute_force():
    """[2,2,2,4] (test/ops/fused_batchnorm_op_test.py:26) by explicit loops."""
    eps = 1e-3
    x, scale, offset = _bn_case((2, 2, 2, 4), seed=3)
    y, bm, bv, sm, sv = oracle.bn_fwd(x, scale, offset, epsilon=eps)
    for c in range(4):
        vals = [float(x[n, h, w, c]) for n in range(2) for h in range(2) for w in range(2)]
        mu = sum(vals) / 8
        var = sum((v - mu) ** 2 for v in vals) / 8
        assert abs(sm[c] - mu) <= 1e-6 and abs(sv[c] - var) <= 1e-6 * max(var, 1)
        assert abs(bv[c] - var * 8 / 7) <= 1e-6 * max(var, 1)
        for n in range(2):
            for h in range(2):
                for w in range(2):
                    want = (float(x[n, h, w, c]) - mu) / np.sqrt(var + eps) * scale[c] + offset[c]
                    assert abs(y[n, h, w, c] - want) <= 1e-5


def test_bn_invariants_and_layouts():
    eps = 1e-3
    x, scale, offset = _bn_case((8, 6, 6, 12), seed=5)
    y, bm, bv, sm, sv = oracle.bn_fwd(x, scale, offset, epsilon=eps)
    yd = y.astype(np.float64).reshape(-1, 12)
    np.testing.assert_allclose(yd.mean(0), offset, atol=1e-6)
    var = x.astype(np.float64).reshape(-1, 12).var(0)
    np.testing.assert_allclose(yd.var(0), scale.astype(np.float64) ** 2 * var / (var + eps),
                               rtol=1e-5)
    # NCHW is the same computation on the transposed tensor.
    xn = np.ascontiguousarray(x.transpose(0, 3, 1, 2))
    yn, bmn, bvn, smn, svn = oracle.bn_fwd(xn, scale, offset, epsilon=eps, data_format="NCHW")
    np.testing.assert_allclose(yn.transpose(0, 2, 3, 1), y, rtol=0, atol=1e-6)
    np.testing.assert_allclose(svn, sv, rtol=1e-6)


def test_bn_special_cases():
    # One element per channel: variance 0, Bessel guard divides by 1.
    x = np.array([[[[1.5, -2.0, 3.0]]]], np.float32)
    y, bm, bv, sm, sv = oracle.bn_fwd(x, np.ones(3, np.float32), np.array([0.5, 0, -1], np.float32),
                                      epsilon=1e-3)
    np.testing.assert_array_equal(bv, 0.0)
    np.testing.assert_array_equal(y.ravel(), [0.5, 0, -1])
    # Exponential average factor blends the running statistics (float64 check).
    xx, scale, offset = _bn_case((4, 3, 3, 5), seed=9)
    rm = np.linspace(-1, 1, 5).astype(np.float32)
    rv = np.linspace(0.5, 2, 5).astype(np.float32)
    _, bm, bv, sm, sv = oracle.bn_fwd(xx, scale, offset, rm, rv, epsilon=1e-3,
                                      exponential_avg_factor=0.25)
    xd = xx.astype(np.float64).reshape(-1, 5)
    np.testing.assert_allclose(bm, 0.75 * rm + 0.25 * xd.mean(0), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(bv, 0.75 * rv + 0.25 * xd.var(0, ddof=1), rtol=1e-6)
    np.testing.assert_allclose(sv, xd.var(0), rtol=1e-6)
    # Inference: y from the given statistics.
    y, bm, bv, _, _ = oracle.bn_fwd(xx, scale, offset, rm, rv, epsilon=1e-3, is_training=False)
    want = (xd - rm) / np.sqrt(rv.astype(np.float64) + 1e-3) * scale + offset
    np.testing.assert_allclose(y.reshape(-1, 5), want, atol=1e-5)
    np.testing.assert_array_equal(bm, rm)
    # Empty batch: NaN statistics.
    _, bm, bv, _, _ = oracle.bn_fwd(np.zeros((0, 2, 2, 3), np.float32), np.ones(3, np.float32),
                                    np.zeros(3, np.float32))
    assert np.isnan(bm).all() and np.isnan(bv).all()


def test_bn_large_mean_is_accurate():
    x, scale, offset = _bn_case((16, 8, 8, 8), seed=2, loc=1000.0)
    _, _, _, sm, sv = oracle.bn_fwd(x, scale, offset, epsilon=1e-3)
    xd = x.astype(np.float64).reshape(-1, 8)
    np.testing.assert_allclose(sv, xd.var(0), rtol=1e-5)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_bn_low_precision_activations(dtype):
    x, scale, offset = _bn_case((8, 5, 5, 16), dtype=dtype, seed=4)
    y, _, _, sm, sv = oracle.bn_fwd(x, scale, offset, epsilon=1e-3, dtype=dtype)
    xf = oracle.to_f32(x, dtype).astype(np.float64)
    _, _, _, yt = _torch_bn_f64(xf, scale, offset, 1e-3)
    y_ref = yt.detach().permute(0, 2, 3, 1).numpy()
    err = np.max(np.abs(oracle.to_f32(y, dtype) - y_ref)) / np.max(np.abs(y_ref))
    assert err < (2 ** -8 if dtype == "float16" else 2 ** -7)


# ---------------------------------------------------------------------------
# FusedBatchNormGradV3
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape", [(2, 2, 2, 4), (4, 5, 5, 8), (16, 3, 3, 32)])
def test_bn_grad_vs_torch_autograd_f64(shape):
    eps = 1e-3
    x, scale, offset = _bn_case(shape, seed=11)
    dy = np.random.default_rng(12).standard_normal(shape).astype(np.float32)
    _, _, _, sm, sv = oracle.bn_fwd(x, scale, offset, epsilon=eps)
    dx, dscale, doffset = oracle.bn_grad(dy, x, scale, sm, sv, epsilon=eps)
    xt, w, b, yt = _torch_bn_f64(x, scale, offset, eps)
    yt.backward(torch.from_numpy(dy.astype(np.float64)).permute(0, 3, 1, 2))
    rel = lambda a, b: np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30)
    assert rel(dx, xt.grad.permute(0, 2, 3, 1).numpy()) < 2e-6
    assert rel(dscale, w.grad.numpy()) < 2e-6
    assert rel(doffset, b.grad.numpy()) < 2e-6
    # Invariants per channel: sum(dx) = 0, and with xc = x - mean,
    # S = sum(dy*xc), k = rsqrt(var+eps): sum(dx*xc) = scale*k*S*eps/(var+eps)
    # (zero only when eps = 0, since sum(xc^2) = n*var).
    c = shape[-1]
    xc = (x.astype(np.float64) - sm).reshape(-1, c)
    dxd = dx.astype(np.float64).reshape(-1, c)
    S = (dy.astype(np.float64).reshape(-1, c) * xc).sum(0)
    var = sv.astype(np.float64)
    k = 1 / np.sqrt(var + eps)
    tol = 1e-5 * np.abs(dxd).max() * xc.shape[0]
    assert np.max(np.abs(dxd.sum(0))) < tol
    want = scale * k * S * eps / (var + eps)
    assert np.max(np.abs((dxd * xc).sum(0) - want)) < tol * np.abs(xc).max()


def test_bn_grad_finite_differences():
    """L = sum(y * dy): dL/dx by central differences in float64 vs the
    oracle's dx on a tiny input."""
    eps = 1e-3
    x, scale, offset = _bn_case((2, 2, 3, 3), seed=21)
    dy = np.random.default_rng(22).standard_normal(x.shape)

    def loss(xv):
        xd = xv.reshape(-1, 3)
        mu, var = xd.mean(0), xd.var(0)
        y = (xd - mu) / np.sqrt(var + eps) * scale + offset
        return float(np.sum(y * dy.reshape(-1, 3)))

    xd = x.astype(np.float64)
    fd = np.zeros_like(xd)
    h = 1e-6
    for i in np.ndindex(xd.shape):
        p, m = xd.copy(), xd.copy()
        p[i] += h
        m[i] -= h
        fd[i] = (loss(p) - loss(m)) / (2 * h)
    _, _, _, sm, sv = oracle.bn_fwd(x, scale, offset, epsilon=eps)
    dx, _, _ = oracle.bn_grad(dy.astype(np.float32), x, scale, sm, sv, epsilon=eps)
    np.testing.assert_allclose(dx, fd, atol=1e-4 * np.max(np.abs(fd)))


def test_bn_grad_inference_mode():
    eps = 1e-3
    x, scale, offset = _bn_case((3, 4, 4, 6), seed=31)
    dy = np.random.default_rng(32).standard_normal(x.shape).astype(np.float32)
    mean = np.linspace(-0.5, 0.5, 6).astype(np.float32)
    var = np.linspace(0.5, 1.5, 6).astype(np.float32)
    dx, ds, do = oracle.bn_grad(dy, x, scale, mean, var, epsilon=eps, is_training=False)
    k = 1 / np.sqrt(var.astype(np.float64) + eps)
    np.testing.assert_allclose(dx, dy * scale * k, rtol=1e-6)
    xd = x.astype(np.float64)
    np.testing.assert_allclose(ds, (dy * (xd - mean) * k).reshape(-1, 6).sum(0), rtol=1e-5)
    np.testing.assert_allclose(do, dy.astype(np.float64).reshape(-1, 6).sum(0), rtol=1e-5)


# ---------------------------------------------------------------------------
# ResourceApplyAdam
# ---------------------------------------------------------------------------
def test_adam_matches_torch_adam_f64_without_epsilon():
    """With epsilon -> 0, TF's update var -= alpha*m/(sqrt(v)+eps) equals
    torch.optim.Adam's bias-corrected update (eps = 0) exactly in real
    arithmetic; ten float32 steps stay within float32 rounding of it."""
    rng = np.random.default_rng(40)
    n = 5000
    var0 = (0.02 * rng.standard_normal(n)).astype(np.float32)
    grads = [(1e-3 * rng.standard_normal(n)).astype(np.float32) for _ in range(10)]
    var, m, v = var0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    p = torch.nn.Parameter(torch.from_numpy(var0.astype(np.float64)))
    opt = torch.optim.Adam([p], lr=1e-3, betas=(0.9, 0.999), eps=0.0)
    b1p = b2p = np.float32(1)
    for g in grads:
        b1p, b2p = np.float32(b1p * np.float32(0.9)), np.float32(b2p * np.float32(0.999))
        oracle.adam(var, m, v, g, b1p, b2p, np.float32(1e-3), np.float32(0.9),
                    np.float32(0.999), 1e-30)
        p.grad = torch.from_numpy(g.astype(np.float64))
        opt.step()
    upd = var.astype(np.float64) - var0
    upd_ref = p.detach().numpy() - var0
    assert np.max(np.abs(upd - upd_ref)) / np.max(np.abs(upd_ref)) < 1e-5


def test_adam_first_step_closed_form():
    rng = np.random.default_rng(41)
    n = 4096
    g = (1e-3 * rng.standard_normal(n)).astype(np.float32)
    g[:4] = 0.0
    var0 = (0.02 * rng.standard_normal(n)).astype(np.float32)
    for nesterov in (False, True):
        var, m, v = var0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
        b1, b2, lr, eps = 0.9, 0.999, 1e-3, 1e-7
        oracle.adam(var, m, v, g, np.float32(b1), np.float32(b2), np.float32(lr), np.float32(b1),
                    np.float32(b2), np.float32(eps), use_nesterov=nesterov)
        gd = g.astype(np.float64)
        f = lambda a: np.float64(np.float32(a))
        m1 = gd * (1 - f(b1))
        v1 = gd * gd * (1 - f(b2))
        alpha = f(lr) * np.sqrt(1 - f(b2)) / (1 - f(b1))
        num = (gd * (1 - f(b1)) + f(b1) * m1) if nesterov else m1
        var1 = var0 - alpha * num / (np.sqrt(v1) + f(eps))
        np.testing.assert_allclose(m, m1, rtol=2e-7, atol=0)
        np.testing.assert_allclose(v, v1, rtol=5e-7, atol=0)
        # var1 = var0 - upd with |upd| ~ lr: float32 rounds upd to ~1e-7 of
        # itself, so the bound is relative to the update, not to var.
        # plus half an ulp for rounding var1 itself to float32.
        upd = np.max(np.abs(var1 - var0))
        bound = 2e-6 * upd + np.spacing(np.abs(var1).astype(np.float32)).astype(np.float64)
        assert np.all(np.abs(var - var1) <= bound)
        # g = 0 with m = v = 0: the variable is untouched.
        np.testing.assert_array_equal(var[:4], var0[:4])


@pytest.mark.parametrize("gdt", ["float16", "bfloat16"])
def test_adam_mixed_first_step_closed_form(gdt):
    """fp32 state with a 16-bit grad: the first step from m = v = 0 in float64
    from the 16-bit grad's exact value (m = g(1-b1), v = g^2(1-b2), var -=
    alpha*m/(sqrt(v)+eps)).  A grad rounded to anything coarser than its own
    value, or a state rounded to 16 bits, misses the float32-level bound."""
    rng = np.random.default_rng(43)
    n = 4096
    g = oracle.to_storage(1e-3 * rng.standard_normal(n), gdt)
    var0 = (0.02 * rng.standard_normal(n)).astype(np.float32)
    var, m, v = var0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    f = lambda a: np.float64(np.float32(a))
    b1, b2, lr, eps = 0.9, 0.999, 1e-3, 1e-7
    oracle.adam_mixed(var, m, v, g, f(b1), f(b2), f(lr), f(b1), f(b2), f(eps), grad_dtype=gdt)
    gd = oracle.to_f32(g, gdt).astype(np.float64)
    m1 = gd * (1 - f(b1))
    v1 = gd * gd * (1 - f(b2))
    alpha = f(lr) * np.sqrt(1 - f(b2)) / (1 - f(b1))
    var1 = var0 - alpha * m1 / (np.sqrt(v1) + f(eps))
    np.testing.assert_allclose(m, m1, rtol=2e-7, atol=0)
    np.testing.assert_allclose(v, v1, rtol=5e-7, atol=0)
    upd = np.max(np.abs(var1 - var0))
    bound = 2e-6 * upd + np.spacing(np.abs(var1).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(var - var1) <= bound)


@pytest.mark.parametrize("dtype,tol", [("float16", 2e-3), ("bfloat16", 1.6e-2),
                                       ("float64", 1e-12)])
def test_adam_other_dtypes_vs_f64(dtype, tol):
    rng = np.random.default_rng(42)
    n = 3000
    var0 = 0.02 * rng.standard_normal(n)
    # |g| in [0.5, 1): g*g*(1-beta2) stays a normal float16.
    g0 = rng.choice([-1.0, 1.0], n) * rng.uniform(0.5, 1.0, n)
    var = oracle.to_storage(var0, dtype)
    m = oracle.to_storage(np.zeros(n), dtype)
    v = oracle.to_storage(np.zeros(n), dtype)
    g = oracle.to_storage(g0, dtype)
    vd = oracle.to_f32(var, dtype).astype(np.float64) if dtype != "float64" else var.copy()
    gd = oracle.to_f32(g, dtype).astype(np.float64) if dtype != "float64" else g.copy()
    # Scalars representable in every T (bfloat16 keeps 8 significant bits).
    oracle.adam(var, m, v, g, 0.875, 0.99609375, 0.0009765625, 0.875, 0.99609375,
                0.0, dtype=dtype)
    m1 = gd * 0.125
    v1 = gd * gd * 0.00390625
    alpha = 0.0009765625 * np.sqrt(1 - 0.99609375) / 0.125
    want = vd - alpha * m1 / np.sqrt(v1)
    got = oracle.to_f32(var, dtype).astype(np.float64) if dtype != "float64" else var
    mg = oracle.to_f32(m, dtype).astype(np.float64) if dtype != "float64" else m
    assert np.max(np.abs(mg - m1)) <= tol * np.max(np.abs(m1))
    assert np.max(np.abs((got - vd) - (want - vd))) <= tol * 8 * np.max(np.abs(want - vd))


# ---------------------------------------------------------------------------
# Elementwise
# ---------------------------------------------------------------------------
# ---------------------------------------------------------------------------
# Integer ResourceApplyAdam (the reference's int32 / int64 registration)
# ---------------------------------------------------------------------------
def _adam_int_python(var, m, v, g, b1p, b2p, lr, b1, b2, eps, bits):
    """Element by element with Python integers reduced modulo 2**bits,
    math.isqrt and sign-magnitude truncating division - an implementation
    independent of the oracle's numpy wrap and fmod arithmetic."""
    import math
    half, mod = 1 << (bits - 1), 1 << bits
    w = lambda x: (x + half) % mod - half
    if abs(1.0 - float(b1p)) < 1e-10:
        a = float(lr)
    elif 1.0 - float(b2p) < 0:
        a = float("nan")
    else:
        a = float(lr) * math.sqrt(1.0 - float(b2p)) / (1.0 - float(b1p))
    alpha = -half if (a != a or not (-half <= math.trunc(a) < half)) else math.trunc(a)
    b1, b2, eps = w(b1), w(b2), w(eps)
    out = []
    for x, mi, vi, gi in zip(var.tolist(), m.tolist(), v.tolist(), g.tolist()):
        mi = w(w(mi * b1) + w(gi * w(1 - b1)))
        vi = w(w(vi * b2) + w(w(gi * gi) * w(1 - b2)))
        d = w((math.isqrt(vi) if vi > 0 else 0) + eps)
        if d == 0:
            q = 0
        else:
            q = abs(mi) // abs(d)
            q = w(-q if (mi < 0) != (d < 0) else q)
        out.append((w(x - w(q * alpha)), mi, vi))
    return [np.array(c, dtype=var.dtype) for c in zip(*out)]


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
def test_adam_int_matches_python_integers(dtype):
    """The oracle's integer chain against a big-integer restatement, on random
    values and on the edge cases: products that wrap, v <= 0 (root 0), a zero
    divisor (epsilon = -root), MIN / -1, and every alpha regime (beta1_power
    1 -> lr; beta2_power > 1 -> NaN -> MIN; an alpha outside T's range)."""
    info = np.iinfo(dtype)
    bits = info.bits
    rng = np.random.default_rng(bits)
    n = 4000
    var = rng.integers(info.min, info.max, n, dtype=dtype, endpoint=True)
    m = rng.integers(info.min, info.max, n, dtype=dtype, endpoint=True)
    v = rng.integers(info.min, info.max, n, dtype=dtype, endpoint=True)
    g = rng.integers(info.min, info.max, n, dtype=dtype, endpoint=True)
    small = slice(0, n // 2)  # half the elements small enough not to wrap
    for a in (var, m, v, g):
        a[small] = rng.integers(-1000, 1000, n // 2)
    v[:64] = np.arange(-32, 32)
    m[64:80] = info.min
    scalars = [
        (3, 1, 9, 2, 3, 1), (0, 0, 5, 0, 0, 0), (1, 0, 11, 1, 1, -1), (2, 5, 7, 0, 1, 0),
        (4, 0, info.max, 3, 2, 2), (2, -3, info.max, 3, 2, 2), (-3, -8, -6, 7, -2, 5),
        (0, 0, 3, 0, 0, -1),
    ]
    for sc in scalars:
        xs, ms, vs = var.copy(), m.copy(), v.copy()
        oracle.adam_int(xs, ms, vs, g, *sc)
        ex, em, ev = _adam_int_python(var, m, v, g, *sc, bits)
        np.testing.assert_array_equal(ms, em, err_msg=str(sc))
        np.testing.assert_array_equal(vs, ev, err_msg=str(sc))
        np.testing.assert_array_equal(xs, ex, err_msg=str(sc))


def test_adam_int_closed_form():
    """beta1 = beta2 = 0 and epsilon = 0: m = grad, v = grad^2, the root is
    |grad| and the update is sign(grad) * alpha with alpha = trunc(lr *
    sqrt(1 - beta2_power) / (1 - beta1_power)); here lr = 10,
    beta1_power = -1, beta2_power = -3 -> alpha = trunc(10 * 2 / 2) = 10."""
    g = np.array([5, -7, 0, 1, -1, 123456], dtype=np.int64)
    var = np.full(6, 100, dtype=np.int64)
    m = np.zeros(6, dtype=np.int64)
    v = np.zeros(6, dtype=np.int64)
    oracle.adam_int(var, m, v, g, -1, -3, 10, 0, 0, 0)
    np.testing.assert_array_equal(m, g)
    np.testing.assert_array_equal(v, g * g)
    np.testing.assert_array_equal(var, 100 - 10 * np.sign(g))


def test_relu_reference_known_answers():
    """test/ops/relu_op_test.py:45-96 literal [-2,-1,0,1,2]."""
    x = np.array([-2.0, -1.0, 0.0, 1.0, 2.0], np.float32)
    np.testing.assert_array_equal(oracle.eltwise("relu", [x]), [0, 0, 0, 1, 2])
    z = oracle.eltwise("relu", [np.array([-0.0, np.nan, -np.inf], np.float32)])
    assert np.signbit(z[0]) and np.isnan(z[1]) and z[2] == 0


@pytest.mark.parametrize("xs,ys", [((64, 33), (33,)), ((64, 33), (64, 1)), ((4, 1, 5), (3, 1)),
                                   ((7,), ()), ((2, 3, 4), (2, 3, 4))])
def test_eltwise_f32_matches_numpy(xs, ys):
    rng = np.random.default_rng(50)
    x = rng.standard_normal(xs).astype(np.float32)
    y = rng.standard_normal(ys).astype(np.float32)
    np.testing.assert_array_equal(oracle.eltwise("add", [x, y]), x + y)
    np.testing.assert_array_equal(oracle.eltwise("mul", [x, y]), x * y)
    np.testing.assert_array_equal(oracle.eltwise("add_relu", [x, y]), np.maximum(x + y, 0))
    b = rng.standard_normal(ys).astype(np.float32)
    np.testing.assert_array_equal(oracle.eltwise("mul_add", [x, y, b]), (x * y) + b)


def test_eltwise_f16_matches_numpy_half_arithmetic():
    rng = np.random.default_rng(51)
    x = rng.standard_normal((128, 77)).astype(np.float16)
    y = rng.standard_normal(77).astype(np.float16)
    b = rng.standard_normal((128, 77)).astype(np.float16)
    np.testing.assert_array_equal(oracle.eltwise("add", [x, y], "float16"), x + y)
    np.testing.assert_array_equal(oracle.eltwise("mul_add", [x, y, b], "float16"), (x * y) + b)
    np.testing.assert_array_equal(oracle.eltwise("add_relu", [x, y], "float16"),
                                  np.maximum(x + y, np.float16(0)))


def test_eltwise_bf16_matches_torch_bf16_arithmetic():
    rng = np.random.default_rng(52)
    xt = torch.from_numpy(rng.standard_normal((96, 40)).astype(np.float32)).bfloat16()
    yt = torch.from_numpy(rng.standard_normal(40).astype(np.float32)).bfloat16()
    bt = torch.from_numpy(rng.standard_normal((96, 40)).astype(np.float32)).bfloat16()
    bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)
    x, y, b = bits(xt), bits(yt), bits(bt)
    np.testing.assert_array_equal(oracle.eltwise("add", [x, y], "bfloat16"), bits(xt + yt))
    np.testing.assert_array_equal(oracle.eltwise("mul_add", [x, y, b], "bfloat16"),
                                  bits((xt * yt) + bt))
    np.testing.assert_array_equal(oracle.eltwise("add_relu", [x, y], "bfloat16"),
                                  bits(torch.relu(xt + yt)))


def _baseline_operand(rng, shape, dtype):
    """Normal values with planted -0, +0, values whose sum cancels to a
    signed zero, and large values whose sum or product overflows the half
    types."""
    v = rng.standard_normal(shape).astype(np.float32)
    flat = v.reshape(-1)
    k = flat.size
    flat[rng.integers(0, k, k // 16)] = -0.0
    flat[rng.integers(0, k, k // 16)] = 0.0
    flat[rng.integers(0, k, k // 32)] = 60000.0
    flat[rng.integers(0, k, k // 32)] = -3.0e38 if dtype == "bfloat16" else -60000.0
    if dtype == "float16":
        return v.astype(np.float16)
    if dtype == "bfloat16":
        return oracle.f32_to_bf16_bits(v)
    return v


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("rows,cols", [(37, 203), (8, 8), (3, 5), (64, 1024)])
def test_baseline_rows_equals_checker(dtype, rows, cols):
    """bench.py times the cfg4 chains on the CPU with the vectorized row
    kernels of oracle_baseline_rows (F16C/AVX2 half conversion, row
    loops); they must give the checker's bits (oracle_eltwise, pinned
    against numpy / torch arithmetic above) for every op and operand
    shape they are timed on, including a column count that leaves a
    scalar tail after the 8-wide vectors."""
    rng = np.random.default_rng(54)
    x = _baseline_operand(rng, (rows, cols), dtype)
    full = _baseline_operand(rng, (rows, cols), dtype)
    row = _baseline_operand(rng, (cols,), dtype)
    c = _baseline_operand(rng, (rows, cols), dtype)
    c_row = _baseline_operand(rng, (cols,), dtype)
    cases = [("add", [x, full]), ("add", [x, row]), ("add_relu", [x, full]),
             ("add_relu", [x, row]), ("mul_add", [x, full, c]), ("mul_add", [x, row, c]),
             ("mul_add", [x, row, c_row]), ("mul_add", [x, full, c_row])]
    for op, ins in cases:
        with np.errstate(over="ignore"):
            want = oracle.eltwise(op, ins, dtype)
        got = oracle.baseline_rows(op, *ins, dtype=dtype)
        assert_bitwise(got, want, f"{op} {dtype} b{ins[1].shape} c{ins[2].shape if len(ins) > 2 else None}")
    # the planted signed zeros reach the outputs: add_relu keeps -0 and clears negatives
    z = oracle.baseline_rows("add_relu", x, full, dtype=dtype)
    zf = z.astype(np.float32) if dtype != "bfloat16" else oracle.bf16_bits_to_f32(z)
    assert (zf >= 0).all()


def _ord16_np(bits):
    """uint16 half / bfloat16 bits -> integers ordered like the values."""
    b = bits.astype(np.int32)
    return np.where(b >= 0x8000, -(b & 0x7FFF), b)


def _bn_ulps(got, want, dtype, atol):
    """Largest ulp distance over elements whose difference exceeds atol."""
    if dtype == "float32":
        d = ulp_diff_f32(got, want)
        d[np.abs(got - want) <= atol] = 0
        return int(d.max())
    g = got.view(np.uint16)
    w = want.view(np.uint16)
    gv = g.view(np.float16).astype(np.float32) if dtype == "float16" else oracle.bf16_bits_to_f32(g)
    wv = w.view(np.float16).astype(np.float32) if dtype == "float16" else oracle.bf16_bits_to_f32(w)
    d = np.abs(_ord16_np(g) - _ord16_np(w))
    d[np.abs(gv - wv) <= atol] = 0
    return int(d.max())


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("shape", [(4, 7, 5, 64), (3, 9, 1, 12), (2, 300, 1, 24)])
@pytest.mark.parametrize("threads", [1, 3])
def test_baseline_bn_matches_checker(dtype, shape, threads):
    """bench.py times the BatchNorm CPU baseline with the vectorized two-pass
    kernels of oracle_baseline_bn_fwd / _grad (float block sums, channel
    vectors of 8, a scalar tail for C % 8); against the checker
    (oracle_bn_fwd / oracle_bn_grad, pinned against torch float64 and the
    reference's known answers above) on data whose mean is far from zero:
    statistics within float32 rounding, 16-bit outputs within 1 ulp outside
    a 1e-6 absolute floor, float32 outputs within 1 ulp outside a floor of 4
    float32 ulps of max|x| (a last-bit difference of the float32 mean moves
    x - mean by that much)."""
    rng = np.random.default_rng(55)
    c = shape[-1]
    x32 = (2.0 * rng.standard_normal(shape) + 3.0).astype(np.float32)
    dy32 = rng.standard_normal(shape).astype(np.float32)
    conv = {"float32": lambda a: a, "float16": lambda a: a.astype(np.float16),
            "bfloat16": oracle.f32_to_bf16_bits}[dtype]
    x, dy = conv(x32), conv(dy32)
    scale = rng.uniform(0.5, 1.5, c).astype(np.float32)
    offset = (0.1 * rng.standard_normal(c)).astype(np.float32)
    eps = 1.001e-5
    old = oracle.get_threads()
    oracle.set_threads(threads)
    try:
        y, m, v = oracle.baseline_bn_fwd(x, scale, offset, eps, dtype)
        ry, _, _, sm, sv = oracle.bn_fwd(x, scale, offset, epsilon=eps, dtype=dtype)
        np.testing.assert_allclose(m, sm, rtol=2e-6, atol=1e-6)
        np.testing.assert_allclose(v, sv, rtol=2e-5)
        floor = 4 * 1.2e-7 * float(np.abs(x32).max()) if dtype == "float32" else 1e-6
        assert _bn_ulps(y, ry, dtype, floor) <= 1
        dx, sbp, obp = oracle.baseline_bn_grad(dy, x, scale, sm, sv, eps, dtype)
        rdx, rsbp, robp = oracle.bn_grad(dy, x, scale, sm, sv, epsilon=eps, dtype=dtype)
        np.testing.assert_allclose(obp, robp, rtol=1e-4, atol=1e-4 * np.abs(robp).max())
        np.testing.assert_allclose(sbp, rsbp, rtol=1e-4, atol=1e-4 * np.abs(rsbp).max())
        assert _bn_ulps(dx, rdx, dtype, floor) <= 1
    finally:
        oracle.set_threads(old)


@pytest.mark.parametrize("n", [1, 7, 8, 1003, 65536 + 5])
def test_baseline_adam_equals_checker(n):
    """bench.py times float32 Adam on the CPU with oracle_baseline_adam_f32
    (8-wide AVX, no per-element dtype dispatch); ten steps of it give the
    checker's bits (oracle_adam, pinned against torch.optim.Adam and the
    closed forms above), including the scalar tail past the last 8."""
    rng = np.random.default_rng(56)
    var0 = (0.02 * rng.standard_normal(n)).astype(np.float32)
    state = [var0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)]
    ref = [var0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)]
    for t in range(1, 11):
        g = (1e-3 * rng.standard_normal(n)).astype(np.float32)
        b1p, b2p = np.float32(0.9) ** t, np.float32(0.999) ** t
        oracle.baseline_adam_f32(*state, g, b1p, b2p, 1e-3, 0.9, 0.999, 1e-7)
        oracle.adam(*ref, g, b1p, b2p, 1e-3, 0.9, 0.999, 1e-7)
    for got, want, name in zip(state, ref, ("var", "m", "v")):
        assert_bitwise(got, want, name)


INT_EDGES = {"int32": [0, 1, -1, 2**31 - 1, -2**31, 2**30, -2**30 - 7, 46341, -46341],
             "int64": [0, 1, -1, 2**63 - 1, -2**63, 2**62, 3037000500, -3037000500, 2**32 + 1],
             "uint8": [0, 1, 2, 127, 128, 200, 255, 16, 17]}


def _int_inputs(rng, dtype, shape):
    info = np.iinfo(dtype)
    x = rng.integers(info.min, info.max, size=shape, dtype=dtype, endpoint=True)
    flat = x.reshape(-1)
    e = np.array(INT_EDGES[dtype], dtype=dtype)
    flat[:min(e.size, flat.size)] = e[:flat.size]
    return x


@pytest.mark.parametrize("dtype", ["int32", "int64", "uint8"])
@pytest.mark.parametrize("xs,ys", [((64, 33), (33,)), ((64, 33), (64, 1)), ((4, 1, 5), (3, 1)),
                                   ((9,), ()), ((9, 9), (9, 9))])
def test_eltwise_integers_wrap_like_numpy_and_python_ints(dtype, xs, ys):
    """Integer add / mul wrap modulo 2^bits: against numpy's integer array
    arithmetic (which wraps silently) and against Python's unbounded
    integers reduced modulo 2^bits into the type's range, including the
    extremes (INT_MIN + -1, INT_MAX * 2, 255 + 1 ...)."""
    rng = np.random.default_rng(53)
    x, y = _int_inputs(rng, dtype, xs), _int_inputs(rng, dtype, ys)
    bits = np.iinfo(dtype).bits
    signed = np.iinfo(dtype).min < 0

    def wrap(v):
        v %= 1 << bits
        return v - (1 << bits) if signed and v >= 1 << (bits - 1) else v

    xb, yb = np.broadcast_arrays(x, y)
    ops = {"add": (np.add, lambda a, b: a + b)}
    if dtype != "uint8":
        ops["mul"] = (np.multiply, lambda a, b: a * b)
    for op, (npf, pyf) in ops.items():
        got = oracle.eltwise(op, [x, y], dtype)
        assert got.dtype == np.dtype(dtype) and got.shape == xb.shape
        with np.errstate(over="ignore"):
            np.testing.assert_array_equal(got, npf(x, y))
        want = np.array([wrap(pyf(int(a), int(b))) for a, b in zip(xb.ravel(), yb.ravel())],
                        dtype=object)
        np.testing.assert_array_equal(got.ravel().astype(object), want)
    with pytest.raises(ValueError):
        oracle.eltwise("add_relu", [x, y], dtype)


def test_bias_add_nchw_channel_dim():
    """NCHW bias runs along dim 1 (musa_biasadd_op.cc:31-52)."""
    x = np.zeros((2, 3, 2, 2), np.float32)
    b = np.array([1, 2, 3], np.float32)
    out = oracle.bias_add(x, b, data_format="NCHW")
    for c in range(3):
        assert np.all(out[:, c] == b[c])
    out = oracle.bias_add(np.zeros((2, 2, 3), np.float32), b)
    assert np.all(out[..., 2] == 3)


# ---------------------------------------------------------------------------
# ReluGrad / BiasAddGrad
# ---------------------------------------------------------------------------
def test_relu_grad_matches_numpy_multiply():
    """ReluGrad = gradients * (features > 0) as a multiply: checked against
    numpy's float32 / float16 multiply and torch's bfloat16 one, including the
    special values (NaN and inf gradients, -0, features = 0)."""
    rng = np.random.default_rng(50)
    g = rng.standard_normal(4000)
    f = rng.standard_normal(4000)
    g[:6] = [np.nan, np.inf, -np.inf, -2.0, 0.0, -0.0]
    f[:6] = [-1.0, 0.0, 1.0, -3.0, 0.0, 5.0]
    for dt, npdt in (("float32", np.float32), ("float16", np.float16)):
        gs, fs = g.astype(npdt), f.astype(npdt)
        want = gs * (fs > 0).astype(npdt)
        got = oracle.eltwise("relu_grad", [gs, fs], dt)
        assert_bitwise(got, want, dt)
    gb, fb = oracle.to_storage(g, "bfloat16"), oracle.to_storage(f, "bfloat16")
    tg = torch.from_numpy(gb.view(np.int16)).view(torch.bfloat16)
    tf_ = torch.from_numpy(fb.view(np.int16)).view(torch.bfloat16)
    want = (tg * (tf_ > 0).to(torch.bfloat16)).view(torch.int16).numpy().view(np.uint16)
    got = oracle.eltwise("relu_grad", [gb, fb], "bfloat16")
    # NaN payloads differ (Eigen's canonical 0x7fc0/0xffc0 vs torch's): compare
    # NaN positions, and every other element bitwise.
    nan_w = np.isnan(oracle.to_f32(want, "bfloat16"))
    assert np.array_equal(np.isnan(oracle.to_f32(got, "bfloat16")), nan_w)
    assert_bitwise(got[~nan_w], want[~nan_w], "bfloat16")


@pytest.mark.parametrize("shape,fmt", [((2, 8, 8, 32), "NHWC"), ((2, 32, 8, 8), "NCHW"),
                                       ((37, 5), "NHWC"), ((3, 4, 5, 6, 7), "NCHW")])
def test_bias_add_grad_matches_numpy(shape, fmt):
    """Against numpy's float64 sum over the non-channel axes (the reference's
    own test shapes, test/ops/biasadd_grad_op_test.py:16-86, and two more)."""
    rng = np.random.default_rng(51)
    x = rng.standard_normal(shape)
    axes = tuple(i for i in range(len(shape)) if i != (1 if fmt == "NCHW" else len(shape) - 1))
    want = x.sum(axis=axes)
    np.testing.assert_allclose(oracle.bias_add_grad(x.astype(np.float32), fmt, "float32"), want,
                               rtol=1e-6, atol=1e-5)
    assert np.max(np.abs(oracle.bias_add_grad(x, fmt, "float64") - want)) < 1e-12
    h = x.astype(np.float16)
    got = oracle.to_f32(oracle.bias_add_grad(h, fmt, "float16"), "float16")
    np.testing.assert_allclose(got, h.astype(np.float64).sum(axis=axes), rtol=1e-3, atol=1e-2)


def test_bias_add_grad_integers_wrap_and_special_ranks():
    x32 = np.full((3, 5), 2**30, dtype=np.int32)  # sum 3 * 2^30 wraps in int32
    assert_bitwise(oracle.bias_add_grad(x32, "NHWC", "int32"),
                   np.sum(x32, axis=0, dtype=np.int32), "int32")
    x64 = np.arange(24, dtype=np.int64).reshape(2, 3, 4)
    np.testing.assert_array_equal(oracle.bias_add_grad(x64, "NCHW", "int64"), x64.sum(axis=(0, 2)))
    v = np.arange(7, dtype=np.float32)
    np.testing.assert_array_equal(oracle.bias_add_grad(v, "NHWC", "float32"), v)  # rank 1
    np.testing.assert_array_equal(oracle.bias_add_grad(np.zeros((0, 16), np.float32), "NHWC",
                                                       "float32"), np.zeros(16, np.float32))
