"""Writes tests/golden/golden.npz: small seeded inputs and the TF-CPU oracle's
outputs for every op on the hot path.

The reference ships no golden vectors for these ops (its tests evaluate TF-CPU
at run time, test/musa_test_utils.py:82-111), so the fixtures come from this
repository's oracle.  Before writing, every BN and Adam case is checked
against an independent float64 reference (torch's batch_norm and autograd,
the Adam closed form), so a fixture can only hold oracle outputs that the
mathematics confirms.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle  # noqa: E402

OUT = os.path.join(HERE, "golden.npz")


def bn_cases(store):
    rng = np.random.default_rng(2024)
    cases = [("bn_nhwc_f32", (2, 2, 2, 4), "float32", "NHWC"),   # reference test shape
             ("bn_nhwc_f32_c3", (2, 4, 5, 3), "float32", "NHWC"),
             ("bn_nhwc_f16", (4, 3, 3, 16), "float16", "NHWC"),
             ("bn_nhwc_bf16", (4, 3, 3, 16), "bfloat16", "NHWC"),
             ("bn_nchw_f32", (2, 3, 4, 5), "float32", "NCHW")]
    for name, shape, dt, fmt in cases:
        c = shape[-1] if fmt == "NHWC" else shape[1]
        x = oracle.to_storage(rng.standard_normal(shape), dt)
        dy = oracle.to_storage(rng.standard_normal(shape), dt)
        scale = rng.uniform(0.5, 1.5, c).astype(np.float32)
        offset = (0.1 * rng.standard_normal(c)).astype(np.float32)
        eps = 1e-3
        y, bm, bv, sm, sv = oracle.bn_fwd(x, scale, offset, epsilon=eps, data_format=fmt, dtype=dt)
        dx, dsc, dof = oracle.bn_grad(dy, x, scale, sm, sv, epsilon=eps, data_format=fmt, dtype=dt)
        # float64 cross-check with torch (NCHW layout for torch).
        xf = oracle.to_f32(x, dt).astype(np.float64)
        dyf = oracle.to_f32(dy, dt).astype(np.float64)
        xt = torch.from_numpy(xf if fmt == "NCHW" else xf.transpose(0, 3, 1, 2).copy())
        dyt = torch.from_numpy(dyf if fmt == "NCHW" else dyf.transpose(0, 3, 1, 2).copy())
        xt.requires_grad_(True)
        w = torch.from_numpy(scale.astype(np.float64)).requires_grad_(True)
        b = torch.from_numpy(offset.astype(np.float64)).requires_grad_(True)
        yt = torch.nn.functional.batch_norm(xt, None, None, w, b, training=True, eps=eps)
        yt.backward(dyt)
        to_fmt = (lambda t: t.detach().numpy()) if fmt == "NCHW" else (
            lambda t: t.detach().numpy().transpose(0, 2, 3, 1))
        tol = 1e-5 if dt == "float32" else 1e-2
        rel = lambda a, r: np.max(np.abs(a - r)) / max(np.max(np.abs(r)), 1e-30)
        assert rel(oracle.to_f32(y, dt), to_fmt(yt)) < tol, name
        assert rel(oracle.to_f32(dx, dt), to_fmt(xt.grad)) < tol, name
        assert rel(dsc, w.grad.numpy()) < 1e-5 and rel(dof, b.grad.numpy()) < 1e-5, name
        for k, v in dict(x=x, dy=dy, scale=scale, offset=offset, y=y, batch_mean=bm,
                         batch_variance=bv, reserve_space_1=sm, reserve_space_2=sv, dx=dx,
                         scale_backprop=dsc, offset_backprop=dof).items():
            store[f"{name}/{k}"] = v


def adam_cases(store):
    rng = np.random.default_rng(7)
    for dt in ("float32", "float16", "bfloat16"):
        n = 1031
        var = oracle.to_storage(0.02 * rng.standard_normal(n), dt)
        m = oracle.to_storage(np.zeros(n), dt)
        v = oracle.to_storage(np.zeros(n), dt)
        g = oracle.to_storage(rng.choice([-1.0, 1.0], n) * rng.uniform(0.5, 1.0, n), dt)
        store[f"adam_{dt}/var0"], store[f"adam_{dt}/grad"] = var.copy(), g.copy()
        # Scalars exactly representable in every T (bfloat16 keeps 8 significant bits).
        b1p, b2p, lr, b1, b2, eps = 0.875, 0.99609375, 0.0009765625, 0.875, 0.99609375, 0.0078125
        oracle.adam(var, m, v, g, b1p, b2p, lr, b1, b2, eps, dtype=dt)
        gd = oracle.to_f32(g, dt).astype(np.float64)
        v0 = oracle.to_f32(store[f"adam_{dt}/var0"], dt).astype(np.float64)
        alpha = lr * np.sqrt(1 - b2p) / (1 - b1p)
        want = v0 - alpha * (gd * (1 - b1)) / (np.sqrt(gd * gd * (1 - b2)) + eps)
        got = oracle.to_f32(var, dt).astype(np.float64)
        # Bound: a few roundings of the update plus one rounding of var to T.
        tol = {"float32": 1e-6, "float16": 4e-3, "bfloat16": 3e-2}[dt]
        ulp = {"float32": 2.0 ** -23, "float16": 2.0 ** -10, "bfloat16": 2.0 ** -7}[dt]
        bound = tol * np.max(np.abs(want - v0)) + ulp * np.abs(want)
        assert np.all(np.abs(got - want) <= bound), dt
        store[f"adam_{dt}/var"], store[f"adam_{dt}/m"], store[f"adam_{dt}/v"] = var, m, v
        store[f"adam_{dt}/scalars"] = np.array([b1p, b2p, lr, b1, b2, eps])


def eltwise_cases(store):
    rng = np.random.default_rng(11)
    for dt in ("float32", "float16", "bfloat16"):
        x = oracle.to_storage(rng.standard_normal((33, 17)), dt)
        bias = oracle.to_storage(rng.standard_normal(17), dt)
        a = oracle.to_storage(rng.standard_normal((33, 17)), dt)
        b = oracle.to_storage(rng.standard_normal(17), dt)
        store[f"ew_{dt}/x"], store[f"ew_{dt}/bias"] = x, bias
        store[f"ew_{dt}/a"], store[f"ew_{dt}/b"] = a, b
        store[f"ew_{dt}/bias_add_relu"] = oracle.bias_add(x, bias, relu=True, dtype=dt)
        store[f"ew_{dt}/add_v2_relu"] = oracle.eltwise("add_relu", [x, bias], dt)
        store[f"ew_{dt}/mul_add"] = oracle.eltwise("mul_add", [x, a, b], dt)
        store[f"ew_{dt}/relu"] = oracle.eltwise("relu", [x], dt)


def backward_cases(store):
    """ReluGrad, BiasAddGrad and mixed-precision Adam (fp32 state, 16-bit grad)."""
    rng = np.random.default_rng(13)
    for dt in ("float32", "float16", "bfloat16"):
        g = rng.standard_normal((33, 17))
        f = rng.standard_normal((33, 17))
        g.ravel()[:6] = [np.nan, np.inf, -np.inf, -2.0, 0.0, -0.0]
        f.ravel()[:6] = [-1.0, 0.0, 1.0, -3.0, 0.0, 5.0]
        gs, fs = oracle.to_storage(g, dt), oracle.to_storage(f, dt)
        rg = oracle.eltwise("relu_grad", [gs, fs], dt)
        with np.errstate(invalid="ignore"):  # inf * 0 is NaN, as in TF
            want = oracle.to_f32(gs, dt).astype(np.float64) * (oracle.to_f32(fs, dt) > 0)
            got = oracle.to_f32(rg, dt).astype(np.float64)
            assert np.array_equal(np.isnan(got), np.isnan(want))
            ok = ~np.isnan(want)
            assert np.array_equal(got[ok], want[ok]) and np.array_equal(
                np.signbit(got[ok]), np.signbit(want[ok])), dt
        store[f"relu_grad_{dt}/g"], store[f"relu_grad_{dt}/f"], store[f"relu_grad_{dt}/out"] = gs, fs, rg
        for shape, fmt in (((2, 8, 8, 32), "NHWC"), ((2, 32, 8, 8), "NCHW")):
            x = oracle.to_storage(rng.standard_normal(shape), dt)
            out = oracle.bias_add_grad(x, fmt, dt)
            axes = tuple(i for i in range(4) if i != (1 if fmt == "NCHW" else 3))
            ref = oracle.to_f32(x, dt).astype(np.float64).sum(axis=axes)
            tol = 1e-6 if dt == "float32" else 1e-2
            assert np.max(np.abs(oracle.to_f32(out, dt) - ref)) <= tol * np.max(np.abs(ref))
            store[f"bias_add_grad_{dt}_{fmt}/x"], store[f"bias_add_grad_{dt}_{fmt}/out"] = x, out
    for gdt in ("float16", "bfloat16"):
        n = 1031
        var = (0.02 * rng.standard_normal(n)).astype(np.float32)
        m = np.zeros(n, np.float32)
        v = np.zeros(n, np.float32)
        g = oracle.to_storage(1e-3 * rng.standard_normal(n), gdt)
        store[f"adam_mixed_{gdt}/var0"], store[f"adam_mixed_{gdt}/grad"] = var.copy(), g.copy()
        sc = [np.float32(a) for a in (0.9, 0.999, 1e-3, 0.9, 0.999, 1e-7)]
        oracle.adam_mixed(var, m, v, g, *[float(a) for a in sc], grad_dtype=gdt)
        gd = oracle.to_f32(g, gdt).astype(np.float64)
        f = lambda a: np.float64(np.float32(a))
        m1 = gd * (1 - f(0.9))
        assert np.allclose(m, m1, rtol=2e-7, atol=0), gdt
        store[f"adam_mixed_{gdt}/var"], store[f"adam_mixed_{gdt}/m"], store[f"adam_mixed_{gdt}/v"] = var, m, v
        store[f"adam_mixed_{gdt}/scalars"] = np.array([float(a) for a in sc])


def main():
    store = {}
    bn_cases(store)
    adam_cases(store)
    eltwise_cases(store)
    backward_cases(store)
    np.savez_compressed(OUT, **store)
    print(f"wrote {OUT}: {len(store)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
