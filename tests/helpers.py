"""Shared helpers for the parity tests: seeded inputs in each storage dtype,
torch<->numpy transfer that keeps bfloat16 bits, and tolerance checks."""
import numpy as np
import torch

from oracle import oracle

TORCH_DT = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16,
            "float64": torch.float64}


def to_dev(a, dtype, dev):
    """numpy storage array (bfloat16 = uint16 bits) -> device tensor."""
    a = np.ascontiguousarray(a)
    if dtype == "bfloat16":
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(dev)
    return torch.from_numpy(a).to(dev)


def to_np(t, dtype):
    """device tensor -> numpy storage array (bfloat16 = uint16 bits)."""
    t = t.detach().cpu().contiguous()
    if dtype == "bfloat16":
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def gen(rng, shape, dtype, kind="normal", scale=1.0, loc=0.0):
    if dtype in ("int32", "int64", "uint8"):
        # the whole range of the type (sums and products wrap)
        info = np.iinfo(dtype)
        return rng.integers(info.min, info.max, size=shape, dtype=dtype, endpoint=True)
    if kind == "normal":
        a = loc + scale * rng.standard_normal(shape)
    elif kind == "uniform":
        a = rng.uniform(loc, scale, shape)
    else:
        raise ValueError(kind)
    return oracle.to_storage(a, dtype)


def max_rel_err(got, ref, dtype, floor=None):
    g = oracle.to_f32(got, dtype).astype(np.float64)
    r = oracle.to_f32(ref, dtype).astype(np.float64)
    denom = max(float(np.max(np.abs(r))) if r.size else 0.0, floor or 1e-30)
    return float(np.max(np.abs(g - r))) / denom if r.size else 0.0


def assert_close(got, ref, dtype, rtol, name=""):
    """max|got-ref| <= rtol * max|ref| (a norm-relative bound: elementwise
    relative error is meaningless for entries that cancel to ~0)."""
    err = max_rel_err(got, ref, dtype)
    assert err <= rtol, f"{name}: max error {err:.3e} (relative to max|ref|) > {rtol}"


def assert_bitwise(got, ref, name=""):
    g = np.ascontiguousarray(got)
    r = np.ascontiguousarray(ref)
    assert g.shape == r.shape, f"{name}: shape {g.shape} != {r.shape}"
    bits = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[g.dtype.itemsize]
    gb, rb = g.view(bits), r.view(bits)
    bad = np.flatnonzero(gb != rb)
    assert bad.size == 0, (f"{name}: {bad.size} of {g.size} elements differ, first at "
                           f"{bad[:5]}: got {g.ravel()[bad[:5]]} want {r.ravel()[bad[:5]]}")


def ulp_diff_f32(a, b):
    ai = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, np.int64(-(2**31)) - ai, ai)
    bi = np.where(bi < 0, np.int64(-(2**31)) - bi, bi)
    return np.abs(ai - bi)


def _ord16(t):
    """float16/bfloat16 device tensor -> int32 tensor ordered like the values
    (adjacent representable values differ by 1; -0 and +0 both map to 0)."""
    b = t.contiguous().view(torch.int16).int()
    return torch.where(b < 0, -(b & 0x7FFF), b)


# Absolute floor of the elementwise 16-bit BN checks: the closed forms take
# the difference of float32 terms of size O(1)-O(10) (dy - mean_dy and
# (x - mean) * c2 for dx; (x - mean) * a and b for y), each rounded to
# float32 (an ulp of 8 is 9.5e-7), so where the difference cancels to near
# zero two float32 evaluations of it - the kernel's and the reference's, whose
# coefficients can differ in their last bit - agree only to about that
# much.  bfloat16 keeps float32's exponent range, so near zero its grid is far
# finer than that (at 1e-6 an ulp is 7.5e-9) and "within 1 ulp" alone would
# demand more than float32 arithmetic holds; half's grid stops at 6e-8.
BN16_ATOL = 1e-6


def bn_max_ulp(got, ref_fn, rows, c, rows_per=1 << 20, atol=BN16_ATOL):
    """Largest distance in units of the last place between a 16-bit BN output
    got ([rows, c] viewable) and ref_fn(r0, r1) - the float32 closed form for
    rows [r0, r1), rounded to got's dtype here - over every element whose
    absolute difference exceeds atol, in chunks of rows_per rows (all on the
    device)."""
    worst = 0
    g2 = got.view(rows, c)
    for r in range(0, rows, rows_per):
        r1 = min(rows, r + rows_per)
        ref32 = ref_fn(r, r1)
        ref = ref32.to(got.dtype)
        d = (_ord16(g2[r:r1]) - _ord16(ref)).abs()
        d[(g2[r:r1].float() - ref32).abs() <= atol] = 0
        worst = max(worst, int(d.max()))
    return worst


def max_ulp_vs(got, ref, dtype, atol=BN16_ATOL, chunk=1 << 24):
    """Largest distance in units of the last place between a float16 /
    bfloat16 device tensor `got` and a reference numpy storage array `ref`
    (float16, or bfloat16 as uint16 bits) of the same element count, over
    every element whose absolute difference exceeds atol (the BN16_ATOL
    floor above); computed on the device in chunks."""
    g = got.reshape(-1)
    r = np.ascontiguousarray(ref).reshape(-1)
    assert g.numel() == r.size
    worst = 0
    for i in range(0, r.size, chunk):
        rc = to_dev(r[i:i + chunk], dtype, got.device)
        gc = g[i:i + chunk]
        d = (_ord16(gc) - _ord16(rc)).abs()
        d[(gc.float() - rc.float()).abs() <= atol] = 0
        worst = max(worst, int(d.max()))
    return worst


def bn_fwd_ref32(x, mean, var, scale, offset, eps, rows, c):
    """float32 y = (x - mean) * (1/sqrt(var + eps) * scale) + offset,
    in the fused kernel's operation order, per row range (for bn_max_ulp)."""
    a = (1.0 / torch.sqrt(var + eps)) * scale
    xv = x.view(rows, c)
    return lambda r0, r1: (xv[r0:r1].float() - mean) * a + offset


def bn_grad_ref32(dy, x, scale, mean, var, offset_bp, scale_bp, eps, rows, c):
    """float32 dx = scale*k * ((dy - mean_dy) - (x - mean) * k^2 * mean(dy*(x-mean)))
    from the kernel's own outputs (offset_bp = sum dy, scale_bp = k * sum
    dy*(x-mean)), in the fused kernel's operation order (for bn_max_ulp)."""
    k = 1.0 / torch.sqrt(var + eps)
    gk = scale * k
    mean_dy = (offset_bp.double() / rows).float()
    k2 = (k * k) * (scale_bp.double() / k.double() / rows).float()
    xv, dv = x.view(rows, c), dy.view(rows, c)
    return lambda r0, r1: gk * ((dv[r0:r1].float() - mean_dy) - (xv[r0:r1].float() - mean) * k2)


def bn_scale_backprop_ref64(dy, x, mean, var, eps, rows, c, rows_per=1 << 20):
    """scale_backprop from its definition, independent of the kernel's
    gradient: rsqrt(var + eps) * sum over rows of dy * (x - mean), with the
    mean and variance the gradient op was given, summed in float64 on the
    device in chunks of rows_per rows."""
    acc = torch.zeros(c, dtype=torch.float64, device=dy.device)
    xv, dv = x.view(rows, c), dy.view(rows, c)
    m = mean.double()
    for r in range(0, rows, rows_per):
        r1 = min(rows, r + rows_per)
        acc += (dv[r:r1].double() * (xv[r:r1].double() - m)).sum(0)
    return acc / torch.sqrt(var.double() + eps)
