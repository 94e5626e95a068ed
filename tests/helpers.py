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
    bits = {2: np.uint16, 4: np.uint32, 8: np.uint64}[g.dtype.itemsize]
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
