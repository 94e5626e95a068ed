"""The allocation-free BiasAddGrad entry point (TFMA_BiasAddGradNoAlloc),
called through the C ABI, against TFMA_BiasAddGrad (caller workspace) on the
same inputs: bitwise equal, on two calls in a row with the second on a
smaller input (the static scratch keeps the first call's partials, which the
second must not see), in every dtype and both layouts; an input whose
partials exceed the static scratch is refused with INVALID_ARGUMENT."""
import ctypes

import numpy as np
import pytest
import torch

import tensorflow_musa_extension_amd as tfma
from tensorflow_musa_extension_amd import _lib
from tests.helpers import assert_bitwise, to_np

pytestmark = pytest.mark.gpu
ops = tfma.raw_ops

def _rand(shape, dtype, dev, gen):
    if dtype in (torch.int32, torch.int64):
        return torch.randint(-1000, 1000, shape, generator=gen, device=dev, dtype=dtype)
    return torch.randn(shape, generator=gen, device=dev).to(dtype)


def _bits(t):
    return np.ascontiguousarray(to_np(t, "bfloat16") if t.dtype == torch.bfloat16
                                else t.cpu().numpy())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16, torch.float64,
                                   torch.int32, torch.int64])
@pytest.mark.parametrize("shapes,fmt", [
    (((8192, 4096), (96, 7, 7, 520)), "NHWC"),
    (((64, 256, 14, 14), (3, 40, 5, 5)), "NCHW"),
])
def test_no_alloc_matches_workspace_entry_point(dev, dtype, shapes, fmt):
    gen = torch.Generator(device=dev)
    gen.manual_seed(21)
    for shape in shapes:  # the second call's input is smaller
        x = _rand(shape, dtype, dev, gen)
        c = shape[1] if fmt == "NCHW" else shape[-1]
        want = ops.BiasAddGrad(x, data_format=fmt)
        got = torch.full((c,), 7, dtype=dtype, device=dev)
        ops.bias_add_grad_no_alloc(x, got, data_format=fmt)
        assert ops.last_kernel_name() == "tfma_bias_add_grad_finalize"
        torch.cuda.synchronize()
        assert_bitwise(_bits(got), _bits(want), f"{shape} {dtype} {fmt}")


def test_no_alloc_calls_on_two_streams_are_ordered(dev):
    """Allocation-free calls issued alternately on two streams with no
    synchronization between them share the static scratch: the library
    chains each call to the previous call's end on the other stream, so
    every result equals TFMA_BiasAddGrad's bit for bit (a large reduction
    then a small one, so an unordered small call would read or overwrite the
    large one's partials mid-flight)."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(23)
    shapes = [(8192, 4096), (64, 96), (4096, 2048), (257, 33)] * 3
    xs = [torch.randn(s, generator=gen, device=dev).half() for s in shapes]
    wants = [ops.BiasAddGrad(x) for x in xs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [torch.full((s[-1],), 7, dtype=torch.half, device=dev) for s in shapes]
    torch.cuda.synchronize()
    for i, (x, o) in enumerate(zip(xs, outs)):
        with torch.cuda.stream(streams[i % 2]):
            ops.bias_add_grad_no_alloc(x, o)
    torch.cuda.synchronize()
    for i, (o, w) in enumerate(zip(outs, wants)):
        assert_bitwise(_bits(o), _bits(w), f"call {i} {shapes[i]}")


def test_no_alloc_refuses_inputs_beyond_the_scratch(dev):
    """1.5M float channels need 6 MB of partials: more than the 4 MiB static
    scratch, so the call is refused before any launch."""
    x = torch.zeros((2, 1_500_000), device=dev)
    out = torch.zeros(1_500_000, device=dev)
    with pytest.raises(tfma.InvalidArgumentError, match="static"):
        ops.bias_add_grad_no_alloc(x, out)
    # Small and rank-1 inputs still work right after.
    x1 = torch.randn(300, device=dev)
    o1 = torch.empty(300, device=dev)
    ops.bias_add_grad_no_alloc(x1, o1)
    torch.cuda.synchronize()
    assert torch.equal(o1, x1)


def test_no_alloc_declared_in_the_c_abi():
    lib = _lib.load()
    assert hasattr(lib, "TFMA_BiasAddGradNoAlloc")
