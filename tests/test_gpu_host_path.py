"""Host data path (staged copies, stream dependencies, host callbacks) on the
GPU.  Copies are checked byte for byte; the reference's behaviour they
mirror is musa_ext/mu/musa_se_plugin.cc:127-211 (pinned bounce H2D),
:365-432 (stream dependency) and :808-835 (host callback)."""
import time

import numpy as np
import pytest
import torch

import tensorflow_musa_extension_amd as tfma

pytestmark = pytest.mark.gpu
se = tfma.stream_executor
MIB = 1 << 20
SIZES = [1, 4095, 4 * MIB, 4 * MIB + 3, 37 * MIB + 5]  # within, at and across 4 MiB chunks


def _wait_for(pred, seconds=10.0):
    """Polls with sleeps (which release the GIL, so a Python host callback
    can run) instead of blocking in a device synchronize."""
    end = time.monotonic() + seconds
    while not pred():
        assert time.monotonic() < end, "host callback did not run"
        time.sleep(0.001)


@pytest.mark.parametrize("sync", [True, False])
@pytest.mark.parametrize("size", SIZES)
def test_htod_pageable(dev, size, sync):
    rng = np.random.default_rng(size)
    src = rng.integers(0, 256, size, dtype=np.uint8)
    want = src.copy()
    dst = torch.zeros(size, dtype=torch.uint8, device=dev)
    se.memcpy_htod(dst, src, sync=sync)
    src[:] = 0  # the call returned: the source is free for reuse, even when async
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), want)


@pytest.mark.parametrize("size", [4095, 9 * MIB + 1])
def test_htod_pinned_and_device_sources(dev, size):
    rng = np.random.default_rng(7)
    want = torch.from_numpy(rng.integers(0, 256, size, dtype=np.uint8))
    pinned = want.pin_memory()
    dst = torch.zeros(size, dtype=torch.uint8, device=dev)
    se.memcpy_htod(dst, pinned)
    torch.cuda.synchronize()
    assert torch.equal(dst.cpu(), want)
    dst2 = torch.zeros(size, dtype=torch.uint8, device=dev)
    se.memcpy_htod(dst2, dst, sync=True)  # a device source: device-to-device
    assert torch.equal(dst2.cpu(), want)


def test_htod_is_stream_ordered(dev):
    """An async staged copy runs after the work enqueued before it on its
    stream (a fill of the same buffer)."""
    s = torch.cuda.Stream()
    n = 12 * MIB + 7
    src = np.full(n, 5, np.uint8)
    dst = torch.empty(n, dtype=torch.uint8, device=dev)
    with torch.cuda.stream(s):
        for _ in range(20):
            dst.fill_(9)
        se.memcpy_htod(dst, src, stream=s)
    s.synchronize()
    assert bool((dst == 5).all())


@pytest.mark.parametrize("size", SIZES)
def test_dtoh_pageable_sync(dev, size):
    rng = np.random.default_rng(size + 1)
    want = rng.integers(0, 256, size, dtype=np.uint8)
    src = torch.from_numpy(want).to(dev)
    out = np.zeros(size, np.uint8)
    se.memcpy_dtoh(out, src, sync=True)
    assert np.array_equal(out, want)


def test_dtoh_async_into_pinned_then_host_callback(dev):
    """An async D2H into pinned memory followed by a host callback on the same
    stream: the callback runs after the copy and sees its data."""
    s = torch.cuda.Stream()
    src = torch.full((1024,), 42, dtype=torch.int32, device=dev)
    pinned = torch.zeros(1024, dtype=torch.int32).pin_memory()
    seen = []
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        se.memcpy_dtoh(pinned, src, stream=s, sync=False)
        se.host_callback(s, lambda: seen.append(int(pinned[0]) + int(pinned[-1])))
    _wait_for(lambda: seen)
    assert seen == [84]


def test_host_callbacks_run_in_order(dev):
    s = torch.cuda.Stream()
    order = []
    for i in range(8):
        se.host_callback(s, lambda i=i: order.append(i))
    _wait_for(lambda: len(order) == 8)
    assert order == list(range(8))


def test_stream_dependency(dev):
    """B reads what a slow producer on A writes; without the dependency B
    would read the buffer while A still works on it."""
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    m = torch.randn(4096, 4096, device=dev)
    torch.cuda.synchronize()
    for rep in range(20):
        with torch.cuda.stream(a):
            t = torch.full((4096,), float(rep), device=dev)
            for _ in range(3):
                m = m @ m.T * 1e-4  # keeps A busy for a while
            t.add_(1.0)
        se.create_stream_dependency(b, a)
        with torch.cuda.stream(b):
            got = t.clone()
        b.synchronize()
        assert bool((got == rep + 1.0).all())
        a.synchronize()
    torch.cuda.synchronize()
    _, _, _, pending = se.staging_pool_stats()
    assert pending == 0  # every dependency event was reclaimed


def test_staging_pool_reuses_blocks(dev):
    n = 8 * MIB
    dst = torch.empty(n, dtype=torch.uint8, device=dev)
    src = np.ones(n, np.uint8)
    for _ in range(40):
        se.memcpy_htod(dst, src)
    torch.cuda.synchronize()
    blocks, allocs, reuses, pending = se.staging_pool_stats()
    assert blocks <= 32 and allocs == blocks
    assert reuses >= 40 * 2 - 32
    assert pending == 0


def test_stream_copy(dev):
    """TFMA_StreamCopy (the bench's measuring stick) copies exactly, and
    rejects sizes and pointers that are not 16-byte multiples."""
    src = torch.randint(0, 2**31 - 1, ((64 << 20) // 4 + 12,), dtype=torch.int32, device=dev)
    dst = torch.zeros_like(src)
    tfma.raw_ops.stream_copy(dst, src)
    torch.cuda.synchronize()
    assert torch.equal(dst, src)
    with pytest.raises(tfma.InvalidArgumentError, match="16-byte"):
        tfma.raw_ops.stream_copy(dst[1:5], src[1:5])
