"""The PluggableDevice adapter (libtfma_tf.so) on the GPU, driven through
the fake TensorFlow runtime as TensorFlow drives a plugin: the
StreamExecutor table on a real device (memory, copies, fills, streams,
events, timers, host callbacks), and every registered kernel family run
through its TF_InitKernel registration on a plugin stream, with outputs and
temporaries allocated through the plugin's own allocate.  Results are
compared bitwise with the library's direct C ABI (same kernels) and with the
TF-CPU oracle at the bars of the op tests (BN 1e-5 f32 / 1e-2 16-bit
activations and 1e-5 statistics; Adam and elementwise bitwise)."""
import ctypes

import numpy as np
import pytest
import torch

import tensorflow_musa_extension_amd as tfma
from oracle import oracle
from tests import tf_harness as th
from tests.helpers import assert_bitwise, assert_close, gen, to_dev, to_np

pytestmark = pytest.mark.gpu
ops = tfma.raw_ops
NP = {"float": np.float32, "half": np.float16, "bfloat16": np.uint16, "double": np.float64,
      "int32": np.int32, "int64": np.int64, "uint8": np.uint8}
ORACLE_DT = {"float": "float32", "half": "float16", "bfloat16": "bfloat16",
             "double": "float64"}


class Plugin:
    def __init__(self):
        self.h = th.harness()
        code, msg, self.params, self.platform, self.fns = self.h.init_plugin()
        assert code == th.TF_OK, msg
        self.dev = self.h.device(self.fns, 0)
        self.se = self.h.stream_executor(self.fns)
        s = ctypes.c_void_p()
        code, msg = self.h.call(self.se, "create_stream", ctypes.byref(self.dev), ctypes.byref(s))
        assert code == th.TF_OK, msg
        self.stream = s
        self.h.init_kernels()

    def sync(self):
        code, msg = self.h.call(self.se, "block_host_until_done", ctypes.byref(self.dev),
                                self.stream)
        assert code == th.TF_OK, msg

    def mem(self, ptr, size):
        return th.SP_DeviceMemoryBase(struct_size=ctypes.sizeof(th.SP_DeviceMemoryBase),
                                      opaque=ptr, size=size)

    def to_host(self, ptr, dtype, shape):
        out = np.empty(shape, NP[dtype])
        if out.nbytes:
            m = self.mem(ptr, out.nbytes)
            code, msg = self.h.call(self.se, "sync_memcpy_dtoh", ctypes.byref(self.dev),
                                    ctypes.c_void_p(out.ctypes.data), ctypes.byref(m),
                                    out.nbytes)
            assert code == th.TF_OK, msg
        return out

    def run(self, op, types, inputs, attrs=None, expect=th.TF_OK):
        """inputs: (pointer, dtype, shape, kind) with kind in {"dev", "host",
        "var", "fwd"}; returns the KernelRun (caller frees it)."""
        torch.cuda.synchronize()  # inputs were written on torch's stream
        kr = th.KernelRun(self.h, self.stream, self.se, self.dev)
        for ptr, dt, shape, kind in inputs:
            kr.input(ptr, dt, shape, variable=kind == "var", forwardable=kind == "fwd")
        kr.attrs(**(attrs or {}))
        code, msg = kr.run(self.h.kernel_index(op, **types))
        self.sync()
        assert code == expect, f"{op}: {code} {msg}"
        kr.message = msg
        return kr

    def out(self, kr, i):
        ptr, dt, shape, fwd = kr.output(i)
        name = [k for k, v in th.DT.items() if v == dt][0]
        return self.to_host(ptr, name, shape)


@pytest.fixture(scope="module")
def plugin(dev):
    return Plugin()


def T(t, kind="dev"):
    """A device (or host) torch tensor as a kernel input."""
    name = {torch.float32: "float", torch.float16: "half", torch.bfloat16: "bfloat16",
            torch.float64: "double", torch.int32: "int32", torch.int64: "int64",
            torch.uint8: "uint8"}[t.dtype]
    return (ctypes.c_void_p(t.data_ptr()), name, tuple(t.shape), kind)


def H(a, dtype="float"):
    """A 0-d host scalar input (HostMemory); the array must stay alive."""
    return (ctypes.c_void_p(a.ctypes.data), dtype, (), "host")


def test_device_and_memory(plugin):
    p, h = plugin, plugin.h
    assert b"gfx950" in p.dev.hardware_name and p.dev.device_vendor == b"AMD"
    assert p.dev.pci_bus_id
    dfns = th.SP_DeviceFns(struct_size=ctypes.sizeof(th.SP_DeviceFns))
    prm = th.SE_CreateDeviceFnsParams(struct_size=ctypes.sizeof(th.SE_CreateDeviceFnsParams),
                                      device_fns=ctypes.pointer(dfns))
    assert h.call(p.fns, "create_device_fns", None, ctypes.byref(prm))[0] == th.TF_OK
    bw = ctypes.CFUNCTYPE(ctypes.c_int64, th.DEV)(dfns.get_memory_bandwidth)(ctypes.byref(p.dev))
    assert bw > 1e12  # HBM3E: several TB/s
    n = 1 << 20
    m = th.SP_DeviceMemoryBase(struct_size=ctypes.sizeof(th.SP_DeviceMemoryBase))
    th.fn(p.se, "allocate")(ctypes.byref(p.dev), n, 0, ctypes.byref(m))
    assert m.opaque and m.size == n
    st = th.SP_AllocatorStats(struct_size=ctypes.sizeof(th.SP_AllocatorStats))
    assert th.fn(p.se, "get_allocator_stats")(ctypes.byref(p.dev), ctypes.byref(st)) == 1
    assert st.num_allocs >= 1 and st.bytes_in_use >= n
    free, total = ctypes.c_int64(), ctypes.c_int64()
    assert th.fn(p.se, "device_memory_usage")(ctypes.byref(p.dev), ctypes.byref(free),
                                              ctypes.byref(total)) == 1
    assert total.value > 200 * 2**30 and 0 < free.value <= total.value
    # memset32 then a synchronous copy back.
    assert p.h.call(p.se, "memset32", ctypes.byref(p.dev), p.stream, ctypes.byref(m),
                    0xDEADBEEF, n)[0] == th.TF_OK
    p.sync()
    got = p.to_host(m.opaque, "int32", (n // 4,)).view(np.uint32)
    assert np.all(got == 0xDEADBEEF)
    # Pageable host -> device (async, staged) -> device -> host round trip.
    src = np.random.default_rng(0).integers(0, 255, n, dtype=np.uint8)
    assert p.h.call(p.se, "memcpy_htod", ctypes.byref(p.dev), p.stream, ctypes.byref(m),
                    ctypes.c_void_p(src.ctypes.data), n)[0] == th.TF_OK
    m2 = th.SP_DeviceMemoryBase(struct_size=ctypes.sizeof(th.SP_DeviceMemoryBase))
    th.fn(p.se, "allocate")(ctypes.byref(p.dev), n, 0, ctypes.byref(m2))
    assert p.h.call(p.se, "memcpy_dtod", ctypes.byref(p.dev), p.stream, ctypes.byref(m2),
                    ctypes.byref(m), n)[0] == th.TF_OK
    dst = np.zeros(n, np.uint8)
    assert p.h.call(p.se, "memcpy_dtoh", ctypes.byref(p.dev), p.stream,
                    ctypes.c_void_p(dst.ctypes.data), ctypes.byref(m2), n)[0] == th.TF_OK
    p.sync()
    assert np.array_equal(dst, src)
    assert p.h.call(p.se, "mem_zero", ctypes.byref(p.dev), p.stream, ctypes.byref(m2),
                    n)[0] == th.TF_OK
    p.sync()
    assert not p.to_host(m2.opaque, "int32", (n // 4,)).any()
    for mm in (m, m2):
        th.fn(p.se, "deallocate")(ctypes.byref(p.dev), ctypes.byref(mm))
        assert not mm.opaque


def test_streams_events_timers_and_callbacks(plugin):
    p, h = plugin, plugin.h
    d = ctypes.byref(p.dev)
    s2 = ctypes.c_void_p()
    assert h.call(p.se, "create_stream", d, ctypes.byref(s2))[0] == th.TF_OK
    ev = ctypes.c_void_p()
    assert h.call(p.se, "create_event", d, ctypes.byref(ev))[0] == th.TF_OK
    timer = ctypes.c_void_p()
    assert h.call(p.se, "create_timer", d, ctypes.byref(timer))[0] == th.TF_OK
    n = 256 << 20
    m = th.SP_DeviceMemoryBase(struct_size=ctypes.sizeof(th.SP_DeviceMemoryBase))
    th.fn(p.se, "allocate")(d, n, 0, ctypes.byref(m))
    assert h.call(p.se, "start_timer", d, p.stream, timer)[0] == th.TF_OK
    assert h.call(p.se, "memset", d, p.stream, ctypes.byref(m), 7, n)[0] == th.TF_OK
    assert h.call(p.se, "stop_timer", d, p.stream, timer)[0] == th.TF_OK
    assert h.call(p.se, "record_event", d, p.stream, ev)[0] == th.TF_OK
    # Stream 2 waits for the fill, then zeroes the first word.
    assert h.call(p.se, "wait_for_event", d, s2, ev)[0] == th.TF_OK
    assert h.call(p.se, "create_stream_dependency", d, s2, p.stream)[0] == th.TF_OK
    assert h.call(p.se, "memset32", d, s2, ctypes.byref(m), 0, 4)[0] == th.TF_OK
    calls = []
    cb = th.STATUS_CB(lambda arg, status: calls.append(arg))
    assert th.fn(p.se, "host_callback")(d, s2, ctypes.cast(cb, ctypes.c_void_p), 1234) == 1
    assert h.call(p.se, "block_host_for_event", d, ev)[0] == th.TF_OK
    assert th.fn(p.se, "get_event_status")(d, ev) == 3  # SE_EVENT_COMPLETE
    assert h.call(p.se, "block_host_until_done", d, s2)[0] == th.TF_OK
    assert h.call(p.se, "get_stream_status", d, s2)[0] == th.TF_OK
    assert h.call(p.se, "synchronize_all_activity", d)[0] == th.TF_OK
    assert calls == [1234]
    ns = th.PROTO["nanoseconds"](_timer_ns(p))(timer)
    assert 1_000 < ns < 1_000_000_000
    head = p.to_host(m.opaque, "int32", (2,)).view(np.uint32)
    assert head[0] == 0 and head[1] == 0x07070707
    th.fn(p.se, "deallocate")(d, ctypes.byref(m))
    th.fn(p.se, "destroy_timer")(d, timer)
    th.fn(p.se, "destroy_event")(d, ev)
    th.fn(p.se, "destroy_stream")(d, s2)


def _timer_ns(p):
    tf = th.SP_TimerFns(struct_size=ctypes.sizeof(th.SP_TimerFns))
    assert p.h.call(p.fns, "create_timer_fns", None, ctypes.byref(tf))[0] == th.TF_OK
    return tf.nanoseconds


@pytest.mark.parametrize("version,dtype", [("V3", "half"), ("V3", "bfloat16"), ("", "float"),
                                           ("V2", "half")])
def test_batch_norm_kernels(plugin, version, dtype):
    """FusedBatchNorm{,V2,V3} + Grad through their registrations: bitwise
    equal to the direct C ABI call (same kernels), and to the oracle within
    the op bars.  reserve_space_4/5 are TensorFlow's empty placeholders."""
    p = plugin
    odt = ORACLE_DT[dtype]
    rng = np.random.default_rng(3)
    shape, c, eps = (8, 14, 14, 256), 256, 1.001e-5
    x = to_dev(gen(rng, shape, odt), odt, "cuda")
    dy = to_dev(gen(rng, shape, odt), odt, "cuda")
    scale = torch.from_numpy(rng.uniform(0.5, 1.5, c).astype(np.float32)).cuda()
    offset = torch.from_numpy((0.1 * rng.standard_normal(c)).astype(np.float32)).cuda()
    empty = torch.empty(0, device="cuda")
    types = {"T": dtype} if version == "" else {"T": dtype, "U": "float"}
    attrs = dict(epsilon=eps, data_format="NHWC", is_training=True)
    if version == "V3":
        attrs["exponential_avg_factor"] = 1.0
    fk = p.run("FusedBatchNorm" + version, types,
               [T(x), T(scale), T(offset), T(empty), T(empty)], attrs)
    n_out = 6 if version == "V3" else 5
    assert [fk.output(i) is not None for i in range(7)] == [True] * n_out + [False] * (7 - n_out)
    y = p.out(fk, 0)
    stats = [p.out(fk, i) for i in range(1, 5)]
    if version == "V3":
        assert fk.output(5)[2] == () and p.out(fk, 5) == 0
    want = ops.FusedBatchNormV3(x, scale, offset, empty, empty, epsilon=eps)
    torch.cuda.synchronize()
    assert_bitwise(y, to_np(want.y, odt), "y")
    for got, w in zip(stats, want[1:5]):
        assert_bitwise(got, w.cpu().numpy(), "stats")
    ry, rbm, rbv, rsm, rsv = oracle.bn_fwd(to_np(x, odt), scale.cpu().numpy(),
                                          offset.cpu().numpy(), epsilon=eps, dtype=odt)
    assert_close(y, ry, odt, 1e-2 if dtype != "float" else 1e-5, "y vs oracle")
    assert_close(stats[1], rbv, "float32", 1e-5, "batch_variance vs oracle")
    # Grad, consuming the forward's reserve spaces (device outputs of the run).
    r1, r2 = fk.output(3)[0], fk.output(4)[0]
    ginputs = [T(dy), T(x), T(scale), (r1, "float", (c,), "dev"), (r2, "float", (c,), "dev")]
    if version == "V3":
        ginputs.append((fk.output(5)[0], "float", (), "dev"))
    gk = p.run("FusedBatchNormGrad" + version, types, ginputs,
               {k: v for k, v in attrs.items() if k != "exponential_avg_factor"})
    dx, dsc, dof = p.out(gk, 0), p.out(gk, 1), p.out(gk, 2)
    assert gk.output(3)[2] == (0,) and gk.output(4)[2] == (0,)
    wg = ops.FusedBatchNormGradV3(dy, x, scale, want.reserve_space_1, want.reserve_space_2,
                                  want.reserve_space_3, epsilon=eps)
    torch.cuda.synchronize()
    assert_bitwise(dx, to_np(wg.x_backprop, odt), "dx")
    assert_bitwise(dsc, wg.scale_backprop.cpu().numpy(), "scale_backprop")
    assert_bitwise(dof, wg.offset_backprop.cpu().numpy(), "offset_backprop")
    rdx, rsb, rob = oracle.bn_grad(to_np(dy, odt), to_np(x, odt), scale.cpu().numpy(), rsm, rsv,
                                   epsilon=eps, dtype=odt)
    assert_close(dx, rdx, odt, 1e-2 if dtype != "float" else 1e-5, "dx vs oracle")
    assert_close(dsc, rsb, "float32", 1e-5, "scale_backprop vs oracle")
    fk.free()
    gk.free()


def _scalars(dtype="float"):
    vals = [0.9 ** 3, 0.999 ** 3, 1e-3, 0.9, 0.999, 1e-7]
    np_t = np.float32 if dtype == "float" else np.float64
    return [np.array(v, np_t) for v in vals]


@pytest.mark.parametrize("use_locking", [False, True])
def test_resource_apply_adam(plugin, use_locking):
    """ResourceApplyAdam on resource variables (TF_GetInputTensorFromVariable)
    with use_locking taking TensorFlow's variable locks around the update:
    bitwise equal to the oracle."""
    p = plugin
    rng = np.random.default_rng(4)
    n = 100_003
    var = (0.02 * rng.standard_normal(n)).astype(np.float32)
    m = np.abs(1e-4 * rng.standard_normal(n)).astype(np.float32)
    v = np.abs(1e-4 * rng.standard_normal(n)).astype(np.float32)
    g = (1e-3 * rng.standard_normal(n)).astype(np.float32)
    dvar, dm, dv, dg = (torch.from_numpy(a.copy()).cuda() for a in (var, m, v, g))
    sc = _scalars()
    k = p.run("ResourceApplyAdam", {"T": "float"},
              [T(dvar, "var"), T(dm, "var"), T(dv, "var")] + [H(s) for s in sc] + [T(dg)],
              dict(use_locking=use_locking, use_nesterov=False))
    locked, live, reads, reads_locked = k.lock_stats()
    assert (locked, live, reads) == ((3 if use_locking else 0), 0, 3)
    assert reads_locked == (3 if use_locking else 0)
    oracle.adam(var, m, v, g, *[float(s) for s in sc])
    for got, want in ((dvar, var), (dm, m), (dv, v)):
        assert_bitwise(got.cpu().numpy(), want, "adam")
    k.free()


def test_resource_apply_adam_int64(plugin):
    """ResourceApplyAdam with int64 state through the adapter's integer
    registration: host int64 scalars, bitwise equal to the oracle's integer
    chain."""
    p = plugin
    rng = np.random.default_rng(14)
    n = 50_001
    var, m, v, g = (rng.integers(-10_000, 10_000, n).astype(np.int64) for _ in range(4))
    dvar, dm, dv, dg = (torch.from_numpy(a.copy()).cuda() for a in (var, m, v, g))
    sc = [np.array(x, np.int64) for x in (3, 1, 9, 2, 3, 1)]
    k = p.run("ResourceApplyAdam", {"T": "int64"},
              [T(dvar, "var"), T(dm, "var"), T(dv, "var")] + [H(s, "int64") for s in sc] + [T(dg)],
              dict(use_locking=False, use_nesterov=False))
    oracle.adam_int(var, m, v, g, *[int(s) for s in sc])
    for got, want in ((dvar, var), (dm, m), (dv, v)):
        np.testing.assert_array_equal(got.cpu().numpy(), want)
    k.free()


def test_mixed_and_grouped_adam(plugin):
    p = plugin
    rng = np.random.default_rng(5)
    sc = _scalars()
    # MusaResourceApplyAdamMixed: fp32 state, bf16 gradient.
    n = 77_777
    var = (0.02 * rng.standard_normal(n)).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    gb = oracle.to_storage(1e-3 * rng.standard_normal(n), "bfloat16")
    dvar, dm, dv = (torch.from_numpy(a.copy()).cuda() for a in (var, m, v))
    dgb = to_dev(gb, "bfloat16", "cuda")
    k = p.run("MusaResourceApplyAdamMixed", {"T": "bfloat16"},
              [T(dvar, "var"), T(dm, "var"), T(dv, "var")] + [H(s) for s in sc] + [T(dgb)],
              dict(use_locking=False, use_nesterov=False))
    oracle.adam_mixed(var, m, v, gb, *[float(s) for s in sc], grad_dtype="bfloat16")
    for got, want in ((dvar, var), (dm, m), (dv, v)):
        assert_bitwise(got.cpu().numpy(), want, "mixed")
    k.free()
    # MusaGroupedResourceApplyAdam over 3 tensors (float state and grads).
    shapes = [(64, 3, 7, 7), (1000,), (513, 129)]
    st = [[(0.02 * rng.standard_normal(s)).astype(np.float32) for s in shapes],
          [np.zeros(s, np.float32) for s in shapes], [np.zeros(s, np.float32) for s in shapes]]
    gs = [(1e-3 * rng.standard_normal(s)).astype(np.float32) for s in shapes]
    dst = [[torch.from_numpy(a.copy()).cuda() for a in kind] for kind in st]
    dgs = [torch.from_numpy(a).cuda() for a in gs]
    inputs = [T(t, "var") for kind in dst for t in kind] + [H(s) for s in sc] + [T(t) for t in dgs]
    k = p.run("MusaGroupedResourceApplyAdam", {"T": "float", "Tgrad": "float"}, inputs,
              dict(N=3, use_locking=True, use_nesterov=False))
    assert k.lock_stats()[0] == 9
    for i in range(3):
        oracle.adam(st[0][i], st[1][i], st[2][i], gs[i], *[float(s) for s in sc])
        for kind in range(3):
            assert_bitwise(dst[kind][i].cpu().numpy(), st[kind][i], f"grouped {i}/{kind}")
    k.free()


def test_uninitialized_variable_is_failed_precondition(plugin):
    p = plugin
    g = torch.zeros(10, device="cuda")
    sc = _scalars()
    k = p.run("ResourceApplyAdam", {"T": "float"},
              [(None, "float", (10,), "var"), T(g, "var"), T(g, "var")] + [H(s) for s in sc] +
              [T(g)], dict(use_locking=False, use_nesterov=False), expect=9)
    assert k.message == "Adam variables (var/m/v) not initialized."
    k.free()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_elementwise_kernels(plugin, dtype):
    """BiasAdd, MusaBiasAddRelu, Relu, ReluGrad, AddV2, Mul, MusaAddV2Relu,
    MusaShiftedAffineMap and BiasAddGrad through their registrations,
    bitwise against the oracle; in-place forwarding when TensorFlow offers
    the input buffer."""
    p = plugin
    odt = {torch.float32: "float32", torch.float16: "float16",
           torch.bfloat16: "bfloat16"}[dtype]
    tname = {torch.float32: "float", torch.float16: "half", torch.bfloat16: "bfloat16"}[dtype]
    rng = np.random.default_rng(6)
    xs, bs, cs = gen(rng, (64, 96), odt), gen(rng, (96,), odt), gen(rng, (64, 96), odt)
    x, b, c = (to_dev(a, odt, "cuda") for a in (xs, bs, cs))
    ty = {"T": tname}

    def check(kr, want, name, i=0):
        ptr, _, shape, _ = kr.output(i)
        got = p.to_host(ptr, tname, shape)
        assert_bitwise(got, np.ascontiguousarray(want), name)
        kr.free()

    check(p.run("BiasAdd", ty, [T(x), T(b)], dict(data_format="NHWC")),
          oracle.bias_add(xs, bs, dtype=odt), "BiasAdd")
    check(p.run("MusaBiasAddRelu", ty, [T(x), T(b)], dict(data_format="NHWC")),
          oracle.bias_add(xs, bs, relu=True, dtype=odt), "MusaBiasAddRelu")
    check(p.run("Relu", ty, [T(x)]), oracle.eltwise("relu", [xs], odt), "Relu")
    check(p.run("ReluGrad", ty, [T(c), T(x)]), oracle.eltwise("relu_grad", [cs, xs], odt),
          "ReluGrad")
    check(p.run("AddV2", ty, [T(x), T(b)]), oracle.eltwise("add", [xs, bs], odt), "AddV2")
    check(p.run("Mul", ty, [T(b), T(x)]), oracle.eltwise("mul", [bs, xs], odt), "Mul")
    check(p.run("MusaAddV2Relu", ty, [T(x), T(c)]), oracle.eltwise("add_relu", [xs, cs], odt),
          "MusaAddV2Relu")
    check(p.run("MusaShiftedAffineMap", ty, [T(x), T(b), T(c)]),
          oracle.eltwise("mul_add", [xs, bs, cs], odt), "MusaShiftedAffineMap")
    bag = p.run("BiasAddGrad", ty, [T(c)], dict(data_format="NHWC"))
    assert_close(p.out(bag, 0), oracle.bias_add_grad(cs, "NHWC", odt), odt,
                 1e-5 if dtype == torch.float32 else 1e-2, "BiasAddGrad")
    bag.free()
    # Forwarded: MusaBiasAddRelu writes over its offered input buffer.
    xf = x.clone()
    k = p.run("MusaBiasAddRelu", ty, [T(xf, "fwd"), T(b)], dict(data_format="NHWC"))
    assert k.output(0)[3] == 0 and k.output(0)[0] == xf.data_ptr()
    check(k, oracle.bias_add(xs, bs, relu=True, dtype=odt), "forwarded MusaBiasAddRelu")


@pytest.mark.parametrize("tname", ["int32", "int64", "uint8", "float"])
def test_stock_op_registrations_integer_and_legacy_names(plugin, tname):
    """Add (the legacy name), AddV2, Mul, BiasAdd and BiasAddV1 through their
    registrations for the reference's integer dtypes (musa_add_op.cc:455-468,
    musa_multiply_op.cc:315-323, musa_biasadd_op.cc:67-79), bitwise against
    the oracle's wrapping arithmetic; float for the legacy names."""
    p = plugin
    npdt = NP[tname]
    rng = np.random.default_rng(7)
    if tname == "float":
        xs = rng.standard_normal((64, 96)).astype(np.float32)
        bs = rng.standard_normal(96).astype(np.float32)
    else:
        info = np.iinfo(npdt)
        xs = rng.integers(info.min, info.max, (64, 96), dtype=npdt, endpoint=True)
        bs = rng.integers(info.min, info.max, 96, dtype=npdt, endpoint=True)
    odt = ORACLE_DT.get(tname, tname)
    x, b = torch.from_numpy(xs).cuda(), torch.from_numpy(bs).cuda()
    ty = {"T": tname}

    def check(kr, want, name):
        ptr, _, shape, _ = kr.output(0)
        assert_bitwise(p.to_host(ptr, tname, shape), np.ascontiguousarray(want), name)
        kr.free()

    for op in ("AddV2", "Add"):
        check(p.run(op, ty, [T(x), T(b)]), oracle.eltwise("add", [xs, bs], odt), op)
    if tname == "uint8":
        for op in ("Mul", "BiasAdd", "BiasAddV1"):  # not registered for uint8
            with pytest.raises(KeyError):
                p.h.kernel_index(op, **ty)
        return
    check(p.run("Mul", ty, [T(b), T(x)]), oracle.eltwise("mul", [bs, xs], odt), "Mul")
    check(p.run("BiasAdd", ty, [T(x), T(b)], dict(data_format="NHWC")),
          oracle.bias_add(xs, bs, dtype=odt), "BiasAdd")
    check(p.run("BiasAddV1", ty, [T(x), T(b)]), oracle.bias_add(xs, bs, dtype=odt), "BiasAddV1")


def test_elementwise_errors(plugin):
    p = plugin
    a, b = torch.zeros(4, 5, device="cuda"), torch.zeros(3, device="cuda")
    k = p.run("AddV2", {"T": "float"}, [T(a), T(b)], expect=th.TF_INVALID_ARGUMENT)
    assert k.message == "Incompatible shapes for Add: [4,5] and [3]"
    assert k.output(0) is None
    k.free()
    k = p.run("ReluGrad", {"T": "float"}, [T(a), T(torch.zeros(5, 4, device="cuda"))],
              expect=th.TF_INVALID_ARGUMENT)
    assert k.message.startswith("Inputs to ReluGrad must have the same shape")
    k.free()
