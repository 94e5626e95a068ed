"""Drives libtfma_tf.so (the PluggableDevice adapter) the way TensorFlow
does, through the fake TensorFlow C-API runtime in tests/fake_tf (test
infrastructure: TensorFlow is not installed).

Struct layouts mirror tensorflow_musa_extension_amd/csrc/tf_c_api.h; the
plugin's function tables are read as raw pointers and called through
ctypes prototypes.
"""
import ctypes
import json
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PLUGIN_PATH = os.path.join(ROOT, "tensorflow_musa_extension_amd", "libtfma_tf.so")
FAKE_PATH = os.path.join(ROOT, "tests", "fake_tf", "libfake_tf.so")

vp, sz, u64, i64, i32 = (ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_int64,
                         ctypes.c_int32)

TF_OK, TF_INVALID_ARGUMENT, TF_INTERNAL = 0, 3, 13
DT = {"float": 1, "double": 2, "int32": 3, "uint8": 4, "int64": 9, "bfloat16": 14, "half": 19,
      "resource": 20}


class SP_Platform(ctypes.Structure):
    _fields_ = [("struct_size", sz), ("ext", vp), ("name", ctypes.c_char_p),
                ("type", ctypes.c_char_p), ("supports_unified_memory", ctypes.c_ubyte),
                ("use_bfc_allocator", ctypes.c_ubyte), ("force_memory_growth", ctypes.c_ubyte)]


PLATFORM_FNS = ["get_device_count", "create_device", "destroy_device", "create_device_fns",
                "destroy_device_fns", "create_stream_executor", "destroy_stream_executor",
                "create_timer_fns", "destroy_timer_fns"]


class SP_PlatformFns(ctypes.Structure):
    _fields_ = [("struct_size", sz), ("ext", vp)] + [(n, vp) for n in PLATFORM_FNS]


class SE_PlatformRegistrationParams(ctypes.Structure):
    _fields_ = [("struct_size", sz), ("ext", vp), ("major_version", i32),
                ("minor_version", i32), ("patch_version", i32),
                ("platform", ctypes.POINTER(SP_Platform)),
                ("platform_fns", ctypes.POINTER(SP_PlatformFns)),
                ("destroy_platform", vp), ("destroy_platform_fns", vp)]


class SP_Device(ctypes.Structure):
    _fields_ = [("struct_size", sz), ("ext", vp), ("ordinal", i32), ("device_handle", vp),
                ("hardware_name", ctypes.c_char_p), ("device_vendor", ctypes.c_char_p),
                ("pci_bus_id", ctypes.c_char_p)]


class SE_CreateDeviceParams(ctypes.Structure):
    _fields_ = [("struct_size", sz), ("ext", vp), ("ordinal", i32),
                ("device", ctypes.POINTER(SP_Device))]


class SP_DeviceFns(ctypes.Structure):
    _fields_ = [("struct_size", sz), ("ext", vp), ("get_numa_node", vp),
                ("get_memory_bandwidth", vp), ("get_gflops", vp)]


class SE_CreateDeviceFnsParams(ctypes.Structure):
    _fields_ = [("struct_size", sz), ("ext", vp), ("device_fns", ctypes.POINTER(SP_DeviceFns))]


SE_FNS = ["allocate", "deallocate", "host_memory_allocate", "host_memory_deallocate",
          "unified_memory_allocate", "unified_memory_deallocate", "get_allocator_stats",
          "device_memory_usage", "create_stream", "destroy_stream", "create_stream_dependency",
          "get_stream_status", "create_event", "destroy_event", "get_event_status",
          "record_event", "wait_for_event", "create_timer", "destroy_timer", "start_timer",
          "stop_timer", "memcpy_dtoh", "memcpy_htod", "memcpy_dtod", "sync_memcpy_dtoh",
          "sync_memcpy_htod", "sync_memcpy_dtod", "block_host_for_event",
          "block_host_until_done", "synchronize_all_activity", "mem_zero", "memset",
          "memset32", "host_callback"]


class SP_StreamExecutor(ctypes.Structure):
    _fields_ = [("struct_size", sz), ("ext", vp)] + [(n, vp) for n in SE_FNS]


class SE_CreateStreamExecutorParams(ctypes.Structure):
    _fields_ = [("struct_size", sz), ("ext", vp),
                ("stream_executor", ctypes.POINTER(SP_StreamExecutor))]


class SP_TimerFns(ctypes.Structure):
    _fields_ = [("struct_size", sz), ("ext", vp), ("nanoseconds", vp)]


class SP_DeviceMemoryBase(ctypes.Structure):
    _fields_ = [("struct_size", sz), ("ext", vp), ("opaque", vp), ("size", u64),
                ("payload", u64)]


class SP_AllocatorStats(ctypes.Structure):
    _fields_ = [("struct_size", sz), ("num_allocs", i64), ("bytes_in_use", i64),
                ("peak_bytes_in_use", i64), ("largest_alloc_size", i64),
                ("has_bytes_limit", ctypes.c_int8), ("bytes_limit", i64),
                ("bytes_reserved", i64), ("peak_bytes_reserved", i64),
                ("has_bytes_reservable_limit", ctypes.c_int8), ("bytes_reservable_limit", i64),
                ("largest_free_block_bytes", i64)]


class TP_OptimizerConfigs(ctypes.Structure):
    _fields_ = [("struct_size", sz), ("ext", vp)] + [(n, ctypes.c_int) for n in (
        "disable_model_pruning", "implementation_selector", "function_optimization",
        "common_subgraph_elimination", "arithmetic_optimization", "debug_stripper",
        "constant_folding", "shape_optimization", "auto_mixed_precision",
        "auto_mixed_precision_onednn_bfloat16", "auto_mixed_precision_mkl",
        "pin_to_host_optimization", "layout_optimizer", "remapping", "loop_optimization",
        "dependency_optimization", "auto_parallel", "memory_optimization",
        "scoped_allocator_optimization")]


class TP_Optimizer(ctypes.Structure):
    _fields_ = [("struct_size", sz), ("ext", vp), ("create_func", vp), ("optimize_func", vp),
                ("destroy_func", vp)]


class TP_OptimizerRegistrationParams(ctypes.Structure):
    _fields_ = [("struct_size", sz), ("ext", vp), ("major_version", i32),
                ("minor_version", i32), ("patch_version", i32),
                ("device_type", ctypes.c_char_p),
                ("optimizer_configs", ctypes.POINTER(TP_OptimizerConfigs)),
                ("optimizer", ctypes.POINTER(TP_Optimizer))]


class TF_Buffer(ctypes.Structure):
    _fields_ = [("data", vp), ("length", sz), ("data_deallocator", vp)]


def full_size(struct):
    return ctypes.sizeof(struct)


def offset_end(struct, field):
    """TF_OFFSET_OF_END: the STRUCT_SIZE constants of TensorFlow's headers."""
    f = getattr(struct, field)
    return f.offset + f.size


# Prototypes of the table entries the tests call.
P = vp  # opaque pointers (SP_Stream, SP_Event, SP_Timer, TF_Status*)
DEV = ctypes.POINTER(SP_Device)
MEM = ctypes.POINTER(SP_DeviceMemoryBase)
PROTO = {
    "get_device_count": ctypes.CFUNCTYPE(None, vp, ctypes.POINTER(ctypes.c_int), P),
    "create_device": ctypes.CFUNCTYPE(None, vp, ctypes.POINTER(SE_CreateDeviceParams), P),
    "destroy_device": ctypes.CFUNCTYPE(None, vp, DEV),
    "create_device_fns": ctypes.CFUNCTYPE(None, vp, ctypes.POINTER(SE_CreateDeviceFnsParams), P),
    "create_stream_executor": ctypes.CFUNCTYPE(None, vp,
                                               ctypes.POINTER(SE_CreateStreamExecutorParams), P),
    "create_timer_fns": ctypes.CFUNCTYPE(None, vp, ctypes.POINTER(SP_TimerFns), P),
    "allocate": ctypes.CFUNCTYPE(None, DEV, u64, i64, MEM),
    "deallocate": ctypes.CFUNCTYPE(None, DEV, MEM),
    "host_memory_allocate": ctypes.CFUNCTYPE(vp, DEV, u64),
    "host_memory_deallocate": ctypes.CFUNCTYPE(None, DEV, vp),
    "get_allocator_stats": ctypes.CFUNCTYPE(ctypes.c_ubyte, DEV, ctypes.POINTER(SP_AllocatorStats)),
    "device_memory_usage": ctypes.CFUNCTYPE(ctypes.c_ubyte, DEV, ctypes.POINTER(i64),
                                            ctypes.POINTER(i64)),
    "create_stream": ctypes.CFUNCTYPE(None, DEV, ctypes.POINTER(vp), P),
    "destroy_stream": ctypes.CFUNCTYPE(None, DEV, vp),
    "create_stream_dependency": ctypes.CFUNCTYPE(None, DEV, vp, vp, P),
    "get_stream_status": ctypes.CFUNCTYPE(None, DEV, vp, P),
    "create_event": ctypes.CFUNCTYPE(None, DEV, ctypes.POINTER(vp), P),
    "destroy_event": ctypes.CFUNCTYPE(None, DEV, vp),
    "get_event_status": ctypes.CFUNCTYPE(ctypes.c_int, DEV, vp),
    "record_event": ctypes.CFUNCTYPE(None, DEV, vp, vp, P),
    "wait_for_event": ctypes.CFUNCTYPE(None, DEV, vp, vp, P),
    "create_timer": ctypes.CFUNCTYPE(None, DEV, ctypes.POINTER(vp), P),
    "destroy_timer": ctypes.CFUNCTYPE(None, DEV, vp),
    "start_timer": ctypes.CFUNCTYPE(None, DEV, vp, vp, P),
    "stop_timer": ctypes.CFUNCTYPE(None, DEV, vp, vp, P),
    "memcpy_dtoh": ctypes.CFUNCTYPE(None, DEV, vp, vp, MEM, u64, P),
    "memcpy_htod": ctypes.CFUNCTYPE(None, DEV, vp, MEM, vp, u64, P),
    "memcpy_dtod": ctypes.CFUNCTYPE(None, DEV, vp, MEM, MEM, u64, P),
    "sync_memcpy_dtoh": ctypes.CFUNCTYPE(None, DEV, vp, MEM, u64, P),
    "sync_memcpy_htod": ctypes.CFUNCTYPE(None, DEV, MEM, vp, u64, P),
    "sync_memcpy_dtod": ctypes.CFUNCTYPE(None, DEV, MEM, MEM, u64, P),
    "block_host_for_event": ctypes.CFUNCTYPE(None, DEV, vp, P),
    "block_host_until_done": ctypes.CFUNCTYPE(None, DEV, vp, P),
    "synchronize_all_activity": ctypes.CFUNCTYPE(None, DEV, P),
    "mem_zero": ctypes.CFUNCTYPE(None, DEV, vp, MEM, u64, P),
    "memset": ctypes.CFUNCTYPE(None, DEV, vp, MEM, ctypes.c_uint8, u64, P),
    "memset32": ctypes.CFUNCTYPE(None, DEV, vp, MEM, ctypes.c_uint32, u64, P),
    "host_callback": ctypes.CFUNCTYPE(ctypes.c_ubyte, DEV, vp, vp, vp),
    "nanoseconds": ctypes.CFUNCTYPE(u64, vp),
    "optimize_func": ctypes.CFUNCTYPE(None, vp, ctypes.POINTER(TF_Buffer), vp,
                                      ctypes.POINTER(TF_Buffer), P),
}
STATUS_CB = ctypes.CFUNCTYPE(None, vp, vp)


def fn(table, name):
    ptr = getattr(table, name)
    assert ptr, f"{name} is null"
    return PROTO[name](ptr)


class Harness:
    """The fake TF runtime and the plugin, loaded into this process."""

    def __init__(self):
        self.fake = ctypes.CDLL(FAKE_PATH, mode=ctypes.RTLD_GLOBAL)
        self.plugin = ctypes.CDLL(PLUGIN_PATH)
        f = self.fake
        f.TF_NewStatus.restype = vp
        f.TF_DeleteStatus.argtypes = [vp]
        f.TF_GetCode.argtypes = [vp]
        f.TF_Message.argtypes = [vp]
        f.TF_Message.restype = ctypes.c_char_p
        f.TF_SetStatus.argtypes = [vp, ctypes.c_int, ctypes.c_char_p]
        f.fake_kernel_describe.argtypes = [ctypes.c_int, ctypes.c_char_p, ctypes.c_int]
        f.fake_op_describe.argtypes = [ctypes.c_int, ctypes.c_char_p, ctypes.c_int]
        f.fake_op_infer.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_int),
                                    ctypes.POINTER(i64), ctypes.POINTER(ctypes.c_int),
                                    ctypes.POINTER(i64), ctypes.c_char_p, ctypes.c_int]
        f.fake_ctx_new.restype = vp
        f.fake_ctx_new.argtypes = [vp, vp, vp]
        f.fake_ctx_free.argtypes = [vp]
        f.fake_ctx_add_input.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.POINTER(i64),
                                         ctypes.c_int, ctypes.c_int]
        f.fake_ctx_attr_float.argtypes = [vp, ctypes.c_char_p, ctypes.c_float]
        f.fake_ctx_attr_bool.argtypes = [vp, ctypes.c_char_p, ctypes.c_int]
        f.fake_ctx_attr_int.argtypes = [vp, ctypes.c_char_p, i64]
        f.fake_ctx_attr_string.argtypes = [vp, ctypes.c_char_p, ctypes.c_char_p]
        f.fake_ctx_attr_type.argtypes = [vp, ctypes.c_char_p, ctypes.c_int]
        f.fake_ctx_run.argtypes = [vp, ctypes.c_int, ctypes.c_char_p, ctypes.c_int]
        f.fake_ctx_output.restype = vp
        f.fake_ctx_output.argtypes = [vp, ctypes.c_int, ctypes.POINTER(ctypes.c_int),
                                      ctypes.POINTER(ctypes.c_int), ctypes.POINTER(i64),
                                      ctypes.POINTER(ctypes.c_int)]
        f.fake_ctx_has_output.argtypes = [vp, ctypes.c_int]
        f.fake_ctx_lock_stats.argtypes = [vp] + [ctypes.POINTER(ctypes.c_int)] * 4
        f.fake_item_new.restype = vp
        f.fake_item_free.argtypes = [vp]
        f.fake_item_add_fetch.argtypes = [vp, ctypes.c_char_p]
        f.fake_item_add_preserve.argtypes = [vp, ctypes.c_char_p]
        self.plugin.SE_InitPlugin.argtypes = [ctypes.POINTER(SE_PlatformRegistrationParams), vp]
        self.plugin.TF_InitKernel.argtypes = []
        self.plugin.TF_InitGraph.argtypes = [ctypes.POINTER(TP_OptimizerRegistrationParams), vp]
        self._kernels_loaded = False

    # ---- status --------------------------------------------------------
    def status(self):
        return self.fake.TF_NewStatus()

    def code(self, s):
        return self.fake.TF_GetCode(s)

    def message(self, s):
        return self.fake.TF_Message(s).decode()

    def free(self, s):
        self.fake.TF_DeleteStatus(s)

    # ---- SE_InitPlugin -------------------------------------------------
    def init_plugin(self, struct_size=None):
        """Returns (code, message, params, platform, platform_fns)."""
        platform = SP_Platform(struct_size=full_size(SP_Platform))
        fns = SP_PlatformFns(struct_size=full_size(SP_PlatformFns))
        params = SE_PlatformRegistrationParams(
            struct_size=full_size(SE_PlatformRegistrationParams) if struct_size is None
            else struct_size, platform=ctypes.pointer(platform), platform_fns=ctypes.pointer(fns))
        s = self.status()
        self.plugin.SE_InitPlugin(ctypes.byref(params), s)
        out = (self.code(s), self.message(s), params, platform, fns)
        self.free(s)
        return out

    def device(self, fns, ordinal=0):
        dev = SP_Device(struct_size=full_size(SP_Device))
        p = SE_CreateDeviceParams(struct_size=full_size(SE_CreateDeviceParams), ordinal=ordinal,
                                  device=ctypes.pointer(dev))
        s = self.status()
        fn(fns, "create_device")(None, ctypes.byref(p), s)
        code, msg = self.code(s), self.message(s)
        self.free(s)
        assert code == TF_OK, msg
        return dev

    def stream_executor(self, fns):
        se = SP_StreamExecutor(struct_size=full_size(SP_StreamExecutor))
        p = SE_CreateStreamExecutorParams(struct_size=full_size(SE_CreateStreamExecutorParams),
                                          stream_executor=ctypes.pointer(se))
        s = self.status()
        fn(fns, "create_stream_executor")(None, ctypes.byref(p), s)
        code, msg = self.code(s), self.message(s)
        self.free(s)
        assert code == TF_OK, msg
        return se

    def call(self, table, name, *args):
        """Calls a slot that ends with a TF_Status*; returns (code, message)."""
        s = self.status()
        fn(table, name)(*args, s)
        out = self.code(s), self.message(s)
        self.free(s)
        return out

    # ---- TF_InitKernel / registry ----------------------------------------
    def init_kernels(self):
        if not self._kernels_loaded:
            self.plugin.TF_InitKernel()
            self._kernels_loaded = True

    def kernels(self):
        self.init_kernels()
        buf = ctypes.create_string_buffer(1 << 14)
        out = []
        for i in range(self.fake.fake_kernel_count()):
            self.fake.fake_kernel_describe(i, buf, len(buf))
            d = json.loads(buf.value.decode())
            d["index"] = i
            out.append(d)
        return out

    def ops(self):
        self.init_kernels()
        buf = ctypes.create_string_buffer(1 << 14)
        out = []
        for i in range(self.fake.fake_op_count()):
            self.fake.fake_op_describe(i, buf, len(buf))
            d = json.loads(buf.value.decode())
            d["index"] = i
            out.append(d)
        return out

    def kernel_index(self, op, **types):
        """Registration of `op` whose type constraints are exactly `types`
        (attr -> dtype name)."""
        want = sorted((a, DT[t]) for a, t in types.items())
        for k in self.kernels():
            if k["op"] == op and sorted(map(tuple, k["types"])) == want:
                return k["index"]
        raise KeyError(f"{op} {types} not registered")

    def infer(self, op_name, shapes):
        """Output-0 shape from op_name's shape function for input shapes (a
        tuple, or None for unknown rank); None = unknown, 'unset' = no output."""
        idx = [o["index"] for o in self.ops() if o["name"] == op_name][0]
        ranks = (ctypes.c_int * len(shapes))(*[-1 if s is None else len(s) for s in shapes])
        flat = [d for s in shapes if s is not None for d in s]
        dims = (i64 * max(1, len(flat)))(*flat)
        rank = ctypes.c_int(0)
        out = (i64 * 16)()
        msg = ctypes.create_string_buffer(512)
        code = self.fake.fake_op_infer(idx, len(shapes), ranks, dims, ctypes.byref(rank), out,
                                       msg, len(msg))
        assert code == TF_OK, msg.value
        if rank.value == -2:
            return "unset"
        if rank.value < 0:
            return None
        return tuple(out[i] for i in range(rank.value))

    # ---- TF_InitGraph --------------------------------------------------
    def init_graph(self, struct_size=None):
        configs = TP_OptimizerConfigs(struct_size=full_size(TP_OptimizerConfigs))
        opt = TP_Optimizer(struct_size=full_size(TP_Optimizer))
        params = TP_OptimizerRegistrationParams(
            struct_size=full_size(TP_OptimizerRegistrationParams) if struct_size is None
            else struct_size, optimizer_configs=ctypes.pointer(configs),
            optimizer=ctypes.pointer(opt))
        s = self.status()
        self.plugin.TF_InitGraph(ctypes.byref(params), s)
        out = (self.code(s), self.message(s), params, configs, opt)
        self.free(s)
        return out

    def optimize(self, opt, graph_bytes, fetch=(), preserve=()):
        """Runs the plugin optimizer on a serialized GraphDef; returns
        (code, message, optimized bytes)."""
        item = self.fake.fake_item_new()
        for n in fetch:
            self.fake.fake_item_add_fetch(item, n.encode())
        for n in preserve:
            self.fake.fake_item_add_preserve(item, n.encode())
        src = ctypes.create_string_buffer(graph_bytes, len(graph_bytes))
        inp = TF_Buffer(data=ctypes.cast(src, vp), length=len(graph_bytes))
        out = TF_Buffer()
        s = self.status()
        fn(opt, "optimize_func")(None, ctypes.byref(inp), item, ctypes.byref(out), s)
        code, msg = self.code(s), self.message(s)
        self.free(s)
        self.fake.fake_item_free(item)
        data = b""
        if code == TF_OK:
            data = ctypes.string_at(out.data, out.length)
            dealloc = ctypes.CFUNCTYPE(None, vp, sz)(out.data_deallocator)
            dealloc(out.data, out.length)
        return code, msg, data


class KernelRun:
    """One kernel invocation on the fake context: inputs, attrs, run,
    outputs."""

    def __init__(self, h, stream, se, dev):
        self.h = h
        self.ctx = h.fake.fake_ctx_new(stream, ctypes.addressof(se), ctypes.addressof(dev))

    def input(self, ptr, dtype, shape, variable=False, forwardable=False):
        dims = (i64 * max(1, len(shape)))(*shape)
        self.h.fake.fake_ctx_add_input(self.ctx, ptr, DT[dtype], len(shape), dims,
                                       1 if variable else 0, 1 if forwardable else 0)

    def attrs(self, **kw):
        f = self.h.fake
        for k, v in kw.items():
            name = k.encode()
            if isinstance(v, bool):
                f.fake_ctx_attr_bool(self.ctx, name, int(v))
            elif isinstance(v, int):
                f.fake_ctx_attr_int(self.ctx, name, v)
            elif isinstance(v, float):
                f.fake_ctx_attr_float(self.ctx, name, v)
            elif isinstance(v, str):
                f.fake_ctx_attr_string(self.ctx, name, v.encode())
            else:
                raise TypeError(k)

    def run(self, kernel_index):
        msg = ctypes.create_string_buffer(1024)
        code = self.h.fake.fake_ctx_run(self.ctx, kernel_index, msg, len(msg))
        return code, msg.value.decode()

    def output(self, i):
        """(device pointer, dtype code, shape, forwarded input or -1), or None."""
        if not self.h.fake.fake_ctx_has_output(self.ctx, i):
            return None
        dt, nd, fw = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        dims = (i64 * 8)()
        p = self.h.fake.fake_ctx_output(self.ctx, i, ctypes.byref(dt), ctypes.byref(nd), dims,
                                        ctypes.byref(fw))
        return p, dt.value, tuple(dims[q] for q in range(nd.value)), fw.value

    def lock_stats(self):
        v = [ctypes.c_int() for _ in range(4)]
        self.h.fake.fake_ctx_lock_stats(self.ctx, *[ctypes.byref(x) for x in v])
        return tuple(x.value for x in v)

    def free(self):
        self.h.fake.fake_ctx_free(self.ctx)
        self.ctx = None


_harness = None


def harness():
    global _harness
    if _harness is None:
        _harness = Harness()
    return _harness
