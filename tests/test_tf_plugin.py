"""CPU tests of the TensorFlow PluggableDevice adapter (libtfma_tf.so) driven
through the fake TensorFlow C-API runtime (tests/fake_tf), in the manner of
the reference's plugin API tests (test/ops/pluggable_se_api_test.py):
exported entry points, SE_InitPlugin's struct checks and platform fields,
device enumeration without a driver, the StreamExecutor table, kernel
registrations (type constraints and HostMemory arguments of the reference's
REGISTER_KERNEL_BUILDER calls, musa_fused_batchnorm_op.cc:303-325,
musa_applyadam_op.cc:645-682, musa_applyadam_mixed_op.cc:285-300), op
definitions with their shape functions, and the graph optimizer.  Nothing
here touches a device."""
import ctypes
import os
import subprocess

import pytest

from tests import tf_harness as th
from tests.graphdef_pb import DT_FLOAT, G, nodes, parse

AMD = "/job:localhost/replica:0/task:0/device:AMDGPU:0"


@pytest.fixture(scope="module")
def h():
    return th.harness()


def test_exports_exactly_the_three_entry_points():
    out = subprocess.run(["nm", "-D", "--defined-only", th.PLUGIN_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert {"SE_InitPlugin", "TF_InitKernel", "TF_InitGraph"} <= exported
    assert not {s for s in exported if s.startswith("TFMA_")}, "C ABI belongs to libtfma.so"


def test_every_tf_import_is_declared_in_the_restated_header():
    """Each TF_* symbol the adapter imports is declared in tf_c_api.h (and
    so is implemented by the fake runtime, which would otherwise fail to
    load the adapter)."""
    out = subprocess.run(["nm", "-D", "--undefined-only", th.PLUGIN_PATH], capture_output=True,
                         text=True, check=True).stdout
    imports = {l.split()[-1] for l in out.splitlines() if l.split()[-1].startswith("TF_")}
    header = open(os.path.join(th.ROOT, "tensorflow_musa_extension_amd", "csrc",
                               "tf_c_api.h")).read()
    assert imports and all(f" {s}(" in header for s in imports), sorted(imports)


def test_se_init_plugin_platform(h):
    code, msg, params, platform, fns = h.init_plugin()
    assert code == th.TF_OK, msg
    assert (params.major_version, params.minor_version, params.patch_version) == (0, 0, 1)
    assert platform.name == b"AMDGPU_ROCM" and platform.type == b"AMDGPU"
    assert platform.use_bfc_allocator == 1
    assert platform.struct_size == th.offset_end(th.SP_Platform, "force_memory_growth")
    assert fns.struct_size == th.offset_end(th.SP_PlatformFns, "destroy_timer_fns")
    assert platform.supports_unified_memory == 0
    assert params.destroy_platform and params.destroy_platform_fns
    for name in th.PLATFORM_FNS:
        assert getattr(fns, name), name


def test_se_init_plugin_rejects_small_structs(h):
    code, msg, *_ = h.init_plugin(struct_size=8)
    assert code == th.TF_INVALID_ARGUMENT and "struct_size" in msg
    s = h.status()
    h.plugin.SE_InitPlugin(None, s)
    assert h.code(s) == th.TF_INVALID_ARGUMENT
    h.free(s)


def test_device_count_without_a_driver_is_zero_and_ok(h):
    _, _, _, _, fns = h.init_plugin()
    n = ctypes.c_int(-1)
    code, msg = h.call(fns, "get_device_count", None, ctypes.byref(n))
    assert code == th.TF_OK, msg
    assert n.value >= 0
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except ImportError:
        has_gpu = False
    if not has_gpu:
        assert n.value == 0


def test_stream_executor_table_is_complete(h):
    _, _, _, _, fns = h.init_plugin()
    se = h.stream_executor(fns)
    assert se.struct_size == th.offset_end(th.SP_StreamExecutor, "host_callback")
    for name in th.SE_FNS:
        assert getattr(se, name), f"SP_StreamExecutor.{name} is null"
    small = th.SP_StreamExecutor(struct_size=16)
    p = th.SE_CreateStreamExecutorParams(struct_size=th.full_size(th.SE_CreateStreamExecutorParams),
                                         stream_executor=ctypes.pointer(small))
    code, msg = h.call(fns, "create_stream_executor", None, ctypes.byref(p))
    assert code == th.TF_INVALID_ARGUMENT


def test_device_and_timer_function_tables(h):
    _, _, _, _, fns = h.init_plugin()
    dfns = th.SP_DeviceFns(struct_size=th.full_size(th.SP_DeviceFns))
    p = th.SE_CreateDeviceFnsParams(struct_size=th.full_size(th.SE_CreateDeviceFnsParams),
                                    device_fns=ctypes.pointer(dfns))
    assert h.call(fns, "create_device_fns", None, ctypes.byref(p))[0] == th.TF_OK
    assert dfns.get_numa_node and dfns.get_memory_bandwidth and dfns.get_gflops
    tf = th.SP_TimerFns(struct_size=th.full_size(th.SP_TimerFns))
    assert h.call(fns, "create_timer_fns", None, ctypes.byref(tf))[0] == th.TF_OK
    assert tf.nanoseconds


def _reg(h, op):
    return [k for k in h.kernels() if k["op"] == op]


def _types(k):
    return {a: t for a, t in k["types"]}


def test_batch_norm_registrations(h):
    """FusedBatchNorm, V2, V3 and their grads for T in {float, half,
    bfloat16} (U = float on V2/V3), as the reference registers all six
    (musa_fused_batchnorm_op.cc:303-325)."""
    for op in ("FusedBatchNorm", "FusedBatchNormV2", "FusedBatchNormV3", "FusedBatchNormGrad",
               "FusedBatchNormGradV2", "FusedBatchNormGradV3"):
        regs = _reg(h, op)
        assert {_types(k)["T"] for k in regs} == {th.DT["float"], th.DT["half"],
                                                  th.DT["bfloat16"]}, op
        for k in regs:
            assert k["device"] == "AMDGPU" and k["host_memory"] == []
            assert k["has_create"] and k["has_compute"] and k["has_delete"]
            if op.endswith(("V2", "V3")):
                assert _types(k)["U"] == th.DT["float"]


def test_adam_registrations_host_memory(h):
    """ResourceApplyAdam: var, m, v handles and the six scalars in host
    memory, for float, double, half, bfloat16, int64 and int32
    (musa_applyadam_op.cc:645-676); ApplyAdam: the scalars, floating types
    only (:660-681); MusaResourceApplyAdamMixed: float/half/bfloat16
    gradients (musa_applyadam_mixed_op.cc:285-300)."""
    scal = ["beta1_power", "beta2_power", "lr", "beta1", "beta2", "epsilon"]
    regs = _reg(h, "ResourceApplyAdam")
    assert {_types(k)["T"] for k in regs} == {th.DT[t] for t in ("float", "half", "bfloat16",
                                                                 "double", "int32", "int64")}
    assert {_types(k)["T"] for k in _reg(h, "ApplyAdam")} == {
        th.DT[t] for t in ("float", "half", "bfloat16", "double")}
    for k in regs:
        assert k["host_memory"] == ["var", "m", "v"] + scal
    for k in _reg(h, "ApplyAdam"):
        assert k["host_memory"] == scal
    mixed = _reg(h, "MusaResourceApplyAdamMixed")
    assert {_types(k)["T"] for k in mixed} == {th.DT[t] for t in ("float", "half", "bfloat16")}
    for k in mixed:
        assert k["host_memory"] == ["var", "m", "v"] + scal
    grouped = _reg(h, "MusaGroupedResourceApplyAdam")
    pairs = {(_types(k)["T"], _types(k)["Tgrad"]) for k in grouped}
    f, hf, bf, d = (th.DT[t] for t in ("float", "half", "bfloat16", "double"))
    assert pairs == {(f, f), (hf, hf), (bf, bf), (d, d), (f, hf), (f, bf)}
    for k in grouped:
        assert k["host_memory"] == ["vars", "ms", "vs"] + scal


def test_elementwise_registrations(h):
    """Every (op, T) pair the reference registers for these ops: AddV2 and
    Add (musa_add_op.cc:455-468, less bool), Mul (musa_multiply_op.cc:315-323),
    BiasAdd and BiasAddV1 (musa_biasadd_op.cc:67-79), Relu (musa_relu_op.cc:
    45-57), BiasAddGrad (musa_biasadd_grad_op.cc:112-123); ReluGrad takes
    double besides the reference's three; the fused ops are floating only."""
    fp = {th.DT[t] for t in ("float", "half", "bfloat16", "double")}
    i3264 = {th.DT["int32"], th.DT["int64"]}
    want = {"Relu": fp, "ReluGrad": fp, "MusaBiasAddRelu": fp, "MusaAddV2Relu": fp,
            "MusaShiftedAffineMap": fp,
            "AddV2": fp | i3264 | {th.DT["uint8"]}, "Add": fp | i3264 | {th.DT["uint8"]},
            "Mul": fp | i3264, "BiasAdd": fp | i3264, "BiasAddV1": fp | i3264,
            "BiasAddGrad": fp | i3264}
    for op, types in want.items():
        regs = _reg(h, op)
        assert len(regs) == len(types), op  # one registration per type
        assert {_types(k)["T"] for k in regs} == types, op


def test_op_definitions(h):
    ops = {o["name"]: o for o in h.ops()}
    assert set(ops) == {"MusaBiasAddRelu", "MusaAddV2Relu", "MusaShiftedAffineMap",
                        "MusaResourceApplyAdamMixed", "MusaGroupedResourceApplyAdam"}
    mixed = ops["MusaResourceApplyAdamMixed"]
    assert mixed["inputs"] == ["var: resource", "m: resource", "v: resource",
                               "beta1_power: float", "beta2_power: float", "lr: float",
                               "beta1: float", "beta2: float", "epsilon: float", "grad: T"]
    assert mixed["outputs"] == [] and mixed["stateful"]
    assert "T: {float, half, bfloat16}" in mixed["attrs"]
    g = ops["MusaGroupedResourceApplyAdam"]
    assert g["inputs"][0] == "vars: N * resource" and g["inputs"][-1] == "grads: N * Tgrad"
    assert "N: int >= 1" in g["attrs"] and g["stateful"]
    sam = ops["MusaShiftedAffineMap"]
    assert sam["inputs"] == ["data_left: T", "mask: T", "sliced_var_right: T"]
    assert all(o["has_shape_fn"] for o in ops.values())


def test_shape_functions(h):
    assert h.infer("MusaBiasAddRelu", [(8, 4), (4,)]) == (8, 4)
    assert h.infer("MusaAddV2Relu", [(8, 4), (4,)]) == (8, 4)
    assert h.infer("MusaAddV2Relu", [(4,), (3, 1, 4)]) == (3, 1, 4)
    assert h.infer("MusaAddV2Relu", [(8, 1, 4), (3, 1)]) is None  # no single input covers it
    assert h.infer("MusaAddV2Relu", [None, (4,)]) is None
    assert h.infer("MusaShiftedAffineMap", [(2, 5), (5,), (2, 1)]) == (2, 5)
    assert h.infer("MusaResourceApplyAdamMixed", [()] * 10) == "unset"


def test_statuses_are_released(h):
    before = h.fake.fake_statuses_live()
    h.init_plugin()
    h.init_graph()
    assert h.fake.fake_statuses_live() == before


def test_init_graph_registration(h):
    code, msg, params, configs, opt = h.init_graph()
    assert code == th.TF_OK, msg
    assert params.device_type == b"AMDGPU"
    assert opt.optimize_func and not opt.create_func and not opt.destroy_func
    assert configs.struct_size == th.offset_end(th.TP_OptimizerConfigs,
                                                "scoped_allocator_optimization")
    assert opt.struct_size == th.offset_end(th.TP_Optimizer, "destroy_func")
    code, msg, *_ = h.init_graph(struct_size=8)
    assert code == th.TF_INVALID_ARGUMENT


def _bias_relu_graph(device=AMD):
    return (G(device=device).node("x", "Placeholder", dtype=DT_FLOAT)
            .node("b", "Const", dtype=DT_FLOAT)
            .node("ba", "BiasAdd", ["x", "b"], T=DT_FLOAT, data_format="NHWC")
            .node("r", "Relu", ["ba"], T=DT_FLOAT).serialize())


def test_optimizer_fuses_nodes_on_the_plugin_device(h):
    _, _, _, _, opt = h.init_graph()
    code, msg, out = h.optimize(opt, _bias_relu_graph(), fetch=["r"], preserve=["r"])
    assert code == th.TF_OK, msg
    n = nodes(parse(out))
    assert n["r"].op == "MusaBiasAddRelu" and list(n["r"].input) == ["x", "b"]
    assert "ba" not in n


def test_optimizer_keeps_preserved_nodes_and_other_devices(h):
    _, _, _, _, opt = h.init_graph()
    g = _bias_relu_graph()
    # The BiasAdd is fetched: it must survive, so nothing is fused.
    code, _, out = h.optimize(opt, g, fetch=["r", "ba"], preserve=["r", "ba"])
    assert code == th.TF_OK and out == g
    cpu = _bias_relu_graph(device="/job:localhost/replica:0/task:0/device:CPU:0")
    code, _, out = h.optimize(opt, cpu, fetch=["r"])
    assert code == th.TF_OK and out == cpu


def test_optimizer_reports_malformed_graphs(h):
    _, _, _, _, opt = h.init_graph()
    code, msg, _ = h.optimize(opt, b"\x0a\xff\xff\xff")
    assert code == th.TF_INVALID_ARGUMENT


def test_python_loader_finds_the_library_and_needs_tensorflow(monkeypatch, tmp_path):
    """The loader mirrors the reference's (python/_loader.py:79-130): the
    library next to the package, an override path, a clear error when it is
    missing, and a clear error when TensorFlow cannot load it."""
    from tensorflow_musa_extension_amd import tf_plugin
    assert tf_plugin.find_plugin_library() == os.path.normpath(th.PLUGIN_PATH)
    monkeypatch.setenv("TFMA_PLUGIN_PATH", str(tmp_path / "nowhere.so"))
    assert tf_plugin.find_plugin_library() == os.path.normpath(th.PLUGIN_PATH)
    monkeypatch.setenv("TFMA_PLUGIN_PATH", th.PLUGIN_PATH)
    assert tf_plugin.find_plugin_library() == os.path.normpath(th.PLUGIN_PATH)
    monkeypatch.setattr(tf_plugin, "__file__", str(tmp_path / "tf_plugin.py"))
    monkeypatch.delenv("TFMA_PLUGIN_PATH")
    with pytest.raises(FileNotFoundError, match="libtfma_tf.so"):
        tf_plugin.find_plugin_library()
    monkeypatch.undo()
    try:
        import tensorflow  # noqa: F401
        pytest.skip("TensorFlow is installed: loading is exercised for real")
    except ImportError:
        with pytest.raises(RuntimeError, match="load_pluggable_device_library"):
            tf_plugin.load_plugin()
        assert not tf_plugin.is_plugin_loaded()
