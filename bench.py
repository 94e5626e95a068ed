#!/usr/bin/env python3
"""Benchmark: achieved HBM GB/s of the fused data-parallel kernels on one GPU.

Headline workload: FusedBatchNormV3 forward +
FusedBatchNormGradV3, NHWC, is_training, epsilon 1.001e-5, at the four
ResNet-50 stage shapes [256,56,56,256], [256,28,28,512], [256,14,14,1024],
[256,7,7,2048], each in float16 and bfloat16 (float32 scale/offset/stats).
One step = the 8 forwards, then the 8 grads in the same order (no grad finds
its x still in the Infinity Cache from its forward).  Inputs are synthetic
(x, dy ~ N(0,1); scale ~ U(0.5,1.5); offset ~ N(0,0.1)), resident in HBM
before the timed region.

value = algorithmic bytes per step (fwd 2*s*E + grad 3*s*E per pair) x steps
        / wall time of the timed region (HIP events around K steps);
        elements_per_s counts each pair's E elements once for the forward and
        once for the grad.
roofline: the dominant kernel (tfma_bn_grad_fused: reads x, dy, writes dx,
        3*s*E bytes per launch) timed with HIP events on its stream for each
        of its launches in the last --trace-steps steps of the timed region
        (the events are the dispatch's own start/stop events; each costs
        ~5 us of idle GPU between kernels, so only those steps carry them).
cpu_baseline: the TF-CPU restatement (oracle/, C + OpenMP; TensorFlow is
        not installed) on the same BN workload (both dtypes, four shapes),
        repeated for >= 10 s on the box's CPU share (at most 16 threads;
        lscpu model and os.cpu_count() reported), and under "components" the
        same for Adam cfg3, a stated sample of cfg5 and the cfg4 chains.
components: cfg1 (FusedBatchNormV3 forward, f32 [32,56,56,64]), BN on the
        split path (NCHW training fwd and grad, NHWC inference), and the
        other kernels (Adam, mixed-precision Adam, grouped Adam at
        the ResNet-50 and 1.31e9-parameter configs, the elementwise chains,
        ReluGrad, BiasAddGrad) at their config shapes, each of 20 reps timed
        with HIP events after a 1 GiB read that evicts the Infinity Cache
        (median ms with min / max; GB/s, % of peak, Gelem/s from the median),
        then the same reps again with events attached to the kernels' own
        dispatches (kernel_ms, kernel_GB/s, kernel_pct_peak: the kernel's
        mean duration without the dispatch and event overhead).  The flushed
        figure stops the clock with the op's output possibly still dirty in
        the Infinity Cache; "sustained" (Adam, grouped Adam, the elementwise
        chains, ReluGrad, BiasAddGrad) is the rate of back-to-back calls
        cycling over rotating buffer sets of >= 1 GiB in total, so every call
        also pays the write-back of the ones before it (median / min / max
        of 20 timings of >= 4 calls each).  above_copy_ceiling flags a
        flushed rate above the measured stream-copy ceiling.
        traffic_ratio = counter-measured HBM bytes per rep (committed
        profiles/pmc_traffic_components.txt) / algorithmic bytes.
--bn-stamps LIB: with LIB a measurement build of the library
        (make -C tensorflow_musa_extension_amd/csrc EXTRA=-DTFMA_BN_STAMPS
        OBJDIR=../../_build/stamps OUT=../../_build/stamps/libtfma.so
        ../../_build/stamps/libtfma.so), runs the fused BatchNorm kernel at
        cfg1 and the cfg2 shapes (f16; forward, and the grads that run
        unsliced) after a cache flush and prints, per op, when its waves reach
        each phase (mean / slowest wave, microseconds from the first wave's
        start, median of 5 runs); no JSON line.
--profile-components: each component once, then 3 times after a cache
        flush, printing a PROFILE_MANIFEST line that attributes a rocprofv3
        --pmc run's dispatches to components (no JSON line).
host_path: pageable host<->device copies (256 MiB) through the library's
        staged path, beside the HIP runtime's own pageable copy and a pinned
        copy (the PCIe ceiling), in GB/s.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PEAK_GBPS = 8000.0  # MI355X HBM3E
SHAPES = [(256, 56, 56, 256), (256, 28, 28, 512), (256, 14, 14, 1024), (256, 7, 7, 2048)]
EPS = 1.001e-5


def resnet50_shapes():
    """torchvision ResNet-50 parameter shapes: 53 bias-free convs, 53 BN
    gamma/beta pairs, fc weight and bias (161 tensors, 25,557,032 params)."""
    shapes = []

    def conv_bn(cin, cout, k):
        shapes.append((cout, cin, k, k))
        shapes.append((cout,))
        shapes.append((cout,))

    conv_bn(3, 64, 7)
    cin = 64
    for width, blocks in ((64, 3), (128, 4), (256, 6), (512, 3)):
        for b in range(blocks):
            conv_bn(cin, width, 1)
            conv_bn(width, width, 3)
            conv_bn(width, width * 4, 1)
            if b == 0:
                conv_bn(cin, width * 4, 1)
            cin = width * 4
    shapes.append((1000, 2048))
    shapes.append((1000,))
    return shapes


def cfg5_shapes():
    """cfg5: 145 fp32 tensors, 1,310,982,144 parameters (24 x {4 x [2048,2048],
    [2048,8192], [8192,2048]} + [50304,2048])."""
    shapes = []
    for _ in range(24):
        shapes += [(2048, 2048)] * 4 + [(2048, 8192), (8192, 2048)]
    shapes.append((50304, 2048))
    return shapes


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-components", action="store_true",
                   help="skip the Adam / elementwise component lines")
    p.add_argument("--trace", default="tfma_bn_grad_fused",
                   help="kernel timed for the roofline object")
    p.add_argument("--trace-steps", type=int, default=2,
                   help="timed steps (the last ones) whose launches of --trace carry timing "
                        "events; each such launch costs ~5 us of idle GPU between kernels")
    p.add_argument("--bn-stamps", metavar="LIB", default=None,
                   help="phase timestamps of the fused BatchNorm kernel from a library built "
                        "with EXTRA=-DTFMA_BN_STAMPS (prints a table, no JSON)")
    p.add_argument("--profile-components", action="store_true",
                   help="run each component 1 + 3 times (cache flushed before each) and print "
                        "a PROFILE_MANIFEST line for attributing rocprofv3 counters; no JSON")
    p.add_argument("--calibrate", action="store_true",
                   help="also run a plain 256 MiB device copy (torch copy_) so a "
                        "rocprofv3 --pmc run can scale FETCH_SIZE/WRITE_SIZE")
    return p.parse_args()


def read_traffic(key, summary="pmc_traffic.txt"):
    """Counter-derived HBM bytes per launch (or per component rep) of `key`
    from a committed rocprofv3 --pmc summary under profiles/ (lines
    "<key> hbm_bytes_per_launch=<N>"), or None."""
    path = os.path.join(ROOT, "profiles", summary)
    try:
        with open(path) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 2 and parts[0] == key and parts[1].startswith(
                        "hbm_bytes_per_launch="):
                    return int(parts[1].split("=", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def _events(torch):
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def bn_workload(torch, ops, dev):
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    fwds, grads, pairs = [], [], []
    for dt in (torch.float16, torch.bfloat16):
        for shape in SHAPES:
            c = shape[-1]
            x = torch.randn(shape, generator=gen, device=dev).to(dt)
            dy = torch.randn(shape, generator=gen, device=dev).to(dt)
            scale = torch.rand(c, generator=gen, device=dev) + 0.5
            offset = 0.1 * torch.randn(c, generator=gen, device=dev)
            empty = torch.empty(0, device=dev)
            ws = torch.empty(ops.fused_batch_norm_workspace_bytes(x), dtype=torch.uint8,
                             device=dev)
            fwd = ops.bind(ops.FusedBatchNormV3, x, scale, offset, empty, empty, epsilon=EPS,
                           data_format="NHWC", is_training=True, workspace=ws)
            r = fwd.result
            grad = ops.bind(ops.FusedBatchNormGradV3, dy, x, scale, r.reserve_space_1,
                            r.reserve_space_2, r.reserve_space_3, epsilon=EPS,
                            data_format="NHWC", is_training=True, workspace=ws)
            fwds.append(fwd)
            grads.append(grad)
            pairs.append((dt, shape, x.numel(), x.element_size()))
    # A training step runs every forward, then every grad in the same order:
    # the first grad's x was read by the first forward, with all the other
    # forwards' 2.4 GB since, and each later grad's x has at least the
    # earlier grads' traffic since its forward - more than the 256 MB
    # Infinity Cache holds - so no grad finds its x cache-warm.
    return fwds + grads, pairs


def time_calls(torch, calls, steps, warmup, flush=None):
    """ms per pass over `calls`.  Without `flush`: the mean over `steps`
    back-to-back passes under one event pair.  With `flush` (a large device
    buffer): a sorted list of `steps` per-pass times, each pass timed on its
    own after reading the buffer, so the 256 MB Infinity Cache holds none of
    the op's data (cfg1 and the smaller f16 shapes would otherwise fit in
    it)."""
    for _ in range(warmup):
        for c in calls:
            c()
    torch.cuda.synchronize()
    if flush is None:
        t0, t1 = _events(torch)
        t0.record()
        for _ in range(steps):
            for c in calls:
                c()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / steps
    pairs = []
    for _ in range(steps):
        flush.sum()
        t0, t1 = _events(torch)
        t0.record()
        for c in calls:
            c()
        t1.record()
        pairs.append((t0, t1))
    torch.cuda.synchronize()
    return sorted(a.elapsed_time(b) for a, b in pairs)


def median(xs):
    xs = sorted(xs)
    k = len(xs)
    return xs[k // 2] if k % 2 else 0.5 * (xs[k // 2 - 1] + xs[k // 2])


SUSTAIN_BYTES = 1 << 30  # rotating buffer sets add up to at least this much


def time_sustained(torch, c, reps=20):
    """Sustained rate of a component: k back-to-back calls under one event
    pair, cycling over n distinct buffer sets (its own calls and n - 1 more
    from c.make()) with n * bytes >= 1 GiB, so by the time a set comes round
    again more than the 256 MB Infinity Cache has streamed through, and each
    call pays for the write-back of the dirty lines the calls before it left
    (the flushed per-call figure leaves its own output's write-back to the
    next flush).  `reps` such timings back to back; returns (sorted ms per
    call, n, k)."""
    n = max(1, min(16, -(-SUSTAIN_BYTES // c.nbytes)))
    sets = [c.calls] + [c.make() for _ in range(n - 1)]
    k = max(n, 4)
    seq = [sets[i % n] for i in range(k)]
    for calls in seq:  # one warm pass over every set
        for call in calls:
            call()
    torch.cuda.synchronize()
    pairs = []
    for _ in range(reps):
        t0, t1 = _events(torch)
        t0.record()
        for calls in seq:
            for call in calls:
                call()
        t1.record()
        pairs.append((t0, t1))
    torch.cuda.synchronize()
    ms = sorted(a.elapsed_time(b) / k for a, b in pairs)
    del sets, seq
    return ms, n, k


class Component:
    """One measured component: `calls` (bound ops run in order per rep),
    its algorithmic bytes and elements per rep, and the trace-name substring
    of the library kernels it launches."""

    def __init__(self, name, calls, nbytes, elems, kernel, reps=20, note=None, make=None):
        self.name, self.calls, self.nbytes, self.elems = name, calls, nbytes, elems
        self.kernel, self.reps, self.note = kernel, reps, note
        # make(): the same calls on a fresh set of buffers (for the sustained
        # rate over rotating buffer sets); None: no sustained figure.
        self.make = make


def component_groups(torch, ops, dev):
    """Yields the components in groups; each group's tensors are freed
    before the next is built (cfg5 alone holds 21 GB of state)."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)

    # cfg1: FusedBatchNormV3 training forward, NHWC f32 x[32,56,56,64]
    # (the reference's CPU-runnable case; epsilon 1e-3), 2*s*E bytes.
    x1 = torch.randn(32, 56, 56, 64, generator=gen, device=dev)
    sc1 = torch.rand(64, generator=gen, device=dev) + 0.5
    of1 = 0.1 * torch.randn(64, generator=gen, device=dev)
    e1 = torch.empty(0, device=dev)
    ws1 = torch.empty(ops.fused_batch_norm_workspace_bytes(x1), dtype=torch.uint8, device=dev)
    bn1 = ops.bind(ops.FusedBatchNormV3, x1, sc1, of1, e1, e1, epsilon=1e-3, data_format="NHWC",
                   is_training=True, workspace=ws1)
    yield [Component("bn_fwd_f32_cfg1_32x56x56x64", [bn1], 8 * x1.numel(), x1.numel(),
                     "tfma_bn_fwd")]
    del x1, bn1, ws1

    # BatchNorm off the NHWC fused path: NCHW training with at least one
    # channel per CU (one workgroup per channel: 2sE / 3sE algorithmic bytes,
    # plus re-reads of what a workgroup cannot hold on chip) and inference,
    # NHWC and NCHW (one apply kernel, coefficients from the running
    # statistics: 2sE).
    xn = torch.randn(256, 512, 28, 28, generator=gen, device=dev).half()
    dyn = torch.randn(256, 512, 28, 28, generator=gen, device=dev).half()
    scn = torch.rand(512, generator=gen, device=dev) + 0.5
    ofn = 0.1 * torch.randn(512, generator=gen, device=dev)
    wsn = torch.empty(ops.fused_batch_norm_workspace_bytes(xn, "NCHW"), dtype=torch.uint8,
                      device=dev)
    fn_ = ops.bind(ops.FusedBatchNormV3, xn, scn, ofn, e1, e1, epsilon=EPS, data_format="NCHW",
                   is_training=True, workspace=wsn)
    rn = fn_.result
    gn = ops.bind(ops.FusedBatchNormGradV3, dyn, xn, scn, rn.reserve_space_1, rn.reserve_space_2,
                  rn.reserve_space_3, epsilon=EPS, data_format="NCHW", is_training=True,
                  workspace=wsn)
    En = xn.numel()
    xi = torch.randn(256, 56, 56, 256, generator=gen, device=dev).half()
    rm = 0.1 * torch.randn(256, generator=gen, device=dev)
    rv = torch.rand(256, generator=gen, device=dev) + 0.5
    wsi = torch.empty(ops.fused_batch_norm_workspace_bytes(xi), dtype=torch.uint8, device=dev)
    bi = ops.bind(ops.FusedBatchNormV3, xi, scn[:256].contiguous(), ofn[:256].contiguous(), rm,
                  rv, epsilon=EPS, data_format="NHWC", is_training=False, workspace=wsi)
    rmn = 0.1 * torch.randn(512, generator=gen, device=dev)
    rvn = torch.rand(512, generator=gen, device=dev) + 0.5
    bin_ = ops.bind(ops.FusedBatchNormV3, xn, scn, ofn, rmn, rvn, epsilon=EPS, data_format="NCHW",
                    is_training=False, workspace=wsn)
    yield [Component("bn_fwd_f16_nchw_256x512x28x28", [fn_], 4 * En, En, "tfma_bn_fwd",
                     note="one workgroup per channel"),
           Component("bn_grad_f16_nchw_256x512x28x28", [gn], 6 * En, En, "tfma_bn_grad",
                     note="one workgroup per channel"),
           Component("bn_fwd_inference_f16_256x56x56x256", [bi], 4 * xi.numel(), xi.numel(),
                     "tfma_bn_infer", note="coefficients from running statistics, one kernel"),
           Component("bn_fwd_inference_f16_nchw_256x512x28x28", [bin_], 4 * En, En,
                     "tfma_bn_infer", note="NCHW, coefficients from running statistics, one kernel")]
    del xn, dyn, fn_, gn, wsn, xi, wsi, bi, bin_

    # One GPU's share of an 8-way data-parallel job (per-replica statistics,
    # no exchange): the cfg2 BatchNorms at per-replica batch 32 and cfg3's
    # Adam on 25.6M / 8 elements; the kernels only, no collective.
    share = []
    for shp in ((32, 56, 56, 256), (32, 28, 28, 512), (32, 14, 14, 1024), (32, 7, 7, 2048)):
        cs = shp[-1]
        xs_ = torch.randn(*shp, generator=gen, device=dev).half()
        dys = torch.randn(*shp, generator=gen, device=dev).half()
        scs = torch.rand(cs, generator=gen, device=dev) + 0.5
        ofs = 0.1 * torch.randn(cs, generator=gen, device=dev)
        wss = torch.empty(ops.fused_batch_norm_workspace_bytes(xs_), dtype=torch.uint8,
                          device=dev)
        fs = ops.bind(ops.FusedBatchNormV3, xs_, scs, ofs, e1, e1, epsilon=EPS,
                      data_format="NHWC", is_training=True, workspace=wss)
        rs = fs.result
        gs = ops.bind(ops.FusedBatchNormGradV3, dys, xs_, scs, rs.reserve_space_1,
                      rs.reserve_space_2, rs.reserve_space_3, epsilon=EPS, data_format="NHWC",
                      is_training=True, workspace=wss)
        Es = xs_.numel()
        tag = "x".join(map(str, shp))
        share += [Component(f"share8_bn_fwd_f16_{tag}", [fs], 4 * Es, Es, "tfma_bn_fwd",
                            note="one GPU's share of cfg2 at 8-way data parallelism"),
                  Component(f"share8_bn_grad_f16_{tag}", [gs], 6 * Es, Es, "tfma_bn_grad",
                            note="one GPU's share of cfg2 at 8-way data parallelism")]
    ns = 25_600_000 // 8

    def share_adam_set():
        var = 0.02 * torch.randn(ns, generator=gen, device=dev)
        return [ops.bind(ops.ResourceApplyAdam, var, torch.zeros_like(var), torch.zeros_like(var),
                         0.9, 0.999, 1e-3, 0.9, 0.999, 1e-7,
                         1e-3 * torch.randn(ns, generator=gen, device=dev))]

    share.append(Component("share8_adam_f32_3.2M", share_adam_set(), 28 * ns, ns,
                           "tfma_adam_flat", make=share_adam_set,
                           note="one GPU's share of cfg3 at 8-way sharding (ZeRO-1)"))
    yield share
    del share, xs_, dys, wss, fs, gs

    n = 25_600_000
    shapes = resnet50_shapes()

    def adam_set():
        var = 0.02 * torch.randn(n, generator=gen, device=dev)
        m = torch.zeros(n, device=dev)
        v = torch.zeros(n, device=dev)
        g = 1e-3 * torch.randn(n, generator=gen, device=dev)
        return [ops.bind(ops.ResourceApplyAdam, var, m, v, 0.9, 0.999, 1e-3, 0.9, 0.999, 1e-7,
                         g)]

    def mixed_set():
        # Mixed precision (fp32 state, bf16 grad): 24 B of state + 2 B of grad.
        var = 0.02 * torch.randn(n, generator=gen, device=dev)
        m = torch.zeros(n, device=dev)
        v = torch.zeros(n, device=dev)
        gb = (1e-3 * torch.randn(n, generator=gen, device=dev)).to(torch.bfloat16)
        return [ops.bind(ops.MusaResourceApplyAdamMixed, var, m, v, 0.9, 0.999, 1e-3, 0.9, 0.999,
                         1e-7, gb)]

    def grouped_set():
        tv = [0.02 * torch.randn(s, generator=gen, device=dev) for s in shapes]
        tm = [torch.zeros(s, device=dev) for s in shapes]
        tvv = [torch.zeros(s, device=dev) for s in shapes]
        tg = [1e-3 * torch.randn(s, generator=gen, device=dev) for s in shapes]
        return [ops.bind(ops.MusaGroupedResourceApplyAdam, tv, tm, tvv, tg, 0.9, 0.999, 1e-3,
                         0.9, 0.999, 1e-7)]

    total = sum(int(torch.Size(s).numel()) for s in shapes)
    yield [Component("adam_f32_25.6M", adam_set(), 28 * n, n, "tfma_adam_flat", make=adam_set),
           Component("adam_mixed_bf16grad_25.6M", mixed_set(), 26 * n, n, "tfma_adam_flat",
                     make=mixed_set),
           Component("grouped_adam_f32_resnet50_161", grouped_set(), 28 * total, total,
                     "tfma_adam_grouped", make=grouped_set)]

    # cfg5: 1.31B parameters in 145 tensors, 21 GB of state resident (one
    # step streams 36.7 GB, so the sustained rate reuses the one set).
    shapes5 = cfg5_shapes()
    tv = [0.02 * torch.randn(s, generator=gen, device=dev) for s in shapes5]
    tm = [(1e-4 * torch.randn(s, generator=gen, device=dev)).abs_() for s in shapes5]
    tvv = [(1e-4 * torch.randn(s, generator=gen, device=dev)).abs_() for s in shapes5]
    tg = [1e-3 * torch.randn(s, generator=gen, device=dev) for s in shapes5]
    total5 = sum(t.numel() for t in tv)
    grouped5 = ops.bind(ops.MusaGroupedResourceApplyAdam, tv, tm, tvv, tg, 0.9, 0.999, 1e-3,
                        0.9, 0.999, 1e-7)
    yield [Component("grouped_adam_f32_cfg5_145", [grouped5], 28 * total5, total5,
                     "tfma_adam_grouped", make=lambda: [grouped5])]
    del tv, tm, tvv, tg, grouped5
    torch.cuda.empty_cache()

    for dt, name in ((torch.float32, "f32"), (torch.float16, "f16")):
        s = torch.tensor([], dtype=dt).element_size()

        def rnd(*shape, dt=dt):
            return torch.randn(*shape, generator=gen, device=dev).to(dt)

        E = 8192 * 4096
        Eo = 8191 * 4095
        chains = [
            (f"bias_add_relu_{name}_8192x4096", 2 * s * E + s * 4096, E, "tfma_ew_add_relu",
             lambda rnd=rnd: [ops.bind(ops.MusaBiasAddRelu, rnd(8192, 4096), rnd(4096))]),
            (f"add_v2_relu_{name}_8192x4096", 2 * s * E + s * 4096, E, "tfma_ew_add_relu",
             lambda rnd=rnd: [ops.bind(ops.MusaAddV2Relu, rnd(8192, 4096), rnd(4096))]),
            (f"mul_add_full_{name}_8192x4096", 4 * s * E, E, "tfma_ew_mul_add",
             lambda rnd=rnd: [ops.bind(ops.MusaShiftedAffineMap, rnd(8192, 4096), rnd(8192, 4096),
                               rnd(8192, 4096))]),
            (f"mul_add_row_{name}_8192x4096", 2 * s * E + 2 * s * 4096, E, "tfma_ew_mul_add",
             lambda rnd=rnd: [ops.bind(ops.MusaShiftedAffineMap, rnd(8192, 4096), rnd(4096),
                               rnd(4096))]),
            (f"bias_add_relu_{name}_8191x4095", 2 * s * Eo + s * 4095, Eo, "tfma_ew_add_relu",
             lambda rnd=rnd: [ops.bind(ops.MusaBiasAddRelu, rnd(8191, 4095), rnd(4095))]),
            # The backward side of the chains: ReluGrad (2 reads, 1 write)
            # and BiasAddGrad (one read of the gradient).
            (f"relu_grad_{name}_8192x4096", 3 * s * E, E, "tfma_ew_relu_grad",
             lambda rnd=rnd: [ops.bind(ops.ReluGrad, rnd(8192, 4096), rnd(8192, 4096))]),
            (f"bias_add_grad_{name}_8192x4096", s * E + s * 4096, E, "tfma_bias_add_grad",
             lambda rnd=rnd: [ops.bind(ops.BiasAddGrad, rnd(8192, 4096))]),
        ]
        # One group per chain: its buffer sets are freed before the next.
        for cname, nbytes, elems, kernel, make in chains:
            yield [Component(cname, make(), nbytes, elems, kernel, make=make)]


def components(torch, ops, dev, copy_ceiling=None):
    """Every component at its config shape: wall time per rep (HIP events
    around it, dispatch included) after a 1 GiB read that evicts the
    Infinity Cache - median, min and max over the reps - then the kernel
    time from events on the library's own dispatches in a second pass
    (mean), and, for the cfg3 / cfg4 / cfg5 components, the sustained rate
    over rotating buffer sets (time_sustained: median, min, max).  A flushed
    figure above the measured copy ceiling (`copy_ceiling`, GB/s) is flagged:
    the op's output was still in the Infinity Cache, not yet written to HBM,
    when the timing stopped."""
    out = {}
    warm = 3
    flush = torch.ones(1 << 28, device=dev)  # 1 GiB, read between reps
    for group in component_groups(torch, ops, dev):
        for c in group:
            reps = time_calls(torch, c.calls, c.reps, warm, flush=flush)
            ms = median(reps)
            gbps = c.nbytes / (ms / 1e3) / 1e9
            ops.trace_enable(c.kernel)
            time_calls(torch, c.calls, c.reps, 0, flush=flush)
            kms, _ = ops.trace_read()
            ops.trace_enable(None)
            kms = kms / c.reps
            kgbps = c.nbytes / (kms / 1e3) / 1e9 if kms else None
            r = {"ms": round(ms, 4), "ms_min": round(reps[0], 4), "ms_max": round(reps[-1], 4),
                 "reps": len(reps), "GB/s": round(gbps, 1),
                 "pct_peak": round(100 * gbps / PEAK_GBPS, 1),
                 "Gelem/s": round(c.elems / (ms / 1e3) / 1e9, 2),
                 "kernel_ms": round(kms, 4) if kms else None,
                 "kernel_GB/s": round(kgbps, 1) if kgbps else None,
                 "kernel_pct_peak": round(100 * kgbps / PEAK_GBPS, 1) if kgbps else None}
            if c.make is not None:
                sms, nsets, k = time_sustained(torch, c)
                smed = median(sms)
                sg = c.nbytes / (smed / 1e3) / 1e9
                r["sustained"] = {
                    "ms": round(smed, 4), "ms_min": round(sms[0], 4),
                    "ms_max": round(sms[-1], 4), "reps": len(sms),
                    "GB/s": round(sg, 1), "pct_peak": round(100 * sg / PEAK_GBPS, 1),
                    "buffer_sets": nsets, "calls_per_rep": k}
            if copy_ceiling and gbps > copy_ceiling:
                r["above_copy_ceiling"] = True
            traffic = read_traffic(c.name, "pmc_traffic_components.txt")
            if traffic:
                r["traffic_ratio"] = round(traffic / c.nbytes, 3)
            if c.note:
                r["note"] = c.note
            out[c.name] = r
        del group
    torch.cuda.synchronize()
    del flush
    return out


def profile_components(torch, ops, dev, reps=3):
    """Runs every component once to warm up, then `reps` times, each after
    the 1 GiB cache flush, and prints one PROFILE_MANIFEST JSON line: per
    component (in launch order) the library dispatches per rep, so a
    rocprofv3 --pmc run of this command attributes its per-dispatch counters
    to the components (the warm-up rep's dispatches come first)."""
    manifest = []
    flush = torch.ones(1 << 28, device=dev)
    for group in component_groups(torch, ops, dev):
        for c in group:
            torch.cuda.synchronize()
            ops.trace_enable("tfma_")
            for call in c.calls:
                call()
            torch.cuda.synchronize()
            _, launches = ops.trace_read()
            ops.trace_enable(None)
            for _ in range(reps):
                flush.sum()
                for call in c.calls:
                    call()
            torch.cuda.synchronize()
            manifest.append({"name": c.name, "dispatches_per_rep": launches, "reps": reps,
                             "warmup_reps": 1, "algorithmic_bytes": c.nbytes})
        del group
    print("PROFILE_MANIFEST " + json.dumps(manifest), flush=True)


def host_path(torch, tfma, dev, mib=256, reps=5):
    """Host<->device copies of a pageable buffer through the library's staged
    path (TFMA_MemcpyHtoD / TFMA_MemcpyDtoH, synchronous), beside the HIP
    runtime's own pageable copy (torch copy_) and a pinned-source copy (the
    PCIe ceiling).  GB/s, best of `reps`."""
    import numpy as np
    se = tfma.stream_executor
    n = mib << 20
    a = np.random.default_rng(0).integers(0, 256, n, dtype=np.uint8)
    out = np.empty(n, np.uint8)
    d = torch.empty(n, dtype=torch.uint8, device=dev)
    pin = torch.from_numpy(a).pin_memory()

    def best(fn):
        fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        return round(n / min(ts) / 1e9, 1)

    r = {f"h2d_pageable_{mib}MiB": {
            "GB/s": best(lambda: se.memcpy_htod(d, a, sync=True)),
            "runtime_GB/s": best(lambda: d.copy_(torch.from_numpy(a))),
            "pinned_GB/s": best(lambda: d.copy_(pin, non_blocking=True))},
         f"d2h_pageable_{mib}MiB": {
            "GB/s": best(lambda: se.memcpy_dtoh(out, d, sync=True)),
            "runtime_GB/s": best(lambda: torch.from_numpy(out).copy_(d))}}
    if not np.array_equal(out, a):
        raise RuntimeError("host path round trip mismatch")
    return r


def cpu_model():
    """The host CPU's model name (lscpu, else /proc/cpuinfo)."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def _host(torch, t):
    """Device tensor -> numpy array (bfloat16 as uint16 bits)."""
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view("uint16")
    return t.cpu().numpy()


def _timed(fn, min_seconds):
    """Runs fn() until at least min_seconds have passed; returns (calls,
    seconds)."""
    calls, secs = 0, 0.0
    while calls == 0 or secs < min_seconds:
        t = time.perf_counter()
        fn()
        secs += time.perf_counter() - t
        calls += 1
    return calls, secs


def cpu_baseline(torch, dev, min_seconds=10.0, component_seconds=1.5):
    """The TF-CPU restatement (oracle/: C + OpenMP, on the GPU box's CPU share
    of at most 16 threads), timed on the host in the same run.  Headline: the
    bench step's BN workload (FusedBatchNormV3 + GradV3 over the four cfg2
    shapes in float16 and bfloat16) for at least `min_seconds`, run by
    oracle_baseline_bn_fwd / _grad (TF's two passes, vectorized over
    channels with F16C/AVX2 conversions; within 1 ulp of the checker).
    Adam runs oracle_baseline_adam_f32 (8-wide, the checker's bits).  Components:
    Adam cfg3 (25.6M f32, 10 steps), a sample of cfg5 (its [50304,2048]
    embedding and the first layer's six tensors, 153M parameters - the
    1.31B-parameter state would need 21 GB of host memory per pass), and the
    cfg4 chains at [8192,4096], each for at least `component_seconds`.
    The chains run oracle_baseline_rows (row loops, F16C/AVX2 half
    conversion), which gives the checker's bits on the same inputs; the
    broadcasting checker walks N-d coordinates per element and would
    understate the CPU.  Inputs are drawn on the GPU and copied to host
    memory before timing; GB/s counts the same algorithmic bytes as the GPU
    figures."""
    import numpy as np
    sys.path.insert(0, ROOT)
    from oracle import oracle
    threads = min(16, os.cpu_count() or 1)
    oracle.set_threads(threads)
    gen = torch.Generator(device=dev)
    gen.manual_seed(2)
    total_bytes, secs, passes = 0, 0.0, 0
    while passes == 0 or secs < min_seconds:
        for tdt, name in ((torch.float16, "float16"), (torch.bfloat16, "bfloat16")):
            for shape in SHAPES:
                c = shape[-1]
                x = _host(torch, torch.randn(shape, generator=gen, device=dev).to(tdt))
                dy = _host(torch, torch.randn(shape, generator=gen, device=dev).to(tdt))
                scale = np.random.default_rng(0).uniform(0.5, 1.5, c).astype(np.float32)
                offset = np.zeros(c, np.float32)
                t = time.perf_counter()
                _, sm, sv = oracle.baseline_bn_fwd(x, scale, offset, EPS, dtype=name)
                oracle.baseline_bn_grad(dy, x, scale, sm, sv, EPS, dtype=name)
                secs += time.perf_counter() - t
                total_bytes += 10 * x.size
                del x, dy
        passes += 1
    gbps = total_bytes / secs / 1e9

    comps = {}

    def rate(name, nbytes, fn, sample):
        calls, t = _timed(fn, component_seconds)
        comps[name] = {"GB/s": round(nbytes * calls / t / 1e9, 3), "seconds": round(t, 2),
                       "sample": sample}

    # Adam cfg3: 10 steps with the step's beta powers.
    n = 25_600_000
    var = _host(torch, 0.02 * torch.randn(n, generator=gen, device=dev))
    m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
    g = _host(torch, 1e-3 * torch.randn(n, generator=gen, device=dev))

    def ten_steps():
        for t_ in range(1, 11):
            oracle.baseline_adam_f32(var, m, v, g, np.float32(0.9) ** t_,
                                     np.float32(0.999) ** t_, 1e-3, 0.9, 0.999, 1e-7)

    rate("adam_f32_25.6M", 10 * 28 * n, ten_steps, "10 steps (t = 1..10) of 25.6M f32")
    del var, m, v, g
    # cfg5 sample: the embedding and layer 0's six tensors.
    shapes5 = cfg5_shapes()
    sample = [shapes5[-1]] + shapes5[:6]
    st = [[_host(torch, 0.02 * torch.randn(sh, generator=gen, device=dev)),
           _host(torch, (1e-4 * torch.randn(sh, generator=gen, device=dev)).abs_()),
           _host(torch, (1e-4 * torch.randn(sh, generator=gen, device=dev)).abs_()),
           _host(torch, 1e-3 * torch.randn(sh, generator=gen, device=dev))] for sh in sample]
    n5 = sum(a[0].size for a in st)

    def cfg5_step():
        for a in st:
            oracle.baseline_adam_f32(a[0], a[1], a[2], a[3], 0.9, 0.999, 1e-3, 0.9, 0.999, 1e-7)

    rate("grouped_adam_f32_cfg5_145", 28 * n5, cfg5_step,
         f"one step over {len(sample)} of the 145 tensors ({n5} parameters: the [50304,2048] "
         "embedding and the first layer's six), repeated")
    del st
    # cfg4 chains.
    for tdt, name, odt in ((torch.float32, "f32", "float32"), (torch.float16, "f16", "float16")):
        es = 4 if tdt == torch.float32 else 2
        x = _host(torch, torch.randn(8192, 4096, generator=gen, device=dev).to(tdt))
        b = _host(torch, torch.randn(4096, generator=gen, device=dev).to(tdt))
        a = _host(torch, torch.randn(8192, 4096, generator=gen, device=dev).to(tdt))
        c = _host(torch, torch.randn(8192, 4096, generator=gen, device=dev).to(tdt))
        E = x.size
        # BiasAdd+Relu and AddV2+Relu with a [C] row are the same row chain.
        rows = "one call of the vectorized row kernels, repeated"
        rate(f"bias_add_relu_{name}_8192x4096", 2 * es * E + es * 4096,
             lambda: oracle.baseline_rows("add_relu", x, b, dtype=odt), rows)
        rate(f"add_v2_relu_{name}_8192x4096", 2 * es * E + es * 4096,
             lambda: oracle.baseline_rows("add_relu", x, b, dtype=odt), rows)
        rate(f"mul_add_full_{name}_8192x4096", 4 * es * E,
             lambda: oracle.baseline_rows("mul_add", x, a, c, dtype=odt), rows)
        rate(f"mul_add_row_{name}_8192x4096", 2 * es * E + 2 * es * 4096,
             lambda: oracle.baseline_rows("mul_add", x, b, b, dtype=odt), rows)
        del x, b, a, c
    return {"value": round(gbps, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "label": "TF-CPU restatement, not TF (TensorFlow is not installed): vectorized "
                     "two-pass BN and row kernels, checked against the oracle",
            "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(),
            "seconds": round(secs, 2),
            "sample": f"{passes} pass(es) of FusedBatchNormV3+GradV3 over the 4 cfg2 shapes in "
                      "f16 and bf16 (the full bench step); algorithmic bytes / wall time",
            "components": comps}


def stream_copy_ceiling(torch, ops, dev, sizes=(268435456, 1 << 30, 8 << 30), reps=5):
    """The measured stream-copy ceiling (informational; every percentage is
    against 8 TB/s): a plain streaming copy (the library's TFMA_StreamCopy,
    16-byte non-temporal loads and stores) of each size, each rep after the
    1 GiB read that evicts the Infinity Cache; read+write bytes per second,
    median of `reps`."""
    flush = torch.ones(1 << 28, device=dev)
    sink = torch.empty((), device=dev)
    out = {}
    for nbytes in sizes:
        src = torch.ones(nbytes // 4, device=dev)
        dst = torch.empty_like(src)
        ops.stream_copy(dst, src)
        ts = []
        for _ in range(reps):
            torch.sum(flush, dim=0, out=sink)
            a, b = _events(torch)
            a.record()
            ops.stream_copy(dst, src)
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b))
        ts.sort()
        out[f"{nbytes >> 20}MiB"] = round(2 * nbytes / (ts[len(ts) // 2] / 1e3) / 1e9, 1)
        del src, dst
    torch.cuda.empty_cache()
    return {"GB/s": out, "note": "informational: read+write bytes of a plain 16-byte "
            "non-temporal streaming copy, Infinity Cache flushed; percentages are against "
            f"{PEAK_GBPS:.0f} GB/s"}


def calibrate(torch, dev):
    """Five plain 256 MiB device copies (torch copy_): the reference reads and
    writes that scale a rocprofv3 --pmc run's FETCH_SIZE / WRITE_SIZE."""
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


STAMP_POINTS = ["entry", "phase1", "published", "finals", "coefs", "phase3", "tail"]


def bn_stamps(torch, tfma, dev, reps=5):
    """Per-phase timing of the fused BatchNorm kernel (--bn-stamps): for each
    op, every wave's stamps relative to the launch's first wave; mean and
    slowest wave per point, median over `reps` flushed runs."""
    import ctypes

    import numpy as np
    from tensorflow_musa_extension_amd import _lib
    ops = tfma.raw_ops
    lib = _lib.load()
    flush = torch.ones(1 << 28, device=dev)
    buf = (ctypes.c_uint64 * (1024 * 64))()

    def read(blocks):
        st = _lib.TFMA_Status()
        lib.TFMA_FusedBatchNormStamps(buf, len(buf), ctypes.byref(st))
        if st.code:
            raise RuntimeError(st.message.decode())
        a = np.frombuffer(buf, dtype=np.uint64)[:blocks * 64].reshape(blocks, 8, 8)
        a = a.astype(np.int64)
        t0 = a[:, :, 0].min()
        return [((a[:, :, i] - t0).mean() / 100.0, (a[:, :, i] - t0).max() / 100.0)
                for i in range(len(STAMP_POINTS))]

    cases = [((32, 56, 56, 64), torch.float32, 1e-3, "cfg1")] + [
        (s, torch.float16, EPS, "cfg2") for s in SHAPES] + [
        ((32,) + tuple(s[1:]), torch.float16, EPS, "share8") for s in SHAPES]
    print("op | " + " | ".join(STAMP_POINTS) + "   (us, mean / slowest wave)", flush=True)
    for shape, dt, eps, cfg in cases:
        gen = torch.Generator(device=dev)
        gen.manual_seed(0)
        c = shape[-1]
        x = torch.randn(shape, generator=gen, device=dev).to(dt)
        dy = torch.randn(shape, generator=gen, device=dev).to(dt)
        sc = torch.rand(c, generator=gen, device=dev) + 0.5
        of = 0.1 * torch.randn(c, generator=gen, device=dev)
        e = torch.empty(0, device=dev)
        f = ops.FusedBatchNormV3(x, sc, of, e, e, epsilon=eps)
        for which in ("fwd", "grad"):
            runs, plan = [], None
            for _ in range(reps):
                torch.cuda.synchronize()
                flush.sum()
                if which == "fwd":
                    ops.FusedBatchNormV3(x, sc, of, e, e, epsilon=eps)
                else:
                    ops.FusedBatchNormGradV3(dy, x, sc, f.reserve_space_1, f.reserve_space_2,
                                             f.reserve_space_3, epsilon=eps)
                plan = ops.fused_batch_norm_last_plan()
                runs.append(read(min(plan["workgroups"], 1024)))
            name = (f"{cfg} {which} {'x'.join(map(str, shape))} {str(dt).split('.')[-1]} "
                    f"(workgroups {plan['workgroups']}, slices {plan['slices']}, "
                    f"dynamic rows {plan['dynamic_rows']})")
            if plan["slices"] > 1:
                print(f"{name} | sliced: the hand-off-hiding kernel records no stamps",
                      flush=True)
                continue
            med = [(float(np.median([r[i][0] for r in runs])),
                    float(np.median([r[i][1] for r in runs]))) for i in range(len(STAMP_POINTS))]
            print(name + " | " + " | ".join(f"{m:.1f} / {x_:.1f}" for m, x_ in med), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); multi-GPU runs are "
              "not part of this build.", file=sys.stderr)
        sys.exit(2)
    import torch
    sys.path.insert(0, ROOT)
    if args.bn_stamps:
        import tensorflow_musa_extension_amd._lib as _lib_mod
        _lib_mod.LIB_PATH = os.path.abspath(args.bn_stamps)
    import tensorflow_musa_extension_amd as tfma
    ops = tfma.raw_ops
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.bn_stamps:
        bn_stamps(torch, tfma, dev)
        return
    if args.profile_components:
        if args.calibrate:
            calibrate(torch, dev)
        profile_components(torch, ops, dev)
        return

    calls, pairs = bn_workload(torch, ops, dev)
    bytes_per_step = sum(5 * s * e for _, _, e, s in pairs)
    kernel_bytes_per_step = sum(3 * s * e for _, _, e, s in pairs)  # grad apply

    for _ in range(args.warmup):
        for c in calls:
            c()
    torch.cuda.synchronize()
    # The roofline kernel's launches carry HIP timing events (attached to the
    # dispatch itself) during the last trace_steps steps of the timed region.
    traced_from = max(0, args.steps - max(1, args.trace_steps))
    t0, t1 = _events(torch)
    t0.record()
    for step in range(args.steps):
        if step == traced_from:
            ops.trace_enable(args.trace)
        for c in calls:
            c()
    t1.record()
    torch.cuda.synchronize()
    traced_ms, launches = ops.trace_read()
    ops.trace_enable(None)
    ms_per_step = t0.elapsed_time(t1) / args.steps
    value = bytes_per_step / (ms_per_step / 1e3) / 1e9

    traced_steps = args.steps - traced_from
    achieved = (kernel_bytes_per_step * traced_steps / (traced_ms / 1e3) / 1e9
                if traced_ms else None)
    roofline = {
        "kernel": args.trace,
        "bound": "hbm",
        "achieved": round(achieved, 1) if achieved else None,
        "peak": PEAK_GBPS,
        "unit": "GB/s",
        "frac": round(achieved / PEAK_GBPS, 4) if achieved else None,
        "traffic": read_traffic(args.trace),
        "launches": launches,
        "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE+WRITE_SIZE, copy-calibrated)",
        "avg_launch_us": round(1e3 * traced_ms / launches, 2) if launches else None,
        "algorithmic_bytes_per_step": kernel_bytes_per_step,
        "algorithmic_bytes_per_launch": kernel_bytes_per_step // len(pairs),
    }
    result = {
        "metric": "achieved HBM GB/s (% of peak) for FusedBN fwd+grad, fused Adam, eltwise",
        "value": round(value, 1),
        "unit": "GB/s",
        "pct_of_peak": round(100 * value / PEAK_GBPS, 2),
        "elements_per_s": round(2 * sum(e for _, _, e, _ in pairs) / (ms_per_step / 1e3)),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "cfg2: FusedBatchNormV3 fwd + FusedBatchNormGradV3, NHWC, "
                        "is_training, eps=1.001e-5, f16 and bf16 x/dy, f32 stats, shapes "
                        + ", ".join("x".join(map(str, s)) for s in SHAPES),
            "bytes_per_step": bytes_per_step,
            "storage_dtypes": ["f16", "bf16"],
            "parallelism": "single GPU",
        },
        "roofline": roofline,
    }
    if args.calibrate:
        calibrate(torch, dev)
    if not args.no_components:
        result["stream_copy_ceiling"] = stream_copy_ceiling(torch, ops, dev)
        result["components"] = components(
            torch, ops, dev, copy_ceiling=max(result["stream_copy_ceiling"]["GB/s"].values()))
        result["host_path"] = host_path(torch, tfma, dev)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(torch, dev)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
