#!/usr/bin/env python3
"""Benchmark: achieved HBM GB/s of the fused data-parallel kernels on one GPU.

Headline workload: FusedBatchNormV3 forward +
FusedBatchNormGradV3, NHWC, is_training, epsilon 1.001e-5, at the four
ResNet-50 stage shapes [256,56,56,256], [256,28,28,512], [256,14,14,1024],
[256,7,7,2048], each in float16 and bfloat16 (float32 scale/offset/stats).
One step = fwd + grad for all 8 (dtype, shape) pairs.  Inputs are synthetic
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
cpu_baseline: the TF-CPU restatement (oracle/, C + OpenMP) on the same
        BN workload (both dtypes, four shapes), repeated for >= 10 s on up to
        16 host cores.
components: cfg1 (FusedBatchNormV3 forward, f32 [32,56,56,64]) and the
        other kernels (Adam, mixed-precision Adam, grouped Adam at
        the ResNet-50 and 1.31e9-parameter configs, the elementwise chains,
        ReluGrad, BiasAddGrad) at their config shapes, each rep timed with HIP
        events after a 1 GiB read that evicts the Infinity Cache (GB/s, % of
        peak, Gelem/s), then the same reps again with events attached to the
        kernels' own dispatches (kernel_ms, kernel_GB/s, kernel_pct_peak: the
        kernel's duration without the dispatch and event overhead).
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
    p.add_argument("--trace-steps", type=int, default=4,
                   help="timed steps (the last ones) whose launches of --trace carry timing "
                        "events; each such launch costs ~5 us of idle GPU between kernels")
    p.add_argument("--calibrate", action="store_true",
                   help="also run a plain 256 MiB device copy (torch copy_) so a "
                        "rocprofv3 --pmc run can scale FETCH_SIZE/WRITE_SIZE")
    return p.parse_args()


def read_traffic(kernel):
    """Counter-derived HBM bytes per launch of `kernel` from the committed
    rocprofv3 --pmc summary (profiles/pmc_traffic.txt, lines
    "<kernel> hbm_bytes_per_launch=<N>"), or None."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.txt")
    try:
        with open(path) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 2 and parts[0] == kernel and parts[1].startswith(
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
    # A training step runs every forward, then the grads in reverse order, so
    # a grad never finds its x still cache-warm from its own forward.
    return fwds + grads[::-1], pairs


def time_calls(torch, calls, steps, warmup, flush=None):
    """ms per pass over `calls`.  With `flush` (a large device buffer), each
    pass is timed on its own after reading the buffer, so the 256 MB
    Infinity Cache holds none of the op's data (the cache is flushed between
    reps: cfg1 and the smaller f16 shapes would otherwise fit in it)."""
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
    return sum(a.elapsed_time(b) for a, b in pairs) / steps


def components(torch, ops, dev):
    """Adam (cfg3), grouped Adam (cfg3b), elementwise chains (cfg4)."""
    out = {}
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    reps, warm = 20, 3
    flush = torch.ones(1 << 28, device=dev)  # 1 GiB, read between reps

    def rate(calls, nbytes, elems, kernel, reps_=reps):
        """Wall time per call (HIP events around it, which includes the
        dispatch and event overhead), then, in a second pass, the kernel time
        per call from events attached to the library's own dispatches of
        `kernel` (summed over its launches in the call)."""
        ms = time_calls(torch, calls, reps_, warm, flush=flush)
        gbps = nbytes / (ms / 1e3) / 1e9
        ops.trace_enable(kernel)
        time_calls(torch, calls, reps_, 0, flush=flush)
        kms, launches = ops.trace_read()
        ops.trace_enable(None)
        kms = kms / reps_
        kgbps = nbytes / (kms / 1e3) / 1e9 if kms else None
        return {"ms": round(ms, 4), "GB/s": round(gbps, 1),
                "pct_peak": round(100 * gbps / PEAK_GBPS, 1),
                "Gelem/s": round(elems / (ms / 1e3) / 1e9, 2),
                "kernel_ms": round(kms, 4) if kms else None,
                "kernel_GB/s": round(kgbps, 1) if kgbps else None,
                "kernel_pct_peak": round(100 * kgbps / PEAK_GBPS, 1) if kgbps else None}

    # cfg1: FusedBatchNormV3 training forward, NHWC f32 x[32,56,56,64]
    # (the reference's CPU-runnable case; epsilon 1e-3), 2*s*E bytes.
    x1 = torch.randn(32, 56, 56, 64, generator=gen, device=dev)
    sc1 = torch.rand(64, generator=gen, device=dev) + 0.5
    of1 = 0.1 * torch.randn(64, generator=gen, device=dev)
    e1 = torch.empty(0, device=dev)
    ws1 = torch.empty(ops.fused_batch_norm_workspace_bytes(x1), dtype=torch.uint8, device=dev)
    bn1 = ops.bind(ops.FusedBatchNormV3, x1, sc1, of1, e1, e1, epsilon=1e-3, data_format="NHWC",
                   is_training=True, workspace=ws1)
    out["bn_fwd_f32_cfg1_32x56x56x64"] = rate([bn1], 8 * x1.numel(), x1.numel(),
                                              "tfma_bn_fwd")
    del x1, bn1, ws1

    n = 25_600_000
    var = 0.02 * torch.randn(n, generator=gen, device=dev)
    m = torch.zeros(n, device=dev)
    v = torch.zeros(n, device=dev)
    g = 1e-3 * torch.randn(n, generator=gen, device=dev)
    adam = ops.bind(ops.ResourceApplyAdam, var, m, v, 0.9, 0.999, 1e-3, 0.9, 0.999, 1e-7, g)
    out["adam_f32_25.6M"] = rate([adam], 28 * n, n, "tfma_adam_flat")
    # Mixed precision (fp32 state, bf16 grad): 24 B of state + 2 B of grad.
    gb = g.to(torch.bfloat16)
    mixed = ops.bind(ops.MusaResourceApplyAdamMixed, var, m, v, 0.9, 0.999, 1e-3, 0.9, 0.999,
                     1e-7, gb)
    out["adam_mixed_bf16grad_25.6M"] = rate([mixed], 26 * n, n, "tfma_adam_flat")
    del gb

    shapes = resnet50_shapes()
    tv = [0.02 * torch.randn(s, generator=gen, device=dev) for s in shapes]
    tm = [torch.zeros(s, device=dev) for s in shapes]
    tvv = [torch.zeros(s, device=dev) for s in shapes]
    tg = [1e-3 * torch.randn(s, generator=gen, device=dev) for s in shapes]
    total = sum(t.numel() for t in tv)
    grouped = ops.bind(ops.MusaGroupedResourceApplyAdam, tv, tm, tvv, tg, 0.9, 0.999, 1e-3, 0.9,
                       0.999, 1e-7)
    out["grouped_adam_f32_resnet50_161"] = rate([grouped], 28 * total, total,
                                                "tfma_adam_grouped")
    del var, m, v, g, tv, tm, tvv, tg, grouped, adam, mixed

    # cfg5: 1.31B parameters in 145 tensors, 21 GB of state resident.
    shapes5 = cfg5_shapes()
    tv = [0.02 * torch.randn(s, generator=gen, device=dev) for s in shapes5]
    tm = [(1e-4 * torch.randn(s, generator=gen, device=dev)).abs_() for s in shapes5]
    tvv = [(1e-4 * torch.randn(s, generator=gen, device=dev)).abs_() for s in shapes5]
    tg = [1e-3 * torch.randn(s, generator=gen, device=dev) for s in shapes5]
    total5 = sum(t.numel() for t in tv)
    grouped5 = ops.bind(ops.MusaGroupedResourceApplyAdam, tv, tm, tvv, tg, 0.9, 0.999, 1e-3,
                        0.9, 0.999, 1e-7)
    out["grouped_adam_f32_cfg5_145"] = rate([grouped5], 28 * total5, total5,
                                            "tfma_adam_grouped", reps_=10)
    del tv, tm, tvv, tg, grouped5
    torch.cuda.empty_cache()

    for dt, name in ((torch.float32, "f32"), (torch.float16, "f16")):
        s = torch.tensor([], dtype=dt).element_size()
        x = torch.randn(8192, 4096, generator=gen, device=dev).to(dt)
        b = torch.randn(4096, generator=gen, device=dev).to(dt)
        E = x.numel()
        out[f"bias_add_relu_{name}_8192x4096"] = rate([ops.bind(ops.MusaBiasAddRelu, x, b)],
                                                      2 * s * E + s * 4096, E, "tfma_ew_add_relu")
        out[f"add_v2_relu_{name}_8192x4096"] = rate([ops.bind(ops.MusaAddV2Relu, x, b)],
                                                    2 * s * E + s * 4096, E, "tfma_ew_add_relu")
        a_full = torch.randn(8192, 4096, generator=gen, device=dev).to(dt)
        b_full = torch.randn(8192, 4096, generator=gen, device=dev).to(dt)
        out[f"mul_add_full_{name}_8192x4096"] = rate(
            [ops.bind(ops.MusaShiftedAffineMap, x, a_full, b_full)], 4 * s * E, E,
            "tfma_ew_mul_add")
        out[f"mul_add_row_{name}_8192x4096"] = rate(
            [ops.bind(ops.MusaShiftedAffineMap, x, b, b)], 2 * s * E + 2 * s * 4096, E,
            "tfma_ew_mul_add")
        xo = torch.randn(8191, 4095, generator=gen, device=dev).to(dt)
        bo = torch.randn(4095, generator=gen, device=dev).to(dt)
        out[f"bias_add_relu_{name}_8191x4095"] = rate([ops.bind(ops.MusaBiasAddRelu, xo, bo)],
                                                      2 * s * xo.numel() + s * 4095,
                                                      xo.numel(), "tfma_ew_add_relu")
        # The backward side of the chains: ReluGrad (2 reads, 1 write) and
        # BiasAddGrad (one read of the gradient).
        out[f"relu_grad_{name}_8192x4096"] = rate([ops.bind(ops.ReluGrad, a_full, x)], 3 * s * E,
                                                  E, "tfma_ew_relu_grad")
        out[f"bias_add_grad_{name}_8192x4096"] = rate([ops.bind(ops.BiasAddGrad, a_full)],
                                                      s * E + s * 4096, E, "tfma_bias_add_grad")
        del x, b, a_full, b_full, xo, bo
    torch.cuda.synchronize()
    del flush
    return out


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


def cpu_baseline(torch, dev, min_seconds=10.0):
    """TF-CPU restatement (oracle, C + OpenMP on up to 16 host cores) on the
    same workload: FusedBatchNormV3 + FusedBatchNormGradV3 over the four cfg2
    shapes in float16 and bfloat16, repeated until at least `min_seconds` of
    CPU time.  Inputs are drawn on the GPU and copied to host memory before
    timing."""
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
                x = torch.randn(shape, generator=gen, device=dev).to(tdt)
                dy = torch.randn(shape, generator=gen, device=dev).to(tdt)
                if tdt == torch.bfloat16:
                    x = x.view(torch.int16).cpu().numpy().view(np.uint16)
                    dy = dy.view(torch.int16).cpu().numpy().view(np.uint16)
                else:
                    x, dy = x.cpu().numpy(), dy.cpu().numpy()
                scale = np.random.default_rng(0).uniform(0.5, 1.5, c).astype(np.float32)
                offset = np.zeros(c, np.float32)
                t = time.perf_counter()
                _, _, _, sm, sv = oracle.bn_fwd(x, scale, offset, epsilon=EPS, dtype=name)
                oracle.bn_grad(dy, x, scale, sm, sv, epsilon=EPS, dtype=name)
                secs += time.perf_counter() - t
                total_bytes += 10 * x.size
                del x, dy
        passes += 1
    gbps = total_bytes / secs / 1e9
    return {"value": round(gbps, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "seconds": round(secs, 2),
            "sample": f"{passes} pass(es) of FusedBatchNormV3+GradV3 over the 4 cfg2 shapes in "
                      "f16 and bf16 (the full bench step); algorithmic bytes / wall time"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); multi-GPU runs are "
              "not part of this build.", file=sys.stderr)
        sys.exit(2)
    import torch
    sys.path.insert(0, ROOT)
    import tensorflow_musa_extension_amd as tfma
    ops = tfma.raw_ops
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")

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
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if not args.no_components:
        result["components"] = components(torch, ops, dev)
        result["host_path"] = host_path(torch, tfma, dev)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(torch, dev)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
