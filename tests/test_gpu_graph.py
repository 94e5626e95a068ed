"""Ops recorded into a HIP graph (stream capture through torch.cuda.graph)
and replayed.  Every replay must equal the eager run of the same iteration
bit for bit; replays are separated by eager work (other fused BatchNorm
launches, which use the eager barrier counters) and synchronizations, as a
training loop would run them."""
import numpy as np
import pytest
import torch

import tensorflow_musa_extension_amd as tfma
from oracle import oracle

pytestmark = pytest.mark.gpu
ops = tfma.raw_ops
EPS = 1.001e-5


def _inputs(dev, shape, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    c = shape[-1]
    return dict(
        x=torch.randn(shape, generator=g, device=dev).half(),
        dz=torch.randn(shape, generator=g, device=dev).half(),
        scale=torch.rand(c, generator=g, device=dev) + 0.5,
        offset=0.1 * torch.randn(c, generator=g, device=dev),
        bias=torch.randn(c, generator=g, device=dev).half(),
        var=0.02 * torch.randn(1 << 20, generator=g, device=dev),
        m=torch.zeros(1 << 20, device=dev),
        v=torch.zeros(1 << 20, device=dev),
        grad=1e-3 * torch.randn(1 << 20, generator=g, device=dev))


def _step(d):
    e = torch.empty(0, device=d["x"].device)
    f = ops.FusedBatchNormV3(d["x"], d["scale"], d["offset"], e, e, epsilon=EPS)
    z = ops.MusaBiasAddRelu(f.y, d["bias"])
    gz = ops.ReluGrad(d["dz"], z)
    db = ops.BiasAddGrad(gz)
    gr = ops.FusedBatchNormGradV3(gz, d["x"], d["scale"], f.reserve_space_1, f.reserve_space_2,
                                  f.reserve_space_3, epsilon=EPS)
    ops.ResourceApplyAdam(d["var"], d["m"], d["v"], 0.9, 0.999, 1e-3, 0.9, 0.999, 1e-7,
                          d["grad"])
    return [f.y, f.batch_mean, f.batch_variance, z, gz, db, gr.x_backprop, gr.scale_backprop,
            gr.offset_backprop]


def _state(d):
    return [d["var"].clone(), d["m"].clone(), d["v"].clone()]


# (16,14,14,256): every row resident, no dynamic chunks.  (128,56,56,256)
# unsliced (override bn_slice_tw 0): the grad hands out phase-3 chunks, so the
# recorded launch zeroes the chunk counters as well as the barrier counters
# at exit; left to the host, the grad runs in 2 slices of 128 channels
# (hand-offs hidden); with slice_tw 8 in 4 slices of 64 channels.
@pytest.mark.parametrize("shape,slice_tw,slices", [((16, 14, 14, 256), None, 1),
                                                   ((128, 56, 56, 256), 0, 1),
                                                   ((128, 56, 56, 256), None, 2),
                                                   ((128, 56, 56, 256), 8, 4)])
def test_recorded_training_step_replays(dev, tune, shape, slice_tw, slices):
    if slice_tw is not None:
        tune("bn_slice_tw", slice_tw)
    d = _inputs(dev, shape, seed=31)
    other = _inputs(dev, (8, 7, 7, 512), seed=32)
    e = torch.empty(0, device=dev)
    start = _state(d)
    eager = []
    for _ in range(3):
        eager.append([t.clone() for t in _step(d)] + _state(d))
        plan = ops.fused_batch_norm_last_plan()
        assert plan["slices"] == slices, plan
        if slice_tw == 0 and shape[1] == 56:
            assert plan["dynamic_rows"] > 0, plan
    other_ref = ops.FusedBatchNormV3(other["x"], other["scale"], other["offset"], e, e,
                                     epsilon=EPS).y.clone()
    torch.cuda.synchronize()
    for t, s in zip((d["var"], d["m"], d["v"]), start):
        t.copy_(s)
    ops.fused_batch_norm_barrier_timed_out(reset=True)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = _step(d)
    torch.cuda.synchronize()
    for want in eager:
        graph.replay()
        y_other = ops.FusedBatchNormV3(other["x"], other["scale"], other["offset"], e, e,
                                       epsilon=EPS).y
        torch.cuda.synchronize()
        got = [t.clone() for t in outs] + _state(d)
        for k, (w, g) in enumerate(zip(want, got)):
            assert torch.equal(w, g), f"output {k} of a replay differs from the eager run"
        assert torch.equal(y_other, other_ref)
    assert not ops.fused_batch_norm_barrier_timed_out()


@pytest.mark.parametrize("gdtype", [torch.float32, torch.bfloat16])
def test_grouped_adam_recorded_replays(dev, gdtype):
    """MusaGroupedResourceApplyAdam recorded into a graph (its tensor table
    travels in the kernel arguments: 100 tensors, two launches) and replayed
    three times, with eager grouped calls on other tensors between the
    replays: every replay applies one Adam step, bit for bit the oracle's."""
    g = torch.Generator(device=dev)
    g.manual_seed(41)
    sizes = [1 + (37 * k) % 5000 for k in range(100)]
    vars_ = [0.02 * torch.randn(n, generator=g, device=dev) for n in sizes]
    ms = [torch.zeros(n, device=dev) for n in sizes]
    vs = [torch.zeros(n, device=dev) for n in sizes]
    grads = [(1e-3 * torch.randn(n, generator=g, device=dev)).to(gdtype) for n in sizes]
    refs = [[t.cpu().numpy().copy() for t in (v, m, w)] for v, m, w in zip(vars_, ms, vs)]
    other = [torch.randn(4096, device=dev) for _ in range(3)]
    om = [torch.zeros(4096, device=dev) for _ in range(3)]
    ov = [torch.zeros(4096, device=dev) for _ in range(3)]
    og = [torch.randn(4096, device=dev) for _ in range(3)]
    b1p, b2p, lr, b1, b2, eps = 0.9, 0.999, 1e-3, 0.9, 0.999, 1e-7
    f32 = lambda x: float(np.float32(x))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.MusaGroupedResourceApplyAdam(vars_, ms, vs, grads, b1p, b2p, lr, b1, b2, eps)
    torch.cuda.synchronize()
    for _ in range(3):
        graph.replay()
        ops.MusaGroupedResourceApplyAdam(other, om, ov, og, b1p, b2p, lr, b1, b2, eps)
        torch.cuda.synchronize()
        for (rv, rm, rw), gt in zip(refs, grads):
            gn = gt.float().cpu().numpy()
            oracle.adam(rv, rm, rw, gn, f32(b1p), f32(b2p), f32(lr), f32(b1), f32(b2), f32(eps))
    for i, (v, m, w) in enumerate(zip(vars_, ms, vs)):
        for name, t, r in (("var", v, refs[i][0]), ("m", m, refs[i][1]), ("v", w, refs[i][2])):
            assert np.array_equal(t.cpu().numpy().view(np.uint32), r.view(np.uint32)), (i, name)
