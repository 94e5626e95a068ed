"""Ops recorded into a HIP graph (stream capture through torch.cuda.graph)
and replayed.  Every replay must equal the eager run of the same iteration
bit for bit; replays are separated by eager work (other fused BatchNorm
launches, which use the eager barrier counters) and synchronizations, as a
training loop would run them."""
import pytest
import torch

import tensorflow_musa_extension_amd as tfma

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


# (16,14,14,256): every row resident, no dynamic chunks.  (128,56,56,256):
# the grad hands out phase-3 chunks, so the recorded launch zeroes the chunk
# counters as well as the barrier counters at exit; with slice_tw 8 the grad
# runs sliced (4 slices of 64 channels, eager and recorded).
@pytest.mark.parametrize("shape,slice_tw", [((16, 14, 14, 256), None),
                                            ((128, 56, 56, 256), None),
                                            ((128, 56, 56, 256), 8)])
def test_recorded_training_step_replays(dev, monkeypatch, shape, slice_tw):
    if slice_tw is not None:
        monkeypatch.setenv("TFMA_BN_SLICE_TW", str(slice_tw))
    d = _inputs(dev, shape, seed=31)
    other = _inputs(dev, (8, 7, 7, 512), seed=32)
    e = torch.empty(0, device=dev)
    start = _state(d)
    eager = []
    for _ in range(3):
        eager.append([t.clone() for t in _step(d)] + _state(d))
        if slice_tw is not None:
            assert ops.fused_batch_norm_last_plan()["slices"] == 4
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


def test_grouped_adam_refuses_capture(dev):
    vs = [torch.zeros(1000, device=dev) for _ in range(3)]
    ms = [torch.zeros(1000, device=dev) for _ in range(3)]
    vvs = [torch.zeros(1000, device=dev) for _ in range(3)]
    gs = [torch.ones(1000, device=dev) for _ in range(3)]
    ops.MusaGroupedResourceApplyAdam(vs, ms, vvs, gs, 0.9, 0.999, 1e-3, 0.9, 0.999, 1e-7)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(tfma.UnimplementedError, match="cannot be recorded into a graph"):
        with torch.cuda.graph(graph):
            ops.MusaGroupedResourceApplyAdam(vs, ms, vvs, gs, 0.9, 0.999, 1e-3, 0.9, 0.999, 1e-7)
    torch.cuda.synchronize()
