"""The GraphDef rewrite (TFMA_OptimizeGraph), on the CPU.

Structural assertions in the manner of the reference's fusion tests
(test/fusion/linear_relu_fusion_test.py, test/fusion/rgprojection_fusion_test.py:127-258):
the fused node is present; name, device and control edges are preserved; the
absorbed node is gone; negative cases with several consumers, an intervening
op, a device or dtype mismatch or a fetched intermediate leave the graph
alone.  On top of those, seeded random graphs are run through a small float64
interpreter before and after the rewrite: every node that survives must
compute the same value, every edge must resolve, and the graph must stay
acyclic (the grouped Adam node merges nodes, so cycles are the failure to
look for).
"""
import numpy as np
import pytest

from tensorflow_musa_extension_amd import errors
from tensorflow_musa_extension_amd.graph_rewrite import optimize_graph_def
from tests.graphdef_pb import DT_DOUBLE, DT_FLOAT, DT_HALF, G, nodes, parse

CPU = "/job:localhost/replica:0/task:0/device:CPU:0"


def run(g, **kw):
    out, stats = optimize_graph_def(g.serialize(), **kw)
    return parse(out), stats


def producer(inp):
    name = inp[1:] if inp.startswith("^") else inp
    if ":" in name and name.rsplit(":", 1)[1].isdigit():
        name = name.rsplit(":", 1)[0]
    return name


def check_well_formed(gd):
    """Every input resolves to a node and the graph is acyclic."""
    by = nodes(gd)
    assert len(by) == len(gd.node), "duplicate node names"
    indeg = {n.name: 0 for n in gd.node}
    succ = {n.name: [] for n in gd.node}
    for n in gd.node:
        seen_control = False
        for i in n.input:
            p = producer(i)
            assert p in by, f"{n.name} reads missing node {i}"
            succ[p].append(n.name)
            indeg[n.name] += 1
            if i.startswith("^"):
                seen_control = True
            else:
                assert not seen_control, f"{n.name}: data input after a control input"
    order = [k for k, d in indeg.items() if d == 0]
    for k in order:
        for s in succ[k]:
            indeg[s] -= 1
            if indeg[s] == 0:
                order.append(s)
    assert len(order) == len(gd.node), "rewritten graph has a cycle"
    return order


def base(g=None, t=DT_FLOAT):
    g = g or G()
    return (g.node("x", "Placeholder", dtype=t).node("y", "Placeholder", dtype=t)
            .node("b", "Const", dtype=t).node("init", "NoOp"))


# ---------------------------------------------------------------------------
# Relu(BiasAdd)
# ---------------------------------------------------------------------------
def test_bias_add_relu_fused_preserving_name_device_and_control_edges():
    g = base().node("ba", "BiasAdd", ["x", "b", "^init"], T=DT_FLOAT, data_format="NCHW")
    g.node("r", "Relu", ["ba", "^y"], T=DT_FLOAT).node("out", "Identity", ["r:0"], T=DT_FLOAT)
    g.node("after", "NoOp", ["^ba"])
    gd, stats = run(g)
    check_well_formed(gd)
    by = nodes(gd)
    assert "ba" not in by and stats["bias_add_relu"] == 1
    r = by["r"]
    assert r.op == "MusaBiasAddRelu" and r.device == g.device
    assert list(r.input) == ["x", "b", "^y", "^init"]
    assert r.attr["T"].type == DT_FLOAT and r.attr["data_format"].s == b"NCHW"
    assert list(by["out"].input) == ["r:0"]
    assert list(by["after"].input) == ["^r"]  # control consumer of the absorbed node
    assert gd.versions.producer == 1205


def test_bias_add_default_format_and_v1():
    g = base().node("ba", "BiasAddV1", ["x", "b"], T=DT_HALF).node("r", "Relu", ["ba"], T=DT_HALF)
    gd, _ = run(g)
    assert nodes(gd)["r"].op == "MusaBiasAddRelu"
    assert nodes(gd)["r"].attr["data_format"].s == b"NHWC"


@pytest.mark.parametrize("case", ["two_consumers", "intervening", "device", "dtype_mismatch",
                                  "int_dtype", "fetched", "filtered", "disabled", "control_only"])
def test_bias_add_relu_negative(case):
    g = base()
    t_ba = DT_FLOAT
    dev_ba = None
    if case == "dtype_mismatch":
        t_ba = DT_HALF
    if case == "int_dtype":
        t_ba = 3
    if case == "device":
        dev_ba = CPU
    g.node("ba", "BiasAdd", ["x", "b"], device=dev_ba, T=t_ba)
    src = "ba"
    if case == "intervening":
        g.node("id", "Identity", ["ba"], T=DT_FLOAT)
        src = "id"
    t_relu = DT_FLOAT if case == "dtype_mismatch" else t_ba
    if case == "control_only":
        g.node("r", "Relu", ["x", "^ba"], T=t_relu)
    else:
        g.node("r", "Relu", [src], T=t_relu)
    if case == "two_consumers":
        g.node("other", "Identity", ["ba"], T=DT_FLOAT)
    kw = {}
    if case == "fetched":
        kw["fetch"] = ["ba:0"]
    if case == "filtered":
        kw["device_filter"] = "GPU"
    if case == "disabled":
        kw["disabled_patterns"] = ["MusaBiasAddRelu"]
    gd, stats = run(g, **kw)
    assert nodes(gd)["r"].op == "Relu" and "ba" in nodes(gd)
    assert stats["bias_add_relu"] == 0
    assert gd.SerializeToString() == g.serialize()  # untouched byte for byte


def test_device_filter_selects_nodes():
    g = base().node("ba", "BiasAdd", ["x", "b"], T=DT_FLOAT).node("r", "Relu", ["ba"], T=DT_FLOAT)
    g.node("ba2", "BiasAdd", ["y", "b"], device=CPU, T=DT_FLOAT)
    g.node("r2", "Relu", ["ba2"], device=CPU, T=DT_FLOAT)
    gd, stats = run(g, device_filter="MUSA")
    assert nodes(gd)["r"].op == "MusaBiasAddRelu" and nodes(gd)["r2"].op == "Relu"
    assert stats["bias_add_relu"] == 1


def test_chain_reaches_fixed_point():
    g = base()
    prev = "x"
    for i in range(6):
        g.node(f"ba{i}", "BiasAdd", [prev, "b"], T=DT_FLOAT)
        g.node(f"r{i}", "Relu", [f"ba{i}"], T=DT_FLOAT)
        prev = f"r{i}"
    gd, stats = run(g)
    check_well_formed(gd)
    assert stats["bias_add_relu"] == 6
    assert [n.op for n in gd.node if n.name.startswith("r")] == ["MusaBiasAddRelu"] * 6
    assert list(nodes(gd)["r3"].input) == ["r2", "b"]


# ---------------------------------------------------------------------------
# Relu(AddV2) and AddV2(Mul)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("add_op", ["AddV2", "Add"])
def test_add_relu_fused(add_op):
    g = base().node("a", add_op, ["x", "y", "^init"], T=DT_FLOAT)
    g.node("r", "Relu", ["a"], T=DT_FLOAT)
    gd, stats = run(g)
    r = nodes(gd)["r"]
    assert r.op == "MusaAddV2Relu" and list(r.input) == ["x", "y", "^init"]
    assert "a" not in nodes(gd) and stats["add_v2_relu"] == 1


# ---------------------------------------------------------------------------
# AddV2(Mul(Const, mask), Const) -> MusaShiftedAffineMap, the reference's
# topology (musa_ext/graph/fusion/shifted_affine_map_fusion.cc:109-233; its
# graphs, test/fusion/shifted_affine_map_fusion_test.py:59-100)
# ---------------------------------------------------------------------------
DT_INT32, DT_BOOL = 3, 10


def affine_graph(mask_op="Select", identities=True, mul_order=0, add_order=0, t=DT_FLOAT,
                 sink=True):
    """mask = Select(cond, ones, zeros); out = AddV2(Mul(left, mask), right),
    left and right Consts read directly or through Identity nodes (the
    reference's frozen-graph form)."""
    g = G()
    g.node("cond", "Placeholder", dtype=DT_BOOL).node("ones", "Const", dtype=t)
    g.node("zeros", "Const", dtype=t).node("init", "NoOp")
    g.node("mask", mask_op, ["cond", "ones", "zeros"], T=t)
    g.node("left", "Const", dtype=t).node("right", "Const", dtype=t)
    left, right = "left", "right"
    if identities:
        g.node("id_left", "Identity", ["left"], T=t).node("id_right", "Identity", ["right"], T=t)
        left, right = "id_left", "id_right"
    g.node("mul", "Mul", [left, "mask"] if mul_order == 0 else ["mask", left], T=t)
    g.node("out", "AddV2", ["mul", right] if add_order == 0 else [right, "mul"], T=t)
    if sink:
        g.node("sink", "Identity", ["out"], T=t)
    return g, left, right


@pytest.mark.parametrize("identities", [True, False])
@pytest.mark.parametrize("mul_order", [0, 1])
@pytest.mark.parametrize("add_order", [0, 1])
@pytest.mark.parametrize("mask_op", ["Select", "SelectV2", "Identity"])
def test_shifted_affine_map_reference_topology(identities, mul_order, add_order, mask_op):
    g, left, right = affine_graph(mask_op, identities, mul_order, add_order)
    gd, stats = run(g)
    check_well_formed(gd)
    by = nodes(gd)
    out = by["out"]
    assert out.op == "MusaShiftedAffineMap" and stats["mul_add"] == 1
    assert list(out.input) == [left, "mask", right]
    assert out.device.endswith("MUSA:0") and out.attr["T"].type == DT_FLOAT
    assert "mul" not in by and list(by["sink"].input) == ["out"]


def test_shifted_affine_map_keeps_a_shared_or_fetched_mul():
    """The reference fuses whatever else reads the Mul and keeps the Mul then
    (FusionGraphUtils::RemoveNodesIfUnused); a fetched Mul is kept too."""
    g, left, right = affine_graph()
    g.node("other", "Identity", ["mul"], T=DT_FLOAT)
    gd, stats = run(g)
    by = nodes(gd)
    assert by["out"].op == "MusaShiftedAffineMap" and by["mul"].op == "Mul"
    assert list(by["other"].input) == ["mul"] and stats["mul_add"] == 1
    g, left, right = affine_graph()
    gd, stats = run(g, fetch=["mul"])
    by = nodes(gd)
    assert by["out"].op == "MusaShiftedAffineMap" and by["mul"].op == "Mul"


def test_shifted_affine_map_double():
    g, left, right = affine_graph(t=DT_DOUBLE)
    gd, stats = run(g)
    assert nodes(gd)["out"].op == "MusaShiftedAffineMap"
    assert nodes(gd)["out"].attr["T"].type == DT_DOUBLE


def _unfused(g, **kw):
    before = [(n.name, n.op, list(n.input)) for n in g.gd.node]
    gd, stats = run(g, **kw)
    assert stats["mul_add"] == 0
    assert [(n.name, n.op, list(n.input)) for n in gd.node] == before


def test_shifted_affine_map_not_applied_when_pattern_incomplete():
    """The reference's negative case (shifted_affine_map_fusion_test.py:215-242):
    a plain Mul of two placeholders plus a constant is not fused; nor is any
    other graph its matcher rejects."""
    g = G().node("a", "Placeholder", dtype=DT_FLOAT).node("b", "Placeholder", dtype=DT_FLOAT)
    g.node("one", "Const", dtype=DT_FLOAT).node("m", "Mul", ["a", "b"], T=DT_FLOAT)
    g.node("incomplete_output", "AddV2", ["m", "one"], T=DT_FLOAT)
    _unfused(g)
    # Add, not AddV2
    g, _, _ = affine_graph()
    nodes(g.gd)["out"].op = "Add"
    _unfused(g)
    # the AddV2 with a control input (three inputs)
    g, _, _ = affine_graph()
    nodes(g.gd)["out"].input.append("^init")
    _unfused(g)
    # right operand not a Const
    g, _, right = affine_graph(identities=False)
    g.node("p", "Placeholder", dtype=DT_FLOAT)
    out = nodes(g.gd)["out"]
    out.input[1] = "p"
    _unfused(g)
    # the Mul's non-constant operand not a mask op
    g, _, _ = affine_graph(mask_op="Relu")
    _unfused(g)
    # a type the op is not registered for
    g, _, _ = affine_graph(t=DT_INT32)
    _unfused(g)
    # a Mul of three inputs (a control one)
    g, _, _ = affine_graph()
    nodes(g.gd)["mul"].input.append("^init")
    _unfused(g)


def test_priority_bias_relu_before_mul_add():
    # Relu(AddV2(Mul(left, mask), right)): AddV2+Relu (priority 90) wins over
    # Mul+Add (80).
    g, left, right = affine_graph(sink=False)
    g.node("r", "Relu", ["out"], T=DT_FLOAT)
    gd, stats = run(g)
    assert nodes(gd)["r"].op == "MusaAddV2Relu" and nodes(gd)["mul"].op == "Mul"
    assert stats == dict(stats, add_v2_relu=1, mul_add=0)
    gd, stats = run(g, disabled_patterns=["MusaAddV2Relu"])
    assert nodes(gd)["out"].op == "MusaShiftedAffineMap" and nodes(gd)["r"].op == "Relu"


# ---------------------------------------------------------------------------
# Grouped ResourceApplyAdam
# ---------------------------------------------------------------------------
SCALARS = ["b1p", "b2p", "lr", "b1", "b2", "eps"]


def adam_graph(n, t=DT_FLOAT, scalars=None, nesterov=None, deps=(), shared_var=False):
    g = G()
    for s in SCALARS:
        g.node(s, "Const", dtype=t)
    g.node("init", "NoOp")
    for i in range(n):
        for r in ("var", "m", "v"):
            g.node(f"{r}{i}", "VarHandleOp", dtype=t)
        g.node(f"g{i}", "Placeholder", dtype=t)
    for i in range(n):
        sc = (scalars or {}).get(i, SCALARS)
        var = "var0" if shared_var and i == 1 else f"var{i}"
        ins = [var, f"m{i}", f"v{i}"] + sc + [f"g{i}", "^init"]
        ins += [f"^adam{j}" for a, j in deps if a == i]
        attrs = dict(T=t, use_locking=False,
                     use_nesterov=bool((nesterov or {}).get(i, False)))
        g.node(f"adam{i}", "ResourceApplyAdam", ins, **attrs)
    g.node("train", "NoOp", [f"^adam{i}" for i in range(n)])
    return g


def test_adam_grouped_in_one_node():
    gd, stats = run(adam_graph(5))
    check_well_formed(gd)
    assert stats["adam_groups"] == 1 and stats["adam_grouped_nodes"] == 5
    grp = [n for n in gd.node if n.op == "MusaGroupedResourceApplyAdam"]
    assert len(grp) == 1 and not [n for n in gd.node if n.op == "ResourceApplyAdam"]
    gn = grp[0]
    assert gn.name == "adam0/MusaGroupedResourceApplyAdam" and gn.device == G().device
    want = ([f"var{i}" for i in range(5)] + [f"m{i}" for i in range(5)] +
            [f"v{i}" for i in range(5)] + SCALARS + [f"g{i}" for i in range(5)] + ["^init"])
    assert list(gn.input) == want
    assert gn.attr["N"].i == 5 and gn.attr["T"].type == DT_FLOAT
    assert gn.attr["use_locking"].b is False and gn.attr["use_nesterov"].b is False
    assert list(nodes(gd)["train"].input) == ["^" + gn.name]


def test_adam_groups_split_by_scalars_dtype_and_attrs():
    other = ["b1p", "b2p", "lr", "b1", "b2", "b1p"]  # a different epsilon tensor
    g = adam_graph(6, scalars={4: other, 5: other}, nesterov={2: True, 3: True})
    gd, stats = run(g)
    check_well_formed(gd)
    groups = sorted(n.attr["N"].i for n in gd.node if n.op == "MusaGroupedResourceApplyAdam")
    assert groups == [2, 2, 2] and stats["adam_grouped_nodes"] == 6


def test_adam_scalar_port_spelling_is_one_tensor():
    sc = ["b1p:0", "b2p", "lr:0", "b1", "b2", "eps"]
    gd, stats = run(adam_graph(3, scalars={1: sc}))
    assert stats["adam_groups"] == 1 and stats["adam_grouped_nodes"] == 3


def test_adam_dependent_nodes_not_grouped():
    # adam2 waits on adam0: the two cannot be one node.
    gd, stats = run(adam_graph(3, deps=[(2, 0)]))
    check_well_formed(gd)
    assert stats["adam_groups"] == 1 and stats["adam_grouped_nodes"] == 2
    assert nodes(gd)["adam2"].op == "ResourceApplyAdam"
    grp = [n for n in gd.node if n.op == "MusaGroupedResourceApplyAdam"][0]
    assert "^" + grp.name in nodes(gd)["adam2"].input  # edge to the member moved to the group


def test_adam_groups_never_close_a_cycle():
    # Key A = {adam0, adam1} (scalars S), key B = {adam2, adam3} (scalars S').
    # adam0 -> adam2 and adam3 -> adam1: grouping both keys would be a cycle.
    other = ["b1p", "b2p", "lr", "b1", "b2", "b1p"]
    g = adam_graph(4, scalars={2: other, 3: other}, deps=[(2, 0), (1, 3)])
    gd, stats = run(g)
    check_well_formed(gd)
    assert stats["adam_groups"] == 1 and stats["adam_grouped_nodes"] == 2


def test_adam_shared_resource_not_grouped_twice():
    gd, stats = run(adam_graph(3, shared_var=True))
    check_well_formed(gd)
    assert stats["adam_grouped_nodes"] == 2
    assert nodes(gd)["adam1"].op == "ResourceApplyAdam"


def test_adam_not_grouped_when_fetched_filtered_or_disabled():
    for kw in (dict(fetch=["adam1"]), dict(device_filter="GPU"),
               dict(disabled_patterns=["MusaGroupedResourceApplyAdam"])):
        gd, stats = run(adam_graph(2), **kw)
        assert stats["adam_groups"] == 0, kw


def test_adam_resnet50_scale():
    gd, stats = run(adam_graph(161))
    check_well_formed(gd)
    assert stats["adam_groups"] == 1 and stats["adam_grouped_nodes"] == 161


# ---------------------------------------------------------------------------
# Wire-level behaviour and errors
# ---------------------------------------------------------------------------
def test_unknown_fields_and_empty_graph_are_preserved():
    g = base().node("ba", "BiasAdd", ["x", "b"], T=DT_FLOAT).node("r", "Relu", ["ba"], T=DT_FLOAT)
    library = b"\x12\x05\x0a\x03abc"  # GraphDef field 2 (library), opaque to the pass
    out, stats = optimize_graph_def(g.serialize() + library)
    assert out.endswith(library) and stats["bias_add_relu"] == 1
    assert optimize_graph_def(b"")[0] == b""


def test_idempotent():
    g = base().node("ba", "BiasAdd", ["x", "b"], T=DT_FLOAT).node("r", "Relu", ["ba"], T=DT_FLOAT)
    once, _ = optimize_graph_def(adam_graph(4).serialize() + g.serialize())
    twice, stats = optimize_graph_def(once)
    assert twice == once and not any(stats.values())


@pytest.mark.parametrize("data", [b"\x0a\x05\x0a\x01", b"\x0a", b"\xff\xff\xff\xff\xff\xff\xff\xff\xff\xff\xff"])
def test_malformed_graph_def(data):
    with pytest.raises(errors.InvalidArgumentError, match="malformed GraphDef"):
        optimize_graph_def(data)


def test_unknown_pattern_name():
    with pytest.raises(ValueError):
        optimize_graph_def(b"", disabled_patterns=["NoSuchFusion"])


# ---------------------------------------------------------------------------
# Random graphs: values of surviving nodes are unchanged.
# ---------------------------------------------------------------------------
def evaluate(gd, feeds):
    by = nodes(gd)
    vals = {}
    for name in check_well_formed(gd):
        n = by[name]
        a = [vals[producer(i)] for i in n.input if not i.startswith("^")]
        op = n.op
        if op in ("Placeholder", "Const"):
            vals[name] = feeds[name]
        elif op == "NoOp":
            vals[name] = None
        elif op == "Identity":
            vals[name] = a[0]
        elif op in ("BiasAdd", "AddV2", "Add"):
            vals[name] = a[0] + a[1]
        elif op == "Mul":
            vals[name] = a[0] * a[1]
        elif op == "Select":
            vals[name] = np.where(a[0], a[1], a[2])
        elif op == "Relu":
            vals[name] = np.maximum(a[0], 0.0)
        elif op in ("MusaBiasAddRelu", "MusaAddV2Relu"):
            vals[name] = np.maximum(a[0] + a[1], 0.0)
        elif op == "MusaShiftedAffineMap":
            vals[name] = a[0] * a[1] + a[2]
        else:
            raise AssertionError(f"unexpected op {op}")
    return vals


def random_graph(rng, n_ops=60):
    g = G()
    full, feeds = [], {}
    for i in range(3):
        g.node(f"p{i}", "Placeholder", dtype=DT_FLOAT)
        full.append(f"p{i}")
        feeds[f"p{i}"] = rng.standard_normal((4, 6))
    for i in range(2):
        g.node(f"c{i}", "Const", dtype=DT_FLOAT)
        feeds[f"c{i}"] = rng.standard_normal(6)
    g.node("q", "Placeholder", dtype=DT_BOOL)
    feeds["q"] = rng.random((4, 6)) < 0.5
    allnames = list(full)
    for k in range(n_ops):
        name = f"n{k}"
        op = rng.choice(["BiasAdd", "Relu", "Relu", "AddV2", "Add", "Mul", "Identity", "Select",
                         "Affine"])
        recent = full[-6:]
        pick = lambda: str(rng.choice(recent if rng.random() < 0.7 else full))
        if op == "Affine":
            # AddV2(Mul(Const, mask), Const) in a random arrangement: operand
            # order, Identity nodes in front of the Consts, Select or Identity
            # as the mask; later nodes may read the Mul or the AddV2 too.
            def const_edge(tag):
                c = f"c{rng.integers(2)}"
                if rng.random() < 0.5:
                    g.node(f"{name}_{tag}", "Identity", [c], T=DT_FLOAT)
                    return f"{name}_{tag}"
                return c
            mask_op = "Select" if rng.random() < 0.7 else "Identity"
            g.node(f"{name}_mask", mask_op,
                   ["q", pick(), pick()] if mask_op == "Select" else [pick()], T=DT_FLOAT)
            left = const_edge("l")
            mul_in = [left, f"{name}_mask"]
            g.node(f"{name}_mul", "Mul", mul_in if rng.random() < 0.5 else mul_in[::-1],
                   T=DT_FLOAT)
            add_in = [f"{name}_mul", const_edge("r")]
            g.node(name, "AddV2", add_in if rng.random() < 0.5 else add_in[::-1], T=DT_FLOAT)
            for extra in (f"{name}_mask", f"{name}_mul"):
                full.append(extra)
                allnames.append(extra)
            full.append(name)
            allnames.append(name)
            continue
        if op == "BiasAdd":
            ins = [pick(), f"c{rng.integers(2)}"]
        elif op in ("Relu", "Identity"):
            ins = [pick()]
        elif op == "Select":
            ins = ["q", pick(), pick()]
        else:
            ins = [pick(), pick() if rng.random() < 0.8 else f"c{rng.integers(2)}"]
        if rng.random() < 0.5:
            ins = [i + ":0" if rng.random() < 0.3 else i for i in ins]
        if rng.random() < 0.15:
            ins.append("^" + str(rng.choice(allnames)))
        dev = CPU if rng.random() < 0.08 else None
        t = DT_DOUBLE if rng.random() < 0.05 else DT_FLOAT
        g.node(name, op, ins, device=dev, T=t)
        full.append(name)
        allnames.append(name)
    fetch = [str(f) for f in rng.choice(full, size=4, replace=False)]
    return g, feeds, fetch


@pytest.mark.parametrize("seed", range(40))
def test_random_graphs_keep_values(seed):
    rng = np.random.default_rng(seed)
    g, feeds, fetch = random_graph(rng)
    before = evaluate(g.gd, feeds)
    gd, stats = run(g, fetch=fetch)
    after = evaluate(gd, feeds)
    assert set(fetch) <= set(after)
    for name, v in after.items():
        if v is not None:
            np.testing.assert_array_equal(v, before[name], err_msg=name)
    # Each fusion removes its absorbed node, except that Mul+Add keeps a Mul
    # something else still reads.
    removed = len(g.gd.node) - len(gd.node)
    assert stats["bias_add_relu"] + stats["add_v2_relu"] <= removed
    assert removed <= stats["bias_add_relu"] + stats["add_v2_relu"] + stats["mul_add"]
    assert optimize_graph_def(gd.SerializeToString(), fetch=fetch)[1]["bias_add_relu"] == 0


# ---------------------------------------------------------------------------
# Cast folding into MusaResourceApplyAdamMixed (reference MusaAdamMixedFusion)
# ---------------------------------------------------------------------------
DT_BF16 = 14


def mixed_graph(n, src=DT_HALF, dst=DT_FLOAT, t=DT_FLOAT, extra_cast_consumer=False):
    g = G()
    for s in SCALARS:
        g.node(s, "Const", dtype=DT_FLOAT)
    for i in range(n):
        for r in ("var", "m", "v"):
            g.node(f"{r}{i}", "VarHandleOp", dtype=DT_FLOAT)
        g.node(f"g{i}", "Placeholder", dtype=src)
        g.node(f"cast{i}", "Cast", [f"g{i}", "^init"] if i == 0 else [f"g{i}"], SrcT=src, DstT=dst)
    g.node("init", "NoOp")
    for i in range(n):
        g.node(f"adam{i}", "ResourceApplyAdam",
               [f"var{i}", f"m{i}", f"v{i}"] + SCALARS + [f"cast{i}"],
               T=t, use_locking=False, use_nesterov=False)
    if extra_cast_consumer:
        g.node("probe", "Identity", ["cast0"], T=dst)
    return g


def test_cast_folded_into_mixed_adam():
    gd, stats = run(mixed_graph(1), disabled_patterns=["MusaGroupedResourceApplyAdam"])
    check_well_formed(gd)
    a = nodes(gd)["adam0"]
    assert a.op == "MusaResourceApplyAdamMixed" and a.attr["T"].type == DT_HALF
    assert list(a.input) == ["var0", "m0", "v0"] + SCALARS + ["g0", "^init"]
    assert "cast0" not in nodes(gd) and stats["adam_mixed"] == 1


def test_cast_with_other_consumer_is_kept():
    gd, stats = run(mixed_graph(1, src=DT_BF16, extra_cast_consumer=True))
    a = nodes(gd)["adam0"]
    assert a.op == "MusaResourceApplyAdamMixed" and a.attr["T"].type == DT_BF16
    assert a.input[9] == "g0" and "cast0" in nodes(gd)
    assert list(nodes(gd)["probe"].input) == ["cast0"]


@pytest.mark.parametrize("kw", [dict(src=DT_FLOAT), dict(dst=DT_HALF), dict(t=DT_HALF),
                                dict(src=DT_DOUBLE)])
def test_cast_folding_negative(kw):
    gd, stats = run(mixed_graph(1, **kw))
    assert nodes(gd)["adam0"].op == "ResourceApplyAdam" and stats["adam_mixed"] == 0


def test_cast_folding_disabled_by_reference_name_and_filter():
    for kw in (dict(disabled_patterns=["MusaAdamMixedFusion"]),
               dict(disabled_patterns=["MusaResourceApplyAdamMixed"]),
               dict(device_filter="GPU")):
        gd, stats = run(mixed_graph(1), **kw)
        assert stats["adam_mixed"] == 0, kw
    gd, stats = run(mixed_graph(1), fetch=["cast0"],
                    disabled_patterns=["MusaGroupedResourceApplyAdam"])
    assert nodes(gd)["adam0"].op == "MusaResourceApplyAdamMixed" and "cast0" in nodes(gd)


def test_mixed_adam_nodes_grouped_with_tgrad():
    gd, stats = run(mixed_graph(4))
    check_well_formed(gd)
    grp = [n for n in gd.node if n.op == "MusaGroupedResourceApplyAdam"]
    assert len(grp) == 1 and stats["adam_mixed"] == 4 and stats["adam_grouped_nodes"] == 4
    gn = grp[0]
    assert gn.attr["T"].type == DT_FLOAT and gn.attr["Tgrad"].type == DT_HALF
    assert list(gn.input)[-5:] == ["g0", "g1", "g2", "g3", "^init"]
    assert not [n for n in gd.node if n.op == "Cast"]


def test_plain_and_mixed_adam_are_separate_groups():
    g = mixed_graph(2)
    for i in range(2, 4):
        for r in ("var", "m", "v"):
            g.node(f"{r}{i}", "VarHandleOp", dtype=DT_FLOAT)
        g.node(f"g{i}", "Placeholder", dtype=DT_FLOAT)
        g.node(f"adam{i}", "ResourceApplyAdam", [f"var{i}", f"m{i}", f"v{i}"] + SCALARS + [f"g{i}"],
               T=DT_FLOAT, use_locking=False, use_nesterov=False)
    gd, stats = run(g)
    check_well_formed(gd)
    grp = sorted((n.attr["Tgrad"].type, n.attr["N"].i) for n in gd.node
                 if n.op == "MusaGroupedResourceApplyAdam")
    assert grp == [(DT_FLOAT, 2), (DT_HALF, 2)]
