"""tensorflow.GraphDef / NodeDef / AttrValue message classes for tests.

TensorFlow is not installed here, so the messages are declared at run time
with the same package, names and field numbers as tensorflow/core/framework/
graph.proto, node_def.proto and attr_value.proto (only the fields the tests
use; anything else a real GraphDef carries is an unknown field to these
classes and is preserved on the wire).  A GraphDef serialized by these classes
is byte-compatible with TensorFlow's.
"""
from google.protobuf import descriptor_pb2, descriptor_pool, message_factory

FDP = descriptor_pb2.FieldDescriptorProto
DT_FLOAT, DT_DOUBLE, DT_RESOURCE, DT_BFLOAT16, DT_HALF = 1, 2, 20, 14, 19


def _field(msg, name, number, ftype, label=FDP.LABEL_OPTIONAL, type_name=None):
    f = msg.field.add(name=name, number=number, type=ftype, label=label)
    if type_name:
        f.type_name = type_name
    return f


def _build():
    fd = descriptor_pb2.FileDescriptorProto(name="tfma_test_graph.proto",
                                            package="tensorflow", syntax="proto3")
    lv = fd.message_type.add(name="AttrValue")
    lst = lv.nested_type.add(name="ListValue")
    _field(lst, "s", 2, FDP.TYPE_BYTES, FDP.LABEL_REPEATED)
    _field(lst, "i", 3, FDP.TYPE_INT64, FDP.LABEL_REPEATED)
    _field(lst, "type", 6, FDP.TYPE_INT32, FDP.LABEL_REPEATED)
    lv.oneof_decl.add(name="value")
    for name, num, t, tn in (("list", 1, FDP.TYPE_MESSAGE, ".tensorflow.AttrValue.ListValue"),
                             ("s", 2, FDP.TYPE_BYTES, None), ("i", 3, FDP.TYPE_INT64, None),
                             ("f", 4, FDP.TYPE_FLOAT, None), ("b", 5, FDP.TYPE_BOOL, None),
                             ("type", 6, FDP.TYPE_INT32, None)):
        _field(lv, name, num, t, type_name=tn).oneof_index = 0

    nd = fd.message_type.add(name="NodeDef")
    entry = nd.nested_type.add(name="AttrEntry")
    entry.options.map_entry = True
    _field(entry, "key", 1, FDP.TYPE_STRING)
    _field(entry, "value", 2, FDP.TYPE_MESSAGE, type_name=".tensorflow.AttrValue")
    _field(nd, "name", 1, FDP.TYPE_STRING)
    _field(nd, "op", 2, FDP.TYPE_STRING)
    _field(nd, "input", 3, FDP.TYPE_STRING, FDP.LABEL_REPEATED)
    _field(nd, "device", 4, FDP.TYPE_STRING)
    _field(nd, "attr", 5, FDP.TYPE_MESSAGE, FDP.LABEL_REPEATED, ".tensorflow.NodeDef.AttrEntry")

    vd = fd.message_type.add(name="VersionDef")
    _field(vd, "producer", 1, FDP.TYPE_INT32)
    _field(vd, "min_consumer", 2, FDP.TYPE_INT32)

    gd = fd.message_type.add(name="GraphDef")
    _field(gd, "node", 1, FDP.TYPE_MESSAGE, FDP.LABEL_REPEATED, ".tensorflow.NodeDef")
    _field(gd, "versions", 4, FDP.TYPE_MESSAGE, type_name=".tensorflow.VersionDef")

    pool = descriptor_pool.DescriptorPool()
    pool.Add(fd)
    get = lambda n: message_factory.GetMessageClass(pool.FindMessageTypeByName(n))
    return get("tensorflow.GraphDef"), get("tensorflow.NodeDef"), get("tensorflow.AttrValue")


GraphDef, NodeDef, AttrValue = _build()


class G:
    """Small builder: G().node("r", "Relu", ["b"], T=DT_FLOAT).serialize()."""

    def __init__(self, device="/job:localhost/replica:0/task:0/device:MUSA:0"):
        self.gd = GraphDef()
        self.gd.versions.producer = 1205
        self.device = device

    def node(self, name, op, inputs=(), device=None, **attrs):
        n = self.gd.node.add(name=name, op=op, device=self.device if device is None else device)
        n.input.extend(inputs)
        for k, v in attrs.items():
            a = n.attr[k]
            if isinstance(v, bool):
                a.b = v
            elif isinstance(v, str):
                a.s = v.encode()
            elif k in ("T", "dtype", "Tgrad", "U", "SrcT", "DstT"):
                a.type = v
            else:
                a.i = v
        return self

    def serialize(self):
        return self.gd.SerializeToString()


def parse(data):
    gd = GraphDef()
    gd.ParseFromString(data)
    return gd


def nodes(gd):
    return {n.name: n for n in gd.node}
