// Graph rewrite for the hot path: turns the unfused TensorFlow patterns into
// the fused ops of this library, on a serialized GraphDef (the form a
// TF_InitGraph optimizer receives), and groups ResourceApplyAdam nodes.
//
//   Relu(BiasAdd(x, b))        -> MusaBiasAddRelu(x, b)          priority 100
//   Relu(AddV2|Add(x, y))      -> MusaAddV2Relu(x, y)            priority  90
//   AddV2(Mul(Const, mask), Const)
//                              -> MusaShiftedAffineMap           priority  80
//                                 (mask: Select, SelectV2, Where or Identity;
//                                 Consts through Identity nodes; the
//                                 reference's exact topology,
//                                 shifted_affine_map_fusion.cc:109-233)
//   ResourceApplyAdam<float>(..., Cast<half|bfloat16 -> float>(g))
//                              -> MusaResourceApplyAdamMixed(..., g)  priority 40
//                                 (musa_ext/graph/fusion/adam_mixed_fusion.cc:93-216)
//   k >= 2 ResourceApplyAdam / MusaResourceApplyAdamMixed with the same
//   scalars, state and gradient dtypes, attrs and device
//                              -> MusaGroupedResourceApplyAdam
//
// Semantics follow the reference's pattern framework: a pattern matches from
// its output node, patterns run in priority groups, each group sweeps the
// graph forward then in reverse until nothing changes (at most 50 rounds)
// (musa_ext/graph/fusion/fusion_pattern_manager.h:54-82,
// musa_ext/mu/optimizer/musa_graph_optimizer.cc:5843-5994); the fused node
// keeps the output node's name, device and control inputs, and the absorbed
// node goes away (FusionGraphUtils::RemoveNodesIfUnused, .h:189-191).  A
// producer is absorbed only if the pattern's node is its only consumer and it
// is not fetched (MusaShiftedAffineMap, as the reference's, fuses whatever
// else reads the Mul and keeps the Mul then).  Adam grouping follows the reference's grouped-SGD rewrite
// (musa_graph_optimizer.cc:2014-2120) and additionally refuses to group nodes
// where one depends on another, which would create a cycle.
//
// The GraphDef is handled at the protobuf wire level (field numbers of
// tensorflow/core/framework/graph.proto, node_def.proto, attr_value.proto);
// fields this pass does not touch are carried through byte for byte.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <set>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "tfma.h"

namespace tfma {
namespace {

// ---------------------------------------------------------------------------
// Protobuf wire format.
// ---------------------------------------------------------------------------
enum WireType { kVarint = 0, kFixed64 = 1, kLen = 2, kFixed32 = 5 };

struct Reader {
  const uint8_t* p;
  const uint8_t* end;
  bool ok = true;

  Reader(const void* data, size_t n)
      : p(static_cast<const uint8_t*>(data)), end(static_cast<const uint8_t*>(data) + n) {}
  bool done() const { return p >= end || !ok; }

  uint64_t varint() {
    uint64_t v = 0;
    for (int shift = 0; shift < 64; shift += 7) {
      if (p >= end) {
        ok = false;
        return 0;
      }
      const uint8_t b = *p++;
      v |= static_cast<uint64_t>(b & 0x7f) << shift;
      if (!(b & 0x80)) return v;
    }
    ok = false;
    return 0;
  }
  // Reads a tag; returns false at the end or on error.
  bool tag(uint32_t* field, uint32_t* wt) {
    if (done()) return false;
    const uint64_t t = varint();
    *field = static_cast<uint32_t>(t >> 3);
    *wt = static_cast<uint32_t>(t & 7);
    return ok && *field != 0;
  }
  std::string bytes() {
    const uint64_t n = varint();
    if (!ok || n > static_cast<uint64_t>(end - p)) {
      ok = false;
      return std::string();
    }
    std::string s(reinterpret_cast<const char*>(p), static_cast<size_t>(n));
    p += n;
    return s;
  }
  void skip(uint32_t wt) {
    switch (wt) {
      case kVarint: varint(); break;
      case kFixed64: p += 8; break;
      case kLen: bytes(); break;
      case kFixed32: p += 4; break;
      default: ok = false;
    }
    if (p > end) ok = false;
  }
};

struct Writer {
  std::string out;
  void varint(uint64_t v) {
    while (v >= 0x80) {
      out.push_back(static_cast<char>((v & 0x7f) | 0x80));
      v >>= 7;
    }
    out.push_back(static_cast<char>(v));
  }
  void tag(uint32_t field, uint32_t wt) { varint((static_cast<uint64_t>(field) << 3) | wt); }
  void bytes(uint32_t field, const std::string& s) {
    tag(field, kLen);
    varint(s.size());
    out += s;
  }
  void uint(uint32_t field, uint64_t v) {
    tag(field, kVarint);
    varint(v);
  }
};

// Copies the raw bytes of the field that starts at `start` (tag included).
std::string raw_field(const uint8_t* start, const uint8_t* end) {
  return std::string(reinterpret_cast<const char*>(start), static_cast<size_t>(end - start));
}

// ---------------------------------------------------------------------------
// NodeDef / AttrValue.
// ---------------------------------------------------------------------------
struct Node {
  std::string name, op, device;
  std::vector<std::string> inputs;
  std::vector<std::pair<std::string, std::string>> attrs;  // key, AttrValue bytes
  std::string other;  // untouched fields, raw
  bool removed = false;
};

bool parse_node(const std::string& bytes, Node* n) {
  Reader r(bytes.data(), bytes.size());
  uint32_t f, wt;
  while (true) {
    const uint8_t* start = r.p;
    if (!r.tag(&f, &wt)) break;
    if (wt == kLen && f >= 1 && f <= 5) {
      std::string v = r.bytes();
      if (f == 1) n->name = v;
      else if (f == 2) n->op = v;
      else if (f == 3) n->inputs.push_back(v);
      else if (f == 4) n->device = v;
      else {
        Reader e(v.data(), v.size());
        std::string key, val;
        uint32_t ef, ewt;
        while (e.tag(&ef, &ewt)) {
          if (ef == 1 && ewt == kLen) key = e.bytes();
          else if (ef == 2 && ewt == kLen) val = e.bytes();
          else e.skip(ewt);
        }
        if (!e.ok) return false;
        n->attrs.emplace_back(key, val);
      }
    } else {
      r.skip(wt);
      n->other += raw_field(start, r.p);
    }
  }
  return r.ok;
}

std::string serialize_node(const Node& n) {
  Writer w;
  w.bytes(1, n.name);
  w.bytes(2, n.op);
  for (const auto& i : n.inputs) w.bytes(3, i);
  if (!n.device.empty()) w.bytes(4, n.device);
  for (const auto& kv : n.attrs) {
    Writer e;
    e.bytes(1, kv.first);
    e.bytes(2, kv.second);
    w.bytes(5, e.out);
  }
  w.out += n.other;
  return w.out;
}

const std::string* find_attr(const Node& n, const std::string& key) {
  for (const auto& kv : n.attrs)
    if (kv.first == key) return &kv.second;
  return nullptr;
}

// Scalar AttrValue fields: s = 2 (bytes), i = 3, b = 5, type = 6 (varints).
bool attr_varint(const Node& n, const std::string& key, uint32_t field, int64_t* v) {
  const std::string* a = find_attr(n, key);
  if (!a) return false;
  Reader r(a->data(), a->size());
  uint32_t f, wt;
  while (r.tag(&f, &wt)) {
    if (f == field && wt == kVarint) {
      *v = static_cast<int64_t>(r.varint());
      return r.ok;
    }
    r.skip(wt);
  }
  return false;
}

std::string attr_string(const Node& n, const std::string& key, const std::string& dflt) {
  const std::string* a = find_attr(n, key);
  if (!a) return dflt;
  Reader r(a->data(), a->size());
  uint32_t f, wt;
  while (r.tag(&f, &wt)) {
    if (f == 2 && wt == kLen) return r.bytes();
    r.skip(wt);
  }
  return dflt;
}

std::string attr_of_type(int64_t dt) {
  Writer w;
  w.uint(6, static_cast<uint64_t>(dt));
  return w.out;
}
std::string attr_of_string(const std::string& s) {
  Writer w;
  w.bytes(2, s);
  return w.out;
}
std::string attr_of_int(int64_t i) {
  Writer w;
  w.uint(3, static_cast<uint64_t>(i));
  return w.out;
}
std::string attr_of_bool(bool b) {
  Writer w;
  w.uint(5, b ? 1 : 0);
  return w.out;
}

// ---------------------------------------------------------------------------
// Graph.
// ---------------------------------------------------------------------------
bool is_control(const std::string& in) { return !in.empty() && in[0] == '^'; }

// "name", "name:0" -> "name", port 0; "^name" -> "name", port -1.
std::string producer_of(const std::string& in, int* port) {
  if (is_control(in)) {
    *port = -1;
    return in.substr(1);
  }
  const size_t c = in.rfind(':');
  if (c != std::string::npos && c + 1 < in.size() &&
      in.find_first_not_of("0123456789", c + 1) == std::string::npos) {
    *port = atoi(in.c_str() + c + 1);
    return in.substr(0, c);
  }
  *port = 0;
  return in;
}

struct Graph {
  std::vector<Node> nodes;
  std::string other;  // GraphDef fields other than node, raw
  std::unordered_map<std::string, int> index;
  std::set<std::string> fetch;
  std::string device_filter;  // rewrite only nodes whose device contains it

  bool on_device(const Node& n) const {
    return device_filter.empty() || n.device.find(device_filter) != std::string::npos;
  }
  void reindex() {
    index.clear();
    for (int i = 0; i < static_cast<int>(nodes.size()); ++i)
      if (!nodes[i].removed) index[nodes[i].name] = i;
  }
  const Node* producer(const std::string& in, int* port) const {
    const std::string name = producer_of(in, port);
    auto it = index.find(name);
    return it == index.end() ? nullptr : &nodes[it->second];
  }
  // Every live input that refers to `name` (data or control).
  std::vector<std::pair<int, int>> consumers(const std::string& name) const {
    std::vector<std::pair<int, int>> out;  // (node index, input index)
    for (int i = 0; i < static_cast<int>(nodes.size()); ++i) {
      if (nodes[i].removed) continue;
      for (int k = 0; k < static_cast<int>(nodes[i].inputs.size()); ++k) {
        int port;
        if (producer_of(nodes[i].inputs[k], &port) == name) out.emplace_back(i, k);
      }
    }
    return out;
  }
  bool unique_name(const std::string& n) const { return index.find(n) == index.end(); }
};

bool parse_graph(const void* data, size_t n, Graph* g) {
  Reader r(data, n);
  uint32_t f, wt;
  while (true) {
    const uint8_t* start = r.p;
    if (!r.tag(&f, &wt)) break;
    if (f == 1 && wt == kLen) {
      Node node;
      if (!parse_node(r.bytes(), &node)) return false;
      g->nodes.push_back(std::move(node));
    } else {
      r.skip(wt);
      g->other += raw_field(start, r.p);
    }
  }
  if (!r.ok) return false;
  g->reindex();
  return true;
}

std::string serialize_graph(const Graph& g) {
  Writer w;
  for (const auto& n : g.nodes)
    if (!n.removed) w.bytes(1, serialize_node(n));
  w.out += g.other;
  return w.out;
}

// TF_DataType codes accepted by the fused kernels.
bool fusable_type(int64_t t) { return t == TFMA_FLOAT || t == TFMA_HALF || t == TFMA_BFLOAT16; }

void add_control_inputs(const Node& from, std::vector<std::string>* to) {
  for (const auto& in : from.inputs)
    if (is_control(in) && std::find(to->begin(), to->end(), in) == to->end()) to->push_back(in);
}

// ---------------------------------------------------------------------------
// Elementwise patterns.  Each returns true after rewriting one match rooted
// at node `i`.
// ---------------------------------------------------------------------------
struct Pattern {
  const char* name;
  const char* alias;  // the reference's name for the same rewrite, if any
  int priority;
  bool (*apply)(Graph* g, int i);
};

// The producer feeding input `k` of node `out`, if it is op in `ops`, has the
// same device and T as `out`, is not fetched, and has no other data
// consumer.  Control consumers are redirected by absorb().
int fusable_producer(const Graph& g, const Node& out, int k, std::initializer_list<const char*> ops) {
  if (!g.on_device(out) || k >= static_cast<int>(out.inputs.size()) || is_control(out.inputs[k]))
    return -1;
  int port;
  const Node* p = g.producer(out.inputs[k], &port);
  if (!p || port != 0) return -1;
  bool op_ok = false;
  for (const char* op : ops) op_ok |= p->op == op;
  if (!op_ok || p->device != out.device || g.fetch.count(p->name)) return -1;
  int64_t t_out = -1, t_p = -2;
  if (!attr_varint(out, "T", 6, &t_out) || !attr_varint(*p, "T", 6, &t_p) || t_out != t_p ||
      !fusable_type(t_out))
    return -1;
  int data_consumers = 0;
  for (const auto& c : g.consumers(p->name))
    if (!is_control(g.nodes[c.first].inputs[c.second])) ++data_consumers;
  if (data_consumers != 1) return -1;
  return g.index.at(p->name);
}

// Removes node `absorbed` (merged into `fused`): its control inputs join the
// fused node's, and control consumers of it now depend on the fused node.
void absorb(Graph* g, int absorbed, int fused) {
  Node& a = g->nodes[absorbed];
  add_control_inputs(a, &g->nodes[fused].inputs);
  for (const auto& c : g->consumers(a.name)) {
    std::string& in = g->nodes[c.first].inputs[c.second];
    if (is_control(in)) in = "^" + g->nodes[fused].name;
  }
  // Drop duplicate control inputs created by the redirect.
  for (auto& n : g->nodes) {
    std::vector<std::string> seen;
    std::vector<std::string> kept;
    for (auto& in : n.inputs) {
      if (is_control(in)) {
        if (in == "^" + n.name || std::find(seen.begin(), seen.end(), in) != seen.end()) continue;
        seen.push_back(in);
      }
      kept.push_back(in);
    }
    n.inputs.swap(kept);
  }
  a.removed = true;
  g->reindex();
}

// Data inputs then control inputs of the fused node.
void set_inputs(Node* n, std::vector<std::string> data, const std::vector<std::string>& old) {
  for (const auto& in : old)
    if (is_control(in)) data.push_back(in);
  n->inputs = std::move(data);
}

bool apply_bias_add_relu(Graph* g, int i) {
  Node& relu = g->nodes[i];
  if (relu.removed || relu.op != "Relu") return false;
  const int b = fusable_producer(*g, relu, 0, {"BiasAdd", "BiasAddV1"});
  if (b < 0 || g->nodes[b].inputs.size() < 2 || is_control(g->nodes[b].inputs[1])) return false;
  const Node& ba = g->nodes[b];
  int64_t t = 0;
  attr_varint(relu, "T", 6, &t);
  const std::string fmt = attr_string(ba, "data_format", "NHWC");
  const std::vector<std::string> old = relu.inputs;
  set_inputs(&relu, {ba.inputs[0], ba.inputs[1]}, old);
  relu.op = "MusaBiasAddRelu";
  relu.attrs = {{"T", attr_of_type(t)}, {"data_format", attr_of_string(fmt)}};
  absorb(g, b, i);
  return true;
}

bool apply_add_v2_relu(Graph* g, int i) {
  Node& relu = g->nodes[i];
  if (relu.removed || relu.op != "Relu") return false;
  const int a = fusable_producer(*g, relu, 0, {"AddV2", "Add"});
  if (a < 0 || g->nodes[a].inputs.size() < 2 || is_control(g->nodes[a].inputs[1])) return false;
  const Node& add = g->nodes[a];
  int64_t t = 0;
  attr_varint(relu, "T", 6, &t);
  const std::vector<std::string> old = relu.inputs;
  set_inputs(&relu, {add.inputs[0], add.inputs[1]}, old);
  relu.op = "MusaAddV2Relu";
  relu.attrs = {{"T", attr_of_type(t)}};
  absorb(g, a, i);
  return true;
}

// The node an input edge reads, followed through Identity nodes (their
// first input) as the reference's ResolveIdentityLike does
// (shifted_affine_map_fusion.cc:62-68).
const Node* resolve_identity(const Graph& g, const std::string& in) {
  int port;
  const Node* p = g.producer(in, &port);
  for (size_t hops = 0; p && p->op == "Identity" && !p->inputs.empty() &&
                        !is_control(p->inputs[0]) && hops < g.nodes.size();
       ++hops)
    p = g.producer(p->inputs[0], &port);
  return p;
}

// AddV2(Mul(data_left, mask), sliced_var_right) -> MusaShiftedAffineMap,
// matched as the reference matches it (shifted_affine_map_fusion.cc:109-233):
// an AddV2 with exactly two inputs, one produced by a Mul and the other
// resolving through Identity nodes to a Const; the Mul with exactly two
// inputs, one resolving to a Const (data_left) and the other produced by a
// Select, SelectV2, Where or Identity node (the mask).  The fused node keeps
// the AddV2's name, device and T (float when absent) and takes the three
// edges as the Mul and the AddV2 read them (:240-316); the Mul goes away
// only when nothing else reads it.  Two guards the reference lacks: T must be
// a type the op is registered for, and a fetched Mul is kept.
bool apply_mul_add(Graph* g, int i) {
  Node& add = g->nodes[i];
  if (add.removed || add.op != "AddV2" || !g->on_device(add)) return false;
  if (add.inputs.size() != 2 || is_control(add.inputs[0]) || is_control(add.inputs[1])) return false;
  int64_t t = TFMA_FLOAT;
  attr_varint(add, "T", 6, &t);
  if (!fusable_type(t) && t != TFMA_DOUBLE) return false;
  auto produced_by = [&](const std::string& in, std::initializer_list<const char*> ops) {
    int port;
    const Node* p = g->producer(in, &port);
    if (!p) return false;
    for (const char* op : ops)
      if (p->op == op) return true;
    return false;
  };
  auto is_const = [&](const std::string& in) {
    const Node* r = resolve_identity(*g, in);
    return r && r->op == "Const";
  };
  int k;
  if (produced_by(add.inputs[0], {"Mul"}) && is_const(add.inputs[1]))
    k = 0;
  else if (produced_by(add.inputs[1], {"Mul"}) && is_const(add.inputs[0]))
    k = 1;
  else
    return false;
  int port;
  const int m = g->index.at(g->producer(add.inputs[k], &port)->name);
  const Node& mul = g->nodes[m];
  if (mul.inputs.size() != 2 || is_control(mul.inputs[0]) || is_control(mul.inputs[1]))
    return false;
  std::string left, mask;
  const std::initializer_list<const char*> mask_ops = {"Select", "SelectV2", "Where", "Identity"};
  if (is_const(mul.inputs[0]) && produced_by(mul.inputs[1], mask_ops)) {
    left = mul.inputs[0];
    mask = mul.inputs[1];
  } else if (is_const(mul.inputs[1]) && produced_by(mul.inputs[0], mask_ops)) {
    left = mul.inputs[1];
    mask = mul.inputs[0];
  } else {
    return false;
  }
  const std::string mul_name = mul.name;
  add.inputs = {left, mask, add.inputs[1 - k]};
  add.op = "MusaShiftedAffineMap";
  add.attrs = {{"T", attr_of_type(t)}};
  if (g->consumers(mul_name).empty() && !g->fetch.count(mul_name)) {
    g->nodes[m].removed = true;
    g->reindex();
  }
  return true;
}

// ResourceApplyAdam<float> whose grad is Cast(SrcT = half|bfloat16, DstT =
// float): the Adam node becomes MusaResourceApplyAdamMixed (T = SrcT) reading
// the Cast's input; the Cast goes away when nothing else reads it.
bool apply_adam_mixed(Graph* g, int i) {
  Node& adam = g->nodes[i];
  if (adam.removed || adam.op != "ResourceApplyAdam" || !g->on_device(adam)) return false;
  int64_t t = 0;
  if (!attr_varint(adam, "T", 6, &t) || t != TFMA_FLOAT) return false;
  if (adam.inputs.size() < 10 || is_control(adam.inputs[9])) return false;
  int port;
  const Node* cast = g->producer(adam.inputs[9], &port);
  if (!cast || port != 0 || cast->op != "Cast" || cast->inputs.empty() ||
      is_control(cast->inputs[0]))
    return false;
  int64_t src = 0, dst = 0;
  if (!attr_varint(*cast, "DstT", 6, &dst) || dst != TFMA_FLOAT) return false;
  if (!attr_varint(*cast, "SrcT", 6, &src) || (src != TFMA_HALF && src != TFMA_BFLOAT16))
    return false;
  const int ci = g->index.at(cast->name);
  int other = 0;
  for (const auto& c : g->consumers(cast->name))
    if (c.first != i || c.second != 9) ++other;
  adam.op = "MusaResourceApplyAdamMixed";
  for (auto& kv : adam.attrs)
    if (kv.first == "T") kv.second = attr_of_type(src);
  adam.inputs[9] = g->nodes[ci].inputs[0];
  if (other == 0 && !g->fetch.count(g->nodes[ci].name)) absorb(g, ci, i);
  return true;
}

const Pattern kPatterns[] = {
    {"MusaBiasAddRelu", nullptr, 100, apply_bias_add_relu},
    {"MusaAddV2Relu", nullptr, 90, apply_add_v2_relu},
    {"MusaShiftedAffineMap", "MusaShiftedAffineMapFusion", 80, apply_mul_add},
    {"MusaResourceApplyAdamMixed", "MusaAdamMixedFusion", 40, apply_adam_mixed},
};

bool pattern_disabled(const std::set<std::string>& disabled, const Pattern& p) {
  return disabled.count(p.name) > 0 || (p.alias && disabled.count(p.alias) > 0);
}

// ---------------------------------------------------------------------------
// ResourceApplyAdam grouping.
// ---------------------------------------------------------------------------
// Candidates reachable (through any input edge) from each node, as bitsets
// over candidate indices, in topological order; false if the graph has a
// cycle (then nothing is grouped).
bool candidate_ancestors(const Graph& g, const std::vector<int>& cand,
                         std::vector<std::vector<uint64_t>>* anc) {
  const int n = static_cast<int>(g.nodes.size());
  const int words = (static_cast<int>(cand.size()) + 63) / 64;
  std::vector<int> cand_id(n, -1);
  for (int c = 0; c < static_cast<int>(cand.size()); ++c) cand_id[cand[c]] = c;
  std::vector<std::vector<int>> preds(n);
  std::vector<int> indeg(n, 0);
  std::vector<std::vector<int>> succ(n);
  for (int i = 0; i < n; ++i) {
    if (g.nodes[i].removed) continue;
    for (const auto& in : g.nodes[i].inputs) {
      int port;
      auto it = g.index.find(producer_of(in, &port));
      if (it == g.index.end()) continue;
      preds[i].push_back(it->second);
      succ[it->second].push_back(i);
      ++indeg[i];
    }
  }
  std::vector<int> order;
  for (int i = 0; i < n; ++i)
    if (!g.nodes[i].removed && indeg[i] == 0) order.push_back(i);
  for (size_t h = 0; h < order.size(); ++h)
    for (int s : succ[order[h]])
      if (--indeg[s] == 0) order.push_back(s);
  int live = 0;
  for (const auto& nd : g.nodes) live += nd.removed ? 0 : 1;
  if (static_cast<int>(order.size()) != live) return false;
  anc->assign(n, std::vector<uint64_t>(words, 0));
  for (int v : order) {
    auto& a = (*anc)[v];
    for (int p : preds[v]) {
      const auto& ap = (*anc)[p];
      for (int w = 0; w < words; ++w) a[w] |= ap[w];
      if (cand_id[p] >= 0) a[cand_id[p] / 64] |= uint64_t(1) << (cand_id[p] % 64);
    }
  }
  return true;
}

// "x" and "x:0" name the same tensor.
std::string tensor_key(const std::string& in) {
  int port;
  const std::string name = producer_of(in, &port);
  return name + ":" + std::to_string(port);
}

// Forms one grouped Adam node; returns the number of nodes it replaced (0 when
// no group of two or more can be formed).  Called until it returns 0, so the
// ancestor sets always describe the current graph and a group never closes a
// cycle with an earlier one.
int group_adam_once(Graph* g) {
  // State and gradient dtypes: ResourceApplyAdam has both = T;
  // MusaResourceApplyAdamMixed has float state and T gradients.
  auto dtypes = [](const Node& n, int64_t* state, int64_t* grad) {
    int64_t t = 0;
    if (!attr_varint(n, "T", 6, &t)) return false;
    if (n.op == "ResourceApplyAdam") {
      *state = *grad = t;
      return fusable_type(t) || t == TFMA_DOUBLE;
    }
    if (n.op == "MusaResourceApplyAdamMixed") {
      *state = TFMA_FLOAT;
      *grad = t;
      return fusable_type(t);
    }
    return false;
  };
  std::vector<int> cand;
  for (int i = 0; i < static_cast<int>(g->nodes.size()); ++i) {
    const Node& n = g->nodes[i];
    int64_t st = 0, gt = 0;
    if (n.removed || g->fetch.count(n.name) || !g->on_device(n)) continue;
    if (!dtypes(n, &st, &gt)) continue;
    bool ok = n.inputs.size() >= 10;
    for (size_t k = 0; k < n.inputs.size() && ok; ++k) ok = is_control(n.inputs[k]) == (k >= 10);
    if (ok) cand.push_back(i);
  }
  if (cand.size() < 2) return 0;
  std::vector<std::vector<uint64_t>> anc;
  if (!candidate_ancestors(*g, cand, &anc)) return 0;
  std::unordered_map<int, int> cid;
  for (int c = 0; c < static_cast<int>(cand.size()); ++c) cid[cand[c]] = c;
  auto reaches = [&](int from, int to) {  // `from` is an ancestor of `to`
    const int c = cid[from];
    return ((anc[to][c / 64] >> (c % 64)) & 1) != 0;
  };
  // Key: device, T, use_locking, use_nesterov and the six scalar inputs.
  std::map<std::string, std::vector<int>> by_key;
  for (int i : cand) {
    const Node& n = g->nodes[i];
    int64_t st = 0, gt = 0, lock = 0, nest = 0;
    dtypes(n, &st, &gt);
    attr_varint(n, "use_locking", 5, &lock);
    attr_varint(n, "use_nesterov", 5, &nest);
    std::string key = n.device + '\x1f' + std::to_string(st) + '\x1f' + std::to_string(gt) +
                      '\x1f' + std::to_string(lock) + '\x1f' + std::to_string(nest);
    for (int k = 3; k < 9; ++k) key += '\x1f' + tensor_key(n.inputs[k]);
    by_key[key].push_back(i);
  }
  for (auto& kv : by_key) {
    // Greedy, in graph order: a member must not reach or be reached by
    // another member, and var/m/v resources must all be distinct.
    std::vector<int> grp;
    std::set<std::string> resources;
    for (int i : kv.second) {
      bool ok = true;
      for (int j : grp) ok = ok && !reaches(i, j) && !reaches(j, i);
      for (int k = 0; k < 3 && ok; ++k) ok = !resources.count(tensor_key(g->nodes[i].inputs[k]));
      if (!ok) continue;
      grp.push_back(i);
      for (int k = 0; k < 3; ++k) resources.insert(tensor_key(g->nodes[i].inputs[k]));
    }
    if (grp.size() < 2) continue;

    const Node& first = g->nodes[grp[0]];
    Node gn;
    gn.name = first.name + "/MusaGroupedResourceApplyAdam";
    for (int s = 1; !g->unique_name(gn.name); ++s)
      gn.name = first.name + "/MusaGroupedResourceApplyAdam_" + std::to_string(s);
    gn.op = "MusaGroupedResourceApplyAdam";
    gn.device = first.device;
    for (int k = 0; k < 3; ++k)
      for (int i : grp) gn.inputs.push_back(g->nodes[i].inputs[k]);
    for (int k = 3; k < 9; ++k) gn.inputs.push_back(first.inputs[k]);
    for (int i : grp) gn.inputs.push_back(g->nodes[i].inputs[9]);
    std::set<std::string> members;
    for (int i : grp) members.insert(g->nodes[i].name);
    for (int i : grp)
      for (const auto& in : g->nodes[i].inputs)
        if (is_control(in) && !members.count(in.substr(1)) &&
            std::find(gn.inputs.begin(), gn.inputs.end(), in) == gn.inputs.end())
          gn.inputs.push_back(in);
    int64_t st = 0, gt = 0, lock = 0, nest = 0;
    dtypes(first, &st, &gt);
    attr_varint(first, "use_locking", 5, &lock);
    attr_varint(first, "use_nesterov", 5, &nest);
    gn.attrs = {{"N", attr_of_int(static_cast<int64_t>(grp.size()))},
                {"T", attr_of_type(st)},
                {"Tgrad", attr_of_type(gt)},
                {"use_locking", attr_of_bool(lock != 0)},
                {"use_nesterov", attr_of_bool(nest != 0)}};
    // Control consumers of the members now depend on the group (the
    // reference's RedirectNodeOutputs); ResourceApplyAdam has no data output.
    for (auto& n : g->nodes) {
      if (n.removed) continue;
      std::vector<std::string> kept;
      bool added = false;
      for (auto& in : n.inputs) {
        if (is_control(in) && members.count(in.substr(1))) {
          if (!added) kept.push_back("^" + gn.name);
          added = true;
          continue;
        }
        kept.push_back(in);
      }
      n.inputs.swap(kept);
    }
    for (int i : grp) g->nodes[i].removed = true;
    const int replaced = static_cast<int>(grp.size());
    g->nodes.push_back(std::move(gn));
    g->reindex();
    return replaced;
  }
  return 0;
}

int group_adam(Graph* g, int* groups_made) {
  int grouped = 0;
  for (int r; (r = group_adam_once(g)) > 0;) {
    grouped += r;
    ++*groups_made;
  }
  return grouped;
}

int set_error(TFMA_Status* st, int code, const char* msg) {
  if (st) {
    st->code = code;
    snprintf(st->message, sizeof(st->message), "%s", msg);
  }
  return code;
}

}  // namespace
}  // namespace tfma

extern "C" {

int TFMA_OptimizeGraph(const void* graph_def, size_t graph_def_bytes,
                       const char* const* fetch_nodes, int num_fetch,
                       const char* device_filter, const char* disabled_patterns,
                       void** optimized,
                       size_t* optimized_bytes, TFMA_GraphRewriteStats* stats,
                       TFMA_Status* status) {
  using namespace tfma;
  if (!optimized || !optimized_bytes || (!graph_def && graph_def_bytes))
    return set_error(status, TFMA_INVALID_ARGUMENT, "TFMA_OptimizeGraph: null argument");
  *optimized = nullptr;
  *optimized_bytes = 0;
  Graph g;
  if (!parse_graph(graph_def, graph_def_bytes, &g))
    return set_error(status, TFMA_INVALID_ARGUMENT, "TFMA_OptimizeGraph: malformed GraphDef");
  for (int i = 0; i < num_fetch; ++i) {
    int port;
    if (fetch_nodes && fetch_nodes[i]) g.fetch.insert(producer_of(fetch_nodes[i], &port));
  }
  if (device_filter) g.device_filter = device_filter;
  std::set<std::string> disabled;
  if (disabled_patterns) {
    std::string s = disabled_patterns;
    size_t pos = 0;
    while (pos <= s.size()) {
      size_t e = s.find(',', pos);
      if (e == std::string::npos) e = s.size();
      std::string tok = s.substr(pos, e - pos);
      tok.erase(0, tok.find_first_not_of(" \t"));
      tok.erase(tok.find_last_not_of(" \t") + 1);
      if (!tok.empty()) disabled.insert(tok);
      pos = e + 1;
    }
  }
  TFMA_GraphRewriteStats local{};
  // Priority groups, highest first; each pattern sweeps forward then in
  // reverse until a whole round changes nothing (at most 50 rounds).
  std::vector<const Pattern*> pats;
  for (const auto& p : kPatterns)
    if (!pattern_disabled(disabled, p)) pats.push_back(&p);
  std::stable_sort(pats.begin(), pats.end(),
                   [](const Pattern* a, const Pattern* b) { return a->priority > b->priority; });
  for (const Pattern* p : pats) {
    for (int round = 0; round < 50; ++round) {
      int changed = 0;
      const int n = static_cast<int>(g.nodes.size());
      for (int i = 0; i < n; ++i) changed += p->apply(&g, i) ? 1 : 0;
      for (int i = n - 1; i >= 0; --i) changed += p->apply(&g, i) ? 1 : 0;
      if (p->apply == apply_bias_add_relu) local.bias_add_relu += changed;
      else if (p->apply == apply_add_v2_relu) local.add_v2_relu += changed;
      else if (p->apply == apply_mul_add) local.mul_add += changed;
      else local.adam_mixed += changed;
      if (!changed) break;
    }
  }
  if (!disabled.count("MusaGroupedResourceApplyAdam"))
    local.adam_grouped_nodes = group_adam(&g, &local.adam_groups);
  const std::string out = serialize_graph(g);
  void* buf = malloc(out.size() ? out.size() : 1);
  if (!buf) return set_error(status, TFMA_RESOURCE_EXHAUSTED, "TFMA_OptimizeGraph: out of memory");
  memcpy(buf, out.data(), out.size());
  *optimized = buf;
  *optimized_bytes = out.size();
  if (stats) *stats = local;
  return set_error(status, TFMA_OK, "");
}

void TFMA_FreeBuffer(void* p) { free(p); }

}  // extern "C"
