// A stand-in for the TensorFlow runtime side of the C API, for testing the
// PluggableDevice adapter (libtfma_tf.so) without TensorFlow.  TEST
// INFRASTRUCTURE ONLY.
//
// It implements the TF_* functions the adapter imports, recording what the
// adapter registers (kernel builders with their type constraints and
// HostMemory arguments, op definitions with their shape functions) and
// running registered kernels on a context the test builds: inputs are
// caller-provided buffers (device or host), outputs and temporaries are
// allocated through the plugin's own SP_StreamExecutor::allocate (as
// TensorFlow's BFC allocator sits on top of it), the stream is a plugin
// SP_Stream, and resource-variable inputs resolve to caller buffers.  Test
// hooks are the fake_* functions at the end.
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "tf_c_api.h"

struct TF_Status {
  TF_Code code = TF_OK;
  std::string msg;
};

struct TF_Tensor {
  void* data = nullptr;
  TF_DataType dtype = TF_FLOAT;
  std::vector<int64_t> dims;
};

struct KernelReg {
  std::string op, device;
  void* (*create)(TF_OpKernelConstruction*) = nullptr;
  void (*compute)(void*, TF_OpKernelContext*) = nullptr;
  void (*destroy)(void*) = nullptr;
  std::vector<std::pair<std::string, int>> types;
  std::vector<std::string> host_memory;
  int priority = 0;
  bool registered = false;
};
struct TF_KernelBuilder {
  KernelReg reg;
};

struct OpReg {
  std::string name;
  std::vector<std::string> inputs, outputs, attrs;
  bool stateful = false, commutative = false;
  void (*shape_fn)(TF_ShapeInferenceContext*, TF_Status*) = nullptr;
};
struct TF_OpDefinitionBuilder {
  OpReg reg;
};

struct TF_ShapeHandle {
  int rank = -1;  // -1: unknown
  std::vector<int64_t> dims;  // -1: unknown dimension
};
struct TF_DimensionHandle {
  int64_t value = -1;
};
struct TF_ShapeInferenceContext {
  std::vector<TF_ShapeHandle> inputs;
  TF_ShapeHandle output;
  bool output_set = false;
};

struct AttrValue {
  int kind = 0;  // 1 float, 2 bool, 3 int, 4 string, 5 type
  float f = 0.f;
  bool b = false;
  int64_t i = 0;
  std::string s;
};

struct Buffer {
  SP_DeviceMemoryBase mem;
};

struct TF_OpKernelContext {
  SP_Stream stream = nullptr;
  const SP_StreamExecutor* se = nullptr;
  const SP_Device* device = nullptr;
  struct Input {
    TF_Tensor t;
    bool variable = false;
    bool forwardable = false;
  };
  std::vector<Input> inputs;
  std::map<int, TF_Tensor> outputs;
  std::map<int, int> forwarded;  // output -> input
  std::vector<Buffer> allocations;
  std::map<std::string, AttrValue> attrs;
  TF_Status status;
  bool failed = false;
  int locks_taken = 0;
  int lock_holders_live = 0;
  int variable_reads = 0;
  int variable_reads_locked = 0;
  ~TF_OpKernelContext() {
    for (Buffer& b : allocations)
      if (se && se->deallocate) se->deallocate(device, &b.mem);
  }
};
struct TF_OpKernelConstruction {
  TF_OpKernelContext* ctx;
  TF_Status status;
  bool failed = false;
};
struct TF_VariableInputLockHolder {
  TF_OpKernelContext* ctx;
};
struct TF_GrapplerItem {
  std::vector<std::string> fetch, preserve;
};

namespace {
std::mutex g_mu;
std::vector<KernelReg> g_kernels;
std::vector<OpReg> g_ops;
int g_statuses_live = 0;

size_t dtype_size(TF_DataType dt) {
  switch (dt) {
    case TF_HALF: case TF_BFLOAT16: case TF_INT16: case TF_UINT16: return 2;
    case TF_DOUBLE: case TF_INT64: case TF_UINT64: case TF_COMPLEX64: return 8;
    case TF_INT8: case TF_UINT8: case TF_BOOL: return 1;
    case TF_COMPLEX128: return 16;
    default: return 4;
  }
}

int64_t elements(const std::vector<int64_t>& d) {
  int64_t n = 1;
  for (int64_t x : d) n *= x;
  return n;
}

void set(TF_Status* s, TF_Code c, const std::string& m) {
  if (!s) return;
  s->code = c;
  s->msg = m;
}

TF_Tensor* alloc_on_device(TF_OpKernelContext* ctx, TF_DataType dt, const int64_t* dims,
                           int nd, TF_Status* s) {
  auto* t = new TF_Tensor();
  t->dtype = dt;
  t->dims.assign(dims, dims + nd);
  const uint64_t bytes = static_cast<uint64_t>(elements(t->dims)) * dtype_size(dt);
  if (bytes > 0) {
    Buffer b{};
    b.mem.struct_size = SP_DEVICE_MEMORY_BASE_STRUCT_SIZE;
    ctx->se->allocate(ctx->device, bytes, 0, &b.mem);
    if (!b.mem.opaque) {
      delete t;
      set(s, TF_RESOURCE_EXHAUSTED, "fake TF: allocation failed");
      return nullptr;
    }
    ctx->allocations.push_back(b);
    t->data = b.mem.opaque;
  }
  set(s, TF_OK, "");
  return t;
}

std::string json_str(const std::string& v) {
  std::string o = "\"";
  for (char c : v) {
    if (c == '"' || c == '\\') o += '\\';
    o += c;
  }
  return o + "\"";
}
}  // namespace

extern "C" {

// ---- tf_status.h ----------------------------------------------------------
TF_Status* TF_NewStatus(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  ++g_statuses_live;
  return new TF_Status();
}
void TF_DeleteStatus(TF_Status* s) {
  std::lock_guard<std::mutex> lk(g_mu);
  --g_statuses_live;
  delete s;
}
void TF_SetStatus(TF_Status* s, TF_Code code, const char* msg) { set(s, code, msg ? msg : ""); }
TF_Code TF_GetCode(const TF_Status* s) { return s->code; }
const char* TF_Message(const TF_Status* s) { return s->msg.c_str(); }

// ---- tf_tensor.h ----------------------------------------------------------
void TF_DeleteTensor(TF_Tensor* t) { delete t; }
TF_DataType TF_TensorType(const TF_Tensor* t) { return t->dtype; }
int TF_NumDims(const TF_Tensor* t) { return static_cast<int>(t->dims.size()); }
int64_t TF_Dim(const TF_Tensor* t, int i) { return t->dims[i]; }
size_t TF_TensorByteSize(const TF_Tensor* t) {
  return static_cast<size_t>(elements(t->dims)) * dtype_size(t->dtype);
}
void* TF_TensorData(const TF_Tensor* t) { return t->data; }
int64_t TF_TensorElementCount(const TF_Tensor* t) { return elements(t->dims); }

// ---- kernels.h: registration ---------------------------------------------
TF_KernelBuilder* TF_NewKernelBuilder(const char* op, const char* device,
                                      void* (*create)(TF_OpKernelConstruction*),
                                      void (*compute)(void*, TF_OpKernelContext*),
                                      void (*destroy)(void*)) {
  auto* b = new TF_KernelBuilder();
  b->reg.op = op;
  b->reg.device = device;
  b->reg.create = create;
  b->reg.compute = compute;
  b->reg.destroy = destroy;
  return b;
}
void TF_KernelBuilder_TypeConstraint(TF_KernelBuilder* b, const char* attr, const TF_DataType t,
                                     TF_Status* s) {
  b->reg.types.emplace_back(attr, static_cast<int>(t));
  set(s, TF_OK, "");
}
void TF_KernelBuilder_HostMemory(TF_KernelBuilder* b, const char* arg) {
  b->reg.host_memory.emplace_back(arg);
}
void TF_KernelBuilder_Priority(TF_KernelBuilder* b, int32_t p) { b->reg.priority = p; }
void TF_RegisterKernelBuilder(const char* name, TF_KernelBuilder* b, TF_Status* s) {
  std::lock_guard<std::mutex> lk(g_mu);
  b->reg.registered = true;
  if (b->reg.op != name) {
    set(s, TF_INVALID_ARGUMENT, "kernel name differs from op name");
    return;
  }
  g_kernels.push_back(b->reg);
  delete b;  // TensorFlow takes ownership of a registered builder
  set(s, TF_OK, "");
}
void TF_DeleteKernelBuilder(TF_KernelBuilder* b) { delete b; }

// ---- kernels.h: context ---------------------------------------------------
SP_Stream TF_GetStream(TF_OpKernelContext* ctx, TF_Status* s) {
  if (!ctx->stream) {
    set(s, TF_FAILED_PRECONDITION, "fake TF: no stream");
    return nullptr;
  }
  set(s, TF_OK, "");
  return ctx->stream;
}
int TF_NumInputs(TF_OpKernelContext* ctx) { return static_cast<int>(ctx->inputs.size()); }
int TF_NumOutputs(TF_OpKernelContext* ctx) { return static_cast<int>(ctx->outputs.size()); }
void TF_GetInput(TF_OpKernelContext* ctx, int i, TF_Tensor** t, TF_Status* s) {
  if (i < 0 || i >= static_cast<int>(ctx->inputs.size())) {
    set(s, TF_OUT_OF_RANGE, "fake TF: input index out of range");
    return;
  }
  if (ctx->inputs[i].variable) {
    set(s, TF_INVALID_ARGUMENT, "fake TF: TF_GetInput on a resource input");
    return;
  }
  *t = new TF_Tensor(ctx->inputs[i].t);
  set(s, TF_OK, "");
}
void TF_SetOutput(TF_OpKernelContext* ctx, int i, const TF_Tensor* t, TF_Status* s) {
  ctx->outputs[i] = *t;
  set(s, TF_OK, "");
}
void TF_OpKernelContext_Failure(TF_OpKernelContext* ctx, TF_Status* s) {
  ctx->failed = true;
  ctx->status = *s;
}
TF_Tensor* TF_AllocateOutput(TF_OpKernelContext* ctx, int index, TF_DataType dtype,
                             const int64_t* dims, int num_dims, size_t len, TF_Status* s) {
  std::vector<int64_t> d(dims, dims + num_dims);
  if (len != static_cast<size_t>(elements(d)) * dtype_size(dtype)) {
    set(s, TF_INVALID_ARGUMENT, "fake TF: TF_AllocateOutput len does not match the shape");
    return nullptr;
  }
  TF_Tensor* t = alloc_on_device(ctx, dtype, dims, num_dims, s);
  if (t) ctx->outputs[index] = *t;
  return t;
}
TF_Tensor* TF_ForwardInputOrAllocateOutput(TF_OpKernelContext* ctx, const int* cand, int ncand,
                                           int index, const int64_t* dims, int nd, int* fwd,
                                           TF_Status* s) {
  std::vector<int64_t> d(dims, dims + nd);
  for (int k = 0; k < ncand; ++k) {
    const int i = cand[k];
    if (i < 0 || i >= static_cast<int>(ctx->inputs.size())) continue;
    const auto& in = ctx->inputs[i];
    if (in.forwardable && in.t.dims == d) {
      ctx->outputs[index] = in.t;
      ctx->forwarded[index] = i;
      if (fwd) *fwd = i;
      set(s, TF_OK, "");
      return new TF_Tensor(in.t);
    }
  }
  if (fwd) *fwd = -1;
  const TF_DataType dt = ncand > 0 && cand[0] < static_cast<int>(ctx->inputs.size())
                             ? ctx->inputs[cand[0]].t.dtype
                             : TF_FLOAT;
  TF_Tensor* t = alloc_on_device(ctx, dt, dims, nd, s);
  if (t) ctx->outputs[index] = *t;
  return t;
}
TF_Tensor* TF_AllocateTemp(TF_OpKernelContext* ctx, TF_DataType dtype, const int64_t* dims,
                           int nd, TF_AllocatorAttributes* attrs, TF_Status* s) {
  if (attrs && attrs->on_host) {
    set(s, TF_UNIMPLEMENTED, "fake TF: host temporaries are not used by the adapter");
    return nullptr;
  }
  return alloc_on_device(ctx, dtype, dims, nd, s);
}

// ---- kernels.h: construction attributes -------------------------------------
namespace {
const AttrValue* find_attr(TF_OpKernelConstruction* c, const char* name, int kind, TF_Status* s) {
  auto it = c->ctx->attrs.find(name);
  if (it == c->ctx->attrs.end()) {
    set(s, TF_INVALID_ARGUMENT, std::string("fake TF: no attr named ") + name);
    return nullptr;
  }
  if (it->second.kind != kind) {
    set(s, TF_INVALID_ARGUMENT, std::string("fake TF: attr ") + name + " has another type");
    return nullptr;
  }
  set(s, TF_OK, "");
  return &it->second;
}
}  // namespace

void TF_OpKernelConstruction_GetAttrSize(TF_OpKernelConstruction* c, const char* name,
                                         int32_t* list_size, int32_t* total_size, TF_Status* s) {
  if (const AttrValue* a = find_attr(c, name, 4, s)) {
    *list_size = -1;
    *total_size = static_cast<int32_t>(a->s.size());
  }
}
void TF_OpKernelConstruction_GetAttrType(TF_OpKernelConstruction* c, const char* name,
                                         TF_DataType* v, TF_Status* s) {
  if (const AttrValue* a = find_attr(c, name, 5, s)) *v = static_cast<TF_DataType>(a->i);
}
void TF_OpKernelConstruction_GetAttrInt32(TF_OpKernelConstruction* c, const char* name,
                                          int32_t* v, TF_Status* s) {
  if (const AttrValue* a = find_attr(c, name, 3, s)) *v = static_cast<int32_t>(a->i);
}
void TF_OpKernelConstruction_GetAttrFloat(TF_OpKernelConstruction* c, const char* name, float* v,
                                          TF_Status* s) {
  if (const AttrValue* a = find_attr(c, name, 1, s)) *v = a->f;
}
void TF_OpKernelConstruction_GetAttrBool(TF_OpKernelConstruction* c, const char* name,
                                         TF_Bool* v, TF_Status* s) {
  if (const AttrValue* a = find_attr(c, name, 2, s)) *v = a->b ? 1 : 0;
}
void TF_OpKernelConstruction_GetAttrString(TF_OpKernelConstruction* c, const char* name,
                                           char* v, size_t max_length, TF_Status* s) {
  if (const AttrValue* a = find_attr(c, name, 4, s)) {
    const size_t n = a->s.size() < max_length ? a->s.size() : max_length;
    memcpy(v, a->s.data(), n);
  }
}
bool TF_OpKernelConstruction_HasAttr(TF_OpKernelConstruction* c, const char* name,
                                     TF_Status* s) {
  set(s, TF_OK, "");
  return c->ctx->attrs.count(name) != 0;
}
void TF_OpKernelConstruction_Failure(TF_OpKernelConstruction* c, TF_Status* s) {
  c->failed = true;
  c->status = *s;
}

// ---- kernels_experimental.h -----------------------------------------------
void TF_MaybeLockVariableInput(TF_OpKernelContext* ctx, int* inputs, size_t len, bool, bool,
                               void (*)(TF_OpKernelContext*, TF_Tensor*, TF_Tensor*),
                               TF_VariableInputLockHolder** holder, TF_Status* s) {
  for (size_t i = 0; i < len; ++i) {
    if (inputs[i] < 0 || inputs[i] >= static_cast<int>(ctx->inputs.size()) ||
        !ctx->inputs[inputs[i]].variable) {
      set(s, TF_INVALID_ARGUMENT, "fake TF: locking a non-variable input");
      return;
    }
  }
  ctx->locks_taken += static_cast<int>(len);
  ctx->lock_holders_live++;
  *holder = new TF_VariableInputLockHolder{ctx};
  set(s, TF_OK, "");
}
void TF_GetInputTensorFromVariable(TF_OpKernelContext* ctx, int input, bool lock_held, bool,
                                   bool, void (*)(TF_OpKernelContext*, TF_Tensor*, TF_Tensor*),
                                   TF_Tensor** out, TF_Status* s) {
  if (input < 0 || input >= static_cast<int>(ctx->inputs.size()) ||
      !ctx->inputs[input].variable) {
    set(s, TF_INVALID_ARGUMENT, "fake TF: input is not a variable");
    return;
  }
  ctx->variable_reads++;
  if (lock_held) ctx->variable_reads_locked++;
  *out = new TF_Tensor(ctx->inputs[input].t);
  set(s, TF_OK, "");
}
void TF_ReleaseVariableInputLockHolder(TF_VariableInputLockHolder* h) {
  if (!h) return;
  h->ctx->lock_holders_live--;
  delete h;
}

// ---- ops.h -----------------------------------------------------------------
TF_OpDefinitionBuilder* TF_NewOpDefinitionBuilder(const char* name) {
  auto* b = new TF_OpDefinitionBuilder();
  b->reg.name = name;
  return b;
}
void TF_RegisterOpDefinition(TF_OpDefinitionBuilder* b, TF_Status* s) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (const OpReg& o : g_ops)
    if (o.name == b->reg.name) {
      delete b;
      set(s, TF_ALREADY_EXISTS, "fake TF: op already registered");
      return;
    }
  g_ops.push_back(b->reg);
  delete b;
  set(s, TF_OK, "");
}
void TF_DeleteOpDefinitionBuilder(TF_OpDefinitionBuilder* b) { delete b; }
void TF_OpDefinitionBuilderAddAttr(TF_OpDefinitionBuilder* b, const char* spec) {
  b->reg.attrs.emplace_back(spec);
}
void TF_OpDefinitionBuilderAddInput(TF_OpDefinitionBuilder* b, const char* spec) {
  b->reg.inputs.emplace_back(spec);
}
void TF_OpDefinitionBuilderAddOutput(TF_OpDefinitionBuilder* b, const char* spec) {
  b->reg.outputs.emplace_back(spec);
}
void TF_OpDefinitionBuilderSetIsCommutative(TF_OpDefinitionBuilder* b, bool v) {
  b->reg.commutative = v;
}
void TF_OpDefinitionBuilderSetIsStateful(TF_OpDefinitionBuilder* b, bool v) {
  b->reg.stateful = v;
}
void TF_OpDefinitionBuilderSetShapeInferenceFunction(
    TF_OpDefinitionBuilder* b, void (*fn)(TF_ShapeInferenceContext*, TF_Status*)) {
  b->reg.shape_fn = fn;
}
int64_t TF_ShapeInferenceContextNumInputs(TF_ShapeInferenceContext* c) {
  return static_cast<int64_t>(c->inputs.size());
}
TF_ShapeHandle* TF_NewShapeHandle(void) { return new TF_ShapeHandle(); }
void TF_DeleteShapeHandle(TF_ShapeHandle* h) { delete h; }
TF_DimensionHandle* TF_NewDimensionHandle(void) { return new TF_DimensionHandle(); }
void TF_DeleteDimensionHandle(TF_DimensionHandle* h) { delete h; }
void TF_ShapeInferenceContextGetInput(TF_ShapeInferenceContext* c, int i, TF_ShapeHandle* h,
                                      TF_Status* s) {
  if (i < 0 || i >= static_cast<int>(c->inputs.size())) {
    set(s, TF_INVALID_ARGUMENT, "fake TF: shape input out of range");
    return;
  }
  *h = c->inputs[i];
  set(s, TF_OK, "");
}
void TF_ShapeInferenceContextSetOutput(TF_ShapeInferenceContext* c, int i, TF_ShapeHandle* h,
                                       TF_Status* s) {
  if (i != 0) {
    set(s, TF_INVALID_ARGUMENT, "fake TF: only output 0 is recorded");
    return;
  }
  c->output = *h;
  c->output_set = true;
  set(s, TF_OK, "");
}
void TF_ShapeInferenceContextSetUnknownShape(TF_ShapeInferenceContext* c, TF_Status* s) {
  c->output = TF_ShapeHandle();
  c->output_set = true;
  set(s, TF_OK, "");
}
int TF_ShapeInferenceContextRankKnown(TF_ShapeInferenceContext*, TF_ShapeHandle* h) {
  return h->rank >= 0;
}
int64_t TF_ShapeInferenceContextRank(TF_ShapeInferenceContext*, TF_ShapeHandle* h) {
  return h->rank;
}
void TF_ShapeInferenceContextDim(TF_ShapeInferenceContext*, TF_ShapeHandle* h, int64_t i,
                                 TF_DimensionHandle* d) {
  d->value = (i >= 0 && i < h->rank) ? h->dims[i] : -1;
}
int TF_DimensionHandleValueKnown(TF_DimensionHandle* d) { return d->value >= 0; }
int64_t TF_DimensionHandleValue(TF_DimensionHandle* d) { return d->value; }

// ---- grappler.h ------------------------------------------------------------
namespace {
void list_size(const std::vector<std::string>& v, int* n, size_t* bytes) {
  *n = static_cast<int>(v.size());
  *bytes = 0;
  for (const std::string& x : v) *bytes += x.size();
}
void list_values(const std::vector<std::string>& v, char** values, size_t* lengths, int n,
                 void* storage, size_t storage_size, TF_Status* s) {
  char* p = static_cast<char*>(storage);
  size_t used = 0;
  for (int i = 0; i < n && i < static_cast<int>(v.size()); ++i) {
    if (used + v[i].size() > storage_size) {
      set(s, TF_INVALID_ARGUMENT, "fake TF: storage too small");
      return;
    }
    memcpy(p + used, v[i].data(), v[i].size());
    values[i] = p + used;
    lengths[i] = v[i].size();
    used += v[i].size();
  }
  set(s, TF_OK, "");
}
}  // namespace
void TF_GetFetchNodesListSize(const TF_GrapplerItem* item, int* n, size_t* bytes, TF_Status* s) {
  list_size(item->fetch, n, bytes);
  set(s, TF_OK, "");
}
void TF_GetFetchNodesList(const TF_GrapplerItem* item, char** values, size_t* lengths, int n,
                          void* storage, size_t storage_size, TF_Status* s) {
  list_values(item->fetch, values, lengths, n, storage, storage_size, s);
}
void TF_GetNodesToPreserveListSize(const TF_GrapplerItem* item, int* n, size_t* bytes,
                                   TF_Status* s) {
  list_size(item->preserve, n, bytes);
  set(s, TF_OK, "");
}
void TF_GetNodesToPreserveList(const TF_GrapplerItem* item, char** values, size_t* lengths,
                               int n, void* storage, size_t storage_size, TF_Status* s) {
  list_values(item->preserve, values, lengths, n, storage, storage_size, s);
}

// ===========================================================================
// Test hooks.
// ===========================================================================
int fake_kernel_count(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  return static_cast<int>(g_kernels.size());
}

// JSON description of kernel registration i, into buf (NUL-terminated).
int fake_kernel_describe(int i, char* buf, int cap) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (i < 0 || i >= static_cast<int>(g_kernels.size())) return -1;
  const KernelReg& k = g_kernels[i];
  std::string j = "{\"op\": " + json_str(k.op) + ", \"device\": " + json_str(k.device) +
                  ", \"types\": [";
  for (size_t q = 0; q < k.types.size(); ++q)
    j += (q ? ", " : "") + std::string("[") + json_str(k.types[q].first) + ", " +
         std::to_string(k.types[q].second) + "]";
  j += "], \"host_memory\": [";
  for (size_t q = 0; q < k.host_memory.size(); ++q)
    j += (q ? ", " : "") + json_str(k.host_memory[q]);
  j += "], \"has_create\": " + std::string(k.create ? "true" : "false") +
       ", \"has_compute\": " + (k.compute ? "true" : "false") +
       ", \"has_delete\": " + (k.destroy ? "true" : "false") + "}";
  snprintf(buf, cap, "%s", j.c_str());
  return static_cast<int>(j.size());
}

int fake_op_count(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  return static_cast<int>(g_ops.size());
}

int fake_op_describe(int i, char* buf, int cap) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (i < 0 || i >= static_cast<int>(g_ops.size())) return -1;
  const OpReg& o = g_ops[i];
  auto list = [](const std::vector<std::string>& v) {
    std::string r = "[";
    for (size_t q = 0; q < v.size(); ++q) r += (q ? ", " : "") + json_str(v[q]);
    return r + "]";
  };
  std::string j = "{\"name\": " + json_str(o.name) + ", \"inputs\": " + list(o.inputs) +
                  ", \"outputs\": " + list(o.outputs) + ", \"attrs\": " + list(o.attrs) +
                  ", \"stateful\": " + (o.stateful ? "true" : "false") +
                  ", \"has_shape_fn\": " + (o.shape_fn ? "true" : "false") + "}";
  snprintf(buf, cap, "%s", j.c_str());
  return static_cast<int>(j.size());
}

// Runs op i's shape function on inputs given as ranks (-1 unknown) and
// flattened dims (-1 unknown); writes output 0's rank (-1 unknown) and dims.
int fake_op_infer(int i, int n, const int* ranks, const int64_t* dims, int* out_rank,
                  int64_t* out_dims, char* msg, int cap) {
  OpReg o;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    if (i < 0 || i >= static_cast<int>(g_ops.size())) return -1;
    o = g_ops[i];
  }
  TF_ShapeInferenceContext c;
  size_t off = 0;
  for (int k = 0; k < n; ++k) {
    TF_ShapeHandle h;
    h.rank = ranks[k];
    for (int q = 0; q < ranks[k]; ++q) h.dims.push_back(dims[off++]);
    c.inputs.push_back(h);
  }
  TF_Status s;
  o.shape_fn(&c, &s);
  snprintf(msg, cap, "%s", s.msg.c_str());
  *out_rank = c.output_set ? c.output.rank : -2;  // -2: no output set
  for (int q = 0; q < c.output.rank; ++q) out_dims[q] = c.output.dims[q];
  return s.code;
}

int fake_statuses_live(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  return g_statuses_live;
}

TF_OpKernelContext* fake_ctx_new(SP_Stream stream, const SP_StreamExecutor* se,
                                 const SP_Device* device) {
  auto* c = new TF_OpKernelContext();
  c->stream = stream;
  c->se = se;
  c->device = device;
  return c;
}
void fake_ctx_free(TF_OpKernelContext* c) { delete c; }
void fake_ctx_add_input(TF_OpKernelContext* c, void* data, int dtype, int nd,
                        const int64_t* dims, int variable, int forwardable) {
  TF_OpKernelContext::Input in;
  in.t.data = data;
  in.t.dtype = static_cast<TF_DataType>(dtype);
  in.t.dims.assign(dims, dims + nd);
  in.variable = variable != 0;
  in.forwardable = forwardable != 0;
  c->inputs.push_back(in);
}
void fake_ctx_attr_float(TF_OpKernelContext* c, const char* n, float v) {
  AttrValue a;
  a.kind = 1;
  a.f = v;
  c->attrs[n] = a;
}
void fake_ctx_attr_bool(TF_OpKernelContext* c, const char* n, int v) {
  AttrValue a;
  a.kind = 2;
  a.b = v != 0;
  c->attrs[n] = a;
}
void fake_ctx_attr_int(TF_OpKernelContext* c, const char* n, int64_t v) {
  AttrValue a;
  a.kind = 3;
  a.i = v;
  c->attrs[n] = a;
}
void fake_ctx_attr_string(TF_OpKernelContext* c, const char* n, const char* v) {
  AttrValue a;
  a.kind = 4;
  a.s = v;
  c->attrs[n] = a;
}
void fake_ctx_attr_type(TF_OpKernelContext* c, const char* n, int v) {
  AttrValue a;
  a.kind = 5;
  a.i = v;
  c->attrs[n] = a;
}

// Constructs registration i's kernel on ctx's attrs, runs compute, deletes
// it.  Returns the TF_Code (construction or compute failure), message in
// msg.
int fake_ctx_run(TF_OpKernelContext* c, int i, char* msg, int cap) {
  KernelReg k;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    if (i < 0 || i >= static_cast<int>(g_kernels.size())) return -1;
    k = g_kernels[i];
  }
  TF_OpKernelConstruction con{c, TF_Status(), false};
  void* kernel = k.create ? k.create(&con) : nullptr;
  if (con.failed) {
    if (k.destroy && kernel) k.destroy(kernel);
    snprintf(msg, cap, "%s", con.status.msg.c_str());
    return con.status.code;
  }
  k.compute(kernel, c);
  if (k.destroy) k.destroy(kernel);
  snprintf(msg, cap, "%s", c->failed ? c->status.msg.c_str() : "");
  return c->failed ? c->status.code : TF_OK;
}

int fake_ctx_num_outputs(TF_OpKernelContext* c) { return static_cast<int>(c->outputs.size()); }

// Output i: data pointer; dtype, rank and dims through the pointers;
// *forwarded_from = the input it aliases, or -1.  Null if not set.
void* fake_ctx_output(TF_OpKernelContext* c, int i, int* dtype, int* nd, int64_t* dims,
                      int* forwarded_from) {
  auto it = c->outputs.find(i);
  if (it == c->outputs.end()) return nullptr;
  *dtype = it->second.dtype;
  *nd = static_cast<int>(it->second.dims.size());
  for (int q = 0; q < *nd; ++q) dims[q] = it->second.dims[q];
  auto f = c->forwarded.find(i);
  *forwarded_from = f == c->forwarded.end() ? -1 : f->second;
  return it->second.data;
}
int fake_ctx_has_output(TF_OpKernelContext* c, int i) { return c->outputs.count(i) ? 1 : 0; }

// Lock bookkeeping: variable inputs locked, lock holders not released,
// variable reads, and those made with the lock held.
void fake_ctx_lock_stats(TF_OpKernelContext* c, int* locked, int* live, int* reads,
                         int* reads_locked) {
  *locked = c->locks_taken;
  *live = c->lock_holders_live;
  *reads = c->variable_reads;
  *reads_locked = c->variable_reads_locked;
}

TF_GrapplerItem* fake_item_new(void) { return new TF_GrapplerItem(); }
void fake_item_free(TF_GrapplerItem* it) { delete it; }
void fake_item_add_fetch(TF_GrapplerItem* it, const char* name) { it->fetch.emplace_back(name); }
void fake_item_add_preserve(TF_GrapplerItem* it, const char* name) {
  it->preserve.emplace_back(name);
}

}  // extern "C"
