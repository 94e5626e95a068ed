// Op layer of the C ABI: argument validation, TF shape rules, host scalar
// arithmetic and dispatch to the gfx950 kernels.  Each TFMA_* entry point
// mirrors the Compute() of the reference op it replaces (cited per entry
// point in include/tfma.h); error codes and messages follow the reference
// where it defines them and TensorFlow's CPU kernels otherwise.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <cmath>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "device_util.h"
#include "tfma_internal.h"

namespace tfma {
namespace {

// ---------------------------------------------------------------------------
// Status helpers.
// ---------------------------------------------------------------------------
int set_status(TFMA_Status* st, int code, const char* fmt, ...) {
  if (st) {
    st->code = code;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(st->message, sizeof(st->message), fmt, ap);
    va_end(ap);
  }
  return code;
}
int ok(TFMA_Status* st) {
  if (st) {
    st->code = TFMA_OK;
    st->message[0] = '\0';
  }
  return TFMA_OK;
}
int hip_status(TFMA_Status* st, hipError_t e, const char* what) {
  if (e == hipSuccess) return ok(st);
  return set_status(st, TFMA_INTERNAL, "%s launch failed: %s", what,
                    hipGetErrorString(e));
}

std::string shape_str(const TFMA_Tensor* t) {
  std::string s = "[";
  for (int i = 0; i < t->ndims; ++i) {
    if (i) s += ",";
    s += std::to_string(t->dims[i]);
  }
  return s + "]";
}

int64_t num_elements(const TFMA_Tensor* t) {
  int64_t n = 1;
  for (int i = 0; i < t->ndims; ++i) n *= t->dims[i];
  return n;
}

bool same_shape(const TFMA_Tensor* a, const TFMA_Tensor* b) {
  if (a->ndims != b->ndims) return false;
  for (int i = 0; i < a->ndims; ++i)
    if (a->dims[i] != b->dims[i]) return false;
  return true;
}

bool valid_tensor(const TFMA_Tensor* t) {
  if (!t || t->ndims < 0 || t->ndims > TFMA_MAX_DIMS) return false;
  for (int i = 0; i < t->ndims; ++i)
    if (t->dims[i] < 0) return false;
  return true;
}

const char* dtype_name(int dt) {
  switch (dt) {
    case TFMA_FLOAT: return "float";
    case TFMA_DOUBLE: return "double";
    case TFMA_HALF: return "half";
    case TFMA_BFLOAT16: return "bfloat16";
    case TFMA_INT32: return "int32";
    case TFMA_INT64: return "int64";
    case TFMA_UINT8: return "uint8";
  }
  return "unknown";
}

bool to_dtype(int dt, DType* out) {
  switch (dt) {
    case TFMA_FLOAT: *out = DType::kF32; return true;
    case TFMA_HALF: *out = DType::kF16; return true;
    case TFMA_BFLOAT16: *out = DType::kBF16; return true;
    case TFMA_DOUBLE: *out = DType::kF64; return true;
  }
  return false;
}

// Integer dtypes an elementwise op takes besides the floating ones: those the
// reference registers for its stock ops - AddV2 / Add int32, int64 and uint8
// (musa_add_op.cc:455-468), Mul int32 and int64 (musa_multiply_op.cc:315-323),
// BiasAdd / BiasAddV1 int32 and int64 (musa_biasadd_op.cc:67-79).  The fused
// ops, Relu and ReluGrad are floating only.  (The reference's bool Add is
// not taken: its arithmetic is muDNN's and nothing pins it.)
enum class IntTypes { kNone, kI32I64, kI32I64U8 };

bool to_ew_dtype(int dt, IntTypes ints, DType* out) {
  if (to_dtype(dt, out)) return true;
  if (ints == IntTypes::kNone) return false;
  switch (dt) {
    case TFMA_INT32: *out = DType::kI32; return true;
    case TFMA_INT64: *out = DType::kI64; return true;
    case TFMA_UINT8:
      if (ints != IntTypes::kI32I64U8) return false;
      *out = DType::kU8;
      return true;
  }
  return false;
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// ---------------------------------------------------------------------------
// Host half / bfloat16 rounding for the Adam scalars (TF computes alpha and
// 1 - beta in T).
// ---------------------------------------------------------------------------
uint16_t host_f32_to_f16(float f) {
  const uint32_t x = f32_bits(f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t mant = x & 0x7fffffu;
  const int exp = static_cast<int>((x >> 23) & 0xffu);
  if (exp == 255) return static_cast<uint16_t>(sign | 0x7c00u | (mant ? 0x200u | (mant >> 13) : 0u));
  const int e = exp - 127 + 15;
  if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return static_cast<uint16_t>(sign);
    mant |= 0x800000u;
    const int shift = 14 - e;
    uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) ++h;
    return static_cast<uint16_t>(sign | h);
  }
  uint32_t h = (static_cast<uint32_t>(e) << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return static_cast<uint16_t>(sign | h);
}

float host_f16_to_f32(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t mant = h & 0x3ffu;
  if (exp == 0) {
    const float v = static_cast<float>(mant) * (1.0f / 16777216.0f);
    return sign ? -v : v;
  }
  if (exp == 31) return bits_f32(sign | 0x7f800000u | (mant << 13));
  return bits_f32(sign | ((exp + 112u) << 23) | (mant << 13));
}

// Reads a 0-d host scalar of dtype t as a double (exact for every T).
double read_scalar(const TFMA_Tensor* s, DType t) {
  switch (t) {
    case DType::kF32: return *static_cast<const float*>(s->data);
    case DType::kF64: return *static_cast<const double*>(s->data);
    case DType::kF16: return host_f16_to_f32(*static_cast<const uint16_t*>(s->data));
    case DType::kBF16: return bf16_to_f32(*static_cast<const uint16_t*>(s->data));
    default: break;
  }
  return 0.0;
}

// Rounds a float to T's precision (float, half or bfloat16).
float round_to(DType t, float v) {
  switch (t) {
    case DType::kF16: return host_f16_to_f32(host_f32_to_f16(v));
    case DType::kBF16: return bf16_to_f32(f32_to_bf16(v));
    default: return v;
  }
}

// alpha = lr * sqrt(1 - beta2_power) / (1 - beta1_power), each operation in
// T, as TF's CPU ApplyAdam computes it.
AdamScalars adam_scalars(DType t, double b1p, double b2p, double lr,
                         double b1, double b2, double eps) {
  AdamScalars s;
  if (t == DType::kF64) {
    s.alpha = lr * sqrt(1.0 - b2p) / (1.0 - b1p);
    s.one_minus_beta1 = 1.0 - b1;
    s.one_minus_beta2 = 1.0 - b2;
  } else {
    const float fb1p = static_cast<float>(b1p), fb2p = static_cast<float>(b2p);
    const float flr = static_cast<float>(lr);
    const float fb1 = static_cast<float>(b1), fb2 = static_cast<float>(b2);
    volatile float r1 = round_to(t, 1.0f - fb2p);
    volatile float r2 = round_to(t, sqrtf(r1));
    volatile float r3 = round_to(t, flr * r2);
    volatile float r4 = round_to(t, 1.0f - fb1p);
    s.alpha = round_to(t, r3 / r4);
    s.one_minus_beta1 = round_to(t, 1.0f - fb1);
    s.one_minus_beta2 = round_to(t, 1.0f - fb2);
  }
  s.beta1 = b1;
  s.beta2 = b2;
  s.epsilon = eps;
  return s;
}

// ---------------------------------------------------------------------------
// Variable locks: a striped table keyed by the variable's memory; a call
// takes the stripes of var/m/v in ascending order (the reference sorts its
// var/m/v mutexes the same way, musa_applyadam_op.cc:138-156).
// ---------------------------------------------------------------------------
constexpr int kLockStripes = 256;
std::mutex& stripe(int i) {
  static std::mutex* table = new std::mutex[kLockStripes];
  return table[i];
}
int stripe_of(const void* p) {
  const uintptr_t u = reinterpret_cast<uintptr_t>(p);
  return static_cast<int>((u >> 8) * 2654435761u % kLockStripes);
}

class VarLocks {
 public:
  void add(const void* p) { ids_.push_back(stripe_of(p)); }
  void lock() {
    std::sort(ids_.begin(), ids_.end());
    ids_.erase(std::unique(ids_.begin(), ids_.end()), ids_.end());
    for (int i : ids_) stripe(i).lock();
    locked_ = true;
  }
  ~VarLocks() {
    if (!locked_) return;
    for (auto it = ids_.rbegin(); it != ids_.rend(); ++it) stripe(*it).unlock();
  }

 private:
  std::vector<int> ids_;
  bool locked_ = false;
};

// ---------------------------------------------------------------------------
// Pinned staging ring for small host->device uploads (grouped Adam tables).
// A slot is reused only after the event recorded behind its copy completes.
// ---------------------------------------------------------------------------
class PinnedRing {
 public:
  static constexpr size_t kSlotBytes = 1024 * 1024;
  static constexpr int kSlots = 16;

  // Copies `bytes` from `src` to device `dst` on `stream`, in pieces of at
  // most one slot (a table above 1 MiB - more than about 256M parameters of
  // chunk map - takes several slots; only a table larger than the whole ring
  // waits for its own earlier pieces to be copied).
  hipError_t upload(void* dst, const void* src, size_t bytes,
                    hipStream_t stream) {
    std::lock_guard<std::mutex> lk(mu_);
    hipError_t e = ensure();
    if (e != hipSuccess) return e;
    for (size_t off = 0; off < bytes; off += kSlotBytes) {
      const size_t piece = std::min(kSlotBytes, bytes - off);
      const int s = next_;
      next_ = (next_ + 1) % kSlots;
      if (used_[s]) {
        e = hipEventSynchronize(events_[s]);
        if (e != hipSuccess) return e;
      }
      char* slot = static_cast<char*>(host_) + s * kSlotBytes;
      memcpy(slot, static_cast<const char*>(src) + off, piece);
      e = hipMemcpyAsync(static_cast<char*>(dst) + off, slot, piece, hipMemcpyHostToDevice,
                         stream);
      if (e != hipSuccess) return e;
      e = hipEventRecord(events_[s], stream);
      if (e != hipSuccess) return e;
      used_[s] = true;
    }
    return hipSuccess;
  }

 private:
  hipError_t ensure() {
    if (host_) return hipSuccess;
    hipError_t e = hipHostMalloc(&host_, kSlotBytes * kSlots, hipHostMallocDefault);
    if (e != hipSuccess) {
      host_ = nullptr;
      return e;
    }
    for (int i = 0; i < kSlots; ++i) {
      e = hipEventCreateWithFlags(&events_[i], hipEventDisableTiming);
      if (e != hipSuccess) return e;
      used_[i] = false;
    }
    return hipSuccess;
  }
  std::mutex mu_;
  void* host_ = nullptr;
  hipEvent_t events_[kSlots];
  bool used_[kSlots];
  int next_ = 0;
};

// One ring per device: its events belong to the device that was current
// when they were created, and are recorded on that device's streams only.
PinnedRing* pinned_ring(int dev) {
  static PinnedRing* rings[64] = {nullptr};
  static std::mutex mu;
  if (dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lk(mu);
  if (!rings[dev]) rings[dev] = new PinnedRing();
  return rings[dev];
}

// ---------------------------------------------------------------------------
// Device copies of recently used grouped-Adam tables, per device.  Training
// calls the grouped update with the same tensors every step, so the table
// (tensor pointers, sizes, chunk offsets) repeats; a call whose table equals
// a cached one launches on the cached copy and uploads nothing.  A slot is
// refilled only after the event recorded behind its last use has completed;
// a call on another stream first waits for the slot's fill.
// ---------------------------------------------------------------------------
class AdamTableCache {
 public:
  static constexpr int kSlots = 8;
  static constexpr int kDevices = 64;

  // The cached device table equal to `t`, made ready on `stream`, or null.
  // On success the slot is pinned (fill() will not reuse it) until the
  // caller, after enqueuing its launch, calls mark_used(), which records the
  // slot's use behind that launch and unpins it.
  const void* find(int dev, const std::vector<uint8_t>& t, hipStream_t stream, int* slot) {
    std::lock_guard<std::mutex> lk(mu_);
    if (dev < 0 || dev >= kDevices) return nullptr;
    for (int i = 0; i < kSlots; ++i) {
      Slot& s = slots_[dev][i];
      if (!s.valid || s.host.size() != t.size() || memcmp(s.host.data(), t.data(), t.size()) != 0)
        continue;
      // The copy that filled the slot may still be in flight (on any stream:
      // a stream handle can be recycled after its stream is destroyed).
      if (hipEventQuery(s.ready) != hipSuccess && hipStreamWaitEvent(stream, s.ready, 0) != hipSuccess)
        return nullptr;
      s.tick = ++tick_;
      ++s.pins;
      *slot = i;
      return s.dev;
    }
    return nullptr;
  }

  void mark_used(int dev, int slot, hipStream_t stream) {
    std::lock_guard<std::mutex> lk(mu_);
    Slot& s = slots_[dev][slot];
    // `used` completes only after every launch that reads the slot: a use
    // still pending on another stream is chained in before the record (the
    // launch itself, already enqueued, does not wait for it).
    if (s.used_stream != stream && hipEventQuery(s.used) == hipErrorNotReady)
      (void)hipStreamWaitEvent(stream, s.used, 0);
    (void)hipEventRecord(s.used, stream);
    s.used_stream = stream;
    --s.pins;
  }

  // Keeps a copy of the table the caller has just uploaded to `ws` on
  // `stream` (the copy is enqueued behind the launch that reads `ws`).
  // Best effort: any failure just leaves the table uncached.
  void fill(int dev, const std::vector<uint8_t>& t, const void* ws, hipStream_t stream) {
    std::lock_guard<std::mutex> lk(mu_);
    if (dev < 0 || dev >= kDevices) return;
    int pick = -1;
    for (int i = 0; i < kSlots; ++i) {
      Slot& s = slots_[dev][i];
      // Pinned by a call between find() and mark_used(), or still read by
      // an enqueued launch.
      if (s.pins > 0 || (s.valid && hipEventQuery(s.used) != hipSuccess)) continue;
      if (pick < 0 || !s.valid || (slots_[dev][pick].valid && s.tick < slots_[dev][pick].tick))
        pick = i;
      if (!s.valid) break;
    }
    if (pick < 0) return;
    Slot& s = slots_[dev][pick];
    const size_t bytes = t.size();
    s.valid = false;
    if (!s.ready) {
      if (hipEventCreateWithFlags(&s.ready, hipEventDisableTiming) != hipSuccess) return;
      if (hipEventCreateWithFlags(&s.used, hipEventDisableTiming) != hipSuccess) return;
    }
    if (s.cap < bytes) {
      if (s.dev) (void)hipFree(s.dev);  // its last use has completed
      s.dev = nullptr;
      s.cap = 0;
      void* p = nullptr;
      if (hipMalloc(&p, bytes) != hipSuccess) return;
      s.dev = p;
      s.cap = bytes;
    }
    if (hipMemcpyAsync(s.dev, ws, bytes, hipMemcpyDeviceToDevice, stream) != hipSuccess) return;
    if (hipEventRecord(s.ready, stream) != hipSuccess) return;
    if (hipEventRecord(s.used, stream) != hipSuccess) return;
    s.host = t;
    s.used_stream = stream;
    s.tick = ++tick_;
    s.valid = true;
  }

 private:
  struct Slot {
    bool valid = false;
    std::vector<uint8_t> host;
    void* dev = nullptr;
    size_t cap = 0;
    hipEvent_t ready = nullptr;
    hipEvent_t used = nullptr;
    hipStream_t used_stream = nullptr;  // stream of the last record of `used`
    uint64_t tick = 0;
    int pins = 0;  // calls between find() and mark_used()
  };
  std::mutex mu_;
  Slot slots_[kDevices][kSlots];
  uint64_t tick_ = 0;
};

AdamTableCache& adam_table_cache() {
  static AdamTableCache* c = new AdamTableCache();
  return *c;
}

// ---------------------------------------------------------------------------
// Broadcasting (TF BCast rules, right-aligned).
// ---------------------------------------------------------------------------
bool broadcast_shape(const TFMA_Tensor* a, const TFMA_Tensor* b, int* nd,
                     int64_t* dims) {
  const int n = std::max(a->ndims, b->ndims);
  for (int i = 0; i < n; ++i) {
    const int ia = a->ndims - n + i, ib = b->ndims - n + i;
    const int64_t da = ia >= 0 ? a->dims[ia] : 1;
    const int64_t db = ib >= 0 ? b->dims[ib] : 1;
    if (da == db || db == 1) {
      dims[i] = da;
    } else if (da == 1) {
      dims[i] = db;
    } else {
      return false;
    }
  }
  *nd = n;
  return true;
}

// Describes operand t broadcast to out (rank nd, dims od): returns false if
// it needs the general strided path.
bool classify(const TFMA_Tensor* t, int nd, const int64_t* od,
              BcastOperand* o) {
  o->data = t->data;
  // Output dims of size 1 are neutral.  The operand's non-broadcast
  // ("active") dims must form one run, with only broadcast dims outside it.
  int lo = -1, last = -1;
  bool gap = false, any_bcast = false;
  for (int d = 0; d < nd; ++d) {
    const int it = t->ndims - nd + d;
    const int64_t td = it >= 0 ? t->dims[it] : 1;
    if (od[d] == 1) continue;
    if (td == od[d]) {
      if (lo < 0) lo = d;
      else if (gap) return false;
      last = d;
    } else {
      any_bcast = true;
      if (lo >= 0) gap = true;
    }
  }
  o->inner = 1;
  o->period = 1;
  if (lo < 0) {
    o->mode = BcastMode::kScalar;
    return true;
  }
  if (!any_bcast) {
    o->mode = BcastMode::kFull;
    return true;
  }
  int64_t period = 1, inner = 1;
  for (int d = lo; d <= last; ++d) period *= od[d];
  for (int d = last + 1; d < nd; ++d) inner *= od[d];
  o->mode = BcastMode::kPeriodic;
  o->inner = inner;
  o->period = period;
  return true;
}

void strides_for(const TFMA_Tensor* t, int nd, const int64_t* od,
                 int64_t* st) {
  int64_t s = 1;
  for (int d = nd - 1; d >= 0; --d) {
    const int it = t->ndims - nd + d;
    const int64_t td = it >= 0 ? t->dims[it] : 1;
    st[d] = (td == od[d] && td != 1) ? s : 0;
    s *= td;
  }
}

// Runs op over up to three inputs broadcast to `out`.  `a_name` etc. are
// for messages; commutative says whether inputs 0 and 1 may be swapped.
int run_elementwise(void* stream, EwOp op, const char* op_name,
                    const TFMA_Tensor* const* ins, int n_in, TFMA_Tensor* out,
                    bool commutative01, TFMA_Status* st, IntTypes ints = IntTypes::kNone) {
  for (int i = 0; i < n_in; ++i)
    if (!valid_tensor(ins[i]))
      return set_status(st, TFMA_INVALID_ARGUMENT, "%s: invalid input %d", op_name, i);
  if (!valid_tensor(out))
    return set_status(st, TFMA_INVALID_ARGUMENT, "%s: invalid output", op_name);
  const int dt = ins[0]->dtype;
  DType t;
  if (!to_ew_dtype(dt, ints, &t))
    return set_status(st, TFMA_UNIMPLEMENTED, "%s: dtype %s is not supported",
                      op_name, dtype_name(dt));
  for (int i = 1; i < n_in; ++i)
    if (ins[i]->dtype != dt)
      return set_status(st, TFMA_INVALID_ARGUMENT,
                        "%s: input %d has dtype %s, expected %s", op_name, i,
                        dtype_name(ins[i]->dtype), dtype_name(dt));
  if (out->dtype != dt)
    return set_status(st, TFMA_INVALID_ARGUMENT, "%s: output dtype %s, expected %s",
                      op_name, dtype_name(out->dtype), dtype_name(dt));
  // Broadcast shape over all inputs.
  TFMA_Tensor acc = *ins[0];
  for (int i = 1; i < n_in; ++i) {
    TFMA_Tensor next = acc;
    if (!broadcast_shape(&acc, ins[i], &next.ndims, next.dims))
      return set_status(st, TFMA_INVALID_ARGUMENT, "Incompatible shapes for %s: %s and %s",
                        op_name, shape_str(&acc).c_str(), shape_str(ins[i]).c_str());
    acc = next;
  }
  if (!same_shape(&acc, out))
    return set_status(st, TFMA_INVALID_ARGUMENT,
                      "%s: output shape %s does not match broadcast shape %s",
                      op_name, shape_str(out).c_str(), shape_str(&acc).c_str());
  const int64_t n = num_elements(out);
  if (n == 0) return ok(st);
  for (int i = 0; i < n_in; ++i)
    if (!ins[i]->data) return set_status(st, TFMA_INVALID_ARGUMENT, "%s: null input %d", op_name, i);
  if (!out->data) return set_status(st, TFMA_INVALID_ARGUMENT, "%s: null output", op_name);

  const int nd = out->ndims;
  const TFMA_Tensor* ord[3] = {ins[0], n_in > 1 ? ins[1] : ins[0], n_in > 2 ? ins[2] : ins[0]};
  BcastOperand o[3];
  bool fast = true;
  for (int i = 0; i < n_in && fast; ++i) fast = classify(ord[i], nd, out->dims, &o[i]);
  if (fast && o[0].mode != BcastMode::kFull && commutative01 && n_in > 1 &&
      o[1].mode == BcastMode::kFull) {
    std::swap(ord[0], ord[1]);
    std::swap(o[0], o[1]);
  }
  if (fast && o[0].mode != BcastMode::kFull) fast = false;
  if (fast) {
    if (n_in < 2) o[1] = o[0];
    if (n_in < 3) o[2] = o[0];
    fast = ElementwiseFlatOk(n, o[0], o[1], o[2]);
  }
  hipError_t e;
  if (fast) {
    e = LaunchElementwise(t, op, n, o[0], o[1], o[2], out->data, as_stream(stream));
  } else {
    StridedShape sh{};
    sh.ndims = nd;
    for (int d = 0; d < nd; ++d) sh.dims[d] = out->dims[d];
    strides_for(ord[0], nd, out->dims, sh.stride_a);
    strides_for(ord[1], nd, out->dims, sh.stride_b);
    strides_for(ord[2], nd, out->dims, sh.stride_c);
    e = LaunchElementwiseStrided(t, op, n, ord[0]->data, ord[1]->data,
                                 ord[2]->data, sh, out->data, as_stream(stream));
  }
  return hip_status(st, e, op_name);
}

int bias_add_impl(void* stream, const TFMA_Tensor* value, const TFMA_Tensor* bias,
                  const char* data_format, TFMA_Tensor* output, bool relu,
                  TFMA_Status* st) {
  const char* name = relu ? "MusaBiasAddRelu" : "BiasAdd";
  if (!valid_tensor(value) || !valid_tensor(bias) || !valid_tensor(output))
    return set_status(st, TFMA_INVALID_ARGUMENT, "%s: invalid tensor", name);
  const std::string fmt = data_format ? data_format : "NHWC";
  if (fmt != "NHWC" && fmt != "NCHW")
    return set_status(st, TFMA_INVALID_ARGUMENT, "Invalid data format");
  if (value->ndims < 2)
    return set_status(st, TFMA_INVALID_ARGUMENT, "Input tensor must be at least 2D: %s",
                      shape_str(value).c_str());
  if (bias->ndims != 1)
    return set_status(st, TFMA_INVALID_ARGUMENT, "Biases must be 1D: %s",
                      shape_str(bias).c_str());
  DType t;
  if (!to_ew_dtype(value->dtype, relu ? IntTypes::kNone : IntTypes::kI32I64, &t))
    return set_status(st, TFMA_UNIMPLEMENTED, "%s: dtype %s is not supported", name,
                      dtype_name(value->dtype));
  if (bias->dtype != value->dtype || output->dtype != value->dtype)
    return set_status(st, TFMA_INVALID_ARGUMENT, "%s: bias/output dtype must match value", name);
  if (!same_shape(value, output))
    return set_status(st, TFMA_INVALID_ARGUMENT, "%s: output shape %s != input shape %s",
                      name, shape_str(output).c_str(), shape_str(value).c_str());
  const int channel_dim = fmt == "NCHW" ? 1 : value->ndims - 1;
  if (bias->dims[0] != value->dims[channel_dim])
    return set_status(st, TFMA_INVALID_ARGUMENT, "Dimension mismatch in BiasAdd");
  const int64_t n = num_elements(value);
  if (n == 0) return ok(st);
  int64_t inner = 1;
  for (int d = channel_dim + 1; d < value->ndims; ++d) inner *= value->dims[d];
  if (!value->data || !bias->data || !output->data)
    return set_status(st, TFMA_INVALID_ARGUMENT, "%s: null data pointer", name);
  hipError_t e;
  const BcastOperand a{value->data, BcastMode::kFull, 1, 1};
  const BcastOperand b{bias->data, BcastMode::kPeriodic, inner, bias->dims[0]};
  if (ElementwiseFlatOk(n, a, b, a)) {
    e = LaunchElementwise(t, relu ? EwOp::kAddRelu : EwOp::kAdd, n, a, b, a,
                          output->data, as_stream(stream));
  } else {
    StridedShape sh{};
    sh.ndims = value->ndims;
    int64_t s = 1;
    for (int d = value->ndims - 1; d >= 0; --d) {
      sh.dims[d] = value->dims[d];
      sh.stride_a[d] = s;
      sh.stride_b[d] = d == channel_dim ? 1 : 0;
      sh.stride_c[d] = 0;
      s *= value->dims[d];
    }
    e = LaunchElementwiseStrided(t, relu ? EwOp::kAddRelu : EwOp::kAdd, n,
                                 value->data, bias->data, value->data, sh,
                                 output->data, as_stream(stream));
  }
  return hip_status(st, e, name);
}

// ---------------------------------------------------------------------------
// Fused batch norm helpers.
// ---------------------------------------------------------------------------
bool parse_bn_format(const char* f, bool* nhwc) {
  const std::string s = f ? f : "NHWC";
  if (s == "NHWC" || s == "NDHWC") { *nhwc = true; return true; }
  if (s == "NCHW" || s == "NCDHW") { *nhwc = false; return true; }
  return false;
}

BnGeometry bn_geometry(const TFMA_Tensor* x, bool nhwc) {
  BnGeometry g;
  g.nhwc = nhwc;
  g.n = x->dims[0];
  if (nhwc) {
    g.c = x->dims[x->ndims - 1];
    g.h = 1;
    for (int d = 1; d < x->ndims - 1; ++d) g.h *= x->dims[d];
  } else {
    g.c = x->dims[1];
    g.h = 1;
    for (int d = 2; d < x->ndims; ++d) g.h *= x->dims[d];
  }
  g.w = 1;
  g.rows = g.n * g.h * g.w;
  return g;
}

bool is_vec_f32(const TFMA_Tensor* t) {
  return valid_tensor(t) && t->ndims == 1 && t->dtype == TFMA_FLOAT;
}

// An earlier fused BatchNorm launch on this device that gave up a
// grid-wide wait (its grid was not co-resident) wrote NaN statistics and
// outputs for the channels concerned; the next BatchNorm call reports it,
// once, as INTERNAL (the launch-failure code of the reference's ops,
// musa_applyadam_op.cc:258-261) instead of launching.
int check_bn_give_up(TFMA_Status* st) {
  unsigned epoch = 0;
  if (!BnPendingGiveUp(&epoch)) return TFMA_OK;
  int dev = -1;
  (void)hipGetDevice(&dev);
  return set_status(st, TFMA_INTERNAL,
                    "FusedBatchNorm: an earlier fused launch on device %d (epoch %u) gave up "
                    "waiting for another workgroup's values because its grid was not "
                    "co-resident (another persistent kernel held compute units); the "
                    "statistics and outputs of the channels concerned were written as NaN",
                    dev, epoch);
}

}  // namespace

int DeviceCUs() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lk(mu);
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

// Fill a float buffer on the stream (empty-input statistics).
hipError_t LaunchFillF32(float* p, int64_t n, float value, hipStream_t stream);

}  // namespace tfma

using namespace tfma;

// ===========================================================================
// Exported C ABI.
// ===========================================================================
extern "C" {

const char* TFMA_Version(void) { return "tfma 0.1 gfx950"; }

int TFMA_StreamCopy(void* stream, void* dst, const void* src, uint64_t bytes,
                    TFMA_Status* status) {
  if (bytes == 0) return ok(status);
  if (!dst || !src)
    return set_status(status, TFMA_INVALID_ARGUMENT, "StreamCopy: null pointer");
  if (bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(dst) & 15) != 0 ||
      (reinterpret_cast<uintptr_t>(src) & 15) != 0)
    return set_status(status, TFMA_INVALID_ARGUMENT,
                      "StreamCopy: bytes (%llu) and both pointers must be 16-byte multiples",
                      static_cast<unsigned long long>(bytes));
  return hip_status(status,
                    LaunchStreamCopy(dst, src, static_cast<int64_t>(bytes), as_stream(stream)),
                    "StreamCopy");
}

int TFMA_FusedBatchNormStamps(uint64_t* stamps, uint64_t count, TFMA_Status* status) {
  if (!stamps && count)
    return set_status(status, TFMA_INVALID_ARGUMENT, "FusedBatchNormStamps: null buffer");
  const hipError_t e = BnStamps(stamps, count * sizeof(uint64_t));
  if (e == hipErrorNotSupported)
    return set_status(status, TFMA_UNIMPLEMENTED,
                      "FusedBatchNormStamps: the library was built without TFMA_BN_STAMPS");
  return hip_status(status, e, "FusedBatchNormStamps");
}

int TFMA_SetTuningOverride(const char* name, int32_t value, TFMA_Status* status) {
  if (!name || !SetTune(name, value))
    return set_status(status, TFMA_INVALID_ARGUMENT, "SetTuningOverride: unknown name %s",
                      name ? name : "(null)");
  return ok(status);
}

int TFMA_GetDeviceCount(int* count, TFMA_Status* status) {
  if (!count) return set_status(status, TFMA_INVALID_ARGUMENT, "count is null");
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
  *count = n;
  return ok(status);
}

int TFMA_FusedBatchNormBarrierTimedOut(int32_t* timed_out, int32_t reset,
                                       TFMA_Status* status) {
  if (!timed_out) return set_status(status, TFMA_INVALID_ARGUMENT, "timed_out is null");
  bool t = false;
  const hipError_t e = BnBarrierTimedOut(reset != 0, &t);
  if (e != hipSuccess)
    return set_status(status, TFMA_INTERNAL, "FusedBatchNorm barrier flag: %s",
                      hipGetErrorString(e));
  *timed_out = t ? 1 : 0;
  return ok(status);
}

int TFMA_FusedBatchNormLastPlan(TFMA_FusedBatchNormPlan* plan, TFMA_Status* status) {
  if (!plan) return set_status(status, TFMA_INVALID_ARGUMENT, "plan is null");
  *plan = BnLastPlan();
  return ok(status);
}

int TFMA_FusedBatchNormWorkspaceBytes(const TFMA_Tensor* x, const char* data_format,
                                      size_t* bytes, TFMA_Status* status) {
  if (!bytes || !valid_tensor(x))
    return set_status(status, TFMA_INVALID_ARGUMENT, "invalid arguments");
  bool nhwc;
  if (!parse_bn_format(data_format, &nhwc))
    return set_status(status, TFMA_INVALID_ARGUMENT, "Invalid data format");
  if (x->ndims != 4 && x->ndims != 5)
    return set_status(status, TFMA_INVALID_ARGUMENT, "input must be 4 or 5-dimensional%s",
                      shape_str(x).c_str());
  DType t;
  if (!to_dtype(x->dtype, &t) || t == DType::kF64)
    return set_status(status, TFMA_UNIMPLEMENTED, "FusedBatchNorm: dtype %s is not supported",
                      dtype_name(x->dtype));
  const BnGeometry g = bn_geometry(x, nhwc);
  *bytes = g.c > 0 ? BnWorkspaceBytes(t, g) : 0;
  return ok(status);
}

int TFMA_FusedBatchNormV3(void* stream, const TFMA_Tensor* x, const TFMA_Tensor* scale,
                          const TFMA_Tensor* offset, const TFMA_Tensor* mean,
                          const TFMA_Tensor* variance, float epsilon,
                          float exponential_avg_factor, const char* data_format,
                          int is_training, TFMA_Tensor* y, TFMA_Tensor* batch_mean,
                          TFMA_Tensor* batch_variance, TFMA_Tensor* reserve_space_1,
                          TFMA_Tensor* reserve_space_2, TFMA_Tensor* reserve_space_3,
                          void* workspace, size_t workspace_bytes, TFMA_Status* status) {
  bool nhwc;
  if (!parse_bn_format(data_format, &nhwc))
    return set_status(status, TFMA_INVALID_ARGUMENT, "Invalid data format");
  if (!valid_tensor(x) || !valid_tensor(scale) || !valid_tensor(offset) || !valid_tensor(y))
    return set_status(status, TFMA_INVALID_ARGUMENT, "FusedBatchNormV3: invalid tensor");
  if (x->ndims != 4 && x->ndims != 5)
    return set_status(status, TFMA_INVALID_ARGUMENT, "input must be 4 or 5-dimensional%s",
                      shape_str(x).c_str());
  if (scale->ndims != 1)
    return set_status(status, TFMA_INVALID_ARGUMENT, "scale must be 1-dimensional%s",
                      shape_str(scale).c_str());
  if (offset->ndims != 1)
    return set_status(status, TFMA_INVALID_ARGUMENT, "offset must be 1-dimensional%s",
                      shape_str(offset).c_str());
  DType t;
  if (!to_dtype(x->dtype, &t) || t == DType::kF64)
    return set_status(status, TFMA_UNIMPLEMENTED, "FusedBatchNormV3: dtype %s is not supported",
                      dtype_name(x->dtype));
  if (y->dtype != x->dtype || !same_shape(x, y))
    return set_status(status, TFMA_INVALID_ARGUMENT, "FusedBatchNormV3: y must match x (%s %s)",
                      dtype_name(x->dtype), shape_str(x).c_str());
  if (scale->dtype != TFMA_FLOAT || offset->dtype != TFMA_FLOAT)
    return set_status(status, TFMA_INVALID_ARGUMENT, "FusedBatchNormV3: scale/offset must be float");
  const BnGeometry g = bn_geometry(x, nhwc);
  const int64_t c = g.c;
  if (num_elements(scale) != c)
    return set_status(status, TFMA_INVALID_ARGUMENT,
                      "scale must have the same number of elements as the channels of x, got %lld and %lld",
                      (long long)num_elements(scale), (long long)c);
  if (num_elements(offset) != c)
    return set_status(status, TFMA_INVALID_ARGUMENT,
                      "offset must have the same number of elements as the channels of x, got %lld and %lld",
                      (long long)num_elements(offset), (long long)c);
  const bool need_running = !is_training || exponential_avg_factor != 1.0f;
  if (need_running) {
    const char* prefix = is_training ? "When exponential_avg_factor != 1" : "When is_training=false";
    if (!valid_tensor(mean) || num_elements(mean) != c || mean->dtype != TFMA_FLOAT)
      return set_status(status, TFMA_INVALID_ARGUMENT,
                        "%s, mean must have the same number of elements as the channels of x, got %lld and %lld",
                        prefix, (long long)(valid_tensor(mean) ? num_elements(mean) : 0), (long long)c);
    if (!valid_tensor(variance) || num_elements(variance) != c || variance->dtype != TFMA_FLOAT)
      return set_status(status, TFMA_INVALID_ARGUMENT,
                        "%s, variance must have the same number of elements as the channels of x, got %lld and %lld",
                        prefix, (long long)(valid_tensor(variance) ? num_elements(variance) : 0), (long long)c);
  }
  TFMA_Tensor* stats[4] = {batch_mean, batch_variance, reserve_space_1, reserve_space_2};
  const char* stat_names[4] = {"batch_mean", "batch_variance", "reserve_space_1", "reserve_space_2"};
  for (int i = 0; i < 4; ++i)
    if (!is_vec_f32(stats[i]) || num_elements(stats[i]) != c)
      return set_status(status, TFMA_INVALID_ARGUMENT, "%s must be a float vector of length %lld",
                        stat_names[i], (long long)c);
  if (reserve_space_3 && (!valid_tensor(reserve_space_3) || reserve_space_3->ndims != 0 ||
                          reserve_space_3->dtype != TFMA_FLOAT))
    return set_status(status, TFMA_INVALID_ARGUMENT, "reserve_space_3 must be a float scalar");
  float* r3 = reserve_space_3 ? static_cast<float*>(reserve_space_3->data) : nullptr;
  hipStream_t s = as_stream(stream);
  if (c == 0) return ok(status);
  if (num_elements(x) == 0) {
    // Empty batch: statistics are NaN (TF's SetNanFunctor), saved stats 0.
    const float nan = bits_f32(0x7fc00000u);
    hipError_t e = LaunchFillF32(static_cast<float*>(batch_mean->data), c, nan, s);
    if (e == hipSuccess) e = LaunchFillF32(static_cast<float*>(batch_variance->data), c, nan, s);
    if (e == hipSuccess) e = LaunchFillF32(static_cast<float*>(reserve_space_1->data), c, 0.f, s);
    if (e == hipSuccess) e = LaunchFillF32(static_cast<float*>(reserve_space_2->data), c, 0.f, s);
    if (e == hipSuccess && r3) e = LaunchFillF32(r3, 1, 0.f, s);
    return hip_status(status, e, "FusedBatchNormV3");
  }
  if (!x->data || !y->data || !scale->data || !offset->data)
    return set_status(status, TFMA_INVALID_ARGUMENT, "FusedBatchNormV3: null data pointer");
  const size_t need = BnWorkspaceBytes(t, g);
  if (!workspace || workspace_bytes < need)
    return set_status(status, TFMA_INVALID_ARGUMENT,
                      "FusedBatchNormV3: workspace of %zu bytes required, got %zu", need,
                      workspace ? workspace_bytes : size_t(0));
  BnFwdArgs a{};
  a.x = x->data;
  a.scale = static_cast<const float*>(scale->data);
  a.offset = static_cast<const float*>(offset->data);
  a.mean_in = need_running ? static_cast<const float*>(mean->data) : nullptr;
  a.var_in = need_running ? static_cast<const float*>(variance->data) : nullptr;
  a.epsilon = epsilon;
  a.exp_avg_factor = exponential_avg_factor;
  a.is_training = is_training != 0;
  a.y = y->data;
  a.batch_mean = static_cast<float*>(batch_mean->data);
  a.batch_var = static_cast<float*>(batch_variance->data);
  a.saved_mean = static_cast<float*>(reserve_space_1->data);
  a.saved_var = static_cast<float*>(reserve_space_2->data);
  a.reserve3 = r3;
  if (const int rc = check_bn_give_up(status)) return rc;
  return hip_status(status, LaunchBnForward(t, g, a, workspace, workspace_bytes, s),
                    "FusedBatchNormV3");
}

int TFMA_FusedBatchNormGradV3(void* stream, const TFMA_Tensor* y_backprop, const TFMA_Tensor* x,
                              const TFMA_Tensor* scale, const TFMA_Tensor* reserve_space_1,
                              const TFMA_Tensor* reserve_space_2,
                              const TFMA_Tensor* reserve_space_3, float epsilon,
                              const char* data_format, int is_training, TFMA_Tensor* x_backprop,
                              TFMA_Tensor* scale_backprop, TFMA_Tensor* offset_backprop,
                              TFMA_Tensor* reserve_space_4, TFMA_Tensor* reserve_space_5,
                              void* workspace, size_t workspace_bytes, TFMA_Status* status) {
  (void)reserve_space_3;
  bool nhwc;
  if (!parse_bn_format(data_format, &nhwc))
    return set_status(status, TFMA_INVALID_ARGUMENT, "Invalid data format");
  if (!valid_tensor(y_backprop) || !valid_tensor(x) || !valid_tensor(scale) ||
      !valid_tensor(reserve_space_1) || !valid_tensor(reserve_space_2) ||
      !valid_tensor(x_backprop))
    return set_status(status, TFMA_INVALID_ARGUMENT, "FusedBatchNormGradV3: invalid tensor");
  if (y_backprop->ndims != 4 && y_backprop->ndims != 5)
    return set_status(status, TFMA_INVALID_ARGUMENT, "input must be 4 or 5-dimensional%s",
                      shape_str(y_backprop).c_str());
  if (x->ndims != 4 && x->ndims != 5)
    return set_status(status, TFMA_INVALID_ARGUMENT, "input must be 4 or 5-dimensional%s",
                      shape_str(x).c_str());
  if (scale->ndims != 1)
    return set_status(status, TFMA_INVALID_ARGUMENT, "scale must be 1-dimensional%s",
                      shape_str(scale).c_str());
  if (reserve_space_1->ndims != 1)
    return set_status(status, TFMA_INVALID_ARGUMENT, "saved mean must be 1-dimensional%s",
                      shape_str(reserve_space_1).c_str());
  if (reserve_space_2->ndims != 1)
    return set_status(status, TFMA_INVALID_ARGUMENT, "saved variance must be 1-dimensional%s",
                      shape_str(reserve_space_2).c_str());
  if (!same_shape(x, y_backprop))
    return set_status(status, TFMA_INVALID_ARGUMENT,
                      "x and y_backprop must have same shape, but x has shape %s and y_backprop has shape %s",
                      shape_str(x).c_str(), shape_str(y_backprop).c_str());
  DType t;
  if (!to_dtype(x->dtype, &t) || t == DType::kF64)
    return set_status(status, TFMA_UNIMPLEMENTED, "FusedBatchNormGradV3: dtype %s is not supported",
                      dtype_name(x->dtype));
  if (y_backprop->dtype != x->dtype || x_backprop->dtype != x->dtype || !same_shape(x, x_backprop))
    return set_status(status, TFMA_INVALID_ARGUMENT,
                      "FusedBatchNormGradV3: y_backprop and x_backprop must match x");
  if (scale->dtype != TFMA_FLOAT || reserve_space_1->dtype != TFMA_FLOAT ||
      reserve_space_2->dtype != TFMA_FLOAT)
    return set_status(status, TFMA_INVALID_ARGUMENT,
                      "FusedBatchNormGradV3: scale and reserve spaces must be float");
  const BnGeometry g = bn_geometry(x, nhwc);
  const int64_t c = g.c;
  if (num_elements(scale) != c)
    return set_status(status, TFMA_INVALID_ARGUMENT,
                      "scale must have the same number of elements as the channels of x, got %lld and %lld",
                      (long long)num_elements(scale), (long long)c);
  if (num_elements(reserve_space_1) != c)
    return set_status(status, TFMA_INVALID_ARGUMENT,
                      "reserve_space_1 must have the same number of elements as the channels of x, got %lld and %lld",
                      (long long)num_elements(reserve_space_1), (long long)c);
  if (num_elements(reserve_space_2) != c)
    return set_status(status, TFMA_INVALID_ARGUMENT,
                      "reserve_space_2 must have the same number of elements as the channels of x, got %lld and %lld",
                      (long long)num_elements(reserve_space_2), (long long)c);
  if (!is_vec_f32(scale_backprop) || num_elements(scale_backprop) != c ||
      !is_vec_f32(offset_backprop) || num_elements(offset_backprop) != c)
    return set_status(status, TFMA_INVALID_ARGUMENT,
                      "scale_backprop/offset_backprop must be float vectors of length %lld", (long long)c);
  for (TFMA_Tensor* r : {reserve_space_4, reserve_space_5})
    if (r && (!valid_tensor(r) || r->dtype != TFMA_FLOAT))
      return set_status(status, TFMA_INVALID_ARGUMENT, "reserve_space_4/5 must be float");
  hipStream_t s = as_stream(stream);
  float* r4 = reserve_space_4 ? static_cast<float*>(reserve_space_4->data) : nullptr;
  float* r5 = reserve_space_5 ? static_cast<float*>(reserve_space_5->data) : nullptr;
  const int64_t n4 = reserve_space_4 ? num_elements(reserve_space_4) : 0;
  const int64_t n5 = reserve_space_5 ? num_elements(reserve_space_5) : 0;
  if (c == 0) return ok(status);
  if (num_elements(x) == 0) {
    hipError_t e = LaunchFillF32(static_cast<float*>(scale_backprop->data), c, 0.f, s);
    if (e == hipSuccess) e = LaunchFillF32(static_cast<float*>(offset_backprop->data), c, 0.f, s);
    if (e == hipSuccess && n4) e = LaunchFillF32(r4, n4, 0.f, s);
    if (e == hipSuccess && n5) e = LaunchFillF32(r5, n5, 0.f, s);
    return hip_status(status, e, "FusedBatchNormGradV3");
  }
  if (!x->data || !y_backprop->data || !x_backprop->data || !scale->data ||
      !reserve_space_1->data || !reserve_space_2->data)
    return set_status(status, TFMA_INVALID_ARGUMENT, "FusedBatchNormGradV3: null data pointer");
  const size_t need = BnWorkspaceBytes(t, g);
  if (!workspace || workspace_bytes < need)
    return set_status(status, TFMA_INVALID_ARGUMENT,
                      "FusedBatchNormGradV3: workspace of %zu bytes required, got %zu", need,
                      workspace ? workspace_bytes : size_t(0));
  BnGradArgs a{};
  a.dy = y_backprop->data;
  a.x = x->data;
  a.scale = static_cast<const float*>(scale->data);
  a.saved_mean = static_cast<const float*>(reserve_space_1->data);
  a.saved_var = static_cast<const float*>(reserve_space_2->data);
  a.epsilon = epsilon;
  a.is_training = is_training != 0;
  a.dx = x_backprop->data;
  a.scale_backprop = static_cast<float*>(scale_backprop->data);
  a.offset_backprop = static_cast<float*>(offset_backprop->data);
  a.reserve4 = r4;
  a.reserve4_n = n4;
  a.reserve5 = r5;
  a.reserve5_n = n5;
  if (const int rc = check_bn_give_up(status)) return rc;
  return hip_status(status, LaunchBnGrad(t, g, a, workspace, workspace_bytes, s),
                    "FusedBatchNormGradV3");
}

// ---------------------------------------------------------------------------
// Adam
// ---------------------------------------------------------------------------
namespace {

int check_adam_scalars(const TFMA_Tensor* const* sc, int dt, AdamScalars* out, DType t,
                       TFMA_Status* st) {
  static const char* names[6] = {"beta1_power", "beta2_power", "lr", "beta1", "beta2", "epsilon"};
  double v[6];
  for (int i = 0; i < 6; ++i) {
    if (!valid_tensor(sc[i]) || !sc[i]->data)
      return set_status(st, TFMA_INVALID_ARGUMENT, "%s is missing", names[i]);
    if (sc[i]->ndims != 0)
      return set_status(st, TFMA_INVALID_ARGUMENT, "%s is not a scalar: %s", names[i],
                        shape_str(sc[i]).c_str());
    if (sc[i]->dtype != dt)
      return set_status(st, TFMA_INVALID_ARGUMENT, "%s has dtype %s, expected %s", names[i],
                        dtype_name(sc[i]->dtype), dtype_name(dt));
    v[i] = read_scalar(sc[i], t);
  }
  *out = adam_scalars(t, v[0], v[1], v[2], v[3], v[4], v[5]);
  return TFMA_OK;
}

// mixed = false: var, m, v and grad share one dtype (ResourceApplyAdam).
// mixed = true: fp32 var/m/v with a float, half or bfloat16 grad
// (MusaResourceApplyAdamMixed, musa_applyadam_mixed_op.cc:160-183).
// *dt / *gdt receive the state and gradient dtypes.
int check_adam_triple(const TFMA_Tensor* var, const TFMA_Tensor* m, const TFMA_Tensor* v,
                      const TFMA_Tensor* grad, bool mixed, int* dt, int* gdt,
                      TFMA_Status* st) {
  if (!valid_tensor(var) || !valid_tensor(m) || !valid_tensor(v) || !valid_tensor(grad))
    return set_status(st, TFMA_INVALID_ARGUMENT, "ResourceApplyAdam: invalid tensor");
  if ((!var->data && num_elements(var) > 0) || (!m->data && num_elements(m) > 0) ||
      (!v->data && num_elements(v) > 0))
    return set_status(st, TFMA_FAILED_PRECONDITION,
                      mixed ? "Mixed-precision Adam variables (var/m/v) not initialized."
                            : "Adam variables (var/m/v) not initialized.");
  if (mixed) {
    const TFMA_Tensor* state[3] = {var, m, v};
    static const char* names[3] = {"var", "m", "v"};
    for (int i = 0; i < 3; ++i)
      if (state[i]->dtype != TFMA_FLOAT)
        return set_status(st, TFMA_INVALID_ARGUMENT,
                          "MusaResourceApplyAdamMixed requires fp32 %s, got %s", names[i],
                          dtype_name(state[i]->dtype));
  }
  if (!same_shape(var, m))
    return set_status(st, TFMA_INVALID_ARGUMENT, "var and m must have the same shape. var: %s m: %s",
                      shape_str(var).c_str(), shape_str(m).c_str());
  if (!same_shape(var, v))
    return set_status(st, TFMA_INVALID_ARGUMENT, "var and v must have the same shape. var: %s v: %s",
                      shape_str(var).c_str(), shape_str(v).c_str());
  if (!same_shape(var, grad))
    return set_status(st, TFMA_INVALID_ARGUMENT,
                      "var and grad must have the same shape. var: %s grad: %s",
                      shape_str(var).c_str(), shape_str(grad).c_str());
  if (mixed) {
    if (grad->dtype != TFMA_FLOAT && grad->dtype != TFMA_HALF && grad->dtype != TFMA_BFLOAT16)
      return set_status(st, TFMA_INVALID_ARGUMENT,
                        "MusaResourceApplyAdamMixed: grad dtype %s is not float, half or bfloat16",
                        dtype_name(grad->dtype));
  } else if (m->dtype != var->dtype || v->dtype != var->dtype || grad->dtype != var->dtype) {
    return set_status(st, TFMA_INVALID_ARGUMENT,
                      "ResourceApplyAdam: var, m, v and grad must have the same dtype");
  }
  if (!grad->data && num_elements(grad) > 0)
    return set_status(st, TFMA_INVALID_ARGUMENT, "ResourceApplyAdam: grad data is null");
  *dt = var->dtype;
  *gdt = grad->dtype;
  return TFMA_OK;
}

// The double -> T conversion of the reference's static_cast<T>(alpha_val)
// as its x86-64 host performs it: truncation toward zero, and the "integer
// indefinite" value (T's minimum) for NaN or a value outside T's range.
int64_t host_double_to_int(double d, bool is64) {
  const double lim = is64 ? 9223372036854775808.0 : 2147483648.0;
  const int64_t minv = is64 ? INT64_MIN : INT32_MIN;
  if (!(d > -lim - 1.0 && d < lim)) return minv;
  const double t = std::trunc(d);
  if (t < -lim || t >= lim) return minv;
  return static_cast<int64_t>(t);
}

int64_t wrap_to(int64_t x, bool is64) {
  return is64 ? x : static_cast<int64_t>(static_cast<int32_t>(static_cast<uint32_t>(x)));
}

// int32 / int64 ResourceApplyAdam, registered by the reference
// (musa_applyadam_op.cc:645-682) and run there through its generic op chain:
// alpha in double from the scalars, with lr when beta1_power is within 1e-10
// of 1 (:231-246), converted to T; 1 - beta in T (:310-316).
int apply_adam_int(void* stream, TFMA_Tensor* var, TFMA_Tensor* m, TFMA_Tensor* v,
                   const TFMA_Tensor* const* sc, const TFMA_Tensor* grad, int dt,
                   int use_locking, TFMA_Status* status) {
  static const char* names[6] = {"beta1_power", "beta2_power", "lr", "beta1", "beta2", "epsilon"};
  const bool is64 = dt == TFMA_INT64;
  int64_t val[6];
  for (int i = 0; i < 6; ++i) {
    if (!valid_tensor(sc[i]) || !sc[i]->data)
      return set_status(status, TFMA_INVALID_ARGUMENT, "%s is missing", names[i]);
    if (sc[i]->ndims != 0)
      return set_status(status, TFMA_INVALID_ARGUMENT, "%s is not a scalar: %s", names[i],
                        shape_str(sc[i]).c_str());
    if (sc[i]->dtype != dt)
      return set_status(status, TFMA_INVALID_ARGUMENT, "%s has dtype %s, expected %s", names[i],
                        dtype_name(sc[i]->dtype), dtype_name(dt));
    val[i] = is64 ? *static_cast<const int64_t*>(sc[i]->data)
                  : static_cast<int64_t>(*static_cast<const int32_t*>(sc[i]->data));
  }
  const double b1p = static_cast<double>(val[0]), b2p = static_cast<double>(val[1]);
  const double lr = static_cast<double>(val[2]);
  const double omb1p = 1.0 - b1p;
  const double alpha = std::abs(omb1p) < 1e-10 ? lr : lr * std::sqrt(1.0 - b2p) / omb1p;
  IntAdamScalars s;
  s.alpha = host_double_to_int(alpha, is64);
  s.beta1 = val[3];
  s.beta2 = val[4];
  s.eps = val[5];
  s.omb1 = wrap_to(static_cast<int64_t>(1ull - static_cast<uint64_t>(val[3])), is64);
  s.omb2 = wrap_to(static_cast<int64_t>(1ull - static_cast<uint64_t>(val[4])), is64);
  VarLocks locks;
  if (use_locking) {
    locks.add(var->data);
    locks.add(m->data);
    locks.add(v->data);
    locks.lock();
  }
  const int64_t n = num_elements(var);
  if (n == 0) return ok(status);
  return hip_status(status,
                    LaunchApplyAdamInt(is64, var->data, m->data, v->data, grad->data, n, s,
                                       as_stream(stream)),
                    "ResourceApplyAdam");
}

int apply_adam(void* stream, TFMA_Tensor* var, TFMA_Tensor* m, TFMA_Tensor* v,
               const TFMA_Tensor* const* sc, const TFMA_Tensor* grad, int use_locking,
               int use_nesterov, bool mixed, const char* op, TFMA_Status* status) {
  int dt = 0, gdt = 0;
  if (const int rc = check_adam_triple(var, m, v, grad, mixed, &dt, &gdt, status)) return rc;
  if (!mixed && (dt == TFMA_INT32 || dt == TFMA_INT64))
    return apply_adam_int(stream, var, m, v, sc, grad, dt, use_locking, status);
  DType t, tg;
  if (!to_dtype(dt, &t) || !to_dtype(gdt, &tg))
    return set_status(status, TFMA_UNIMPLEMENTED, "%s: dtype %s is not supported", op,
                      dtype_name(dt));
  AdamScalars s;
  if (const int rc = check_adam_scalars(sc, dt, &s, t, status)) return rc;
  VarLocks locks;
  if (use_locking) {
    locks.add(var->data);
    locks.add(m->data);
    locks.add(v->data);
    locks.lock();
  }
  const int64_t n = num_elements(var);
  if (n == 0) return ok(status);
  return hip_status(status,
                    LaunchApplyAdam(t, tg, var->data, m->data, v->data, grad->data, n, s,
                                    use_nesterov != 0, as_stream(stream)),
                    op);
}

}  // namespace

int TFMA_ResourceApplyAdam(void* stream, TFMA_Tensor* var, TFMA_Tensor* m, TFMA_Tensor* v,
                           const TFMA_Tensor* beta1_power, const TFMA_Tensor* beta2_power,
                           const TFMA_Tensor* lr, const TFMA_Tensor* beta1,
                           const TFMA_Tensor* beta2, const TFMA_Tensor* epsilon,
                           const TFMA_Tensor* grad, int use_locking, int use_nesterov,
                           TFMA_Status* status) {
  const TFMA_Tensor* sc[6] = {beta1_power, beta2_power, lr, beta1, beta2, epsilon};
  return apply_adam(stream, var, m, v, sc, grad, use_locking, use_nesterov, false,
                    "ResourceApplyAdam", status);
}

int TFMA_MusaResourceApplyAdamMixed(void* stream, TFMA_Tensor* var, TFMA_Tensor* m,
                                    TFMA_Tensor* v, const TFMA_Tensor* beta1_power,
                                    const TFMA_Tensor* beta2_power, const TFMA_Tensor* lr,
                                    const TFMA_Tensor* beta1, const TFMA_Tensor* beta2,
                                    const TFMA_Tensor* epsilon, const TFMA_Tensor* grad,
                                    int use_locking, int use_nesterov, TFMA_Status* status) {
  const TFMA_Tensor* sc[6] = {beta1_power, beta2_power, lr, beta1, beta2, epsilon};
  return apply_adam(stream, var, m, v, sc, grad, use_locking, use_nesterov, true,
                    "MusaResourceApplyAdamMixed", status);
}

namespace {
// Table blob of the grouped update: the tensor entries, then one uint32
// tensor index per chunk (so a workgroup finds its tensor with one load).
size_t grouped_table_bytes(int entries, int64_t chunks) {
  return static_cast<size_t>(entries) * sizeof(AdamTensorEntry) +
         static_cast<size_t>(chunks) * sizeof(uint32_t);
}
}  // namespace

int TFMA_GroupedApplyAdamWorkspaceBytes(int n, const TFMA_Tensor* vars, size_t* bytes,
                                        TFMA_Status* status) {
  if (n < 1 || !bytes || !vars)
    return set_status(status, TFMA_INVALID_ARGUMENT, "N must be >= 1");
  int64_t chunks = 0;
  for (int i = 0; i < n; ++i) {
    if (!valid_tensor(&vars[i]))
      return set_status(status, TFMA_INVALID_ARGUMENT, "tensor %d: invalid tensor", i);
    chunks += (num_elements(&vars[i]) + kGroupedAdamChunk - 1) / kGroupedAdamChunk;
  }
  *bytes = (grouped_table_bytes(n, chunks) + 255) & ~size_t(255);
  return ok(status);
}

int TFMA_GroupedResourceApplyAdam(void* stream, int n, TFMA_Tensor* vars, TFMA_Tensor* ms,
                                  TFMA_Tensor* vs, const TFMA_Tensor* grads,
                                  const TFMA_Tensor* beta1_power, const TFMA_Tensor* beta2_power,
                                  const TFMA_Tensor* lr, const TFMA_Tensor* beta1,
                                  const TFMA_Tensor* beta2, const TFMA_Tensor* epsilon,
                                  int use_locking, int use_nesterov, void* workspace,
                                  size_t workspace_bytes, TFMA_Status* status) {
  if (n < 1 || !vars || !ms || !vs || !grads)
    return set_status(status, TFMA_INVALID_ARGUMENT, "N must be >= 1");
  // The gradients may be half or bfloat16 under fp32 state (the attr Tgrad
  // of the grouped op, after MusaGroupedResourceApplyGradientDescentMixed's
  // T/Tgrad pair, musa_applygradientdescent_op.cc:305-314).
  const bool mixed = valid_tensor(&vars[0]) && valid_tensor(&grads[0]) &&
                     vars[0].dtype == TFMA_FLOAT && grads[0].dtype != TFMA_FLOAT;
  int dt0 = 0, gdt0 = 0;
  std::vector<AdamTensorEntry> table;
  table.reserve(n);
  int64_t chunks = 0;
  for (int i = 0; i < n; ++i) {
    int dt = 0, gdt = 0;
    TFMA_Status inner;
    if (const int rc = check_adam_triple(&vars[i], &ms[i], &vs[i], &grads[i], mixed, &dt, &gdt,
                                         &inner))
      return set_status(status, rc, "tensor %d: %s", i, inner.message);
    if (i == 0) {
      dt0 = dt;
      gdt0 = gdt;
    }
    if (dt != dt0)
      return set_status(status, TFMA_INVALID_ARGUMENT,
                        "tensor %d has dtype %s, expected %s", i, dtype_name(dt), dtype_name(dt0));
    if (gdt != gdt0)
      return set_status(status, TFMA_INVALID_ARGUMENT,
                        "tensor %d has grad dtype %s, expected %s", i, dtype_name(gdt),
                        dtype_name(gdt0));
    const int64_t ne = num_elements(&vars[i]);
    if (ne == 0) continue;
    AdamTensorEntry e;
    e.var = vars[i].data;
    e.m = ms[i].data;
    e.v = vs[i].data;
    e.grad = grads[i].data;
    e.n = ne;
    e.first_chunk = chunks;
    chunks += (ne + kGroupedAdamChunk - 1) / kGroupedAdamChunk;
    table.push_back(e);
  }
  DType t, tg;
  if (!to_dtype(dt0, &t) || !to_dtype(gdt0, &tg))
    return set_status(status, TFMA_UNIMPLEMENTED,
                      "MusaGroupedResourceApplyAdam: dtype %s is not supported", dtype_name(dt0));
  const TFMA_Tensor* sc[6] = {beta1_power, beta2_power, lr, beta1, beta2, epsilon};
  AdamScalars s;
  if (const int rc = check_adam_scalars(sc, dt0, &s, t, status)) return rc;
  size_t need = 0;
  TFMA_GroupedApplyAdamWorkspaceBytes(n, vars, &need, nullptr);
  if (!workspace || workspace_bytes < need)
    return set_status(status, TFMA_INVALID_ARGUMENT,
                      "MusaGroupedResourceApplyAdam: workspace of %zu bytes required, got %zu",
                      need, workspace ? workspace_bytes : size_t(0));
  // Recorded into a graph, the table travels in the kernel arguments: the
  // staged device table (a pinned ring slot or a cached copy, both reused by
  // later calls) could have changed by the time a replay reads it.
  bool recorded = false;
  {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    const hipError_t ce = hipStreamIsCapturing(as_stream(stream), &cap);
    if (ce != hipSuccess) return hip_status(status, ce, "MusaGroupedResourceApplyAdam");
    recorded = cap != hipStreamCaptureStatusNone;
  }
  VarLocks locks;
  if (use_locking) {
    for (int i = 0; i < n; ++i) {
      locks.add(vars[i].data);
      locks.add(ms[i].data);
      locks.add(vs[i].data);
    }
    locks.lock();
  }
  if (table.empty()) return ok(status);
  if (recorded)
    return hip_status(status,
                      LaunchGroupedApplyAdamArgs(t, tg, table.data(), static_cast<int>(table.size()),
                                                 s, use_nesterov != 0, as_stream(stream)),
                      "MusaGroupedResourceApplyAdam");
  // Blob: entries, then the tensor index of every chunk.
  std::vector<uint8_t> blob(grouped_table_bytes(static_cast<int>(table.size()), chunks));
  memcpy(blob.data(), table.data(), table.size() * sizeof(AdamTensorEntry));
  uint32_t* cmap = reinterpret_cast<uint32_t*>(blob.data() + table.size() * sizeof(AdamTensorEntry));
  for (size_t i = 0; i < table.size(); ++i) {
    const int64_t end = i + 1 < table.size() ? table[i + 1].first_chunk : chunks;
    for (int64_t c = table[i].first_chunk; c < end; ++c) cmap[c] = static_cast<uint32_t>(i);
  }
  hipStream_t strm = as_stream(stream);
  int dev = -1;
  (void)hipGetDevice(&dev);
  int slot = -1;
  AdamTableCache& cache = adam_table_cache();
  if (const void* cached = cache.find(dev, blob, strm, &slot)) {
    hipError_t e = LaunchGroupedApplyAdam(t, tg, static_cast<const AdamTensorEntry*>(cached),
                                          static_cast<int>(table.size()), chunks, s,
                                          use_nesterov != 0, strm);
    cache.mark_used(dev, slot, strm);
    return hip_status(status, e, "MusaGroupedResourceApplyAdam");
  }
  PinnedRing* ring = pinned_ring(dev);
  if (!ring)
    return set_status(status, TFMA_INTERNAL, "MusaGroupedResourceApplyAdam: no current device");
  hipError_t e = ring->upload(workspace, blob.data(), blob.size(), strm);
  if (e != hipSuccess) return hip_status(status, e, "MusaGroupedResourceApplyAdam table upload");
  e = LaunchGroupedApplyAdam(t, tg, static_cast<const AdamTensorEntry*>(workspace),
                             static_cast<int>(table.size()), chunks, s, use_nesterov != 0,
                             strm);
  if (e == hipSuccess) cache.fill(dev, blob, workspace, strm);
  return hip_status(status, e, "MusaGroupedResourceApplyAdam");
}

// ---------------------------------------------------------------------------
// Elementwise
// ---------------------------------------------------------------------------
int TFMA_BiasAdd(void* stream, const TFMA_Tensor* value, const TFMA_Tensor* bias,
                 const char* data_format, TFMA_Tensor* output, TFMA_Status* status) {
  return bias_add_impl(stream, value, bias, data_format, output, false, status);
}

int TFMA_MusaBiasAddRelu(void* stream, const TFMA_Tensor* value, const TFMA_Tensor* bias,
                         const char* data_format, TFMA_Tensor* output, TFMA_Status* status) {
  return bias_add_impl(stream, value, bias, data_format, output, true, status);
}

int TFMA_Relu(void* stream, const TFMA_Tensor* features, TFMA_Tensor* activations,
              TFMA_Status* status) {
  const TFMA_Tensor* ins[1] = {features};
  return run_elementwise(stream, EwOp::kRelu, "Relu", ins, 1, activations, false, status);
}

int TFMA_ReluGrad(void* stream, const TFMA_Tensor* gradients, const TFMA_Tensor* features,
                  TFMA_Tensor* backprops, TFMA_Status* status) {
  if (!valid_tensor(gradients) || !valid_tensor(features))
    return set_status(status, TFMA_INVALID_ARGUMENT, "ReluGrad: invalid tensor");
  if (!same_shape(gradients, features))
    return set_status(status, TFMA_INVALID_ARGUMENT,
                      "Inputs to ReluGrad must have the same shape. gradients: %s, features: %s",
                      shape_str(gradients).c_str(), shape_str(features).c_str());
  const TFMA_Tensor* ins[2] = {gradients, features};
  return run_elementwise(stream, EwOp::kReluGrad, "ReluGrad", ins, 2, backprops, false, status);
}

namespace {

// BiasAddGrad geometry: [outer, C, inner] around the channel dimension.
int bias_grad_geometry(const TFMA_Tensor* x, const char* data_format, const TFMA_Tensor* out,
                       int64_t* outer, int64_t* c, int64_t* inner, TFMA_Status* st) {
  if (!valid_tensor(x) || (out && !valid_tensor(out)))
    return set_status(st, TFMA_INVALID_ARGUMENT, "BiasAddGrad: invalid tensor");
  const std::string fmt = data_format ? data_format : "NHWC";
  if (fmt != "NHWC" && fmt != "NCHW")
    return set_status(st, TFMA_INVALID_ARGUMENT, "Invalid data format");
  if (x->ndims < 1)
    return set_status(st, TFMA_INVALID_ARGUMENT, "Input tensor must be at least 1D: %s",
                      shape_str(x).c_str());
  switch (x->dtype) {
    case TFMA_FLOAT: case TFMA_HALF: case TFMA_BFLOAT16: case TFMA_DOUBLE:
    case TFMA_INT32: case TFMA_INT64:
      break;
    default:
      return set_status(st, TFMA_UNIMPLEMENTED, "BiasAddGrad: dtype %s is not supported",
                        dtype_name(x->dtype));
  }
  const int cd = (fmt == "NCHW" && x->ndims > 1) ? 1 : x->ndims - 1;
  *c = x->dims[cd];
  *outer = 1;
  *inner = 1;
  for (int d = 0; d < cd; ++d) *outer *= x->dims[d];
  for (int d = cd + 1; d < x->ndims; ++d) *inner *= x->dims[d];
  if (out) {
    if (out->dtype != x->dtype)
      return set_status(st, TFMA_INVALID_ARGUMENT, "BiasAddGrad: output dtype %s, expected %s",
                        dtype_name(out->dtype), dtype_name(x->dtype));
    if (out->ndims != 1 || out->dims[0] != *c)
      return set_status(st, TFMA_INVALID_ARGUMENT, "BiasAddGrad: output shape %s, expected [%lld]",
                        shape_str(out).c_str(), static_cast<long long>(*c));
  }
  if (*inner >= (int64_t(1) << 31) || *c >= (int64_t(1) << 31))
    return set_status(st, TFMA_UNIMPLEMENTED, "BiasAddGrad: dimension too large");
  return TFMA_OK;
}

int elem_size(int dt) {
  switch (dt) {
    case TFMA_HALF: case TFMA_BFLOAT16: return 2;
    case TFMA_DOUBLE: case TFMA_INT64: return 8;
    default: return 4;
  }
}

}  // namespace

int TFMA_BiasAddGradWorkspaceBytes(const TFMA_Tensor* out_backprop, const char* data_format,
                                   size_t* bytes, TFMA_Status* status) {
  int64_t outer = 0, c = 0, inner = 0;
  if (const int rc = bias_grad_geometry(out_backprop, data_format, nullptr, &outer, &c, &inner,
                                        status))
    return rc;
  if (!bytes) return set_status(status, TFMA_INVALID_ARGUMENT, "bytes is null");
  *bytes = (out_backprop->ndims < 2 || c == 0)
               ? 0
               : BiasAddGradWorkspaceBytes(out_backprop->dtype, outer, c, inner,
                                           elem_size(out_backprop->dtype));
  return ok(status);
}

int TFMA_BiasAddGrad(void* stream, const TFMA_Tensor* out_backprop, const char* data_format,
                     TFMA_Tensor* output, void* workspace, size_t workspace_bytes,
                     TFMA_Status* status) {
  int64_t outer = 0, c = 0, inner = 0;
  if (const int rc = bias_grad_geometry(out_backprop, data_format, output, &outer, &c, &inner,
                                        status))
    return rc;
  if (c == 0) return ok(status);
  if (!output->data) return set_status(status, TFMA_INVALID_ARGUMENT, "BiasAddGrad: null output");
  const int es = elem_size(out_backprop->dtype);
  hipStream_t strm = as_stream(stream);
  // Rank 1: nothing to reduce; the output is the input (reference :50-58).
  if (out_backprop->ndims == 1) {
    if (!out_backprop->data)
      return set_status(status, TFMA_INVALID_ARGUMENT, "BiasAddGrad: null input");
    return hip_status(status,
                      hipMemcpyAsync(output->data, out_backprop->data, static_cast<size_t>(c) * es,
                                     hipMemcpyDeviceToDevice, strm),
                      "BiasAddGrad");
  }
  // Nothing summed: zeros (reference :64-69).
  if (outer == 0 || inner == 0)
    return hip_status(status, LaunchZeroBytes(output->data, c * es, strm), "BiasAddGrad");
  if (!out_backprop->data)
    return set_status(status, TFMA_INVALID_ARGUMENT, "BiasAddGrad: null input");
  const size_t need = BiasAddGradWorkspaceBytes(out_backprop->dtype, outer, c, inner, es);
  if (!workspace || workspace_bytes < need)
    return set_status(status, TFMA_INVALID_ARGUMENT,
                      "BiasAddGrad: workspace of %zu bytes required, got %zu", need,
                      workspace ? workspace_bytes : size_t(0));
  return hip_status(status,
                    LaunchBiasAddGrad(out_backprop->dtype, out_backprop->data, outer, c, inner,
                                      output->data, workspace, strm),
                    "BiasAddGrad");
}

int TFMA_BiasAddGradNoAlloc(void* stream, const TFMA_Tensor* out_backprop,
                            const char* data_format, TFMA_Tensor* output, TFMA_Status* status) {
  int64_t outer = 0, c = 0, inner = 0;
  if (const int rc = bias_grad_geometry(out_backprop, data_format, output, &outer, &c, &inner,
                                        status))
    return rc;
  if (c == 0) return ok(status);
  if (!output->data) return set_status(status, TFMA_INVALID_ARGUMENT, "BiasAddGrad: null output");
  const int es = elem_size(out_backprop->dtype);
  hipStream_t strm = as_stream(stream);
  if (out_backprop->ndims == 1) {
    if (!out_backprop->data)
      return set_status(status, TFMA_INVALID_ARGUMENT, "BiasAddGrad: null input");
    return hip_status(status,
                      hipMemcpyAsync(output->data, out_backprop->data, static_cast<size_t>(c) * es,
                                     hipMemcpyDeviceToDevice, strm),
                      "BiasAddGrad");
  }
  if (outer == 0 || inner == 0)
    return hip_status(status, LaunchZeroBytes(output->data, c * es, strm), "BiasAddGrad");
  if (!out_backprop->data)
    return set_status(status, TFMA_INVALID_ARGUMENT, "BiasAddGrad: null input");
  const size_t need = BiasAddGradWorkspaceBytes(out_backprop->dtype, outer, c, inner, es);
  if (need > kBiasAddGradScratchBytes)
    return set_status(status, TFMA_INVALID_ARGUMENT,
                      "BiasAddGradNoAlloc: this input needs %zu bytes of scratch, more than the "
                      "library's static %zu bytes; use TFMA_BiasAddGrad with a workspace",
                      need, kBiasAddGradScratchBytes);
  return hip_status(status,
                    LaunchBiasAddGradNoAlloc(out_backprop->dtype, out_backprop->data, outer, c,
                                             inner, output->data, strm),
                    "BiasAddGrad");
}

int TFMA_AddV2(void* stream, const TFMA_Tensor* x, const TFMA_Tensor* y, TFMA_Tensor* z,
               TFMA_Status* status) {
  const TFMA_Tensor* ins[2] = {x, y};
  return run_elementwise(stream, EwOp::kAdd, "Add", ins, 2, z, true, status,
                         IntTypes::kI32I64U8);
}

int TFMA_Mul(void* stream, const TFMA_Tensor* x, const TFMA_Tensor* y, TFMA_Tensor* z,
             TFMA_Status* status) {
  const TFMA_Tensor* ins[2] = {x, y};
  return run_elementwise(stream, EwOp::kMul, "Mul", ins, 2, z, true, status,
                         IntTypes::kI32I64);
}

int TFMA_MusaAddV2Relu(void* stream, const TFMA_Tensor* x, const TFMA_Tensor* y,
                       TFMA_Tensor* z, TFMA_Status* status) {
  const TFMA_Tensor* ins[2] = {x, y};
  return run_elementwise(stream, EwOp::kAddRelu, "MusaAddV2Relu", ins, 2, z, true, status);
}

int TFMA_MusaShiftedAffineMap(void* stream, const TFMA_Tensor* data_left,
                              const TFMA_Tensor* mask, const TFMA_Tensor* sliced_var_right,
                              TFMA_Tensor* output, TFMA_Status* status) {
  const TFMA_Tensor* ins[3] = {data_left, mask, sliced_var_right};
  return run_elementwise(stream, EwOp::kMulAdd, "MusaShiftedAffineMap", ins, 3, output, true,
                         status);
}

}  // extern "C"
