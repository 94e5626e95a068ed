// Adam update kernels for gfx950: single-tensor (ResourceApplyAdam) and
// multi-tensor (grouped) variants.
//
// Per element, in TensorFlow's CPU order (training_ops.cc ApplyAdamNonCuda,
// which the reference's op mirrors for its semantics; reference kernel:
// musa_ext/kernels/training/musa_apply_sparse_adam_kernel.mu:140-157):
//   m   += (g - m) * (1 - beta1)
//   v   += (g*g - v) * (1 - beta2)
//   var -= (m * alpha) / (sqrt(v) + epsilon)
//   nesterov: var -= ((g * (1 - beta1) + beta1 * m) * alpha) / (sqrt(v) + eps)
// Every operation is rounded to T (Eigen evaluates half/bfloat16 in float and
// rounds after each operation); the file is compiled with -ffp-contract=off
// so no multiply-add is fused, and sqrt/divide are the correctly rounded
// IEEE operations.
//
// Mixed precision (MusaResourceApplyAdamMixed, and grouped updates with a
// gradient dtype below the state's): fp32 var/m/v with a half or bfloat16
// gradient.  The gradient is widened to float, which is exact, so the update
// equals TF's Cast(grad, float) followed by the fp32 ResourceApplyAdam - the
// pair this op replaces (reference fusion: musa_ext/graph/fusion/
// adam_mixed_fusion.cc:93-216).
//
// Memory: 16-byte vector loads of var, m, v, grad and 16-byte stores of var,
// m, v (28 B per fp32 element, 26 B with a 16-bit gradient); each workgroup
// streams one contiguous chunk with four vectors per tensor in flight per
// thread.
#include "device_util.h"
#include "tfma_internal.h"

#include <type_traits>

namespace tfma {
namespace {

constexpr int kThreads = 256;

template <typename C>
struct AdamP {
  C alpha, beta1, eps, omb1, omb2;
};

__device__ inline float dsqrt(float x) { return __builtin_sqrtf(x); }
__device__ inline double dsqrt(double x) { return __builtin_sqrt(x); }
__device__ inline float ddiv(float a, float b) { return a / b; }
__device__ inline double ddiv(double a, double b) { return a / b; }

// Tr: state (var/m/v) type; Tg: gradient type (Tg = Tr, or fp32 state with a
// 16-bit gradient).
template <class Tr, class Tg, bool kNesterov>
__device__ inline void adam_elem(typename Tr::S& var, typename Tr::S& m,
                                 typename Tr::S& v, typename Tg::S g,
                                 const AdamP<typename Tr::C>& p) {
  using C = typename Tr::C;
  const C gc = static_cast<C>(Tg::ld(g));
  C mc = Tr::ld(m);
  C vc = Tr::ld(v);
  C xc = Tr::ld(var);
  mc = Tr::rnd(mc + Tr::rnd(Tr::rnd(gc - mc) * p.omb1));
  const C g2 = Tr::rnd(gc * gc);
  vc = Tr::rnd(vc + Tr::rnd(Tr::rnd(g2 - vc) * p.omb2));
  C num;
  if constexpr (kNesterov) {
    num = Tr::rnd(
        Tr::rnd(Tr::rnd(gc * p.omb1) + Tr::rnd(p.beta1 * mc)) * p.alpha);
  } else {
    num = Tr::rnd(mc * p.alpha);
  }
  const C den = Tr::rnd(Tr::rnd(dsqrt(vc)) + p.eps);
  xc = Tr::rnd(xc - Tr::rnd(ddiv(num, den)));
  m = Tr::st(mc);
  v = Tr::st(vc);
  var = Tr::st(xc);
}

// Launches that stream at least this many elements load with non-temporal
// loads: measured on MI355X (f32, Infinity Cache flushed between reps), plain
// loads are 8 % faster at 2^25 elements, both equal at 2^26, non-temporal
// loads 2.6-4.5 % faster from 2^27 up.
constexpr int64_t kStreamElems = int64_t(1) << 26;

// Updates elements [0, len) of one contiguous range with the whole
// workgroup: 16-byte vectors, U per tensor in flight per thread, when every
// pointer is aligned for them; element by element otherwise.
template <class Tr, class Tg, bool kNesterov, bool kStream>
__device__ inline void adam_range(typename Tr::S* __restrict__ var, typename Tr::S* __restrict__ m,
                                  typename Tr::S* __restrict__ v,
                                  const typename Tg::S* __restrict__ g, int64_t len,
                                  const AdamP<typename Tr::C>& p) {
  using S = typename Tr::S;
  using SG = typename Tg::S;
  constexpr int VEC = Tr::kVec;
  const uintptr_t align = reinterpret_cast<uintptr_t>(var) |
                          reinterpret_cast<uintptr_t>(m) |
                          reinterpret_cast<uintptr_t>(v);
  int64_t done = 0;
  if ((align & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(g) & (VEC * sizeof(SG) - 1)) == 0) {
    const int64_t nv = len / VEC;
    constexpr int U = 4;
    int64_t i = threadIdx.x;
    for (; i + (U - 1) * kThreads < nv; i += U * kThreads) {
      S xv[U][VEC], mv[U][VEC], vv[U][VEC];
      SG gv[U][VEC];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t off = (i + u * kThreads) * VEC;
        vload_sel<kStream, SG, VEC>(g + off, gv[u]);
        vload_sel<kStream, S, VEC>(m + off, mv[u]);
        vload_sel<kStream, S, VEC>(v + off, vv[u]);
        vload_sel<kStream, S, VEC>(var + off, xv[u]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int j = 0; j < VEC; ++j)
          adam_elem<Tr, Tg, kNesterov>(xv[u][j], mv[u][j], vv[u][j], gv[u][j], p);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t off = (i + u * kThreads) * VEC;
        vstore_nt<S, VEC>(m + off, mv[u]);
        vstore_nt<S, VEC>(v + off, vv[u]);
        vstore_nt<S, VEC>(var + off, xv[u]);
      }
    }
    for (; i < nv; i += kThreads) {
      S xv[VEC], mv[VEC], vv[VEC];
      SG gv[VEC];
      const int64_t off = i * VEC;
      vload_sel<kStream, SG, VEC>(g + off, gv);
      vload_sel<kStream, S, VEC>(m + off, mv);
      vload_sel<kStream, S, VEC>(v + off, vv);
      vload_sel<kStream, S, VEC>(var + off, xv);
#pragma unroll
      for (int j = 0; j < VEC; ++j)
        adam_elem<Tr, Tg, kNesterov>(xv[j], mv[j], vv[j], gv[j], p);
      vstore_nt<S, VEC>(m + off, mv);
      vstore_nt<S, VEC>(v + off, vv);
      vstore_nt<S, VEC>(var + off, xv);
    }
    done = nv * VEC;
  }
  for (int64_t k = done + threadIdx.x; k < len; k += kThreads) {
    S xs = var[k], ms = m[k], vs = v[k];
    adam_elem<Tr, Tg, kNesterov>(xs, ms, vs, g[k], p);
    var[k] = xs;
    m[k] = ms;
    v[k] = vs;
  }
}

// Single tensor: workgroup b updates elements [b*C, (b+1)*C) with C =
// kGroupedAdamChunk.  Contiguous per-workgroup ranges sustain a higher HBM
// rate than a grid-stride sweep on this read-modify-write pattern (measured
// on MI355X: 5.2 vs 4.8 TB/s at 1.3e9 elements).
template <class Tr, class Tg, bool kNesterov, bool kStream>
__global__ __launch_bounds__(kThreads) void adam_chunk_kernel(
    typename Tr::S* __restrict__ var, typename Tr::S* __restrict__ m,
    typename Tr::S* __restrict__ v, const typename Tg::S* __restrict__ g, int64_t n,
    AdamP<typename Tr::C> p) {
  const int64_t start = static_cast<int64_t>(blockIdx.x) * kGroupedAdamChunk;
  int64_t len = n - start;
  if (len > kGroupedAdamChunk) len = kGroupedAdamChunk;
  adam_range<Tr, Tg, kNesterov, kStream>(var + start, m + start, v + start, g + start, len, p);
}

// Grouped variant: workgroup b updates chunk b of the concatenation of all
// tensors; its tensor is chunk_map[b] (the uint32 array after the n_tensors
// entries), two dependent scalar loads instead of a binary search.
template <class Tr, class Tg, bool kNesterov, bool kStream>
__global__ __launch_bounds__(kThreads) void adam_grouped_kernel(
    const AdamTensorEntry* __restrict__ table, int n_tensors,
    AdamP<typename Tr::C> p) {
  using S = typename Tr::S;
  using SG = typename Tg::S;
  const int64_t b = blockIdx.x;
  const uint32_t* __restrict__ chunk_map = reinterpret_cast<const uint32_t*>(table + n_tensors);
  const AdamTensorEntry e = table[chunk_map[b]];
  const int64_t start = (b - e.first_chunk) * kGroupedAdamChunk;
  int64_t len = e.n - start;
  if (len > kGroupedAdamChunk) len = kGroupedAdamChunk;
  adam_range<Tr, Tg, kNesterov, kStream>(static_cast<S*>(e.var) + start,
                                         static_cast<S*>(e.m) + start,
                                static_cast<S*>(e.v) + start,
                                static_cast<const SG*>(e.grad) + start, len, p);
}

// Grouped variant for launches recorded into a graph: the table travels in
// the kernel arguments, which a recorded launch keeps by value (a device
// table staged per call could have changed by the time a replay reads it).
// Workgroup b finds its tensor by a binary search over the chunk prefix sums,
// read from the kernarg segment through its pointer (indexing the by-value
// argument would copy it to scratch).
template <class Tr, class Tg, bool kNesterov, bool kStream>
__global__ __launch_bounds__(kThreads) void adam_grouped_args_kernel(
    AdamArgTable tab, AdamP<typename Tr::C> p) {
  using S = typename Tr::S;
  using SG = typename Tg::S;
  (void)tab;
  const AdamArgTable* t = (const AdamArgTable*)__builtin_amdgcn_kernarg_segment_ptr();
  const int64_t b = blockIdx.x;
  int lo = 0, hi = t->count - 1;  // the last tensor whose first chunk is <= b
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (t->first_chunk[mid] <= b) lo = mid;
    else hi = mid - 1;
  }
  const int64_t start = (b - t->first_chunk[lo]) * kGroupedAdamChunk;
  int64_t len = t->n[lo] - start;
  if (len > kGroupedAdamChunk) len = kGroupedAdamChunk;
  adam_range<Tr, Tg, kNesterov, kStream>(static_cast<S*>(t->var[lo]) + start,
                                         static_cast<S*>(t->m[lo]) + start,
                                         static_cast<S*>(t->v[lo]) + start,
                                         static_cast<const SG*>(t->grad[lo]) + start, len, p);
}

// Integer state (int32 / int64): the reference's generic op chain for T
// (musa_applyadam_op.cc:300-408), each step one operation in T:
//   m = m * beta1 + grad * (1 - beta1)
//   v = v * beta2 + (grad * grad) * (1 - beta2)
//   var = var - (m / (sqrt(v) + epsilon)) * alpha
// Multiplies, adds and subtracts wrap (two's complement).  The reference
// runs the square root and the division through the closed muDNN library,
// whose integer semantics are not published; here the square root is the
// exact integer square root (0 for v <= 0) and the division truncates
// toward zero, with 0 for a zero divisor and MIN / -1 = MIN.  The chain has
// no Nesterov form (the reference's ignores use_nesterov).
template <typename T>
struct IntOps {
  using U = typename std::make_unsigned<T>::type;
  __device__ static T add(T a, T b) { return static_cast<T>(static_cast<U>(a) + static_cast<U>(b)); }
  __device__ static T sub(T a, T b) { return static_cast<T>(static_cast<U>(a) - static_cast<U>(b)); }
  __device__ static T mul(T a, T b) { return static_cast<T>(static_cast<U>(a) * static_cast<U>(b)); }
  __device__ static T div(T a, T b) {
    if (b == 0) return 0;
    if (b == -1) return sub(0, a);
    return a / b;
  }
  __device__ static T sqrt(T v) {
    if (v <= 0) return 0;
    const uint64_t u = static_cast<uint64_t>(v);
    // The double root is within one of the integer root; s * s and
    // (s + 1) * (s + 1) fit in 64 bits for any v < 2^63.
    uint64_t r = static_cast<uint64_t>(__builtin_sqrt(static_cast<double>(v)));
    while (r * r > u) --r;
    while ((r + 1) * (r + 1) <= u) ++r;
    return static_cast<T>(r);
  }
};

template <typename T>
__global__ __launch_bounds__(kThreads) void adam_int_kernel(T* __restrict__ var, T* __restrict__ m,
                                                           T* __restrict__ v,
                                                           const T* __restrict__ g, int64_t n,
                                                           IntAdamScalars s) {
  using O = IntOps<T>;
  const T b1 = static_cast<T>(s.beta1), b2 = static_cast<T>(s.beta2);
  const T omb1 = static_cast<T>(s.omb1), omb2 = static_cast<T>(s.omb2);
  const T eps = static_cast<T>(s.eps), alpha = static_cast<T>(s.alpha);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride) {
    const T gi = g[i];
    const T mi = O::add(O::mul(m[i], b1), O::mul(gi, omb1));
    const T vi = O::add(O::mul(v[i], b2), O::mul(O::mul(gi, gi), omb2));
    const T upd = O::mul(O::div(mi, O::add(O::sqrt(vi), eps)), alpha);
    var[i] = O::sub(var[i], upd);
    m[i] = mi;
    v[i] = vi;
  }
}

template <class Tr>
AdamP<typename Tr::C> make_params(const AdamScalars& s) {
  using C = typename Tr::C;
  AdamP<C> p;
  p.alpha = static_cast<C>(s.alpha);
  p.beta1 = static_cast<C>(s.beta1);
  p.eps = static_cast<C>(s.epsilon);
  p.omb1 = static_cast<C>(s.one_minus_beta1);
  p.omb2 = static_cast<C>(s.one_minus_beta2);
  return p;
}

template <class Tr, class Tg, bool kNesterov>
hipError_t launch_flat(void* var, void* m, void* v, const void* grad,
                       int64_t n, const AdamScalars& s, hipStream_t stream) {
  using S = typename Tr::S;
  using SG = typename Tg::S;
  constexpr int VEC = Tr::kVec;
  const auto p = make_params<Tr>(s);
  const uintptr_t align =
      reinterpret_cast<uintptr_t>(var) | reinterpret_cast<uintptr_t>(m) |
      reinterpret_cast<uintptr_t>(v);
  const bool vec_ok =
      (align & 15) == 0 && (reinterpret_cast<uintptr_t>(grad) & (VEC * sizeof(SG) - 1)) == 0;
  const int64_t blocks = (n + kGroupedAdamChunk - 1) / kGroupedAdamChunk;
  const char* const kname = vec_ok ? "tfma_adam_flat_vec" : "tfma_adam_flat_scalar";
  if (n >= kStreamElems)
    TFMA_LAUNCH(kname, (adam_chunk_kernel<Tr, Tg, kNesterov, true>), dim3(blocks),
                       dim3(kThreads), 0, stream, static_cast<S*>(var), static_cast<S*>(m),
                       static_cast<S*>(v), static_cast<const SG*>(grad), n, p);
  else
    TFMA_LAUNCH(kname, (adam_chunk_kernel<Tr, Tg, kNesterov, false>), dim3(blocks),
                       dim3(kThreads), 0, stream, static_cast<S*>(var), static_cast<S*>(m),
                       static_cast<S*>(v), static_cast<const SG*>(grad), n, p);
  return hipGetLastError();
}

template <class Tr, class Tg, bool kNesterov>
hipError_t launch_grouped(const AdamTensorEntry* table, int n_tensors,
                          int64_t total_chunks, const AdamScalars& s,
                          hipStream_t stream) {
  const auto p = make_params<Tr>(s);
  if (total_chunks * kGroupedAdamChunk >= kStreamElems)
    TFMA_LAUNCH("tfma_adam_grouped", (adam_grouped_kernel<Tr, Tg, kNesterov, true>), dim3(total_chunks),
                       dim3(kThreads), 0, stream, table, n_tensors, p);
  else
    TFMA_LAUNCH("tfma_adam_grouped", (adam_grouped_kernel<Tr, Tg, kNesterov, false>), dim3(total_chunks),
                       dim3(kThreads), 0, stream, table, n_tensors, p);
  return hipGetLastError();
}

// The table in kernel arguments, kArgTableTensors tensors per launch.
template <class Tr, class Tg, bool kNesterov>
hipError_t launch_grouped_args(const AdamTensorEntry* entries, int n_tensors,
                               const AdamScalars& s, hipStream_t stream) {
  const auto p = make_params<Tr>(s);
  for (int i0 = 0; i0 < n_tensors; i0 += kArgTableTensors) {
    const int cnt = n_tensors - i0 < kArgTableTensors ? n_tensors - i0 : kArgTableTensors;
    AdamArgTable t{};
    int64_t chunks = 0;
    for (int k = 0; k < cnt; ++k) {
      const AdamTensorEntry& e = entries[i0 + k];
      t.first_chunk[k] = chunks;
      t.var[k] = e.var;
      t.m[k] = e.m;
      t.v[k] = e.v;
      t.grad[k] = e.grad;
      t.n[k] = e.n;
      chunks += (e.n + kGroupedAdamChunk - 1) / kGroupedAdamChunk;
    }
    t.first_chunk[cnt] = chunks;
    t.count = cnt;
    if (chunks == 0) continue;
    if (chunks * kGroupedAdamChunk >= kStreamElems)
      TFMA_LAUNCH("tfma_adam_grouped", (adam_grouped_args_kernel<Tr, Tg, kNesterov, true>),
                  dim3(chunks), dim3(kThreads), 0, stream, t, p);
    else
      TFMA_LAUNCH("tfma_adam_grouped", (adam_grouped_args_kernel<Tr, Tg, kNesterov, false>),
                  dim3(chunks), dim3(kThreads), 0, stream, t, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace

hipError_t LaunchGroupedApplyAdamArgs(DType t, DType tg, const AdamTensorEntry* entries,
                                      int n_tensors, const AdamScalars& s, bool nesterov,
                                      hipStream_t stream) {
  if (n_tensors <= 0) return hipSuccess;
#define TFMA_GADAM_ARGS(TR, TG)                                                        \
  return nesterov ? launch_grouped_args<TR, TG, true>(entries, n_tensors, s, stream)  \
                  : launch_grouped_args<TR, TG, false>(entries, n_tensors, s, stream);
  if (tg != t) {
    if (t != DType::kF32) return hipErrorInvalidValue;
    switch (tg) {
      case DType::kF16: TFMA_GADAM_ARGS(TF32, TF16)
      case DType::kBF16: TFMA_GADAM_ARGS(TF32, TBF16)
      default: return hipErrorInvalidValue;
    }
  }
  switch (t) {
    case DType::kF32: TFMA_GADAM_ARGS(TF32, TF32)
    case DType::kF16: TFMA_GADAM_ARGS(TF16, TF16)
    case DType::kBF16: TFMA_GADAM_ARGS(TBF16, TBF16)
    case DType::kF64: TFMA_GADAM_ARGS(TF64, TF64)
    default: break;  // integer state: LaunchApplyAdamInt
  }
#undef TFMA_GADAM_ARGS
  return hipErrorInvalidValue;
}

hipError_t LaunchApplyAdam(DType t, DType tg, void* var, void* m, void* v,
                           const void* grad, int64_t n, const AdamScalars& s,
                           bool nesterov, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
#define TFMA_ADAM_CASE(TR, TG)                                                  \
  return nesterov ? launch_flat<TR, TG, true>(var, m, v, grad, n, s, stream)   \
                  : launch_flat<TR, TG, false>(var, m, v, grad, n, s, stream);
  if (tg != t) {
    if (t != DType::kF32) return hipErrorInvalidValue;
    switch (tg) {
      case DType::kF16: TFMA_ADAM_CASE(TF32, TF16)
      case DType::kBF16: TFMA_ADAM_CASE(TF32, TBF16)
      default: return hipErrorInvalidValue;
    }
  }
  switch (t) {
    case DType::kF32: TFMA_ADAM_CASE(TF32, TF32)
    case DType::kF16: TFMA_ADAM_CASE(TF16, TF16)
    case DType::kBF16: TFMA_ADAM_CASE(TBF16, TBF16)
    case DType::kF64: TFMA_ADAM_CASE(TF64, TF64)
    default: break;  // integer state: LaunchApplyAdamInt
  }
#undef TFMA_ADAM_CASE
  return hipErrorInvalidValue;
}

hipError_t LaunchApplyAdamInt(bool is64, void* var, void* m, void* v, const void* grad,
                              int64_t n, const IntAdamScalars& s, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  int64_t blocks = (n + kThreads - 1) / kThreads;
  const int64_t cap = static_cast<int64_t>(DeviceCUs()) * 8;
  if (blocks > cap) blocks = cap;
  if (is64)
    TFMA_LAUNCH("tfma_adam_int", adam_int_kernel<int64_t>, dim3(blocks), dim3(kThreads), 0,
                stream, static_cast<int64_t*>(var), static_cast<int64_t*>(m),
                static_cast<int64_t*>(v), static_cast<const int64_t*>(grad), n, s);
  else
    TFMA_LAUNCH("tfma_adam_int", adam_int_kernel<int32_t>, dim3(blocks), dim3(kThreads), 0,
                stream, static_cast<int32_t*>(var), static_cast<int32_t*>(m),
                static_cast<int32_t*>(v), static_cast<const int32_t*>(grad), n, s);
  return hipGetLastError();
}

hipError_t LaunchGroupedApplyAdam(DType t, DType tg, const AdamTensorEntry* dev_table,
                                  int n_tensors, int64_t total_chunks,
                                  const AdamScalars& s, bool nesterov,
                                  hipStream_t stream) {
  if (total_chunks <= 0) return hipSuccess;
#define TFMA_GADAM_CASE(TR, TG)                                               \
  return nesterov ? launch_grouped<TR, TG, true>(dev_table, n_tensors,       \
                                                 total_chunks, s, stream)    \
                  : launch_grouped<TR, TG, false>(dev_table, n_tensors,      \
                                                  total_chunks, s, stream);
  if (tg != t) {
    if (t != DType::kF32) return hipErrorInvalidValue;
    switch (tg) {
      case DType::kF16: TFMA_GADAM_CASE(TF32, TF16)
      case DType::kBF16: TFMA_GADAM_CASE(TF32, TBF16)
      default: return hipErrorInvalidValue;
    }
  }
  switch (t) {
    case DType::kF32: TFMA_GADAM_CASE(TF32, TF32)
    case DType::kF16: TFMA_GADAM_CASE(TF16, TF16)
    case DType::kBF16: TFMA_GADAM_CASE(TBF16, TBF16)
    case DType::kF64: TFMA_GADAM_CASE(TF64, TF64)
    default: break;  // integer state: LaunchApplyAdamInt
  }
#undef TFMA_GADAM_CASE
  return hipErrorInvalidValue;
}

}  // namespace tfma
