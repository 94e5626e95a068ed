// Elementwise kernels for gfx950: BiasAdd, Relu, AddV2, Mul and the fused
// chains Relu(BiasAdd), Relu(AddV2) and Mul+Add (MusaShiftedAffineMap).
// Add and Mul also run on int32 / int64 (and add on uint8), wrapping modulo
// 2^bits: the same kernels over 16-byte vectors of 4, 2 or 16 elements.
//
// Numerics follow TensorFlow's CPU kernels: each TF op computes in float and
// rounds to T once, so a fused chain rounds after every op it replaces
// (Mul+Add rounds the product before the add; compiled with
// -ffp-contract=off so it never becomes a fused multiply-add).  Relu keeps
// the input bits unless x < 0, so Relu(-0) = -0 and Relu(NaN) = NaN as with
// Eigen's max.
//
// Memory: the value input and the output are streamed with 16-byte vector
// accesses over the flat index; a broadcast operand is read as a 16-byte
// vector when its period is a multiple of the vector width (row vectors such
// as a BiasAdd bias over the last dimension), as one value per vector when
// its inner extent is (NCHW bias), and gathered per element otherwise (odd
// shapes such as [8191, 4095]).  Broadcast operands are tiny and stay in
// L1/L2, so HBM traffic is the compulsory stream of the full-size tensors.
#include <atomic>

#include "device_util.h"
#include "tfma_internal.h"

namespace tfma {
namespace {

constexpr int kThreads = 256;

// kRowOddK: a row operand (inner extent 1) whose period is not a multiple of
// the vector width - one modulo per vector, then one 16-byte read from the
// operand's shifted copies in LDS (odd_len below).  kGatherK: anything else -
// one division per vector, then an incremental walk of (index, position
// within the inner extent) over a copy of the operand's `period` values in
// LDS.  Each workgroup makes its copies first (per-element gathers from
// global memory are limited by the L1's request rate, not by bytes);
// kGatherGlobalK is the same walk from global memory, for periods larger
// than the LDS copies allow.
enum Kind : int {
  kFullK = 0, kScalarK = 1, kRowK = 2, kChanK = 3, kRowOddK = 4, kGatherK = 5, kGatherGlobalK = 6
};
constexpr bool staged_kind(int k) { return k == kRowOddK || k == kGatherK; }
// Vectors of `a` per thread a staging kernel loads before its staging
// completes; staged kinds are launched only where every thread has them.
constexpr int kStagedPre = 8;

// A staged odd-period row operand is held as odd_copies(es) = 8 / es copies
// (one for 8-byte elements) of odd_len(period, es) positions each, copy s
// at s * odd_len holding element (k + s) mod period at position k.  The
// vector of V = 16 / es elements that starts at element idx is then the 16
// bytes at position idx - s of copy s = idx mod odd_copies: 8-byte aligned
// whatever idx is, one ds_read2_b64, no wrap at the period's end.  (A
// single copy needed five 32-bit reads and four funnel shifts per half
// vector, and an element loop where a vector wraps; V copies, for 16-byte
// aligned reads, measured no faster and take twice the LDS.)  Consecutive
// lanes read consecutive 16-byte spans of one copy.
__host__ __device__ constexpr uint32_t odd_copies(int es) { return es >= 8 ? 1u : 8u / es; }
// Positions per copy: at least period + V - 1, a multiple of V (so every
// copy starts 16-byte aligned).
__host__ __device__ constexpr uint32_t odd_len(uint32_t period, int es) {
  return (period + 2 * (16 / es) - 2) / (16 / es) * (16 / es);
}
// The copies and one 16-byte slot after them that takes the staging's
// stores of positions no copy has (stored there instead of branched around).
__host__ __device__ constexpr uint32_t odd_stage_bytes(uint32_t period, int es) {
  return period == 0 ? 0 : odd_copies(es) * odd_len(period, es) * es + 16;
}
// LDS budget per staged operand: the shifted copies of periods up to 4095
// elements (32848 bytes for half; a thread then stages at most 17 elements),
// the plain copy of kGatherK periods up to 20496 bytes.
constexpr uint32_t kOddStageBytes = 32848;
constexpr uint32_t kGatherStageBytes = 20496;
__host__ __device__ constexpr uint32_t stage_bytes(int kind, uint32_t period, int es) {
  return kind == kRowOddK ? odd_stage_bytes(period, es) : (kind == kGatherK ? period * es : 0);
}
__host__ __device__ constexpr uint32_t round16(uint32_t b) { return (b + 15u) & ~15u; }

struct Operand {
  const void* p;
  int kind;
  uint32_t period;
  uint32_t inner;
  uint32_t olen;  // kRowOddK: odd_len(period, element bytes)
  FastDiv div_inner;
  FastDiv div_period;
};

template <typename S>
__device__ inline S gather_one(const Operand& o, uint32_t i) {
  const S* p = static_cast<const S*>(o.p);
  const uint32_t q = o.div_inner.div(i);
  const uint32_t idx = q - o.div_period.div(q) * o.period;
  return p[idx];
}

// Loads the V operand values for flat indices i0 .. i0+V-1.  K is the
// operand kind when known at compile time (the vector kernels are
// instantiated per kind, so no branch separates the loads of one unrolled
// iteration from the next and every load is in flight before the first use);
// kAnyK switches on o.kind at run time.
constexpr int kAnyK = -1;

// p is the operand's data: o.p, or its LDS copy for the staged kinds.
// NT (the kernel's cache mode): >= 1 loads a full-size operand
// non-temporally, 2 also a row operand.
template <int K, typename S, int V, int NT = 0>
__device__ inline void fetch(const Operand& o, const S* p, uint32_t i0, S (&out)[V]) {
  if constexpr (K == kAnyK) {
    switch (o.kind) {
      case kFullK: fetch<kFullK, S, V>(o, p, i0, out); break;
      case kScalarK: fetch<kScalarK, S, V>(o, p, i0, out); break;
      case kRowK: fetch<kRowK, S, V>(o, p, i0, out); break;
      case kChanK: fetch<kChanK, S, V>(o, p, i0, out); break;
      case kRowOddK:  // only classified for 16-byte vectors
        if constexpr (V * sizeof(S) == 16) {
          fetch<kRowOddK, S, V>(o, p, i0, out);
          break;
        }
        [[fallthrough]];
      default: fetch<kGatherK, S, V>(o, p, i0, out); break;
    }
  } else if constexpr (K == kFullK) {
    vload_sel<(NT >= 1), S, V>(p + i0, out);
  } else if constexpr (K == kScalarK) {
    const S s = p[0];
#pragma unroll
    for (int j = 0; j < V; ++j) out[j] = s;
  } else if constexpr (K == kRowK) {
    const uint32_t idx = i0 - o.div_period.div(i0) * o.period;
    vload_sel<(NT == 2), S, V>(p + idx, out);
  } else if constexpr (K == kChanK) {
    const S s = gather_one<S>(o, i0);
#pragma unroll
    for (int j = 0; j < V; ++j) out[j] = s;
  } else if constexpr (K == kRowOddK) {
    // p is the shifted copies (odd_len).
    constexpr uint32_t kC = odd_copies(sizeof(S));
    static_assert(V * sizeof(S) == 16 && V % kC == 0, "one 16-byte read");
    const uint32_t idx = i0 - o.div_period.div(i0) * o.period;
    const uint32_t sh = idx & (kC - 1);
    const uint2* q = static_cast<const uint2*>(
        __builtin_assume_aligned(p + sh * o.olen + (idx - sh), 8));
    const uint4 w = make_uint4(q[0].x, q[0].y, q[1].x, q[1].y);
    __builtin_memcpy(out, &w, 16);
  } else {
    const uint32_t q = o.div_inner.div(i0);
    uint32_t r = i0 - q * o.inner;
    uint32_t idx = q - o.div_period.div(q) * o.period;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      out[j] = p[idx];
      const bool next = ++r == o.inner;
      r = next ? 0 : r;
      idx = next ? (idx + 1 == o.period ? 0 : idx + 1) : idx;
    }
  }
}

// Elements of the extended period a thread stages (odd_len is at most
// kOddStageBytes / (odd_copies * es); copy s needs odd_len + s positions).
template <typename S>
constexpr uint32_t odd_stage_loads() {
  constexpr uint32_t kC = odd_copies(sizeof(S));
  return ((kOddStageBytes - 16) / (kC * sizeof(S)) + kC - 1 + kThreads - 1) / kThreads;
}

// A workgroup's LDS copy of a staged operand (src: its values in global
// memory), in two steps so that the kernel can issue its first loads of `a`
// between them: issue() starts the global loads, commit() writes LDS (the
// kernel's __syncthreads follows).  kGatherK: the plain copy, in commit().
template <int K, typename S>
struct Stage {
  __device__ void issue(const Operand&, const S*) {}
  __device__ void commit(const Operand& o, const S* src, S* dst) {
#pragma unroll 4
    for (uint32_t k = threadIdx.x; k < o.period; k += kThreads) dst[k] = src[k];
  }
};

// kRowOddK: element t of the extended period (element t mod period, for
// t < odd_len + copies - 1) is loaded once, by thread t mod kThreads, all of
// a thread's loads issued before the first is used, and stored straight
// into every copy s at position t - s (a third of the time of loading copy
// 0 and building the others from it with 16-byte LDS windows).  No load
// or store sits in a branch: load indices past the end are clamped, and a
// position no copy has is stored to the spare slot after the copies.  (A load whose use
// sat in a branch left the compiler's wait analysis treating its register
// as pending in the streaming loop, which then waited for each load before
// issuing the next; and loads in branches make it wait for every
// outstanding load, the kernel's prefetch of `a` included.)
template <typename S>
struct Stage<kRowOddK, S> {
  static constexpr uint32_t kLoads = odd_stage_loads<S>();
  S v0[kLoads];
  __device__ void issue(const Operand& o, const S* src) {
    const uint32_t ext = o.olen + odd_copies(sizeof(S)) - 1;
#pragma unroll
    for (uint32_t r = 0; r < kLoads; ++r) {
      uint32_t k = threadIdx.x + r * kThreads;
      k = k < ext ? k : ext - 1;
      v0[r] = src[k - o.div_period.div(k) * o.period];
    }
  }
  __device__ void commit(const Operand& o, const S*, S* dst) {
    constexpr uint32_t kC = odd_copies(sizeof(S));
    const uint32_t len = o.olen;
#pragma unroll
    for (uint32_t r = 0; r < kLoads; ++r) {
      const uint32_t t = threadIdx.x + r * kThreads;
#pragma unroll
      for (uint32_t sh = 0; sh < kC; ++sh) {
        const bool in = t >= sh && t - sh < len;
        dst[in ? sh * len + (t - sh) : kC * len] = v0[r];
      }
    }
  }
};

template <class Tr, EwOp OP>
__device__ inline typename Tr::S ew_apply(typename Tr::S a, typename Tr::S b,
                                          typename Tr::S c) {
  using C = typename Tr::C;
  const C x = Tr::ld(a);
  if constexpr (OP == EwOp::kAdd) {
    return Tr::st(x + Tr::ld(b));
  } else if constexpr (OP == EwOp::kAddRelu) {
    const typename Tr::S r = Tr::st(x + Tr::ld(b));
    return Tr::ld(r) < C(0) ? Tr::st(C(0)) : r;
  } else if constexpr (OP == EwOp::kMul) {
    return Tr::st(x * Tr::ld(b));
  } else if constexpr (OP == EwOp::kMulAdd) {
    const C t = Tr::rnd(x * Tr::ld(b));
    return Tr::st(t + Tr::ld(c));
  } else if constexpr (OP == EwOp::kReluGrad) {
    // TF: gradients * (features > 0), a multiply - NaN or inf gradients at
    // features <= 0 give NaN, negative ones give -0.
    return Tr::st(x * (Tr::ld(b) > C(0) ? C(1) : C(0)));
  } else {  // kRelu
    return x < C(0) ? Tr::st(C(0)) : a;
  }
}

template <EwOp OP>
constexpr int arity() {
  return OP == EwOp::kRelu ? 1 : (OP == EwOp::kMulAdd ? 3 : 2);
}

// Flat kernel over n < 2^31 elements; `a` is always full-size.  KB / KC are
// the kinds of the b / c operands (kAnyK: decided per access at run time).
// NT: 1 = full-size operands loaded non-temporally, 2 = row operands loaded
// and the output stored non-temporally as well (chosen by size, see
// stream_mode()).
template <class Tr, EwOp OP, int V, int UNROLL, int KB, int KC, int NT>
__global__ __launch_bounds__(kThreads) void ew_flat_kernel(
    const typename Tr::S* __restrict__ a, Operand b, Operand c,
    typename Tr::S* __restrict__ out, uint32_t n) {
  using S = typename Tr::S;
  constexpr int kArity = arity<OP>();
  extern __shared__ __align__(16) unsigned char ew_lds[];
  const S* pb = static_cast<const S*>(b.p);
  const S* pc = static_cast<const S*>(c.p);
  const uint32_t nv = n / V;
  const uint32_t stride = gridDim.x * kThreads;
  const uint32_t tid = blockIdx.x * kThreads + threadIdx.x;
  // A kernel that stages an operand issues the staging loads, then its
  // first kStagedPre vectors of `a`, then completes the staging: those
  // vectors stream in meanwhile instead of the memory system idling while
  // every workgroup stages (the staging of a [4095] half operand takes
  // ~2.5 us).  Loads complete in order, so the staging waits only for its
  // own - which needs straight-line code: no load of the prologue sits in a
  // branch.  The host launches staged kinds only with
  // nv >= kStagedPre * stride (stage_grid), so every prefetched vector
  // exists; the indices are clamped all the same.
  constexpr bool kSB = kArity >= 2 && staged_kind(KB);
  constexpr bool kSC = kArity >= 3 && staged_kind(KC);
  constexpr int kPre = (kSB || kSC) ? kStagedPre : 1;
  [[maybe_unused]] Stage<KB, S> stb;
  [[maybe_unused]] Stage<KC, S> stc;
  if constexpr (kSB) stb.issue(b, pb);
  if constexpr (kSC) stc.issue(c, pc);
  [[maybe_unused]] S ap[kPre][V];
  if constexpr (kSB || kSC) {
#pragma unroll
    for (int q = 0; q < kPre; ++q) {
      const uint32_t iq = tid + q * stride < nv ? tid + q * stride : nv - 1;
      vload_sel<(NT >= 1), S, V>(a + iq * V, ap[q]);
    }
    // Keep the scheduler from sinking these loads below the staging's first
    // waits (it interleaved them with the LDS stores, after the first
    // staging load had returned).
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (kSB) {
    S* l = reinterpret_cast<S*>(ew_lds);
    stb.commit(b, pb, l);
    pb = l;
  }
  if constexpr (kSC) {
    const uint32_t off = kSB ? round16(stage_bytes(KB, b.period, sizeof(S))) : 0;
    S* l = reinterpret_cast<S*>(ew_lds + off);
    stc.commit(c, pc, l);
    pc = l;
  }
  uint32_t i = tid;
  if constexpr (kSB || kSC) {
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kPre; ++q) {
      const uint32_t iq = tid + q * stride < nv ? tid + q * stride : nv - 1;
      S bv[V], cv[V], ov[V];
      if constexpr (kArity >= 2) fetch<KB, S, V, NT>(b, pb, iq * V, bv);
      if constexpr (kArity >= 3) fetch<KC, S, V, NT>(c, pc, iq * V, cv);
#pragma unroll
      for (int j = 0; j < V; ++j)
        ov[j] = ew_apply<Tr, OP>(ap[q][j], kArity >= 2 ? bv[j] : S(0),
                                 kArity >= 3 ? cv[j] : S(0));
      if (tid + q * stride < nv) vstore_sel<(NT == 2), S, V>(out + iq * V, ov);
    }
    i += kPre * stride;
  }
  for (; i + (UNROLL - 1) * stride < nv; i += UNROLL * stride) {
    S av[UNROLL][V], bv[UNROLL][V], cv[UNROLL][V];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const uint32_t i0 = (i + u * stride) * V;
      vload_sel<(NT >= 1), S, V>(a + i0, av[u]);
      if constexpr (kArity >= 2) fetch<KB, S, V, NT>(b, pb, i0, bv[u]);
      if constexpr (kArity >= 3) fetch<KC, S, V, NT>(c, pc, i0, cv[u]);
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      S ov[V];
#pragma unroll
      for (int j = 0; j < V; ++j)
        ov[j] = ew_apply<Tr, OP>(av[u][j], kArity >= 2 ? bv[u][j] : S(0),
                                 kArity >= 3 ? cv[u][j] : S(0));
      vstore_sel<(NT == 2), S, V>(out + (i + u * stride) * V, ov);
    }
  }
  for (; i < nv; i += stride) {
    const uint32_t i0 = i * V;
    S av[V], bv[V], cv[V], ov[V];
    vload_sel<(NT >= 1), S, V>(a + i0, av);
    if constexpr (kArity >= 2) fetch<KB, S, V, NT>(b, pb, i0, bv);
    if constexpr (kArity >= 3) fetch<KC, S, V, NT>(c, pc, i0, cv);
#pragma unroll
    for (int j = 0; j < V; ++j)
      ov[j] = ew_apply<Tr, OP>(av[j], kArity >= 2 ? bv[j] : S(0),
                               kArity >= 3 ? cv[j] : S(0));
    vstore_sel<(NT == 2), S, V>(out + i0, ov);
  }
  const uint32_t tail = n - nv * V;
  if (tid < tail) {
    const uint32_t k = nv * V + tid;
    const S bs = kArity >= 2 ? gather_one<S>(b, k) : S(0);
    const S cs = kArity >= 3 ? gather_one<S>(c, k) : S(0);
    out[k] = ew_apply<Tr, OP>(a[k], bs, cs);
  }
}

// General broadcast: per element coordinate decomposition (64-bit).
template <class Tr, EwOp OP>
__global__ __launch_bounds__(kThreads) void ew_strided_kernel(
    const typename Tr::S* __restrict__ a, const typename Tr::S* __restrict__ b,
    const typename Tr::S* __restrict__ c, StridedShape sh,
    typename Tr::S* __restrict__ out, int64_t n) {
  using S = typename Tr::S;
  constexpr int kArity = arity<OP>();
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
       i < n; i += stride) {
    int64_t rem = i, oa = 0, ob = 0, oc = 0;
    for (int d = sh.ndims - 1; d >= 0; --d) {
      const int64_t coord = rem % sh.dims[d];
      rem /= sh.dims[d];
      oa += coord * sh.stride_a[d];
      ob += coord * sh.stride_b[d];
      oc += coord * sh.stride_c[d];
    }
    out[i] = ew_apply<Tr, OP>(a[oa], kArity >= 2 ? b[ob] : S(0),
                              kArity >= 3 ? c[oc] : S(0));
  }
}

const char* op_kernel_name(EwOp op) {
  switch (op) {
    case EwOp::kAdd: return "tfma_ew_add";
    case EwOp::kAddRelu: return "tfma_ew_add_relu";
    case EwOp::kMul: return "tfma_ew_mul";
    case EwOp::kMulAdd: return "tfma_ew_mul_add";
    case EwOp::kRelu: return "tfma_ew_relu";
    case EwOp::kReluGrad: return "tfma_ew_relu_grad";
  }
  return "tfma_ew";
}

// Workgroups per CU of the grid-stride kernels (TFMA_EW_BLOCKS_PER_CU).
// Measured on MI355X, kernel time at [8192,4096] (f32 / f16 BiasAdd+Relu):
// 1: 55.3 / 31.7 us, 2: 40.3 / 22.5 us, 3: 41.2 / 23.6 us, 8: 44.8 / 24.3 us,
// 16: 46.1 / 26.1 us - fewer, longer-lived workgroups ramp up and drain
// faster; one per CU leaves too few loads in flight for the row-broadcast
// kinds.
int blocks_per_cu() {
  static int v = [] {
    const char* e = getenv("TFMA_EW_BLOCKS_PER_CU");
    const int b = e ? atoi(e) : 0;
    return b > 0 ? b : 2;
  }();
  return v;
}

int64_t grid_for(int64_t units, int unroll) {
  int64_t blocks = (units + kThreads * unroll - 1) / (kThreads * unroll);
  const int64_t max_blocks = static_cast<int64_t>(DeviceCUs()) * blocks_per_cu();
  if (blocks > max_blocks) blocks = max_blocks;
  if (blocks < 1) blocks = 1;
  return blocks;
}

// Classify an operand for vector width V.
Operand make_operand(const BcastOperand& o, int elem_bytes, int V,
                     bool* vec_ok) {
  Operand r;
  r.p = o.data;
  r.period = 1;
  r.inner = 1;
  r.olen = 0;
  const bool aligned = (reinterpret_cast<uintptr_t>(o.data) & 15) == 0;
  switch (o.mode) {
    case BcastMode::kFull:
      r.kind = kFullK;
      r.div_inner = FastDiv(1);
      r.div_period = FastDiv(0x7fffffffu);  // i < 2^31: idx = i
      r.period = 0x7fffffffu;
      if (!aligned) *vec_ok = false;
      break;
    case BcastMode::kScalar:
      r.kind = kScalarK;
      r.div_inner = FastDiv(1);
      r.div_period = FastDiv(1);
      r.period = 1;
      break;
    case BcastMode::kPeriodic:
      r.div_inner = FastDiv(static_cast<uint32_t>(o.inner));
      r.div_period = FastDiv(static_cast<uint32_t>(o.period));
      r.period = static_cast<uint32_t>(o.period);
      r.inner = static_cast<uint32_t>(o.inner);
      if (o.inner == 1 && o.period % V == 0 && aligned) {
        r.kind = kRowK;
      } else if (o.inner % V == 0) {
        r.kind = kChanK;
      } else if (o.inner == 1 ? odd_stage_bytes(r.period, elem_bytes) > kOddStageBytes
                              : o.period * elem_bytes > kGatherStageBytes) {
        r.kind = kGatherGlobalK;
      } else if (o.inner == 1) {
        r.kind = kRowOddK;
        r.olen = odd_len(r.period, elem_bytes);
      } else {
        r.kind = kGatherK;
      }
      break;
  }
  return r;
}

// Cache mode by size (measured on MI355X with the Infinity Cache flushed
// between reps).  By output size, f32 BiasAdd+Relu: plain accesses are
// 5-10 % faster up to 2^26 elements; at 2^27 non-temporal loads of the full
// operands are 13 % faster; from 2^28 on non-temporal loads of every
// operand and non-temporal stores 5-7 % faster than plain.  By the bytes of
// full-size inputs: from 192 MiB non-temporal loads (cfg4 Mul+Add with full
// a and b, kernel time: f32 74.8 -> 81.3 %, f16 74.2 -> 78.3 % of 8 TB/s;
// ReluGrad f32 79.7 -> 80.9 %; at 128 MiB, f16 ReluGrad, plain loads are
// 2 points faster).  Only the kinds that stream (full, scalar, row,
// channel) have the non-temporal variants.  The "ew_nt" override (for
// measurements): 0, 1 or 2 forces the mode.
int stream_mode(int64_t out_bytes, int64_t full_in_bytes) {
  const int forced = TuneValue(kTuneEwNt);
  if (forced >= 0 && forced <= 2) return forced;
  if (out_bytes >= (int64_t(1) << 30)) return 2;
  if (out_bytes >= (int64_t(1) << 29) || full_in_bytes >= (int64_t(192) << 20)) return 1;
  return 0;
}

constexpr bool streams(int k) {
  return k == kFullK || k == kScalarK || k == kRowK || k == kChanK;
}

// Grid of a staging kernel: at most `blocks`, and few enough that every
// thread has kStagedPre vectors (the kernel's prologue loads them
// unconditionally).  launch_ew stages only where nv >= kStagedPre * kThreads.
int64_t stage_grid(int64_t nv, int64_t blocks) {
  const int64_t most = nv / (static_cast<int64_t>(kThreads) * kStagedPre);
  return blocks < most ? blocks : (most > 0 ? most : 1);
}

// Vector-path launch with the operand kinds as compile-time parameters.
template <class Tr, EwOp OP, int KB, int KC>
void launch_vec(const Operand& ob, const Operand& oc, const typename Tr::S* a,
                typename Tr::S* out, uint32_t n, int nt, hipStream_t stream) {
  constexpr int V = Tr::kVec;
  constexpr int U = 2;
  constexpr bool sb = arity<OP>() >= 2 && staged_kind(KB);
  constexpr bool sc = arity<OP>() >= 3 && staged_kind(KC);
  // A staged workgroup copies the operand once; fewer, longer-lived
  // workgroups keep that copy cheap.
  constexpr int kEs = sizeof(typename Tr::S);
  const uint32_t lds_b = sb ? stage_bytes(KB, ob.period, kEs) : 0;
  const size_t lds = sc ? round16(lds_b) + stage_bytes(KC, oc.period, kEs) : lds_b;
  // Two staged operands may need more than the 64 KB a launch gets by default
  // (a failure here is left for the caller's hipGetLastError).
  if (lds > 65536) {
    // Set once per device (setting it again from another thread is harmless;
    // the flag only saves the call).
    static std::atomic<bool> raised[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return;
    if (!raised[dev].load(std::memory_order_acquire)) {
      constexpr int kMaxLds = static_cast<int>(round16(kOddStageBytes) + kOddStageBytes);
      if (hipFuncSetAttribute(
              reinterpret_cast<const void*>(&ew_flat_kernel<Tr, OP, V, U, KB, KC, 0>),
              hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds) != hipSuccess)
        return;
      raised[dev].store(true, std::memory_order_release);
    }
  }
  int64_t blocks = grid_for(n / V, U);
  if (sb || sc) blocks = stage_grid(n / V, blocks);
  if constexpr (streams(KB) && streams(KC)) {
    if (nt == 2) {
      TFMA_LAUNCH(op_kernel_name(OP), (ew_flat_kernel<Tr, OP, V, U, KB, KC, 2>), dim3(blocks),
                         dim3(kThreads), lds, stream, a, ob, oc, out, n);
      return;
    }
    if (nt == 1) {
      TFMA_LAUNCH(op_kernel_name(OP), (ew_flat_kernel<Tr, OP, V, U, KB, KC, 1>), dim3(blocks),
                         dim3(kThreads), lds, stream, a, ob, oc, out, n);
      return;
    }
  }
  TFMA_LAUNCH(op_kernel_name(OP), (ew_flat_kernel<Tr, OP, V, U, KB, KC, 0>), dim3(blocks),
                     dim3(kThreads), lds, stream, a, ob, oc, out, n);
}

template <class Tr, EwOp OP, int KB>
void pick_kc(const Operand& ob, const Operand& oc, const typename Tr::S* a,
             typename Tr::S* out, uint32_t n, int nt, hipStream_t stream) {
  if constexpr (arity<OP>() < 3) {
    launch_vec<Tr, OP, KB, kFullK>(ob, oc, a, out, n, nt, stream);  // c unused
  } else {
    switch (oc.kind) {
      case kFullK: launch_vec<Tr, OP, KB, kFullK>(ob, oc, a, out, n, nt, stream); break;
      case kScalarK: launch_vec<Tr, OP, KB, kScalarK>(ob, oc, a, out, n, nt, stream); break;
      case kRowK: launch_vec<Tr, OP, KB, kRowK>(ob, oc, a, out, n, nt, stream); break;
      case kChanK: launch_vec<Tr, OP, KB, kChanK>(ob, oc, a, out, n, nt, stream); break;
      case kRowOddK: launch_vec<Tr, OP, KB, kRowOddK>(ob, oc, a, out, n, nt, stream); break;
      case kGatherK: launch_vec<Tr, OP, KB, kGatherK>(ob, oc, a, out, n, nt, stream); break;
      default: launch_vec<Tr, OP, KB, kGatherGlobalK>(ob, oc, a, out, n, nt, stream); break;
    }
  }
}

template <class Tr, EwOp OP>
void pick_kb(const Operand& ob, const Operand& oc, const typename Tr::S* a,
             typename Tr::S* out, uint32_t n, int nt, hipStream_t stream) {
  if constexpr (arity<OP>() < 2) {
    launch_vec<Tr, OP, kFullK, kFullK>(ob, oc, a, out, n, nt, stream);  // b, c unused
  } else {
    switch (ob.kind) {
      case kFullK: pick_kc<Tr, OP, kFullK>(ob, oc, a, out, n, nt, stream); break;
      case kScalarK: pick_kc<Tr, OP, kScalarK>(ob, oc, a, out, n, nt, stream); break;
      case kRowK: pick_kc<Tr, OP, kRowK>(ob, oc, a, out, n, nt, stream); break;
      case kChanK: pick_kc<Tr, OP, kChanK>(ob, oc, a, out, n, nt, stream); break;
      case kRowOddK: pick_kc<Tr, OP, kRowOddK>(ob, oc, a, out, n, nt, stream); break;
      case kGatherK: pick_kc<Tr, OP, kGatherK>(ob, oc, a, out, n, nt, stream); break;
      default: pick_kc<Tr, OP, kGatherGlobalK>(ob, oc, a, out, n, nt, stream); break;
    }
  }
}

template <class Tr, EwOp OP>
hipError_t launch_ew(int64_t n, const BcastOperand& a, const BcastOperand& b,
                     const BcastOperand& c, void* out, hipStream_t stream) {
  using S = typename Tr::S;
  constexpr int V = Tr::kVec;
  bool vec_ok = ((reinterpret_cast<uintptr_t>(a.data) |
                  reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  constexpr int kArity = arity<OP>();
  Operand ob = kArity >= 2 ? make_operand(b, sizeof(S), V, &vec_ok)
                           : make_operand(a, sizeof(S), V, &vec_ok);
  Operand oc = kArity >= 3 ? make_operand(c, sizeof(S), V, &vec_ok)
                           : make_operand(a, sizeof(S), V, &vec_ok);
  const uint32_t n32 = static_cast<uint32_t>(n);
  int64_t full_in = n * static_cast<int64_t>(sizeof(S));  // a
  if (kArity >= 2 && b.mode == BcastMode::kFull) full_in += n * static_cast<int64_t>(sizeof(S));
  if (kArity >= 3 && c.mode == BcastMode::kFull) full_in += n * static_cast<int64_t>(sizeof(S));
  // Too few vectors for a staging kernel's prologue: walk such operands in
  // global memory instead.
  if (n / V < static_cast<int64_t>(kThreads) * kStagedPre) {
    if (staged_kind(ob.kind)) ob.kind = kGatherGlobalK;
    if (staged_kind(oc.kind)) oc.kind = kGatherGlobalK;
  }
  if (vec_ok) {
    pick_kb<Tr, OP>(ob, oc, static_cast<const S*>(a.data), static_cast<S*>(out), n32,
                    stream_mode(n * static_cast<int64_t>(sizeof(S)), full_in), stream);
  } else {
    // Re-classify for V = 1 (rows and channels become per-element gathers).
    bool dummy = true;
    ob = kArity >= 2 ? make_operand(b, sizeof(S), 1, &dummy)
                     : make_operand(a, sizeof(S), 1, &dummy);
    oc = kArity >= 3 ? make_operand(c, sizeof(S), 1, &dummy)
                     : make_operand(a, sizeof(S), 1, &dummy);
    constexpr int U = 4;
    TFMA_LAUNCH(op_kernel_name(OP), (ew_flat_kernel<Tr, OP, 1, U, kAnyK, kAnyK, 0>), dim3(grid_for(n, U)),
                       dim3(kThreads), 0, stream, static_cast<const S*>(a.data),
                       ob, oc, static_cast<S*>(out), n32);
  }
  return hipGetLastError();
}

template <class Tr, EwOp OP>
hipError_t launch_ew_strided(int64_t n, const void* a, const void* b,
                             const void* c, const StridedShape& sh, void* out,
                             hipStream_t stream) {
  using S = typename Tr::S;
  TFMA_LAUNCH("tfma_ew_strided", (ew_strided_kernel<Tr, OP>), dim3(grid_for(n, 4)),
                     dim3(kThreads), 0, stream, static_cast<const S*>(a),
                     static_cast<const S*>(b), static_cast<const S*>(c), sh,
                     static_cast<S*>(out), n);
  return hipGetLastError();
}

// Integer types take add and multiply only (the stock ops registered for
// them); the other ops are not instantiated for them.
template <class Tr>
hipError_t dispatch_op(EwOp op, int64_t n, const BcastOperand& a,
                       const BcastOperand& b, const BcastOperand& c, void* out,
                       hipStream_t stream) {
  if constexpr (IsIntTraits<Tr>::value) {
    if (op == EwOp::kAdd) return launch_ew<Tr, EwOp::kAdd>(n, a, b, c, out, stream);
    if (op == EwOp::kMul) return launch_ew<Tr, EwOp::kMul>(n, a, b, c, out, stream);
  } else {
    switch (op) {
      case EwOp::kAdd: return launch_ew<Tr, EwOp::kAdd>(n, a, b, c, out, stream);
      case EwOp::kAddRelu: return launch_ew<Tr, EwOp::kAddRelu>(n, a, b, c, out, stream);
      case EwOp::kMul: return launch_ew<Tr, EwOp::kMul>(n, a, b, c, out, stream);
      case EwOp::kMulAdd: return launch_ew<Tr, EwOp::kMulAdd>(n, a, b, c, out, stream);
      case EwOp::kRelu: return launch_ew<Tr, EwOp::kRelu>(n, a, b, c, out, stream);
      case EwOp::kReluGrad: return launch_ew<Tr, EwOp::kReluGrad>(n, a, b, c, out, stream);
    }
  }
  return hipErrorInvalidValue;
}

template <class Tr>
hipError_t dispatch_strided(EwOp op, int64_t n, const void* a, const void* b,
                            const void* c, const StridedShape& sh, void* out,
                            hipStream_t stream) {
  if constexpr (IsIntTraits<Tr>::value) {
    if (op == EwOp::kAdd) return launch_ew_strided<Tr, EwOp::kAdd>(n, a, b, c, sh, out, stream);
    if (op == EwOp::kMul) return launch_ew_strided<Tr, EwOp::kMul>(n, a, b, c, sh, out, stream);
  } else {
    switch (op) {
      case EwOp::kAdd: return launch_ew_strided<Tr, EwOp::kAdd>(n, a, b, c, sh, out, stream);
      case EwOp::kAddRelu:
        return launch_ew_strided<Tr, EwOp::kAddRelu>(n, a, b, c, sh, out, stream);
      case EwOp::kMul: return launch_ew_strided<Tr, EwOp::kMul>(n, a, b, c, sh, out, stream);
      case EwOp::kMulAdd:
        return launch_ew_strided<Tr, EwOp::kMulAdd>(n, a, b, c, sh, out, stream);
      case EwOp::kRelu: return launch_ew_strided<Tr, EwOp::kRelu>(n, a, b, c, sh, out, stream);
      case EwOp::kReluGrad:
        return launch_ew_strided<Tr, EwOp::kReluGrad>(n, a, b, c, sh, out, stream);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace

namespace {

constexpr int64_t kMaxFlat = (int64_t(1) << 31) - 1;  // flat indices stay 32-bit

int64_t gcd64(int64_t x, int64_t y) {
  while (y) {
    const int64_t r = x % y;
    x = y;
    y = r;
  }
  return x;
}

// Chunk length for n > kMaxFlat: a multiple of 16 elements (16-byte aligned
// chunk starts for every dtype) and of each periodic operand's cycle, so
// every chunk starts at broadcast phase 0; 0 when no such chunk fits.
int64_t flat_chunk(const BcastOperand* ops) {
  int64_t cycle = 16;
  for (int i = 0; i < 3; ++i) {
    if (ops[i].mode != BcastMode::kPeriodic) continue;
    const int64_t len = ops[i].inner * ops[i].period;
    if (len <= 0 || len > kMaxFlat) return 0;
    cycle = cycle / gcd64(cycle, len) * len;
    if (cycle > kMaxFlat) return 0;
  }
  return kMaxFlat / cycle * cycle;
}

BcastOperand shifted(const BcastOperand& o, int64_t off, int esize) {
  BcastOperand r = o;
  if (o.mode == BcastMode::kFull) r.data = static_cast<const char*>(o.data) + off * esize;
  return r;
}

hipError_t dispatch_flat(DType t, EwOp op, int64_t n, const BcastOperand& a,
                         const BcastOperand& b, const BcastOperand& c, void* out,
                         hipStream_t stream) {
  switch (t) {
    case DType::kF32: return dispatch_op<TF32>(op, n, a, b, c, out, stream);
    case DType::kF16: return dispatch_op<TF16>(op, n, a, b, c, out, stream);
    case DType::kBF16: return dispatch_op<TBF16>(op, n, a, b, c, out, stream);
    case DType::kF64: return dispatch_op<TF64>(op, n, a, b, c, out, stream);
    case DType::kI32: return dispatch_op<TI32>(op, n, a, b, c, out, stream);
    case DType::kI64: return dispatch_op<TI64>(op, n, a, b, c, out, stream);
    case DType::kU8: return dispatch_op<TU8>(op, n, a, b, c, out, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace

bool ElementwiseFlatOk(int64_t n, const BcastOperand& a, const BcastOperand& b,
                       const BcastOperand& c) {
  if (n <= kMaxFlat) return true;
  const BcastOperand ops[3] = {a, b, c};
  return flat_chunk(ops) > 0;
}

hipError_t LaunchElementwise(DType t, EwOp op, int64_t n,
                             const BcastOperand& a, const BcastOperand& b,
                             const BcastOperand& c, void* out,
                             hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  if (n <= kMaxFlat) return dispatch_flat(t, op, n, a, b, c, out, stream);
  const BcastOperand ops[3] = {a, b, c};
  const int64_t chunk = flat_chunk(ops);
  if (chunk <= 0) return hipErrorInvalidValue;
  const int esize = DTypeBytes(t);
  for (int64_t off = 0; off < n; off += chunk) {
    const int64_t len = n - off < chunk ? n - off : chunk;
    const hipError_t e =
        dispatch_flat(t, op, len, shifted(a, off, esize), shifted(b, off, esize),
                      shifted(c, off, esize), static_cast<char*>(out) + off * esize, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t LaunchElementwiseStrided(DType t, EwOp op, int64_t n,
                                    const void* a, const void* b,
                                    const void* c, const StridedShape& shape,
                                    void* out, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  switch (t) {
    case DType::kF32: return dispatch_strided<TF32>(op, n, a, b, c, shape, out, stream);
    case DType::kF16: return dispatch_strided<TF16>(op, n, a, b, c, shape, out, stream);
    case DType::kBF16: return dispatch_strided<TBF16>(op, n, a, b, c, shape, out, stream);
    case DType::kF64: return dispatch_strided<TF64>(op, n, a, b, c, shape, out, stream);
    case DType::kI32: return dispatch_strided<TI32>(op, n, a, b, c, shape, out, stream);
    case DType::kI64: return dispatch_strided<TI64>(op, n, a, b, c, shape, out, stream);
    case DType::kU8: return dispatch_strided<TU8>(op, n, a, b, c, shape, out, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace tfma
