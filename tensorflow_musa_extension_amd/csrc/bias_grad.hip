// BiasAddGrad for gfx950: the per-channel sum of out_backprop over every
// dimension but the channel one (reference op:
// musa_ext/kernels/nn/musa_biasadd_grad_op.cc:24-110, channel dimension
// :31-40; TF-CPU semantics: half and bfloat16 accumulate in float, float in
// float, double in double, int32/int64 wrap).
//
// x is viewed as [outer, C, inner]: inner = 1 for NHWC (and any rank with the
// channel last), inner = H*W... for NCHW.
//   stage 1, inner == 1 ("rows"): workgroup (g, tile) sums a range of rows for
//            a tile of channel vectors - lanes along 16-byte channel vectors,
//            so a wave reads whole row segments - then the rows of the
//            workgroup through LDS; one partial per (g, channel).
//   stage 1, inner > 1 ("planes"): workgroup (g, channel) sums the channel's
//            planes of a range of images; one partial per (g, channel).
//   stage 2: per channel, the partials in group order, cast to T.
// Every sum runs in a fixed order, so results are deterministic.  Memory:
// one read of x (s*E bytes), partials of G*C accumulators.
#include <mutex>
#include <type_traits>

#include "device_util.h"
#include "tfma_internal.h"

namespace tfma {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 8;

// Per dtype: storage type S, accumulator A, the widening load and the
// final conversion back to S.
template <typename TS, typename TA>
struct Plain {
  using S = TS;
  using A = TA;
  __device__ static A ld(S s) { return static_cast<A>(s); }
  __device__ static S out(A a) { return static_cast<S>(a); }
};
using BagF32 = Plain<float, float>;
using BagF64 = Plain<double, double>;
using BagI32 = Plain<int32_t, uint32_t>;  // wraps modulo 2^32 like TF's int32 sum
using BagI64 = Plain<int64_t, uint64_t>;
template <class Tr>
struct Narrow {  // half / bfloat16, accumulated in float
  using S = uint16_t;
  using A = float;
  __device__ static A ld(S s) { return Tr::ld(s); }
  __device__ static S out(A a) { return Tr::st(a); }
};
using BagF16 = Narrow<TF16>;
using BagBF16 = Narrow<TBF16>;

// The one-launch form (kTag): a 1-D grid of ct * groups reducing workgroups
// (workgroup b: tile b % ct, group b / ct) followed by the finalizing ones;
// partials are stored as epoch-tagged words (TagArgs).  Otherwise a 2-D grid
// (tile, group) writing plain partials for bag_finalize_kernel.
struct TagArgs {
  unsigned long long* slots;  // [groups][c] {partial bits, epoch}
  unsigned epoch;
  int ct;                     // tiles (rows) or channels (planes) per group
  int64_t groups;
  unsigned spin_limit;
};

// Tagged partial words: {value bits (low 32), epoch (high 32)}, written and
// read with relaxed agent-scope atomics (coherent across the XCDs' L2s; one
// single-copy-atomic word, so a word validates itself).  Float accumulators
// only (f32, f16, bf16).
__device__ inline uint32_t acc_bits(float v) { return __builtin_bit_cast(uint32_t, v); }
__device__ inline float acc_from(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ inline void store_tagged(const TagArgs& tg, int64_t slot, float v) {
  __hip_atomic_store(tg.slots + slot,
                     (static_cast<unsigned long long>(tg.epoch) << 32) | acc_bits(v),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LDS bytes of bag_rows_kernel's reduction: ry rows of lanes * (VEC + 1)
// accumulators (VEC for VEC = 1), i.e. kThreads * stride.
inline size_t bag_rows_smem(int vec, size_t acc_bytes) {
  return static_cast<size_t>(kThreads) * (vec > 1 ? vec + 1 : 1) * acc_bytes;
}

template <class B, int VEC, bool kTag = false>
__global__ __launch_bounds__(kThreads) void bag_rows_kernel(
    const typename B::S* __restrict__ x, int64_t rows, int c, int64_t cv, int tx_shift,
    int64_t rows_per_g, typename B::A* __restrict__ partial, TagArgs tg,
    typename B::S* __restrict__ out);

template <class B, bool kTag>
__device__ void bag_finalize_block(const typename B::A* __restrict__ partial, int64_t groups,
                                   int c, int fb, typename B::S* __restrict__ out,
                                   const TagArgs& tg);

template <class B, int VEC, bool kTag>
__global__ __launch_bounds__(kThreads) void bag_rows_kernel(
    const typename B::S* __restrict__ x, int64_t rows, int c, int64_t cv, int tx_shift,
    int64_t rows_per_g, typename B::A* __restrict__ partial, TagArgs tg,
    typename B::S* __restrict__ out) {
  using S = typename B::S;
  using A = typename B::A;
  extern __shared__ unsigned char bag_lds[];
  A* red = reinterpret_cast<A*>(bag_lds);  // [ry][lanes * (VEC + 1)] (bag_rows_smem)
  int64_t bx = blockIdx.x, by = blockIdx.y;
  if constexpr (kTag) {
    const int64_t b = blockIdx.x;
    if (b >= tg.ct * tg.groups) {
      bag_finalize_block<B, true>(nullptr, tg.groups, c, static_cast<int>(b - tg.ct * tg.groups),
                                  out, tg);
      return;
    }
    bx = b % tg.ct;
    by = b / tg.ct;
  }
  const int tx = threadIdx.x & ((1 << tx_shift) - 1);
  const int ty = threadIdx.x >> tx_shift;
  const int ry = kThreads >> tx_shift;
  const int width = (1 << tx_shift) * VEC;
  // Channel tiles vary fastest across workgroups, so the workgroups running
  // together read adjacent segments of the same rows instead of one column
  // of many rows (which concentrates on few memory channels).
  const int64_t cvi = bx * (1 << tx_shift) + tx;
  const int64_t r0 = by * rows_per_g;
  int64_t r1 = r0 + rows_per_g;
  if (r1 > rows) r1 = rows;
  A acc[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) acc[j] = A(0);
  if (cvi < cv) {
    const S* __restrict__ p = x + cvi * VEC;
    int64_t r = r0 + ty;
    // Whole batches of kUnroll rows.  For 2-byte types software-pipelined:
    // the next batch's loads are issued before the current batch is summed,
    // so a thread keeps up to 2 * kUnroll loads in flight instead of
    // draining to zero at every batch (measured at [8192,4096] f16: 56.8 ->
    // 58.5 % of 8 TB/s kernel time; f32, whose 1024 workgroups - 4 per CU -
    // already keep more loads in flight, 66.0 -> 65.5, so it keeps the plain
    // loop).  The rows
    // are summed in the same order either way (bitwise the same sums).
    const int64_t step = static_cast<int64_t>(kUnroll) * ry;
    const int64_t nb =
        sizeof(S) == 2 && r < r1 ? (r1 - r + ry - 1) / ry / kUnroll : 0;
    auto load = [&](S (&v)[kUnroll][VEC], int64_t rr) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) vload_nt<S, VEC>(p + (rr + u * ry) * c, v[u]);
    };
    auto sum = [&](const S (&v)[kUnroll][VEC]) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[j] += B::ld(v[u][j]);
    };
    if (nb > 0) {
      S va[kUnroll][VEC], vb[kUnroll][VEC];
      load(va, r);
      int64_t b = 0;
      for (; b + 2 < nb; b += 2) {  // batches b + 1 and b + 2 exist
        load(vb, r + step);
        sum(va);
        load(va, r + 2 * step);
        sum(vb);
        r += 2 * step;
      }
      if (b + 1 < nb) {
        load(vb, r + step);
        sum(va);
        sum(vb);
        r += 2 * step;
      } else {
        sum(va);
        r += step;
      }
    }
    for (; r + (kUnroll - 1) * ry < r1; r += step) {  // other types: plain batches
      S v[kUnroll][VEC];
      load(v, r);
      sum(v);
    }
    for (; r < r1; r += ry) {
      S v[VEC];
      vload_nt<S, VEC>(p + r * c, v);
#pragma unroll
      for (int j = 0; j < VEC; ++j) acc[j] += B::ld(v[j]);
    }
  }
  // The row lanes' sums through LDS, a lane's VEC channels at a stride of
  // VEC + 1 words (odd for VEC > 1): the writes of one channel slot from
  // consecutive lanes, and the reads of consecutive channels, fall on
  // distinct banks (a stride of VEC made the writes 8-way conflicts for
  // half: 3.4 conflicts per access).  Row ty starts at ty * row_words.
  constexpr int kStride = VEC > 1 ? VEC + 1 : 1;
  const int row_words = (1 << tx_shift) * kStride;
#pragma unroll
  for (int j = 0; j < VEC; ++j) red[ty * row_words + tx * kStride + j] = acc[j];
  __syncthreads();
  const int64_t ch = bx * width + threadIdx.x;
  if (static_cast<int>(threadIdx.x) < width && ch < c) {
    const int slot = static_cast<int>(threadIdx.x) / VEC * kStride + static_cast<int>(threadIdx.x) % VEC;
    A s = A(0);
    for (int k = 0; k < ry; ++k) s += red[k * row_words + slot];
    if constexpr (kTag)
      store_tagged(tg, by * c + ch, s);
    else
      partial[by * c + ch] = s;
  }
}

// VEC > 1 when every plane is a whole number of aligned 16-byte vectors
// (inner % VEC == 0 and x aligned): `inner` and the flat index then count
// vectors.
template <class B, int VEC, bool kTag = false>
__global__ __launch_bounds__(kThreads) void bag_planes_kernel(
    const typename B::S* __restrict__ x, int64_t outer, int c, int64_t inner,
    int64_t outer_per_g, FastDiv div_inner, typename B::A* __restrict__ partial,
    TagArgs tg, typename B::S* __restrict__ out) {
  using S = typename B::S;
  using A = typename B::A;
  __shared__ A red[kThreads / 64];
  int64_t bx = blockIdx.x, by = blockIdx.y;
  if constexpr (kTag) {
    const int64_t b = blockIdx.x;
    if (b >= tg.ct * tg.groups) {
      bag_finalize_block<B, true>(nullptr, tg.groups, c, static_cast<int>(b - tg.ct * tg.groups),
                                  out, tg);
      return;
    }
    bx = b % tg.ct;
    by = b / tg.ct;
  }
  const int ch = static_cast<int>(bx);
  const int64_t o0 = by * outer_per_g;
  int64_t o1 = o0 + outer_per_g;
  if (o1 > outer) o1 = outer;
  const int64_t count = (o1 - o0) * inner;  // < 2^31 (checked by the host)
  A acc = A(0);
  constexpr int U = VEC > 1 ? 4 : 8;
  auto at = [&](int64_t k, S (&v)[VEC]) {
    const uint32_t q = div_inner.div(static_cast<uint32_t>(k));
    const int64_t i = k - static_cast<int64_t>(q) * inner;
    vload_nt<S, VEC>(x + (((o0 + q) * c + ch) * inner + i) * VEC, v);
  };
  int64_t k = threadIdx.x;
  for (; k + (U - 1) * kThreads < count; k += U * kThreads) {
    S v[U][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u) at(k + u * kThreads, v[u]);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < VEC; ++j) acc += B::ld(v[u][j]);
  }
  for (; k < count; k += kThreads) {
    S v[VEC];
    at(k, v);
#pragma unroll
    for (int j = 0; j < VEC; ++j) acc += B::ld(v[j]);
  }
  // Fixed-order reduction: lanes by shuffle, then the waves in order.
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    A s = A(0);
    for (int w = 0; w < kThreads / 64; ++w) s += red[w];
    if constexpr (kTag)
      store_tagged(tg, by * c + ch, s);
    else
      partial[by * c + ch] = s;
  }
}

// kFinLoads partial loads in flight per lane, each wave reading 64
// consecutive partials of a group.  (One wave per channel, its lanes reading
// one partial each C elements apart, took 4.1 us for 64 groups x 4096
// channels.)
constexpr int kFinLoads = 16;
// The one-launch form's finalizing code polls smaller batches: a poll round
// checks and reloads every word of its batch, so a batch no larger than a
// lane's groups turns around sooner (4 for 2-byte rows, whose 256 reducing
// workgroups give a lane 4 groups at [8192,4096]; 8 for 4-byte rows, 1024
// workgroups).  Measured in-box against 16 (kernel time, % of 8 TB/s, 5
// rounds): f16 57.9 -> 60.1 %, f32 65.3 -> 66.2 %.  The groups are summed
// in the same order whatever the batch.
template <class S>
constexpr int kTagFinLoads = sizeof(S) == 2 ? 4 : 8;

// Workgroup fb finishes channels [64 fb, 64 fb + 64): lane l of wave w sums
// channel 64 fb + l over groups w, w + 4, w + 8, ... in order, then wave 0
// adds the four waves' sums in order - the same additions in the same order
// in both forms, so both give the same bits.  kTag: the partials are the
// epoch-tagged words, polled until every one carries this launch's epoch
// (the reducing workgroups precede this one in dispatch order and wait for
// nothing, so they all run; the spin is bounded all the same, and a partial
// that never arrives is taken as NaN).
template <class B, bool kTag>
__device__ void bag_finalize_block(const typename B::A* __restrict__ partial, int64_t groups,
                                   int c, int fb, typename B::S* __restrict__ out,
                                   const TagArgs& tg) {
  using A = typename B::A;
  constexpr int kWaves = kThreads / 64;
  __shared__ A fred[kWaves][64];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t ch = static_cast<int64_t>(fb) * 64 + lane;
  const bool active = ch < c;
  const int64_t c0 = active ? ch : 0;
  A s = A(0);
  int64_t g = w;
  if constexpr (kTag) {
    const unsigned long long want = static_cast<unsigned long long>(tg.epoch);
    for (; g < groups; g += kTagFinLoads<typename B::S> * kWaves) {
      unsigned long long v[kTagFinLoads<typename B::S>];
#pragma unroll
      for (int u = 0; u < kTagFinLoads<typename B::S>; ++u) {
        const int64_t gg = g + u * kWaves;
        v[u] = gg < groups ? __hip_atomic_load(tg.slots + gg * c + c0, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT)
                           : (want << 32);
      }
      unsigned spins = 0;
      while (true) {
        bool ready = true;
#pragma unroll
        for (int u = 0; u < kTagFinLoads<typename B::S>; ++u) ready = ready && (v[u] >> 32) == want;
        if (ready) break;
        if (++spins > tg.spin_limit) {
#pragma unroll
          for (int u = 0; u < kTagFinLoads<typename B::S>; ++u)
            if ((v[u] >> 32) != want) v[u] = (want << 32) | 0x7fc00000u;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int u = 0; u < kTagFinLoads<typename B::S>; ++u) {
          const int64_t gg = g + u * kWaves;
          if ((v[u] >> 32) != want)
            v[u] = __hip_atomic_load(tg.slots + gg * c + c0, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
        }
      }
#pragma unroll
      for (int u = 0; u < kTagFinLoads<typename B::S>; ++u)
        if (g + u * kWaves < groups) s += acc_from(static_cast<uint32_t>(v[u]));
    }
  } else {
    const A* __restrict__ p = partial + c0;
    for (; g + (kFinLoads - 1) * kWaves < groups; g += kFinLoads * kWaves) {
      A v[kFinLoads];
#pragma unroll
      for (int u = 0; u < kFinLoads; ++u) v[u] = p[(g + u * kWaves) * c];
#pragma unroll
      for (int u = 0; u < kFinLoads; ++u) s += v[u];
    }
    for (; g < groups; g += kWaves) s += p[g * c];
  }
  fred[w][lane] = s;
  __syncthreads();
  if (w == 0 && active) {
    A t = fred[0][lane];
#pragma unroll
    for (int k = 1; k < kWaves; ++k) t += fred[k][lane];
    out[ch] = B::out(t);
  }
}

template <class B>
__global__ __launch_bounds__(kThreads) void bag_finalize_kernel(
    const typename B::A* __restrict__ partial, int64_t groups, int c,
    typename B::S* __restrict__ out) {
  bag_finalize_block<B, false>(partial, groups, c, blockIdx.x, out, TagArgs{});
}

__global__ __launch_bounds__(kThreads) void zero_bytes_kernel(uint8_t* __restrict__ p, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kThreads)
    p[i] = 0;
}

struct BagPlan {
  bool rows;         // inner == 1
  int vec;
  int64_t cv;
  int tx_shift;
  int ct;
  int64_t per_g;     // rows (or images) per group
  int64_t groups;
};

// Reducing workgroups aimed for: 1024, and 256 for the rows form with 2-byte
// elements - longer-lived workgroups and a quarter of the partials.
// Measured in one launch at [8192,4096] (kernel time, % of 8 TB/s): f16 53.5
// -> 56.8 % with 256 (1024: 53.5, 512: 55.6); f32 unchanged within noise
// (256: 63.7, 512: 66.1, 1024: 65.5-66.5, 2048: 65.7-67.3).
constexpr int64_t kTargetBlocks = 1024;
constexpr int64_t kTargetBlocksRows16 = 256;

BagPlan make_bag_plan(int64_t outer, int64_t c, int64_t inner, int esize, bool aligned) {
  BagPlan p{};
  p.rows = inner == 1;
  if (p.rows) {
    const int kv = 16 / esize;
    p.vec = (aligned && c % kv == 0) ? kv : 1;
    p.cv = c / p.vec;
    int s = 0;
    while ((int64_t(1) << s) < p.cv && s < 5) ++s;  // at most 32 lanes along channels
    p.tx_shift = s;
    const int ry = kThreads >> s;
    p.ct = static_cast<int>((p.cv + (1 << s) - 1) >> s);
    int64_t gt = (esize == 2 ? kTargetBlocksRows16 : kTargetBlocks) / p.ct;
    if (gt < 1) gt = 1;
    int64_t rpg = (outer + gt - 1) / gt;
    const int64_t min_rows = static_cast<int64_t>(ry) * kUnroll;
    if (rpg < min_rows) rpg = min_rows;
    p.per_g = rpg;
    p.groups = (outer + rpg - 1) / rpg;
  } else {
    const int kv = 16 / esize;
    p.vec = (aligned && inner % kv == 0) ? kv : 1;
    int64_t gt = kTargetBlocks / c;
    if (gt < 1) gt = 1;
    int64_t opg = (outer + gt - 1) / gt;
    const int64_t min_imgs = (static_cast<int64_t>(kThreads) * 8 * p.vec + inner - 1) / inner;
    if (opg < min_imgs) opg = min_imgs;
    // The flat index within a group stays below 2^31.
    const int64_t max_imgs = ((int64_t(1) << 31) - 1) / inner;
    if (opg > max_imgs) opg = max_imgs;
    if (opg < 1) opg = 1;
    p.per_g = opg;
    p.groups = (outer + opg - 1) / opg;
  }
  if (p.groups < 1) p.groups = 1;
  return p;
}

// ---- one launch: tagged partials and trailing finalizing workgroups ------
// Per device: the tagged partial slots (library-owned, zeroed once), the
// last epoch, and the end event and stream of the last launch.  Launches on
// one device are chained (one on another stream than the previous waits for
// its end), so two launches never share the slots at once; eager epochs stay
// below 2^31 and the slots are zeroed again at the wrap.
constexpr size_t kTagSlots = size_t(1) << 19;  // 4 MiB of tagged partials
constexpr unsigned kTagSpinLimit = 1u << 20;
struct TagState {
  std::mutex mu;
  unsigned long long* slots = nullptr;
  unsigned epoch = 0;
  LaunchChain chain;
};

TagState* tag_state() {
  static TagState states[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  return &states[dev];
}

// Whether the one-launch form applies: float accumulators (f32, f16, bf16),
// an eager launch (under stream capture the graph would keep this launch's
// epoch), partials that fit the slots, and not switched off (override
// "bag_fused" 0).
template <class B>
bool tag_applies(const BagPlan& p, int64_t c, hipStream_t stream) {
  if constexpr (!std::is_same<typename B::A, float>::value) {
    return false;
  } else {
    if (TuneValue(kTuneBagFused) == 0) return false;
    if (static_cast<size_t>(p.groups) * static_cast<size_t>(c) > kTagSlots) return false;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess) return false;
    return cap == hipStreamCaptureStatusNone;
  }
}

// One launch: ct * groups (rows) or c * groups (planes) reducing workgroups,
// then ceil(c / 64) finalizing ones; same plan, partials and summation order
// as the two-kernel form, so the same bits.  The finalizers come last in the
// 1-D grid, so they are dispatched after every reducing workgroup.
template <class B>
hipError_t launch_bag_tagged(const BagPlan& p, const void* x, int64_t outer, int64_t c,
                             int64_t inner, void* out, hipStream_t stream) {
  using S = typename B::S;
  TagState* ts = tag_state();
  if (!ts) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(ts->mu);
  hipError_t e;
  if (!ts->slots) {
    void* q = nullptr;
    e = hipMalloc(&q, kTagSlots * sizeof(unsigned long long));
    if (e != hipSuccess) return e;
    e = hipMemset(q, 0, kTagSlots * sizeof(unsigned long long));
    if (e != hipSuccess) {
      (void)hipFree(q);
      return e;
    }
    ts->slots = static_cast<unsigned long long*>(q);
  }
  e = ts->chain.before(stream);
  if (e != hipSuccess) return e;
  if (ts->epoch + 1 >= (1u << 31)) {  // after the wait above: no launch still reads them
    e = hipMemsetAsync(ts->slots, 0, kTagSlots * sizeof(unsigned long long), stream);
    if (e != hipSuccess) return e;
    ts->epoch = 0;
  }
  TagArgs tg;
  tg.slots = ts->slots;
  tg.epoch = ++ts->epoch;
  tg.groups = p.groups;
  tg.spin_limit = kTagSpinLimit;
  const int64_t fin = (c + 63) / 64;
  const S* xs = static_cast<const S*>(x);
  S* o = static_cast<S*>(out);
  constexpr const char* kName = "tfma_bias_add_grad_fused";
  SetLastKernel(kName);
  const TraceEvents tev = TraceTake(kName);
  hipEvent_t end = ts->chain.end_event(tev.end);
  constexpr int V = 16 / sizeof(S);
  if (p.rows) {
    tg.ct = p.ct;
    const dim3 grid(static_cast<unsigned>(p.ct * p.groups + fin));
    const size_t smem = bag_rows_smem(p.vec, sizeof(float));
    if (p.vec == V)
      hipExtLaunchKernelGGL((bag_rows_kernel<B, V, true>), grid, dim3(kThreads), smem, stream,
                            tev.start, end, 0, xs, outer, static_cast<int>(c), p.cv, p.tx_shift,
                            p.per_g, static_cast<float*>(nullptr), tg, o);
    else
      hipExtLaunchKernelGGL((bag_rows_kernel<B, 1, true>), grid, dim3(kThreads), smem, stream,
                            tev.start, end, 0, xs, outer, static_cast<int>(c), p.cv, p.tx_shift,
                            p.per_g, static_cast<float*>(nullptr), tg, o);
  } else {
    tg.ct = static_cast<int>(c);
    const dim3 grid(static_cast<unsigned>(c * p.groups + fin));
    if (p.vec > 1) {
      const int64_t iv = inner / V;
      hipExtLaunchKernelGGL((bag_planes_kernel<B, V, true>), grid, dim3(kThreads), 0, stream,
                            tev.start, end, 0, xs, outer, static_cast<int>(c), iv, p.per_g,
                            FastDiv(static_cast<uint32_t>(iv)), static_cast<float*>(nullptr), tg,
                            o);
    } else {
      hipExtLaunchKernelGGL((bag_planes_kernel<B, 1, true>), grid, dim3(kThreads), 0, stream,
                            tev.start, end, 0, xs, outer, static_cast<int>(c), inner, p.per_g,
                            FastDiv(static_cast<uint32_t>(inner)), static_cast<float*>(nullptr),
                            tg, o);
    }
  }
  TraceCommit(tev);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  ts->chain.after(stream, end);
  return hipSuccess;
}

// chain_end (the allocation-free path): in, the event the finalize dispatch
// ends with, or null for none (hipExtLaunchKernelGGL's own stop event: no
// marker packet between kernels); out, the event that marks its end (a trace
// event instead when tracing is on for the finalize kernel).
template <class B>
hipError_t launch_bag(const void* x, int64_t outer, int64_t c, int64_t inner, void* out,
                      void* workspace, hipStream_t stream, hipEvent_t* chain_end = nullptr) {
  using S = typename B::S;
  using A = typename B::A;
  const bool aligned = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  const BagPlan p = make_bag_plan(outer, c, inner, sizeof(S), aligned);
  if constexpr (std::is_same<A, float>::value) {
    if (!chain_end && tag_applies<B>(p, c, stream))
      return launch_bag_tagged<B>(p, x, outer, c, inner, out, stream);
  }
  A* partial = static_cast<A*>(workspace);
  const S* xs = static_cast<const S*>(x);
  {
    if (p.rows) {
      const size_t smem = bag_rows_smem(p.vec, sizeof(A));
      constexpr int V = 16 / sizeof(S);
      if (p.vec == V) {
        TFMA_LAUNCH("tfma_bias_add_grad_reduce", (bag_rows_kernel<B, V>), dim3(p.ct, p.groups), dim3(kThreads), smem,
                           stream, xs, outer, static_cast<int>(c), p.cv, p.tx_shift, p.per_g,
                           partial, TagArgs{}, static_cast<S*>(nullptr));
      } else {
        TFMA_LAUNCH("tfma_bias_add_grad_reduce", (bag_rows_kernel<B, 1>), dim3(p.ct, p.groups), dim3(kThreads), smem,
                           stream, xs, outer, static_cast<int>(c), p.cv, p.tx_shift, p.per_g,
                           partial, TagArgs{}, static_cast<S*>(nullptr));
      }
    } else if (p.vec > 1) {
      constexpr int V = 16 / sizeof(S);
      const int64_t iv = inner / V;
      TFMA_LAUNCH("tfma_bias_add_grad_reduce", (bag_planes_kernel<B, V>), dim3(c, p.groups), dim3(kThreads), 0, stream,
                         xs, outer, static_cast<int>(c), iv, p.per_g,
                         FastDiv(static_cast<uint32_t>(iv)), partial, TagArgs{},
                         static_cast<S*>(nullptr));
    } else {
      TFMA_LAUNCH("tfma_bias_add_grad_reduce", (bag_planes_kernel<B, 1>), dim3(c, p.groups), dim3(kThreads), 0, stream,
                         xs, outer, static_cast<int>(c), inner, p.per_g,
                         FastDiv(static_cast<uint32_t>(inner)), partial, TagArgs{},
                         static_cast<S*>(nullptr));
    }
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  constexpr const char* kFinalize = "tfma_bias_add_grad_finalize";
  if (!chain_end) {
    TFMA_LAUNCH(kFinalize, (bag_finalize_kernel<B>), dim3((c + 63) / 64), dim3(kThreads), 0,
                stream, partial, p.groups, static_cast<int>(c), static_cast<S*>(out));
    return hipGetLastError();
  }
  SetLastKernel(kFinalize);
  const TraceEvents tev = TraceTake(kFinalize);
  hipEvent_t end = tev.end ? tev.end : *chain_end;  // may be null: no end event
  hipExtLaunchKernelGGL((bag_finalize_kernel<B>), dim3((c + 63) / 64), dim3(kThreads), 0, stream,
                        tev.start, end, 0, partial, p.groups, static_cast<int>(c),
                        static_cast<S*>(out));
  TraceCommit(tev);
  *chain_end = end;
  return hipGetLastError();
}

size_t acc_bytes(int dt) {
  return (dt == TFMA_DOUBLE || dt == TFMA_INT64) ? 8 : 4;
}

// Scratch of the allocation-free BiasAddGrad: the per-group partials live in
// this file-scope array instead of a caller workspace.  Each device holds its
// own copy for the life of the process.  In host code `bag_scratch` names a
// host-side stand-in, not device memory: kernels get the device address that
// hipGetSymbolAddress returns for the current device (BiasAddGradScratch).
static __device__ __align__(256) unsigned char bag_scratch[kBiasAddGradScratchBytes];

}  // namespace

hipError_t BiasAddGradScratch(void** ptr) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* addr[kMaxDevices] = {nullptr};
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(bag_scratch));
    if (e != hipSuccess) return e;
    addr[dev] = p;
  }
  *ptr = addr[dev];
  return hipSuccess;
}

size_t BiasAddGradWorkspaceBytes(int dt, int64_t outer, int64_t c, int64_t inner, int esize) {
  const BagPlan p = make_bag_plan(outer, c, inner, esize, true);
  const BagPlan q = make_bag_plan(outer, c, inner, esize, false);
  const int64_t g = p.groups > q.groups ? p.groups : q.groups;
  return (static_cast<size_t>(g) * c * acc_bytes(dt) + 255) & ~size_t(255);
}

namespace {
hipError_t dispatch_bag(int dt, const void* x, int64_t outer, int64_t c, int64_t inner,
                        void* out, void* ws, hipStream_t stream, hipEvent_t* chain_end) {
  switch (dt) {
    case TFMA_FLOAT: return launch_bag<BagF32>(x, outer, c, inner, out, ws, stream, chain_end);
    case TFMA_HALF: return launch_bag<BagF16>(x, outer, c, inner, out, ws, stream, chain_end);
    case TFMA_BFLOAT16:
      return launch_bag<BagBF16>(x, outer, c, inner, out, ws, stream, chain_end);
    case TFMA_DOUBLE: return launch_bag<BagF64>(x, outer, c, inner, out, ws, stream, chain_end);
    case TFMA_INT32: return launch_bag<BagI32>(x, outer, c, inner, out, ws, stream, chain_end);
    case TFMA_INT64: return launch_bag<BagI64>(x, outer, c, inner, out, ws, stream, chain_end);
  }
  return hipErrorInvalidValue;
}

// Per device: the allocation-free calls share one scratch, so a call on
// another stream than the previous call's first waits for that call's
// finalize to end (LaunchChain); calls on one stream are ordered by the
// stream.  The mutex keeps the wait, the launches and the bookkeeping of one
// call together.
struct NoAllocChain {
  std::mutex mu;
  LaunchChain chain;
};
}  // namespace

hipError_t LaunchBiasAddGrad(int dt, const void* x, int64_t outer, int64_t c, int64_t inner,
                             void* out, void* workspace, hipStream_t stream) {
  return dispatch_bag(dt, x, outer, c, inner, out, workspace, stream, nullptr);
}

hipError_t LaunchBiasAddGradNoAlloc(int dt, const void* x, int64_t outer, int64_t c,
                                    int64_t inner, void* out, hipStream_t stream) {
  void* scratch = nullptr;
  hipError_t e = BiasAddGradScratch(&scratch);
  if (e != hipSuccess) return e;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(stream, &cap);
  if (e != hipSuccess) return e;
  // Under capture the graph orders its nodes; a replay must not overlap
  // other allocation-free BiasAddGrad work on the device.
  if (cap != hipStreamCaptureStatusNone)
    return dispatch_bag(dt, x, outer, c, inner, out, scratch, stream, nullptr);
  int dev = 0;
  e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  static NoAllocChain chains[64];
  NoAllocChain& ch = chains[dev];
  std::lock_guard<std::mutex> lk(ch.mu);
  e = ch.chain.before(stream);
  if (e != hipSuccess) return e;
  hipEvent_t end = ch.chain.end_event(nullptr);
  e = dispatch_bag(dt, x, outer, c, inner, out, scratch, stream, &end);
  if (e != hipSuccess) return e;
  ch.chain.after(stream, end);
  return hipSuccess;
}

namespace {
// Streaming copy for the measured ceiling: 16-byte non-temporal loads and
// stores, four of each in flight per thread, grid-stride.
typedef unsigned u32x4v __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(kThreads) void stream_copy_kernel(const u32x4v* __restrict__ src,
                                                               u32x4v* __restrict__ dst,
                                                               int64_t n) {
  constexpr int U = 4;
  const int64_t nth = static_cast<int64_t>(gridDim.x) * kThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  for (; i + (U - 1) * nth < n; i += U * nth) {
    u32x4v v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(src + i + u * nth);
#pragma unroll
    for (int u = 0; u < U; ++u) __builtin_nontemporal_store(v[u], dst + i + u * nth);
  }
  for (; i < n; i += nth) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}
}  // namespace

hipError_t LaunchStreamCopy(void* dst, const void* src, int64_t bytes, hipStream_t stream) {
  if (bytes <= 0) return hipSuccess;
  const int64_t n = bytes / 16;
  // One workgroup per CU: measured (Infinity Cache flushed, read + write
  // bytes) 6.0-6.3 TB/s at 128 MiB-1 GiB and 5.5 TB/s at 8 GiB, against
  // 5.4-5.8 / 5.1 with 2 per CU and 4.3-4.9 / 4.9 with 8 per CU.
  int64_t blocks = DeviceCUs();
  const int64_t need = (n + kThreads - 1) / kThreads;
  if (blocks > need) blocks = need;
  TFMA_LAUNCH("tfma_stream_copy", stream_copy_kernel, dim3(blocks), dim3(kThreads), 0, stream,
              static_cast<const u32x4v*>(src), static_cast<u32x4v*>(dst), n);
  return hipGetLastError();
}

hipError_t LaunchZeroBytes(void* p, int64_t n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  int64_t blocks = (n + kThreads - 1) / kThreads;
  if (blocks > 1024) blocks = 1024;
  TFMA_LAUNCH("tfma_zero_bytes", zero_bytes_kernel, dim3(blocks), dim3(kThreads), 0, stream,
                     static_cast<uint8_t*>(p), n);
  return hipGetLastError();
}

}  // namespace tfma
