// FusedBatchNormV3 / FusedBatchNormGradV3 kernels for gfx950.
//
// Semantics (TF CPU kernels, which the reference's op reproduces; reference
// conventions at musa_ext/kernels/nn/musa_fused_batchnorm_op.cc:13-15,
// 60-62, 141-170, 265-277):
//   forward, training, per channel c over the n = N*H*W elements:
//     mean = sum(x)/n, var = sum((x-mean)^2)/n  (population variance)
//     y = (x - mean) * (rsqrt(var + eps) * scale) + offset
//     batch_mean = mean, batch_variance = var * n/(n-1)  (Bessel)
//       (blended with the running values when exponential_avg_factor != 1)
//     reserve_space_1 = mean, reserve_space_2 = var, reserve_space_3 = 0
//   grad, training (reserve_space_1/2 = mean / population variance):
//     k = rsqrt(var + eps), xc = x - mean
//     offset_backprop = sum(dy), scale_backprop = k * sum(dy * xc)
//     dx = scale*k * ((dy - sum(dy)/n) - xc * (k*k * sum(dy*xc)/n))
//
// Structure: three kernels per op.
//   1. reduce:   each workgroup owns a row range x channel tile and writes
//                one float2 partial per channel (shifted sums for the
//                forward, sum(dy) / sum(dy*xc) for the grad).  16-byte loads,
//                8 loads in flight per thread, lanes mapped to channel
//                vectors so a wave reads whole 512-byte row segments.
//   2. finalize: per channel, a double-precision sum over the partials;
//                writes the statistics outputs and 4 per-channel
//                coefficients.
//   3. apply:    y (or dx) from x (and dy) and the coefficients.  Row ranges
//                are walked in the reverse of the reduce order, so the
//                lines the reduce touched last - still in the 256 MB
//                Infinity Cache - are re-read first.
// The forward statistics use sums of (x - K) with K = chan_shift(), the
// median of five of the channel's elements, which keeps sum((x-K)^2) -
// sum(x-K)^2/n free of cancellation when |mean| >> std and when single
// elements are outliers; partials add exactly like plain sums because every
// workgroup uses the same K.
#include <hip/hip_ext.h>

#include <atomic>
#include <mutex>

#include "device_util.h"
#include "tfma_internal.h"

namespace tfma {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 8;
constexpr int kFinCh = 8;          // channels per finalize workgroup
constexpr int kFinThreads = 256;   // 32 partial slices x 8 channels

struct Plan {
  bool nhwc;
  int vec;          // elements per thread access
  int64_t cv;       // channel vectors per row (NHWC) / vectors per plane (NCHW)
  int tx_shift;     // log2(threads along channels) (NHWC)
  int ct;           // channel tiles (NHWC) / channels (NCHW)
  int64_t rows_per_g;
  int64_t groups;   // G: row groups (NHWC) / image groups (NCHW)
};

int pow2_ceil_log2(int64_t v) {
  int s = 0;
  while ((int64_t(1) << s) < v) ++s;
  return s;
}

int target_wgs() {
  static int t = [] {
    const char* e = getenv("TFMA_BN_TARGET_WGS");
    int v = e ? atoi(e) : 0;
    return v > 0 ? v : 1024;
  }();
  return t;
}

int vec_of(DType t) { return t == DType::kF32 ? 4 : 8; }
int elem_bytes(DType t) { return t == DType::kF32 ? 4 : 2; }

Plan make_plan(DType t, const BnGeometry& g, bool aligned) {
  Plan p;
  p.nhwc = g.nhwc;
  const int kv = vec_of(t);
  if (g.nhwc) {
    p.vec = (aligned && g.c % kv == 0) ? kv : 1;
    p.cv = g.c / p.vec;
    int s = pow2_ceil_log2(p.cv);
    if (s > 5) s = 5;  // at most 32 lanes along channels
    p.tx_shift = s;
    const int tx = 1 << s;
    const int ry = kThreads / tx;
    p.ct = static_cast<int>((p.cv + tx - 1) / tx);
    int64_t gt = target_wgs() / p.ct;
    if (gt < 1) gt = 1;
    int64_t rpg = (g.rows + gt - 1) / gt;
    const int64_t min_rows = static_cast<int64_t>(ry) * kUnroll;
    if (rpg < min_rows) rpg = min_rows;
    rpg = (rpg + ry - 1) / ry * ry;
    p.rows_per_g = rpg;
    p.groups = (g.rows + rpg - 1) / rpg;
    if (p.groups < 1) p.groups = 1;
  } else {
    const int64_t plane = g.h * g.w;
    p.vec = (aligned && plane % kv == 0) ? kv : 1;
    p.cv = plane / p.vec;
    p.tx_shift = 0;
    p.ct = static_cast<int>(g.c);
    int64_t gt = target_wgs() / g.c;
    if (gt < 1) gt = 1;
    // Images per group: enough vectors per workgroup to keep it busy.
    int64_t ipg = (g.n + gt - 1) / gt;
    const int64_t min_imgs = (kThreads * 4 + p.cv - 1) / p.cv;
    if (ipg < min_imgs) ipg = min_imgs;
    if (ipg > g.n) ipg = g.n;
    if (ipg < 1) ipg = 1;
    p.rows_per_g = ipg;
    p.groups = (g.n + ipg - 1) / ipg;
    if (p.groups < 1) p.groups = 1;
  }
  return p;
}

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

size_t partial_bytes(const Plan& p, const BnGeometry& g) {
  return align256(static_cast<size_t>(p.groups) * g.c * sizeof(float2));
}
size_t coef_bytes(const BnGeometry& g) {
  return align256(static_cast<size_t>(g.c) * sizeof(float4));
}

// ---------------------------------------------------------------------------
// Shift K of the forward's sums of (x - K) and (x - K)^2: the median of five
// elements spread over the channel (its elements 0, n/4, n/2, 3n/4, n-1),
// truncated toward zero to a multiple of a power of two near 1/16 of the
// samples' spread.  The variance sum((x-K)^2) - sum(x-K)^2 / n cancels in
// proportion to ((mean - K) / std)^2, so K must sit near the mean: the
// channel's first element would do unless it is an outlier (one at 1e3 among
// N(0,1) values put the float32 statistics off by 1e-4); the median of five
// stays within a few standard deviations unless three of the five are
// outliers, and the truncation moves it by less than 1/16 of the spread.
// The truncation keeps K on a grid no finer than the data's own: a median
// near zero (|K| ~ 1e-3 among N(0,1) half values) carries bits far below the
// data's quantum, every term x - K then carries those same bits, and the
// float32 running sums round them the same way at every add - a bias that
// put the mean of [256,56,56,256] half data off by 1e-7 (5e-5 of its largest
// value); on the coarse grid the terms add exactly.  A non-finite median
// gives K = 0, so infinities and NaNs reach the sums as in an unshifted sum.
// Every kernel and the finals compute K with these functions from the same
// five elements, so they agree bit for bit.
__device__ inline float coarse_shift(float k, float spread) {
  if (!(spread > 0.f) || !__builtin_isfinite(spread)) return k;
  const int es = static_cast<int>((__builtin_bit_cast(uint32_t, spread) >> 23) & 0xffu);
  uint32_t kb = __builtin_bit_cast(uint32_t, k);
  int ek = static_cast<int>((kb >> 23) & 0xffu);
  if (ek == 0) ek = 1;  // subnormal: same bit weights as exponent field 1
  // Clear the mantissa bits worth less than 2^(es - 4 - 127).
  const int drop = (es - 4) - ek + 23;
  if (drop <= 0) return k;
  if (drop >= 24) return __builtin_bit_cast(float, kb & 0x80000000u);
  kb &= ~((1u << drop) - 1u);
  return __builtin_bit_cast(float, kb);
}
// ---------------------------------------------------------------------------
__device__ inline void cmp_swap(float& lo, float& hi) {
  const float a = fminf(lo, hi), b = fmaxf(lo, hi);
  lo = a;
  hi = b;
}

__device__ inline float shift_of(float (&v)[5]) {
  // Optimal 9-comparator sorting network for five elements.
  cmp_swap(v[0], v[1]);
  cmp_swap(v[3], v[4]);
  cmp_swap(v[2], v[4]);
  cmp_swap(v[2], v[3]);
  cmp_swap(v[0], v[3]);
  cmp_swap(v[0], v[2]);
  cmp_swap(v[1], v[4]);
  cmp_swap(v[1], v[3]);
  cmp_swap(v[1], v[2]);
  return __builtin_isfinite(v[2]) ? coarse_shift(v[2], v[3] - v[1]) : 0.f;
}

// The shifts of the VEC channels of five sample vectors (the fused kernel's
// K).  Same selection as shift_of() per channel.  For half the network runs
// on packed channel pairs (v_pk_min/max_f16, IEEE minNum/maxNum like fminf/
// fmaxf): widening half to float is exact and order-preserving, so the
// median is the same element, and the five samples stay packed in 20
// registers instead of 40 floats - registers the resident rows can use.
template <class Tr>
__device__ inline void shift_words(const uint4 (&kw)[5], float (&k)[Tr::kVec]) {
  using S = typename Tr::S;
#pragma unroll
  for (int j = 0; j < Tr::kVec; ++j) {
    float v[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) {
      S sv[Tr::kVec];
      __builtin_memcpy(sv, &kw[i], 16);
      v[i] = Tr::ld(sv[j]);
    }
    k[j] = shift_of(v);
  }
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ inline void cmp_swap2(half2v& lo, half2v& hi) {
  const half2v a = __builtin_elementwise_min(lo, hi), b = __builtin_elementwise_max(lo, hi);
  lo = a;
  hi = b;
}

template <>
__device__ inline void shift_words<TF16>(const uint4 (&kw)[5], float (&k)[8]) {
  half2v v[5][4];
#pragma unroll
  for (int i = 0; i < 5; ++i) __builtin_memcpy(v[i], &kw[i], 16);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    cmp_swap2(v[0][w], v[1][w]);
    cmp_swap2(v[3][w], v[4][w]);
    cmp_swap2(v[2][w], v[4][w]);
    cmp_swap2(v[2][w], v[3][w]);
    cmp_swap2(v[0][w], v[3][w]);
    cmp_swap2(v[0][w], v[2][w]);
    cmp_swap2(v[1][w], v[4][w]);
    cmp_swap2(v[1][w], v[3][w]);
    cmp_swap2(v[1][w], v[2][w]);
    const float lo = static_cast<float>(v[2][w].x), hi = static_cast<float>(v[2][w].y);
    const float slo = static_cast<float>(v[3][w].x) - static_cast<float>(v[1][w].x);
    const float shi = static_cast<float>(v[3][w].y) - static_cast<float>(v[1][w].y);
    k[2 * w] = __builtin_isfinite(lo) ? coarse_shift(lo, slo) : 0.f;
    k[2 * w + 1] = __builtin_isfinite(hi) ? coarse_shift(hi, shi) : 0.f;
  }
}

// Element j of channel ch: NHWC (hw = 1) at j*c + ch, NCHW at
// (j / hw)*c*hw + ch*hw + j % hw.
__device__ inline int64_t chan_elem(int64_t j, int64_t ch, int64_t c, int64_t hw) {
  return (j / hw) * c * hw + ch * hw + j % hw;
}

__device__ inline void shift_rows(int64_t n, int64_t (&js)[5]) {
  js[0] = 0;
  js[1] = n / 4;
  js[2] = n / 2;
  js[3] = (3 * n) / 4;
  js[4] = n - 1;
}

template <class Tr>
__device__ inline float chan_shift(const typename Tr::S* x, int64_t ch, int64_t n, int64_t c,
                                   int64_t hw) {
  if (n <= 0) return 0.f;
  int64_t js[5];
  shift_rows(n, js);
  float v[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) v[i] = Tr::ld(x[chan_elem(js[i], ch, c, hw)]);
  return shift_of(v);
}

// ---------------------------------------------------------------------------
// 1. Reduce.
// ---------------------------------------------------------------------------
// kGrad = false: s1 += x - K, s2 += (x - K)^2, K = chan_shift() of the channel.
// kGrad = true:  s1 += dy,    s2 += dy * (x - mean).
template <class Tr, int VEC, bool kGrad>
__device__ inline void accum(const typename Tr::S (&xv)[VEC],
                             const typename Tr::S (&dv)[VEC],
                             const float (&k)[VEC], float (&s1)[VEC],
                             float (&s2)[VEC]) {
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    const float xc = Tr::ld(xv[j]) - k[j];
    if constexpr (kGrad) {
      const float d = Tr::ld(dv[j]);
      s1[j] += d;
      s2[j] += d * xc;
    } else {
      s1[j] += xc;
      s2[j] += xc * xc;
    }
  }
}

template <class Tr, int VEC, bool kGrad>
__global__ __launch_bounds__(kThreads) void bn_nhwc_reduce_kernel(
    const typename Tr::S* __restrict__ x, const typename Tr::S* __restrict__ dy,
    const float* __restrict__ mean_in, int64_t rows, int c, int64_t cv,
    int tx_shift, int64_t rows_per_g, float2* __restrict__ partial) {
  using S = typename Tr::S;
  extern __shared__ float2 red[];  // [ry][tx*VEC]
  const int tx = threadIdx.x & ((1 << tx_shift) - 1);
  const int ty = threadIdx.x >> tx_shift;
  const int ry = kThreads >> tx_shift;
  const int width = (1 << tx_shift) * VEC;
  // Channel tiles vary fastest across workgroups (adjacent row segments
  // are read together rather than one column of many rows).
  const int64_t cvi = static_cast<int64_t>(blockIdx.x) * (1 << tx_shift) + tx;
  const int64_t g = blockIdx.y;
  const int64_t r0 = g * rows_per_g;
  int64_t r1 = r0 + rows_per_g;
  if (r1 > rows) r1 = rows;
  float s1[VEC], s2[VEC], k[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) { s1[j] = 0.f; s2[j] = 0.f; }
  if (cvi < cv) {
    const int64_t c0 = cvi * VEC;
    if constexpr (kGrad) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) k[j] = mean_in[c0 + j];
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) k[j] = chan_shift<Tr>(x, c0 + j, rows, c, 1);
    }
    const S* __restrict__ px = x + c0;
    const S* __restrict__ pd = kGrad ? dy + c0 : nullptr;
    int64_t r = r0 + ty;
    for (; r + (kUnroll - 1) * ry < r1; r += kUnroll * ry) {
      S xv[kUnroll][VEC], dv[kUnroll][VEC];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        vload<S, VEC>(px + (r + u * ry) * c, xv[u]);
        if constexpr (kGrad) vload<S, VEC>(pd + (r + u * ry) * c, dv[u]);
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) accum<Tr, VEC, kGrad>(xv[u], dv[u], k, s1, s2);
    }
    for (; r < r1; r += ry) {
      S xv[VEC], dv[VEC];
      vload<S, VEC>(px + r * c, xv);
      if constexpr (kGrad) vload<S, VEC>(pd + r * c, dv);
      accum<Tr, VEC, kGrad>(xv, dv, k, s1, s2);
    }
  }
#pragma unroll
  for (int j = 0; j < VEC; ++j) red[ty * width + tx * VEC + j] = make_float2(s1[j], s2[j]);
  __syncthreads();
  const int64_t cbase = static_cast<int64_t>(blockIdx.x) * width;
  for (int cl = threadIdx.x; cl < width; cl += kThreads) {
    if (cbase + cl >= c) break;
    float a = 0.f, b = 0.f;
    for (int t = 0; t < ry; ++t) {
      const float2 v = red[t * width + cl];
      a += v.x;
      b += v.y;
    }
    partial[g * c + cbase + cl] = make_float2(a, b);
  }
}

// NCHW: workgroup (g, ch) reduces images [g*ipg, ...) of channel ch.
template <class Tr, int VEC, bool kGrad>
__global__ __launch_bounds__(kThreads) void bn_nchw_reduce_kernel(
    const typename Tr::S* __restrict__ x, const typename Tr::S* __restrict__ dy,
    const float* __restrict__ mean_in, int64_t nimg, int c, int64_t plane,
    int64_t pv, int64_t ipg, FastDiv div_pv, float2* __restrict__ partial) {
  using S = typename Tr::S;
  __shared__ float2 red[kThreads];
  const int ch = blockIdx.y;
  const int64_t g = blockIdx.x;
  const int64_t n0 = g * ipg;
  int64_t n1 = n0 + ipg;
  if (n1 > nimg) n1 = nimg;
  float kk = kGrad ? mean_in[ch] : chan_shift<Tr>(x, ch, nimg * plane, c, plane);
  float k[VEC], s1[VEC], s2[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) { k[j] = kk; s1[j] = 0.f; s2[j] = 0.f; }
  const uint32_t count = static_cast<uint32_t>((n1 - n0) * pv);
  for (uint32_t e = threadIdx.x; e < count; e += kThreads) {
    uint32_t q, r;
    div_pv.divmod(e, q, r);
    const int64_t off = ((n0 + q) * c + ch) * plane + static_cast<int64_t>(r) * VEC;
    S xv[VEC], dv[VEC];
    vload<S, VEC>(x + off, xv);
    if constexpr (kGrad) vload<S, VEC>(dy + off, dv);
    accum<Tr, VEC, kGrad>(xv, dv, k, s1, s2);
  }
  float a = 0.f, b = 0.f;
#pragma unroll
  for (int j = 0; j < VEC; ++j) { a += s1[j]; b += s2[j]; }
  red[threadIdx.x] = make_float2(a, b);
  __syncthreads();
  for (int s = kThreads / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      red[threadIdx.x].x += red[threadIdx.x + s].x;
      red[threadIdx.x].y += red[threadIdx.x + s].y;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) partial[g * c + ch] = red[0];
}

// ---------------------------------------------------------------------------
// 2. Finalize: per channel, double sums over the G partials.
// ---------------------------------------------------------------------------
struct FinArgs {
  int64_t groups;
  int c;
  int64_t n;          // elements per channel
  const void* x;      // forward shift source (chan_shift() samples)
  int64_t k_stride;   // element stride between channels (1 NHWC, H*W NCHW)
  const float* scale;
  const float* offset;
  const float* mean_in;
  const float* var_in;
  float eps;
  float f;            // exponential_avg_factor
  float* batch_mean;
  float* batch_var;
  float* saved_mean;
  float* saved_var;
  float* reserve3;
  // grad
  float* scale_bp;
  float* offset_bp;
  float* reserve4;
  int64_t reserve4_n;
  float* reserve5;
  int64_t reserve5_n;
  bool is_training;
};

// The per-channel inputs finish_channel() needs besides the sums, loaded
// where they are used (FinLoad) or all at once ahead of the sums (FinIn,
// from fin_inputs()), so a caller can issue the loads before it waits for
// the sums and their latency overlaps the wait (the forward's shift K
// re-reads five elements of x).
template <class Tr>
struct FinLoad {
  const FinArgs& a;
  int ch;
  __device__ float kshift() const {
    return chan_shift<Tr>(static_cast<const typename Tr::S*>(a.x), ch, a.n, a.c, a.k_stride);
  }
  __device__ float scale() const { return a.scale[ch]; }
  __device__ float offset() const { return a.offset[ch]; }
  __device__ float mean_in() const { return a.mean_in[ch]; }
  __device__ float var_in() const { return a.var_in[ch]; }
};

struct FinIn {
  float k, sc, of, mi, vi;  // shift (forward), scale, offset (forward), mean_in, var_in
  __device__ float kshift() const { return k; }
  __device__ float scale() const { return sc; }
  __device__ float offset() const { return of; }
  __device__ float mean_in() const { return mi; }
  __device__ float var_in() const { return vi; }
};

// FinIn of channel ch; kshift = the forward's shift K (unused by the grad).
// mean_in and var_in are read by the grad, and by a forward whose
// exponential_avg_factor is not 1 (only then are they given).
template <class Tr, bool kGrad>
__device__ inline FinIn fin_inputs(const FinArgs& a, int ch, float kshift) {
  FinIn p{kshift, 0.f, 0.f, 0.f, 0.f};
  if (kGrad || a.f != 1.0f) {
    p.mi = a.mean_in[ch];
    p.vi = a.var_in[ch];
  }
  p.sc = a.scale[ch];
  if constexpr (!kGrad) p.of = a.offset[ch];
  return p;
}

template <class Tr, bool kGrad>
__device__ inline FinIn fin_inputs(const FinArgs& a, int ch) {
  return fin_inputs<Tr, kGrad>(a, ch, kGrad ? 0.f : FinLoad<Tr>{a, ch}.kshift());
}

// Final statistics and apply coefficients of channel ch from the double
// sums s1, s2 over all of the channel's elements and its inputs p (FinIn or
// FinLoad); writes the op's per-channel outputs and returns the coefficients
// {mean, a, b, c2} for apply_one().
template <class Tr, bool kGrad, class In>
__device__ inline float4 finish_channel(const FinArgs& a, int ch, double s1, double s2,
                                        const In& p) {
  const double n = static_cast<double>(a.n);
  if constexpr (!kGrad) {
    const double mean = static_cast<double>(p.kshift()) + s1 / n;
    double m2 = s2 - s1 * s1 / n;
    if (m2 < 0.0) m2 = 0.0;
    const float mean_f = static_cast<float>(mean);
    const float var_f = static_cast<float>(m2 / n);
    const float nf = static_cast<float>(a.n);
    const float nm1 = static_cast<float>(a.n > 1 ? a.n - 1 : 1);
    const float adj = nf / nm1;
    a.saved_mean[ch] = mean_f;
    a.saved_var[ch] = var_f;
    if (a.f == 1.0f) {
      a.batch_mean[ch] = mean_f;
      a.batch_var[ch] = var_f * adj;
    } else {
      const float omf = 1.0f - a.f;
      a.batch_mean[ch] = p.mean_in() * omf + mean_f * a.f;
      a.batch_var[ch] = p.var_in() * omf + (var_f * adj) * a.f;
    }
    const float inv = 1.0f / __builtin_sqrtf(var_f + a.eps);
    return make_float4(mean_f, inv * p.scale(), p.offset(), 0.f);
  } else {
    const float mu = p.mean_in();
    const float k = 1.0f / __builtin_sqrtf(p.var_in() + a.eps);
    a.offset_bp[ch] = static_cast<float>(s1);
    a.scale_bp[ch] = static_cast<float>(s2 * static_cast<double>(k));
    if (a.is_training) {
      const float mean_dy = static_cast<float>(s1 / n);
      const float mean_dyxc = static_cast<float>(s2 / n);
      return make_float4(mu, p.scale() * k, mean_dy, (k * k) * mean_dyxc);
    } else {
      return make_float4(mu, p.scale() * k, 0.f, 0.f);
    }
  }
}

template <class Tr, bool kGrad>
__device__ inline float4 finish_channel(const FinArgs& a, int ch, double s1, double s2) {
  return finish_channel<Tr, kGrad>(a, ch, s1, s2, FinLoad<Tr>{a, ch});
}

// Zero-filled side outputs (reserve_space_3 of the forward, reserve_space_4/5
// of the grad), spread over the whole grid.
template <bool kGrad>
__device__ inline void zero_side_outputs(const FinArgs& a) {
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t gstride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  if constexpr (!kGrad) {
    if (gtid == 0 && a.reserve3) a.reserve3[0] = 0.f;
  } else {
    for (int64_t i = gtid; i < a.reserve4_n; i += gstride) a.reserve4[i] = 0.f;
    for (int64_t i = gtid; i < a.reserve5_n; i += gstride) a.reserve5[i] = 0.f;
  }
}

// Split-path finalize: workgroup b owns kFinCh consecutive channels; its
// threads stride over the G partial rows (kFinCh*8 contiguous bytes per row)
// and combine in double through LDS.
template <class Tr, bool kGrad>
__global__ __launch_bounds__(kFinThreads) void bn_finalize_kernel(
    const float2* __restrict__ partial, FinArgs a, float4* __restrict__ coef) {
  constexpr int kSlices = kFinThreads / kFinCh;
  __shared__ double2 red[kSlices][kFinCh];
  const int lane = threadIdx.x % kFinCh;
  const int slice = threadIdx.x / kFinCh;
  const int ch = blockIdx.x * kFinCh + lane;
  double s1 = 0.0, s2 = 0.0;
  if (ch < a.c) {
    for (int64_t g = slice; g < a.groups; g += kSlices) {
      const float2 v = partial[g * a.c + ch];
      s1 += v.x;
      s2 += v.y;
    }
  }
  red[slice][lane] = make_double2(s1, s2);
  __syncthreads();
  if (slice == 0 && ch < a.c) {
    for (int s = 1; s < kSlices; ++s) {
      s1 += red[s][lane].x;
      s2 += red[s][lane].y;
    }
    coef[ch] = finish_channel<Tr, kGrad>(a, ch, s1, s2);
  }
  zero_side_outputs<kGrad>(a);
}

// Inference-mode forward coefficients from the running statistics.
// Inference forward: the statistics outputs are the running mean and
// variance, and each apply thread forms its channels' coefficients itself
// (no coefficient kernel, no second launch).  infer_stats: the statistics
// outputs, spread over the whole grid (lid, nthreads: the calling thread's
// linear index in it and its size).
__device__ inline float4 infer_coef(const FinArgs& a, int64_t ch) {
  const float inv = 1.0f / __builtin_sqrtf(a.var_in[ch] + a.eps);
  return make_float4(a.mean_in[ch], inv * a.scale[ch], a.offset[ch], 0.f);
}
__device__ inline void infer_stats(const FinArgs& a, int64_t lid, int64_t nthreads) {
  if (lid == 0 && a.reserve3) a.reserve3[0] = 0.f;
  for (int64_t ch = lid; ch < a.c; ch += nthreads) {
    const float mu = a.mean_in[ch];
    const float var = a.var_in[ch];
    a.batch_mean[ch] = mu;
    a.batch_var[ch] = var;
    a.saved_mean[ch] = mu;
    a.saved_var[ch] = var;
  }
}

// ---------------------------------------------------------------------------
// 3. Apply.
// ---------------------------------------------------------------------------
template <class Tr, bool kGrad>
__device__ inline typename Tr::S apply_one(typename Tr::S xs, typename Tr::S ds,
                                           float4 cf) {
  const float xc = Tr::ld(xs) - cf.x;
  if constexpr (kGrad) {
    const float t = Tr::ld(ds) - cf.z;
    return Tr::st(cf.y * (t - xc * cf.w));
  } else {
    return Tr::st(xc * cf.y + cf.z);
  }
}

template <class Tr, int VEC, bool kGrad, bool kInfer>
__global__ __launch_bounds__(kThreads) void bn_nhwc_apply_kernel(
    const typename Tr::S* __restrict__ x, const typename Tr::S* __restrict__ dy,
    typename Tr::S* __restrict__ out, const float4* __restrict__ coef,
    int64_t rows, int c, int64_t cv, int tx_shift, int64_t rows_per_g,
    int64_t groups, FinArgs fa) {
  using S = typename Tr::S;
  if constexpr (kInfer)
    infer_stats(fa, (static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x) * kThreads +
                        threadIdx.x,
                static_cast<int64_t>(gridDim.x) * gridDim.y * kThreads);
  const int tx = threadIdx.x & ((1 << tx_shift) - 1);
  const int ty = threadIdx.x >> tx_shift;
  const int ry = kThreads >> tx_shift;
  const int64_t cvi = static_cast<int64_t>(blockIdx.x) * (1 << tx_shift) + tx;
  if (cvi >= cv) return;
  const int64_t g = groups - 1 - blockIdx.y;  // reverse of the reduce order
  const int64_t r0 = g * rows_per_g;
  int64_t r1 = r0 + rows_per_g;
  if (r1 > rows) r1 = rows;
  const int64_t c0 = cvi * VEC;
  float4 cf[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) cf[j] = kInfer ? infer_coef(fa, c0 + j) : coef[c0 + j];
  if (r0 + ty >= r1) return;
  static_assert((kThreads & (kThreads - 1)) == 0, "ry = kThreads >> tx_shift is a power of two");
  const int64_t nr = (r1 - r0 - ty + ry - 1) >> (__builtin_ctz(kThreads) - tx_shift);  // rows of this thread
  const S* __restrict__ px = x + c0;
  const S* __restrict__ pd = kGrad ? dy + c0 : nullptr;
  S* __restrict__ po = out + c0;
  // Walk this thread's rows last-to-first.  The inference forward reads x
  // once: non-temporal loads, which leave the Infinity Cache to the output
  // (measured, [256,56,56,256] f16 kernel time: 69.8 -> 79.3 % of 8 TB/s;
  // non-temporal stores as well 62.8 %, stores alone 61.9 %).  The split
  // training path re-reads lines its reduce kernel just read: plain loads.
  int64_t k = nr - 1;
  for (; k >= kUnroll - 1; k -= kUnroll) {
    S xv[kUnroll][VEC], dv[kUnroll][VEC];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t r = r0 + ty + (k - u) * ry;
      vload_sel<kInfer, S, VEC>(px + r * c, xv[u]);
      if constexpr (kGrad) vload<S, VEC>(pd + r * c, dv[u]);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t r = r0 + ty + (k - u) * ry;
      S ov[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j)
        ov[j] = apply_one<Tr, kGrad>(xv[u][j], kGrad ? dv[u][j] : xv[u][j], cf[j]);
      vstore<S, VEC>(po + r * c, ov);
    }
  }
  for (; k >= 0; --k) {
    const int64_t r = r0 + ty + k * ry;
    S xv[VEC], dv[VEC], ov[VEC];
    vload_sel<kInfer, S, VEC>(px + r * c, xv);
    if constexpr (kGrad) vload<S, VEC>(pd + r * c, dv);
#pragma unroll
    for (int j = 0; j < VEC; ++j)
      ov[j] = apply_one<Tr, kGrad>(xv[j], kGrad ? dv[j] : xv[j], cf[j]);
    vstore<S, VEC>(po + r * c, ov);
  }
}

// NCHW apply: flat over vectors (plane % VEC == 0 keeps a vector inside one
// (image, channel) plane); channel = (i / plane) % C.  Reverse order.
template <class Tr, int VEC, bool kGrad, bool kInfer>
__global__ __launch_bounds__(kThreads) void bn_nchw_apply_kernel(
    const typename Tr::S* __restrict__ x, const typename Tr::S* __restrict__ dy,
    typename Tr::S* __restrict__ out, const float4* __restrict__ coef,
    int64_t nvec, int64_t pv, int c, FinArgs fa) {
  using S = typename Tr::S;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  const int64_t lid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if constexpr (kInfer) infer_stats(fa, lid, stride);
  int last = -1;
  float4 cf = make_float4(0.f, 0.f, 0.f, 0.f);
  // Vector i = q * pv + r of channel q mod c.  One division at the start,
  // then each step back by `stride` vectors updates (r, ch) by subtraction
  // with a borrow (a 64-bit division and modulo per vector made this kernel
  // issue 58k VALU instructions per MB).
  const int64_t i0 = nvec - 1 - lid;
  const int64_t q0 = i0 >= 0 ? i0 / pv : 0;
  int64_t r = i0 >= 0 ? i0 - q0 * pv : 0;
  int64_t chv = q0 % c;
  const int64_t dq = stride / pv;
  const int64_t dr = stride - dq * pv;
  const int64_t dch = dq % c;
  for (int64_t i = i0; i >= 0; i -= stride) {
    const int ch = static_cast<int>(chv);
    r -= dr;
    const int64_t borrow = r < 0 ? 1 : 0;
    r += borrow * pv;
    chv -= dch + borrow;  // dch + borrow <= c: at most one wrap
    chv += chv < 0 ? c : 0;
    if (kInfer ? ch != last : true) {
      cf = kInfer ? infer_coef(fa, ch) : coef[ch];
      last = ch;
    }
    S xv[VEC], dv[VEC], ov[VEC];
    vload<S, VEC>(x + i * VEC, xv);
    if constexpr (kGrad) vload<S, VEC>(dy + i * VEC, dv);
#pragma unroll
    for (int j = 0; j < VEC; ++j)
      ov[j] = apply_one<Tr, kGrad>(xv[j], kGrad ? dv[j] : xv[j], cf);
    vstore<S, VEC>(out + i * VEC, ov);
  }
}

// ---------------------------------------------------------------------------
// 4. Fused persistent kernel (NHWC, 16-byte vectors): one launch per op, one
//    workgroup of 512 threads per CU, all workgroups co-resident.
//    phase 1: statistics partials.  Each thread's rows are split three ways:
//             its first KR row-vectors stay in VGPRs, the next KL in LDS
//             (about 150 KB per workgroup), the rest are streamed;
//    phase 2: per-channel finals, channels spread over workgroups, each
//             waiting only for its channel's partials;
//    phase 3: outputs, each workgroup waiting only for its channel tile's
//             coefficients - streamed rows re-read last-to-first, then the
//             LDS- and register-resident rows, which are not read again.
//    On-chip residency is what removes the second read: on MI355X re-reads
//    served by the Infinity Cache run at about the same rate as HBM reads.
//    No grid barrier: every value that crosses workgroups (partials,
//    coefficients) is a 64-bit word {value, epoch} written and read with
//    agent-scope atomics (coherent across the XCDs' L2s), and its consumer
//    polls until the word carries this launch's epoch.  A two-level grid
//    barrier (relaxed atomics, ~3 us; a cooperative launch's grid sync costs
//    ~33 us) cost 8-11 us per op between the slowest wave's phase-1 end and
//    phase 3: the stores' acknowledgement, two atomic levels and the poll,
//    twice; the epoch words made the 16-op benchmark step 2.9 % faster
//    (4-6 us on each 7x7 op).  A launch that hands out phase-3 chunks, or
//    is recorded into a graph, still counts its exit to reset what the next
//    launch needs reset.
// ---------------------------------------------------------------------------
constexpr int kFusedThreads = 512;
// Polls of a cross-workgroup wait before it gives up (~0.5 s).  A wait can
// only run out when the grid is not co-resident - another persistent kernel
// (another process's, or a graph replay overlapping an eager launch) holds
// CUs this grid's missing workgroups need.  The waiting wave then stops
// waiting, poisons what it computes (the channel's statistics and
// coefficients, hence its outputs, become NaN) and stores the launch's epoch
// into a host-visible word; the host reports it as an error from the next
// FusedBatchNorm call on the device (BnPendingGiveUp).
constexpr unsigned kSpinLimit = 1u << 24;
// Epoch-tagged partials: at most 8 row groups per lane of a finishing wave.
constexpr int kEpochPerLane = 8;
constexpr int64_t kMaxEpochGroups = 64 * kEpochPerLane;
// Copies of the epoch-tagged coefficient words (at most kCoefCopies, one
// per kPollersPerCopy row groups of a tile): the finishing waves store every
// channel's coefficients into each copy and the workgroups of row group g
// poll copy g mod copies, so the polls of a tile's workgroups are spread
// over as many line sets instead of queueing on the few lines of one.
#ifndef TFMA_COEF_COPIES
#define TFMA_COEF_COPIES 8
#endif
constexpr int kCoefCopies = TFMA_COEF_COPIES;
constexpr int kPollersPerCopy = 32;
// Resident 16-byte vectors per thread and per input tensor: KR in VGPRs (the
// largest counts that compile without spills at 256 VGPRs), KL in LDS (the
// LDS budget split over the inputs).  kOpaque*: the register rows are made
// opaque right after their phase-1 use; without it the compiler keeps half
// rows split into 16-bit pieces (8 registers per row instead of 4) until
// phase 3, and with it the bf16 and f32 forwards schedule worse - so it is
// chosen per type and direction, by the spill-free KR it allows.
// kRegFwdSmall: the forward's register rows when a thread has at most
// kSmallFwdRows rows (the 14x14 and 7x7 stage shapes): there fewer register
// rows measured faster even where that leaves rows to stream (each register
// row adds unrolled code to a kernel run about once, and the resident loads
// arrive as one burst that streams worse than the pipelined loop).
// PA/PB: streamed vectors per tensor prefetched for phase 3 while the
// cross-workgroup values are pending - PA after the partials are published
// (by waves with no phase-2 channel), PB after the finals (by every wave).
// Both 0: without the grid barriers the wait is short, and no prefetch was
// 0.35 % faster over the 16-op benchmark step and frees the registers for
// 2-3 more resident rows per type.
template <class Tr> struct Resident {
  static constexpr bool kOpaqueFwd = false, kOpaqueGrad = true;
  static constexpr int kRegFwd = 29, kRegGrad = 13, kLdsFwd = 18, kLdsGrad = 9;
  static constexpr int kRegGradSliced = 11;
  static constexpr int kRegGradOverlap = 17;
  static constexpr int kRegFwdSmall = 8;
  static constexpr int kPaFwd = 0, kPbFwd = 0, kPaGrad = 0, kPbGrad = 0;
};
template <> struct Resident<TF16> {
  static constexpr bool kOpaqueFwd = true, kOpaqueGrad = true;
  static constexpr int kRegFwd = 32, kRegGrad = 13, kLdsFwd = 18, kLdsGrad = 9;
  static constexpr int kRegGradSliced = 12;
  static constexpr int kRegGradOverlap = 15;
  static constexpr int kRegFwdSmall = 8;
  static constexpr int kPaFwd = 0, kPbFwd = 0, kPaGrad = 0, kPbGrad = 0;
};
template <> struct Resident<TBF16> {
  static constexpr bool kOpaqueFwd = false, kOpaqueGrad = true;
  static constexpr int kRegFwd = 32, kRegGrad = 11, kLdsFwd = 18, kLdsGrad = 9;
  static constexpr int kRegGradSliced = 9;
  static constexpr int kRegGradOverlap = 14;
  static constexpr int kRegFwdSmall = 8;
  static constexpr int kPaFwd = 0, kPbFwd = 0, kPaGrad = 0, kPbGrad = 0;
};

struct FusedArgs {
  const void* x;
  const void* dy;
  void* out;
  int64_t rows;
  int c;
  int64_t cv;
  int tx_shift;
  int ct;                       // channel tiles
  int ct_conc;                  // sliced kernel: tiles run at once (ct / slices)
  int slices;                   // sliced kernel: tiles each workgroup runs in turn
  int64_t groups;
  int64_t rows_per_g;
  unsigned long long* barrier;  // device-wide exit-arrival counter
  unsigned long long base;      // its value when this launch starts
  unsigned* sub;                // 8 arrival counters (workgroup id mod 8), 256 B apart
  unsigned sub_last[8];         // value class r's last exit arrival sees
  unsigned* gave_up;             // host-visible word: epoch of a launch whose wait ran out
  unsigned spin_limit;          // polls before a wait gives up (kSpinLimit)
  unsigned wait_xor;            // 0; a test hook flips an epoch bit no launch publishes
  unsigned* queues;             // [ct][wave] chunk counters, zero between launches
  int reset_at_exit;            // recorded into a graph: zero every counter at exit
  int dyn_rows;                 // streamed rows per thread handed out dynamically
  int dyn_chunk;                // rows per thread in one dynamic chunk
  int shards;                   // chunk counters per (ct, wave)
  // Values that cross workgroups carry the launch's epoch: each partial is
  // published as two 64-bit words {value, epoch} in `eslots` ([groups * c]
  // [2]) and each channel's coefficients as four in `ecoef` ([c][4]), both
  // library-owned and zeroed once; the waves finishing a channel poll for
  // its partials, and each workgroup for its tile's coefficients.  Eager
  // launches get the epoch from the host (`epoch`, below 2^31); a launch
  // recorded into a graph reads it from `epoch_dev` (2^31 and up) and its
  // last workgroup to exit advances it for the next replay.
  unsigned long long* eslots;
  unsigned long long* ecoef;
  int64_t coef_copy;            // words from one copy of `ecoef` to the next
  int coef_copies;              // copies in use (1 .. kCoefCopies)
  // The forward's shift K of every channel ([c], one word each), published
  // by the first row group's workgroups with their partials, so the waves
  // finishing a channel read it with the partials instead of re-reading
  // five elements of x.
  unsigned long long* ekey;
  unsigned epoch;
  unsigned* epoch_dev;
  FinArgs fin;
};

// Per-wave phase timestamps of the fused NHWC kernel, compiled in only with
// -DTFMA_BN_STAMPS (a measurement build: make EXTRA=-DTFMA_BN_STAMPS).  Lane
// 0 of each wave stores s_memrealtime (a 100 MHz clock) at kStampCount
// points into bn_stamps[(blockIdx.x * 8 + wave) * kStampCount + point]; the
// host reads them with TFMA_FusedBatchNormStamps.  Points: 0 entry, 1 phase
// 1 summed, 2 partials published, 3 finals done, 4 coefficients in, 5 static
// phase-3 rows written, 6 dynamic tail done; slot 7 holds the wave's XCD.  A
// sliced launch keeps its last slice's stamps.
#ifdef TFMA_BN_STAMPS
constexpr int kStampCount = 8;
constexpr int kStampBlocks = 1024;
__device__ unsigned long long bn_stamps[kStampBlocks * 8 * kStampCount];
__device__ inline void stamp(int point) {
  if ((threadIdx.x & 63) == 0 && blockIdx.x < kStampBlocks) {
    unsigned long long* p = bn_stamps + (blockIdx.x * 8 + (threadIdx.x >> 6)) * kStampCount;
    p[point] = __builtin_amdgcn_s_memrealtime();
    // Point 7: the XCD the wave runs on (HW_REG_XCC_ID bits 3:0).
    if (point == 0) p[7] = __builtin_amdgcn_s_getreg((3 << 11) | 20) & 15;
  }
}
#else
__device__ inline void stamp(int) {}
#endif

__device__ inline double2 wave_sum(double a, double b) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    a += __shfl_xor(a, off, 64);
    b += __shfl_xor(b, off, 64);
  }
  return make_double2(a, b);
}

// Coherent (agent-scope) 8-byte store/load for values shared across XCDs.
__device__ inline void store_shared(void* p, uint64_t v) {
  __hip_atomic_store(static_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint64_t load_shared(const void* p) {
  return __hip_atomic_load(static_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// Exit arrivals (launches that hand out phase-3 chunks, and launches
// recorded into a graph) are counted in two levels: workgroup b counts
// itself on counter b mod 8 (consecutive workgroups sit on different XCDs),
// and the last of each of those classes counts the class on the global
// counter; 256 atomics on one address queue for ~4 us, 8 classes of 32 do
// not.  The workgroup that completes the count resets what the next launch
// needs reset.
__device__ inline unsigned barrier_classes() { return gridDim.x < 8 ? gridDim.x : 8; }

template <class Tr, bool kGrad>
__device__ inline void accum_words(const uint4& xw, const uint4& dw, const float (&k)[Tr::kVec],
                                   float (&s1)[Tr::kVec], float (&s2)[Tr::kVec]) {
  typename Tr::S xv[Tr::kVec], dv[Tr::kVec];
  __builtin_memcpy(xv, &xw, 16);
  if constexpr (kGrad) __builtin_memcpy(dv, &dw, 16);
  accum<Tr, Tr::kVec, kGrad>(xv, dv, k, s1, s2);
}

template <class Tr, bool kGrad>
__device__ inline uint4 apply_words(const uint4& xw, const uint4& dw,
                                    const float4 (&cf)[Tr::kVec]) {
  typename Tr::S xv[Tr::kVec], dv[Tr::kVec], ov[Tr::kVec];
  __builtin_memcpy(xv, &xw, 16);
  if constexpr (kGrad) __builtin_memcpy(dv, &dw, 16);
#pragma unroll
  for (int j = 0; j < Tr::kVec; ++j)
    ov[j] = apply_one<Tr, kGrad>(xv[j], kGrad ? dv[j] : xv[j], cf[j]);
  uint4 o;
  __builtin_memcpy(&o, ov, 16);
  return o;
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ inline uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
// Phase-3 re-reads are the last use of their lines: non-temporal loads keep
// them from displacing the lines the remaining re-reads will still hit in the
// Infinity Cache (measured: the grad kernel 1.9 % faster on cfg2; making the
// phase-1 loads non-temporal as well is 17 % slower).
__device__ inline uint4 ld16_last(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}
// Loads of a workgroup's own rows through a buffer resource (gfx9 word 3
// 0x00020000: raw, stride 0) that covers rows [r0, r1) of one tensor.  An
// offset at or past its end - a row past the group, or any row of an
// inactive lane (offset + 2^31) - is out of range: the load returns zeros
// and makes no memory request.  Loads that may not be needed are issued that
// way instead of inside a branch: a load inside `if (q < nk)` ended up
// waiting for its data before the next load issued (the compiler copies the
// loaded registers at the branch join), which serialized the resident-row
// loads of the forward kernels.  Offsets are 32-bit (one VGPR per address
// instead of two); the host keeps a group's span below 2^31 bytes.
constexpr uint32_t kOutOfRange = 0x80000000u;
__device__ inline __amdgpu_buffer_rsrc_t rows_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0,
                                           static_cast<int>(bytes > 0 ? bytes : 0), 0x00020000);
}
__device__ inline uint4 bld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ inline uint4 bld16_last(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2 /* nt */);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// A channel's two partial words of one row group - {sum 1, epoch} and {sum
// 2, epoch}, adjacent and 16-byte aligned - moved in one 16-byte access
// with the cache policy of the agent-scope atomics (sc1: coherent across
// the XCDs' L2s) instead of two 8-byte ones: half the requests for the
// finishing waves' polls, which gather one slot per row group.  Each 8-byte
// half carries its own tag, so a read that saw one half before the other
// was written looks not yet ready and is polled again.  These are plain
// loads to the compiler: a poll loop reloads them after a compiler barrier.
// Their words are read as floats through bits_f32 (by value): this clang's
// __builtin_bit_cast applied to an element of an ext_vector_type value
// reads element 0 whatever the index.
constexpr int kSc1 = 16;  // buffer cache policy bit sc1
__device__ inline __amdgpu_buffer_rsrc_t slots_rsrc(const void* slots, int64_t groups, int c) {
  return rows_rsrc(slots, groups * c * 16);
}
__device__ inline u32x4 load_pair(__amdgpu_buffer_rsrc_t r, int64_t slot) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<uint32_t>(slot) * 16u, 0, kSc1);
}
__device__ inline void store_pair(__amdgpu_buffer_rsrc_t r, int64_t slot, uint32_t epoch,
                                  float sa, float sb) {
  const u32x4 w = {__builtin_bit_cast(uint32_t, sa), epoch, __builtin_bit_cast(uint32_t, sb),
                   epoch};
  __builtin_amdgcn_raw_buffer_store_b128(w, r, static_cast<uint32_t>(slot) * 16u, 0, kSc1);
}
__device__ inline bool pair_tagged(const u32x4& v, uint32_t wtag) {
  return v[1] == wtag && v[3] == wtag;
}
// Outputs are written once and not read again by the op: non-temporal.
__device__ inline void st16(void* p, const uint4& v) {
  __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4*>(p));
}

// Phase-1 end of a channel tile: the threads' partial sums, summed over the
// row lanes of each wave with shuffles, then over the waves through LDS
// (`red`), published as one epoch-tagged pair of words per channel.
// Sums s1, s2 over the row lanes of each wave (shuffles); lanes
// 0 .. 2^tx_shift - 1 of the wave then hold the wave's sums of their channels.
template <int VEC>
__device__ __forceinline__ void wave_row_sums(const FusedArgs& a, float (&s1)[VEC],
                                              float (&s2)[VEC]) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    if (off < (1 << a.tx_shift)) break;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      s1[j] += __shfl_xor(s1[j], off, 64);
      s2[j] += __shfl_xor(s2[j], off, 64);
    }
  }
}

// The workgroup's sums of its threads' s1, s2 per channel of the tile, for
// thread tid < width (channel tid), through `red`: wave sums by shuffles,
// then the waves in a fixed order.  Every thread calls it (two barriers);
// `red` must be free on entry.
template <int VEC>
__device__ __forceinline__ float2 workgroup_sums(const FusedArgs& a, float2* red,
                                                float (&s1)[VEC], float (&s2)[VEC], int tid,
                                                int width) {
  const int wave = tid >> 6;
  const int lane = tid & 63;
  wave_row_sums<VEC>(a, s1, s2);
  __syncthreads();
  if (lane < (1 << a.tx_shift)) {
#pragma unroll
    for (int j = 0; j < VEC; ++j) red[wave * width + lane * VEC + j] = make_float2(s1[j], s2[j]);
  }
  __syncthreads();
  float2 r = make_float2(0.f, 0.f);
  if (tid < width) {
#pragma unroll
    for (int w = 0; w < kFusedThreads / 64; ++w) {
      const float2 v = red[w * width + tid];
      r.x += v.x;
      r.y += v.y;
    }
  }
  return r;
}

// `pend` (thread tid < width, channel tid of the tile): sums of earlier rows
// of the workgroup for that channel, added last.
template <int VEC>
__device__ __forceinline__ void publish_partials(const FusedArgs& a, float2* red,
                                                 float (&s1)[VEC], float (&s2)[VEC], int tid,
                                                 int width, int ct, int64_t g, uint64_t etag,
                                                 float2 pend = make_float2(0.f, 0.f)) {
  const int wave = tid >> 6;
  const int lane = tid & 63;
  wave_row_sums<VEC>(a, s1, s2);
  if (lane < (1 << a.tx_shift)) {
#pragma unroll
    for (int j = 0; j < VEC; ++j) red[wave * width + lane * VEC + j] = make_float2(s1[j], s2[j]);
  }
  __syncthreads();
  if (tid < width && static_cast<int64_t>(ct) * width + tid < static_cast<int64_t>(a.cv) * VEC) {
    float sa = 0.f, sb = 0.f;
#pragma unroll
    for (int w = 0; w < kFusedThreads / 64; ++w) {
      const float2 v = red[w * width + tid];
      sa += v.x;
      sb += v.y;
    }
    sa += pend.x;
    sb += pend.y;
    const int64_t slot = g * a.c + static_cast<int64_t>(ct) * width + tid;
    store_pair(slots_rsrc(a.eslots, a.groups, a.c), slot, static_cast<uint32_t>(etag >> 32), sa,
               sb);
  }
}

// Stores the coefficients of a finished channel block into every copy:
// lanes [0, B) hold channels cb .. cb + B - 1 (lane l's channel is ch, the
// one of lane l mod B; chv: it exists); lane l stores copies l / B,
// l / B + 64 / B, ...  Every lane of the wave takes part (shuffles).
__device__ __forceinline__ void store_coefs(const FusedArgs& a, int ch, bool chv, float4 cfc,
                                            int lane, int B, uint64_t etag) {
  const int src = lane % B;
  const float v4[4] = {__shfl(cfc.x, src, 64), __shfl(cfc.y, src, 64), __shfl(cfc.z, src, 64),
                       __shfl(cfc.w, src, 64)};
  if (!chv) return;
  // Two 16-byte pairs per channel and copy (a copy is an even number of
  // words, so every channel's four words start 16-byte aligned).
  const auto rc = rows_rsrc(a.ecoef, a.coef_copies * a.coef_copy * 8);
  const uint32_t e = static_cast<uint32_t>(etag >> 32);
  for (int r = lane / B; r < a.coef_copies; r += 64 / B) {
    const int64_t pr = (r * a.coef_copy + 4 * static_cast<int64_t>(ch)) / 2;
    store_pair(rc, pr, e, v4[0], v4[1]);
    store_pair(rc, pr + 1, e, v4[2], v4[3]);
  }
}

// Phase 2 for channels [cs0, cs1): channel ch is finished by wave
// (ch - cs0) / gridDim.x of workgroup (ch - cs0) % gridDim.x, one channel
// at a time per wave, so all of a workgroup's partial loads are in flight
// together.  A wait that runs out stores the launch's epoch into the
// host-visible give-up word and poisons the channel.
template <class Tr, bool kGrad>
__device__ __forceinline__ void finish_channels(const FusedArgs& a, int cs0, int cs1, int wave,
                                                int lane, uint32_t wtag, uint64_t etag,
                                                unsigned epoch) {
  constexpr int kWaves = kFusedThreads / 64;
  auto give_up = [&]() {
    __hip_atomic_store(a.gave_up, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  };
  for (int ch = cs0 + blockIdx.x + wave * gridDim.x; ch < cs1; ch += kWaves * gridDim.x) {
    // The channel's other inputs, in flight while its partials are polled;
    // the forward's shift K comes with them (lane 0 polls its word).
    FinIn fin_in = fin_inputs<Tr, kGrad>(a.fin, ch, 0.f);
    double t1 = 0.0, t2 = 0.0;
    {
      // Lane l sums groups l, l + 64, ... (at most kMaxGroups / 64 of them):
      // all their slots are loaded at once, then the ones not yet tagged
      // with this launch's epoch are polled again.
      const uint64_t tag = static_cast<uint64_t>(wtag) << 32;
      const bool has_key = !kGrad && lane == 0;
      uint64_t vk = has_key ? load_shared(a.ekey + ch) : tag;
      // Slots past the groups are out of range: they read as zeros and are
      // treated as tagged.
      const auto rs = slots_rsrc(a.eslots, a.groups, a.c);
      auto pslot = [&](int i) -> int64_t {
        const int64_t gg = lane + 64 * i;
        return gg < a.groups ? gg * a.c + ch : int64_t(kOutOfRange / 16);
      };
      auto ok = [&](const u32x4& v, int i) {
        return lane + 64 * i >= a.groups || pair_tagged(v, wtag);
      };
      u32x4 v[kEpochPerLane];
#pragma unroll
      for (int i = 0; i < kEpochPerLane; ++i) v[i] = load_pair(rs, pslot(i));
      unsigned spins = 0;
      bool lost = false;
      while (true) {
        bool ready = (vk >> 32) == (tag >> 32);
#pragma unroll
        for (int i = 0; i < kEpochPerLane; ++i) ready = ready && ok(v[i], i);
        if (ready) break;
        if (++spins > a.spin_limit) {
          lost = true;
          give_up();
          break;
        }
        __builtin_amdgcn_s_sleep(1);
        if ((vk >> 32) != (tag >> 32)) vk = load_shared(a.ekey + ch);
        asm volatile("" ::: "memory");  // the reloads below are not the loads above
#pragma unroll
        for (int i = 0; i < kEpochPerLane; ++i)
          if (!ok(v[i], i)) v[i] = load_pair(rs, pslot(i));
      }
      fin_in.k = __builtin_bit_cast(float, static_cast<uint32_t>(vk));
#pragma unroll
      for (int i = 0; i < kEpochPerLane; ++i) {
        if (lane + 64 * i < a.groups) {
          t1 += bits_f32(v[i][0]);
          t2 += bits_f32(v[i][2]);
        }
      }
      // A lane whose partials never arrived poisons the channel's sums (the
      // wave sum below spreads the NaN to its statistics and coefficients).
      if (lost) t1 = t2 = __builtin_nan("");
    }
    const double2 w = wave_sum(t1, t2);
    float4 cfc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (lane == 0) cfc = finish_channel<Tr, kGrad>(a.fin, ch, w.x, w.y, fin_in);
    store_coefs(a, ch, true, cfc, lane, 1, etag);
  }
}

// Phase 2 in blocks of B consecutive channels (every fused kernel whose
// registers allow it): block j of [cs0, cs1) is finished by wave j / gridDim.x of
// workgroup j % gridDim.x.  Lane l reads channel l % B of groups l / B,
// l / B + 64 / B, ... - so each group's B channels are one contiguous
// segment of partial words (B * 16 bytes) instead of B words a line apart
// - sums them in group order, then across the lanes of its channel; lanes
// 0 .. B-1 finish one channel each.  B = 16, or smaller where the groups
// need more than kEpochPerLane words per lane.  Same give-up behaviour as
// finish_channels.
template <class Tr, bool kGrad>
__device__ __forceinline__ void finish_channel_blocks(const FusedArgs& a, int cs0, int cs1,
                                                      int wave, int lane, uint32_t wtag,
                                                      uint64_t etag, unsigned epoch) {
  constexpr int kWaves = kFusedThreads / 64;
  int B = 16;
  while (B > 1 && static_cast<int64_t>(64 / B) * kEpochPerLane < a.groups) B >>= 1;
  const int gpl = 64 / B;
  const int cl = lane % B, gl = lane / B;
  const int nb = (cs1 - cs0 + B - 1) / B;
  const uint64_t tag = static_cast<uint64_t>(wtag) << 32;
  auto tagged = [&](uint64_t v) { return (v >> 32) == (tag >> 32); };
  for (int blk = blockIdx.x + wave * gridDim.x; blk < nb; blk += kWaves * gridDim.x) {
    const int ch = cs0 + blk * B + cl;
    const bool chv = ch < cs1;
    FinIn fin_in = fin_inputs<Tr, kGrad>(a.fin, chv ? ch : cs1 - 1, 0.f);
    uint64_t vk = !kGrad && chv ? load_shared(a.ekey + ch) : tag;
    // Slots of absent channels or past the groups are out of range: they
    // read as zeros and are treated as tagged.
    const auto rs = slots_rsrc(a.eslots, a.groups, a.c);
    auto has = [&](int i) { return chv && gl + static_cast<int64_t>(gpl) * i < a.groups; };
    auto pslot = [&](int i) -> int64_t {
      return has(i) ? (gl + static_cast<int64_t>(gpl) * i) * a.c + ch
                    : int64_t(kOutOfRange / 16);
    };
    u32x4 v[kEpochPerLane];
#pragma unroll
    for (int i = 0; i < kEpochPerLane; ++i) v[i] = load_pair(rs, pslot(i));
    unsigned spins = 0;
    bool lost = false;
    while (true) {
      bool ready = tagged(vk);
#pragma unroll
      for (int i = 0; i < kEpochPerLane; ++i)
        ready = ready && (!has(i) || pair_tagged(v[i], wtag));
      if (ready) break;
      if (++spins > a.spin_limit) {
        lost = true;
        __hip_atomic_store(a.gave_up, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      if (!tagged(vk)) vk = load_shared(a.ekey + ch);
      asm volatile("" ::: "memory");  // the reloads below are not the loads above
#pragma unroll
      for (int i = 0; i < kEpochPerLane; ++i)
        if (has(i) && !pair_tagged(v[i], wtag)) v[i] = load_pair(rs, pslot(i));
    }
    fin_in.k = __builtin_bit_cast(float, static_cast<uint32_t>(vk));
    double t1 = 0.0, t2 = 0.0;
#pragma unroll
    for (int i = 0; i < kEpochPerLane; ++i) {
      if (chv && gl + static_cast<int64_t>(gpl) * i < a.groups) {
        t1 += bits_f32(v[i][0]);
        t2 += bits_f32(v[i][2]);
      }
    }
    // A lane whose partials never arrived poisons its channel's sums.
    if (lost) t1 = t2 = __builtin_nan("");
    for (int off = 32; off >= B; off >>= 1) {
      t1 += __shfl_xor(t1, off, 64);
      t2 += __shfl_xor(t2, off, 64);
    }
    float4 cfc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (lane < B && chv) cfc = finish_channel<Tr, kGrad>(a.fin, ch, t1, t2, fin_in);
    store_coefs(a, ch, chv, cfc, lane, B, etag);
  }
}

// The coefficients of channel tile ct (4 words per channel, at most 1024
// words: one 16-byte pair per thread, consecutive pairs to consecutive
// threads, so the cross-XCD loads stay coalesced), polled until tagged with
// this launch's epoch, then shared through `red`, free since phase 1's
// reduction (the first __syncthreads below orders those reads before these
// writes).  LDS: component c of channel cl (= tx * VEC + j) at c * kW + cl +
// cl / VEC - a stride kW = 8 (mod 32) between components and one pad word
// per channel vector, so the reads (lane tx at tx * (VEC + 1) + j) hit
// distinct banks.  Coefficients that never arrive are used as NaN.
template <class Tr>
__device__ __forceinline__ void tile_coefs(const FusedArgs& a, float2* red, int tid, int tx, int ct,
                                           int width, bool active, uint32_t wtag, unsigned epoch,
                                           float4 (&cf)[Tr::kVec]) {
  constexpr int VEC = Tr::kVec;
  constexpr int kW = VEC == 8 ? 296 : 168;  // >= 32 * (VEC + 1), = 8 mod 32
  static_assert(kW >= 32 * (VEC + 1) && kW % 32 == 8, "coefficient layout");
  static_assert(4 * kW * sizeof(float) <= (kFusedThreads / 64) * 32 * VEC * sizeof(float2),
                "coefficients fit in red");
  float* const cs = reinterpret_cast<float*>(red);
  // Row group blockIdx.x / ct_conc polls its copy.  Thread t polls the pair
  // of words 2t, 2t + 1: components 2 (t & 1) and 2 (t & 1) + 1 of channel
  // t / 2; a pair it does not need is out of range and not polled.
  const int64_t copy0 = ((blockIdx.x / a.ct_conc) % a.coef_copies) * a.coef_copy;
  const auto rc = rows_rsrc(a.ecoef, a.coef_copies * a.coef_copy * 8);
  const int cl = tid >> 1;
  const int64_t chn = static_cast<int64_t>(ct) * width + cl;
  const bool need = cl < width && chn < a.c;
  const int64_t pr = need ? (copy0 + 4 * chn) / 2 + (tid & 1) : int64_t(kOutOfRange / 16);
  u32x4 v = load_pair(rc, pr);
  unsigned spins = 0;
  while (need && !pair_tagged(v, wtag)) {
    if (++spins > a.spin_limit) {
      if (v[1] != wtag) v[0] = 0x7fc00000u;
      if (v[3] != wtag) v[2] = 0x7fc00000u;
      __hip_atomic_store(a.gave_up, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
    asm volatile("" ::: "memory");  // the reload is not the load above
    v = load_pair(rc, pr);
  }
  __syncthreads();
  if (need) {
    const int c2 = 2 * (tid & 1);
    cs[c2 * kW + cl + cl / VEC] = bits_f32(v[0]);
    cs[(c2 + 1) * kW + cl + cl / VEC] = bits_f32(v[2]);
  }
  __syncthreads();
  const int cb = tx * (VEC + 1);
#pragma unroll
  for (int j = 0; j < VEC; ++j)
    cf[j] = active ? make_float4(cs[cb + j], cs[kW + cb + j], cs[2 * kW + cb + j],
                                 cs[3 * kW + cb + j])
                   : make_float4(0.f, 0.f, 0.f, 0.f);
}

template <class Tr, bool kGrad, int KR, int KL, bool kSliced>
__global__ __launch_bounds__(kFusedThreads) void bn_fused_nhwc_kernel(FusedArgs a) {
  using S = typename Tr::S;
  constexpr int VEC = Tr::kVec;
  constexpr int kIn = kGrad ? 2 : 1;
  constexpr int U = kGrad ? 4 : 8;  // streamed vectors per tensor in flight
  extern __shared__ uint4 lds_rows[];  // [KL][kIn][kFusedThreads]
  __shared__ float2 red[(kFusedThreads / 64) * 32 * VEC];  // [wave][tx * VEC + j]
  constexpr int kWaves = kFusedThreads / 64;
  // Channel tiles of this workgroup.  Unsliced: one, tile blockIdx % ct of
  // row group blockIdx / ct.  Sliced: the workgroup owns row group
  // blockIdx / ct_conc and runs the whole two-phase pass once per slice, on
  // tile blockIdx % ct_conc + s * ct_conc in slice s, so a slice's rows fit
  // (or nearly fit) in the resident registers and LDS and are not re-read.
  const int nslices = kSliced ? a.slices : 1;
  const int width = (1 << a.tx_shift) * VEC;  // channels of a tile

  stamp(0);
  // This launch's epoch, in the upper half of the tag word (recorded
  // launches: 2^31 + 1 + (device word mod 2^31 - 1)), and the tag the waits
  // look for (wait_xor is 0 except under the host's forced-give-up test
  // hook).  Read once the first phase-1 loads are issued: the branch and
  // its kernel-argument loads would otherwise stand before them.
  unsigned epoch = 0;
  uint64_t etag = 0;
  uint32_t wtag = 0;
  auto read_epoch = [&]() {
    epoch = a.epoch_dev ? 0x80000001u + __hip_atomic_load(a.epoch_dev, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT) %
                                            0x7fffffffu
                        : a.epoch;
    etag = static_cast<uint64_t>(epoch) << 32;
    wtag = epoch ^ a.wait_xor;
  };

#pragma clang loop unroll(disable)
  for (int sl = 0; sl < nslices; ++sl) {
  int tid_v = threadIdx.x;
  if constexpr (kSliced) asm volatile("" : "+v"(tid_v));
  const int tid = tid_v;
  const int tx = tid & ((1 << a.tx_shift) - 1);
  const int ty = tid >> a.tx_shift;
  const int ry = kFusedThreads >> a.tx_shift;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int ct_conc = kSliced ? a.ct_conc : a.ct;
  const int64_t g = blockIdx.x / ct_conc;
  const int64_t r0 = g * a.rows_per_g;
  int64_t r1 = r0 + a.rows_per_g;
  if (r1 > a.rows) r1 = a.rows;
  const int ct = static_cast<int>(blockIdx.x % ct_conc) + sl * ct_conc;
  // The channels whose finals this slice computes.
  const int cs0 = sl * ct_conc * width;
  const int cs1 = a.c < cs0 + ct_conc * width ? a.c : cs0 + ct_conc * width;
  // The previous slice's reads of its coefficients from `red` come before
  // this slice's phase-1 reduction writes it.
  if (kSliced && sl > 0) __syncthreads();
  const int64_t cvi = static_cast<int64_t>(ct) * (1 << a.tx_shift) + tx;
  const bool active = cvi < a.cv;
  static_assert(kFusedThreads == 512, "ry = 2^(9 - tx_shift)");
  const int ry_shift = 9 - a.tx_shift;
  const int64_t nk = (active && r0 + ty < r1) ? (r1 - r0 - ty + ry - 1) >> ry_shift : 0;
  // The wave's last LDS row (see the LDS loops below); the large forwards
  // keep all KL slots (bounded, their phase 1 was scheduled worse: the
  // 56x56 forward 178 -> 194 us).
  constexpr bool kWaveLds = kGrad || KR == Resident<Tr>::kRegFwdSmall;
  const int nk_w = __builtin_amdgcn_readfirstlane(static_cast<int>(nk));
  const int kl_w =
      !kWaveLds ? KL : (nk_w - KR < 0 ? 0 : (nk_w - KR < KL ? nk_w - KR : KL));
  const int64_t c0 = active ? cvi * VEC : 0;
  const S* __restrict__ px = static_cast<const S*>(a.x) + c0;
  const S* __restrict__ pd = kGrad ? static_cast<const S*>(a.dy) + c0 : nullptr;
  S* __restrict__ po = static_cast<S*>(a.out) + c0;
  const int64_t rstride = static_cast<int64_t>(ry) * a.c;  // elements between my rows
  const int64_t base = (r0 + ty) * a.c;                     // my first row
  auto xrow = [&](int64_t q) { return px + base + q * rstride; };
  auto drow = [&](int64_t q) { return pd + base + q * rstride; };
  // This group's rows as buffer resources: roff(q) is the byte offset of my
  // row q, out of range past the group (and for an inactive lane);
  // roff_if(q, false) is out of range.
  const int64_t gbytes = (r1 - r0) * a.c * static_cast<int64_t>(sizeof(S));
  const auto rx = rows_rsrc(static_cast<const S*>(a.x) + r0 * a.c, gbytes);
  const auto rd = rows_rsrc(kGrad ? static_cast<const S*>(a.dy) + r0 * a.c : a.x, gbytes);
  const uint32_t lane_off =
      active ? static_cast<uint32_t>((ty * a.c + c0) * static_cast<int64_t>(sizeof(S)))
             : kOutOfRange;
  const uint32_t rstride_b = static_cast<uint32_t>(rstride * static_cast<int64_t>(sizeof(S)));
  auto roff = [&](int64_t q) { return lane_off + static_cast<uint32_t>(q) * rstride_b; };
  auto roff_if = [&](int64_t q, bool use) { return use ? roff(q) : kOutOfRange; };
  auto lds = [&](int q2, int which) -> uint4& {
    return lds_rows[(q2 * kIn + which) * kFusedThreads + tid];
  };

  // ---- phase 1: partial statistics --------------------------------------
  float k[VEC], s1[VEC], s2[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    s1[j] = 0.f;
    s2[j] = 0.f;
    k[j] = 0.f;
  }
  if (active) {
#pragma unroll
    for (int j = 0; j < VEC; ++j) k[j] = kGrad ? a.fin.mean_in[c0 + j] : 0.f;
  }
  // The shift samples: an inactive lane (px = x) reads channels 0..VEC-1 of
  // the same rows, in bounds, and its k is never used.
  uint4 kw[kGrad ? 1 : 5];
  if constexpr (!kGrad) {
    int64_t js[5];
    shift_rows(a.rows, js);
#pragma unroll
    for (int i = 0; i < 5; ++i) kw[i] = ld16(px + js[i] * a.c);
  }
  // Register- and LDS-resident rows: all loads issued before any is used,
  // none of them in a branch (rows past nk are out of range).
  uint4 xr[KR];
  uint4 dr[kGrad ? KR : 1];
  uint4 xl[KL];
  uint4 dl[kGrad ? KL : 1];
  // These rows are never read from memory again (phase 3 takes them from
  // registers and LDS), so their loads are non-temporal: they leave the
  // Infinity Cache to the streamed rows that phase 3 re-reads (measured: the
  // 16-op cfg2 step 1.825 -> 1.802 ms, the 56x56 grads 3 % faster).
#pragma unroll
  for (int q = 0; q < KR; ++q) {
    xr[q] = bld16_last(rx, roff(q));
    if constexpr (kGrad) dr[q] = bld16_last(rd, roff(q));
  }
#pragma unroll
  for (int q = 0; q < KL; ++q) {
    xl[q] = bld16_last(rx, roff(KR + q));
    if constexpr (kGrad) dl[q] = bld16_last(rd, roff(KR + q));
  }
  if (sl == 0) read_epoch();
  if constexpr (!kGrad) shift_words<Tr>(kw, k);
  // After its phase-1 use a register row is made opaque, so the compiler
  // keeps its packed words to phase 3 rather than the half-width pieces it
  // split them into (for half: twice the registers).
#pragma unroll
  for (int q = 0; q < KR; ++q) {
    if (q < nk) accum_words<Tr, kGrad>(xr[q], dr[kGrad ? q : 0], k, s1, s2);
    if constexpr (kGrad ? Resident<Tr>::kOpaqueGrad : Resident<Tr>::kOpaqueFwd) {
      asm volatile("" : "+v"(xr[q].x), "+v"(xr[q].y), "+v"(xr[q].z), "+v"(xr[q].w));
      if constexpr (kGrad)
        asm volatile("" : "+v"(dr[q].x), "+v"(dr[q].y), "+v"(dr[q].z), "+v"(dr[q].w));
    }
  }
  // LDS rows: stored as they arrive, then accumulated from LDS in a loop,
  // not unrolled - the unrolled per-row code made the kernel about as large
  // as the 64 KB instruction cache a CU pair shares, which the small shapes
  // (code run once) paid for.  Both loops, and phase 3's, stop at the
  // wave's last LDS row (kl_w, wave-uniform: lane 0 has the wave's smallest
  // ty, hence its largest nk) instead of running all KL slots; slots past a
  // lane's own nk are never read.
#pragma unroll
  for (int q = 0; q < KL; ++q) {
    if (q < kl_w) {
      lds(q, 0) = xl[q];
      if constexpr (kGrad) lds(q, kGrad ? 1 : 0) = dl[kGrad ? q : 0];
    }
  }
#pragma unroll 2
  for (int q = 0; q < kl_w; ++q) {
    if (KR + q < nk) {
      const uint4 xw = lds(q, 0);
      const uint4 dw = kGrad ? lds(q, kGrad ? 1 : 0) : xw;
      accum_words<Tr, kGrad>(xw, dw, k, s1, s2);
    }
  }
  // Streamed rows, U vectors per tensor in flight.
  int64_t q = KR + KL;
  for (; q + U <= nk; q += U) {
    uint4 xw[U], dw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      xw[u] = ld16(xrow(q + u));
      if constexpr (kGrad) dw[u] = ld16(drow(q + u));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) accum_words<Tr, kGrad>(xw[u], dw[u], k, s1, s2);
  }
  // Fewer than U rows left: all of their loads in flight at once (rows past
  // nk out of range), not one load-and-wait per row.
  if (q < nk) {
    uint4 xw[U], dw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      xw[u] = bld16(rx, roff(q + u));
      if constexpr (kGrad) dw[u] = bld16(rd, roff(q + u));
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (q + u < nk) accum_words<Tr, kGrad>(xw[u], dw[u], k, s1, s2);
  }
  stamp(1);
  if constexpr (!kGrad) {
    if (g == 0 && ty == 0 && active) {
#pragma unroll
      for (int j = 0; j < VEC; ++j)
        store_shared(a.ekey + c0 + j, etag | __builtin_bit_cast(uint32_t, k[j]));
    }
  }
  publish_partials<VEC>(a, red, s1, s2, tid, width, ct, g, etag);
  stamp(2);

  // Phase-3 prefetch, part A: the last streamed rows (phase 3 runs
  // last-to-first), loaded by the waves that have no phase-2 channel so the
  // partial loads of the others do not queue behind them.
  constexpr int PA = kGrad ? Resident<Tr>::kPaGrad : Resident<Tr>::kPaFwd;
  constexpr int PB = kGrad ? Resident<Tr>::kPbGrad : Resident<Tr>::kPbFwd;
  const bool pre_a =
      PA > 0 && static_cast<int>(blockIdx.x) + wave * static_cast<int>(gridDim.x) >= cs1 - cs0;
  uint4 pax[PA > 0 ? PA : 1], pad[kGrad && PA > 0 ? PA : 1];
  if (pre_a) {
#pragma unroll
    for (int p = 0; p < PA; ++p) {
      const uint32_t o = roff_if(nk - 1 - p, nk - 1 - p >= KR + KL);
      pax[p] = bld16(rx, o);
      if constexpr (kGrad) pad[p] = bld16(rd, o);
    }
  }
  const int64_t qb = nk - 1 - (pre_a ? PA : 0);  // first row of part B

  // ---- phase 2: per-channel finals ---------------------------------------
  // In channel blocks where the registers allow it (all but the unsliced
  // float grad, which would spill), else a channel per wave.
  constexpr bool kBlockFin = !(kGrad && !kSliced && sizeof(S) == 4);
  if constexpr (kBlockFin)
    finish_channel_blocks<Tr, kGrad>(a, cs0, cs1, wave, lane, wtag, etag, epoch);
  else
    finish_channels<Tr, kGrad>(a, cs0, cs1, wave, lane, wtag, etag, epoch);
  if (sl == 0) zero_side_outputs<kGrad>(a.fin);
  stamp(3);

  // Prefetch part B: the next rows, in flight while the tile's coefficients
  // are polled.
  uint4 pbx[PB > 0 ? PB : 1], pbd[kGrad && PB > 0 ? PB : 1];
#pragma unroll
  for (int p = 0; p < PB; ++p) {
    const uint32_t o = roff_if(qb - p, qb - p >= KR + KL);
    pbx[p] = bld16(rx, o);
    if constexpr (kGrad) pbd[p] = bld16(rd, o);
  }

  // ---- phase 3: outputs --------------------------------------------------
  // Make the resident words opaque so only the packed words (not their
  // phase-1 float conversions) stay live across the barriers.
#pragma unroll
  for (int r = 0; r < KR; ++r) {
    asm volatile("" : "+v"(xr[r].x), "+v"(xr[r].y), "+v"(xr[r].z), "+v"(xr[r].w));
    if constexpr (kGrad)
      asm volatile("" : "+v"(dr[r].x), "+v"(dr[r].y), "+v"(dr[r].z), "+v"(dr[r].w));
  }
  float4 cf[VEC];
  tile_coefs<Tr>(a, red, tid, tx, ct, width, active, wtag, epoch, cf);
  stamp(4);
  // Prefetched rows first, then the remaining streamed rows last-to-first.
  if (pre_a) {
#pragma unroll
    for (int p = 0; p < PA; ++p)
      if (nk - 1 - p >= KR + KL)
        st16(po + base + (nk - 1 - p) * rstride,
             apply_words<Tr, kGrad>(pax[p], pad[kGrad ? p : 0], cf));
  }
#pragma unroll
  for (int p = 0; p < PB; ++p)
    if (qb - p >= KR + KL)
      st16(po + base + (qb - p) * rstride, apply_words<Tr, kGrad>(pbx[p], pbd[kGrad ? p : 0], cf));
  // The lowest dyn_rows streamed rows of every thread are not processed by
  // their owner but handed out in chunks after the owner's other rows.
  const int64_t qlo = KR + KL + a.dyn_rows;
  // Phase-3 rows in flight per tensor: the grad's loop has the registers for
  // 6 (0.8 % faster than 4); the forward gains nothing beyond its 8.
  constexpr int U3 = kGrad ? 6 : U;
  q = qb - PB;
  for (; q >= qlo + U3 - 1; q -= U3) {
    uint4 xw[U3], dw[U3];
#pragma unroll
    for (int u = 0; u < U3; ++u) {
      xw[u] = ld16_last(xrow(q - u));
      if constexpr (kGrad) dw[u] = ld16_last(drow(q - u));
    }
#pragma unroll
    for (int u = 0; u < U3; ++u)
      st16(po + base + (q - u) * rstride, apply_words<Tr, kGrad>(xw[u], dw[u], cf));
  }
  if (q >= qlo) {  // fewer than U3 rows left: loads issued together
    uint4 xw[U3], dw[U3];
#pragma unroll
    for (int u = 0; u < U3; ++u) {
      const uint32_t o = roff_if(q - u, q - u >= qlo);
      xw[u] = bld16_last(rx, o);
      if constexpr (kGrad) dw[u] = bld16_last(rd, o);
    }
#pragma unroll
    for (int u = 0; u < U3; ++u)
      if (q - u >= qlo) st16(po + base + (q - u) * rstride, apply_words<Tr, kGrad>(xw[u], dw[u], cf));
  }
#pragma unroll 2
  for (int q2 = 0; q2 < kl_w; ++q2) {
    if (KR + q2 < nk) {
      const uint4 xw = lds(q2, 0);
      const uint4 dw = kGrad ? lds(q2, kGrad ? 1 : 0) : xw;
      st16(po + base + (KR + q2) * rstride, apply_words<Tr, kGrad>(xw, dw, cf));
    }
  }
#pragma unroll
  for (int r = 0; r < KR; ++r)
    if (r < nk) st16(po + base + r * rstride, apply_words<Tr, kGrad>(xr[r], dr[kGrad ? r : 0], cf));
  stamp(5);

  // Dynamic tail: chunk j of group g' covers the owner rows q in
  // [KR+KL + j*B, KR+KL + (j+1)*B) below the owner's static rows.  Wave w of
  // any workgroup of channel tile ct takes chunks of wave w of the others
  // (same lanes, same channels, same coefficients).  Groups are split into
  // `shards` of whole runs of 8 consecutive groups (8 consecutive workgroups
  // sit on the 8 different XCDs), each with its own counter per (ct, w), so
  // no single counter serializes the whole grid.  The next claim is issued
  // before the current chunk is processed.  Results do not depend on which
  // wave writes them.
  if (a.dyn_rows > 0) {
    const int B = a.dyn_chunk;
    const int S = a.shards;
    const int64_t nb8 = (a.groups + 7) / 8;
    const int shard = static_cast<int>((g / 8) % S);
    const int64_t kb = shard < nb8 ? (nb8 - shard + S - 1) / S : 0;
    const int64_t members = kb * 8;
    const unsigned jn = static_cast<unsigned>((a.dyn_rows + B - 1) / B);
    const unsigned total = jn * static_cast<unsigned>(members);
    unsigned* ctr = a.queues + (static_cast<int64_t>(ct) * S + shard) * kWaves + wave;
    auto claim = [&]() {
      unsigned v = 0;
      if (lane == 0) v = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return v;
    };
    unsigned next = claim();
    while (true) {
      const unsigned cidx = __builtin_amdgcn_readfirstlane(next);
      if (cidx >= total) break;
      next = claim();
      const int64_t i = cidx % static_cast<unsigned>(members);
      const int64_t j = cidx / static_cast<unsigned>(members);
      const int64_t go = 8 * (shard + static_cast<int64_t>(S) * (i / 8)) + (i % 8);
      if (go >= a.groups) continue;
      const int64_t o0 = go * a.rows_per_g;
      int64_t o1 = o0 + a.rows_per_g;
      if (o1 > a.rows) o1 = a.rows;
      const int64_t onk = (active && o0 + ty < o1) ? (o1 - o0 - ty + ry - 1) >> ry_shift : 0;
      const bool opre = PA > 0 && static_cast<int>(go * ct_conc + ct - sl * ct_conc) +
                                          wave * static_cast<int>(gridDim.x) >= cs1 - cs0;
      int64_t qhi = onk - 1 - (opre ? PA : 0) - PB;  // owner's last streamed row
      if (qhi > qlo - 1) qhi = qlo - 1;              // owner's static rows end at qlo
      const int64_t qa = KR + KL + j * B;
      int64_t qb2 = qa + B - 1;
      if (qb2 > qhi) qb2 = qhi;
      const int64_t obase = (o0 + ty) * a.c;
      int64_t qq = qa;
      for (; qq + U - 1 <= qb2; qq += U) {
        uint4 xw[U], dw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          xw[u] = ld16_last(px + obase + (qq + u) * rstride);
          if constexpr (kGrad) dw[u] = ld16_last(pd + obase + (qq + u) * rstride);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
          st16(po + obase + (qq + u) * rstride, apply_words<Tr, kGrad>(xw[u], dw[u], cf));
      }
      for (; qq <= qb2; ++qq) {
        const uint4 xw = ld16_last(px + obase + qq * rstride);
        uint4 dw = xw;
        if constexpr (kGrad) dw = ld16_last(pd + obase + qq * rstride);
        st16(po + obase + qq * rstride, apply_words<Tr, kGrad>(xw, dw, cf));
      }
    }
  }
  stamp(6);

  }  // slices
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;

  // Exit (when chunks were handed out, and in a launch recorded into a
  // graph): counted in two levels - class counter, then the global counter -
  // and the workgroup that completes the count zeroes the chunk counters for
  // the next launch; in a recorded launch also the exit and class counters,
  // so every replay starts from zero, and it advances the replays' epoch
  // word.  Relaxed:
  // every counter this workgroup touched was updated by atomics whose
  // results it has already used, and no workgroup reads a counter after its
  // exit arrival.
  if (a.dyn_rows > 0 || a.reset_at_exit) {
    __syncthreads();
    if (wave == 0) {
      unsigned done = 0;
      if (lane == 0) {
        const unsigned r = blockIdx.x & 7;
        // Uniform selects over the by-value arguments (a dynamic index
        // would put them in scratch memory).
        unsigned last = a.sub_last[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) last = r == static_cast<unsigned>(i) ? a.sub_last[i] : last;
        const unsigned old =
            __hip_atomic_fetch_add(a.sub + 64 * r, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == last) {
          const unsigned long long g =
              __hip_atomic_fetch_add(a.barrier, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          done = g == a.base + barrier_classes() - 1;
        }
      }
      if (__builtin_amdgcn_readfirstlane(done)) {
        if (a.dyn_rows > 0) {
          for (int i = lane; i < a.ct * a.shards * kWaves; i += 64)
            __hip_atomic_store(a.queues + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (a.reset_at_exit) {
          if (lane < 8)
            __hip_atomic_store(a.sub + 64 * lane, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (lane == 0) {
            __hip_atomic_store(a.barrier, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // Every workgroup read the epoch word at its start: the next
            // replay gets the next epoch.
            if (a.epoch_dev)
              __hip_atomic_store(a.epoch_dev, (epoch - 0x80000001u + 1u) % 0x7fffffffu,
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 4b. Sliced gradient with the hand-offs hidden (NHWC, every workgroup one
//     row group running the channel tiles - slices - in turn).
//     After publishing slice s's partials, a workgroup does not wait idle
//     for slice s's coefficients: it first reads the streamed (not resident)
//     rows of slice s + 1 - their x and dy need no storage, only their sums,
//     which the workgroup reduces per channel into one register pair of the
//     thread owning the channel (`pend`) - then takes slice s's
//     coefficients, writes slice s's outputs (re-reading its streamed rows),
//     loads slice s + 1's resident rows into the freed registers and LDS,
//     and publishes slice s + 1's partials (resident rows, then `pend`).
//     Only the last slice's hand-off is a wait.  Registers in use are those
//     of the plain sliced pass plus `pend`.
// ---------------------------------------------------------------------------
// A copy of a row's words that the compiler cannot see through.
__device__ inline uint4 opaque_words(uint4 w) {
  asm volatile("" : "+v"(w.x), "+v"(w.y), "+v"(w.z), "+v"(w.w));
  return w;
}

template <class Tr, int KR, int KL>
__global__ __launch_bounds__(kFusedThreads) void bn_sliced_grad_kernel(FusedArgs a) {
  using S = typename Tr::S;
  constexpr int VEC = Tr::kVec;
  constexpr int U = 4;   // streamed vectors per tensor in flight, phase 1
  // Phase 3: 4 rows in flight, which leaves the registers for 3 more
  // resident rows per thread than 6 in flight (f16 15 against 12, bf16 14
  // against 11, f32 17 against 14; cfg2 16-op step 1.778 -> 1.770 ms, the
  // 28x28 bf16 grad 159 -> 155 us).
  constexpr int U3 = 4;
  extern __shared__ uint4 lds_rows[];  // [KL][2][kFusedThreads]
  __shared__ float2 red[(kFusedThreads / 64) * 32 * VEC];
  const int nslices = a.slices;
  const int width = (1 << a.tx_shift) * VEC;  // channels of a slice
  const unsigned epoch =
      a.epoch_dev ? 0x80000001u + __hip_atomic_load(a.epoch_dev, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT) % 0x7fffffffu
                  : a.epoch;
  const uint64_t etag = static_cast<uint64_t>(epoch) << 32;
  const uint32_t wtag = epoch ^ a.wait_xor;
  const int ry = kFusedThreads >> a.tx_shift;
  const int64_t g = blockIdx.x;  // one row group per workgroup, every slice
  const int64_t r0 = g * a.rows_per_g;
  int64_t r1 = r0 + a.rows_per_g;
  if (r1 > a.rows) r1 = a.rows;
  const int64_t gbytes = (r1 - r0) * a.c * static_cast<int64_t>(sizeof(S));
  const auto rx = rows_rsrc(static_cast<const S*>(a.x) + r0 * a.c, gbytes);
  const auto rd = rows_rsrc(static_cast<const S*>(a.dy) + r0 * a.c, gbytes);
  const uint32_t rstride_b =
      static_cast<uint32_t>(static_cast<int64_t>(ry) * a.c * static_cast<int64_t>(sizeof(S)));
  const int64_t rstride = static_cast<int64_t>(ry) * a.c;

  // Per-lane geometry of slice s for thread tid (tid is an opaque copy of
  // threadIdx.x made in each slice, so none of this stays live across the
  // slice loop).
  struct Lane {
    int tx, ty;
    bool active;
    int64_t nk, c0;
    uint32_t off;  // byte offset of row 0 in the group's buffer resources
  };
  auto lane_of = [&](int tid, int s) {
    Lane l;
    l.tx = tid & ((1 << a.tx_shift) - 1);
    l.ty = tid >> a.tx_shift;
    const int64_t cvi = static_cast<int64_t>(s) * (1 << a.tx_shift) + l.tx;
    l.active = cvi < a.cv;
    l.nk = l.active && r0 + l.ty < r1 ? (r1 - r0 - l.ty + ry - 1) >> (9 - a.tx_shift) : 0;
    l.c0 = l.active ? cvi * VEC : 0;
    l.off = l.active ? static_cast<uint32_t>((l.ty * static_cast<int64_t>(a.c) + l.c0) *
                                             static_cast<int64_t>(sizeof(S)))
                     : kOutOfRange;
    return l;
  };
  auto opaque_tid = []() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
  };
  auto load_k = [&](const Lane& l, float (&k)[VEC]) {
#pragma unroll
    for (int j = 0; j < VEC; ++j) k[j] = l.active ? a.fin.mean_in[l.c0 + j] : 0.f;
  };
  auto lds = [&](int tid, int q2, int which) -> uint4& {
    return lds_rows[(q2 * 2 + which) * kFusedThreads + tid];
  };
  // Streamed rows [KR + KL, nk) of lane l, accumulated.  Plain loads: phase
  // 3 re-reads these lines, and finding them in the Infinity Cache matters
  // (non-temporal loads here made the 56x56 grads 325 us instead of 285-289).
  auto stream_accum = [&](const Lane& l, const float (&k)[VEC], float (&s1)[VEC],
                          float (&s2)[VEC]) {
    const S* px = static_cast<const S*>(a.x) + (r0 + l.ty) * a.c + l.c0;
    const S* pd = static_cast<const S*>(a.dy) + (r0 + l.ty) * a.c + l.c0;
    int64_t q = KR + KL;
    for (; q + U <= l.nk; q += U) {
      uint4 xw[U], dw[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        xw[u] = ld16(px + (q + u) * rstride);
        dw[u] = ld16(pd + (q + u) * rstride);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) accum_words<Tr, true>(xw[u], dw[u], k, s1, s2);
    }
    if (q < l.nk) {
      uint4 xw[U], dw[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t o = l.off + static_cast<uint32_t>(q + u) * rstride_b;
        xw[u] = bld16(rx, o);
        dw[u] = bld16(rd, o);
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (q + u < l.nk) accum_words<Tr, true>(xw[u], dw[u], k, s1, s2);
    }
  };
  // Resident rows of lane l: KR into registers, KL into LDS, all loads in
  // flight before any is used (never re-read from memory: non-temporal),
  // then accumulated.
  uint4 xr[KR], dr[KR];
  auto resident_accum = [&](int tid, const Lane& l, const float (&k)[VEC], float (&s1)[VEC],
                            float (&s2)[VEC]) {
    uint4 xl[KL], dl[KL];
#pragma unroll
    for (int q = 0; q < KR; ++q) {
      const uint32_t o = l.off + static_cast<uint32_t>(q) * rstride_b;
      xr[q] = bld16_last(rx, o);
      dr[q] = bld16_last(rd, o);
    }
#pragma unroll
    for (int q = 0; q < KL; ++q) {
      const uint32_t o = l.off + static_cast<uint32_t>(KR + q) * rstride_b;
      xl[q] = bld16_last(rx, o);
      dl[q] = bld16_last(rd, o);
    }
    // Register rows are only ever used through opaque copies: rows loaded
    // here and used as 16-bit values in the next slice's phase 3 were
    // otherwise split into their halves at the load, both pieces live
    // across the hand-off (8 registers per row instead of 4; it spilled).
#pragma unroll
    for (int q = 0; q < KR; ++q)
      if (q < l.nk) accum_words<Tr, true>(opaque_words(xr[q]), opaque_words(dr[q]), k, s1, s2);
#pragma unroll
    for (int q = 0; q < KL; ++q) {
      lds(tid, q, 0) = xl[q];
      lds(tid, q, 1) = dl[q];
    }
#pragma unroll 2
    for (int q = 0; q < KL; ++q) {
      if (KR + q < l.nk) accum_words<Tr, true>(lds(tid, q, 0), lds(tid, q, 1), k, s1, s2);
    }
  };

  // Slice 0: the whole phase 1, then its partials.
  {
    const int tid = opaque_tid();
    const Lane l = lane_of(tid, 0);
    float k[VEC], s1[VEC], s2[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) s1[j] = s2[j] = 0.f;
    load_k(l, k);
    resident_accum(tid, l, k, s1, s2);
    stream_accum(l, k, s1, s2);
    publish_partials<VEC>(a, red, s1, s2, tid, width, 0, g, etag);
  }

#pragma clang loop unroll(disable)
  for (int sl = 0; sl < nslices; ++sl) {
    const int tid = opaque_tid();
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const Lane l = lane_of(tid, sl);
    const int cs0 = sl * width;
    const int cs1 = a.c < cs0 + width ? a.c : cs0 + width;
    // ---- phase 2 of slice sl ----
    finish_channel_blocks<Tr, true>(a, cs0, cs1, wave, lane, wtag, etag, epoch);
    if (sl == 0) zero_side_outputs<true>(a.fin);
    const bool more = sl + 1 < nslices;
    // ---- while slice sl's coefficients are pending: the streamed rows of
    // slice sl + 1, summed per channel into `pend` ----
    float2 pend = make_float2(0.f, 0.f);
    if (more) {
      const Lane ln = lane_of(tid, sl + 1);
      float k[VEC], s1[VEC], s2[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) s1[j] = s2[j] = 0.f;
      load_k(ln, k);
      stream_accum(ln, k, s1, s2);
      pend = workgroup_sums<VEC>(a, red, s1, s2, tid, width);
    }
    // ---- phase 3 of slice sl ----
    float4 cf[VEC];
    tile_coefs<Tr>(a, red, tid, l.tx, sl, width, l.active, wtag, epoch, cf);
    {
      const S* px = static_cast<const S*>(a.x) + (r0 + l.ty) * a.c + l.c0;
      const S* pd = static_cast<const S*>(a.dy) + (r0 + l.ty) * a.c + l.c0;
      S* po = static_cast<S*>(a.out) + (r0 + l.ty) * a.c + l.c0;
      const int64_t qlo = KR + KL;
      int64_t q = l.nk - 1;
      for (; q >= qlo + U3 - 1; q -= U3) {
        uint4 xw[U3], dw[U3];
#pragma unroll
        for (int u = 0; u < U3; ++u) {
          xw[u] = ld16_last(px + (q - u) * rstride);
          dw[u] = ld16_last(pd + (q - u) * rstride);
        }
#pragma unroll
        for (int u = 0; u < U3; ++u)
          st16(po + (q - u) * rstride, apply_words<Tr, true>(xw[u], dw[u], cf));
      }
      if (q >= qlo) {  // fewer than U3 rows left: loads issued together
        uint4 xw[U3], dw[U3];
#pragma unroll
        for (int u = 0; u < U3; ++u) {
          const uint32_t o = q - u >= qlo ? l.off + static_cast<uint32_t>(q - u) * rstride_b
                                          : kOutOfRange;
          xw[u] = bld16_last(rx, o);
          dw[u] = bld16_last(rd, o);
        }
#pragma unroll
        for (int u = 0; u < U3; ++u)
          if (q - u >= qlo) st16(po + (q - u) * rstride, apply_words<Tr, true>(xw[u], dw[u], cf));
      }
#pragma unroll 2
      for (int q2 = 0; q2 < KL; ++q2) {
        if (KR + q2 < l.nk)
          st16(po + (KR + q2) * rstride,
               apply_words<Tr, true>(lds(tid, q2, 0), lds(tid, q2, 1), cf));
      }
#pragma unroll
      for (int r = 0; r < KR; ++r)
        if (r < l.nk)
          st16(po + r * rstride, apply_words<Tr, true>(opaque_words(xr[r]), opaque_words(dr[r]), cf));
    }
    // ---- phase 1 of slice sl + 1: its resident rows, then its partials ----
    if (more) {
      const Lane ln = lane_of(tid, sl + 1);
      float k[VEC], s1[VEC], s2[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) s1[j] = s2[j] = 0.f;
      load_k(ln, k);
      resident_accum(tid, ln, k, s1, s2);
      // Every thread has read slice sl's coefficients out of `red` before
      // the reduction below writes it.
      __syncthreads();
      publish_partials<VEC>(a, red, s1, s2, tid, width, sl + 1, g, etag, pend);
    }
  }
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  // Exit of a launch recorded into a graph: counted in two levels; the
  // workgroup completing the count zeroes the counters and advances the
  // replays' epoch word (as in bn_fused_nhwc_kernel, which documents the
  // orderings).
  if (a.reset_at_exit) {
    __syncthreads();
    if (wave == 0) {
      unsigned done = 0;
      if (lane == 0) {
        const unsigned r = blockIdx.x & 7;
        unsigned last = a.sub_last[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) last = r == static_cast<unsigned>(i) ? a.sub_last[i] : last;
        const unsigned old =
            __hip_atomic_fetch_add(a.sub + 64 * r, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == last) {
          const unsigned long long gg =
              __hip_atomic_fetch_add(a.barrier, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          done = gg == a.base + barrier_classes() - 1;
        }
      }
      if (__builtin_amdgcn_readfirstlane(done)) {
        if (lane < 8)
          __hip_atomic_store(a.sub + 64 * lane, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0) {
          __hip_atomic_store(a.barrier, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (a.epoch_dev)
            __hip_atomic_store(a.epoch_dev, (epoch - 0x80000001u + 1u) % 0x7fffffffu,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 5. NCHW, one channel per workgroup: workgroup ch sums, finishes and applies
//    channel ch alone, so no value crosses workgroups - no waits, no
//    co-residency assumption, any number of workgroups in flight.  The
//    channel's vectors (its N planes, 16 bytes each, plane % VEC == 0) are
//    dealt to the 512 threads in turn: vector i = tid + q * 512 of the
//    channel is the thread's row q.  As in the NHWC kernel, a thread's first
//    KR rows stay in VGPRs, the next KL in LDS, the rest are re-read in
//    phase 3 (last-to-first, from the Infinity Cache when they are still
//    there).  All loads go through one buffer resource over the channel's
//    span of the tensor (the host keeps the tensor below 2^31 bytes): a row
//    past the channel's last vector lies past the span, reads zeros and
//    makes no memory request, so no load needs a branch.
// ---------------------------------------------------------------------------
struct NchwArgs {
  const void* x;
  const void* dy;
  void* out;
  int64_t n;      // images
  int c;          // channels
  int64_t plane;  // elements per (image, channel) plane
  int64_t pv;     // 16-byte vectors per plane
  FinArgs fin;
};

// Register rows per thread (the largest spill-free counts; LDS rows as in the
// NHWC kernel).
template <class Tr> struct OwnedRows { static constexpr int kFwd = 30, kGrad = 16; };
template <> struct OwnedRows<TF16> { static constexpr int kFwd = 30, kGrad = 17; };
template <> struct OwnedRows<TBF16> { static constexpr int kFwd = 31, kGrad = 15; };

template <class Tr, bool kGrad, int KR, int KL>
__global__ __launch_bounds__(kFusedThreads) void bn_nchw_owned_kernel(NchwArgs a) {
  using S = typename Tr::S;
  constexpr int VEC = Tr::kVec;
  constexpr int kIn = kGrad ? 2 : 1;
  constexpr int U = kGrad ? 4 : 8;  // streamed vectors per tensor in flight
  constexpr int kWaves = kFusedThreads / 64;
  extern __shared__ uint4 lds_rows[];  // [KL][kIn][kFusedThreads]
  __shared__ double red[2][kWaves];
  __shared__ float cfs[4];
  const int tid = threadIdx.x;
  const int ch = blockIdx.x;
  const int64_t nv = a.n * a.pv;  // vectors of the channel
  const int64_t nk = tid < nv ? (nv - tid + kFusedThreads - 1) / kFusedThreads : 0;
  // Byte offset of this thread's row q from the channel's first plane:
  // img * c * plane * s + v * 16 for channel vector (img, v).  Rows advance
  // by kFusedThreads vectors: dimg images and dv vectors (with carry).
  const uint32_t img_b = static_cast<uint32_t>(a.c * a.plane * static_cast<int64_t>(sizeof(S)));
  const uint32_t dimg = static_cast<uint32_t>(kFusedThreads / a.pv);
  const uint32_t dv = static_cast<uint32_t>(kFusedThreads % a.pv);
  const uint32_t pv = static_cast<uint32_t>(a.pv);
  uint32_t img0 = static_cast<uint32_t>(tid / a.pv), v0 = static_cast<uint32_t>(tid % a.pv);
  auto step = [&](uint32_t& img, uint32_t& v) {
    v += dv;
    const bool carry = v >= pv;
    v = carry ? v - pv : v;
    img += dimg + (carry ? 1u : 0u);
  };
  auto off_of = [&](uint32_t img, uint32_t v) { return img * img_b + v * 16u; };
  const int64_t chan0 = static_cast<int64_t>(ch) * a.plane;  // element offset of plane (0, ch)
  const int64_t span = ((a.n - 1) * a.c * a.plane + a.plane) * static_cast<int64_t>(sizeof(S));
  const auto rx = rows_rsrc(static_cast<const S*>(a.x) + chan0, span);
  const auto rd = rows_rsrc(kGrad ? static_cast<const S*>(a.dy) + chan0 : a.x, span);
  char* const obase = reinterpret_cast<char*>(static_cast<S*>(a.out) + chan0);
  auto lds = [&](int q2, int which) -> uint4& {
    return lds_rows[(q2 * kIn + which) * kFusedThreads + tid];
  };

  // ---- phase 1: the channel's sums ----------------------------------------
  const float kk = kGrad ? a.fin.mean_in[ch]
                         : chan_shift<Tr>(static_cast<const S*>(a.x), ch, a.n * a.plane, a.c,
                                          a.plane);
  float k[VEC], s1[VEC], s2[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    k[j] = kk;
    s1[j] = 0.f;
    s2[j] = 0.f;
  }
  uint4 xr[KR];
  uint4 dr[kGrad ? KR : 1];
  uint4 xl[KL];
  uint4 dl[kGrad ? KL : 1];
  uint32_t img = img0, v = v0;
#pragma unroll
  for (int q = 0; q < KR; ++q) {
    const uint32_t o = off_of(img, v);
    xr[q] = bld16(rx, o);
    if constexpr (kGrad) dr[q] = bld16(rd, o);
    step(img, v);
  }
#pragma unroll
  for (int q = 0; q < KL; ++q) {
    const uint32_t o = off_of(img, v);
    xl[q] = bld16(rx, o);
    if constexpr (kGrad) dl[q] = bld16(rd, o);
    step(img, v);
  }
  const uint32_t img_s = img, v_s = v;  // first streamed row
#pragma unroll
  for (int q = 0; q < KR; ++q) {
    if (q < nk) accum_words<Tr, kGrad>(xr[q], dr[kGrad ? q : 0], k, s1, s2);
    if constexpr (kGrad ? Resident<Tr>::kOpaqueGrad : Resident<Tr>::kOpaqueFwd) {
      asm volatile("" : "+v"(xr[q].x), "+v"(xr[q].y), "+v"(xr[q].z), "+v"(xr[q].w));
      if constexpr (kGrad)
        asm volatile("" : "+v"(dr[q].x), "+v"(dr[q].y), "+v"(dr[q].z), "+v"(dr[q].w));
    }
  }
#pragma unroll
  for (int q = 0; q < KL; ++q) {
    lds(q, 0) = xl[q];
    if constexpr (kGrad) lds(q, kGrad ? 1 : 0) = dl[kGrad ? q : 0];
  }
#pragma unroll 2
  for (int q = 0; q < KL; ++q) {
    if (KR + q < nk) {
      const uint4 xw = lds(q, 0);
      const uint4 dw = kGrad ? lds(q, kGrad ? 1 : 0) : xw;
      accum_words<Tr, kGrad>(xw, dw, k, s1, s2);
    }
  }
  // Streamed rows, U in flight (rows past nk read zeros and are not summed).
  for (int64_t q = KR + KL; q < nk; q += U) {
    uint4 xw[U], dw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t o = off_of(img, v);
      xw[u] = bld16(rx, o);
      if constexpr (kGrad) dw[u] = bld16(rd, o);
      step(img, v);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (q + u < nk) accum_words<Tr, kGrad>(xw[u], dw[u], k, s1, s2);
  }
  // The forward's other inputs (K is kk; scale, offset in flight during the
  // reduction below).  The grad loads its inputs after the reduction: loaded
  // here, they cost the grad kernels registers they do not have.
  FinIn fin_in{};
  if constexpr (!kGrad) fin_in = fin_inputs<Tr, kGrad>(a.fin, ch, kk);
  // The workgroup's sums: per thread in float, then in double across the
  // threads in a fixed order (wave shuffles, then the waves in order).
  float ta = 0.f, tb = 0.f;
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    ta += s1[j];
    tb += s2[j];
  }
  const double2 w = wave_sum(static_cast<double>(ta), static_cast<double>(tb));
  const int wave = tid >> 6;
  if ((tid & 63) == 0) {
    red[0][wave] = w.x;
    red[1][wave] = w.y;
  }
  __syncthreads();
  if (tid == 0) {
    double t1 = 0.0, t2 = 0.0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
      t1 += red[0][i];
      t2 += red[1][i];
    }
    float4 cf;
    if constexpr (kGrad)
      cf = finish_channel<Tr, kGrad>(a.fin, ch, t1, t2);
    else
      cf = finish_channel<Tr, kGrad>(a.fin, ch, t1, t2, fin_in);
    cfs[0] = cf.x;
    cfs[1] = cf.y;
    cfs[2] = cf.z;
    cfs[3] = cf.w;
  }
  zero_side_outputs<kGrad>(a.fin);
  __syncthreads();
  const float4 cone = make_float4(cfs[0], cfs[1], cfs[2], cfs[3]);
  float4 cf[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) cf[j] = cone;

  // ---- phase 3: outputs ----------------------------------------------------
  // Streamed rows last-to-first: walk forward to find the last row's
  // position, then step backwards.
#pragma unroll
  for (int r = 0; r < KR; ++r) {
    asm volatile("" : "+v"(xr[r].x), "+v"(xr[r].y), "+v"(xr[r].z), "+v"(xr[r].w));
    if constexpr (kGrad)
      asm volatile("" : "+v"(dr[r].x), "+v"(dr[r].y), "+v"(dr[r].z), "+v"(dr[r].w));
  }
  if (nk > KR + KL) {
    // Row nk - 1's position: (nk - 1 - (KR + KL)) steps past the first
    // streamed row.
    const uint64_t steps = static_cast<uint64_t>(nk - 1 - (KR + KL));
    const uint64_t vv = v_s + steps * dv;
    uint32_t bimg = img_s + static_cast<uint32_t>(steps * dimg + vv / pv);
    uint32_t bv = static_cast<uint32_t>(vv % pv);
    auto back = [&](uint32_t& im, uint32_t& vi) {
      const bool borrow = vi < dv;
      vi = borrow ? vi + pv - dv : vi - dv;
      im -= dimg + (borrow ? 1u : 0u);
    };
    int64_t q = nk - 1;
    for (; q >= KR + KL + U - 1; q -= U) {
      uint4 xw[U], dw[U];
      uint32_t os[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        os[u] = off_of(bimg, bv);
        xw[u] = bld16_last(rx, os[u]);
        if constexpr (kGrad) dw[u] = bld16_last(rd, os[u]);
        back(bimg, bv);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) st16(obase + os[u], apply_words<Tr, kGrad>(xw[u], dw[u], cf));
    }
    for (; q >= KR + KL; --q) {
      const uint32_t o = off_of(bimg, bv);
      const uint4 xw = bld16_last(rx, o);
      uint4 dw = xw;
      if constexpr (kGrad) dw = bld16_last(rd, o);
      st16(obase + o, apply_words<Tr, kGrad>(xw, dw, cf));
      back(bimg, bv);
    }
  }
  img = img0;
  v = v0;
#pragma unroll
  for (int r = 0; r < KR; ++r) {
    if (r < nk) st16(obase + off_of(img, v), apply_words<Tr, kGrad>(xr[r], dr[kGrad ? r : 0], cf));
    step(img, v);
  }
#pragma unroll 2
  for (int q2 = 0; q2 < KL; ++q2) {
    if (KR + q2 < nk) {
      const uint4 xw = lds(q2, 0);
      const uint4 dw = kGrad ? lds(q2, kGrad ? 1 : 0) : xw;
      st16(obase + off_of(img, v), apply_words<Tr, kGrad>(xw, dw, cf));
    }
    step(img, v);
  }
}

// ---------------------------------------------------------------------------
// Host drivers.
// ---------------------------------------------------------------------------
template <class Tr, int VEC, bool kGrad>
hipError_t launch_reduce(const Plan& p, const BnGeometry& g, const void* x,
                         const void* dy, const float* mean_in, float2* partial,
                         hipStream_t stream) {
  using S = typename Tr::S;
  if (p.nhwc) {
    const size_t smem = static_cast<size_t>(kThreads) * VEC * sizeof(float2);
    TFMA_LAUNCH(kGrad ? "tfma_bn_grad_reduce" : "tfma_bn_fwd_reduce", (bn_nhwc_reduce_kernel<Tr, VEC, kGrad>),
                       dim3(p.ct, p.groups), dim3(kThreads), smem, stream,
                       static_cast<const S*>(x), static_cast<const S*>(dy),
                       mean_in, g.rows, static_cast<int>(g.c), p.cv, p.tx_shift,
                       p.rows_per_g, partial);
  } else {
    TFMA_LAUNCH(kGrad ? "tfma_bn_grad_reduce_nchw" : "tfma_bn_fwd_reduce_nchw", (bn_nchw_reduce_kernel<Tr, VEC, kGrad>),
                       dim3(p.groups, g.c), dim3(kThreads), 0, stream,
                       static_cast<const S*>(x), static_cast<const S*>(dy),
                       mean_in, g.n, static_cast<int>(g.c), g.h * g.w, p.cv,
                       p.rows_per_g, FastDiv(static_cast<uint32_t>(p.cv)),
                       partial);
  }
  return hipGetLastError();
}

// kInfer: the inference forward (coefficients from fa's running statistics,
// statistics outputs written by the same launch; coef unused).
template <class Tr, int VEC, bool kGrad, bool kInfer = false>
hipError_t launch_apply(const Plan& p, const BnGeometry& g, const void* x,
                        const void* dy, void* out, const float4* coef,
                        hipStream_t stream, const FinArgs& fa = FinArgs{}) {
  using S = typename Tr::S;
  if (p.nhwc) {
    TFMA_LAUNCH(kInfer ? "tfma_bn_infer_apply" : (kGrad ? "tfma_bn_grad_apply" : "tfma_bn_fwd_apply"),
                       (bn_nhwc_apply_kernel<Tr, VEC, kGrad, kInfer>),
                       dim3(p.ct, p.groups), dim3(kThreads), 0, stream,
                       static_cast<const S*>(x), static_cast<const S*>(dy),
                       static_cast<S*>(out), coef, g.rows, static_cast<int>(g.c),
                       p.cv, p.tx_shift, p.rows_per_g, p.groups, fa);
  } else {
    const int64_t nvec = g.n * g.c * p.cv;
    int64_t blocks = (nvec + kThreads * 4 - 1) / (kThreads * 4);
    const int64_t maxb = static_cast<int64_t>(DeviceCUs()) * 16;
    if (blocks > maxb) blocks = maxb;
    if (blocks < 1) blocks = 1;
    TFMA_LAUNCH(kInfer ? "tfma_bn_infer_apply_nchw"
                       : (kGrad ? "tfma_bn_grad_apply_nchw" : "tfma_bn_fwd_apply_nchw"),
                (bn_nchw_apply_kernel<Tr, VEC, kGrad, kInfer>), dim3(blocks),
                       dim3(kThreads), 0, stream, static_cast<const S*>(x),
                       static_cast<const S*>(dy), static_cast<S*>(out), coef,
                       nvec, p.cv, static_cast<int>(g.c), fa);
  }
  return hipGetLastError();
}

template <class Tr, bool kGrad>
hipError_t launch_finalize(const Plan& p, const FinArgs& fa,
                           const float2* partial, float4* coef,
                           hipStream_t stream) {
  const int blocks = (fa.c + kFinCh - 1) / kFinCh;
  TFMA_LAUNCH(kGrad ? "tfma_bn_grad_finalize" : "tfma_bn_fwd_finalize", (bn_finalize_kernel<Tr, kGrad>), dim3(blocks), dim3(kFinThreads), 0,
                     stream, partial, fa, coef);
  (void)p;
  return hipGetLastError();
}

// ---- fused path host side --------------------------------------------------
bool fused_enabled() {
  static bool on = [] {
    const char* e = getenv("TFMA_BN_FUSED");
    return !(e && e[0] == '0');
  }();
  return on;
}

// Upper bound on fused workgroups (one or two per CU); sizes the partials.
int64_t fused_group_bound() { return 2 * static_cast<int64_t>(DeviceCUs()); }

template <class Tr, bool kGrad>
constexpr int fused_kr() { return kGrad ? Resident<Tr>::kRegGrad : Resident<Tr>::kRegFwd; }
template <class Tr, bool kGrad>
constexpr int fused_kl() { return kGrad ? Resident<Tr>::kLdsGrad : Resident<Tr>::kLdsFwd; }

constexpr int64_t kSmallFwdRows = 64;

template <class Tr, bool kGrad, int KR = fused_kr<Tr, kGrad>(), bool kSliced = false>
const void* fused_kernel() {
  return reinterpret_cast<const void*>(
      &bn_fused_nhwc_kernel<Tr, kGrad, KR, fused_kl<Tr, kGrad>(), kSliced>);
}

template <class Tr, bool kGrad>
size_t fused_smem() {
  return static_cast<size_t>(fused_kl<Tr, kGrad>()) * (kGrad ? 2 : 1) * kFusedThreads * 16;
}

// The sliced grad kernel (the slice loop costs registers: kRegGradSliced is
// the largest spill-free count).
template <class Tr>
const void* sliced_kernel() {
  return fused_kernel<Tr, true, Resident<Tr>::kRegGradSliced, true>();
}

// The sliced grad that hides its slices' hand-offs (8-vector tiles, no
// dynamic tail): the plain sliced kernel's residency.
template <class Tr>
const void* sliced_overlap_kernel() {
  return reinterpret_cast<const void*>(
      &bn_sliced_grad_kernel<Tr, Resident<Tr>::kRegGradOverlap, Resident<Tr>::kLdsGrad>);
}

// The "bn_sliced_overlap" override 0 (tests and measurements): sliced grads
// run the plain sliced kernel.
bool sliced_overlap_enabled() { return TuneValue(kTuneBnSlicedOverlap) != 0; }

// Per device: the sliced kernel has the unsliced kernel's occupancy (set by
// fused_blocks_per_cu before it publishes its count).
template <class Tr, bool kGrad>
std::atomic<bool>* sliced_ok() {
  static std::atomic<bool> ok[64];
  return ok;
}

// Co-resident workgroups per CU for the fused kernel (0 if it cannot run).
// Computed once per device; threads that race to compute it store the same
// values.
template <class Tr, bool kGrad>
int fused_blocks_per_cu() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  const int known = cached[dev].load(std::memory_order_acquire);
  if (known != 0) return known;
  {
    int nb = 0, sliced_ns = 0;
    hipError_t e = hipFuncSetAttribute(fused_kernel<Tr, kGrad>(),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(fused_smem<Tr, kGrad>()));
    if constexpr (!kGrad) {  // the small-shape forward: same LDS, fewer VGPRs
      if (e == hipSuccess)
        e = hipFuncSetAttribute(fused_kernel<Tr, kGrad, Resident<Tr>::kRegFwdSmall>(),
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(fused_smem<Tr, kGrad>()));
    }
    if constexpr (kGrad) {  // the sliced grads: same LDS, and they must fit as often
      int overlap_ns = 0;
      if (e == hipSuccess)
        e = hipFuncSetAttribute(sliced_kernel<Tr>(), hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(fused_smem<Tr, kGrad>()));
      if (e == hipSuccess)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&sliced_ns, sliced_kernel<Tr>(),
                                                         kFusedThreads, fused_smem<Tr, kGrad>());
      if (e == hipSuccess)
        e = hipFuncSetAttribute(sliced_overlap_kernel<Tr>(),
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(fused_smem<Tr, kGrad>()));
      if (e == hipSuccess)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&overlap_ns, sliced_overlap_kernel<Tr>(),
                                                         kFusedThreads, fused_smem<Tr, kGrad>());
      if (overlap_ns < sliced_ns) sliced_ns = overlap_ns;
    }
    if (e == hipSuccess)
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fused_kernel<Tr, kGrad>(),
                                                       kFusedThreads, fused_smem<Tr, kGrad>());
    if (e != hipSuccess || nb < 1) nb = -1;
    const int count = nb > 2 ? 2 : nb;
    sliced_ok<Tr, kGrad>()[dev].store(nb >= 1 && sliced_ns >= count, std::memory_order_relaxed);
    cached[dev].store(count, std::memory_order_release);
    return count;
  }
}

struct FusedPlan {
  int tx_shift;
  int ct;
  int ct_conc = 0;  // tiles in flight at once (= ct unless sliced)
  int slices = 1;   // > 1: each workgroup runs ct / ct_conc tiles in turn
  int64_t cv;
  int64_t groups;
  int64_t rows_per_g;
  int blocks;
  int dyn_rows;   // per-thread streamed rows handed out dynamically
  int dyn_chunk;  // rows per thread in one chunk
};

// Channels of the largest fused plan (at most 2 workgroups per CU, tiles of
// at most 256 channels), and the words from one copy of the epoch-tagged
// coefficients ([C][4]) to the next: 4 KiB + 256 B more than a copy holds,
// so the copies start at different offsets within a page.
int64_t max_fused_channels() { return static_cast<int64_t>(2 * DeviceCUs()) * 256; }
size_t coef_copy_words() { return static_cast<size_t>(max_fused_channels()) * 4 + 544; }

// Share of each thread's streamed rows (after the prefetched ones) that is
// handed out dynamically in phase 3 (percent; TFMA_BN_DYN_PCT, default 20).
int dyn_pct() {
  static int v = [] {
    const char* e = getenv("TFMA_BN_DYN_PCT");
    const int p = e ? atoi(e) : 20;
    return p < 0 ? 0 : (p > 100 ? 100 : p);
  }();
  return v;
}

bool make_fused_plan(const BnGeometry& g, int vec, int blocks_per_cu, FusedPlan* fp) {
  if (!g.nhwc || blocks_per_cu < 1 || g.c % vec != 0) return false;
  fp->cv = g.c / vec;
  int s = pow2_ceil_log2(fp->cv);
  if (s > 5) s = 5;
  fp->tx_shift = s;
  const int tx = 1 << s;
  fp->ct = static_cast<int>((fp->cv + tx - 1) / tx);
  const int64_t max_blocks = static_cast<int64_t>(blocks_per_cu) * DeviceCUs();
  int64_t groups = max_blocks / fp->ct;
  if (groups < 1) return false;
  const int ry = kFusedThreads / tx;
  // Fewer groups when rows are scarce: every thread gets at least one row.
  const int64_t max_groups = (g.rows + ry - 1) / ry;
  if (groups > max_groups) groups = max_groups;
  if (groups > fused_group_bound()) groups = fused_group_bound();
  if (groups > kMaxEpochGroups) groups = kMaxEpochGroups;  // partials a finishing wave reads
  fp->rows_per_g = (g.rows + groups - 1) / groups;
  // The kernel reads a workgroup's own rows through a buffer resource with
  // 32-bit offsets (rows past the group are out of range and read nothing):
  // the group's span plus the rows a thread may address past its last one
  // (fewer than 64 row passes) must stay below 2^31 bytes.
  const int64_t esz = 16 / vec;
  if ((fp->rows_per_g + 64 * static_cast<int64_t>(ry)) * g.c * esz >= (int64_t{1} << 31))
    return false;
  fp->groups = (g.rows + fp->rows_per_g - 1) / fp->rows_per_g;
  fp->blocks = static_cast<int>(fp->groups * fp->ct);
  fp->ct_conc = fp->ct;
  fp->slices = 1;
  fp->dyn_rows = 0;
  fp->dyn_chunk = 1;
  return true;
}

// Sliced plan: tiles of 2^tx_shift channel vectors, ct_conc of them in
// flight, each workgroup running ct / ct_conc of them in turn (one row group
// of all blocks / ct_conc per workgroup).
bool make_sliced_plan(const BnGeometry& g, int vec, int blocks_per_cu, int tx_shift, int ct_conc,
                      FusedPlan* fp) {
  if (!g.nhwc || blocks_per_cu < 1 || g.c % vec != 0 || tx_shift < 0 || tx_shift > 5 ||
      ct_conc < 1)
    return false;
  fp->cv = g.c / vec;
  fp->tx_shift = tx_shift;
  const int tx = 1 << tx_shift;
  const int64_t tiles = (fp->cv + tx - 1) / tx;
  if (tiles < 2 || tiles % ct_conc != 0 || tiles / ct_conc < 2) return false;
  fp->ct = static_cast<int>(tiles);
  fp->ct_conc = ct_conc;
  fp->slices = static_cast<int>(tiles / ct_conc);
  const int64_t max_blocks = static_cast<int64_t>(blocks_per_cu) * DeviceCUs();
  int64_t groups = max_blocks / ct_conc;
  if (groups < 1) return false;
  const int ry = kFusedThreads / tx;
  const int64_t max_groups = (g.rows + ry - 1) / ry;
  if (groups > max_groups) groups = max_groups;
  if (groups > fused_group_bound()) groups = fused_group_bound();
  if (groups > kMaxEpochGroups) groups = kMaxEpochGroups;
  // The epoch-tagged partial slots hold at most 512 * CUs (group, channel)
  // values.
  if (groups * g.c > 512 * static_cast<int64_t>(DeviceCUs())) return false;
  fp->rows_per_g = (g.rows + groups - 1) / groups;
  const int64_t esz = 16 / vec;
  if ((fp->rows_per_g + 64 * static_cast<int64_t>(ry)) * g.c * esz >= (int64_t{1} << 31))
    return false;
  fp->groups = (g.rows + fp->rows_per_g - 1) / fp->rows_per_g;
  fp->blocks = static_cast<int>(fp->groups * ct_conc);
  fp->dyn_rows = 0;
  fp->dyn_chunk = 1;
  return true;
}

// A gradient is sliced when the x + dy rows its unsliced plan re-reads in
// phase 3 exceed kGradSliceAbove (more than the 256 MB Infinity Cache keeps
// for the re-read), into the fewest slices whose re-read stays below
// kGradSliceStreamMax.
constexpr int64_t kGradSliceAbove = int64_t(192) << 20;
constexpr int64_t kGradSliceStreamMax = int64_t(128) << 20;

// The fused plan of an NHWC op.  A gradient whose unsliced plan re-reads more
// x + dy in phase 3 than the Infinity Cache keeps for it runs sliced: every
// workgroup runs the two-phase pass once per channel tile in turn, with the
// widest tiles (fewest slices and hand-offs) whose per-slice re-read stays
// below kGradSliceStreamMax - cfg2's 256x56x56x256 in 4 slices of 8
// vectors (128-byte row segments, the narrowest that read whole cache
// lines), 256x28x28x512 in 2 of 32.  Forwards are not sliced (measured
// slower: a slice's read-only phase 1 and write-only phase 3 stream slower
// than the unsliced phase 3, which reads and writes at once).
// The "bn_slice_tw" override (tests and measurements): 0 never slices; 4,
// 8, 16 or 32 slices every grad that has such a plan, with tiles of that
// many vectors.
template <class Tr, bool kGrad>
bool choose_fused_plan(const BnGeometry& g, int vec, FusedPlan* fp) {
  const int bpc = fused_blocks_per_cu<Tr, kGrad>();
  if (!make_fused_plan(g, vec, bpc, fp)) return false;
  if constexpr (kGrad) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64 ||
        !sliced_ok<Tr, kGrad>()[dev].load(std::memory_order_relaxed))
      return true;
    const int tw = TuneValue(kTuneBnSliceTw);
    if (tw == 0) return true;
    if (tw == 4 || tw == 8 || tw == 16 || tw == 32) {
      FusedPlan sp;
      if (make_sliced_plan(g, vec, bpc, __builtin_ctz(tw), 1, &sp) &&
          sp.slices <= 8)
        *fp = sp;
      return true;
    }
    // x + dy rows that phase 3 re-reads (those not held on chip), in bytes.
    constexpr int kRes = Resident<Tr>::kRegGradOverlap + Resident<Tr>::kLdsGrad;
    const int64_t threads = static_cast<int64_t>(fp->blocks) * kFusedThreads;
    auto streamed_bytes = [&](const FusedPlan& p) {
      const int ry = kFusedThreads >> p.tx_shift;
      const int64_t nk = (p.rows_per_g + ry - 1) / ry;
      return (nk > kRes ? nk - kRes : 0) * 32 * threads;
    };
    if (streamed_bytes(*fp) <= kGradSliceAbove) return true;
    for (int shift = 5; shift >= 3; --shift) {
      FusedPlan sp;
      if (!make_sliced_plan(g, vec, bpc, shift, 1, &sp) || sp.slices > 8) continue;
      if (streamed_bytes(sp) > kGradSliceStreamMax) continue;
      *fp = sp;
      return true;
    }
    // Too large for any slice to keep its re-read in the cache: the
    // narrowest tiles (fewest rows on chip to re-read per slice).
    FusedPlan sp;
    if (make_sliced_plan(g, vec, bpc, 3, 1, &sp) && sp.slices <= 8) *fp = sp;
  }
  return true;
}

// Fills in the dynamic share for kernel <Tr, kGrad>: resident rows KR + KL,
// prefetched rows PA + PB and U rows per loop step (chunks of 2U rows).
void set_dynamic_share(FusedPlan* fp, int resident, int prefetched, int u) {
  const int ry = kFusedThreads >> fp->tx_shift;
  const int64_t nk = (fp->rows_per_g + ry - 1) / ry;
  const int64_t streamed = nk - resident - prefetched;
  static const int mult = [] {
    const char* e = getenv("TFMA_BN_DYN_CHUNK");  // chunk = mult * U rows per thread
    const int m = e ? atoi(e) : 2;
    return m < 1 ? 1 : (m > 8 ? 8 : m);
  }();
  const int chunk = mult * u;
  int64_t d = streamed * dyn_pct() / 100 / chunk * chunk;
  if (d < chunk) d = 0;
  fp->dyn_rows = static_cast<int>(d);
  fp->dyn_chunk = chunk;
}

// Per-device state of the fused kernels: a monotonic exit-arrival counter in
// device memory (zeroed once), its value before the next launch, the
// epoch-tagged value regions and the last epoch, and the launch chain
// (LaunchChain: a launch on another stream than the previous one waits for
// it; once a device has seen two streams every launch carries the
// dispatch's own end event, hipExtLaunchKernelGGL's stop event, not a marker
// after it - a marker between kernels costs microseconds).  So at most one
// persistent grid is resident at a time and every launch knows the
// counter's starting value.
// The allocation also holds the dynamic-chunk counters (from byte 256),
// which the last workgroup of each launch zeroes again.  A second, identical
// region serves launches recorded into a graph (stream capture): they start
// from zero counters and zero them again at exit, so replays need no host
// bookkeeping; they are not chained to other fused launches (the graph
// orders them), so a replay must not overlap other fused BatchNorm work on
// the device.
constexpr size_t kEpochOffset = 16;  // recorded region: the replays' epoch word
constexpr size_t kQueueOffset = 256;
constexpr size_t kQueueBytes = 4096 * sizeof(unsigned);  // <= 512 tiles x 8 waves
constexpr size_t kSubOffset = kQueueOffset + kQueueBytes;  // 8 class counters, 256 B apart
constexpr size_t kStateBytes = kSubOffset + 8 * 256;
struct BarrierState {
  std::mutex mu;
  unsigned long long* counter = nullptr;  // [0] arrivals
  unsigned long long base = 0;
  unsigned sub_base[8] = {0, 0, 0, 0, 0, 0, 0, 0};  // class counters (mod 2^32)
  LaunchChain chain;           // orders launches from different streams
  unsigned long long* eslots = nullptr;  // epoch-tagged partials, zeroed at creation
  size_t eslot_bytes = 0;
  unsigned long long* ecoef = nullptr;   // epoch-tagged coefficients, zeroed at creation
  size_t ecoef_bytes = 0;
  unsigned epoch = 0;                    // last epoch handed to a launch (< 2^31)
  // Give-up word in pinned host memory (coherent, mapped): a launch whose
  // wait ran out stores its epoch there; the host reads it without any
  // device synchronization.  `reported`: the value last turned into an error.
  volatile unsigned* gave_up_host = nullptr;
  unsigned* gave_up_dev = nullptr;
  unsigned reported = 0;
};

// Test hook (TFMA_BN_FORCE_GIVE_UP=1, read once): every eager fused launch
// waits for an epoch no launch publishes, with a short spin limit, so each
// wait gives up and the kernels still exit normally.
bool force_give_up() {
  static const bool on = [] {
    const char* e = getenv("TFMA_BN_FORCE_GIVE_UP");
    return e && e[0] == '1';
  }();
  return on;
}


// Plan of the calling thread's last FusedBatchNorm launch
// (TFMA_FusedBatchNormLastPlan).
thread_local TFMA_FusedBatchNormPlan t_last_plan{};

void note_split_plan(const Plan& p) {
  t_last_plan = TFMA_FusedBatchNormPlan{};
  t_last_plan.row_groups = p.groups;
  t_last_plan.channel_tiles = p.ct;
}

BarrierState* barrier_state() {
  static BarrierState states[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  return &states[dev];
}

template <class Tr, bool kGrad>
hipError_t launch_fused(const FusedPlan& fp, const BnGeometry& g, const void* x,
                        const void* dy, void* out, const FinArgs& fin, hipStream_t stream) {
  BarrierState* bs = barrier_state();
  if (!bs) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(bs->mu);
  if (!bs->counter) {
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, 2 * kStateBytes);
    if (e != hipSuccess) return e;
    e = hipMemset(p, 0, 2 * kStateBytes);
    if (e != hipSuccess) {
      (void)hipFree(p);
      return e;
    }
    bs->counter = static_cast<unsigned long long*>(p);
  }
  if (!bs->gave_up_host) {
    void* h = nullptr;
    hipError_t e = hipHostMalloc(&h, 64, hipHostMallocCoherent | hipHostMallocMapped);
    if (e != hipSuccess) return e;
    *static_cast<volatile unsigned*>(h) = 0;
    void* d = nullptr;
    e = hipHostGetDevicePointer(&d, h, 0);
    if (e != hipSuccess) {
      (void)hipHostFree(h);
      return e;
    }
    bs->gave_up_host = static_cast<volatile unsigned*>(h);
    bs->gave_up_dev = static_cast<unsigned*>(d);
  }
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  {
    const hipError_t e = hipStreamIsCapturing(stream, &cap);
    if (e != hipSuccess) return e;
  }
  const bool recorded = cap != hipStreamCaptureStatusNone;
  // Epoch-tagged values: partial slots for every (group, channel) and
  // coefficient words for every channel of the largest fused plan (at most
  // 2 workgroups per CU, each channel tile at most 256 channels wide and
  // served by at least one workgroup, so G*C and C are both at most
  // 512 * CUs), tagged with the launch's epoch, so a value from an earlier
  // launch never matches.  Eager epochs stay below 2^31; at the wrap both
  // regions are zeroed again.
  if (!bs->eslots) {
    const size_t slot_bytes = static_cast<size_t>(2 * DeviceCUs()) * 256 * 16;
    // kCoefCopies copies of 4 words per channel, then 1 key word per channel.
    const size_t coef_bytes =
        (kCoefCopies * coef_copy_words() + static_cast<size_t>(max_fused_channels())) * 8;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, slot_bytes + coef_bytes);
    if (e != hipSuccess) return e;
    e = hipMemset(p, 0, slot_bytes + coef_bytes);
    if (e != hipSuccess) {
      (void)hipFree(p);
      return e;
    }
    bs->eslots = static_cast<unsigned long long*>(p);
    bs->eslot_bytes = slot_bytes;
    bs->ecoef = reinterpret_cast<unsigned long long*>(static_cast<char*>(p) + slot_bytes);
    bs->ecoef_bytes = coef_bytes;
    // First eager epoch - 1 (TFMA_BN_EPOCH_START, default 0): a test starts
    // just below the wrap to run launches across it.
    const char* es = getenv("TFMA_BN_EPOCH_START");
    const unsigned long long start = es ? strtoull(es, nullptr, 10) : 0ull;
    bs->epoch = start < (1ull << 31) ? static_cast<unsigned>(start) : 0u;
  }
  if (fp.groups > kMaxEpochGroups || fp.ct_conc < 1 ||
      static_cast<size_t>(fp.groups) * g.c * 16 > bs->eslot_bytes ||
      g.c > max_fused_channels())
    return hipErrorInvalidValue;  // excluded by make_fused_plan
  unsigned long long* region =
      recorded ? reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(bs->counter) +
                                                       kStateBytes)
               : bs->counter;
  if (!recorded) {
    hipError_t e = bs->chain.before(stream);
    if (e != hipSuccess) return e;
  }
  // The epoch, after the wait above: zeroing the regions at the wrap must
  // follow the previous fused launch, which may be on another stream.
  unsigned epoch = 0;
  if (!recorded) {
    if (bs->epoch + 1 >= (1u << 31)) {
      hipError_t e = hipMemsetAsync(bs->eslots, 0, bs->eslot_bytes + bs->ecoef_bytes, stream);
      if (e != hipSuccess) return e;
      bs->epoch = 0;
    }
    epoch = ++bs->epoch;
  }
  FusedArgs fa;
  fa.x = x;
  fa.dy = dy;
  fa.out = out;
  fa.rows = g.rows;
  fa.c = static_cast<int>(g.c);
  fa.cv = fp.cv;
  fa.tx_shift = fp.tx_shift;
  fa.ct = fp.ct;
  fa.ct_conc = fp.ct_conc;
  fa.slices = fp.slices;
  fa.groups = fp.groups;
  fa.rows_per_g = fp.rows_per_g;
  fa.barrier = region;
  fa.base = recorded ? 0 : bs->base;
  fa.sub = reinterpret_cast<unsigned*>(reinterpret_cast<char*>(region) + kSubOffset);
  for (int r = 0; r < 8; ++r) {
    const unsigned members = static_cast<unsigned>((fp.blocks + 7 - r) / 8);
    const unsigned sb = recorded ? 0u : bs->sub_base[r];
    fa.sub_last[r] = sb + members - 1;
  }
  fa.gave_up = bs->gave_up_dev;
  const bool forced = force_give_up() && !recorded;
  fa.spin_limit = forced ? 2000u : kSpinLimit;
  fa.wait_xor = forced ? 0x40000000u : 0u;
  fa.queues = reinterpret_cast<unsigned*>(reinterpret_cast<char*>(region) + kQueueOffset);
  fa.reset_at_exit = recorded ? 1 : 0;
  fa.eslots = bs->eslots;
  fa.ecoef = bs->ecoef;
  fa.coef_copy = static_cast<int64_t>(coef_copy_words());
  fa.coef_copies = static_cast<int>(std::min<int64_t>(
      kCoefCopies, std::max<int64_t>(1, fp.groups / kPollersPerCopy)));
  // The key words after the last copy of the coefficients.
  fa.ekey = bs->ecoef + kCoefCopies * coef_copy_words();
  fa.epoch = epoch;
  fa.epoch_dev = recorded ? reinterpret_cast<unsigned*>(reinterpret_cast<char*>(region) +
                                                        kEpochOffset)
                          : nullptr;
  const int ry = kFusedThreads >> fp.tx_shift;
  const int64_t nk_max = (fp.rows_per_g + ry - 1) / ry;  // rows of a thread
  const bool sliced = kGrad && fp.slices > 1;
  const bool small = !kGrad && nk_max <= kSmallFwdRows;
  int kr = small ? Resident<Tr>::kRegFwdSmall : fused_kr<Tr, kGrad>();
  if constexpr (kGrad) {
    if (sliced) kr = Resident<Tr>::kRegGradSliced;
  }
  {
    FusedPlan fd = fp;
    constexpr int kPre = kGrad ? Resident<Tr>::kPaGrad + Resident<Tr>::kPbGrad
                               : Resident<Tr>::kPaFwd + Resident<Tr>::kPbFwd;
    set_dynamic_share(&fd, kr + fused_kl<Tr, kGrad>(), kPre, kGrad ? 4 : 8);
    fa.dyn_chunk = fd.dyn_chunk;
    const size_t slots = kQueueBytes / sizeof(unsigned);
    const size_t per_shard = static_cast<size_t>(fp.ct) * (kFusedThreads / 64);
    size_t shards = slots / per_shard;
    if (shards > 16) shards = 16;
    fa.shards = shards > 0 ? static_cast<int>(shards) : 1;
    fa.dyn_rows = shards > 0 ? fd.dyn_rows : 0;
  }
  fa.fin = fin;
  fa.fin.groups = fp.groups;
  t_last_plan = TFMA_FusedBatchNormPlan{};
  t_last_plan.fused = 1;
  t_last_plan.workgroups = fp.blocks;
  t_last_plan.row_groups = fp.groups;
  t_last_plan.channel_tiles = fp.ct;
  t_last_plan.dynamic_rows = fa.dyn_rows;
  t_last_plan.dynamic_chunk = fa.dyn_chunk;
  t_last_plan.register_rows = kr;
  t_last_plan.lds_rows = fused_kl<Tr, kGrad>();
  t_last_plan.slices = fp.slices;
  const char* name = kGrad ? "tfma_bn_grad_fused" : "tfma_bn_fwd_fused";
  SetLastKernel(name);
  const void* kern = fused_kernel<Tr, kGrad>();
  if constexpr (kGrad) {
    if (sliced) {
      kern = sliced_kernel<Tr>();
      // No dynamic tail: the kernel that hides the slices' hand-offs.
      if (fp.ct_conc == 1 && fa.dyn_rows == 0 && sliced_overlap_enabled()) {
        kern = sliced_overlap_kernel<Tr>();
        t_last_plan.register_rows = Resident<Tr>::kRegGradOverlap;
      }
    }
  }
  if constexpr (!kGrad) {
    if (small) kern = fused_kernel<Tr, kGrad, Resident<Tr>::kRegFwdSmall>();
  }
  const size_t smem = fused_smem<Tr, kGrad>();
  void* kargs[] = {&fa};
  if (recorded) {  // no events, no tracing, no chain bookkeeping inside a graph
    hipError_t le = hipLaunchKernel(kern, dim3(fp.blocks), dim3(kFusedThreads), kargs, smem,
                                    stream);
    return le != hipSuccess ? le : hipGetLastError();
  }
  const TraceEvents tev = TraceTake(name);
  hipEvent_t end = bs->chain.end_event(tev.end);
  {
    hipError_t le = hipExtLaunchKernel(kern, dim3(fp.blocks), dim3(kFusedThreads), kargs, smem,
                                       stream, tev.start, end, 0);
    if (le != hipSuccess) return le;
  }
  TraceCommit(tev);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // Per exit count (when chunks were handed out): each class counter gets
  // one arrival per member, the global counter one per non-empty class.
  const unsigned rounds = fa.dyn_rows > 0 ? 1u : 0u;  // the exit arrival
  const unsigned long long classes = fp.blocks < 8 ? fp.blocks : 8;
  for (int r = 0; r < 8; ++r)
    bs->sub_base[r] += rounds * static_cast<unsigned>((fp.blocks + 7 - r) / 8);
  bs->base += rounds * classes;
  bs->chain.after(stream, end);
  return hipSuccess;
}

}  // namespace

hipError_t BnStamps(void* host, size_t bytes) {
#ifdef TFMA_BN_STAMPS
  if (bytes > sizeof(bn_stamps)) bytes = sizeof(bn_stamps);
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return e;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(bn_stamps), bytes, 0, hipMemcpyDeviceToHost);
#else
  (void)host;
  (void)bytes;
  return hipErrorNotSupported;
#endif
}

hipError_t BnBarrierTimedOut(bool reset, bool* timed_out) {
  *timed_out = false;
  BarrierState* bs = barrier_state();
  if (!bs) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(bs->mu);
  if (!bs->gave_up_host) return hipSuccess;  // no fused launch on this device yet
  const hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return e;
  *timed_out = *bs->gave_up_host != 0;
  if (reset) {
    *bs->gave_up_host = 0;
    bs->reported = 0;
  }
  return hipSuccess;
}

TFMA_FusedBatchNormPlan BnLastPlan() { return t_last_plan; }

bool BnPendingGiveUp(unsigned* epoch) {
  BarrierState* bs = barrier_state();
  if (!bs) return false;
  std::lock_guard<std::mutex> lk(bs->mu);
  if (!bs->gave_up_host) return false;
  const unsigned v = *bs->gave_up_host;
  if (v == 0 || v == bs->reported) return false;
  bs->reported = v;
  *epoch = v;
  return true;
}

namespace {

// Partial-sum region: large enough for the split plan (either alignment)
// and for the fused plan's at most fused_group_bound() row groups.
size_t partial_region_bytes(DType t, const BnGeometry& g) {
  const Plan pv = make_plan(t, g, true);
  const Plan ps = make_plan(t, g, false);
  size_t r = partial_bytes(pv, g);
  if (partial_bytes(ps, g) > r) r = partial_bytes(ps, g);
  const size_t f = align256(static_cast<size_t>(fused_group_bound()) * g.c * sizeof(float2));
  return r > f ? r : f;
}

// The channel-per-workgroup NCHW kernel: training, 16-byte plane vectors, at
// least one channel per CU (fewer channels leave CUs idle: the split path's
// reduce spreads every channel over many workgroups), and offsets that fit
// the kernel's 32-bit buffer offsets (rows up to 16 images past the tensor's
// end).  The "bn_nchw_owned" override 0 keeps the split path.
bool nchw_owned_ok(const BnGeometry& g, int vec, int elem) {
  if (g.nhwc || vec <= 1 || g.c < DeviceCUs()) return false;
  if (TuneValue(kTuneBnNchwOwned) == 0) return false;
  const int64_t plane = g.h * g.w;
  return plane % vec == 0 && (g.n + 16) * g.c * plane * elem < (int64_t{1} << 31);
}

template <class Tr, bool kGrad>
hipError_t launch_nchw_owned(const BnGeometry& g, const void* x, const void* dy, void* out,
                             const FinArgs& fin, hipStream_t stream) {
  constexpr int KR = kGrad ? OwnedRows<Tr>::kGrad : OwnedRows<Tr>::kFwd;
  constexpr int KL = fused_kl<Tr, kGrad>();
  const auto kern = &bn_nchw_owned_kernel<Tr, kGrad, KR, KL>;
  const size_t smem = static_cast<size_t>(KL) * (kGrad ? 2 : 1) * kFusedThreads * 16;
  static std::atomic<bool> attr_set[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  if (!attr_set[dev].load(std::memory_order_acquire)) {
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
    if (e != hipSuccess) return e;
    attr_set[dev].store(true, std::memory_order_release);
  }
  NchwArgs na;
  na.x = x;
  na.dy = dy;
  na.out = out;
  na.n = g.n;
  na.c = static_cast<int>(g.c);
  na.plane = g.h * g.w;
  na.pv = na.plane / Tr::kVec;
  na.fin = fin;
  t_last_plan = TFMA_FusedBatchNormPlan{};
  t_last_plan.fused = 2;
  t_last_plan.workgroups = static_cast<int32_t>(g.c);
  t_last_plan.row_groups = 1;
  t_last_plan.channel_tiles = static_cast<int32_t>(g.c);
  t_last_plan.register_rows = KR;
  t_last_plan.lds_rows = KL;
  t_last_plan.slices = 1;
  TFMA_LAUNCH(kGrad ? "tfma_bn_grad_nchw_owned" : "tfma_bn_fwd_nchw_owned", kern,
              dim3(static_cast<unsigned>(g.c)), dim3(kFusedThreads), smem, stream, na);
  return hipGetLastError();
}

bool ptr_aligned(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

template <class Tr>
hipError_t forward_t(const BnGeometry& g, const BnFwdArgs& a, void* ws,
                     size_t ws_bytes, hipStream_t stream) {
  const bool aligned = ptr_aligned(a.x) && ptr_aligned(a.y);
  const DType dt = Tr::kVec == 4 ? DType::kF32 : DType::kF16;
  const Plan p = make_plan(dt, g, aligned);
  const size_t pb = partial_region_bytes(dt, g);
  if (ws_bytes < pb + coef_bytes(g)) return hipErrorInvalidValue;
  float2* partial = static_cast<float2*>(ws);
  float4* coef = reinterpret_cast<float4*>(static_cast<char*>(ws) + pb);
  FinArgs fa{};
  fa.groups = p.groups;
  fa.c = static_cast<int>(g.c);
  fa.n = g.rows;
  fa.x = a.x;
  fa.k_stride = g.nhwc ? 1 : g.h * g.w;
  fa.scale = a.scale;
  fa.offset = a.offset;
  fa.mean_in = a.mean_in;
  fa.var_in = a.var_in;
  fa.eps = a.epsilon;
  fa.f = a.exp_avg_factor;
  fa.batch_mean = a.batch_mean;
  fa.batch_var = a.batch_var;
  fa.saved_mean = a.saved_mean;
  fa.saved_var = a.saved_var;
  fa.reserve3 = a.reserve3;
  fa.is_training = a.is_training;
  hipError_t e;
  FusedPlan fp;
  if (a.is_training && nchw_owned_ok(g, p.vec, sizeof(typename Tr::S)))
    return launch_nchw_owned<Tr, false>(g, a.x, nullptr, a.y, fa, stream);
  if (a.is_training && p.vec > 1 && fused_enabled() &&
      choose_fused_plan<Tr, false>(g, p.vec, &fp)) {
    return launch_fused<Tr, false>(fp, g, a.x, nullptr, a.y, fa,
                                                  stream);
  }
  note_split_plan(p);
  if (!a.is_training)
    return p.vec == 1
               ? launch_apply<Tr, 1, false, true>(p, g, a.x, nullptr, a.y, nullptr, stream, fa)
               : launch_apply<Tr, Tr::kVec, false, true>(p, g, a.x, nullptr, a.y, nullptr, stream,
                                                        fa);
  e = p.vec == 1 ? launch_reduce<Tr, 1, false>(p, g, a.x, nullptr, nullptr, partial, stream)
                 : launch_reduce<Tr, Tr::kVec, false>(p, g, a.x, nullptr, nullptr, partial, stream);
  if (e != hipSuccess) return e;
  e = launch_finalize<Tr, false>(p, fa, partial, coef, stream);
  if (e != hipSuccess) return e;
  return p.vec == 1 ? launch_apply<Tr, 1, false>(p, g, a.x, nullptr, a.y, coef, stream)
                    : launch_apply<Tr, Tr::kVec, false>(p, g, a.x, nullptr, a.y, coef, stream);
}

template <class Tr>
hipError_t grad_t(const BnGeometry& g, const BnGradArgs& a, void* ws,
                  size_t ws_bytes, hipStream_t stream) {
  const bool aligned = ptr_aligned(a.x) && ptr_aligned(a.dy) && ptr_aligned(a.dx);
  const DType dt = Tr::kVec == 4 ? DType::kF32 : DType::kF16;
  const Plan p = make_plan(dt, g, aligned);
  const size_t pb = partial_region_bytes(dt, g);
  if (ws_bytes < pb + coef_bytes(g)) return hipErrorInvalidValue;
  float2* partial = static_cast<float2*>(ws);
  float4* coef = reinterpret_cast<float4*>(static_cast<char*>(ws) + pb);
  FinArgs fa{};
  fa.groups = p.groups;
  fa.c = static_cast<int>(g.c);
  fa.n = g.rows;
  fa.scale = a.scale;
  fa.mean_in = a.saved_mean;
  fa.var_in = a.saved_var;
  fa.eps = a.epsilon;
  fa.scale_bp = a.scale_backprop;
  fa.offset_bp = a.offset_backprop;
  fa.reserve4 = a.reserve4;
  fa.reserve4_n = a.reserve4 ? a.reserve4_n : 0;
  fa.reserve5 = a.reserve5;
  fa.reserve5_n = a.reserve5 ? a.reserve5_n : 0;
  fa.is_training = a.is_training;
  FusedPlan fp;
  if (nchw_owned_ok(g, p.vec, sizeof(typename Tr::S)))
    return launch_nchw_owned<Tr, true>(g, a.x, a.dy, a.dx, fa, stream);
  if (p.vec > 1 && fused_enabled() &&
      choose_fused_plan<Tr, true>(g, p.vec, &fp)) {
    return launch_fused<Tr, true>(fp, g, a.x, a.dy, a.dx, fa,
                                                  stream);
  }
  note_split_plan(p);
  hipError_t e =
      p.vec == 1 ? launch_reduce<Tr, 1, true>(p, g, a.x, a.dy, a.saved_mean, partial, stream)
                 : launch_reduce<Tr, Tr::kVec, true>(p, g, a.x, a.dy, a.saved_mean, partial, stream);
  if (e != hipSuccess) return e;
  e = launch_finalize<Tr, true>(p, fa, partial, coef, stream);
  if (e != hipSuccess) return e;
  return p.vec == 1 ? launch_apply<Tr, 1, true>(p, g, a.x, a.dy, a.dx, coef, stream)
                    : launch_apply<Tr, Tr::kVec, true>(p, g, a.x, a.dy, a.dx, coef, stream);
}

__global__ void fill_f32_kernel(float* __restrict__ p, int64_t n, float v) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    p[i] = v;
}

}  // namespace

hipError_t LaunchFillF32(float* p, int64_t n, float value, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 1024) blocks = 1024;
  TFMA_LAUNCH("tfma_fill_f32", fill_f32_kernel, dim3(blocks), dim3(256), 0, stream, p, n, value);
  return hipGetLastError();
}

size_t BnWorkspaceBytes(DType t, const BnGeometry& g) {
  return partial_region_bytes(t, g) + coef_bytes(g);
}

hipError_t LaunchBnForward(DType t, const BnGeometry& g, const BnFwdArgs& a,
                           void* ws, size_t ws_bytes, hipStream_t stream) {
  switch (t) {
    case DType::kF32: return forward_t<TF32>(g, a, ws, ws_bytes, stream);
    case DType::kF16: return forward_t<TF16>(g, a, ws, ws_bytes, stream);
    case DType::kBF16: return forward_t<TBF16>(g, a, ws, ws_bytes, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t LaunchBnGrad(DType t, const BnGeometry& g, const BnGradArgs& a,
                        void* ws, size_t ws_bytes, hipStream_t stream) {
  switch (t) {
    case DType::kF32: return grad_t<TF32>(g, a, ws, ws_bytes, stream);
    case DType::kF16: return grad_t<TF16>(g, a, ws, ws_bytes, stream);
    case DType::kBF16: return grad_t<TBF16>(g, a, ws, ws_bytes, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace tfma
