// Device-side helpers shared by the gfx950 kernels: storage/compute type
// traits with TensorFlow-CPU rounding points, 16-byte vector access, and a
// 32-bit fast divider.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace tfma {

// ---------------------------------------------------------------------------
// Type traits.  S = storage type in HBM, C = compute type in registers.
// `rnd` rounds a compute value to the storage precision and back; TF's CPU
// kernels (Eigen) evaluate half/bfloat16 arithmetic as float and round to the
// storage type after every operation, which `rnd` reproduces.
// ---------------------------------------------------------------------------

__host__ __device__ inline uint32_t f32_bits(float f) {
  return __builtin_bit_cast(uint32_t, f);
}
__host__ __device__ inline float bits_f32(uint32_t u) {
  return __builtin_bit_cast(float, u);
}

// float -> bfloat16, round to nearest even; NaN -> quiet NaN with the sign
// kept (0x7fc0 / 0xffc0), the convention of Eigen's float_to_bfloat16_rtne.
__host__ __device__ inline uint16_t f32_to_bf16(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u & 0x80000000u) ? 0xffc0u : 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__host__ __device__ inline float bf16_to_f32(uint16_t h) {
  return bits_f32(static_cast<uint32_t>(h) << 16);
}

struct TF32 {
  using S = float;
  using C = float;
  static constexpr int kVec = 4;  // elements per 16-byte access
  __device__ static inline C ld(S s) { return s; }
  __device__ static inline S st(C c) { return c; }
  __device__ static inline C rnd(C c) { return c; }
};

struct TF16 {
  using S = uint16_t;
  using C = float;
  static constexpr int kVec = 8;
  __device__ static inline C ld(S s) {
    return static_cast<float>(__builtin_bit_cast(_Float16, s));
  }
  __device__ static inline S st(C c) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(c));
  }
  __device__ static inline C rnd(C c) { return ld(st(c)); }
};

struct TBF16 {
  using S = uint16_t;
  using C = float;
  static constexpr int kVec = 8;
  __device__ static inline C ld(S s) { return bf16_to_f32(s); }
  // gfx950 converts with v_cvt_pk_bf16_f32 (round to nearest even, as
  // f32_to_bf16; NaN payloads may differ from the host helper's).
  __device__ static inline S st(C c) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(c)); }
  __device__ static inline C rnd(C c) { return ld(st(c)); }
};

struct TF64 {
  using S = double;
  using C = double;
  static constexpr int kVec = 2;
  __device__ static inline C ld(S s) { return s; }
  __device__ static inline S st(C c) { return c; }
  __device__ static inline C rnd(C c) { return c; }
};

// Integer storage types.  They compute in the unsigned type of the same width
// (uint8 in 32 bits) so that add and multiply wrap modulo 2^bits, the
// two's-complement result TF's CPU kernels produce, with no signed overflow
// in the device code; st() keeps the low bits.
template <typename SS, typename CC>
struct TInt {
  using S = SS;
  using C = CC;
  static constexpr bool kInt = true;
  static constexpr int kVec = 16 / static_cast<int>(sizeof(SS));
  __device__ static inline C ld(S s) {
    if constexpr (sizeof(S) == sizeof(C))
      return __builtin_bit_cast(C, s);
    else
      return static_cast<C>(s);
  }
  __device__ static inline S st(C c) {
    if constexpr (sizeof(S) == sizeof(C))
      return __builtin_bit_cast(S, c);
    else
      return static_cast<S>(c);
  }
  __device__ static inline C rnd(C c) { return c; }
};
using TI32 = TInt<int32_t, uint32_t>;
using TI64 = TInt<int64_t, uint64_t>;
using TU8 = TInt<uint8_t, uint32_t>;

// Whether Tr is one of the integer traits (the others have no kInt member).
template <class Tr, class = void>
struct IsIntTraits : std::false_type {};
template <class Tr>
struct IsIntTraits<Tr, std::void_t<decltype(Tr::kInt)>> : std::true_type {};

// ---------------------------------------------------------------------------
// Vector access: N consecutive storage elements at p (p aligned to
// N*sizeof(S) bytes when N*sizeof(S) is 16, 8 or 4).
// ---------------------------------------------------------------------------
template <typename S, int N>
struct Raw {
  static constexpr int kBytes = N * static_cast<int>(sizeof(S));
  using Word = typename std::conditional<
      kBytes == 16, uint4,
      typename std::conditional<
          kBytes == 8, uint2,
          typename std::conditional<
              kBytes == 4, uint32_t,
              typename std::conditional<kBytes == 2, uint16_t, S>::type>::type>::type>::type;
};

template <typename S, int N>
__device__ inline void vload(const S* __restrict__ p, S (&out)[N]) {
  using W = typename Raw<S, N>::Word;
  if constexpr (sizeof(W) == sizeof(S) * N) {
    W w = *reinterpret_cast<const W*>(p);
    __builtin_memcpy(out, &w, sizeof(W));
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) out[j] = p[j];
  }
}

template <typename S, int N>
__device__ inline void vstore(S* __restrict__ p, const S (&in)[N]) {
  using W = typename Raw<S, N>::Word;
  if constexpr (sizeof(W) == sizeof(S) * N) {
    W w;
    __builtin_memcpy(&w, in, sizeof(W));
    *reinterpret_cast<W*>(p) = w;
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) p[j] = in[j];
  }
}

// Non-temporal variants (the line is not kept in the caches for reuse).
// Measured on MI355X with the Infinity Cache flushed between reps: loads of
// BiasAddGrad's single-use input 5 % faster, Adam's stores 0.5-2 % faster;
// Adam's loads and the elementwise kernels' loads and stores only pay off
// above a size (their launchers choose with vload_sel / vstore_sel).
typedef unsigned int nt_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int nt_u32x2 __attribute__((ext_vector_type(2)));
template <typename W> struct NtWord { using T = W; };
template <> struct NtWord<uint4> { using T = nt_u32x4; };
template <> struct NtWord<uint2> { using T = nt_u32x2; };

template <typename S, int N>
__device__ inline void vload_nt(const S* __restrict__ p, S (&out)[N]) {
  using W = typename Raw<S, N>::Word;
  if constexpr (sizeof(W) == sizeof(S) * N) {
    using T = typename NtWord<W>::T;
    const T w = __builtin_nontemporal_load(reinterpret_cast<const T*>(p));
    __builtin_memcpy(out, &w, sizeof(W));
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) out[j] = __builtin_nontemporal_load(p + j);
  }
}

template <typename S, int N>
__device__ inline void vstore_nt(S* __restrict__ p, const S (&in)[N]) {
  using W = typename Raw<S, N>::Word;
  if constexpr (sizeof(W) == sizeof(S) * N) {
    using T = typename NtWord<W>::T;
    T w;
    __builtin_memcpy(&w, in, sizeof(W));
    __builtin_nontemporal_store(w, reinterpret_cast<T*>(p));
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) __builtin_nontemporal_store(in[j], p + j);
  }
}

template <bool kNt, typename S, int N>
__device__ inline void vload_sel(const S* __restrict__ p, S (&out)[N]) {
  if constexpr (kNt)
    vload_nt<S, N>(p, out);
  else
    vload<S, N>(p, out);
}

template <bool kNt, typename S, int N>
__device__ inline void vstore_sel(S* __restrict__ p, const S (&in)[N]) {
  if constexpr (kNt)
    vstore_nt<S, N>(p, in);
  else
    vstore<S, N>(p, in);
}

// ---------------------------------------------------------------------------
// Unsigned 32-bit division by a runtime-invariant divisor d >= 1 with a
// multiply-high (round-up method, Granlund & Montgomery, PLDI 1994):
// q = (mulhi(n, m) + n) >> s with s = ceil(log2 d), m = floor(2^32 (2^s - d)
// / d) + 1.  Exact for all n < 2^32.
// ---------------------------------------------------------------------------
struct FastDiv {
  uint32_t d;
  uint32_t m;
  uint32_t s;
  __host__ __device__ FastDiv() : d(1), m(0), s(0) {}
  __host__ explicit FastDiv(uint32_t div) : d(div) {
    uint32_t sh = 0;
    while (sh < 32 && (uint64_t(1) << sh) < div) ++sh;
    s = sh;
    uint64_t num = (uint64_t(1) << 32) * ((uint64_t(1) << sh) - div);
    m = static_cast<uint32_t>(num / div + 1);
  }
  __device__ inline uint32_t div(uint32_t n) const {
    uint32_t hi = __umulhi(n, m);
    return static_cast<uint32_t>((static_cast<uint64_t>(hi) + n) >> s);
  }
  __device__ inline void divmod(uint32_t n, uint32_t& q, uint32_t& r) const {
    q = div(n);
    r = n - q * d;
  }
};

}  // namespace tfma
