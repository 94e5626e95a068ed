/*
 * tfcpu_oracle.c - CPU restatement of TensorFlow's CPU kernels for the hot
 * path (FusedBatchNormV3 / FusedBatchNormGradV3, ResourceApplyAdam, the
 * elementwise ops behind BiasAdd+Relu, AddV2+Relu, Mul+Add, and their
 * backward counterparts ReluGrad and BiasAddGrad).
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library and the CPU baseline ("port") that bench.py times; nothing in the
 * product links, loads or calls it.
 *
 * The reference (MooreThreads/tensorflow_musa_extension) defers this
 * arithmetic to closed muDNN kernels and judges it against TF's CPU kernels
 * (test/musa_test_utils.py:82-111), so the oracle restates TF-CPU semantics,
 * with the conventions the reference documents:
 *   - BN statistics, Bessel factor and reserve-space meaning:
 *     musa_ext/kernels/nn/musa_fused_batchnorm_op.cc:13-15, 60-62, 141-170,
 *     265-277 (grad takes population variance + epsilon).
 *   - Adam inputs / alpha / dtypes: musa_ext/kernels/training/
 *     musa_applyadam_op.cc:158-186, 224-246, 645-682 (alpha is computed the
 *     TF-CPU way, in T, not in double as the reference does).
 *   - BiasAdd channel dimension: musa_ext/kernels/nn/musa_biasadd_op.cc:31-52;
 *     BiasAddGrad: musa_ext/kernels/nn/musa_biasadd_grad_op.cc:31-69;
 *     ReluGrad: musa_ext/kernels/nn/musa_relu_grad_op.cc:19-46.
 *   - Broadcasting: musa_ext/kernels/math/musa_add_op.cc:194-220, 397-403;
 *     musa_ext/kernels/fusion/musa_shifted_affine_map_op.cc:108-165.
 * Summation order is the one deliberate difference from TF: BN sums are
 * accumulated in double (TF sums in float in Eigen's tree order), so the
 * oracle is closer to the exact value than TF; the rest rounds exactly where
 * TF does.  Build with -ffp-contract=off (see Makefile).
 *
 * dtype codes are TF_DataType values: 1 float, 2 double, 3 int32, 4 uint8,
 * 9 int64, 14 bfloat16, 19 half.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { DT_FLOAT = 1, DT_DOUBLE = 2, DT_INT32 = 3, DT_UINT8 = 4, DT_INT64 = 9,
       DT_BFLOAT16 = 14, DT_HALF = 19 };

/* ------------------------------------------------------------------------ */
/* half / bfloat16 <-> float, round to nearest even                          */
/* ------------------------------------------------------------------------ */
static inline uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t oracle_f32_to_f16(float f) {
  uint32_t x = fbits(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  int32_t exp = (int32_t)((x >> 23) & 0xff);
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u));
  int32_t e = exp - 112; /* rebias 127 -> 15 */
  if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    uint32_t sh = (uint32_t)(14 - e);
    uint32_t q = man >> sh, r = man & ((1u << sh) - 1u), hw = 1u << (sh - 1u);
    if (r > hw || (r == hw && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t q = ((uint32_t)e << 10) | (man >> 13), r = man & 0x1fffu;
  if (r > 0x1000u || (r == 0x1000u && (q & 1u))) q++;
  return (uint16_t)(sign | q);
}

float oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
  if (exp == 0) {
    float v = (float)man * 5.9604644775390625e-8f; /* 2^-24 */
    return sign ? -v : v;
  }
  if (exp == 0x1f) return bitsf(sign | 0x7f800000u | (man << 13));
  return bitsf(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u = fbits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u & 0x80000000u) ? 0xffc0u : 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t h) { return bitsf((uint32_t)h << 16); }

static inline float ld(int dt, const void* p, int64_t i) {
  switch (dt) {
    case DT_FLOAT: return ((const float*)p)[i];
    case DT_HALF: return oracle_f16_to_f32(((const uint16_t*)p)[i]);
    case DT_BFLOAT16: return oracle_bf16_to_f32(((const uint16_t*)p)[i]);
  }
  return 0.f;
}
static inline void st(int dt, void* p, int64_t i, float v) {
  switch (dt) {
    case DT_FLOAT: ((float*)p)[i] = v; break;
    case DT_HALF: ((uint16_t*)p)[i] = oracle_f32_to_f16(v); break;
    case DT_BFLOAT16: ((uint16_t*)p)[i] = oracle_f32_to_bf16(v); break;
  }
}
/* round a float to T and back */
static inline float rnd(int dt, float v) {
  switch (dt) {
    case DT_HALF: return oracle_f16_to_f32(oracle_f32_to_f16(v));
    case DT_BFLOAT16: return oracle_bf16_to_f32(oracle_f32_to_bf16(v));
  }
  return v;
}

static int g_threads = 1;
void oracle_set_threads(int n) { g_threads = n > 0 ? n : 1; }
int oracle_get_threads(void) { return g_threads; }

/* element (image n, channel c, spatial s) of an NHWC or NCHW tensor */
static inline int64_t bn_index(int nhwc, int64_t n, int64_t c, int64_t s, int64_t C, int64_t S) {
  return nhwc ? (n * S + s) * C + c : (n * C + c) * S + s;
}

/* Per-channel double sums of f(x[, dy]) over all N*S positions, parallel
 * over images with per-thread accumulators combined in thread order. */
typedef struct {
  int dt, nhwc;
  const void* x;
  const void* dy;
  int64_t N, C, S;
  const float* center; /* per-channel value subtracted from x (float op) */
  const float* k;      /* grad: per-channel rsqrt, for sum(dy * (xc*k)) */
} bn_sum_args;

/* mode 0: s1 = sum x
 * mode 1: s1 = sum (xc)^2 where xc = x - center (float)
 * mode 2: s1 = sum dy, s2 = sum (dy*xc) (float product), s3 = sum dy*(xc*k) */
static void bn_sums(const bn_sum_args* a, int mode, double* s1, double* s2, double* s3) {
  const int64_t C = a->C;
  int nt = g_threads;
  if (nt > a->N) nt = (int)(a->N > 0 ? a->N : 1);
  double* acc = (double*)calloc((size_t)nt * 3 * (size_t)C, sizeof(double));
#ifdef _OPENMP
#pragma omp parallel num_threads(nt)
#endif
  {
#ifdef _OPENMP
    int t = omp_get_thread_num();
#else
    int t = 0;
#endif
    double* p1 = acc + (size_t)t * 3 * C;
    double* p2 = p1 + C;
    double* p3 = p2 + C;
    int64_t nb = a->N * t / nt, ne = a->N * (t + 1) / nt;
    for (int64_t n = nb; n < ne; ++n) {
      for (int64_t s = 0; s < a->S; ++s) {
        for (int64_t c = 0; c < C; ++c) {
          int64_t i = bn_index(a->nhwc, n, c, s, C, a->S);
          float xv = ld(a->dt, a->x, i);
          if (mode == 0) {
            p1[c] += xv;
          } else if (mode == 1) {
            float xc = xv - a->center[c];
            p1[c] += (double)xc * (double)xc;
          } else {
            float d = ld(a->dt, a->dy, i);
            float xc = xv - a->center[c];
            p1[c] += d;
            p2[c] += (double)(d * xc);
            p3[c] += (double)(d * (xc * a->k[c]));
          }
        }
      }
    }
  }
  for (int64_t c = 0; c < C; ++c) {
    double a1 = 0, a2 = 0, a3 = 0;
    for (int t = 0; t < nt; ++t) {
      a1 += acc[(size_t)t * 3 * C + c];
      a2 += acc[(size_t)t * 3 * C + C + c];
      a3 += acc[(size_t)t * 3 * C + 2 * C + c];
    }
    if (s1) s1[c] = a1;
    if (s2) s2[c] = a2;
    if (s3) s3[c] = a3;
  }
  free(acc);
}

/* FusedBatchNormV3 forward (TF CPU FusedBatchNorm<CPUDevice, T, float>). */
void oracle_bn_fwd(int dt, int nhwc, const void* x, int64_t N, int64_t C, int64_t S,
                   const float* scale, const float* offset, const float* mean_in,
                   const float* var_in, float eps, float f, int is_training, void* y,
                   float* batch_mean, float* batch_var, float* saved_mean, float* saved_var) {
  const int64_t n = N * S;
  float* mean = (float*)malloc(sizeof(float) * (size_t)(C > 0 ? C : 1));
  float* var = (float*)malloc(sizeof(float) * (size_t)(C > 0 ? C : 1));
  float* scaling = (float*)malloc(sizeof(float) * (size_t)(C > 0 ? C : 1));
  if (is_training) {
    if (n == 0) {
      for (int64_t c = 0; c < C; ++c) {
        batch_mean[c] = NAN; batch_var[c] = NAN; saved_mean[c] = 0.f; saved_var[c] = 0.f;
      }
      free(mean); free(var); free(scaling);
      return;
    }
    double* s = (double*)malloc(sizeof(double) * (size_t)C);
    bn_sum_args a = {dt, nhwc, x, NULL, N, C, S, NULL, NULL};
    bn_sums(&a, 0, s, NULL, NULL);
    for (int64_t c = 0; c < C; ++c) mean[c] = (float)(s[c] / (double)n);
    a.center = mean;
    bn_sums(&a, 1, s, NULL, NULL);
    for (int64_t c = 0; c < C; ++c) var[c] = (float)(s[c] / (double)n);
    free(s);
    const float adj = (float)n / (float)(n > 1 ? n - 1 : 1);
    for (int64_t c = 0; c < C; ++c) {
      saved_mean[c] = mean[c];
      saved_var[c] = var[c];
      if (f == 1.0f) {
        batch_mean[c] = mean[c];
        batch_var[c] = var[c] * adj;
      } else {
        const float omf = 1.0f - f;
        batch_mean[c] = mean_in[c] * omf + mean[c] * f;
        batch_var[c] = var_in[c] * omf + (var[c] * adj) * f;
      }
    }
  } else {
    for (int64_t c = 0; c < C; ++c) {
      mean[c] = mean_in[c];
      var[c] = var_in[c];
      batch_mean[c] = mean_in[c];
      batch_var[c] = var_in[c];
      saved_mean[c] = mean_in[c];
      saved_var[c] = var_in[c];
    }
  }
  for (int64_t c = 0; c < C; ++c) scaling[c] = (1.0f / sqrtf(var[c] + eps)) * scale[c];
#ifdef _OPENMP
#pragma omp parallel for num_threads(g_threads) schedule(static)
#endif
  for (int64_t nn = 0; nn < N; ++nn)
    for (int64_t s = 0; s < S; ++s)
      for (int64_t c = 0; c < C; ++c) {
        int64_t i = bn_index(nhwc, nn, c, s, C, S);
        float xc = ld(dt, x, i) - mean[c];
        st(dt, y, i, xc * scaling[c] + offset[c]);
      }
  free(mean); free(var); free(scaling);
}

/* FusedBatchNormGradV3 (TF CPU FusedBatchNormGrad<CPUDevice, T, float>);
 * mean/var are reserve_space_1/2 (population variance). */
void oracle_bn_grad(int dt, int nhwc, const void* dy, const void* x, int64_t N, int64_t C,
                    int64_t S, const float* scale, const float* mean, const float* var,
                    float eps, int is_training, void* dx, float* scale_bp, float* offset_bp) {
  const int64_t n = N * S;
  if (C == 0) return;
  if (n == 0) {
    for (int64_t c = 0; c < C; ++c) { scale_bp[c] = 0.f; offset_bp[c] = 0.f; }
    return;
  }
  float* k = (float*)malloc(sizeof(float) * (size_t)C);
  float* coef1 = (float*)malloc(sizeof(float) * (size_t)C);
  float* coef2 = (float*)malloc(sizeof(float) * (size_t)C);
  float* mdy = (float*)malloc(sizeof(float) * (size_t)C);
  double* s1 = (double*)malloc(sizeof(double) * (size_t)C);
  double* s2 = (double*)malloc(sizeof(double) * (size_t)C);
  double* s3 = (double*)malloc(sizeof(double) * (size_t)C);
  for (int64_t c = 0; c < C; ++c) k[c] = 1.0f / sqrtf(var[c] + eps);
  bn_sum_args a = {dt, nhwc, x, dy, N, C, S, mean, k};
  bn_sums(&a, 2, s1, s2, s3);
  for (int64_t c = 0; c < C; ++c) {
    offset_bp[c] = (float)s1[c];
    scale_bp[c] = (float)s3[c];
    coef1[c] = scale[c] * k[c];
    if (is_training) {
      mdy[c] = (float)(s1[c] / (double)n);
      coef2[c] = (k[c] * k[c]) * (float)(s2[c] / (double)n);
    } else {
      mdy[c] = 0.f;
      coef2[c] = 0.f;
    }
  }
#ifdef _OPENMP
#pragma omp parallel for num_threads(g_threads) schedule(static)
#endif
  for (int64_t nn = 0; nn < N; ++nn)
    for (int64_t s = 0; s < S; ++s)
      for (int64_t c = 0; c < C; ++c) {
        int64_t i = bn_index(nhwc, nn, c, s, C, S);
        float xc = ld(dt, x, i) - mean[c];
        float d = ld(dt, dy, i);
        float r = is_training ? coef1[c] * ((d - mdy[c]) - xc * coef2[c]) : d * coef1[c];
        st(dt, dx, i, r);
      }
  free(k); free(coef1); free(coef2); free(mdy); free(s1); free(s2); free(s3);
}

/* ResourceApplyAdam (TF CPU ApplyAdamNonCuda): in place on var/m/v; the
 * scalars are given as doubles holding T values exactly. */
void oracle_adam(int dt, void* var, void* m, void* v, const void* grad, int64_t n, double b1p_,
                 double b2p_, double lr_, double b1_, double b2_, double eps_, int nesterov) {
  if (dt == DT_DOUBLE) {
    double* X = (double*)var; double* M = (double*)m; double* V = (double*)v;
    const double* G = (const double*)grad;
    const double alpha = lr_ * sqrt(1.0 - b2p_) / (1.0 - b1p_);
    const double omb1 = 1.0 - b1_, omb2 = 1.0 - b2_;
#ifdef _OPENMP
#pragma omp parallel for num_threads(g_threads) schedule(static)
#endif
    for (int64_t i = 0; i < n; ++i) {
      double g = G[i];
      M[i] += (g - M[i]) * omb1;
      V[i] += (g * g - V[i]) * omb2;
      if (nesterov)
        X[i] -= ((g * omb1 + b1_ * M[i]) * alpha) / (sqrt(V[i]) + eps_);
      else
        X[i] -= (M[i] * alpha) / (sqrt(V[i]) + eps_);
    }
    return;
  }
  /* The scalars are T tensors in TF: round them to T first. */
  const float b1p = rnd(dt, (float)b1p_), b2p = rnd(dt, (float)b2p_), lr = rnd(dt, (float)lr_);
  const float b1 = rnd(dt, (float)b1_), b2 = rnd(dt, (float)b2_), eps = rnd(dt, (float)eps_);
  /* alpha = lr * sqrt(1 - beta2_power) / (1 - beta1_power), in T */
  const float alpha = rnd(dt, rnd(dt, lr * rnd(dt, sqrtf(rnd(dt, 1.0f - b2p)))) /
                                  rnd(dt, 1.0f - b1p));
  const float omb1 = rnd(dt, 1.0f - b1), omb2 = rnd(dt, 1.0f - b2);
#ifdef _OPENMP
#pragma omp parallel for num_threads(g_threads) schedule(static)
#endif
  for (int64_t i = 0; i < n; ++i) {
    const float g = ld(dt, grad, i);
    float mm = ld(dt, m, i), vv = ld(dt, v, i), xx = ld(dt, var, i);
    mm = rnd(dt, mm + rnd(dt, rnd(dt, g - mm) * omb1));
    vv = rnd(dt, vv + rnd(dt, rnd(dt, rnd(dt, g * g) - vv) * omb2));
    float num;
    if (nesterov)
      num = rnd(dt, rnd(dt, rnd(dt, g * omb1) + rnd(dt, b1 * mm)) * alpha);
    else
      num = rnd(dt, mm * alpha);
    const float den = rnd(dt, rnd(dt, sqrtf(vv)) + eps);
    xx = rnd(dt, xx - rnd(dt, num / den));
    st(dt, m, i, mm);
    st(dt, v, i, vv);
    st(dt, var, i, xx);
  }
}

/* Elementwise ops with TF broadcasting (integer dtypes: add and mul only).
 * op: 0 add, 1 add+relu, 2 mul,
 * 3 mul+add (in0*in1 rounded, + in2), 4 relu, 5 relu grad (in0 = gradients,
 * in1 = features: gradients * (features > 0), TF's ReluGrad as a multiply,
 * so a NaN or infinite gradient at features <= 0 gives NaN and a negative
 * gradient gives -0).  Each input i has rank
 * in_ndims[i] <= 8 and dims in_dims[8*i ...]; out has rank out_ndims. */
void oracle_eltwise(int dt, int op, int nin, const void* const* ins, const int64_t* in_dims,
                    const int* in_ndims, int out_ndims, const int64_t* out_dims, void* out) {
  int64_t strides[3][8];
  int64_t total = 1;
  for (int d = 0; d < out_ndims; ++d) total *= out_dims[d];
  for (int k = 0; k < nin; ++k) {
    int64_t s = 1;
    for (int d = out_ndims - 1; d >= 0; --d) {
      int it = in_ndims[k] - out_ndims + d;
      int64_t td = it >= 0 ? in_dims[8 * k + it] : 1;
      strides[k][d] = (td == out_dims[d]) ? s : 0;
      s *= td;
    }
  }
#ifdef _OPENMP
#pragma omp parallel for num_threads(g_threads) schedule(static)
#endif
  for (int64_t i = 0; i < total; ++i) {
    int64_t off[3] = {0, 0, 0};
    int64_t rem = i;
    for (int d = out_ndims - 1; d >= 0; --d) {
      int64_t coord = rem % out_dims[d];
      rem /= out_dims[d];
      for (int k = 0; k < nin; ++k) off[k] += coord * strides[k][d];
    }
    if (dt == DT_INT32 || dt == DT_INT64 || dt == DT_UINT8) {
      /* Integer add / mul wrap modulo 2^bits (two's complement), as TF's CPU
       * kernels' int32 / int64 / uint8 arithmetic does: computed in uint64,
       * the low bits kept. */
      uint64_t x, y;
      if (dt == DT_INT32) {
        x = (uint64_t)(int64_t)((const int32_t*)ins[0])[off[0]];
        y = (uint64_t)(int64_t)((const int32_t*)ins[1])[off[1]];
      } else if (dt == DT_INT64) {
        x = (uint64_t)((const int64_t*)ins[0])[off[0]];
        y = (uint64_t)((const int64_t*)ins[1])[off[1]];
      } else {
        x = ((const uint8_t*)ins[0])[off[0]];
        y = ((const uint8_t*)ins[1])[off[1]];
      }
      const uint64_t z = op == 2 ? x * y : x + y;
      if (dt == DT_INT32) ((int32_t*)out)[i] = (int32_t)(uint32_t)z;
      else if (dt == DT_INT64) ((int64_t*)out)[i] = (int64_t)z;
      else ((uint8_t*)out)[i] = (uint8_t)z;
      continue;
    }
    float a = ld(dt, ins[0], off[0]);
    float r;
    switch (op) {
      case 0: r = a + ld(dt, ins[1], off[1]); break;
      case 1: r = rnd(dt, a + ld(dt, ins[1], off[1])); r = r < 0.f ? 0.f : r; break;
      case 2: r = a * ld(dt, ins[1], off[1]); break;
      case 3: r = rnd(dt, a * ld(dt, ins[1], off[1])) + ld(dt, ins[2], off[2]); break;
      case 5: r = a * (ld(dt, ins[1], off[1]) > 0.f ? 1.f : 0.f); break;
      default: r = a < 0.f ? 0.f : a; break;
    }
    if (op == 4 && !(a < 0.f)) {
      /* keep the input bits (Relu(-0) = -0, NaN stays NaN) */
      if (dt == DT_FLOAT) ((float*)out)[i] = ((const float*)ins[0])[off[0]];
      else ((uint16_t*)out)[i] = ((const uint16_t*)ins[0])[off[0]];
    } else {
      st(dt, out, i, r);
    }
  }
}

/* BiasAddGrad: out[c] = sum of x over every dimension except the channel
 * dimension (the last for NHWC, 1 for NCHW; reference
 * musa_ext/kernels/nn/musa_biasadd_grad_op.cc:31-52).  x is viewed as
 * [outer, C, inner].  Floating types are summed in double and rounded once to
 * T (TF sums half/bfloat16 in float, float in float, in Eigen's order);
 * int32 / int64 wrap modulo 2^32 / 2^64 as TF's integer sum does. */
void oracle_bias_add_grad(int dt, const void* x, int64_t outer, int64_t c, int64_t inner,
                          void* out) {
#ifdef _OPENMP
#pragma omp parallel for num_threads(g_threads) schedule(static)
#endif
  for (int64_t ch = 0; ch < c; ++ch) {
    if (dt == 3 || dt == 9) {
      uint64_t acc = 0;
      for (int64_t o = 0; o < outer; ++o)
        for (int64_t k = 0; k < inner; ++k) {
          const int64_t idx = (o * c + ch) * inner + k;
          acc += dt == 3 ? (uint64_t)(int64_t)((const int32_t*)x)[idx]
                         : (uint64_t)((const int64_t*)x)[idx];
        }
      if (dt == 3) ((int32_t*)out)[ch] = (int32_t)(uint32_t)acc;
      else ((int64_t*)out)[ch] = (int64_t)acc;
      continue;
    }
    double acc = 0.0;
    for (int64_t o = 0; o < outer; ++o)
      for (int64_t k = 0; k < inner; ++k) {
        const int64_t idx = (o * c + ch) * inner + k;
        acc += dt == DT_DOUBLE ? ((const double*)x)[idx] : (double)ld(dt, x, idx);
      }
    if (dt == DT_DOUBLE) ((double*)out)[ch] = acc;
    else st(dt, out, ch, (float)acc);
  }
}

/* ------------------------------------------------------------------------ */
/* CPU baseline of the cfg4 chains (bench.py's cpu_baseline leg; the parity  */
/* checker is oracle_eltwise above).  Contiguous [rows, cols] x with b and c  */
/* either full or a [cols] row vector, run as TF-CPU's vectorized kernels run */
/* them: a contiguous inner loop per row (OpenMP over rows, SIMD within),     */
/* and hardware half conversions (F16C) where the host has them.  Same        */
/* rounding points as oracle_eltwise, which tests/test_oracle.py checks bit   */
/* for bit.  op: 0 add, 1 add+relu, 3 mul+add (x*b rounded, + c).             */
/* ------------------------------------------------------------------------ */
#if defined(__x86_64__)
#include <immintrin.h>
__attribute__((target("avx2,f16c"))) static void rows_f16_hw(int op, const uint16_t* x,
                                                             const uint16_t* b, int b_row,
                                                             const uint16_t* c, int c_row,
                                                             int64_t rows, int64_t cols,
                                                             uint16_t* out) {
#ifdef _OPENMP
#pragma omp parallel for num_threads(g_threads) schedule(static)
#endif
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* xr = x + r * cols;
    const uint16_t* br = b ? (b_row ? b : b + r * cols) : NULL;
    const uint16_t* cr = c ? (c_row ? c : c + r * cols) : NULL;
    uint16_t* orow = out + r * cols;
    int64_t j = 0;
    for (; j + 8 <= cols; j += 8) {
      const __m256 xv = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(xr + j)));
      const __m256 bv = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(br + j)));
      __m256 v;
      if (op == 3) {
        const __m128i p = _mm256_cvtps_ph(_mm256_mul_ps(xv, bv), _MM_FROUND_TO_NEAREST_INT);
        const __m256 cv = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(cr + j)));
        v = _mm256_add_ps(_mm256_cvtph_ps(p), cv);
      } else {
        v = _mm256_add_ps(xv, bv);
      }
      __m128i h = _mm256_cvtps_ph(v, _MM_FROUND_TO_NEAREST_INT);
      if (op == 1) {
        /* relu on the rounded half: a value below zero - sign bit set,
         * magnitude nonzero (not -0) and at most infinity's (not NaN) -
         * becomes +0; everything else keeps its bits. */
        const __m128i mag = _mm_and_si128(h, _mm_set1_epi16(0x7fff));
        const __m128i sign = _mm_cmplt_epi16(h, _mm_setzero_si128());
        const __m128i zero = _mm_cmpeq_epi16(mag, _mm_setzero_si128());
        const __m128i num = _mm_cmplt_epi16(mag, _mm_set1_epi16(0x7c01));
        const __m128i neg = _mm_andnot_si128(zero, _mm_and_si128(sign, num));
        h = _mm_andnot_si128(neg, h);
      }
      _mm_storeu_si128((__m128i*)(orow + j), h);
    }
    for (; j < cols; ++j) {
      float v;
      const float xv = oracle_f16_to_f32(xr[j]), bv = oracle_f16_to_f32(br[j]);
      if (op == 3) v = oracle_f16_to_f32(oracle_f32_to_f16(xv * bv)) + oracle_f16_to_f32(cr[j]);
      else v = xv + bv;
      uint16_t h = oracle_f32_to_f16(v);
      if (op == 1 && oracle_f16_to_f32(h) < 0.f) h = 0;
      orow[j] = h;
    }
  }
}
#endif

void oracle_baseline_rows(int dt, int op, const void* x, const void* b, int b_row, const void* c,
                          int c_row, int64_t rows, int64_t cols, void* out) {
#if defined(__x86_64__)
  if (dt == DT_HALF && __builtin_cpu_supports("f16c") && __builtin_cpu_supports("avx2")) {
    rows_f16_hw(op, (const uint16_t*)x, (const uint16_t*)b, b_row, (const uint16_t*)c, c_row,
                rows, cols, (uint16_t*)out);
    return;
  }
#endif
#ifdef _OPENMP
#pragma omp parallel for num_threads(g_threads) schedule(static)
#endif
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t o = r * cols;
    const int64_t ob = b_row ? 0 : o, oc = c_row ? 0 : o;
    if (dt == DT_FLOAT) {
      const float* xr = (const float*)x + o;
      const float* br = (const float*)b + ob;
      const float* cr = c ? (const float*)c + oc : NULL;
      float* orow = (float*)out + o;
      if (op == 3) {
#ifdef _OPENMP
#pragma omp simd
#endif
        for (int64_t j = 0; j < cols; ++j) orow[j] = xr[j] * br[j] + cr[j];
      } else if (op == 1) {
#ifdef _OPENMP
#pragma omp simd
#endif
        for (int64_t j = 0; j < cols; ++j) {
          const float v = xr[j] + br[j];
          orow[j] = v < 0.f ? 0.f : v;
        }
      } else {
#ifdef _OPENMP
#pragma omp simd
#endif
        for (int64_t j = 0; j < cols; ++j) orow[j] = xr[j] + br[j];
      }
    } else {
      for (int64_t j = 0; j < cols; ++j) {
        const float xv = ld(dt, x, o + j), bv = ld(dt, b, ob + j);
        float v = op == 3 ? rnd(dt, xv * bv) + ld(dt, c, oc + j) : xv + bv;
        if (op == 1) {
          v = rnd(dt, v);
          v = v < 0.f ? 0.f : v;
        }
        st(dt, out, o + j, v);
      }
    }
  }
}

/* ------------------------------------------------------------------------ */
/* CPU baseline of the NHWC training BatchNorm (bench.py's cpu_baseline      */
/* leg; the checker is oracle_bn_fwd / oracle_bn_grad above).  x is          */
/* [rows, C] contiguous.  The same two passes as TF's CPU kernel (statistics, */
/* then the outputs), vectorized over channels: per-thread sums over blocks  */
/* of 64 rows in float, added into per-thread double sums and combined in    */
/* thread order; the forward's sums are shifted by the first row (no         */
/* cancellation when |mean| >> std).  Outputs round to T once (bfloat16:     */
/* round-to-nearest-even on finite values).                                  */
/* ------------------------------------------------------------------------ */
#if defined(__x86_64__)
#define BL_TARGET __attribute__((target("avx2,f16c")))
BL_TARGET static inline __m256 bl_ld8(int dt, const void* p, int64_t i) {
  if (dt == DT_FLOAT) return _mm256_loadu_ps((const float*)p + i);
  const __m128i h = _mm_loadu_si128((const __m128i*)((const uint16_t*)p + i));
  if (dt == DT_HALF) return _mm256_cvtph_ps(h);
  return _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(h), 16));
}
BL_TARGET static inline void bl_st8(int dt, void* p, int64_t i, __m256 v) {
  if (dt == DT_FLOAT) {
    _mm256_storeu_ps((float*)p + i, v);
    return;
  }
  __m128i h;
  if (dt == DT_HALF) {
    h = _mm256_cvtps_ph(v, _MM_FROUND_TO_NEAREST_INT);
  } else {
    __m256i u = _mm256_castps_si256(v);
    const __m256i lsb = _mm256_and_si256(_mm256_srli_epi32(u, 16), _mm256_set1_epi32(1));
    u = _mm256_srli_epi32(_mm256_add_epi32(u, _mm256_add_epi32(_mm256_set1_epi32(0x7fff), lsb)),
                          16);
    /* 32 -> 16 bits: packus works within each 128-bit half; keep qwords 0, 2 */
    const __m256i pk = _mm256_permute4x64_epi64(_mm256_packus_epi32(u, u), 0x08);
    h = _mm256_castsi256_si128(pk);
  }
  _mm_storeu_si128((__m128i*)((uint16_t*)p + i), h);
}
#define BL_HW 1
#else
#define BL_TARGET
#define BL_HW 0
#endif

enum { BL_BLOCK = 64 };

/* Per-channel sums over rows [r0, r1) of thread t's share.  mode 0:
 * (x - K), (x - K)^2; mode 1: dy, dy * (x - K) (K = the mean). */
BL_TARGET static void bl_sums(int dt, int mode, const void* x, const void* dy, int64_t r0,
                              int64_t r1, int64_t C, const float* K, float* a1, float* a2,
                              double* d1, double* d2) {
  const int64_t cv = BL_HW ? C / 8 * 8 : 0;
  for (int64_t r = r0; r < r1; r += BL_BLOCK) {
    const int64_t re = r + BL_BLOCK < r1 ? r + BL_BLOCK : r1;
    for (int64_t c = 0; c < C; ++c) a1[c] = a2[c] = 0.f;
    for (int64_t rr = r; rr < re; ++rr) {
      const int64_t o = rr * C;
      int64_t c = 0;
#if BL_HW
      for (; c < cv; c += 8) {
        const __m256 xc = _mm256_sub_ps(bl_ld8(dt, x, o + c), _mm256_loadu_ps(K + c));
        __m256 s1 = _mm256_loadu_ps(a1 + c), s2 = _mm256_loadu_ps(a2 + c);
        if (mode == 0) {
          s1 = _mm256_add_ps(s1, xc);
          s2 = _mm256_add_ps(s2, _mm256_mul_ps(xc, xc));
        } else {
          const __m256 d = bl_ld8(dt, dy, o + c);
          s1 = _mm256_add_ps(s1, d);
          s2 = _mm256_add_ps(s2, _mm256_mul_ps(d, xc));
        }
        _mm256_storeu_ps(a1 + c, s1);
        _mm256_storeu_ps(a2 + c, s2);
      }
#endif
      for (; c < C; ++c) {
        const float xc = ld(dt, x, o + c) - K[c];
        if (mode == 0) {
          a1[c] += xc;
          a2[c] += xc * xc;
        } else {
          const float d = ld(dt, dy, o + c);
          a1[c] += d;
          a2[c] += d * xc;
        }
      }
    }
    for (int64_t c = 0; c < C; ++c) {
      d1[c] += a1[c];
      d2[c] += a2[c];
    }
  }
}

/* Sums over all rows, per-thread then in thread order: s1, s2 [C]. */
static void bl_all_sums(int dt, int mode, const void* x, const void* dy, int64_t rows, int64_t C,
                        const float* K, double* s1, double* s2) {
  const int nt = g_threads;
  double* part = (double*)calloc((size_t)nt * 2 * (size_t)C, sizeof(double));
  float* blk = (float*)malloc((size_t)nt * 2 * (size_t)C * sizeof(float));
#ifdef _OPENMP
#pragma omp parallel for num_threads(nt) schedule(static, 1)
#endif
  for (int t = 0; t < nt; ++t) {
    const int64_t r0 = rows * t / nt, r1 = rows * (t + 1) / nt;
    bl_sums(dt, mode, x, dy, r0, r1, C, K, blk + (size_t)t * 2 * C, blk + (size_t)t * 2 * C + C,
            part + (size_t)t * 2 * C, part + (size_t)t * 2 * C + C);
  }
  for (int64_t c = 0; c < C; ++c) s1[c] = s2[c] = 0.0;
  for (int t = 0; t < nt; ++t)
    for (int64_t c = 0; c < C; ++c) {
      s1[c] += part[(size_t)t * 2 * C + c];
      s2[c] += part[(size_t)t * 2 * C + C + c];
    }
  free(part);
  free(blk);
}

/* out[r, c] = (x - m[c]) * a[c] + b[c] (forward), or with dy: a[c] * ((dy -
 * b[c]) - (x - m[c]) * e[c]) (gradient). */
BL_TARGET static void bl_apply(int dt, int grad, const void* x, const void* dy, int64_t rows,
                               int64_t C, const float* m, const float* a, const float* b,
                               const float* e, void* out) {
  const int64_t cv = BL_HW ? C / 8 * 8 : 0;
#ifdef _OPENMP
#pragma omp parallel for num_threads(g_threads) schedule(static)
#endif
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t o = r * C;
    int64_t c = 0;
#if BL_HW
    for (; c < cv; c += 8) {
      const __m256 xc = _mm256_sub_ps(bl_ld8(dt, x, o + c), _mm256_loadu_ps(m + c));
      __m256 v;
      if (!grad) {
        v = _mm256_add_ps(_mm256_mul_ps(xc, _mm256_loadu_ps(a + c)), _mm256_loadu_ps(b + c));
      } else {
        const __m256 d = _mm256_sub_ps(bl_ld8(dt, dy, o + c), _mm256_loadu_ps(b + c));
        v = _mm256_mul_ps(_mm256_loadu_ps(a + c),
                          _mm256_sub_ps(d, _mm256_mul_ps(xc, _mm256_loadu_ps(e + c))));
      }
      bl_st8(dt, out, o + c, v);
    }
#endif
    for (; c < C; ++c) {
      const float xc = ld(dt, x, o + c) - m[c];
      const float v = grad ? a[c] * ((ld(dt, dy, o + c) - b[c]) - xc * e[c]) : xc * a[c] + b[c];
      st(dt, out, o + c, v);
    }
  }
}

/* Training forward: y, and the population mean and variance per channel. */
void oracle_baseline_bn_fwd(int dt, const void* x, int64_t rows, int64_t C, const float* scale,
                            const float* offset, float eps, void* y, float* mean, float* var) {
  if (rows <= 0 || C <= 0) return;
  float* K = (float*)malloc(sizeof(float) * 4 * (size_t)C);
  float* a = K + C;
  float* b = a + C;
  float* m = b + C;
  double* s = (double*)malloc(sizeof(double) * 2 * (size_t)C);
  for (int64_t c = 0; c < C; ++c) K[c] = ld(dt, x, c);
  bl_all_sums(dt, 0, x, NULL, rows, C, K, s, s + C);
  for (int64_t c = 0; c < C; ++c) {
    const double d = s[c] / (double)rows;
    m[c] = (float)((double)K[c] + d);
    const double v = s[C + c] / (double)rows - d * d;
    mean[c] = m[c];
    var[c] = (float)(v > 0.0 ? v : 0.0);
    a[c] = (1.0f / sqrtf(var[c] + eps)) * scale[c];
    b[c] = offset[c];
  }
  bl_apply(dt, 0, x, NULL, rows, C, m, a, b, NULL, y);
  free(K);
  free(s);
}

/* Training gradient from the forward's mean and population variance. */
void oracle_baseline_bn_grad(int dt, const void* dy, const void* x, int64_t rows, int64_t C,
                             const float* scale, const float* mean, const float* var, float eps,
                             void* dx, float* scale_bp, float* offset_bp) {
  if (rows <= 0 || C <= 0) return;
  float* k = (float*)malloc(sizeof(float) * 4 * (size_t)C);
  float* a = k + C;
  float* b = a + C;
  float* e = b + C;
  double* s = (double*)malloc(sizeof(double) * 2 * (size_t)C);
  bl_all_sums(dt, 1, x, dy, rows, C, mean, s, s + C);
  for (int64_t c = 0; c < C; ++c) {
    k[c] = 1.0f / sqrtf(var[c] + eps);
    offset_bp[c] = (float)s[c];
    scale_bp[c] = (float)(s[C + c] * (double)k[c]);
    a[c] = scale[c] * k[c];
    b[c] = (float)(s[c] / (double)rows);
    e[c] = (k[c] * k[c]) * (float)(s[C + c] / (double)rows);
  }
  bl_apply(dt, 1, x, dy, rows, C, mean, a, b, e, dx);
  free(k);
  free(s);
}

/* CPU baseline of float ResourceApplyAdam (bench.py's cpu_baseline leg; the
 * checker is oracle_adam): the checker's float operations in its order,
 * without the per-element dtype dispatch, so the loop vectorizes (8-wide
 * IEEE sqrt and divide give the scalar loop's bits). */
BL_TARGET void oracle_baseline_adam_f32(float* var, float* m, float* v, const float* grad,
                                        int64_t n, double b1p_, double b2p_, double lr_,
                                        double b1_, double b2_, double eps_) {
  const float b1p = (float)b1p_, b2p = (float)b2p_, lr = (float)lr_;
  const float b1 = (float)b1_, b2 = (float)b2_, eps = (float)eps_;
  const float alpha = (lr * sqrtf(1.0f - b2p)) / (1.0f - b1p);
  const float omb1 = 1.0f - b1, omb2 = 1.0f - b2;
  (void)b1;
  const int64_t nv = BL_HW ? n / 8 : 0;
#ifdef _OPENMP
#pragma omp parallel for num_threads(g_threads) schedule(static)
#endif
  for (int64_t k = 0; k < nv; ++k) {
#if BL_HW
    const int64_t i = 8 * k;
    const __m256 g = _mm256_loadu_ps(grad + i);
    const __m256 m0 = _mm256_loadu_ps(m + i), v0 = _mm256_loadu_ps(v + i);
    const __m256 mm =
        _mm256_add_ps(m0, _mm256_mul_ps(_mm256_sub_ps(g, m0), _mm256_set1_ps(omb1)));
    const __m256 vv = _mm256_add_ps(
        v0, _mm256_mul_ps(_mm256_sub_ps(_mm256_mul_ps(g, g), v0), _mm256_set1_ps(omb2)));
    _mm256_storeu_ps(m + i, mm);
    _mm256_storeu_ps(v + i, vv);
    const __m256 den = _mm256_add_ps(_mm256_sqrt_ps(vv), _mm256_set1_ps(eps));
    const __m256 step = _mm256_div_ps(_mm256_mul_ps(mm, _mm256_set1_ps(alpha)), den);
    _mm256_storeu_ps(var + i, _mm256_sub_ps(_mm256_loadu_ps(var + i), step));
#endif
  }
  for (int64_t i = 8 * nv; i < n; ++i) {
    const float g = grad[i];
    const float mm = m[i] + (g - m[i]) * omb1;
    const float vv = v[i] + (g * g - v[i]) * omb2;
    m[i] = mm;
    v[i] = vv;
    var[i] = var[i] - (mm * alpha) / (sqrtf(vv) + eps);
  }
}
