/*
 * Oracle for the int8 frozen-weight LoRA linear (CPU restatement of Reels.jl).
 * TEST INFRASTRUCTURE ONLY: see oracle.h for who may call it and what pins each function.
 * Build: plain gcc, -O2 -fopenmp, no -ffast-math (IEEE division, rint ties-to-even and
 * denormals must behave as Julia's Float32 arithmetic does).
 */
#include "oracle.h"
#include <math.h>
#include <string.h>
#include <stdlib.h>

/* ---- bf16 conversions: src/models/interface.jl:13-25 ---------------------------------- */
float oracle_bf16_to_f32(uint16_t h) {
  /* float32_values: UInt32(bits) << 16 reinterpreted (interface.jl:13-16) */
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t oracle_f32_to_bf16(float f) {
  /* bfloat16_values: (bits + 0x7fff + ((bits >> 16) & 1)) >> 16 in wrapping UInt32
   * arithmetic (interface.jl:19-25) */
  uint32_t u;
  memcpy(&u, &f, 4);
  u = u + 0x00007fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

void oracle_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_bf16(in[i]);
}

void oracle_bf16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_bf16_to_f32(in[i]);
}

/* ---- f16 helpers (IEEE binary16, round-to-nearest-even) -------------------------------- */
static float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff;
  float f;
  if (exp == 0) {
    f = ldexpf((float)man, -24);
    if (sign) f = -f;
    return f;
  }
  if (exp == 31) {
    uint32_t u = sign | 0x7f800000u | (man << 13);
    memcpy(&f, &u, 4);
    return f;
  }
  uint32_t u = sign | ((exp + 112) << 23) | (man << 13);
  memcpy(&f, &u, 4);
  return f;
}

static uint16_t f32_to_f16(float f) {
  /* Round an f32 to the nearest binary16, ties to even (textbook; handles subnormals). */
  uint32_t u;
  memcpy(&u, &f, 4);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000);
  float a = fabsf(f);
  if (isnan(f)) return sign | 0x7e00;
  if (a >= 65520.0f) return sign | 0x7c00; /* rounds to infinity */
  if (a < ldexpf(1.0f, -14)) {
    /* subnormal range: quantum 2^-24, nearbyint rounds ties to even */
    float m = nearbyintf(a * 16777216.0f);
    return sign | (uint16_t)m; /* m <= 1024 gives the smallest normal when it carries */
  }
  int e;
  float mant = frexpf(a, &e); /* a = mant * 2^e, mant in [0.5, 1) */
  float scaled = nearbyintf(mant * 2048.0f); /* 11 significant bits */
  if (scaled >= 2048.0f) { scaled = 1024.0f; e += 1; }
  int exp16 = e - 1 + 15;
  if (exp16 >= 31) return sign | 0x7c00;
  return sign | (uint16_t)((exp16 << 10) | ((int)scaled - 1024));
}

void oracle_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f16_to_f32(in[i]);
}

void oracle_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_f16(in[i]);
}

/* value of a 16-bit element: elt 0 = bf16 bits, 1 = IEEE binary16 bits (both exact in f32) */
static float in16(uint16_t h, int elt) { return elt ? f16_to_f32(h) : oracle_bf16_to_f32(h); }
static uint16_t out16(float f, int elt) { return elt ? f32_to_f16(f) : oracle_f32_to_bf16(f); }
/* element i of an activation / adapter array: elt 0 = bf16, 1 = f16 (16-bit codes), 2 = f32 */
static float inel(const void* p, int64_t i, int elt) {
  return elt == 2 ? ((const float*)p)[i] : in16(((const uint16_t*)p)[i], elt);
}
static void outel(void* p, int64_t i, float f, int elt) {
  if (elt == 2) ((float*)p)[i] = f;
  else ((uint16_t*)p)[i] = out16(f, elt);
}

/* ---- quantize_frozen_matrix: src/layers/quantization.jl:35-44 --------------------------- */
static float load_elem(const void* w, int dtype, int64_t idx) {
  if (dtype == 0) return ((const float*)w)[idx];
  if (dtype == 1) return oracle_bf16_to_f32(((const uint16_t*)w)[idx]);
  return f16_to_f32(((const uint16_t*)w)[idx]);
}

int oracle_pack(const void* w, int dtype, int64_t N, int64_t K, int64_t ld, int8_t* q, float* s) {
  if (N < 0 || K <= 0 || ld < K || dtype < 0 || dtype > 2) return -1;
  int status = 0;
#pragma omp parallel for schedule(static) reduction(| : status)
  for (int64_t n = 0; n < N; ++n) {
    const int64_t base = n * ld;
    /* maxima = vec(maximum(abs, host; dims=2)) (line 38); Julia's max propagates NaN */
    float m = 0.0f;
    int has_nan = 0;
    for (int64_t k = 0; k < K; ++k) {
      float a = fabsf(load_elem(w, dtype, base + k));
      if (isnan(a)) has_nan = 1;
      else if (a > m) m = a;
    }
    if (has_nan) m = NAN;
    /* scales = maxima ./ 127f0 (line 39), IEEE f32 division */
    volatile float scale = m / 127.0f;
    /* scales[maxima .== 0f0] .= 1f0 (line 40) */
    if (m == 0.0f) scale = 1.0f;
    s[n] = scale;
    /* values = Int8.(round.(clamp.(host ./ scale, -127f0, 127f0))) (lines 41-42) */
    for (int64_t k = 0; k < K; ++k) {
      volatile float v = load_elem(w, dtype, base + k) / scale;
      float cl = v > 127.0f ? 127.0f : (v < -127.0f ? -127.0f : v); /* Base.clamp */
      float rd = rintf(cl); /* round(x) = RoundNearest = ties to even */
      if (!isfinite(rd)) { /* Int8(NaN) throws InexactError */
        status = 1;
        q[n * K + k] = 0;
      } else {
        q[n * K + k] = (int8_t)rd;
      }
    }
  }
  return status;
}

/* ---- dequantization: quantization.jl:25-29 (_host_dequantize), 61-64 -------------------- */
void oracle_dequant(const int8_t* q, const float* s, int64_t N, int64_t K, int mode, void* out) {
  for (int64_t n = 0; n < N; ++n) {
    uint16_t s16 = f32_to_f16(s[n]);
    float s16f = f16_to_f32(s16);
    for (int64_t k = 0; k < K; ++k) {
      int64_t i = n * K + k;
      if (mode == 0) {
        ((float*)out)[i] = (float)q[i] * s[n];
      } else if (mode == 1) {
        /* Float16(q) * Float16(s): Julia computes Float16 products in Float32 and rounds once;
         * the product of two binary16 values is exact in Float32. */
        ((uint16_t*)out)[i] = f32_to_f16((float)q[i] * s16f);
      } else {
        ((uint16_t*)out)[i] = oracle_f32_to_bf16((float)q[i] * s[n]);
      }
    }
  }
}

/* ---- lora_forward: src/layers/lora.jl:56-95 ------------------------------------------- */
void oracle_lora_forward(const void* x, const int8_t* q, const float* s, const void* A,
                         const void* B, const void* bias, int64_t M, int64_t K, int64_t N,
                         int64_t r, float c, const int64_t* rows, int64_t nrows, double* y_out,
                         double* h_out, int elt) {
  if (!rows) nrows = M;
  double* Ad = (double*)malloc(sizeof(double) * (size_t)(K * (r > 0 ? r : 1)));
  double* Bd = (double*)malloc(sizeof(double) * (size_t)((r > 0 ? r : 1) * N));
  for (int64_t i = 0; i < K * r; ++i) Ad[i] = inel(A, i, elt);
  for (int64_t i = 0; i < r * N; ++i) Bd[i] = inel(B, i, elt);
#pragma omp parallel
  {
    double* xr = (double*)malloc(sizeof(double) * (size_t)K);
    double* hr = (double*)malloc(sizeof(double) * (size_t)(r > 0 ? r : 1));
#pragma omp for schedule(dynamic, 4)
    for (int64_t ii = 0; ii < nrows; ++ii) {
      int64_t m = rows ? rows[ii] : ii;
      for (int64_t k = 0; k < K; ++k) xr[k] = inel(x, m * K + k, elt);
      /* A * z (lora.jl:86) */
      for (int64_t j = 0; j < r; ++j) hr[j] = 0.0;
      for (int64_t k = 0; k < K; ++k)
        for (int64_t j = 0; j < r; ++j) hr[j] += xr[k] * Ad[k * r + j];
      if (h_out)
        for (int64_t j = 0; j < r; ++j) h_out[ii * r + j] = hr[j];
      if (y_out) {
        for (int64_t n = 0; n < N; ++n) {
          /* _weight_mul: deq(W) * x (quantization.jl:73-74) */
          const int8_t* qr = q + n * K;
          double acc = 0.0;
          for (int64_t k = 0; k < K; ++k) acc += xr[k] * (double)qr[k];
          double y = acc * (double)s[n];
          /* bias: mixed_add(y, bias) (lora.jl:64-67) */
          if (bias) y += inel(bias, n, elt);
          /* adapter = c * B * (A * z) (lora.jl:86-94) */
          double ad = 0.0;
          for (int64_t j = 0; j < r; ++j) ad += hr[j] * Bd[j * N + n];
          y_out[ii * N + n] = y + (double)c * ad;
        }
      }
    }
    free(xr);
    free(hr);
  }
  free(Ad);
  free(Bd);
}

/* ---- lora_backward: src/layers/lora.jl:106-118 ------------------------------------------ */
void oracle_lora_backward(const void* dy, const void* x, const int8_t* q, const float* s,
                          const void* A, const void* B, int64_t M, int64_t K, int64_t N,
                          int64_t r, float c, const int64_t* rows, int64_t nrows,
                          const int64_t* kcols, int64_t nk, const int64_t* ncols, int64_t nn,
                          double* dx_out, double* dA_out, double* dB_out, int elt) {
  if (!rows) nrows = M;
  if (!kcols) nk = K;
  if (!ncols) nn = N;
  const int64_t rr = r > 0 ? r : 1;
  double* Ad = (double*)malloc(sizeof(double) * (size_t)(K * rr));
  double* Bd = (double*)malloc(sizeof(double) * (size_t)(rr * N));
  for (int64_t i = 0; i < K * r; ++i) Ad[i] = inel(A, i, elt);
  for (int64_t i = 0; i < r * N; ++i) Bd[i] = inel(B, i, elt);
  /* u = B' * dy and h = A * x for every token (lora.jl:112-113) */
  double* u = (double*)malloc(sizeof(double) * (size_t)(M * rr));
  double* h = (double*)malloc(sizeof(double) * (size_t)(M * rr));
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t j = 0; j < r; ++j) { u[m * r + j] = 0.0; h[m * r + j] = 0.0; }
    for (int64_t n = 0; n < N; ++n) {
      double d = inel(dy, m * N + n, elt);
      for (int64_t j = 0; j < r; ++j) u[m * r + j] += d * Bd[j * N + n];
    }
    if (dB_out)
      for (int64_t k = 0; k < K; ++k) {
        double xv = inel(x, m * K + k, elt);
        for (int64_t j = 0; j < r; ++j) h[m * r + j] += xv * Ad[k * r + j];
      }
  }
  if (dx_out) {
    /* dx = _weight_transpose_mul(W, dy) + c * A' * (B' * dy) (lora.jl:115-116) */
#pragma omp parallel
    {
      double* acc = (double*)malloc(sizeof(double) * (size_t)K);
#pragma omp for schedule(dynamic, 4)
      for (int64_t ii = 0; ii < nrows; ++ii) {
        int64_t m = rows ? rows[ii] : ii;
        for (int64_t k = 0; k < K; ++k) acc[k] = 0.0;
        for (int64_t n = 0; n < N; ++n) {
          double d = (double)inel(dy, m * N + n, elt) * (double)s[n];
          const int8_t* qr = q + n * K;
          for (int64_t k = 0; k < K; ++k) acc[k] += d * (double)qr[k];
        }
        for (int64_t k = 0; k < K; ++k) {
          double l = 0.0;
          for (int64_t j = 0; j < r; ++j) l += u[m * r + j] * Ad[k * r + j];
          dx_out[ii * K + k] = acc[k] + (double)c * l;
        }
      }
      free(acc);
    }
  }
  if (dA_out) {
    /* dA = c * (B' * dy) * x' (lora.jl:113) */
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t kk = 0; kk < nk; ++kk) {
      int64_t k = kcols ? kcols[kk] : kk;
      double accj[256];
      for (int64_t j = 0; j < r; ++j) accj[j] = 0.0;
      for (int64_t m = 0; m < M; ++m) {
        double xv = inel(x, m * K + k, elt);
        for (int64_t j = 0; j < r; ++j) accj[j] += u[m * r + j] * xv;
      }
      for (int64_t j = 0; j < r; ++j) dA_out[kk * r + j] = (double)c * accj[j];
    }
  }
  if (dB_out) {
    /* dB = c * dy * (A x)' (lora.jl:114) */
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t nn_i = 0; nn_i < nn; ++nn_i) {
      int64_t n = ncols ? ncols[nn_i] : nn_i;
      double accj[256];
      for (int64_t j = 0; j < r; ++j) accj[j] = 0.0;
      for (int64_t m = 0; m < M; ++m) {
        double d = inel(dy, m * N + n, elt);
        for (int64_t j = 0; j < r; ++j) accj[j] += h[m * r + j] * d;
      }
      for (int64_t j = 0; j < r; ++j) dB_out[j * nn + nn_i] = (double)c * accj[j];
    }
  }
  free(u);
  free(h);
  free(Ad);
  free(Bd);
}

/* ---- gelu_tanh: src/layers/linear.jl:61-68 ----------------------------------------------- */
static float gelu_f32(float x) {
  float cubic = x * x * x;                      /* x32 .^ 3 */
  float inner = x + 0.044715f * cubic;          /* x32 .+ 0.044715f0 .* cubic */
  float k = (float)sqrt(2.0 / 3.14159265358979323846); /* sqrt(Float32(2 / pi)) */
  float activated = tanhf(k * inner);
  return 0.5f * x * (1.0f + activated);
}

void oracle_gelu_tanh(const void* x, void* y, int64_t n, int elt) {
  for (int64_t i = 0; i < n; ++i) outel(y, i, gelu_f32(inel(x, i, elt)), elt);
}

void oracle_gelu_tanh_backward(const void* x, const void* dy, void* dx, int64_t n,
                               int elt) {
  /* d/dx 0.5x(1+tanh(k(x+a x^3))) = 0.5(1+t) + 0.5x(1-t^2)k(1+3a x^2) */
  const double k = sqrt(2.0 / 3.14159265358979323846), a = 0.044715;
  for (int64_t i = 0; i < n; ++i) {
    double xv = inel(x, i, elt);
    double t = tanh(k * (xv + a * xv * xv * xv));
    double d = 0.5 * (1.0 + t) + 0.5 * xv * (1.0 - t * t) * k * (1.0 + 3.0 * a * xv * xv);
    outel(dx, i, (float)(d * (double)inel(dy, i, elt)), elt);
  }
}

/* ---- Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11) ------------------------------------ */
/* ---- attention (attention.jl:106-221) ---------------------------------------------------- */
static double att_scale(int64_t D) { return (double)(1.0f / sqrtf((float)D)); }

static int att_visible(const uint8_t* mask, int causal, int64_t Sk, int64_t i, int64_t j) {
  if (mask && !mask[i * Sk + j]) return 0;
  if (causal && j > i) return 0;
  return 1;
}

/* scores and probabilities of query i of head (b, h): p[j] = exp(s_j - m) / l over visible keys,
 * 0 elsewhere; returns lse (NaN when no key is visible, p then all NaN-free zeros) */
static double att_row(const void* q, const void* k, const uint8_t* mask, int causal, int64_t b,
                      int64_t i, int64_t h, int64_t Sq, int64_t Sk, int64_t H, int64_t D, int elt,
                      double* s, double* p) {
  const double sc = att_scale(D);
  const int64_t qo = ((b * Sq + i) * H + h) * D;
  double m = -INFINITY;
  int any = 0;
  for (int64_t j = 0; j < Sk; ++j) {
    if (!att_visible(mask, causal, Sk, i, j)) { s[j] = -INFINITY; continue; }
    const int64_t ko = ((b * Sk + j) * H + h) * D;
    double acc = 0.0;
    for (int64_t d = 0; d < D; ++d) acc += (double)inel(q, qo + d, elt) * (double)inel(k, ko + d, elt);
    s[j] = acc * sc;
    if (s[j] > m) m = s[j];
    any = 1;
  }
  if (!any) {
    for (int64_t j = 0; j < Sk; ++j) p[j] = 0.0;
    return Sk == 0 ? -INFINITY : NAN;  /* -Inf + log(0) without keys; NaN from exp(-Inf - -Inf) */
  }
  double l = 0.0;
  for (int64_t j = 0; j < Sk; ++j) { p[j] = isfinite(s[j]) ? exp(s[j] - m) : 0.0; l += p[j]; }
  for (int64_t j = 0; j < Sk; ++j) p[j] /= l;
  return m + log(l);
}

void oracle_attention_forward(const void* q, const void* k, const void* v, const uint8_t* mask,
                              int causal, int64_t B, int64_t Sq, int64_t Sk, int64_t H, int64_t D,
                              int elt, double* out, double* lse) {
  double* s = (double*)malloc(sizeof(double) * (size_t)(Sk > 0 ? Sk : 1));
  double* p = (double*)malloc(sizeof(double) * (size_t)(Sk > 0 ? Sk : 1));
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < H; ++h)
      for (int64_t i = 0; i < Sq; ++i) {
        const double L = att_row(q, k, mask, causal, b, i, h, Sq, Sk, H, D, elt, s, p);
        if (lse) lse[(b * H + h) * Sq + i] = L;
        if (!out) continue;
        double* o = out + ((b * Sq + i) * H + h) * D;
        const int none = !isfinite(L);
        for (int64_t d = 0; d < D; ++d) o[d] = none ? NAN : 0.0;
        if (none) continue;
        for (int64_t j = 0; j < Sk; ++j) {
          if (p[j] == 0.0) continue;
          const int64_t vo = ((b * Sk + j) * H + h) * D;
          for (int64_t d = 0; d < D; ++d) o[d] += p[j] * (double)inel(v, vo + d, elt);
        }
      }
  free(s);
  free(p);
}

void oracle_attention_backward(const void* q, const void* k, const void* v, const void* dy,
                               const uint8_t* mask, int causal, int64_t B, int64_t Sq, int64_t Sk,
                               int64_t H, int64_t D, int elt, double* dq, double* dk, double* dv) {
  const double sc = att_scale(D);
  double* s = (double*)malloc(sizeof(double) * (size_t)(Sk > 0 ? Sk : 1));
  double* p = (double*)malloc(sizeof(double) * (size_t)(Sk > 0 ? Sk : 1));
  double* o = (double*)malloc(sizeof(double) * (size_t)(D > 0 ? D : 1));
  if (dq) for (int64_t i = 0; i < B * Sq * H * D; ++i) dq[i] = 0.0;
  if (dk) for (int64_t i = 0; i < B * Sk * H * D; ++i) dk[i] = 0.0;
  if (dv) for (int64_t i = 0; i < B * Sk * H * D; ++i) dv[i] = 0.0;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < H; ++h)
      for (int64_t i = 0; i < Sq; ++i) {
        const double L = att_row(q, k, mask, causal, b, i, h, Sq, Sk, H, D, elt, s, p);
        const int64_t qo = ((b * Sq + i) * H + h) * D;
        /* the output of this query, and the correction sum(dy .* out) (attention.jl:190) */
        for (int64_t d = 0; d < D; ++d) o[d] = isfinite(L) ? 0.0 : NAN;
        if (isfinite(L))
          for (int64_t j = 0; j < Sk; ++j) {
            if (p[j] == 0.0) continue;
            const int64_t vo = ((b * Sk + j) * H + h) * D;
            for (int64_t d = 0; d < D; ++d) o[d] += p[j] * (double)inel(v, vo + d, elt);
          }
        double corr = 0.0;
        for (int64_t d = 0; d < D; ++d) corr += (double)inel(dy, qo + d, elt) * o[d];
        for (int64_t j = 0; j < Sk; ++j) {
          if (!isfinite(s[j])) continue;  /* masked: probability 0, no contribution */
          const int64_t ko = ((b * Sk + j) * H + h) * D;
          double dp = 0.0;
          for (int64_t d = 0; d < D; ++d) dp += (double)inel(dy, qo + d, elt) * (double)inel(v, ko + d, elt);
          const double ds = p[j] * (dp - corr);
          for (int64_t d = 0; d < D; ++d) {
            if (dq) dq[qo + d] += sc * ds * (double)inel(k, ko + d, elt);
            if (dk) dk[ko + d] += sc * ds * (double)inel(q, qo + d, elt);
            if (dv) dv[ko + d] += p[j] * (double)inel(dy, qo + d, elt);
          }
        }
      }
  free(s);
  free(p);
  free(o);
}

void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
  uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
  uint32_t k0 = key[0], k1 = key[1];
  for (int round = 0; round < 10; ++round) {
    uint64_t p0 = (uint64_t)M0 * c0, p1 = (uint64_t)M1 * c2;
    uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    uint32_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    k0 += W0; k1 += W1;
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

static double philox_normal(uint64_t seed, uint32_t stream, int64_t i, uint32_t words[4]) {
  uint32_t ctr[4] = {(uint32_t)i, (uint32_t)((uint64_t)i >> 32), stream, 0u};
  uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  oracle_philox4x32_10(ctr, key, words);
  double u1 = ((double)words[0] + 1.0) / 4294967296.0; /* (0, 1] */
  double u2 = (double)words[1] / 4294967296.0;         /* [0, 1) */
  return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

void oracle_normal_bf16(uint64_t seed, uint32_t stream, int64_t n, double sigma,
                        double outlier_rate, double outlier_sigma, uint16_t* out) {
  const double thresh = outlier_rate * 4294967296.0;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    uint32_t w[4];
    double z = philox_normal(seed, stream, i, w);
    double v = z * sigma;
    if (outlier_rate > 0.0 && (double)w[2] < thresh)
      v = ((w[3] & 1u) ? -outlier_sigma : outlier_sigma) * sigma;
    out[i] = oracle_f32_to_bf16((float)v);
  }
}

void oracle_normal_f32(uint64_t seed, uint32_t stream, int64_t n, double sigma, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    uint32_t w[4];
    out[i] = (float)(philox_normal(seed, stream, i, w) * sigma);
  }
}
