// Shared device/host helpers for the reels_hip kernels (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>
#include <type_traits>

#include "../../include/reels_hip.h"

namespace reels {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short i16x4;

#define LDS_PTR(T, p) ((__attribute__((address_space(3))) T*)(p))

// ---- bf16 <-> f32 ---------------------------------------------------------------------------
// bf16 -> f32 is exact (bits << 16); f32 -> bf16 rounds to nearest even with the same integer
// formula as the reference's bfloat16_values (src/models/interface.jl:19-25).
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
// two f32 -> packed bf16x2 (lo in bits 0-15), RNE
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

// ---- int8 -> bf16 (exact: |q| <= 127 has at most 8 significant bits) ------------------------
// Converts 4 packed int8 to 2 dwords of packed bf16. The f32 value of each code is exact and so
// is its top half, so the bf16 is taken by truncation (v_perm), no rounding needed.
__device__ __forceinline__ void i8x4_to_bf16x4(uint32_t w, uint32_t& o0, uint32_t& o1) {
  float f0 = (float)(int8_t)(w & 0xff);
  float f1 = (float)(int8_t)((w >> 8) & 0xff);
  float f2 = (float)(int8_t)((w >> 16) & 0xff);
  float f3 = (float)((int32_t)w >> 24);
  o0 = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
  o1 = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
}

__device__ __forceinline__ bf16x8 i8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
  u32x4 r;
  uint32_t a, b, c, d;
  i8x4_to_bf16x4(lo, a, b);
  i8x4_to_bf16x4(hi, c, d);
  r[0] = a; r[1] = b; r[2] = c; r[3] = d;
  return __builtin_bit_cast(bf16x8, r);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// ---- 16-bit element types of the LoRA linear --------------------------------------------------
// Elt<REELS_HIP_BF16> and Elt<REELS_HIP_F16> give each kernel its element arithmetic: unpack to
// f32 (exact), round f32 to the element (nearest even), the MFMA shapes, the exact int8
// conversion and the dequantized-weight element of the compute type.
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;

// HBM -> LDS copy of 16 bytes per lane (buffer_load_dwordx4 ... lds): lane i's data lands at
// LDS byte ldsaddr + 16 i (ldsaddr in M0). Issued through inline asm so the compiler does not
// order the kernel's LDS reads behind it: the kernel synchronises these copies itself (explicit
// vmcnt waits followed by a workgroup barrier).
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
__device__ __forceinline__ i32x4 buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = (int)(uint32_t)b;
  r[1] = (int)((b >> 32) & 0xffffu);  // stride 0
  r[2] = (int)bytes;                  // num_records: reads past it return 0
  r[3] = 0x00020000;                  // raw buffer, 32-bit data format
  return r;
}
// The compiler writes M0 right before the asm but does not know that the copy reads it: on
// this GPU generation an LDS-DMA instruction needs one wait state after an SALU write of M0,
// hence the s_nop.
__device__ __forceinline__ void dma16(const i32x4& rsrc, uint32_t voff, uint32_t soff,
                                      const uint8_t* lds) {
  const uint32_t ldsaddr = (uint32_t)(uintptr_t)LDS_PTR(const uint8_t, lds);
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc),
               "s"(soff), "{m0}"(ldsaddr)
               : "memory");
}

// the same with the LDS byte address given as a (wave-uniform) integer
__device__ __forceinline__ void dma16_at(const i32x4& rsrc, uint32_t voff, uint32_t soff,
                                         uint32_t ldsaddr) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc),
               "s"(soff), "{m0}"(ldsaddr)
               : "memory");
}

// Reductions over lanes l, l^16, l^32, l^48. v_permlane16_swap (v_permlane32_swap) with x as both
// operands hands every lane the values of lanes l and l^16 (l^32), in an order that depends on
// the lane: a VALU exchange instead of an LDS round trip (ds_bpermute). The sums are the same
// bits as (x_l + x_l^16) + (x_l^32 + x_l^48) in any lane order, since a + b == b + a.
__device__ __forceinline__ float wave_max16(float x) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
__device__ __forceinline__ float wave_sum16(float x) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// tanh(u) from one exponential and one reciprocal: |t| = 1 - 2 / (1 + 2^(2 |u| log2 e)) with the
// sign of u (v_exp_f32 and v_rcp_f32, each within 1 ulp; no overflow path: a huge |u| gives
// 2 / inf = 0, |t| = 1; NaN stays NaN). Within 2^-23 of tanh(u) absolute, so 1 + t and 1 - t^2
// below carry the same cancellation as with a correctly rounded tanh (for u << 0, 1 + t is
// rounded near -1 in both). About 6 VALU operations against ~25 for the libm tanhf, whose range
// reduction made the GELU passes VALU-bound.
__device__ __forceinline__ float tanh_f(float u) {
  const float e = __builtin_amdgcn_exp2f(fabsf(u) * 2.8853900817779268f);  // 2 log2(e)
  const float m = fmaf(-2.0f, __builtin_amdgcn_rcpf(1.0f + e), 1.0f);
  return copysignf(m, u);
}

// gelu_tanh, src/layers/linear.jl:61-68, in f32, and its analytic derivative
__device__ __forceinline__ float gelu_f(float x) {
  const float k = 0.7978845608028654f;  // sqrt(Float32(2 / pi))
  const float inner = x + 0.044715f * (x * x * x);
  return 0.5f * x * (1.0f + tanh_f(k * inner));
}
__device__ __forceinline__ float gelu_grad_f(float x) {
  const float k = 0.7978845608028654f, a = 0.044715f;
  const float t = tanh_f(k * (x + a * x * x * x));
  return 0.5f * (1.0f + t) + 0.5f * x * (1.0f - t * t) * k * (1.0f + 3.0f * a * x * x);
}
template <int ELT> struct Elt;

template <> struct Elt<REELS_HIP_BF16> {
  typedef bf16x8 v8;
  static __device__ __forceinline__ float to_f32(uint16_t h) { return bf16_to_f32(h); }
  static __device__ __forceinline__ float lo(uint32_t w) { return bf16_lo(w); }
  static __device__ __forceinline__ float hi(uint32_t w) { return bf16_hi(w); }
  static __device__ __forceinline__ uint32_t bits(float f) { return f32_to_bf16_bits(f); }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) { return pack_bf16x2(a, b); }
  // the same rounding for finite values in one v_cvt_pk_bf16_f32 (NaN patterns may differ from
  // pack2's, and f32 denormals follow the denormal mode): for MFMA operands computed in a kernel
  static __device__ __forceinline__ uint32_t pack2_fast(float a, float b) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    const bf2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
  static __device__ __forceinline__ v8 as8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
  static __device__ __forceinline__ v8 from_i8x8(uint32_t l, uint32_t h) { return i8x8_to_bf16x8(l, h); }
  static __device__ __forceinline__ f32x4 mfma16(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x16 mfma32(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  // dequantized weight for bf16 compute: bf16(fl32(q s)) (_host_dequantize with T = BFloat16,
  // src/layers/quantization.jl:25-29)
  static __device__ __forceinline__ uint32_t deq(float q, float s) { return f32_to_bf16_bits(q * s); }
  // w[i] * s[i] rounded to bf16 (s: 8 bf16 patterns); the int8 dX path scales the activations
  // instead, so this exists for the generic template only
  static __device__ __forceinline__ v8 scale8(v8 w, u32x4 s) {
    const u32x4 wb = __builtin_bit_cast(u32x4, w);
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = pack2(lo(wb[i]) * lo(s[i]), hi(wb[i]) * hi(s[i]));
    return as8(o);
  }
};

template <> struct Elt<REELS_HIP_F16> {
  typedef f16x8 v8;
  static __device__ __forceinline__ float to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
  static __device__ __forceinline__ float lo(uint32_t w) { return to_f32((uint16_t)(w & 0xffffu)); }
  static __device__ __forceinline__ float hi(uint32_t w) { return to_f32((uint16_t)(w >> 16)); }
  static __device__ __forceinline__ uint32_t bits(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
  }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) { return bits(a) | (bits(b) << 16); }
  static __device__ __forceinline__ uint32_t pack2_fast(float a, float b) { return pack2(a, b); }
  static __device__ __forceinline__ v8 as8(u32x4 v) { return __builtin_bit_cast(f16x8, v); }
  // int8 -> binary16 is exact (|q| <= 127 fits the 11-bit significand)
  // exact: 1024 + (q + 128) is a binary16 value (ulp 1 on [1024, 2048)). Each code byte with its
  // sign bit flipped (q + 128) becomes the low mantissa byte under the exponent byte of 1024
  // (0x64), then one packed binary16 subtraction of 1152 per two codes leaves q
  static __device__ __forceinline__ v8 from_i8x8(uint32_t l, uint32_t h) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const uint32_t e = 0x64646464u, ul = l ^ 0x80808080u, uh = h ^ 0x80808080u;
    const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const uint32_t w[4] = {__builtin_amdgcn_perm(e, ul, 0x04010400u), __builtin_amdgcn_perm(e, ul, 0x04030402u),
                           __builtin_amdgcn_perm(e, uh, 0x04010400u), __builtin_amdgcn_perm(e, uh, 0x04030402u)};
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, w[i]) - bias);
    return __builtin_bit_cast(v8, r);
  }
  static __device__ __forceinline__ f32x4 mfma16(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x16 mfma32(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  // dequantized weight for fp16 compute: Float16(q) * Float16(s) (_dequantize_for_compute,
  // quantization.jl:61-62), one binary16 multiply (equal to rounding the exact f32 product
  // once). Written as an f32 product rounded to f16, hipcc folds it into v_fma_mixlo_f16 with a
  // +0 addend, which turns a -0 product (q < 0, f16(s) == 0) into +0.
  static __device__ __forceinline__ uint32_t deq(float q, float s) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)((_Float16)q * (_Float16)s));
  }
  // w[i] * s[i] in binary16 (one correctly rounded multiply each, v_pk_mul_f16): with w the exact
  // codes and s = f16(scales) this is Float16(q) * Float16(s) of _dequantize_for_compute
  static __device__ __forceinline__ v8 scale8(v8 w, u32x4 s) { return w * as8(s); }
};

// calls f(std::integral_constant<int, ELT>) for the run-time element code (bf16 or f16)
template <typename F>
inline void with_elt(int elt, F&& f) {
  if (elt == REELS_HIP_F16) f(std::integral_constant<int, REELS_HIP_F16>{});
  else f(std::integral_constant<int, REELS_HIP_BF16>{});
}

// ---- host-side error state -----------------------------------------------------------------
void set_error(const std::string& msg);
void clear_error();
int fail(int code, const std::string& msg);
int check_launch(const char* what);

// kernel timing instrumentation (abi.hip): no-ops unless reels_hip_trace_start was called
void trace_before(hipStream_t st, const char* name);
void trace_after(hipStream_t st);
struct TraceScope {
  hipStream_t st;
  TraceScope(hipStream_t s, const char* name) : st(s) { trace_before(s, name); }
  ~TraceScope() { trace_after(st); }
};

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace reels
