// Shared device/host helpers for the reels_hip kernels (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

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
