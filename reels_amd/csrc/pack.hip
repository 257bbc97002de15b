// Per-output-channel symmetric int8 packing: quantize_frozen_matrix,
// src/layers/quantization.jl:35-44, bit-exact.
//
// One wavefront per output row n (64 lanes). Lane l owns the 16-byte chunks l, l+64, l+128, ...
// of the row, so every load and store instruction of a wave is one contiguous, coalesced span.
//   pass 1: absmax over the row as an unsigned maximum of magnitude bits (sign cleared): for
//           IEEE formats that order equals the order of |x|, with every NaN above Inf, so a NaN
//           anywhere in the row shows up as a maximum above the Inf pattern and propagates like
//           Julia's maximum (quantization.jl:38); bf16 / f16 rows take two elements per packed
//           16-bit max, then a wave max via xor shuffles
//   scale = absmax / 127f0 (IEEE division), 1 where absmax == 0 (quantization.jl:39-40)
//   pass 2: q = rint(clamp(w / scale, -127, 127)), ties to even (quantization.jl:41-42)
// The row stays in registers when it fits in MAXC chunks per lane; otherwise pass 2 re-reads it
// (an L2 hit: the wave read the same bytes moments before).
// Built without fast-math: the division is the correctly rounded IEEE one and f32 denormals are
// preserved, so results equal the reference's Float32 arithmetic bit for bit.
#include "common.h"

namespace reels {

template <typename T>
struct Elem;
// Per element type: unpack a 16-byte chunk to f32, fold a chunk into the running maximum of
// magnitude bits (mag), and turn that maximum into |x|max as f32 (absmax).
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a),
                                                                __builtin_bit_cast(u16x2, b)));
}
template <>
struct Elem<float> {
  static constexpr int E = 4;  // elements per 16-byte chunk
  __device__ static void unpack(const u32x4& c, float* v) {
    for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(c[i]);
  }
  __device__ static void mag(const u32x4& c, uint32_t& m) {
    for (int i = 0; i < 4; ++i) m = max(m, c[i] & 0x7fffffffu);
  }
  __device__ static float absmax(uint32_t m) { return __uint_as_float(m); }
};
template <>
struct Elem<__bf16> {
  static constexpr int E = 8;
  __device__ static void unpack(const u32x4& c, float* v) {
    for (int i = 0; i < 4; ++i) { v[2 * i] = bf16_lo(c[i]); v[2 * i + 1] = bf16_hi(c[i]); }
  }
  __device__ static void mag(const u32x4& c, uint32_t& m) {  // both halves at once
    for (int i = 0; i < 4; ++i) m = pk_max_u16(m, c[i] & 0x7fff7fffu);
  }
  __device__ static float absmax(uint32_t m) { return __uint_as_float(max(m & 0xffffu, m >> 16) << 16); }
};
template <>
struct Elem<_Float16> {
  static constexpr int E = 8;
  __device__ static void unpack(const u32x4& c, float* v) {
    for (int i = 0; i < 4; ++i) {
      _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)(c[i] & 0xffff));
      _Float16 hi = __builtin_bit_cast(_Float16, (uint16_t)(c[i] >> 16));
      v[2 * i] = (float)lo;
      v[2 * i + 1] = (float)hi;
    }
  }
  __device__ static void mag(const u32x4& c, uint32_t& m) {
    for (int i = 0; i < 4; ++i) m = pk_max_u16(m, c[i] & 0x7fff7fffu);
  }
  __device__ static float absmax(uint32_t m) {  // f16 NaN converts to an f32 NaN
    return (float)__builtin_bit_cast(_Float16, (uint16_t)max(m & 0xffffu, m >> 16));
  }
};

__device__ __forceinline__ float wave_max(float v) {
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  for (int off = 32; off >= 1; off >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, off, 64));
  return v;
}

// Quantizes E values with one scale; returns codes packed little-endian (E/4 dwords) and sets
// bad if any code is non-finite (Julia: Int8(NaN) throws InexactError).
//
// Exact shortcut for the IEEE division: when the scale s is a normal float, inv = fl(1/s) is
// computed once per row and t = fl(w * inv) differs from w/s by at most 2^-23 |w/s| <= 2^-16
// (|w/s| <= 127 * (1 + 2^-23)), while the correctly rounded quotient fl(w/s) differs from w/s by at
// most 2^-17. Whenever t lies more than 2^-12 away from every half-integer, t and fl(w/s) are
// on the same side of it, so rint(clamp(t)) == rint(clamp(fl(w/s))) — the reference's code. The
// few elements within 2^-12 of a half-integer (and rows whose scale is 0, denormal, Inf or NaN)
// take the IEEE division itself, so every code is bit-identical to quantization.jl:41-42.
__device__ __forceinline__ int quantize_one(float w, float scale, float inv, bool fast, bool& bad) {
  float t = w * inv;
  const float rt = __builtin_rintf(t);
  if (!fast || __builtin_fabsf(t - rt) > 0.5f - 0x1p-12f) t = w / scale;
  const float c = t > 127.0f ? 127.0f : (t < -127.0f ? -127.0f : t);
  const float rd = __builtin_rintf(c);
  if (__builtin_isfinite(rd)) return (int)rd;
  bad = true;
  return 0;
}

template <int E>
__device__ __forceinline__ void quantize_chunk(const float* v, float scale, float inv, bool fast,
                                               uint32_t* out, bool& bad) {
#pragma unroll
  for (int d = 0; d < E / 4; ++d) {
    uint32_t word = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int code = quantize_one(v[d * 4 + b], scale, inv, fast, bad);
      word |= ((uint32_t)(code & 0xff)) << (8 * b);
    }
    out[d] = word;
  }
}

// Fast path of quantize_chunk for a normal finite scale (every element of such a row is finite):
// t = w * inv, c = clamp(t) (v_med3), and u = c + 1.5 * 2^23 rounds c to the nearest integer,
// ties to even, leaving the two's complement code in u's low byte (c + 1.5 * 2^23 lies in
// [2^23, 2^24), where the float spacing is 1). Returns true when some |c - rint(c)| exceeds
// 0.5 - 2^-12: that chunk is redone with the IEEE division (the shortcut argument above).
// Clamping before rounding equals the reference's clamp-then-round: the bounds are integers.
template <int E>
__device__ __forceinline__ bool quantize_chunk_fast(const float* v, float inv, uint32_t* out) {
  constexpr float MAGIC = 12582912.0f;  // 1.5 * 2^23
  float emax = 0.0f;
  uint32_t ub[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float c = __builtin_amdgcn_fmed3f(v[e] * inv, -127.0f, 127.0f);
    const float u = c + MAGIC;
    emax = fmaxf(emax, __builtin_fabsf(c - (u - MAGIC)));
    ub[e] = __float_as_uint(u);
  }
#pragma unroll
  for (int d = 0; d < E / 4; ++d) {
    const uint32_t lo = __builtin_amdgcn_perm(ub[4 * d + 1], ub[4 * d + 0], 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(ub[4 * d + 3], ub[4 * d + 2], 0x0c0c0400u);
    out[d] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
  }
  return emax > 0.5f - 0x1p-12f;
}

// scale is a finite normal float: the multiply shortcut applies (see quantize_one)
__device__ __forceinline__ bool fast_scale(float scale) {
  return scale >= 0x1p-126f && scale <= 3.4028234663852886e38f;
}

template <typename T, int MAXC>
__global__ __launch_bounds__(256) void pack_rows_kernel(const T* __restrict__ w, int64_t N, int64_t K,
                                                        int64_t ld, int8_t* __restrict__ q,
                                                        float* __restrict__ scales, int32_t* status) {
  constexpr int E = Elem<T>::E;
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int64_t chunks = K / E;
  const u32x4* row = reinterpret_cast<const u32x4*>(w + n * ld);

  u32x4 cache[MAXC > 0 ? MAXC : 1];
  uint32_t mb = 0;
  if (MAXC > 0) {
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      int64_t c = lane + 64 * (int64_t)i;
      if (c < chunks) cache[i] = __builtin_nontemporal_load(row + c);
    }
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      int64_t c = lane + 64 * (int64_t)i;
      if (c < chunks) Elem<T>::mag(cache[i], mb);
    }
    // every cached load has been used: saying so outside the branches keeps the compiler from
    // waiting before each store below (its wait would include the earlier stores)
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  } else {
    for (int64_t c = lane; c < chunks; c += 64) Elem<T>::mag(row[c], mb);
  }
  // this lane's |x|max as f32 bits (non-negative floats order as unsigned integers, NaN above Inf)
  const uint32_t wm = wave_max_u32(__float_as_uint(Elem<T>::absmax(mb)));
  const float m = wm > 0x7f800000u ? __builtin_nanf("") : __uint_as_float(wm);
  float scale = m / 127.0f;
  if (m == 0.0f) scale = 1.0f;
  if (lane == 0) scales[n] = scale;
  const bool fast = fast_scale(scale);
  const float inv = fast ? 1.0f / scale : 0.0f;

  bool bad = false;
  int8_t* qrow = q + n * K;
  if (MAXC > 0) {
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      int64_t c = lane + 64 * (int64_t)i;
      if (c < chunks) {
        float v[E];
        Elem<T>::unpack(cache[i], v);
        uint32_t out[E / 4];
        if (!fast || quantize_chunk_fast<E>(v, inv, out))
          quantize_chunk<E>(v, scale, inv, false, out, bad);
        if (E == 8) {
          u32x2 o = {out[0], out[1 % (E / 4)]};
          __builtin_nontemporal_store(o, reinterpret_cast<u32x2*>(qrow + c * E));
        } else {
          __builtin_nontemporal_store(out[0], reinterpret_cast<uint32_t*>(qrow + c * E));
        }
      }
    }
  } else {
    for (int64_t c = lane; c < chunks; c += 64) {
      float v[E];
      Elem<T>::unpack(row[c], v);
      uint32_t out[E / 4];
      if (!fast || quantize_chunk_fast<E>(v, inv, out))
        quantize_chunk<E>(v, scale, inv, false, out, bad);
      if (E == 8) {
        u32x2 o = {out[0], out[1 % (E / 4)]};
        __builtin_nontemporal_store(o, reinterpret_cast<u32x2*>(qrow + c * E));
      } else {
        __builtin_nontemporal_store(out[0], reinterpret_cast<uint32_t*>(qrow + c * E));
      }
    }
  }
  if (status != nullptr && __any(bad) && lane == 0) *status = 1;
}

// Any shape / alignment: one wave per row, scalar element loads.
template <typename T>
__global__ __launch_bounds__(256) void pack_rows_scalar_kernel(const T* __restrict__ w, int64_t N,
                                                               int64_t K, int64_t ld,
                                                               int8_t* __restrict__ q,
                                                               float* __restrict__ scales,
                                                               int32_t* status) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const T* row = w + n * ld;
  float m = 0.0f;
  bool nan_seen = false;
  for (int64_t k = lane; k < K; k += 64) {
    float a = fabsf((float)row[k]);
    nan_seen |= (a != a);
    m = fmaxf(m, a);
  }
  m = wave_max(m);
  if (__any(nan_seen)) m = __builtin_nanf("");
  float scale = m / 127.0f;
  if (m == 0.0f) scale = 1.0f;
  if (lane == 0) scales[n] = scale;
  bool bad = false;
  for (int64_t k = lane; k < K; k += 64) {
    float t = (float)row[k] / scale;
    float c = t > 127.0f ? 127.0f : (t < -127.0f ? -127.0f : t);
    float rd = __builtin_rintf(c);
    int code = 0;
    if (__builtin_isfinite(rd)) code = (int)rd; else bad = true;
    q[n * K + k] = (int8_t)code;
  }
  if (status != nullptr && __any(bad) && lane == 0) *status = 1;
}

__global__ void clear_i32_kernel(int32_t* p) { *p = 0; }

template <typename T>
static int launch_pack(const T* w, int64_t N, int64_t K, int64_t ld, int8_t* q, float* s,
                       int32_t* status, hipStream_t st) {
  constexpr int E = Elem<T>::E;
  const dim3 grid((unsigned)ceil_div(N, 4)), block(256);
  const bool vec = aligned16(w) && (K % E == 0) && (ld % E == 0) && (K % 16 == 0) && aligned16(q);
  if (!vec) {
    { TraceScope _ts(st, "pack_rows_scalar_kernel<T>"); pack_rows_scalar_kernel<T><<<grid, block, 0, st>>>(w, N, K, ld, q, s, status); }
    return check_launch("pack_rows_scalar_kernel");
  }
  const int64_t chunks_per_lane = ceil_div(K / E, 64);
  if (chunks_per_lane <= 4)
    { TraceScope _ts(st, "pack_rows_kernel<T,4>"); pack_rows_kernel<T, 4><<<grid, block, 0, st>>>(w, N, K, ld, q, s, status); }
  else if (chunks_per_lane <= 12)
    { TraceScope _ts(st, "pack_rows_kernel<T,12>"); pack_rows_kernel<T, 12><<<grid, block, 0, st>>>(w, N, K, ld, q, s, status); }
  else if (chunks_per_lane <= 28)
    { TraceScope _ts(st, "pack_rows_kernel<T,28>"); pack_rows_kernel<T, 28><<<grid, block, 0, st>>>(w, N, K, ld, q, s, status); }
  else
    { TraceScope _ts(st, "pack_rows_kernel<T,0>"); pack_rows_kernel<T, 0><<<grid, block, 0, st>>>(w, N, K, ld, q, s, status); }
  return check_launch("pack_rows_kernel");
}

}  // namespace reels

using namespace reels;

extern "C" int reels_hip_i8_pack(const void* w, int dtype, int64_t N, int64_t K, int64_t ld_w,
                                 int8_t* q, float* scales, int32_t* status, void* stream) {
  clear_error();
  if (N < 0 || K <= 0 || ld_w < K)
    return fail(REELS_HIP_EINVAL, "reels_hip_i8_pack: need N >= 0, K > 0 and ld_w >= K (Julia's "
                                  "maximum over an empty row throws)");
  if (dtype != REELS_HIP_F32 && dtype != REELS_HIP_BF16 && dtype != REELS_HIP_F16)
    return fail(REELS_HIP_EDTYPE, "reels_hip_i8_pack: dtype must be REELS_HIP_F32, "
                                  "REELS_HIP_BF16 or REELS_HIP_F16");
  if (N > 0 && (w == nullptr || q == nullptr || scales == nullptr))
    return fail(REELS_HIP_EINVAL, "reels_hip_i8_pack: NULL w, q or scales");
  if (N > ((int64_t)1 << 33))
    return fail(REELS_HIP_EINVAL, "reels_hip_i8_pack: N too large for one launch");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (status != nullptr) {
    { TraceScope _ts(st, "clear_i32_kernel"); clear_i32_kernel<<<1, 1, 0, st>>>(status); }
    int rc = check_launch("clear_i32_kernel");
    if (rc) return rc;
  }
  if (N == 0) return REELS_HIP_OK;
  if (dtype == REELS_HIP_F32)
    return launch_pack<float>(static_cast<const float*>(w), N, K, ld_w, q, scales, status, st);
  if (dtype == REELS_HIP_BF16)
    return launch_pack<__bf16>(static_cast<const __bf16*>(w), N, K, ld_w, q, scales, status, st);
  return launch_pack<_Float16>(static_cast<const _Float16*>(w), N, K, ld_w, q, scales, status, st);
}
