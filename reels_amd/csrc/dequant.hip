// Dequantization for compute: _dequantize_for_compute / _host_dequantize
// (src/layers/quantization.jl:25-29, 54-64), out = cast(T, q * s) per output channel.
//   f32:  fl32(q * s)             Float32.(values) .* Float32.(scales)
//   f16:  f16(q * f16(s))         Float16.(values) .* Float16.(scales) (the product of two
//                                 binary16 values is exact in f32, then one rounding)
//   bf16: bf16(fl32(q * s))       the weight the bf16 GEMMs of the LoRA linear multiply
// The bf16 and f16 forms (the weights the LoRA linear's GEMMs multiply) have streaming kernels
// (four groups of 16 codes per thread; four 64 x 64 LDS tiles per block for the transpose); every
// other case runs one element per thread.
#include <algorithm>

#include "i8gemm.h"

namespace reels {

// Both streaming kernels issue all of a thread's code loads before converting any of them: with
// one 16-byte load in flight per thread the passes were bound by memory latency (2.2-2.8 TB/s on
// 5120 x 5120); four per thread keep enough bytes in flight per CU for the HBM rate.
constexpr int kDeqGroups = 4;  // 16-code groups per thread (rows) / 64 x 64 tiles per block (transpose)

// block b covers the 1024 consecutive 16-code groups from 1024 b (row-major over [N][K / 16]);
// group j of a thread is 1024 b + 256 j + t, so each load instruction of a wave reads 1 KiB
template <int ELT>
__global__ __launch_bounds__(256) void dequant_rows_kernel(const int8_t* __restrict__ q, int64_t ldq,
                                                           const float* __restrict__ s, int64_t N,
                                                           int64_t K, uint16_t* __restrict__ wd) {
  constexpr int G = kDeqGroups;
  const uint32_t groups = (uint32_t)(K >> 4), total = (uint32_t)(N * (K >> 4));  // < 2^31
  const uint32_t base = blockIdx.x * (256u * G) + threadIdx.x;
  u32x4 v[G];
  float sc[G];
  uint32_t n[G], c[G];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const uint32_t i = base + 256u * j;
    n[j] = i / groups;
    c[j] = i - n[j] * groups;
    v[j] = u32x4{0u, 0u, 0u, 0u};
    sc[j] = 0.0f;
    if (i < total) {
      v[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(q + (int64_t)n[j] * ldq + c[j] * 16));
      sc[j] = s[n[j]];
    }
  }
#pragma unroll
  for (int j = 0; j < G; ++j) {
    if (base + 256u * j >= total) break;
    u32x4 o[2];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t x = v[j][d];
      const float q0 = (float)(int8_t)(x & 0xff), q1 = (float)(int8_t)((x >> 8) & 0xff);
      const float q2 = (float)(int8_t)((x >> 16) & 0xff), q3 = (float)((int32_t)x >> 24);
      o[d >> 1][(d & 1) * 2] = Elt<ELT>::deq(q0, sc[j]) | (Elt<ELT>::deq(q1, sc[j]) << 16);
      o[d >> 1][(d & 1) * 2 + 1] = Elt<ELT>::deq(q2, sc[j]) | (Elt<ELT>::deq(q3, sc[j]) << 16);
    }
    u32x4* dst = reinterpret_cast<u32x4*>(wd + (int64_t)n[j] * K + c[j] * 16);
    dst[0] = o[0];
    dst[1] = o[1];
  }
}

// 64 x 64 tiles through LDS, kDeqGroups consecutive tiles along k per block (their loads issued
// together): a thread reads 16 codes of one row n and writes them as bf16 into column n of the
// [k][n] tile; it then stores 16 consecutive n of one row k (two 16-byte stores). K and N are
// multiples of 64.
template <int ELT>
__global__ __launch_bounds__(256) void dequant_transpose_kernel(const int8_t* __restrict__ q,
                                                                int64_t ldq,
                                                                const float* __restrict__ s,
                                                                int64_t N, int64_t K,
                                                                uint16_t* __restrict__ wt) {
  constexpr int G = kDeqGroups;
  __shared__ uint16_t tile[64][66];  // [k][n], rows padded to 132 bytes
  const int64_t n0 = (int64_t)blockIdx.y * 64, kb = (int64_t)blockIdx.x * 64 * G;
  const int t = threadIdx.x;
  const int nl = t >> 2, kl = (t & 3) * 16;
  u32x4 v[G];
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int64_t k0 = kb + 64 * i;
    v[i] = u32x4{0u, 0u, 0u, 0u};
    if (k0 < K) v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(q + (n0 + nl) * ldq + k0 + kl));
  }
  const float sc = s[n0 + nl];
  const int kr = t >> 2, nc = (t & 3) * 16;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int64_t k0 = kb + 64 * i;
    if (k0 >= K) break;  // uniform over the block
    if (i > 0) __syncthreads();  // the previous tile's rows have been read
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      tile[kl + j][nl] = (uint16_t)Elt<ELT>::deq((float)(int8_t)((v[i][j >> 2] >> (8 * (j & 3))) & 0xff), sc);
    }
    __syncthreads();
    const uint32_t* row = reinterpret_cast<const uint32_t*>(&tile[kr][nc]);
    u32x4 o0 = {row[0], row[1], row[2], row[3]}, o1 = {row[4], row[5], row[6], row[7]};
    u32x4* dst = reinterpret_cast<u32x4*>(wt + (k0 + kr) * N + n0 + nc);
    dst[0] = o0;
    dst[1] = o1;
  }
}

template <int DT, bool TRANS>  // DT: REELS_HIP_F32 / F16 / BF16
__global__ __launch_bounds__(256) void dequant_generic_kernel(const int8_t* __restrict__ q,
                                                              int64_t ldq,
                                                              const float* __restrict__ s,
                                                              int64_t N, int64_t K, void* out) {
  const int64_t total = N * K, stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) {
    int64_t n, k;  // out index i is row-major in the output layout, so stores coalesce
    if (TRANS) { k = i / N; n = i - k * N; } else { n = i / K; k = i - n * K; }
    const float qv = (float)q[n * ldq + k];
    if (DT == REELS_HIP_F32) static_cast<float*>(out)[i] = qv * s[n];
    else if (DT == REELS_HIP_F16) static_cast<uint16_t*>(out)[i] = (uint16_t)Elt<REELS_HIP_F16>::deq(qv, s[n]);
    else static_cast<uint16_t*>(out)[i] = (uint16_t)Elt<REELS_HIP_BF16>::deq(qv, s[n]);
  }
}

int launch_dequant_rows(int elt, const int8_t* q, int64_t ldq, const float* s, int64_t N, int64_t K,
                        uint16_t* wd, hipStream_t st) {
  const int64_t n = N * (K >> 4);
  if (n >= ((int64_t)1 << 31)) {  // the streaming kernel indexes groups in 32 bits
    const unsigned grid = (unsigned)std::min<int64_t>(ceil_div(N * K, 256), 1 << 16);
    { TraceScope _ts(st, "dequant_generic_kernel");
      if (elt == REELS_HIP_F16) dequant_generic_kernel<REELS_HIP_F16, false><<<grid, 256, 0, st>>>(q, ldq, s, N, K, wd);
      else dequant_generic_kernel<REELS_HIP_BF16, false><<<grid, 256, 0, st>>>(q, ldq, s, N, K, wd); }
    return check_launch("dequant_generic_kernel");
  }
  { TraceScope _ts(st, "dequant_rows_kernel");
    with_elt(elt, [&](auto e) {
      dequant_rows_kernel<decltype(e)::value><<<(unsigned)ceil_div(n, 256 * kDeqGroups), 256, 0, st>>>(q, ldq, s, N, K, wd);
    }); }
  return check_launch("dequant_rows_kernel");
}

int launch_dequant_transpose(int elt, const int8_t* q, int64_t ldq, const float* s, int64_t N,
                             int64_t K, uint16_t* wt, hipStream_t st) {
  { TraceScope _ts(st, "dequant_transpose_kernel");
    with_elt(elt, [&](auto e) {
      dequant_transpose_kernel<decltype(e)::value><<<dim3((unsigned)ceil_div(K, 64 * kDeqGroups), (unsigned)(N / 64)), 256, 0, st>>>(q, ldq, s, N, K, wt);
    }); }
  return check_launch("dequant_transpose_kernel");
}

}  // namespace reels

using namespace reels;

extern "C" int reels_hip_i8_dequant(const int8_t* q, const float* scales, int64_t N, int64_t K,
                                    int64_t ld_q, int dtype, int transpose, void* out,
                                    void* stream) {
  clear_error();
  if (N < 0 || K < 0 || ld_q < K)
    return fail(REELS_HIP_EINVAL, "reels_hip_i8_dequant: need N >= 0, K >= 0 and ld_q >= K");
  if (dtype != REELS_HIP_F32 && dtype != REELS_HIP_BF16 && dtype != REELS_HIP_F16)
    return fail(REELS_HIP_EDTYPE, "reels_hip_i8_dequant: dtype must be REELS_HIP_F32, "
                                  "REELS_HIP_BF16 or REELS_HIP_F16");
  if (transpose != 0 && transpose != 1)
    return fail(REELS_HIP_EINVAL, "reels_hip_i8_dequant: transpose must be 0 or 1");
  if (N == 0 || K == 0) return REELS_HIP_OK;
  if (q == nullptr || scales == nullptr || out == nullptr)
    return fail(REELS_HIP_EINVAL, "reels_hip_i8_dequant: NULL q, scales or out");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool al = aligned16(q) && aligned16(out) && ld_q % 16 == 0;
  const bool half = dtype == REELS_HIP_BF16 || dtype == REELS_HIP_F16;
  if (half && !transpose && al && K % 16 == 0)
    return launch_dequant_rows(dtype, q, ld_q, scales, N, K, static_cast<uint16_t*>(out), st);
  if (half && transpose && al && N % 64 == 0 && K % 64 == 0)
    return launch_dequant_transpose(dtype, q, ld_q, scales, N, K, static_cast<uint16_t*>(out), st);
  const unsigned grid = (unsigned)std::min<int64_t>(ceil_div(N * K, 256), 1 << 16);  // grid-stride
  { TraceScope _ts(st, "dequant_generic_kernel");
    if (dtype == REELS_HIP_F32) {
      if (transpose) dequant_generic_kernel<REELS_HIP_F32, true><<<grid, 256, 0, st>>>(q, ld_q, scales, N, K, out);
      else dequant_generic_kernel<REELS_HIP_F32, false><<<grid, 256, 0, st>>>(q, ld_q, scales, N, K, out);
    } else if (dtype == REELS_HIP_F16) {
      if (transpose) dequant_generic_kernel<REELS_HIP_F16, true><<<grid, 256, 0, st>>>(q, ld_q, scales, N, K, out);
      else dequant_generic_kernel<REELS_HIP_F16, false><<<grid, 256, 0, st>>>(q, ld_q, scales, N, K, out);
    } else {
      if (transpose) dequant_generic_kernel<REELS_HIP_BF16, true><<<grid, 256, 0, st>>>(q, ld_q, scales, N, K, out);
      else dequant_generic_kernel<REELS_HIP_BF16, false><<<grid, 256, 0, st>>>(q, ld_q, scales, N, K, out);
    }
  }
  return check_launch("dequant_generic_kernel");
}
