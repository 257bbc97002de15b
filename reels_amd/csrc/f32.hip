// fp32 compute with int8 frozen weights: the reference's Float32 path (_dequantize_for_compute
// with T = Float32, src/layers/quantization.jl:61-64: W = Float32.(values) .* scales; lora_forward
// and lora_backward in Float32, src/layers/lora.jl:56-118). Every operand, intermediate and
// result is fp32; the dequantized weight fl32(q s) is materialised once per call, as the
// reference does, and multiplied on fp32 MFMA (v_mfma_f32_16x16x4_f32).
//
// Fast path: K % 4 == 0, N % 4 == 0, 16-byte aligned pointers, r <= 128. Other shapes take the
// one-output-per-thread kernels at the end of this file.
#include <mutex>
#include <type_traits>

#include "common.h"
#include "i8gemm.h"

namespace reels {

// ---------------------------------------------------------------------------------------------
// dequantization to fp32: wd[n][k] = fl32(q[n][k] s[n]), or transposed wt[k][n]
__global__ __launch_bounds__(256) void deq_f32_rows_kernel(const int8_t* __restrict__ q,
                                                           const float* __restrict__ s, int64_t N,
                                                           int64_t K, float* __restrict__ wd) {
  const int64_t total4 = N * K / 4, stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total4; i += stride) {
    const int64_t e = i * 4, n = e / K;  // K % 4 == 0: the 4 elements share a row
    const uint32_t w = *reinterpret_cast<const uint32_t*>(q + e);
    const float sc = s[n];
    f32x4 o;
#pragma unroll
    for (int b = 0; b < 4; ++b) o[b] = (float)(int8_t)((w >> (8 * b)) & 0xffu) * sc;
    *reinterpret_cast<f32x4*>(wd + e) = o;
  }
}

// 64 x 64 tiles through LDS: rows of q read along k, rows of wt written along n
__global__ __launch_bounds__(256) void deq_f32_transpose_kernel(const int8_t* __restrict__ q,
                                                                const float* __restrict__ s,
                                                                int64_t N, int64_t K,
                                                                float* __restrict__ wt) {
  __shared__ float tile[64][65];
  const int t = threadIdx.x;
  const int64_t n0 = (int64_t)blockIdx.y * 64, k0 = (int64_t)blockIdx.x * 64;
  for (int i = t; i < 64 * 64; i += 256) {
    const int rn = i >> 6, ck = i & 63;
    const int64_t n = n0 + rn, k = k0 + ck;
    tile[rn][ck] = (n < N && k < K) ? (float)q[n * K + k] * s[n] : 0.0f;
  }
  __syncthreads();
  for (int i = t; i < 64 * 64; i += 256) {
    const int rk = i >> 6, cn = i & 63;
    const int64_t k = k0 + rk, n = n0 + cn;
    if (k < K && n < N) wt[k * N + n] = tile[cn][rk];
  }
}

// out[c][r] = in[r][c] (in [rows][cols] fp32)
__global__ __launch_bounds__(256) void transpose_f32_kernel(const float* __restrict__ in,
                                                            int64_t rows, int64_t cols,
                                                            float* __restrict__ out) {
  __shared__ float tile[32][33];
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
  for (int i = ty; i < 32; i += 8)
    tile[i][tx] = (r0 + i < rows && c0 + tx < cols) ? in[(r0 + i) * cols + c0 + tx] : 0.0f;
  __syncthreads();
  for (int i = ty; i < 32; i += 8)
    if (c0 + i < cols && r0 + tx < rows) out[(c0 + i) * rows + r0 + tx] = tile[tx][i];
}

// ---------------------------------------------------------------------------------------------
// GEMM: out[m][n] = (sum_k act[m][k] wd[n][k] + bias[n]) + c sum_j L[m][j] R[n][j]
// (the reference's order: _weight_mul, mixed_add of the bias, then the scaled adapter).
struct F32GemmArgs {
  const float* act;   // [M][Kred]
  const float* wd;    // [Ncols][Kred]
  const float* L;     // [M][r] or nullptr
  const float* R;     // [Ncols][r]
  const float* bias;  // [Ncols] or nullptr
  float* out;         // [M][Ncols]
  int64_t M, Ncols, Kred;
  int r;
  float c;
};

namespace f32g {
constexpr int BM = 128, BN = 128, BK = 16, NT = 256;
constexpr int TILE = 128 * BK * 4;  // 8 KiB: 128 rows of 16 floats
constexpr int STAGE = 2 * TILE;     // activation tile + weight tile
constexpr int NS = 5;               // ring depth: copies run 3 steps ahead of the MFMAs
constexpr int LDS = NS * STAGE;     // 80 KiB: two workgroups per CU
constexpr int GM = 4;
}  // namespace f32g

// 128 x 128 output tile, reduction step 16, 4 waves of 64 tokens x 64 columns (4 x 4 tiles of
// v_mfma_f32_16x16x4_f32). Tiles [128][16] fp32 arrive through LDS-DMA copies into a five-stage
// ring, issued three steps before their fragments are read; a wave waits only for the copies of
// the step it is about to read (vmcnt counts its later copies still in flight). Rows are 64 bytes; the 16-byte chunk c of
// row i sits in slot c ^ ((i >> 1) & 3), so the 8 rows read together by a fragment load (4 row
// pairs sharing a 128-byte line) hit distinct banks. A lane reads 4 consecutive k of its row with
// one ds_read_b128 and feeds them to 4 MFMAs, element j to the j-th: every lane of a 16-lane
// group supplies the same k, so A and B agree on the k order and the sum is the full reduction.
// D register v of lane l is output column 4 (l / 16) + v, token l % 16 of the 16 x 16 tile.
__global__ __launch_bounds__(256, 2) void f32gemm_kernel(F32GemmArgs a, int tiles_n, int tiles_m) {
  using namespace f32g;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = w >> 1, wn = w & 1;
  const int l16 = lane & 15, lq = lane >> 4;
  const int64_t M = a.M, Ncols = a.Ncols, Kred = a.Kred;

  // tile order as in the bf16 GEMM: an XCD's resident tiles form groups of GM token blocks
  const int nt = tiles_n * tiles_m;
  const int b = blockIdx.x;
  const int xcd = b & 7, idx = b >> 3;
  const int lo = nt >> 3, rem = nt & 7;
  const int logical = xcd * lo + (xcd < rem ? xcd : rem) + idx;
  const int group = GM * tiles_n;
  const int g = logical / group;
  const int first_m = g * GM;
  const int gm = (tiles_m - first_m) < GM ? (tiles_m - first_m) : GM;
  const int within = logical - g * group;
  const int64_t m0 = (int64_t)(first_m + within % gm) * BM;
  const int64_t n0 = (int64_t)(within / gm) * BN;

  // copies: copy i (0..1) of wave w fills rows (2w + i) * 16 + lane / 4, slot lane % 4 (chunk
  // (lane % 4) ^ ((row >> 1) & 3)), 1 KiB of LDS. Rows past M / Ncols and chunks past Kred read
  // beyond the buffer: zeros.
  const i32x4 ract = buffer_rsrc(a.act, (uint32_t)(M * Kred * 4));
  const i32x4 rw = buffer_rsrc(a.wd, (uint32_t)(Ncols * Kred * 4));
  uint32_t voa[2], vow[2];
  int kc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = (w * 2 + i) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ ((row >> 1) & 3);
    kc[i] = c * 4;
    voa[i] = (uint32_t)(((m0 + row) * Kred + c * 4) * 4);
    vow[i] = (uint32_t)(((n0 + row) * Kred + c * 4) * 4);
  }
  const int nk = (int)((Kred + BK - 1) / BK);
  auto issue = [&](int kt) {
    uint8_t* base = smem + (kt % NS) * STAGE;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const bool in = (int64_t)kt * BK + kc[i] < Kred;
      const uint32_t adv = (uint32_t)kt * (BK * 4);
      dma16(ract, in ? voa[i] + adv : 0xFFFFFFF0u, 0u, base + (w * 2 + i) * 1024);
      dma16(rw, in ? vow[i] + adv : 0xFFFFFFF0u, 0u, base + TILE + (w * 2 + i) * 1024);
    }
  };

  f32x4 acc[4][4];  // [output-column tile][token tile]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int off = (lq ^ ((l16 >> 1) & 3)) << 4;  // fragment rows start at multiples of 16
  const uint32_t frag = (uint32_t)(uintptr_t)LDS_PTR(const uint8_t, smem) + off;
  const uint32_t fx = frag + (wm * 64 + l16) * 64, fw = frag + TILE + (wn * 64 + l16) * 64;
  // The fragment reads are inline assembly, invisible to the compiler's wait insertion: the
  // reads of the next step then overlap this step's MFMAs, and the waits are placed by hand.
  // A wait names the fragments it releases as operands, so no MFMA moves above it.
  auto rd = [&](int kt, f32x4(&xf)[4], f32x4(&wf)[4]) {
    const uint32_t sb = (uint32_t)((kt % NS) * STAGE);
    asm volatile(
        "ds_read_b128 %0, %8\n\t"
        "ds_read_b128 %1, %8 offset:1024\n\t"
        "ds_read_b128 %2, %8 offset:2048\n\t"
        "ds_read_b128 %3, %8 offset:3072\n\t"
        "ds_read_b128 %4, %9\n\t"
        "ds_read_b128 %5, %9 offset:1024\n\t"
        "ds_read_b128 %6, %9 offset:2048\n\t"
        "ds_read_b128 %7, %9 offset:3072"
        : "=&v"(xf[0]), "=&v"(xf[1]), "=&v"(xf[2]), "=&v"(xf[3]), "=&v"(wf[0]), "=&v"(wf[1]),
          "=&v"(wf[2]), "=&v"(wf[3])  // early clobber: the data returns while addresses are in use
        : "v"(fx + sb), "v"(fw + sb)
        : "memory");
  };
  // lgkmcnt(n): at most n of this wave's LDS reads still in flight
  auto release = [&](f32x4(&xf)[4], f32x4(&wf)[4], auto n) {
    asm volatile("s_waitcnt lgkmcnt(%8)"
                 : "+v"(xf[0]), "+v"(xf[1]), "+v"(xf[2]), "+v"(xf[3]), "+v"(wf[0]), "+v"(wf[1]),
                   "+v"(wf[2]), "+v"(wf[3])
                 : "n"(decltype(n)::value));
  };
  auto mm = [&](const f32x4(&xf)[4], const f32x4(&wf)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int ti = 0; ti < 4; ++ti)
#pragma unroll
        for (int tj = 0; tj < 4; ++tj)
          acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x4f32(wf[ti][j], xf[tj][j], acc[ti][tj], 0, 0, 0);
  };
  // wait until this wave's copies of step s have landed, given that the copies of every step up
  // to min(last, nk - 1) were issued after them (4 per step)
  auto wait_step = [&](int s, int last) {
    const int later = (last < nk - 1 ? last : nk - 1) - s;
    if (later >= 3) __builtin_amdgcn_s_waitcnt(0x0F7C);       // vmcnt(12)
    else if (later == 2) __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8)
    else if (later == 1) __builtin_amdgcn_s_waitcnt(0x0F74);  // vmcnt(4)
    else __builtin_amdgcn_s_waitcnt(0x0F70);                  // vmcnt(0)
  };
  using zero = std::integral_constant<int, 0>;
  using eight = std::integral_constant<int, 8>;
  // Fragments are read one step ahead into the second register set. At the barrier of step kt
  // every wave's copies of step kt + 1 have landed and every wave has consumed its fragments of
  // step kt - 1, whose stage the copies of step kt + 4 then refill. Scheduling fences keep every
  // LDS access on its side of the barriers.
  f32x4 xa[4], wa[4], xb[4], wb[4];
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nk) issue(s);
  wait_step(0, NS - 2);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  rd(0, xa, wa);
  release(xa, wa, zero());  // lgkmcnt holds 15: never more than 8 reads in flight
  __builtin_amdgcn_sched_barrier(0);
  auto step = [&](int kt, f32x4(&xc)[4], f32x4(&wc)[4], f32x4(&xn)[4], f32x4(&wn_)[4]) {
    if (kt + 1 < nk) {
      wait_step(kt + 1, kt + NS - 2);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      if (kt + NS - 1 < nk) issue(kt + NS - 1);
      rd(kt + 1, xn, wn_);
      release(xc, wc, eight());  // the 8 reads just issued may still be in flight
    } else {
      release(xc, wc, zero());
    }
    __builtin_amdgcn_sched_barrier(0);
    mm(xc, wc);
    __builtin_amdgcn_sched_barrier(0);
  };
  // steady state, no branches: the copies of steps kt + 2 and kt + 3 stay in flight
  int kt = 0;
  for (; kt + NS < nk; kt += 2) {
    __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue(kt + NS - 1);
    rd(kt + 1, xb, wb);
    release(xa, wa, eight());
    __builtin_amdgcn_sched_barrier(0);
    mm(xa, wa);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0x0F78);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue(kt + NS);
    rd(kt + 2, xa, wa);
    release(xb, wb, eight());
    __builtin_amdgcn_sched_barrier(0);
    mm(xb, wb);
    __builtin_amdgcn_sched_barrier(0);
  }
  // the last steps: fewer copies in flight, nothing to read after the final one
  for (; kt + 1 < nk; kt += 2) {
    step(kt, xa, wa, xb, wb);
    step(kt + 1, xb, wb, xa, wa);
  }
  if (kt < nk) step(kt, xa, wa, xb, wb);

  // epilogue: the rank-r term on MFMA from global L and R (k in steps of 16: lane supplies 4
  // consecutive j, zeros past r), bias, fp32 stores of 4 consecutive columns per lane. With
  // r % 4 == 0 (rows 16-byte aligned) the 4 j of a lane come in one load.
  const int r = a.r;
  // the bias of this lane's 4 x 4 output columns, loaded before any store: a load between the
  // stores would make each store wait for the previous ones (vmcnt counts both)
  f32x4 bs[4];
#pragma unroll
  for (int ti = 0; ti < 4; ++ti) {
    const int64_t nb = n0 + wn * 64 + ti * 16 + lq * 4;
    bs[ti] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (a.bias != nullptr && nb < Ncols) bs[ti] = *reinterpret_cast<const f32x4*>(a.bias + nb);
  }
  f32x4 lor[4][4];
#pragma unroll
  for (int ti = 0; ti < 4; ++ti)
#pragma unroll
    for (int tj = 0; tj < 4; ++tj) lor[ti][tj] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if (a.L != nullptr) {
    const bool vec = (r & 3) == 0;
    for (int j0 = 0; j0 < r; j0 += 16) {
      const int jl = j0 + lq * 4;
      f32x4 lv[4], rv[4];
#pragma unroll
      for (int tj = 0; tj < 4; ++tj) {
        const int64_t m = m0 + wm * 64 + tj * 16 + l16;
        lv[tj] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (m < M && jl < r) {
          if (vec) {
            lv[tj] = *reinterpret_cast<const f32x4*>(a.L + m * r + jl);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (jl + e < r) lv[tj][e] = a.L[m * r + jl + e];
          }
        }
      }
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) {
        const int64_t nrow = n0 + wn * 64 + ti * 16 + l16;  // this lane's R row
        rv[ti] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (nrow < Ncols && jl < r) {
          if (vec) {
            rv[ti] = *reinterpret_cast<const f32x4*>(a.R + nrow * r + jl);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (jl + e < r) rv[ti][e] = a.R[nrow * r + jl + e];
          }
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int ti = 0; ti < 4; ++ti)
#pragma unroll
          for (int tj = 0; tj < 4; ++tj)
            lor[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x4f32(rv[ti][e], lv[tj][e], lor[ti][tj], 0, 0, 0);
    }
  }
  // one wait for every load, outside any branch: the compiler then knows the bias has arrived
  // on every path and puts no wait (which would include the stores) between the stores
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
#pragma unroll
  for (int ti = 0; ti < 4; ++ti) {
    const int64_t nb = n0 + wn * 64 + ti * 16 + lq * 4;  // this lane's 4 output columns
#pragma unroll
    for (int tj = 0; tj < 4; ++tj) {
      const int64_t m = m0 + wm * 64 + tj * 16 + l16;
      if (m < M && nb < Ncols) {
        f32x4 o;
#pragma unroll
        for (int v = 0; v < 4; ++v) o[v] = (acc[ti][tj][v] + bs[ti][v]) + a.c * lor[ti][tj][v];
        *reinterpret_cast<f32x4*>(a.out + m * Ncols + nb) = o;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// rank-r projection: out[m][j] = sum_k src[m][k] P[j][k] (P [r][Kd] fp32, rows contiguous).
// 4 waves x 16 tokens per workgroup; MFMA A = P rows (j), B = token rows, so a lane holds 4
// consecutive j of one token. Operands straight from global memory, 4 k-chunks of 16 in flight.
__global__ __launch_bounds__(256) void rowproj_f32_kernel(const float* __restrict__ src, int64_t M,
                                                          int64_t Kd, const float* __restrict__ P,
                                                          int r, float* __restrict__ out) {
  constexpr int JT = 8;  // up to 128 ranks
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int l16 = lane & 15, lq = lane >> 4;
  const int64_t m = (int64_t)blockIdx.x * 64 + w * 16 + l16;
  const int jt_n = (r + 15) >> 4;
  f32x4 acc[JT];
#pragma unroll
  for (int i = 0; i < JT; ++i) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int U = 8;  // 8 k-chunks (8 KiB per wave) in flight
  for (int64_t k0 = 0; k0 < Kd; k0 += 16 * U) {
    f32x4 xv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t k = k0 + u * 16 + lq * 4;
      xv[u] = (m < M && k < Kd) ? *reinterpret_cast<const f32x4*>(src + m * Kd + k) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int jt = 0; jt < JT; ++jt) {
      if (jt >= jt_n) break;
      const int j = jt * 16 + l16;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t k = k0 + u * 16 + lq * 4;
        const f32x4 pv = (j < r && k < Kd) ? *reinterpret_cast<const f32x4*>(P + (int64_t)j * Kd + k) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(pv[e], xv[u][e], acc[jt], 0, 0, 0);
      }
    }
  }
  // D: lane holds j = jt*16 + 4 (l/16) + v for token l % 16 of the wave's 16
  const int64_t mo = (int64_t)blockIdx.x * 64 + w * 16 + l16;
  if (mo >= M) return;
#pragma unroll
  for (int jt = 0; jt < JT; ++jt) {
    if (jt >= jt_n) break;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int j = jt * 16 + lq * 4 + v;
      if (j < r) out[mo * r + j] = acc[jt][v];
    }
  }
}

// ---------------------------------------------------------------------------------------------
// split-M column gradients: part[sp][o][j] = sum over the split's tokens of src[m][o] Lm[m][j]
// (src [M][Od], Lm [M][r]). A workgroup takes 64 columns o (16 per wave) of one split; token
// tiles of 64 pass through LDS; MFMA A = Lm^T rows (j), B = src^T rows (o), k = tokens, with
// single-element LDS reads (the k of lane l is token 4 step + l / 16 for both operands).
namespace f32c {
constexpr int TM = 64, BO = 64;
}
__global__ __launch_bounds__(256) void colgrad_f32_kernel(const float* __restrict__ src, int64_t M,
                                                          int64_t Od, const float* __restrict__ Lm,
                                                          int r, int64_t tokens_per_split,
                                                          float* __restrict__ part) {
  using namespace f32c;
  constexpr int JT = 8;
  __shared__ float ss[TM][BO + 1];
  __shared__ __attribute__((aligned(16))) float sl[TM * 128];  // [tok][j], row stride r
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int l16 = lane & 15, lq = lane >> 4;
  const int64_t o0 = (int64_t)blockIdx.x * BO;
  const int sp = blockIdx.y;
  const int64_t mbeg = (int64_t)sp * tokens_per_split;
  const int64_t mend = (mbeg + tokens_per_split < M) ? mbeg + tokens_per_split : M;
  const int jt_n = (r + 15) >> 4;
  f32x4 acc[JT];
#pragma unroll
  for (int i = 0; i < JT; ++i) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // the next token tile is loaded into registers while the current one is multiplied: the src
  // tile [64 tokens][64 o] as 4 f32x4 per thread, the Lm tile [64 tokens][r] (64 r contiguous
  // floats of Lm) as up to 8 f32x4 per thread
  f32x4 rs[4], rl[8];
  const int nl4 = TM * r / 4;
  auto load = [&](int64_t mb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int id = t + 256 * i, row = id >> 4, c4 = (id & 15) * 4;
      const int64_t mm = mb + row, o = o0 + c4;
      rs[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (mm < mend && o < Od) rs[i] = *reinterpret_cast<const f32x4*>(src + mm * Od + o);
    }
    const int64_t lim = (mend - mb) * r;  // floats of the tile that belong to this split
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int id = t + 256 * i;
      rl[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      const int64_t e0 = (int64_t)id * 4;  // whole vectors inside the split; the one across its
      if (id < nl4 && e0 + 3 < lim) {      // end (r odd) element by element: no read past M r
        rl[i] = *reinterpret_cast<const f32x4*>(Lm + mb * r + e0);
      } else if (id < nl4 && e0 < lim) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (e0 + e < lim) rl[i][e] = Lm[mb * r + e0 + e];
      }
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int id = t + 256 * i, row = id >> 4, c4 = (id & 15) * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) ss[row][c4 + e] = rs[i][e];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int id = t + 256 * i;
      if (id < nl4) *reinterpret_cast<f32x4*>(&sl[id * 4]) = rl[i];
    }
  };
  if (mbeg < mend) load(mbeg);
  for (int64_t mb = mbeg; mb < mend; mb += TM) {
    stash();
    __syncthreads();
    if (mb + TM < mend) load(mb + TM);
#pragma unroll 4
    for (int ks = 0; ks < TM / 4; ++ks) {
      const int tok = ks * 4 + lq;
      const float bv = ss[tok][w * 16 + l16];
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) {
        if (jt >= jt_n) break;
        const int j = jt * 16 + l16;
        const float av = j < r ? sl[tok * r + j] : 0.0f;
        acc[jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[jt], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  // D: lane holds j = jt*16 + 4 (l/16) + v for column o = o0 + 16 w + l % 16
  const int64_t o = o0 + w * 16 + l16;
  if (o >= Od) return;
#pragma unroll
  for (int jt = 0; jt < JT; ++jt) {
    if (jt >= jt_n) break;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int j = jt * 16 + lq * 4 + v;
      if (j < r) part[((int64_t)sp * Od + o) * r + j] = acc[jt][v];
    }
  }
}

// ---------------------------------------------------------------------------------------------
// generic kernels (any shape / alignment): one output per thread, f32 sums in k order
__global__ void gf_rowproj_kernel(const float* __restrict__ src, int64_t M, int64_t Kd,
                                  const float* __restrict__ P, int64_t ps_k, int64_t ps_j, int r,
                                  float* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * r) return;
  const int64_t m = idx / r, j = idx % r;
  float acc = 0.0f;
  for (int64_t k = 0; k < Kd; ++k) acc += src[m * Kd + k] * P[k * ps_k + j * ps_j];
  out[idx] = acc;
}

// y = (sum_k x w + bias) + c sum_j h B, w = fl32(q s)
__global__ void gf_fwd_kernel(const float* __restrict__ x, const int8_t* __restrict__ q,
                              const float* __restrict__ s, const float* __restrict__ h,
                              const float* __restrict__ B, const float* __restrict__ bias,
                              int64_t M, int64_t K, int64_t N, int r, float c,
                              float* __restrict__ y) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * N) return;
  const int64_t m = idx / N, n = idx % N;
  float acc = 0.0f;
  for (int64_t k = 0; k < K; ++k) acc += x[m * K + k] * ((float)q[n * K + k] * s[n]);
  float lo = 0.0f;
  for (int j = 0; j < r; ++j) lo += h[m * r + j] * B[(int64_t)j * N + n];
  y[idx] = (acc + (bias ? bias[n] : 0.0f)) + c * lo;
}

// dx = sum_n dy w + c sum_j u A, w = fl32(q s)
__global__ void gf_dx_kernel(const float* __restrict__ dy, const int8_t* __restrict__ q,
                             const float* __restrict__ s, const float* __restrict__ u,
                             const float* __restrict__ A, int64_t M, int64_t K, int64_t N, int r,
                             float c, float* __restrict__ dx) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * K) return;
  const int64_t m = idx / K, k = idx % K;
  float acc = 0.0f;
  for (int64_t n = 0; n < N; ++n) acc += dy[m * N + n] * ((float)q[n * K + k] * s[n]);
  float lo = 0.0f;
  for (int j = 0; j < r; ++j) lo += u[m * r + j] * A[k * r + j];
  dx[idx] = acc + c * lo;
}

// out[o][j] (or [j][o] when TRANS) = c * sum_m src[m][o] Lm[m][j]
template <bool TRANS>
__global__ void gf_colgrad_kernel(const float* __restrict__ src, int64_t M, int64_t Od,
                                  const float* __restrict__ Lm, int r, float c,
                                  float* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= Od * r) return;
  int64_t o, j;
  if (TRANS) { j = idx / Od; o = idx % Od; } else { o = idx / r; j = idx % r; }
  float acc = 0.0f;
  for (int64_t m = 0; m < M; ++m) acc += src[m * Od + o] * Lm[m * r + j];
  out[idx] = c * acc;
}

__global__ void zero_f32_kernel(float* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

__global__ void gelu_f32_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = gelu_f(x[i]);
}
__global__ void gelu_bwd_f32_kernel(const float* __restrict__ x, const float* __restrict__ dy,
                                    float* __restrict__ dx, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dx[i] = dy[i] * gelu_grad_f(x[i]);
}

// ---------------------------------------------------------------------------------------------
// host side
static unsigned g1(int64_t n) { return (unsigned)ceil_div(n, 256); }

struct PlanF32 {
  bool fast;
  int splits;
  int64_t tps;
};

static PlanF32 plan_f32(int64_t M, int64_t K, int64_t N, int64_t r, bool aligned) {
  PlanF32 p;
  p.fast = aligned && K % 4 == 0 && N % 4 == 0 && r <= 128 && M * K * 4 < ((int64_t)1 << 31) &&
           M * N * 4 < ((int64_t)1 << 31) && N * K * 4 < ((int64_t)1 << 31);
  int64_t s = (M + 1023) / 1024;
  if (s < 1) s = 1;
  if (s > 32) s = 32;
  p.tps = ((M + s - 1) / s + 63) / 64 * 64;
  if (p.tps < 64) p.tps = 64;
  p.splits = (int)((M + p.tps - 1) / p.tps);
  if (p.splits < 1) p.splits = 1;
  return p;
}

struct WsF32 {
  size_t at, bt, h, wd, u, pa, pb, pbias, total;
};

static WsF32 ws_f32(int64_t M, int64_t K, int64_t N, int64_t r, int which, const PlanF32& p) {
  WsF32 w{};
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off = align_up(off + bytes, 256); return o; };
  w.at = take((size_t)r * K * 4);
  w.h = take((size_t)M * r * 4);
  w.wd = take(p.fast ? (size_t)N * K * 4 : 0);
  if (which == REELS_HIP_WS_FWD) {
    w.bt = take((size_t)N * r * 4);
  } else {
    w.u = take((size_t)M * r * 4);
    w.pa = take(p.fast && r > 0 ? (size_t)p.splits * K * r * 4 : 0);
    w.pb = take(p.fast && r > 0 ? (size_t)p.splits * N * r * 4 : 0);
    w.pbias = take(colsum_partial_bytes(M, N));  // the bias gradient's split partials
  }
  w.total = off == 0 ? 256 : off;
  return w;
}

// mode 0 = forward, 1 = dX (names the launch in the kernel trace)
static int launch_f32gemm(int mode, const F32GemmArgs& a, hipStream_t st) {
  using namespace f32g;
  static std::once_flag once;
  static hipError_t attr_err = hipSuccess;
  std::call_once(once, [&] {
    attr_err = hipFuncSetAttribute((const void*)f32gemm_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, LDS);
  });
  if (attr_err != hipSuccess)
    return fail(REELS_HIP_EHIP, std::string("f32gemm: hipFuncSetAttribute: ") + hipGetErrorString(attr_err));
  if (a.M == 0 || a.Ncols == 0) return REELS_HIP_OK;
  const int tn = (int)ceil_div(a.Ncols, BN), tm = (int)ceil_div(a.M, BM);
  { TraceScope _ts(st, mode == 0 ? "f32gemm_kernel<0>" : "f32gemm_kernel<1>"); f32gemm_kernel<<<tn * tm, NT, LDS, st>>>(a, tn, tm); }
  return check_launch("f32gemm_kernel");
}

static int launch_rowproj_f32(const float* src, int64_t M, int64_t Kd, const float* P, int r,
                              float* out, hipStream_t st) {
  if (M == 0 || r == 0) return REELS_HIP_OK;
  { TraceScope _ts(st, "rowproj_f32_kernel"); rowproj_f32_kernel<<<(unsigned)ceil_div(M, 64), 256, 0, st>>>(src, M, Kd, P, r, out); }
  return check_launch("rowproj_f32_kernel");
}

static int launch_colgrad_f32(const float* src, int64_t M, int64_t Od, const float* Lm, int r,
                              const PlanF32& p, float c, float* part, float* out, bool trans,
                              hipStream_t st) {
  const dim3 grid((unsigned)ceil_div(Od, f32c::BO), (unsigned)p.splits);
  { TraceScope _ts(st, "colgrad_f32_kernel"); colgrad_f32_kernel<<<grid, 256, 0, st>>>(src, M, Od, Lm, r, p.tps, part); }
  if (int rc = check_launch("colgrad_f32_kernel")) return rc;
  return launch_reduce_partials(part, p.splits, Od, r, r, c, out, trans, st);
}

static int launch_transpose_f32(const float* in, int64_t rows, int64_t cols, float* out, hipStream_t st) {
  { TraceScope _ts(st, "transpose_f32_kernel"); transpose_f32_kernel<<<dim3((unsigned)ceil_div(cols, 32), (unsigned)ceil_div(rows, 32)), 256, 0, st>>>(in, rows, cols, out); }
  return check_launch("transpose_f32_kernel");
}

static int i8lora_fwd_f32_impl(const float* x, const int8_t* q, const float* scales, const float* A,
                               const float* B, const float* bias, int64_t M, int64_t K, int64_t N,
                               int64_t r, float c, float* y, float* h_save, void* workspace,
                               size_t ws_bytes, hipStream_t st) {
  const char* fn = "reels_hip_i8lora_fwd_f32";
  if (M < 0 || K <= 0 || N <= 0 || r < 0 || r > 4096)
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": need M >= 0, K > 0, N > 0, 0 <= r <= 4096");
  if (!(c == c)) return fail(REELS_HIP_EINVAL, std::string(fn) + ": lora_scale is NaN");
  if (M == 0) return REELS_HIP_OK;
  if (!x || !q || !scales || !y || (r > 0 && (!A || !B)))
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": NULL x, q, scales, y, or A/B with r > 0");
  const bool aligned = aligned16(x) && aligned16(q) && aligned16(scales) && aligned16(A) &&
                       aligned16(B) && aligned16(bias) && aligned16(y) && aligned16(h_save) &&
                       aligned16(workspace);
  const PlanF32 p = plan_f32(M, K, N, r, aligned);
  const WsF32 w = ws_f32(M, K, N, r, REELS_HIP_WS_FWD, p);
  if (!workspace || ws_bytes < w.total)
    return fail(REELS_HIP_EWORKSPACE, std::string(fn) + ": workspace NULL or smaller than "
                                      "reels_hip_i8lora_workspace_bytes_f32(..., REELS_HIP_WS_FWD)");
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  float* h = h_save ? h_save : reinterpret_cast<float*>(ws + w.h);
  int rc;
  if (!p.fast) {
    if (r > 0) {
      // h = x A (A [K][r]: P(j, k) = A[k * r + j])
      { TraceScope _ts(st, "gf_rowproj_kernel"); gf_rowproj_kernel<<<g1(M * r), 256, 0, st>>>(x, M, K, A, r, 1, (int)r, h); }
      if ((rc = check_launch("gf_rowproj_kernel"))) return rc;
    }
    { TraceScope _ts(st, "gf_fwd_kernel"); gf_fwd_kernel<<<g1(M * N), 256, 0, st>>>(x, q, scales, h, B, bias, M, K, N, (int)r, c, y); }
    return check_launch("gf_fwd_kernel");
  }
  float* bt = nullptr;
  if (r > 0) {
    float* at = reinterpret_cast<float*>(ws + w.at);
    bt = reinterpret_cast<float*>(ws + w.bt);
    if ((rc = launch_transpose_f32(A, K, r, at, st))) return rc;  // At [r][K]
    if ((rc = launch_transpose_f32(B, r, N, bt, st))) return rc;  // Bt [N][r]
    if ((rc = launch_rowproj_f32(x, M, K, at, (int)r, h, st))) return rc;
  }
  float* wd = reinterpret_cast<float*>(ws + w.wd);
  if (K > 0) {
    { TraceScope _ts(st, "deq_f32_rows_kernel");
      const int64_t blocks = ceil_div(N * K / 4, 256);
      deq_f32_rows_kernel<<<(unsigned)(blocks < 65536 ? blocks : 65536), 256, 0, st>>>(q, scales, N, K, wd); }
    if ((rc = check_launch("deq_f32_rows_kernel"))) return rc;
  }
  F32GemmArgs g{};
  g.act = x; g.wd = wd; g.L = r > 0 ? h : nullptr; g.R = bt; g.bias = bias; g.out = y;
  g.M = M; g.Ncols = N; g.Kred = K; g.r = (int)r; g.c = c;
  return launch_f32gemm(0, g, st);
}

static int i8lora_bwd_f32_impl(const char* fn, const float* dy, const float* x, const float* hh,
                               const int8_t* q, const float* scales, const float* A,
                               const float* B, int64_t M, int64_t K, int64_t N, int64_t r, float c,
                               float* dx, float* dA, float* dB, float* dbias, void* workspace,
                               size_t ws_bytes, hipStream_t st) {
  if (M < 0 || K <= 0 || N <= 0 || r < 0 || r > 4096)
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": need M >= 0, K > 0, N > 0, 0 <= r <= 4096");
  if (!(c == c)) return fail(REELS_HIP_EINVAL, std::string(fn) + ": lora_scale is NaN");
  if (r == 0) { dA = nullptr; dB = nullptr; }
  int rc;
  if (M == 0) {  // empty token set: the reductions over tokens are zero
    if (dA && K * r > 0) {
      { TraceScope _ts(st, "zero_f32_kernel"); zero_f32_kernel<<<g1(K * r), 256, 0, st>>>(dA, K * r); }
      if ((rc = check_launch("zero_f32_kernel"))) return rc;
    }
    if (dB && N * r > 0) {
      { TraceScope _ts(st, "zero_f32_kernel"); zero_f32_kernel<<<g1(N * r), 256, 0, st>>>(dB, N * r); }
      if ((rc = check_launch("zero_f32_kernel"))) return rc;
    }
    if (dbias) {
      { TraceScope _ts(st, "zero_f32_kernel"); zero_f32_kernel<<<g1(N), 256, 0, st>>>(dbias, N); }
      if ((rc = check_launch("zero_f32_kernel"))) return rc;
    }
    return REELS_HIP_OK;
  }
  if (!dy || !q || !scales || (r > 0 && (!A || !B)) || ((dA || (dB && !hh)) && !x))
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": NULL dy, q, scales, A/B with r > 0, or x "
                                  "needed for dA / recomputing h");
  if (!dx && !dA && !dB && !dbias) return REELS_HIP_OK;
  const bool aligned = aligned16(dy) && aligned16(x) && aligned16(hh) && aligned16(q) &&
                       aligned16(scales) && aligned16(A) && aligned16(B) && aligned16(dx) &&
                       aligned16(dA) && aligned16(dB) && aligned16(workspace);
  const PlanF32 p = plan_f32(M, K, N, r, aligned);
  const WsF32 w = ws_f32(M, K, N, r, REELS_HIP_WS_BWD, p);
  if (!workspace || ws_bytes < w.total)
    return fail(REELS_HIP_EWORKSPACE, std::string(fn) + ": workspace NULL or smaller than "
                                      "reels_hip_i8lora_workspace_bytes_f32(..., REELS_HIP_WS_BWD)");
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  float* u = reinterpret_cast<float*>(ws + w.u);
  if (!p.fast) {
    if (r > 0) {
      // u = dy B^T (B [r][N]: P(j, n) = B[j * N + n])
      { TraceScope _ts(st, "gf_rowproj_kernel"); gf_rowproj_kernel<<<g1(M * r), 256, 0, st>>>(dy, M, N, B, 1, N, (int)r, u); }
      if ((rc = check_launch("gf_rowproj_kernel"))) return rc;
    }
    if (dx) {
      { TraceScope _ts(st, "gf_dx_kernel"); gf_dx_kernel<<<g1(M * K), 256, 0, st>>>(dy, q, scales, u, A, M, K, N, (int)r, c, dx); }
      if ((rc = check_launch("gf_dx_kernel"))) return rc;
    }
    if (dA) {
      { TraceScope _ts(st, "gf_colgrad_kernel<false>"); gf_colgrad_kernel<false><<<g1(K * r), 256, 0, st>>>(x, M, K, u, (int)r, c, dA); }
      if ((rc = check_launch("gf_colgrad_kernel"))) return rc;
    }
    if (dB) {
      const float* hp = hh;
      if (!hp) {
        float* hw = reinterpret_cast<float*>(ws + w.h);
        { TraceScope _ts(st, "gf_rowproj_kernel"); gf_rowproj_kernel<<<g1(M * r), 256, 0, st>>>(x, M, K, A, r, 1, (int)r, hw); }
        if ((rc = check_launch("gf_rowproj_kernel"))) return rc;
        hp = hw;
      }
      { TraceScope _ts(st, "gf_colgrad_kernel<true>"); gf_colgrad_kernel<true><<<g1(N * r), 256, 0, st>>>(dy, M, N, hp, (int)r, c, dB); }
      if ((rc = check_launch("gf_colgrad_kernel"))) return rc;
    }
    if (dbias)
      return launch_colsum(REELS_HIP_F32, dy, M, N, reinterpret_cast<float*>(ws + w.pbias), dbias, st);
    return REELS_HIP_OK;
  }
  // 1. u = dy B^T (B [r][N] rows are the projection rows); 2. dx = dy wt^T + c u A^T
  if (r > 0 && (dx || dA)) {
    if ((rc = launch_rowproj_f32(dy, M, N, B, (int)r, u, st))) return rc;
  }
  if (dx) {
    float* wt = reinterpret_cast<float*>(ws + w.wd);
    if (K > 0) {
      { TraceScope _ts(st, "deq_f32_transpose_kernel");
        deq_f32_transpose_kernel<<<dim3((unsigned)ceil_div(K, 64), (unsigned)ceil_div(N, 64)), 256, 0, st>>>(q, scales, N, K, wt); }
      if ((rc = check_launch("deq_f32_transpose_kernel"))) return rc;
    }
    F32GemmArgs g{};
    g.act = dy; g.wd = wt; g.L = r > 0 ? u : nullptr; g.R = A; g.bias = nullptr; g.out = dx;
    g.M = M; g.Ncols = K; g.Kred = N; g.r = (int)r; g.c = c;
    if ((rc = launch_f32gemm(1, g, st))) return rc;
  }
  // 3. dA = c x^T u ; dB = c (dy^T h)^T
  if (dA) {
    if ((rc = launch_colgrad_f32(x, M, K, u, (int)r, p, c, reinterpret_cast<float*>(ws + w.pa), dA, false, st))) return rc;
  }
  if (dB) {
    const float* hp = hh;
    if (!hp) {
      float* at = reinterpret_cast<float*>(ws + w.at);
      float* hw = reinterpret_cast<float*>(ws + w.h);
      if ((rc = launch_transpose_f32(A, K, r, at, st))) return rc;
      if ((rc = launch_rowproj_f32(x, M, K, at, (int)r, hw, st))) return rc;
      hp = hw;
    }
    if ((rc = launch_colgrad_f32(dy, M, N, hp, (int)r, p, c, reinterpret_cast<float*>(ws + w.pb), dB, true, st))) return rc;
  }
  if (dbias)
    return launch_colsum(REELS_HIP_F32, dy, M, N, reinterpret_cast<float*>(ws + w.pbias), dbias, st);
  return REELS_HIP_OK;
}

}  // namespace reels

using namespace reels;

extern "C" size_t reels_hip_i8lora_workspace_bytes_f32(int64_t M, int64_t K, int64_t N, int64_t r,
                                                       int which) {
  if (M < 0 || K < 0 || N < 0 || r < 0) return 0;
  if (which != REELS_HIP_WS_FWD && which != REELS_HIP_WS_BWD) return 0;
  const PlanF32 p = plan_f32(M, K, N, r, true);  // the fast layout is never smaller
  return ws_f32(M, K, N, r, which, p).total;
}

extern "C" int reels_hip_i8lora_fwd_f32(const float* x, const int8_t* q, const float* scales,
                                        const float* A, const float* B, const float* bias,
                                        int64_t M, int64_t K, int64_t N, int64_t r,
                                        float lora_scale, float* y, float* h_save, void* workspace,
                                        size_t ws_bytes, void* stream) {
  clear_error();
  return i8lora_fwd_f32_impl(x, q, scales, A, B, bias, M, K, N, r, lora_scale, y, h_save,
                             workspace, ws_bytes, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int reels_hip_i8lora_bwd_f32(const float* dy, const float* x, const float* h,
                                        const int8_t* q, const float* scales, const float* A,
                                        const float* B, int64_t M, int64_t K, int64_t N, int64_t r,
                                        float lora_scale, float* dx, float* dA, float* dB,
                                        void* workspace, size_t ws_bytes, void* stream) {
  clear_error();
  return i8lora_bwd_f32_impl("reels_hip_i8lora_bwd_f32", dy, x, h, q, scales, A, B, M, K, N, r,
                             lora_scale, dx, dA, dB, nullptr, workspace, ws_bytes,
                             reinterpret_cast<hipStream_t>(stream));
}

extern "C" int reels_hip_i8lora_bwd_bias_f32(const float* dy, const float* x, const float* h,
                                             const int8_t* q, const float* scales, const float* A,
                                             const float* B, int64_t M, int64_t K, int64_t N,
                                             int64_t r, float lora_scale, float* dx, float* dA,
                                             float* dB, float* dbias, void* workspace,
                                             size_t ws_bytes, void* stream) {
  clear_error();
  return i8lora_bwd_f32_impl("reels_hip_i8lora_bwd_bias_f32", dy, x, h, q, scales, A, B, M, K, N,
                             r, lora_scale, dx, dA, dB, dbias, workspace, ws_bytes,
                             reinterpret_cast<hipStream_t>(stream));
}

extern "C" int reels_hip_gelu_tanh_f32(const float* x, float* y, int64_t n, void* stream) {
  clear_error();
  if (n < 0) return fail(REELS_HIP_EINVAL, "reels_hip_gelu_tanh_f32: n < 0");
  if (n == 0) return REELS_HIP_OK;
  if (!x || !y) return fail(REELS_HIP_EINVAL, "reels_hip_gelu_tanh_f32: NULL pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  { TraceScope _ts(st, "gelu_f32_kernel"); gelu_f32_kernel<<<g1(n), 256, 0, st>>>(x, y, n); }
  return check_launch("gelu_f32_kernel");
}

extern "C" int reels_hip_gelu_tanh_bwd_f32(const float* x, const float* dy, float* dx, int64_t n,
                                           void* stream) {
  clear_error();
  if (n < 0) return fail(REELS_HIP_EINVAL, "reels_hip_gelu_tanh_bwd_f32: n < 0");
  if (n == 0) return REELS_HIP_OK;
  if (!x || !dy || !dx) return fail(REELS_HIP_EINVAL, "reels_hip_gelu_tanh_bwd_f32: NULL pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  { TraceScope _ts(st, "gelu_bwd_f32_kernel"); gelu_bwd_f32_kernel<<<g1(n), 256, 0, st>>>(x, dy, dx, n); }
  return check_launch("gelu_bwd_f32_kernel");
}
