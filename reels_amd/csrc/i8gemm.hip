// GEMMs of the int8 LoRA linear, bf16 MFMA on gfx950.
//
//   FWD (_weight_mul, src/layers/quantization.jl:73-74, inside lora_forward, lora.jl:56-95):
//     out[m][n] = bf16( sum_k act[m][k] deq(W)[n][k] + c * sum_j L[m][j] R[n][j] + bias[n] )
//     act = x [M][K], L = h [M][rp], R = B^T [N][rp]
//   DX  (_weight_transpose_mul, quantization.jl:75-76, inside lora_backward, lora.jl:115-116):
//     out[m][k] = bf16( sum_n act[m][n] deq(W)[n][k] + c * sum_j L[m][j] R[k][j] )
//     act = dy [M][N], L = u [M][rp], R = A [K][rp]
//
// Kernels in this file:
// * dequant_rows_kernel / dequant_transpose_kernel + bfgemm_kernel: the path for K and N
//   multiples of 64 (every Wan / LTX projection): deq(W) = bf16(fl32(q * s)) written once per
//   call (transposed for DX, scale folded in), then a bf16 GEMM with the LoRA epilogue.
// * i8gemm_v3_kernel (reduction a multiple of 64) and i8gemm_kernel (any reduction multiple of
//   16): the int8 codes themselves are staged in LDS and converted exactly to bf16 in registers;
//   the FWD scale s[n] is applied to the f32 sum. DX in bf16 takes act = bf16(dy * s) (bf16 has
//   f32's exponent range, so the pre-scaled operand cannot underflow); DX in f16 multiplies the
//   raw dy by the reference's binary16 weight f16(q * f16(s[n])) (quantization.jl:61-62), built
//   in registers from the int8 codes and the step's scales staged in LDS (i8gemm_kernel only),
//   so dy * s never has to fit binary16's exponent range.
//
// i8gemm_kernel: block tile 256 output columns (n in FWD, k in DX) x 256 tokens, reduction step
// 64, 256 threads = 4 waves in a 2 x 2 grid, each wave 128 x 128 = 4 x 4 tiles of
// v_mfma_f32_32x32x16_bf16. The MFMA A operand is the weight (rows = output columns) and the B
// operand the activations (columns = tokens), so each lane ends with 4 consecutive output
// columns of one token and the epilogue stores 8 bytes per lane. LDS (double-buffered, 96 KiB):
//   activations: [256 tokens][64] bf16, 16-byte chunks XOR-swizzled by f(row) so the 32-row
//                MFMA operand reads (ds_read_b128) hit distinct banks;
//   weights: int8 as loaded from HBM (half the LDS bytes of bf16), converted exactly to bf16 in
//            registers after the read:
//     FWD [256 n][64 k]: operand = 8 consecutive k of one row n -> ds_read_b64
//     DX  [64 n][256 k]: operand = 8 consecutive n of one column k -> ds_read_b64_tr_b8 (gfx950
//         transpose read: lane i of a 16-lane group receives byte i%8 of the 8 bytes addressed
//         by lane 2j + i/8, j = 0..7)
#include "i8gemm.h"

#include <mutex>

namespace reels {

namespace gemm {
constexpr int BM = 256;  // tokens per block
constexpr int BN = 256;  // output columns per block
constexpr int BK = 64;   // reduction per step
constexpr int NT = 256;
constexpr int ACT_BYTES = BM * BK * 2;  // 32 KiB
constexpr int W_BYTES = BN * BK;        // 16 KiB
constexpr int S_BYTES = BK * 2;          // DX with redscale: f16(s[n]) of the step's 64 n
constexpr int STAGE_BYTES = ACT_BYTES + W_BYTES + S_BYTES;
}  // namespace gemm


// swizzles (see the header comment); all map [0, 8) or [0, 16) onto itself for a fixed row
__device__ __forceinline__ int act_swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int wf_swz(int row) { return ((row >> 1) & 7) ^ ((row >> 4) & 1); }
__device__ __forceinline__ int wd_swz(int row) { return (row & 7) | ((row & 1) << 3); }
// bf16 GEMM tiles ([rows][64] bf16, 8 chunks of 16 bytes per row): chunk ^ (row & 7). Its
// 16x16x32 fragment reads (lanes 0-15 rows r..r+15 of one chunk, lanes 16-63 the next three
// chunks) are free of bank conflicts; act_swz's extra ^ (row >> 3) costs 2 of 5 LDS cycles per
// ds_read_b128 in this pattern (SQ_LDS_BANK_CONFLICT).
__device__ __forceinline__ int bf_swz(int row) { return row & 7; }

template <int MODE, int ELT>  // MODE 0 = FWD, 1 = DX; ELT the 16-bit element type
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void i8gemm_kernel(GemmArgs a) {
  using E = Elt<ELT>;
  typedef typename E::v8 V8;
  using namespace gemm;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t n0 = (int64_t)blockIdx.x * BN;  // output column block
  const int64_t m0 = (int64_t)blockIdx.y * BM;  // token block
  const int64_t M = a.M, Ncols = a.Ncols, Kred = a.Kred;
  const int nk = (int)((Kred + BK - 1) / BK);

  // ---- global -> register staging --------------------------------------------------------
  u32x4 ra[8], rw[4];
  uint32_t rs = 0;  // DX with redscale: f16(s[n]) for n = r0 + t (threads 0..63)
  const bool dxs = MODE == 1 && a.redscale != nullptr;
  auto load_tiles = [&](int kt) {
    const int64_t r0 = (int64_t)kt * BK;
    if (dxs && t < BK) {
      const int64_t n = r0 + t;
      rs = n < Kred ? E::bits(a.redscale[n]) : 0u;  // f16(s): E::bits rounds to the element type
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = (t >> 3) + 32 * i, c = t & 7;
      const int64_t m = m0 + row, k = r0 + c * 8;
      const bool ok = (m < M) && (k < Kred);
      const int64_t mc = m < M ? m : M - 1, kc = k < Kred ? k : 0;
      u32x4 v = *reinterpret_cast<const u32x4*>(a.act + mc * Kred + kc);
      ra[i] = ok ? v : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int64_t wr, wc;
      bool ok;
      if (MODE == 0) {  // rows n (output columns), 64 contiguous k
        const int row = (t >> 2) + 64 * i, c = t & 3;
        wr = n0 + row; wc = r0 + c * 16;
        ok = (wr < Ncols) && (wc < Kred);
        if (wr >= Ncols) wr = Ncols - 1;
        if (wc >= Kred) wc = 0;
      } else {          // rows n (reduction), 256 contiguous k (output columns)
        const int row = (t >> 4) + 16 * i, c = t & 15;
        wr = r0 + row; wc = n0 + c * 16;
        ok = (wr < Kred) && (wc < Ncols);
        if (wr >= Kred) wr = Kred - 1;
        if (wc >= Ncols) wc = 0;
      }
      u32x4 v = *reinterpret_cast<const u32x4*>(a.q + wr * a.ldq + wc);
      rw[i] = ok ? v : u32x4{0, 0, 0, 0};
    }
  };

  // ---- register -> LDS ------------------------------------------------------------------
  auto store_tiles = [&](int buf) {
    uint8_t* sa = smem + buf * STAGE_BYTES;
    uint8_t* sw = sa + ACT_BYTES;
    if (dxs && t < BK) reinterpret_cast<uint16_t*>(sw + W_BYTES)[t] = (uint16_t)rs;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = (t >> 3) + 32 * i, c = t & 7;
      *reinterpret_cast<u32x4*>(sa + row * 128 + ((c ^ act_swz(row)) << 4)) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (MODE == 0) {
        const int row = (t >> 2) + 64 * i, c = t & 3;
        const int g = wf_swz(row);
        u32x4 v = rw[i];
        if (g & 1) v = u32x4{v[2], v[3], v[0], v[1]};
        *reinterpret_cast<u32x4*>(sw + row * 64 + ((c ^ (g >> 1)) << 4)) = v;
      } else {
        const int row = (t >> 4) + 16 * i, c = t & 15;
        *reinterpret_cast<u32x4*>(sw + row * 256 + ((c ^ wd_swz(row)) << 4)) = rw[i];
      }
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // per-lane LDS read offsets (independent of the k step)
  const int l32 = lane & 31, lhi = lane >> 5;

  auto compute = [&](int buf) {
    const uint8_t* sa = smem + buf * STAGE_BYTES;
    const uint8_t* sw = sa + ACT_BYTES;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      V8 bfr[4], afr[4];
#pragma unroll
      for (int tj = 0; tj < 4; ++tj) {
        const int row = wm * 128 + tj * 32 + l32;
        const int c = kk * 2 + lhi;
        bfr[tj] = E::as8(*reinterpret_cast<const u32x4*>(sa + row * 128 + ((c ^ act_swz(row)) << 4)));
      }
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) {
        u32x2 raw;
        if (MODE == 0) {
          const int row = wn * 128 + ti * 32 + l32;
          const int sub = kk * 2 + lhi;
          raw = *reinterpret_cast<const u32x2*>(sw + row * 64 + ((sub ^ wf_swz(row)) << 3));
        } else {
          const int g = lane >> 4, i16 = lane & 15;
          const int row = kk * 16 + (g >> 1) * 8 + (i16 >> 1);
          const int col = wn * 128 + ti * 32 + 16 * (g & 1) + 8 * (i16 & 1);
          const int sub = col >> 3;  // 0..31
          const uint8_t* p = sw + row * 256 + ((sub ^ (wd_swz(row) << 1)) << 3);
          i32x2 v = __builtin_amdgcn_ds_read_tr8_b64_v2i32(LDS_PTR(i32x2, p));
          raw = u32x2{(uint32_t)v[0], (uint32_t)v[1]};
        }
        afr[ti] = E::from_i8x8(raw[0], raw[1]);
        if (dxs) {
          // the 8 bytes this lane received are rows n = kk*16 + (lane/32)*8 + (0..7) of the step
          // (byte j from providing lane 2j + i/8, whose row is kk*16 + (g/2)*8 + j): multiply each
          // exact code by its f16 scale, one binary16 rounding, as Float16(q) * Float16(s)
          const int nrow = kk * 16 + (lane >> 5) * 8;
          const u32x4 s8 = *reinterpret_cast<const u32x4*>(sw + W_BYTES + nrow * 2);
          afr[ti] = E::scale8(afr[ti], s8);
        }
      }
#pragma unroll
      for (int ti = 0; ti < 4; ++ti)
#pragma unroll
        for (int tj = 0; tj < 4; ++tj)
          acc[ti][tj] = E::mfma32(afr[ti], bfr[tj], acc[ti][tj]);
    }
  };

  load_tiles(0);
  store_tiles(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tiles(kt + 1);
    compute(cur);
    if (kt + 1 < nk) store_tiles(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: scale, LoRA up-projection on MFMA, bias, one bf16 rounding ----------------
  const int nsteps = a.rp >> 4;
#pragma unroll
  for (int ti = 0; ti < 4; ++ti) {
    const int64_t nrow = n0 + wn * 128 + ti * 32 + l32;  // R operand row of this lane
    const int64_t nrc = nrow < Ncols ? nrow : Ncols - 1;
    // per-lane output columns: n = nbase + g4*8 + (0..3)
    const int64_t nbase = n0 + wn * 128 + ti * 32 + lhi * 4;
    float sc[16], bs[16];
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int64_t n = nbase + g4 * 8;
      const bool ok = n < Ncols;
      f32x4 s4 = {1.0f, 1.0f, 1.0f, 1.0f};
      if (a.colscale != nullptr && ok) s4 = *reinterpret_cast<const f32x4*>(a.colscale + n);
      u32x2 b2 = {0, 0};
      if (a.bias != nullptr && ok) b2 = *reinterpret_cast<const u32x2*>(a.bias + n);
#pragma unroll
      for (int e = 0; e < 4; ++e) sc[g4 * 4 + e] = s4[e];
      bs[g4 * 4 + 0] = E::lo(b2[0]); bs[g4 * 4 + 1] = E::hi(b2[0]);
      bs[g4 * 4 + 2] = E::lo(b2[1]); bs[g4 * 4 + 3] = E::hi(b2[1]);
    }
#pragma unroll
    for (int tj = 0; tj < 4; ++tj) {
      const int64_t m = m0 + wm * 128 + tj * 32 + l32;
      const int64_t mc = m < M ? m : M - 1;
      f32x16 lo;
#pragma unroll
      for (int v = 0; v < 16; ++v) lo[v] = 0.0f;
      for (int s = 0; s < nsteps; ++s) {
        u32x4 rv = *reinterpret_cast<const u32x4*>(a.R + nrc * a.rp + s * 16 + lhi * 8);
        u32x4 lv = *reinterpret_cast<const u32x4*>(a.L + mc * a.rp + s * 16 + lhi * 8);
        if (nrow >= Ncols) rv = u32x4{0, 0, 0, 0};
        if (m >= M) lv = u32x4{0, 0, 0, 0};
        lo = E::mfma32(E::as8(rv), E::as8(lv), lo);
      }
      if (m < M) {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int64_t n = nbase + g4 * 8;
          if (n < Ncols) {
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int v = g4 * 4 + e;
              o[e] = sc[v] * acc[ti][tj][v] + a.c * lo[v] + bs[v];
            }
            u32x2 pk = {E::pack2(o[0], o[1]), E::pack2(o[2], o[3])};
            *reinterpret_cast<u32x2*>(a.out + m * Ncols + n) = pk;
          }
        }
      }
    }
  }
}

// FWD weight tile of the three-stage kernel: [256 n][64 k] int8, 16-byte slots XOR-swizzled
// within the 64-byte row so 32-row fragment reads (ds_read_b128) hit distinct banks
__device__ __forceinline__ int wf2_swz(int row) { return ((row >> 1) & 3) ^ ((row >> 3) & 1); }

// =============================================================================================
// Main kernel, used whenever the reduction length is a multiple of 64 (every Wan / LTX shape).
//
// * HBM -> LDS with buffer_load_dwordx4 ... lds (no staging registers, no VALU for the copy),
//   three LDS stages (3 x 48 KiB): the loads for step k+2 are in flight while step k is computed.
//   SGPR base + per-lane 32-bit voffset; the k advance is the scalar soffset.
// * 8 waves (two per SIMD, so one wave's MFMAs cover the other's LDS reads, int8 -> bf16
//   conversion and copies), 256 x 256 block tile, reduction step 64. A four-wave layout with
//   128 x 128 wave tiles (half the LDS read traffic, explicitly interleaved schedule) measured
//   the same throughput on the Wan shapes.
// * FWD reads a weight fragment for two MFMA steps with one ds_read_b128: the 64 reduction
//   indices of a step pair are assigned so that lane half lhi, step 2p+e uses k = 32p + 16lhi +
//   8e + (0..7); the activation fragment of that step is 16-byte chunk 4p + 2lhi + e of the row.
//   (The pairing only reorders the reduction; both operands use the same k for each product.)
// * DX reads weight fragments with ds_read_b64_tr_b8 as the general kernel does.
// * Tiles are mapped to XCDs (block b runs on XCD b % 8): each XCD takes a contiguous range of
//   the tile order, and the order walks 4 token blocks before moving to the next column block,
//   so the ~32 tiles resident on one XCD share activation and weight tiles in its L2. Wave w owns tokens [128*(w/4), +128) and output columns [64*(w%4), +64): 4 x 2 tiles
// of 32x32 (128 accumulator registers). Per 64-step and wave: 16 activation fragment reads, 4
// (FWD, ds_read_b128) or 8 (DX, ds_read_b64_tr_b8) weight fragment reads, 32 MFMAs.
namespace gemm3 {
constexpr int BM = 256, BN = 256, BK = 64, NT = 512;
constexpr int ACT = BM * BK * 2;   // 32 KiB
constexpr int WB = BN * BK;        // 16 KiB
constexpr int STAGE = ACT + WB;    // 48 KiB
constexpr int NSTAGE = 3;
constexpr int GM = 4;
}  // namespace gemm3

// SPLIT: one of a.ksplit reduction ranges of the tile, written as an f32 partial (colscale
// applied, LoRA term in split 0, no bias), as in the bf16 GEMM below
template <int MODE, int ELT, bool SPLIT>
__global__ __launch_bounds__(512)
void i8gemm_v3_kernel(GemmArgs a, int tiles_n, int tiles_m) {
  using E = Elt<ELT>;
  typedef typename E::v8 V8;
  using namespace gemm3;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = w >> 2, wn = w & 3;
  const int l32 = lane & 31, lhi = lane >> 5;
  const int64_t M = a.M, Ncols = a.Ncols, Kred = a.Kred;

  const int nt = tiles_n * tiles_m;
  const int ks = SPLIT ? a.ksplit : 1;  // reduction splits: a tile's are consecutive
  const int b = blockIdx.x;
  const int xcd = b & 7, idx = b >> 3;
  const int lo = (nt * ks) >> 3, rem = (nt * ks) & 7;
  const int lall = xcd * lo + (xcd < rem ? xcd : rem) + idx;
  const int logical = lall / ks, split = lall - logical * ks;
  const int group = GM * tiles_n;
  const int g = logical / group;
  const int first_m = g * GM;
  const int gm = (tiles_m - first_m) < GM ? (tiles_m - first_m) : GM;
  const int within = logical - g * group;
  const int64_t m0 = (int64_t)(first_m + within % gm) * BM;
  const int64_t n0 = (int64_t)(within / gm) * BN;

  // this workgroup's reduction steps [kb, kb + nk) of 64
  const int nkt = (int)(Kred / BK);
  const int kb = (int)((int64_t)split * nkt / ks);
  const int nk = (int)((int64_t)(split + 1) * nkt / ks) - kb;
  const i32x4 ract = buffer_rsrc(a.act, (uint32_t)(M * Kred * 2));
  const i32x4 rq = buffer_rsrc(a.q, (uint32_t)(Ncols * Kred));
  uint32_t voa[4], vow[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = (w * 4 + i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ act_swz(row);
    const int64_t m = (m0 + row < M) ? m0 + row : M - 1;
    voa[i] = (uint32_t)((m * Kred + (int64_t)kb * BK + c * 8) * 2);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (MODE == 0) {
      const int row = (w * 2 + i) * 16 + (lane >> 2);
      const int j = (lane & 3) ^ wf2_swz(row);
      const int64_t n = (n0 + row < Ncols) ? n0 + row : Ncols - 1;
      vow[i] = (uint32_t)(n * Kred + (int64_t)kb * BK + j * 16);
    } else {
      const int row = (w * 2 + i) * 4 + (lane >> 4);
      const int c = (lane & 15) ^ wd_swz(row);
      int64_t kc = n0 + c * 16;
      if (kc >= Ncols) kc = Ncols - 16;
      vow[i] = (uint32_t)(((int64_t)kb * BK + row) * a.ldq + kc);
    }
  }
  auto issue = [&](int kt, int stage) {
    uint8_t* base = smem + stage * STAGE;
    const uint32_t sa = (uint32_t)kt * (BK * 2);
    const uint32_t sw = MODE == 0 ? (uint32_t)kt * BK : (uint32_t)kt * (uint32_t)(BK * a.ldq);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dma16(ract, voa[i], sa, base + (w * 4 + i) * 1024);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      dma16(rq, vow[i], sw, base + ACT + (w * 2 + i) * 1024);
  };

  f32x16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // ---- k loop ----------------------------------------------------------------------------
  // Registers carry, across the barrier, the weight fragments of the next step and the
  // activation fragments of its first MFMA sub-step: the barrier (and the wait for the next
  // stage's loads) sits before the last sub-step of each step, whose MFMAs then cover the LDS
  // latency of the next step's first reads. Stage j+2 is issued right after the barrier of step
  // j, into the buffer of step j-1, which every wave has finished reading by then.
  auto xchunk = [&](int s) { return MODE == 0 ? 4 * (s >> 1) + 2 * lhi + (s & 1) : 2 * s + lhi; };
  auto read_x = [&](const uint8_t* sa, int s, V8* xf) {
    const int c = xchunk(s);
#pragma unroll
    for (int tj = 0; tj < 4; ++tj) {
      const int row = wm * 128 + tj * 32 + l32;
      xf[tj] = E::as8(*reinterpret_cast<const u32x4*>(sa + row * 128 + ((c ^ act_swz(row)) << 4)));
    }
  };
  u32x4 wr[2][2];   // FWD: raw int8 weight slots [pair][ti]
  i32x2 wt[4][2];   // DX: transposed raw int8 [step][ti]
  auto read_w = [&](const uint8_t* sw) {
    if (MODE == 0) {
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) {
          const int row = wn * 64 + ti * 32 + l32;
          const int j = 2 * pp + lhi;
          wr[pp][ti] = *reinterpret_cast<const u32x4*>(sw + row * 64 + ((j ^ wf2_swz(row)) << 4));
        }
    } else {
      const int gq = lane >> 4, i16 = lane & 15;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) {
          const int row = kk * 16 + (gq >> 1) * 8 + (i16 >> 1);
          const int col = wn * 64 + ti * 32 + 16 * (gq & 1) + 8 * (i16 & 1);
          const uint8_t* p = sw + row * 256 + (((col >> 3) ^ (wd_swz(row) << 1)) << 3);
          wt[kk][ti] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(LDS_PTR(i32x2, p));
        }
    }
  };
  auto convert = [&](int s, V8* af) {
#pragma unroll
    for (int ti = 0; ti < 2; ++ti) {
      if (MODE == 0) {
        const u32x4& r = wr[s >> 1][ti];
        af[ti] = (s & 1) ? E::from_i8x8(r[2], r[3]) : E::from_i8x8(r[0], r[1]);
      } else {
        af[ti] = E::from_i8x8((uint32_t)wt[s][ti][0], (uint32_t)wt[s][ti][1]);
      }
    }
  };
  auto mfma8 = [&](const V8* af, const V8* xf) {
#pragma unroll
    for (int tj = 0; tj < 4; ++tj)
#pragma unroll
      for (int ti = 0; ti < 2; ++ti)
        acc[ti][tj] = E::mfma32(af[ti], xf[tj], acc[ti][tj]);
  };

  V8 xa[4], xb[4], af[2];
  issue(0, 0);
  if (nk > 1) issue(1, 1);
  if (nk > 1) __builtin_amdgcn_s_waitcnt(0x0F76);  // vmcnt(6): stage 1 may stay in flight
  else __builtin_amdgcn_s_waitcnt(0x0F70);
  __builtin_amdgcn_s_barrier();
  read_w(smem + ACT);
  read_x(smem, 0, xa);
  for (int kt = 0; kt < nk; ++kt) {
    const uint8_t* sa = smem + (kt % NSTAGE) * STAGE;
    __builtin_amdgcn_iglp_opt(MODE == 0 ? 1 : 0);
    convert(0, af);
    read_x(sa, 1, xb);
    mfma8(af, xa);
    convert(1, af);
    read_x(sa, 2, xa);
    mfma8(af, xb);
    convert(2, af);
    read_x(sa, 3, xb);
    mfma8(af, xa);
    convert(3, af);
    if (kt + 1 < nk) {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): stage kt+1 has landed
      __builtin_amdgcn_s_barrier();
      if (kt + 2 < nk) issue(kt + 2, (kt + 2) % NSTAGE);
      const uint8_t* sn = smem + ((kt + 1) % NSTAGE) * STAGE;
      read_w(sn + ACT);
      read_x(sn, 0, xa);
    }
    mfma8(af, xb);
  }

  // ---- epilogue: scale, LoRA up-projection on MFMA, bias, one bf16 rounding; the finished
  // 256 x 256 bf16 tile is staged in LDS (rows of 512 bytes, 16-byte chunks XOR-swizzled by row)
  // and written to HBM as whole 512-byte row segments.
  __syncthreads();  // every wave is done reading the last stage
  uint8_t* stile = smem;
  const int nsteps = split == 0 ? a.rp >> 4 : 0;  // the LoRA term: in split 0 only
#pragma unroll
  for (int ti = 0; ti < 2; ++ti) {
    const int64_t nrow = n0 + wn * 64 + ti * 32 + l32;
    const int64_t nrc = nrow < Ncols ? nrow : Ncols - 1;
    const int nloc = wn * 64 + ti * 32 + lhi * 4;  // tile-local column of this lane's group 0
    const int64_t nbase = n0 + nloc;
    float sc[16], bs[16];
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int64_t n = nbase + g4 * 8;
      const bool ok = n < Ncols;
      f32x4 s4 = {1.0f, 1.0f, 1.0f, 1.0f};
      if (a.colscale != nullptr && ok) s4 = *reinterpret_cast<const f32x4*>(a.colscale + n);
      u32x2 b2 = {0, 0};
      if (a.bias != nullptr && ok) b2 = *reinterpret_cast<const u32x2*>(a.bias + n);
#pragma unroll
      for (int e = 0; e < 4; ++e) sc[g4 * 4 + e] = s4[e];
      bs[g4 * 4 + 0] = E::lo(b2[0]); bs[g4 * 4 + 1] = E::hi(b2[0]);
      bs[g4 * 4 + 2] = E::lo(b2[1]); bs[g4 * 4 + 3] = E::hi(b2[1]);
    }
#pragma unroll
    for (int tj = 0; tj < 4; ++tj) {
      const int mloc = wm * 128 + tj * 32 + l32;
      const int64_t m = m0 + mloc;
      const int64_t mc = m < M ? m : M - 1;
      f32x16 lo;
#pragma unroll
      for (int v = 0; v < 16; ++v) lo[v] = 0.0f;
      for (int s = 0; s < nsteps; ++s) {
        u32x4 rv = *reinterpret_cast<const u32x4*>(a.R + nrc * a.rp + s * 16 + lhi * 8);
        u32x4 lv = *reinterpret_cast<const u32x4*>(a.L + mc * a.rp + s * 16 + lhi * 8);
        if (nrow >= Ncols) rv = u32x4{0, 0, 0, 0};
        if (m >= M) lv = u32x4{0, 0, 0, 0};
        lo = E::mfma32(E::as8(rv), E::as8(lv), lo);
      }
      if constexpr (SPLIT) {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int64_t n = nbase + g4 * 8;
          f32x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int v = g4 * 4 + e;
            o[e] = sc[v] * acc[ti][tj][v] + (split == 0 ? a.c * lo[v] : 0.0f);
          }
          if (m < M && n < Ncols) *reinterpret_cast<f32x4*>(a.part + ((int64_t)split * M + m) * Ncols + n) = o;
        }
        continue;
      }
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int v = g4 * 4 + e;
          o[e] = sc[v] * acc[ti][tj][v] + a.c * lo[v] + bs[v];
        }
        const u32x2 pk = {E::pack2(o[0], o[1]), E::pack2(o[2], o[3])};
        const int col = nloc + g4 * 8;                       // 4 columns, 8 bytes
        const int chunk = (col >> 3) ^ (mloc & 31);          // 16-byte chunk, swizzled
        *reinterpret_cast<u32x2*>(stile + mloc * 512 + chunk * 16 + (col & 7) * 2) = pk;
      }
    }
  }
  if constexpr (SPLIT) return;  // the partials went straight to global memory
  __syncthreads();
  // 256 rows x 32 chunks of 16 bytes; a wave stores two whole 512-byte row segments per instruction
#pragma unroll 4
  for (int i = 0; i < 16; ++i) {
    const int id = t + 512 * i, row = id >> 5, c = id & 31;
    const int64_t m = m0 + row, n = n0 + c * 8;
    if (m < M && n < Ncols) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(stile + row * 512 + ((c ^ (row & 31)) << 4));
      *reinterpret_cast<u32x4*>(a.out + m * Ncols + n) = v;
    }
  }
}

// =============================================================================================
// Dequantized-weight path (every shape whose K and N are multiples of 64, i.e. every Wan / LTX
// projection). Like the reference's _materialize_weight (src/layers/quantization.jl:54-64,
// dequantize then GEMM), the int8 weight is expanded once per call into a bf16 copy
// wd = bf16(fl32(q * s)) in the caller's workspace, and a plain bf16 GEMM with the LoRA epilogue
// runs on it. For dX the copy is written transposed, wt[k][n] = bf16(fl32(q[n][k] * s[n])), so
// the same GEMM computes dx = dy wt^T with the scale folded into the weight. Against the int8
// GEMM above this takes the int8 -> bf16 conversion (VALU in every wave's inner loop) out of the
// GEMM at the cost of a streaming pass over the weight (~1-2% of the GEMM's time); the passes
// are in dequant.hip.

// bf16 GEMM: 256 x 256 block tile, reduction step 64, 8 waves (two per SIMD), each wave 128
// tokens x 64 output columns; HBM -> LDS copies into a two-stage ring of 64 KiB stages
// (activation and weight tiles [256][64] bf16 with the same 16-byte XOR swizzle). At the barrier
// that ends step kt every wave has finished reading stage kt (lgkmcnt(0) before it), so the copy
// of step kt+2 goes into it right away and has one step to land. XCD-aware tile order and the
// epilogue as in the int8 kernel (minus the column scale).
namespace bfg {
constexpr int BM = 256, BN = 256, BK = 64, NT = 512;
constexpr int ACT = BM * BK * 2;   // 32 KiB
constexpr int WB = BN * BK * 2;    // 32 KiB
constexpr int LDS = 3 * ACT + 2 * WB;  // 160 KiB: activation ring of 3 stages, weight ring of 2
constexpr int GM = 4;
}  // namespace bfg

// MFMA shape: v_mfma_f32_16x16x32_bf16, so a wave's 128 x 64 is 8 x 4 tiles of 16 x 16 and a
// step is two sub-steps of k = 32. Per flop it moves half the accumulator registers of
// v_mfma_f32_32x32x16_bf16 (4 per 16K flops against 16 per 32K); the GPU runs at its power cap
// under this load, and sustained register-only loops of the 16 x 16 form run 10-13% faster
// (this GEMM: +3.5% over the same kernel on 32 x 32 tiles). Lane l supplies row l % 16 of both
// operands with k = 8 (l / 16) + (0..7) (any k order shared by the two operands gives the same
// sum); D register v of lane l is output column 4 (l / 16) + v, token l % 16 of the tile.
// SPLIT: the workgroup takes one of a.ksplit reduction ranges of its tile and writes an f32
// partial (a separate instantiation, so the unsplit kernel's registers stay as they are).
// EPI (unsplit only): 0 plain; 1 writes gout = rnd(gelu_tanh(out)) beside out (the FFN's first
// projection followed by its GELU), and 2 writes out = rnd(rnd(sum) * gelu_tanh'(gx)), the GELU's
// pullback of the product; both from the rounded 16-bit values the plain kernel stores, so the
// bits equal the separate GELU passes.
template <int ELT, bool SPLIT, int EPI = 0>
__global__ __launch_bounds__(512)
void bfgemm_kernel(GemmArgs a, const uint16_t* __restrict__ wd, int tiles_n, int tiles_m) {
  static_assert(EPI == 0 || !SPLIT, "the GELU epilogues run on the unsplit kernel");
  using E = Elt<ELT>;
  typedef typename E::v8 V8;
  using namespace bfg;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = w >> 2, wn = w & 3;
  const int l16 = lane & 15, lq = lane >> 4;
  const int64_t M = a.M, Ncols = a.Ncols, Kred = a.Kred;

  const int nt = tiles_n * tiles_m;
  const int ks = SPLIT ? a.ksplit : 1;  // reduction splits: a tile's are consecutive
  const int b = blockIdx.x;
  const int xcd = b & 7, idx = b >> 3;
  const int lo = (nt * ks) >> 3, rem = (nt * ks) & 7;
  const int lall = xcd * lo + (xcd < rem ? xcd : rem) + idx;
  const int logical = lall / ks, split = lall - logical * ks;
  const int group = GM * tiles_n;
  const int g = logical / group;
  const int first_m = g * GM;
  const int gm = (tiles_m - first_m) < GM ? (tiles_m - first_m) : GM;
  const int within = logical - g * group;
  const int64_t m0 = (int64_t)(first_m + within % gm) * BM;
  const int64_t n0 = (int64_t)(within / gm) * BN;

  // this workgroup's reduction steps [kb, kb + nk) of 64
  const int nkt = (int)(Kred / BK);
  const int kb = (int)((int64_t)split * nkt / ks);
  const int nk = (int)((int64_t)(split + 1) * nkt / ks) - kb;
  const i32x4 ract = buffer_rsrc(a.act, (uint32_t)(M * Kred * 2));
  const i32x4 rw = buffer_rsrc(wd, (uint32_t)(Ncols * Kred * 2));
  uint32_t voa[4], vow[4];  // copies i: rows (w*4+i)*8 + lane/8 of each tile, 16 bytes per lane
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = (w * 4 + i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ bf_swz(row);
    const int64_t m = (m0 + row < M) ? m0 + row : M - 1;
    const int64_t n = (n0 + row < Ncols) ? n0 + row : Ncols - 1;
    voa[i] = (uint32_t)((m * Kred + (int64_t)kb * BK + c * 8) * 2);
    vow[i] = (uint32_t)((n * Kred + (int64_t)kb * BK + c * 8) * 2);
  }
  const i32x4 rnone = buffer_rsrc(a.act, 0u);  // zero records: a copy through it reads nothing
  // LDS: activation ring of 3 stages [0, 96 KiB), weight ring of 2 stages [96, 160 KiB); step kt
  // uses activation stage kt % 3 and weight stage kt % 2
  auto abase = [&](int kt) { return smem + (kt % 3) * ACT; };
  auto wbase = [&](int kt) { return smem + 3 * ACT + (kt & 1) * WB; };
  auto issue_act = [&](int kt, int i) {
    dma16(ract, voa[i], (uint32_t)kt * (BK * 2), abase(kt) + (w * 4 + i) * 1024);
  };
  auto issue_w = [&](int kt, int i) {
    dma16(rw, vow[i], (uint32_t)kt * (BK * 2), wbase(kt) + (w * 4 + i) * 1024);
  };
  // LoRA operands (rank up to 32): the L tile [256 tokens][32] and the R tile [256 columns][32],
  // rows of 64 bytes, zeros past the rank, copied before the first steps' copies into activation
  // stage 2 (free until step 0 issues step 2's copies, after the prologue's barrier) as bytes
  // [0, 16) and [16, 32) KiB (copies 0-1 L, 2-3 R; copy i of wave w fills 1 KiB = 16 rows). A
  // 16 x 32 fragment is then 1 KiB of contiguous LDS. The accumulators start at c L R^T, computed
  // while the first steps' copies land, so the epilogue adds only the bias and rounds. Higher
  // ranks read L and R from global memory in the epilogue.
  const int rp = a.rp;
  const bool lora = rp > 0 && a.L != nullptr && split == 0;  // split 0 carries the LoRA term
  const bool lr_lds = lora && rp <= 32;
  auto issue_lr = [&](int kt, int k) {  // copy k (0..3) into activation stage kt
    const bool isr = k >= 2;
    const int ci = w * 2 + (k & 1);
    const int row = ci * 16 + (lane >> 2), c = lane & 3;
    const int64_t origin = isr ? n0 : m0, rows = isr ? Ncols : M;
    const uint32_t vo = (c * 8 < rp) ? (uint32_t)((origin + row) * rp * 2 + c * 16) : 0xFFFFFFF0u;
    const i32x4 rs = lr_lds ? buffer_rsrc(isr ? a.R : a.L, (uint32_t)(rows * rp * 2)) : rnone;
    dma16(rs, vo, 0u, abase(kt) + (isr ? 16384 : 0) + ci * 1024);
  };

  f32x4 acc[4][8];  // [output-column tile][token tile]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = 0.0f;

  // fragment reads: sub-step s of a step uses the 16-byte chunk 4 s + l / 16 of each row; rows of
  // a 16-row tile start at multiples of 16, so the row swizzle depends on the lane only
  const int swz = bf_swz(l16);
  auto read_w = [&](const uint8_t* sw, int s, V8* wf) {  // sw: a weight stage
    const int off = ((4 * s + lq) ^ swz) << 4;
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
      wf[ti] = E::as8(*reinterpret_cast<const u32x4*>(sw + (wn * 64 + ti * 16 + l16) * 128 + off));
  };
  auto read_x = [&](const uint8_t* sa, int s, int tj) {
    const int off = ((4 * s + lq) ^ swz) << 4;
    return E::as8(*reinterpret_cast<const u32x4*>(sa + (wm * 128 + tj * 16 + l16) * 128 + off));
  };
  auto mfma4 = [&](const V8* wf, const V8& xf, int tj) {
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
      acc[ti][tj] = E::mfma16(wf[ti], xf, acc[ti][tj]);
  };

  V8 w0[4], w1[4], x[8];
  // L and R first (through the zero-record descriptor when they stay in global memory: the copy
  // counts of the waits below are the same either way), then steps 0 and 1
#pragma unroll
  for (int k = 0; k < 4; ++k) issue_lr(2, k);
#pragma unroll
  for (int i = 0; i < 4; ++i) { issue_act(0, i); issue_w(0, i); }
  if (nk > 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) { issue_act(1, i); issue_w(1, i); }
  }
  if (lr_lds) {
    // acc = c L R^T: the same L fragments serve every column tile
    if (nk > 1) __builtin_amdgcn_s_waitcnt(0x4F70);  // vmcnt(16): L and R have landed
    else __builtin_amdgcn_s_waitcnt(0x0F78);         // vmcnt(8)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");  // the L and R reads stay after the barrier
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* sL = abase(2);
    const uint8_t* sR = sL + 16384;
    V8 lf[8], rf[4];
#pragma unroll
    for (int tj = 0; tj < 8; ++tj)
      lf[tj] = E::as8(*reinterpret_cast<const u32x4*>(sL + (wm * 128 + tj * 16 + l16) * 64 + lq * 16));
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
      rf[ti] = E::as8(*reinterpret_cast<const u32x4*>(sR + (wn * 64 + ti * 16 + l16) * 64 + lq * 16));
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
      for (int tj = 0; tj < 8; ++tj) acc[ti][tj] = E::mfma16(rf[ti], lf[tj], acc[ti][tj]);
    if (a.c != 1.0f) {
#pragma unroll
      for (int ti = 0; ti < 4; ++ti)
#pragma unroll
        for (int tj = 0; tj < 8; ++tj)
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[ti][tj][v] *= a.c;
    }
  }
  asm volatile("" ::: "memory");  // ... and before the waits and barrier below
  __builtin_amdgcn_sched_barrier(0);
  if (nk > 1) __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8): step 1 may stay in flight
  else __builtin_amdgcn_s_waitcnt(0x0F70);
  // every wave has read L and R (the barrier orders those reads before step 0's copies of step 2
  // into their stage)
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  // no scalar loads pending at the loop entry, so the waits at its head count LDS reads only
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_sched_barrier(0);
  read_w(wbase(0), 0, w0);
#pragma unroll
  for (int tj = 0; tj < 8; ++tj) x[tj] = read_x(abase(0), 0, tj);
  // Steps 0 .. nk-2 (the last one is peeled). Step kt:
  // - sub-step 0 reads sub-step 1's fragments and issues the activation copies of step kt+2 (one
  //   per eight MFMAs) into the activation stage of step kt-1, free since the barrier of step kt-1;
  // - the barrier: step kt+1 has landed, the four newer activation copies may stay in flight;
  // - sub-step 1 reads step kt+1's sub-step-0 fragments and issues the weight copies of step kt+2
  //   into the weight stage of step kt, free since this barrier.
  // The L2-to-LDS path moves about 64 bytes per clock per CU; eight copies in one sub-step stall
  // their issue, four per sub-step do not. Step nk-2 (LR) has no step nk to copy: its copies go
  // through a zero-record descriptor (they move no memory and write zeros into stages no wave
  // reads any more), so every step's waits count the same copies.
  //
  // Waves w and w + 4 share a SIMD. With equal priorities the older one (w < 4) wins every MFMA
  // issue slot it wants, runs a whole sub-step ahead, and the younger one then finishes its
  // sub-step 0 alone, where one wave keeps the pipe only about three quarters busy. The younger
  // wave therefore takes the higher priority for sub-step 1 and gives it up for sub-step 0, so
  // both reach the barrier together.
  auto kstep = [&](int kt, auto lr) {
    constexpr bool LR = decltype(lr)::value;
    if (w >= 4) __builtin_amdgcn_s_setprio(0);
    const uint8_t* sa = abase(kt);
    const uint8_t* sw = wbase(kt);
#pragma unroll
    for (int tj = 0; tj < 8; ++tj) {
      mfma4(w0, x[tj], tj);
      __builtin_amdgcn_sched_barrier(0);
      x[tj] = read_x(sa, 1, tj);
      if (tj == 0) read_w(sw, 1, w1);
      if (tj & 1) {
        if constexpr (LR) dma16(rnone, 0u, 0u, abase(kt + 2) + (w * 4 + (tj >> 1)) * 1024);
        else issue_act(kt + 2, tj >> 1);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // lgkmcnt(7): the weight fragments of this step have been read (the weight copies issued
    // after the barrier overwrite their stage). The seven activation reads issued after them may
    // still be queued at the LDS, which serves requests in order: the activation copies into that
    // stage are issued a full sub-step after the barrier and land a memory latency later.
    __builtin_amdgcn_s_waitcnt(0xC77F);
    __builtin_amdgcn_s_waitcnt(0x0F74);  // vmcnt(4): step kt+1 has landed
    __builtin_amdgcn_s_barrier();
    if (w >= 4) __builtin_amdgcn_s_setprio(1);
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* san = abase(kt + 1);
    const uint8_t* swn = wbase(kt + 1);
    read_w(swn, 0, w0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int tj = 0; tj < 8; ++tj) {
      mfma4(w1, x[tj], tj);
      __builtin_amdgcn_sched_barrier(0);
      x[tj] = read_x(san, 0, tj);
      if (tj & 1) {
        if constexpr (LR) dma16(rnone, 0u, 0u, wbase(kt + 2) + (w * 4 + (tj >> 1)) * 1024);
        else issue_w(kt + 2, tj >> 1);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  for (int kt = 0; kt + 2 < nk; ++kt) kstep(kt, std::false_type{});
  if (nk > 1) kstep(nk - 2, std::true_type{});
  if (w >= 4) __builtin_amdgcn_s_setprio(0);
  {
    const uint8_t* sa = abase(nk - 1);
    read_w(wbase(nk - 1), 1, w1);
#pragma unroll
    for (int tj = 0; tj < 8; ++tj) {
      mfma4(w0, x[tj], tj);
      x[tj] = read_x(sa, 1, tj);
    }
#pragma unroll
    for (int tj = 0; tj < 8; ++tj) mfma4(w1, x[tj], tj);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // the last zero-record copies have landed

  // epilogue: bias and one rounding per output (acc + bias, the LoRA term already in acc; ranks
  // above 32 add c lor here, their up-projection on MFMA with k = 32 per instruction and lanes
  // past the rank supplying zeros); each wave stages its 128 x 64 outputs in LDS and stores them
  // as 128-byte row segments. The staging tile's rows of 512 bytes (16-byte chunks XOR-swizzled
  // by row) fill, 64 rows at a time, four of the five stages (all copies have landed).
  __syncthreads();
  const int lrs = nk % 3;
  auto srow = [&](int r) { const int q = r >> 6; return smem + (q < lrs ? q : q + 1) * ACT + (r & 63) * 512; };
  const int nsteps = (rp + 31) >> 5;
  // bias of this lane's four output columns of each 16-column tile, loaded together
  u32x2 braw[4];
#pragma unroll
  for (int ti = 0; ti < 4; ++ti) {
    const int64_t nb = n0 + wn * 64 + ti * 16 + lq * 4;
    braw[ti] = u32x2{0u, 0u};
    if (a.bias != nullptr && nb < Ncols) braw[ti] = *reinterpret_cast<const u32x2*>(a.bias + nb);
  }

  // acc (+ c lor with UL) + bias, rounded once, into the staging tile
  auto finish = [&](int ti, const f32x4* lor, auto ul) {
    constexpr bool UL = decltype(ul)::value;
    const int nloc = wn * 64 + ti * 16 + lq * 4;  // this lane's four output columns
    if constexpr (SPLIT) {
      // split partial: acc (+ c lor in split 0), f32, 16 bytes per lane and token
#pragma unroll
      for (int tj = 0; tj < 8; ++tj) {
        const int64_t m = m0 + wm * 128 + tj * 16 + l16, n = n0 + nloc;
        f32x4 o = acc[ti][tj];
        if (UL && lora) {
#pragma unroll
          for (int v = 0; v < 4; ++v) o[v] += a.c * lor[tj][v];
        }
        if (m < M && n < Ncols) *reinterpret_cast<f32x4*>(a.part + ((int64_t)split * M + m) * Ncols + n) = o;
      }
      return;
    }
    const float bs[4] = {E::lo(braw[ti][0]), E::hi(braw[ti][0]), E::lo(braw[ti][1]), E::hi(braw[ti][1])};
#pragma unroll
    for (int tj = 0; tj < 8; ++tj) {
      const int mloc = wm * 128 + tj * 16 + l16;
      float o[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) o[v] = UL ? acc[ti][tj][v] + a.c * lor[tj][v] + bs[v] : acc[ti][tj][v] + bs[v];
      const u32x2 pk = {E::pack2_fast(o[0], o[1]), E::pack2_fast(o[2], o[3])};
      const int chunk = (nloc >> 3) ^ (mloc & 31);
      *reinterpret_cast<u32x2*>(srow(mloc) + chunk * 16 + (nloc & 7) * 2) = pk;
    }
  };
  if (lr_lds || !lora) {
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) finish(ti, nullptr, std::false_type{});
  } else {
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      f32x4 lor[8];
#pragma unroll
      for (int tj = 0; tj < 8; ++tj)
#pragma unroll
        for (int v = 0; v < 4; ++v) lor[tj][v] = 0.0f;
      if (lora) {
        const int64_t nrow = n0 + wn * 64 + ti * 16 + l16;  // A-operand row of this lane
        const int64_t nrc = nrow < Ncols ? nrow : Ncols - 1;
        for (int s = 0; s < nsteps; ++s) {
          const int k0 = s * 32 + lq * 8;
          u32x4 rv = {0, 0, 0, 0};
          if (k0 < rp && nrow < Ncols) rv = *reinterpret_cast<const u32x4*>(a.R + nrc * rp + k0);
#pragma unroll
          for (int tj = 0; tj < 8; ++tj) {
            const int64_t m = m0 + wm * 128 + tj * 16 + l16;
            u32x4 lv = {0, 0, 0, 0};
            if (k0 < rp && m < M) lv = *reinterpret_cast<const u32x4*>(a.L + m * rp + k0);
            lor[tj] = E::mfma16(E::as8(rv), E::as8(lv), lor[tj]);
          }
        }
      }
      finish(ti, lor, std::true_type{});
    }
  }
  if constexpr (SPLIT) return;  // the partials went straight to global memory
  // each wave stores the region it staged itself (128 rows x 64 columns: 128-byte row segments,
  // whole cache lines), so no barrier waits for the other waves
  if constexpr (EPI == 2) {
    // the GELU inputs of the 16 row segments this lane stores, all loaded at once once the
    // accumulators are dead (earlier, with them live, the registers spill), then the products
    u32x4 gv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = wm * 128 + 8 * i + (lane >> 3), c = wn * 8 + (lane & 7);
      const int64_t m = m0 + row, n = n0 + c * 8;
      gv[i] = u32x4{0u, 0u, 0u, 0u};
      if (m < M && n < Ncols) gv[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.gx + m * Ncols + n));
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's staging writes are done
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = wm * 128 + 8 * i + (lane >> 3), c = wn * 8 + (lane & 7);
      const int64_t m = m0 + row, n = n0 + c * 8;
      if (m < M && n < Ncols) {
        const u32x4 d = *reinterpret_cast<const u32x4*>(srow(row) + ((c ^ (row & 31)) << 4));
        u32x4 o;
#pragma unroll
        for (int k = 0; k < 4; ++k)
          o[k] = E::bits(E::lo(d[k]) * gelu_grad_f(E::lo(gv[i][k]))) |
                 (E::bits(E::hi(d[k]) * gelu_grad_f(E::hi(gv[i][k]))) << 16);
        __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(a.out + m * Ncols + n));
      }
    }
    return;
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's staging writes are done
  // nontemporal stores: every CU stores its tile at about the same time at the end of a round
  // (1536-deep GEMMs on 32760 tokens: 1.3% faster over the six Wan-1.3B projections; the
  // 5120-deep ones and a chain whose next projection reads the output unchanged)
#pragma unroll 4
  for (int i = 0; i < 16; ++i) {
    const int row = wm * 128 + 8 * i + (lane >> 3), c = wn * 8 + (lane & 7);
    const int64_t m = m0 + row, n = n0 + c * 8;
    if (m < M && n < Ncols) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(srow(row) + ((c ^ (row & 31)) << 4));
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(a.out + m * Ncols + n));
      if constexpr (EPI == 1) {
        u32x4 gv;
#pragma unroll
        for (int k = 0; k < 4; ++k)
          gv[k] = E::bits(gelu_f(E::lo(v[k]))) | (E::bits(gelu_f(E::hi(v[k]))) << 16);
        __builtin_nontemporal_store(gv, reinterpret_cast<u32x4*>(a.gout + m * Ncols + n));
      }
    }
  }
}

// out = rnd(sum over splits of part[sp][m][n] (split order) + bias[n]) for the split bf16 GEMM;
// four outputs per thread and step, grid-stride
template <int ELT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, int ks,
                                                            int64_t M, int64_t Ncols,
                                                            const uint16_t* __restrict__ bias,
                                                            uint16_t* __restrict__ out) {
  using E = Elt<ELT>;
  const int64_t n4 = Ncols / 4, total = M * n4, plane = M * Ncols;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += step) {
    const int64_t m = i / n4, n = (i - m * n4) * 4;
    const float* p = part + m * Ncols + n;
    f32x4 sum = *reinterpret_cast<const f32x4*>(p);
    for (int sp = 1; sp < ks; ++sp) sum += *reinterpret_cast<const f32x4*>(p + sp * plane);
    if (bias != nullptr) {
      const u32x2 b = *reinterpret_cast<const u32x2*>(bias + n);
      sum[0] += E::lo(b[0]); sum[1] += E::hi(b[0]); sum[2] += E::lo(b[1]); sum[3] += E::hi(b[1]);
    }
    *reinterpret_cast<u32x2*>(out + m * Ncols + n) = u32x2{E::pack2_fast(sum[0], sum[1]), E::pack2_fast(sum[2], sum[3])};
  }
}

static int launch_splitk_reduce(int elt, const GemmArgs& a, hipStream_t st) {
  const int64_t n4 = a.M * (a.Ncols / 4);
  const unsigned grid = (unsigned)(ceil_div(n4, 256) < 4096 ? ceil_div(n4, 256) : 4096);
  { TraceScope _ts(st, "splitk_reduce_kernel");
    with_elt(elt, [&](auto e) {
      splitk_reduce_kernel<decltype(e)::value><<<grid, 256, 0, st>>>(a.part, a.ksplit, a.M, a.Ncols, a.bias, a.out);
    }); }
  return check_launch("splitk_reduce_kernel");
}

int bfgemm_splits(int64_t M, int64_t Ncols, int64_t Kred) {
  const int64_t tiles = ceil_div(M, bfg::BM) * ceil_div(Ncols, bfg::BN);
  if (tiles <= 0 || tiles >= 128) return 1;
  int64_t s = (256 + tiles / 2) / tiles;
  const int64_t nk = Kred / bfg::BK;
  if (s > nk / 4) s = nk / 4;
  if (s > 16) s = 16;
  return s < 2 ? 1 : (int)s;
}

bool bfgemm_fuses_gelu(const GemmArgs& a) {
  const auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  return a.ksplit <= 1 && a.Ncols % 8 == 0 && al(a.out) && al(a.gx);
}

bool bfgemm_fuses_gelu_fwd(const GemmArgs& a) {
  const auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  return a.ksplit <= 1 && a.Ncols % 8 == 0 && al(a.out) && al(a.gout);
}

bool bfgemm_supported(int64_t M, int64_t Ncols, int64_t Kred) {
  (void)M;  // any token count: launch_bfgemm splits the tokens into chunks (below)
  return Kred % bfg::BK == 0 && Ncols % 16 == 0 && Ncols * Kred * 2 < ((int64_t)1 << 31);
}

int launch_bfgemm(int mode, int elt, const GemmArgs& a, const uint16_t* wd, hipStream_t st) {
  if (!bfgemm_supported(a.M, a.Ncols, a.Kred))
    return fail(REELS_HIP_EINVAL, "bfgemm: shape not supported (reduction not a multiple of 64 or operands of 2 GiB or more)");
  static std::once_flag once;
  static hipError_t attr_err = hipSuccess;
  std::call_once(once, [&] {
    const void* ks[] = {(const void*)bfgemm_kernel<REELS_HIP_BF16, false>, (const void*)bfgemm_kernel<REELS_HIP_F16, false>,
                        (const void*)bfgemm_kernel<REELS_HIP_BF16, true>, (const void*)bfgemm_kernel<REELS_HIP_F16, true>,
                        (const void*)bfgemm_kernel<REELS_HIP_BF16, false, 2>, (const void*)bfgemm_kernel<REELS_HIP_F16, false, 2>,
                        (const void*)bfgemm_kernel<REELS_HIP_BF16, false, 1>, (const void*)bfgemm_kernel<REELS_HIP_F16, false, 1>};
    for (const void* k : ks)
      if (attr_err == hipSuccess) attr_err = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, bfg::LDS);
  });
  if (attr_err != hipSuccess)
    return fail(REELS_HIP_EHIP, std::string("bfgemm: hipFuncSetAttribute: ") + hipGetErrorString(attr_err));
  // The activation copies address their buffer with 32-bit offsets: token counts whose
  // activations reach 2 GiB run as consecutive launches over token chunks (multiples of the
  // 256-token tile) with the activation, output and L pointers advanced.
  const int64_t chunk = ((((int64_t)1 << 31) - 1) / (a.Kred * 2)) / bfg::BM * bfg::BM;
  if (a.gx && !bfgemm_fuses_gelu(a))
    return fail(REELS_HIP_EINVAL, "bfgemm: the GELU epilogue needs the unsplit kernel and 16-byte aligned buffers");
  if (a.gout && (a.gx || !bfgemm_fuses_gelu_fwd(a)))
    return fail(REELS_HIP_EINVAL, "bfgemm: the forward GELU epilogue needs the unsplit kernel, 16-byte aligned buffers and no pullback");
  if (a.ksplit > 1) {
    // split reduction: few tiles (one chunk of tokens), partials in a.part, then the reduction pass
    if (a.M > chunk || a.part == nullptr || a.Ncols % 4 != 0)
      return fail(REELS_HIP_EINVAL, "bfgemm: split reduction needs one token chunk, a partials buffer and Ncols % 4 == 0");
    const int tn = (int)ceil_div(a.Ncols, bfg::BN), tm = (int)ceil_div(a.M, bfg::BM);
    { TraceScope _ts(st, mode == 0 ? "bfgemm_kernel<0>" : "bfgemm_kernel<1>");
      with_elt(elt, [&](auto e) {
        bfgemm_kernel<decltype(e)::value, true><<<tn * tm * a.ksplit, bfg::NT, bfg::LDS, st>>>(a, wd, tn, tm);
      }); }
    if (int rc = check_launch("bfgemm_kernel")) return rc;
    return launch_splitk_reduce(elt, a, st);
  }
  for (int64_t m0 = 0; m0 < a.M; m0 += chunk) {
    GemmArgs c = a;
    c.M = (a.M - m0 < chunk) ? a.M - m0 : chunk;
    c.act = a.act + m0 * a.Kred;
    c.out = a.out + m0 * a.Ncols;
    if (a.L) c.L = a.L + m0 * a.rp;
    if (a.gx) c.gx = a.gx + m0 * a.Ncols;
    if (a.gout) c.gout = a.gout + m0 * a.Ncols;
    const int tn = (int)ceil_div(c.Ncols, bfg::BN), tm = (int)ceil_div(c.M, bfg::BM);
    { TraceScope _ts(st, mode == 0 ? "bfgemm_kernel<0>" : "bfgemm_kernel<1>");
      with_elt(elt, [&](auto e) {
        constexpr int EL = decltype(e)::value;
        if (c.gx) bfgemm_kernel<EL, false, 2><<<tn * tm, bfg::NT, bfg::LDS, st>>>(c, wd, tn, tm);
        else if (c.gout) bfgemm_kernel<EL, false, 1><<<tn * tm, bfg::NT, bfg::LDS, st>>>(c, wd, tn, tm);
        else bfgemm_kernel<EL, false><<<tn * tm, bfg::NT, bfg::LDS, st>>>(c, wd, tn, tm);
      }); }
    if (int rc = check_launch("bfgemm_kernel")) return rc;
  }
  return REELS_HIP_OK;
}

int launch_i8gemm(int mode, int elt, const GemmArgs& a, hipStream_t st) {
  using namespace gemm;
  // the main kernel needs a reduction in whole 64-steps and 32-bit buffer offsets
  const int64_t act_bytes = a.M * a.Kred * 2, q_bytes = a.Ncols * a.Kred;
  // the DX weight scale (f16 path) is applied only by the register-staged kernel
  const bool v3 = (a.Kred % gemm3::BK == 0) && act_bytes < ((int64_t)1 << 31) &&
                  q_bytes < ((int64_t)1 << 31) && (a.ldq * gemm3::BK) < ((int64_t)1 << 31) &&
                  !(mode == 1 && a.redscale != nullptr);
  static std::once_flag once;
  static hipError_t attr_err = hipSuccess;
  std::call_once(once, [&] {
    const int l1 = 2 * STAGE_BYTES, l2 = gemm3::NSTAGE * gemm3::STAGE;
    const void* k1[] = {(const void*)i8gemm_kernel<0, REELS_HIP_BF16>, (const void*)i8gemm_kernel<1, REELS_HIP_BF16>,
                        (const void*)i8gemm_kernel<0, REELS_HIP_F16>, (const void*)i8gemm_kernel<1, REELS_HIP_F16>};
    const void* k3[] = {(const void*)i8gemm_v3_kernel<0, REELS_HIP_BF16, false>, (const void*)i8gemm_v3_kernel<1, REELS_HIP_BF16, false>,
                        (const void*)i8gemm_v3_kernel<0, REELS_HIP_F16, false>, (const void*)i8gemm_v3_kernel<1, REELS_HIP_F16, false>,
                        (const void*)i8gemm_v3_kernel<0, REELS_HIP_BF16, true>, (const void*)i8gemm_v3_kernel<1, REELS_HIP_BF16, true>,
                        (const void*)i8gemm_v3_kernel<0, REELS_HIP_F16, true>, (const void*)i8gemm_v3_kernel<1, REELS_HIP_F16, true>};
    for (const void* k : k1)
      if (attr_err == hipSuccess) attr_err = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, l1);
    for (const void* k : k3)
      if (attr_err == hipSuccess) attr_err = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, l2);
  });
  if (attr_err != hipSuccess)
    return fail(REELS_HIP_EHIP, std::string("i8gemm: hipFuncSetAttribute: ") + hipGetErrorString(attr_err));
  if (v3 && a.ksplit > 1) {
    // split reduction (few tiles): partials in a.part, then the reduction pass of the bf16 GEMM
    if (a.part == nullptr || a.Ncols % 4 != 0)
      return fail(REELS_HIP_EINVAL, "i8gemm: split reduction needs a partials buffer and Ncols % 4 == 0");
    const int tn = (int)ceil_div(a.Ncols, gemm3::BN), tm = (int)ceil_div(a.M, gemm3::BM);
    const size_t lds = gemm3::NSTAGE * gemm3::STAGE;
    {
      TraceScope _ts(st, mode == 0 ? "i8gemm_v3_kernel<0>" : "i8gemm_v3_kernel<1>");
      with_elt(elt, [&](auto e) {
        constexpr int T = decltype(e)::value;
        if (mode == 0) i8gemm_v3_kernel<0, T, true><<<tn * tm * a.ksplit, gemm3::NT, lds, st>>>(a, tn, tm);
        else i8gemm_v3_kernel<1, T, true><<<tn * tm * a.ksplit, gemm3::NT, lds, st>>>(a, tn, tm);
      });
    }
    if (int rc = check_launch(mode == 0 ? "i8gemm_v3_kernel<FWD>" : "i8gemm_v3_kernel<DX>")) return rc;
    return launch_splitk_reduce(elt, a, st);
  }
  if (v3) {
    const int tn = (int)ceil_div(a.Ncols, gemm3::BN), tm = (int)ceil_div(a.M, gemm3::BM);
    const size_t lds = gemm3::NSTAGE * gemm3::STAGE;
    TraceScope _ts(st, mode == 0 ? "i8gemm_v3_kernel<0>" : "i8gemm_v3_kernel<1>");
    with_elt(elt, [&](auto e) {
      constexpr int T = decltype(e)::value;
      if (mode == 0) i8gemm_v3_kernel<0, T, false><<<tn * tm, gemm3::NT, lds, st>>>(a, tn, tm);
      else i8gemm_v3_kernel<1, T, false><<<tn * tm, gemm3::NT, lds, st>>>(a, tn, tm);
    });
  } else {
    dim3 grid((unsigned)ceil_div(a.Ncols, BN), (unsigned)ceil_div(a.M, BM));
    const size_t lds = 2 * STAGE_BYTES;
    TraceScope _ts(st, mode == 0 ? "i8gemm_kernel<0>" : "i8gemm_kernel<1>");
    with_elt(elt, [&](auto e) {
      constexpr int T = decltype(e)::value;
      if (mode == 0) i8gemm_kernel<0, T><<<grid, NT, lds, st>>>(a);
      else i8gemm_kernel<1, T><<<grid, NT, lds, st>>>(a);
    });
  }
  const char* what = v3 ? (mode == 0 ? "i8gemm_v3_kernel<FWD>" : "i8gemm_v3_kernel<DX>")
                        : (mode == 0 ? "i8gemm_kernel<FWD>" : "i8gemm_kernel<DX>");
  return check_launch(what);
}

}  // namespace reels
