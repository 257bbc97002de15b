// Few-token path of the int8 LoRA linear: a large frozen weight against at most a few hundred
// tokens, e.g. the cross-attention K/V projections over 77-512 text tokens
// (src/models/wan21/transformer.jl:185-188, I2V 225-235, through quantization.jl:73-76). There
// the weight stream is the whole cost, so the int8 codes are read once, coalesced, straight from
// HBM into registers (no bf16 copy of the weight) and converted there; the tokens sit on the
// 16-wide side of v_mfma_f32_16x16x32 (77 tokens = 2 blocks of 3 tiles of 16).
//
//   skinny_kernel      block (o-block of 64 output rows, reduction split sp, token block tb of up
//                      to 64 tokens): each of its 4 waves takes a quarter of the split's 64-wide
//                      reduction chunks, accumulating 64 rows x 16T tokens; the 4 wave partials are summed in LDS in
//                      wave order and written as f32 partials part[sp][m][col]. Blocks past the
//                      output rows compute the adapter's rank-r projection partials (h = x A in
//                      the forward, u = dy B^T for dX) into the columns past Ncols.
//   skinny_epilogue    sums the splits in split order, rounds h (u) once to the element type and
//                      writes out = rnd(scale * sum + c * h R + bias).
//
// FWD: out[m][n] = rnd(s[n] sum_k x[m][k] q[n][k] + c sum_j h[m][j] B[j][n] + bias[n]),
//      h = rnd(x A): the int8 path's formula (the scale on the f32 sum).
// DX:  out[m][k] = rnd(sum_n dy[m][n] W[n][k] + c sum_j u[m][j] A[k][j]), u = rnd(dy B^T), with
//      W = bf16(fl32(q[n][k] s[n])) for bf16 (the weight of the large-token bf16 path) and
//      f16(q[n][k] f16(s[n])) for f16 (the reference's binary16 weight, quantization.jl:61-62),
//      made from the codes in registers; the weight columns of a reduction chunk reach the MFMA
//      through ds_read_b64_tr_b8 from a per-wave LDS tile.
// Deterministic: fixed wave order, fixed split order, no atomics.
#include "i8gemm.h"

#include <mutex>

namespace reels {

namespace sk {
constexpr int NB = 64;       // output rows per block: 4 MFMA tiles of 16
constexpr int NBL = 32;      // adapter rows per adapter block: 2 MFMA tiles of 16
constexpr int KC = 64;       // reduction chunk
constexpr int MAXT = 5;      // token tiles of 16 per block (80 tokens)
constexpr int STAGE = 4096;  // per-wave LDS staging (DX weight tile, FWD adapter chunk: 4 KiB each)
}  // namespace sk

struct SkArgs {
  const uint16_t* act;  // [M][Kred] 16-bit: x (FWD) or dy (DX)
  const int8_t* q;      // codes [N][K], row stride ldq
  const float* s;       // DX: scale of the reduction index n
  const uint16_t* lw;   // adapter operand: FWD A [Kred][rp] (zeros past r), DX B [r][Kred]
  float* part;          // [S][M][ldp] f32 partials
  int64_t M, Kred, Ncols, ldq;
  int r, rp, S, ldp, nblk;  // nblk: output blocks; adapter blocks follow
  int tb, blocks;           // token blocks; all blocks of the launch
  int blk0;                 // first block index (nblk: the adapter blocks alone)
};

// Block b runs on XCD b % 8. Each XCD takes a contiguous range of the logical order, which walks
// the token blocks of one (row block, split) first: the blocks that read the same weight rows
// run on one XCD, close in time, and share them through its L2.
struct SkBlock {
  int blk, sp, tb;
};
__device__ __forceinline__ SkBlock skinny_decode(const SkArgs& a) {
  const int b = blockIdx.x, xcd = b & 7, idx = b >> 3;
  const int per = a.blocks >> 3, rem = a.blocks & 7;
  const int logical = xcd * per + (xcd < rem ? xcd : rem) + idx;
  SkBlock d;
  d.tb = logical % a.tb;
  const int rest = logical / a.tb;
  d.sp = rest % a.S;
  d.blk = a.blk0 + rest / a.S;
  return d;
}

static constexpr int skinny_lds(int T) {
  return (4 * 4 * T * 4 * 64 * 4) > 4 * sk::STAGE ? (4 * 4 * T * 4 * 64 * 4) : 4 * sk::STAGE;
}

// One block's work; LORA: an adapter block (rows j of A^T in the forward, of B for dX) rather than
// an output block of the int8 weight.
template <int T, int MODE, int ELT, bool LORA>
__device__ __forceinline__ void skinny_block(const SkArgs& a, const SkBlock& d, uint8_t* smem) {
  using E = Elt<ELT>;
  typedef typename E::v8 V8;
  constexpr bool lora = LORA;
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  const int blk = d.blk, sp = d.sp;
  const int64_t tok0 = (int64_t)d.tb * (16 * T);
  constexpr int NI = lora ? 2 : 4;  // MFMA row tiles of 16
  const int64_t o0 = lora ? (int64_t)(blk - a.nblk) * sk::NBL : (int64_t)blk * sk::NB;
  const int nc = (int)(a.Kred / sk::KC);
  const int c0 = (int)((int64_t)sp * nc / a.S), c1 = (int)((int64_t)(sp + 1) * nc / a.S);

  // Descriptors: reads past num_records return zeros (tokens past M, weight rows past the
  // matrix, adapter rows past the rank, chunks past the split).
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.act), (short)0, (int)(a.M * a.Kred * 2), 0x00020000);
  const int64_t wbytes = lora ? (MODE == 0 ? a.Kred * a.rp * 2 : (int64_t)a.r * a.Kred * 2)
                              : (MODE == 0 ? a.Ncols * a.ldq : a.Kred * a.ldq);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(lora ? (const void*)a.lw : (const void*)a.q), (short)0, (int)wbytes,
      0x00020000);

  // FWD output blocks take the 16 bytes of a row at k = 16 g + (0..15) of the chunk and feed
  // MFMA step e with k = 16 g + 8 e + (0..7); every other operand uses k = 32 e + 8 g + (0..7).
  // Both operands of one product always use the same assignment.
  //
  // Per-lane offsets are fixed for the whole walk; the chunk's advance is uniform and goes in
  // the loads' scalar offset, so a chunk costs no vector address arithmetic. A lane whose row lies
  // past its operand (tokens past M, adapter rows past the rank) gets an offset past the
  // descriptor and reads zeros.
  constexpr uint32_t OOB = 0x80000000u;
  constexpr bool perm = MODE == 0 && !lora;
  uint32_t vx[T][2];
#pragma unroll
  for (int tt = 0; tt < T; ++tt)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int64_t tok = tok0 + 16 * tt + l16;
      const int64_t k = perm ? 16 * g + 8 * e : 32 * e + 8 * g;
      vx[tt][e] = tok < a.M ? (uint32_t)((tok * a.Kred + k) * 2) : OOB;
    }
  constexpr int NWL = 4;  // weight / adapter loads per chunk
  constexpr int NSC = (MODE == 1 && !lora) ? 4 : 1;
  uint32_t vw[NWL];
  uint32_t wstep;  // bytes per chunk along the reduction
#pragma unroll
  for (int i = 0; i < NWL; ++i) {
    if (!lora && MODE == 0) {         // row o0 + 16 i + l16, 16 bytes at 16 g
      vw[i] = (uint32_t)((o0 + 16 * i + l16) * a.ldq + 16 * g);
    } else if (!lora) {               // DX tile [64 n][64 k]: row 16 i + lane/4, 16 bytes at 16 (lane % 4)
      vw[i] = (uint32_t)((16 * i + (lane >> 2)) * a.ldq + o0 + 16 * (lane & 3));
    } else if (MODE == 0) {           // A chunk [64 k][32 j] bf16: row 16 i + lane/4, 8 columns at 8 (lane % 4)
      const int64_t j = o0 + 8 * (lane & 3);
      vw[i] = j < a.rp ? (uint32_t)(((16 * i + (lane >> 2)) * a.rp + j) * 2) : OOB;
    } else {                          // B rows j = o0 + 16 (i / 2) + l16, 8 values at 32 (i % 2) + 8 g
      const int64_t j = o0 + 16 * (i >> 1) + l16;
      vw[i] = j < a.r ? (uint32_t)((j * a.Kred + 32 * (i & 1) + 8 * g) * 2) : OOB;
    }
  }
  wstep = (!lora && MODE == 0) ? (uint32_t)sk::KC
        : !lora                ? (uint32_t)(sk::KC * a.ldq)
        : MODE == 0            ? (uint32_t)(sk::KC * a.rp * 2)
                               : (uint32_t)(sk::KC * 2);

  struct Stage {
    u32x4 wq[NWL];
    u32x4 x[T][2];
    f32x4 sc[NSC];  // DX: s[n] for n = 32 e + 8 g + (0..7), [2 e + half]
  };
  Stage st0, st1;
  // valid = false (a step past the wave's run): every offset of the step moves past its
  // descriptor, so the step reads zeros and adds nothing (no branch around the loads or the
  // multiply, which keeps the compiler's waits exact)
  auto load = [&](int c, bool valid, Stage& s) {
    const uint32_t sw = (uint32_t)c * wstep, sx = (uint32_t)c * (uint32_t)(sk::KC * 2);
#pragma unroll
    for (int i = 0; i < NWL; ++i)
      s.wq[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, valid ? vw[i] : OOB, sw, !lora ? 2 : 0));
#pragma unroll
    for (int tt = 0; tt < T; ++tt)
#pragma unroll
      for (int e = 0; e < 2; ++e)
        s.x[tt][e] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, valid ? vx[tt][e] : OOB, sx, 0));
    if constexpr (MODE == 1 && !lora) {  // the scales of a zero step multiply zeros
      const float* sp8 = a.s + (int64_t)c * sk::KC + 8 * g;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        s.sc[2 * e] = *reinterpret_cast<const f32x4*>(sp8 + 32 * e);
        s.sc[2 * e + 1] = *reinterpret_cast<const f32x4*>(sp8 + 32 * e + 4);
      }
    }
  };

  f32x4 acc[NI][T];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int tt = 0; tt < T; ++tt) acc[i][tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  uint8_t* wst = smem + w * sk::STAGE;  // this wave's staging area
  auto compute = [&](const Stage& s) {
    V8 af[NI][2];
    if constexpr (!lora && MODE == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        af[i][0] = E::from_i8x8(s.wq[i][0], s.wq[i][1]);
        af[i][1] = E::from_i8x8(s.wq[i][2], s.wq[i][3]);
      }
    } else if constexpr (!lora) {
      // the DX tile to LDS as loaded ([64 n][64 k], 64-byte rows), then per 16-k tile i and step
      // e the transposed read: providing lane p of a 16-lane group addresses row
      // 32 e + 8 g + p / 2, columns 16 i + 8 (p % 2) .. +7; lane l16 receives k = 16 i + l16,
      // n = 32 e + 8 g + (0..7)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<u32x4*>(wst + (16 * i + (lane >> 2)) * 64 + 16 * (lane & 3)) = s.wq[i];
#pragma unroll
      for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint8_t* p = wst + (32 * e + 8 * g + (l16 >> 1)) * 64 + 16 * i + 8 * (l16 & 1);
          const i32x2 v = __builtin_amdgcn_ds_read_tr8_b64_v2i32(LDS_PTR(i32x2, p));
          af[i][e] = E::from_i8x8((uint32_t)v[0], (uint32_t)v[1]);
          const f32x4 s0 = s.sc[2 * e], s1 = s.sc[2 * e + 1];  // s[n] for this lane's 8 n
          if constexpr (ELT == REELS_HIP_F16) {  // Float16(q) * Float16(s[n])
            const u32x4 s16 = {E::pack2(s0[0], s0[1]), E::pack2(s0[2], s0[3]),
                               E::pack2(s1[0], s1[1]), E::pack2(s1[2], s1[3])};
            af[i][e] = E::scale8(af[i][e], s16);
          } else {  // bf16(fl32(q * s[n])), the dequantized weight of the bf16 path
            const u32x4 qv = __builtin_bit_cast(u32x4, af[i][e]);
            const u32x4 o = {E::pack2_fast(E::lo(qv[0]) * s0[0], E::hi(qv[0]) * s0[1]),
                             E::pack2_fast(E::lo(qv[1]) * s0[2], E::hi(qv[1]) * s0[3]),
                             E::pack2_fast(E::lo(qv[2]) * s1[0], E::hi(qv[2]) * s1[1]),
                             E::pack2_fast(E::lo(qv[3]) * s1[2], E::hi(qv[3]) * s1[3])};
            af[i][e] = E::as8(o);
          }
        }
    } else if constexpr (MODE == 0) {
      // the A chunk [64 k][32 j] to LDS (64-byte rows); row tile i (j = 16 i + l16), step e:
      // two transposed 16-bit reads give k = 32 e + 8 g + 4 h + (0..3), h = 0, 1: providing lane
      // p addresses row 32 e + 8 g + 4 h + p / 4, columns 16 i + 4 (p % 4) .. +3
#pragma unroll
      for (int i = 0; i < NWL; ++i)
        *reinterpret_cast<u32x4*>(wst + (16 * i + (lane >> 2)) * 64 + 16 * (lane & 3)) = s.wq[i];
#pragma unroll
      for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          u32x4 v;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint8_t* p = wst + (32 * e + 8 * g + 4 * h + (l16 >> 2)) * 64 +
                               2 * (16 * i + 4 * (l16 & 3));
            const i16x4 r4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(i16x4, p));
            v[2 * h] = (uint16_t)r4[0] | ((uint32_t)(uint16_t)r4[1] << 16);
            v[2 * h + 1] = (uint16_t)r4[2] | ((uint32_t)(uint16_t)r4[3] << 16);
          }
          af[i][e] = E::as8(v);
        }
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        af[i][0] = E::as8(s.wq[2 * i]);
        af[i][1] = E::as8(s.wq[2 * i + 1]);
      }
    }
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int tt = 0; tt < T; ++tt) {
        const V8 xf = E::as8(s.x[tt][e]);
#pragma unroll
        for (int i = 0; i < NI; ++i) acc[i][tt] = E::mfma16(af[i][e], xf, acc[i][tt]);
      }
  };

  // Wave w takes a contiguous quarter of the split's chunks (each weight row read sequentially)
  // and walks it from a rotation that depends on the logical block: rows of the weight (and of
  // the activations) lie a multiple of 1 KiB apart, so blocks that walked the same k offsets at
  // the same time would pile onto a few memory channels. Two register stages: the copies of step
  // i + 2 are issued while step i is multiplied; steps past the wave's run read zeros (the steps
  // come in pairs).
  const int q = (c1 - c0 + 3) / 4;
  const int wb = c0 + w * q;
  const int nw = (wb + q < c1 ? wb + q : c1) - wb;
  const int rot = nw > 0 ? (int)(((int64_t)blk * 5 + (int64_t)tok0 / 16 * 3) % nw) : 0;
  auto chunk = [&](int i) {
    const int p = rot + i;
    return i < nw ? wb + (p < nw ? p : p - nw) : c0;
  };
  // (scheduling barriers keep each stage's loads together and in program order, so the waits at
  // the loop head only cover the older stage)
  load(chunk(0), 0 < nw, st0);
  __builtin_amdgcn_sched_barrier(0);
  load(chunk(1), 1 < nw, st1);
  __builtin_amdgcn_sched_barrier(0);
  for (int i = 0; i < nw; i += 2) {
    compute(st0);
    __builtin_amdgcn_sched_barrier(0);
    load(chunk(i + 2), i + 2 < nw, st0);
    __builtin_amdgcn_sched_barrier(0);
    compute(st1);
    __builtin_amdgcn_sched_barrier(0);
    load(chunk(i + 3), i + 3 < nw, st1);
    __builtin_amdgcn_sched_barrier(0);
  }

  // the 4 wave partials [i][tt][v][lane] in LDS, summed in wave order
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);
  constexpr int PER = NI * T * 4 * 64;
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int tt = 0; tt < T; ++tt)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[w * PER + ((i * T + tt) * 4 + v) * 64 + lane] = acc[i][tt][v];
  __syncthreads();
  const int64_t limit = lora ? a.rp : a.Ncols;
  const int64_t col0 = lora ? a.Ncols : 0;
  // thread -> (token, 4 consecutive outputs): value (o = 16 i + 4 qd + v, token 16 tt + c) sits at
  // [i][tt][v][16 qd + c] of each wave's block; the 4 waves summed in wave order, stored as 16
  // bytes, so a token's NB outputs go out as one contiguous row segment
  constexpr int QUADS = NI * 4;  // output quads per token
  for (int idx = t; idx < 16 * T * QUADS; idx += 256) {
    const int tl = idx / QUADS, n4 = idx % QUADS;
    const int i = n4 >> 2, qd = n4 & 3, tt = tl >> 4, cc = tl & 15;
    f32x4 o;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int e = ((i * T + tt) * 4 + v) * 64 + 16 * qd + cc;
      o[v] = ((red[e] + red[PER + e]) + red[2 * PER + e]) + red[3 * PER + e];
    }
    const int64_t tok = tok0 + tl, ob = o0 + 4 * n4;
    if (tok < a.M && ob < limit)
      *reinterpret_cast<f32x4*>(a.part + ((int64_t)sp * a.M + tok) * a.ldp + col0 + ob) = o;
  }
}

template <int T, int MODE, int ELT>
__global__ __launch_bounds__(256, 2) void skinny_kernel(SkArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const SkBlock d = skinny_decode(a);
  if (d.blk >= a.nblk) skinny_block<T, MODE, ELT, true>(a, d, smem);
  else skinny_block<T, MODE, ELT, false>(a, d, smem);
}

// out[m][o] = rnd(scale[o] * sum_sp part[sp][m][o] + c * sum_j l[m][j] R(o, j) + bias[o]) with
// l[m][j] = rnd(sum_sp part[sp][m][Ncols + j]) (h in the forward, u for dX); R(o, j) = B[j][o]
// (MODE 0, row stride ldr) or R[o][j] (MODE 1, rows of ldr >= rp elements, zeros past r). One
// output per thread; the split partials and the adapter operand are loaded in independent batches
// (the epilogue is latency-bound: few bytes, many blocks). lsave[m][j] (j < lsave_cols, zeros
// past r) receives l from the blocks of column block 0.
template <int MODE, int ELT>
__global__ __launch_bounds__(256) void skinny_epilogue_kernel(
    const float* __restrict__ part, int S, int64_t M, int64_t Ncols, int ldp, int r, int rp,
    const float* __restrict__ colscale, const uint16_t* __restrict__ R, int64_t ldr,
    const uint16_t* __restrict__ bias, float c, uint16_t* __restrict__ out,
    uint16_t* __restrict__ lsave, int64_t ld_lsave, int lsave_cols) {
  using E = Elt<ELT>;
  extern __shared__ float hl[];  // rp values of l for this token
  const int t = threadIdx.x;
  const int64_t m = blockIdx.y;
  const float* pm = part + m * ldp;
  const int64_t sstride = M * ldp;
  auto split_sum = [&](int64_t col) {  // sum over the splits in split order, 8 loads in flight
    float v = 0.0f;
    for (int s = 0; s < S; s += 8) {
      float p[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) p[u] = s + u < S ? pm[(int64_t)(s + u) * sstride + col] : 0.0f;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (s + u < S) v += p[u];
    }
    return v;
  };
  for (int j = t; j < rp; j += 256) {
    const float v = split_sum(Ncols + j);
    const uint32_t b = j < r ? E::bits(v) : 0u;
    hl[j] = E::to_f32((uint16_t)b);
    if (blockIdx.x == 0 && lsave != nullptr && j < lsave_cols) lsave[m * ld_lsave + j] = (uint16_t)b;
  }
  __syncthreads();
  const int64_t o = (int64_t)blockIdx.x * 256 + t;
  if (out == nullptr || o >= Ncols) return;
  const float acc = split_sum(o);
  float lo = 0.0f;
  if (MODE == 0) {
    for (int j0 = 0; j0 < r; j0 += 16) {
      float b[16];
#pragma unroll
      for (int u = 0; u < 16; ++u)
        b[u] = j0 + u < r ? E::to_f32(R[(int64_t)(j0 + u) * ldr + o]) : 0.0f;
#pragma unroll
      for (int u = 0; u < 16; ++u) lo += hl[j0 + u < rp ? j0 + u : 0] * b[u];
    }
  } else {
    const uint16_t* ro = R + o * ldr;
    for (int j0 = 0; j0 < rp; j0 += 32) {
      u32x4 a4[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        a4[u] = j0 + 8 * u < rp ? *reinterpret_cast<const u32x4*>(ro + j0 + 8 * u) : u32x4{0, 0, 0, 0};
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int j = j0 + 8 * u + 2 * q;
          if (j < rp) lo += hl[j] * E::lo(a4[u][q]) + hl[j + 1] * E::hi(a4[u][q]);
        }
    }
  }
  const float sc = colscale ? colscale[o] * acc : acc;
  const float bs = bias ? E::to_f32(bias[o]) : 0.0f;
  out[m * Ncols + o] = (uint16_t)E::bits(sc + c * lo + bs);
}

bool skinny_supported(int64_t M, int64_t K, int64_t N, int rp) {
  // the reduction in whole 64-chunks, whole 64-row blocks, 32-bit buffer offsets (with room for
  // the token-block overrun), the epilogue's LDS row of l
  return M > 0 && M <= kSkinnyMaxTokens && K % 64 == 0 && N % 64 == 0 &&
         (M + 128) * (K > N ? K : N) * 2 < ((int64_t)1 << 31) && N * K < ((int64_t)1 << 31) &&
         (int64_t)rp * (K > N ? K : N) * 2 < ((int64_t)1 << 31) && rp <= 4096;
}

SkinnyPlan skinny_plan(int64_t M, int64_t Kred, int64_t Ncols, int rp) {
  SkinnyPlan p;
  p.tb = (int)ceil_div(M, 16 * sk::MAXT);
  p.T = (int)ceil_div(ceil_div(M, p.tb), 16);
  const int64_t blocks = (Ncols / sk::NB + ceil_div(rp, sk::NBL)) * p.tb;
  const int64_t nc = Kred / sk::KC;
  // about two blocks per CU, each wave at least one chunk
  int64_t S = (kSkinnyTargetBlocks + blocks / 2) / (blocks > 0 ? blocks : 1);
  if (S > nc / 4) S = nc / 4;
  if (S < 1) S = 1;
  p.S = (int)S;
  return p;
}

size_t skinny_part_bytes(const SkinnyPlan& p, int64_t M, int64_t Ncols, int rp) {
  return (size_t)p.S * (size_t)M * (size_t)(Ncols + rp) * 4;
}

template <int MODE, int ELT, int T>
static hipError_t launch_skinny_t(const SkArgs& a, dim3 grid, hipStream_t st) {
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [] {
    attr = hipFuncSetAttribute((const void*)skinny_kernel<T, MODE, ELT>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, skinny_lds(T));
  });
  if (attr != hipSuccess) return attr;
  skinny_kernel<T, MODE, ELT><<<grid, 256, skinny_lds(T), st>>>(a);
  return hipSuccess;
}

int launch_skinny(int mode, int elt, const SkinnyPlan& p, const uint16_t* act, const int8_t* q,
                  int64_t ldq, const float* s, const uint16_t* lw, float* part, int64_t M,
                  int64_t Kred, int64_t Ncols, int r, int rp, const float* colscale,
                  const uint16_t* R, int64_t ldr, const uint16_t* bias, float c, uint16_t* out,
                  uint16_t* lsave, int64_t ld_lsave, int lsave_cols, hipStream_t st,
                  bool adapter_only) {
  SkArgs a;
  a.act = act; a.q = q; a.s = s; a.lw = lw; a.part = part;
  a.M = M; a.Kred = Kred; a.Ncols = Ncols; a.ldq = ldq;
  a.r = r; a.rp = r > 0 ? rp : 0; a.S = p.S; a.ldp = (int)(Ncols + a.rp);
  a.nblk = (int)(Ncols / sk::NB);
  const int lblk = (int)ceil_div(a.rp, sk::NBL);
  a.tb = p.tb;
  a.blk0 = adapter_only ? a.nblk : 0;
  a.blocks = (adapter_only ? lblk : a.nblk + lblk) * p.S * p.tb;
  const dim3 grid((unsigned)a.blocks);
  hipError_t attr = hipSuccess;
  {
    TraceScope _ts(st, mode == 0 ? "skinny_kernel<0>" : "skinny_kernel<1>");
    with_elt(elt, [&](auto e) {
      constexpr int EL = decltype(e)::value;
      auto go = [&](auto m) {
        constexpr int MD = decltype(m)::value;
        switch (p.T) {
          case 1: attr = launch_skinny_t<MD, EL, 1>(a, grid, st); break;
          case 2: attr = launch_skinny_t<MD, EL, 2>(a, grid, st); break;
          case 3: attr = launch_skinny_t<MD, EL, 3>(a, grid, st); break;
          case 4: attr = launch_skinny_t<MD, EL, 4>(a, grid, st); break;
          default: attr = launch_skinny_t<MD, EL, 5>(a, grid, st); break;
        }
      };
      if (mode == 0) go(std::integral_constant<int, 0>{});
      else go(std::integral_constant<int, 1>{});
    });
  }
  if (attr != hipSuccess)
    return fail(REELS_HIP_EHIP, std::string("skinny_kernel: hipFuncSetAttribute: ") + hipGetErrorString(attr));
  if (int rc = check_launch("skinny_kernel")) return rc;
  {
    TraceScope _ts(st, mode == 0 ? "skinny_epilogue_kernel<0>" : "skinny_epilogue_kernel<1>");
    const dim3 eg(adapter_only ? 1u : (unsigned)ceil_div(Ncols, 256), (unsigned)M);
    const size_t lds = (size_t)(a.rp > 0 ? a.rp : 1) * 4;
    with_elt(elt, [&](auto e) {
      constexpr int EL = decltype(e)::value;
      if (mode == 0)
        skinny_epilogue_kernel<0, EL><<<eg, 256, lds, st>>>(part, p.S, M, Ncols, a.ldp, r, a.rp,
                                                             colscale, R, ldr, bias, c,
                                                             adapter_only ? nullptr : out, lsave,
                                                             ld_lsave, lsave_cols);
      else
        skinny_epilogue_kernel<1, EL><<<eg, 256, lds, st>>>(part, p.S, M, Ncols, a.ldp, r, a.rp,
                                                             colscale, R, ldr, bias, c, out, lsave,
                                                             ld_lsave, lsave_cols);
    });
  }
  return check_launch("skinny_epilogue_kernel");
}

}  // namespace reels
