// Exact scaled dot-product attention with an online softmax: memory_efficient_attention and its
// backward (src/layers/attention.jl:106-221 CPU, 225-371 CUDA), for bf16 / f16 tensors with f32
// arithmetic, head_dim 64 or 128 (f32 tensors and the other head dims up to 128 go to the
// generic kernels of attention_g.hip).
//
// Layouts (row-major; the reference's (head_dim, heads, tokens, batch) arrays): q, out, dq
// [B][Sq][H][D]; k, v, dk, dv [B][Sk][H][D]; lse [B][H][Sq] f32; mask [Sq][Sk] uint8 (nonzero =
// visible; the reference's (key_tokens, query_tokens) Bool array), causal: key <= query.
//
// Forward: a workgroup takes 128 queries of one (batch, head), 32 per wave as two 16-query MFMA
// tiles, and streams the keys in tiles of 64 through a two-stage LDS ring (LDS-DMA copies). Per
// key tile: S^T = K Q^T on v_mfma_f32_16x16x32 (lane l holds keys 4(l/16)+v of a 16-key tile for
// query l%16), the running maximum and sum in the base-2 domain, P rounded to the element type
// (v_cvt_pk_bf16_f32 for bf16),
// O^T += V^T P^T with V^T fragments read transposed from LDS (ds_read_b64_tr_b16). The P operand
// takes its 8 keys per lane as keys {4g..4g+3} and {16+4g..16+4g+3} of a 32-key block (g = l/16):
// exactly what the score accumulators hold, so no lane exchange is needed; the V^T reads use the
// same key order.
//
// Backward (deterministic, no atomics): correction[q] = sum(dy .* out) (attention.jl:190); a
// key-tile kernel accumulates dK and dV over all query tiles; a query-tile kernel accumulates dQ
// over all key tiles. Both recompute P from lse.
#include <cstdlib>
#include <cstring>

#include "attention_g.h"

namespace reels {

namespace att {
constexpr int KT = 64;    // keys per tile
constexpr int QW = 32;    // queries per wave (forward, dQ)
constexpr int QB = 128;   // queries per workgroup (forward, dQ)
constexpr int KW = 16;    // keys per wave (dK / dV)
constexpr int KB = 64;    // keys per workgroup (dK / dV)
constexpr int QT = 64;    // queries per step (dK / dV)
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
}  // namespace att

// LDS slot of 16-byte chunk c of row r is c ^ swz<D>(r). The tiles are read in two patterns:
// - fragment reads (ds_read_b128): 16 rows of an aligned 16-row block, one chunk per 16-lane
//   group (chunks 4 kb + 0..3);
// - transposed reads (read_tr, ds_read_b64_tr_b16): 8 rows of an aligned 8-row block per
//   32-lane pass, 32 bytes of each (chunks 2 i and 2 i + 1).
// The transposed reads need distinct chunk pairs (swz >> 1) within 8 rows; the fragment reads
// need the 16-lane passes of ds_read_b128 to meet distinct banks, and that instruction's passes
// pair 8-lane groups {0, 3}, {1, 2}, {4, 7}, {5, 6} (measured on gfx950 with
// SQ_LDS_BANK_CONFLICT, like the swizzles themselves). For D = 128 (each row covers all 64
// banks) swz = 2 (r mod 8) meets both: the row swizzle r mod 16 left the transposed reads
// two-way conflicted. For D = 64 (two rows per 256 bytes) r mod 8 meets both.
template <int D>
__device__ __forceinline__ int swz(int r) {
  if constexpr (D == 128) return (r & 7) << 1;
  else return r & 7;
}

// byte offset of element d of row r in a tile with rows of D elements (16-byte chunks
// XOR-swizzled by the row, swz above)
template <int D>
__device__ __forceinline__ uint32_t toff(int r, int d) {
  return (uint32_t)(r * D * 2 + (((d >> 3) ^ swz<D>(r)) << 4) + (d & 7) * 2);
}

// 2^x on v_exp_f32 alone: exp2f adds a range scaling for results below 2^-126, probabilities
// that make no difference to any sum here
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }


// A operand of 8 rows-transposed elements from an LDS tile: element e < 4 is row r0 + e,
// element e >= 4 is row r1 + e - 4, column c (the lane's 4-column piece chosen by the caller's
// addresses, see ds_read_b64_tr_b16)
template <int D>
__device__ __forceinline__ u32x4 read_tr(const uint8_t* tile, int r0, int r1, int c, int i16) {
  const int rr0 = r0 + (i16 >> 2), rr1 = r1 + (i16 >> 2), cc = c + 4 * (i16 & 3);
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(i16x4, tile + toff<D>(rr0, cc)));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(i16x4, tile + toff<D>(rr1, cc)));
  u32x4 r;
  r[0] = (uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16);
  r[1] = (uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16);
  r[2] = (uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16);
  r[3] = (uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16);
  return r;
}

struct AttArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* out;   // backward: the forward's output
  const uint16_t* dy;
  const float* lse;
  const float* corr;     // backward: sum(dy .* out) per query, [B][H][Sq]
  float* corr_out;       // the correction kernel's output (the same buffer)
  const uint8_t* mask;
  uint16_t* o;           // forward output / dq
  uint16_t* dk;
  uint16_t* dv;
  float* lse_out;
  int64_t Sq, Sk, H;
  int causal;
  float scale;           // 1 / sqrt(Float32(D)) (attention.jl:129)
};

// Visibility modes, fixed at compile time so that the common case carries no branch in the
// kernels' inner loops: VM 0 = no mask, not causal (bounds only); VM 1 = causal; VM 2 = a mask
// (and causal when a.causal).
template <int VM>
__device__ __forceinline__ bool att_visible(const AttArgs& a, int64_t qi, int64_t kj) {
  const bool in = (kj < a.Sk) & (qi < a.Sq);
  if constexpr (VM == 0) return in;
  if constexpr (VM == 1) return in & (kj <= qi);
  if (!in) return false;
  if (a.causal && kj > qi) return false;
  return a.mask[qi * a.Sk + kj] != 0;
}

// Visibility of key kj to query qi inside a key tile of the forward or dQ kernel. Without a mask
// only keys past Sk are invisible (a query past Sq computes values nobody stores), and only the
// last key tile holds such keys: tiles wholly below Sk (FULL) need no check.
template <int VM, bool FULL>
__device__ __forceinline__ bool att_visible_tile(const AttArgs& a, int64_t qi, int64_t kj) {
  if constexpr (VM == 0) return FULL || kj < a.Sk;
  return att_visible<VM>(a, qi, kj);
}

// Copies of one 64-row tile of a [B][S][H][D] tensor (rows = tokens of one batch and head) into
// LDS with the toff swizzle: copy c of the tile covers LDS rows c * (64 / CH) .. + 64 / CH - 1,
// lane L row c * (64 / CH) + L / CH, LDS slot L % CH holding chunk (L % CH) ^ swz<D>(row).
// Rows past the tensor's end read zeros (buffer range).
template <int D>
struct TileCopy {
  static constexpr int CH = D / 8, RPC = 64 / CH, NC = CH / 4;  // chunks per row, rows per copy, copies per wave
  uint32_t off[NC];  // this lane's byte offset of copy i within a tile that starts at row 0
  uint32_t lds0;     // LDS byte address of this wave's first copy in a tile (scalar)
};
template <int D>
__device__ __forceinline__ TileCopy<D> tile_copy(int64_t H, int w, int lane, const uint8_t* smem) {
  TileCopy<D> tc;
#pragma unroll
  for (int i = 0; i < TileCopy<D>::NC; ++i) {
    const int c = w * TileCopy<D>::NC + i;
    const int row = c * TileCopy<D>::RPC + lane / TileCopy<D>::CH;
    const int chunk = (lane % TileCopy<D>::CH) ^ swz<D>(row);
    tc.off[i] = (uint32_t)((row * H * D + chunk * 8) * 2);
  }
  tc.lds0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)LDS_PTR(const uint8_t, smem) + (uint32_t)(w * TileCopy<D>::NC * 1024));
  return tc;
}
// one wave's copies of the tile at rows row0 .. into the LDS tile at byte offset dst (scalar).
// The row offset goes into the per-lane (vector) offsets, one add per copy, where the buffer's
// range check that turns rows past the tensor's end into zeros applies to it.
template <int D>
__device__ __forceinline__ void copy_tile(const i32x4& rsrc, const TileCopy<D>& tc, int64_t row0,
                                          int64_t H, uint32_t dst) {
  const uint32_t roff = (uint32_t)(row0 * H * D * 2);
#pragma unroll
  for (int i = 0; i < TileCopy<D>::NC; ++i) dma16_at(rsrc, tc.off[i] + roff, 0u, tc.lds0 + dst + i * 1024);
}

// ---------------------------------------------------------------------------------------------
// forward
template <int ELT, int D, int VM>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(AttArgs a) {
  using E = Elt<ELT>;
  using namespace att;
  constexpr int TB = KT * D * 2;  // bytes of one K or V tile
  constexpr int NKB = D / 32;     // k-blocks of the score MFMA
  constexpr int NDT = D / 16;     // 16-wide d tiles of the output
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int64_t b = blockIdx.z, h = blockIdx.y;
  const int64_t q0 = (int64_t)blockIdx.x * QB + w * QW;
  const int64_t Sq = a.Sq, Sk = a.Sk, H = a.H;
  const float sl2 = a.scale * LOG2E;

  // this wave's query fragments (B operand of S^T): query q0 + 16 qt + l16, d = 32 kb + 8 g ..
  u32x4 qf[2][NKB];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int64_t qi = q0 + 16 * qt + l16;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      qf[qt][kb] = u32x4{0, 0, 0, 0};
      if (qi < Sq) qf[qt][kb] = *reinterpret_cast<const u32x4*>(a.q + ((b * Sq + qi) * H + h) * D + kb * 32 + g * 8);
    }
  }
  const uint16_t* kbase = a.k + (b * Sk * H + h) * D;
  const uint16_t* vbase = a.v + (b * Sk * H + h) * D;
  const uint32_t nrec = (uint32_t)(((Sk - 1) * H + 1) * D * 2);
  const i32x4 rk = buffer_rsrc(kbase, nrec), rv = buffer_rsrc(vbase, nrec);
  const TileCopy<D> tc = tile_copy<D>(H, w, lane, smem);
  auto issue = [&](int j, int stg) {
    const uint32_t st = (uint32_t)(stg * 2 * TB);
    copy_tile<D>(rk, tc, (int64_t)j * KT, H, st);
    copy_tile<D>(rv, tc, (int64_t)j * KT, H, st + TB);
  };

  f32x4 oacc[NDT][2];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) oacc[dt][qt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float mrun[2] = {-INFINITY, -INFINITY}, lrun[2] = {0.0f, 0.0f};  // lrun: this lane's part

  // keys past the last one any query of this workgroup can see (causal) need no tile
  int64_t kend = Sk;
  if (a.causal) {
    const int64_t qlast = (int64_t)blockIdx.x * QB + QB - 1;
    kend = qlast + 1 < Sk ? qlast + 1 : Sk;
  }
  const int ntiles = (int)((kend + KT - 1) / KT);
  // tiles wholly below Sk (checked per score only with a mask or causal)
  const int nfull = VM == 0 ? (int)(kend / KT) : 0;
  if (ntiles > 0) issue(0, 0);
  // step j uses ring stage j % 2: STG 0 or 1 when the caller knows it (the LDS addresses are then
  // constant offsets of the lane's base), -1 to compute it
  auto step = [&](int j, auto full, auto stage) {
    constexpr bool FULL = decltype(full)::value;
    constexpr int STG = decltype(stage)::value;
    const int stg = STG >= 0 ? STG : (j & 1);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's copies of tile j have landed
    __syncthreads();                     // every wave's; every wave is done with tile j - 1
    if (j + 1 < ntiles) issue(j + 1, stg ^ 1);
    const uint8_t* sk = smem + stg * 2 * TB;
    const uint8_t* sv = sk + TB;
    const int64_t key0 = (int64_t)j * KT;

    // S^T tiles: s[kt][qt] lane: keys key0 + 16 kt + 4 g + v, query q0 + 16 qt + l16
    // (k-block outer: eight independent accumulators between two MFMAs on the same one)
    f32x4 s[4][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) s[kt][0] = s[kt][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // raised wave priority over the score MFMAs (their fragment reads issue ahead of the other
    // wave's softmax): forward -0.6%; over the softmax or the P.V MFMAs it is slower
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      u32x4 kf[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
        kf[kt] = *reinterpret_cast<const u32x4*>(sk + toff<D>(16 * kt + l16, kb * 32 + g * 8));
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        s[kt][0] = E::mfma16(E::as8(kf[kt]), E::as8(qf[0][kb]), s[kt][0]);
        s[kt][1] = E::mfma16(E::as8(kf[kt]), E::as8(qf[1][kb]), s[kt][1]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
    // online softmax per query (base 2): masked scores are -inf and get probability 0. The
    // maximum is taken on the raw scores (the scale sl2 is positive) and each exponent is one
    // fma, s sl2 - m. The running maximum m is only moved (and O and l rescaled) when a query's
    // tile maximum exceeds it by more than TAU = 8 somewhere in the wave (one wave-uniform
    // branch); otherwise P = 2^(s sl2 - m) <= 2^8, exact in the sums and in the lse, and the
    // rounding of P to the element type is relative as before.
    constexpr float TAU = 8.0f;
    float ml[2];  // this lane's maximum raw score per query tile
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const int64_t qi = q0 + 16 * qt + l16;
      float m = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int64_t kj = key0 + 16 * kt + 4 * g + v;
          const float x = att_visible_tile<VM, FULL>(a, qi, kj) ? s[kt][qt][v] : -INFINITY;
          s[kt][qt][v] = x;
          m = fmaxf(m, x);
        }
      ml[qt] = m;
    }
    // a query with no visible key so far keeps m = -inf (nothing accumulated); the first tile
    // always moves m (-inf + TAU < any finite maximum). The test needs no exchange between lanes:
    // some lane's own maximum exceeds its row's running maximum + TAU exactly when the row's
    // maximum does (scaling by sl2 > 0 keeps the order), and the ballot asks for any row
    if (__builtin_amdgcn_ballot_w64((ml[0] * sl2 > mrun[0] + TAU) || (ml[1] * sl2 > mrun[1] + TAU))) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        const float mnew = fmaxf(mrun[qt], wave_max16(ml[qt]) * sl2);
        const float alpha = (VM == 2 && mnew == -INFINITY) ? 1.0f : ex2(mrun[qt] - mnew);
        mrun[qt] = mnew;
        lrun[qt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int v = 0; v < 4; ++v) oacc[dt][qt][v] *= alpha;
      }
    }
    u32x4 pb[2][2];  // P operand: [32-key block][qt]
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const float mu = mrun[qt];
      float ps = 0.0f;
      float p[4][4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float x = s[kt][qt][v];
          p[kt][v] = (VM == 2 && x == -INFINITY) ? 0.0f : ex2(__builtin_fmaf(x, sl2, -mu));
          ps += p[kt][v];
        }
      lrun[qt] += ps;
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2) {
        pb[kb2][qt][0] = E::pack2_fast(p[2 * kb2][0], p[2 * kb2][1]);
        pb[kb2][qt][1] = E::pack2_fast(p[2 * kb2][2], p[2 * kb2][3]);
        pb[kb2][qt][2] = E::pack2_fast(p[2 * kb2 + 1][0], p[2 * kb2 + 1][1]);
        pb[kb2][qt][3] = E::pack2_fast(p[2 * kb2 + 1][2], p[2 * kb2 + 1][3]);
      }
    }
    // O^T += V^T P^T: A = V^T rows d = 16 dt + l16, keys {32 kb2 + 4 g ..} and {32 kb2 + 16 + 4 g ..}
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const u32x4 vf = read_tr<D>(sv, 32 * kb2 + 4 * g, 32 * kb2 + 16 + 4 * g, 16 * dt, l16);
        oacc[dt][0] = E::mfma16(E::as8(vf), E::as8(pb[kb2][0]), oacc[dt][0]);
        oacc[dt][1] = E::mfma16(E::as8(vf), E::as8(pb[kb2][1]), oacc[dt][1]);
      }
  };
  // (run-time stage: with constant stages this kernel spills and runs slower)
  using SR = std::integral_constant<int, -1>;
  int j = 0;
  for (; j < nfull; ++j) step(j, std::true_type{}, SR{});
  for (; j < ntiles; ++j) step(j, std::false_type{}, SR{});

  // out = O / l, lse = (m + log2 l) ln 2; a query with no visible key gets NaN for both, as the
  // reference's online softmax gives
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int64_t qi = q0 + 16 * qt + l16;
    const float l = wave_sum16(lrun[qt]);
    const bool none = !(l > 0.0f);
    const float inv = none ? __builtin_nanf("") : 1.0f / l;
    // no keys at all: lse = -Inf + log(0) as the reference computes it; keys, none visible: NaN
    const float lnone = Sk == 0 ? -INFINITY : __builtin_nanf("");
    if (qi < Sq) {
      uint16_t* orow = a.o + ((b * Sq + qi) * H + h) * D;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const u32x2 pk = {E::pack2(oacc[dt][qt][0] * inv, oacc[dt][qt][1] * inv),
                          E::pack2(oacc[dt][qt][2] * inv, oacc[dt][qt][3] * inv)};
        *reinterpret_cast<u32x2*>(orow + 16 * dt + 4 * g) = pk;
      }
      if (a.lse_out != nullptr && g == 0)
        a.lse_out[(b * H + h) * Sq + qi] = none ? lnone : (mrun[qt] + log2f(l)) * LN2;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// backward: correction[b][h][q] = sum_d dy * out (f32). D / 8 lanes per query row, 16 bytes of
// dy and of out each (whole rows per load instruction, where one row per thread made every load
// touch 64 rows), then a fixed-order sum over the row's lanes: the same bits on every run.
template <int ELT, int D>
__global__ __launch_bounds__(256) void attn_corr_kernel(AttArgs a, int64_t B) {
  using E = Elt<ELT>;
  constexpr int LPR = D / 8, RPB = 256 / LPR;  // lanes per row, rows per block
  const int t = threadIdx.x, c = t % LPR;
  const int64_t i = (int64_t)blockIdx.x * RPB + t / LPR;  // ((b * Sq + q) * H + h)
  const bool in = i < B * a.Sq * a.H;
  float acc = 0.0f;
  if (in) {
    const u32x4 x = reinterpret_cast<const u32x4*>(a.dy + i * D)[c];
    const u32x4 y = reinterpret_cast<const u32x4*>(a.out + i * D)[c];
#pragma unroll
    for (int e = 0; e < 4; ++e) acc += E::lo(x[e]) * E::lo(y[e]) + E::hi(x[e]) * E::hi(y[e]);
  }
#pragma unroll
  for (int off = LPR / 2; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, LPR);
  if (in && c == 0) {
    const int64_t h = i % a.H, bq = i / a.H, qi = bq % a.Sq, b = bq / a.Sq;
    a.corr_out[(b * a.H + h) * a.Sq + qi] = acc;
  }
}

// dK, dV: a workgroup takes 64 keys of one (batch, head), 16 per wave, and streams the queries
// in steps of 64 (Q and dY tiles through a two-stage LDS ring, lse and correction beside them).
// Per step: S = Q K^T and dP = dY V^T (lane l: queries 16 qt + 4 g + v, key l16), P from lse,
// dS = P (dP - correction), dV^T += dY^T P and dK^T += Q^T dS (A operands read transposed, the
// query order {4g..4g+3, 16+4g..16+4g+3} of each 32-query block of the accumulators).
template <int ELT, int D, int VM>
__global__ __launch_bounds__(256, 2) void attn_dkdv_kernel(AttArgs a) {
  using E = Elt<ELT>;
  using namespace att;
  constexpr int TB = QT * D * 2;  // bytes of one Q or dY step tile
  constexpr int NKB = D / 32, NDT = D / 16;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int64_t b = blockIdx.z, h = blockIdx.y;
  const int64_t k0 = (int64_t)blockIdx.x * KB + w * KW;
  const int64_t Sq = a.Sq, Sk = a.Sk, H = a.H;
  const float sl2 = a.scale * LOG2E;
  const int64_t kj = k0 + l16;  // this lane's key

  // K and V fragments (B operands): key kj, d = 32 kb + 8 g ..
  u32x4 kf[NKB], vf[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    kf[kb] = vf[kb] = u32x4{0, 0, 0, 0};
    if (kj < Sk) {
      kf[kb] = *reinterpret_cast<const u32x4*>(a.k + ((b * Sk + kj) * H + h) * D + kb * 32 + g * 8);
      vf[kb] = *reinterpret_cast<const u32x4*>(a.v + ((b * Sk + kj) * H + h) * D + kb * 32 + g * 8);
    }
  }
  const uint16_t* qbase = a.q + (b * Sq * H + h) * D;
  const uint16_t* dbase = a.dy + (b * Sq * H + h) * D;
  const uint32_t nrec = (uint32_t)(((Sq - 1) * H + 1) * D * 2);
  const i32x4 rq = buffer_rsrc(qbase, nrec), rd = buffer_rsrc(dbase, nrec);
  float* sstat = reinterpret_cast<float*>(smem + 4 * TB);  // [2 stages][lse QT, corr QT]
  static_assert(QT == 64, "the step tiles are the 64-row tiles of copy_tile");
  const TileCopy<D> tc = tile_copy<D>(H, w, lane, smem);
  auto issue = [&](int j) {
    const uint32_t st = (uint32_t)((j & 1) * 2 * TB);
    copy_tile<D>(rq, tc, (int64_t)j * QT, H, st);
    copy_tile<D>(rd, tc, (int64_t)j * QT, H, st + TB);
  };
  // lse and correction of a step's queries (threads 0..63): loaded into a register with the
  // step's copies and written to LDS after the wait that ends the previous step, so the loads
  // never make the compiler wait for copies it cannot see
  float stv = 0.0f;
  auto stats_load = [&](int j) {
    if (t < 2 * QT) {
      const int64_t qi = (int64_t)j * QT + (t % QT);
      stv = 0.0f;
      if (qi < Sq) stv = (t < QT) ? a.lse[(b * H + h) * Sq + qi] : a.corr[(b * H + h) * Sq + qi];
    }
  };
  // lse to base 2 here, after the step's wait: a product at the load made the wave wait for the
  // load before issuing the step's copies
  auto stats_store = [&](int j) {
    if (t < 2 * QT) sstat[(j & 1) * 2 * QT + t] = t < QT ? stv * LOG2E : stv;
  };

  f32x4 dvacc[NDT], dkacc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) dvacc[dt] = dkacc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // causal: queries before the first key of this workgroup see none of its keys
  int jbeg = 0;
  if (a.causal) jbeg = (int)(((int64_t)blockIdx.x * KB) / QT);
  const int nsteps = (int)((Sq + QT - 1) / QT);
  if (jbeg < nsteps) { stats_load(jbeg); issue(jbeg); }
  for (int j = jbeg; j < nsteps; ++j) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // this wave's copies and statistics of step j
    stats_store(j);
    __syncthreads();
    if (j + 1 < nsteps) { stats_load(j + 1); issue(j + 1); }
    __builtin_amdgcn_s_setprio(0);
    const uint8_t* sq = smem + (j & 1) * 2 * TB;
    const uint8_t* sd = sq + TB;
    const float* ls = sstat + (j & 1) * 2 * QT;
    constexpr int NQT = QT / 16;  // 16-query tiles per step
    // S and dP tiles [qt]: lane queries 16 qt + 4 g + v, key l16 (k-block outer: independent
    // accumulators between two MFMAs on the same one)
    f32x4 s[NQT], dp[NQT];
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) s[qt] = dp[qt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int qt = 0; qt < NQT; ++qt) {
        const u32x4 qa = *reinterpret_cast<const u32x4*>(sq + toff<D>(16 * qt + l16, kb * 32 + g * 8));
        const u32x4 da = *reinterpret_cast<const u32x4*>(sd + toff<D>(16 * qt + l16, kb * 32 + g * 8));
        s[qt] = E::mfma16(E::as8(qa), E::as8(kf[kb]), s[qt]);
        dp[qt] = E::mfma16(E::as8(da), E::as8(vf[kb]), dp[qt]);
      }
    // B operands per 32-query block kb2: key l16, queries {32 kb2 + 4g ..+3, 32 kb2 + 16 + 4g ..+3}
    u32x4 pb[NQT / 2], db[NQT / 2];
#pragma unroll
    for (int kb2 = 0; kb2 < NQT / 2; ++kb2) {
      float p[2][4], ds[2][4];
#pragma unroll
      for (int hq = 0; hq < 2; ++hq) {
        const int qt = 2 * kb2 + hq;
        // lse and correction of this lane's 4 queries 16 qt + 4 g .. + 3: one read each
        const f32x4 lq4 = *reinterpret_cast<const f32x4*>(ls + 16 * qt + 4 * g);
        const f32x4 cq4 = *reinterpret_cast<const f32x4*>(ls + QT + 16 * qt + 4 * g);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int ql = 16 * qt + 4 * g + v;
          const int64_t qi = (int64_t)j * QT + ql;
          // without a mask nothing needs hiding here: a query past Sq has zero Q and dY rows
          // (and zero statistics), so its P is 1 and its dS 0 and both products add zeros; a
          // key past Sk only affects its own, unstored, dK and dV column
          const bool vis = VM == 0 || att_visible<VM>(a, qi, kj);
          p[hq][v] = vis ? ex2(s[qt][v] * sl2 - lq4[v]) : 0.0f;
          ds[hq][v] = vis ? p[hq][v] * (dp[qt][v] - cq4[v]) : 0.0f;
        }
      }
      pb[kb2][0] = E::pack2_fast(p[0][0], p[0][1]); pb[kb2][1] = E::pack2_fast(p[0][2], p[0][3]);
      pb[kb2][2] = E::pack2_fast(p[1][0], p[1][1]); pb[kb2][3] = E::pack2_fast(p[1][2], p[1][3]);
      db[kb2][0] = E::pack2_fast(ds[0][0], ds[0][1]); db[kb2][1] = E::pack2_fast(ds[0][2], ds[0][3]);
      db[kb2][2] = E::pack2_fast(ds[1][0], ds[1][1]); db[kb2][3] = E::pack2_fast(ds[1][2], ds[1][3]);
    }
    // The gradient MFMAs run at raised wave priority, kept through the next step's wait, barrier
    // and copy issue and dropped before its score reads: a wave in this phase issues ahead of
    // the other wave on its SIMD (which is in its score reads or softmax), so the matrix core
    // gets one wave's dense MFMA run while the other's LDS reads and VALU work proceed beside it
    // (dK/dV 41.9 -> 39.6 ms; the same around the score MFMAs or the softmax, or in dQ and the
    // forward, is slower)
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int kb2 = 0; kb2 < NQT / 2; ++kb2)
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const u32x4 da = read_tr<D>(sd, 32 * kb2 + 4 * g, 32 * kb2 + 16 + 4 * g, 16 * dt, l16);
        const u32x4 qa = read_tr<D>(sq, 32 * kb2 + 4 * g, 32 * kb2 + 16 + 4 * g, 16 * dt, l16);
        dvacc[dt] = E::mfma16(E::as8(da), E::as8(pb[kb2]), dvacc[dt]);
        dkacc[dt] = E::mfma16(E::as8(qa), E::as8(db[kb2]), dkacc[dt]);
      }
  }
  __builtin_amdgcn_s_setprio(0);
  // dV[kj][d], dK[kj][d] = scale dK^T: lane holds d = 16 dt + 4 g + v of key kj
  if (kj < Sk) {
    uint16_t* dvrow = a.dv + ((b * Sk + kj) * H + h) * D;
    uint16_t* dkrow = a.dk + ((b * Sk + kj) * H + h) * D;
    const float sc = a.scale;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const u32x2 pv = {E::pack2(dvacc[dt][0], dvacc[dt][1]), E::pack2(dvacc[dt][2], dvacc[dt][3])};
      const u32x2 pk = {E::pack2(dkacc[dt][0] * sc, dkacc[dt][1] * sc), E::pack2(dkacc[dt][2] * sc, dkacc[dt][3] * sc)};
      *reinterpret_cast<u32x2*>(dvrow + 16 * dt + 4 * g) = pv;
      *reinterpret_cast<u32x2*>(dkrow + 16 * dt + 4 * g) = pk;
    }
  }
}

// dK, dV for head dim 128 on 32 x 32 x 16 MFMAs: a workgroup of eight waves takes 256 keys of one
// (batch, head), 32 per wave, and streams the queries in steps of 64 (Q and dY tiles through a
// two-stage LDS ring, the workgroup's V rows in LDS for the whole pass, K in registers). Each
// step is two blocks of 32 queries; per block and wave: S = Q K^T and dP = dY V^T as one 32 x 32
// tile each (lane l: key l % 32; accumulator element v: query 8 (v / 4) + 4 (l / 32) + v % 4),
// P from lse, dS = P (dP - correction), then dV^T += dY^T P and dK^T += Q^T dS over two
// 16-query MFMA steps b. Step b's B operands are accumulator elements 8 b .. 8 b + 7 as they are
// (queries 16 b + 4 (l / 32) + 0..3 and 16 b + 8 + 4 (l / 32) + 0..3), its A operands dY^T and
// Q^T read transposed from the step tiles in that query order. Each fragment read from LDS feeds
// one 32 x 32 x 16 MFMA: 40 KB of LDS reads per wave and 32 queries against 64 KB for the same
// products on 16 x 16 x 32 tiles with 16 keys per wave. Eight waves share each Q / dY tile (half
// the L2 reads of four-wave workgroups: measured 1.73 -> 1.79 GHz under the power cap, dK/dV
// 36.7 -> 36.0 ms), and the 64-query steps keep one barrier per 64 queries.
namespace att {
constexpr int KW2 = 32;   // keys per wave
constexpr int KB2 = 256;  // keys per workgroup
constexpr int NW2 = 8;    // waves per workgroup
constexpr int QT2 = 64;   // queries per step (two 32-query blocks)
constexpr int QS = 32;    // queries per MFMA block
}  // namespace att

// Chunk swizzle of this kernel's tiles (rows of 128 elements, 256 bytes: each row covers all 64
// banks): the slot of chunk c of row r is c ^ swz32(r), swz32(r) = 4 (r mod 4) + (r / 4 mod 2)
// + 2 (r / 8 mod 2), a bijection on r mod 16.
// - fragment reads (ds_read_b128, lane l: row l % 32, chunk 2 s + l / 32): the instruction's
//   16-lane passes (8-lane groups {0, 3}, {1, 2}, {4, 7}, {5, 6}) take rows {0..7, 24..31} or
//   {8..15, 16..23} at one chunk: 16 distinct r mod 16, 16 distinct slots;
// - transposed reads (read_tr32, ds_read_b64_tr_b16; a 32-lane pass reads rows 4 i .. 4 i + 3,
//   chunks 4 t .. 4 t + 3): swz32(r) / 4 = r mod 4 differs between the four rows, so the four
//   rows' chunk quads land on four distinct quads of slots.
__device__ __forceinline__ int swz32(int r) {
  return ((r & 3) << 2) | ((r >> 2) & 1) | (((r >> 3) & 1) << 1);
}
__device__ __forceinline__ uint32_t toff32(int r, int d) {
  return (uint32_t)(r * 256 + (((d >> 3) ^ swz32(r)) << 4) + (d & 7) * 2);
}
// read_tr on the swz32 layout: element e < 4 is row r0 + e, e >= 4 row r1 + e - 4, column
// c + (lane % 16)
__device__ __forceinline__ u32x4 read_tr32(const uint8_t* tile, int r0, int r1, int c, int i16) {
  const int rr0 = r0 + (i16 >> 2), rr1 = r1 + (i16 >> 2), cc = c + 4 * (i16 & 3);
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(i16x4, tile + toff32(rr0, cc)));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(i16x4, tile + toff32(rr1, cc)));
  u32x4 r;
  r[0] = (uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16);
  r[1] = (uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16);
  r[2] = (uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16);
  r[3] = (uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16);
  return r;
}

// LDS: [V rows of the workgroup, 64 KB][2 stages x (Q 16 KB, dY 16 KB)][2 stages x (lse 64, corr 64) f32]
constexpr int kDkdv32Lds = att::KB2 * 256 + 2 * 2 * att::QT2 * 256 + 2 * 2 * att::QT2 * 4;

template <int ELT, int VM>
__global__ __launch_bounds__(512, 1) void attn_dkdv32_kernel(AttArgs a) {
  using E = Elt<ELT>;
  using namespace att;
  constexpr int D = 128;
  constexpr int TQ = QT2 * D * 2;  // bytes of one Q or dY step tile
  constexpr int TV = KB2 * D * 2;  // bytes of the V rows
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int l32 = lane & 31, hf = lane >> 5, l16 = lane & 15, g = lane >> 4;
  const int64_t b = blockIdx.z, h = blockIdx.y;
  const int64_t kb0 = (int64_t)blockIdx.x * KB2;
  const int64_t Sq = a.Sq, Sk = a.Sk, H = a.H;
  const float sl2 = a.scale * LOG2E;
  const int64_t kj = kb0 + w * KW2 + l32;  // this lane's key

  // K fragments (B operands of S): key kj, d = 16 s + 8 hf ..
  u32x4 kf[D / 16];
#pragma unroll
  for (int s = 0; s < D / 16; ++s) {
    kf[s] = u32x4{0, 0, 0, 0};
    if (kj < Sk) kf[s] = *reinterpret_cast<const u32x4*>(a.k + ((b * Sk + kj) * H + h) * D + 16 * s + 8 * hf);
  }
  const uint32_t nrq = (uint32_t)(((Sq - 1) * H + 1) * D * 2);
  const uint32_t nrk = (uint32_t)(((Sk - 1) * H + 1) * D * 2);
  const i32x4 rq = buffer_rsrc(a.q + (b * Sq * H + h) * D, nrq);
  const i32x4 rd = buffer_rsrc(a.dy + (b * Sq * H + h) * D, nrq);
  const i32x4 rv = buffer_rsrc(a.v + (b * Sk * H + h) * D, nrk);
  // LDS-DMA copies of 1 KiB (4 rows): lane L writes row 4 c + L / 16 of copy c, slot L % 16, with
  // chunk (L % 16) ^ swz32(row) of that row. Per step wave w copies rows 8 w .. 8 w + 7 of the
  // 64-row Q and dY tiles; before the first step, its own 32 V rows. Rows past the tensor's end
  // read zeros (buffer range).
  const int crow = lane >> 4, cslot = lane & 15;
  uint32_t qoff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = 8 * w + 4 * i + crow;
    qoff[i] = (uint32_t)((row * H * D + (cslot ^ swz32(row)) * 8) * 2);
  }
  // LDS addresses of the copies (M0) in scalar registers
  const uint32_t sbase = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)LDS_PTR(const uint8_t, smem));
  const int wu = __builtin_amdgcn_readfirstlane(w);
  auto issue = [&](int j) {
    const uint32_t roff = (uint32_t)((int64_t)j * QT2 * H * D * 2);
    const uint32_t st = sbase + (uint32_t)(TV + (j & 1) * 2 * TQ + wu * 2048);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      dma16_at(rq, qoff[i] + roff, 0u, st + i * 1024);
      dma16_at(rd, qoff[i] + roff, 0u, st + TQ + i * 1024);
    }
  };
  auto issue_v = [&]() {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = 32 * w + 4 * i + crow;
      const uint32_t off = (uint32_t)(((kb0 + row) * H * D + (cslot ^ swz32(row)) * 8) * 2);
      dma16_at(rv, off, 0u, sbase + (uint32_t)(32 * wu + 4 * i) * 256);
    }
  };
  float* sstat = reinterpret_cast<float*>(smem + TV + 4 * TQ);  // [2 stages][lse QT2, corr QT2]
  // lse (to base 2 at the store) and correction of a step's queries (threads 0..63), loaded with
  // the step's copies and written to LDS after the wait that ends the previous step
  float stv = 0.0f;
  auto stats_load = [&](int j) {
    if (t < 2 * QT2) {
      const int64_t qi = (int64_t)j * QT2 + (t % QT2);
      stv = 0.0f;
      if (qi < Sq) stv = (t < QT2) ? a.lse[(b * H + h) * Sq + qi] : a.corr[(b * H + h) * Sq + qi];
    }
  };
  auto stats_store = [&](int j) {
    if (t < 2 * QT2) sstat[(j & 1) * 2 * QT2 + t] = t < QT2 ? stv * LOG2E : stv;
  };

  f32x16 dvacc[D / 32], dkacc[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int v = 0; v < 16; ++v) dvacc[dt][v] = dkacc[dt][v] = 0.0f;

  // causal: queries before the first key of this workgroup see none of its keys
  int jbeg = 0;
  if (a.causal) jbeg = (int)(kb0 / QT2);
  const int nsteps = (int)((Sq + QT2 - 1) / QT2);
  if (jbeg < nsteps) { issue_v(); stats_load(jbeg); issue(jbeg); }
  const uint8_t* sv = smem + w * KW2 * 256;
  for (int j = jbeg; j < nsteps; ++j) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // this wave's copies and statistics of step j
    stats_store(j);
    __syncthreads();
    if (j + 1 < nsteps) { stats_load(j + 1); issue(j + 1); }
    // the two 32-query blocks (kept as a loop: unrolled, the compiler interleaves them and spills)
#pragma unroll 1
    for (int sb = 0; sb < QT2 / QS; ++sb) {
    __builtin_amdgcn_s_setprio(0);
    const uint8_t* sq = smem + TV + (j & 1) * 2 * TQ + sb * QS * 256;
    const uint8_t* sd = sq + TQ;
    const float* ls0 = sstat + (j & 1) * 2 * QT2 + sb * QS;
    f32x16 s, dp;
#pragma unroll
    for (int v = 0; v < 16; ++v) s[v] = dp[v] = 0.0f;
#pragma unroll
    for (int ds = 0; ds < D / 16; ++ds) {
      const u32x4 qa = *reinterpret_cast<const u32x4*>(sq + toff32(l32, 16 * ds + 8 * hf));
      const u32x4 da = *reinterpret_cast<const u32x4*>(sd + toff32(l32, 16 * ds + 8 * hf));
      const u32x4 va = *reinterpret_cast<const u32x4*>(sv + toff32(l32, 16 * ds + 8 * hf));
      s = E::mfma32(E::as8(qa), E::as8(kf[ds]), s);
      dp = E::mfma32(E::as8(da), E::as8(va), dp);
    }
    float p[16], dsv[16];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      // lse and correction of this lane's queries 8 c + 4 hf .. + 3: one read each
      const f32x4 lq4 = *reinterpret_cast<const f32x4*>(ls0 + 8 * c + 4 * hf);
      const f32x4 cq4 = *reinterpret_cast<const f32x4*>(ls0 + QT2 + 8 * c + 4 * hf);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int v = 4 * c + e;
        const int64_t qi = (int64_t)j * QT2 + sb * QS + 8 * c + 4 * hf + e;
        // without a mask nothing needs hiding: a query past Sq has zero Q and dY rows and zero
        // statistics (P = 1, dS = 0, both products add zeros); a key past Sk only affects its
        // own, unstored, dK and dV column
        const bool vis = VM == 0 || att_visible<VM>(a, qi, kj);
        p[v] = vis ? ex2(s[v] * sl2 - lq4[e]) : 0.0f;
        dsv[v] = vis ? p[v] * (dp[v] - cq4[e]) : 0.0f;
      }
    }
    u32x4 pb[2], db[2];
#pragma unroll
    for (int bb = 0; bb < 2; ++bb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pb[bb][i] = E::pack2_fast(p[8 * bb + 2 * i], p[8 * bb + 2 * i + 1]);
        db[bb][i] = E::pack2_fast(dsv[8 * bb + 2 * i], dsv[8 * bb + 2 * i + 1]);
      }
    // gradient MFMAs at raised wave priority, as in attn_dkdv_kernel: the two waves of a SIMD
    // belong to this workgroup and leave each barrier together, and the priority puts the one
    // that reaches its gradient MFMAs first ahead, so that its MFMAs run beside the other's
    // softmax (without it: 63.2 against 36.7 ms; over the score MFMAs instead: 37.0 ms)
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int bb = 0; bb < 2; ++bb)
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        const int r0 = 16 * bb + 4 * hf, c = 32 * dt + 16 * (g & 1);
        const u32x4 da = read_tr32(sd, r0, r0 + 8, c, l16);
        const u32x4 qa = read_tr32(sq, r0, r0 + 8, c, l16);
        dvacc[dt] = E::mfma32(E::as8(da), E::as8(pb[bb]), dvacc[dt]);
        dkacc[dt] = E::mfma32(E::as8(qa), E::as8(db[bb]), dkacc[dt]);
      }
    }
  }
  __builtin_amdgcn_s_setprio(0);
  // dV[kj][d], dK[kj][d] = scale dK^T: element v of tile dt is d = 32 dt + 8 (v / 4) + 4 hf + v % 4
  if (kj < Sk) {
    uint16_t* dvrow = a.dv + ((b * Sk + kj) * H + h) * D;
    uint16_t* dkrow = a.dk + ((b * Sk + kj) * H + h) * D;
    const float sc = a.scale;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d = 32 * dt + 8 * c + 4 * hf;
        const u32x2 pv = {E::pack2(dvacc[dt][4 * c], dvacc[dt][4 * c + 1]),
                          E::pack2(dvacc[dt][4 * c + 2], dvacc[dt][4 * c + 3])};
        const u32x2 pk = {E::pack2(dkacc[dt][4 * c] * sc, dkacc[dt][4 * c + 1] * sc),
                          E::pack2(dkacc[dt][4 * c + 2] * sc, dkacc[dt][4 * c + 3] * sc)};
        *reinterpret_cast<u32x2*>(dvrow + d) = pv;
        *reinterpret_cast<u32x2*>(dkrow + d) = pk;
      }
  }
}

// dQ: the forward's structure. Per key tile: S^T = K Q^T and dP^T = V dY^T (A operands K and V
// rows from LDS, B operands this wave's Q and dY fragments), P from lse, dS = P (dP - corr),
// dQ^T += K^T dS^T with K^T read transposed in the accumulators' key order.
template <int ELT, int D, int VM>
__global__ __launch_bounds__(256, 2) void attn_dq_kernel(AttArgs a) {
  using E = Elt<ELT>;
  using namespace att;
  constexpr int TB = KT * D * 2;
  constexpr int NKB = D / 32, NDT = D / 16;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int64_t b = blockIdx.z, h = blockIdx.y;
  const int64_t q0 = (int64_t)blockIdx.x * QB + w * QW;
  const int64_t Sq = a.Sq, Sk = a.Sk, H = a.H;
  const float sl2 = a.scale * LOG2E;

  u32x4 qf[2][NKB], df[2][NKB];
  float lse2[2], cr[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int64_t qi = q0 + 16 * qt + l16;
    lse2[qt] = qi < Sq ? a.lse[(b * H + h) * Sq + qi] * LOG2E : 0.0f;
    cr[qt] = qi < Sq ? a.corr[(b * H + h) * Sq + qi] : 0.0f;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      qf[qt][kb] = df[qt][kb] = u32x4{0, 0, 0, 0};
      if (qi < Sq) {
        qf[qt][kb] = *reinterpret_cast<const u32x4*>(a.q + ((b * Sq + qi) * H + h) * D + kb * 32 + g * 8);
        df[qt][kb] = *reinterpret_cast<const u32x4*>(a.dy + ((b * Sq + qi) * H + h) * D + kb * 32 + g * 8);
      }
    }
  }
  const uint16_t* kbase = a.k + (b * Sk * H + h) * D;
  const uint16_t* vbase = a.v + (b * Sk * H + h) * D;
  const uint32_t nrec = (uint32_t)(((Sk - 1) * H + 1) * D * 2);
  const i32x4 rk = buffer_rsrc(kbase, nrec), rv = buffer_rsrc(vbase, nrec);
  const TileCopy<D> tc = tile_copy<D>(H, w, lane, smem);
  auto issue = [&](int j, int stg) {
    const uint32_t st = (uint32_t)(stg * 2 * TB);
    copy_tile<D>(rk, tc, (int64_t)j * KT, H, st);
    copy_tile<D>(rv, tc, (int64_t)j * KT, H, st + TB);
  };
  f32x4 qacc[NDT][2];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) qacc[dt][0] = qacc[dt][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  int64_t kend = Sk;
  if (a.causal) {
    const int64_t qlast = (int64_t)blockIdx.x * QB + QB - 1;
    kend = qlast + 1 < Sk ? qlast + 1 : Sk;
  }
  const int ntiles = (int)((kend + KT - 1) / KT);
  // tiles wholly below Sk (keys past Sk must get P = 0 here: their zero K rows would not cancel
  // an overflowing P)
  const int nfull = VM == 0 ? (int)(kend / KT) : 0;
  if (ntiles > 0) issue(0, 0);
  auto step = [&](int j, auto full, auto stage) {  // stage as in the forward
    constexpr bool FULL = decltype(full)::value;
    constexpr int STG = decltype(stage)::value;
    const int stg = STG >= 0 ? STG : (j & 1);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    if (j + 1 < ntiles) issue(j + 1, stg ^ 1);
    const uint8_t* sk = smem + stg * 2 * TB;
    const uint8_t* sv = sk + TB;
    const int64_t key0 = (int64_t)j * KT;
    u32x4 db[2][2];  // dS operand [32-key block][qt]
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2) {
      float dsv[2][2][4];  // [key tile within the block][qt][v]
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int kt = 2 * kb2 + half;
        f32x4 s[2], dp[2];
        s[0] = s[1] = dp[0] = dp[1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          const u32x4 ka = *reinterpret_cast<const u32x4*>(sk + toff<D>(16 * kt + l16, kb * 32 + g * 8));
          const u32x4 va = *reinterpret_cast<const u32x4*>(sv + toff<D>(16 * kt + l16, kb * 32 + g * 8));
#pragma unroll
          for (int qt = 0; qt < 2; ++qt) {
            s[qt] = E::mfma16(E::as8(ka), E::as8(qf[qt][kb]), s[qt]);
            dp[qt] = E::mfma16(E::as8(va), E::as8(df[qt][kb]), dp[qt]);
          }
        }
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
          const int64_t qi = q0 + 16 * qt + l16;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int64_t kj = key0 + 16 * kt + 4 * g + v;
            const bool vis = att_visible_tile<VM, FULL>(a, qi, kj);
            const float p = vis ? ex2(s[qt][v] * sl2 - lse2[qt]) : 0.0f;
            dsv[half][qt][v] = vis ? p * (dp[qt][v] - cr[qt]) : 0.0f;
          }
        }
      }
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        db[kb2][qt][0] = E::pack2_fast(dsv[0][qt][0], dsv[0][qt][1]);
        db[kb2][qt][1] = E::pack2_fast(dsv[0][qt][2], dsv[0][qt][3]);
        db[kb2][qt][2] = E::pack2_fast(dsv[1][qt][0], dsv[1][qt][1]);
        db[kb2][qt][3] = E::pack2_fast(dsv[1][qt][2], dsv[1][qt][3]);
      }
    }
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const u32x4 kt_ = read_tr<D>(sk, 32 * kb2 + 4 * g, 32 * kb2 + 16 + 4 * g, 16 * dt, l16);
        qacc[dt][0] = E::mfma16(E::as8(kt_), E::as8(db[kb2][0]), qacc[dt][0]);
        qacc[dt][1] = E::mfma16(E::as8(kt_), E::as8(db[kb2][1]), qacc[dt][1]);
      }
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using SR = std::integral_constant<int, -1>;
  int j = 0;
  for (; j + 1 < nfull; j += 2) {
    step(j, std::true_type{}, S0{});
    step(j + 1, std::true_type{}, S1{});
  }
  for (; j < nfull; ++j) step(j, std::true_type{}, SR{});
  for (; j < ntiles; ++j) step(j, std::false_type{}, SR{});
  const float sc = a.scale;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int64_t qi = q0 + 16 * qt + l16;
    if (qi >= Sq) continue;
    uint16_t* row = a.o + ((b * Sq + qi) * H + h) * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const u32x2 pk = {E::pack2(qacc[dt][qt][0] * sc, qacc[dt][qt][1] * sc),
                        E::pack2(qacc[dt][qt][2] * sc, qacc[dt][qt][3] * sc)};
      *reinterpret_cast<u32x2*>(row + 16 * dt + 4 * g) = pk;
    }
  }
}

// zero fill of n 16-bit elements (a kernel rather than hipMemsetAsync: callers may capture the
// backward in a graph)
__global__ __launch_bounds__(256) void attn_zero_kernel(uint16_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0;
}

// ---------------------------------------------------------------------------------------------
// host side
// bf16 / f16 with head dim 64 or 128 take the tuned kernels above; f32 and the other head dims
// up to 128 the generic kernels of attention_g.hip
static bool attn_tuned(int dtype, int64_t D) {
  return (dtype == REELS_HIP_BF16 || dtype == REELS_HIP_F16) && (D == 64 || D == 128);
}

static int attn_validate(const char* fn, const void* q, const void* k, const void* v, int64_t B,
                         int64_t Sq, int64_t Sk, int64_t H, int64_t D, int dtype) {
  if (B < 0 || Sq < 0 || Sk < 0 || H < 0)
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": need B, Sq, Sk, H >= 0");
  if (dtype != REELS_HIP_BF16 && dtype != REELS_HIP_F16 && dtype != REELS_HIP_F32)
    return fail(REELS_HIP_EDTYPE, std::string(fn) + ": dtype must be REELS_HIP_BF16, REELS_HIP_F16 or REELS_HIP_F32");
  if (D < 1 || D > 128)
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": head_dim must be between 1 and 128");
  if (H >= 65536 || B >= 65536)
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": B and H must be below 65536");
  const int64_t es = dtype == REELS_HIP_F32 ? 4 : 2;
  if (Sq * H * D * es >= ((int64_t)1 << 31) || Sk * H * D * es >= ((int64_t)1 << 31))
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": one batch of q or k over 2 GiB");
  if (B * Sq * H == 0) return 1;  // nothing to compute
  // k and v may be NULL without keys (empty tensors): nothing reads them then
  if (!q || (Sk > 0 && (!k || !v))) return fail(REELS_HIP_EINVAL, std::string(fn) + ": NULL q, k or v");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v))
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": q, k, v must be 16-byte aligned");
  return 0;
}

template <typename K>
static hipError_t set_lds(K kernel, int bytes) {
  return hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

// calls f(std::integral_constant<int, VM>) for the arguments' visibility mode
template <typename F>
static int with_vm(const AttArgs& a, F&& f) {
  if (a.mask != nullptr) return f(std::integral_constant<int, 2>{});
  if (a.causal) return f(std::integral_constant<int, 1>{});
  return f(std::integral_constant<int, 0>{});
}

template <int ELT, int D>
static int launch_attn_fwd(const AttArgs& a, int64_t B, hipStream_t st) {
  return with_vm(a, [&](auto vm) {
    constexpr int VM = decltype(vm)::value;
    const int lds = 4 * att::KT * D * 2;
    if (hipError_t e = set_lds(attn_fwd_kernel<ELT, D, VM>, lds))
      return fail(REELS_HIP_EHIP, std::string("attention fwd: hipFuncSetAttribute: ") + hipGetErrorString(e));
    const dim3 grid((unsigned)ceil_div(a.Sq, att::QB), (unsigned)a.H, (unsigned)B);
    { TraceScope _ts(st, "attn_fwd_kernel"); attn_fwd_kernel<ELT, D, VM><<<grid, 256, lds, st>>>(a); }
    return check_launch("attn_fwd_kernel");
  });
}

// dK / dV at head dim 128: the 256-key workgroups of attn_dkdv32_kernel (one per CU, 256 CUs)
// or the 64-key ones of attn_dkdv_kernel (two per CU), whichever grid needs less time counted in
// rounds of workgroups over the CUs. A 256-key round takes 1.74 times as long as a 64-key one
// (36.0 ms for 20 rounds against 41.4 ms for 40 at 32760 x 32760 x 40 heads), so few keys, as in
// cross-attention on text tokens, go to the 64-key kernel. Backward at 32760 queries x 40 heads,
// 64- / 256-key kernel: 77 keys 1.24 / 1.84 ms, 512 keys 1.78 / 2.13, 1024 keys 2.96 / 2.61,
// 2048 keys 4.90 / 5.35, 3072 keys 6.91 / 6.20, 4096 keys 8.56 / 8.86, 8192 keys 16.7 / 15.2:
// the rule picks the faster one at each. REELS_HIP_ATTN_DKDV_KEYS=256 or =64 fixes the choice
// (the tests run both kernels on the same shapes).
static bool dkdv_wide(int64_t Sk, int64_t H, int64_t B) {
  if (const char* e = std::getenv("REELS_HIP_ATTN_DKDV_KEYS")) {
    if (std::strcmp(e, "256") == 0) return true;
    if (std::strcmp(e, "64") == 0) return false;
  }
  const int64_t nw = ceil_div(Sk, att::KB2) * H * B, n64 = ceil_div(Sk, att::KB) * H * B;
  return ceil_div(nw, 256) * 174 < ceil_div(n64, 512) * 100;
}

template <int ELT, int D>
static int launch_attn_bwd(const AttArgs& a, int64_t B, hipStream_t st) {
  {
    TraceScope _ts(st, "attn_corr_kernel");
    attn_corr_kernel<ELT, D><<<(unsigned)ceil_div(B * a.Sq * a.H, 256 / (D / 8)), 256, 0, st>>>(a, B);
  }
  if (int rc = check_launch("attn_corr_kernel")) return rc;
  return with_vm(a, [&](auto vm) {
    constexpr int VM = decltype(vm)::value;
    bool wide = false;
    if constexpr (D == 128) wide = dkdv_wide(a.Sk, a.H, B);
    if (a.Sk > 0 && wide) {
      if (hipError_t e = set_lds(attn_dkdv32_kernel<ELT, VM>, kDkdv32Lds))
        return fail(REELS_HIP_EHIP, std::string("attention bwd: hipFuncSetAttribute: ") + hipGetErrorString(e));
      const dim3 grid((unsigned)ceil_div(a.Sk, att::KB2), (unsigned)a.H, (unsigned)B);
      { TraceScope _ts(st, "attn_dkdv32_kernel"); attn_dkdv32_kernel<ELT, VM><<<grid, 64 * att::NW2, kDkdv32Lds, st>>>(a); }
      if (int rc = check_launch("attn_dkdv32_kernel")) return rc;
    } else if (a.Sk > 0) {
      const int lds = 4 * att::QT * D * 2 + 2 * 2 * att::QT * 4;  // Q, dY rings + lse / corr
      if (hipError_t e = set_lds(attn_dkdv_kernel<ELT, D, VM>, lds))
        return fail(REELS_HIP_EHIP, std::string("attention bwd: hipFuncSetAttribute: ") + hipGetErrorString(e));
      const dim3 grid((unsigned)ceil_div(a.Sk, att::KB), (unsigned)a.H, (unsigned)B);
      { TraceScope _ts(st, "attn_dkdv_kernel"); attn_dkdv_kernel<ELT, D, VM><<<grid, 256, lds, st>>>(a); }
      if (int rc = check_launch("attn_dkdv_kernel")) return rc;
    }
    const int lds = 4 * att::KT * D * 2;
    if (hipError_t e = set_lds(attn_dq_kernel<ELT, D, VM>, lds))
      return fail(REELS_HIP_EHIP, std::string("attention bwd: hipFuncSetAttribute: ") + hipGetErrorString(e));
    const dim3 grid((unsigned)ceil_div(a.Sq, att::QB), (unsigned)a.H, (unsigned)B);
    { TraceScope _ts(st, "attn_dq_kernel"); attn_dq_kernel<ELT, D, VM><<<grid, 256, lds, st>>>(a); }
    return check_launch("attn_dq_kernel");
  });
}

template <typename F>
static int with_att(int dtype, int64_t D, F&& f) {
  if (dtype == REELS_HIP_F16) {
    if (D == 64) return f(std::integral_constant<int, REELS_HIP_F16>{}, std::integral_constant<int, 64>{});
    return f(std::integral_constant<int, REELS_HIP_F16>{}, std::integral_constant<int, 128>{});
  }
  if (D == 64) return f(std::integral_constant<int, REELS_HIP_BF16>{}, std::integral_constant<int, 64>{});
  return f(std::integral_constant<int, REELS_HIP_BF16>{}, std::integral_constant<int, 128>{});
}

}  // namespace reels

using namespace reels;

extern "C" size_t reels_hip_attention_workspace_bytes(int64_t B, int64_t Sq, int64_t H) {
  if (B < 0 || Sq < 0 || H < 0) return 0;
  const size_t n = (size_t)B * (size_t)Sq * (size_t)H * 4;
  return n == 0 ? 256 : (n + 255) / 256 * 256;
}

extern "C" int reels_hip_attention_fwd(const void* q, const void* k, const void* v,
                                       const uint8_t* mask, int causal, int64_t B, int64_t Sq,
                                       int64_t Sk, int64_t H, int64_t D, int dtype, void* out,
                                       float* lse, void* stream) {
  clear_error();
  const char* fn = "reels_hip_attention_fwd";
  if (int rc = attn_validate(fn, q, k, v, B, Sq, Sk, H, D, dtype)) return rc < 0 ? rc : REELS_HIP_OK;
  if (!out) return fail(REELS_HIP_EINVAL, std::string(fn) + ": NULL out");
  if (!aligned16(out)) return fail(REELS_HIP_EINVAL, std::string(fn) + ": out must be 16-byte aligned");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (!attn_tuned(dtype, D)) {
    AttgArgs g{};
    g.q = q; g.k = k; g.v = v; g.mask = mask; g.o = out; g.lse_out = lse;
    g.Sq = Sq; g.Sk = Sk; g.H = H; g.D = D;
    g.causal = causal ? 1 : 0;
    g.scale = 1.0f / sqrtf((float)D);
    return attn_generic_fwd(g, dtype, B, st);
  }
  AttArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.mask = mask;
  a.o = static_cast<uint16_t*>(out);
  a.lse_out = lse;
  a.Sq = Sq; a.Sk = Sk; a.H = H;
  a.causal = causal ? 1 : 0;
  a.scale = 1.0f / sqrtf((float)D);
  return with_att(dtype, D, [&](auto e, auto d) { return launch_attn_fwd<decltype(e)::value, decltype(d)::value>(a, B, st); });
}

extern "C" int reels_hip_attention_bwd(const void* q, const void* k, const void* v,
                                       const void* out, const void* dy, const float* lse,
                                       const uint8_t* mask, int causal, int64_t B, int64_t Sq,
                                       int64_t Sk, int64_t H, int64_t D, int dtype, void* dq,
                                       void* dk, void* dv, void* workspace, size_t ws_bytes,
                                       void* stream) {
  clear_error();
  const char* fn = "reels_hip_attention_bwd";
  if (int rc = attn_validate(fn, q, k, v, B, Sq, Sk, H, D, dtype)) {
    if (rc < 0) return rc;
    // no queries: dk and dv are zero (the reference's zero(k), zero(v))
    if (B * Sk * H > 0 && dk && dv) {
      hipStream_t st = reinterpret_cast<hipStream_t>(stream);
      const int64_t n = B * Sk * H * D * (dtype == REELS_HIP_F32 ? 2 : 1);  // 16-bit words
      const unsigned grid = (unsigned)(ceil_div(n, 256) < 4096 ? ceil_div(n, 256) : 4096);
      { TraceScope _ts(st, "attn_zero_kernel"); attn_zero_kernel<<<grid, 256, 0, st>>>(static_cast<uint16_t*>(dk), n); }
      { TraceScope _ts(st, "attn_zero_kernel"); attn_zero_kernel<<<grid, 256, 0, st>>>(static_cast<uint16_t*>(dv), n); }
      return check_launch("attn_zero_kernel");
    }
    return REELS_HIP_OK;
  }
  if (!out || !dy || !lse || !dq || (Sk > 0 && (!dk || !dv)))
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": NULL out, dy, lse, dq, dk or dv");
  if (!aligned16(out) || !aligned16(dy) || !aligned16(dq) || !aligned16(dk) || !aligned16(dv))
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": out, dy, dq, dk, dv must be 16-byte aligned");
  if (!workspace || ws_bytes < reels_hip_attention_workspace_bytes(B, Sq, H))
    return fail(REELS_HIP_EWORKSPACE, std::string(fn) + ": workspace NULL or smaller than "
                                      "reels_hip_attention_workspace_bytes(B, Sq, H)");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (!attn_tuned(dtype, D)) {
    AttgArgs g{};
    g.q = q; g.k = k; g.v = v; g.out = out; g.dy = dy; g.lse = lse;
    g.corr = static_cast<float*>(workspace);
    g.mask = mask; g.o = dq; g.dk = dk; g.dv = dv;
    g.Sq = Sq; g.Sk = Sk; g.H = H; g.D = D;
    g.causal = causal ? 1 : 0;
    g.scale = 1.0f / sqrtf((float)D);
    return attn_generic_bwd(g, dtype, B, st);
  }
  AttArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.out = static_cast<const uint16_t*>(out);
  a.dy = static_cast<const uint16_t*>(dy);
  a.lse = lse;
  a.corr = static_cast<const float*>(workspace);
  a.corr_out = static_cast<float*>(workspace);
  a.mask = mask;
  a.o = static_cast<uint16_t*>(dq);
  a.dk = static_cast<uint16_t*>(dk);
  a.dv = static_cast<uint16_t*>(dv);
  a.Sq = Sq; a.Sk = Sk; a.H = H;
  a.causal = causal ? 1 : 0;
  a.scale = 1.0f / sqrtf((float)D);
  return with_att(dtype, D, [&](auto e, auto d) { return launch_attn_bwd<decltype(e)::value, decltype(d)::value>(a, B, st); });
}
