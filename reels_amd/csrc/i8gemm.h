// Arguments and launcher of the int8-weight MFMA GEMM (i8gemm.hip), shared with lora.hip.
#pragma once
#include "common.h"

namespace reels {

struct GemmArgs {
  const uint16_t* act;     // [M][Kred] bf16
  const int8_t* q;         // [N][K] int8, row length ldq
  const float* colscale;   // per output column scale (FWD: s) or nullptr (= 1)
  const float* redscale;   // DX only: per reduction index scale s[n] applied to the weight as
                           // E::deq(q, s) (the f16 path), or nullptr: act is already scaled
  const uint16_t* L;       // [M][rp] bf16 or nullptr
  const uint16_t* R;       // [Ncols][rp] bf16 or nullptr
  const uint16_t* bias;    // [Ncols] bf16 or nullptr
  uint16_t* out;           // [M][Ncols] bf16
  int64_t M, Ncols, Kred, ldq;
  int rp;                  // LoRA rank (multiple of 16, 0 = none)
  float c;                 // LoRA scale alpha / r
  // bfgemm only: the reduction split over ksplit workgroups per tile (0 or 1 = none); each writes
  // its f32 partial to part [ksplit][M][Ncols] (the first split's with c L R^T added) and a
  // reduction pass sums them in split order, adds the bias and rounds once
  int ksplit;
  float* part;
  // bfgemm only, without a split reduction: the GELU's pullback fused into the epilogue,
  // out = rnd(rnd(sum) * gelu_tanh'(gx)) with gx [M][Ncols] the GELU's input (the same bits as
  // gelu_bwd_kernel on the stored product), when gx != nullptr
  const uint16_t* gx;
  // bfgemm only, without a split reduction: gout [M][Ncols] = gelu_tanh(out) from the rounded
  // 16-bit outputs (the same bits as gelu_kernel on out), written beside out when != nullptr
  uint16_t* gout;
};

// mode 0 = FWD (out = s * act q^T + c L R^T + bias), 1 = DX (out = act q + c L R^T, or
// out = act deq(q, redscale) + c L R^T when redscale is set); elt is the 16-bit element type of
// act, L, R, bias and out (REELS_HIP_BF16 or REELS_HIP_F16)
int launch_i8gemm(int mode, int elt, const GemmArgs& a, hipStream_t st);

// 16-bit GEMM with the LoRA epilogue: out = rnd(act wd^T + c L R^T + bias), wd [Ncols][Kred] (a
// dequantized weight) of element type elt like every other operand; a.q and a.colscale are
// unused. Needs Kred % 64 == 0, 16-byte aligned operands and a weight below 2^31 bytes
// (bfgemm_supported); any token count (split into chunks of activations below 2^31 bytes).
bool bfgemm_supported(int64_t M, int64_t Ncols, int64_t Kred);
// reduction splits for token counts whose 256 x 256 tiles leave most CUs idle (1 = none): about
// one round of 256 workgroups, at least 4 reduction steps of 64 per split
int bfgemm_splits(int64_t M, int64_t Ncols, int64_t Kred);
// mode only labels the trace record ("bfgemm_kernel<0>" forward, "<1>" dX). a.gx needs
// a.ksplit <= 1 and 16-byte aligned buffers (bfgemm_fuses_gelu)
int launch_bfgemm(int mode, int elt, const GemmArgs& a, const uint16_t* wd, hipStream_t st);
bool bfgemm_fuses_gelu(const GemmArgs& a);
// a.gout (the forward GELU epilogue) needs the same: a.ksplit <= 1 and 16-byte aligned buffers
bool bfgemm_fuses_gelu_fwd(const GemmArgs& a);

// wd[n][k] = deq(q[n][k], s[n]) in element type elt (bf16: bf16(fl32(q s)); f16: f16(q f16(s))),
// q [N][K] row stride ldq (K % 16 == 0)
int launch_dequant_rows(int elt, const int8_t* q, int64_t ldq, const float* s, int64_t N, int64_t K,
                        uint16_t* wd, hipStream_t st);
// wt[k][n] = deq(q[n][k], s[n]) (N % 64 == 0, K % 64 == 0)
int launch_dequant_transpose(int elt, const int8_t* q, int64_t ldq, const float* s, int64_t N,
                             int64_t K, uint16_t* wt, hipStream_t st);

// Few-token path (skinny.hip): int8 codes streamed straight into registers, tokens on the MFMA's
// 16-wide side, the reduction split over blocks and finished in the same launch by the last block
// of each tile (split order). mode 0 = FWD (act = x, rows of q are outputs, lw = A [Kred][rp]
// zero-padded), 1 = DX (act = dy, rows of q are the reduction, lw = B [r][Kred], s = the
// reduction's scale).
// up to 240 tokens (three 80-token blocks), or 1024 on weights of at most 4M elements; beyond,
// and wherever they fill the GPU, the row-wave output tiles (skinny_rw_kernel) run instead
constexpr int64_t kSkinnyMaxTokens = 240;
constexpr int64_t kSkinnySmallWeightTokens = 1024;
constexpr int64_t kSkinnyTargetBlocks = 256;  // about one block per CU
struct SkinnyPlan {
  int T;   // token tiles of 16 per block (the adapter blocks; also the output blocks unless rw)
  int tb;  // token blocks (ditto)
  int S;   // reduction splits (ditto)
  // row-wave output tiles: 64 NI rows x 16 To tokens over the whole reduction in one block,
  // orb x otb of them; the adapter blocks keep T, tb and S
  bool rw = false;
  int NI = 0, To = 0, orb = 0, otb = 0;
};
bool skinny_supported(int64_t M, int64_t K, int64_t N, int rp);
// mode 0: the forward (Kred = K, Ncols = N); 1: dX (Kred = N, Ncols = K)
SkinnyPlan skinny_plan(int64_t M, int64_t Kred, int64_t Ncols, int rp, int mode);
// workspace of one launch: the split partials and l [M][rp]
size_t skinny_ws_bytes(const SkinnyPlan& p, int64_t M, int64_t Ncols, int rp);
// out = rnd(colscale * act W + c l R + bias) with l = rnd(act L) (h or u), written to lsave
// ([M][ld_lsave], lsave_cols columns, zeros past r) when not NULL; R(o, j) = R[j][o] (mode 0,
// row stride ldr) or R[o][j] (mode 1, rows of ldr >= rp elements, zeros past r). adapter_only: l
// alone, from the same blocks and split order as a full launch (so a recomputed h equals the
// forward's bit for bit). The launch's counters live in ws (cleared by a kernel before it), so
// launches with their own workspaces may run concurrently.
int launch_skinny(int mode, int elt, const SkinnyPlan& p, const uint16_t* act, const int8_t* q,
                  int64_t ldq, const float* s, const uint16_t* lw, void* ws, int64_t M,
                  int64_t Kred, int64_t Ncols, int r, int rp, const float* colscale,
                  const uint16_t* R, int64_t ldr, const uint16_t* bias, float c, uint16_t* out,
                  uint16_t* lsave, int64_t ld_lsave, int lsave_cols, hipStream_t st,
                  bool adapter_only = false);

// out = c * sum over splits of part[sp][o][j] (split order): out[o][j], or out[j][o] with trans
int launch_reduce_partials(const float* part, int splits, int64_t Od, int rp, int r, float c,
                           float* out, bool trans, hipStream_t st);

// out[o] = sum_m src[m][o] in f32 (src [M][Od] of element type elt: REELS_HIP_F32, _BF16 or
// _F16): the bias gradient. Split-M partials in part (colsum_partial_bytes(M, Od) bytes), summed
// in split order; the same splits and order as the dB gradient pass's fused column sums.
int launch_colsum(int elt, const void* src, int64_t M, int64_t Od, float* part, float* out,
                  hipStream_t st);
size_t colsum_partial_bytes(int64_t M, int64_t Od);

}  // namespace reels
