// Arguments and launcher of the int8-weight MFMA GEMM (i8gemm.hip), shared with lora.hip.
#pragma once
#include "common.h"

namespace reels {

struct GemmArgs {
  const uint16_t* act;     // [M][Kred] bf16
  const int8_t* q;         // [N][K] int8, row length ldq
  const float* colscale;   // per output column scale (FWD: s) or nullptr (= 1)
  const uint16_t* L;       // [M][rp] bf16 or nullptr
  const uint16_t* R;       // [Ncols][rp] bf16 or nullptr
  const uint16_t* bias;    // [Ncols] bf16 or nullptr
  uint16_t* out;           // [M][Ncols] bf16
  int64_t M, Ncols, Kred, ldq;
  int rp;                  // LoRA rank (multiple of 16, 0 = none)
  float c;                 // LoRA scale alpha / r
};

// mode 0 = FWD (out = s * act q^T + c L R^T + bias), 1 = DX (out = act q + c L R^T)
int launch_i8gemm(int mode, const GemmArgs& a, hipStream_t st);

// bf16 x bf16 GEMM with the LoRA epilogue: out = bf16(act wd^T + c L R^T + bias), wd [Ncols][Kred]
// bf16 (a dequantized weight); a.q and a.colscale are unused. Needs Kred % 64 == 0, 16-byte
// aligned operands and byte sizes below 2^31 (bfgemm_supported).
bool bfgemm_supported(int64_t M, int64_t Ncols, int64_t Kred);
// mode only labels the trace record ("bfgemm_kernel<0>" forward, "<1>" dX)
int launch_bfgemm(int mode, const GemmArgs& a, const uint16_t* wd, hipStream_t st);

// wd[n][k] = bf16(fl32(q[n][k] * s[n])), q [N][K] row stride ldq (K % 16 == 0)
int launch_dequant_rows(const int8_t* q, int64_t ldq, const float* s, int64_t N, int64_t K,
                        uint16_t* wd, hipStream_t st);
// wt[k][n] = bf16(fl32(q[n][k] * s[n])) (N % 64 == 0, K % 64 == 0)
int launch_dequant_transpose(const int8_t* q, int64_t ldq, const float* s, int64_t N, int64_t K,
                             uint16_t* wt, hipStream_t st);

}  // namespace reels
