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

}  // namespace reels
