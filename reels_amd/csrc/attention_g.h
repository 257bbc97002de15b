// Attention for element types and head dims outside the tuned kernels (attention_g.hip):
// arguments and launchers, called by the entry points of attention.hip.
#pragma once
#include "common.h"

namespace reels {

struct AttgArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* out;   // backward: the forward's output
  const void* dy;
  const float* lse;  // backward: [B][H][Sq]
  float* corr;       // backward: sum(dy .* out) per query, [B][H][Sq] (workspace)
  const uint8_t* mask;
  void* o;           // forward output / dq
  void* dk;
  void* dv;
  float* lse_out;
  int64_t Sq, Sk, H, D;
  int causal;
  float scale;       // 1 / sqrt(Float32(D)) (attention.jl:129)
};

// forward (out, lse) and backward (dq, dk, dv; corr is the [B][H][Sq] f32 workspace) for dtype
// REELS_HIP_F32, _BF16 or _F16 and 1 <= D <= 128; the caller has checked the arguments
int attn_generic_fwd(const AttgArgs& a, int dtype, int64_t B, hipStream_t st);
int attn_generic_bwd(const AttgArgs& a, int dtype, int64_t B, hipStream_t st);

}  // namespace reels
