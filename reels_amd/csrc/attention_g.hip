// Attention for the element types and head dims the tuned kernels of attention.hip do not take:
// f32 tensors (the reference's Float32 path, the partner of the f32 int8 LoRA linear), and bf16 /
// f16 tensors whose head dim is not 64 or 128 (any D up to 128). memory_efficient_attention and
// its backward (src/layers/attention.jl:106-221) are generic in both.
//
// Every product and sum runs in f32 on v_mfma_f32_16x16x4_f32, with the operands converted
// exactly from the element type; unlike the tuned kernels the probabilities stay in f32 (the
// reference's own order: scores, softmax and P V in Float32), and only the results are rounded
// to the element type. Deterministic: no atomics, fixed summation order.
//
// MFMA layouts (v_mfma_f32_16x16x4_f32): lane l holds A[l % 16][l / 16] and B[l / 16][l % 16]
// (the four k slots are the four 16-lane groups g = l / 16) and D[4 g + v][l % 16], v = 0..3. A
// score product S^T = K Q^T leaves lane (query l % 16, g) holding keys 4 g + v of a 16-key tile;
// the product that consumes those probabilities maps its k slot g of step t to key 4 g + t, so
// each lane feeds register t of its own scores to step t: no lane exchange.
#include "attention_g.h"

namespace reels {

// one element as f32 (exact) and an f32 result rounded to the element type
template <int ELT> struct GElt;
template <> struct GElt<REELS_HIP_F32> {
  static __device__ __forceinline__ float ld(const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }
  static __device__ __forceinline__ void st(void* p, int64_t i, float x) { static_cast<float*>(p)[i] = x; }
};
template <> struct GElt<REELS_HIP_BF16> {
  static __device__ __forceinline__ float ld(const void* p, int64_t i) {
    return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
  static __device__ __forceinline__ void st(void* p, int64_t i, float x) {
    static_cast<uint16_t*>(p)[i] = (uint16_t)f32_to_bf16_bits(x);
  }
};
template <> struct GElt<REELS_HIP_F16> {
  static __device__ __forceinline__ float ld(const void* p, int64_t i) {
    return Elt<REELS_HIP_F16>::to_f32(static_cast<const uint16_t*>(p)[i]);
  }
  static __device__ __forceinline__ void st(void* p, int64_t i, float x) {
    static_cast<uint16_t*>(p)[i] = (uint16_t)Elt<REELS_HIP_F16>::bits(x);
  }
};

namespace attg {
constexpr int QW = 16;   // queries (forward, dQ) or keys (dK / dV) per wave
constexpr int WB = 64;   // per workgroup (four waves)
constexpr int KT = 32;   // keys per LDS tile (forward, dQ)
constexpr int QT = 32;   // queries per LDS tile (dK / dV)
}  // namespace attg

// visibility modes as in attention.hip: 0 bounds only, 1 causal, 2 mask (and causal if set)
template <int VM>
__device__ __forceinline__ bool attg_visible(const AttgArgs& a, int64_t qi, int64_t kj) {
  const bool in = (kj < a.Sk) & (qi < a.Sq);
  if constexpr (VM == 0) return in;
  if constexpr (VM == 1) return in & (kj <= qi);
  if (!in) return false;
  if (a.causal && kj > qi) return false;
  return a.mask[qi * a.Sk + kj] != 0;
}

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// rows r0 .. r0 + R - 1 (tokens) of one (batch, head) of a [B][S][H][D] tensor into an LDS tile
// [R][DP + 1] f32 (the odd row stride spreads a column's rows over the banks); zeros past S or D
template <int ELT, int R, int DP>
__device__ __forceinline__ void attg_tile(float* dst, const void* src, int64_t b, int64_t h,
                                          int64_t r0, int64_t S, int64_t H, int64_t D) {
  for (int i = threadIdx.x; i < R * DP; i += 256) {
    const int r = i / DP, d = i % DP;
    const int64_t row = r0 + r;
    float x = 0.0f;
    if (row < S && d < D) x = GElt<ELT>::ld(src, ((b * S + row) * H + h) * D + d);
    dst[r * (DP + 1) + d] = x;
  }
}

// ---------------------------------------------------------------------------------------------
// forward: a workgroup takes 64 queries of one (batch, head), 16 per wave; 32-key tiles of K and
// V in LDS. The online softmax follows attention.jl:136-160 (block maximum, rescale of the
// running sum and accumulator, probabilities of the visible keys).
template <int ELT, int DP, int VM>
__global__ __launch_bounds__(256) void attng_fwd_kernel(AttgArgs a) {
  using namespace attg;
  constexpr int SP = DP + 1;
  __shared__ float sk[KT * SP], sv[KT * SP];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, l16 = lane & 15, g = lane >> 4;
  const int64_t b = blockIdx.z, h = blockIdx.y, H = a.H, D = a.D, Sq = a.Sq, Sk = a.Sk;
  const int64_t qi = (int64_t)blockIdx.x * WB + w * QW + l16;  // this lane's query
  float qf[DP / 4];  // B operand of S^T = K Q^T: Q[qi][4 s + g]
#pragma unroll
  for (int s = 0; s < DP / 4; ++s) {
    const int64_t d = 4 * s + g;
    qf[s] = (qi < Sq && d < D) ? GElt<ELT>::ld(a.q, ((b * Sq + qi) * H + h) * D + d) : 0.0f;
  }
  f32x4 oacc[DP / 16];  // O^T: lane holds d = 16 dt + 4 g + v of query qi
#pragma unroll
  for (int dt = 0; dt < DP / 16; ++dt) oacc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m = -INFINITY, l = 0.0f;
  for (int64_t k0 = 0; k0 < Sk; k0 += KT) {
    __syncthreads();  // every wave is done with the previous tile
    attg_tile<ELT, KT, DP>(sk, a.k, b, h, k0, Sk, H, D);
    attg_tile<ELT, KT, DP>(sv, a.v, b, h, k0, Sk, H, D);
    __syncthreads();
    // S^T per 16-key half u: lane holds keys k0 + 16 u + 4 g + v of query qi
    float sc[2][4];
    float bmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      f32x4 s = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int st = 0; st < DP / 4; ++st) s = mfma4(sk[(16 * u + l16) * SP + 4 * st + g], qf[st], s);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t kj = k0 + 16 * u + 4 * g + v;
        sc[u][v] = attg_visible<VM>(a, qi, kj) ? s[v] * a.scale : -INFINITY;
        bmax = fmaxf(bmax, sc[u][v]);
      }
    }
    bmax = wave_max16(bmax);  // over the key groups of this query
    const float nmax = fmaxf(m, bmax);
    // with no visible key so far (nmax = -Inf) there is nothing to rescale; the reference's
    // exp(-Inf - -Inf) = NaN there would only reach queries that see no key at all
    const float ps = nmax == -INFINITY ? 1.0f : expf(m - nmax);
    float p[2][4];
    float bsum = 0.0f;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        p[u][v] = sc[u][v] == -INFINITY ? 0.0f : expf(sc[u][v] - nmax);
        bsum += p[u][v];
      }
    l = ps * l + wave_sum16(bsum);
    // O^T = O^T ps + V^T P^T: step (u, tt) takes key 16 u + 4 g + tt in k slot g
#pragma unroll
    for (int dt = 0; dt < DP / 16; ++dt) {
      f32x4 o = oacc[dt] * ps;
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) o = mfma4(sv[(16 * u + 4 * g + tt) * SP + 16 * dt + l16], p[u][tt], o);
      oacc[dt] = o;
    }
    m = nmax;
  }
  if (qi >= Sq) return;
  // out = acc / l, lse = m + log(l); a query without a visible key: NaN output, lse NaN (-Inf
  // without keys: the reference's -Inf + log(0))
  const bool none = m == -INFINITY;
  const int64_t ob = ((b * Sq + qi) * H + h) * D;
#pragma unroll
  for (int dt = 0; dt < DP / 16; ++dt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t d = 16 * dt + 4 * g + v;
      if (d < D) GElt<ELT>::st(a.o, ob + d, none ? NAN : oacc[dt][v] / l);
    }
  if (g == 0 && a.lse_out) a.lse_out[(b * H + h) * Sq + qi] = none ? (Sk == 0 ? -INFINITY : NAN) : m + logf(l);
}

// correction[q] = sum(dy .* out) over the head dim (attention.jl:190), in f32
template <int ELT>
__global__ __launch_bounds__(256) void attng_corr_kernel(AttgArgs a, int64_t B) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (b, q, h) in memory order
  if (i >= B * a.Sq * a.H) return;
  const int64_t h = i % a.H, q = (i / a.H) % a.Sq, b = i / (a.H * a.Sq);
  float s = 0.0f;
  for (int64_t d = 0; d < a.D; ++d) s += GElt<ELT>::ld(a.dy, i * a.D + d) * GElt<ELT>::ld(a.out, i * a.D + d);
  a.corr[(b * a.H + h) * a.Sq + q] = s;
}

// dK and dV: a workgroup takes 64 keys of one (batch, head), 16 per wave, and walks every query
// tile (from the first that can see them when causal). With S = Q K^T a lane holds queries
// 4 g + v of a 16-query half for key kj, and the dV / dK products take query 4 g + tt in k slot
// g of step tt: dV^T += dY^T P, dK^T += Q^T dS with dS = P (dP - correction), dP = dY V^T.
template <int ELT, int DP, int VM>
__global__ __launch_bounds__(256) void attng_dkdv_kernel(AttgArgs a) {
  using namespace attg;
  constexpr int SP = DP + 1;
  __shared__ float sq[QT * SP], sdy[QT * SP], slse[QT], scorr[QT];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, l16 = lane & 15, g = lane >> 4;
  const int64_t b = blockIdx.z, h = blockIdx.y, H = a.H, D = a.D, Sq = a.Sq, Sk = a.Sk;
  const int64_t kb = (int64_t)blockIdx.x * WB;
  const int64_t kj = kb + w * QW + l16;  // this lane's key
  float kf[DP / 4], vf[DP / 4];  // B operands: K[kj][4 s + g], V[kj][4 s + g]
#pragma unroll
  for (int s = 0; s < DP / 4; ++s) {
    const int64_t d = 4 * s + g;
    const bool ok = kj < Sk && d < D;
    kf[s] = ok ? GElt<ELT>::ld(a.k, ((b * Sk + kj) * H + h) * D + d) : 0.0f;
    vf[s] = ok ? GElt<ELT>::ld(a.v, ((b * Sk + kj) * H + h) * D + d) : 0.0f;
  }
  f32x4 dka[DP / 16], dva[DP / 16];
#pragma unroll
  for (int dt = 0; dt < DP / 16; ++dt) dka[dt] = dva[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // causal: queries before the workgroup's first key see none of its keys
  const int64_t qstart = VM == 1 ? kb / QT * QT : 0;
  for (int64_t q0 = qstart; q0 < Sq; q0 += QT) {
    __syncthreads();
    attg_tile<ELT, QT, DP>(sq, a.q, b, h, q0, Sq, H, D);
    attg_tile<ELT, QT, DP>(sdy, a.dy, b, h, q0, Sq, H, D);
    if (t < QT) {
      const int64_t qq = q0 + t;
      slse[t] = qq < Sq ? a.lse[(b * H + h) * Sq + qq] : 0.0f;
      scorr[t] = qq < Sq ? a.corr[(b * H + h) * Sq + qq] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      f32x4 s = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, dp = s;
#pragma unroll
      for (int st = 0; st < DP / 4; ++st) {
        const int r = (16 * u + l16) * SP + 4 * st + g;
        s = mfma4(sq[r], kf[st], s);
        dp = mfma4(sdy[r], vf[st], dp);
      }
      // a hidden pair adds nothing (its query's correction is NaN when that query sees no key)
      float p[4], ds[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int qq = 16 * u + 4 * g + v;
        const bool vis = attg_visible<VM>(a, q0 + qq, kj);
        p[v] = vis ? expf(s[v] * a.scale - slse[qq]) : 0.0f;
        ds[v] = vis ? p[v] * (dp[v] - scorr[qq]) : 0.0f;
      }
#pragma unroll
      for (int dt = 0; dt < DP / 16; ++dt) {
        f32x4 x = dva[dt], y = dka[dt];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          const int r = (16 * u + 4 * g + tt) * SP + 16 * dt + l16;
          x = mfma4(sdy[r], p[tt], x);
          y = mfma4(sq[r], ds[tt], y);
        }
        dva[dt] = x;
        dka[dt] = y;
      }
    }
  }
  if (kj >= Sk) return;
  const int64_t ob = ((b * Sk + kj) * H + h) * D;
#pragma unroll
  for (int dt = 0; dt < DP / 16; ++dt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t d = 16 * dt + 4 * g + v;
      if (d < D) {
        GElt<ELT>::st(a.dk, ob + d, dka[dt][v] * a.scale);
        GElt<ELT>::st(a.dv, ob + d, dva[dt][v]);
      }
    }
}

// dQ: a workgroup takes 64 queries, 16 per wave, and walks the key tiles: dQ^T += K^T dS^T with
// dS^T = P^T (dP^T - correction), dP^T = V dY^T (the forward's orientation).
template <int ELT, int DP, int VM>
__global__ __launch_bounds__(256) void attng_dq_kernel(AttgArgs a) {
  using namespace attg;
  constexpr int SP = DP + 1;
  __shared__ float sk[KT * SP], sv[KT * SP];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, l16 = lane & 15, g = lane >> 4;
  const int64_t b = blockIdx.z, h = blockIdx.y, H = a.H, D = a.D, Sq = a.Sq, Sk = a.Sk;
  const int64_t qi = (int64_t)blockIdx.x * WB + w * QW + l16;
  float qf[DP / 4], df[DP / 4];
#pragma unroll
  for (int s = 0; s < DP / 4; ++s) {
    const int64_t d = 4 * s + g;
    const bool ok = qi < Sq && d < D;
    qf[s] = ok ? GElt<ELT>::ld(a.q, ((b * Sq + qi) * H + h) * D + d) : 0.0f;
    df[s] = ok ? GElt<ELT>::ld(a.dy, ((b * Sq + qi) * H + h) * D + d) : 0.0f;
  }
  const float lse = qi < Sq ? a.lse[(b * H + h) * Sq + qi] : 0.0f;
  const float corr = qi < Sq ? a.corr[(b * H + h) * Sq + qi] : 0.0f;
  f32x4 dqa[DP / 16];
#pragma unroll
  for (int dt = 0; dt < DP / 16; ++dt) dqa[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // causal: keys past the workgroup's last query are seen by none of its queries
  const int64_t kend = VM == 1 ? std::min(Sk, (int64_t)(blockIdx.x + 1) * WB) : Sk;
  for (int64_t k0 = 0; k0 < kend; k0 += KT) {
    __syncthreads();
    attg_tile<ELT, KT, DP>(sk, a.k, b, h, k0, Sk, H, D);
    attg_tile<ELT, KT, DP>(sv, a.v, b, h, k0, Sk, H, D);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      f32x4 s = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, dp = s;
#pragma unroll
      for (int st = 0; st < DP / 4; ++st) {
        const int r = (16 * u + l16) * SP + 4 * st + g;
        s = mfma4(sk[r], qf[st], s);
        dp = mfma4(sv[r], df[st], dp);
      }
      float ds[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t kk = k0 + 16 * u + 4 * g + v;
        ds[v] = attg_visible<VM>(a, qi, kk) ? expf(s[v] * a.scale - lse) * (dp[v] - corr) : 0.0f;
      }
#pragma unroll
      for (int dt = 0; dt < DP / 16; ++dt) {
        f32x4 x = dqa[dt];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) x = mfma4(sk[(16 * u + 4 * g + tt) * SP + 16 * dt + l16], ds[tt], x);
        dqa[dt] = x;
      }
    }
  }
  if (qi >= Sq) return;
  const int64_t ob = ((b * Sq + qi) * H + h) * D;
#pragma unroll
  for (int dt = 0; dt < DP / 16; ++dt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t d = 16 * dt + 4 * g + v;
      if (d < D) GElt<ELT>::st(a.o, ob + d, dqa[dt][v] * a.scale);
    }
}

// ---------------------------------------------------------------------------------------------
// host side (called by the entry points of attention.hip after their argument checks)
template <typename F>
static int attg_dispatch(int dtype, int64_t D, const AttgArgs& a, F&& f) {
  auto by_vm = [&](auto e, auto dp) {
    if (a.mask != nullptr) return f(e, dp, std::integral_constant<int, 2>{});
    if (a.causal) return f(e, dp, std::integral_constant<int, 1>{});
    return f(e, dp, std::integral_constant<int, 0>{});
  };
  auto by_dp = [&](auto e) {
    if (D <= 32) return by_vm(e, std::integral_constant<int, 32>{});
    if (D <= 64) return by_vm(e, std::integral_constant<int, 64>{});
    return by_vm(e, std::integral_constant<int, 128>{});
  };
  if (dtype == REELS_HIP_F32) return by_dp(std::integral_constant<int, REELS_HIP_F32>{});
  if (dtype == REELS_HIP_F16) return by_dp(std::integral_constant<int, REELS_HIP_F16>{});
  return by_dp(std::integral_constant<int, REELS_HIP_BF16>{});
}

int attn_generic_fwd(const AttgArgs& a, int dtype, int64_t B, hipStream_t st) {
  return attg_dispatch(dtype, a.D, a, [&](auto e, auto dp, auto vm) {
    constexpr int ELT = decltype(e)::value, DP = decltype(dp)::value, VM = decltype(vm)::value;
    const dim3 grid((unsigned)ceil_div(a.Sq, attg::WB), (unsigned)a.H, (unsigned)B);
    { TraceScope _ts(st, "attng_fwd_kernel"); attng_fwd_kernel<ELT, DP, VM><<<grid, 256, 0, st>>>(a); }
    return check_launch("attng_fwd_kernel");
  });
}

int attn_generic_bwd(const AttgArgs& a, int dtype, int64_t B, hipStream_t st) {
  return attg_dispatch(dtype, a.D, a, [&](auto e, auto dp, auto vm) {
    constexpr int ELT = decltype(e)::value, DP = decltype(dp)::value, VM = decltype(vm)::value;
    {
      TraceScope _ts(st, "attng_corr_kernel");
      attng_corr_kernel<ELT><<<(unsigned)ceil_div(B * a.Sq * a.H, 256), 256, 0, st>>>(a, B);
    }
    if (int rc = check_launch("attng_corr_kernel")) return rc;
    if (a.Sk > 0) {
      const dim3 grid((unsigned)ceil_div(a.Sk, attg::WB), (unsigned)a.H, (unsigned)B);
      { TraceScope _ts(st, "attng_dkdv_kernel"); attng_dkdv_kernel<ELT, DP, VM><<<grid, 256, 0, st>>>(a); }
      if (int rc = check_launch("attng_dkdv_kernel")) return rc;
    }
    const dim3 grid((unsigned)ceil_div(a.Sq, attg::WB), (unsigned)a.H, (unsigned)B);
    { TraceScope _ts(st, "attng_dq_kernel"); attng_dq_kernel<ELT, DP, VM><<<grid, 256, 0, st>>>(a); }
    return check_launch("attng_dq_kernel");
  });
}

}  // namespace reels
