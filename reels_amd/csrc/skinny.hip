// Few-token path of the int8 LoRA linear: a large frozen weight against at most a few hundred
// tokens, e.g. the cross-attention K/V projections over 77-512 text tokens
// (src/models/wan21/transformer.jl:185-188, I2V 225-235, through quantization.jl:73-76). There
// the weight stream is the whole cost, so the int8 codes are read once, coalesced, straight from
// HBM into registers (no bf16 copy of the weight) and converted there; the tokens sit on the
// 16-wide side of v_mfma_f32_16x16x32 (77 tokens = 5 tiles of 16).
//
// One launch does everything. A block is (tile, split): a tile is 64 output rows (or 32 rows of
// the adapter's rank projection) x up to 16T tokens, a split a contiguous range of 64-wide
// reduction chunks. The block's 8 waves take the split's chunks round by round (wave w every
// eighth chunk); their accumulators are summed in LDS in a fixed wave order. With more than one
// split the other splits store that sum as an f32 partial and announce it under the launch's
// key; split 0 waits for those keys, sums the tile's partials in split order (its own from
// registers) and finishes the tile:
//   adapter tile: l = rnd(sum) (h = x A in the forward, u = dy B^T for dX) into the workspace
//                 (and lsave), announced under the key;
//   output tile:  waits for its tokens' adapter tiles' keys, then
//                 out = rnd(scale * sum + c * l R + bias), the l R product on the MFMA.
// The adapter blocks come first in the logical order and wait for nothing but their splits, so
// their keys are normally there long before an output tile looks; every wait is bounded all the
// same, and a block that gives up computes what it waited for itself with the same code and
// order (same bits), so the result never depends on how the grid is scheduled.
// The keys, partials and l live in the call's own workspace and a key names one launch (its
// dispatch in its queue and the host call's nonce), so nothing needs clearing before a launch and
// nothing is shared between calls: calls on any streams, and HIP graphs that capture them, may
// run at the same time. Deterministic: fixed wave order, fixed split order.
//
// FWD: out[m][n] = rnd(s[n] sum_k x[m][k] q[n][k] + c sum_j h[m][j] B[j][n] + bias[n]),
//      h = rnd(x A): the int8 path's formula (the scale on the f32 sum).
// DX:  out[m][k] = rnd(sum_n dy[m][n] W[n][k] + c sum_j u[m][j] A[k][j]), u = rnd(dy B^T), with
//      W = bf16(fl32(q[n][k] s[n])) for bf16 (the weight of the large-token bf16 path) and
//      f16(q[n][k] f16(s[n])) for f16 (the reference's binary16 weight, quantization.jl:61-62),
//      made from the codes in registers; the weight columns of a reduction chunk reach the MFMA
//      through ds_read_b64_tr_b8 from a per-wave LDS tile.
#include "i8gemm.h"

#include <atomic>
#include <chrono>
#include <cstdlib>
#include <mutex>
#include <random>

namespace reels {

namespace sk {
constexpr int NB = 64;       // output rows per tile: 4 MFMA tiles of 16
constexpr int NBL = 32;      // adapter rows per tile: 2 MFMA tiles of 16
constexpr int KC = 64;       // reduction chunk
constexpr int MAXT = 5;      // token tiles of 16 per block (80 tokens)
constexpr int MAXS = 8;      // reduction splits
constexpr int STAGE = 4096;  // per-wave LDS staging (DX weight tile, FWD adapter chunk: 4 KiB each)
constexpr int NWV = 8;       // waves per block (two per SIMD)
constexpr int kMaxTiles = 4096;
constexpr uint32_t kSpinLimit = 1u << 12;  // wait rounds of s_sleep 8 (about 1 ms) before computing l
}  // namespace sk

struct SkArgs {
  const uint16_t* act;  // [M][Kred] 16-bit: x (FWD) or dy (DX)
  const int8_t* q;      // codes [N][K], row stride ldq
  const float* s;       // DX: scale of the reduction index n
  const uint16_t* lw;   // adapter operand: FWD A [Kred][rp] (zeros past r), DX B [r][Kred]
  float* part;          // split partials in MFMA fragment order (output tiles, then adapter tiles)
  uint16_t* hl;         // [M][rp] l rounded to the element type (zeros past r)
  const float* colscale;
  const uint16_t* R;    // FWD B [r][Ncols] (row stride ldr), DX A [Ncols][ldr] (zeros past r)
  const uint16_t* bias;
  uint16_t* out;        // [M][Ncols]
  uint16_t* lsave;      // [M][ld_lsave], lsave_cols columns (or NULL)
  uint32_t* keys;       // [nta] adapter tile's l stored, then [tiles][S] split partial stored
  uint32_t nonce_lo, nonce_hi;  // the host call's nonce (the keys' first words)
  int64_t M, Kred, Ncols, ldq, ldr, ld_lsave;
  float c;
  int r, rp, S, nblk, lblk, tb, lsave_cols;
  int blocks;  // of the launch
  int nad;     // adapter blocks: the first blocks of the logical order
  int ntm;     // output tiles (nblk * tb; 0 for an adapter-only launch)
  uint32_t spin;  // wait rounds before an output tile computes l itself
  int nta;     // adapter tiles (lblk * tb)
  int64_t lpart0;  // first partial fragment of the adapter tiles (after the output tiles')
  int otb;     // row-wave output tiles: token tiles (the output tile is ti / otb, ti % otb)
};

struct SkBlock {
  int blk, sp, tb, tile;  // blk >= nblk: adapter row block blk - nblk
};

// dynamic LDS: the waves' staging areas during the loop, 4 wave sums (4 x 4T fragments of 1 KiB)
// after it, then 16 bytes for the block's arrival count and ready flag
static constexpr int skinny_lds(int T) {
  return ((4 * 4 * T * 64 * 16) > sk::NWV * sk::STAGE ? (4 * 4 * T * 64 * 16) : sk::NWV * sk::STAGE) + 16;
}

// Data one block hands to another (split partials, l, and the keys that announce them) is
// stored and loaded with device-scope coherence (sc1: what the compiler emits for agent-scope
// relaxed atomics), so it never sits in one XCD's L2 where another XCD cannot see it, and no
// cache-wide write-back or invalidate is needed.
constexpr int kSC1 = 16;  // cache policy bit: device scope
// every memory operation of this wave complete (and no compiler motion across it)
__device__ __forceinline__ void sk_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ __amdgpu_buffer_rsrc_t sk_rsrc(const void* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// A launch hands l and the split partials over under a key rather than counters, so nothing has
// to zero memory before the launch (a zeroing launch in front cost about 4 us per call, a tenth
// of a 512-token forward). A key is 16 bytes: the host call's nonce (two
// words), the dispatch's packet index in its queue and the queue's address. A (queue, packet
// index) pair names one dispatch for the queue's life, graph replays included, and the nonce
// differs between host calls and between processes, so whatever an earlier launch (or anything
// else) left in the workspace does not hold this launch's key. A block stores its data, waits for
// those stores (vmcnt 0 in every wave, then the barrier), and then thread 0 stores the key with
// one 16-byte device-scope store; a reader loads the key with device-scope loads and issues its
// data loads after seeing it.
extern "C" __device__ uint64_t reels_dispatch_id() __asm("llvm.amdgcn.dispatch.id");
// The dispatch's two key words go to the block's words [0] and [3] in LDS as the block starts
// (so the registers that bring them in are free for the rest of the block), and the key is read
// back after a barrier.
__device__ __forceinline__ void sk_stash_key(uint32_t* words) {
  if (threadIdx.x == 0) {
    const uint64_t did = reels_dispatch_id();
    const uint64_t q = (uint64_t)__builtin_amdgcn_queue_ptr();
    words[0] = (uint32_t)did;
    words[3] = (uint32_t)(q >> 6) ^ (uint32_t)(did >> 32);
  }
}
__device__ __forceinline__ u32x4 sk_key(const SkArgs& a, const uint32_t* words) {
  return u32x4{a.nonce_lo, a.nonce_hi, words[0], words[3]};
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t sk_keys_rsrc(const SkArgs& a) {
  return sk_rsrc(a.keys, ((int64_t)a.nta + (int64_t)(a.ntm + a.nta) * a.S) * 16);
}
__device__ __forceinline__ void sk_put_key(const SkArgs& a, int idx, u32x4 key) {
  __builtin_amdgcn_raw_buffer_store_b128(key, sk_keys_rsrc(a), (uint32_t)idx * 16u, 0, kSC1);
}
// whether entry idx holds the key (reloaded on every call: the clobber keeps the compiler from
// reusing an earlier load)
__device__ __forceinline__ bool sk_has_key(const SkArgs& a, int idx, u32x4 key) {
  asm volatile("" ::: "memory");
  const u32x4 v = __builtin_bit_cast(
      u32x4, __builtin_amdgcn_raw_buffer_load_b128(sk_keys_rsrc(a), (uint32_t)idx * 16u, 0, kSC1));
  return v[0] == key[0] && v[1] == key[1] && v[2] == key[2] && v[3] == key[3];
}
// waits for the key at entry idx, spending the shared budget of wait rounds (s_sleep 8 each);
// false once the budget is spent without it. A budget of 0 (tests) looks at nothing.
__device__ __forceinline__ bool sk_wait_key(const SkArgs& a, int idx, u32x4 key, uint32_t& rounds) {
  if (a.spin == 0u) return false;
  while (!sk_has_key(a, idx, key)) {
    if (++rounds > a.spin) return false;
    __builtin_amdgcn_s_sleep(8);
  }
  return true;
}

// One wave's share of a (row block, split, token block): acc[i][tt] = rows 16 i + (0..15) x
// tokens 16 tt + (0..15) over the wave's chunks of the split (every eighth). LORA: a block of the
// adapter's rank projection (rows j of A^T in the forward, of B for dX) rather than of the int8
// weight.
template <int T, int MODE, int ELT, bool LORA>
__device__ __forceinline__ void skinny_acc(const SkArgs& a, int blk, int sp, int64_t tok0,
                                           uint8_t* smem, f32x4 (&acc)[LORA ? 2 : 4][T]) {
  using E = Elt<ELT>;
  typedef typename E::v8 V8;
  constexpr bool lora = LORA;
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int l16 = lane & 15, g = lane >> 4;
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

  struct WStage {
    u32x4 wq[NWL];
    f32x4 sc[NSC];  // DX: s[n] for n = 32 e + 8 g + (0..7), [2 e + half]
  };
  struct XStage {
    u32x4 x[T][2];
  };
  // valid = false (a step past the wave's run): every offset of the step moves past its
  // descriptor, so the step reads zeros and adds nothing (no branch around the loads or the
  // multiply, which keeps the compiler's waits exact)
  auto load_x = [&](int c, bool valid, XStage& s) {
    const uint32_t sx = (uint32_t)c * (uint32_t)(sk::KC * 2);
#pragma unroll
    for (int tt = 0; tt < T; ++tt)
#pragma unroll
      for (int e = 0; e < 2; ++e)
        s.x[tt][e] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, valid ? vx[tt][e] : OOB, sx, 0));
  };
  auto load_w = [&](int c, bool valid, WStage& s) {
    const uint32_t sw = (uint32_t)c * wstep;
#pragma unroll
    for (int i = 0; i < NWL; ++i)
      s.wq[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, valid ? vw[i] : OOB, sw, !lora ? 2 : 0));
    if constexpr (MODE == 1 && !lora) {  // the scales of a zero step multiply zeros
      const float* sp8 = a.s + (int64_t)c * sk::KC + 8 * g;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        s.sc[2 * e] = *reinterpret_cast<const f32x4*>(sp8 + 32 * e);
        s.sc[2 * e + 1] = *reinterpret_cast<const f32x4*>(sp8 + 32 * e + 4);
      }
    }
  };

#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int tt = 0; tt < T; ++tt) acc[i][tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  uint8_t* wst = smem + w * sk::STAGE;  // this wave's staging area
  auto compute = [&](const WStage& s, const XStage& xs) {
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
        const V8 xf = E::as8(xs.x[tt][e]);
#pragma unroll
        for (int i = 0; i < NI; ++i) acc[i][tt] = E::mfma16(af[i][e], xf, acc[i][tt]);
      }
  };

  // The split's chunks go round by round: in round rr the block's 8 waves take the 8 consecutive
  // chunks c0 + 8 rr + w, so at any time the block streams one 512-byte stretch of each of its 64
  // weight rows (DRAM pages stay open) and each wave owns a fixed residue of the chunk index. The
  // rounds start at a rotation that depends on the block: rows of the weight (and of the
  // activations) lie a multiple of 1 KiB apart, so blocks that walked the same k offsets at the
  // same time would pile onto a few memory channels. Slots past the split (the last round) read
  // zeros and add nothing.
  const int nk = c1 - c0;
  const int nw = (nk + sk::NWV - 1) / sk::NWV;  // rounds, the same for every wave
  const int rot = nw > 0 ? (int)(((int64_t)blk * 5 + (int64_t)tok0 / 16 * 3) % nw) : 0;
  auto round_of = [&](int i) {
    const int p = rot + i;
    return p < nw ? p : p - nw;
  };
  auto valid = [&](int i) { return i < nw && sk::NWV * round_of(i) + w < nk; };
  // an empty slot names the split's first chunk: every address formed from it stays in bounds
  // (dX reads its scales with plain loads; its zero weights then multiply them)
  auto chunk = [&](int i) { return valid(i) ? c0 + sk::NWV * round_of(i) + w : c0; };
  // (scheduling barriers keep each step's loads together and in program order, so the waits
  // before a multiply cover exactly its own operands)
  if constexpr (MODE == 0 && !lora) {
    // the forward's weight stream runs DW steps ahead; the activations (cache hits) one step
    // ahead, issued before the weight refill so that waiting for them never waits for it
    constexpr int DW = 2;
    WStage ws[DW];
    XStage xs[2];
#pragma unroll
    for (int j = 0; j < DW; ++j) {
      load_w(chunk(j), valid(j), ws[j]);
      __builtin_amdgcn_sched_barrier(0);
    }
    load_x(chunk(0), valid(0), xs[0]);
    __builtin_amdgcn_sched_barrier(0);
    for (int i = 0; i < nw; i += DW) {
#pragma unroll
      for (int j = 0; j < DW; ++j) {
        load_x(chunk(i + j + 1), valid(i + j + 1), xs[(j + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        compute(ws[j], xs[j & 1]);
        __builtin_amdgcn_sched_barrier(0);
        load_w(chunk(i + j + DW), valid(i + j + DW), ws[j]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  } else {
    // dX and the adapter blocks: the weight (with dX's scales) two steps ahead, the activations
    // loaded at the start of their step (the other wave of the SIMD covers that wait)
    WStage w0, w1;
    XStage x0;
    load_w(chunk(0), valid(0), w0);
    __builtin_amdgcn_sched_barrier(0);
    load_w(chunk(1), valid(1), w1);
    __builtin_amdgcn_sched_barrier(0);
    for (int i = 0; i < nw; i += 2) {
      load_x(chunk(i), valid(i), x0);
      __builtin_amdgcn_sched_barrier(0);
      compute(w0, x0);
      __builtin_amdgcn_sched_barrier(0);
      load_w(chunk(i + 2), valid(i + 2), w0);
      __builtin_amdgcn_sched_barrier(0);
      load_x(chunk(i + 1), valid(i + 1), x0);
      __builtin_amdgcn_sched_barrier(0);
      compute(w1, x0);
      __builtin_amdgcn_sched_barrier(0);
      load_w(chunk(i + 3), valid(i + 3), w1);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// The block's sum of its 8 waves' accumulators, in a fixed order: waves 4-7 hand theirs to waves
// 0-3 through LDS (p_w = acc_w + acc_{w+4}), then the four p_w go to LDS as MFMA fragments (wave,
// fragment f = i T + tt, lane) and are summed in wave order, ((p0 + p1) + p2) + p3, by the wave that
// owns the fragment: wave w owns f = w, w + 8, ... with the same lane slot (each thread reads and
// writes 16 consecutive bytes per fragment).
template <int NF> constexpr int sk_fpw() { return (NF + sk::NWV - 1) / sk::NWV; }

template <int T, int NI>
__device__ __forceinline__ void skinny_sum(f32x4 (&acc)[NI][T], uint8_t* smem,
                                           f32x4 (&sum)[sk_fpw<NI * T>()]) {
  constexpr int NF = NI * T, FPW = sk_fpw<NF>();
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  f32x4* red = reinterpret_cast<f32x4*>(smem);
  __syncthreads();
  if (w >= 4) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int tt = 0; tt < T; ++tt) red[((w - 4) * NF + i * T + tt) * 64 + lane] = acc[i][tt];
  }
  __syncthreads();
  if (w < 4) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int tt = 0; tt < T; ++tt) acc[i][tt] += red[(w * NF + i * T + tt) * 64 + lane];
  }
  __syncthreads();
  if (w < 4) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int tt = 0; tt < T; ++tt) red[(w * NF + i * T + tt) * 64 + lane] = acc[i][tt];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < FPW; ++k) {
    const int f = w + sk::NWV * k;
    sum[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (f < NF)
      sum[k] = ((red[f * 64 + lane] + red[(NF + f) * 64 + lane]) + red[(2 * NF + f) * 64 + lane]) +
               red[(3 * NF + f) * 64 + lane];
  }
  __syncthreads();  // LDS free again
}

// l = rnd(sum) of an adapter tile (rows j = o0 + 16 i + 4 g + v of fragment (i, tt), token
// 16 tt + l16) into hl (device scope) and, with lsave set, into lsave
template <int T, int ELT>
__device__ __forceinline__ void skinny_put_l(const SkArgs& a, int64_t o0, int64_t tok0,
                                             const f32x4 (&sum)[sk_fpw<2 * T>()], bool lsave) {
  using E = Elt<ELT>;
  constexpr int NF = 2 * T, FPW = sk_fpw<NF>();
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  const __amdgpu_buffer_rsrc_t rl = sk_rsrc(a.hl, a.M * a.rp * 2);
#pragma unroll
  for (int k = 0; k < FPW; ++k) {
    const int f = w + sk::NWV * k;
    if (f >= NF) continue;
    const int i = f / T, tt = f % T;
    const int64_t tok = tok0 + 16 * tt + l16, j = o0 + 16 * i + 4 * g;
    if (tok >= a.M || j >= a.rp) continue;
    uint32_t b[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) b[v] = j + v < a.r ? E::bits(sum[k][v]) : 0u;
    typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;
    __builtin_amdgcn_raw_buffer_store_b64(u32x2{b[0] | (b[1] << 16), b[2] | (b[3] << 16)}, rl,
                                          (uint32_t)((tok * a.rp + j) * 2), 0, kSC1);
    if (lsave && a.lsave != nullptr && a.lsave != a.hl) {
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (j + v < a.lsave_cols) a.lsave[tok * a.ld_lsave + j + v] = (uint16_t)b[v];
    }
  }
}

// One block: its accumulators, the tile's split reduction, then the tile's results (l for an
// adapter tile, out for an output tile). Split 0 of a tile reduces it, after the other splits
// have stored their partials under the launch's key; a split whose key has not come after a
// bounded wait it computes itself, with that split's code (the same bits). An adapter tile
// announces its l under the key.
template <int T, int MODE, int ELT, bool LORA>
__device__ __forceinline__ void skinny_block(const SkArgs& a, const SkBlock& d, uint8_t* smem) {
  using E = Elt<ELT>;
  constexpr bool lora = LORA;
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  const int blk = d.blk, sp = d.sp;
  const int64_t tok0 = (int64_t)d.tb * (16 * T);
  constexpr int NI = lora ? 2 : 4;
  const int64_t o0 = lora ? (int64_t)(blk - a.nblk) * sk::NBL : (int64_t)blk * sk::NB;
  constexpr int NF = NI * T, FPW = sk_fpw<NF>();
  // [0], [3] the dispatch's key words, [1] splits seen, [2] l ready
  uint32_t* words = reinterpret_cast<uint32_t*>(smem + skinny_lds(T) - 16);
  sk_stash_key(words);
  f32x4 sum[FPW];
  {
    f32x4 acc[NI][T];
    skinny_acc<T, MODE, ELT, LORA>(a, blk, sp, tok0, smem, acc);
    skinny_sum<T, NI>(acc, smem, sum);
  }
  const u32x4 key = sk_key(a, words);
  // An output tile's epilogue operands: the column scales and bias of this thread's rows and
  // (forward) the first 32 rank rows of R for the tile's 64 columns, which threads 0-255 stage in
  // LDS. With split partials they are loaded before the hand-over, whose round trips cover their
  // latency; with one split just before the epilogue (loaded early there they ran slower).
  f32x4 cs[FPW];
  u32x2 bsv[FPW];
  u32x4 rpre;
  auto load_epi = [&]() {
#pragma unroll
    for (int k = 0; k < FPW; ++k) {
      const int f = w + sk::NWV * k;
      const int64_t o = o0 + 16 * (f / T) + 4 * g;
      cs[k] = f32x4{1.0f, 1.0f, 1.0f, 1.0f};
      bsv[k] = u32x2{0u, 0u};
      if (f < NF && a.colscale) cs[k] = *reinterpret_cast<const f32x4*>(a.colscale + o);
      if (f < NF && a.bias) bsv[k] = *reinterpret_cast<const u32x2*>(a.bias + o);
    }
    rpre = u32x4{0u, 0u, 0u, 0u};
    if (MODE == 0 && a.nad > 0 && t < 256 && (t >> 3) < a.r)
      rpre = *reinterpret_cast<const u32x4*>(a.R + (int64_t)(t >> 3) * a.ldr + o0 + 8 * (t & 7));
  };
  if constexpr (!lora)
    if (a.S > 1) load_epi();
  const __amdgpu_buffer_rsrc_t rl = sk_rsrc(a.hl, a.M * a.rp * 2);
  // Output tiles of a launch with an adapter look for the keys of their tokens' adapter tiles now
  // (each wave looks; a key once there stays) and, when all are there, load their tokens' l for
  // the first 32 rank columns while the partial is handed over.
  const bool wants_l = !lora && a.nad > 0;
  uint32_t up = 0;
  if (wants_l) {
    up = 1;
    for (int lb = 0; lb < a.lblk && up; ++lb) up = sk_has_key(a, lb * a.tb + d.tb, key);
  }
  u32x4 hv[FPW];  // B operand of the l R product: l[tok][j .. j + 7], j = 8 g (first rank chunk)
  auto load_l = [&](int j0, u32x4 (&dst)[FPW]) {
    // (the lane index through an empty asm: the offsets are computed here, not kept in
    // registers across the main loop)
    int l16v = l16;
    asm volatile("" : "+v"(l16v));
#pragma unroll
    for (int k = 0; k < FPW; ++k) {
      const int f = w + sk::NWV * k;
      const int64_t tok = tok0 + 16 * (f % T) + l16v;
      const int jj = j0 + 8 * g;
      dst[k] = u32x4{0u, 0u, 0u, 0u};
      if (f < NF && tok < a.M && jj < a.rp)
        dst[k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                               rl, (uint32_t)((tok * a.rp + jj) * 2), 0, kSC1));
    }
  };
  if (a.S > 1) {
    // partial [tile][split][fragment][lane] (16 bytes); output tiles first, then adapter tiles
    const int64_t tbase = lora ? a.lpart0 + (int64_t)(d.tile - a.ntm) * a.S * (NF * 64)
                               : (int64_t)d.tile * a.S * (NF * 64);
    const __amdgpu_buffer_rsrc_t rp_ = sk_rsrc(reinterpret_cast<f32x4*>(a.part) + tbase, (int64_t)a.S * NF * 64 * 16);
    // every split stores its partial (split 0's is loaded back with the others', so no value of
    // it stays in registers across a wait or a recomputation)
    auto put_part = [&](int s, const f32x4 (&v)[FPW]) {
#pragma unroll
      for (int k = 0; k < FPW; ++k) {
        const int f = w + sk::NWV * k;
        if (f < NF)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[k]), rp_,
                                                 (uint32_t)((s * (NF * 64) + f * 64 + lane) * 16), 0, kSC1);
      }
    };
    put_part(sp, sum);
    sk_drain();
    __syncthreads();
    if (sp != 0) {
      if (t == 0) sk_put_key(a, a.nta + d.tile * a.S + sp, key);
      return;
    }
    // split 0: the other splits' keys
    if (t == 0) {
      const int k0 = a.nta + d.tile * a.S;
      uint32_t seen = 0, rounds = 0;
      for (int s = 1; s < a.S; ++s)
        if (sk_wait_key(a, k0 + s, key, rounds)) seen |= 1u << s;
      words[1] = seen;
    }
    __syncthreads();
    const uint32_t seen = words[1], others = ((1u << a.S) - 1u) & ~1u;
    if ((seen & others) != others) {
      // (block-uniform) the splits not seen: their partials computed here with their code and
      // stored in their place; the epilogue operands loaded again after
      for (int s = 1; s < a.S; ++s) {
        if ((seen >> s) & 1u) continue;
        f32x4 ps[FPW];
        {
          f32x4 acc[NI][T];
          skinny_acc<T, MODE, ELT, LORA>(a, blk, s, tok0, smem, acc);
          skinny_sum<T, NI>(acc, smem, ps);
        }
        put_part(s, ps);
      }
      sk_drain();
      __syncthreads();
      if constexpr (!lora) load_epi();
    }
    if (wants_l && up) load_l(0, hv);
    asm volatile("" ::: "memory");
    // the tile's sum in split order, the partials loaded in batches of SB splits
    constexpr int SB = 4;
    f32x4 tot[FPW];
#pragma unroll
    for (int k = 0; k < FPW; ++k) tot[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < a.S; s0 += SB) {
      f32x4 v[SB][FPW];
#pragma unroll
      for (int u = 0; u < SB; ++u)
#pragma unroll
        for (int k = 0; k < FPW; ++k) {
          const int f = w + sk::NWV * k, s = s0 + u;
          v[u][k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          if (f < NF && s < a.S)
            v[u][k] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                    rp_, (uint32_t)((s * (NF * 64) + f * 64 + lane) * 16), 0, kSC1));
        }
#pragma unroll
      for (int u = 0; u < SB; ++u)
        if (s0 + u < a.S) {
#pragma unroll
          for (int k = 0; k < FPW; ++k) tot[k] += v[u][k];
        }
    }
#pragma unroll
    for (int k = 0; k < FPW; ++k) sum[k] = tot[k];
  } else {
#pragma unroll
    for (int k = 0; k < FPW; ++k) sum[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f} + sum[k];
    if (wants_l && up) load_l(0, hv);
  }

  if constexpr (lora) {
    skinny_put_l<T, ELT>(a, o0, tok0, sum, true);
    sk_drain();
    __syncthreads();
    if (t == 0) sk_put_key(a, d.tile - a.ntm, key);
    return;
  } else {
    // l complete: the adapter blocks come first in the logical order and wait for nothing but
    // their splits, so their keys are normally there by the time an output tile gets here. Should
    // they not have come after a bounded wait (a grid that cannot be resident at once, behind
    // other work), the block computes l for its tokens itself, with the adapter blocks' code,
    // splits and order, so the values are the same bits either way.
    if (wants_l) {
      if (t == 0) {
        uint32_t rounds = 0, ok = 1;
        for (int lb = 0; lb < a.lblk && ok; ++lb) ok = sk_wait_key(a, lb * a.tb + d.tb, key, rounds);
        words[2] = ok;
      }
      __syncthreads();
      if (words[2] == 0u) {
        for (int lb = 0; lb < a.lblk; ++lb) {
          constexpr int FA = sk_fpw<2 * T>();
          f32x4 tl[FA];
#pragma unroll
          for (int k = 0; k < FA; ++k) tl[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          for (int s = 0; s < a.S; ++s) {
            f32x4 acc[2][T], ps[FA];
            skinny_acc<T, MODE, ELT, true>(a, a.nblk + lb, s, tok0, smem, acc);
            skinny_sum<T, 2>(acc, smem, ps);
#pragma unroll
            for (int k = 0; k < FA; ++k) tl[k] += ps[k];
          }
          skinny_put_l<T, ELT>(a, (int64_t)lb * sk::NBL, tok0, tl, false);
        }
        sk_drain();
        __syncthreads();
      }
      asm volatile("" ::: "memory");
      if (!up) load_l(0, hv);  // the waves that found the flag down load l now
    }
    if (a.S == 1 || (wants_l && words[2] == 0u)) load_epi();  // (not kept across the path above)
    // lo = l R for this tile on the MFMA, 32 rank columns per step: A operand rows o = 16 i + l16
    // with j = 32 jc + 8 g + (0..7), B operand the tokens' l[tok][j .. j + 7]
    f32x4 lo[FPW];
#pragma unroll
    for (int k = 0; k < FPW; ++k) lo[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int njc = wants_l ? (a.rp + 31) / 32 : 0;
    uint16_t* rst = reinterpret_cast<uint16_t*>(smem);  // FWD: R rows [32 j][64 o]
    for (int jc = 0; jc < njc; ++jc) {
      const int j0 = 32 * jc;
      if (jc > 0) load_l(j0, hv);
      if constexpr (MODE == 0) {
        __syncthreads();
        if (t < 256) {
          const int row = t >> 3, col = 8 * (t & 7);
          u32x4 v = rpre;
          if (jc > 0) {
            v = u32x4{0u, 0u, 0u, 0u};
            if (j0 + row < a.r) v = *reinterpret_cast<const u32x4*>(a.R + (int64_t)(j0 + row) * a.ldr + o0 + col);
          }
          *reinterpret_cast<u32x4*>(rst + row * 64 + col) = v;
        }
        __syncthreads();
      }
#pragma unroll
      for (int k = 0; k < FPW; ++k) {
        const int f = w + sk::NWV * k;
        if (f >= NF) continue;
        const int i = f / T;
        u32x4 av;
        if constexpr (MODE == 0) {
          // transposed 16-bit reads: providing lane p addresses row 8 g + 4 h + p / 4, columns
          // 16 i + 4 (p % 4) .. +3; lane l16 receives o = 16 i + l16, j = 8 g + 4 h + (0..3)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint16_t* p = rst + (8 * g + 4 * h + (l16 >> 2)) * 64 + 16 * i + 4 * (l16 & 3);
            const i16x4 r4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(i16x4, p));
            av[2 * h] = (uint16_t)r4[0] | ((uint32_t)(uint16_t)r4[1] << 16);
            av[2 * h + 1] = (uint16_t)r4[2] | ((uint32_t)(uint16_t)r4[3] << 16);
          }
        } else {
          const int jj = j0 + 8 * g;
          av = jj < a.rp ? *reinterpret_cast<const u32x4*>(a.R + (o0 + 16 * i + l16) * a.ldr + jj)
                         : u32x4{0u, 0u, 0u, 0u};
        }
        lo[k] = E::mfma16(E::as8(av), E::as8(hv[k]), lo[k]);
      }
    }
    // out = rnd(scale * sum + c * lo + bias) for rows o = o0 + 16 i + 4 g + v, token 16 tt + l16
#pragma unroll
    for (int k = 0; k < FPW; ++k) {
      const int f = w + sk::NWV * k;
      if (f >= NF) continue;
      const int i = f / T, tt = f % T;
      const int64_t tok = tok0 + 16 * tt + l16, o = o0 + 16 * i + 4 * g;
      if (tok >= a.M) continue;
      const float bv[4] = {E::lo(bsv[k][0]), E::hi(bsv[k][0]), E::lo(bsv[k][1]), E::hi(bsv[k][1])};
      uint32_t b[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float sc = a.colscale ? cs[k][v] * sum[k][v] : sum[k][v];
        b[v] = E::bits(sc + a.c * lo[k][v] + bv[v]);
      }
      *reinterpret_cast<uint2*>(a.out + tok * a.Ncols + o) = uint2{b[0] | (b[1] << 16), b[2] | (b[3] << 16)};
    }
  }
}

// ---- row-wave output tiles: a few hundred tokens on a large weight ------------------------------
// With more tokens than one 80-token block the tiles above re-read the activations once per
// 64-row block and hand split partials between blocks. A row-wave tile instead covers 64 NI
// output rows x 16 To tokens and the whole reduction in one block, so no partial leaves it: wave
// w takes rows 16 NI (w & 3) .. + 16 NI of the tile and, in step s, the 64-wide reduction chunk
// 2 s + (w >> 2); waves w and w + 4 meet once at the end. A step's operands (the activations of
// two chunks x 16 To tokens, and the block's codes) are copied from memory straight into an LDS
// ring by the buffer unit, several steps ahead (rw_acc_dma), and every wave reads its fragments
// there:
//   FWD: the codes of a step, 64 NI rows x 128 bytes, are copied as whole 128-byte row segments
//        (8 rows per copy instruction); a lane reads 16 codes of row 16 i + l16 at
//        k = 64 par + 16 g + (0..15) and feeds MFMA step e with k = 64 par + 16 g + 8 e + (0..7),
//        the activations using the same k. Converted exactly to bf16 (f16); the row scale
//        multiplies the f32 sum at the end.
//   DX:  the codes of a step, 128 rows n x 64 NI bytes k, are copied as whole row segments too;
//        a wave's [64 n][16 NI k] share reaches the MFMA through ds_read_b64_tr_b8 (lane:
//        k = 16 i + l16, n = 32 e + 8 g + (0..7)), each code scaled by s[n] from a table of the
//        block's scales in LDS: bf16(fl32(q s[n])) (f16: f16(q f16(s))), the dequantized weight
//        of the large-token dX.
// (Measured against register-staged loads: codes loaded straight in the MFMA layout touched 16
// rows' half lines per instruction (FWD) or 16 bytes of each of 64 rows (DX); whole row segments
// through LDS, then copies that bypass the registers, took 77 / 333 / 512 tokens on 5120 x 5120
// from 20.1 / 34.4 / 46.6 to 17.3 / 30.0 / 40.6 us forward and 32.0 / 56.7 / 73.0 to
// 29.1 / 43.7 / 54.2 us backward.)
// LDS rows of the activations are 128 bytes (64 bf16), their 16-byte units swizzled per row
// (rw_swz) so that the fragment reads hit distinct banks.
constexpr int align16(int v) { return (v + 15) & ~15; }

// The 16-byte unit u of activation row r sits at u ^ rw_swz<MODE>(r). A fragment read takes
// unit 2 g + e (FWD) or 4 e + g (DX) of rows r .. r + 15 in each 16-lane group g, and
// ds_read_b128 serves two 8-lane groups per pass; with these swizzles any two groups that may
// share a pass (lanes 0-7 with 16-23 or with 24-31, and so on) hit distinct banks: bits 1-2 of
// the row pick the swizzle from {0, 1, 4, 5} (FWD, never flipping unit bit 1, which separates
// g from g ^ 1) or {0, 2, 4, 6} (DX, never flipping bit 0), and bit 0 of the row already picks
// the other half of the 64 banks.
template <int MODE> __device__ __forceinline__ int rw_swz(int row) {
  return MODE == 0 ? ((row >> 1) & 1) | (((row >> 2) & 1) << 2) : ((row >> 1) & 3) << 1;
}
// Code slot of a step: FWD 64 NI rows x 128 bytes, DX 128 rows x 64 NI bytes. FWD row r's unit
// u sits at u ^ rw_wswz(r): the code reads (rows l16 of a 16-row tile, unit 4 par + g) meet
// distinct banks in a pass. DX row n's unit u sits at u ^ rw_dswz(n), so that the 16 rows of a
// transposed read's 32-lane pass (one unit each) meet distinct banks.
constexpr int rw_wslot(int NI) { return 64 * NI * 128; }
__device__ __forceinline__ int rw_wswz(int row) { return ((row >> 1) & 3) << 1; }
template <int NI> __device__ __forceinline__ int rw_dswz(int row) {
  return NI == 2 ? ((row >> 1) & 7) : ((row >> 2) & 3);
}

// The same products with both operands copied from memory straight into LDS by the buffer unit
// (buffer_load ... lds), no register staging: a ring of RS step slots (activations
// [2 par][16 To tokens][128 bytes] as above, then the codes: FWD [64 NI rows][128 bytes], units
// XOR-swizzled by rw_wswz; DX [128 n][64 NI bytes], units swizzled by rw_dswz, then the step's
// 128 scales s[n] in a 1 KiB tail, copied by wave 0), the copies of step s + L = s + RS - 1
// issued right after the barrier that opens step s. At that barrier every wave has finished
// reading the previous step's slot (lgkmcnt(0)) and waited for its own copies of step s (the
// copies of the L - 1 later steps may stay in flight), so the barrier publishes step s and frees
// slot (s - 1) % RS, which the new copies fill. Copies past the reduction read zeros (a
// 2^30-byte offset past the descriptor) into slots nobody reads; the last of them are drained
// before returning.
constexpr int rw_fstep(int To, int NI, int MODE) { return 2 * 16 * To * 128 + rw_wslot(NI) + (MODE == 1 ? 1024 : 0); }
constexpr int rw_fslots(int To, int NI, int MODE) {
  return (160 * 1024 - 16) / rw_fstep(To, NI, MODE) > 8 ? 8 : (160 * 1024 - 16) / rw_fstep(To, NI, MODE);
}

template <int To, int NI, int MODE, int ELT>
__device__ __forceinline__ void rw_acc_dma(const SkArgs& a, int64_t r0, int64_t tok0, int rot,
                                           uint8_t* smem, f32x4 (&acc)[NI][To]) {
  using E = Elt<ELT>;
  typedef typename E::v8 V8;
  constexpr int BN = 16 * To, XL = To / 2, SLOT = 2 * BN * 128, WSLOT = rw_wslot(NI);
  constexpr int RS = rw_fslots(To, NI, MODE), L = RS - 1, STEP = rw_fstep(To, NI, MODE);
  static_assert(RS >= 3, "at least two steps in flight");
  constexpr uint32_t OOB = 0x80000000u, PAST = 0x40000000u;
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wr = w & 3, par = w >> 2;
  const int l16 = lane & 15, g = lane >> 4;
  const int nsteps = (int)(a.Kred / 128);
  const i32x4 rx = buffer_rsrc(a.act, (uint32_t)(a.M * a.Kred * 2));
  const i32x4 rq = buffer_rsrc(a.q, (uint32_t)((MODE == 0 ? a.Ncols : a.Kred) * a.ldq));
  // DX: wave 0's lanes 0-31 copy a step's 128 scales (lanes 32-63 read zeros past the descriptor)
  const i32x4 rs = buffer_rsrc(a.s, (uint32_t)(MODE == 1 ? a.Kred * 4 : 0));
  const uint32_t vsc = lane < 32 ? (uint32_t)lane * 16u : OOB;
  // activations: copy j of wave w fills LDS unit (8 j + w) 64 + lane of the slot (as rw_acc)
  uint32_t vx[XL];
#pragma unroll
  for (int j = 0; j < XL; ++j) {
    const int u = (8 * j + w) * 64 + lane;
    const int p = u / (BN * 8), rem = u % (BN * 8), row = rem >> 3;
    const int col = (rem & 7) ^ rw_swz<MODE>(row);
    const int64_t tok = tok0 + row;
    vx[j] = tok < a.M ? (uint32_t)(tok * a.Kred * 2 + p * 128 + col * 16) : OOB;
  }
  // codes: copy i of wave w fills the slot's 16-byte units (NI w + i) 64 + lane. FWD: ring row
  // 8 (NI w + i) + lane / 8, unit lane % 8, which holds the row's unit (lane % 8) ^ rw_wswz(row);
  // DX: flat unit idx of [128 n][4 NI], holding unit (idx % 4 NI) ^ rw_dswz(n) of row n
  uint32_t vw[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    if constexpr (MODE == 0) {
      const int R = (NI * w + i) * 8 + (lane >> 3);
      const int64_t grow = r0 + R;
      vw[i] = grow < a.Ncols ? (uint32_t)(grow * a.ldq + 16 * ((lane & 7) ^ rw_wswz(R))) : OOB;
    } else {
      const int idx = (NI * w + i) * 64 + lane, n = idx / (4 * NI);
      const int64_t col = r0 + 16 * ((idx % (4 * NI)) ^ rw_dswz<NI>(n));
      vw[i] = col < a.Ncols ? (uint32_t)(n * a.ldq + col) : OOB;
    }
  }
  const uint32_t wstep = MODE == 0 ? 128u : (uint32_t)(128 * a.ldq);
  auto at = [&](int s) { const int v = s + rot; return v >= nsteps ? v - nsteps : v; };
  auto issue = [&](int s, int slot) {
    const bool ok = s < nsteps;
    const int sr = at(s);
    const uint32_t sx = ok ? (uint32_t)sr * 256u : PAST, sw = ok ? (uint32_t)sr * wstep : PAST;
    uint8_t* base = smem + slot * STEP;
#pragma unroll
    for (int j = 0; j < XL; ++j) dma16(rx, vx[j], sx, base + (8 * j + w) * 1024);
#pragma unroll
    for (int i = 0; i < NI; ++i) dma16(rq, vw[i], sw, base + SLOT + (NI * w + i) * 1024);
    if (MODE == 1 && w == 0) dma16(rs, vsc, ok ? (uint32_t)sr * 512u : PAST, base + SLOT + WSLOT);
  };
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int tt = 0; tt < To; ++tt) acc[i][tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // the wait that opens a step: this wave's LDS reads done, its copies of the step landed (the
  // copies of the L - 1 steps after it may stay in flight)
  constexpr int NV = (L - 1) * (XL + NI), NV0 = (L - 1) * (XL + NI + (MODE == 1 ? 1 : 0));
  static_assert(NV0 < 64, "vmcnt field");
  constexpr int WAIT = (NV & 15) | ((NV >> 4) << 14) | (7 << 4);  // lgkmcnt(0), vmcnt(NV)
  constexpr int WAIT0 = (NV0 & 15) | ((NV0 >> 4) << 14) | (7 << 4);  // wave 0 (DX: the scales)
  auto step = [&](int s, int slot) {
    if (w == 0) __builtin_amdgcn_s_waitcnt(WAIT0);
    else __builtin_amdgcn_s_waitcnt(WAIT);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue(s + L, (slot + L) % RS);
    const uint8_t* base = smem + slot * STEP;
    V8 af[NI][2];
    u32x4 cv[NI];
    if constexpr (MODE == 0) {
      // codes of rows 16 i + l16 (unit 4 par + g: k = 64 par + 16 g + (0..15)), read before the
      // activations (unit 2 g + e of the par half: k = 64 par + 16 g + 8 e + (0..7))
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int row = 16 * NI * wr + 16 * i + l16;
        cv[i] = *reinterpret_cast<const u32x4*>(base + SLOT + row * 128 + (((4 * par + g) ^ rw_wswz(row)) << 4));
      }
    }
    const uint8_t* xs = base + par * (BN * 128);
    const int sw = rw_swz<MODE>(l16);
    u32x4 xv[2][To];
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int tt = 0; tt < To; ++tt) {
        // FWD: k = 16 g + 8 e + (0..7) (unit 2 g + e); DX: n = 32 e + 8 g + (0..7) (unit 4 e + g)
        const int unit = MODE == 0 ? 2 * g + e : 4 * e + g;
        xv[e][tt] = *reinterpret_cast<const u32x4*>(xs + (16 * tt + l16) * 128 + ((unit ^ sw) << 4));
      }
    if constexpr (MODE == 0) {
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int e = 0; e < 2; ++e) af[i][e] = E::from_i8x8(cv[i][2 * e], cv[i][2 * e + 1]);
    } else {
      // per 16-k tile i and half e the transposed read: providing lane p of a 16-lane group
      // addresses row n = 64 par + 32 e + 8 g + p / 2, unit NI wr + i, bytes 8 (p % 2) .. +7;
      // lane l16 receives k = 16 (NI wr + i) + l16, n = 64 par + 32 e + 8 g + (0..7), each code
      // scaled by s[n] from the slot's scales
      const float* sc = reinterpret_cast<const float*>(base + SLOT + WSLOT) + 64 * par;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const f32x4 s0 = *reinterpret_cast<const f32x4*>(sc + 32 * e + 8 * g);
        const f32x4 s1 = *reinterpret_cast<const f32x4*>(sc + 32 * e + 8 * g + 4);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const int row = 64 * par + 32 * e + 8 * g + (l16 >> 1);
          const uint8_t* p = base + SLOT + row * (64 * NI) + (((NI * wr + i) ^ rw_dswz<NI>(row)) << 4) + 8 * (l16 & 1);
          const i32x2 v = __builtin_amdgcn_ds_read_tr8_b64_v2i32(LDS_PTR(i32x2, p));
          if constexpr (ELT == REELS_HIP_F16) {  // Float16(q) * Float16(s[n])
            const u32x4 s16 = {E::pack2(s0[0], s0[1]), E::pack2(s0[2], s0[3]),
                               E::pack2(s1[0], s1[1]), E::pack2(s1[2], s1[3])};
            af[i][e] = E::scale8(E::from_i8x8((uint32_t)v[0], (uint32_t)v[1]), s16);
          } else {  // bf16(fl32(q * s[n]))
            const uint32_t lo = (uint32_t)v[0], hi = (uint32_t)v[1];
            const u32x4 o = {E::pack2_fast((float)(int8_t)(lo & 0xffu) * s0[0], (float)(int8_t)((lo >> 8) & 0xffu) * s0[1]),
                             E::pack2_fast((float)(int8_t)((lo >> 16) & 0xffu) * s0[2], (float)((int32_t)lo >> 24) * s0[3]),
                             E::pack2_fast((float)(int8_t)(hi & 0xffu) * s1[0], (float)(int8_t)((hi >> 8) & 0xffu) * s1[1]),
                             E::pack2_fast((float)(int8_t)((hi >> 16) & 0xffu) * s1[2], (float)((int32_t)hi >> 24) * s1[3])};
            af[i][e] = E::as8(o);
          }
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int tt = 0; tt < To; ++tt)
#pragma unroll
        for (int i = 0; i < NI; ++i) acc[i][tt] = E::mfma16(af[i][e], E::as8(xv[e][tt]), acc[i][tt]);
  };
#pragma unroll
  for (int d = 0; d < L; ++d) issue(d, d);
  const int nfull = nsteps / RS * RS;
  for (int s0 = 0; s0 < nfull; s0 += RS) {
#pragma unroll
    for (int j = 0; j < RS; ++j) step(s0 + j, j);
  }
#pragma unroll
  for (int j = 0; j < RS; ++j)
    if (nfull + j < nsteps) step(nfull + j, j);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the copies past the reduction have landed
}

// lo[i][tt] (rows 16 i + 4 g + v of the wave's 16 NI, tokens of the wave's token tiles) += the
// adapter term l R over rank columns [0, rp): FWD R(o, j) = B[j][o] staged per wave in LDS and
// read transposed, DX R(k, j) = A[k][j] read straight from memory; l = h or u from the workspace
template <int NI, int TH, int MODE, int ELT>
__device__ __forceinline__ void rw_lora(const SkArgs& a, int64_t ob, int64_t tok0, uint8_t* wst,
                                        f32x4 (&lo)[NI][TH]) {
  using E = Elt<ELT>;
  const int lane = threadIdx.x & 63, l16 = lane & 15, g = lane >> 4;
  const __amdgpu_buffer_rsrc_t rl = sk_rsrc(a.hl, a.M * a.rp * 2);
  const int njc = (a.rp + 31) / 32;
  for (int jc = 0; jc < njc; ++jc) {
    const int j0 = 32 * jc;
    u32x4 hv[TH];
#pragma unroll
    for (int tt = 0; tt < TH; ++tt) {
      const int64_t tok = tok0 + 16 * tt + l16;
      const int jj = j0 + 8 * g;
      hv[tt] = u32x4{0u, 0u, 0u, 0u};
      if (tok < a.M && jj < a.rp)
        hv[tt] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rl, (uint32_t)((tok * a.rp + jj) * 2), 0, kSC1));
    }
    u32x4 av[NI];
    if constexpr (MODE == 0) {
      // rows j0 .. j0 + 31 of B, columns ob .. ob + 16 NI, into the wave's tile [32 j][16 NI o]
      // (2 NI lanes per row, 16 bytes each), then transposed 16-bit reads: providing lane p
      // addresses row 8 g + 4 h + p / 4, columns 16 i + 4 (p % 4) .. +3; lane l16 receives
      // o = 16 i + l16, j = 8 g + 4 h + (0..3)
      uint16_t* rst = reinterpret_cast<uint16_t*>(wst);
#pragma unroll
      for (int k = 0; k < NI; ++k) {
        const int idx = lane + 64 * k, row = idx / (2 * NI), c8 = 8 * (idx % (2 * NI));
        u32x4 v = u32x4{0u, 0u, 0u, 0u};
        if (j0 + row < a.r && ob + c8 < a.Ncols)
          v = *reinterpret_cast<const u32x4*>(a.R + (int64_t)(j0 + row) * a.ldr + ob + c8);
        *reinterpret_cast<u32x4*>(rst + row * (16 * NI) + c8) = v;
      }
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint16_t* p = rst + (8 * g + 4 * h + (l16 >> 2)) * (16 * NI) + 16 * i + 4 * (l16 & 3);
          const i16x4 r4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(i16x4, p));
          av[i][2 * h] = (uint16_t)r4[0] | ((uint32_t)(uint16_t)r4[1] << 16);
          av[i][2 * h + 1] = (uint16_t)r4[2] | ((uint32_t)(uint16_t)r4[3] << 16);
        }
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int64_t k = ob + 16 * i + l16;
        const int jj = j0 + 8 * g;
        av[i] = (k < a.Ncols && jj < a.rp) ? *reinterpret_cast<const u32x4*>(a.R + k * a.ldr + jj)
                                           : u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int tt = 0; tt < TH; ++tt) lo[i][tt] = E::mfma16(E::as8(av[i]), E::as8(hv[tt]), lo[i][tt]);
  }
}

// One row-wave output tile: the wave's accumulators, the pair sum of waves w and w + 4 (each
// keeps half the token tiles), l when the adapter blocks have published it (or computed here with
// their code, splits and order when they have not), then out = rnd(scale sum + c l R + bias).
template <int To, int NI, int Ta, int MODE, int ELT>
__device__ __forceinline__ void rw_block(const SkArgs& a, int rb, int tbo, uint8_t* smem,
                                         int lds_bytes) {
  using E = Elt<ELT>;
  constexpr int TH = To / 2;
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wr = w & 3, par = w >> 2;
  const int l16 = lane & 15, g = lane >> 4;
  const int64_t r0 = (int64_t)rb * (64 * NI), tok0 = (int64_t)tbo * (16 * To);
  const int64_t ob = r0 + 16 * NI * wr;          // the wave's first output row
  const int64_t tw0 = tok0 + (int64_t)par * (16 * TH);  // the wave's first token after the pair sum
  uint32_t* words = reinterpret_cast<uint32_t*>(smem + lds_bytes - 16);  // [0], [3] key, [2] l ready
  const bool wants_l = a.nad > 0;
  sk_stash_key(words);

  f32x4 sum[NI][TH];
  {
    f32x4 acc[NI][To];
    // The walk over the reduction starts at a rotation per XCD (block b runs on XCD b % 8): the
    // blocks of one XCD walk together, so the activations of a token tile that several row
    // blocks read meet in that XCD's L2, and the 8 XCDs' weight reads spread over the channels.
    // (A rotation per row block spread the channels as well but re-fetched the activations per
    // row block: 512 tokens on 5120 x 5120 40.4 against 35.1 us forward.)
    const int nsteps = (int)(a.Kred / 128);
    const int rot = (int)(((int64_t)(blockIdx.x & 7) * nsteps) / 8);
    rw_acc_dma<To, NI, MODE, ELT>(a, r0, tok0, rot, smem, acc);
    // waves 4-7 give their first half of the token tiles, waves 0-3 their second, through LDS;
    // each then adds (partner + own, wave w's value first: the same sum for both halves)
    f32x4* ex = reinterpret_cast<f32x4*>(smem);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int tt = 0; tt < TH; ++tt)
        ex[((w * NI + i) * TH + tt) * 64 + lane] = acc[i][par == 0 ? TH + tt : tt];
    __syncthreads();
    const int pw = w ^ 4;
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int tt = 0; tt < TH; ++tt) {
        const f32x4 other = ex[((pw * NI + i) * TH + tt) * 64 + lane];
        const f32x4 own = acc[i][par == 0 ? tt : TH + tt];
        sum[i][tt] = par == 0 ? own + other : other + own;
      }
    __syncthreads();  // LDS free again
  }

  if (wants_l) {
    // the adapter tiles of this tile's tokens: they come first in the logical order and wait for
    // nothing but their splits, so their keys are normally there; after a bounded wait the block
    // computes l for its tokens itself, with the adapter blocks' code, splits and order (the same
    // bits)
    const int tb_lo = (int)(tok0 / (16 * Ta));
    const int tb_hi = std::min((int)((tok0 + 16 * To + 16 * Ta - 1) / (16 * Ta)), a.tb);
    if (t == 0) {
      const u32x4 key = sk_key(a, words);
      uint32_t rounds = 0, ok = 1;
      for (int lb = 0; lb < a.lblk && ok; ++lb)
        for (int tba = tb_lo; tba < tb_hi && ok; ++tba) ok = sk_wait_key(a, lb * a.tb + tba, key, rounds);
      words[2] = ok;
    }
    __syncthreads();
    if (words[2] == 0u) {
      for (int tba = tb_lo; tba < tb_hi; ++tba)
        for (int lb = 0; lb < a.lblk; ++lb) {
          constexpr int FA = sk_fpw<2 * Ta>();
          f32x4 tl[FA];
#pragma unroll
          for (int k = 0; k < FA; ++k) tl[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          for (int s = 0; s < a.S; ++s) {
            f32x4 acc[2][Ta], ps[FA];
            skinny_acc<Ta, MODE, ELT, true>(a, a.nblk + lb, s, (int64_t)tba * (16 * Ta), smem, acc);
            skinny_sum<Ta, 2>(acc, smem, ps);
#pragma unroll
            for (int k = 0; k < FA; ++k) tl[k] += ps[k];
          }
          skinny_put_l<Ta, ELT>(a, (int64_t)lb * sk::NBL, (int64_t)tba * (16 * Ta), tl, false);
        }
      sk_drain();
      __syncthreads();
    }
    asm volatile("" ::: "memory");
  }

  f32x4 lo[NI][TH];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int tt = 0; tt < TH; ++tt) lo[i][tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if (wants_l) rw_lora<NI, TH, MODE, ELT>(a, ob, tw0, smem + w * (1024 * NI), lo);

  // out = rnd(scale * sum + c * lo + bias), rows o = ob + 16 i + 4 g + v, token 16 tt + l16
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int64_t o = ob + 16 * i + 4 * g;
    if (o >= a.Ncols) continue;
    f32x4 cs = f32x4{1.0f, 1.0f, 1.0f, 1.0f};
    if (a.colscale) cs = *reinterpret_cast<const f32x4*>(a.colscale + o);
    u32x2 bsv = u32x2{0u, 0u};
    if (a.bias) bsv = *reinterpret_cast<const u32x2*>(a.bias + o);
    const float bv[4] = {E::lo(bsv[0]), E::hi(bsv[0]), E::lo(bsv[1]), E::hi(bsv[1])};
#pragma unroll
    for (int tt = 0; tt < TH; ++tt) {
      const int64_t tok = tw0 + 16 * tt + l16;
      if (tok >= a.M) continue;
      uint32_t b[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float sc = a.colscale ? cs[v] * sum[i][tt][v] : sum[i][tt][v];
        b[v] = E::bits(sc + a.c * lo[i][tt][v] + bv[v]);
      }
      *reinterpret_cast<uint2*>(a.out + tok * a.Ncols + o) = uint2{b[0] | (b[1] << 16), b[2] | (b[3] << 16)};
    }
  }
}

template <int To, int NI, int Ta, int MODE, int ELT>
__global__ __launch_bounds__(64 * sk::NWV, 1) void skinny_rw_kernel(SkArgs a, int lds_bytes) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  // the logical order and XCD mapping of skinny_kernel: adapter blocks first, then the output
  // tiles with the token tile fastest, so the tiles that read the same weight rows run on one
  // XCD, close in time
  const int b = (int)blockIdx.x, xcd = b & 7, idx = b >> 3;
  const int per = a.blocks >> 3, rem = a.blocks & 7;
  const int tk = xcd * per + (xcd < rem ? xcd : rem) + idx;
  if (tk < a.nad) {
    int rest = tk;
    SkBlock d;
    d.tb = rest % a.tb;
    rest /= a.tb;
    d.sp = rest % a.S;
    const int rb = rest / a.S;
    d.blk = a.nblk + rb;
    d.tile = a.ntm + rb * a.tb + d.tb;
    skinny_block<Ta, MODE, ELT, true>(a, d, smem);
  } else {
    const int ti = tk - a.nad;
    rw_block<To, NI, Ta, MODE, ELT>(a, ti / a.otb, ti % a.otb, smem, lds_bytes);
  }
}

template <int T, int MODE, int ELT>
__global__ __launch_bounds__(64 * sk::NWV, 1) void skinny_kernel(SkArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  // logical order: adapter blocks, then output blocks; within each (row block, split, token
  // block) with the token block fastest. Block b runs on XCD b % 8, and each XCD takes a
  // contiguous range of the logical order, so the token blocks that read the same weight rows
  // run on one XCD, close in time, and share those rows through its L2.
  const int b = (int)blockIdx.x, xcd = b & 7, idx = b >> 3;
  const int per = a.blocks >> 3, rem = a.blocks & 7;
  const int tk = xcd * per + (xcd < rem ? xcd : rem) + idx;
  const bool lora = tk < a.nad;
  int rest = lora ? tk : tk - a.nad;
  SkBlock d;
  d.tb = rest % a.tb;
  rest /= a.tb;
  d.sp = rest % a.S;
  const int rb = rest / a.S;
  d.blk = lora ? a.nblk + rb : rb;
  d.tile = lora ? a.ntm + rb * a.tb + d.tb : rb * a.tb + d.tb;
  if (lora) skinny_block<T, MODE, ELT, true>(a, d, smem);
  else skinny_block<T, MODE, ELT, false>(a, d, smem);
}

// Row-wave tiles (NI, To) for a launch: the candidates whose output tiles and adapter blocks fit
// one round of the 256 CUs and fill most of it (or, on short reductions, some of it); among them
// the least estimated clocks per
// 128-deep step on a CU (the largest of the matrix cores, the LDS reads, the vector memory and,
// for dX, the VALU scaling of the codes), then the least padded work.
struct RwCand { int NI, To; };
constexpr RwCand kRwCands[] = {{1, 2}, {1, 4}, {2, 4}, {2, 6}};
constexpr int kRwLdsMax = 160 * 1024;

static int rw_lds_bytes(int NI, int To, int mode, int64_t Kred) {
  const int slot = 2 * 16 * To * 128, ta = To <= 4 ? To : To / 2;
  (void)Kred;
  int v = rw_fslots(To, NI, mode) * rw_fstep(To, NI, mode);
  v = std::max(v, 8 * NI * (To / 2) * 1024);
  v = std::max(v, skinny_lds(ta));
  v = std::max(v, 8 * 1024 * NI);
  return v + 16;
}

static bool rw_choose(int64_t M, int64_t Kred, int64_t Ncols, int rp, int mode, SkinnyPlan& out) {
  if (M <= 0 || Kred % 128 != 0 || Ncols % 64 != 0 || Kred > 16384) return false;
  // the kernel moves steps past the operands with a scalar offset of 2^30 bytes
  if (M * Kred * 2 > ((int64_t)1 << 30) || Ncols * Kred > ((int64_t)1 << 30)) return false;
  // Tiles that fill most of the GPU; on reductions up to 4096 deep also fewer (down to 32): a
  // whole-reduction tile there is short, and beats split tiles that hand partials over (77 tokens
  // on 1536 x 1536 forward 15.7 -> 10.4 us, backward 20.7 -> 15.2 us; the 4096-deep dX of 160
  // tokens on 1024 -> 4096 backward 34.8 -> 25.9 us), while on longer ones the split tiles win
  // (3 tokens on 5120 x 5120 forward 11.6 against 13.9 us; the 8960-deep dX of 77 tokens on
  // 1536 -> 8960 backward 28.3 against 36.6 us)
  const int64_t min_tiles = Kred <= 4096 ? 32 : kSkinnyTargetBlocks / 2;
  bool found = false;
  int64_t best_cost = 0, best_work = 0;
  for (const RwCand& c : kRwCands) {
    const int64_t orb = ceil_div(Ncols, 64 * c.NI), otb = ceil_div(M, 16 * c.To);
    const int ta = c.To <= 4 ? c.To : c.To / 2;
    const int64_t tba = ceil_div(M, 16 * ta), lblk = ceil_div(rp, sk::NBL);
    const int64_t tiles = orb * otb, nad = rp > 0 ? lblk * tba : 0;
    if (tiles + nad > kSkinnyTargetBlocks || tiles < min_tiles) continue;
    if (rw_lds_bytes(c.NI, c.To, mode, Kred) > kRwLdsMax) continue;
    const int64_t mf = 64 * c.NI * c.To, lds = 128 * c.To, vm = 128 * c.NI + 64 * c.To;
    const int64_t valu = (mode == 1 ? 384 : 192) * c.NI;
    const int64_t cost = std::max(std::max(mf, lds), std::max(vm, valu));
    const int64_t work = orb * 64 * c.NI * otb * 16 * c.To;
    if (!found || cost < best_cost || (cost == best_cost && work < best_work)) {
      found = true;
      best_cost = cost;
      best_work = work;
      out.rw = true;
      out.NI = c.NI; out.To = c.To;
      out.orb = (int)orb; out.otb = (int)otb;
      out.T = ta; out.tb = (int)tba;
      // adapter splits: as many as the round leaves room for (shorter adapter blocks publish l
      // sooner), each wave at least one chunk
      int64_t S = nad > 0 ? (kSkinnyTargetBlocks - tiles) / nad : 1;
      if (S > Kred / sk::KC / 4) S = Kred / sk::KC / 4;
      if (S > sk::MAXS) S = sk::MAXS;
      if (S < 1) S = 1;
      out.S = (int)S;
    }
  }
  return found;
}

static bool skinny_limits(int64_t M, int64_t K, int64_t N, int rp) {
  // the reduction in whole 64-chunks, whole 64-row blocks, 32-bit buffer offsets (with room for
  // the token-block overrun), a bounded tile count
  const int64_t tb = ceil_div(M, 16 * sk::MAXT);
  const int64_t mx = K > N ? K : N;
  return M > 0 && K % 64 == 0 && N % 64 == 0 &&
         (M + 128) * mx * 2 < ((int64_t)1 << 31) && N * K < ((int64_t)1 << 31) &&
         (int64_t)rp * mx * 2 < ((int64_t)1 << 31) && rp <= 4096 &&
         (mx / sk::NB + ceil_div(rp, sk::NBL)) * tb <= sk::kMaxTiles;
}

bool skinny_supported(int64_t M, int64_t K, int64_t N, int rp) {
  if (!skinny_limits(M, K, N, rp)) return false;
  // up to 240 tokens, or up to 1024 on a small weight (at most 4M elements, which stays in L2
  // across the token blocks): there one launch beats the 256 x 256-tile GEMM's few tiles
  if (M <= kSkinnyMaxTokens || (M <= kSkinnySmallWeightTokens && N * K <= ((int64_t)1 << 22)))
    return true;
  // a few hundred tokens on a large weight: row-wave tiles in both directions
  SkinnyPlan f, d;
  return M <= kSkinnySmallWeightTokens && rw_choose(M, K, N, rp, 0, f) && rw_choose(M, N, K, rp, 1, d);
}

SkinnyPlan skinny_plan(int64_t M, int64_t Kred, int64_t Ncols, int rp, int mode) {
  SkinnyPlan p;
  // row-wave tiles wherever they fill the GPU (with the codes loaded as whole row segments they
  // beat the split tiles in both directions: 77 tokens on 5120 x 5120, dX + dA + dB 29.5 against
  // 32.0 us), split tiles elsewhere
  if (rw_choose(M, Kred, Ncols, rp, mode, p)) return p;
  p.tb = (int)ceil_div(M, 16 * sk::MAXT);
  p.T = (int)ceil_div(ceil_div(M, p.tb), 16);
  const int64_t blocks = (Ncols / sk::NB + ceil_div(rp, sk::NBL)) * p.tb;
  const int64_t nc = Kred / sk::KC;
  // about one block per CU, each wave at least one chunk
  int64_t S = (kSkinnyTargetBlocks + blocks / 2) / (blocks > 0 ? blocks : 1);
  if (S > nc / 4) S = nc / 4;
  if (S > sk::MAXS) S = sk::MAXS;
  if (S < 1) S = 1;
  p.S = (int)S;
  return p;
}

// workspace of one launch: split partials, l [M][rp], then the keys; the offsets are the same in
// sizing and use
struct SkWs {
  size_t part, hl, keys, total;
  int ntiles;
};
static SkWs skinny_ws(const SkinnyPlan& p, int64_t M, int64_t Ncols, int rp) {
  SkWs w;
  // split partials in MFMA fragments: the output tiles' (none for row-wave tiles), then the
  // adapter tiles'
  const size_t ofrags = p.rw ? 0 : (size_t)(Ncols / sk::NB) * p.tb * (4 * p.T);
  const size_t frags = ofrags + (size_t)ceil_div(rp, sk::NBL) * p.tb * (2 * p.T);
  const int64_t otiles = p.rw ? (int64_t)p.orb * p.otb : (Ncols / sk::NB) * p.tb;
  w.ntiles = (int)(otiles + ceil_div(rp, sk::NBL) * p.tb);
  w.part = 0;
  w.hl = align_up(p.S > 1 ? frags * p.S * 64 * 16 : 0, 256);
  w.keys = align_up(w.hl + (size_t)M * rp * 2, 256);
  // 16-byte keys: one per adapter tile (l stored), then one per tile and split (partial stored)
  const size_t nta = (size_t)ceil_div(rp, sk::NBL) * p.tb;
  w.total = align_up(w.keys + (nta + (size_t)w.ntiles * p.S) * 16, 256);
  return w;
}

size_t skinny_ws_bytes(const SkinnyPlan& p, int64_t M, int64_t Ncols, int rp) {
  return skinny_ws(p, M, Ncols, rp).total;
}

template <int MODE, int ELT, int T>
static hipError_t launch_skinny_t(const SkArgs& a, hipStream_t st) {
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [] {
    attr = hipFuncSetAttribute((const void*)skinny_kernel<T, MODE, ELT>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, skinny_lds(T));
  });
  if (attr != hipSuccess) return attr;
  skinny_kernel<T, MODE, ELT><<<dim3((unsigned)a.blocks), 64 * sk::NWV, skinny_lds(T), st>>>(a);
  return hipSuccess;
}

template <int To, int NI, int Ta, int MODE, int ELT>
static hipError_t launch_rw_t(const SkArgs& a, int lds, hipStream_t st) {
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [] {
    attr = hipFuncSetAttribute((const void*)skinny_rw_kernel<To, NI, Ta, MODE, ELT>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, kRwLdsMax);
  });
  if (attr != hipSuccess) return attr;
  skinny_rw_kernel<To, NI, Ta, MODE, ELT><<<dim3((unsigned)a.blocks), 64 * sk::NWV, lds, st>>>(a, lds);
  return hipSuccess;
}

// the nonce of a row-wave launch's keys: a process-wide count from a random start (so two
// processes, or two calls, do not share one)
static uint64_t sk_next_nonce() {
  static std::atomic<uint64_t> next{[] {
    std::random_device rd;
    const uint64_t t = (uint64_t)std::chrono::steady_clock::now().time_since_epoch().count();
    return (((uint64_t)rd() << 32) ^ (uint64_t)rd() ^ (t * 0x9E3779B97F4A7C15ull));
  }()};
  return next.fetch_add(1, std::memory_order_relaxed);
}

int launch_skinny(int mode, int elt, const SkinnyPlan& p, const uint16_t* act, const int8_t* q,
                  int64_t ldq, const float* s, const uint16_t* lw, void* ws, int64_t M,
                  int64_t Kred, int64_t Ncols, int r, int rp, const float* colscale,
                  const uint16_t* R, int64_t ldr, const uint16_t* bias, float c, uint16_t* out,
                  uint16_t* lsave, int64_t ld_lsave, int lsave_cols, hipStream_t st,
                  bool adapter_only) {
  SkArgs a;
  a.act = act; a.q = q; a.s = s; a.lw = lw;
  a.M = M; a.Kred = Kred; a.Ncols = Ncols; a.ldq = ldq;
  a.r = r; a.rp = r > 0 ? rp : 0; a.S = p.S;
  a.nblk = (int)(Ncols / sk::NB);
  a.lblk = (int)ceil_div(a.rp, sk::NBL);
  a.tb = p.tb;
  a.colscale = colscale; a.R = R; a.ldr = ldr; a.bias = bias; a.c = c;
  a.out = out; a.lsave = lsave; a.ld_lsave = ld_lsave; a.lsave_cols = lsave_cols;
  a.ntm = adapter_only ? 0 : (p.rw ? p.orb * p.otb : a.nblk * p.tb);
  a.nta = a.lblk * p.tb;
  a.otb = p.otb;
  a.lpart0 = p.rw ? 0 : (int64_t)a.ntm * p.S * (4 * p.T * 64);
  // REELS_HIP_SKINNY_SPIN (tests): wait rounds before an output tile computes l itself; 0 makes
  // every output tile take that path
  a.spin = sk::kSpinLimit;
  if (const char* e = std::getenv("REELS_HIP_SKINNY_SPIN")) a.spin = (uint32_t)std::strtoul(e, nullptr, 10);
  a.nad = a.nta * p.S;
  a.blocks = a.nad + a.ntm * (p.rw ? 1 : p.S);
  if (a.blocks <= 0) return REELS_HIP_OK;
  const SkWs w = skinny_ws(p, M, Ncols, a.rp);
  uint8_t* wb = static_cast<uint8_t*>(ws);
  a.part = reinterpret_cast<float*>(wb + w.part);
  uint16_t* hl = reinterpret_cast<uint16_t*>(wb + w.hl);
  // l straight into lsave when the layouts agree
  a.hl = (lsave != nullptr && ld_lsave == a.rp && lsave_cols >= a.rp) ? lsave : hl;
  a.keys = reinterpret_cast<uint32_t*>(wb + w.keys);
  const uint64_t nonce = sk_next_nonce();
  a.nonce_lo = (uint32_t)nonce;
  a.nonce_hi = (uint32_t)(nonce >> 32);

  hipError_t attr = hipSuccess;
  if (p.rw) {
    TraceScope _ts(st, mode == 0 ? "skinny_rw_kernel<0>" : "skinny_rw_kernel<1>");
    const int lds = rw_lds_bytes(p.NI, p.To, mode, Kred);
    with_elt(elt, [&](auto el) {
      constexpr int EL = decltype(el)::value;
      auto go = [&](auto m) {
        constexpr int MD = decltype(m)::value;
        if (p.NI == 1 && p.To == 2) attr = launch_rw_t<2, 1, 2, MD, EL>(a, lds, st);
        else if (p.NI == 1 && p.To == 4) attr = launch_rw_t<4, 1, 4, MD, EL>(a, lds, st);
        else if (p.NI == 2 && p.To == 4) attr = launch_rw_t<4, 2, 4, MD, EL>(a, lds, st);
        else attr = launch_rw_t<6, 2, 3, MD, EL>(a, lds, st);
      };
      if (mode == 0) go(std::integral_constant<int, 0>{});
      else go(std::integral_constant<int, 1>{});
    });
  } else {
    TraceScope _ts(st, mode == 0 ? "skinny_kernel<0>" : "skinny_kernel<1>");
    with_elt(elt, [&](auto el) {
      constexpr int EL = decltype(el)::value;
      auto go = [&](auto m) {
        constexpr int MD = decltype(m)::value;
        switch (p.T) {
          case 1: attr = launch_skinny_t<MD, EL, 1>(a, st); break;
          case 2: attr = launch_skinny_t<MD, EL, 2>(a, st); break;
          case 3: attr = launch_skinny_t<MD, EL, 3>(a, st); break;
          case 4: attr = launch_skinny_t<MD, EL, 4>(a, st); break;
          default: attr = launch_skinny_t<MD, EL, 5>(a, st); break;
        }
      };
      if (mode == 0) go(std::integral_constant<int, 0>{});
      else go(std::integral_constant<int, 1>{});
    });
  }
  if (attr != hipSuccess)
    return fail(REELS_HIP_EHIP, std::string("skinny_kernel: hipFuncSetAttribute: ") + hipGetErrorString(attr));
  return check_launch("skinny_kernel");
}

}  // namespace reels
