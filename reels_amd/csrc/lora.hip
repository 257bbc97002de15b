// LoRA-side kernels and the forward/backward entry points of the int8 LoRA linear.
//
// Forward (lora_forward, src/layers/lora.jl:56-95):
//   1. transpose A [K][r] -> At [r][K], B [r][N] -> Bt [N][rp]           (tiny)
//   2. rowproj:  h = bf16(x * A)                      [M][rp]            (HBM-bound, reads x once)
//   3. i8gemm<FWD>: y = bf16(s * (x q^T) + c * h Bt^T + bias)            (MFMA-bound)
// Backward (lora_backward, lora.jl:106-118):
//   1. rowproj (+ scaled copy): u = bf16(dy * B^T), dys = bf16(dy * s)   (reads dy once)
//   2. i8gemm<DX>: dx = bf16(dys q + c * u A^T)                          (MFMA-bound)
//   3. colgrad: dA = c x^T u, dB = c (dy^T h)^T as split-M partials, then a fixed-order sum
//      (no float atomics: bitwise reproducible)                          (HBM-bound)
// Every rank takes the fast kernels: the LoRA panels h, u and the adapter operands live in the
// workspace with rp = round_up(r, 16) columns (zeros past r), and the projection and gradient
// kernels run in rank chunks of up to 128. Shapes the fast kernels do not take (K or N not
// multiples of 16, unaligned pointers) run through the generic kernels at the bottom, which
// compute the same formulas with the same bf16 rounding points, one output element per thread.
#include "i8gemm.h"

#include <mutex>

namespace reels {



// ---------------------------------------------------------------------------------------------
// transpose: out[c][r] = in[r][c] for r < rows, zero for rows <= r < rows_pad (bf16)
// up to two transposes in one launch: job 0 takes the first nb0 blocks; a job's blocks are 32 x 32
// tiles, column tile fastest
struct TpJob {
  const uint16_t* in;
  uint16_t* out;
  int64_t rows, cols, rows_pad;
  int gx;  // column tiles
};
__global__ void transpose_pad_kernel(TpJob j0, TpJob j1, int nb0) {
  __shared__ uint16_t tile[32][33];
  const bool second = (int)blockIdx.x >= nb0;
  const int b = second ? (int)blockIdx.x - nb0 : (int)blockIdx.x;
  const uint16_t* __restrict__ in = second ? j1.in : j0.in;
  uint16_t* __restrict__ out = second ? j1.out : j0.out;
  const int64_t rows = second ? j1.rows : j0.rows, cols = second ? j1.cols : j0.cols;
  const int64_t rows_pad = second ? j1.rows_pad : j0.rows_pad;
  const int gx = second ? j1.gx : j0.gx;
  const int64_t r0 = (int64_t)(b / gx) * 32, c0 = (int64_t)(b % gx) * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 256 threads: 32 x 8
  for (int i = ty; i < 32; i += 8) {
    const int64_t r = r0 + i, c = c0 + tx;
    tile[i][tx] = (r < rows && c < cols) ? in[r * cols + c] : (uint16_t)0;
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int64_t c = c0 + i, r = r0 + tx;
    if (c < cols && r < rows_pad) out[c * rows_pad + r] = tile[tx][i];
  }
}

// ---------------------------------------------------------------------------------------------
// rowproj: out[m][j] = bf16(sum_k src[m][k] * P[j][k]) for j < r, 0 for r <= j < rp (rp <= 128;
// out rows of ld_out elements). src [M][Kd] bf16 (x or dy), P [r][Kd] bf16 (At or B). Ranks above
// 128 run as launches over rank chunks of 128 (P and out advanced). When SCALED, also writes
// scaled[m][k] = bf16(src[m][k] * s[k]) (the dy * s operand of the DX GEMM).
// HBM-bound: a block of 256 threads owns ROWS rows (32 or 64) and streams them in chunks of 256
// columns. Each wave-instruction loads two contiguous 512-byte row segments; the chunk goes to a
// padded LDS tile (row stride 528 bytes: 8 consecutive rows fall in distinct banks) while the
// next chunk is already in flight into registers. Wave w multiplies columns [64w, 64w+64) of the
// chunk on MFMA (A = 32 src rows per row group, B = 32 rows of P staged the same way); the four
// wave partials are summed in wave order at the end. Every block streams all of P (r x Kd, from
// L2), so 64-row blocks halve that traffic per output row; 32-row blocks are used when there are
// too few tokens to give every CU a 64-row block.
namespace rowp {
constexpr int KC = 256, LROW = KC + 8;  // LDS row: 264 bf16 = 528 bytes
}  // namespace rowp

// With part set (few tokens), blockIdx.y splits the columns: the block streams chunks
// [c0, c1) of its rows and writes its f32 sums to part[split][m][rp_]; rowproj_reduce_kernel then
// sums the splits in order and rounds once.
template <int RT, bool SCALED, int ROWS, int ELT>
__global__ __launch_bounds__(256) void rowproj_kernel(const uint16_t* __restrict__ src, int64_t M,
                                                      int64_t Kd, const uint16_t* __restrict__ P,
                                                      int r, int rp_, uint16_t* __restrict__ out,
                                                      int ld_out, const float* __restrict__ s,
                                                      uint16_t* __restrict__ scaled,
                                                      float* __restrict__ part) {
  using E = Elt<ELT>;
  typedef typename E::v8 V8;
  using namespace rowp;
  constexpr int RG = ROWS / 32;  // 32-row MFMA groups
  __shared__ __attribute__((aligned(16))) uint16_t xs[ROWS * LROW];
  __shared__ __attribute__((aligned(16))) uint16_t ps[32 * RT * LROW];
  __shared__ float red[RG][RT][16][64];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int l32 = lane & 31, lhi = lane >> 5;
  const int64_t m0 = (int64_t)blockIdx.x * ROWS;
  const int nchunks = (int)((Kd + KC - 1) / KC);
  const int ks = (int)gridDim.y, sp = (int)blockIdx.y;
  const int cbeg = (int)((int64_t)sp * nchunks / ks), cend = (int)((int64_t)(sp + 1) * nchunks / ks);
  // loader roles: X chunk = ROWS rows x 32 16-byte chunks, ROWS/8 per thread; P chunk = 32RT
  // rows, 4RT per thread
  // two register stages: the copies of chunks ck + 1 and ck + 2 are in flight while chunk ck is
  // multiplied
  typedef u32x4 XS[ROWS / 8];
  typedef u32x4 PS[4 * RT];
  XS rx0, rx1;
  PS rp0, rp1;
  // Buffer loads: a descriptor over this block's rows of src (and one over P) returns zeros for
  // offsets past its end, so rows past M, columns past Kd (offset moved out of range) and chunks
  // past the last need no branch. Branch-free loads keep the compiler's waits exact: a stash
  // waits only for its own stage.
  const int64_t rows_here = (M - m0) < ROWS ? (M - m0) : ROWS;
  const __amdgpu_buffer_rsrc_t rsx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(src + m0 * Kd), (short)0, (int)(rows_here * Kd * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsp = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(r > 0 ? P : src), (short)0, r > 0 ? (int)(r * Kd * 2) : 0, 0x00020000);
  auto load = [&](int ck, XS& rx, PS& rpv) {
    const int64_t k0 = (int64_t)ck * KC;
    const bool in = ck < cend;  // chunks of the next split read zeros
#pragma unroll
    for (int i = 0; i < ROWS / 8; ++i) {
      const int row = (t >> 5) + 8 * i, c = t & 31;
      const int64_t k = k0 + c * 8;
      const uint32_t off = (in && k < Kd) ? (uint32_t)((row * Kd + k) * 2) : 0x80000000u;
      rx[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsx, off, 0, 2));  // nt
    }
#pragma unroll
    for (int i = 0; i < 4 * RT; ++i) {
      const int row = (t >> 5) + 8 * i, c = t & 31;
      const int64_t k = k0 + c * 8;
      const uint32_t off = (in && k < Kd) ? (uint32_t)((row * Kd + k) * 2) : 0x80000000u;
      rpv[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsp, off, 0, 0));
    }
  };
  auto stash = [&](int ck, const XS& rx, const PS& rpv) {
    const int64_t k0 = (int64_t)ck * KC;
#pragma unroll
    for (int i = 0; i < ROWS / 8; ++i) {
      const int row = (t >> 5) + 8 * i, c = t & 31;
      *reinterpret_cast<u32x4*>(&xs[row * LROW + c * 8]) = rx[i];
      if (SCALED) {
        const int64_t m = m0 + row, k = k0 + c * 8;
        if (m < M && k < Kd && ck < cend) {
          const f32x4 sa = *reinterpret_cast<const f32x4*>(s + k);
          const f32x4 sb = *reinterpret_cast<const f32x4*>(s + k + 4);
          const u32x4 x = rx[i];
          u32x4 o;
          o[0] = E::pack2(E::lo(x[0]) * sa[0], E::hi(x[0]) * sa[1]);
          o[1] = E::pack2(E::lo(x[1]) * sa[2], E::hi(x[1]) * sa[3]);
          o[2] = E::pack2(E::lo(x[2]) * sb[0], E::hi(x[2]) * sb[1]);
          o[3] = E::pack2(E::lo(x[3]) * sb[2], E::hi(x[3]) * sb[3]);
          *reinterpret_cast<u32x4*>(scaled + m * Kd + k) = o;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4 * RT; ++i) {
      const int row = (t >> 5) + 8 * i, c = t & 31;
      *reinterpret_cast<u32x4*>(&ps[row * LROW + c * 8]) = rpv[i];
    }
  };
  f32x16 acc[RG][RT];
#pragma unroll
  for (int g = 0; g < RG; ++g)
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[g][j][v] = 0.0f;
  auto compute = [&]() {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int col = wave * 64 + ks * 16 + lhi * 8;
      V8 a[RG];
#pragma unroll
      for (int g = 0; g < RG; ++g)
        a[g] = E::as8(*reinterpret_cast<const u32x4*>(&xs[(g * 32 + l32) * LROW + col]));
#pragma unroll
      for (int j = 0; j < RT; ++j) {
        const V8 bv = E::as8(*reinterpret_cast<const u32x4*>(&ps[(j * 32 + l32) * LROW + col]));
#pragma unroll
        for (int g = 0; g < RG; ++g)
          acc[g][j] = E::mfma32(a[g], bv, acc[g][j]);
      }
    }
  };
  // chunk ck: its registers to LDS, the copies of chunk ck + 2 into the freed registers, the
  // MFMAs on chunk ck
  // (a chunk past the end reads only zeros: its columns are past Kd)
  auto step = [&](int ck, XS& rx, PS& rpv) {
    stash(ck, rx, rpv);
    __syncthreads();
    load(ck + 2, rx, rpv);
    compute();
    __syncthreads();
  };
  // steps in pairs, the second unconditional (with an odd chunk count the last one is all
  // zeros): a branch around it would make the compiler's waits drain both stages
  load(cbeg, rx0, rp0);
  load(cbeg + 1, rx1, rp1);
  for (int ck = cbeg; ck < cend; ck += 2) {
    step(ck, rx0, rp0);
    step(ck + 1, rx1, rp1);
  }
  if (out == nullptr) return;
  // D lane layout: row (token) = g*32 + (v/4)*8 + lhi*4 + v%4, column (j) = t*32 + l32.
  // Sum the four wave partials in wave order (deterministic), one wave at a time.
  for (int w = 0; w < 4; ++w) {
    if (wave == w) {
#pragma unroll
      for (int g = 0; g < RG; ++g)
#pragma unroll
        for (int j = 0; j < RT; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            red[g][j][v][lane] = (w == 0 ? 0.0f : red[g][j][v][lane]) + acc[g][j][v];
    }
    __syncthreads();
  }
  for (int idx = t; idx < ROWS * 32 * RT; idx += 256) {
    const int g = idx / (1024 * RT), j0 = (idx / 1024) % RT, rem = idx % 1024;
    const int row = rem / 32, col = rem % 32;
    const int v = (row / 8) * 4 + (row % 4), ln = ((row / 4) & 1) * 32 + col;
    const float sum = red[g][j0][v][ln];
    const int64_t mm = m0 + g * 32 + row;
    const int j = j0 * 32 + col;
    if (part != nullptr) {
      if (mm < M && j < rp_) part[((int64_t)sp * M + mm) * rp_ + j] = sum;
    } else {
      if (mm < M && j < rp_) out[mm * ld_out + j] = j < r ? (uint16_t)E::bits(sum) : (uint16_t)0;
    }
  }
}

// out[m][j] = rnd(sum over splits of part[sp][m][j]) in split order (j < r; zeros up to rp)
template <int ELT>
__global__ __launch_bounds__(256) void rowproj_reduce_kernel(const float* __restrict__ part, int ks,
                                                             int64_t M, int r, int rp,
                                                             uint16_t* __restrict__ out, int ld_out) {
  using E = Elt<ELT>;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * rp) return;
  const int64_t m = i / rp;
  const int j = (int)(i - m * rp);
  float sum = 0.0f;
  for (int sp = 0; sp < ks; ++sp) sum += part[((int64_t)sp * M + m) * rp + j];
  out[m * ld_out + j] = j < r ? (uint16_t)E::bits(sum) : (uint16_t)0;
}

// ---------------------------------------------------------------------------------------------
// colgrad partials: part[sp][o][j] = sum over this split's tokens of src[m][o] * Lm[m][j]
// (o < Od output index, j < rp <= 128; Lm rows of ld_lm, part rows of ld_part elements; ranks
// above 128 run as launches over rank chunks). D = src^T Lm on MFMA; both operands need 8 consecutive tokens
// per lane, read transposed out of row-major LDS tiles with ds_read_b64_tr_b16 (lane i of a
// 16-lane group receives element i%4 of the 4 elements addressed by lane 4j + i/4, j = 0..3).
namespace cg {
constexpr int BO = 128;           // output rows (o) per block: 4 waves x 32
constexpr int TM = 64;            // tokens per step
constexpr int SROW = BO + 16;     // padded LDS row (elements)
constexpr int LROW = 128 + 16;    // Lm tile row (rp <= 128)
}  // namespace cg

// One launch runs up to two such passes (dA over x with u, dB over dy with h): job 0 takes the
// first nb0 blocks. A job's blocks are (column block, split), column block fastest.
struct CgJob {
  const uint16_t* src;  // [M][Od]
  const uint16_t* Lm;   // [M][ld_lm]
  float* part;          // partials, or NULL with out set
  float* out;           // one split: c * sum written here ([Od][r], or [r][Od] with trans)
  float* bpart;         // column sums of src (the bias gradient): split partials [splits][Od],
  float* bout;          // or with one split the sums themselves [Od]; both NULL: none
  int64_t Od, tps;      // output rows; tokens per split
  int nbx, trans;       // column blocks
};

// BS: jobs with bpart or bout set also sum the columns of src (sum_m src[m][o], unscaled) from
// the registers the tile copies pass through, in the order of colsum_kernel: per 64-token step
// thread (c = tid % 16, g = tid / 16) adds rows g, g + 16, g + 32, g + 48 of columns 8c..8c+7,
// steps in token order, then the 16 row groups are added in order g = 0..15
template <int RT, int ELT, bool BS>
__global__ __launch_bounds__(256) void colgrad_kernel(CgJob j0, CgJob j1, int nb0, int64_t M,
                                                      int ld_lm, int rp, int ld_part, float c,
                                                      int r) {
  using E = Elt<ELT>;
  using namespace cg;
  __shared__ __attribute__((aligned(16))) uint16_t ssrc[TM * SROW];
  __shared__ __attribute__((aligned(16))) uint16_t slm[TM * LROW];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool second = (int)blockIdx.x >= nb0;
  const int bj = second ? (int)blockIdx.x - nb0 : (int)blockIdx.x;
  const uint16_t* __restrict__ src = second ? j1.src : j0.src;
  const uint16_t* __restrict__ Lm = second ? j1.Lm : j0.Lm;
  float* __restrict__ part = second ? j1.part : j0.part;
  float* __restrict__ out = second ? j1.out : j0.out;
  const int64_t Od = second ? j1.Od : j0.Od;
  const int64_t tokens_per_split = second ? j1.tps : j0.tps;
  const int nbx = second ? j1.nbx : j0.nbx;
  const int trans = second ? j1.trans : j0.trans;
  float* __restrict__ bpart = second ? j1.bpart : j0.bpart;
  float* __restrict__ bout = second ? j1.bout : j0.bout;
  const bool bsum = BS && (bpart != nullptr || bout != nullptr);  // uniform over the block
  float csum[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) csum[e] = 0.0f;
  const int64_t o0 = (int64_t)(bj % nbx) * BO;
  const int sp = bj / nbx;
  const int64_t mbeg = (int64_t)sp * tokens_per_split;
  const int64_t mend = (mbeg + tokens_per_split < M) ? mbeg + tokens_per_split : M;
  f32x16 acc[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[t][v] = 0.0f;

  const int g = lane >> 4, i16 = lane & 15;
  const int jj = i16 >> 2, qq = i16 & 3;  // providing-lane roles for the transpose reads
  // register staging, two stages: src tile [64 tokens][128 o] (4 chunks per thread), Lm tile
  // [64 tokens][32*RT] (RT chunks per thread); the copies of token steps s + 1 and s + 2 are in
  // flight while step s is multiplied. Buffer loads through descriptors over the step's tokens
  // return zeros past their end (tokens past the split, a step past the last) and for offsets
  // moved out of range (columns past Od or rp), so the loads need no branch and the compiler's
  // waits count only the older stage.
  typedef u32x4 SS[4];
  typedef u32x4 LS[RT];
  SS rs0, rs1;
  LS rl0, rl1;
  auto load = [&](int64_t mb, SS& rs, LS& rl) {
    const int64_t nt = mend - mb < TM ? (mend - mb > 0 ? mend - mb : 0) : TM;
    const int64_t mc = mb < mend ? mb : mbeg;  // a valid base for an empty descriptor
    const __amdgpu_buffer_rsrc_t rss = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(src + mc * Od), (short)0, (int)(nt * Od * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsl = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(Lm + mc * ld_lm), (short)0, (int)(nt * ld_lm * 2), 0x00020000);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int id = tid + 256 * i, row = id >> 4, c = id & 15;
      const int64_t o = o0 + c * 8;
      const uint32_t off = o < Od ? (uint32_t)((row * Od + o) * 2) : 0x80000000u;
      rs[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rss, off, 0, 2));  // nt
    }
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const int id = tid + 256 * i, row = id / (RT * 4), c = id % (RT * 4);
      const uint32_t off = c * 8 < rp ? (uint32_t)((row * ld_lm + c * 8) * 2) : 0x80000000u;
      rl[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsl, off, 0, 0));
    }
  };
  auto stash = [&](const SS& rs, const LS& rl) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int id = tid + 256 * i, row = id >> 4, c = id & 15;
      *reinterpret_cast<u32x4*>(&ssrc[row * SROW + c * 8]) = rs[i];
    }
    if (BS && bsum) {
      // rows past the split or M arrive as zeros, which leave the sums unchanged
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          csum[2 * e] += E::lo(rs[i][e]);
          csum[2 * e + 1] += E::hi(rs[i][e]);
        }
    }
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const int id = tid + 256 * i, row = id / (RT * 4), c = id % (RT * 4);
      if (row < TM) *reinterpret_cast<u32x4*>(&slm[row * LROW + c * 8]) = rl[i];
    }
  };
  auto compute = [&]() {
#pragma unroll
    for (int ks = 0; ks < TM / 16; ++ks) {
      // A operand: src^T rows o = wave*32 + (0..31), tokens ks*16 + (lane/32)*8 + (0..7)
      u32x4 av;
      {
        const int rowb = ks * 16 + (g >> 1) * 8 + jj;
        const int col = wave * 32 + 16 * (g & 1) + 4 * qq;
        i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(i16x4, &ssrc[rowb * SROW + col]));
        i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(i16x4, &ssrc[(rowb + 4) * SROW + col]));
        av[0] = (uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16);
        av[1] = (uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16);
        av[2] = (uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16);
        av[3] = (uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16);
      }
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        u32x4 bv;
        const int rowb = ks * 16 + (g >> 1) * 8 + jj;
        const int col = t * 32 + 16 * (g & 1) + 4 * qq;
        i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(i16x4, &slm[rowb * LROW + col]));
        i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(i16x4, &slm[(rowb + 4) * LROW + col]));
        bv[0] = (uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16);
        bv[1] = (uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16);
        bv[2] = (uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16);
        bv[3] = (uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16);
        acc[t] = E::mfma32(E::as8(av), E::as8(bv), acc[t]);
      }
    }
  };
  // token step at mb: its registers to LDS, the copies of step mb + 2 TM into the freed
  // registers, the MFMAs on step mb
  auto step = [&](int64_t mb, SS& rs, LS& rl) {
    stash(rs, rl);
    __syncthreads();
    load(mb + 2 * TM, rs, rl);
    compute();
    __syncthreads();
  };
  // steps in pairs, the second unconditional (past the split's end it reads only zeros): a
  // branch around it would make the compiler's waits drain both stages
  load(mbeg, rs0, rl0);
  load(mbeg + TM, rs1, rl1);
  for (int64_t mb = mbeg; mb < mend; mb += 2 * TM) {
    step(mb, rs0, rl0);
    step(mb + TM, rs1, rl1);
  }
  if (BS && bsum) {
    // the 16 row groups' sums through LDS (the step loop ended with a barrier: ssrc is free)
    float* red = reinterpret_cast<float*>(ssrc);  // [16][BO]
    const int cc = tid & 15, gg = tid >> 4;
#pragma unroll
    for (int e = 0; e < 8; ++e) red[gg * BO + cc * 8 + e] = csum[e];
    __syncthreads();
    if (tid < BO) {
      float sum = 0.0f;
#pragma unroll
      for (int q = 0; q < 16; ++q) sum += red[q * BO + tid];
      const int64_t o = o0 + tid;
      if (o < Od) {
        if (bout != nullptr) bout[o] = sum;
        else bpart[(int64_t)sp * Od + o] = sum;
      }
    }
  }
  // D lane layout: row (o) = wave*32 + (v/4)*8 + (lane/32)*4 + v%4, column j = t*32 + lane%32
  const int l32 = lane & 31, lhi = lane >> 5;
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const int j = t * 32 + l32;
    if (j >= rp) continue;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t o = o0 + wave * 32 + (v / 4) * 8 + lhi * 4 + (v % 4);
      if (o >= Od) continue;
      if (out == nullptr) {
        part[((int64_t)sp * Od + o) * ld_part + j] = acc[t][v];
      } else if (j < r) {
        // one split: the result itself, as the reduction pass would write it (c (0 + sum))
        const float val = c * (0.0f + acc[t][v]);
        if (trans) out[(int64_t)j * Od + o] = val;
        else out[o * r + j] = val;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Column sums sum_m src[m][o] of a [M][Od] operand: the gradient of a trainable bias, the
// pullback of mixed_add (src/layers/linear.jl:7-13) for LoRALinear's bias when train_bias is set
// (src/layers/lora.jl:37-38, 64-67), dbias[n] = sum over tokens of dy[m][n], in f32.
// Split-M partials part[sp][o] (or, with one split, the sums written to out), then
// colsum_reduce_kernel adds the splits in order. The block and thread order is the one the dB
// gradient pass uses when it sums dy's columns beside its MFMAs (colgrad_kernel with BS): blocks
// are (column block of 128, split), column block fastest; per 64-token step thread
// (c = tid % 16, g = tid / 16) adds rows g, g + 16, g + 32, g + 48 of columns 8c..8c+7, steps in
// token order; then the 16 row groups are added in order. Same splits, same bits.
// VEC: 16-byte loads (16-byte aligned rows, Od a multiple of 8), else one element at a time.
template <int ELT, bool VEC>
__global__ __launch_bounds__(256) void colsum_kernel(const uint16_t* __restrict__ src, int64_t M,
                                                     int64_t Od, int64_t tps,
                                                     float* __restrict__ part,
                                                     float* __restrict__ out) {
  using E = Elt<ELT>;
  constexpr int BO = cg::BO, TM = cg::TM;
  __shared__ float red[16 * BO];
  const int tid = threadIdx.x, cc = tid & 15, gg = tid >> 4;
  const int nbx = (int)((Od + BO - 1) / BO);
  const int64_t o0 = (int64_t)(blockIdx.x % nbx) * BO;
  const int sp = (int)(blockIdx.x / nbx);
  const int64_t mbeg = (int64_t)sp * tps;
  const int64_t mend = mbeg + tps < M ? mbeg + tps : M;
  const int64_t oc = o0 + cc * 8;
  float csum[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) csum[e] = 0.0f;
  auto add_row = [&](int64_t m) {
    const uint16_t* row = src + m * Od;
    if (VEC) {
      if (oc < Od) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(row + oc);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          csum[2 * e] += E::lo(v[e]);
          csum[2 * e + 1] += E::hi(v[e]);
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (oc + e < Od) csum[e] += E::to_f32(row[oc + e]);
    }
  };
  int64_t mb = mbeg;
  for (; mb + TM <= mend; mb += TM) {
#pragma unroll
    for (int i = 0; i < 4; ++i) add_row(mb + gg + 16 * i);
  }
  if (mb < mend) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (mb + gg + 16 * i < mend) add_row(mb + gg + 16 * i);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) red[gg * BO + cc * 8 + e] = csum[e];
  __syncthreads();
  if (tid < BO) {
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q) sum += red[q * BO + tid];
    const int64_t o = o0 + tid;
    if (o < Od) {
      if (part == nullptr) out[o] = sum;
      else part[(int64_t)sp * Od + o] = sum;
    }
  }
}

// The same over f32 src (the fp32 path): per 64-token step thread (c = tid % 32, g = tid / 32)
// adds rows g, g + 8, ..., g + 56 of columns 4c..4c+3; then the 8 row groups in order.
template <bool VEC>
__global__ __launch_bounds__(256) void colsum_f32_kernel(const float* __restrict__ src, int64_t M,
                                                         int64_t Od, int64_t tps,
                                                         float* __restrict__ part,
                                                         float* __restrict__ out) {
  constexpr int BO = cg::BO, TM = cg::TM;
  __shared__ float red[8 * BO];
  const int tid = threadIdx.x, cc = tid & 31, gg = tid >> 5;
  const int nbx = (int)((Od + BO - 1) / BO);
  const int64_t o0 = (int64_t)(blockIdx.x % nbx) * BO;
  const int sp = (int)(blockIdx.x / nbx);
  const int64_t mbeg = (int64_t)sp * tps;
  const int64_t mend = mbeg + tps < M ? mbeg + tps : M;
  const int64_t oc = o0 + cc * 4;
  float csum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  auto add_row = [&](int64_t m) {
    const float* row = src + m * Od;
    if (VEC) {
      if (oc < Od) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(row + oc);
#pragma unroll
        for (int e = 0; e < 4; ++e) csum[e] += v[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (oc + e < Od) csum[e] += row[oc + e];
    }
  };
  int64_t mb = mbeg;
  for (; mb + TM <= mend; mb += TM) {
#pragma unroll
    for (int i = 0; i < 8; ++i) add_row(mb + gg + 8 * i);
  }
  if (mb < mend) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (mb + gg + 8 * i < mend) add_row(mb + gg + 8 * i);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) red[gg * BO + cc * 4 + e] = csum[e];
  __syncthreads();
  if (tid < BO) {
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) sum += red[q * BO + tid];
    const int64_t o = o0 + tid;
    if (o < Od) {
      if (part == nullptr) out[o] = sum;
      else part[(int64_t)sp * Od + o] = sum;
    }
  }
}

// out[o] = sum_sp part[sp][o] in split order
__global__ __launch_bounds__(256) void colsum_reduce_kernel(const float* __restrict__ part,
                                                            int splits, int64_t Od,
                                                            float* __restrict__ out) {
  const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= Od) return;
  float sum = 0.0f;
  for (int sp = 0; sp < splits; ++sp) sum += part[(int64_t)sp * Od + o];
  out[o] = sum;
}

// out = c * sum_sp part[sp][o][j] in split order; TRANS: out[j][o] (dB [r][N]) else out[o][j].
// One sum per thread, j fastest, so the partials are read contiguously; the split loop is
// unrolled so that each thread has several independent loads in flight.
template <bool TRANS>
__global__ __launch_bounds__(256) void reduce_partials_kernel(const float* __restrict__ part, int splits,
                                                              int64_t Od, int rp, int r, float c,
                                                              float* __restrict__ out) {
  if (!TRANS) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= Od * r) return;
    const int64_t o = idx / r, j = idx % r;
    float sum = 0.0f;
#pragma unroll 8
    for (int sp = 0; sp < splits; ++sp) sum += part[((int64_t)sp * Od + o) * rp + j];
    out[idx] = c * sum;
    return;
  }
  // 8 x 32 tiles of (o, j); the [r][Od] output is written along o through an LDS transpose
  __shared__ float tile[8][33];
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  const int64_t o = (int64_t)blockIdx.x * 8 + ty;
  const int j = blockIdx.y * 32 + tx;
  float sum = 0.0f;
  if (o < Od && j < r) {
#pragma unroll 8
    for (int sp = 0; sp < splits; ++sp) sum += part[((int64_t)sp * Od + o) * rp + j];
  }
  tile[ty][tx] = c * sum;
  __syncthreads();
  const int wo = threadIdx.x & 7, wj = threadIdx.x >> 3;  // 32 rows of 8 outputs
  const int64_t oo = (int64_t)blockIdx.x * 8 + wo;
  const int jj = blockIdx.y * 32 + wj;
  if (jj < r && oo < Od) out[(int64_t)jj * Od + oo] = tile[wo][wj];
}

// The dA (out[o][j]) and dB (out[j][o]) reductions of one backward in one launch: blocks
// [0, nb0) reduce dA as reduce_partials_kernel<false> (256 outputs per block), the rest dB as
// <true> (8 x 32 tiles, row of tiles fastest); same sums in the same order
struct RpJob {
  const float* part;
  float* out;
  int64_t Od;
  int splits;
};
// blocks from nbs on sum the column-sum partials bj.part [splits][Od] into bj.out (as
// colsum_reduce_kernel; nbs = gridDim.x: none)
__global__ __launch_bounds__(256) void reduce_partials2_kernel(RpJob ja, RpJob jb, int nb0, int rp,
                                                               int r, float c, RpJob bj, int nbs) {
  __shared__ float tile[8][33];
  if ((int)blockIdx.x >= nbs) {
    const int64_t o = (int64_t)((int)blockIdx.x - nbs) * blockDim.x + threadIdx.x;
    if (o >= bj.Od) return;
    float sum = 0.0f;
    for (int sp = 0; sp < bj.splits; ++sp) sum += bj.part[(int64_t)sp * bj.Od + o];
    bj.out[o] = sum;
    return;
  }
  if ((int)blockIdx.x < nb0) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= ja.Od * r) return;
    const int64_t o = idx / r, j = idx % r;
    float sum = 0.0f;
#pragma unroll 8
    for (int sp = 0; sp < ja.splits; ++sp) sum += ja.part[((int64_t)sp * ja.Od + o) * rp + j];
    ja.out[idx] = c * sum;
    return;
  }
  const int b = (int)blockIdx.x - nb0;
  const int gx = (int)((jb.Od + 7) / 8);
  const int bx = b % gx, by = b / gx;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  const int64_t o = (int64_t)bx * 8 + ty;
  const int j = by * 32 + tx;
  float sum = 0.0f;
  if (o < jb.Od && j < r) {
#pragma unroll 8
    for (int sp = 0; sp < jb.splits; ++sp) sum += jb.part[((int64_t)sp * jb.Od + o) * rp + j];
  }
  tile[ty][tx] = c * sum;
  __syncthreads();
  const int wo = threadIdx.x & 7, wj = threadIdx.x >> 3;
  const int64_t oo = (int64_t)bx * 8 + wo;
  const int jj = by * 32 + wj;
  if (jj < r && oo < jb.Od) jb.out[(int64_t)jj * jb.Od + oo] = tile[wo][wj];
}

__global__ void fill_f32_kernel(float* p, int64_t n, float v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// dst[i][j] = j < cols ? src[i][j] : 0 for j < cols_dst (16-bit elements; rows of ld_src and
// ld_dst): widens a [rows][r] LoRA operand to the padded [rows][rp] layout of the fast kernels,
// or (cols = cols_dst = r) compacts a padded one back to [rows][r]
__global__ void pad_cols_kernel(const uint16_t* __restrict__ src, int64_t rows, int cols,
                                int64_t ld_src, uint16_t* __restrict__ dst, int cols_dst,
                                int64_t ld_dst) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * cols_dst) return;
  const int64_t row = i / cols_dst;
  const int j = (int)(i % cols_dst);
  dst[row * ld_dst + j] = j < cols ? src[row * ld_src + j] : (uint16_t)0;
}

// ---------------------------------------------------------------------------------------------
// generic kernels (any shape / alignment)
// out[m][j] = bf16(sum_k src[m*Kd + k] * P[k*ps_k + j*ps_j]) (j < r), row stride ld_out
template <int ELT>
__global__ void g_rowproj_kernel(const uint16_t* __restrict__ src, int64_t M, int64_t Kd,
                                 const uint16_t* __restrict__ P, int64_t ps_k, int64_t ps_j, int r,
                                 uint16_t* __restrict__ out, int64_t ld_out) {
  using E = Elt<ELT>;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * r) return;
  const int64_t m = idx / r, j = idx % r;
  float acc = 0.0f;
  for (int64_t k = 0; k < Kd; ++k) acc += E::to_f32(src[m * Kd + k]) * E::to_f32(P[k * ps_k + j * ps_j]);
  out[m * ld_out + j] = (uint16_t)E::bits(acc);
}

template <int ELT>
__global__ void g_fwd_kernel(const uint16_t* __restrict__ x, const int8_t* __restrict__ q,
                             const float* __restrict__ s, const uint16_t* __restrict__ h,
                             int64_t ldh, const uint16_t* __restrict__ B,
                             const uint16_t* __restrict__ bias, int64_t M, int64_t K, int64_t N,
                             int r, float c, uint16_t* __restrict__ y) {
  using E = Elt<ELT>;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * N) return;
  const int64_t m = idx / N, n = idx % N;
  float acc = 0.0f;
  for (int64_t k = 0; k < K; ++k) acc += E::to_f32(x[m * K + k]) * (float)q[n * K + k];
  float lo = 0.0f;
  for (int j = 0; j < r; ++j) lo += E::to_f32(h[m * ldh + j]) * E::to_f32(B[(int64_t)j * N + n]);
  float o = s[n] * acc + c * lo + (bias ? E::to_f32(bias[n]) : 0.0f);
  y[idx] = (uint16_t)E::bits(o);
}

template <int ELT>
__global__ void g_dx_kernel(const uint16_t* __restrict__ dy, const int8_t* __restrict__ q,
                            const float* __restrict__ s, const uint16_t* __restrict__ u,
                            int64_t ldu, const uint16_t* __restrict__ A, int64_t M, int64_t K,
                            int64_t N, int r, float c, uint16_t* __restrict__ dx) {
  using E = Elt<ELT>;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * K) return;
  const int64_t m = idx / K, k = idx % K;
  float acc = 0.0f;
  if (ELT == REELS_HIP_F16) {
    // the reference's binary16 weight f16(q * f16(s)) times the raw dy (quantization.jl:61-62):
    // dy * s itself may lie below binary16's normal range
    for (int64_t n = 0; n < N; ++n)
      acc += E::to_f32(dy[m * N + n]) * E::to_f32((uint16_t)E::deq((float)q[n * K + k], s[n]));
  } else {
    // bf16 keeps f32's exponent range: bf16(dy * s) times the exact code
    for (int64_t n = 0; n < N; ++n) {
      const float dys = E::to_f32((uint16_t)E::bits(E::to_f32(dy[m * N + n]) * s[n]));
      acc += dys * (float)q[n * K + k];
    }
  }
  float lo = 0.0f;
  for (int j = 0; j < r; ++j) lo += E::to_f32(u[m * ldu + j]) * E::to_f32(A[k * r + j]);
  dx[idx] = (uint16_t)E::bits(acc + c * lo);
}

// out[o][j] (or [j][o] when TRANS) = c * sum_m src[m][o] * Lm[m][j]
template <bool TRANS, int ELT>
__global__ void g_colgrad_kernel(const uint16_t* __restrict__ src, int64_t M, int64_t Od,
                                 const uint16_t* __restrict__ Lm, int64_t ldl, int r, float c,
                                 float* __restrict__ out) {
  using E = Elt<ELT>;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= Od * r) return;
  int64_t o, j;
  if (TRANS) { j = idx / Od; o = idx % Od; } else { o = idx / r; j = idx % r; }
  float acc = 0.0f;
  for (int64_t m = 0; m < M; ++m) acc += E::to_f32(src[m * Od + o]) * E::to_f32(Lm[m * ldl + j]);
  out[idx] = c * acc;
}

// ---------------------------------------------------------------------------------------------
// gelu_tanh, src/layers/linear.jl:61-68 (f32 math, 16-bit in/out; gelu_f in common.h)
// Streaming passes: with 16-byte aligned operands a thread takes 8 elements per 16-byte load
// (nontemporal, grid-stride), the rest (n mod 8, or unaligned operands) one element per thread.
template <int ELT>
__global__ __launch_bounds__(256) void gelu_kernel(const uint16_t* __restrict__ x,
                                                   uint16_t* __restrict__ y, int64_t n, int vec) {
  using E = Elt<ELT>;
  const int64_t nv = vec ? n / 8 : 0;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv; i += step) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x) + i);
    u32x4 o;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      o[k] = E::bits(gelu_f(E::lo(v[k]))) | (E::bits(gelu_f(E::hi(v[k]))) << 16);
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(y) + i);
  }
  for (int64_t i = nv * 8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step)
    y[i] = (uint16_t)E::bits(gelu_f(E::to_f32(x[i])));
}
template <int ELT>
// (dx may be dy: each element is read before the same thread writes it)
__global__ __launch_bounds__(256) void gelu_bwd_kernel(const uint16_t* __restrict__ x,
                                                       const uint16_t* dy, uint16_t* dx, int64_t n,
                                                       int vec) {
  using E = Elt<ELT>;
  const int64_t nv = vec ? n / 8 : 0;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv; i += step) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x) + i);
    const u32x4 d = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(dy) + i);
    u32x4 o;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      o[k] = E::bits(E::lo(d[k]) * gelu_grad_f(E::lo(v[k]))) |
             (E::bits(E::hi(d[k]) * gelu_grad_f(E::hi(v[k]))) << 16);
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(dx) + i);
  }
  for (int64_t i = nv * 8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step)
    dx[i] = (uint16_t)E::bits(E::to_f32(dy[i]) * gelu_grad_f(E::to_f32(x[i])));
}

// ---------------------------------------------------------------------------------------------
// host side
// Split-M plan of one gradient pass over a [M][Od] operand: enough token splits that the
// ceil(Od / 128) column blocks times the splits fill one round of the GPU's workgroup slots
// (256 CUs x 4 resident gradient workgroups), at most 32 splits (the partials buffer), tokens per
// split a multiple of 128 (the kernel takes token steps of 64 in pairs). Up to 512 tokens one
// split: the pass writes its result itself and no reduction launch follows (5120 x 5120 backward
// at 333 / 512 tokens 42.2 -> 40.6 and 51.5 -> 49.6 us; capping the splits at 2 or 4 up to 1024
// tokens slowed 1536 x 1536 at 1024 tokens, 21.5 -> 22.7-23.6 us).
struct Split {
  int splits;
  int64_t tps;  // tokens per split
};

static Split split_for(int64_t M, int64_t Od) {
  constexpr int64_t kSlots = 1024;
  const int64_t colblocks = (Od + cg::BO - 1) / cg::BO;
  int64_t s = kSlots / (colblocks > 0 ? colblocks : 1);
  if (s > 32) s = 32;
  if (s > (M + 127) / 128) s = (M + 127) / 128;
  if (M <= 512) s = 1;
  if (s < 1) s = 1;
  Split sp;
  sp.tps = ((M + s - 1) / s + 127) / 128 * 128;
  if (sp.tps < 128) sp.tps = 128;
  sp.splits = (int)((M + sp.tps - 1) / sp.tps);
  if (sp.splits < 1) sp.splits = 1;
  return sp;
}

struct Plan {
  bool fast;
  bool deq;     // fast and K, N multiples of 64: dequantized weight + bf16 GEMM
  bool skinny;  // few tokens: the int8 codes streamed into registers (skinny.hip), both directions
  int rp;       // row stride of the h/u panels and padded adapter operands: round_up(r, 16)
  bool padded;  // rp != r: h, h_save and A go through padded copies in the workspace
  Split sa;     // dA: columns of x (K)
  Split sb;     // dB: columns of dy (N)
  SkinnyPlan skf, skb;  // the few-token forward (reduction K) and dX (reduction N)
  int ksf, ksb;  // reduction splits of the forward and dX GEMMs (1 = none)
  bool i8f;      // deq shapes with a split forward: the forward multiplies the int8 codes (no
                 // weight copy; faster there), dX keeps the dequantized weight (faster there)
};

// rank chunk of the projection and gradient kernels (their LDS tiles hold 128 rank columns)
constexpr int kRankChunk = 128;

// Column splits of a rank projection over few tokens (32-row blocks that leave most CUs idle):
// about 256 blocks, at most 16 splits, one rank chunk (rp <= 128); 1 = none
static int rowproj_splits(int64_t M, int64_t Kd, int rp) {
  const int64_t blocks = ceil_div(M, 32);
  if (blocks >= 128 || rp > kRankChunk || rp <= 0) return 1;
  int64_t s = ceil_div(256, blocks);
  const int64_t nch = ceil_div(Kd, rowp::KC);
  if (s > nch) s = nch;
  if (s > 16) s = 16;
  return s < 2 ? 1 : (int)s;
}


// The plan of reels_hip_i8lora_fwd_noalloc: never the dequantized-weight copy (its N*K*2 bytes
// are what would not fit a modest scratch) and no split-reduction partials
static void noalloc_plan(Plan& p) {
  p.deq = false;
  p.i8f = false;
  p.ksf = p.ksb = 1;
}

static Plan make_plan(int64_t M, int64_t K, int64_t N, int64_t r, bool ptrs_aligned) {
  Plan p;
  // K, N < 2^22 keeps the projection and gradient kernels' buffer descriptors (64 rows, or a
  // rank chunk of 128 rows, of one row length) below 2^31 bytes
  p.fast = ptrs_aligned && (K % 16 == 0) && (N % 16 == 0) &&
           K < ((int64_t)1 << 22) && N < ((int64_t)1 << 22);
  p.deq = p.fast && bfgemm_supported(M, N, K) && bfgemm_supported(M, K, N);
  p.rp = (int)((r + 15) / 16 * 16);
  p.padded = p.fast && p.rp != r;
  p.skinny = p.fast && skinny_supported(M, K, N, p.rp);
  if (p.skinny) {
    p.skf = skinny_plan(M, K, N, r > 0 ? p.rp : 0, 0);
    p.skb = skinny_plan(M, N, K, r > 0 ? p.rp : 0, 1);
  }
  p.sa = split_for(M, K);
  p.sb = split_for(M, N);
  p.ksf = p.fast && !p.skinny ? bfgemm_splits(M, N, K) : 1;
  p.ksb = p.fast && !p.skinny ? bfgemm_splits(M, K, N) : 1;
  p.i8f = p.deq && p.ksf > 1;
  return p;
}

// workspace layout (byte offsets, 256-aligned); identical computation for sizing and use
struct WsLayout {
  size_t h, u, dys, wd, at, bt, ap, pa, pb, pbias, kp, rq, total;
};

static WsLayout ws_layout(int64_t M, int64_t K, int64_t N, int64_t r, int which, const Plan& p) {
  WsLayout w{};
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off = align_up(off + bytes, 256); return o; };
  const size_t rp = (size_t)p.rp;
  const int rpl = r > 0 ? p.rp : 0;
  if (p.skinny) {
    // few tokens: the f32 split partials instead of a dequantized weight; A zero-padded to rp for
    // the forward's adapter blocks; u (and h for the dB pass) as in the other plans
    if (which == REELS_HIP_WS_FWD) {
      w.ap = take(p.padded && r > 0 ? (size_t)K * rp * 2 : 0);
      w.pa = take(skinny_ws_bytes(p.skf, M, N, rpl));
    } else {
      w.h = take((size_t)M * rp * 2);
      w.at = take(r > 0 ? (size_t)K * rp * 2 : 0);  // A^T, or A padded to rp for recomputing h
      w.ap = take(p.padded && r > 0 ? (size_t)K * rp * 2 : 0);  // A [K][rp] for the dX epilogue
      w.u = take((size_t)M * rp * 2);
      // dX partials, or the forward's when h is recomputed
      const size_t pb = skinny_ws_bytes(p.skb, M, K, rpl), pf = skinny_ws_bytes(p.skf, M, N, rpl);
      w.wd = take(pb > pf ? pb : pf);
      w.pa = take(r > 0 ? (size_t)p.sa.splits * K * rp * 4 : 0);
      w.pb = take(r > 0 ? (size_t)p.sb.splits * N * rp * 4 : 0);
      w.pbias = take(colsum_partial_bytes(M, N));
    }
    w.total = off == 0 ? 256 : off;
    return w;
  }
  w.h = take((size_t)M * rp * 2);
  w.at = take(r > 0 ? (size_t)r * K * 2 : 0);
  {  // column-split partials of the rank projections over few tokens (h over K, u over N)
    const int rs = r > 0 && p.fast ? std::max(rowproj_splits(M, K, p.rp), rowproj_splits(M, N, p.rp)) : 1;
    w.rq = take(rs > 1 ? (size_t)rs * M * rp * 4 : 0);
  }
  // bf16 copy of the dequantized weight (dX, and the forward unless it multiplies the codes)
  w.wd = take(p.deq && !(which == REELS_HIP_WS_FWD && p.i8f) ? (size_t)N * K * 2 : 0);
  if (which == REELS_HIP_WS_FWD) {
    w.bt = take(p.fast ? (size_t)N * rp * 2 : 0);
    w.kp = take(p.ksf > 1 ? (size_t)p.ksf * M * N * 4 : 0);  // split GEMM partials
  } else {
    w.kp = take(p.ksb > 1 ? (size_t)p.ksb * M * K * 4 : 0);
    w.u = take((size_t)M * rp * 2);
    w.ap = take(p.padded ? (size_t)K * rp * 2 : 0);  // A [K][rp], zeros past r
    w.dys = take(p.fast && !p.deq ? (size_t)M * N * 2 : 0);
    w.pa = take(p.fast && r > 0 ? (size_t)p.sa.splits * K * rp * 4 : 0);
    w.pb = take(p.fast && r > 0 ? (size_t)p.sb.splits * N * rp * 4 : 0);
    w.pbias = take(colsum_partial_bytes(M, N));  // the bias gradient's split partials
  }
  w.total = off == 0 ? 256 : off;
  return w;
}

static int grid1(int64_t n, int bs = 256) { return (int)ceil_div(n, bs); }

// out[c][r] = in[r][c] (rows_pad >= rows output rows, zeros past rows) for one or two matrices
// in one launch (in1 NULL: one)
static TpJob tp_job(const uint16_t* in, int64_t rows, int64_t cols, int64_t rows_pad, uint16_t* out) {
  TpJob j{};
  j.in = in; j.out = out; j.rows = rows; j.cols = cols; j.rows_pad = rows_pad;
  j.gx = (int)ceil_div(cols, 32);
  return j;
}
static int launch_transpose_pad(const TpJob& a, const TpJob* b, hipStream_t st) {
  const int nb0 = a.gx * (int)ceil_div(a.rows_pad, 32);
  const int nb1 = b ? b->gx * (int)ceil_div(b->rows_pad, 32) : 0;
  { TraceScope _ts(st, "transpose_pad_kernel");
    transpose_pad_kernel<<<(unsigned)(nb0 + nb1), 256, 0, st>>>(a, b ? *b : a, nb0); }
  return check_launch("transpose_pad_kernel");
}
// grid of a grid-stride streaming pass over n 16-bit elements (8 per thread and step): enough
// blocks to fill the GPU several times over, fewer for small n
static int grid_stream(int64_t n) {
  const int64_t b = ceil_div(ceil_div(n, 8), 256);
  return (int)(b < 8192 ? (b > 0 ? b : 1) : 8192);
}

template <bool SCALED, int ROWS>
static void launch_rowproj_t(int elt, int rt, const uint16_t* src, int64_t M, int64_t Kd,
                             const uint16_t* P, int r, int rp, uint16_t* out, int ld_out,
                             const float* s, uint16_t* scaled, hipStream_t st,
                             float* part = nullptr, int ks = 1) {
  const dim3 grid((unsigned)ceil_div(M, ROWS), (unsigned)ks);
  TraceScope _ts(st, SCALED ? (rt <= 1 ? "rowproj_kernel<1,true>" : rt == 2 ? "rowproj_kernel<2,true>" : "rowproj_kernel<4,true>")
                            : (rt <= 1 ? "rowproj_kernel<1,false>" : rt == 2 ? "rowproj_kernel<2,false>" : "rowproj_kernel<4,false>"));
  with_elt(elt, [&](auto e) {
    constexpr int T = decltype(e)::value;
    float* pt = ks > 1 ? part : nullptr;
    if (rt <= 1) rowproj_kernel<1, SCALED, ROWS, T><<<grid, 256, 0, st>>>(src, M, Kd, P, r, rp, out, ld_out, s, scaled, pt);
    else if (rt == 2) rowproj_kernel<2, SCALED, ROWS, T><<<grid, 256, 0, st>>>(src, M, Kd, P, r, rp, out, ld_out, s, scaled, pt);
    else rowproj_kernel<4, SCALED, ROWS, T><<<grid, 256, 0, st>>>(src, M, Kd, P, r, rp, out, ld_out, s, scaled, pt);
  });
}

// out [M][rp] = bf16(src P^T) (zeros in columns r..rp), P [r][Kd]; one launch per rank chunk of
// 128 (the scaled copy, when asked for, comes with the first). part (rowproj_splits(M, Kd, rp)
// x M x rp f32, or NULL): with few tokens the columns are split and a second pass sums them.
static int launch_rowproj(int elt, const uint16_t* src, int64_t M, int64_t Kd, const uint16_t* P,
                          int r, int rp, uint16_t* out, const float* s, uint16_t* scaled,
                          hipStream_t st, float* part = nullptr) {
  const bool wide = ceil_div(M, 64) >= 256;  // enough tokens for a 64-row block on every CU
  const int ks = (part != nullptr && out != nullptr) ? rowproj_splits(M, Kd, rp) : 1;
  if (ks > 1) {
    const int rt = (rp + 31) / 32;
    if (scaled) launch_rowproj_t<true, 32>(elt, rt, src, M, Kd, P, r, rp, out, rp, s, scaled, st, part, ks);
    else launch_rowproj_t<false, 32>(elt, rt, src, M, Kd, P, r, rp, out, rp, s, scaled, st, part, ks);
    if (int rcode = check_launch("rowproj_kernel")) return rcode;
    { TraceScope _ts(st, "rowproj_reduce_kernel");
      with_elt(elt, [&](auto e) {
        rowproj_reduce_kernel<decltype(e)::value><<<grid1(M * rp), 256, 0, st>>>(part, ks, M, r, rp, out, rp);
      }); }
    return check_launch("rowproj_reduce_kernel");
  }
  for (int c0 = 0; c0 < (rp > 0 ? rp : 1); c0 += kRankChunk) {
    const int rpc = rp - c0 < kRankChunk ? rp - c0 : kRankChunk;     // columns of this chunk
    const int rc = r - c0 < 0 ? 0 : (r - c0 < rpc ? r - c0 : rpc);  // of them, rows of P
    const int rt = (rpc + 31) / 32;
    const uint16_t* Pc = P + (int64_t)c0 * Kd;
    uint16_t* oc = out ? out + c0 : nullptr;
    uint16_t* sc = c0 == 0 ? scaled : nullptr;
    if (sc) {
      if (wide) launch_rowproj_t<true, 64>(elt, rt, src, M, Kd, Pc, rc, rpc, oc, rp, s, sc, st);
      else launch_rowproj_t<true, 32>(elt, rt, src, M, Kd, Pc, rc, rpc, oc, rp, s, sc, st);
    } else {
      if (wide) launch_rowproj_t<false, 64>(elt, rt, src, M, Kd, Pc, rc, rpc, oc, rp, s, sc, st);
      else launch_rowproj_t<false, 32>(elt, rt, src, M, Kd, Pc, rc, rpc, oc, rp, s, sc, st);
    }
    if (int rcode = check_launch("rowproj_kernel")) return rcode;
  }
  return REELS_HIP_OK;
}

// Lm [M][rp]; partials part[sp][Od][rp], one launch per rank chunk of 128, then the fixed-order
// reduction over the splits
// One gradient pass over [M][Od] operands: out = c * src^T Lm (trans: its transpose), through
// split partials and the reduction pass, or written directly with one split.
struct CgPass {
  const uint16_t* src;
  int64_t Od;
  const uint16_t* Lm;
  Split sp;
  float* part;
  float* out;
  bool trans;
  float* bpart = nullptr;  // column sums of src too (the bias gradient): split partials
  float* bout = nullptr;   // [sp.splits][Od] and the result [Od]; NULL bout: none
};

// dA and dB passes (either may be absent: src NULL) in one colgrad launch per rank chunk, then
// the reduction passes of those that need one
static int launch_colgrad2(int elt, int64_t M, int r, int rp, float c, const CgPass& pa,
                           const CgPass& pb, hipStream_t st) {
  const CgPass* ps[2] = {pa.src ? &pa : nullptr, pb.src ? &pb : nullptr};
  if (!ps[0] && !ps[1]) return REELS_HIP_OK;
  if (!ps[0]) { ps[0] = ps[1]; ps[1] = nullptr; }
  bool direct[2];
  for (int i = 0; i < 2; ++i) direct[i] = ps[i] && ps[i]->sp.splits == 1 && rp <= kRankChunk;
  for (int c0 = 0; c0 < rp; c0 += kRankChunk) {
    const int rpc = rp - c0 < kRankChunk ? rp - c0 : kRankChunk;
    const int rt = (rpc + 31) / 32;
    CgJob j[2] = {};
    int nb[2] = {0, 0};
    bool bs = false;
    for (int i = 0; i < 2; ++i) {
      if (!ps[i]) continue;
      const CgPass& q = *ps[i];
      j[i].src = q.src; j[i].Lm = q.Lm + c0; j[i].part = q.part + c0;
      j[i].out = direct[i] ? q.out : nullptr;
      if (q.bout && c0 == 0) {  // the column sums ride on the first rank chunk's launch
        if (q.sp.splits == 1) j[i].bout = q.bout;
        else j[i].bpart = q.bpart;
        bs = true;
      }
      j[i].Od = q.Od; j[i].tps = q.sp.tps; j[i].trans = q.trans ? 1 : 0;
      j[i].nbx = (int)ceil_div(q.Od, cg::BO);
      nb[i] = j[i].nbx * q.sp.splits;
    }
    const unsigned grid = (unsigned)(nb[0] + nb[1]);
    {
      TraceScope _ts(st, rt <= 1 ? (bs ? "colgrad_kernel<1,bias>" : "colgrad_kernel<1>")
                         : rt == 2 ? (bs ? "colgrad_kernel<2,bias>" : "colgrad_kernel<2>")
                                   : (bs ? "colgrad_kernel<4,bias>" : "colgrad_kernel<4>"));
      with_elt(elt, [&](auto e) {
        constexpr int T = decltype(e)::value;
        if (bs) {
          if (rt <= 1) colgrad_kernel<1, T, true><<<grid, 256, 0, st>>>(j[0], j[1], nb[0], M, rp, rpc, rp, c, r);
          else if (rt == 2) colgrad_kernel<2, T, true><<<grid, 256, 0, st>>>(j[0], j[1], nb[0], M, rp, rpc, rp, c, r);
          else colgrad_kernel<4, T, true><<<grid, 256, 0, st>>>(j[0], j[1], nb[0], M, rp, rpc, rp, c, r);
        } else {
          if (rt <= 1) colgrad_kernel<1, T, false><<<grid, 256, 0, st>>>(j[0], j[1], nb[0], M, rp, rpc, rp, c, r);
          else if (rt == 2) colgrad_kernel<2, T, false><<<grid, 256, 0, st>>>(j[0], j[1], nb[0], M, rp, rpc, rp, c, r);
          else colgrad_kernel<4, T, false><<<grid, 256, 0, st>>>(j[0], j[1], nb[0], M, rp, rpc, rp, c, r);
        }
      });
    }
    if (int rc = check_launch("colgrad_kernel")) return rc;
  }
  // the column-sum partials still to be added up (at most one pass carries them)
  const CgPass* bias_red = nullptr;
  for (int i = 0; i < 2; ++i)
    if (ps[i] && ps[i]->bout && ps[i]->sp.splits > 1) bias_red = ps[i];
  // the reductions: dA and dB together in one launch when both need one
  const CgPass* need[2] = {nullptr, nullptr};
  int nn = 0;
  for (int i = 0; i < 2; ++i)
    if (ps[i] && !direct[i]) need[nn++] = ps[i];
  if (nn == 2 && !need[0]->trans && need[1]->trans) {
    const RpJob ja{need[0]->part, need[0]->out, need[0]->Od, need[0]->sp.splits};
    const RpJob jb{need[1]->part, need[1]->out, need[1]->Od, need[1]->sp.splits};
    const int nb0 = (int)ceil_div(ja.Od * r, 256);
    const int nb1 = (int)(ceil_div(jb.Od, 8) * ceil_div(r, 32));
    RpJob bj{};
    int nb2 = 0;
    if (bias_red) {
      bj = RpJob{bias_red->bpart, bias_red->bout, bias_red->Od, bias_red->sp.splits};
      nb2 = (int)ceil_div(bj.Od, 256);
      bias_red = nullptr;
    }
    { TraceScope _ts(st, "reduce_partials2_kernel");
      reduce_partials2_kernel<<<(unsigned)(nb0 + nb1 + nb2), 256, 0, st>>>(ja, jb, nb0, rp, r, c, bj, nb0 + nb1); }
    return check_launch("reduce_partials2_kernel");
  }
  for (int i = 0; i < nn; ++i) {
    const CgPass& q = *need[i];
    if (int rc = launch_reduce_partials(q.part, q.sp.splits, q.Od, rp, r, c, q.out, q.trans, st)) return rc;
  }
  if (bias_red) {
    { TraceScope _ts(st, "colsum_reduce_kernel");
      colsum_reduce_kernel<<<(unsigned)ceil_div(bias_red->Od, 256), 256, 0, st>>>(
          bias_red->bpart, bias_red->sp.splits, bias_red->Od, bias_red->bout); }
    return check_launch("colsum_reduce_kernel");
  }
  return REELS_HIP_OK;
}

// Column sums out[o] = sum_m src[m][o] of a [M][Od] operand of element type elt (F32, BF16 or
// F16), in the split plan of the dB gradient pass (split_for(M, Od)): partials in part
// (colsum_partial_bytes(M, Od) bytes), then the ordered sum over the splits
int launch_colsum(int elt, const void* src, int64_t M, int64_t Od, float* part, float* out,
                  hipStream_t st) {
  if (Od <= 0) return REELS_HIP_OK;
  if (M == 0) {
    { TraceScope _ts(st, "fill_f32_kernel"); fill_f32_kernel<<<grid1(Od), 256, 0, st>>>(out, Od, 0.0f); }
    return check_launch("fill_f32_kernel");
  }
  const Split sp = split_for(M, Od);
  const unsigned grid = (unsigned)(ceil_div(Od, cg::BO) * sp.splits);
  float* pt = sp.splits > 1 ? part : nullptr;
  const size_t esz = elt == REELS_HIP_F32 ? 4 : 2;
  const bool vec = aligned16(src) && (Od * (int64_t)esz) % 16 == 0;
  {
    TraceScope _ts(st, "colsum_kernel");
    if (elt == REELS_HIP_F32) {
      const float* f = static_cast<const float*>(src);
      if (vec) colsum_f32_kernel<true><<<grid, 256, 0, st>>>(f, M, Od, sp.tps, pt, out);
      else colsum_f32_kernel<false><<<grid, 256, 0, st>>>(f, M, Od, sp.tps, pt, out);
    } else {
      const uint16_t* h = static_cast<const uint16_t*>(src);
      with_elt(elt, [&](auto e) {
        constexpr int T = decltype(e)::value;
        if (vec) colsum_kernel<T, true><<<grid, 256, 0, st>>>(h, M, Od, sp.tps, pt, out);
        else colsum_kernel<T, false><<<grid, 256, 0, st>>>(h, M, Od, sp.tps, pt, out);
      });
    }
  }
  if (int rc = check_launch("colsum_kernel")) return rc;
  if (sp.splits == 1) return REELS_HIP_OK;
  { TraceScope _ts(st, "colsum_reduce_kernel");
    colsum_reduce_kernel<<<(unsigned)ceil_div(Od, 256), 256, 0, st>>>(part, sp.splits, Od, out); }
  return check_launch("colsum_reduce_kernel");
}

size_t colsum_partial_bytes(int64_t M, int64_t Od) {
  const Split sp = split_for(M, Od);
  return sp.splits > 1 ? (size_t)sp.splits * (size_t)Od * 4 : 0;
}

// dst [rows][cols_dst] (row stride ld_dst) from src [rows][cols] (row stride ld_src), zeros past cols
static int launch_pad_cols(const uint16_t* src, int64_t rows, int cols, int64_t ld_src,
                           uint16_t* dst, int cols_dst, int64_t ld_dst, hipStream_t st) {
  { TraceScope _ts(st, "pad_cols_kernel");
    pad_cols_kernel<<<grid1(rows * cols_dst), 256, 0, st>>>(src, rows, cols, ld_src, dst, cols_dst, ld_dst); }
  return check_launch("pad_cols_kernel");
}

int launch_reduce_partials(const float* part, int splits, int64_t Od, int rp, int r, float c,
                           float* out, bool trans, hipStream_t st) {
  if (trans) { TraceScope _ts(st, "reduce_partials_kernel<true>"); reduce_partials_kernel<true><<<dim3((unsigned)ceil_div(Od, 8), (unsigned)ceil_div(r, 32)), 256, 0, st>>>(part, splits, Od, rp, r, c, out); }
  else { TraceScope _ts(st, "reduce_partials_kernel<false>"); reduce_partials_kernel<false><<<(unsigned)ceil_div(Od * r, 256), 256, 0, st>>>(part, splits, Od, rp, r, c, out); }
  return check_launch("reduce_partials_kernel");
}

}  // namespace reels

using namespace reels;

extern "C" size_t reels_hip_i8lora_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t r,
                                                   int which) {
  if (M < 0 || K < 0 || N < 0 || r < 0) return 0;
  if (which != REELS_HIP_WS_FWD && which != REELS_HIP_WS_BWD && which != REELS_HIP_WS_FWD_NOALLOC)
    return 0;
  // sized for the fast layout when the shape allows it (pointer alignment cannot be known here;
  // the fast layout is never smaller than the generic one)
  Plan p = make_plan(M, K, N, r, true);
  if (which == REELS_HIP_WS_FWD_NOALLOC) {
    noalloc_plan(p);
    which = REELS_HIP_WS_FWD;
  }
  return ws_layout(M, K, N, r, which, p).total;
}

static bool all_aligned(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if (p != nullptr && !aligned16(p)) return false;
  return true;
}

// ---- allocation-free forward ----------------------------------------------------------------
// Scratch of reels_hip_i8lora_fwd_noalloc: one array per GPU, held until the process ends. Host
// code never uses the array's name as an address (on the host it is a stand-in symbol); the
// device address comes from hipGetSymbolAddress, once per device, on that device's first call.
constexpr size_t kScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices] = {};

static int scratch_for_current_device(const char* fn, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail(REELS_HIP_EHIP, std::string(fn) + ": hipGetDevice: " + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(REELS_HIP_EHIP, std::string(fn) + ": device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(REELS_HIP_EHIP, std::string(fn) + ": hipGetSymbolAddress(scratch): " +
                                      hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return REELS_HIP_OK;
}

// noalloc: never the dequantized-weight plan (its N*K*2-byte copy is what would not fit a modest
// scratch), the workspace is the device's scratch array
static int i8lora_fwd_impl(int elt, const char* fn, const void* x, const int8_t* q,
                           const float* scales, const void* A, const void* B, const void* bias,
                           int64_t M, int64_t K, int64_t N, int64_t r, float lora_scale, void* y,
                           void* h_save, void* workspace, size_t ws_bytes, void* stream,
                           bool noalloc = false, void* gout = nullptr, bool* gelu_fused = nullptr) {
  clear_error();
  if (M < 0 || K <= 0 || N <= 0 || r < 0 || r > 4096)
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": " "need M >= 0, K > 0, N > 0, 0 <= r <= 4096");
  if (!(lora_scale == lora_scale))
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": " "lora_scale is NaN");
  if (M == 0) return REELS_HIP_OK;
  if (!x || !q || !scales || !y || (r > 0 && (!A || !B)))
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": " "NULL x, q, scales, y, or A/B with r > 0");
  const bool al = all_aligned({x, q, scales, A, B, y, h_save}) &&
                  (bias == nullptr || (reinterpret_cast<uintptr_t>(bias) & 7u) == 0);
  Plan p = make_plan(M, K, N, r, al);
  if (noalloc) noalloc_plan(p);
  WsLayout w = ws_layout(M, K, N, r, REELS_HIP_WS_FWD, p);
  if (noalloc) {
    if (w.total > kScratchBytes)
      return fail(REELS_HIP_EINVAL,
                  std::string(fn) + ": these sizes need " + std::to_string(w.total) +
                      " bytes of scratch, more than the " + std::to_string(kScratchBytes) +
                      " this entry point holds (use reels_hip_i8lora_fwd with a workspace)");
    int rc0 = scratch_for_current_device(fn, &workspace);
    if (rc0) return rc0;
    ws_bytes = kScratchBytes;
  }
  if (workspace == nullptr || ws_bytes < w.total)
    return fail(REELS_HIP_EWORKSPACE, std::string(fn) + ": " "workspace NULL or smaller than "
                                      "reels_hip_i8lora_workspace_bytes(..., REELS_HIP_WS_FWD)");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const uint16_t* xb = static_cast<const uint16_t*>(x);
  int rc;
  if (p.skinny) {
    // few tokens: y and h from the int8 codes in one launch
    const uint16_t* Ap = static_cast<const uint16_t*>(A);
    if (r > 0 && p.padded) {
      uint16_t* ap = reinterpret_cast<uint16_t*>(ws + w.ap);
      if ((rc = launch_pad_cols(Ap, K, (int)r, r, ap, p.rp, p.rp, st))) return rc;
      Ap = ap;
    }
    return launch_skinny(0, elt, p.skf, xb, q, K, nullptr, r > 0 ? Ap : nullptr,
                         reinterpret_cast<float*>(ws + w.pa), M, K, N, (int)r, p.rp, scales,
                         static_cast<const uint16_t*>(B), N, static_cast<const uint16_t*>(bias),
                         lora_scale, static_cast<uint16_t*>(y), static_cast<uint16_t*>(h_save), r,
                         (int)r, st);
  }
  // h [M][rp]: straight into h_save unless padded columns make the layouts differ
  uint16_t* h = r > 0 ? ((h_save && !p.padded) ? static_cast<uint16_t*>(h_save)
                                               : reinterpret_cast<uint16_t*>(ws + w.h))
                      : nullptr;
  if (!p.fast) {
    if (r > 0) {
      { TraceScope _ts(st, "g_rowproj_kernel"); with_elt(elt, [&](auto e) { g_rowproj_kernel<decltype(e)::value><<<grid1(M * r), 256, 0, st>>>(xb, M, K, static_cast<const uint16_t*>(A), r, 1,
                                                    (int)r, h, r); }); }
      if ((rc = check_launch("g_rowproj_kernel"))) return rc;
    }
    { TraceScope _ts(st, "g_fwd_kernel"); with_elt(elt, [&](auto e) { g_fwd_kernel<decltype(e)::value><<<grid1(M * N), 256, 0, st>>>(xb, q, scales, h, r, static_cast<const uint16_t*>(B),
                                              static_cast<const uint16_t*>(bias), M, K, N, (int)r,
                                              lora_scale, static_cast<uint16_t*>(y)); }); }
    return check_launch("g_fwd_kernel");
  }
  uint16_t* bt = nullptr;
  if (r > 0) {
    uint16_t* at = reinterpret_cast<uint16_t*>(ws + w.at);
    bt = reinterpret_cast<uint16_t*>(ws + w.bt);
    // At [r][K] from A [K][r]; Bt [N][rp] from B [r][N] (one launch)
    const TpJob ja = tp_job(static_cast<const uint16_t*>(A), K, r, K, at);
    const TpJob jb = tp_job(static_cast<const uint16_t*>(B), r, N, p.rp, bt);
    if ((rc = launch_transpose_pad(ja, &jb, st))) return rc;
    if ((rc = launch_rowproj(elt, xb, M, K, at, (int)r, p.rp, h, nullptr, nullptr, st,
                             reinterpret_cast<float*>(ws + w.rq)))) return rc;
    if (p.padded && h_save &&
        (rc = launch_pad_cols(h, M, (int)r, p.rp, static_cast<uint16_t*>(h_save), (int)r, r, st)))
      return rc;
  }
  GemmArgs g{};
  g.act = xb; g.q = q; g.colscale = scales; g.L = h; g.R = bt;
  g.bias = static_cast<const uint16_t*>(bias); g.out = static_cast<uint16_t*>(y);
  g.M = M; g.Ncols = N; g.Kred = K; g.ldq = K; g.rp = r > 0 ? p.rp : 0; g.c = lora_scale;
  g.ksplit = p.ksf; g.part = reinterpret_cast<float*>(ws + w.kp);
  if (p.deq && !p.i8f) {
    uint16_t* wd = reinterpret_cast<uint16_t*>(ws + w.wd);
    if ((rc = launch_dequant_rows(elt, q, K, scales, N, K, wd, st))) return rc;
    g.q = nullptr; g.colscale = nullptr;
    g.gout = static_cast<uint16_t*>(gout);
    if (g.gout && !bfgemm_fuses_gelu_fwd(g)) g.gout = nullptr;
    if (g.gout && gelu_fused) *gelu_fused = true;
    return launch_bfgemm(0, elt, g, wd, st);
  }
  return launch_i8gemm(0, elt, g, st);
}

static int i8lora_bwd_impl(int elt, const char* fn, const void* dy, const void* x, const void* h,
                           const int8_t* q, const float* scales, const void* A, const void* B,
                           int64_t M, int64_t K, int64_t N, int64_t r, float lora_scale, void* dx,
                           float* dA, float* dB, float* dbias, void* workspace, size_t ws_bytes,
                           void* stream, const void* gx = nullptr, bool* gelu_fused = nullptr) {
  clear_error();
  if (M < 0 || K <= 0 || N <= 0 || r < 0 || r > 4096)
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": " "need M >= 0, K > 0, N > 0, 0 <= r <= 4096");
  if (!(lora_scale == lora_scale))
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": " "lora_scale is NaN");
  if (r == 0) { dA = nullptr; dB = nullptr; }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  int rc;
  if (M == 0) {  // empty token set: the reductions over tokens are zero
    if (dA) {
      { TraceScope _ts(st, "fill_f32_kernel"); fill_f32_kernel<<<grid1(K * r), 256, 0, st>>>(dA, K * r, 0.0f); }
      if ((rc = check_launch("fill_f32_kernel"))) return rc;
    }
    if (dB) {
      { TraceScope _ts(st, "fill_f32_kernel"); fill_f32_kernel<<<grid1(N * r), 256, 0, st>>>(dB, N * r, 0.0f); }
      if ((rc = check_launch("fill_f32_kernel"))) return rc;
    }
    if (dbias) {
      { TraceScope _ts(st, "fill_f32_kernel"); fill_f32_kernel<<<grid1(N), 256, 0, st>>>(dbias, N, 0.0f); }
      if ((rc = check_launch("fill_f32_kernel"))) return rc;
    }
    return REELS_HIP_OK;
  }
  if (!dy || !q || !scales || (r > 0 && (!A || !B)) || ((dA || (dB && !h)) && !x))
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": " "NULL dy, q, scales, A/B with r > 0, or x "
                                  "needed for dA / recomputing h");
  if (!dx && !dA && !dB && !dbias) return REELS_HIP_OK;
  const bool al = all_aligned({dy, x, h, q, scales, A, B, dx, dA, dB, dbias});
  Plan p = make_plan(M, K, N, r, al);
  WsLayout w = ws_layout(M, K, N, r, REELS_HIP_WS_BWD, p);
  if (workspace == nullptr || ws_bytes < w.total)
    return fail(REELS_HIP_EWORKSPACE, std::string(fn) + ": " "workspace NULL or smaller than "
                                      "reels_hip_i8lora_workspace_bytes(..., REELS_HIP_WS_BWD)");
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const uint16_t* dyb = static_cast<const uint16_t*>(dy);
  const uint16_t* xb = static_cast<const uint16_t*>(x);
  const uint16_t* Ab = static_cast<const uint16_t*>(A);
  const uint16_t* Bb = static_cast<const uint16_t*>(B);
  uint16_t* u = reinterpret_cast<uint16_t*>(ws + w.u);
  const uint16_t* hh = static_cast<const uint16_t*>(h);
  const bool need_h = (dB != nullptr) && r > 0;

  if (!p.fast) {
    if (r > 0 && (dx || dA)) {
      { TraceScope _ts(st, "g_rowproj_kernel"); with_elt(elt, [&](auto e) { g_rowproj_kernel<decltype(e)::value><<<grid1(M * r), 256, 0, st>>>(dyb, M, N, Bb, 1, N, (int)r, u, r); }); }
      if ((rc = check_launch("g_rowproj_kernel"))) return rc;
    }
    if (need_h && !hh) {
      uint16_t* hw = reinterpret_cast<uint16_t*>(ws + w.h);
      { TraceScope _ts(st, "g_rowproj_kernel"); with_elt(elt, [&](auto e) { g_rowproj_kernel<decltype(e)::value><<<grid1(M * r), 256, 0, st>>>(xb, M, K, Ab, r, 1, (int)r, hw, r); }); }
      if ((rc = check_launch("g_rowproj_kernel"))) return rc;
      hh = hw;
    }
    if (dx) {
      { TraceScope _ts(st, "g_dx_kernel"); with_elt(elt, [&](auto e) { g_dx_kernel<decltype(e)::value><<<grid1(M * K), 256, 0, st>>>(dyb, q, scales, u, r, Ab, M, K, N, (int)r, lora_scale,
                                               static_cast<uint16_t*>(dx)); }); }
      if ((rc = check_launch("g_dx_kernel"))) return rc;
    }
    if (dA) {
      { TraceScope _ts(st, "g_colgrad_kernel<false>"); with_elt(elt, [&](auto e) { g_colgrad_kernel<false, decltype(e)::value><<<grid1(K * r), 256, 0, st>>>(xb, M, K, u, r, (int)r, lora_scale, dA); }); }
      if ((rc = check_launch("g_colgrad_kernel"))) return rc;
    }
    if (dB) {
      { TraceScope _ts(st, "g_colgrad_kernel<true>"); with_elt(elt, [&](auto e) { g_colgrad_kernel<true, decltype(e)::value><<<grid1(N * r), 256, 0, st>>>(dyb, M, N, hh, r, (int)r, lora_scale, dB); }); }
      if ((rc = check_launch("g_colgrad_kernel"))) return rc;
    }
    if (dbias)
      return launch_colsum(elt, dyb, M, N, reinterpret_cast<float*>(ws + w.pbias), dbias, st);
    return REELS_HIP_OK;
  }

  uint16_t* dys = reinterpret_cast<uint16_t*>(ws + w.dys);
  const bool f16 = elt == REELS_HIP_F16;
  // the dX epilogue's A and the dB pass's h in the padded [.][rp] layout
  const uint16_t* Ar = Ab;
  if (p.padded && dx) {
    uint16_t* ap = reinterpret_cast<uint16_t*>(ws + w.ap);
    if ((rc = launch_pad_cols(Ab, K, (int)r, r, ap, p.rp, p.rp, st))) return rc;
    Ar = ap;
  }
  if (p.padded && need_h && hh) {
    uint16_t* hw = reinterpret_cast<uint16_t*>(ws + w.h);
    if ((rc = launch_pad_cols(hh, M, (int)r, r, hw, p.rp, p.rp, st))) return rc;
    hh = hw;
  }
  if (p.skinny && dx) {
    // few tokens: dx and u = rnd(dy B^T) from one launch over the int8 codes (u lands in the
    // workspace for the dA pass)
    if ((rc = launch_skinny(1, elt, p.skb, dyb, q, K, scales, r > 0 ? Bb : nullptr,
                            reinterpret_cast<float*>(ws + w.wd), M, N, K, (int)r, p.rp, nullptr,
                            Ar, p.rp, nullptr, lora_scale, static_cast<uint16_t*>(dx),
                            r > 0 ? u : nullptr, p.rp, p.rp, st)))
      return rc;
  } else if (p.skinny) {
    if (r > 0 && dA &&
        (rc = launch_rowproj(elt, dyb, M, N, Bb, (int)r, p.rp, u, nullptr, nullptr, st)))
      return rc;
  } else if (p.deq) {
    // 1. u = dy B^T; 2. dx = dy wt^T + c u A^T with wt[k][n] = bf16(q[n][k] s[n])
    if (r > 0 && (dx || dA)) {
      if ((rc = launch_rowproj(elt, dyb, M, N, Bb, (int)r, p.rp, u, nullptr, nullptr, st,
                               reinterpret_cast<float*>(ws + w.rq)))) return rc;
    }
    if (dx) {
      uint16_t* wt = reinterpret_cast<uint16_t*>(ws + w.wd);
      if ((rc = launch_dequant_transpose(elt, q, K, scales, N, K, wt, st))) return rc;
      GemmArgs g{};
      g.act = dyb; g.q = nullptr; g.colscale = nullptr; g.L = r > 0 ? u : nullptr; g.R = Ar;
      g.bias = nullptr; g.out = static_cast<uint16_t*>(dx);
      g.M = M; g.Ncols = K; g.Kred = N; g.ldq = N; g.rp = r > 0 ? p.rp : 0; g.c = lora_scale;
      g.ksplit = p.ksb; g.part = reinterpret_cast<float*>(ws + w.kp);
      g.gx = static_cast<const uint16_t*>(gx);
      if (g.gx && !bfgemm_fuses_gelu(g)) g.gx = nullptr;
      if (g.gx && gelu_fused) *gelu_fused = true;
      if ((rc = launch_bfgemm(1, elt, g, wt, st))) return rc;
    }
  } else if (r > 0 || (dx && !f16)) {
    // 1. u = dy B^T and (bf16) dys = dy * s in one pass over dy (the scaled copy only when dx is
    // wanted); f16 keeps dy as it is and scales the weight inside the dX GEMM instead
    uint16_t* scaled = (dx && !f16) ? dys : nullptr;
    if (r > 0) {
      if ((rc = launch_rowproj(elt, dyb, M, N, Bb, (int)r, p.rp, u, scales, scaled, st,
                               reinterpret_cast<float*>(ws + w.rq)))) return rc;
    } else {
      // r = 0: only the scaled copy is needed (no projection output)
      if ((rc = launch_rowproj(elt, dyb, M, N, Bb, 0, 0, nullptr, scales, scaled, st))) return rc;
    }
  }
  // 2. dx = dys q + c u A^T (bf16), dx = dy f16(q f16(s)) + c u A^T (f16)
  if (dx && !p.deq && !p.skinny) {
    GemmArgs g{};
    g.act = f16 ? dyb : dys; g.q = q; g.colscale = nullptr; g.redscale = f16 ? scales : nullptr;
    g.L = r > 0 ? u : nullptr; g.R = Ar; g.bias = nullptr;
    g.out = static_cast<uint16_t*>(dx);
    g.M = M; g.Ncols = K; g.Kred = N; g.ldq = K; g.rp = r > 0 ? p.rp : 0; g.c = lora_scale;
    g.ksplit = p.ksb; g.part = reinterpret_cast<float*>(ws + w.kp);
    if ((rc = launch_i8gemm(1, elt, g, st))) return rc;
  }
  // 3. dA = c x^T u ; dB = c (dy^T h)^T, in one launch (h recomputed first when not given)
  if (dB) {
    if (!hh && p.skinny) {
      // recompute h exactly as the few-token forward computed it (same blocks, same split order)
      uint16_t* hw = reinterpret_cast<uint16_t*>(ws + w.h);
      const uint16_t* Ap = Ab;
      if (p.padded) {
        uint16_t* ap = reinterpret_cast<uint16_t*>(ws + w.at);  // A [K][rp] in the A^T slot
        if ((rc = launch_pad_cols(Ab, K, (int)r, r, ap, p.rp, p.rp, st))) return rc;
        Ap = ap;
      }
      if ((rc = launch_skinny(0, elt, p.skf, xb, q, K, nullptr, Ap, reinterpret_cast<float*>(ws + w.wd),
                              M, K, N, (int)r, p.rp, nullptr, nullptr, N, nullptr, lora_scale, nullptr,
                              hw, p.rp, p.rp, st, true)))
        return rc;
      hh = hw;
    }
    if (!hh) {
      uint16_t* at = reinterpret_cast<uint16_t*>(ws + w.at);
      uint16_t* hw = reinterpret_cast<uint16_t*>(ws + w.h);
      if ((rc = launch_transpose_pad(tp_job(Ab, K, r, K, at), nullptr, st))) return rc;
      if ((rc = launch_rowproj(elt, xb, M, K, at, (int)r, p.rp, hw, nullptr, nullptr, st,
                               reinterpret_cast<float*>(ws + w.rq)))) return rc;
      hh = hw;
    }
  }
  {
    CgPass ga{}, gb{};
    if (dA) ga = CgPass{xb, K, u, p.sa, reinterpret_cast<float*>(ws + w.pa), dA, false};
    if (dB) {
      gb = CgPass{dyb, N, hh, p.sb, reinterpret_cast<float*>(ws + w.pb), dB, true};
      // the bias gradient from the same pass over dy
      gb.bpart = reinterpret_cast<float*>(ws + w.pbias);
      gb.bout = dbias;
    }
    if ((rc = launch_colgrad2(elt, M, (int)r, p.rp, lora_scale, ga, gb, st))) return rc;
  }
  if (dbias && !dB)
    return launch_colsum(elt, dyb, M, N, reinterpret_cast<float*>(ws + w.pbias), dbias, st);
  return REELS_HIP_OK;
}

static int gelu_impl(int elt, const char* fn, const void* x, void* y, int64_t n, void* stream) {
  clear_error();
  if (n < 0) return fail(REELS_HIP_EINVAL, std::string(fn) + ": " "n < 0");
  if (n == 0) return REELS_HIP_OK;
  if (!x || !y) return fail(REELS_HIP_EINVAL, std::string(fn) + ": " "NULL pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int vec = aligned16(x) && aligned16(y);
  { TraceScope _ts(st, "gelu_kernel");
    with_elt(elt, [&](auto e) { gelu_kernel<decltype(e)::value><<<grid_stream(n), 256, 0, st>>>(static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), n, vec); }); }
  return check_launch("gelu_kernel");
}

static int gelu_bwd_impl(int elt, const char* fn, const void* x, const void* dy, void* dx, int64_t n,
                         void* stream) {
  clear_error();
  if (n < 0) return fail(REELS_HIP_EINVAL, std::string(fn) + ": " "n < 0");
  if (n == 0) return REELS_HIP_OK;
  if (!x || !dy || !dx) return fail(REELS_HIP_EINVAL, std::string(fn) + ": " "NULL pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int vec = aligned16(x) && aligned16(dy) && aligned16(dx);
  { TraceScope _ts(st, "gelu_bwd_kernel");
    with_elt(elt, [&](auto e) { gelu_bwd_kernel<decltype(e)::value><<<grid_stream(n), 256, 0, st>>>(static_cast<const uint16_t*>(x),
                                              static_cast<const uint16_t*>(dy),
                                              static_cast<uint16_t*>(dx), n, vec); }); }
  return check_launch("gelu_bwd_kernel");
}

extern "C" int reels_hip_i8lora_fwd(const void* x, const int8_t* q, const float* scales,
                                    const void* A, const void* B, const void* bias, int64_t M,
                                    int64_t K, int64_t N, int64_t r, float lora_scale, void* y,
                                    void* h_save, void* workspace, size_t ws_bytes, void* stream) {
  return i8lora_fwd_impl(REELS_HIP_BF16, "reels_hip_i8lora_fwd", x, q, scales, A, B, bias, M, K, N,
                         r, lora_scale, y, h_save, workspace, ws_bytes, stream);
}

extern "C" int reels_hip_i8lora_fwd_noalloc(const void* x, const int8_t* q, const float* scales,
                                            const void* A, const void* B, const void* bias,
                                            int64_t M, int64_t K, int64_t N, int64_t r,
                                            float lora_scale, void* y, void* h_save, void* stream) {
  return i8lora_fwd_impl(REELS_HIP_BF16, "reels_hip_i8lora_fwd_noalloc", x, q, scales, A, B, bias,
                         M, K, N, r, lora_scale, y, h_save, nullptr, 0, stream, true);
}

extern "C" int reels_hip_i8lora_fwd_f16(const void* x, const int8_t* q, const float* scales,
                                        const void* A, const void* B, const void* bias, int64_t M,
                                        int64_t K, int64_t N, int64_t r, float lora_scale, void* y,
                                        void* h_save, void* workspace, size_t ws_bytes,
                                        void* stream) {
  return i8lora_fwd_impl(REELS_HIP_F16, "reels_hip_i8lora_fwd_f16", x, q, scales, A, B, bias, M, K,
                         N, r, lora_scale, y, h_save, workspace, ws_bytes, stream);
}

extern "C" int reels_hip_i8lora_bwd(const void* dy, const void* x, const void* h, const int8_t* q,
                                    const float* scales, const void* A, const void* B, int64_t M,
                                    int64_t K, int64_t N, int64_t r, float lora_scale, void* dx,
                                    float* dA, float* dB, void* workspace, size_t ws_bytes,
                                    void* stream) {
  return i8lora_bwd_impl(REELS_HIP_BF16, "reels_hip_i8lora_bwd", dy, x, h, q, scales, A, B, M, K, N,
                         r, lora_scale, dx, dA, dB, nullptr, workspace, ws_bytes, stream);
}

extern "C" int reels_hip_i8lora_bwd_bias(const void* dy, const void* x, const void* h,
                                         const int8_t* q, const float* scales, const void* A,
                                         const void* B, int64_t M, int64_t K, int64_t N,
                                         int64_t r, float lora_scale, void* dx, float* dA,
                                         float* dB, float* dbias, void* workspace,
                                         size_t ws_bytes, void* stream) {
  return i8lora_bwd_impl(REELS_HIP_BF16, "reels_hip_i8lora_bwd_bias", dy, x, h, q, scales, A, B, M,
                         K, N, r, lora_scale, dx, dA, dB, dbias, workspace, ws_bytes, stream);
}

extern "C" int reels_hip_i8lora_bwd_bias_f16(const void* dy, const void* x, const void* h,
                                             const int8_t* q, const float* scales, const void* A,
                                             const void* B, int64_t M, int64_t K, int64_t N,
                                             int64_t r, float lora_scale, void* dx, float* dA,
                                             float* dB, float* dbias, void* workspace,
                                             size_t ws_bytes, void* stream) {
  return i8lora_bwd_impl(REELS_HIP_F16, "reels_hip_i8lora_bwd_bias_f16", dy, x, h, q, scales, A, B,
                         M, K, N, r, lora_scale, dx, dA, dB, dbias, workspace, ws_bytes, stream);
}

extern "C" int reels_hip_i8lora_bwd_f16(const void* dy, const void* x, const void* h,
                                        const int8_t* q, const float* scales, const void* A,
                                        const void* B, int64_t M, int64_t K, int64_t N, int64_t r,
                                        float lora_scale, void* dx, float* dA, float* dB,
                                        void* workspace, size_t ws_bytes, void* stream) {
  return i8lora_bwd_impl(REELS_HIP_F16, "reels_hip_i8lora_bwd_f16", dy, x, h, q, scales, A, B, M, K,
                         N, r, lora_scale, dx, dA, dB, nullptr, workspace, ws_bytes, stream);
}

// The first FFN projection's forward followed by the GELU (transformer.jl:289-292, linear.jl:61-68):
// g = gelu_tanh(y) written by the GEMM's epilogue beside y where the forward runs on the unsplit
// dequantized-weight GEMM, otherwise by the separate pass after it (the same bits either way).
static int i8lora_fwd_gelu_impl(int elt, const char* fn, const void* x, const int8_t* q,
                                const float* scales, const void* A, const void* B,
                                const void* bias, int64_t M, int64_t K, int64_t N, int64_t r,
                                float lora_scale, void* y, void* g, void* h_save, void* workspace,
                                size_t ws_bytes, void* stream) {
  if (M > 0 && !g) {
    clear_error();
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": NULL g");
  }
  bool fused = false;
  if (int rc = i8lora_fwd_impl(elt, fn, x, q, scales, A, B, bias, M, K, N, r, lora_scale, y, h_save,
                               workspace, ws_bytes, stream, false, g, &fused))
    return rc;
  if (fused || M == 0) return REELS_HIP_OK;
  return gelu_impl(elt, fn, y, g, M * N, stream);
}

extern "C" int reels_hip_i8lora_fwd_gelu(const void* x, const int8_t* q, const float* scales,
                                         const void* A, const void* B, const void* bias, int64_t M,
                                         int64_t K, int64_t N, int64_t r, float lora_scale, void* y,
                                         void* g, void* h_save, void* workspace, size_t ws_bytes,
                                         void* stream) {
  return i8lora_fwd_gelu_impl(REELS_HIP_BF16, "reels_hip_i8lora_fwd_gelu", x, q, scales, A, B, bias,
                              M, K, N, r, lora_scale, y, g, h_save, workspace, ws_bytes, stream);
}

extern "C" int reels_hip_i8lora_fwd_gelu_f16(const void* x, const int8_t* q, const float* scales,
                                             const void* A, const void* B, const void* bias,
                                             int64_t M, int64_t K, int64_t N, int64_t r,
                                             float lora_scale, void* y, void* g, void* h_save,
                                             void* workspace, size_t ws_bytes, void* stream) {
  return i8lora_fwd_gelu_impl(REELS_HIP_F16, "reels_hip_i8lora_fwd_gelu_f16", x, q, scales, A, B,
                              bias, M, K, N, r, lora_scale, y, g, h_save, workspace, ws_bytes,
                              stream);
}

// The second FFN projection's backward with the GELU's pullback (transformer.jl:289-292,
// linear.jl:61-68): fused into the dX GEMM's epilogue where dX runs on the unsplit
// dequantized-weight GEMM, otherwise the separate pass after it (the same bits either way).
static int i8lora_bwd_gelu_impl(int elt, const char* fn, const void* dy, const void* x,
                                const void* h, const int8_t* q, const float* scales, const void* A,
                                const void* B, const void* gx, int64_t M, int64_t K, int64_t N,
                                int64_t r, float lora_scale, void* dx, float* dA, float* dB,
                                float* dbias, void* workspace, size_t ws_bytes, void* stream) {
  if (M > 0 && dx && !gx) {
    clear_error();
    return fail(REELS_HIP_EINVAL, std::string(fn) + ": NULL gx with dx");
  }
  bool fused = false;
  if (int rc = i8lora_bwd_impl(elt, fn, dy, x, h, q, scales, A, B, M, K, N, r, lora_scale, dx, dA,
                               dB, dbias, workspace, ws_bytes, stream, dx ? gx : nullptr, &fused))
    return rc;
  if (fused || M == 0 || !dx) return REELS_HIP_OK;
  return gelu_bwd_impl(elt, fn, gx, dx, dx, M * K, stream);
}

extern "C" int reels_hip_i8lora_bwd_gelu(const void* dy, const void* x, const void* h,
                                         const int8_t* q, const float* scales, const void* A,
                                         const void* B, const void* gx, int64_t M, int64_t K,
                                         int64_t N, int64_t r, float lora_scale, void* dx,
                                         float* dA, float* dB, float* dbias, void* workspace,
                                         size_t ws_bytes, void* stream) {
  return i8lora_bwd_gelu_impl(REELS_HIP_BF16, "reels_hip_i8lora_bwd_gelu", dy, x, h, q, scales, A,
                              B, gx, M, K, N, r, lora_scale, dx, dA, dB, dbias, workspace,
                              ws_bytes, stream);
}

extern "C" int reels_hip_i8lora_bwd_gelu_f16(const void* dy, const void* x, const void* h,
                                             const int8_t* q, const float* scales, const void* A,
                                             const void* B, const void* gx, int64_t M, int64_t K,
                                             int64_t N, int64_t r, float lora_scale, void* dx,
                                             float* dA, float* dB, float* dbias, void* workspace,
                                             size_t ws_bytes, void* stream) {
  return i8lora_bwd_gelu_impl(REELS_HIP_F16, "reels_hip_i8lora_bwd_gelu_f16", dy, x, h, q, scales,
                              A, B, gx, M, K, N, r, lora_scale, dx, dA, dB, dbias, workspace,
                              ws_bytes, stream);
}

extern "C" int reels_hip_gelu_tanh(const void* x, void* y, int64_t n, void* stream) {
  return gelu_impl(REELS_HIP_BF16, "reels_hip_gelu_tanh", x, y, n, stream);
}

extern "C" int reels_hip_gelu_tanh_f16(const void* x, void* y, int64_t n, void* stream) {
  return gelu_impl(REELS_HIP_F16, "reels_hip_gelu_tanh_f16", x, y, n, stream);
}

extern "C" int reels_hip_gelu_tanh_bwd(const void* x, const void* dy, void* dx, int64_t n, void* stream) {
  return gelu_bwd_impl(REELS_HIP_BF16, "reels_hip_gelu_tanh_bwd", x, dy, dx, n, stream);
}

extern "C" int reels_hip_gelu_tanh_bwd_f16(const void* x, const void* dy, void* dx, int64_t n,
                                           void* stream) {
  return gelu_bwd_impl(REELS_HIP_F16, "reels_hip_gelu_tanh_bwd_f16", x, dy, dx, n, stream);
}
