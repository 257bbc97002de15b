/*
 * Oracle for the int8 frozen-weight LoRA linear: a plain-C, CPU-only restatement of
 * Reels.jl's algorithm (file:line citations are relative to the Reels.jl repository).
 *
 * TEST INFRASTRUCTURE ONLY. The only callers are tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py, and only as the reference results to compare with. The product
 * path (reels_amd/) never links, loads or calls anything here.
 *
 * Physical layouts (row-major, "[a][b]" = a rows of b contiguous elements), identical to the
 * Julia column-major arrays they restate:
 *   x  [M][K] bf16   (Julia x::(K,M))          q  [N][K] int8 (Julia values::(N,K) as transpose)
 *   s  [N]    f32                              A  [K][r] bf16 (Julia A::(r,K))
 *   B  [r][N] bf16   (Julia B::(N,r))          y  [M][N]      (Julia y::(N,M))
 *   dy [M][N]        dx [M][K]                 dA [K][r]      dB [r][N]
 *
 * Parity status of each function is stated beside it.
 */
#ifndef REELS_ORACLE_H
#define REELS_ORACLE_H
#include <stdint.h>
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif

/* bf16 <-> f32 exactly as src/models/interface.jl:13-25 (RNE bit trick, no NaN special case).
 * Pinned by: exhaustive 2^16 round trip, textbook RNE ties, torch's bf16 cast on finite values. */
float    oracle_bf16_to_f32(uint16_t h);
uint16_t oracle_f32_to_bf16(float f);
void     oracle_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n);
void     oracle_bf16_to_f32_array(const uint16_t* in, float* out, int64_t n);

/* quantize_frozen_matrix, src/layers/quantization.jl:35-44.
 * w: [N][K] with leading dimension ld (elements). dtype: 0 = f32, 1 = bf16, 2 = f16.
 * Returns 0, or 1 if any element is non-finite (Julia's Int8(NaN) InexactError), in which case
 * the rows holding non-finite codes are left with the value 0 in q. -1 on bad arguments.
 * Pinned by: a second independent numpy restatement (bit-exact agreement), closed-form special
 * cases (zero rows, exact scale 1 and 2 ties-to-even rows, single spikes, denormal absmax),
 * invariants, and committed golden codes for the real Wan weights in
 * test/fixtures/wan21_block_tiny.safetensors. */
int oracle_pack(const void* w, int dtype, int64_t N, int64_t K, int64_t ld, int8_t* q, float* s);

/* Dequantization variants, src/layers/quantization.jl:25-29 and 61-64.
 * mode 0: Float32(q)*s (f32 out); mode 1: Float16(q)*Float16(s) rounded to f16 (u16 bits out);
 * mode 2: bf16_rne(Float32(q)*s) (u16 bits out). Pinned by closed forms per element. */
void oracle_dequant(const int8_t* q, const float* s, int64_t N, int64_t K, int mode, void* out);

/* 16-bit element codes of the forward / backward / gelu inputs: 0 = bf16 bits, 1 = IEEE binary16
 * bits (the reference's Float16 compute). Both decode exactly to f32. The f16 conversions are
 * exported for tests: f16 -> f32 exact, f32 -> f16 round to nearest even (with subnormals).
 * Pinned by: every one of the 65536 binary16 patterns against numpy's float16, and numpy's
 * float16 rounding on random and boundary f32 values. */
void oracle_f16_to_f32_array(const uint16_t* in, float* out, int64_t n);
void oracle_f32_to_f16_array(const float* in, uint16_t* out, int64_t n);

/* lora_forward, src/layers/lora.jl:56-95 with _weight_mul (quantization.jl:73-74), computed in
 * f64 from 16-bit inputs (the exact value of the math): for each listed row m,
 *   y[m][n] = sum_k x[m][k]*q[n][k]*s[n] + c*sum_j h[m][j]*B[j][n] + bias[n],
 *   h[m][j] = sum_k x[m][k]*A[k][j].
 * rows: row indices to compute (NULL = all M; nrows then ignored). Output rows are packed in
 * the order given (y_out [nrows][N], h_out [nrows][r], either may be NULL). bias may be NULL.
 * Pinned by: brute-force small cases with integer-valued inputs (exact in f64), linearity,
 * B = 0 reducing to the base GEMM (test/unit/lora.jl:6), merged-weight identity (lora.jl:8). */
void oracle_lora_forward(const void* x, const int8_t* q, const float* s, const void* A,
                         const void* B, const void* bias, int64_t M, int64_t K, int64_t N,
                         int64_t r, float c, const int64_t* rows, int64_t nrows, double* y_out,
                         double* h_out, int elt);

/* lora_backward, src/layers/lora.jl:106-118 (and the frozen-weight rrule of
 * src/training/ad_rules.jl:70-80), in f64:
 *   u[m][j]  = sum_n dy[m][n]*B[j][n]
 *   dx[m][k] = sum_n dy[m][n]*s[n]*q[n][k] + c*sum_j u[m][j]*A[k][j]   (listed rows only)
 *   dA[k][j] = c*sum_m u[m][j]*x[m][k]       (all M; listed k columns only, kcols NULL = all)
 *   dB[j][n] = c*sum_m h[m][j]*dy[m][n]      (all M; listed n columns only, ncols NULL = all)
 * with h = x*A in f64. Outputs packed in listed order: dx_out [nrows][K], dA_out [nk][r],
 * dB_out [r][nn]; any may be NULL. Pinned by: central finite differences of
 * oracle_lora_forward (as test/unit/lora.jl:12-21), brute-force integer cases. */
void oracle_lora_backward(const void* dy, const void* x, const int8_t* q, const float* s,
                          const void* A, const void* B, int64_t M, int64_t K, int64_t N,
                          int64_t r, float c, const int64_t* rows, int64_t nrows,
                          const int64_t* kcols, int64_t nk, const int64_t* ncols, int64_t nn,
                          double* dx_out, double* dA_out, double* dB_out, int elt);

/* gelu_tanh, src/layers/linear.jl:61-68, in f32 on bf16 / f16 / f32 inputs, result rounded to
 * the input type, and its analytic derivative applied to an upstream gradient (dx = rnd(dy * gelu'(x))).
 * Pinned by: closed-form values (gelu(0)=0, odd-part identity gelu(x)-gelu(-x)=x), central
 * finite differences for the derivative. */
void oracle_gelu_tanh(const void* x, void* y, int64_t n, int elt);
void oracle_gelu_tanh_backward(const void* x, const void* dy, void* dx, int64_t n,
                               int elt);

/* memory_efficient_attention, src/layers/attention.jl:106-172 (and reference_attention 30-63),
 * as exact scaled dot-product attention in f64 from 16-bit or f32 inputs (elt as above, 2 = f32).
 * Layouts (row-major; the Julia (D, H, tokens, batch) arrays): q [B][Sq][H][D], k and v
 * [B][Sk][H][D], mask [Sq][Sk] uint8 (nonzero = visible; Julia's (key_tokens, query_tokens) Bool
 * array) or NULL, causal: key index <= query index. scale = 1/sqrt(Float32(D)) rounded to f32,
 * as attention.jl:129. out [B][Sq][H][D] and lse [B][H][Sq] (either may be NULL). A query with no
 * visible key gets NaN output and NaN lse, as the reference's online softmax gives (its first
 * rescale is exp(-Inf - -Inf)); with no keys at all (Sk = 0) the lse is -Inf + log(0) = -Inf.
 * Pinned by: q = 0 (uniform weights: the mean of the visible values, lse = log(count)), causal
 * row 0 (= v of key 0), an independent numpy restatement, mask/causal equivalences. */
void oracle_attention_forward(const void* q, const void* k, const void* v, const uint8_t* mask,
                              int causal, int64_t B, int64_t Sq, int64_t Sk, int64_t H, int64_t D,
                              int elt, double* out, double* lse);
/* memory_efficient_attention_backward, attention.jl:174-221, in f64: P from the exact scores,
 * dP = dy V^T, correction = sum(dy .* out) per query (the reference uses its cached output),
 * dS = P (dP - correction), dq = scale dS K, dk = scale dS^T Q, dv = P^T dy. Outputs in the q / k
 * / v layouts, f64 (any may be NULL). Pinned by central finite differences of
 * oracle_attention_forward (as test/unit/layers.jl:56-71 does for reference_attention). */
void oracle_attention_backward(const void* q, const void* k, const void* v, const void* dy,
                               const uint8_t* mask, int causal, int64_t B, int64_t Sq, int64_t Sk,
                               int64_t H, int64_t D, int elt, double* dq, double* dk, double* dv);

/* Philox4x32-10 (Salmon et al., SC'11) counter-based generator for seeded test inputs.
 * Pinned by the published Random123 known-answer vectors. */
void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
/* Normal(0, sigma) values from Philox + Box-Muller (in f64), element i uses counter
 * (i_lo, i_hi, stream, 0) and key (seed_lo, seed_hi). Outliers: if outlier_rate > 0 an element
 * whose third word is < outlier_rate*2^32 becomes +-outlier_sigma*sigma (sign: bit 0 of the
 * fourth word). Written as bf16 (RNE) or f32. */
void oracle_normal_bf16(uint64_t seed, uint32_t stream, int64_t n, double sigma,
                        double outlier_rate, double outlier_sigma, uint16_t* out);
void oracle_normal_f32(uint64_t seed, uint32_t stream, int64_t n, double sigma, float* out);

#ifdef __cplusplus
}
#endif
#endif
