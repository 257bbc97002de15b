/*
 * reels_hip: MI355X (gfx950) HIP kernels for Reels.jl's int8 frozen-weight LoRA linear.
 *
 * C ABI only: plain pointers, sizes and a hipStream_t passed as void*. Every pointer argument
 * is a device pointer unless stated otherwise. The caller owns every buffer; the library never
 * allocates caller-visible memory, never frees and keeps no pointer past return. All work is
 * enqueued on `stream` (NULL = the default stream) without host synchronisation, so buffers must
 * stay alive until the caller synchronises that stream.
 *
 * Conventions follow the reference's only native bridge (deps/sentencepiece_bridge.cpp:11-87):
 * an int status (0 = success, negative = error) and a thread-local message retrieved with
 * reels_hip_last_error(), valid until the next call on the same thread.
 *
 * Physical layouts (row-major "[a][b]": a rows of b contiguous elements). They are the memory
 * of the reference's column-major Julia arrays, so a Julia caller passes its arrays unchanged:
 *   x  [M][K] bf16  = Julia x::(K,M)            q  [N][K] int8 = transpose(Julia (K,N) Int8)
 *   s  [N]    f32   = QuantizedMatrix.scales     A  [K][r] bf16 = Julia A::(r,K)
 *   B  [r][N] bf16  = Julia B::(N,r)             y  [M][N] bf16 = Julia y::(N,M)
 *   dy [M][N] bf16, dx [M][K] bf16, dA [K][r] f32 (= Julia (r,K)), dB [r][N] f32 (= (N,r))
 * M = tokens, K = in_features, N = out_features, r = LoRA rank, lora_scale = alpha / r.
 */
#ifndef REELS_HIP_H
#define REELS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define REELS_HIP_ABI_VERSION 1

/* element type codes */
#define REELS_HIP_F32 0
#define REELS_HIP_BF16 1
#define REELS_HIP_F16 2

/* status codes */
#define REELS_HIP_OK 0
#define REELS_HIP_EINVAL (-1)     /* bad argument: NULL pointer, shape, leading dimension */
#define REELS_HIP_EDTYPE (-2)     /* unsupported element type */
#define REELS_HIP_EWORKSPACE (-3) /* workspace NULL or smaller than reels_hip_*_workspace_bytes */
#define REELS_HIP_EHIP (-4)       /* HIP runtime or launch failure */

/* workspace selectors for reels_hip_i8lora_workspace_bytes */
#define REELS_HIP_WS_FWD 0
#define REELS_HIP_WS_BWD 1
#define REELS_HIP_WS_FWD_NOALLOC 2 /* the scratch reels_hip_i8lora_fwd_noalloc needs */

/* ABI version of the loaded library; compare with REELS_HIP_ABI_VERSION. No reference
 * counterpart (the reference has no native library for this path). */
int reels_hip_abi_version(void);

/* Message for the last failed call on this thread ("" if none). Mirrors reels_sp_last_error,
 * deps/sentencepiece_bridge.cpp:11-16 and 83-87. */
const char* reels_hip_last_error(void);

/*
 * quantize_frozen_matrix(W, T), src/layers/quantization.jl:35-44: per output channel
 * (row n of W), absmax over K in f32, scale = absmax / 127f0 (IEEE divide), scale = 1 for a zero
 * row, q = Int8(round_ties_even(clamp(w / scale, -127, 127))). Bit-exact with the reference.
 *   w      [N][ld_w] of dtype REELS_HIP_BF16, REELS_HIP_F16 or REELS_HIP_F32 (ld_w >= K)
 *   q      [N][K] int8 out; scales [N] f32 out
 *   status one device int32, set to 0 then to 1 if any weight is non-finite (the reference
 *          throws InexactError from Int8(NaN)); such elements are written as 0. May be NULL.
 * Replaces the host-CPU packing in _move_weight (quantization.jl:111-125) and
 * quantized_umt5_state_dict (src/models/wan21/text_encoder.jl:318).
 */
int reels_hip_i8_pack(const void* w, int dtype, int64_t N, int64_t K, int64_t ld_w, int8_t* q,
                      float* scales, int32_t* status, void* stream);

/*
 * Dequantization for compute, _dequantize_for_compute / _host_dequantize
 * (src/layers/quantization.jl:25-29, 54-64): out = cast(T, q * s) per output channel n.
 *   REELS_HIP_F32   out = fl32(q[n][k] * s[n])            Float32.(values) .* Float32.(scales)
 *   REELS_HIP_F16   out = f16(q[n][k] * f16(s[n]))        Float16.(values) .* Float16.(scales)
 *   REELS_HIP_BF16  out = bf16(fl32(q[n][k] * s[n]))      the weight the bf16 GEMMs multiply
 *   q [N][ld_q] int8 (ld_q >= K), scales [N] f32
 *   transpose = 0: out [N][K] (row stride K); 1: out [K][N] (row stride N)
 * The int8 LoRA linear runs the BF16 form internally (plain for the forward, transposed for dX);
 * this entry point exposes it, e.g. for merged_weight.
 */
int reels_hip_i8_dequant(const int8_t* q, const float* scales, int64_t N, int64_t K, int64_t ld_q,
                         int dtype, int transpose, void* out, void* stream);

/* Bytes of device workspace needed by reels_hip_i8lora_fwd (which = REELS_HIP_WS_FWD) or
 * reels_hip_i8lora_bwd (REELS_HIP_WS_BWD) for these sizes, or of the library's scratch that
 * reels_hip_i8lora_fwd_noalloc would use (REELS_HIP_WS_FWD_NOALLOC). Always a multiple of 256;
 * 0 for negative sizes or another selector. */
size_t reels_hip_i8lora_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t r, int which);

/*
 * lora_forward(layer, x), src/layers/lora.jl:56-95, for a LoRALinear whose weight is a
 * QuantizedMatrix (_weight_mul, quantization.jl:73-74), bf16 activations:
 *   h = bf16(x * A)                                    [M][r]
 *   y = bf16(sum_k x[m][k] W[n][k] + lora_scale * sum_j h[m][j] B[j][n] + bias[n])
 * with W = bf16(fl32(q * s)) written into the workspace once per call when K and N are multiples
 * of 64 and there are many tokens (the reference's _materialize_weight, quantization.jl:54-64);
 * otherwise W = q * s exact with s[n] applied to the f32 sum: K or N not a multiple of 64, and the
 * few-token path (M <= 240, or M <= 1024 with N * K <= 2^22; K and N multiples of 64), which
 * reads the int8 codes without a weight copy. With few 256 x 256 output tiles (a few hundred
 * tokens) the GEMM splits its reduction over several workgroups and sums their f32 partials in a
 * fixed order before the one rounding (the workspace holds them); the forward then multiplies the
 * int8 codes with s on the f32 sum, no weight copy. bias may be NULL. r = 0 (A, B NULL) gives the base-only
 * linear(::DenseLayer) of src/layers/linear.jl:38-46. h_save ([M][r] or NULL) receives h for the
 * backward. workspace: device memory of reels_hip_i8lora_workspace_bytes(M, K, N, r,
 * REELS_HIP_WS_FWD).
 */
int reels_hip_i8lora_fwd(const void* x, const int8_t* q, const float* scales, const void* A,
                         const void* B, const void* bias, int64_t M, int64_t K, int64_t N,
                         int64_t r, float lora_scale, void* y, void* h_save, void* workspace,
                         size_t ws_bytes, void* stream);

/*
 * The same with binary16 x, A, B, bias, y and h_save: the reference's own int8 compute
 * precision (Float16, quantization.jl:61-62 and lora.jl:56-95 with T = Float16). Every bf16
 * rounding above becomes an f16 rounding (nearest even). The weight is the one the bf16 entry
 * point's shape rules pick, in binary16: where that entry point multiplies a dequantized copy
 * (K and N multiples of 64, many tokens), W = f16(q * f16(s)) as _dequantize_for_compute
 * computes it; where it multiplies the int8 codes (the few-token path, the split-reduction
 * forward over a few hundred tokens, K or N not a multiple of 64), s[n] is applied to the f32
 * sum of x * q, so y can differ from the f16(q * f16(s)) product in the last f16 bit. The
 * backward (reels_hip_i8lora_bwd_f16) always multiplies f16(q * f16(s)). Same workspace size.
 */
int reels_hip_i8lora_fwd_f16(const void* x, const int8_t* q, const float* scales, const void* A,
                             const void* B, const void* bias, int64_t M, int64_t K, int64_t N,
                             int64_t r, float lora_scale, void* y, void* h_save, void* workspace,
                             size_t ws_bytes, void* stream);

/*
 * reels_hip_i8lora_fwd without a workspace argument: it allocates nothing (no hipMalloc, hipFree
 * or allocating library call), for callers that cannot allocate - code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc. No counterpart in the reference (its
 * forward allocates per call). Same arguments, results and errors as reels_hip_i8lora_fwd except:
 *   - the scratch (the h panel, transposed adapter operands, the few-token kernel's split
 *     partials and keys, the rank projection's split partials) is a 32 MiB device array
 *     inside the library, one per GPU, held until the process ends; sizes for which
 *     reels_hip_i8lora_workspace_bytes(M, K, N, r, REELS_HIP_WS_FWD_NOALLOC) exceeds 32 MiB
 *     return REELS_HIP_EINVAL before any work;
 *   - it always multiplies the int8 codes (s applied to the f32 sum), never a dequantized bf16
 *     copy, so its y can differ from reels_hip_i8lora_fwd's in the last bf16 bit where that entry
 *     point takes the dequantized-weight path (K and N multiples of 64);
 *   - calls that overlap on one GPU (other streams or threads) race on the shared scratch.
 */
int reels_hip_i8lora_fwd_noalloc(const void* x, const int8_t* q, const float* scales,
                                 const void* A, const void* B, const void* bias, int64_t M,
                                 int64_t K, int64_t N, int64_t r, float lora_scale, void* y,
                                 void* h_save, void* stream);

/*
 * lora_backward(layer, x, dy), src/layers/lora.jl:106-118, with the frozen-weight pullback of
 * src/training/ad_rules.jl:70-80 (_weight_transpose_mul, quantization.jl:75-76):
 *   u  = bf16(dy * B^T)                                                      [M][r]
 *   dx = bf16(sum_n dy[m][n] W[n][k] + lora_scale * sum_j u[m][j] A[k][j])
 *   dA = lora_scale * x^T u   (f32 [K][r]);   dB = lora_scale * h^T dy   (f32 [r][N])
 * W = bf16(fl32(q * s)) when K and N are multiples of 64 (a transposed copy in the workspace, or,
 * on the few-token path of reels_hip_i8lora_fwd, built in registers from the codes); when K or N
 * is not a multiple of 64 the product is taken as sum_n bf16(dy[m][n] s[n]) q[n][k]. h: the
 * forward's h_save ([M][r]) or NULL to recompute it.
 * dx, dA, dB may each be NULL to skip that output. r = 0 gives dx = deq(W)^T dy alone
 * (_weight_transpose_mul). dA and dB are overwritten (not accumulated) and are bitwise
 * reproducible run to run.
 */
int reels_hip_i8lora_bwd(const void* dy, const void* x, const void* h, const int8_t* q,
                         const float* scales, const void* A, const void* B, int64_t M, int64_t K,
                         int64_t N, int64_t r, float lora_scale, void* dx, float* dA, float* dB,
                         void* workspace, size_t ws_bytes, void* stream);

/* The same with binary16 dy, x, h, A, B and dx (dA, dB stay f32); roundings and W as in
 * reels_hip_i8lora_fwd_f16. On every path dx multiplies the raw dy by the binary16 weight
 * f16(q * f16(s)) with f32 sums (the reference's Float16 _weight_transpose_mul): dy * s is never
 * rounded to binary16, whose normal range it can fall below. */
int reels_hip_i8lora_bwd_f16(const void* dy, const void* x, const void* h, const int8_t* q,
                             const float* scales, const void* A, const void* B, int64_t M,
                             int64_t K, int64_t N, int64_t r, float lora_scale, void* dx, float* dA,
                             float* dB, void* workspace, size_t ws_bytes, void* stream);

/*
 * lora_backward with the gradient of a trainable bias: LoRALinear's bias when train_bias is set
 * (src/layers/lora.jl:37-38, lora_parameters, and 64-67, where the forward adds it with
 * mixed_add, src/layers/linear.jl:7-13). The reference lets Zygote differentiate that add, which
 * gives dbias[n] = sum over tokens m of dy[m][n]; here it is
 *   dbias [N] f32 = sum_m dy[m][n]   (f32 sums in a fixed order: bitwise reproducible)
 * beside the outputs of reels_hip_i8lora_bwd (same arguments, same meaning, same workspace size:
 * reels_hip_i8lora_workspace_bytes(..., REELS_HIP_WS_BWD)). When dB is computed, the column sums
 * come from the dB gradient pass's own read of dy; otherwise (dB NULL, r = 0) from a pass of
 * their own with the same summation order, so dbias does not depend on which outputs are asked
 * for. dbias NULL gives exactly reels_hip_i8lora_bwd.
 */
int reels_hip_i8lora_bwd_bias(const void* dy, const void* x, const void* h, const int8_t* q,
                              const float* scales, const void* A, const void* B, int64_t M,
                              int64_t K, int64_t N, int64_t r, float lora_scale, void* dx,
                              float* dA, float* dB, float* dbias, void* workspace,
                              size_t ws_bytes, void* stream);
/* The same with binary16 dy, x, h, A, B and dx (reels_hip_i8lora_bwd_f16); dbias stays f32. */
int reels_hip_i8lora_bwd_bias_f16(const void* dy, const void* x, const void* h, const int8_t* q,
                                  const float* scales, const void* A, const void* B, int64_t M,
                                  int64_t K, int64_t N, int64_t r, float lora_scale, void* dx,
                                  float* dA, float* dB, float* dbias, void* workspace,
                                  size_t ws_bytes, void* stream);

/* gelu_tanh, src/layers/linear.jl:61-68: y = bf16(0.5x(1 + tanh(sqrt(2/pi)(x + 0.044715x^3))))
 * computed in f32 on bf16 x[n]. */
int reels_hip_gelu_tanh(const void* x, void* y, int64_t n, void* stream);
/* The same on binary16 x and y. */
int reels_hip_gelu_tanh_f16(const void* x, void* y, int64_t n, void* stream);

/* Pullback of gelu_tanh (the reference lets Zygote differentiate linear.jl:61-68):
 * dx = bf16(dy * gelu'(x)) with the analytic derivative in f32. */
int reels_hip_gelu_tanh_bwd(const void* x, const void* dy, void* dx, int64_t n, void* stream);
/* The same on binary16 x, dy and dx. */
int reels_hip_gelu_tanh_bwd_f16(const void* x, const void* dy, void* dx, int64_t n, void* stream);

/*
 * The forward of the Wan FFN's first projection followed by its GELU, transformer.jl:289-292
 * (ffn.0 -> gelu_tanh), in one call. No single counterpart in the reference (its FFN calls the
 * linear, lora.jl:56-95, then gelu_tanh, linear.jl:61-68, in turn); the results are those of the
 * two calls, bit for bit: y [M][N] as reels_hip_i8lora_fwd (the GELU's input, which the
 * backward's reels_hip_i8lora_bwd_gelu takes as gx) and g [M][N] = gelu_tanh(y). Where the
 * forward runs on the dequantized-weight GEMM without a split reduction (many tokens, K and N
 * multiples of 64, 16-byte aligned buffers) the GELU runs in the GEMM's epilogue on the rounded
 * outputs (y is not read back); elsewhere the separate pass runs after it. Workspace as for
 * reels_hip_i8lora_fwd. _f16: binary16 operands, as reels_hip_i8lora_fwd_f16.
 */
int reels_hip_i8lora_fwd_gelu(const void* x, const int8_t* q, const float* scales, const void* A,
                              const void* B, const void* bias, int64_t M, int64_t K, int64_t N,
                              int64_t r, float lora_scale, void* y, void* g, void* h_save,
                              void* workspace, size_t ws_bytes, void* stream);
int reels_hip_i8lora_fwd_gelu_f16(const void* x, const int8_t* q, const float* scales,
                                  const void* A, const void* B, const void* bias, int64_t M,
                                  int64_t K, int64_t N, int64_t r, float lora_scale, void* y,
                                  void* g, void* h_save, void* workspace, size_t ws_bytes,
                                  void* stream);

/*
 * The backward of the Wan FFN's second projection with the GELU's pullback before it,
 * transformer.jl:289-292 (ffn.0 -> gelu_tanh -> ffn.2), in one call. No single counterpart in the
 * reference (its FFN pullback calls the linear's, then gelu_tanh's, linear.jl:61-68, in turn);
 * the results are those of the two calls, bit for bit: reels_hip_i8lora_bwd_bias for the second
 * projection (dbias may be NULL) with dx replaced by gelu_tanh_bwd(gx, dx), gx [M][K] the
 * GELU's input (the first projection's y). Where dX runs on the dequantized-weight GEMM without
 * a split reduction (many tokens, K and N multiples of 64, 16-byte aligned buffers) the pullback
 * runs in the GEMM's epilogue (the product is neither stored nor read back);
 * elsewhere that pass runs after it. Workspace as for reels_hip_i8lora_bwd. _f16: binary16
 * operands, as reels_hip_i8lora_bwd_f16.
 */
int reels_hip_i8lora_bwd_gelu(const void* dy, const void* x, const void* h, const int8_t* q,
                              const float* scales, const void* A, const void* B, const void* gx,
                              int64_t M, int64_t K, int64_t N, int64_t r, float lora_scale,
                              void* dx, float* dA, float* dB, float* dbias, void* workspace,
                              size_t ws_bytes, void* stream);
int reels_hip_i8lora_bwd_gelu_f16(const void* dy, const void* x, const void* h, const int8_t* q,
                                  const float* scales, const void* A, const void* B,
                                  const void* gx, int64_t M, int64_t K, int64_t N, int64_t r,
                                  float lora_scale, void* dx, float* dA, float* dB, float* dbias,
                                  void* workspace, size_t ws_bytes, void* stream);

/*
 * fp32 compute, the reference's Float32 path with int8 frozen weights (_dequantize_for_compute
 * with T = Float32, src/layers/quantization.jl:61-64, and lora_forward / lora_backward in
 * Float32, src/layers/lora.jl:56-118). Every operand, intermediate and result is f32:
 *   W = fl32(q[n][k] * s[n])                   materialised in the workspace once per call
 *   h = x * A                                  [M][r]
 *   y = (x W^T + bias) + lora_scale * (h B)    (the reference's order: mixed_add, then adapter)
 *   u = dy B^T;  dx = dy W + lora_scale * u A^T;  dA = lora_scale x^T u;  dB = lora_scale h^T dy
 * with the layouts of the bf16 entry points (x [M][K], A [K][r], B [r][N], y [M][N], dA [K][r],
 * dB [r][N]). The sums run in f32 on fp32 MFMA. workspace: reels_hip_i8lora_workspace_bytes_f32.
 */
size_t reels_hip_i8lora_workspace_bytes_f32(int64_t M, int64_t K, int64_t N, int64_t r,
                                            int which);
int reels_hip_i8lora_fwd_f32(const float* x, const int8_t* q, const float* scales, const float* A,
                             const float* B, const float* bias, int64_t M, int64_t K, int64_t N,
                             int64_t r, float lora_scale, float* y, float* h_save, void* workspace,
                             size_t ws_bytes, void* stream);
int reels_hip_i8lora_bwd_f32(const float* dy, const float* x, const float* h, const int8_t* q,
                             const float* scales, const float* A, const float* B, int64_t M,
                             int64_t K, int64_t N, int64_t r, float lora_scale, float* dx,
                             float* dA, float* dB, void* workspace, size_t ws_bytes, void* stream);
/* reels_hip_i8lora_bwd_f32 with the trainable bias's gradient dbias [N] = sum_m dy[m][n] (f32,
 * fixed order), as reels_hip_i8lora_bwd_bias; same workspace as reels_hip_i8lora_bwd_f32. */
int reels_hip_i8lora_bwd_bias_f32(const float* dy, const float* x, const float* h,
                                  const int8_t* q, const float* scales, const float* A,
                                  const float* B, int64_t M, int64_t K, int64_t N, int64_t r,
                                  float lora_scale, float* dx, float* dA, float* dB, float* dbias,
                                  void* workspace, size_t ws_bytes, void* stream);
/* gelu_tanh and its pullback on f32 x, dy (linear.jl:61-68 with T = Float32: no rounding). */
int reels_hip_gelu_tanh_f32(const float* x, float* y, int64_t n, void* stream);
int reels_hip_gelu_tanh_bwd_f32(const float* x, const float* dy, float* dx, int64_t n,
                                void* stream);

/*
 * Exact scaled dot-product attention with an online softmax. Replaces
 * memory_efficient_attention (src/layers/attention.jl:106-172 CPU, 225-304 CUDA) and
 * memory_efficient_attention_backward (attention.jl:174-221, 306-371), which the Wan model calls
 * for self- and cross-attention (src/models/wan21/transformer.jl:199, 238-239).
 * Layouts (row-major, the reference's (head_dim, heads, tokens, batch) arrays):
 *   q, out, dy, dq [B][Sq][H][D];  k, v, dk, dv [B][Sk][H][D];  lse [B][H][Sq] f32
 *   mask [Sq][Sk] uint8, nonzero = visible (the reference's (key_tokens, query_tokens) Bool
 *   array), or NULL; causal != 0: key index <= query index.
 * dtype REELS_HIP_BF16, REELS_HIP_F16 or REELS_HIP_F32 for q, k, v, out, dy, dq, dk, dv; head
 * dim 1 <= D <= 128; 16-byte aligned tensors; one batch of q or k below 2 GiB. Scores, softmax
 * and sums run in f32 with scale 1/sqrt(Float32(D)) (attention.jl:129). bf16 / f16 with D = 64
 * or 128 take the tuned kernels, which round P to dtype for the P V product; f32 and other head
 * dims take kernels that keep P in f32 (the reference's order) at a lower rate.
 * A query with no visible key gets NaN output and NaN lse (-Inf when Sk = 0), as the reference;
 * it contributes nothing to dq, dk, dv (in the reference its NaN correction reaches every dk of
 * the head). The reference's query_block / key_block do not change the result and have no
 * parameter here.
 *   reels_hip_attention_fwd: out and (when lse != NULL) lse, the cache the backward needs.
 *   reels_hip_attention_bwd: dq, dk, dv from dy, the forward's out and lse; workspace of
 *     reels_hip_attention_workspace_bytes(B, Sq, H) bytes (the per-query sum(dy .* out)).
 * Deterministic: no atomics, fixed summation order. At D = 128 the backward picks one of two dK/dV
 * kernels by grid size (256 or 64 keys per workgroup; their results differ in rounding, within
 * the same tolerance of the exact math); the environment variable REELS_HIP_ATTN_DKDV_KEYS=256 or
 * =64 fixes the choice.
 */
size_t reels_hip_attention_workspace_bytes(int64_t B, int64_t Sq, int64_t H);
int reels_hip_attention_fwd(const void* q, const void* k, const void* v, const uint8_t* mask,
                            int causal, int64_t B, int64_t Sq, int64_t Sk, int64_t H, int64_t D,
                            int dtype, void* out, float* lse, void* stream);
int reels_hip_attention_bwd(const void* q, const void* k, const void* v, const void* out,
                            const void* dy, const float* lse, const uint8_t* mask, int causal,
                            int64_t B, int64_t Sq, int64_t Sk, int64_t H, int64_t D, int dtype,
                            void* dq, void* dk, void* dv, void* workspace, size_t ws_bytes,
                            void* stream);

/*
 * Kernel timing instrumentation. No counterpart in the reference (it has no profiler hooks);
 * used by benchmarks to time individual kernels with HIP events on the stream each kernel is
 * launched on. While enabled, every kernel the library enqueues is bracketed by two event
 * records (events are created on first use and kept). Not thread-safe against concurrent calls
 * of the entry points on other threads while enabled.
 *   reels_hip_trace_start(capacity): clear old records and record up to `capacity` launches
 *   reels_hip_trace_stop(): stop recording; returns the number of launches recorded
 *   reels_hip_trace_get(i, &name, &ms): kernel name and duration of launch i; the caller must
 *     have synchronised the streams first. Returns REELS_HIP_EINVAL for a bad index.
 *   reels_hip_trace_only(name_part): from now on bracket and record only kernels whose name
 *     contains name_part (NULL or "": every kernel), so the events of a timed loop cost less
 */
int reels_hip_trace_start(int capacity);
int reels_hip_trace_only(const char* name_part);
int reels_hip_trace_stop(void);
int reels_hip_trace_get(int index, const char** name, float* ms);

#ifdef __cplusplus
}
#endif
#endif /* REELS_HIP_H */
