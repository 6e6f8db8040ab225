/*
 * libqvggt_hip.so -- C ABI of the MI355X (gfx950) replacement for QVGGT's
 * `awq_inference_engine` extension.
 *
 * Plain pointers and sizes only: every pointer is a device pointer to
 * contiguous row-major data unless stated otherwise, `stream` is a
 * hipStream_t (NULL = the null stream), and every call is asynchronous on
 * that stream.  Return value: QV_OK (0) or a negative QV_E* code; the
 * message for the calling thread's last error is qv_last_error().
 *
 * 16-bit float buffers are passed as `void*` with a `dtype` of QV_F16 or
 * QV_BF16.  Reference citations are paths under
 * qvggt/runtime/awq_inference_engine/csrc/ of the reference repository.
 */
#ifndef QVGGT_HIP_H
#define QVGGT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QV_OK 0
#define QV_EINVAL (-1)      /* bad shape / dtype / alignment / group size */
#define QV_EHIP (-2)        /* HIP runtime reported an error */
#define QV_EUNSUPPORTED (-3)

#define QV_F16 0
#define QV_BF16 1
#define QV_F32 2

/* GEMM epilogues (fusion of qmodule.py:367 `out + bias` and the MLP GELU). */
#define QV_EPI_NONE 0
#define QV_EPI_BIAS 1
#define QV_EPI_BIAS_GELU 2  /* exact-erf GELU after the bias */
#define QV_EPI_GELU 3

/* Message of the calling thread's last failed call ("" if none). */
const char* qv_last_error(void);

/* Library version string. */
const char* qv_version(void);

/*
 * AWQ W4A16 group-128 GEMM:  out[M,N] = x[M,K] . dequant(qweight)^T (+ epilogue)
 *
 * Replaces gemm_forward_cuda_new (quantization_new/gemm/gemm_cuda.h:3,
 * gemm_cuda.cu:1125-1235).  qweight is the AWQ-v2 int16 (N/4, K) layout of
 * awq/qmodule.py:43-99; scales / scaled_zeros are (rows >= K/128, N) tables
 * (qmodule.py:169-211); dequant w = fp16_rn(q*s + sz) as in
 * quantization_new/dequantize.cuh:8-51 + gemm_cuda.cu:911-916.
 * Accumulation is fp32 (the reference accumulates fp16 in fp16).
 * Requires K % 128 == 0, N % 16 == 0, M >= 0.  bias (N) may be NULL unless the
 * epilogue uses it.
 */
int qv_w4a16_gemm(const void* x, const void* qweight, const void* scales,
                  const void* scaled_zeros, const void* bias, void* out,
                  int64_t M, int64_t N, int64_t K, int dtype, int epilogue,
                  void* stream);

/*
 * The launch plan qv_w4a16_gemm (and its residual / q/k-RoPE variants, which
 * plan the same way) picks for an M x K -> N linear, written to plan[4]:
 * plan[0] = 0 skinny kernel (M <= 64), 1 streamed tiles, 2 streamed tiles
 * with K split between two wave groups of one workgroup, 3 streamed tiles
 * with 128-k pipeline stages (2 and 3: launches of at most one tile per CU);
 * plan[1] = tile height of rows [0, plan[2]); plan[3] = tile height of the
 * remaining rows (0: one range).  No device work.  The
 * reference has no counterpart (its gemm_cuda.cu:1125-1235 picks kernels by
 * M bucket internally); it is here for tests and profiling, which need to
 * know which summation order a launch uses.
 */
int qv_w4a16_plan(int64_t M, int64_t N, int64_t K, int epilogue, int32_t* plan);

/*
 * Skinny-M W4A16 GEMV, 1 <= M <= 16 (channels across the grid, 128-k groups
 * across the waves of a workgroup, products on 16x16x32 MFMA, wave partials
 * summed through LDS; the GEMM entry runs M <= 64 on the same kernel).
 * Replaces gemv_forward_cuda_new (quantization_new/gemv/gemv_cuda.h:4-12,
 * gemv_cuda.cu:197-281; the reference accepts M in 1..7 and group 128 only).
 */
int qv_w4a16_gemv(const void* x, const void* qweight, const void* scales,
                  const void* scaled_zeros, const void* bias, void* out,
                  int64_t M, int64_t N, int64_t K, int group_size, int dtype,
                  int epilogue, void* stream);

/*
 * Dequantise the packed weights to a dense (N, K) 16-bit matrix:
 * w[n,k] = fp16_rn(q[n,k]*s[k/128,n] + sz[k/128,n]).  Exposes the reference's
 * device-side dequantisation (dequantize.cuh:8-51 + the hfma2 of
 * gemm_cuda.cu:911-916) as a checkable op; bit-exact by contract.
 */
int qv_w4a16_dequant(const void* qweight, const void* scales,
                     const void* scaled_zeros, void* out_w, int64_t N,
                     int64_t K, int dtype, void* stream);

/*
 * W4A16 linear fused with the LayerScale residual update of a VGGT block:
 * residual[M,N] = residual + gamma[n] * fp16_rn(x . dequant(W)^T + bias[n]),
 * the linear output rounded to the 16-bit type first and the update in fp32
 * with one rounding (the order of `x.addcmul_(proj(h), gamma)` in torch).
 * Same operands and layout checks as qv_w4a16_gemm; bias and gamma (N) are
 * required, residual is read and written in place (16-byte aligned).  The
 * reference has no counterpart: the update is vggt-hf's `x + ls(attn(...))` /
 * `x + ls(mlp(...))` around the quantised proj / fc2 linears
 * (qmodule.py:331-369 computes the linear, then torch adds).
 */
int qv_w4a16_gemm_residual(const void* x, const void* qweight, const void* scales,
                           const void* scaled_zeros, const void* bias, const void* gamma,
                           void* residual, int64_t M, int64_t N, int64_t K, int dtype,
                           void* stream);

/*
 * The VGGT qkv projection fused with what follows it: out (M, 3*H*64) =
 * fp16(x @ W^T + bias), then for every token the per-head LayerNorm of the q
 * and k heads (q_gamma/q_beta, k_gamma/k_beta (64) fp16, eps) rounded to
 * fp16, then the VGGT 2-D RoPE of qv_qknorm_rope2d (positions int32 (M, 2),
 * fp32 cos/sin tables (table_rows, 16)); the v heads get the bias only.
 * fp16 only.  The reference has no single op for this: it is
 * WQLinear.forward (qmodule.py:331-369, gemm_forward_cuda_new) followed by
 * vggt-hf's q_norm / k_norm and RoPE, i.e. qv_w4a16_gemm then
 * qv_qknorm_rope2d, which this entry replaces with one kernel for M > 64
 * (for M <= 64 it runs exactly those two).  The LayerNorm statistics are
 * summed in another order than qv_qknorm_rope2d's, so the q and k outputs
 * may differ from the two-step path in the last bit.
 */
int qv_w4a16_gemm_qkrope(const void* x, const void* qweight, const void* scales,
                         const void* scaled_zeros, const void* bias, void* out,
                         int64_t M, int64_t N, int64_t K, const int32_t* positions,
                         const float* cos_table, const float* sin_table, int64_t table_rows,
                         const void* q_gamma, const void* q_beta, const void* k_gamma,
                         const void* k_beta, float eps, int64_t H, void* stream);

/*
 * qv_w4a16_gemm that allocates nothing: same arguments, kernels, split plan
 * and bit-identical output.  No counterpart in the reference; it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The skinny path's
 * split-K partials and counters live in a fixed file-scope device array of
 * 8 MiB + 16 KiB per GPU, held until the process ends.  A split that would
 * not fit there (more than 4096 channel blocks or 2 Mi partial values) runs
 * unsplit, exactly as qv_w4a16_gemm plans it, so no shape is refused for the
 * array's size.  The first split-K call on a device resolves the array's
 * address and clears its counters (a kernel, then a wait), so make it outside
 * stream capture (under capture it fails with QV_EINVAL); after that, calls
 * may be captured.  All calls on one GPU share the array: calls that overlap
 * (concurrent streams or threads) race.
 */
int qv_w4a16_gemm_noalloc(const void* x, const void* qweight, const void* scales,
                          const void* scaled_zeros, const void* bias, void* out,
                          int64_t M, int64_t N, int64_t K, int dtype, int epilogue,
                          void* stream);

/*
 * Quantise + pack: the buffers WQLinear.from_linear stores
 * (awq/qmodule.py:225-329, pack_intweight at qmodule.py:43-99), computed on
 * the GPU.  weight (N, K), scales and zeros (N, K/group_size) in `dtype`
 * (zeros integer-valued).  q = round((w + z*s) / s) with every operation
 * rounded to `dtype`, packed into qweight int16 (N/4, K) (low 16 bits of the
 * unmasked nibble OR, as the reference); scales_out / scaled_zeros_out
 * (calculate_zeros_width(K, group_size) * 8, N) = s^T and -(s * int(z))^T,
 * zero-padded.  group_size 32, 64, >= 128 dividing K, or -1 (one group).
 * Requires N % 4 == 0, K % 64 == 0; weight and qweight 16-byte aligned.
 */
int qv_w4a16_pack(const void* weight, const void* scales, const void* zeros,
                  void* qweight, void* scales_out, void* scaled_zeros_out,
                  int64_t N, int64_t K, int group_size, int dtype,
                  void* stream);

/* ------------------------------------------------------------ W8A8 family */

/*
 * W8A8 GEMM: out[M,N] fp16 = fp16_rn((float(sum_k a[m,k] b[n,k]) * ws[n]) * as[m] (+ bias[n])).
 * a int8 (M,K), b int8 (N,K), ws fp16 (N), as fp16 (M), bias fp16 (N) or NULL.
 * Replaces w8a8_gemm_forward_cuda / w8a8_gemm_fuse_bias_forward_cuda
 * (w8a8/w8a8_gemm_cuda.h:3-4, w8a8_gemm_cuda.cu:564-607, 881-922).
 * Requires K % 64 == 0, N % 16 == 0.
 */
int qv_w8a8_gemm(const int8_t* a, const int8_t* b, const void* wscales, const void* ascales,
                 const void* bias, void* out, int64_t M, int64_t N, int64_t K, void* stream);

/*
 * W8A8 GEMM + bias fused with a LayerScale residual update, in place:
 * residual[M,N] = fp16(residual + gamma[n] * o), o = the fp16 output of
 * qv_w8a8_gemm with the bias.  No reference op: a VGGT block's W8A8 proj /
 * fc2 (w8a8_gemm_fuse_bias_forward_cuda, w8a8_gemm_cuda.cu:564-607) followed
 * by vggt-hf's LayerScale residual add (x.addcmul_(o, gamma)), fused into the
 * GEMM's store loop.  gamma fp16 (N), 16-byte aligned; bias required.
 */
int qv_w8a8_gemm_residual(const int8_t* a, const int8_t* b, const void* wscales, const void* ascales,
                          const void* bias, const void* gamma, void* residual, int64_t M, int64_t N,
                          int64_t K, void* stream);

/*
 * The raw int32 accumulators of qv_w8a8_gemm (same kernel, no epilogue):
 * out[M,N] int32 = a . b^T.  Exposes dense_kernel0's accumulators
 * (w8a8_gemm_cuda.cu:609-850) as a bit-exact check.
 */
int qv_w8a8_gemm_i32(const int8_t* a, const int8_t* b, int32_t* out, int64_t M, int64_t N,
                     int64_t K, void* stream);

/*
 * Packed W8A8 weights.  No counterpart in the reference: its int8 GEMM reads
 * the (N, K) weight as stored.  For callers that keep a weight across calls
 * (the W8A8 linear module), a one-time re-layout lets the GEMM load each
 * wave's weight fragments straight to registers with one contiguous 1 KB
 * load per instruction.  qv_w8a8_packed_bytes(N, K) is the packed size
 * (N rounded up to 32, times K); qv_w8a8_pack_weight writes it from the
 * (N, K) int8 weight (K a multiple of 64, N of 16).  qv_w8a8_gemm_packed
 * computes what qv_w8a8_gemm computes (gamma NULL; bias optional), or what
 * qv_w8a8_gemm_residual computes (gamma given; bias required, `out` the
 * residual, updated in place), from the packed weight: the same int32
 * accumulators and fp16 results, bit for bit.
 */
int64_t qv_w8a8_packed_bytes(int64_t N, int64_t K);
int qv_w8a8_pack_weight(const int8_t* w, int8_t* packed, int64_t N, int64_t K, void* stream);
int qv_w8a8_gemm_packed(const int8_t* a, const int8_t* packed_b, const void* wscales,
                        const void* ascales, const void* bias, const void* gamma, void* out,
                        int64_t M, int64_t N, int64_t K, void* stream);

/*
 * Per-token int8 quantisation of x (M,D) (dtype QV_F16/QV_BF16/QV_F32):
 * scale[m] fp16 = amax/127, q = sat(rint(x * 127/amax)).
 * Replaces invoke_quant (w8a8/quantization.h:2-4, quantization.cu:42-96).
 */
int qv_quant_per_token(const void* x, int dtype, int8_t* q, void* scale, int64_t M, int64_t D,
                       void* stream);

/*
 * LayerNorm (E[x^2] - mean^2 variance) fused with int8 quantisation.
 * per_token != 0: scale (M) fp16 is written (amax of the rounded LN / 127);
 * per_token == 0: scale[0] fp16 is read and beta is ignored.
 * Replaces rms_norm_general (w8a8/layernorm.h:3-9, layernorm.cu:155-191).
 */
int qv_layernorm_quant(const void* x, int dtype, const void* gamma, const void* beta, int8_t* q,
                       void* scale, float eps, int per_token, int64_t M, int64_t D, void* stream);

/*
 * tanh-GELU (fp16 arithmetic) fused with per-token int8 quantisation; tmp
 * receives the fp16 GELU output.  Replaces gelu_and_quant (w8a8/act.h:5-10,
 * act.cu:22-90).  tmp may be NULL (an extension: the reference always writes
 * it, as the scratch its kernel re-reads): q and scale are the same, and the
 * 2 bytes per element of tmp are not written.
 */
int qv_gelu_quant(const void* x, int8_t* q, void* scale, void* tmp, int64_t M, int64_t D,
                  void* stream);

/* ------------------------------------------------------- normalisation */

/*
 * T5 RMSNorm: out = (x * rsqrt(mean(x^2) + eps)) * gamma, fp16 outputs clamped
 * to +-64504.  Replaces layernorm_forward_cuda (layernorm/layernorm.h:3,
 * layernorm.cu:31-116).
 */
int qv_rmsnorm(const void* x, const void* gamma, void* out, float eps, int64_t M, int64_t D,
               int dtype, void* stream);

/*
 * LayerNorm with torch.nn.LayerNorm semantics (fp32 statistics, two-pass
 * variance, affine).  The VGGT blocks' norm1/norm2; no counterpart in the
 * reference extension (the model graph lives in the external vggt-hf).
 */
int qv_layernorm(const void* x, const void* gamma, const void* beta, void* out, float eps,
                 int64_t M, int64_t D, int dtype, void* stream);

/* ---------------------------------------------------------------- RoPE */

/*
 * Rotate-half RoPE on x[S][B][H][D] with arbitrary element strides
 * (x_strides / out_strides: 4 int64 each, order s,b,h,d) and fp32 angles
 * freqs[B][S][D2]; dims >= D2 copied.  Replaces
 * fused_rope_with_pos_forward_func (rope_new/fused_rope_with_pos.h:3-5,
 * fused_rope_with_pos.cu:19-164).
 */
int qv_rope_with_pos(const void* x, const float* freqs, void* out, int dtype, int64_t S,
                     int64_t B, int64_t H, int64_t D, int64_t D2, const int64_t* x_strides,
                     const int64_t* out_strides, void* stream);

/*
 * VGGT 2-D RoPE (head_dim 64: y on dims [0,32), x on [32,64)) applied to the
 * q and k parts of a fused fp16 qkv buffer (T tokens, token stride
 * src_token_stride elements, layout [3][H][64] per token).  Results go to
 * out + t*dst_token_stride + part*dst_part_stride (part 0 = q, 1 = k); out
 * may alias qkv for in-place use.  positions: int32 (T,2) = (y, x) in
 * [0, table_rows) (out-of-range values are clamped); cos/sin tables fp32
 * (table_rows,16).  Built from fused_rope_with_pos semantics
 * (rope_new/fused_rope_with_pos.cu:19-57); the 2-D split follows VGGT.
 */
int qv_rope2d(const void* qkv, void* out, const int32_t* positions, const float* cos_table,
              const float* sin_table, int64_t table_rows, int64_t T, int64_t H,
              int64_t src_token_stride, int64_t dst_token_stride, int64_t dst_part_stride,
              void* stream);

/*
 * VGGT attention prologue fused in one pass, in place on a fp16 qkv buffer
 * (T tokens x token_stride elements, [3][H][64] per token): per-head
 * LayerNorm of q and k over the 64 head dims (q_gamma/q_beta, k_gamma/k_beta
 * fp16 (64), eps), rounded to fp16, then the 2-D RoPE of qv_rope2d.  No
 * counterpart in the reference extension (VGGT's qk-norm is in vggt-hf).
 */
int qv_qknorm_rope2d(void* qkv, const int32_t* positions, const float* cos_table,
                     const float* sin_table, int64_t table_rows, const void* q_gamma,
                     const void* q_beta, const void* k_gamma, const void* k_beta, float eps,
                     int64_t T, int64_t H, int64_t token_stride, void* stream);

/* ----------------------------------------------------------- attention */

/*
 * Flash attention, fp16 in/out, fp32 softmax/accumulation, no mask:
 * for each of B sequences of L tokens and each of H heads,
 * out = softmax(q k^T * scale) v with head_dim 64 (the only size supported).
 * q/k/v/out are token-major with the given token strides (elements) and head
 * stride 64, so q, k, v can point into a fused (tokens, 3, H, 64) buffer.
 * VGGT frame attention is B = frames, L = 1374; global attention B = 1,
 * L = frames * 1374.  No counterpart in the reference extension (its
 * single_query_attention is an LLM decode kernel, out of scope; VGGT's SDPA
 * lives in the external vggt-hf).
 */
int qv_attention_fwd(const void* q, const void* k, const void* v, void* out, int64_t B,
                     int64_t L, int64_t H, int64_t head_dim, int64_t q_token_stride,
                     int64_t k_token_stride, int64_t v_token_stride, int64_t out_token_stride,
                     float scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QVGGT_HIP_H */
