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
 * Skinny-M W4A16 GEMV, 1 <= M <= 16 (wavefront reductions, no MFMA).
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

#ifdef __cplusplus
}
#endif

#endif /* QVGGT_HIP_H */
