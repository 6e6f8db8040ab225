// Row kernels of the W8A8 / normalisation family for gfx950: per-token int8
// quantisation, LayerNorm + int8 quantisation, tanh-GELU + int8
// quantisation, T5 RMSNorm and (VGGT) LayerNorm.
//
// All are HBM-bound row operations: one wave per row (4 rows per 256-thread
// workgroup), 16-byte loads/stores, every value kept in registers between the
// reduction and the write-out, so each element is read once and written once.
//
// Arithmetic contract (matches the CPU oracle bit for bit): IEEE fp32 ops,
// one rounding each, no contraction into FMA (pragma below); IEEE division and
// square root; row reductions in a fixed order -- chunk c (8 elements) of a
// row belongs to lane c % 64, each lane accumulates its elements in order,
// then a butterfly over lane distances 1, 2, 4, 8, 16, 32.
#include "common.h"

#pragma clang fp contract(off)

namespace qv {

constexpr int ROWS_PER_WG = 4;

template <int DT>
__device__ __forceinline__ void load8(const void* base, size_t e, float (&v)[8]) {
  if constexpr (DT == QV_F32) {
    const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + e);
    const float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 u = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + e);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = to_f32((uint16_t)(w[i] & 0xFFFF), DT == QV_BF16);
      v[2 * i + 1] = to_f32((uint16_t)(w[i] >> 16), DT == QV_BF16);
    }
  }
}

template <int DT>
__device__ __forceinline__ float round_to(float v) {  // fp32 -> storage type -> fp32
  if constexpr (DT != QV_F32) asm volatile("" : "+v"(v));  // no mul+convert fusion (see from_f32)
  if constexpr (DT == QV_F16) return (float)(_Float16)v;
  if constexpr (DT == QV_BF16) return (float)(__bf16)v;
  return v;
}

template <int DT>
__device__ __forceinline__ void store8(void* base, size_t e, const float (&v)[8]) {
  if constexpr (DT == QV_F32) {
    float4* p = reinterpret_cast<float4*>(reinterpret_cast<float*>(base) + e);
    p[0] = make_float4(v[0], v[1], v[2], v[3]);
    p[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    uint4 u;
    u.x = pack2<DT == QV_BF16>(v[0], v[1]);
    u.y = pack2<DT == QV_BF16>(v[2], v[3]);
    u.z = pack2<DT == QV_BF16>(v[4], v[5]);
    u.w = pack2<DT == QV_BF16>(v[6], v[7]);
    *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(base) + e) = u;
  }
}

// cvt.rni.sat.s8 semantics: round half to even, saturate, NaN -> 0.
// v_cvt_i32_f32 already maps NaN to 0 and saturates out-of-range values, so
// rint + convert + integer clamp (v_med3_i32) is the whole operation.  The
// convert is inline asm: a C++ float -> int cast of NaN or of an
// out-of-range value is undefined, and the hardware behaviour is the contract.
__device__ __forceinline__ int sat_s8(float v) {
  int i;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(i) : "v"(__builtin_rintf(v)));
  return i < -128 ? -128 : (i > 127 ? 127 : i);
}

// four int8 (low bytes of a, b, c, d) -> one word, a in the low byte
__device__ __forceinline__ uint32_t pack_s8x4(int a, int b, int c, int d) {
  const uint32_t ab = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);  // [a0, b0, 0, 0]
  const uint32_t cd = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x0c0c0400u);  // [c0, d0, 0, 0]
  return __builtin_amdgcn_perm(cd, ab, 0x05040100u);                                 // [a0, b0, c0, d0]
}

__device__ __forceinline__ void store_q8(int8_t* q, size_t e, const float (&t)[8], float mul) {
  const uint32_t lo = pack_s8x4(sat_s8(t[0] * mul), sat_s8(t[1] * mul), sat_s8(t[2] * mul), sat_s8(t[3] * mul));
  const uint32_t hi = pack_s8x4(sat_s8(t[4] * mul), sat_s8(t[5] * mul), sat_s8(t[6] * mul), sat_s8(t[7] * mul));
  *reinterpret_cast<uint2*>(q + e) = make_uint2(lo, hi);
}

// Cross-lane steps without LDS round trips: DPP within 16-lane rows, the
// gfx950 permlane swaps across rows.  Each returns the partner lane's value
// for the step's pairing; after steps 1..k every 2^k-lane group holds one
// value, which is what lets the mirrors stand in for xor 4 and xor 8.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
// x[l ^ 16] (v_permlane16_swap: rows 1 and 3 of the first operand trade
// places with rows 0 and 2 of the second) and x[l ^ 32] (v_permlane32_swap).
// Inline asm with the VALU -> permlane hazard covered by s_nop.
__device__ __forceinline__ float xor16(float v) {
  float a = v, b = v;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  return (threadIdx.x & 16) ? a : b;
}
__device__ __forceinline__ float xor32(float v) {
  float a = v, b = v;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  return (threadIdx.x & 32) ? a : b;
}

// Butterfly over lane distances 1, 2, 4, 8, 16, 32 (every lane ends with the
// wave total; the pairing is exact, so the fp32 result is the same on every
// lane and equals the oracle's lane tree).
__device__ __forceinline__ float bfly_sum(float v) {
  v = v + dpp<0xB1>(v);   // quad_perm [1,0,3,2]: l ^ 1
  v = v + dpp<0x4E>(v);   // quad_perm [2,3,0,1]: l ^ 2
  v = v + dpp<0x141>(v);  // row_half_mirror: l ^ 4 once quads are uniform
  v = v + dpp<0x140>(v);  // row_mirror: l ^ 8 once 8-lane groups are uniform
  v = v + xor16(v);
  v = v + xor32(v);
  return v;
}

__device__ __forceinline__ float bfly_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  v = fmaxf(v, xor16(v));
  v = fmaxf(v, xor32(v));
  return v;
}

// Row loader shared by every kernel: J chunks of 8 per lane, chunk c = lane + 64*j.
template <int DT, int J>
__device__ __forceinline__ void load_row(const void* x, size_t row, int D, int lane, float (&v)[J][8],
                                         bool (&ok)[J]) {
  const int nch = D >> 3;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = lane + 64 * j;
    ok[j] = c < nch;
    if (ok[j]) {
      load8<DT>(x, row * (size_t)D + (size_t)c * 8, v[j]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[j][e] = 0.0f;
    }
  }
}

template <int J>
__device__ __forceinline__ float row_sum(const float (&v)[J][8]) {
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = acc + v[j][e];
  return bfly_sum(acc);
}

template <int J>
__device__ __forceinline__ float row_sumsq(const float (&v)[J][8]) {
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = acc + v[j][e] * v[j][e];
  return bfly_sum(acc);
}

#define QV_ROW_PROLOGUE                                  \
  const int lane = threadIdx.x & 63;                     \
  const size_t row = (size_t)blockIdx.x * ROWS_PER_WG + (threadIdx.x >> 6); \
  if (row >= (size_t)M) return;

// ------------------------------------------------- per-token quantisation
// quantization.cu:42-96: scale = fp16(amax/127), q = sat(rint(x * (127/amax))).
template <int DT, int J>
__global__ __launch_bounds__(256) void quant_rows_kernel(const void* __restrict__ x, int8_t* __restrict__ q,
                                                         uint16_t* __restrict__ scale, int M, int D) {
  QV_ROW_PROLOGUE
  float v[J][8];
  bool ok[J];
  load_row<DT, J>(x, row, D, lane, v, ok);
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, __builtin_fabsf(v[j][e]));
  amax = bfly_max(amax);
  if (lane == 0) scale[row] = from_f32<false>(amax / 127.0f);
  const float inv = 127.0f / amax;
#pragma unroll
  for (int j = 0; j < J; ++j)
    if (ok[j]) store_q8(q, row * (size_t)D + (size_t)(lane + 64 * j) * 8, v[j], inv);
}

// ------------------------------------------ LayerNorm + int8 quantisation
// layernorm.cu:20-151 (rms_norm_general): mean and E[x^2] in fp32,
// var = E[x^2] - mean^2, y = ((x - mean) * rs) * g (+ b).  Per token: amax over
// y rounded to the input type (floor 1e-6 in that type), int8 from the fp32 y.
// Per tensor: int8 = sat(rint(float(T(y)) * scale)), no beta.  amax is taken
// over |y| in fp32 and rounded once: rounding to the storage type is
// monotonic and odd, so that equals the max over the rounded values.
template <int DT, int J, bool PER_TOKEN>
__global__ __launch_bounds__(256) void ln_quant_kernel(const void* __restrict__ x, const void* __restrict__ gamma,
                                                       const void* __restrict__ beta, int8_t* __restrict__ q,
                                                       uint16_t* __restrict__ scale, float eps, int M, int D) {
  QV_ROW_PROLOGUE
  float v[J][8];
  bool ok[J];
  load_row<DT, J>(x, row, D, lane, v, ok);
  const float s = row_sum<J>(v);
  const float s2 = row_sumsq<J>(v);
  const float mean = s / (float)D;
  const float var = s2 / (float)D - mean * mean;
  const float rs = 1.0f / __builtin_sqrtf(var + eps);
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if (!ok[j]) continue;
    float g[8], b[8];
    const size_t e0 = (size_t)(lane + 64 * j) * 8;
    load8<DT>(gamma, e0, g);
    if constexpr (PER_TOKEN) load8<DT>(beta, e0, b);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float t = (v[j][e] - mean) * rs;
      t = t * g[e];
      if constexpr (PER_TOKEN) t = t + b[e];
      v[j][e] = t;
      if constexpr (PER_TOKEN) amax = fmaxf(amax, __builtin_fabsf(t));
    }
  }
  if constexpr (PER_TOKEN) {
    amax = fmaxf(round_to<DT>(1e-6f), round_to<DT>(bfly_max(amax)));
    const float dyn = 127.0f / amax;
#pragma unroll
    for (int j = 0; j < J; ++j)
      if (ok[j]) store_q8(q, row * (size_t)D + (size_t)(lane + 64 * j) * 8, v[j], dyn);
    if (lane == 0) scale[row] = from_f32<false>(amax / 127.0f);
  } else {
    const float sc = to_f32(scale[0], false);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if (!ok[j]) continue;
      float r[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = round_to<DT>(v[j][e]);
      store_q8(q, row * (size_t)D + (size_t)(lane + 64 * j) * 8, r, sc);
    }
  }
}

// ------------------------------------------------------- T5 RMSNorm
// layernorm/layernorm.cu:31-57: y = (x * rsqrt(mean(x^2) + eps)) * g; fp16
// outputs clamped to +-(65504 - 1000) first (reduction.cuh:60-71).
template <int DT, int J>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const void* __restrict__ x, const void* __restrict__ gamma,
                                                      void* __restrict__ out, float eps, int M, int D) {
  QV_ROW_PROLOGUE
  float v[J][8];
  bool ok[J];
  load_row<DT, J>(x, row, D, lane, v, ok);
  const float s2 = row_sumsq<J>(v);
  const float rs = 1.0f / __builtin_sqrtf(s2 / (float)D + eps);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if (!ok[j]) continue;
    float g[8];
    const size_t e0 = (size_t)(lane + 64 * j) * 8;
    load8<DT>(gamma, e0, g);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float t = (v[j][e] * rs) * g[e];
      if constexpr (DT == QV_F16) t = t > 0.0f ? fminf(t, 65504.0f - 1000.0f) : fmaxf(t, -65504.0f + 1000.0f);
      v[j][e] = t;
    }
    store8<DT>(out, row * (size_t)D + e0, v[j]);
  }
}

// ------------------------------------------------------ VGGT LayerNorm
// torch.nn.LayerNorm semantics (fp32 statistics, two-pass variance):
// y = ((x - mean) * rsqrt(var + eps)) * g + b.
template <int DT, int J>
__global__ __launch_bounds__(256) void layernorm_kernel(const void* __restrict__ x, const void* __restrict__ gamma,
                                                        const void* __restrict__ beta, void* __restrict__ out,
                                                        float eps, int M, int D) {
  QV_ROW_PROLOGUE
  float v[J][8];
  bool ok[J];
  load_row<DT, J>(x, row, D, lane, v, ok);
  const float mean = row_sum<J>(v) / (float)D;
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) v[j][e] = ok[j] ? v[j][e] - mean : 0.0f;
  const float var = row_sumsq<J>(v) / (float)D;
  const float rs = 1.0f / __builtin_sqrtf(var + eps);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if (!ok[j]) continue;
    float g[8], b[8];
    const size_t e0 = (size_t)(lane + 64 * j) * 8;
    load8<DT>(gamma, e0, g);
    load8<DT>(beta, e0, b);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[j][e] = (v[j][e] * rs) * g[e] + b[e];
    store8<DT>(out, row * (size_t)D + e0, v[j]);
  }
}

// --------------------------------------------- tanh-GELU + quantisation
// act.cu:22-75 with T = half: every operation of gelu_fast is one fp16
// rounding; tanh is evaluated in fp64 and rounded to fp32 (then to fp16).
// amax folds t > fp16(1e-4) ? t : -t (act.cu:47-48); the quantiser multiplies
// fp16(127/amax) * tmp in fp16 before the int8 conversion (act.cu:65).
__device__ __forceinline__ _Float16 gelu_fast_h(_Float16 x) {
  const _Float16 a = x * (_Float16)0.79788456f;
  const _Float16 b = ((_Float16)0.044715f * x) * x;
  const _Float16 c = (_Float16)1.0f + b;
  const _Float16 u = a * c;
  const _Float16 t = (_Float16)(float)tanh((double)u);
  return ((_Float16)0.5f * x) * ((_Float16)1.0f + t);
}

template <int J>
__global__ __launch_bounds__(256) void gelu_quant_kernel(const uint16_t* __restrict__ x, int8_t* __restrict__ q,
                                                         uint16_t* __restrict__ scale, uint16_t* __restrict__ tmp,
                                                         int M, int D) {
  QV_ROW_PROLOGUE
  const int nch = D >> 3;
  _Float16 t[J][8];
  float amax = 0.0f;
  const _Float16 zero = (_Float16)0.0001f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = lane + 64 * j;
    if (c >= nch) continue;
    const size_t e0 = row * (size_t)D + (size_t)c * 8;
    const f16x8 xv = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(x + e0));
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      t[j][e] = gelu_fast_h(xv[e]);
      const _Float16 f = t[j][e] > zero ? t[j][e] : -t[j][e];
      amax = fmaxf(amax, (float)f);
    }
    f16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = t[j][e];
    *reinterpret_cast<uint4*>(tmp + e0) = __builtin_bit_cast(uint4, o);
  }
  amax = bfly_max(amax);
  if (lane == 0) scale[row] = from_f32<false>(amax / 127.0f);
  const _Float16 hs = (_Float16)(127.0f / amax);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = lane + 64 * j;
    if (c >= nch) continue;
    float p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) p[e] = (float)(_Float16)(hs * t[j][e]);
    store_q8(q, row * (size_t)D + (size_t)c * 8, p, 1.0f);
  }
}

// ---------------------------------------------------------------- host
static int row_chunks(int64_t D, int& J) {
  const int64_t nch = D / 8;
  const int64_t per_lane = (nch + 63) / 64;
  if (per_lane <= 1) J = 1;
  else if (per_lane <= 2) J = 2;
  else if (per_lane <= 4) J = 4;
  else if (per_lane <= 8) J = 8;
  else if (per_lane <= 16) J = 16;
  else return QV_EINVAL;
  return QV_OK;
}

#define QV_ROW_CHECK(D, M)                                                                                \
  QV_CHECK_ARG((M) >= 0 && (M) <= INT32_MAX, "bad row count %lld", (long long)(M));                      \
  QV_CHECK_ARG((D) > 0 && (D) % 8 == 0 && (D) <= 8192, "row length %lld must be a positive multiple of 8, <= 8192", \
               (long long)(D));

}  // namespace qv

using namespace qv;

static dim3 row_grid(int64_t M) { return dim3((unsigned)((M + ROWS_PER_WG - 1) / ROWS_PER_WG)); }

#define QV_DT_SWITCH(dt, ...)                                         \
  switch (dt) {                                                       \
    case QV_F16: { constexpr int DT = QV_F16; __VA_ARGS__; } break;    \
    case QV_BF16: { constexpr int DT = QV_BF16; __VA_ARGS__; } break;  \
    case QV_F32: { constexpr int DT = QV_F32; __VA_ARGS__; } break;    \
    default: ::qv::set_error("unsupported dtype %d", dt); return QV_EINVAL; \
  }

template <int DT, int J>
static void launch_quant(const void* x, int8_t* q, uint16_t* s, int M, int D, hipStream_t st) {
  hipLaunchKernelGGL((quant_rows_kernel<DT, J>), row_grid(M), dim3(256), 0, st, x, q, s, M, D);
}

extern "C" int qv_quant_per_token(const void* x, int dtype, int8_t* q, void* scale, int64_t M, int64_t D,
                                  void* stream) {
  QV_ROW_CHECK(D, M);
  if (M == 0) return QV_OK;
  QV_CHECK_ARG(x && q && scale, "null pointer argument");
  QV_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)q % 8) == 0, "x must be 16-byte and q 8-byte aligned");
  int J;
  row_chunks(D, J);
  hipStream_t st = (hipStream_t)stream;
  QV_DT_SWITCH(dtype, {
    switch (J) {
      case 1: launch_quant<DT, 1>(x, q, (uint16_t*)scale, (int)M, (int)D, st); break;
      case 2: launch_quant<DT, 2>(x, q, (uint16_t*)scale, (int)M, (int)D, st); break;
      case 4: launch_quant<DT, 4>(x, q, (uint16_t*)scale, (int)M, (int)D, st); break;
      case 8: launch_quant<DT, 8>(x, q, (uint16_t*)scale, (int)M, (int)D, st); break;
      default: launch_quant<DT, 16>(x, q, (uint16_t*)scale, (int)M, (int)D, st); break;
    }
  });
  return check_launch("quant_per_token");
}

template <int DT, int J>
static void launch_lnq(const void* x, const void* g, const void* b, int8_t* q, uint16_t* s, float eps, bool per_token,
                       int M, int D, hipStream_t st) {
  if (per_token)
    hipLaunchKernelGGL((ln_quant_kernel<DT, J, true>), row_grid(M), dim3(256), 0, st, x, g, b, q, s, eps, M, D);
  else
    hipLaunchKernelGGL((ln_quant_kernel<DT, J, false>), row_grid(M), dim3(256), 0, st, x, g, b, q, s, eps, M, D);
}

extern "C" int qv_layernorm_quant(const void* x, int dtype, const void* gamma, const void* beta, int8_t* q,
                                  void* scale, float eps, int per_token, int64_t M, int64_t D, void* stream) {
  QV_ROW_CHECK(D, M);
  if (M == 0) return QV_OK;
  QV_CHECK_ARG(x && gamma && q && scale && (beta || !per_token), "null pointer argument");
  QV_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)gamma % 16) == 0 && ((uintptr_t)q % 8) == 0 &&
                   (!beta || ((uintptr_t)beta % 16) == 0),
               "x, gamma, beta must be 16-byte and q 8-byte aligned");
  int J;
  row_chunks(D, J);
  hipStream_t st = (hipStream_t)stream;
  QV_DT_SWITCH(dtype, {
    switch (J) {
      case 1: launch_lnq<DT, 1>(x, gamma, beta, q, (uint16_t*)scale, eps, per_token, (int)M, (int)D, st); break;
      case 2: launch_lnq<DT, 2>(x, gamma, beta, q, (uint16_t*)scale, eps, per_token, (int)M, (int)D, st); break;
      case 4: launch_lnq<DT, 4>(x, gamma, beta, q, (uint16_t*)scale, eps, per_token, (int)M, (int)D, st); break;
      case 8: launch_lnq<DT, 8>(x, gamma, beta, q, (uint16_t*)scale, eps, per_token, (int)M, (int)D, st); break;
      default: launch_lnq<DT, 16>(x, gamma, beta, q, (uint16_t*)scale, eps, per_token, (int)M, (int)D, st); break;
    }
  });
  return check_launch("layernorm_quant");
}

extern "C" int qv_gelu_quant(const void* x, int8_t* q, void* scale, void* tmp, int64_t M, int64_t D, void* stream) {
  QV_ROW_CHECK(D, M);
  if (M == 0) return QV_OK;
  QV_CHECK_ARG(x && q && scale && tmp, "null pointer argument");
  QV_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)tmp % 16) == 0 && ((uintptr_t)q % 8) == 0,
               "x, tmp must be 16-byte and q 8-byte aligned");
  int J;
  row_chunks(D, J);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = row_grid(M), block(256);
  switch (J) {
    case 1: hipLaunchKernelGGL((gelu_quant_kernel<1>), grid, block, 0, st, (const uint16_t*)x, q, (uint16_t*)scale, (uint16_t*)tmp, (int)M, (int)D); break;
    case 2: hipLaunchKernelGGL((gelu_quant_kernel<2>), grid, block, 0, st, (const uint16_t*)x, q, (uint16_t*)scale, (uint16_t*)tmp, (int)M, (int)D); break;
    case 4: hipLaunchKernelGGL((gelu_quant_kernel<4>), grid, block, 0, st, (const uint16_t*)x, q, (uint16_t*)scale, (uint16_t*)tmp, (int)M, (int)D); break;
    case 8: hipLaunchKernelGGL((gelu_quant_kernel<8>), grid, block, 0, st, (const uint16_t*)x, q, (uint16_t*)scale, (uint16_t*)tmp, (int)M, (int)D); break;
    default: hipLaunchKernelGGL((gelu_quant_kernel<16>), grid, block, 0, st, (const uint16_t*)x, q, (uint16_t*)scale, (uint16_t*)tmp, (int)M, (int)D); break;
  }
  return check_launch("gelu_quant");
}

template <int DT, int J>
static void launch_rms(const void* x, const void* g, void* out, float eps, int M, int D, hipStream_t st) {
  hipLaunchKernelGGL((rmsnorm_kernel<DT, J>), row_grid(M), dim3(256), 0, st, x, g, out, eps, M, D);
}

extern "C" int qv_rmsnorm(const void* x, const void* gamma, void* out, float eps, int64_t M, int64_t D, int dtype,
                          void* stream) {
  QV_ROW_CHECK(D, M);
  if (M == 0) return QV_OK;
  QV_CHECK_ARG(x && gamma && out, "null pointer argument");
  QV_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)gamma % 16) == 0 && ((uintptr_t)out % 16) == 0,
               "buffers must be 16-byte aligned");
  int J;
  row_chunks(D, J);
  hipStream_t st = (hipStream_t)stream;
  QV_DT_SWITCH(dtype, {
    switch (J) {
      case 1: launch_rms<DT, 1>(x, gamma, out, eps, (int)M, (int)D, st); break;
      case 2: launch_rms<DT, 2>(x, gamma, out, eps, (int)M, (int)D, st); break;
      case 4: launch_rms<DT, 4>(x, gamma, out, eps, (int)M, (int)D, st); break;
      case 8: launch_rms<DT, 8>(x, gamma, out, eps, (int)M, (int)D, st); break;
      default: launch_rms<DT, 16>(x, gamma, out, eps, (int)M, (int)D, st); break;
    }
  });
  return check_launch("rmsnorm");
}

template <int DT, int J>
static void launch_ln(const void* x, const void* g, const void* b, void* out, float eps, int M, int D, hipStream_t st) {
  hipLaunchKernelGGL((layernorm_kernel<DT, J>), row_grid(M), dim3(256), 0, st, x, g, b, out, eps, M, D);
}

extern "C" int qv_layernorm(const void* x, const void* gamma, const void* beta, void* out, float eps, int64_t M,
                            int64_t D, int dtype, void* stream) {
  QV_ROW_CHECK(D, M);
  if (M == 0) return QV_OK;
  QV_CHECK_ARG(x && gamma && beta && out, "null pointer argument");
  QV_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)gamma % 16) == 0 && ((uintptr_t)beta % 16) == 0 &&
                   ((uintptr_t)out % 16) == 0,
               "buffers must be 16-byte aligned");
  int J;
  row_chunks(D, J);
  hipStream_t st = (hipStream_t)stream;
  QV_DT_SWITCH(dtype, {
    switch (J) {
      case 1: launch_ln<DT, 1>(x, gamma, beta, out, eps, (int)M, (int)D, st); break;
      case 2: launch_ln<DT, 2>(x, gamma, beta, out, eps, (int)M, (int)D, st); break;
      case 4: launch_ln<DT, 4>(x, gamma, beta, out, eps, (int)M, (int)D, st); break;
      case 8: launch_ln<DT, 8>(x, gamma, beta, out, eps, (int)M, (int)D, st); break;
      default: launch_ln<DT, 16>(x, gamma, beta, out, eps, (int)M, (int)D, st); break;
    }
  });
  return check_launch("layernorm");
}
