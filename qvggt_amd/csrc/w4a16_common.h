// Shared pieces of the W4A16 kernels: AWQ-v2 nibble decoding, the exact
// dequantisation, MFMA wrappers and the fused epilogue.
//
// Packed layout (awq/qmodule.py:43-99, interleave 4, kstride 64): weight
// (n, k) lives in qweight row n/4.  The 16 bytes at int16 columns
// 64*kb + 16*(n%4) + 8*c .. +7 hold the 32 nibbles of row n for
// k in [64*kb + 32*c, +32) as four little-endian u32 words f = 0..3; nibble
// i = 4*e + h of word f is k = 64*kb + 32*c + 8*h + 2*f + e.  So one 16-byte
// load gives one row's full 32-k chunk, and "pair h" of each word -- nibbles
// (h, h+4) -- is the two consecutive k = 8*h + 2*f + {0,1}.
#pragma once

#include "common.h"

namespace qv {

// Pair t of word w -> two fp16 weights fp16_rn(q*s + sz), one fused rounding.
// (w & 0x000f000f) | 0x64006400 is the fp16 pair (1024+q_lo, 1024+q_hi); the
// 0x00f000f0 mask gives (1024+16q); both are made exact integers q first.
template <int t>
__device__ __forceinline__ uint32_t dq_pair_f16(uint32_t w, uint32_t w_hi, f16x2 s2, f16x2 z2) {
  const uint32_t src = (t < 2) ? w : w_hi;
  const uint32_t mask = (t & 1) ? 0x00f000f0u : 0x000f000fu;
  // One v_and_or_b32 (mask from an SGPR, magic from a VGPR: gfx9 VOP3 takes
  // no literal and one constant-bus operand).
  uint32_t bits;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(bits) : "v"(src), "s"(mask), "v"(0x64006400u));
  const f16x2 h = __builtin_bit_cast(f16x2, bits);
  f16x2 q;
  if constexpr ((t & 1) == 0) {
    q = h - (f16x2){(_Float16)1024.0f, (_Float16)1024.0f};
  } else {
    q = __builtin_elementwise_fma(h, (f16x2){(_Float16)0.0625f, (_Float16)0.0625f},
                                  (f16x2){(_Float16)-64.0f, (_Float16)-64.0f});
  }
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q, s2, z2));
}

// bf16: q*s + sz is exact in fp32 for tables built as sz = -bf16(s*z) (at most
// 13 significant bits), so fp32 FMA then one RNE rounding to bf16 equals the
// fused bf16 operation of the reference.
template <int t>
__device__ __forceinline__ uint32_t dq_pair_bf16(uint32_t w, float s, float z) {
  const float q0 = (float)((w >> (4 * t)) & 0xFu);
  const float q1 = (float)((w >> (4 * t + 16)) & 0xFu);
  const bf16x2 r = {(__bf16)__builtin_fmaf(q0, s, z), (__bf16)__builtin_fmaf(q1, s, z)};
  return __builtin_bit_cast(uint32_t, r);
}

// Weight fragment for k-step t: 8 slots = pair t of words 0..3.
template <bool BF16, int t>
__device__ __forceinline__ uint4 dq_frag(const uint4& wq, uint32_t s_bits, uint32_t z_bits) {
  uint4 r;
  if constexpr (!BF16) {
    const f16x2 s2 = __builtin_bit_cast(f16x2, s_bits * 0x10001u);
    const f16x2 z2 = __builtin_bit_cast(f16x2, z_bits * 0x10001u);
    r.x = dq_pair_f16<t>(wq.x, wq.x >> 8, s2, z2);
    r.y = dq_pair_f16<t>(wq.y, wq.y >> 8, s2, z2);
    r.z = dq_pair_f16<t>(wq.z, wq.z >> 8, s2, z2);
    r.w = dq_pair_f16<t>(wq.w, wq.w >> 8, s2, z2);
  } else {
    const float s = __builtin_bit_cast(float, s_bits << 16);
    const float z = __builtin_bit_cast(float, z_bits << 16);
    r.x = dq_pair_bf16<t>(wq.x, s, z);
    r.y = dq_pair_bf16<t>(wq.y, s, z);
    r.z = dq_pair_bf16<t>(wq.z, s, z);
    r.w = dq_pair_bf16<t>(wq.w, s, z);
  }
  return r;
}

// dq_frag with the scale and scaled zero as 32-bit words holding two
// channels' 16-bit values; sel (a v_perm_b32 byte selector, 0x01000100 or
// 0x03020302) picks this lane's half and splats it.
template <bool BF16, int t>
__device__ __forceinline__ uint4 dq_frag_w(const uint4& wq, uint32_t s_word, uint32_t z_word, uint32_t sel) {
  const uint32_t s_sp = __builtin_amdgcn_perm(s_word, s_word, sel), z_sp = __builtin_amdgcn_perm(z_word, z_word, sel);
  uint4 r;
  if constexpr (!BF16) {
    const f16x2 s2 = __builtin_bit_cast(f16x2, s_sp);
    const f16x2 z2 = __builtin_bit_cast(f16x2, z_sp);
    r.x = dq_pair_f16<t>(wq.x, wq.x >> 8, s2, z2);
    r.y = dq_pair_f16<t>(wq.y, wq.y >> 8, s2, z2);
    r.z = dq_pair_f16<t>(wq.z, wq.z >> 8, s2, z2);
    r.w = dq_pair_f16<t>(wq.w, wq.w >> 8, s2, z2);
  } else {
    const float s = __builtin_bit_cast(float, s_sp << 16);
    const float z = __builtin_bit_cast(float, z_sp << 16);
    r.x = dq_pair_bf16<t>(wq.x, s, z);
    r.y = dq_pair_bf16<t>(wq.y, s, z);
    r.z = dq_pair_bf16<t>(wq.z, s, z);
    r.w = dq_pair_bf16<t>(wq.w, s, z);
  }
  return r;
}

template <bool BF16>
__device__ __forceinline__ f32x4 mfma16(const uint4& a, const uint4& b, f32x4 c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

template <bool BF16>
__device__ __forceinline__ f32x16 mfma32(const uint4& a, const uint4& b, f32x16 c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// Offset (in u32 units) of the 16-byte chunk (row n, 32-k chunk g of the
// 128-k group kt) inside qweight.
__device__ __forceinline__ size_t qw_chunk_u32(int n, int kt, int g, int K) {
  return (size_t)(n >> 2) * (size_t)(K >> 1) + (size_t)kt * 64 + (g >> 1) * 32 + (n & 3) * 8 +
         (g & 1) * 4;
}

// Internal epilogue id (not part of the qv_w4a16_gemm contract): bias, then
// the LayerScale residual update out = out + gamma * fp16(acc + bias), in
// place on the residual stream (qv_w4a16_gemm_residual).
constexpr int QV_EPI_BIAS_RESID = 4;
// Internal epilogue id of qv_w4a16_gemm_qkrope (fp16 only): the VGGT qkv
// projection with its per-head q/k LayerNorm and 2-D RoPE (see QkRopeArgs).
constexpr int QV_EPI_QKROPE = 5;

// Operands of the QV_EPI_QKROPE epilogue.  Output columns [0, qk_cols) are the
// q heads then the k heads (64 columns each), the rest pass through with the
// bias; positions are int32 (y, x) per output row, cos/sin fp32 (P, 16).
struct QkRopeArgs {
  const int* pos = nullptr;
  const float* cos_t = nullptr;
  const float* sin_t = nullptr;
  const uint16_t* qg = nullptr;
  const uint16_t* qb = nullptr;
  const uint16_t* kg = nullptr;
  const uint16_t* kb = nullptr;
  int P = 1;
  int qk_cols = 0;
  float eps = 0.f;
};

// whether an epilogue adds a bias
template <int EPI>
constexpr bool epi_has_bias() {
  return EPI == QV_EPI_BIAS || EPI == QV_EPI_BIAS_GELU || EPI == QV_EPI_BIAS_RESID || EPI == QV_EPI_QKROPE;
}

// Bias / GELU on four consecutive channels (fp32, before the single rounding
// to the 16-bit output type); b holds their four bias values, already loaded
// (ignored without bias).
template <bool BF16, int EPI>
__device__ __forceinline__ void epilogue_apply4v(const uint2& b, float (&r)[4]) {
  if constexpr (epi_has_bias<EPI>()) {
    r[0] += to_f32((uint16_t)(b.x & 0xFFFF), BF16);
    r[1] += to_f32((uint16_t)(b.x >> 16), BF16);
    r[2] += to_f32((uint16_t)(b.y & 0xFFFF), BF16);
    r[3] += to_f32((uint16_t)(b.y >> 16), BF16);
  }
  if constexpr (EPI == QV_EPI_BIAS_GELU || EPI == QV_EPI_GELU) {
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = gelu_erf(r[i]);
  }
}

// Tile plan of one streamed launch: rows [0, rows_a) in (32 mt_a)-row tiles
// and rows [rows_a, M) in (32 mt_b)-row tiles; mt_b = 0: every row in
// (32 mt_a)-row tiles.  Pairs (4, 3), (4, 2), (3, 2); rows_a a multiple of
// 32 mt_a.
struct StreamPlan {
  int mt_a = 4, rows_a = 0, mt_b = 0;
  bool ksplit = false;   // one range of mt_a tiles, K split between two 4-wave groups
  int sub = 1;           // 64-k sub-stages per pipeline stage (2: one range of 64- or 96-row tiles, K % 256 == 0)
};

// Streamed (LDS-pipelined, 32x32 MFMA) GEMM, tiles (32 mt) x 256.
template <bool BF16>
int launch_w4a16_stream(const void* x, const void* qw, const void* s, const void* z, const void* bias,
                        const void* gamma, void* out, int M, int N, int K, int epi, const StreamPlan& plan,
                        hipStream_t st, const QkRopeArgs* qk = nullptr);

}  // namespace qv
