// Shared device/host helpers for the gfx950 kernels of libqvggt_hip.so.
//
// Every kernel here is written for CDNA4 (gfx950): 64-wide wavefronts,
// MFMA matrix cores, 160 KB of LDS per CU.  Host entry points are the
// extern "C" functions declared in include/qvggt_hip.h; they validate their
// arguments, launch on the caller's HIP stream and return a status code
// (0 = ok, negative = error, message via qv_last_error()).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <stdio.h>
#include <stdarg.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/qvggt_hip.h"

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

namespace qv {

// ------------------------------------------------------------ error state
void set_error(const char* fmt, ...);

#define QV_CHECK_ARG(cond, ...)                  \
  do {                                           \
    if (!(cond)) {                               \
      ::qv::set_error(__VA_ARGS__);              \
      return QV_EINVAL;                          \
    }                                            \
  } while (0)

// Report the launch status of the last kernel.
int check_launch(const char* what);

// ------------------------------------------------------- scalar conversions
__device__ __forceinline__ float to_f32(uint16_t bits, bool bf16) {
  if (bf16) return __builtin_bit_cast(float, (uint32_t)bits << 16);
  return (float)__builtin_bit_cast(_Float16, bits);
}

template <bool BF16>
__device__ __forceinline__ float ld_f32(const uint16_t* p) {
  return to_f32(*p, BF16);
}

// fp32 -> 16-bit float, round to nearest even.  The empty asm pins v as an
// fp32 value: otherwise the backend may fold the multiply that produced it
// and this conversion into one v_fma_mixlo_f16 (one rounding instead of the
// fp32-then-fp16 roundings the kernels promise).
template <bool BF16>
__device__ __forceinline__ uint16_t from_f32(float v) {
  asm volatile("" : "+v"(v));
  if constexpr (BF16) {
    return __builtin_bit_cast(uint16_t, (__bf16)v);
  } else {
    return __builtin_bit_cast(uint16_t, (_Float16)v);
  }
}

template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (BF16) {
    return (uint32_t)from_f32<true>(a) | ((uint32_t)from_f32<true>(b) << 16);
  } else {
    // gfx950's v_cvt_pk_f16_f32 rounds both halves to nearest even like two
    // v_cvt_f16_f32, in one instruction (inline asm: no fusion with the
    // producer either)
    uint32_t r;
    asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
  }
}

// v_fma_mix_f32 with 16-bit float operands taken from half K (0 = low, 1 =
// high) of a 32-bit register: the fp16 -> fp32 conversion is exact and free,
// and each result is the exact value rounded once to fp32, so these equal
// the conversion followed by the plain fp32 operation bit for bit.
template <int K>
__device__ __forceinline__ float mix_add(uint32_t h2, float c) {  // float(h) + c
  float d;
  if constexpr (K == 0) asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(d) : "v"(h2), "v"(c));
  else asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(h2), "v"(c));
  return d;
}
template <int K>
__device__ __forceinline__ float mix_sq_add(uint32_t h2, float c) {  // float(h)^2 + c (the square is exact)
  float d;
  if constexpr (K == 0) asm("v_fma_mix_f32 %0, %1, %1, %2 op_sel_hi:[1,1,0]" : "=v"(d) : "v"(h2), "v"(c));
  else asm("v_fma_mix_f32 %0, %1, %1, %2 op_sel:[1,1,0] op_sel_hi:[1,1,0]" : "=v"(d) : "v"(h2), "v"(c));
  return d;
}
template <int K>
__device__ __forceinline__ float mix_mul(float a, uint32_t h2) {  // a * float(h), as a * h + (-0)
  float d;
  if constexpr (K == 0) asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(d) : "v"(a), "v"(h2), "v"(-0.0f));
  else asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(d) : "v"(a), "v"(h2), "v"(-0.0f));
  return d;
}

// GELU with the exact-erf definition of torch.nn.GELU(), 0.5 v (1 + erf(v / sqrt 2))
// = v * Phi(v), rewritten with the normal tail Q(a) = Phi(-a), a = |v|:
//   GELU(v) = max(v, 0) - a * Q(a),
// Q(a) = 2^P(a), P a degree-5 near-minimax (Lawson-weighted Chebyshev
// least-squares) fit of log2 Q on [0, 6], |P - log2 Q| <= 5.4e-4 there, i.e.
// a relative error of Q below 3.7e-4 (0.75 of an fp16 ulp).  P has no turning
// point on [0, inf) and falls faster than log2 Q beyond 6, so a * 2^P(a) tends
// to 0 with no clamp of a.  Checked on the CPU for every finite fp16 input, in
// fp32 with fused Horner steps and exp2 off by up to 2 fp32 ulps: the
// fp16-rounded output is within one ulp of the correctly rounded GELU
// (including v < -90, where the product must round to -0).  One exp2, no
// divide, 9 VALU slots per element with the bias add.
__device__ __forceinline__ float gelu_erf(float v) {
  const float a = __builtin_fabsf(v);
  float p = -2.016825019e-04f;
  p = __builtin_fmaf(p, a, 4.467580467e-03f);
  p = __builtin_fmaf(p, a, -4.283261672e-02f);
  p = __builtin_fmaf(p, a, -4.727858603e-01f);
  p = __builtin_fmaf(p, a, -1.144399643e+00f);
  p = __builtin_fmaf(p, a, -1.000531793e+00f);
  return __builtin_fmaf(-a, __builtin_amdgcn_exp2f(p), __builtin_fmaxf(v, 0.0f));
}

// {v[l], v[l ^ 32]} in some order in a and b (v_permlane32_swap with both
// operands holding v): a + b or max(a, b) is the 32-apart butterfly step.
// Inline asm with the VALU -> permlane hazard covered by s_nop.
__device__ __forceinline__ void pair32(float v, float& a, float& b) {
  a = v;
  b = v;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

// LayerScale residual update of 8 consecutive channels (the W4A16 and W8A8
// GEMMs' residual epilogues): r + o * g per element in fp32, o the already
// rounded 16-bit linear output, one rounding of the result (the order of
// torch's x.addcmul_(o, gamma) on 16-bit tensors; o * g is exact in fp32 for
// 16-bit o and g, so a fused multiply-add gives the same value).
template <bool BF16>
__device__ __forceinline__ uint4 resid_update8(const uint4& r, const uint4& o, const uint4& g) {
  const uint32_t rw[4] = {r.x, r.y, r.z, r.w}, ow[4] = {o.x, o.y, o.z, o.w}, gw[4] = {g.x, g.y, g.z, g.w};
  uint32_t res[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = to_f32((uint16_t)(rw[i] & 0xFFFF), BF16) +
                     to_f32((uint16_t)(ow[i] & 0xFFFF), BF16) * to_f32((uint16_t)(gw[i] & 0xFFFF), BF16);
    const float hi = to_f32((uint16_t)(rw[i] >> 16), BF16) +
                     to_f32((uint16_t)(ow[i] >> 16), BF16) * to_f32((uint16_t)(gw[i] >> 16), BF16);
    res[i] = pack2<BF16>(lo, hi);
  }
  return make_uint4(res[0], res[1], res[2], res[3]);
}

// Byte offset of (row, byte) in a GEMM epilogue staging area of 128-byte rows
// (a wave's 64-channel fp16 output tile): 16-byte chunk c of row r sits at
// c ^ ((r >> 1) & 7).  The staging writes (8 bytes, one row per lane, the same
// column) and the row read-back (16 bytes, eight lanes per row) then each put
// the lanes of a 16-lane group on distinct banks; with unswizzled rows padded to
// 144 bytes the SQ_LDS_BANK_CONFLICT counter read ~0.5 conflict cycles per LDS
// instruction of the W4A16 GEMM.
__device__ __forceinline__ uint32_t stg_off(int row, int byte) {
  return (uint32_t)(row * 128 + ((((byte >> 4) ^ (row >> 1)) & 7) << 4) + (byte & 15));
}

// Raw buffer descriptor (gfx9 dword3 = 32-bit data format) over `bytes`
// bytes from `base`; loads at offsets >= bytes return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint64_t bytes) {
  const int n = bytes >= 0xFFFFFFFFull ? (int)0xFFFFFFFFu : (int)(uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

// Streaming 16- and 8-byte global accesses (nt-flagged loads / stores) for
// data a kernel touches exactly once -- the row kernels' inputs and outputs:
// measured 8-9 % more HBM throughput for LayerNorm and per-token quant on
// buffers larger than the caches.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ld_stream16(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void st_stream16(void* p, const uint4& u) {
  const u32x4_t v = {u.x, u.y, u.z, u.w};
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(p));
}
__device__ __forceinline__ void st_stream8(void* p, const uint2& u) {
  const u32x2_t v = {u.x, u.y};
  __builtin_nontemporal_store(v, reinterpret_cast<u32x2_t*>(p));
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
  return __builtin_bit_cast(uint4, v);
}

// ---- asynchronous global -> LDS copies ("LDS DMA") under explicit control.
// Issued through inline asm so the compiler neither waits for them before
// unrelated LDS reads nor before barriers: the kernel orders them itself with
// s_waitcnt vmcnt(n) + lds_barrier().  Each lane's 16 (or 4) bytes land at
// lds_base + 16*lane (4*lane); M0 carries the wave-uniform LDS base.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                          uint32_t lds_base) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(r), "s"(soff), "{m0}"(__builtin_amdgcn_readfirstlane(lds_base))
               : "memory");
}
__device__ __forceinline__ void lds_dma4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                         uint32_t lds_base) {
  asm volatile("buffer_load_dword %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(r), "s"(soff), "{m0}"(__builtin_amdgcn_readfirstlane(lds_base))
               : "memory");
}
// Workgroup barrier that only drains this wave's LDS operations (not its
// outstanding global loads, which the caller waits for with s_waitcnt).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Map the hardware workgroup id to a logical tile id so that the workgroups
// one XCD receives (the dispatcher deals ids round-robin over the 8 XCDs)
// form one contiguous range of logical tiles; neighbouring tiles then share
// that XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int nwg) {
  constexpr int NXCD = 8;
  const int q = nwg / NXCD, r = nwg % NXCD;
  const int xcd = bid % NXCD;
  const int start = xcd * q + (xcd < r ? xcd : r);
  return start + bid / NXCD;
}

}  // namespace qv
