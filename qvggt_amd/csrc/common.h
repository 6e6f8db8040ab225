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

// fp32 -> 16-bit float, round to nearest even.
template <bool BF16>
__device__ __forceinline__ uint16_t from_f32(float v) {
  if constexpr (BF16) {
    return __builtin_bit_cast(uint16_t, (__bf16)v);
  } else {
    return __builtin_bit_cast(uint16_t, (_Float16)v);
  }
}

template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return (uint32_t)from_f32<BF16>(a) | ((uint32_t)from_f32<BF16>(b) << 16);
}

// Exact-erf GELU, fp32 (torch.nn.GELU() semantics).
__device__ __forceinline__ float gelu_erf(float v) {
  return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
}

// Raw buffer descriptor (gfx9 dword3 = 32-bit data format) over `bytes`
// bytes from `base`; loads at offsets >= bytes return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint64_t bytes) {
  const int n = bytes >= 0xFFFFFFFFull ? (int)0xFFFFFFFFu : (int)(uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
  return __builtin_bit_cast(uint4, v);
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
