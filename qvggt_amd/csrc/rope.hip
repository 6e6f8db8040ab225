// Rotary position embeddings for gfx950.
//
// qv_rope_with_pos: fused_rope_with_pos_forward_func of the reference
// (rope_new/fused_rope_with_pos.cu:19-164): rotate-half RoPE on the first d2
// dims of x[s][b][h][:] (arbitrary element strides) with fp32 angles
// freqs[b][s][0:d2]; dims >= d2 are copied.  cos/sin are evaluated in fp64
// (one sincos: a shared argument reduction) and rounded to fp32 (the
// reference used the fast-math sincosf), once per (s, b, d) and shared by the
// heads.
//
// qv_rope2d: the VGGT 2-D RoPE on the q and k parts of a fused qkv buffer
// (tokens, 3, H, 64).  Head dims [0,32) rotate with the token's y position,
// [32,64) with its x position; inside each half, dims (d, d+16) form the
// rotate-half pair with frequency index d (0..15).  cos/sin come from fp32
// tables (positions x 16) built on the host; special tokens carry position 0
// (cos 1, sin 0: unrotated).  out = x*cos - x_pair*sin (first of the pair),
// x*cos + x_pair*sin (second), fp32 ops with one rounding each.
#include "common.h"

#pragma clang fp contract(off)

namespace qv {

template <int DT>
__device__ __forceinline__ float ld1(const void* p, size_t i) {
  if constexpr (DT == QV_F32) return reinterpret_cast<const float*>(p)[i];
  else return to_f32(reinterpret_cast<const uint16_t*>(p)[i], DT == QV_BF16);
}
template <int DT>
__device__ __forceinline__ void st1(void* p, size_t i, float v) {
  if constexpr (DT == QV_F32) reinterpret_cast<float*>(p)[i] = v;
  else reinterpret_cast<uint16_t*>(p)[i] = from_f32<DT == QV_BF16>(v);
}

// Eight elements at e of a 16- or 32-bit row, as fp32 (16-byte aligned).
template <int DT>
__device__ __forceinline__ void ld8(const void* p, long e, float (&v)[8]) {
  if constexpr (DT == QV_F32) {
    const uint4 a = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(p) + e);
    const uint4 b = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(p) + e + 4);
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __builtin_bit_cast(float, w[i]);
  } else {
    const uint4 u = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p) + e);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = to_f32((uint16_t)(w[i] & 0xFFFF), DT == QV_BF16);
      v[2 * i + 1] = to_f32((uint16_t)(w[i] >> 16), DT == QV_BF16);
    }
  }
}
// The same eight elements as raw 16-byte words (one for 16-bit types, two for
// fp32), converted later with cvt8: a load whose use comes much later.
template <int DT>
struct Raw8 {
  uint4 w[DT == QV_F32 ? 2 : 1];
};
template <int DT>
__device__ __forceinline__ Raw8<DT> ld8_raw(const void* p, long e) {
  Raw8<DT> r;
  if constexpr (DT == QV_F32) {
    r.w[0] = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(p) + e);
    r.w[1] = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(p) + e + 4);
  } else {
    r.w[0] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p) + e);
  }
  return r;
}
template <int DT>
__device__ __forceinline__ void cvt8(const Raw8<DT>& r, float (&v)[8]) {
  if constexpr (DT == QV_F32) {
    const uint32_t w[8] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w, r.w[1].x, r.w[1].y, r.w[1].z, r.w[1].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __builtin_bit_cast(float, w[i]);
  } else {
    const uint32_t w[4] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = to_f32((uint16_t)(w[i] & 0xFFFF), DT == QV_BF16);
      v[2 * i + 1] = to_f32((uint16_t)(w[i] >> 16), DT == QV_BF16);
    }
  }
}

template <int DT>
__device__ __forceinline__ void st8(void* p, long e, const float (&v)[8]) {
  if constexpr (DT == QV_F32) {
    float* q = reinterpret_cast<float*>(p) + e;
    *reinterpret_cast<uint4*>(q) = make_uint4(__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                                              __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3]));
    *reinterpret_cast<uint4*>(q + 4) = make_uint4(__builtin_bit_cast(uint32_t, v[4]), __builtin_bit_cast(uint32_t, v[5]),
                                                  __builtin_bit_cast(uint32_t, v[6]), __builtin_bit_cast(uint32_t, v[7]));
  } else {
    constexpr bool BF = DT == QV_BF16;
    *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(p) + e) =
        make_uint4(pack2<BF>(v[0], v[1]), pack2<BF>(v[2], v[3]), pack2<BF>(v[4], v[5]), pack2<BF>(v[6], v[7]));
  }
}

// qv_rope_with_pos.  One wave per (s, b) position at a time (grid-stride).
// The rotation angles freqs[b][s][0, d2) are the same for all H heads of a
// position, so the wave first evaluates their cos / sin once (fp64, rounded
// to fp32) into a wave-private LDS row, then rotates the heads from it.
// VEC (unit element stride of the head dims in x and out, 16-byte aligned
// rows, d2/2 and d - d2 multiples of 8): a lane moves 8 dims of the first
// half and their 8 partners of the second half with 16-byte accesses, then
// the pass-through dims in 8-element chunks; otherwise a lane takes one
// (head, pair) at a time with element accesses.  The angles and a lane's
// first 16-byte pair are loaded before the table is evaluated, so their
// latency runs under the fp64 cos / sin (with VGGT's 16 heads of 64, d2 = 64,
// that first pair is all a lane moves).  d2 above RWP_MAX_D2 skips the table
// and evaluates cos / sin per element.
constexpr int RWP_WAVES = 4;
constexpr int RWP_MAX_D2 = 512;

template <int DT, bool VEC, bool TAB>
__global__ __launch_bounds__(64 * RWP_WAVES) void rope_with_pos_kernel(
    const void* __restrict__ x, const float* __restrict__ freqs, void* __restrict__ out, int S, int B, int H,
    int D, int D2, long sx_s, long sx_b, long sx_h, long sx_d, long so_s, long so_b, long so_h, long so_d) {
  __shared__ float cs_l[TAB ? RWP_WAVES : 1][TAB ? RWP_MAX_D2 : 1], sn_l[TAB ? RWP_WAVES : 1][TAB ? RWP_MAX_D2 : 1];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int half = D2 / 2;
  const int nch = half >> 3;           // VEC: 8-dim chunks per half
  const int items = H * nch;           // VEC: (head, chunk) items of a position
  float* cs = cs_l[TAB ? wave : 0];
  float* sn = sn_l[TAB ? wave : 0];
  const long npos = (long)S * B;
  for (long pidx = (long)blockIdx.x * RWP_WAVES + wave; pidx < npos; pidx += (long)gridDim.x * RWP_WAVES) {
    const int ss = (int)(pidx / B), bb = (int)(pidx % B);
    const float* f = freqs + ((long)bb * S + ss) * D2;
    auto cosv = [&](int d) {
      if constexpr (TAB) return cs[d];
      else return (float)cos((double)f[d]);
    };
    auto sinv = [&](int d) {
      if constexpr (TAB) return sn[d];
      else return (float)sin((double)f[d]);
    };
    const long xb = ss * sx_s + bb * sx_b, ob = ss * so_s + bb * so_b;
    // angle of the lane's first table entry, then (VEC) the lane's first item,
    // loaded unconditionally (clamped indices, in bounds) and kept raw, so no
    // branch or conversion makes the wave wait for them before the table
    const float th0 = TAB ? f[lane < D2 ? lane : D2 - 1] : 0.0f;
    Raw8<DT> a0r, p0r;
    if constexpr (VEC) {
      const int t0 = lane < items ? lane : items - 1;
      const int hh = t0 / nch, c = 8 * (t0 - hh * nch);
      a0r = ld8_raw<DT>(x, xb + hh * sx_h + c);
      p0r = ld8_raw<DT>(x, xb + hh * sx_h + half + c);
    }
    if constexpr (TAB) {
      // every lane evaluates its first entry (clamped), so the angle load is
      // not sunk behind the x loads into a branch
      double sd0, cd0;
      sincos((double)th0, &sd0, &cd0);
      const float c0 = (float)cd0, s0 = (float)sd0;
      if (lane < D2) {
        cs[lane] = c0;
        sn[lane] = s0;
      }
      for (int d = lane + 64; d < D2; d += 64) {
        double sd, cd;
        sincos((double)f[d], &sd, &cd);
        cs[d] = (float)cd;
        sn[d] = (float)sd;
      }
      // the wave's LDS accesses run in order: make the compiler keep them so
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
    if constexpr (VEC) {
      auto rotate = [&](int t, const float (&a)[8], const float (&pp)[8]) {
        const int hh = t / nch, c = 8 * (t - hh * nch);
        float o1[8], o2[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          o1[e] = a[e] * cosv(c + e) + (-pp[e]) * sinv(c + e);
          o2[e] = pp[e] * cosv(half + c + e) + a[e] * sinv(half + c + e);
        }
        st8<DT>(out, ob + hh * so_h + c, o1);
        st8<DT>(out, ob + hh * so_h + half + c, o2);
      };
      if (lane < items) {
        float a0[8], p0[8];
        cvt8<DT>(a0r, a0);
        cvt8<DT>(p0r, p0);
        rotate(lane, a0, p0);
      }
      for (int t = lane + 64; t < items; t += 64) {
        const int hh = t / nch, c = 8 * (t - hh * nch);
        float a[8], pp[8];
        ld8<DT>(x, xb + hh * sx_h + c, a);
        ld8<DT>(x, xb + hh * sx_h + half + c, pp);
        rotate(t, a, pp);
      }
      const int npass = (D - D2) >> 3;
      for (int t = lane; t < H * npass; t += 64) {
        const int hh = t / npass, c = D2 + 8 * (t - hh * npass);
        float v[8];
        ld8<DT>(x, xb + hh * sx_h + c, v);
        st8<DT>(out, ob + hh * so_h + c, v);
      }
    } else {
      for (int t = lane; t < H * half; t += 64) {
        const int hh = t / half, j = t - hh * half;
        const long xi = xb + hh * sx_h, oi = ob + hh * so_h;
        const float a = ld1<DT>(x, xi + j * sx_d);
        const float pp = ld1<DT>(x, xi + (j + half) * sx_d);
        st1<DT>(out, oi + j * so_d, a * cosv(j) + (-pp) * sinv(j));
        st1<DT>(out, oi + (j + half) * so_d, pp * cosv(j + half) + a * sinv(j + half));
      }
      const int npass = D - D2;
      for (int t = lane; t < H * npass; t += 64) {
        const int hh = t / npass, d = D2 + (t - hh * npass);
        st1<DT>(out, ob + hh * so_h + d * so_d, ld1<DT>(x, xb + hh * sx_h + d * sx_d));
      }
    }
    if constexpr (TAB) {
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");   // reads done before the next position's writes
      __builtin_amdgcn_wave_barrier();
    }
  }
}

// Lane exchange inside 8-lane row groups (DPP, no LDS).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float sum8_lanes(float v) {
  v = v + dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]: j ^ 1
  v = v + dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]: j ^ 2
  v = v + dpp_f<0x141>(v);  // row_half_mirror: j ^ 4 once quads are uniform
  return v;
}

// VGGT 2-D RoPE.  Eight lanes per (token, part in {q,k}, head) row of 64
// dims: lane j holds dims 8j..8j+7 (one 16-byte load and store), so a wave
// moves 8 whole 128-byte rows per instruction.  Each 8-lane group handles NR
// rows, 32 apart.  Lanes 0-3 hold the y half (dims 0..31), 4-7 the x half;
// within a half, lanes with (j & 2) == 0 hold dims i < 16 and rotate against
// lane j ^ 2 (DPP quad_perm).  Dead lanes shadow row 0 and store nothing.
// The loads run in three phases, fenced from the compiler's scheduler (which
// otherwise sinks each load next to its use and so serialises their
// latencies): every row's token position, then every row's data, then --
// once the positions are in, with the data still in flight -- every row's
// cos / sin table entries.
__device__ __forceinline__ void row_coords(long r, int H, int hshift, int& tok, int& part, int& head) {
  if (hshift >= 0) {                        // H = 2^hshift: shifts instead of 64-bit divisions
    tok = (int)(r >> (hshift + 1));
    part = (int)(r >> hshift) & 1;
    head = (int)r & ((1 << hshift) - 1);
  } else {
    tok = (int)(r / (2 * H));
    const int rr = (int)(r % (2 * H));
    part = rr / H;
    head = rr % H;
  }
}

// cos / sin of the 8 frequencies i0 .. i0 + 7 of table row p (clamped to the table)
struct Angles8 {
  float4 c0, c1, s0, s1;
};
__device__ __forceinline__ Angles8 load_angles(const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                               int p, int P, int i0) {
  p = p < 0 ? 0 : (p >= P ? P - 1 : p);
  const float4* cp = reinterpret_cast<const float4*>(cos_t + p * 16 + i0);
  const float4* sp = reinterpret_cast<const float4*>(sin_t + p * 16 + i0);
  return Angles8{cp[0], cp[1], sp[0], sp[1]};
}

// the rotation of one lane's 8 packed fp16 values y against lane j ^ 2's
__device__ __forceinline__ uint4 rotate8(const uint32_t (&yw)[4], const Angles8& a, bool lo) {
  const float cs[8] = {a.c0.x, a.c0.y, a.c0.z, a.c0.w, a.c1.x, a.c1.y, a.c1.z, a.c1.w};
  // the first of a rotation pair subtracts the partner term: x*c - o*s = x*c + o*(-s)
  const float sg = lo ? -1.0f : 1.0f;
  const float sn[8] = {sg * a.s0.x, sg * a.s0.y, sg * a.s0.z, sg * a.s0.w,
                       sg * a.s1.x, sg * a.s1.y, sg * a.s1.z, sg * a.s1.w};
  uint32_t ow[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t other = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)yw[m], 0x4E, 0xF, 0xF, true);  // lane j ^ 2
    ow[m] = pack2<false>(mix_mul<0>(cs[2 * m], yw[m]) + mix_mul<0>(sn[2 * m], other),
                         mix_mul<1>(cs[2 * m + 1], yw[m]) + mix_mul<1>(sn[2 * m + 1], other));
  }
  return make_uint4(ow[0], ow[1], ow[2], ow[3]);
}

template <int NR>
__global__ __launch_bounds__(256) void rope2d_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                          const int* __restrict__ pos, const float* __restrict__ cos_t,
                                                          const float* __restrict__ sin_t, int P, int T, int H,
                                                          long src_tok, long dst_tok, long dst_part, int hshift) {
  const long nrows = (long)T * 2 * H;
  const long g0 = (long)blockIdx.x * (32 * NR) + (threadIdx.x >> 3);
  const int j = threadIdx.x & 7;
  const int half = j >> 2;
  const int i0 = 8 * (j & 1);
  const bool lo = (j & 2) == 0;
  uint32_t xw[NR][4];   // the row's 8 fp16 values, packed (read through v_fma_mix_f32)
  bool live[NR];
  int pv[NR];
  long soff[NR], doff[NR];
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    const long r = g0 + 32 * k;
    live[k] = r < nrows;
    int tok, part, head;
    row_coords(live[k] ? r : 0, H, hshift, tok, part, head);
    soff[k] = (long)tok * src_tok + (long)part * H * 64 + (long)head * 64 + 8 * j;
    doff[k] = (long)tok * dst_tok + (long)part * dst_part + (long)head * 64 + 8 * j;
    pv[k] = pos[2 * tok + half];
  }
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    const uint4 v = ld_stream16(src + soff[k]);
    xw[k][0] = v.x; xw[k][1] = v.y; xw[k][2] = v.z; xw[k][3] = v.w;
  }
  __builtin_amdgcn_sched_barrier(0);
  Angles8 an[NR];
#pragma unroll
  for (int k = 0; k < NR; ++k) an[k] = load_angles(cos_t, sin_t, pv[k], P, i0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    const uint4 o = rotate8(xw[k], an[k], lo);
    if (live[k]) st_stream16(dst + doff[k], o);
  }
}

// VGGT attention prologue, fused: per-head LayerNorm of q and k (qk-norm,
// affine, over the 64 head dims), rounded to fp16, then the 2-D RoPE of rope2d_kernel,
// in place in the fused qkv buffer.  Eight lanes per (token, part, head) row:
// lane j of the row holds dims 8j..8j+7 (one 16-byte load and store), so a
// wave moves 8 whole rows per instruction; NR rows per 8-lane group, all
// loaded first.  Statistics in fp32: each lane sums
// its 8 values in order, then a butterfly over lanes j ^ 1, j ^ 2, j ^ 4
// (DPP, no LDS); two-pass variance; one rounding per fp32 operation.  The
// rotation partner of dim d (d +- 16 in its half) sits in lane j ^ 2.
constexpr int QKN_ROWS_PER_WG = 32;  // 4 waves x 8 rows per row slot; NR slots per workgroup

// q/k LayerNorm of one row's 8 values in a lane (packed fp16 xw, the row
// spread over 8 lanes): mean, two-pass variance, affine, rounded to fp16 yw.
__device__ __forceinline__ void qk_norm8(const uint32_t (&xw)[4], const uint4& g, const uint4& b, float eps,
                                         uint32_t (&yw)[4]) {
  float s = 0.f;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    s = mix_add<0>(xw[m], s);
    s = mix_add<1>(xw[m], s);
  }
  const float nm = -(sum8_lanes(s) / 64.0f);
  float d[8], s2 = 0.f;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    d[2 * m] = mix_add<0>(xw[m], nm);
    d[2 * m + 1] = mix_add<1>(xw[m], nm);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) s2 = s2 + d[e] * d[e];
  const float rs = 1.0f / __builtin_sqrtf(sum8_lanes(s2) / 64.0f + eps);
  const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
  for (int m = 0; m < 4; ++m)
    yw[m] = pack2<false>(mix_add<0>(bw[m], mix_mul<0>(d[2 * m] * rs, gw[m])),
                         mix_add<1>(bw[m], mix_mul<1>(d[2 * m + 1] * rs, gw[m])));
}
template <int NR>
__global__ __launch_bounds__(256) void qknorm_rope2d_kernel(
    uint16_t* __restrict__ qkv, const int* __restrict__ pos, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, int P, const uint16_t* __restrict__ qg, const uint16_t* __restrict__ qb,
    const uint16_t* __restrict__ kg, const uint16_t* __restrict__ kb, float eps, int T, int H, long tok_stride,
    int hshift) {
  const long nrows = (long)T * 2 * H;
  const long g0 = (long)blockIdx.x * (QKN_ROWS_PER_WG * NR) + (threadIdx.x >> 3);
  const int j = threadIdx.x & 7;
  const int half = j >> 2;
  const int i0 = 8 * (j & 1);
  const bool lo = (j & 2) == 0;
  // the row's 8 fp16 values stay packed (pairs 2m, 2m+1 in word m) and enter
  // the fp32 arithmetic through v_fma_mix_f32 (mix_add / mix_mul), which
  // converts exactly for free: the same values as converting first
  uint32_t xw[NR][4];
  bool live[NR];
  int partv[NR], pv[NR];
  uint16_t* row[NR];
  // load phases as in rope2d_kernel: positions, rows and the q / k norm
  // weights, then (positions in) the cos / sin entries
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    const long r = g0 + QKN_ROWS_PER_WG * k;
    live[k] = r < nrows;
    int tok, part, head;
    row_coords(live[k] ? r : 0, H, hshift, tok, part, head);   // dead lanes shadow row 0
    partv[k] = part;
    row[k] = qkv + (size_t)tok * tok_stride + (size_t)part * H * 64 + (size_t)head * 64;
    pv[k] = pos[2 * tok + half];
  }
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    const uint4 v = ld_stream16(row[k] + 8 * j);
    xw[k][0] = v.x; xw[k][1] = v.y; xw[k][2] = v.z; xw[k][3] = v.w;
  }
  const uint4 gq = reinterpret_cast<const uint4*>(qg)[j], bq = reinterpret_cast<const uint4*>(qb)[j];
  const uint4 gk = reinterpret_cast<const uint4*>(kg)[j], bk = reinterpret_cast<const uint4*>(kb)[j];
  __builtin_amdgcn_sched_barrier(0);
  Angles8 an[NR];
#pragma unroll
  for (int k = 0; k < NR; ++k) an[k] = load_angles(cos_t, sin_t, pv[k], P, i0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    uint32_t yw[4];
    qk_norm8(xw[k], partv[k] ? gk : gq, partv[k] ? bk : bq, eps, yw);
    const uint4 o = rotate8(yw, an[k], lo);
    if (live[k]) st_stream16(row[k] + 8 * j, o);
  }
}

// Token blocks.  When H is a multiple of 16 a token's 2H rows are whole
// 32-row blocks, so the 32 rows of one block share a token and its position
// pair.  A wave takes one block: group g (lanes 8g .. 8g + 7) takes rows
// g, g + 8, g + 16, g + 24 of it, and each lane loads its 8 cos / sin pairs
// once for all four.  With the angles held once instead of per row, four rows
// per lane are in flight at full occupancy (the per-row form holds two).
// Results are those of the per-row kernels bit for bit (the same arithmetic
// per row).
constexpr int TOK_ROWS = 4;        // rows per 8-lane group
constexpr int TOK_WAVES = 4;       // waves (32-row blocks) per workgroup

__global__ __launch_bounds__(64 * TOK_WAVES) void rope2d_tok_kernel(
    const uint16_t* __restrict__ src, uint16_t* __restrict__ dst, const int* __restrict__ pos,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, int P, int T, int H, long src_tok,
    long dst_tok, long dst_part, int hshift) {
  const long base = ((long)blockIdx.x * TOK_WAVES + (threadIdx.x >> 6)) * 32;
  if (base >= (long)T * 2 * H) return;   // whole block past the end (wave-uniform; no barriers)
  const int g = (threadIdx.x >> 3) & 7, j = threadIdx.x & 7;
  const int half = j >> 2, i0 = 8 * (j & 1);
  const bool lo = (j & 2) == 0;
  int tok, part0, head0;
  row_coords(base, H, hshift, tok, part0, head0);
  const int rr0 = part0 * H + head0 + g;   // row of the token (q heads, then k heads)
  const int pv = pos[2 * tok + half];
  const uint16_t* s0 = src + (size_t)tok * src_tok + 8 * j;
  uint32_t xw[TOK_ROWS][4];
#pragma unroll
  for (int k = 0; k < TOK_ROWS; ++k) {
    const uint4 v = ld_stream16(s0 + (size_t)(rr0 + 8 * k) * 64);
    xw[k][0] = v.x; xw[k][1] = v.y; xw[k][2] = v.z; xw[k][3] = v.w;
  }
  __builtin_amdgcn_sched_barrier(0);
  const Angles8 an = load_angles(cos_t, sin_t, pv, P, i0);
  __builtin_amdgcn_sched_barrier(0);
  uint16_t* d0 = dst + (size_t)tok * dst_tok + 8 * j;
#pragma unroll
  for (int k = 0; k < TOK_ROWS; ++k) {
    const int rr = rr0 + 8 * k;
    const int part = rr >= H;
    const int head = rr - (part ? H : 0);
    st_stream16(d0 + (size_t)part * dst_part + (size_t)head * 64, rotate8(xw[k], an, lo));
  }
}

__global__ __launch_bounds__(64 * TOK_WAVES) void qknorm_rope2d_tok_kernel(
    uint16_t* __restrict__ qkv, const int* __restrict__ pos, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, int P, const uint16_t* __restrict__ qg, const uint16_t* __restrict__ qb,
    const uint16_t* __restrict__ kg, const uint16_t* __restrict__ kb, float eps, int T, int H, long tok_stride,
    int hshift) {
  const long base = ((long)blockIdx.x * TOK_WAVES + (threadIdx.x >> 6)) * 32;
  if (base >= (long)T * 2 * H) return;   // whole block past the end (wave-uniform; no barriers)
  const int g = (threadIdx.x >> 3) & 7, j = threadIdx.x & 7;
  const int half = j >> 2, i0 = 8 * (j & 1);
  const bool lo = (j & 2) == 0;
  int tok, part0, head0;
  row_coords(base, H, hshift, tok, part0, head0);
  const int rr0 = part0 * H + head0 + g;
  const int pv = pos[2 * tok + half];
  uint16_t* r0 = qkv + (size_t)tok * tok_stride + 8 * j;
  uint32_t xw[TOK_ROWS][4];
#pragma unroll
  for (int k = 0; k < TOK_ROWS; ++k) {
    const uint4 v = ld_stream16(r0 + (size_t)(rr0 + 8 * k) * 64);
    xw[k][0] = v.x; xw[k][1] = v.y; xw[k][2] = v.z; xw[k][3] = v.w;
  }
  const uint4 gq = reinterpret_cast<const uint4*>(qg)[j], bq = reinterpret_cast<const uint4*>(qb)[j];
  const uint4 gk = reinterpret_cast<const uint4*>(kg)[j], bk = reinterpret_cast<const uint4*>(kb)[j];
  __builtin_amdgcn_sched_barrier(0);
  const Angles8 an = load_angles(cos_t, sin_t, pv, P, i0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < TOK_ROWS; ++k) {
    const int rr = rr0 + 8 * k;
    const bool kpart = rr >= H;
    uint32_t yw[4];
    qk_norm8(xw[k], kpart ? gk : gq, kpart ? bk : bq, eps, yw);
    st_stream16(r0 + (size_t)rr * 64, rotate8(yw, an, lo));
  }
}

}  // namespace qv

using namespace qv;

// the token-block kernels' grid: one wave per 32 rows, a 32-bit workgroup count
static bool tok_blocks_ok(long rows) { return rows / 32 / TOK_WAVES < INT32_MAX; }

extern "C" int qv_qknorm_rope2d(void* qkv, const int32_t* positions, const float* cos_table, const float* sin_table,
                                int64_t table_rows, const void* q_gamma, const void* q_beta, const void* k_gamma,
                                const void* k_beta, float eps, int64_t T, int64_t H, int64_t token_stride,
                                void* stream) {
  QV_CHECK_ARG(T >= 0 && H > 0 && table_rows > 0 && table_rows <= INT32_MAX, "bad shape");
  if (T == 0) return QV_OK;
  QV_CHECK_ARG(qkv && positions && cos_table && sin_table && q_gamma && q_beta && k_gamma && k_beta,
               "null pointer argument");
  QV_CHECK_ARG(token_stride % 8 == 0 && token_stride >= 2 * H * 64 && ((uintptr_t)qkv % 16) == 0,
               "qkv rows must be 16-byte aligned and hold q and k");
  QV_CHECK_ARG(((uintptr_t)cos_table % 16) == 0 && ((uintptr_t)sin_table % 16) == 0 &&
                   ((uintptr_t)q_gamma % 16) == 0 && ((uintptr_t)q_beta % 16) == 0 &&
                   ((uintptr_t)k_gamma % 16) == 0 && ((uintptr_t)k_beta % 16) == 0,
               "tables and norm weights must be 16-byte aligned");
  const long rows = T * 2 * H;
  QV_CHECK_ARG(rows / QKN_ROWS_PER_WG < INT32_MAX, "too many rows");
  const int hshift = (H & (H - 1)) == 0 ? __builtin_ctzll((unsigned long long)H) : -1;
  if (H % 16 == 0 && tok_blocks_ok(rows)) {
    hipLaunchKernelGGL(qknorm_rope2d_tok_kernel, dim3((unsigned)((rows / 32 + TOK_WAVES - 1) / TOK_WAVES)),
                       dim3(64 * TOK_WAVES), 0, (hipStream_t)stream, (uint16_t*)qkv, positions, cos_table,
                       sin_table, (int)table_rows, (const uint16_t*)q_gamma, (const uint16_t*)q_beta,
                       (const uint16_t*)k_gamma, (const uint16_t*)k_beta, eps, (int)T, (int)H, (long)token_stride,
                       hshift);
    return check_launch("qknorm_rope2d");
  }
  constexpr int NR = 2;   // two rows per 8-lane group: 3 % faster than one at S = 32
  hipLaunchKernelGGL(qknorm_rope2d_kernel<NR>,
                     dim3((unsigned)((rows + QKN_ROWS_PER_WG * NR - 1) / (QKN_ROWS_PER_WG * NR))), dim3(256), 0,
                     (hipStream_t)stream, (uint16_t*)qkv, positions, cos_table, sin_table, (int)table_rows,
                     (const uint16_t*)q_gamma, (const uint16_t*)q_beta, (const uint16_t*)k_gamma,
                     (const uint16_t*)k_beta, eps, (int)T, (int)H, (long)token_stride, hshift);
  return check_launch("qknorm_rope2d");
}

extern "C" int qv_rope_with_pos(const void* x, const float* freqs, void* out, int dtype, int64_t S, int64_t B,
                                int64_t H, int64_t D, int64_t D2, const int64_t* x_strides,
                                const int64_t* out_strides, void* stream) {
  QV_CHECK_ARG(S >= 0 && B >= 0 && H >= 0 && D > 0, "bad shape");
  QV_CHECK_ARG(D2 > 0 && D2 <= D && D2 % 2 == 0, "rotary dim d2=%lld must be even and <= d=%lld", (long long)D2,
               (long long)D);
  QV_CHECK_ARG(x_strides && out_strides, "null stride array");
  if (S * B * H == 0) return QV_OK;
  QV_CHECK_ARG(x && freqs && out, "null pointer argument");
  QV_CHECK_ARG(S <= INT32_MAX && B <= INT32_MAX && H * D <= INT32_MAX, "shape too large");
  QV_CHECK_ARG(dtype == QV_F16 || dtype == QV_BF16 || dtype == QV_F32, "unsupported dtype %d", dtype);
  const long* xs = (const long*)x_strides;
  const long* os = (const long*)out_strides;
  // 16-byte vector accesses: unit dim strides, aligned rows, whole 8-element chunks
  const long align = dtype == QV_F32 ? 4 : 8;
  const bool vec = xs[3] == 1 && os[3] == 1 && (D2 / 2) % 8 == 0 && (D - D2) % 8 == 0 &&
                   xs[0] % align == 0 && xs[1] % align == 0 && xs[2] % align == 0 && os[0] % align == 0 &&
                   os[1] % align == 0 && os[2] % align == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)out % 16) == 0;
  const bool tab = D2 <= RWP_MAX_D2;
  const long npos = S * B;
  const long blocks = (npos + RWP_WAVES - 1) / RWP_WAVES;
  const dim3 grid((unsigned)(blocks < 16384 ? blocks : 16384)), block(64 * RWP_WAVES);
  hipStream_t st = (hipStream_t)stream;
#define QV_ROPE(DTV, V, T)                                                                                        \
  hipLaunchKernelGGL((rope_with_pos_kernel<DTV, V, T>), grid, block, 0, st, x, freqs, out, (int)S, (int)B, (int)H, \
                     (int)D, (int)D2, xs[0], xs[1], xs[2], xs[3], os[0], os[1], os[2], os[3])
#define QV_ROPE_DT(DTV) \
  if (vec && tab) QV_ROPE(DTV, true, true); else if (vec) QV_ROPE(DTV, true, false); \
  else if (tab) QV_ROPE(DTV, false, true); else QV_ROPE(DTV, false, false);
  switch (dtype) {
    case QV_F16: QV_ROPE_DT(QV_F16) break;
    case QV_BF16: QV_ROPE_DT(QV_BF16) break;
    default: QV_ROPE_DT(QV_F32) break;
  }
#undef QV_ROPE_DT
#undef QV_ROPE
  return check_launch("rope_with_pos");
}

extern "C" int qv_rope2d(const void* qkv, void* out, const int32_t* positions, const float* cos_table,
                         const float* sin_table, int64_t table_rows, int64_t T, int64_t H,
                         int64_t src_token_stride, int64_t dst_token_stride, int64_t dst_part_stride,
                         void* stream) {
  QV_CHECK_ARG(T >= 0 && H > 0, "bad shape T=%lld H=%lld", (long long)T, (long long)H);
  QV_CHECK_ARG(table_rows > 0 && table_rows <= INT32_MAX, "bad table size %lld", (long long)table_rows);
  if (T == 0) return QV_OK;
  QV_CHECK_ARG(qkv && out && positions && cos_table && sin_table, "null pointer argument");
  QV_CHECK_ARG(src_token_stride % 8 == 0 && dst_token_stride % 8 == 0 && dst_part_stride % 8 == 0 &&
                   ((uintptr_t)qkv % 16) == 0 && ((uintptr_t)out % 16) == 0 && ((uintptr_t)cos_table % 16) == 0 &&
                   ((uintptr_t)sin_table % 16) == 0,
               "rope2d needs 16-byte aligned rows and tables");
  const long nrows = T * 2 * H;
  const int hshift = (H & (H - 1)) == 0 ? __builtin_ctzll((unsigned long long)H) : -1;
  if (H % 16 == 0 && tok_blocks_ok(nrows)) {
    hipLaunchKernelGGL(rope2d_tok_kernel, dim3((unsigned)((nrows / 32 + TOK_WAVES - 1) / TOK_WAVES)),
                       dim3(64 * TOK_WAVES), 0, (hipStream_t)stream, (const uint16_t*)qkv, (uint16_t*)out, positions,
                       cos_table, sin_table, (int)table_rows, (int)T, (int)H, (long)src_token_stride,
                       (long)dst_token_stride, (long)dst_part_stride, hshift);
    return check_launch("rope2d");
  }
  // two rows per 8-lane group: 10 % faster than one at S = 32, four no better
  constexpr int NR = 2;
  hipLaunchKernelGGL(rope2d_kernel<NR>, dim3((unsigned)((nrows + 32 * NR - 1) / (32 * NR))), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)qkv, (uint16_t*)out, positions, cos_table, sin_table,
                     (int)table_rows, (int)T, (int)H, (long)src_token_stride, (long)dst_token_stride,
                     (long)dst_part_stride, hshift);
  return check_launch("rope2d");
}
