// Streamed W4A16 group-128 GEMM for gfx950 (the large-M path).
//
// Workgroup tile BM (= 32*MT, m) x 256 (n); the 4 waves sit side by side
// along n, each owning BM x 64 = MT x 2 tiles of v_mfma_f32_32x32x16 (so every
// dequantised weight fragment feeds MT MFMAs of 32x32x16).  All operands
// stream global -> LDS with direct buffer loads (no register staging) through
// 3 stages of 64 k:
//   A   BM rows x 128 B activations; 16-byte chunk c of row r stored at
//       c ^ fA(r), fA(r) = (r & 7) ^ ((r >> 3) & 1)
//   B   256 channels x 32 B: the stage's two 16-byte 32-k chunks per channel,
//       chunk cc of channel n stored at cc ^ fB(n), fB(n) = ((n>>2) ^ (n>>3)) & 1
//   S,Z the 256 fp16 scales / scaled zeros of the stage's 128-k group
// Both swizzles make every 8-lane and every 16-lane group of a b128 read hit
// distinct banks (whichever the hardware groups per cycle), and each 1 KB
// direct write is contiguous.
//
// K-slots: MFMA operand lanes split as h = lane/32 (k-half) and l = lane%32.
// In k-step s (0..3) of a stage, lane half h takes 32-k chunk h and nibble
// pair s of its four words, i.e. stage-local k = 32*h + 8*s + slot on BOTH
// operands (activations: 8 contiguous halves of chunk 4h + s).  Output: lane
// (h, l), register r holds out[m = l][n = 8*(r/4) + 4*h + r%4] of the tile.
// LDS per workgroup: 3 x (BM*128 + 9 KB); BM = 128 -> 75 KB, 2 workgroups/CU.
// The epilogue reuses that LDS to stage each wave's BM x 64 output tile and
// writes it back as whole 128-byte rows.
#include "w4a16_common.h"

namespace qv {

template <bool BF16, int MT, int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void w4a16_stream32_kernel(const uint16_t* __restrict__ x, const uint32_t* __restrict__ qw,
                           const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
                           const uint16_t* __restrict__ bias, const uint16_t* __restrict__ gamma,
                           uint16_t* __restrict__ out, int M, int N,
                           int K, int tiles_n) {
  constexpr int BM = 32 * MT, BN = 256, NT = 2;
  constexpr int A_BYTES = BM * 128, B_BYTES = BN * 32, S_BYTES = BN * 2;
  constexpr int STAGE = A_BYTES + B_BYTES + 2 * S_BYTES;
  constexpr int NSTAGE = 3;
  constexpr int A_INSTR = BM / 32;                // 1 KB direct loads per wave for A
  constexpr int VM_PER_STAGE = A_INSTR + 2 + 1;   // + B (2) + S or Z (1)
  static_assert(VM_PER_STAGE < 16, "vmcnt immediate");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NSTAGE * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int h = lane >> 5, l32 = lane & 31;
  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  const int m0 = (lid / tiles_n) * BM;
  const int n0 = (lid % tiles_n) * BN;
  const int K2 = K * 2;
  const int KS = K >> 6;

  const auto rsA = make_rsrc(x + (size_t)m0 * K, (uint64_t)(M - m0) * K2);
  const auto rsB = make_rsrc(qw + (size_t)(n0 >> 2) * (K >> 1), (uint64_t)((N - n0) >> 2) * K2);
  const auto rsS = make_rsrc((wave < 2 ? scales : zeros) + n0, ((uint64_t)(K >> 7) * N - n0) * 2);

  // A: instruction q covers rows r0 = 8*(A_INSTR*wave + q) .. +7; lane L lands
  // at row r0 + L/8, physical chunk L%8 and so fetches logical chunk
  // (L%8) ^ fA(row) = (L%8) ^ (L/8) ^ ((r0 >> 3) & 1).
  uint32_t a_voff[2];
#pragma unroll
  for (int v = 0; v < 2; ++v)
    a_voff[v] = (uint32_t)((lane >> 3) * K2 + (((lane & 7) ^ (lane >> 3) ^ v) * 16));
  // B: instruction q covers channels r0 = 32*(2*wave + q) .. +31; lane L lands
  // at channel r0 + L/2, physical chunk L&1 = logical cc ^ fB(L/2).
  const int bn = lane >> 1;
  const int bcc = (lane & 1) ^ (((lane >> 3) ^ (lane >> 4)) & 1);
  const uint32_t b_voff = (uint32_t)((bn >> 2) * K2 + 32 * (bn & 3) + 16 * bcc);

  const uint32_t lds0 = lds_addr(lds);
  auto issue = [&](int ks, int st) {
    const uint32_t base = lds0 + st * STAGE;
#pragma unroll
    for (int q = 0; q < A_INSTR; ++q) {
      const int r0 = 8 * (A_INSTR * wave + q);
      lds_dma16(rsA, a_voff[(r0 >> 3) & 1], r0 * K2 + ks * 128, base + r0 * 128);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int r0 = 32 * (2 * wave + q);
      lds_dma16(rsB, b_voff, (r0 >> 2) * K2 + ks * 128, base + A_BYTES + r0 * 32);
    }
    // waves 0,1: the two halves of the scales; waves 2,3: of the scaled zeros
    lds_dma4(rsS, lane * 4, (ks >> 1) * N * 2 + (wave & 1) * 256,
             base + A_BYTES + B_BYTES + (wave >> 1) * S_BYTES + (wave & 1) * 256);
  };

  f32x16 acc[NT][MT];
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.f;

  // per-lane LDS byte offsets that do not depend on the stage
  uint32_t b_off[NT], s_off[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int n = 64 * wave + 32 * j + l32;
    b_off[j] = (uint32_t)(A_BYTES + n * 32 + ((h ^ (((n >> 2) ^ (n >> 3)) & 1)) * 16));
    s_off[j] = (uint32_t)(A_BYTES + B_BYTES + n * 2);
  }
  const int fa = (l32 & 7) ^ ((l32 >> 3) & 1);  // fA(32*i + l32) is the same for all i

  auto dq = [&](int s, const uint4 (&wq)[NT], const uint32_t (&sv)[NT], const uint32_t (&zv)[NT], uint4 (&wf)[NT]) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      switch (s) {
        case 0: wf[j] = dq_frag<BF16, 0>(wq[j], sv[j], zv[j]); break;
        case 1: wf[j] = dq_frag<BF16, 1>(wq[j], sv[j], zv[j]); break;
        case 2: wf[j] = dq_frag<BF16, 2>(wq[j], sv[j], zv[j]); break;
        default: wf[j] = dq_frag<BF16, 3>(wq[j], sv[j], zv[j]); break;
      }
    }
  };
  // One stage: k-step s issues the LDS reads of step s+1's activations, then
  // its own MFMAs, then dequantises step s+1's weights (VALU that co-issues
  // with the MFMAs in flight).  The scheduling fences keep the compiler from
  // sinking the reads next to their use, which would expose LDS latency.
  auto compute = [&](int st) {
    const uint8_t* base = lds + st * STAGE;
    uint4 wq[NT];
    uint32_t sv[NT], zv[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      wq[j] = *reinterpret_cast<const uint4*>(base + b_off[j]);
      sv[j] = *reinterpret_cast<const uint16_t*>(base + s_off[j]);
      zv[j] = *reinterpret_cast<const uint16_t*>(base + s_off[j] + S_BYTES);
    }
    uint4 af[2][MT], wf[2][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
      af[0][i] = *reinterpret_cast<const uint4*>(base + (32 * i + l32) * 128 + (uint32_t)(((4 * h) ^ fa) * 16));
    dq(0, wq, sv, zv, wf[0]);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s < 3) {
        const uint32_t col = (uint32_t)(((4 * h + s + 1) ^ fa) * 16);
#pragma unroll
        for (int i = 0; i < MT; ++i)
          af[(s + 1) & 1][i] = *reinterpret_cast<const uint4*>(base + (32 * i + l32) * 128 + col);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[j][i] = mfma32<BF16>(wf[s & 1][j], af[s & 1][i], acc[j][i]);
      }
      if (s < 3) dq(s + 1, wq, sv, zv, wf[(s + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  issue(0, 0);
  if (KS > 1) issue(1, 1);
  for (int ks = 0; ks < KS; ++ks) {
    // this wave's loads for stage ks have landed; after the barrier everyone's
    // have, and every wave is done with stage ks-1 (overwritten next)
    if (ks + 1 < KS) {
      __builtin_amdgcn_s_waitcnt(0x0F70 | VM_PER_STAGE);  // vmcnt(VM_PER_STAGE)
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);                 // vmcnt(0)
    }
    lds_barrier();
    if (ks + 2 < KS) issue(ks + 2, (ks + 2) % NSTAGE);
    compute(ks % NSTAGE);
  }

  // ---- epilogue: the wave's BM x 64 output tile goes through LDS so that the
  // global stores are whole 128-byte rows (direct 8-byte stores from the MFMA
  // layout cost ~3x the output size in HBM write traffic).
  lds_barrier();  // every wave is done reading the pipeline stages
  constexpr int EP = 144;  // bytes per staged row: 64 fp16 + 16 B pad
  static_assert(4 * BM * EP <= NSTAGE * STAGE, "epilogue staging fits in the pipeline LDS");
  uint8_t* stg = lds + wave * (BM * EP);
#pragma unroll
  for (int j = 0; j < NT; ++j) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int nl = 32 * j + 8 * q + 4 * h;
      const int n = n0 + 64 * wave + nl;
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        float r[4] = {acc[j][i][4 * q], acc[j][i][4 * q + 1], acc[j][i][4 * q + 2], acc[j][i][4 * q + 3]};
        epilogue_apply4<BF16, EPI>(bias, r, n < N ? n : 0);
        uint2 o;
        o.x = pack2<BF16>(r[0], r[1]);
        o.y = pack2<BF16>(r[2], r[3]);
        *reinterpret_cast<uint2*>(stg + (32 * i + l32) * EP + nl * 2) = o;
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's staging writes are done
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int it = 0; it < BM * 8 / 64; ++it) {
    const int idx = it * 64 + lane;
    const int row = idx >> 3, c = idx & 7;
    const int m = m0 + row, n = n0 + 64 * wave + 8 * c;
    if (m < M && n < N) {
      uint4 v = *reinterpret_cast<const uint4*>(stg + row * EP + c * 16);
      if constexpr (EPI == QV_EPI_BIAS_RESID)
        v = resid_update8<BF16>(*reinterpret_cast<const uint4*>(out + (size_t)m * N + n), v,
                                *reinterpret_cast<const uint4*>(gamma + n));
      *reinterpret_cast<uint4*>(out + (size_t)m * N + n) = v;
    }
  }
}

template <bool BF16, int MT>
static void launch_mt(const void* x, const void* qw, const void* s, const void* z, const void* bias,
                      const void* gamma, void* out, int M, int N, int K, int epi, hipStream_t st) {
  const int tiles_m = (M + 32 * MT - 1) / (32 * MT), tiles_n = (N + 255) / 256;
  const dim3 grid(tiles_m * tiles_n), block(256);
#define QV_ARGS                                                                                \
  (const uint16_t*)x, (const uint32_t*)qw, (const uint16_t*)s, (const uint16_t*)z,             \
      (const uint16_t*)bias, (const uint16_t*)gamma, (uint16_t*)out, M, N, K, tiles_n
  switch (epi) {
    case QV_EPI_NONE:
      hipLaunchKernelGGL((w4a16_stream32_kernel<BF16, MT, QV_EPI_NONE>), grid, block, 0, st, QV_ARGS);
      break;
    case QV_EPI_BIAS:
      hipLaunchKernelGGL((w4a16_stream32_kernel<BF16, MT, QV_EPI_BIAS>), grid, block, 0, st, QV_ARGS);
      break;
    case QV_EPI_BIAS_GELU:
      hipLaunchKernelGGL((w4a16_stream32_kernel<BF16, MT, QV_EPI_BIAS_GELU>), grid, block, 0, st, QV_ARGS);
      break;
    case QV_EPI_GELU:
      hipLaunchKernelGGL((w4a16_stream32_kernel<BF16, MT, QV_EPI_GELU>), grid, block, 0, st, QV_ARGS);
      break;
    default:
      hipLaunchKernelGGL((w4a16_stream32_kernel<BF16, MT, QV_EPI_BIAS_RESID>), grid, block, 0, st, QV_ARGS);
      break;
  }
#undef QV_ARGS
}

template <bool BF16>
int launch_w4a16_stream(const void* x, const void* qw, const void* s, const void* z, const void* bias,
                        const void* gamma, void* out, int M, int N, int K, int epi, int bm, hipStream_t st) {
  if (bm == 128) launch_mt<BF16, 4>(x, qw, s, z, bias, gamma, out, M, N, K, epi, st);
  else if (bm == 96) launch_mt<BF16, 3>(x, qw, s, z, bias, gamma, out, M, N, K, epi, st);
  else if (bm == 64) launch_mt<BF16, 2>(x, qw, s, z, bias, gamma, out, M, N, K, epi, st);
  else launch_mt<BF16, 1>(x, qw, s, z, bias, gamma, out, M, N, K, epi, st);
  return check_launch("w4a16_stream32");
}

template int launch_w4a16_stream<false>(const void*, const void*, const void*, const void*, const void*,
                                        const void*, void*, int, int, int, int, int, hipStream_t);
template int launch_w4a16_stream<true>(const void*, const void*, const void*, const void*, const void*,
                                       const void*, void*, int, int, int, int, int, hipStream_t);

}  // namespace qv
