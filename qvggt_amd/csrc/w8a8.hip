// W8A8 GEMM for gfx950: int8 activations (per-token scale) x int8 weights
// (per-output-channel scale), exact int32 accumulation on
// v_mfma_i32_32x32x32_i8, epilogue fp16_rn((float(acc) * ws[n]) * as[m] (+ bias[n])).
// Replaces dense_kernel0 / dense_kernel0_fuse_bias of the reference
// (w8a8/w8a8_gemm_cuda.cu:284-607, 609-922).
//
// Workgroup tile BM (= 32*MT, m) x 256 (n); the 4 waves sit side by side along
// n, each owning BM x 64 = MT x 2 MFMA tiles of 32x32.  Activations and
// weights stream global -> LDS with direct buffer loads through 3 stages of
// 64 k (A: BM x 64 B, B: 256 x 64 B).  Rows are 64 B = four 16-byte chunks;
// chunk c of row r is stored at c ^ f(r), f(r) = (r + (r >> 2)) & 3.  Chosen by
// measurement: with f(r) = ((r >> 1) + (r >> 3)) & 3 the fragment reads cost
// ~4 bank-conflict cycles per LDS instruction (SQ_LDS_BANK_CONFLICT); with
// this f they cost none, and the fc1 shape ran 71.1 -> 68.6 us.
// K-slots: k-step s (0..1) of a stage, lane half h: k = 32*s + 16*h + 0..15
// (16 contiguous bytes = chunk 2s + h) on both operands.  Output: lane (h, l),
// register r holds out[m = l][n = 8*(r/4) + 4*h + r%4] of the wave's tile.
// Packed weights (PACKED, qv_w8a8_gemm_packed): the weights are re-laid out
// once (qv_w8a8_pack_weight) so that the 16-byte B fragment of lane L for
// column block cb (32 channels), stage ks and k-step s sits at byte
// ((cb * KS + ks) * 2 + s) * 1024 + 16 * L: each wave then loads its own
// 64 columns straight to registers, one stage ahead, every load instruction
// one contiguous 1 KB, and the LDS holds only the activations.  (Loaded
// straight from the N x K layout, each 16-byte lane load touches 32 rows in
// 32-byte pieces: measured 10-26 % slower than the LDS path; packed, 12-16 %
// faster than it.)
// Outputs are written with non-temporal stores so that they do not evict the
// operand rows the XCD's other tiles still read from L2.  The residual form
// (OUT 3, qv_w8a8_gemm_residual) reads the residual row chunk and LayerScale
// gamma in the store loop and writes residual + gamma * fp16(epilogue) in
// place, which replaces torch's x.addcmul_(o, gamma) pass of a VGGT block.
#include <type_traits>

#include "common.h"

#pragma clang fp contract(off)

namespace qv {

__device__ __forceinline__ int f8(int r) { return (r + (r >> 2)) & 3; }

// OUT: 0 = fp16 (scaled), 1 = fp16 (scaled + bias), 2 = raw int32,
// 3 = fp16 (scaled + bias) LayerScale-added to `out` in place
template <int MT, int OUT, bool PACKED>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void w8a8_gemm_kernel(const int8_t* __restrict__ a, const int8_t* __restrict__ b,
                      const uint16_t* __restrict__ ws, const uint16_t* __restrict__ as,
                      const uint16_t* __restrict__ bias, const uint16_t* __restrict__ gamma,
                      void* __restrict__ out, int M, int N, int K, int tiles_n, int gn) {
  constexpr bool BIAS = OUT == 1 || OUT == 3;
  constexpr int BM = 32 * MT, BN = 256, NT = 2;
  constexpr int A_BYTES = BM * 64, B_BYTES = PACKED ? 0 : BN * 64;
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int NSTAGE = 3;
  constexpr int A_INSTR = BM / 64;   // 1 KB direct loads per wave per stage (A)
  constexpr int B_INSTR = 4;         // 16 KB / 1 KB / 4 waves (LDS path)
  constexpr int EP = 128;            // bytes per staged epilogue row (64 fp16, chunk-swizzled: stg_off)
  constexpr int LDS_BYTES = NSTAGE * STAGE > 4 * BM * EP ? NSTAGE * STAGE : 4 * BM * EP;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;
  // Tiles are numbered column group by column group (gn n-tiles wide), row
  // by row inside a group, and each XCD takes a contiguous range of that
  // order (xcd_remap): the weight slices of one group stay in the XCD's L2
  // while it walks down the rows (w8a8_col_group picks gn).
  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  const int tiles_m = (M + BM - 1) / BM;
  const int g = lid / (tiles_m * gn);
  const int r = lid - g * tiles_m * gn;
  const int gw = tiles_n - g * gn < gn ? tiles_n - g * gn : gn;
  const int m0 = (r / gw) * BM;
  const int n0 = (g * gn + r % gw) * BN;
  const int KS = K >> 6;

  // The epilogue's per-channel scales / bias and per-token scales, loaded
  // before the main loop so their latency hides under it (read after the
  // loop they cost one exposed global-load wait per 4-column group).  Only
  // the 128-row tiles of multi-round launches: in a one-round launch of
  // 64-row tiles the early loads delay the first stage more than they save
  // (measured, mean of four same-process A/B runs: fc1 at 10,992 tokens
  // -2.2 %, qkv at 10,992 tokens -3.1 %; qkv at 1,374 tokens +2 % when the
  // 64-row tiles prefetched too).
  constexpr bool PREF = OUT != 2 && MT >= 4;
  uint2 wsv[NT][4], bsv[NT][4];
  uint16_t asv[MT];
  if constexpr (PREF) {
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int n = min(n0 + 64 * wave + 32 * j + 8 * qd + 4 * h, N - 4);
        wsv[j][qd] = *reinterpret_cast<const uint2*>(ws + n);
        if constexpr (BIAS) bsv[j][qd] = *reinterpret_cast<const uint2*>(bias + n);
      }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int m = m0 + 32 * i + l32;
      asv[i] = as[m < M ? m : M - 1];
    }
  }

  const auto rsA = make_rsrc(a + (size_t)m0 * K, (uint64_t)(M - m0) * K);
  // packed: column blocks of 32 channels, 32 K bytes each, N rounded up to 32
  const auto rsB = PACKED ? make_rsrc(b + (size_t)n0 * K, (uint64_t)(((N + 31) & ~31) - n0) * K)
                          : make_rsrc(b + (size_t)n0 * K, (uint64_t)(N - n0) * K);

  // Direct loads: instruction covers 16 rows r0..r0+15 (r0 % 16 == 0); lane L
  // lands at row r0 + L/4, physical chunk L%4, so it fetches logical chunk
  // (L%4) ^ f(r0 + L/4); voff[v] serves r0 % 32 == 16 v.
  uint32_t voff[2];
#pragma unroll
  for (int v = 0; v < 2; ++v) {
    const int c = (lane & 3) ^ f8(16 * v + (lane >> 2));
    voff[v] = (uint32_t)((lane >> 2) * K + c * 16);
  }
  const uint32_t lds0 = lds_addr(lds);
  auto issue = [&](int ks, int st) {
    const uint32_t base = lds0 + st * STAGE;
#pragma unroll
    for (int q = 0; q < A_INSTR; ++q) {
      const int r0 = 16 * (A_INSTR * wave + q);
      lds_dma16(rsA, voff[(r0 >> 4) & 1], r0 * K + ks * 64, base + r0 * 64);
    }
    if constexpr (!PACKED) {
#pragma unroll
      for (int q = 0; q < B_INSTR; ++q) {
        const int r0 = 16 * (B_INSTR * wave + q);
        lds_dma16(rsB, voff[(r0 >> 4) & 1], r0 * K + ks * 64, base + A_BYTES + r0 * 64);
      }
    }
  };

  i32x16 acc[NT][MT];
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][i][r] = 0;

  const int fl = f8(l32);  // f has period 16: f(32*i + l32) == f(l32), and f(64*w + 32*j + l32) too
  if constexpr (PACKED) {
    // Activation fragments of k-step s of the stage in LDS buffer st.
    auto read_a = [&](int st, int s, uint4 (&av)[MT]) {
      const uint8_t* base = lds + st * STAGE;
      const uint32_t col = (uint32_t)(((2 * s + h) ^ fl) * 16);
#pragma unroll
      for (int i = 0; i < MT; ++i) av[i] = *reinterpret_cast<const uint4*>(base + (32 * i + l32) * 64 + col);
    };
    // Weights of column block 2 * wave + j, stage ks, k-step s: one 1 KB load.
    uint32_t b_voff[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) b_voff[j] = (uint32_t)((2 * wave + j) * 32 * K + 16 * lane);
    auto load_b = [&](int ks, uint4 (&bw)[NT][2]) {
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
          bw[j][s2] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsB, b_voff[j], ks * 2048 + 1024 * s2, 0));
    };
    auto mfmas = [&](const uint4 (&bw)[NT][2], int s, const uint4 (&av)[MT]) {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
          acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, bw[j][s]),
                                                            __builtin_bit_cast(i32x4, av[i]), acc[j][i], 0, 0, 0);
    };
    // One stage (LDS buffer st, weights bw), as in the LDS path below: step 0
    // issues the activation reads of step 1, then its MFMAs; step 1 those of
    // the next stage's step 0 (buffer nst), then its MFMAs.
    uint4 a0[MT];
    // mid(): run between the stage's two k-steps (the weight requests)
    auto compute = [&](int st, int nst, const uint4 (&bw)[NT][2], auto&& mid) {
      uint4 a1[MT];
      read_a(st, 1, a1);
      __builtin_amdgcn_sched_barrier(0);
      mfmas(bw, 0, a0);
      __builtin_amdgcn_sched_barrier(0);
      mid();
      __builtin_amdgcn_sched_barrier(0);
      read_a(nst, 0, a0);
      __builtin_amdgcn_sched_barrier(0);
      mfmas(bw, 1, a1);
      __builtin_amdgcn_sched_barrier(0);
    };
    // Stage s uses LDS buffer s % 4 and weight register set s % 3.  At its
    // top, vmcnt(A_INSTR + W_OPS) lands this wave's activation copy of stage
    // s + 1 and its weights of stage s, both issued two stages earlier (only
    // the previous stage's copy and weight loads stay in flight); the barrier
    // publishes the copies and frees buffer (s + 3) % 4, the previous stage's,
    // which receives stage s + 3, and the weights of stage s + 2 go into the
    // register set stage s - 1 used, requested between stage s's k-steps.  Requests one stage ahead (3 buffers, 2
    // register sets) left their latency exposed: same-box A/B, bit-identical,
    // fc1 at 10,992 tokens 60.2 -> 57.1 us, fc2 54.7 -> 52.7 us, qkv 47.9 ->
    // 46.0 us, 2748 x 4096 -> 1024 35.5 -> 21.3 us.  Three stages run per
    // iteration (constant register-set indices), a remainder of one or two
    // after the loop; loads past the last stage repeat it (valid addresses,
    // into a buffer or register set nobody reads), so every stage issues the
    // same count and the wait above stays exact.
    constexpr int NB = 4;                      // LDS buffers of the activation copies
    constexpr int W_OPS = 2 * NT;              // weight loads per stage
    constexpr int WAIT_TOP = 0x0F70 | (A_INSTR + W_OPS);
    static_assert(A_INSTR + W_OPS < 16, "vmcnt immediate");
    static_assert(NB * STAGE <= LDS_BYTES, "the activation buffers fit the LDS allocation");
    uint4 bw3[3][NT][2];
    const int last = KS - 1;
    issue(0, 0);
    issue(KS > 1 ? 1 : last, 1);
    issue(KS > 2 ? 2 : last, 2);
    load_b(0, bw3[0]);
    load_b(KS > 1 ? 1 : last, bw3[1]);
    __builtin_amdgcn_s_waitcnt(0x0070);   // vmcnt(0) lgkmcnt(0), as in the LDS path
    lds_barrier();
    read_a(0, 0, a0);
    auto stage = [&](int s, auto pc) __attribute__((always_inline)) {
      constexpr int p = decltype(pc)::value, p2 = (p + 2) % 3;
      if (s > 0) {
        __builtin_amdgcn_s_waitcnt(WAIT_TOP);   // A(s + 1), B(s): issued two stages ago
        lds_barrier();
      }
      const int s3 = s + 3 < KS ? s + 3 : last, s2 = s + 2 < KS ? s + 2 : last;
      issue(s3, (s + 3) & (NB - 1));
      // the weight requests between the stage's k-steps rather than at its
      // top: 1-6 % faster on most shapes, bitwise identical (fc1 at 10,992
      // tokens 59.6 -> 57.9 us, proj 18.8 -> 17.7 us, qkv at 1,374 tokens
      // 11.2 -> 10.8 us; qkv at 10,992 tokens level)
      compute(s & (NB - 1), (s + 1) & (NB - 1), bw3[p], [&]() __attribute__((always_inline)) { load_b(s2, bw3[p2]); });
    };
    int i = 0;
    for (; i + 3 <= KS; i += 3) {
      stage(i, std::integral_constant<int, 0>());
      stage(i + 1, std::integral_constant<int, 1>());
      stage(i + 2, std::integral_constant<int, 2>());
    }
    if (i < KS) stage(i, std::integral_constant<int, 0>());
    if (i + 1 < KS) stage(i + 1, std::integral_constant<int, 1>());
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the repeated loads land before the epilogue
  } else {
    // Fragments of k-step s of the stage in LDS buffer st (weights, activations).
    auto read = [&](int st, int s, uint4 (&bw)[NT], uint4 (&av)[MT]) {
      const uint8_t* base = lds + st * STAGE;
      const uint32_t col = (uint32_t)(((2 * s + h) ^ fl) * 16);
#pragma unroll
      for (int j = 0; j < NT; ++j)
        bw[j] = *reinterpret_cast<const uint4*>(base + A_BYTES + (64 * wave + 32 * j + l32) * 64 + col);
#pragma unroll
      for (int i = 0; i < MT; ++i) av[i] = *reinterpret_cast<const uint4*>(base + (32 * i + l32) * 64 + col);
    };
    auto mfmas = [&](const uint4 (&bw)[NT], const uint4 (&av)[MT]) {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
          acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, bw[j]),
                                                            __builtin_bit_cast(i32x4, av[i]), acc[j][i], 0, 0, 0);
    };
    // One stage (buffer st).  On entry b0 / a0 hold its k-step 0 fragments.
    // Step 0 issues the reads of step 1, then its MFMAs; step 1 issues the
    // reads of the NEXT stage's k-step 0 (buffer nst), then its MFMAs, so no
    // stage starts with its MFMAs waiting behind the barrier for LDS reads.
    // The fences keep the compiler from sinking each read next to its use.
    uint4 b0[NT], a0[MT];
    auto compute = [&](int st, int nst) {
      uint4 b1[NT], a1[MT];
      read(st, 1, b1, a1);
      __builtin_amdgcn_sched_barrier(0);
      mfmas(b0, a0);
      __builtin_amdgcn_sched_barrier(0);
      read(nst, 0, b0, a0);
      __builtin_amdgcn_sched_barrier(0);
      mfmas(b1, a1);
      __builtin_amdgcn_sched_barrier(0);
    };

    // Stage ks uses buffer ks % 3.  At its top: vmcnt(0) lands this wave's
    // copies of stage ks + 1 (issued one stage earlier), and the barrier makes
    // every wave's visible and guarantees every wave is done with buffer
    // (ks + 2) % 3 = the previous stage's, which then receives stage ks + 2.
    // Stages past KS - 1 are not copied; the last stage's read of the "next"
    // stage reads a buffer nobody uses again (its values are dropped).
    issue(0, 0);
    if (KS > 1) issue(1, 1);
    // vmcnt(0): stages 0 and 1; lgkmcnt(0), as a builtin the compiler sees:
    // a scalar load it hoisted here (a kernel argument of the epilogue) would
    // otherwise count as pending through the loop, and since scalar loads
    // return out of order the compiler would wait lgkmcnt(0) for every LDS read
    __builtin_amdgcn_s_waitcnt(0x0070);
    lds_barrier();
    read(0, 0, b0, a0);
    for (int ks = 0; ks < KS; ++ks) {
      __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
      lds_barrier();
      if (ks + 2 < KS) issue(ks + 2, (ks + 2) % NSTAGE);
      compute(ks % NSTAGE, (ks + 1) % NSTAGE);
    }
  }

  if constexpr (OUT == 2) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int n = n0 + 64 * wave + 32 * j + 8 * qd + 4 * h;
        if (n >= N) continue;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          const int m = m0 + 32 * i + l32;
          if (m >= M) continue;
          int4 o = make_int4(acc[j][i][4 * qd], acc[j][i][4 * qd + 1], acc[j][i][4 * qd + 2], acc[j][i][4 * qd + 3]);
          st_stream16(reinterpret_cast<int32_t*>(out) + (size_t)m * N + n, __builtin_bit_cast(uint4, o));
        }
      }
    }
  } else {
    // fp16 output: the wave's BM x 64 tile is staged in LDS (reusing the
    // pipeline buffers) and written back as whole 128-byte rows.
    lds_barrier();  // every wave is done reading the pipeline stages
    uint8_t* stg = lds + wave * (BM * EP);
    float am[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      if constexpr (PREF) {
        am[i] = to_f32(asv[i], false);
      } else {
        const int m = m0 + 32 * i + l32;
        am[i] = to_f32(as[m < M ? m : M - 1], false);
      }
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int nl = 32 * j + 8 * qd + 4 * h;
        const int n = min(n0 + 64 * wave + nl, N - 4);
        float wsn[4], bn[4] = {0.f, 0.f, 0.f, 0.f};
        uint2 wv;
        if constexpr (PREF) wv = wsv[j][qd];
        else wv = *reinterpret_cast<const uint2*>(ws + n);
        wsn[0] = to_f32((uint16_t)(wv.x & 0xFFFF), false);
        wsn[1] = to_f32((uint16_t)(wv.x >> 16), false);
        wsn[2] = to_f32((uint16_t)(wv.y & 0xFFFF), false);
        wsn[3] = to_f32((uint16_t)(wv.y >> 16), false);
        if constexpr (BIAS) {
          uint2 bv;
          if constexpr (PREF) bv = bsv[j][qd];
          else bv = *reinterpret_cast<const uint2*>(bias + n);
          bn[0] = to_f32((uint16_t)(bv.x & 0xFFFF), false);
          bn[1] = to_f32((uint16_t)(bv.x >> 16), false);
          bn[2] = to_f32((uint16_t)(bv.y & 0xFFFF), false);
          bn[3] = to_f32((uint16_t)(bv.y >> 16), false);
        }
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          float r[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float t = (float)acc[j][i][4 * qd + e] * wsn[e];
            t = t * am[i];
            if constexpr (BIAS) t = t + bn[e];
            // keep the fp32 rounding of t: without this the backend fuses the last
            // multiply and the fp16 conversion into one v_fma_mixlo_f16 (one rounding)
            asm volatile("" : "+v"(t));
            r[e] = t;
          }
          uint2 o;
          o.x = pack2<false>(r[0], r[1]);
          o.y = pack2<false>(r[2], r[3]);
          *reinterpret_cast<uint2*>(stg + stg_off(32 * i + l32, nl * 2)) = o;
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's staging writes are done
    __builtin_amdgcn_wave_barrier();
    uint16_t* o16 = reinterpret_cast<uint16_t*>(out);
    // Write-back: iteration it moves row (it * 64 + lane) / 8 of the wave's
    // tile, 16-byte chunk lane % 8 -- the same 8 columns in every iteration.
    constexpr int IT = BM * 8 / 64;
    const int c = lane & 7;
    const int n = n0 + 64 * wave + 8 * c;
    if constexpr (OUT == 3) {
      // residual rows read in place of the output, all before the first
      // store (a read of `out` cannot move past a store to it, so in one loop
      // each read waited for the previous store); gamma read once
      const uint4 gv = n < N ? *reinterpret_cast<const uint4*>(gamma + n) : make_uint4(0, 0, 0, 0);
      uint4 rv[IT];
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const int m = m0 + ((it * 64 + lane) >> 3);
        rv[it] = m < M && n < N ? *reinterpret_cast<const uint4*>(o16 + (size_t)m * N + n) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const int row = (it * 64 + lane) >> 3;
        const int m = m0 + row;
        if (m < M && n < N)
          st_stream16(o16 + (size_t)m * N + n,
                      resid_update8<false>(rv[it], *reinterpret_cast<const uint4*>(stg + stg_off(row, c * 16)), gv));
      }
    } else {
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const int row = (it * 64 + lane) >> 3;
        const int m = m0 + row;
        if (m < M && n < N) st_stream16(o16 + (size_t)m * N + n, *reinterpret_cast<const uint4*>(stg + stg_off(row, c * 16)));
      }
    }
  }
}

// Re-layout of an N x K int8 weight for the PACKED kernel: 16-byte chunk
// ((cb * KS + ks) * 2 + s) * 64 + L of the output is bytes
// [64 ks + 32 s + 16 (L / 32), +16) of row 32 cb + L % 32 (zeros for rows past
// N, which is rounded up to 32).  One thread per output chunk.
__global__ __launch_bounds__(256) void w8a8_pack_kernel(const int8_t* __restrict__ w, int8_t* __restrict__ p,
                                                        int N, int K, long nchunks) {
  const long c = (long)blockIdx.x * 256 + threadIdx.x;
  if (c >= nchunks) return;
  const int KS = K >> 6;
  const int L = (int)(c & 63);
  const long blk = c >> 6;                  // (cb * KS + ks) * 2 + s
  const int s = (int)(blk & 1);
  const long cbks = blk >> 1;
  const int ks = (int)(cbks % KS);
  const int cb = (int)(cbks / KS);
  const int n = 32 * cb + (L & 31);
  uint4 v = make_uint4(0, 0, 0, 0);
  if (n < N) v = *reinterpret_cast<const uint4*>(w + (size_t)n * K + 64 * ks + 32 * s + 16 * (L >> 5));
  *reinterpret_cast<uint4*>(p + c * 16) = v;
}

// Width (in 256-column tiles) of the column groups the tile order walks.  A
// read model per launch: every column group reads all of A once (its rows
// are shared by the gn tiles of a row, which run side by side on one XCD),
// and every XCD reads the weight slices of the groups it works on, once when
// they fit in about half of its 4 MB L2 next to the A rows in flight, else
// once per round of its 64 resident tiles.  fc1 of an MLP at 11 k tokens
// (K = 1024, N = 4096): whole rows read the 4 MB weight matrix ~2.7 times per
// XCD (~97 MB), groups of 8 tiles read A twice and the weights once per XCD
// (~38 MB).
static int w8a8_col_group(long tiles_m, int tiles_n, long M, long K) {
  const double a_bytes = (double)M * K, slice = 256.0 * K;
  const double xcd_rounds = (double)tiles_m * tiles_n / (8.0 * 64.0);
  int best = tiles_n;
  double best_cost = 0;
  for (int gn = tiles_n; gn >= 1; --gn) {
    const int groups = (tiles_n + gn - 1) / gn;
    const double groups_per_xcd = groups > 8 ? groups / 8.0 : 1.0;
    const double w_xcd = gn * slice <= 2.0 * 1024 * 1024 ? groups_per_xcd * gn * slice
                                                         : (xcd_rounds > 1 ? xcd_rounds : 1) * gn * slice;
    const double cost = a_bytes * groups + 8.0 * w_xcd;
    if (gn == tiles_n || cost < best_cost) best = gn, best_cost = cost;
  }
  return best;
}

template <int MT, int OUT, bool PACKED>
static void launch(const void* a, const void* b, const void* ws, const void* as, const void* bias,
                   const void* gamma, void* out, int M, int N, int K, hipStream_t st) {
  const int tiles_m = (M + 32 * MT - 1) / (32 * MT), tiles_n = (N + 255) / 256;
  const int gn = w8a8_col_group(tiles_m, tiles_n, M, K);
  hipLaunchKernelGGL((w8a8_gemm_kernel<MT, OUT, PACKED>), dim3(tiles_m * tiles_n), dim3(256), 0, st,
                     (const int8_t*)a, (const int8_t*)b, (const uint16_t*)ws, (const uint16_t*)as,
                     (const uint16_t*)bias, (const uint16_t*)gamma, out, M, N, K, tiles_n, gn);
}

// mode: 0 = fp16 out, 1 = fp16 out + bias, 2 = int32 accumulators,
// 3 = bias + LayerScale residual into `out` (the residual stream);
// packed: b is the qv_w8a8_pack_weight layout (modes 0, 1, 3)
static int w8a8_run(const void* a, const void* b, const void* ws, const void* as, const void* bias,
                    const void* gamma, void* out, int64_t M, int64_t N, int64_t K, int mode, void* stream,
                    bool packed = false) {
  QV_CHECK_ARG(M >= 0 && N > 0 && K > 0, "bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  QV_CHECK_ARG(K % 64 == 0, "K=%lld must be a multiple of 64", (long long)K);
  QV_CHECK_ARG(N % 16 == 0, "N=%lld must be a multiple of 16", (long long)N);
  QV_CHECK_ARG(M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX, "shape too large");
  QV_CHECK_ARG((uint64_t)((N + 31) & ~31) * K < (1ull << 32) && (uint64_t)128 * K < (1ull << 31),
               "weight too large for 32-bit offsets");
  if (M == 0) return QV_OK;
  QV_CHECK_ARG(a && b && out && (mode == 2 || (ws && as)) && ((mode != 1 && mode != 3) || bias) &&
                   (mode != 3 || gamma),
               "null pointer argument");
  QV_CHECK_ARG(((uintptr_t)a % 16) == 0 && ((uintptr_t)b % 16) == 0, "a and b must be 16-byte aligned");
  QV_CHECK_ARG(((uintptr_t)out % 16) == 0, "out must be 16-byte aligned");
  QV_CHECK_ARG(mode == 2 || ((uintptr_t)ws % 8) == 0, "wscales must be 8-byte aligned");
  QV_CHECK_ARG((mode != 1 && mode != 3) || ((uintptr_t)bias % 8) == 0, "bias must be 8-byte aligned");
  QV_CHECK_ARG(mode != 3 || ((uintptr_t)gamma % 16) == 0, "gamma must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  const long big_tiles = (long)((M + 127) / 128) * ((N + 255) / 256);
  const bool big = big_tiles >= 256;
  QV_CHECK_ARG(!packed || mode != 2, "the packed weight layout has no int32 output");
#define QV_W8(MT, P)                                                                                \
  switch (mode) {                                                                                   \
    case 0: launch<MT, 0, P>(a, b, ws, as, bias, gamma, out, (int)M, (int)N, (int)K, st); break;    \
    case 1: launch<MT, 1, P>(a, b, ws, as, bias, gamma, out, (int)M, (int)N, (int)K, st); break;    \
    case 3: launch<MT, 3, P>(a, b, ws, as, bias, gamma, out, (int)M, (int)N, (int)K, st); break;    \
    default:                                                                                        \
      if constexpr (!P) launch<MT, 2, P>(a, b, ws, as, bias, gamma, out, (int)M, (int)N, (int)K, st); \
      break;                                                                                        \
  }
  if (big) {
    if (packed) { QV_W8(4, true) } else { QV_W8(4, false) }
  } else {
    if (packed) { QV_W8(2, true) } else { QV_W8(2, false) }
  }
#undef QV_W8
  return check_launch("w8a8_gemm");
}

}  // namespace qv

extern "C" int qv_w8a8_gemm(const int8_t* a, const int8_t* b, const void* wscales, const void* ascales,
                            const void* bias, void* out, int64_t M, int64_t N, int64_t K, void* stream) {
  return qv::w8a8_run(a, b, wscales, ascales, bias, nullptr, out, M, N, K, bias ? 1 : 0, stream);
}

extern "C" int qv_w8a8_gemm_residual(const int8_t* a, const int8_t* b, const void* wscales, const void* ascales,
                                     const void* bias, const void* gamma, void* residual, int64_t M, int64_t N,
                                     int64_t K, void* stream) {
  return qv::w8a8_run(a, b, wscales, ascales, bias, gamma, residual, M, N, K, 3, stream);
}

extern "C" int qv_w8a8_gemm_i32(const int8_t* a, const int8_t* b, int32_t* out, int64_t M, int64_t N, int64_t K,
                                void* stream) {
  return qv::w8a8_run(a, b, nullptr, nullptr, nullptr, nullptr, out, M, N, K, 2, stream);
}

extern "C" int64_t qv_w8a8_packed_bytes(int64_t N, int64_t K) {
  return N > 0 && K > 0 ? (N + 31) / 32 * 32 * K : 0;
}

extern "C" int qv_w8a8_pack_weight(const int8_t* w, int8_t* packed, int64_t N, int64_t K, void* stream) {
  QV_CHECK_ARG(N > 0 && K > 0 && K % 64 == 0 && N % 16 == 0,
               "bad weight shape N=%lld K=%lld (K a multiple of 64, N of 16)", (long long)N, (long long)K);
  QV_CHECK_ARG((uint64_t)((N + 31) & ~31) * K < (1ull << 32), "weight too large for 32-bit offsets");
  QV_CHECK_ARG(w && packed, "null pointer argument");
  QV_CHECK_ARG(((uintptr_t)w % 16) == 0 && ((uintptr_t)packed % 16) == 0, "w and packed must be 16-byte aligned");
  const long nchunks = (long)((N + 31) / 32) * (K / 64) * 2 * 64;
  hipLaunchKernelGGL(qv::w8a8_pack_kernel, dim3((unsigned)((nchunks + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, w, packed, (int)N, (int)K, nchunks);
  return qv::check_launch("w8a8_pack_weight");
}

extern "C" int qv_w8a8_gemm_packed(const int8_t* a, const int8_t* packed_b, const void* wscales,
                                   const void* ascales, const void* bias, const void* gamma, void* out, int64_t M,
                                   int64_t N, int64_t K, void* stream) {
  return qv::w8a8_run(a, packed_b, wscales, ascales, bias, gamma, out, M, N, K, gamma ? 3 : (bias ? 1 : 0), stream,
                      true);
}
