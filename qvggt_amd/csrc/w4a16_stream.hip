// Streamed W4A16 group-128 GEMM for gfx950 (the large-M path).
//
// Workgroup tile BM (= 32*MT, m) x 256 (n); the 4 waves sit side by side
// along n, each owning BM x 64 = MT x 2 tiles of v_mfma_f32_32x32x16 (so every
// dequantised weight fragment feeds MT MFMAs of 32x32x16).  The activations,
// which all four waves read, stream global -> LDS with direct buffer loads
// (no register staging) through 3 stages of 64 k: BM rows x 128 B, 16-byte
// chunk c of row r stored at c ^ fA(r), fA(r) = (r & 7) ^ ((r >> 3) & 1), which
// makes every 8-lane and every 16-lane group of a b128 read hit distinct banks
// while each 1 KB direct write stays contiguous.  The packed weights and the
// group scales / scaled zeros of a wave's own 64 channels go straight to its
// registers with ordinary buffer loads one stage ahead: no other wave reads
// them, and routing them through LDS cost more than its share (the direct
// LDS writes of a stage contend with the fragment reads).
//
// K-slots: MFMA operand lanes split as h = lane/32 (k-half) and l = lane%32.
// In k-step s (0..3) of a stage, lane half h takes 32-k chunk h and nibble
// pair s of its four words, i.e. stage-local k = 32*h + 8*s + slot on BOTH
// operands (activations: 8 contiguous halves of chunk 4h + s).  Output: lane
// (h, l), register r holds out[m = l][n = 8*(r/4) + 4*h + r%4] of the tile.
// LDS per workgroup: max(3 stages x BM*128, the epilogue staging of 4 x BM x
// 128 B); BM = 128 -> 64 KB, 2 workgroups/CU.  One launch may cover its rows
// in two ranges of different tile heights (StreamPlan): whole rounds of the
// larger tile, then shorter tiles that fill the slots freed first; a tile's
// results do not depend on its height.  The epilogue stages each wave's
// BM x 64 output tile there and writes it back as whole 128-byte rows, with
// non-temporal stores: the output (90 MB for an MLP linear at 43 k tokens)
// would otherwise evict the weight matrix and the activation rows that the
// other tiles of the XCD still read from its L2 (fc1 at M = 10992: HBM reads
// 94.7 -> 43.0 MB per launch).
#include <type_traits>

#include "w4a16_common.h"

namespace qv {

constexpr int EP = 128;  // bytes per staged epilogue row (64 fp16, chunk-swizzled: stg_off)

// Main loop of one tile over its 64-k stages [k0, k1): acc += the tile's
// products (acc is not cleared here).  Returns with every load landed.
// MID: the k-step of a stage after which the stage's weight requests (for
// the stage two ahead) are issued; -1 issues them at the stage top.  ADMA
// likewise for the activation copy of the stage two ahead (ADMA <= MID: the
// copy precedes the weight requests).
template <bool BF16, int MT, int SUB = 1, int MID = -1, int ADMA = -1>
__device__ __forceinline__ void stream_mainloop(uint8_t* __restrict__ lds, const uint16_t* __restrict__ x,
                                                const uint32_t* __restrict__ qw,
                                                const uint16_t* __restrict__ scales,
                                                const uint16_t* __restrict__ zeros, int M, int N, int K, int m0,
                                                int n0, int k0, int k1, f32x16 (&acc)[2][MT]) {
  constexpr int BM = 32 * MT, NT = 2;
  constexpr int A_BYTES = BM * 128;
  constexpr int STAGE = SUB * A_BYTES;
  // VMEM instructions of one stage's weight loads (load_b), and the wait at a
  // stage's end that leaves exactly those of the stage two ahead in flight
  constexpr int W_OPS = SUB * NT;
  constexpr int SCL = 3 * STAGE;   // the stages' scale / zero rows: 3 x 1 KB after the activation stages
  static_assert(W_OPS < 16, "vmcnt immediate");
  constexpr int WAIT_NEXT = 0x0F70 | W_OPS;
  constexpr int A_INSTR = BM / 32;                // 1 KB direct loads per wave for A
  static_assert(SUB * A_INSTR < 16, "vmcnt immediate");
  static_assert(SUB == 1 || SUB == 2, "64- or 128-k stages");

  // threadIdx.x through an empty asm: the lane-dependent addresses below are
  // then computed here, not hoisted out of a caller's loop over tiles and
  // kept live across it (in a kernel that loops over tiles, that hoisting
  // made the accumulators spill).  The index within the 4-wave group: the
  // K-split kernel runs two such groups in one workgroup.
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  tid &= 255;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int h = lane >> 5, l32 = lane & 31;
  const int K2 = K * 2;

  const auto rsA = make_rsrc(x + (size_t)m0 * K, (uint64_t)(M - m0) * K2);
  const auto rsB = make_rsrc(qw + (size_t)(n0 >> 2) * (K >> 1), (uint64_t)((N - n0) >> 2) * K2);
  const auto rsS = make_rsrc(scales + n0, ((uint64_t)(K >> 7) * N - n0) * 2);
  const auto rsZ = make_rsrc(zeros + n0, ((uint64_t)(K >> 7) * N - n0) * 2);

  // A: instruction q covers rows r0 = 8*(A_INSTR*wave + q) .. +7; lane L lands
  // at row r0 + L/8, physical chunk L%8 and so fetches logical chunk
  // (L%8) ^ fA(row) = (L%8) ^ (L/8) ^ ((r0 >> 3) & 1).
  uint32_t a_voff[2];
#pragma unroll
  for (int v = 0; v < 2; ++v)
    a_voff[v] = (uint32_t)((lane >> 3) * K2 + (((lane & 7) ^ (lane >> 3) ^ v) * 16));
  // B: lane (h, l) of channel block j loads 32-k chunk h of channel
  // n = 64*wave + 32*j + l, i.e. bytes 32*(n&3) + 16*h of the stage's 128-byte
  // segment of packed row n/4 (one 1 KB instruction covers 8 whole segments);
  // S / Z: the 32-bit word holding the channel's 16-bit scale (scaled zero)
  // of the stage's group and its even / odd neighbour's; dq_frag_w picks the
  // half.  The workgroup's 256-channel row of each table comes with the
  // stage's activation copy (one 256-byte LDS DMA per wave) into a 3 x 1 KB
  // ring after the stages, and each lane reads its two words from there:
  // the per-lane 32-bit global loads this replaces (which measured 0.2-2 %
  // faster than 16-bit ones) cost 0-2 % on the multi-round shapes and 2-7 %
  // on one-round ones (1374 x 4096 -> 1024 24.95 -> 23.43 us, proj at
  // M = 10992 25.3 -> 24.8 us; same box, bit-identical).
  uint32_t b_voff[NT], sz_voff[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int n = 64 * wave + 32 * j + l32;
    b_voff[j] = (uint32_t)((n >> 2) * K2 + 32 * (n & 3) + 16 * h);
    sz_voff[j] = (uint32_t)((n & ~1) * 2);   // byte offset of the channel's word in a 512-byte row
  }
  auto load_b = [&](int ks, uint4 (&wq)[SUB][NT]) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
#pragma unroll
      for (int u = 0; u < SUB; ++u)
        wq[u][j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsB, b_voff[j], (SUB * ks + u) * 128, 0));
    }
  };

  const uint32_t lds0 = lds_addr(lds);
  auto issue = [&](int ks, int st) {
#pragma unroll
    for (int u = 0; u < SUB; ++u) {
      const uint32_t base = lds0 + st * STAGE + u * A_BYTES;
#pragma unroll
      for (int q = 0; q < A_INSTR; ++q) {
        const int r0 = 8 * (A_INSTR * wave + q);
        lds_dma16(rsA, a_voff[(r0 >> 3) & 1], r0 * K2 + (SUB * ks + u) * 128, base + r0 * 128);
      }
    }
    // the stage's group row of the workgroup's 256 scales (waves 0, 1) and
    // scaled zeros (waves 2, 3), 256 bytes per wave, into ring entry st
    lds_dma4(wave < 2 ? rsS : rsZ, (uint32_t)((64 * (wave & 1) + lane) * 4), (uint32_t)(((SUB * ks) >> 1) * N * 2),
             lds0 + SCL + st * 1024 + wave * 256);
  };
  auto read_s = [&](int st, uint32_t (&sv)[NT], uint32_t (&zv)[NT]) {
    const uint8_t* base = lds + SCL + st * 1024;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      sv[j] = *reinterpret_cast<const uint32_t*>(base + sz_voff[j]);
      zv[j] = *reinterpret_cast<const uint32_t*>(base + 512 + sz_voff[j]);
    }
  };

  const int fa = (l32 & 7) ^ ((l32 >> 3) & 1);  // fA(32*i + l32) is the same for all i

  // the lane's channel is odd (high half of the loaded word) iff l32 is
  const uint32_t sz_sel = (l32 & 1) ? 0x03020302u : 0x01000100u;
  auto dq = [&](int s, const uint4 (&wq)[NT], const uint32_t (&sv)[NT], const uint32_t (&zv)[NT], uint4 (&wf)[NT]) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      switch (s) {
        case 0: wf[j] = dq_frag_w<BF16, 0>(wq[j], sv[j], zv[j], sz_sel); break;
        case 1: wf[j] = dq_frag_w<BF16, 1>(wq[j], sv[j], zv[j], sz_sel); break;
        case 2: wf[j] = dq_frag_w<BF16, 2>(wq[j], sv[j], zv[j], sz_sel); break;
        default: wf[j] = dq_frag_w<BF16, 3>(wq[j], sv[j], zv[j], sz_sel); break;
      }
    }
  };
  // activation fragments of k-step s of 64-k half u of the stage in LDS buffer st
  auto read_a = [&](int st, int u, int s, uint4 (&af)[MT]) {
    const uint8_t* base = lds + st * STAGE + u * A_BYTES;
    const uint32_t col = (uint32_t)(((4 * h + s) ^ fa) * 16);
#pragma unroll
    for (int i = 0; i < MT; ++i) af[i] = *reinterpret_cast<const uint4*>(base + (32 * i + l32) * 128 + col);
  };
  // One stage (LDS buffer st, weights wq/sv/zv).  On entry af0 / wf0 hold the
  // stage's k-step 0 fragments; k-step s issues the LDS reads of step s+1's
  // activations, then its own MFMAs, then dequantises step s+1's weights
  // (VALU that co-issues with the MFMAs in flight).  Step 3 does the same for
  // k-step 0 of the NEXT stage (buffer nst, weights nwq/nsv/nzv), so the next
  // stage's first MFMAs do not wait behind its barrier for LDS reads and a
  // dequantisation; af0 / wf0 hold those fragments on exit.  The scheduling
  // fences keep the compiler from sinking the reads next to their use.
  auto compute = [&](int st, int nst, const uint4 (&wq)[SUB][NT], const uint32_t (&sv)[NT], const uint32_t (&zv)[NT],
                     const uint4 (&nwq)[SUB][NT], uint32_t (&nsv)[NT], uint32_t (&nzv)[NT], uint4 (&af0)[MT],
                     uint4 (&wf0)[NT], auto&& mid, auto&& mida) {
    constexpr int T = 4 * SUB;   // k-steps per stage
    static_assert(MID < T - 1 && ADMA <= MID, "the activation copy, then the weight requests, before the last k-step");
    uint4 af[2][MT], wf[2][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i) af[0][i] = af0[i];
#pragma unroll
    for (int j = 0; j < NT; ++j) wf[0][j] = wf0[j];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if (t < T - 1) {
        read_a(st, (t + 1) >> 2, (t + 1) & 3, af[(t + 1) & 1]);
      } else {
        read_a(nst, 0, 0, af[0]);
        read_s(nst, nsv, nzv);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[j][i] = mfma32<BF16>(wf[t & 1][j], af[t & 1][i], acc[j][i]);
      }
      if (t < T - 1) {
        dq((t + 1) & 3, wq[(t + 1) >> 2], sv, zv, wf[(t + 1) & 1]);
        if (t == ADMA) mida();
        if (t == MID) mid();
      } else {
        // the next stage's weights and every copy issued before this
        // stage's own weight loads have landed
        __builtin_amdgcn_s_waitcnt(WAIT_NEXT);
        dq(0, nwq[0], nsv, nzv, wf[0]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) af0[i] = af[0][i];
#pragma unroll
    for (int j = 0; j < NT; ++j) wf0[j] = wf[0][j];
  };

  // Stage i = ks - k0 uses LDS buffer i % 3 and weight register set i % 3.
  // Per stage: barrier (every wave is done reading buffer (i + 2) % 3, the
  // previous stage's, and sees A(ks + 1)), the copy of A(ks + 2) into that
  // buffer, the weight loads B(ks + 2) into register set (i + 2) % 3, then
  // the stage's compute, whose last step waits for every load but those of
  // B(ks + 2) (vmcnt(W_OPS): A(ks + 2) and B(ks + 1) have landed) and reads
  // stage ks + 1's first fragments -- A(ks + 1) landed at the same point of
  // the previous stage, before the barrier that published it.  So a stage's
  // weights are requested about two stages before their first use, where
  // one stage (two register sets) left their latency exposed: fc1 at
  // M = 10992 95.7 -> 92.6 us, qkv 67.2 -> 65.6 us, config-1 qkv 14.2 ->
  // 13.6 us, the K split at 1374 x 4096 -> 1024 26.9 -> 25.1 us (same box,
  // bit-identical).  The A copies are inline asm the compiler does not
  // count; its own waits for B(ks + 1), by its count of weight loads alone,
  // are no later than that vmcnt(W_OPS).  Three stages run per iteration, so
  // every register-set index is a constant; a remainder of one or two stages
  // runs after the loop.  Loads past k1 - 1 repeat stage k1 - 1 (valid
  // addresses; A into a buffer nobody reads, B into a dead register set), so
  // every stage issues the same count.
  uint4 wq[3][SUB][NT];
  uint32_t sv[3][NT], zv[3][NT];   // scale / zero words, read from the ring
  uint4 af0[MT], wf0[NT];
  // stage indices in units of SUB x 64 k
  const int L0 = k0 / SUB, L1 = k1 / SUB;
  const int last = L1 - 1, nks = L1 - L0;
  issue(L0, 0);
  issue(L0 + 1 < L1 ? L0 + 1 : last, 1);
  load_b(L0, wq[0]);
  load_b(L0 + 1 < L1 ? L0 + 1 : last, wq[1]);
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): A(k0), A(k0 + 1), B(k0), B(k0 + 1)
  lds_barrier();
  read_a(0, 0, 0, af0);
  read_s(0, sv[0], zv[0]);
  dq(0, wq[0][0], sv[0], zv[0], wf0);
  auto stage = [&](int s, auto pc) __attribute__((always_inline)) {
    constexpr int p = decltype(pc)::value, p1 = (p + 1) % 3, p2 = (p + 2) % 3;
    lds_barrier();
    const int s2 = s + 2 < L1 ? s + 2 : last;
    auto req_a = [&]() __attribute__((always_inline)) { issue(s2, p2); };
    if constexpr (ADMA < 0) req_a();
    auto req_b = [&]() __attribute__((always_inline)) { load_b(s2, wq[p2]); };
    if constexpr (MID < 0) req_b();
    compute(p, p1, wq[p], sv[p], zv[p], wq[p1], sv[p1], zv[p1], af0, wf0, req_b, req_a);
  };
  int i = 0;
  for (; i + 3 <= nks; i += 3) {
    stage(L0 + i, std::integral_constant<int, 0>());
    stage(L0 + i + 1, std::integral_constant<int, 1>());
    stage(L0 + i + 2, std::integral_constant<int, 2>());
  }
  if (i < nks) stage(L0 + i, std::integral_constant<int, 0>());
  if (i + 1 < nks) stage(L0 + i + 1, std::integral_constant<int, 1>());
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the repeated loads may not land during the epilogue
}

// Epilogue of one tile: the wave's BM x 64 output tile goes through LDS so
// that the global stores are whole 128-byte rows (direct 8-byte stores from
// the MFMA layout cost ~3x the output size in HBM write traffic).  Starts
// with a workgroup barrier (every wave is done reading the pipeline stages).
// BIAS_IN_ACC: the accumulators already hold the bias (init_acc); the
// epilogue then adds none.
template <bool BF16, int MT, int EPI, bool BIAS_IN_ACC = false>
__device__ __forceinline__ void stream_epilogue(uint8_t* __restrict__ lds, const uint16_t* __restrict__ bias,
                                                const uint16_t* __restrict__ gamma, uint16_t* __restrict__ out,
                                                int M, int N, const QkRopeArgs& qk, int m0, int n0,
                                                const f32x16 (&acc)[2][MT]) {
  constexpr int BM = 32 * MT, NT = 2;
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));  // as in stream_mainloop
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;
  // the bias values of the wave's columns, all requested before the barrier
  // (each of the NT x 4 column groups waited for its own load otherwise)
  uint2 bv[NT][4];
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n0 + 64 * wave + 32 * j + 8 * q + 4 * h;
      bv[j][q] = epi_has_bias<EPI>() && !BIAS_IN_ACC ? *reinterpret_cast<const uint2*>(bias + (n < N ? n : 0))
                                                     : make_uint2(0, 0);
    }
  // q/k RoPE: the token positions of the lane's MT rows, likewise early (the
  // cos / sin reads depend on them)
  int2 ppv[EPI == QV_EPI_QKROPE ? MT : 1];
  if constexpr (EPI == QV_EPI_QKROPE) {
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int m = m0 + 32 * i + l32;
      ppv[i] = *reinterpret_cast<const int2*>(qk.pos + 2 * (m < M ? m : M - 1));
    }
  }
  lds_barrier();
  uint8_t* stg = lds + wave * (BM * EP);
  bool staged = false;
  if constexpr (EPI == QV_EPI_QKROPE && !BF16) {
    // The wave's 64 columns are one head.  For a q or k head, per output row
    // (token): y = fp16(acc + bias); per-head LayerNorm over the 64 values
    // (each lane holds 32 of them, the other 32 sit in lane ^ 32), rounded
    // to fp16; then the 2-D RoPE of rope2d_kernel: columns [0, 32) rotate
    // with the token's y position, [32, 64) with its x position, and the
    // pair (d, d + 16) of a half is registers q and q + 2 of one lane.
    const int nw = n0 + 64 * wave;
    if (nw < qk.qk_cols) {
      staged = true;
      const bool is_k = nw >= (qk.qk_cols >> 1);
      const uint16_t* gp = is_k ? qk.kg : qk.qg;
      const uint16_t* bp = is_k ? qk.kb : qk.qb;
      // the head's norm weights for the lane's 32 columns, read once for all
      // MT row blocks (the main loop's registers are free by now)
      uint2 gv[NT][4], bev[NT][4];
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int dl = 32 * j + 8 * q + 4 * h;
          gv[j][q] = *reinterpret_cast<const uint2*>(gp + dl);
          bev[j][q] = *reinterpret_cast<const uint2*>(bp + dl);
        }
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        uint32_t yw[NT][4][2];
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint2 b2 = bv[j][q];
            yw[j][q][0] = pack2<false>(mix_add<0>(b2.x, acc[j][i][4 * q]), mix_add<1>(b2.x, acc[j][i][4 * q + 1]));
            yw[j][q][1] = pack2<false>(mix_add<0>(b2.y, acc[j][i][4 * q + 2]), mix_add<1>(b2.y, acc[j][i][4 * q + 3]));
#pragma unroll
            for (int w = 0; w < 2; ++w) {
              sum = mix_add<0>(yw[j][q][w], sum);
              sum = mix_add<1>(yw[j][q][w], sum);
            }
          }
        float pa, pb;
        pair32(sum, pa, pb);
        const float nm = -((pa + pb) * (1.0f / 64.0f));
        float d[NT][4][4];
        float s2 = 0.f;
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int w = 0; w < 2; ++w) {
              d[j][q][2 * w] = mix_add<0>(yw[j][q][w], nm);
              d[j][q][2 * w + 1] = mix_add<1>(yw[j][q][w], nm);
              s2 = s2 + d[j][q][2 * w] * d[j][q][2 * w];
              s2 = s2 + d[j][q][2 * w + 1] * d[j][q][2 * w + 1];
            }
        pair32(s2, pa, pb);
        const float rs = 1.0f / __builtin_sqrtf((pa + pb) * (1.0f / 64.0f) + qk.eps);
        const int2 pp = ppv[i];
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          int p = j == 0 ? pp.x : pp.y;
          p = p < 0 ? 0 : (p >= qk.P ? qk.P - 1 : p);
          uint32_t zw[4][2];   // LayerNorm output of this half, rounded to fp16
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t gw[2] = {gv[j][q].x, gv[j][q].y}, bw[2] = {bev[j][q].x, bev[j][q].y};
#pragma unroll
            for (int w = 0; w < 2; ++w)
              zw[q][w] = pack2<false>(mix_add<0>(bw[w], mix_mul<0>(d[j][q][2 * w] * rs, gw[w])),
                                      mix_add<1>(bw[w], mix_mul<1>(d[j][q][2 * w + 1] * rs, gw[w])));
          }
#pragma unroll
          for (int qq = 0; qq < 2; ++qq) {
            // frequencies 8 qq + 4 h + e (e = 0..3) of this half, shared by the pair (qq, qq + 2)
            const float4 c4 = *reinterpret_cast<const float4*>(qk.cos_t + p * 16 + 8 * qq + 4 * h);
            const float4 s4 = *reinterpret_cast<const float4*>(qk.sin_t + p * 16 + 8 * qq + 4 * h);
            const float cs[4] = {c4.x, c4.y, c4.z, c4.w}, sn[4] = {s4.x, s4.y, s4.z, s4.w};
            uint32_t o1[2], o2[2];
#pragma unroll
            for (int w = 0; w < 2; ++w) {
              const uint32_t a = zw[qq][w], b = zw[qq + 2][w];
              // first of the pair: a c - b s; second: b c + a s
              o1[w] = pack2<false>(mix_mul<0>(cs[2 * w], a) - mix_mul<0>(sn[2 * w], b),
                                   mix_mul<1>(cs[2 * w + 1], a) - mix_mul<1>(sn[2 * w + 1], b));
              o2[w] = pack2<false>(mix_mul<0>(cs[2 * w], b) + mix_mul<0>(sn[2 * w], a),
                                   mix_mul<1>(cs[2 * w + 1], b) + mix_mul<1>(sn[2 * w + 1], a));
            }
            *reinterpret_cast<uint2*>(stg + stg_off(32 * i + l32, (32 * j + 8 * qq + 4 * h) * 2)) =
                make_uint2(o1[0], o1[1]);
            *reinterpret_cast<uint2*>(stg + stg_off(32 * i + l32, (32 * j + 8 * (qq + 2) + 4 * h) * 2)) =
                make_uint2(o2[0], o2[1]);
          }
        }
      }
    }
  }
  if (!staged) {
#pragma unroll
  for (int j = 0; j < NT; ++j) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int nl = 32 * j + 8 * q + 4 * h;
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        float r[4] = {acc[j][i][4 * q], acc[j][i][4 * q + 1], acc[j][i][4 * q + 2], acc[j][i][4 * q + 3]};
        // with the bias in the accumulators only the GELU (if any) is left
        constexpr int AEPI = !BIAS_IN_ACC ? EPI
                                          : (EPI == QV_EPI_BIAS_GELU || EPI == QV_EPI_GELU ? QV_EPI_GELU : QV_EPI_NONE);
        epilogue_apply4v<BF16, AEPI>(bv[j][q], r);
        uint2 o;
        o.x = pack2<BF16>(r[0], r[1]);
        o.y = pack2<BF16>(r[2], r[3]);
        *reinterpret_cast<uint2*>(stg + stg_off(32 * i + l32, nl * 2)) = o;
      }
    }
  }
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's staging writes are done
  __builtin_amdgcn_wave_barrier();
  // Write-back: iteration it moves row (it * 64 + lane) / 8 of the wave's
  // tile, 16-byte chunk lane % 8 -- the same 8 columns in every iteration.
  constexpr int IT = BM * 8 / 64;
  const int c = lane & 7;
  const int n = n0 + 64 * wave + 8 * c;
  if constexpr (EPI == QV_EPI_BIAS_RESID) {
    // The residual rows are read in place of the output; every read is
    // issued before the first store (the compiler cannot move a read of
    // `out` past a store to it, and in the loop below each read waited for
    // the previous iteration's store: IT serial memory latencies), and
    // gamma, the same in every iteration, is read once.
    const uint4 gv = n < N ? *reinterpret_cast<const uint4*>(gamma + n) : make_uint4(0, 0, 0, 0);
    uint4 rv[IT];
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int m = m0 + ((it * 64 + lane) >> 3);
      rv[it] = m < M && n < N ? *reinterpret_cast<const uint4*>(out + (size_t)m * N + n) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int row = (it * 64 + lane) >> 3;
      const int m = m0 + row;
      if (m < M && n < N)
        st_stream16(out + (size_t)m * N + n,
                    resid_update8<BF16>(rv[it], *reinterpret_cast<const uint4*>(stg + stg_off(row, c * 16)), gv));
    }
  } else {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int row = (it * 64 + lane) >> 3;
      const int m = m0 + row;
      if (m < M && n < N) st_stream16(out + (size_t)m * N + n, *reinterpret_cast<const uint4*>(stg + stg_off(row, c * 16)));
    }
  }
}

// One whole tile: logical tile lid of the rows from m_base.
// Every epilogue with a bias folds it into the accumulators' start value
// (fp32), so the epilogue adds none: the bias enters the fp32 sum first
// instead of last (the same rounding count; 1-2 % faster on the MLP and qkv
// shapes, e.g. qkv at M = 10992 66.8 -> 65.2 us, fc1 97.3 -> 96.3 us,
// config 1 12.35 -> 12.12 us, same box).  All of them fold, so a fused
// epilogue (residual, q/k RoPE) sees the same linear output as the bias-only
// one it replaces.
// acc = the lane's bias values (with_bias) or zero; lane (h, l) of wave w
// holds channels n0 + 64 w + 32 j + 8 (r / 4) + 4 h + r % 4 in register r of
// acc[j][*].
template <bool BF16, int MT>
__device__ __forceinline__ void init_acc(f32x16 (&acc)[2][MT], const uint16_t* __restrict__ bias, int N, int n0,
                                         bool with_bias) {
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));  // as in stream_mainloop
  tid &= 255;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), h = (tid & 63) >> 5;
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n0 + 64 * wave + 32 * j + 8 * q + 4 * h;
      const uint2 b2 = with_bias && n < N ? *reinterpret_cast<const uint2*>(bias + n) : make_uint2(0, 0);
      const float bf[4] = {to_f32((uint16_t)(b2.x & 0xFFFF), BF16), to_f32((uint16_t)(b2.x >> 16), BF16),
                           to_f32((uint16_t)(b2.y & 0xFFFF), BF16), to_f32((uint16_t)(b2.y >> 16), BF16)};
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[j][i][4 * q + e] = bf[e];
    }
}

template <bool BF16, int MT, int EPI, int SUB = 1, int MID = -1, int ADMA = -1>
__device__ __forceinline__ void stream_tile(uint8_t* __restrict__ lds, const uint16_t* __restrict__ x,
                                            const uint32_t* __restrict__ qw, const uint16_t* __restrict__ scales,
                                            const uint16_t* __restrict__ zeros, const uint16_t* __restrict__ bias,
                                            const uint16_t* __restrict__ gamma, uint16_t* __restrict__ out, int M,
                                            int N, int K, int tiles_n, const QkRopeArgs& qk, int lid, int m_base) {
  const int m0 = m_base + (lid / tiles_n) * (32 * MT);
  const int n0 = (lid % tiles_n) * 256;
  f32x16 acc[2][MT];
  if constexpr (epi_has_bias<EPI>()) {
    init_acc<BF16, MT>(acc, bias, N, n0, true);
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.f;
  }
  stream_mainloop<BF16, MT, SUB, MID, ADMA>(lds, x, qw, scales, zeros, M, N, K, m0, n0, 0, K >> 6, acc);
  stream_epilogue<BF16, MT, EPI, epi_has_bias<EPI>()>(lds, bias, gamma, out, M, N, qk, m0, n0, acc);
}

// One launch over two row ranges: blocks [0, n_first) take 32*MT-row tiles of
// rows [0, m_split), the rest 32*MT2-row tiles of rows [m_split, M) (MT2 = 0:
// one range).  Each range maps its blocks to tiles on its own (xcd_remap of
// the block's index within the range).
template <bool BF16, int MT, int MT2, int EPI, int SUB = 1>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void w4a16_stream32_kernel(const uint16_t* __restrict__ x, const uint32_t* __restrict__ qw,
                           const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
                           const uint16_t* __restrict__ bias, const uint16_t* __restrict__ gamma,
                           uint16_t* __restrict__ out, int M, int N, int K, int tiles_n, QkRopeArgs qk,
                           int n_first, int m_split) {
  constexpr int MTX = MT > MT2 ? MT : MT2;
  // max(3 stages + their 3 KB scale / zero ring, the epilogue staging)
  constexpr int LDS_B = (SUB == 2 ? 6 : 4) * 32 * MTX * 128 > 3 * SUB * 32 * MTX * 128 + 3072
                            ? (SUB == 2 ? 6 : 4) * 32 * MTX * 128
                            : 3 * SUB * 32 * MTX * 128 + 3072;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_B];
  // Weight requests after a stage's second k-step (1.5 stages ahead of use)
  // measured 1-4 % faster than at the stage top for 96- and 128-row tiles and
  // the one-round 128-k stages (fc1 at M = 10992 99.2 -> 97.9 us, config-1
  // qkv 13.6 -> 13.1 us, M = 43968 fc1 392.7 -> 382.6 us), but 1-4 % slower
  // in launches with 64-row 64-k tiles (fc2 at M = 10992, 128- then 64-row
  // tiles: 85.5 -> 87.1 us; 8244 x 4096 -> 1024 71.7 -> 74.9 us), whose
  // stages are half as long; those keep the requests at the stage top.
  constexpr int MID = (MT2 == 2 || (MT <= 2 && SUB == 1)) ? -1 : 1;
  // The activation copy after the first k-step instead of at the stage top
  // (0.75 of a stage ahead of use): 1-4 % faster for one-round 128-k stages
  // (2748 x 1024 -> 1024 11.0 -> 10.6 us, 1000 x 1024 -> 3072 10.8 -> 10.6
  // us; config-1 qkv +2.5 % and +0.1 % in two runs) and one-range 96-row
  // tiles (proj at M = 10992 +0.6-2 %), within 1 % for 128-row tiles, 2-7 %
  // slower with 64-row 64-k tiles.
  constexpr int ADMA = (SUB == 2 || (MT2 == 0 && MT == 3)) ? 0 : -1;
  const int b = blockIdx.x;
  if (MT2 == 0 || b < n_first) {
    stream_tile<BF16, MT, EPI, SUB, MID, ADMA>(lds, x, qw, scales, zeros, bias, gamma, out, M, N, K, tiles_n, qk,
                               xcd_remap(b, MT2 == 0 ? (int)gridDim.x : n_first), 0);
  } else {
    stream_tile<BF16, (MT2 > 0 ? MT2 : 1), EPI, 1, MID, ADMA>(lds, x, qw, scales, zeros, bias, gamma, out, M, N, K, tiles_n, qk,
                                                xcd_remap(b - n_first, (int)gridDim.x - n_first), m_split);
  }
}

// K split inside the workgroup, for launches of at most one tile per CU
// (where the 4-wave kernel runs one wave per SIMD and nothing hides a wave's
// own LDS, dequantisation and barrier latencies behind another's MFMAs).
// Eight waves: group g = wave / 4 runs the main loop of the 4-wave kernel
// over stages [g K/128, (g + 1) K/128) in its own three LDS stage buffers, so
// each SIMD holds one wave of each group.  Then group 1 hands its fp32
// partial sums to group 0 through LDS (one 16-byte slot per lane and
// register quad: contiguous 1 KB per wave instruction), group 0 adds them
// (its own first-half sum + the second half's) and runs the epilogue of the
// 4-wave kernel.  Both groups run the same number of stages, so every
// per-stage barrier of the main loop is reached by all eight waves; group 1
// also takes part in the epilogue's opening barrier, after which it is done.
template <int MT>
constexpr int ksplit_lds_bytes() {
  constexpr int stages = 2 * (3 * 32 * MT * 128 + 3072), part = 32 * MT * 256 * 4, stage_out = 4 * 32 * MT * EP;
  return stages > part ? (stages > stage_out ? stages : stage_out) : (part > stage_out ? part : stage_out);
}

template <bool BF16, int MT, int EPI>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void w4a16_ksplit_kernel(const uint16_t* __restrict__ x, const uint32_t* __restrict__ qw,
                         const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
                         const uint16_t* __restrict__ bias, const uint16_t* __restrict__ gamma,
                         uint16_t* __restrict__ out, int M, int N, int K, int tiles_n, QkRopeArgs qk) {
  constexpr int BM = 32 * MT;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[ksplit_lds_bytes<MT>()];
  const int grp = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 8));
  const int lid = xcd_remap(blockIdx.x, (int)gridDim.x);
  const int m0 = (lid / tiles_n) * BM;
  const int n0 = (lid % tiles_n) * 256;
  const int half = K >> 7;   // stages per group (K % 256 == 0: an even count)
  f32x16 acc[2][MT];
  // group 0 starts from the bias where the epilogue folds it (stream_tile)
  init_acc<BF16, MT>(acc, bias, N, n0, epi_has_bias<EPI>() && grp == 0);
  // weight requests after each stage's second k-step and the activation copy
  // after its first (as in stream_tile; measured faster for every tile height
  // here: 1374 x 4096 -> 1024 24.8 -> 23.6 -> 23.6 us, 2748 x 4096 -> 1024
  // 31.2 -> 30.2 -> 29.4 us)
  stream_mainloop<BF16, MT, 1, 1, 0>(lds + grp * (3 * BM * 128 + 3072), x, qw, scales, zeros, M, N, K, m0, n0, grp * half,
                            (grp + 1) * half, acc);
  // every wave is done reading its group's stage buffers
  lds_barrier();
  const int lane = threadIdx.x & 63;
  const int wv = (threadIdx.x >> 6) & 3;
  float4* part = reinterpret_cast<float4*>(lds) + (wv * (2 * MT * 4)) * 64 + lane;
  if (grp == 1) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          part[((j * MT + i) * 4 + q) * 64] =
              make_float4(acc[j][i][4 * q], acc[j][i][4 * q + 1], acc[j][i][4 * q + 2], acc[j][i][4 * q + 3]);
  }
  lds_barrier();
  if (grp == 0) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float4 p = part[((j * MT + i) * 4 + q) * 64];
          acc[j][i][4 * q] += p.x;
          acc[j][i][4 * q + 1] += p.y;
          acc[j][i][4 * q + 2] += p.z;
          acc[j][i][4 * q + 3] += p.w;
        }
    // its opening barrier (matched by group 1 below) also orders these
    // reads before the staging writes that reuse the same LDS
    stream_epilogue<BF16, MT, EPI, epi_has_bias<EPI>()>(lds, bias, gamma, out, M, N, qk, m0, n0, acc);
  } else {
    lds_barrier();
  }
}

template <bool BF16, int MT>
static void launch_ksplit(const void* x, const void* qw, const void* s, const void* z, const void* bias,
                          const void* gamma, void* out, int M, int N, int K, int epi, hipStream_t st,
                          const QkRopeArgs& qk) {
  const int tiles_n = (N + 255) / 256;
  const dim3 grid((M + 32 * MT - 1) / (32 * MT) * tiles_n), block(512);
#define QV_ARGS                                                                                \
  (const uint16_t*)x, (const uint32_t*)qw, (const uint16_t*)s, (const uint16_t*)z,             \
      (const uint16_t*)bias, (const uint16_t*)gamma, (uint16_t*)out, M, N, K, tiles_n, qk
  switch (epi) {
    case QV_EPI_NONE:
      hipLaunchKernelGGL((w4a16_ksplit_kernel<BF16, MT, QV_EPI_NONE>), grid, block, 0, st, QV_ARGS);
      break;
    case QV_EPI_BIAS:
      hipLaunchKernelGGL((w4a16_ksplit_kernel<BF16, MT, QV_EPI_BIAS>), grid, block, 0, st, QV_ARGS);
      break;
    case QV_EPI_BIAS_GELU:
      hipLaunchKernelGGL((w4a16_ksplit_kernel<BF16, MT, QV_EPI_BIAS_GELU>), grid, block, 0, st, QV_ARGS);
      break;
    case QV_EPI_GELU:
      hipLaunchKernelGGL((w4a16_ksplit_kernel<BF16, MT, QV_EPI_GELU>), grid, block, 0, st, QV_ARGS);
      break;
    case QV_EPI_QKROPE:
      if constexpr (!BF16) hipLaunchKernelGGL((w4a16_ksplit_kernel<BF16, MT, QV_EPI_QKROPE>), grid, block, 0, st, QV_ARGS);
      break;
    default:
      hipLaunchKernelGGL((w4a16_ksplit_kernel<BF16, MT, QV_EPI_BIAS_RESID>), grid, block, 0, st, QV_ARGS);
      break;
  }
#undef QV_ARGS
}

template <bool BF16, int MT, int MT2 = 0, int SUB = 1>
static void launch_mt(const void* x, const void* qw, const void* s, const void* z, const void* bias,
                      const void* gamma, void* out, int M, int N, int K, int epi, hipStream_t st,
                      const QkRopeArgs& qk, int m_split = 0) {
  const int tiles_n = (N + 255) / 256;
  const int rows1 = MT2 ? m_split : M;
  const int n_first = (rows1 + 32 * MT - 1) / (32 * MT) * tiles_n;
  const int n_second = MT2 ? (M - m_split + 32 * MT2 - 1) / (32 * MT2) * tiles_n : 0;
  const dim3 grid(n_first + n_second), block(256);
#define QV_ARGS                                                                                \
  (const uint16_t*)x, (const uint32_t*)qw, (const uint16_t*)s, (const uint16_t*)z,             \
      (const uint16_t*)bias, (const uint16_t*)gamma, (uint16_t*)out, M, N, K, tiles_n, qk, n_first, m_split
  switch (epi) {
    case QV_EPI_NONE:
      hipLaunchKernelGGL((w4a16_stream32_kernel<BF16, MT, MT2, QV_EPI_NONE, SUB>), grid, block, 0, st, QV_ARGS);
      break;
    case QV_EPI_BIAS:
      hipLaunchKernelGGL((w4a16_stream32_kernel<BF16, MT, MT2, QV_EPI_BIAS, SUB>), grid, block, 0, st, QV_ARGS);
      break;
    case QV_EPI_BIAS_GELU:
      hipLaunchKernelGGL((w4a16_stream32_kernel<BF16, MT, MT2, QV_EPI_BIAS_GELU, SUB>), grid, block, 0, st, QV_ARGS);
      break;
    case QV_EPI_GELU:
      hipLaunchKernelGGL((w4a16_stream32_kernel<BF16, MT, MT2, QV_EPI_GELU, SUB>), grid, block, 0, st, QV_ARGS);
      break;
    case QV_EPI_QKROPE:
      if constexpr (!BF16) hipLaunchKernelGGL((w4a16_stream32_kernel<BF16, MT, MT2, QV_EPI_QKROPE, SUB>), grid, block, 0, st, QV_ARGS);
      break;
    default:
      hipLaunchKernelGGL((w4a16_stream32_kernel<BF16, MT, MT2, QV_EPI_BIAS_RESID, SUB>), grid, block, 0, st, QV_ARGS);
      break;
  }
#undef QV_ARGS
}

template <bool BF16>
int launch_w4a16_stream(const void* x, const void* qw, const void* s, const void* z, const void* bias,
                        const void* gamma, void* out, int M, int N, int K, int epi, const StreamPlan& p,
                        hipStream_t st, const QkRopeArgs* qk) {
  const QkRopeArgs a = qk ? *qk : QkRopeArgs();
  if (p.ksplit) {
    QV_CHECK_ARG(p.mt_b == 0 && K % 256 == 0, "bad tile plan: K split of K=%d", K);
    if (p.mt_a == 4) launch_ksplit<BF16, 4>(x, qw, s, z, bias, gamma, out, M, N, K, epi, st, a);
    else if (p.mt_a == 3) launch_ksplit<BF16, 3>(x, qw, s, z, bias, gamma, out, M, N, K, epi, st, a);
    else if (p.mt_a == 2) launch_ksplit<BF16, 2>(x, qw, s, z, bias, gamma, out, M, N, K, epi, st, a);
    else launch_ksplit<BF16, 1>(x, qw, s, z, bias, gamma, out, M, N, K, epi, st, a);
  } else if (p.mt_b) {
    QV_CHECK_ARG(p.rows_a > 0 && p.rows_a < M && p.rows_a % (32 * p.mt_a) == 0,
                 "bad tile plan: %d rows of %d-row tiles for M=%d", p.rows_a, 32 * p.mt_a, M);
    if (p.mt_a == 4 && p.mt_b == 3) launch_mt<BF16, 4, 3>(x, qw, s, z, bias, gamma, out, M, N, K, epi, st, a, p.rows_a);
    else if (p.mt_a == 4 && p.mt_b == 2) launch_mt<BF16, 4, 2>(x, qw, s, z, bias, gamma, out, M, N, K, epi, st, a, p.rows_a);
    else if (p.mt_a == 3 && p.mt_b == 2) launch_mt<BF16, 3, 2>(x, qw, s, z, bias, gamma, out, M, N, K, epi, st, a, p.rows_a);
    else QV_CHECK_ARG(false, "bad tile plan: tile pair %d/%d", p.mt_a, p.mt_b);
  } else if (p.sub == 2) {
    QV_CHECK_ARG(K % 256 == 0 && (p.mt_a == 2 || p.mt_a == 3),
                 "bad tile plan: 128-k stages need K %% 256 == 0 and 64- or 96-row tiles (K=%d, tile %d)", K,
                 32 * p.mt_a);
    if (p.mt_a == 3) launch_mt<BF16, 3, 0, 2>(x, qw, s, z, bias, gamma, out, M, N, K, epi, st, a);
    else launch_mt<BF16, 2, 0, 2>(x, qw, s, z, bias, gamma, out, M, N, K, epi, st, a);
  } else if (p.mt_a == 4) {
    launch_mt<BF16, 4>(x, qw, s, z, bias, gamma, out, M, N, K, epi, st, a);
  } else if (p.mt_a == 3) {
    launch_mt<BF16, 3>(x, qw, s, z, bias, gamma, out, M, N, K, epi, st, a);
  } else if (p.mt_a == 2) {
    launch_mt<BF16, 2>(x, qw, s, z, bias, gamma, out, M, N, K, epi, st, a);
  } else {
    launch_mt<BF16, 1>(x, qw, s, z, bias, gamma, out, M, N, K, epi, st, a);
  }
  return check_launch("w4a16_stream32");
}

template int launch_w4a16_stream<false>(const void*, const void*, const void*, const void*, const void*,
                                        const void*, void*, int, int, int, int, const StreamPlan&, hipStream_t,
                                        const QkRopeArgs*);
template int launch_w4a16_stream<true>(const void*, const void*, const void*, const void*, const void*,
                                       const void*, void*, int, int, int, int, const StreamPlan&, hipStream_t,
                                       const QkRopeArgs*);

}  // namespace qv
