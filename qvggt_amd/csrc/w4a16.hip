// AWQ W4A16 group-128 dispatcher, skinny-M kernel (the GEMV entry and every
// M <= 64), dequantisation and GPU packing for gfx950.  The AWQ-v2 nibble
// layout and the exact dequantisation are documented in w4a16_common.h; the
// large-M streamed GEMM lives in w4a16_stream.hip.
#include "w4a16_common.h"

#include <map>
#include <mutex>
#include <queue>
#include <tuple>
#include <utility>
#include <vector>

namespace qv {

// ------------------------------------------------- skinny-M MFMA kernel
// For M <= 64: one workgroup per 16 NB output channels whose W waves split
// the 128-k groups round-robin, as in the GEMV,
// but the products run on v_mfma_f32_16x16x32 with the dequantised weights
// as the A operand (row = channel) and up to four 16-token column blocks of
// activations as B, read with buffer loads straight from L2 (tokens >= M
// fall outside the descriptor and read as zero).  Lane (g = lane/16,
// l = lane%16): channel n0 + l; in k-step t of a 128-k group, k-slot s of the
// lane is k = 32g + 8t + s on BOTH operands (activations: 8 contiguous
// halves; weights: nibble pair t of the lane's four words of 32-k chunk g);
// accumulator block mb holds out[m = 16 mb + l][n = n0 + 4g + r], r = 0..3.
// Each weight byte is read once; the activations (M x K, at most 1 MiB at
// K = 8192) stay L2-resident but are re-read by every workgroup, so NB > 1
// (each activation fragment feeding NB channel blocks) cuts that L2 -> CU
// traffic by NB at the cost of NB-fold fewer workgroups.  Wave partials are
// summed through LDS.
//
// Split K (gridDim.y = SK > 1): workgroup (b, ks) takes the 128-k groups
// [ks*KT/SK, (ks+1)*KT/SK) of channel block b, so a launch with few channel
// blocks (e.g. 8192 -> 2048: 128 blocks) still fills the CUs.  Each split
// writes its fp32 partial (M x 16 NB) to workspace slot (b, ks) with
// agent-coherent (sc1) stores, waits for them (vmcnt 0) and bumps block b's
// arrival counter with a wrapping increment (global_atomic_inc with limit
// SK - 1: SK - 1 -> 0), so the split that sees SK - 1 arrives last and the
// same atomic has already returned the counter to zero for the next launch.
// The counters of one SK serve only launches with that SK (cnt points at
// that range), so every launch adds exactly SK increments to each counter it
// touches and leaves it as it found it, even if launches that wrongly share
// a workspace overlap.  The last split reads the SK partials back in ks
// order -- the sum order never depends on arrival order -- and runs the
// epilogue.  No workgroup waits on another.
template <bool BF16, int MB, int NB, bool SPLIT>
__global__ __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(MB * NB == 1 ? 8 : 1))) void w4a16_skinny_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ qw,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    const uint16_t* __restrict__ bias, const uint16_t* __restrict__ gamma, uint16_t* __restrict__ out,
    int M, int N, int K, int epi, float* __restrict__ part, int* __restrict__ cnt) {
  __shared__ f32x4 red[16][MB][64];
  __shared__ int s_arrived;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwaves = blockDim.x >> 6;
  const int g = lane >> 4, li = lane & 15;
  const int n0 = blockIdx.x * 16 * NB;
  // SPLIT: gridDim.y > 1; the unsplit instance carries no fix-up code
  const int SK = SPLIT ? (int)gridDim.y : 1, ks = SPLIT ? (int)blockIdx.y : 0;
  // SK is 1, 2 or 4 (launch_skinny): the k-range bounds by shifts -- a 64-bit
  // division here expanded to ~300 instructions ahead of the first load, which
  // cost the unsplit launches 6-19 % (measured against the build without it)
  const int sk_log = __builtin_ctz((unsigned)SK);
  const int kt_lo = (ks * (K >> 7)) >> sk_log, kt_hi = ((ks + 1) * (K >> 7)) >> sk_log;
  const uint32_t K2 = (uint32_t)K * 2;
  const auto rsX = make_rsrc(x, (uint64_t)M * K2);
  const uint32_t x_voff = (uint32_t)li * K2 + (uint32_t)g * 64;

  f32x4 acc[NB][MB];
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[j][mb] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // One 128-k group per step.  The next step's weights and group scales (HBM)
  // are loaded before this step's dequant + MFMAs, and so are its activations
  // (L2), where the 128-VGPR budget of a 1024-thread group allows (weights for
  // MB * NB < 8, activations for MB * NB == 2), so a wave with several groups
  // (K > 128 * waves) keeps the next group in flight.  The single-block
  // instance (M <= 16, NB = 1) skips the activation prefetch to stay within 64
  // VGPRs, so two 16-wave workgroups share a CU and a launch over N / 16
  // workgroups is one round (M = 1, 2048 -> 8192: 5.90 -> 4.78 us).
  constexpr bool PREW = MB * NB < 8, PREX = MB * NB == 2;
  uint4 wq[NB], xb[MB][4];
  uint32_t sj[NB], zj[NB];
  auto load_w = [&](int k, uint4 (&w)[NB], uint32_t (&sv)[NB], uint32_t (&zv)[NB]) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int n = n0 + 16 * j + li;
      w[j] = *reinterpret_cast<const uint4*>(qw + qw_chunk_u32(n, k, g, K));
      sv[j] = scales[(size_t)k * N + n];
      zv[j] = zeros[(size_t)k * N + n];
    }
  };
  auto load_x = [&](int k, uint4 (&xv)[MB][4]) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int t = 0; t < 4; ++t) xv[mb][t] = buf_load16(rsX, x_voff, mb * 16 * K2 + k * 256 + t * 16);
  };
  if constexpr (!PREW) {
    for (int kt = kt_lo + wave; kt < kt_hi; kt += nwaves) {
      load_w(kt, wq, sj, zj);
      load_x(kt, xb);
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        uint4 wf[4];
        wf[0] = dq_frag<BF16, 0>(wq[j], sj[j], zj[j]);
        wf[1] = dq_frag<BF16, 1>(wq[j], sj[j], zj[j]);
        wf[2] = dq_frag<BF16, 2>(wq[j], sj[j], zj[j]);
        wf[3] = dq_frag<BF16, 3>(wq[j], sj[j], zj[j]);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) acc[j][mb] = mfma16<BF16>(wf[t], xb[mb][t], acc[j][mb]);
      }
    }
  } else {
    int kt = kt_lo + wave;
    if (kt < kt_hi) {
      load_w(kt, wq, sj, zj);
      load_x(kt, xb);
    }
    for (; kt < kt_hi; kt += nwaves) {
      const int kn = kt + nwaves;
      uint4 wq2[NB], xb2[MB][4];
      uint32_t sj2[NB], zj2[NB];
      if (kn < kt_hi) {
        load_w(kn, wq2, sj2, zj2);
        if constexpr (PREX) load_x(kn, xb2);
      }
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        uint4 wf[4];
        wf[0] = dq_frag<BF16, 0>(wq[j], sj[j], zj[j]);
        wf[1] = dq_frag<BF16, 1>(wq[j], sj[j], zj[j]);
        wf[2] = dq_frag<BF16, 2>(wq[j], sj[j], zj[j]);
        wf[3] = dq_frag<BF16, 3>(wq[j], sj[j], zj[j]);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) acc[j][mb] = mfma16<BF16>(wf[t], xb[mb][t], acc[j][mb]);
      }
      if (kn < kt_hi) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          wq[j] = wq2[j];
          sj[j] = sj2[j];
          zj[j] = zj2[j];
        }
        if constexpr (PREX) {
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int t = 0; t < 4; ++t) xb[mb][t] = xb2[mb][t];
        } else {
          load_x(kn, xb);
        }
      }
    }
  }
  // Cross-wave sums, one 16-channel block at a time through the same LDS.
  // Element e of a block is token m = 16 mb + (l & 15), channel
  // nn = n0 + 16 j + 4 (l >> 4) + r; with split K it goes to partial slot
  // ((b * SK + ks) * NB + j) * M * 16 + m * 16 + (nn - n0 - 16 j).
  auto epilogue = [&](float v, int m, int nn) {
    if (epi == QV_EPI_BIAS || epi == QV_EPI_BIAS_GELU || epi == QV_EPI_BIAS_RESID) v += to_f32(bias[nn], BF16);
    if (epi == QV_EPI_BIAS_GELU || epi == QV_EPI_GELU) v = gelu_erf(v);
    if (epi == QV_EPI_BIAS_RESID)  // out + gamma * o, o rounded first (resid_update8)
      v = to_f32(out[(size_t)m * N + nn], BF16) + to_f32(from_f32<BF16>(v), BF16) * to_f32(gamma[nn], BF16);
    out[(size_t)m * N + nn] = from_f32<BF16>(v);
  };
  const auto rsP = make_rsrc(part, part ? (uint64_t)gridDim.x * SK * NB * M * 16 * 4 : 0);
  auto slot = [&](int k_split, int j, int m, int c) {
    return (uint32_t)(((((blockIdx.x * SK + k_split) * NB + j) * M + m) * 16 + c) * 4);
  };
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    if (j) __syncthreads();
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) red[wave][mb][lane] = acc[j][mb];
    __syncthreads();
    for (int e = tid; e < MB * 256; e += blockDim.x) {
      const int mb = e >> 8, l = (e >> 2) & 63, r = e & 3;
      const int m = 16 * mb + (l & 15);
      if (m >= M) continue;
      float v = 0.f;
      for (int w = 0; w < nwaves; ++w) v += red[w][mb][l][r];
      const int c = 4 * (l >> 4) + r;
      // (!SPLIT || SK == 1): the split instances keep a runtime test for a
      // one-split grid -- with the epilogue branch folded away the compiler
      // rotated this loop around the partial stores, and the 4-way split
      // launches measured 5-9 % slower (M = 16..64 at 8192 -> 2048)
      if (!SPLIT || SK == 1)
        epilogue(v, m, n0 + 16 * j + c);
      else
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, v), rsP, slot(ks, j, m, c), 0, 16 /*sc1*/);
    }
  }
  if (!SPLIT || SK == 1) return;
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's partial values are stored
  __syncthreads();
  if (tid == 0)
    s_arrived = (int)__builtin_amdgcn_atomic_inc32(reinterpret_cast<unsigned*>(cnt) + blockIdx.x, (unsigned)(SK - 1),
                                                   __ATOMIC_RELAXED, "agent");
  __syncthreads();
  if (s_arrived != SK - 1) return;   // another split finishes the block
  for (int e = tid; e < M * 16 * NB; e += blockDim.x) {
    const int m = e / (16 * NB), cn = e % (16 * NB), j = cn >> 4, c = cn & 15;
    // the partials of up to four splits are loaded together (one L2 round
    // trip, not one per split), then added in split order
    float v = 0.f;
    for (int k0 = 0; k0 < SK; k0 += 4) {
      float t[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        t[u] = k0 + u < SK ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                           rsP, slot(k0 + u, j, m, c), 0, 16))
                           : 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (k0 + u < SK) v = k0 + u == 0 ? t[u] : v + t[u];
    }
    epilogue(v, m, n0 + cn);
  }
}

// ---------------------------------------------------------- dequant kernel
// One thread per (row n, 32-k chunk): writes 32 weights in natural k order.
template <bool BF16>
__global__ __launch_bounds__(256) void w4a16_dequant_kernel(
    const uint32_t* __restrict__ qw, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ zeros, uint16_t* __restrict__ w, int N, int K) {
  const int chunks_per_row = K >> 5;
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)N * chunks_per_row) return;
  const int n = (int)(idx / chunks_per_row);
  const int c = (int)(idx % chunks_per_row);
  const int kt = c >> 2, g = c & 3;
  const uint4 wq = *reinterpret_cast<const uint4*>(qw + qw_chunk_u32(n, kt, g, K));
  const uint32_t s = scales[(size_t)kt * N + n];
  const uint32_t z = zeros[(size_t)kt * N + n];
  uint4* dst = reinterpret_cast<uint4*>(w + (size_t)n * K + (size_t)c * 32);
  dst[0] = dq_frag<BF16, 0>(wq, s, z);
  dst[1] = dq_frag<BF16, 1>(wq, s, z);
  dst[2] = dq_frag<BF16, 2>(wq, s, z);
  dst[3] = dq_frag<BF16, 3>(wq, s, z);
}

// ------------------------------------------------------------ pack kernels
// WQLinear.from_linear on the GPU (qmodule.py:255-327).  One thread per (row
// n, 32-k chunk): q = rint(r(r(w + r(z * s)) / s)), r() rounding to the model
// dtype after every operation as the reference's 16-bit tensor ops do (each
// computed in fp32, IEEE division, rint = round half to even as torch.round),
// then the chunk's 32 values go into its 8 int16 of the AWQ-v2 layout: int16
// 8c + 2f + e of row r in 64-k block kb holds k = 64kb + 32c + 8h + 2f + e at
// bit 4h (the unmasked OR of qmodule.py:84-92, low 16 bits, so values outside
// 0..15 pack exactly as the reference packs them).
template <bool BF16>
__device__ __forceinline__ float rnd16(float v) {
  return to_f32(from_f32<BF16>(v), BF16);
}

template <bool BF16>
__global__ __launch_bounds__(256) void w4a16_pack_kernel(
    const uint16_t* __restrict__ w, const uint16_t* __restrict__ s, const uint16_t* __restrict__ z,
    uint16_t* __restrict__ qw, int N, int K, int gs, int G) {
  const int chunks = K >> 5;
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)N * chunks) return;
  const int n = (int)(idx / chunks), ch = (int)(idx % chunks);
  const int k0 = ch * 32, g = k0 / gs;
  const float sf = to_f32(s[(size_t)n * G + g], BF16);
  const float szf = rnd16<BF16>(to_f32(z[(size_t)n * G + g], BF16) * sf);
  const uint4* src = reinterpret_cast<const uint4*>(w + (size_t)n * K + k0);
  int q[32];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const uint4 u = src[v];
    const uint32_t words[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float wf = to_f32((uint16_t)(words[i >> 1] >> (16 * (i & 1))), BF16);
      const float t = rnd16<BF16>(wf + szf);
      const float d = rnd16<BF16>(t / sf);
      q[8 * v + i] = (int)__builtin_rintf(d);
    }
  }
  uint32_t out[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {  // int16 pair (2p, 2p + 1) = f = p, e = 0 / 1
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      lo |= (uint32_t)q[8 * h + 2 * p] << (4 * h);
      hi |= (uint32_t)q[8 * h + 2 * p + 1] << (4 * h);
    }
    out[p] = (lo & 0xFFFFu) | (hi << 16);
  }
  const int rg = n >> 2, r = n & 3, kb = k0 >> 6, c = (k0 >> 5) & 1;
  *reinterpret_cast<uint4*>(qw + (size_t)rg * K + 64 * kb + 16 * r + 8 * c) =
      make_uint4(out[0], out[1], out[2], out[3]);
}

// scales (rows, N) = s^T zero-padded; scaled_zeros = -r(float(s) * float(int(z)))
// (qmodule.py:262-283, 317-327: zeros truncated to int32, product in fp32,
// one rounding, negated), zero-padded.
template <bool BF16>
__global__ __launch_bounds__(256) void w4a16_pack_tables_kernel(
    const uint16_t* __restrict__ s, const uint16_t* __restrict__ z, uint16_t* __restrict__ s_out,
    uint16_t* __restrict__ sz_out, int N, int G, int rows) {
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)rows * N) return;
  const int g = (int)(idx / N), n = (int)(idx % N);
  uint16_t sv = 0, zv = 0;
  if (g < G) {
    sv = s[(size_t)n * G + g];
    const float zi = (float)(int)to_f32(z[(size_t)n * G + g], BF16);
    zv = from_f32<BF16>(to_f32(sv, BF16) * zi) ^ 0x8000u;
  }
  s_out[idx] = sv;
  sz_out[idx] = zv;
}

// ------------------------------------------------------------- launchers
// Kernel choice (w4_pick_tile): M <= 64 goes to the skinny kernel (5), whose
// grid covers the channels instead of M x N tiles; a grid that the 32-row
// tile keeps within one tile per CU takes that tile (6); everything else
// goes to the streamed kernel with the tile plan of w4_stream_plan below.
// Two workgroups run per CU (512 slots on 256 CUs).
static int w4_pick_tile(int M, int N, int K) {
  // the skinny kernel addresses the activations with 32-bit buffer offsets
  const bool skinny_ok = M <= 64 && (int64_t)M * K * 2 < ((int64_t)1 << 31);
  if (skinny_ok) return 5;
  // Estimated time per candidate, in units of one 32-row tile step:
  //  * at most one tile per CU (256 tiles): latency-bound, a tile costs its
  //    pipeline fill + epilogue (~130 rows' worth) plus its rows;
  //  * more: ceil(tiles / 512 slots) rounds of (130 + bm) / eff, eff the
  //    measured per-row efficiency of the tile (larger tiles spread the
  //    dequantisation over more MFMAs).
  // Fitted to single-launch timings at M = 1374 .. 43968, K = 1024 / 4096,
  // N = 1024 .. 4096 (the W4 linears of the VGGT blocks); it picks the
  // measured fastest tile at each of them.
  const struct { int id, bm; double eff; } cand[] = {{1, 128, 1.00}, {2, 96, 0.93}, {3, 64, 0.82}, {6, 32, 0.62}};
  int best = 1;
  double best_t = 1e300;
  for (const auto& c : cand) {
    const double tiles = (double)((M + c.bm - 1) / c.bm) * ((N + 255) / 256);
    const double t = tiles <= 256.0 ? 130.0 + c.bm : __builtin_ceil(tiles / 512.0) * (130.0 + c.bm) / c.eff;
    if (t < best_t) { best_t = t; best = c.id; }
  }
  return best;
}

// Tile plan of the streamed kernel (w4_stream_plan).  A launch whose last
// round of tiles leaves slots idle loses up to a tile's time; covering the
// rows in two ranges, whole rounds of 128- or 96-row tiles and then shorter
// tiles, lets the short tiles fill the slots that free up first.  The plan
// is chosen with an event-driven model of the launch: 256 CUs x 2 workgroup
// slots, workgroups dispatched in grid order to the slot that frees first
// (simultaneous completions refill the CUs breadth-first), a tile's work
// = prologue + stages x per-stage time of its height + epilogue per row,
// and two co-resident tiles each progressing at 0.62 of the rate of a tile
// alone on its CU.  The constants (microseconds, shader clock ~2.1 GHz) are
// fitted to 28 timings of single- and two-range launches at M = 1374 ..
// 43968, K = 1024 / 4096, N = 1024 .. 4096 (rms error ~5 %).  Only the
// ranking matters; the model is run once per shape and cached.
namespace {
constexpr int PLAN_CUS = 256;
constexpr double PLAN_SHARED_RATE = 0.623;

double w4_tile_us(int mt, int K, bool gelu) {
  const double per_stage = mt == 4 ? 0.907 : (mt == 3 ? 0.779 : 0.567);
  return 1.48 + (K / 64) * per_stage + 32 * mt * (gelu ? 0.0482 : 0.0080);
}

// Finish time of n_a tiles of work w_a followed (in dispatch order) by n_b
// tiles of work w_b.  Slot s = pass * PLAN_CUS + cu; its CU partner is
// s +- PLAN_CUS.  A full round of identical tiles starts on every slot at
// once and ends at once (w_a at the shared rate), after which the state is
// the starting one: all but the last full round of the first range are
// skipped in closed form.
double w4_simulate(int n_a, double w_a, int n_b, double w_b) {
  const int slots = 2 * PLAN_CUS;
  const int skip = n_a / slots > 1 ? n_a / slots - 1 : 0;
  const double t_skip = skip * (w_a / PLAN_SHARED_RATE);
  n_a -= skip * slots;
  struct Slot { double rem = 0, t0 = 0; int ver = 0; bool busy = false; };
  std::vector<Slot> slot(2 * PLAN_CUS);
  using Ev = std::pair<double, std::pair<int, int>>;
  std::priority_queue<Ev, std::vector<Ev>, std::greater<Ev>> pq;
  const int total = n_a + n_b;
  int next = 0;
  double now = 0, end = 0;
  auto mate = [](int s) { return s < PLAN_CUS ? s + PLAN_CUS : s - PLAN_CUS; };
  auto rate = [&](int s) { return slot[mate(s)].busy ? PLAN_SHARED_RATE : 1.0; };
  auto take = [&](int s) {
    slot[s].busy = next < total;
    if (slot[s].busy) {
      slot[s].rem = next < n_a ? w_a : w_b;
      slot[s].t0 = now;
      ++next;
    }
  };
  auto push = [&](int s) {
    if (!slot[s].busy) return;
    ++slot[s].ver;
    pq.push({now + slot[s].rem / rate(s), {s, slot[s].ver}});
  };
  for (int s = 0; s < 2 * PLAN_CUS; ++s) take(s);
  for (int s = 0; s < 2 * PLAN_CUS; ++s) push(s);
  while (!pq.empty()) {
    const Ev e = pq.top();
    pq.pop();
    const int s = e.second.first, o = mate(s);
    if (!slot[s].busy || e.second.second != slot[s].ver) continue;
    now = end = e.first;
    if (slot[o].busy) {  // the partner ran at the shared rate until now
      slot[o].rem -= (now - slot[o].t0) * rate(o);
      slot[o].t0 = now;
    }
    take(s);
    push(s);
    push(o);
  }
  return t_skip + end;
}

double w4_plan_time(int M, int N, int K, bool gelu, const StreamPlan& p) {
  const int tn = (N + 255) / 256;
  const int rows_a = p.mt_b ? p.rows_a : M;
  const int n_a = (rows_a + 32 * p.mt_a - 1) / (32 * p.mt_a) * tn;
  const int n_b = p.mt_b ? (M - rows_a + 32 * p.mt_b - 1) / (32 * p.mt_b) * tn : 0;
  return w4_simulate(n_a, w4_tile_us(p.mt_a, K, gelu), n_b, p.mt_b ? w4_tile_us(p.mt_b, K, gelu) : 0.0);
}

StreamPlan w4_stream_plan_uncached(int M, int N, int K, bool gelu) {
  const int tn = (N + 255) / 256;
  // Long K (>= 4096, 64 stages) in at most one round of slots: one 128-row
  // tile per CU first, the remaining rows in 64-row tiles.  Measured at
  // K = 4096: two co-resident tiles of one height each progress at only
  // 0.48 (128-row) to 0.57 (64-row) of their solo rate -- they start
  // together and stall together -- while a 128-row tile beside a 64-row one
  // progresses at ~0.65, so this plan beats every single-height one (fc2 of
  // the MLP at M = 10992: 87.7-89.9 us against 91.1-99.8 us for 96-row
  // tiles, two boxes).  The event model below assumes one co-residence rate
  // and misses this.
  if (K >= 4096) {
    const int rows_a = PLAN_CUS / tn * 128;
    const int64_t tiles = (int64_t)rows_a / 128 * tn + (int64_t)(M - rows_a + 63) / 64 * tn;
    if (rows_a > 0 && rows_a < M && tiles <= 2 * PLAN_CUS) {
      StreamPlan p;
      p.mt_a = 4;
      p.rows_a = rows_a;
      p.mt_b = 2;
      return p;
    }
  }
  StreamPlan best;
  double best_t = 1e300;
  for (int mt : {4, 3, 2}) {
    StreamPlan p;
    p.mt_a = mt;
    const double t = w4_plan_time(M, N, K, gelu, p);
    if (t < best_t) best_t = t, best = p;
  }
  // Past 16 rounds of 128-row tiles the last round is < 7 % of the launch.
  if ((int64_t)(M + 127) / 128 * tn > 16 * 2 * PLAN_CUS) return best;
  const double single_t = best_t;
  const StreamPlan single = best;
  const int pairs[3][2] = {{4, 3}, {4, 2}, {3, 2}};
  // The second range fills the last rounds: first ranges that end more than
  // 2.5 rounds of 128-row tiles before the launch does are not tried.
  const double rounds128 = (double)((M + 127) / 128) * tn / (2 * PLAN_CUS);
  for (const auto& pr : pairs) {
    const int bm = 32 * pr[0];
    const int jmax = (M - 1) / bm;  // rows_a = j * bm < M
    const double min_tiles = (rounds128 - 2.5) * 2 * PLAN_CUS;
    const int jmin = min_tiles > tn ? (int)(min_tiles / tn) : 1;
    if (jmax < jmin) continue;
    const int span = jmax - jmin + 1;
    const int step = span > 16 ? span / 16 : 1;
    int best_j = 0;
    double pair_t = 1e300;
    auto eval = [&](int j) {
      StreamPlan p;
      p.mt_a = pr[0];
      p.rows_a = j * bm;
      p.mt_b = pr[1];
      const double t = w4_plan_time(M, N, K, gelu, p);
      if (t < pair_t) pair_t = t, best_j = j;
    };
    // a coarse scan plus every split whose first range ends within two tile
    // rows of a whole number of rounds, then the neighbours of the best
    for (int j = jmin; j <= jmax; ++j) {
      const int r = (int)((int64_t)j * tn % (2 * PLAN_CUS));
      if ((j - jmin) % step == 0 || r <= 2 * tn || 2 * PLAN_CUS - r <= 2 * tn) eval(j);
    }
    const int c = best_j;
    for (int j = c - step + 1; j < c + step; ++j)
      if (j >= jmin && j <= jmax && j != c) eval(j);
    if (pair_t < best_t) {
      best_t = pair_t;
      best.mt_a = pr[0];
      best.rows_a = best_j * bm;
      best.mt_b = pr[1];
    }
  }
  // keep one tile height unless two ranges are predicted > 2 % faster
  return best_t < 0.98 * single_t ? best : single;
}

StreamPlan w4_stream_plan(int M, int N, int K, bool gelu) {
  static std::mutex mu;
  static std::map<std::tuple<int, int, int, bool>, StreamPlan> cache;
  const auto key = std::make_tuple(M, N, K, gelu);
  {
    std::lock_guard<std::mutex> g(mu);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  const StreamPlan p = w4_stream_plan_uncached(M, N, K, gelu);
  std::lock_guard<std::mutex> g(mu);
  if (cache.size() >= 4096) cache.clear();
  cache[key] = p;
  return p;
}

#ifndef QV_W4_KSPLIT
#define QV_W4_KSPLIT 1
#endif
StreamPlan w4_plan_for(int tile, int M, int N, int K, int epi) {
  StreamPlan p;
  if (tile == 6) {  // a grid of at most one tile per CU: the 32-row tile
    p.mt_a = 1;
  } else {
    p = w4_stream_plan(M, N, K, epi == QV_EPI_BIAS_GELU || epi == QV_EPI_GELU);
  }
  // One range of at most one tile per CU runs one wave per SIMD: split K
  // between two 4-wave groups of one workgroup (whole 128-k groups each)
  // where that measured faster -- long K (K >= 2048: M = 1374 and 2748 at
  // 4096 -> 1024, -14 %) and the 32-row tile (1374 x 1024 -> 1024, -6 %).
  // At K = 1024 with taller tiles the two groups, held in step by the
  // shared per-stage barriers, wait on their loads together and the split
  // measured 2-4 % slower (config 1: 14.67 -> 14.98 us).
  const long tiles = (long)((M + 32 * p.mt_a - 1) / (32 * p.mt_a)) * ((N + 255) / 256);
  p.ksplit = QV_W4_KSPLIT && p.mt_b == 0 && tiles <= 256 && K % 256 == 0 && (K >= 2048 || p.mt_a == 1);
  // The other one-round launches of 64- and 96-row tiles pipeline 128-k
  // stages: a stage's loads get twice the time to land behind one wave's
  // MFMAs, and half as many barriers (config 1, 1374 x 1024 -> 3072:
  // 15.0 -> 14.5 us; 1000 x 1024 -> 3072 -3 %; bit-identical).  With two
  // workgroups per CU the shorter stages measured equal or faster.
  p.sub = (p.mt_b == 0 && !p.ksplit && tiles <= 256 && K % 256 == 0 && (p.mt_a == 2 || p.mt_a == 3)) ? 2 : 1;
  return p;
}
}  // namespace

// Split-K workspace of the skinny kernel: fp32 partials and the arrival
// counters, SPLIT_MAX_BLOCKS per split factor (2 and 4: counters
// [0, 256) serve two-way launches, [256, 512) four-way ones).  The counters
// start at zero (cleared when the workspace is made) and every complete
// launch returns each counter it uses to zero with its last wrapping
// increment (see w4a16_skinny_kernel), so no launch clears them.
struct SplitWorkspace {
  float* part = nullptr;
  int* cnt = nullptr;
  size_t part_floats = 0;
  int cnt_n = 0;
};
constexpr size_t SPLIT_PART_FLOATS = (size_t)2 << 20;   // 8 MiB of partials
constexpr int SPLIT_MAX_BLOCKS = 256;                    // a split launch has < 256 channel blocks
constexpr int SPLIT_COUNTERS = 4096;                     // >= 2 x SPLIT_MAX_BLOCKS
static_assert(SPLIT_COUNTERS >= 2 * SPLIT_MAX_BLOCKS, "one counter range per split factor");

static int split_workspace(hipStream_t st, SplitWorkspace& ws);

template <bool BF16>
static int launch_skinny(const void* x, const void* qw, const void* s, const void* z, const void* bias,
                         void* out, int M, int N, int K, int epi, hipStream_t st, const void* gamma,
                         const SplitWorkspace& ws);

template <bool BF16>
static int launch_gemm(const void* x, const void* qw, const void* s, const void* z, const void* bias,
                       void* out, int M, int N, int K, int epi, hipStream_t st, const void* gamma = nullptr) {
  const int tile = w4_pick_tile(M, N, K);
  if (tile == 5) {
    SplitWorkspace ws;
    const int rc = split_workspace(st, ws);
    if (rc) return rc;
    return launch_skinny<BF16>(x, qw, s, z, bias, out, M, N, K, epi, st, gamma, ws);
  }
  return launch_w4a16_stream<BF16>(x, qw, s, z, bias, gamma, out, M, N, K, epi, w4_plan_for(tile, M, N, K, epi), st);
}

// Channel blocks per skinny workgroup: NB = 2 from M = 5 when N >= 4096
// (>= 128 workgroups remain), else 1 -- measured on the VGGT camera-head and
// aggregator shapes, where NB = 4 never won.
static int w4_skinny_nb(int M, int N) {
  int nb = (M > 4 && N >= 4096) ? 2 : 1;
  if (N % (16 * nb)) nb = 1;
  return nb;
}

// Split factor of the skinny kernel: only long K (>= 64 groups) with fewer
// than 256 channel blocks is split -- 2 ways for M <= 8, else 4 ways with
// 32-channel blocks, which halves the activation re-reads.  Measured from
// graph replays over > 1 GB of rotating weights (8192 -> 2048: M = 32
// 19.9 -> 10.5 us, M = 8 8.1 -> 7.2 us, M = 1 6.4 -> 6.2 us); splitting K <= 2048
// or shapes that already give >= 256 blocks measured equal or slower.  A
// split that the workspace cannot hold (partials or counters) runs unsplit.
static void w4_skinny_plan(int M, int N, int K, const SplitWorkspace& ws, int& nb, int& sk) {
  nb = w4_skinny_nb(M, N);
  sk = 1;
  if (K / 128 < 64 || N / (16 * nb) >= SPLIT_MAX_BLOCKS) return;
  if (M > 8 && N % 32 == 0) {
    nb = 2;
    sk = 4;
  } else {
    sk = 2;
  }
  if ((size_t)N * M * sk > ws.part_floats || N / (16 * nb) >= SPLIT_MAX_BLOCKS) {
    nb = w4_skinny_nb(M, N);
    sk = 1;
  }
}

// zero n counters of a new workspace (a kernel on the stream that will use
// it, not a synchronous memset on the null stream)
__global__ __launch_bounds__(256) void zero_counters_kernel(int* __restrict__ c, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) c[i] = 0;
}

template <bool BF16>
static int launch_skinny(const void* x, const void* qw, const void* s, const void* z, const void* bias,
                         void* out, int M, int N, int K, int epi, hipStream_t st, const void* gamma,
                         const SplitWorkspace& ws) {
  int nb, sk;
  w4_skinny_plan(M, N, K, ws, nb, sk);
  const int KT = K / 128 / sk;
  const int waves = KT < 16 ? KT : 16;
  const dim3 grid(N / (16 * nb), sk), block(64 * waves);
  float* part = sk > 1 ? ws.part : nullptr;
  int* cnt = sk > 1 ? ws.cnt + (sk == 2 ? 0 : SPLIT_MAX_BLOCKS) : nullptr;
  QV_CHECK_ARG(sk == 1 || ((sk == 2 || sk == 4) && (int)grid.x < SPLIT_MAX_BLOCKS && ws.cnt_n >= 2 * SPLIT_MAX_BLOCKS),
               "w4a16 skinny: bad split plan (%d splits over %d blocks)", sk, (int)grid.x);
#define QV_SKINNY_L(MB, NB, SP)                                                                       \
  hipLaunchKernelGGL((w4a16_skinny_kernel<BF16, MB, NB, SP>), grid, block, 0, st, (const uint16_t*)x, \
                     (const uint32_t*)qw, (const uint16_t*)s, (const uint16_t*)z,                     \
                     (const uint16_t*)bias, (const uint16_t*)gamma, (uint16_t*)out, M, N, K, epi, part, cnt)
#define QV_SKINNY(MB, NB)                   \
  do {                                      \
    if (sk > 1) QV_SKINNY_L(MB, NB, true);  \
    else QV_SKINNY_L(MB, NB, false);        \
  } while (0)
#define QV_SKINNY_M(NB)            \
  if (M <= 16) QV_SKINNY(1, NB);   \
  else if (M <= 32) QV_SKINNY(2, NB); \
  else if (M <= 48) QV_SKINNY(3, NB); \
  else QV_SKINNY(4, NB);
  if (nb == 2) { QV_SKINNY_M(2) }
  else { QV_SKINNY_M(1) }
#undef QV_SKINNY_M
#undef QV_SKINNY
#undef QV_SKINNY_L
  return check_launch("w4a16_skinny");
}

// ------------------------------------------------- device scratch
// File-scope device scratch: the split partials and counters of a
// SplitWorkspace, fixed at 8 MiB + 16 KiB per GPU for the life of the
// process.  qv_w4a16_gemm_noalloc always uses it; the allocating entries use
// it for a launch captured into a graph on a stream that has no workspace of
// its own yet (see split_workspace).  In host code `scratch` only names the
// symbol; its device address comes from hipGetSymbolAddress, once per device
// with that device current (scratch_workspace), and only that address is
// passed to kernels.  That first call also clears the counters (a kernel on
// the caller's stream, then a wait for it), so it has to run outside stream
// capture.  Split launches that overlap on one GPU and use the scratch share
// it and so race.
static __device__ __align__(256) uint8_t scratch[SPLIT_PART_FLOATS * sizeof(float) + SPLIT_COUNTERS * sizeof(int)];

static int scratch_workspace(hipStream_t st, SplitWorkspace& ws) {
  constexpr int MAX_DEV = 64;
  static std::mutex mu;
  static void* ptr[MAX_DEV] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) {
    set_error("w4a16 no-alloc: no usable current device");
    return QV_EHIP;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!ptr[dev]) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cap) != hipSuccess) {
      set_error("w4a16 skinny: hipStreamIsCapturing failed (%s)", hipGetErrorString(hipGetLastError()));
      return QV_EHIP;
    }
    QV_CHECK_ARG(cap == hipStreamCaptureStatusNone,
                 "w4a16 skinny: the first split-K call on a device clears the device scratch and must run "
                 "outside stream capture (make one eager call first)");
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("w4a16 no-alloc: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
      return QV_EHIP;
    }
    int* cnt = reinterpret_cast<int*>(reinterpret_cast<uint8_t*>(p) + SPLIT_PART_FLOATS * sizeof(float));
    hipLaunchKernelGGL(zero_counters_kernel, dim3((SPLIT_COUNTERS + 255) / 256), dim3(256), 0, st, cnt,
                       SPLIT_COUNTERS);
    const int rc = check_launch("zero_counters");
    if (rc) return rc;
    if (hipStreamSynchronize(st) != hipSuccess) {
      set_error("w4a16 skinny: clearing the device scratch failed (%s)", hipGetErrorString(hipGetLastError()));
      return QV_EHIP;
    }
    ptr[dev] = p;
  }
  ws.part = reinterpret_cast<float*>(ptr[dev]);
  ws.cnt = reinterpret_cast<int*>(reinterpret_cast<uint8_t*>(ptr[dev]) + SPLIT_PART_FLOATS * sizeof(float));
  ws.part_floats = SPLIT_PART_FLOATS;
  ws.cnt_n = SPLIT_COUNTERS;
  return QV_OK;
}

// Eager launches: one split workspace per (device, stream), allocated on the
// stream's first skinny call; launches on one stream run in order and share
// it, another stream gets its own, so eager skinny calls on different streams
// may overlap.  Launches captured into a graph always use the device scratch
// instead: capture cannot allocate, the split plan (and with it every output
// bit) is then the same as an eager call's, and a graph -- which keeps the
// workspace it was captured with and may be replayed on any stream -- never
// shares memory with eager calls.  Graphs with split launches that are
// replayed concurrently with each other (or with qv_w4a16_gemm_noalloc
// calls) on one GPU race.
static int split_workspace(hipStream_t st, SplitWorkspace& ws) {
  static std::mutex mu;
  static std::map<std::pair<int, hipStream_t>, SplitWorkspace> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    set_error("w4a16 skinny: hipGetDevice failed");
    return QV_EHIP;
  }
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cap) != hipSuccess) {
    set_error("w4a16 skinny: hipStreamIsCapturing failed (%s)", hipGetErrorString(hipGetLastError()));
    return QV_EHIP;
  }
  if (cap != hipStreamCaptureStatusNone) return scratch_workspace(st, ws);
  {
    std::lock_guard<std::mutex> lock(mu);
    const auto it = cache.find(std::make_pair(dev, st));
    if (it != cache.end()) {
      ws = it->second;
      return QV_OK;
    }
  }
  // set the device scratch up now, outside capture, for a later capture on a
  // stream that has no workspace
  SplitWorkspace sc;
  int rc = scratch_workspace(st, sc);
  if (rc) return rc;
  SplitWorkspace n;
  n.part_floats = SPLIT_PART_FLOATS;
  n.cnt_n = SPLIT_COUNTERS;
  if (hipMalloc(&n.part, n.part_floats * sizeof(float)) != hipSuccess ||
      hipMalloc(&n.cnt, n.cnt_n * sizeof(int)) != hipSuccess) {
    set_error("w4a16 skinny: split workspace allocation failed (%s)", hipGetErrorString(hipGetLastError()));
    return QV_EHIP;
  }
  // the counters start at zero; only this stream (and graphs captured on it)
  // will use them, after this kernel
  hipLaunchKernelGGL(zero_counters_kernel, dim3((n.cnt_n + 255) / 256), dim3(256), 0, st, n.cnt, n.cnt_n);
  rc = check_launch("zero_counters");
  if (rc) return rc;
  std::lock_guard<std::mutex> lock(mu);
  cache[std::make_pair(dev, st)] = n;
  ws = n;
  return QV_OK;
}

static int check_common(const void* x, const void* qw, const void* s, const void* z, const void* bias,
                        const void* out, int64_t M, int64_t N, int64_t K, int dtype, int epi) {
  QV_CHECK_ARG(dtype == QV_F16 || dtype == QV_BF16, "unsupported dtype %d (expected fp16 or bf16)", dtype);
  QV_CHECK_ARG(M >= 0 && N > 0 && K > 0, "bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  QV_CHECK_ARG(K % 128 == 0, "K=%lld must be a multiple of the group size 128", (long long)K);
  QV_CHECK_ARG(N % 16 == 0, "N=%lld must be a multiple of 16", (long long)N);
  QV_CHECK_ARG(M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX && M * K <= (int64_t)1 << 40, "shape too large");
  QV_CHECK_ARG(epi >= QV_EPI_NONE && epi <= QV_EPI_GELU, "bad epilogue %d", epi);
  QV_CHECK_ARG(bias != nullptr || !(epi == QV_EPI_BIAS || epi == QV_EPI_BIAS_GELU), "epilogue needs a bias pointer");
  QV_CHECK_ARG(M == 0 || (x && qw && s && z && out), "null pointer argument");
  QV_CHECK_ARG(((uintptr_t)x % 16) == 0 && ((uintptr_t)qw % 16) == 0, "x and qweight must be 16-byte aligned");
  QV_CHECK_ARG(((uintptr_t)s % 4) == 0 && ((uintptr_t)z % 4) == 0, "scale tables must be 4-byte aligned");
  QV_CHECK_ARG(((uintptr_t)out % 16) == 0, "out must be 16-byte aligned");
  QV_CHECK_ARG(bias == nullptr || ((uintptr_t)bias % 8) == 0, "bias must be 8-byte aligned");
  return QV_OK;
}

}  // namespace qv

using namespace qv;

extern "C" int qv_w4a16_gemm(const void* x, const void* qweight, const void* scales,
                             const void* scaled_zeros, const void* bias, void* out, int64_t M,
                             int64_t N, int64_t K, int dtype, int epilogue, void* stream) {
  int rc = check_common(x, qweight, scales, scaled_zeros, bias, out, M, N, K, dtype, epilogue);
  if (rc) return rc;
  if (M == 0) return QV_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == QV_BF16)
    return launch_gemm<true>(x, qweight, scales, scaled_zeros, bias, out, (int)M, (int)N, (int)K,
                             epilogue, st);
  return launch_gemm<false>(x, qweight, scales, scaled_zeros, bias, out, (int)M, (int)N, (int)K,
                            epilogue, st);
}

extern "C" int qv_w4a16_gemv(const void* x, const void* qweight, const void* scales,
                             const void* scaled_zeros, const void* bias, void* out, int64_t M,
                             int64_t N, int64_t K, int group_size, int dtype, int epilogue,
                             void* stream) {
  QV_CHECK_ARG(group_size == 128, "unsupported group size %d for the GEMV (only 128)", group_size);
  QV_CHECK_ARG(M >= 1 && M <= 16, "unsupported batch size M=%lld for the GEMV (1..16)", (long long)M);
  int rc = check_common(x, qweight, scales, scaled_zeros, bias, out, M, N, K, dtype, epilogue);
  if (rc) return rc;
  // the skinny kernel addresses the activations with 32-bit buffer offsets
  QV_CHECK_ARG(M * K * 2 < ((int64_t)1 << 31), "K=%lld too large for the GEMV", (long long)K);
  hipStream_t st = (hipStream_t)stream;
  SplitWorkspace ws;
  rc = split_workspace(st, ws);
  if (rc) return rc;
  if (dtype == QV_BF16)
    return launch_skinny<true>(x, qweight, scales, scaled_zeros, bias, out, (int)M, (int)N, (int)K, epilogue, st,
                               nullptr, ws);
  return launch_skinny<false>(x, qweight, scales, scaled_zeros, bias, out, (int)M, (int)N, (int)K, epilogue, st,
                              nullptr, ws);
}

extern "C" int qv_w4a16_dequant(const void* qweight, const void* scales, const void* scaled_zeros,
                                void* out_w, int64_t N, int64_t K, int dtype, void* stream) {
  QV_CHECK_ARG(dtype == QV_F16 || dtype == QV_BF16, "unsupported dtype %d", dtype);
  QV_CHECK_ARG(N > 0 && K > 0 && K % 128 == 0 && N % 4 == 0, "bad shape N=%lld K=%lld", (long long)N, (long long)K);
  QV_CHECK_ARG(N <= INT32_MAX && K <= INT32_MAX, "shape too large");
  QV_CHECK_ARG(qweight && scales && scaled_zeros && out_w, "null pointer argument");
  QV_CHECK_ARG(((uintptr_t)qweight % 16) == 0 && ((uintptr_t)out_w % 16) == 0, "buffers must be 16-byte aligned");
  const size_t total = (size_t)N * (size_t)(K / 32);
  const dim3 grid((unsigned)((total + 255) / 256)), block(256);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == QV_BF16)
    hipLaunchKernelGGL((w4a16_dequant_kernel<true>), grid, block, 0, st, (const uint32_t*)qweight,
                       (const uint16_t*)scales, (const uint16_t*)scaled_zeros, (uint16_t*)out_w, (int)N, (int)K);
  else
    hipLaunchKernelGGL((w4a16_dequant_kernel<false>), grid, block, 0, st, (const uint32_t*)qweight,
                       (const uint16_t*)scales, (const uint16_t*)scaled_zeros, (uint16_t*)out_w, (int)N, (int)K);
  return check_launch("w4a16_dequant");
}

// Rows of the scale tables: calculate_zeros_width(K, group_size) * 8
// (qmodule.py:13-41; group_size -1 = one group of K, multiplier 1).
static int64_t w4_scale_rows(int64_t K, int group_size) {
  const int gs = group_size == -1 ? (int)K : group_size;
  int mult = 1;
  if (group_size == 64) mult = 2;
  else if (group_size == 32) mult = 4;
  const int64_t base = (K / gs + 7) / 8;
  return (base + mult - 1) / mult * mult * 8;
}

extern "C" int qv_w4a16_pack(const void* weight, const void* scales, const void* zeros, void* qweight,
                             void* scales_out, void* scaled_zeros_out, int64_t N, int64_t K,
                             int group_size, int dtype, void* stream) {
  QV_CHECK_ARG(dtype == QV_F16 || dtype == QV_BF16, "unsupported dtype %d", dtype);
  QV_CHECK_ARG(N > 0 && K > 0 && N % 4 == 0 && K % 64 == 0, "bad shape N=%lld K=%lld (need N %% 4 == 0, K %% 64 == 0)",
               (long long)N, (long long)K);
  QV_CHECK_ARG(N <= INT32_MAX && K <= INT32_MAX, "shape too large");
  const int gs = group_size == -1 ? (int)K : group_size;
  QV_CHECK_ARG(gs >= 32 && gs % 32 == 0 && K % gs == 0 && (gs >= 128 || gs == 64 || gs == 32),
               "unsupported group size %d for K=%lld", group_size, (long long)K);
  QV_CHECK_ARG(weight && scales && zeros && qweight && scales_out && scaled_zeros_out, "null pointer argument");
  QV_CHECK_ARG(((uintptr_t)weight % 16) == 0 && ((uintptr_t)qweight % 16) == 0, "weight and qweight must be 16-byte aligned");
  const int G = (int)(K / gs);
  const int64_t rows = w4_scale_rows(K, group_size);
  hipStream_t st = (hipStream_t)stream;
  const size_t total = (size_t)N * (size_t)(K / 32), ttot = (size_t)rows * (size_t)N;
  const dim3 block(256), grid((unsigned)((total + 255) / 256)), tgrid((unsigned)((ttot + 255) / 256));
  if (dtype == QV_BF16) {
    hipLaunchKernelGGL((w4a16_pack_kernel<true>), grid, block, 0, st, (const uint16_t*)weight,
                       (const uint16_t*)scales, (const uint16_t*)zeros, (uint16_t*)qweight, (int)N, (int)K, gs, G);
    hipLaunchKernelGGL((w4a16_pack_tables_kernel<true>), tgrid, block, 0, st, (const uint16_t*)scales,
                       (const uint16_t*)zeros, (uint16_t*)scales_out, (uint16_t*)scaled_zeros_out, (int)N, G, (int)rows);
  } else {
    hipLaunchKernelGGL((w4a16_pack_kernel<false>), grid, block, 0, st, (const uint16_t*)weight,
                       (const uint16_t*)scales, (const uint16_t*)zeros, (uint16_t*)qweight, (int)N, (int)K, gs, G);
    hipLaunchKernelGGL((w4a16_pack_tables_kernel<false>), tgrid, block, 0, st, (const uint16_t*)scales,
                       (const uint16_t*)zeros, (uint16_t*)scales_out, (uint16_t*)scaled_zeros_out, (int)N, G, (int)rows);
  }
  return check_launch("w4a16_pack");
}

extern "C" int qv_w4a16_gemm_residual(const void* x, const void* qweight, const void* scales,
                                      const void* scaled_zeros, const void* bias, const void* gamma,
                                      void* residual, int64_t M, int64_t N, int64_t K, int dtype, void* stream) {
  int rc = check_common(x, qweight, scales, scaled_zeros, bias, residual, M, N, K, dtype, QV_EPI_BIAS);
  if (rc) return rc;
  QV_CHECK_ARG(gamma != nullptr && ((uintptr_t)gamma % 16) == 0, "gamma must be a 16-byte aligned pointer");
  QV_CHECK_ARG(((uintptr_t)residual % 16) == 0, "residual must be 16-byte aligned");
  if (M == 0) return QV_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == QV_BF16)
    return launch_gemm<true>(x, qweight, scales, scaled_zeros, bias, residual, (int)M, (int)N, (int)K,
                             QV_EPI_BIAS_RESID, st, gamma);
  return launch_gemm<false>(x, qweight, scales, scaled_zeros, bias, residual, (int)M, (int)N, (int)K,
                            QV_EPI_BIAS_RESID, st, gamma);
}

extern "C" int qv_w4a16_gemm_qkrope(const void* x, const void* qweight, const void* scales,
                                    const void* scaled_zeros, const void* bias, void* out, int64_t M, int64_t N,
                                    int64_t K, const int32_t* positions, const float* cos_table,
                                    const float* sin_table, int64_t table_rows, const void* q_gamma,
                                    const void* q_beta, const void* k_gamma, const void* k_beta, float eps,
                                    int64_t H, void* stream) {
  int rc = check_common(x, qweight, scales, scaled_zeros, bias, out, M, N, K, QV_F16, QV_EPI_BIAS);
  if (rc) return rc;
  QV_CHECK_ARG(bias != nullptr, "the fused q/k-norm + RoPE projection needs its bias");
  QV_CHECK_ARG(H > 0 && N == 3 * H * 64, "N=%lld must be 3 x heads x 64 (heads=%lld)", (long long)N, (long long)H);
  QV_CHECK_ARG(table_rows > 0 && table_rows <= INT32_MAX, "bad table_rows %lld", (long long)table_rows);
  QV_CHECK_ARG(positions && cos_table && sin_table && q_gamma && q_beta && k_gamma && k_beta,
               "null pointer argument");
  QV_CHECK_ARG(((uintptr_t)cos_table % 16) == 0 && ((uintptr_t)sin_table % 16) == 0 &&
                   ((uintptr_t)positions % 8) == 0,
               "cos/sin tables must be 16-byte and positions 8-byte aligned");
  QV_CHECK_ARG(((uintptr_t)q_gamma % 16) == 0 && ((uintptr_t)q_beta % 16) == 0 && ((uintptr_t)k_gamma % 16) == 0 &&
                   ((uintptr_t)k_beta % 16) == 0,
               "norm weights must be 16-byte aligned");
  if (M == 0) return QV_OK;
  const int tile = w4_pick_tile((int)M, (int)N, (int)K);
  if (tile == 5) {  // skinny M: the projection, then the standalone q/k-norm + RoPE pass
    rc = qv_w4a16_gemm(x, qweight, scales, scaled_zeros, bias, out, M, N, K, QV_F16, QV_EPI_BIAS, stream);
    if (rc) return rc;
    return qv_qknorm_rope2d(out, positions, cos_table, sin_table, table_rows, q_gamma, q_beta, k_gamma, k_beta,
                            eps, M, H, N, stream);
  }
  QkRopeArgs a;
  a.pos = positions;
  a.cos_t = cos_table;
  a.sin_t = sin_table;
  a.qg = (const uint16_t*)q_gamma;
  a.qb = (const uint16_t*)q_beta;
  a.kg = (const uint16_t*)k_gamma;
  a.kb = (const uint16_t*)k_beta;
  a.P = (int)table_rows;
  a.qk_cols = (int)(2 * H * 64);
  a.eps = eps;
  return launch_w4a16_stream<false>(x, qweight, scales, scaled_zeros, bias, nullptr, out, (int)M, (int)N, (int)K,
                                    QV_EPI_QKROPE, w4_plan_for(tile, (int)M, (int)N, (int)K, QV_EPI_QKROPE),
                                    (hipStream_t)stream, &a);
}

extern "C" int qv_w4a16_plan(int64_t M, int64_t N, int64_t K, int epilogue, int32_t* plan) {
  QV_CHECK_ARG(plan != nullptr, "null plan pointer");
  QV_CHECK_ARG(M > 0 && N > 0 && K > 0 && K % 128 == 0 && N % 16 == 0 && M <= INT32_MAX && N <= INT32_MAX &&
                   K <= INT32_MAX,
               "bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  QV_CHECK_ARG(epilogue >= QV_EPI_NONE && epilogue <= QV_EPI_GELU, "bad epilogue %d", epilogue);
  const int tile = w4_pick_tile((int)M, (int)N, (int)K);
  if (tile == 5) {
    plan[0] = 0;
    plan[1] = plan[2] = plan[3] = 0;
    return QV_OK;
  }
  const StreamPlan p = w4_plan_for(tile, (int)M, (int)N, (int)K, epilogue);
  plan[0] = p.ksplit ? 2 : (p.sub == 2 ? 3 : 1);
  plan[1] = 32 * p.mt_a;
  plan[2] = p.mt_b ? p.rows_a : (int32_t)M;
  plan[3] = 32 * p.mt_b;
  return QV_OK;
}

extern "C" int qv_w4a16_gemm_noalloc(const void* x, const void* qweight, const void* scales,
                                     const void* scaled_zeros, const void* bias, void* out, int64_t M,
                                     int64_t N, int64_t K, int dtype, int epilogue, void* stream) {
  int rc = check_common(x, qweight, scales, scaled_zeros, bias, out, M, N, K, dtype, epilogue);
  if (rc) return rc;
  if (M == 0) return QV_OK;
  hipStream_t st = (hipStream_t)stream;
  if (w4_pick_tile((int)M, (int)N, (int)K) != 5) {   // the large-M kernels use no scratch
    if (dtype == QV_BF16)
      return launch_gemm<true>(x, qweight, scales, scaled_zeros, bias, out, (int)M, (int)N, (int)K, epilogue, st);
    return launch_gemm<false>(x, qweight, scales, scaled_zeros, bias, out, (int)M, (int)N, (int)K, epilogue, st);
  }
  // The skinny path splits K into the scratch when its plan fits there
  // (w4_skinny_plan runs every other shape unsplit, as qv_w4a16_gemm does).
  SplitWorkspace ws;
  rc = scratch_workspace(st, ws);
  if (rc) return rc;
  if (dtype == QV_BF16)
    return launch_skinny<true>(x, qweight, scales, scaled_zeros, bias, out, (int)M, (int)N, (int)K, epilogue, st,
                               nullptr, ws);
  return launch_skinny<false>(x, qweight, scales, scaled_zeros, bias, out, (int)M, (int)N, (int)K, epilogue, st,
                              nullptr, ws);
}
