// Flash attention (fp16 in/out, fp32 softmax and accumulation, head_dim 64,
// no mask) for VGGT's frame and global attention on gfx950.
//
// Sequences: B sequences of L tokens each (frame attention: B = frames,
// L = 1374; global attention: B = 1, L = frames * 1374).  q/k/v/out are
// token-major with arbitrary token strides and head stride 64, so q, k and v
// can be read straight out of the fused qkv projection output.
//
// Workgroup: ATT_WAVES waves, 64 queries each (64 * ATT_WAVES queries of one
// (sequence, head)).
// Per 64-key tile a wave computes S^T = K Q^T for its two 32-query blocks
// (2 x 2 x 4 v_mfma_f32_32x32x16_f16, every K fragment read from LDS feeding
// both blocks), the online softmax in registers, and O^T += V^T P^T (16 more
// MFMAs, each V^T fragment again feeding both blocks).
// The softmax is trimmed to what the MFMAs cannot hide: key masking only on
// the last (partial) tile; Q pre-scaled by scale * log2(e) and the score
// accumulators started at -m (the running reference), so P = 2^S takes one
// exp2 per score and nothing else; row sums by v_dot2 on the fp16 P values;
// and a lazy rescale -- the reference moves only when a tile exceeds it by
// 2^8, so most tiles skip the O *= alpha pass, and the tile maximum itself is
// only computed when a lane's tile sum says some P may have exceeded 2^8.
// Layouts:
//  * S^T layout: lane (h = lane/32, q = lane%32) holds, for key block kb,
//    keys 32kb + 8*(r/4) + 4h + r%4 (r = 0..15) of query q.  A query's 64
//    scores are split between lanes q and q+32: one cross-lane exchange per
//    max / sum.
//  * P^T is the PV B operand without any shuffle: k-step s = 2kb + p takes
//    registers 8p..8p+7 of block kb, i.e. keys 32kb + 16p + {0..3, 8..11} + 4h.
//  * K and V tiles arrive by LDS DMA in their natural [key][dim] layout
//    (128-byte rows; 16-byte chunk c of row r at c ^ fk(r) for K and
//    c ^ fv(r) for V), one DMA tile ahead.  In the 4-wave form a DMA tile
//    holds 128 keys, consumed as two 64-key compute tiles, so the workgroup
//    meets at one barrier per 128 keys (1-2 % faster than one per 64,
//    bit-identical); the 2-wave form copies 64-key tiles.
//  * V^T (the PV A operand) comes out of LDS through ds_read_b64_tr_b16: two
//    transposed 8-byte reads give each lane its dim's 8 keys in k-slot order,
//    with no register staging or transposed stores.
#include "common.h"

namespace qv {

constexpr int ATT_QW = 64;                 // queries per wave (two 32-query blocks)
constexpr int ATT_BK = 64;                 // keys per compute tile
// The kernel's two forms (template WAVES, SUB): 4 waves per workgroup with
// 128-key DMA tiles (64 KB of K / V buffers, two workgroups per CU), and, for
// launches that would not fill one round of those, 2 waves with 64-key DMA
// tiles (32 KB, four workgroups per CU), which spreads the queries over twice
// as many workgroups (bit-identical: the key order of every query is the
// same; 4 x 1374 frame tokens 0.5-5 % and one 5496-token sequence 1.8 %
// faster, two boxes).  At 8 x 1374 (1.5 rounds of the 4-wave form) the
// 2-wave form was 7-8 % slower: twice the K / V copies per query and a
// barrier per 64 keys.

constexpr float RESCALE_SLACK = 8.0f;  // log2 units: P <= 256 between rescales
constexpr float P_SUM_LIMIT = 256.0f;  // 2^RESCALE_SLACK: a lane's tile sum above it may hide a P above it

__device__ __forceinline__ int fk(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// V rows swizzle: 16-byte chunk c of key row r sits at c ^ fv(r).  The
// transposed reads below touch 4 consecutive rows per 16-lane group; fv moves
// rows r and r + 2 to opposite halves of the 128-byte row, so each 32-lane
// half of a read covers all 64 banks once.
__device__ __forceinline__ int fv(int r) { return 4 * ((r >> 1) & 1); }

typedef short v4i16 __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16: within each 16-lane group, lane j = 4a + b receives
// element b of the 8-byte segments addressed by lanes a, a + 4, a + 8, a + 12.
__device__ __forceinline__ uint2 lds_read_tr16(const uint8_t* p) {
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16*)(__attribute__((address_space(3))) uint8_t*)p);
  return __builtin_bit_cast(uint2, r);
}

// max / sum of x over lanes l and l ^ 32.  v_permlane32_swap exchanges the
// upper half of its first operand with the lower half of its second; with
// both holding x, lane l ends with {x[l & 31], x[(l & 31) + 32]} in the pair.
// Written as inline asm: the compiler's model of the builtin folds the two
// results into one when both operands carry the same value.  The s_nop
// covers the VALU-write -> permlane-read hazard.
__device__ __forceinline__ void half_pair(float x, float& a, float& b) {
  a = x;
  b = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float half_max(float x) {
  float a, b;
  half_pair(x, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float half_sum(float x) {
  float a, b;
  half_pair(x, a, b);
  return a + b;
}

template <int WAVES, int SUB>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(2, 2))) void attention_fwd_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    uint16_t* __restrict__ out, int L, int H, long q_ts, long kv_ts, long v_ts, long o_ts, float scale_log2) {
  constexpr int ATT_WAVES = WAVES;               // waves per workgroup
  constexpr int ATT_BQ = ATT_WAVES * ATT_QW;     // queries per workgroup
  constexpr int ATT_SUB = SUB;                   // compute tiles per DMA tile (one barrier per DMA tile)
  constexpr int ATT_BKD = ATT_BK * ATT_SUB;      // keys per DMA tile
  constexpr int ATT_DMA = ATT_BKD / 8 / ATT_WAVES;  // 1 KB (8-key) DMA rows per wave per DMA tile, K and V each
  static_assert(ATT_DMA * 8 * ATT_WAVES == ATT_BKD, "DMA rows split evenly over the waves");
  __shared__ __attribute__((aligned(1024))) uint8_t k_lds[2][ATT_BKD * 128];
  __shared__ __attribute__((aligned(1024))) uint8_t v_lds[2][ATT_BKD * 128];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;
  const int qtiles = (L + ATT_BQ - 1) / ATT_BQ;
  // consecutive q-tiles of one (sequence, head) share an XCD (and its L2),
  // which then streams that head's K / V once for all of them
  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = lid % qtiles;
  const int head = (lid / qtiles) % H;
  const int seq = lid / (qtiles * H);
  const long tok0 = (long)seq * L;
  const bool live = qt * ATT_BQ + wave * ATT_QW < L;   // wave-uniform

  // ---- Q^T fragments (B operand of S^T = K Q^T): per query block, 4 k-steps of 16 dims
  uint4 qf[2][4];
  int qi[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    qi[qb] = qt * ATT_BQ + wave * ATT_QW + 32 * qb + l32;     // query index in the sequence
    const int qc = qi[qb] < L ? qi[qb] : L - 1;
    const uint16_t* qp = q + (tok0 + qc) * q_ts + (long)head * 64;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      // pre-scaled by scale * log2(e) (one fp16 rounding), so the MFMA yields
      // scores in log2 units and the softmax needs no per-score multiply
      const uint4 raw = *reinterpret_cast<const uint4*>(qp + 16 * s + 8 * h);
      const uint32_t rw[4] = {raw.x, raw.y, raw.z, raw.w};
      uint32_t sw[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f16x2 hv = __builtin_bit_cast(f16x2, rw[e]);
        const f16x2 sv = {(_Float16)((float)hv[0] * scale_log2), (_Float16)((float)hv[1] * scale_log2)};
        sw[e] = __builtin_bit_cast(uint32_t, sv);
      }
      qf[qb][s] = make_uint4(sw[0], sw[1], sw[2], sw[3]);
    }
  }

  // ---- K tile DMA: 16 x 1 KB per DMA tile, 4 per wave; lane L lands at key
  // r0 + L/8, physical chunk L%8, so it fetches logical chunk (L%8) ^ fk(row).
  const auto rsK = make_rsrc(k + tok0 * kv_ts + (long)head * 64, (uint64_t)L * kv_ts * 2);
  uint32_t k_voff[ATT_DMA];
#pragma unroll
  for (int w2 = 0; w2 < ATT_DMA; ++w2) {
    const int row = 8 * (ATT_DMA * wave + w2) + (lane >> 3);
    const int c = (lane & 7) ^ fk(row);
    k_voff[w2] = (uint32_t)((lane >> 3) * kv_ts * 2 + c * 16);
  }
  const uint32_t klds0 = lds_addr(k_lds);
  auto issue_k = [&](int tile, int buf) {
#pragma unroll
    for (int w2 = 0; w2 < ATT_DMA; ++w2) {
      const int r0 = 8 * (ATT_DMA * wave + w2);
      lds_dma16(rsK, k_voff[w2], (uint32_t)((tile * ATT_BKD + r0) * kv_ts * 2),
                klds0 + buf * (ATT_BKD * 128) + r0 * 128);
    }
  };
  // ---- V tile DMA, natural [key][dim] layout with the fv swizzle
  const auto rsV = make_rsrc(v + tok0 * v_ts + (long)head * 64, (uint64_t)L * v_ts * 2);
  uint32_t v_voff[ATT_DMA];
#pragma unroll
  for (int w2 = 0; w2 < ATT_DMA; ++w2) {
    const int row = 8 * (ATT_DMA * wave + w2) + (lane >> 3);
    const int c = (lane & 7) ^ fv(row);
    v_voff[w2] = (uint32_t)((lane >> 3) * v_ts * 2 + c * 16);
  }
  const uint32_t vlds0 = lds_addr(v_lds);
  auto issue_v = [&](int tile, int buf) {
#pragma unroll
    for (int w2 = 0; w2 < ATT_DMA; ++w2) {
      const int r0 = 8 * (ATT_DMA * wave + w2);
      lds_dma16(rsV, v_voff[w2], (uint32_t)((tile * ATT_BKD + r0) * v_ts * 2),
                vlds0 + buf * (ATT_BKD * 128) + r0 * 128);
    }
  };
  // Transposed V^T fragments: for k-step st (keys 16 st + {0..3, 8..11} + 4h
  // in k-slot order) and dim block db, lane (group G = lane / 16, i = lane % 16)
  // addresses key 16 st + 8 r + 4h + i / 4, dims 32 db + 16 (G & 1) + 4 (i & 3)
  // for reads r = 0, 1; the transpose hands lane l32 its dim's 8 keys.
  const int tr_key = 4 * h + ((lane & 15) >> 2);
  const int tr_dim = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const int ntiles = (L + ATT_BKD - 1) / ATT_BKD;   // DMA tiles
  f32x16 o[2][2];   // [query block][dim block]
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[qb][db][r] = 0.f;
  // m_use: the running reference maximum in log2 units.  It is only raised
  // when a tile's maximum exceeds it by more than RESCALE_SLACK, so P values
  // stay <= 2^RESCALE_SLACK and most tiles skip the O rescale.
  float m_use[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
  // base: the reference the score accumulators start from (S' = S - base,
  // the MFMA's C input), equal to m_use after the first tile, so P = 2^S'
  // needs one exp2 per score and nothing else
  float base[2] = {0.f, 0.f};
  const f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};

  // one 64-key compute tile: keys key0.., K / V rows at kb_lds / vb
  auto ctile = [&](int key0, const uint8_t* kb_lds, const uint8_t* vb, bool mask) __attribute__((always_inline)) {
    {
      // ---- S^T = K Q^T for the 64 keys of the tile, both query blocks (raw dot products)
      f32x16 sc[2][2];   // [query block][key block]
  #pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int row = 32 * kb + l32;
  #pragma unroll
        for (int st = 0; st < 4; ++st) {
          const int c = 2 * st + h;
          const uint4 kf = *reinterpret_cast<const uint4*>(kb_lds + row * 128 + ((c ^ fk(row)) * 16));
  #pragma unroll
          for (int qb = 0; qb < 2; ++qb)
            sc[qb][kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                __builtin_bit_cast(f16x8, kf), __builtin_bit_cast(f16x8, qf[qb][st]),
                st == 0 ? f32x16{} - base[qb] : sc[qb][kb], 0, 0, 0);
        }
      }
      // ---- V^T fragments of this tile, read before the softmax so their LDS
      // latency hides behind it (the PV MFMAs below consume them)
      uint4 vfr[2][4];
  #pragma unroll
      for (int db = 0; db < 2; ++db) {
        const int dim = 32 * db + tr_dim;
  #pragma unroll
        for (int st = 0; st < 4; ++st) {
          uint2 vv[2];
  #pragma unroll
          for (int r = 0; r < 2; ++r) {
            const int key = 16 * st + 8 * r + tr_key;
            vv[r] = lds_read_tr16(vb + key * 128 + (((dim >> 3) ^ fv(key)) * 16) + ((dim >> 2) & 1) * 8);
          }
          vfr[db][st] = make_uint4(vv[0].x, vv[0].y, vv[1].x, vv[1].y);
        }
      }
      uint4 pf[2][4];
  #pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        if (mask) {
          const int kh = key0 + 4 * h;
  #pragma unroll
          for (int kb = 0; kb < 2; ++kb)
  #pragma unroll
            for (int r = 0; r < 16; ++r)
              if (kh + 32 * kb + 8 * (r >> 2) + (r & 3) >= L) sc[qb][kb][r] = -INFINITY;
        }
        // ---- P = 2^S' = 2^(S - m_use) in fp16 against the current reference,
        // with this tile's partial row sum t (v_dot2 on the fp16 values).  The
        // tile maximum is only needed when some P could exceed 2^RESCALE_SLACK,
        // and every such P makes t exceed it too (P >= 0), so the maximum is
        // computed only for waves where some lane's t does, and on the first
        // tile (no reference yet).
        float t = 0.f;
        auto make_p = [&](bool shift, float off) {
  #pragma unroll
          for (int kb = 0; kb < 2; ++kb)
  #pragma unroll
            for (int pp = 0; pp < 2; ++pp) {
              uint32_t w[4];
  #pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float s0 = sc[qb][kb][8 * pp + 2 * e], s1 = sc[qb][kb][8 * pp + 2 * e + 1];
                const float p0 = __builtin_amdgcn_exp2f(shift ? s0 + off : s0);
                const float p1 = __builtin_amdgcn_exp2f(shift ? s1 + off : s1);
                const f16x2 ph = {(_Float16)p0, (_Float16)p1};
                t = __builtin_amdgcn_fdot2(ph, ones, t, false);
                w[e] = __builtin_bit_cast(uint32_t, ph);
              }
              pf[qb][2 * kb + pp] = make_uint4(w[0], w[1], w[2], w[3]);
            }
        };
        make_p(false, 0.f);
        if (__builtin_amdgcn_ballot_w64(!(t <= P_SUM_LIMIT) || m_use[qb] == -INFINITY)) {
          // ---- tile maximum of this query (both lane halves hold 32 keys each)
          float mx = sc[qb][0][0];
  #pragma unroll
          for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sc[qb][0][r]);
  #pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[qb][1][r]);
          mx = half_max(mx) + base[qb];
          // ---- lazy rescale: the reference moves when the tile maximum exceeds
          // it by more than the slack; then P is recomputed against it
          const bool need = mx > m_use[qb] + RESCALE_SLACK;
          if (__builtin_amdgcn_ballot_w64(need)) {
            const float m_new = need ? mx : m_use[qb];
            const float alpha = __builtin_amdgcn_exp2f(m_use[qb] - m_new);  // 0 on the first tile, 1 if !need
            m_use[qb] = m_new;
            l_run[qb] *= alpha;
  #pragma unroll
            for (int db = 0; db < 2; ++db)
  #pragma unroll
              for (int r = 0; r < 16; ++r) o[qb][db][r] *= alpha;
            t = 0.f;
            make_p(true, base[qb] - m_new);
          }
          base[qb] = m_use[qb];
        }
        l_run[qb] += t;
        // ---- O^T += V^T P^T for this query block (each V^T fragment feeds
        // both blocks), issued before the next block's softmax so these
        // MFMAs run under its VALU work
  #pragma unroll
        for (int db = 0; db < 2; ++db)
  #pragma unroll
          for (int st = 0; st < 4; ++st)
            o[qb][db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, vfr[db][st]),
                                                              __builtin_bit_cast(f16x8, pf[qb][st]), o[qb][db], 0, 0, 0);
      }
    }
  };
  auto tile = [&](int j, bool last) {
    const int buf = j & 1;
    const bool more = j + 1 < ntiles;
    if (more) {
      issue_k(j + 1, buf ^ 1);
      issue_v(j + 1, buf ^ 1);
    }
    // a wave whose 64 queries all lie past the sequence end (the last query
    // tile of a frame) only issues its share of the DMA and keeps the barriers
    if (live) {
#pragma unroll
      for (int u = 0; u < ATT_SUB; ++u) {
        const int key0 = j * ATT_BKD + u * ATT_BK;
        if (!last) {
          ctile(key0, k_lds[buf] + u * ATT_BK * 128, v_lds[buf] + u * ATT_BK * 128, false);
        } else if (key0 < L) {
          ctile(key0, k_lds[buf] + u * ATT_BK * 128, v_lds[buf] + u * ATT_BK * 128, key0 + ATT_BK > L);
        }
      }
    }
    if (more) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): next K and V tiles landed
    lds_barrier();
  };

  issue_k(0, 0);
  issue_v(0, 0);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  lds_barrier();
  const int nfull = L / ATT_BKD;       // DMA tiles with every key valid
  for (int j = 0; j < nfull; ++j) tile(j, false);
  if (nfull < ntiles) tile(nfull, true);

  // ---- normalise and store: lane (h, q) holds dims 32db + 8*(r/4) + 4h + r%4
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float l_tot = half_sum(l_run[qb]);
    const float inv = 1.0f / l_tot;
    if (qi[qb] < L) {
      uint16_t* op = out + (tok0 + qi[qb]) * o_ts + (long)head * 64;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          uint2 w;
          w.x = pack2<false>(o[qb][db][4 * g] * inv, o[qb][db][4 * g + 1] * inv);
          w.y = pack2<false>(o[qb][db][4 * g + 2] * inv, o[qb][db][4 * g + 3] * inv);
          *reinterpret_cast<uint2*>(op + 32 * db + 8 * g + 4 * h) = w;
        }
    }
  }
}

}  // namespace qv

extern "C" int qv_attention_fwd(const void* q, const void* k, const void* v, void* out, int64_t B, int64_t L,
                                int64_t H, int64_t head_dim, int64_t q_token_stride, int64_t k_token_stride,
                                int64_t v_token_stride, int64_t out_token_stride, float scale, void* stream) {
  QV_CHECK_ARG(head_dim == 64, "only head_dim 64 is supported (got %lld)", (long long)head_dim);
  QV_CHECK_ARG(B >= 0 && L >= 0 && H > 0, "bad shape B=%lld L=%lld H=%lld", (long long)B, (long long)L, (long long)H);
  if (B == 0 || L == 0) return QV_OK;
  QV_CHECK_ARG(q && k && v && out, "null pointer argument");
  QV_CHECK_ARG(q_token_stride % 8 == 0 && k_token_stride % 8 == 0 && v_token_stride % 8 == 0 &&
                   out_token_stride % 4 == 0 && q_token_stride >= H * 64 && k_token_stride >= H * 64 &&
                   v_token_stride >= H * 64 && out_token_stride >= H * 64,
               "token strides must cover the heads and keep 16-byte alignment");
  QV_CHECK_ARG(((uintptr_t)q % 16) == 0 && ((uintptr_t)k % 16) == 0 && ((uintptr_t)v % 16) == 0 &&
                   ((uintptr_t)out % 8) == 0,
               "q, k, v must be 16-byte and out 8-byte aligned");
  QV_CHECK_ARG((uint64_t)L * k_token_stride * 2 < (1ull << 32) && (uint64_t)L * v_token_stride * 2 < (1ull << 32),
               "sequence too long for 32-bit offsets");
  // 4-wave workgroups (256 queries) when they fill at least one round of
  // the 512 workgroup slots (two per CU); else 2-wave workgroups
  const long qtiles4 = (L + 4 * qv::ATT_QW - 1) / (4 * qv::ATT_QW);
  const bool wide = B * H * qtiles4 >= 512;
  const long bq = wide ? 4 * qv::ATT_QW : 2 * qv::ATT_QW;
  const long nwg = B * H * ((L + bq - 1) / bq);
  QV_CHECK_ARG(nwg <= INT32_MAX, "grid too large");
  const float scale_log2 = scale * 1.4426950408889634f;
#define QV_ATT_ARGS                                                                                       \
  (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)out, (int)L, (int)H, (long)q_token_stride, \
      (long)k_token_stride, (long)v_token_stride, (long)out_token_stride, scale_log2
  if (wide)
    hipLaunchKernelGGL((qv::attention_fwd_kernel<4, 2>), dim3((unsigned)nwg), dim3(256), 0, (hipStream_t)stream,
                       QV_ATT_ARGS);
  else
    hipLaunchKernelGGL((qv::attention_fwd_kernel<2, 1>), dim3((unsigned)nwg), dim3(128), 0, (hipStream_t)stream,
                       QV_ATT_ARGS);
#undef QV_ATT_ARGS
  return qv::check_launch("attention_fwd");
}
