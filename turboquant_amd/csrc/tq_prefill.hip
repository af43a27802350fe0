// tq_prefill.hip -- causal GQA flash attention of a prefill chunk (fp16 K/V,
// head size 64, 128 or 256).
//
// Semantics: o[i, h] = softmax_j(q[i, h] . k[j, h / ratio] * sm_scale) v[j, h / ratio]
// over keys j <= (Lk - Lq) + i (causal, aligned to the end of the keys: a
// chunk of Lq new tokens whose keys are the Lk - Lq earlier tokens of its
// sequence followed by its own).  This is the attention the backend's prefill
// path needs (reference turboquant/vllm_backend_fused.py:335-371 runs it over
// the fresh chunk only, in flash-attn; TurboQuantFusedImpl here prepends the
// cached context read back from the quantized cache).
//
// gfx950 design:
//  * One workgroup = 32 NW query rows of one q head (NW waves x 32 rows,
//    NW = 8 when the grid of such blocks still fills the CUs, else 4); grid
//    (q heads, query blocks): the longest (last) query blocks are dispatched
//    first, and the q heads of one kv head are neighbours (their K/V tiles
//    are shared in L2).  Eight waves (one workgroup per CU at two waves per
//    SIMD) copy each K/V tile into LDS once for 256 rows instead of twice
//    for two workgroups of 128, and take 128-key tiles in the LDS that frees
//    (half the per-tile max, rescale and barrier steps): 7-9% faster on long
//    prompts than the four-wave, 64-key shape.
//  * Scores are computed transposed, S^T = K Q^T, with
//    v_mfma_f32_32x32x16_f16 (A = K rows from LDS, B = q columns held in
//    registers for the whole kernel): the C layout then gives each lane one
//    query row (lane % 32) and 16 key rows per 32-key block, so the softmax
//    max and sum are in-lane plus one permlane32 swap, and the lane's
//    probabilities are, in order, the B operand of O^T = V^T P^T (the MFMA's
//    reduction order is the C layout's row order; V^T is read in the same
//    order).  O^T's C layout again gives each lane its own query row, so the
//    online-softmax rescale is a per-lane scalar.
//  * K and V tiles (64 or 128 keys) stream into LDS as rows with
//    direct-to-LDS 16-byte copies, their 16-byte chunks XOR-swizzled by row:
//    the K reads (16 bytes of one row per lane, issued four MFMAs ahead of
//    their use) and the V transpose reads (ds_read_b64_tr_b16: four keys of
//    one dim per lane, the V^T operand without a transposing copy) are
//    conflict-free.  Two buffers of each (distinct LDS arrays, so the
//    compiler does not wait for the copies in flight into the other buffer),
//    one barrier per tile.
//  * Short chunks over long contexts (too few query blocks to fill the
//    CUs): each query block's tiles are split over several workgroups
//    (grid z), which leave their normalised O (fp16), reference max and row
//    sum in a caller-owned workspace; prefill_merge_kernel combines them.
//  * Online softmax in the exp2 domain with a lazy rescale (the running max
//    moves only when a tile exceeds it by more than 8 / scale); probabilities
//    enter the PV MFMA as fp16 (round to nearest), accumulation is fp32;
//    at head size 64 the row sum is taken from those fp16 values.
#include <atomic>

#include "tq_common.h"

namespace tq {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// two floats as an fp16 pair, round to nearest even (one v_cvt_pk_f16_f32)
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, half2_t));
}

constexpr int kBNmax = 128;  // largest tile (keys)

struct PrefillParams {
  const _Float16* q;
  const _Float16* k;
  const _Float16* v;
  _Float16* o;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh;  // strides in elements
  int lq, lk, ratio, nqb;
  float c;  // sm_scale * log2(e)
  // split-KV mode: workgroup z of a (head, query block) covers its tiles
  // [z tps, (z + 1) tps) and leaves its rows' O / row sum (fp16) and
  // (reference max in log2 units, row sum) in the workspace for
  // prefill_merge_kernel
  int nsplit, tps;
  _Float16* ws_o;  // [nsplit][lq][Hq][D]
  float* ws_ml;    // [nsplit][lq][Hq][2]
};

// max / sum of x over lanes l and l ^ 32: v_permlane32_swap of x with
// itself returns (x, x of lane l ^ 32) in some order in every lane
__device__ __forceinline__ float max32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// WPE: waves per SIMD the register budget is sized for (2 at head size 64
// and 128; 1 at 256, whose q operand and output accumulators alone take 192
// registers per lane)
template <int kD, int NW, int kBN, bool SPLIT, int WPE = 2>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void prefill_kernel(PrefillParams p) {
  constexpr int kKRow = kD * 2;       // bytes of one K row in LDS
  constexpr int kCH = kD / 8;         // 16-byte chunks per K row
  constexpr int kRPC = 1024 / kKRow;  // K rows per 1 KB copy
  constexpr int kBM = 32 * NW;  // query rows per workgroup
  constexpr int kNU = kBN / 32, kNS = kBN / 16;  // 32-key score blocks, 16-key PV steps
  // 64-byte quarters of a row the V swizzle rotates over (D >= 128: four;
  // 64: two)
  constexpr int kQS = kD >= 128 ? 0 : 1;  // row % 4 >> kQS selects the quarter
  __shared__ __attribute__((aligned(16))) uint8_t kbuf0[kBN * kKRow];
  __shared__ __attribute__((aligned(16))) uint8_t kbuf1[kBN * kKRow];
  __shared__ __attribute__((aligned(16))) uint8_t vbuf0[kBN * kKRow];
  __shared__ __attribute__((aligned(16))) uint8_t vbuf1[kBN * kKRow];

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int hh = lane >> 5, n = lane & 31;
  const int qb = p.nqb - 1 - (int)blockIdx.y;
  const int head = blockIdx.x, g = head / p.ratio;
  const int q0 = qb * kBM;
  const int off = p.lk - p.lq;
  const int qrow = q0 + 32 * w + n;  // this lane's query row
  const int kend = min(p.lk, off + min(q0 + kBM, p.lq));  // keys any row here sees
  const int ntiles = (kend + kBN - 1) / kBN;

  // q^T as the B operand of S^T = K Q^T: k-step s covers dims 16s .. 16s+15,
  // lane (hh, n) holds dims 16s + 8hh .. +7 of query row qrow
  half8_t qB[kD / 16];
  {
    const _Float16* qp = p.q + (int64_t)qrow * p.q_st + (int64_t)head * p.q_sh + 8 * hh;
#pragma unroll
    for (int s = 0; s < kD / 16; s++) {
      u32x4 x = {0u, 0u, 0u, 0u};
      if (qrow < p.lq) x = *reinterpret_cast<const u32x4*>(qp + 16 * s);
      qB[s] = __builtin_bit_cast(half8_t, x);
    }
  }

  // K and V copies: copy j fills LDS bytes [1024 j, 1024 j + 1024) of a
  // buffer = rows kRPC j .. kRPC j + kRPC - 1; lane l writes row
  // kRPC j + l / kCH, physical 16-byte chunk l % kCH.  K rows hold logical
  // chunk (l % kCH) ^ (row % kCH) there (the score MFMAs' A reads, 16 bytes
  // of one row per lane, hit distinct chunks); V rows hold logical chunk
  // (l % kCH) ^ 4 ((row % 4) >> kQS), which moves the 64-byte quarters of
  // four consecutive rows apart for the transpose reads of the PV MFMAs (and
  // lets their addresses be a per-lane base xor 64 d plus an immediate).
  // Wave w issues copies j = w + NW i of both.
  constexpr int kKC = (kBN / kRPC) / NW;  // copies per wave, tile and tensor
  const int kst_b = (int)(p.k_st * 2), vst_b = (int)(p.v_st * 2);
  uint32_t koff[kKC], voff[kKC];  // per-lane byte offsets of this wave's copies in a tile
#pragma unroll
  for (int i = 0; i < kKC; i++) {
    const int j = w + NW * i, row = kRPC * j + lane / kCH;
    koff[i] = (uint32_t)(row * kst_b + (((lane % kCH) ^ (row % kCH)) * 16));
    voff[i] = (uint32_t)(row * vst_b + (((lane % kCH) ^ (4 * ((row & 3) >> kQS))) * 16));
  }
  // buffer resource over rows [kb, Lk) of a K or V tile (wave-uniform base
  // and size; rows past Lk read as zeros)
  auto tile_rsrc = [&](const _Float16* base, int64_t st, int kb) {
    const int rows = min(kBN, p.lk - kb);
    const uint64_t a = (uint64_t)(uintptr_t)(base + (int64_t)kb * st);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    const int nrec = __builtin_amdgcn_readfirstlane(rows * (int)(st * 2));
    return __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)(((uint64_t)hi << 32) | lo),
                                             (short)0, nrec, 0x00020000);
  };
  const _Float16* const kbase = p.k + (int64_t)g * p.k_sh;
  const _Float16* const vbase = p.v + (int64_t)g * p.v_sh;
  auto issue = [&](int kt, uint8_t* kb, uint8_t* vb) {
#if defined(__HIP_DEVICE_COMPILE__)  // the LDS-copy builtin has no host form
    const __amdgpu_buffer_rsrc_t rk = tile_rsrc(kbase, p.k_st, kt * kBN);
    const __amdgpu_buffer_rsrc_t rv = tile_rsrc(vbase, p.v_st, kt * kBN);
#pragma unroll
    for (int i = 0; i < kKC; i++) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (void*)(kb + 1024 * (w + NW * i)), 16,
                                               koff[i], 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (void*)(vb + 1024 * (w + NW * i)), 16,
                                               voff[i], 0, 0, 0);
    }
#else
    (void)kt;
    (void)kb;
    (void)vb;
    (void)tile_rsrc;
    (void)kbase;
    (void)vbase;
#endif
  };
  // PV transpose reads (ds_read_b64_tr_b16): in each 16-lane group gq, source
  // lane s reads 4 halves V[K0 + s/4][D0 + 4 (s % 4) .. +3] and result lane i
  // receives V^T[D0 + i][K0 .. K0 + 3] (D0 = 32 d + 16 (gq % 2), K0 = 16 st +
  // 4 hh, plus 8 for the second read): the A operand of O^T = V^T P^T.
  // vread_base is this lane's byte offset for d = 0, st = 0.
  const int vgq = lane >> 4, vsl = lane & 15, vt4 = vsl >> 2;
  const uint32_t vread_base =
      (uint32_t)((4 * hh + vt4) * kKRow +
                 ((2 * (vgq & 1) + ((vsl & 3) >> 1)) ^ (4 * (vt4 >> kQS))) * 16 + 8 * (vsl & 1));

  f32x16 oacc[kD / 32];
#pragma unroll
  for (int d = 0; d < kD / 32; d++)
#pragma unroll
    for (int j = 0; j < 16; j++) oacc[d][j] = 0.0f;
  float m = -INFINITY, mc = -INFINITY, lsum = 0.0f;
  const int qlim = off + qrow;  // last key of this lane's row

  auto tile = [&](int kt, const uint8_t* kbuf, const uint8_t* vt) {
    const int kb = kt * kBN;
    // the wave's rows are q0 + 32w .. +31: nothing to do when all its keys
    // in this tile are beyond every row (uniform)
    if (kb > off + q0 + 32 * w + 31) return;
    // S^T blocks: MFMA i = s * kNU + u adds k-step s of key block u.  The K
    // fragments are read kKP ahead of their MFMA and the schedule is pinned
    // (one MFMA, then one read): left to itself the compiler issued each
    // read one or two MFMAs ahead and waited for it in full (1.5-2.5% slower)
    constexpr int kKP = 4;
    constexpr int kNI = kNU * (kD / 16);
    f32x16 sacc[kNU];
#pragma unroll
    for (int u = 0; u < kNU; u++)
#pragma unroll
      for (int j = 0; j < 16; j++) sacc[u][j] = 0.0f;
    auto kfrag = [&](int i) {
      const int u = i % kNU, s = i / kNU, row = 32 * u + n;
      return *reinterpret_cast<const u32x4*>(kbuf + row * kKRow +
                                             (((2 * s + hh) ^ (row % kCH)) * 16));
    };
    u32x4 fr[kKP];
#pragma unroll
    for (int j = 0; j < kKP; j++) fr[j] = kfrag(j);
#pragma unroll
    for (int i = 0; i < kNI; i++) {
      const u32x4 a = fr[i % kKP];
      if (i + kKP < kNI) fr[i % kKP] = kfrag(i + kKP);
      sacc[i % kNU] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
          __builtin_bit_cast(half8_t, a), qB[i / kNU], sacc[i % kNU], 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, kKP, 0);  // the first kKP reads
#pragma unroll
    for (int i = 0; i < kNI; i++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA i
      if (i + kKP < kNI) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // read i + kKP
    }
    // mask keys beyond the row (causal) or beyond Lk (uniform test): lim is
    // the lane's last visible key relative to key 4 hh of the tile, and the
    // score at tile key 4 hh + kk gets -inf (the sign bits of lim - kk spread
    // into 0xff800000) or +0 added; no compare masks, so no scalar registers
    // for them
    if (kb + kBN - 1 > off + q0 + 32 * w || kb + kBN > p.lk) {
      const int lim = min(qlim, p.lk - 1) - kb - 4 * hh;
#pragma unroll
      for (int u = 0; u < kNU; u++)
#pragma unroll
        for (int j = 0; j < 16; j++) {
          const int kk = 32 * u + 8 * (j >> 2) + (j & 3);
          sacc[u][j] += __int_as_float(((lim - kk) >> 31) & (int)0xff800000u);
        }
    }
    float tmax = -INFINITY;
#if defined(TQ_PREFILL_PROBE) && TQ_PREFILL_PROBE >= 2
    tmax = sacc[0][0];  // measurement probe: no row max
#else
#pragma unroll
    for (int u = 0; u < kNU; u++)
#pragma unroll
      for (int j = 0; j < 16; j++) tmax = fmaxf(tmax, sacc[u][j]);
    tmax = max32(tmax);
#endif
    const float m_new = fmaxf(m, tmax);
    // lazy rescale: p = exp2((s - m) c) stays below 2^8 between rescales
    if (__builtin_amdgcn_ballot_w64(m_new * p.c > mc + 8.0f) != 0) {
      const float alpha = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mc - m_new * p.c);
#pragma unroll
      for (int d = 0; d < kD / 32; d++) oacc[d] *= alpha;
      lsum *= alpha;
      m = m_new;
      mc = m_new * p.c;
    }
    // a row with no visible key yet (possible in split mode, where a split's
    // first tiles can lie wholly beyond a row) keeps mc = -inf while the
    // wave's ballot above may fire for other rows: its exponent offset is
    // then 0, so its probabilities are exp2(-inf) = 0 instead of NaN, and
    // the split leaves sum 0 and O = 0 for it
    const float mce = mc == -INFINITY ? 0.0f : mc;
    half8_t pB[kNS];  // B operand of O^T = V^T P^T for k-steps (u, t)
#pragma unroll
    for (int u = 0; u < kNU; u++)
#pragma unroll
      for (int t = 0; t < 2; t++) {
        float pr[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
#if defined(TQ_PREFILL_PROBE) && TQ_PREFILL_PROBE >= 1
          pr[i] = __builtin_fmaf(sacc[u][8 * t + i], p.c, -mce);  // measurement probe: no exp2
#else
          pr[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[u][8 * t + i], p.c, -mce));
#endif
          if constexpr (kD != 64) lsum += pr[i];
        }
        u32x4 pk;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const half2_t h = __builtin_convertvector(f32x2{pr[2 * i], pr[2 * i + 1]}, half2_t);
          // head size 64 (two scores per MFMA, the softmax weighs more): the
          // row sum of the fp16 probabilities the PV MFMAs take, two per
          // v_dot2 against (1, 1) with an fp32 accumulator.  (Dot2 of an
          // element extracted from a u32x4 miscompiled here: the same source
          // register for all four; the sum reads the half2 values.)
          if constexpr (kD == 64)
            lsum = __builtin_amdgcn_fdot2(h, half2_t{(_Float16)1.0f, (_Float16)1.0f}, lsum, false);
          pk[i] = __builtin_bit_cast(uint32_t, h);
        }
        pB[2 * u + t] = __builtin_bit_cast(half8_t, pk);
      }
    // O^T += V^T P^T: k-step (u, t) reduces keys 32u + 16t + {4hh + 0..3,
    // 8 + 4hh + 0..3} (the C-layout rows of the lane's probabilities)
#pragma unroll
    for (int st = 0; st < kNS; st++) {
#pragma unroll
      for (int d = 0; d < kD / 32; d++) {
        typedef __attribute__((address_space(3))) uint8_t lds_u8;
        typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
        lds_u8* const pd = (lds_u8*)vt + (vread_base ^ (uint32_t)(64 * d)) + 16 * st * kKRow;
        const u32x2 a0 =
            __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)pd));
        const u32x2 a1 = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(pd + 8 * kKRow)));
        const u32x4 a = {a0[0], a0[1], a1[0], a1[1]};
        oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a), pB[st],
                                                         oacc[d], 0, 0, 0);
      }
    }
  };

  // this workgroup's tiles: all of them, or split z's share
  int t0 = 0, t1 = ntiles;
  if constexpr (SPLIT) {
    t0 = (int)blockIdx.z * p.tps;
    t1 = min(ntiles, t0 + p.tps);
  }
  if (t0 < t1) issue(t0, kbuf0, vbuf0);
  for (int kt = t0; kt < t1; kt += 2) {
    // tile kt: buffers 0
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's copies of tile kt
    __syncthreads();                     // everyone's copies of tile kt
    if (kt + 1 < t1) issue(kt + 1, kbuf1, vbuf1);
    tile(kt, kbuf0, vbuf0);
    if (kt + 1 >= t1) break;
    // tile kt + 1: buffers 1
    __builtin_amdgcn_s_waitcnt(0x0f70);
    __syncthreads();
    if (kt + 2 < t1) issue(kt + 2, kbuf0, vbuf0);
    tile(kt + 1, kbuf1, vbuf1);
  }

  if constexpr (SPLIT) {
    // this split's O / row sum (a convex combination of V rows: fp16 is
    // safe) and (mc, row sum); a split that held no visible key for a row
    // leaves mc = -inf, sum 0, O = 0
    lsum = sum32(lsum);
    if (qrow < p.lq) {
      const int64_t r = ((int64_t)blockIdx.z * p.lq + qrow) * gridDim.x + head;
      const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
      _Float16* const wo = p.ws_o + r * kD + 4 * hh;
#pragma unroll
      for (int d = 0; d < kD / 32; d++)
#pragma unroll
        for (int jq = 0; jq < 4; jq++) {
          const uint32_t lo = pack_h2(oacc[d][4 * jq] * inv, oacc[d][4 * jq + 1] * inv);
          const uint32_t hi = pack_h2(oacc[d][4 * jq + 2] * inv, oacc[d][4 * jq + 3] * inv);
          *reinterpret_cast<u32x2*>(wo + 32 * d + 8 * jq) = u32x2{lo, hi};
        }
      if (hh == 0) *reinterpret_cast<f32x2*>(p.ws_ml + 2 * r) = f32x2{mc, lsum};
    }
    return;
  }

  // o = O / sum, lane (hh, n) holds dims 32d + 8jq + 4hh + 0..3 of row qrow
  lsum = sum32(lsum);
  if (qrow < p.lq) {
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    _Float16* op = p.o + (int64_t)qrow * p.o_st + (int64_t)head * p.o_sh + 4 * hh;
#pragma unroll
    for (int d = 0; d < kD / 32; d++)
#pragma unroll
      for (int jq = 0; jq < 4; jq++) {
        const uint32_t lo = pack_h2(oacc[d][4 * jq] * inv, oacc[d][4 * jq + 1] * inv);
        const uint32_t hi = pack_h2(oacc[d][4 * jq + 2] * inv, oacc[d][4 * jq + 3] * inv);
        *reinterpret_cast<u32x2*>(op + 32 * d + 8 * jq) = u32x2{lo, hi};
      }
  }
}

// The same attention with RB row blocks of 32 query rows per wave: each K
// fragment and each V^T fragment read from LDS feeds RB MFMAs instead of
// one, so a tile's LDS reads per MFMA drop by RB.  Non-split only.  Row block
// rb of wave w holds rows q0 + 32 (RB w + rb) + n.  Used at head size 64
// (RB 2, 64-key tiles: 217 VGPRs, two waves per SIMD), where the registers
// of two row blocks fit; at head size 128 they do not (one wave per SIMD,
// measured slower).
template <int kD, int NW, int kBN, int RB, int WPE>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void prefill_rb_kernel(PrefillParams p) {
  constexpr int kKRow = kD * 2;
  constexpr int kCH = kD / 8;
  constexpr int kRPC = 1024 / kKRow;
  constexpr int kBM = 32 * NW * RB;
  constexpr int kNU = kBN / 32, kNS = kBN / 16;
  constexpr int kQS = kD >= 128 ? 0 : 1;
  __shared__ __attribute__((aligned(16))) uint8_t kbuf0[kBN * kKRow];
  __shared__ __attribute__((aligned(16))) uint8_t kbuf1[kBN * kKRow];
  __shared__ __attribute__((aligned(16))) uint8_t vbuf0[kBN * kKRow];
  __shared__ __attribute__((aligned(16))) uint8_t vbuf1[kBN * kKRow];

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int hh = lane >> 5, n = lane & 31;
  const int qb = p.nqb - 1 - (int)blockIdx.y;
  const int head = blockIdx.x, g = head / p.ratio;
  const int q0 = qb * kBM;
  const int off = p.lk - p.lq;
  const int wrow0 = q0 + 32 * RB * w;  // the wave's first row
  const int kend = min(p.lk, off + min(q0 + kBM, p.lq));
  const int ntiles = (kend + kBN - 1) / kBN;

  half8_t qB[RB][kD / 16];
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    const int qrow = wrow0 + 32 * rb + n;
    const _Float16* qp = p.q + (int64_t)qrow * p.q_st + (int64_t)head * p.q_sh + 8 * hh;
#pragma unroll
    for (int s = 0; s < kD / 16; s++) {
      u32x4 x = {0u, 0u, 0u, 0u};
      if (qrow < p.lq) x = *reinterpret_cast<const u32x4*>(qp + 16 * s);
      qB[rb][s] = __builtin_bit_cast(half8_t, x);
    }
  }

  constexpr int kKC = (kBN / kRPC) / NW;
  const int kst_b = (int)(p.k_st * 2), vst_b = (int)(p.v_st * 2);
  uint32_t koff[kKC], voff[kKC];
#pragma unroll
  for (int i = 0; i < kKC; i++) {
    const int j = w + NW * i, row = kRPC * j + lane / kCH;
    koff[i] = (uint32_t)(row * kst_b + (((lane % kCH) ^ (row % kCH)) * 16));
    voff[i] = (uint32_t)(row * vst_b + (((lane % kCH) ^ (4 * ((row & 3) >> kQS))) * 16));
  }
  auto tile_rsrc = [&](const _Float16* base, int64_t st, int kb) {
    const int rows = min(kBN, p.lk - kb);
    const uint64_t a = (uint64_t)(uintptr_t)(base + (int64_t)kb * st);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    const int nrec = __builtin_amdgcn_readfirstlane(rows * (int)(st * 2));
    return __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)(((uint64_t)hi << 32) | lo),
                                             (short)0, nrec, 0x00020000);
  };
  const _Float16* const kbase = p.k + (int64_t)g * p.k_sh;
  const _Float16* const vbase = p.v + (int64_t)g * p.v_sh;
  auto issue = [&](int kt, uint8_t* kb, uint8_t* vb) {
#if defined(__HIP_DEVICE_COMPILE__)
    const __amdgpu_buffer_rsrc_t rk = tile_rsrc(kbase, p.k_st, kt * kBN);
    const __amdgpu_buffer_rsrc_t rv = tile_rsrc(vbase, p.v_st, kt * kBN);
#pragma unroll
    for (int i = 0; i < kKC; i++) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (void*)(kb + 1024 * (w + NW * i)), 16,
                                               koff[i], 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (void*)(vb + 1024 * (w + NW * i)), 16,
                                               voff[i], 0, 0, 0);
    }
#else
    (void)kt;
    (void)kb;
    (void)vb;
    (void)tile_rsrc;
    (void)kbase;
    (void)vbase;
#endif
  };
  const int vgq = lane >> 4, vsl = lane & 15, vt4 = vsl >> 2;
  const uint32_t vread_base =
      (uint32_t)((4 * hh + vt4) * kKRow +
                 ((2 * (vgq & 1) + ((vsl & 3) >> 1)) ^ (4 * (vt4 >> kQS))) * 16 + 8 * (vsl & 1));

  f32x16 oacc[RB][kD / 32];
  float m[RB], mc[RB], lsum[RB];
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
#pragma unroll
    for (int d = 0; d < kD / 32; d++)
#pragma unroll
      for (int j = 0; j < 16; j++) oacc[rb][d][j] = 0.0f;
    m[rb] = -INFINITY;
    mc[rb] = -INFINITY;
    lsum[rb] = 0.0f;
  }

  auto tile = [&](int kt, const uint8_t* kbuf, const uint8_t* vt) {
    const int kb = kt * kBN;
    if (kb > off + wrow0 + 32 * RB - 1) return;  // beyond every row of the wave
    constexpr int kKP = 4;
    constexpr int kNI = kNU * (kD / 16);
    f32x16 sacc[RB][kNU];
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
      for (int u = 0; u < kNU; u++)
#pragma unroll
        for (int j = 0; j < 16; j++) sacc[rb][u][j] = 0.0f;
    auto kfrag = [&](int i) {
      const int u = i % kNU, s = i / kNU, row = 32 * u + n;
      return *reinterpret_cast<const u32x4*>(kbuf + row * kKRow +
                                             (((2 * s + hh) ^ (row % kCH)) * 16));
    };
    u32x4 fr[kKP];
#pragma unroll
    for (int j = 0; j < kKP; j++) fr[j] = kfrag(j);
#pragma unroll
    for (int i = 0; i < kNI; i++) {
      const u32x4 a = fr[i % kKP];
      if (i + kKP < kNI) fr[i % kKP] = kfrag(i + kKP);
#pragma unroll
      for (int rb = 0; rb < RB; rb++)
        sacc[rb][i % kNU] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
            __builtin_bit_cast(half8_t, a), qB[rb][i / kNU], sacc[rb][i % kNU], 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, kKP, 0);
#pragma unroll
    for (int i = 0; i < kNI; i++) {
      __builtin_amdgcn_sched_group_barrier(0x008, RB, 0);  // the RB MFMAs of read i
      if (i + kKP < kNI) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    half8_t pB[RB][kNS];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
      const int rfirst = wrow0 + 32 * rb;
      if (kb + kBN - 1 > off + rfirst || kb + kBN > p.lk) {
        const int lim = min(off + rfirst + n, p.lk - 1) - kb - 4 * hh;
#pragma unroll
        for (int u = 0; u < kNU; u++)
#pragma unroll
          for (int j = 0; j < 16; j++) {
            const int kk = 32 * u + 8 * (j >> 2) + (j & 3);
            sacc[rb][u][j] += __int_as_float(((lim - kk) >> 31) & (int)0xff800000u);
          }
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int u = 0; u < kNU; u++)
#pragma unroll
        for (int j = 0; j < 16; j++) tmax = fmaxf(tmax, sacc[rb][u][j]);
      tmax = max32(tmax);
      const float m_new = fmaxf(m[rb], tmax);
      if (__builtin_amdgcn_ballot_w64(m_new * p.c > mc[rb] + 8.0f) != 0) {
        const float alpha =
            m[rb] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mc[rb] - m_new * p.c);
#pragma unroll
        for (int d = 0; d < kD / 32; d++) oacc[rb][d] *= alpha;
        lsum[rb] *= alpha;
        m[rb] = m_new;
        mc[rb] = m_new * p.c;
      }
      const float mce = mc[rb] == -INFINITY ? 0.0f : mc[rb];
#pragma unroll
      for (int u = 0; u < kNU; u++)
#pragma unroll
        for (int t = 0; t < 2; t++) {
          float pr[8];
#pragma unroll
          for (int i = 0; i < 8; i++) {
            pr[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[rb][u][8 * t + i], p.c, -mce));
            if constexpr (kD != 64) lsum[rb] += pr[i];
          }
          u32x4 pk;
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const half2_t h = __builtin_convertvector(f32x2{pr[2 * i], pr[2 * i + 1]}, half2_t);
            if constexpr (kD == 64)
              lsum[rb] = __builtin_amdgcn_fdot2(h, half2_t{(_Float16)1.0f, (_Float16)1.0f},
                                                lsum[rb], false);
            pk[i] = __builtin_bit_cast(uint32_t, h);
          }
          pB[rb][2 * u + t] = __builtin_bit_cast(half8_t, pk);
        }
    }
#pragma unroll
    for (int st = 0; st < kNS; st++) {
#pragma unroll
      for (int d = 0; d < kD / 32; d++) {
        typedef __attribute__((address_space(3))) uint8_t lds_u8;
        typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
        lds_u8* const pd = (lds_u8*)vt + (vread_base ^ (uint32_t)(64 * d)) + 16 * st * kKRow;
        const u32x2 a0 =
            __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)pd));
        const u32x2 a1 = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(pd + 8 * kKRow)));
        const u32x4 a = {a0[0], a0[1], a1[0], a1[1]};
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
          oacc[rb][d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
              __builtin_bit_cast(half8_t, a), pB[rb][st], oacc[rb][d], 0, 0, 0);
      }
    }
  };

  if (ntiles > 0) issue(0, kbuf0, vbuf0);
  for (int kt = 0; kt < ntiles; kt += 2) {
    __builtin_amdgcn_s_waitcnt(0x0f70);
    __syncthreads();
    if (kt + 1 < ntiles) issue(kt + 1, kbuf1, vbuf1);
    tile(kt, kbuf0, vbuf0);
    if (kt + 1 >= ntiles) break;
    __builtin_amdgcn_s_waitcnt(0x0f70);
    __syncthreads();
    if (kt + 2 < ntiles) issue(kt + 2, kbuf0, vbuf0);
    tile(kt + 1, kbuf1, vbuf1);
  }

#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    const int qrow = wrow0 + 32 * rb + n;
    const float ls = sum32(lsum[rb]);
    if (qrow < p.lq) {
      const float inv = ls > 0.0f ? 1.0f / ls : 0.0f;
      _Float16* op = p.o + (int64_t)qrow * p.o_st + (int64_t)head * p.o_sh + 4 * hh;
#pragma unroll
      for (int d = 0; d < kD / 32; d++)
#pragma unroll
        for (int jq = 0; jq < 4; jq++) {
          const uint32_t lo =
              pack_h2(oacc[rb][d][4 * jq] * inv, oacc[rb][d][4 * jq + 1] * inv);
          const uint32_t hi =
              pack_h2(oacc[rb][d][4 * jq + 2] * inv, oacc[rb][d][4 * jq + 3] * inv);
          *reinterpret_cast<u32x2*>(op + 32 * d + 8 * jq) = u32x2{lo, hi};
        }
    }
  }
}

// Merge of the splits of split-KV mode: one wave per (query row, q head),
// o = sum_z w_z (O_z / l_z) / sum_z w_z, w_z = 2^(mc_z - M) l_z, fp16 out.
template <int kD>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillParams p, int hq) {
  constexpr int V = kD / 64;  // dims per lane
  const int lane = threadIdx.x & 63;
  const int64_t idx = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // row * hq + head
  if (idx >= (int64_t)p.lq * hq) return;
  const int row = (int)(idx / hq), head = (int)(idx % hq);
  const int64_t zs = (int64_t)p.lq * hq;  // rows of one split
  float mx = -INFINITY;
  for (int z = 0; z < p.nsplit; z++) mx = fmaxf(mx, p.ws_ml[2 * (z * zs + idx)]);
  float den = 0.0f, acc[V];
#pragma unroll
  for (int i = 0; i < V; i++) acc[i] = 0.0f;
  for (int z = 0; z < p.nsplit; z++) {
    const f32x2 ml = *reinterpret_cast<const f32x2*>(p.ws_ml + 2 * (z * zs + idx));
    if (ml[0] == -INFINITY) continue;  // no visible key in this split
    const float wgt = __builtin_amdgcn_exp2f(ml[0] - mx) * ml[1];
    den += wgt;
    const _Float16* const src = p.ws_o + (z * zs + idx) * kD + V * lane;
#pragma unroll
    for (int i = 0; i < V; i++) acc[i] += wgt * (float)src[i];
  }
  const float inv = den > 0.0f ? 1.0f / den : 0.0f;
  _Float16* const op = p.o + (int64_t)row * p.o_st + (int64_t)head * p.o_sh + V * lane;
#pragma unroll
  for (int i = 0; i < V; i++) op[i] = (_Float16)(acc[i] * inv);
}

// the workgroup shapes, at head size 64 or 128: 256 query rows (eight waves
// with 128-key tiles at head size 128; four waves of two row blocks with
// 64-key tiles at head size 64); four waves, 64-key tiles; four waves split
// over the keys (then merged).
// Head size 256: four waves, 64-key tiles (128 KB of LDS for the K and V
// double buffers), one wave per SIMD, split or not.
template <int D>
hipError_t launch_prefill(int nw, int heads, hipStream_t st, const PrefillParams& p) {
  if constexpr (D == 256) {
    (void)nw;
    if (p.nsplit <= 1) {
      hipLaunchKernelGGL((prefill_kernel<D, 4, 64, false, 1>), dim3(heads, p.nqb), dim3(256), 0,
                         st, p);
    } else {
      hipLaunchKernelGGL((prefill_kernel<D, 4, 64, true, 1>), dim3(heads, p.nqb, p.nsplit),
                         dim3(256), 0, st, p);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      const int64_t waves = (int64_t)p.lq * heads;
      hipLaunchKernelGGL((prefill_merge_kernel<D>), dim3((unsigned)((waves + 3) / 4)), dim3(256),
                         0, st, p, heads);
    }
  } else if (nw == 8 && D == 64) {
    // head size 64: four waves of 64 rows (two row blocks each), 64-key tiles
    hipLaunchKernelGGL((prefill_rb_kernel<D, 4, 64, 2, 2>), dim3(heads, p.nqb), dim3(256), 0, st,
                       p);
  } else if (nw == 8) {
    hipLaunchKernelGGL((prefill_kernel<D, 8, 128, false>), dim3(heads, p.nqb), dim3(512), 0, st,
                       p);
  } else if (p.nsplit <= 1) {
    hipLaunchKernelGGL((prefill_kernel<D, 4, 64, false>), dim3(heads, p.nqb), dim3(256), 0, st,
                       p);
  } else {
    hipLaunchKernelGGL((prefill_kernel<D, 4, 64, true>), dim3(heads, p.nqb, p.nsplit), dim3(256),
                       0, st, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t waves = (int64_t)p.lq * heads;
    hipLaunchKernelGGL((prefill_merge_kernel<D>), dim3((unsigned)((waves + 3) / 4)), dim3(256),
                       0, st, p, heads);
  }
  return hipGetLastError();
}


// Launch plan of one call: the workgroup shape and, when the grid would
// leave CUs idle (short chunks over long contexts), a split of the keys.
struct PrefillPlan {
  int nw = 4, nqb = 0, nsplit = 1, tps = 0;
  int64_t ws_bytes = 0;  // workspace the split needs (0: none)
};
PrefillPlan plan_prefill(int q_len, int kv_len, int heads, int head_dim) {
  PrefillPlan sp;
  const int cus = device_cus();
  const int64_t nqb8 = (q_len + 255) / 256;
  if (head_dim != 256 && (int64_t)heads * nqb8 >= (int64_t)cus) {
    // 256-row workgroups (8 waves, one per CU) when they still give every CU one
    sp.nw = 8;
    sp.nqb = (int)nqb8;
    return sp;
  }
  // else 128-row workgroups (4 waves, two per CU; one at head size 256);
  // with fewer than two per CU, the keys of each query block are split so that the grid fills the
  // chip, each split at least 8 tiles (512 keys)
  sp.nqb = (q_len + 127) / 128;
  const int64_t wgs = (int64_t)heads * sp.nqb;
  const int ntl = (kv_len + 63) / 64;  // tiles of the last (longest) query block
  if (cus > 0 && wgs < 2LL * cus && ntl >= 16) {
    int64_t S = (2LL * cus + wgs - 1) / wgs;
    if (S > ntl / 8) S = ntl / 8;
    if (S > 64) S = 64;
    if (S >= 2) {
      sp.tps = (int)((ntl + S - 1) / S);
      sp.nsplit = (ntl + sp.tps - 1) / sp.tps;
      sp.ws_bytes = (int64_t)sp.nsplit * q_len * heads * (head_dim * 2 + 8);
    }
  }
  return sp;
}

}  // namespace
}  // namespace tq

extern "C" int64_t tq_prefill_workspace_bytes(int32_t q_len, int32_t kv_len, int32_t num_qo_heads,
                                              int32_t num_kv_heads, int32_t head_dim) {
  if (q_len <= 0 || kv_len < q_len || num_qo_heads <= 0 || num_kv_heads <= 0 ||
      (head_dim != 64 && head_dim != 128 && head_dim != 256))
    return 0;
  (void)num_kv_heads;
  return tq::plan_prefill(q_len, kv_len, num_qo_heads, head_dim).ws_bytes;
}

extern "C" int tq_prefill_attention_ws(
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k,
    int64_t k_stride_tok, int64_t k_stride_head, const void* v, int64_t v_stride_tok,
    int64_t v_stride_head, void* o, int64_t o_stride_tok, int64_t o_stride_head, int32_t q_len,
    int32_t kv_len, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, float sm_scale,
    void* workspace, int64_t workspace_bytes, tq_stream_t stream) {
  using namespace tq;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) {
    set_error("prefill_attention: head_dim %d unsupported (64, 128 or 256 only)", head_dim);
    return kEinval;
  }
  if (num_kv_heads <= 0 || num_qo_heads <= 0 || num_qo_heads % num_kv_heads != 0) {
    set_error("prefill_attention: num_qo_heads %d not a multiple of num_kv_heads %d",
              num_qo_heads, num_kv_heads);
    return kEinval;
  }
  if (q_len < 0 || kv_len < q_len) {
    set_error("prefill_attention: need 0 <= q_len (%d) <= kv_len (%d)", q_len, kv_len);
    return kEinval;
  }
  if (!q || !k || !v || !o) {
    set_error("prefill_attention: null pointer");
    return kEinval;
  }
  const int64_t strides[8] = {q_stride_tok, q_stride_head, k_stride_tok, k_stride_head,
                              v_stride_tok, v_stride_head, o_stride_tok, o_stride_head};
  for (int i = 0; i < 8; i++) {
    if (strides[i] < 0 || strides[i] % 8 != 0) {
      set_error("prefill_attention: strides must be non-negative multiples of 8 elements");
      return kEinval;
    }
  }
  if (k_stride_tok < head_dim || v_stride_tok < head_dim ||
      (k_stride_tok > v_stride_tok ? k_stride_tok : v_stride_tok) * 2 * (int64_t)kBNmax > INT32_MAX) {
    set_error("prefill_attention: k / v token strides out of range");
    return kEinval;
  }
  const uintptr_t al = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)o;
  if (al & 15) {
    set_error("prefill_attention: tensors must be 16-byte aligned");
    return kEinval;
  }
  if (q_len == 0) return 0;
  PrefillParams p;
  p.q = static_cast<const _Float16*>(q);
  p.k = static_cast<const _Float16*>(k);
  p.v = static_cast<const _Float16*>(v);
  p.o = static_cast<_Float16*>(o);
  p.q_st = q_stride_tok;
  p.q_sh = q_stride_head;
  p.k_st = k_stride_tok;
  p.k_sh = k_stride_head;
  p.v_st = v_stride_tok;
  p.v_sh = v_stride_head;
  p.o_st = o_stride_tok;
  p.o_sh = o_stride_head;
  p.lq = q_len;
  p.lk = kv_len;
  p.ratio = num_qo_heads / num_kv_heads;
  p.c = sm_scale * 1.4426950408889634f;
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const PrefillPlan sp = plan_prefill(q_len, kv_len, num_qo_heads, head_dim);
  p.nqb = sp.nqb;
  p.nsplit = 1;
  p.tps = 0;
  p.ws_o = nullptr;
  p.ws_ml = nullptr;
  // the split runs only with a workspace that holds it (else one workgroup
  // per query block, the same result)
  if (sp.nsplit > 1 && workspace && workspace_bytes >= sp.ws_bytes &&
      ((uintptr_t)workspace & 15) == 0) {
    p.nsplit = sp.nsplit;
    p.tps = sp.tps;
    p.ws_o = static_cast<_Float16*>(workspace);
    p.ws_ml = reinterpret_cast<float*>(p.ws_o + (int64_t)sp.nsplit * q_len * num_qo_heads *
                                                    head_dim);
  }
  if (head_dim == 64) return (int)launch_prefill<64>(sp.nw, num_qo_heads, st, p);
  if (head_dim == 128) return (int)launch_prefill<128>(sp.nw, num_qo_heads, st, p);
  return (int)launch_prefill<256>(sp.nw, num_qo_heads, st, p);
}

extern "C" int tq_prefill_attention(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                    const void* k, int64_t k_stride_tok, int64_t k_stride_head,
                                    const void* v, int64_t v_stride_tok, int64_t v_stride_head,
                                    void* o, int64_t o_stride_tok, int64_t o_stride_head,
                                    int32_t q_len, int32_t kv_len, int32_t num_qo_heads,
                                    int32_t num_kv_heads, int32_t head_dim, float sm_scale,
                                    tq_stream_t stream) {
  return tq_prefill_attention_ws(q, q_stride_tok, q_stride_head, k, k_stride_tok, k_stride_head,
                                 v, v_stride_tok, v_stride_head, o, o_stride_tok, o_stride_head,
                                 q_len, kv_len, num_qo_heads, num_kv_heads, head_dim, sm_scale,
                                 nullptr, 0, stream);
}
