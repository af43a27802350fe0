// tq_decode.hip -- split-KV GQA decode attention over the packed paged cache.
//
// Semantics: dequantize-then-attend of the reference
// (turboquant/triton_decode_ref.py:89-131, :264-299) computed in the rotated
// domain as the reference's v5 kernel does
// (csrc/include/flashinfer_decode_turboquant_v5_tc.cuh:106-795): q is rotated
// once, q' = FWHT(s*q)/sqrt(pd); K^ = codebook[code]*norm/sqrt(pd);
// softmax(q'.K^ * sm_scale) V^ per split, LSE merge across splits
// (flashinfer_decode_turboquant_combine.cuh:18-79), then the inverse rotation
// o = s * FWHT(o')/sqrt(pd), applied once per (sequence, head) after the merge.
//
// gfx950 design (not the reference's):
//  * One workgroup per (sequence, split, group of G kv heads), one wave64 per
//    kv head; all G heads of a token share 80-byte neighbours in the same
//    cache lines, so a workgroup consumes whole lines.
//  * A 16-token tile is one MFMA block.  QK^T: v_mfma_f32_16x16x32_f16 with
//    A = dequantized K (row = token, lane l loads 16 B of token l%16 with one
//    dwordx4), B = q' as fp16 hi + lo parts (column = q head; GQA heads
//    padded to 16).  The C layout
//    (row 4*(l/16)+r = token, column l%16 = head) is exactly the B layout of
//    the PV product v_mfma_f32_16x16x16_f16 (A = V^T: row = dim slot l%16,
//    k = tokens 4*(l/16)..+3), so probabilities never leave registers.
//  * 4-bit -> fp16 dequant without memory lookups: the codebook is odd
//    (c[15-i] = -c[i]); codes are folded to (sign, 3-bit magnitude) with
//    bit tricks on 8 nibbles at once, magnitudes come from two v_perm_b32
//    byte tables (high and low byte of the fp16 value), the sign is OR-ed into
//    the high byte, and v_perm interleaves the bytes into packed fp16 pairs.
//  * The K norm scales the score; the V norm and 1/sqrt(pd) fold into the
//    probability, so dequantized operands are (scaled) codebook values.
//  * Accuracy: q' and the probabilities enter the MFMAs as fp16 hi + lo
//    pairs and the codebook tables are pre-scaled to fp16-friendly values,
//    keeping the result within ~1e-3 of fp32 math even for heavy-tailed keys.
//  * Online softmax in the exp2 domain with a lazy rescale (the running max
//    only moves when a tile exceeds it by more than 2^3), bounding p <= 8.
#include <math.h>

#include "tq_common.h"

namespace tq {

namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// The dequant tables hold fp16(kCbScale * c[8+m]), m = 0..7: the positive
// centroids scaled by kCbScale = 1.48098 (fp32 0x3fbd90c1), a factor chosen by
// search so that all eight products sit close to fp16 grid points (max
// relative rounding error 8.7e-5 instead of 4.7e-4 for the unscaled values).
// 1/kCbScale is folded into the score and probability scales, so the math is
// unchanged and the fp16 operands carry ~5x less codebook rounding.
// fp16 bits: 0x3216 0x3899 0x3bc8 0x3d95 0x3f71 0x40cb 0x4221 0x440c, split
// into a high-byte table and a low-byte table of 8 bytes each (byte m).
constexpr float kCbScale = 1.4809800386428833f;
constexpr uint32_t kHi0 = 0x3d3b3832u, kHi1 = 0x4442403fu;
constexpr uint32_t kLo0 = 0x95c89916u, kLo1 = 0x0c21cb71u;

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  // byte i of the result = byte sel_i of the 8-byte value {hi:lo} (lo = bytes 0-3)
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// Dequantize 8 codes (one dword, byte k = code[2k] << 4 | code[2k+1]) to 8
// fp16 codebook values, as 4 packed pairs:
//   x[0] = (byte0 low, byte1 low)   x[1] = (byte2 low, byte3 low)
//   x[2] = (byte0 high, byte1 high) x[3] = (byte2 high, byte3 high)
// i.e. element order {1,3,5,7,0,2,4,6} of the 8 dims the dword holds.
__device__ __forceinline__ void dq8(uint32_t D, uint32_t* x) {
  // fold: nibble n -> (neg flag in bit 3, magnitude index m in bits 0-2) with
  // c[n] = (n >= 8) ? M[n-8] : -M[7-n]
  const uint32_t a = D & 0x88888888u;
  const uint32_t F = ~D ^ (a - (a >> 3));
  const uint32_t SL = F & 0x07070707u;
  const uint32_t SH = (F >> 4) & 0x07070707u;
  const uint32_t hL = perm(kHi1, kHi0, SL) | ((F << 4) & 0x80808080u);
  const uint32_t lL = perm(kLo1, kLo0, SL);
  const uint32_t hH = perm(kHi1, kHi0, SH) | (F & 0x80808080u);
  const uint32_t lH = perm(kLo1, kLo0, SH);
  x[0] = perm(hL, lL, 0x05010400u);
  x[1] = perm(hL, lL, 0x07030602u);
  x[2] = perm(hH, lH, 0x05010400u);
  x[3] = perm(hH, lH, 0x07030602u);
}

__device__ __forceinline__ half8_t as_half8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u32x4 u = {a, b, c, d};
  return __builtin_bit_cast(half8_t, u);
}
__device__ __forceinline__ half4_t as_half4(uint32_t a, uint32_t b) {
  u32x2 u = {a, b};
  return __builtin_bit_cast(half4_t, u);
}

// broadcast lane r of each quad (DPP quad_perm, no LDS)
template <int R>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, R * 0x55, 0xf, 0xf, false);
}

__device__ __forceinline__ float h2f(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

struct DecodeParams {
  const _Float16* q;
  int64_t q_sb, q_sh;
  const uint8_t* ks;
  const uint8_t* vs;
  const int32_t* indices;
  const int32_t* indptr;
  const int32_t* seq_lens;
  const float* signs;
  float* po;
  float* plse;
  int num_blocks;  // clamped to INT_MAX (page ids are int32)
  int B, Hq, Hkv, ratio, block_size, ebs, S, cs, G, HG;
  float qk_scale;     // sm_scale * log2(e) / (sqrt(pd) * kCbScale)
  float inv_sqrt_pd;  // 1/sqrt(pd)
  float pv_scale;     // 1/(sqrt(pd) * kCbScale)
};

template <int PD>
struct Tile {
  static constexpr int KD = PD / 32;               // K dwords per lane = QK MFMA pairs
  static constexpr int VB = PD / 32;               // V bytes per lane per token
  static constexpr int VW = VB >= 4 ? VB / 4 : 1;  // V dwords per lane per token
  uint32_t k[KD];
  uint32_t v[4][VW];
  uint32_t nk, nv;
};

// Per-lane byte offsets inside one 16-token tile of one kv head, relative to
// the tile's first entry (constant over the whole loop).
struct LaneOffsets {
  uint32_t k;     // K codes: token n, bytes [q4*PD/8, (q4+1)*PD/8)
  uint32_t v[4];  // V codes: token 4*q4 + j, bytes [n*PD/32, (n+1)*PD/32)
  uint32_t nrm;   // norm of token 4*q4 + (lane & 3)
};

// Issue the loads of one tile through buffer resources whose base is the
// tile's first entry of this kv head (wave-uniform) and whose size is the
// tile's extent, or 0 for a tile that is not fetched: out-of-range buffer
// loads return zeros without touching memory, so every tile issues the same
// instruction sequence and the load counters stay in order.
template <int PD>
__device__ __forceinline__ void load_tile(__amdgpu_buffer_rsrc_t kr, __amdgpu_buffer_rsrc_t vr,
                                          const LaneOffsets& o, Tile<PD>& t) {
  if constexpr (PD == 64) {
    const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(kr, o.k, 0, 0);
    t.k[0] = w[0]; t.k[1] = w[1];
  } else if constexpr (PD == 128) {
    const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(kr, o.k, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) t.k[i] = w[i];
  } else {
    const u32x4 w0 = __builtin_amdgcn_raw_buffer_load_b128(kr, o.k, 0, 0);
    const u32x4 w1 = __builtin_amdgcn_raw_buffer_load_b128(kr, o.k + 16, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) { t.k[i] = w0[i]; t.k[4 + i] = w1[i]; }
  }
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if constexpr (PD == 64) {
      t.v[j][0] = __builtin_amdgcn_raw_buffer_load_b16(vr, o.v[j], 0, 0);
    } else if constexpr (PD == 128) {
      t.v[j][0] = __builtin_amdgcn_raw_buffer_load_b32(vr, o.v[j], 0, 0);
    } else {
      const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(vr, o.v[j], 0, 0);
      t.v[j][0] = w[0]; t.v[j][1] = w[1];
    }
  }
  t.nk = __builtin_amdgcn_raw_buffer_load_b16(kr, o.nrm, 0, 0);
  t.nv = __builtin_amdgcn_raw_buffer_load_b16(vr, o.nrm, 0, 0);
}

// 4x4 byte transpose: E_k byte j = byte k of D_j
__device__ __forceinline__ void transpose4(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3,
                                           uint32_t* e) {
  const uint32_t a01 = perm(d1, d0, 0x05010400u), b01 = perm(d1, d0, 0x07030602u);
  const uint32_t a23 = perm(d3, d2, 0x05010400u), b23 = perm(d3, d2, 0x07030602u);
  e[0] = perm(a23, a01, 0x05040100u);
  e[1] = perm(a23, a01, 0x07060302u);
  e[2] = perm(b23, b01, 0x05040100u);
  e[3] = perm(b23, b01, 0x07060302u);
}

// Online-softmax state of one wave: O[i][r] = unnormalised o[h = n][dim
// (4*q4 + r)*NO + i] in the rotated domain (times pv_scale^-1, see below),
// m = running max of the scores (log2 units, per column h), lsum = this
// lane's share of the denominator.  Probabilities are formed as
// p' = exp2(s - mb), mb = m + Lpv with Lpv = -log2(pv_scale), i.e. p' = p *
// pv_scale: the V norm then multiplies in without leaving the fp16 range;
// o = pv_scale * O / lsum', and mb + log2(lsum') is the LSE (log2 units).
template <int PD>
struct SoftmaxState {
  static constexpr int NO = PD / 16;
  float4_t O[NO];
  float m;
  float mb;
  float lsum;
};

__device__ __forceinline__ float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// fp16 value held in the low / high half of a dword
__device__ __forceinline__ float lo_half(uint32_t v) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu));
}
__device__ __forceinline__ float hi_half(uint32_t v) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
}

// One 16-token tile of one kv head.  `full` (wave-uniform): every token of
// the tile is valid (page valid and inside [c0, c1)), so no masking is needed.
template <int PD>
__device__ __forceinline__ void attend_tile(bool full, const Tile<PD>& cur, bool ok, int tile, int c0,
                                            int c1, int q4, int n, int ratio,
                                            const half8_t* qhi, const half8_t* qlo, float lpv,
                                            SoftmaxState<PD>& st) {
  constexpr int KD = PD / 32;
  constexpr int VB = PD / 32;
  constexpr int NO = PD / 16;
  // ---- scores S[t = 4*q4 + r][h = n]; q' carries sm_scale*log2(e)/(sqrt(pd)*kCbScale)
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < KD; c++) {
    uint32_t x[4];
    dq8(cur.k[c], x);
    const half8_t kv8 = as_half8(x[0], x[1], x[2], x[3]);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv8, qhi[c], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv8, qlo[c], acc, 0, 0, 0);
  }
  // norms of tokens 4*q4 + r: K norm in the low half, V norm in the high half
  const uint32_t nkv = cur.nk | (cur.nv << 16);
  const uint32_t nr[4] = {quad_bcast<0>(nkv), quad_bcast<1>(nkv), quad_bcast<2>(nkv),
                          quad_bcast<3>(nkv)};
  float sc[4];
  bool valid[4];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    sc[r] = acc[r] * lo_half(nr[r]);
    valid[r] = true;
  }
  if (!full) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int t = tile * kTile + 4 * q4 + r;
      valid[r] = ok && t >= c0 && t < c1;
      sc[r] = valid[r] ? sc[r] : -INFINITY;
    }
  }
  float tmax = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
  tmax = xor16_max(tmax);
  tmax = xor32_max(tmax);
  const float m_new = fmaxf(st.m, tmax);
  const bool need = (n < ratio) && (m_new > st.m + 3.0f);
  if (__any(need)) {
    const float alpha = (m_new == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(st.m - m_new);
#pragma unroll
    for (int i = 0; i < NO; i++) st.O[i] *= alpha;
    st.lsum *= alpha;
    st.m = m_new;
    st.mb = m_new + lpv;
  }
  float pr[4];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    pr[r] = __builtin_amdgcn_exp2f(sc[r] - st.mb);
  }
  if (!full) {
#pragma unroll
    for (int r = 0; r < 4; r++) pr[r] = valid[r] ? pr[r] : 0.0f;
  }
  st.lsum += (pr[0] + pr[1]) + (pr[2] + pr[3]);
  // fp16 hi + lo parts of p' * norm_v
  half4_t pvh, pvl;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const float x = pr[r] * hi_half(nr[r]);
    const _Float16 hi = (_Float16)x;
    pvh[r] = hi;
    pvl[r] = (_Float16)(x - (float)hi);
  }
  // ---- O[h][dim slot] += V^T P^T
  uint32_t e[VB];
  if constexpr (PD == 64) {
    const uint32_t p01 = cur.v[0][0] | (cur.v[1][0] << 16);
    const uint32_t p23 = cur.v[2][0] | (cur.v[3][0] << 16);
    e[0] = perm(p23, p01, 0x06040200u);
    e[1] = perm(p23, p01, 0x07050301u);
  } else if constexpr (PD == 128) {
    transpose4(cur.v[0][0], cur.v[1][0], cur.v[2][0], cur.v[3][0], e);
  } else {
    transpose4(cur.v[0][0], cur.v[1][0], cur.v[2][0], cur.v[3][0], e);
    transpose4(cur.v[0][1], cur.v[1][1], cur.v[2][1], cur.v[3][1], e + 4);
  }
#pragma unroll
  for (int k = 0; k < VB; k++) {
    uint32_t x[4];
    dq8(e[k], x);
    const half4_t lo4 = as_half4(x[0], x[1]), hi4 = as_half4(x[2], x[3]);
    st.O[2 * k + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(lo4, pvh, st.O[2 * k + 1], 0, 0, 0);
    st.O[2 * k + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(lo4, pvl, st.O[2 * k + 1], 0, 0, 0);
    st.O[2 * k] = __builtin_amdgcn_mfma_f32_16x16x16f16(hi4, pvh, st.O[2 * k], 0, 0, 0);
    st.O[2 * k] = __builtin_amdgcn_mfma_f32_16x16x16f16(hi4, pvl, st.O[2 * k], 0, 0, 0);
  }
}

template <int PD>
__device__ __forceinline__ void attend(const Tile<PD>& cur, bool ok, int tile, int c0, int c1,
                                       int q4, int n, int ratio, const half8_t* qhi,
                                       const half8_t* qlo, float lpv, SoftmaxState<PD>& st) {
  const bool full = ok && tile * kTile >= c0 && tile * kTile + kTile <= c1;
  attend_tile<PD>(full, cur, ok, tile, c0, c1, q4, n, ratio, qhi, qlo, lpv, st);
}

template <int PD>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(PD == 256 ? 2 : 4)))
void decode_partials_kernel(DecodeParams p) {
  constexpr int KD = PD / 32;
  constexpr int NO = PD / 16;  // PV MFMAs = dim slots per lane
  extern __shared__ float smem[];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int q4 = lane >> 4, n = lane & 15;
  int bid = blockIdx.x;
  const int hg = bid % p.HG;
  bid /= p.HG;
  const int s = bid % p.S;
  const int b = bid / p.S;
  const int kvh = hg * p.G + w;
  const int ratio = p.ratio;

  // ---- q' = FWHT(s*q)/sqrt(pd) for this wave's `ratio` heads, in LDS
  float* qs = smem + (size_t)w * ratio * PD;
  for (int i = lane; i < ratio * PD; i += 64) {
    const int r = i / PD, d = i - r * PD;
    float x = (float)p.q[b * p.q_sb + (int64_t)(kvh * ratio + r) * p.q_sh + d];
    if (p.signs) x = x * p.signs[d];
    qs[i] = x;
  }
  __syncthreads();
  if (p.signs) {
    for (int h = 1; h < PD; h <<= 1) {
      for (int i = lane; i < ratio * PD / 2; i += 64) {
        const int r = i / (PD / 2), j = i - r * (PD / 2);
        const int lo = r * PD + (j / h) * 2 * h + (j % h);
        const float a = qs[lo], c = qs[lo + h];
        qs[lo] = a + c;
        qs[lo + h] = a - c;
      }
      __syncthreads();
    }
  }
  const float qsc = (p.signs ? p.inv_sqrt_pd : 1.0f) * p.qk_scale;
  // q' is split into fp16 high and low parts (q' = hi + lo to ~22 bits), two
  // MFMAs per K block, so the scores keep fp32-level accuracy even for
  // heavy-tailed keys.
  half8_t qhi[KD], qlo[KD];
  {
    constexpr int ord[8] = {1, 3, 5, 7, 0, 2, 4, 6};
#pragma unroll
    for (int c = 0; c < KD; c++) {
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const int d = q4 * (PD / 4) + 8 * c + ord[e];
        const float x = (n < ratio) ? qs[n * PD + d] * qsc : 0.0f;
        const _Float16 hi = (_Float16)x;
        qhi[c][e] = hi;
        qlo[c][e] = (_Float16)(x - (float)hi);
      }
    }
  }

  SoftmaxState<PD> st;
#pragma unroll
  for (int i = 0; i < NO; i++) st.O[i] = float4_t{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.mb = -INFINITY;
  st.lsum = 0.f;
  const float lpv = -__log2f(p.pv_scale);

  const int L = p.seq_lens[b];
  const int c0 = s * p.cs;
  const int c1 = min(c0 + p.cs, L);
  if (c0 < c1) {
    const int tile0 = c0 / kTile, tile1 = (c1 - 1) / kTile;
    const int tpp = p.block_size / kTile;  // tiles per page
    const int64_t tokstride = (int64_t)p.Hkv * p.ebs;
    const int ip = p.indptr[b];
    LaneOffsets lo;
    lo.k = (uint32_t)(n * tokstride + q4 * (PD / 8));
#pragma unroll
    for (int j = 0; j < 4; j++) lo.v[j] = (uint32_t)((4 * q4 + j) * tokstride + n * (PD / 32));
    lo.nrm = (uint32_t)((4 * q4 + (lane & 3)) * tokstride + PD / 2);
    const uint8_t* kslab = p.ks + (int64_t)kvh * p.ebs;
    const uint8_t* vslab = p.vs + (int64_t)kvh * p.ebs;
    const int tile_bytes = (int)(kTile * tokstride);

    // windows of 64 tiles: lane i holds the page id of tile w0 + i
    for (int w0 = tile0; w0 <= tile1; w0 += 64) {
      const int wend = min(w0 + 63, tile1);
      int vpage = -1;
      if (w0 + lane <= wend) vpage = p.indices[ip + (w0 + lane) / tpp];

      // Issue tile t's loads into `t_`; tiles past the window fetch nothing.
      auto issue = [&](int t, Tile<PD>& t_, bool& ok_) {
        const int rel = t - w0;
        int pg = __builtin_amdgcn_readlane(vpage, rel & 63);
        ok_ = rel <= wend - w0 && pg >= 0 && pg < p.num_blocks;
        const int64_t off =
            ok_ ? ((int64_t)pg * p.block_size + (t % tpp) * kTile) * tokstride : 0;
        const int nrec = ok_ ? tile_bytes : 0;
        const __amdgpu_buffer_rsrc_t kr =
            __builtin_amdgcn_make_buffer_rsrc((void*)(kslab + off), (short)0, nrec, 0x00020000);
        const __amdgpu_buffer_rsrc_t vr =
            __builtin_amdgcn_make_buffer_rsrc((void*)(vslab + off), (short)0, nrec, 0x00020000);
        load_tile<PD>(kr, vr, lo, t_);
      };

      // three-deep register ring: tiles t+1 and t+2 are in flight while t runs
      Tile<PD> b0, b1, b2;
      bool ok0, ok1, ok2;
      issue(w0, b0, ok0);
      issue(w0 + 1, b1, ok1);
      // Whole groups of three tiles: a tile past the window end is fetched as
      // an empty buffer and fully masked, so the body has no early exits.
      for (int t = w0; t <= wend; t += 3) {
        issue(t + 2, b2, ok2);
        attend<PD>(b0, ok0, t, c0, c1, q4, n, ratio, qhi, qlo, lpv, st);
        issue(t + 3, b0, ok0);
        attend<PD>(b1, ok1, t + 1, c0, c1, q4, n, ratio, qhi, qlo, lpv, st);
        issue(t + 4, b1, ok1);
        attend<PD>(b2, ok2, t + 2, c0, c1, q4, n, ratio, qhi, qlo, lpv, st);
      }
    }
  }

  // ---- finish: O[i][r] = o[h = n][dim (4*q4 + r)*NO + i]
  const float lt = xor32_sum(xor16_sum(st.lsum));
  if (n < ratio) {
    // o = pv_scale * O / lsum' (p' = p * pv_scale in both O and lsum')
    const float inv = lt > 0.f ? p.pv_scale / lt : 0.0f;
    const int64_t row = ((int64_t)b * p.S + s) * p.Hq + kvh * ratio + n;
    float* out = p.po + row * PD + q4 * (PD / 4);
#pragma unroll
    for (int r = 0; r < 4; r++) {
#pragma unroll
      for (int i = 0; i < NO; i += 4) {
        float4_t v = {st.O[i][r] * inv, st.O[i + 1][r] * inv, st.O[i + 2][r] * inv,
                      st.O[i + 3][r] * inv};
        *reinterpret_cast<float4_t*>(out + r * NO + i) = v;
      }
    }
    // natural-log LSE: (m + log2(sum p)) * ln 2 = (mb + log2(lsum')) * ln 2
    if (q4 == 0)
      p.plse[row] = lt > 0.f ? (st.mb + __log2f(lt)) * 0.69314718055994531f : -INFINITY;
  }
}

template <int PD>
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ po,
                                                      const float* __restrict__ plse, int S,
                                                      int Hq, const float* __restrict__ signs,
                                                      float inv_sqrt_pd, _Float16* __restrict__ o) {
  constexpr int C = PD / 4;        // float4 columns
  constexpr int NG = 256 / C;      // split groups
  constexpr int V = PD / 64;       // dims per lane in the FWHT
  extern __shared__ float sm[];    // [S] weights, then [NG][PD] partial sums
  __shared__ float red[8];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int b = blockIdx.x / Hq, h = blockIdx.x % Hq;
  const int64_t row0 = (int64_t)b * S * Hq + h;  // row of split s: row0 + s*Hq

  float mx = -INFINITY;
  for (int s = tid; s < S; s += 256) mx = fmaxf(mx, plse[row0 + (int64_t)s * Hq]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  if (lane == 0) red[wv] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float den = 0.f;
  for (int s = tid; s < S; s += 256) {
    const float l = plse[row0 + (int64_t)s * Hq];
    const float wgt = (l > -INFINITY && mx > -INFINITY) ? __expf(l - mx) : 0.0f;
    sm[s] = wgt;
    den += wgt;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) den += __shfl_xor(den, off);
  __syncthreads();  // red[] reads done, weights visible
  if (lane == 0) red[4 + wv] = den;
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
  const int col = tid % C, grp = tid / C;
  for (int s = grp; s < S; s += NG) {
    const float wgt = sm[s];
    if (wgt != 0.0f) {
      const float4_t v = *reinterpret_cast<const float4_t*>(po + (row0 + (int64_t)s * Hq) * PD + col * 4);
      acc += wgt * v;
    }
  }
  __syncthreads();  // weights no longer needed; reuse LDS for group sums
  float* part = sm;
  *reinterpret_cast<float4_t*>(part + grp * PD + col * 4) = acc;
  __syncthreads();
  if (wv == 0) {
    den = (red[4] + red[5]) + (red[6] + red[7]);
    const float inv = den > 0.f ? 1.0f / den : 0.0f;
    float x[V];
#pragma unroll
    for (int i = 0; i < V; i++) {
      float t = 0.f;
      for (int g = 0; g < NG; g++) t += part[g * PD + lane * V + i];
      x[i] = t * inv;
    }
    if (signs) {
#pragma unroll
      for (int hh = 1; hh < V; hh <<= 1)
#pragma unroll
        for (int i = 0; i < V; i += 2 * hh)
#pragma unroll
          for (int k = 0; k < hh; k++) {
            const float a = x[i + k], c = x[i + k + hh];
            x[i + k] = a + c;
            x[i + k + hh] = a - c;
          }
#pragma unroll
      for (int delta = 1; delta < 64; delta <<= 1)
#pragma unroll
        for (int i = 0; i < V; i++) {
          const float partner = __shfl_xor(x[i], delta);
          x[i] = (lane & delta) ? (partner - x[i]) : (x[i] + partner);
        }
#pragma unroll
      for (int i = 0; i < V; i++) x[i] = x[i] * inv_sqrt_pd * signs[lane * V + i];
    }
    _Float16* dst = o + ((int64_t)b * Hq + h) * PD + lane * V;
#pragma unroll
    for (int i = 0; i < V; i++) dst[i] = (_Float16)x[i];
  }
}

int check_geometry(int pd, int hq, int hkv, int bs, int ebs, const char* who) {
  if (pd != 64 && pd != 128 && pd != 256) {
    set_error("%s: padded_dim must be 64, 128 or 256, got %d", who, pd);
    return kEinval;
  }
  if (hkv <= 0 || hq <= 0 || hq % hkv != 0 || hq / hkv > 16) {
    set_error("%s: num_qo_heads %d / num_kv_heads %d must be an integer <= 16", who, hq, hkv);
    return kEinval;
  }
  if (bs <= 0 || bs % kTile != 0) {
    set_error("%s: block_size %d must be a positive multiple of 16", who, bs);
    return kEinval;
  }
  if (ebs % 16 != 0 || ebs < pd / 2 + 2 * (pd / 64)) {
    set_error("%s: ebs %d must be a multiple of 16 and >= %d", who, ebs, pd / 2 + 2 * (pd / 64));
    return kEinval;
  }
  return 0;
}

}  // namespace
}  // namespace tq

extern "C" int tq_decode_partials(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                  const uint8_t* k_slab, const uint8_t* v_slab,
                                  const int32_t* indices, const int32_t* indptr,
                                  const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads,
                                  int32_t num_kv_heads, int32_t padded_dim, int32_t block_size,
                                  int32_t ebs, int64_t num_blocks, float sm_scale,
                                  const float* signs, int32_t num_splits, int32_t kv_chunk_size,
                                  float* partition_o, float* partition_lse, tq_stream_t stream) {
  using namespace tq;
  int rc = check_geometry(padded_dim, num_qo_heads, num_kv_heads, block_size, ebs, "decode");
  if (rc) return rc;
  if (batch < 0 || num_splits < 1 || kv_chunk_size < 1) {
    set_error("decode: batch %d, num_splits %d, kv_chunk_size %d out of range", batch,
              num_splits, kv_chunk_size);
    return kEinval;
  }
  if (batch == 0) return 0;
  if (!q || !k_slab || !v_slab || !indices || !indptr || !seq_lens || !partition_o ||
      !partition_lse) {
    set_error("decode: null pointer");
    return kEinval;
  }
  if ((uintptr_t)k_slab % 16 || (uintptr_t)v_slab % 16 || (uintptr_t)partition_o % 16) {
    set_error("decode: cache slabs and partition_o must be 16-byte aligned");
    return kEinval;
  }
  const int pd = padded_dim;
  const int ratio = num_qo_heads / num_kv_heads;
  int G = 1;
  for (int g = 8; g >= 1; g--)
    if (num_kv_heads % g == 0 && g * ratio * pd <= 16384) {
      G = g;
      break;
    }
  DecodeParams p;
  p.q = static_cast<const _Float16*>(q);
  p.q_sb = q_stride_b;
  p.q_sh = q_stride_h;
  p.ks = k_slab;
  p.vs = v_slab;
  p.indices = indices;
  p.indptr = indptr;
  p.seq_lens = seq_lens;
  p.signs = signs;
  p.po = partition_o;
  p.plse = partition_lse;
  p.num_blocks = num_blocks > 0x7fffffffLL ? 0x7fffffff : (int)num_blocks;
  p.B = batch;
  p.Hq = num_qo_heads;
  p.Hkv = num_kv_heads;
  p.ratio = ratio;
  p.block_size = block_size;
  p.ebs = ebs;
  p.S = num_splits;
  p.cs = kv_chunk_size;
  p.G = G;
  p.HG = num_kv_heads / G;
  p.inv_sqrt_pd = 1.0f / sqrtf((float)pd);
  p.qk_scale = sm_scale * 1.4426950408889634f * p.inv_sqrt_pd / kCbScale;
  p.pv_scale = p.inv_sqrt_pd / kCbScale;
  const int64_t blocks = (int64_t)batch * num_splits * p.HG;
  if (blocks > 0x7fffffffLL) {
    set_error("decode: grid too large");
    return kEinval;
  }
  const size_t lds = (size_t)G * ratio * pd * sizeof(float);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((unsigned)blocks), block(64 * G);
  switch (pd) {
    case 64:
      hipLaunchKernelGGL(decode_partials_kernel<64>, grid, block, lds, st, p);
      break;
    case 128:
      hipLaunchKernelGGL(decode_partials_kernel<128>, grid, block, lds, st, p);
      break;
    default:
      hipLaunchKernelGGL(decode_partials_kernel<256>, grid, block, lds, st, p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("decode: launch failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}

extern "C" int tq_combine_splits(const float* partition_o, const float* partition_lse,
                                 int32_t batch, int32_t num_splits, int32_t num_qo_heads,
                                 int32_t padded_dim, const float* signs, void* o,
                                 tq_stream_t stream) {
  using namespace tq;
  const int pd = padded_dim;
  if (pd != 64 && pd != 128 && pd != 256) {
    set_error("combine: padded_dim must be 64, 128 or 256, got %d", pd);
    return kEinval;
  }
  if (batch < 0 || num_splits < 1 || num_qo_heads < 1) {
    set_error("combine: bad sizes");
    return kEinval;
  }
  if (batch == 0) return 0;
  if (!partition_o || !partition_lse || !o) {
    set_error("combine: null pointer");
    return kEinval;
  }
  const int64_t blocks = (int64_t)batch * num_qo_heads;
  if (blocks > 0x7fffffffLL) {
    set_error("combine: grid too large");
    return kEinval;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const float isq = 1.0f / sqrtf((float)pd);
  _Float16* out = static_cast<_Float16*>(o);
  // LDS: split weights, later reused for the group partial sums (256*4 floats)
  const size_t lds = sizeof(float) * (size_t)(num_splits > 1024 ? num_splits : 1024);
  if (lds > 60 * 1024) {
    set_error("combine: num_splits %d too large", num_splits);
    return kEinval;
  }
  dim3 grid((unsigned)blocks), block(256);
  switch (pd) {
    case 64:
      hipLaunchKernelGGL(combine_kernel<64>, grid, block, lds, st, partition_o, partition_lse,
                         num_splits, num_qo_heads, signs, isq, out);
      break;
    case 128:
      hipLaunchKernelGGL(combine_kernel<128>, grid, block, lds, st, partition_o, partition_lse,
                         num_splits, num_qo_heads, signs, isq, out);
      break;
    default:
      hipLaunchKernelGGL(combine_kernel<256>, grid, block, lds, st, partition_o, partition_lse,
                         num_splits, num_qo_heads, signs, isq, out);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("combine: launch failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}

extern "C" int tq_decode_paged_splitkv(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                       const uint8_t* k_slab, const uint8_t* v_slab,
                                       const int32_t* indices, const int32_t* indptr,
                                       const int32_t* seq_lens, int32_t batch,
                                       int32_t num_qo_heads, int32_t num_kv_heads,
                                       int32_t head_dim, int32_t padded_dim, int32_t block_size,
                                       int32_t ebs, int64_t num_blocks, float sm_scale,
                                       const float* signs, int32_t num_splits,
                                       int32_t kv_chunk_size, float* partition_o,
                                       float* partition_lse, void* o, tq_stream_t stream) {
  using namespace tq;
  if (head_dim <= 0 || head_dim > padded_dim) {
    set_error("decode: head_dim %d exceeds padded_dim %d", head_dim, padded_dim);
    return kEinval;
  }
  int rc = tq_decode_partials(q, q_stride_b, q_stride_h, k_slab, v_slab, indices, indptr,
                              seq_lens, batch, num_qo_heads, num_kv_heads, padded_dim,
                              block_size, ebs, num_blocks, sm_scale, signs, num_splits,
                              kv_chunk_size, partition_o, partition_lse, stream);
  if (rc) return rc;
  return tq_combine_splits(partition_o, partition_lse, batch, num_splits, num_qo_heads,
                           padded_dim, signs, o, stream);
}
