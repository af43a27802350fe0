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
// tables indexed by 7 - m (byte j holds magnitude 7 - j)
constexpr uint32_t kHiR0 = 0x3f404244u, kHiR1 = 0x32383b3du;
constexpr uint32_t kLoR0 = 0x71cb210cu, kLoR1 = 0x1699c895u;

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
  // c[n] = (n >= 8) ? M[n-8] : -M[7-n].  G = D ^ (7 in every nibble whose
  // bit 3 is set): the low 3 bits of each nibble of G are 7 - magnitude
  // index and bit 3 stays set exactly for the non-negative codes.
  const uint32_t a = D & 0x88888888u;
  const uint32_t G = D ^ (a - (a >> 3));
  const uint32_t SL = G & 0x07070707u;
  const uint32_t SH = (G >> 4) & 0x07070707u;
  const uint32_t hL = perm(kHiR1, kHiR0, SL) | (~(G << 4) & 0x80808080u);
  const uint32_t lL = perm(kLoR1, kLoR0, SL);
  const uint32_t hH = perm(kHiR1, kHiR0, SH) | (~G & 0x80808080u);
  const uint32_t lH = perm(kLoR1, kLoR0, SH);
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
  int share0;         // two splits per workgroup: 256ths of the pair's tokens for the first
};

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
// rotate by 8 lanes inside each 16-lane row (DPP row_ror:8)
__device__ __forceinline__ float ror8(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xf, 0xf, false));
}
// fp16 value held in the low / high half of a dword
__device__ __forceinline__ float lo_half(uint32_t v) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu));
}
__device__ __forceinline__ float hi_half(uint32_t v) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
}

// Static LDS geometry of the decode kernel.  A step is two 16-token tiles;
// one staged step holds, for the workgroup's G heads, the K slab then the V
// slab, each [32 token rows][G*ebs bytes].  ROW = the largest G*ebs a
// workgroup may take for this head size.
template <int PD>
struct DecodeGeom {
  static constexpr int KD = PD / 32;  // K dwords per lane per tile = QK MFMA pairs
  static constexpr int VB = PD / 32;  // V bytes per lane per token
  static constexpr int NO = PD / 16;  // PV MFMAs = output dim slots per lane
  static constexpr int EBS = PD == 64 ? 48 : (PD == 128 ? 80 : 144);  // entry bytes
  static constexpr int MAXG = PD == 256 ? 4 : 8;          // kv heads (waves) per workgroup
  static constexpr int WAVE_STEP = 2 * 2 * kTile * EBS;  // one wave's staged step (K+V, 2 tiles)
};

// Online-softmax state of one wave.  O[i][r] = unnormalised o[h = l%16][dim
// (4*q4 + r)*NO + i] in the rotated domain.  m = running max of the scores
// (log2 units, replicated over the lanes of a head), lsum = this lane's
// share of the denominator.  Probabilities are formed as p' = exp2(s - mb),
// mb = m + Lpv with Lpv = -log2(pv_scale), i.e. p' = p * pv_scale: the V
// norm then multiplies in without leaving the fp16 range; o = pv_scale * O /
// lsum', and mb + log2(lsum') is the LSE (log2 units).
template <int PD>
struct SoftmaxState {
  float4_t O[DecodeGeom<PD>::NO];
  float m, mb, lsum;
};

// LDS byte address of dequant-table entry `byte k of w` for this lane.  The
// table sits at LDS address 0 with LREP copies of each entry side by side
// (entry e, copy r at dword e * LREP + r).  With 64 copies lane l reads
// copy l, so a table read never has a bank conflict, and the address is one
// byte permute: byte 0 = 4 l (lane4), byte 1 = the code byte.
template <int LREP>
__device__ __forceinline__ uint32_t lut_addr(uint32_t w, int k, uint32_t lane4) {
  if constexpr (LREP == 64) {
    return perm(w, lane4, 0x0c0c0000u | ((4u + (uint32_t)k) << 8));
  } else {
    static_assert(LREP == 1, "table copies: 1 or 64");
    (void)lane4;
    return ((w >> (8 * k)) & 0xffu) << 2;
  }
}

// Eight table reads and one wait (inline assembly: the compiler does not
// see them, so it adds no conservative wait for the copies in flight).
__device__ __forceinline__ void lut_read8(const uint32_t* a, uint32_t* x) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile(
      "ds_read_b32 %0, %8\n\t"
      "ds_read_b32 %1, %9\n\t"
      "ds_read_b32 %2, %10\n\t"
      "ds_read_b32 %3, %11\n\t"
      "ds_read_b32 %4, %12\n\t"
      "ds_read_b32 %5, %13\n\t"
      "ds_read_b32 %6, %14\n\t"
      "ds_read_b32 %7, %15\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]), "=&v"(x[3]), "=&v"(x[4]), "=&v"(x[5]),
        "=&v"(x[6]), "=&v"(x[7])
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]),
        "v"(a[7])
      : "memory");
#else
  for (int i = 0; i < 8; i++) x[i] = a[i];
#endif
}

// Scores of one tile, S[t = 4*q4 + r][h = l%16]: the K codes this lane
// holds (token l%16, dims of quarter q4; byte j of dword c = dims 8c + 2j,
// 8c + 2j + 1) are dequantized through the LDS table (code byte -> fp16
// values of its high and low nibble, one ds_read each), then the QK MFMAs
// run against q' (pre-scaled to log2 units) as fp16 hi + lo parts.  QC: the
// B operand holds the hi parts in columns 0..7 and the lo parts in columns
// 8..15 (GQA ratio <= 8), one MFMA per K block, and the two halves are added
// across lanes n and n+8 (both end up with the sum); otherwise qb/ql are
// separate hi/lo operands, two MFMAs per K block.
template <int PD, bool QC, int LREP>
__device__ __forceinline__ float4_t tile_scores(const uint32_t* kw, const half8_t* qb,
                                                const half8_t* ql, uint32_t lane4) {
  constexpr int KD = PD / 32;
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < KD; c += 2) {
    // two K blocks per batch of 8 table reads and one wait
    uint32_t a[8], x[8];
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
      for (int j = 0; j < 4; j++) a[4 * u + j] = lut_addr<LREP>(kw[c + u], j, lane4);
    lut_read8(a, x);
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const half8_t kv8 = as_half8(x[4 * u], x[4 * u + 1], x[4 * u + 2], x[4 * u + 3]);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv8, qb[c + u], acc, 0, 0, 0);
      if constexpr (!QC)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv8, ql[c + u], acc, 0, 0, 0);
    }
  }
  if constexpr (QC) {
#pragma unroll
    for (int r = 0; r < 4; r++) acc[r] = acc[r] + ror8(acc[r]);
  }
  return acc;
}

// O[h][dim slot] += V^T P^T over the 32 tokens of one step with
// v_mfma_f32_16x16x32_f16: the 8 k-values of a lane are tokens 4*q4 + 0..3
// of tile 0 followed by the same tokens of tile 1, in both A (dequantized
// V^T, row = dim slot) and B (probabilities p * nv, column = head).
// v0 / v1[j] = this lane's V code bytes of token 4*q4 + j of tile 0 / 1
// (dword w = bytes 4w..4w+3 of the lane's PD/32).  The A operand needs
// fp16 pairs of one dim over two tokens, so the table index of a pair is
// built from the two tokens' nibbles of one code byte (first token's
// nibble high): the table maps it to (value of the first, value of the
// second).  Byte k's low nibbles give dim slot 2k + 1, its high nibbles
// dim slot 2k.
template <int PD, int LREP>
__device__ __forceinline__ void step_pv(const uint32_t (*v0)[(PD / 32) >= 4 ? PD / 128 : 1],
                                        const uint32_t (*v1)[(PD / 32) >= 4 ? PD / 128 : 1],
                                        half8_t p, SoftmaxState<PD>& st, uint32_t lane4) {
  constexpr int VB = PD / 32;
  constexpr int VW = VB >= 4 ? VB / 4 : 1;
  // ix[T][pair][nibble][w]: pair 0 = tokens 0, 1; pair 1 = tokens 2, 3;
  // nibble 0 = low nibbles, 1 = high nibbles
  uint32_t ix[2][2][2][VW];
#pragma unroll
  for (int T = 0; T < 2; T++) {
    const uint32_t (*v)[VW] = T ? v1 : v0;
#pragma unroll
    for (int pr = 0; pr < 2; pr++)
#pragma unroll
      for (int w = 0; w < VW; w++) {
        const uint32_t a = v[2 * pr][w], b = v[2 * pr + 1][w];
        ix[T][pr][0][w] = ((a << 4) & 0xf0f0f0f0u) | (b & 0x0f0f0f0fu);
        ix[T][pr][1][w] = (a & 0xf0f0f0f0u) | ((b >> 4) & 0x0f0f0f0fu);
      }
  }
#pragma unroll
  for (int k = 0; k < VB; k++) {
    const int w = k / 4, j = k % 4;
    uint32_t a[8], x[8];
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
#pragma unroll
      for (int T = 0; T < 2; T++)
#pragma unroll
        for (int pr = 0; pr < 2; pr++)
          a[4 * nb + 2 * T + pr] = lut_addr<LREP>(ix[T][pr][nb][w], j, lane4);
    lut_read8(a, x);
    const half8_t lo8 = as_half8(x[0], x[1], x[2], x[3]);
    const half8_t hi8 = as_half8(x[4], x[5], x[6], x[7]);
    st.O[2 * k + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(lo8, p, st.O[2 * k + 1], 0, 0, 0);
    st.O[2 * k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(hi8, p, st.O[2 * k], 0, 0, 0);
  }
}

// This wave's share of one staged step, read from LDS into registers.
template <int PD>
struct StepData {
  static constexpr int KD = PD / 32;
  static constexpr int VW = (PD / 32) >= 4 ? PD / 128 : 1;
  uint32_t k[2][KD];     // K codes of tiles 0 and 1
  uint32_t v[2][4][VW];  // V codes of tiles 0 and 1, tokens 4*q4 + j
  uint32_t nkv[2];       // norms (K low, V high) of the packed tokens, per group
};

// s_waitcnt immediate that waits until at most n vector-memory operations
// are outstanding (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] |
// vmcnt[5:4] in [15:14]; expcnt and lgkmcnt left at their maximum).
__host__ __device__ constexpr int vmcnt_imm(int n) {
  return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14);
}

// LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* ptr) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)ptr;
}

// This wave's V share of one staged step, read from LDS into registers, as
// inline assembly ending in lgkmcnt(0): the compiler does not see these LDS
// reads, so it adds no conservative wait for the copies in flight; the
// caller waits for exactly the copy it reads (vmcnt).  Staged layout of one
// step of one wave: regions V t0, V t1 of TB bytes; a region holds the 16
// tokens' codes (CB bytes each, token-major) followed by their 16-byte entry
// tails (norm copies and pad).  nv[T] = V norm bits of token
// 4*q4 + (lane & 3) of tile T (PACK 2 reads only the lane's own tile).
template <int PD, int PACK>
__device__ __forceinline__ void read_v_asm(const uint8_t* wslot, uint32_t voff, uint32_t noff,
                                           StepData<PD>& d, uint32_t* nv) {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass only needs the kernel stubs
  constexpr int CB = PD / 2;            // code bytes per token
  constexpr int TB = kTile * (CB + 16);  // one staged tile
  constexpr int N1 = PACK == 2 ? 0 : TB;  // second norm: tile 1 (PACK 1 only)
  const uint32_t base = lds_addr(wslot);
  const uint32_t va = base + voff;
  const uint32_t na = base + noff;
  if constexpr (PD == 128 || PD == 64) {
    uint32_t v0, v1, v2, v3, v4, v5, v6, v7;
    if constexpr (PD == 128) {
      asm volatile(
          "ds_read_b32 %0, %10\n\t"
          "ds_read_b32 %1, %10 offset:%12\n\t"
          "ds_read_b32 %2, %10 offset:%13\n\t"
          "ds_read_b32 %3, %10 offset:%14\n\t"
          "ds_read_b32 %4, %10 offset:%15\n\t"
          "ds_read_b32 %5, %10 offset:%16\n\t"
          "ds_read_b32 %6, %10 offset:%17\n\t"
          "ds_read_b32 %7, %10 offset:%18\n\t"
          "ds_read_u16 %8, %11\n\t"
          "ds_read_u16 %9, %11 offset:%19\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3), "=&v"(v4), "=&v"(v5), "=&v"(v6),
            "=&v"(v7), "=&v"(nv[0]), "=&v"(nv[1])
          : "v"(va), "v"(na), "i"(CB), "i"(2 * CB), "i"(3 * CB), "i"(TB), "i"(TB + CB),
            "i"(TB + 2 * CB), "i"(TB + 3 * CB), "i"(N1)
          : "memory");
    } else {
      asm volatile(
          "ds_read_u16 %0, %10\n\t"
          "ds_read_u16 %1, %10 offset:%12\n\t"
          "ds_read_u16 %2, %10 offset:%13\n\t"
          "ds_read_u16 %3, %10 offset:%14\n\t"
          "ds_read_u16 %4, %10 offset:%15\n\t"
          "ds_read_u16 %5, %10 offset:%16\n\t"
          "ds_read_u16 %6, %10 offset:%17\n\t"
          "ds_read_u16 %7, %10 offset:%18\n\t"
          "ds_read_u16 %8, %11\n\t"
          "ds_read_u16 %9, %11 offset:%19\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3), "=&v"(v4), "=&v"(v5), "=&v"(v6),
            "=&v"(v7), "=&v"(nv[0]), "=&v"(nv[1])
          : "v"(va), "v"(na), "i"(CB), "i"(2 * CB), "i"(3 * CB), "i"(TB), "i"(TB + CB),
            "i"(TB + 2 * CB), "i"(TB + 3 * CB), "i"(N1)
          : "memory");
    }
    d.v[0][0][0] = v0; d.v[0][1][0] = v1; d.v[0][2][0] = v2; d.v[0][3][0] = v3;
    d.v[1][0][0] = v4; d.v[1][1][0] = v5; d.v[1][2][0] = v6; d.v[1][3][0] = v7;
  } else {
    u32x2 v0, v1, v2, v3, v4, v5, v6, v7;
    asm volatile(
        "ds_read_b64 %0, %10\n\t"
        "ds_read_b64 %1, %10 offset:%12\n\t"
        "ds_read_b64 %2, %10 offset:%13\n\t"
        "ds_read_b64 %3, %10 offset:%14\n\t"
        "ds_read_b64 %4, %10 offset:%15\n\t"
        "ds_read_b64 %5, %10 offset:%16\n\t"
        "ds_read_b64 %6, %10 offset:%17\n\t"
        "ds_read_b64 %7, %10 offset:%18\n\t"
        "ds_read_u16 %8, %11\n\t"
        "ds_read_u16 %9, %11 offset:%19\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3), "=&v"(v4), "=&v"(v5), "=&v"(v6),
          "=&v"(v7), "=&v"(nv[0]), "=&v"(nv[1])
        : "v"(va), "v"(na), "i"(CB), "i"(2 * CB), "i"(3 * CB), "i"(TB), "i"(TB + CB),
          "i"(TB + 2 * CB), "i"(TB + 3 * CB), "i"(N1)
        : "memory");
    const u32x2 vv[8] = {v0, v1, v2, v3, v4, v5, v6, v7};
#pragma unroll
    for (int T = 0; T < 2; T++)
#pragma unroll
      for (int j = 0; j < 4; j++) { d.v[T][j][0] = vv[4 * T + j][0]; d.v[T][j][1] = vv[4 * T + j][1]; }
  }
#else
  (void)wslot; (void)voff; (void)noff; (void)d; nv[0] = nv[1] = 0;
#endif
}

// Online softmax over the NV score values this lane holds for one step
// (PACK 2: 4 values, tile (l%16)/8, head l%8; PACK 1: 8 values, tile 0 then
// tile 1, head l%16; tokens 4*q4 + r).  nk / nv: the tokens' K and V norms.
// valid: token masks, `full` when all are valid.  Writes p * nv (fp16) to
// pv; the running max only moves when the step exceeds it by more than 2^3,
// so p <= 8.
template <int PD, int NV>
__device__ __forceinline__ void softmax_step(float* sc, const float* nk, const float* nv,
                                             bool full, const bool* valid, bool rot8, int head,
                                             int ratio, float lpv, SoftmaxState<PD>& st,
                                             _Float16* pv) {
  constexpr int NO = PD / 16;
#pragma unroll
  for (int r = 0; r < NV; r++) sc[r] = sc[r] * nk[r];
  if (!full) {
#pragma unroll
    for (int r = 0; r < NV; r++) sc[r] = valid[r] ? sc[r] : -INFINITY;
  }
  float tmax = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
  if constexpr (NV == 8) tmax = fmaxf(tmax, fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
  if (rot8) tmax = fmaxf(tmax, ror8(tmax));
  tmax = xor16_max(tmax);
  tmax = xor32_max(tmax);
  const float m_new = fmaxf(st.m, tmax);
  const bool need = (head < ratio) && (m_new > st.m + 3.0f);
  if (__any(need)) {
    const float alpha = (m_new == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(st.m - m_new);
#pragma unroll
    for (int i = 0; i < NO; i++) st.O[i] *= alpha;
    st.lsum *= alpha;
    st.m = m_new;
    st.mb = m_new + lpv;
  }
  float pr[NV];
#pragma unroll
  for (int r = 0; r < NV; r++) pr[r] = __builtin_amdgcn_exp2f(sc[r] - st.mb);
  if (!full) {
#pragma unroll
    for (int r = 0; r < NV; r++) pr[r] = valid[r] ? pr[r] : 0.0f;
  }
  float ls = (pr[0] + pr[1]) + (pr[2] + pr[3]);
  if constexpr (NV == 8) ls += (pr[4] + pr[5]) + (pr[6] + pr[7]);
  st.lsum += ls;
#pragma unroll
  for (int r = 0; r < NV; r++) {
    float x = pr[r] * nv[r];
    if (!full) x = valid[r] ? x : 0.0f;  // masked entries may hold any bits
    pv[r] = (_Float16)x;
  }
}

// Bring tile 1's packed probabilities (lanes 8..15 of each row) to lanes
// 0..7 (DPP row_shl:8), the B-operand position of the PV MFMA.
__device__ __forceinline__ half4_t shl8(half4_t v) {
  u32x2 u = __builtin_bit_cast(u32x2, v);
  u[0] = (uint32_t)__builtin_amdgcn_mov_dpp((int)u[0], 0x108, 0xf, 0xf, false);
  u[1] = (uint32_t)__builtin_amdgcn_mov_dpp((int)u[1], 0x108, 0xf, 0xf, false);
  return __builtin_bit_cast(half4_t, u);
}

// Split-KV partials.  Workgroup = (sequence b, split s, group hg of G kv
// heads), one wave per kv head.  Each wave streams its own head's cache
// entries of each step (two 16-token tiles, K and V) into its own region of
// NSLOT LDS slots with direct-to-LDS 16-byte loads, NSLOT - 1 steps ahead of
// the step it computes.  Waves never wait on each other after the q setup:
// the slots are distinct LDS arrays, so the compiler ties every LDS read to
// the one copy it depends on and leaves the later copies in flight.
template <int PD, int PACK, bool QC, int SPW>
__global__ __launch_bounds__(64 * DecodeGeom<PD>::MAXG * SPW)
__attribute__((amdgpu_waves_per_eu(PD == 256 ? 2 : (PACK == 1 ? 3 : 4))))
void decode_partials_kernel(DecodeParams p) {
  using Geo = DecodeGeom<PD>;
  constexpr int KD = Geo::KD;
  constexpr int NO = Geo::NO;
  constexpr int EBS = Geo::EBS;
  constexpr int WB = 2 * kTile * EBS;  // bytes of one staged step (V, two tiles) of one wave
  constexpr int MG = Geo::MAXG;
  // dequant table copies: one per lane when two splits share the workgroup
  // (which then has the CU's LDS to itself), else one
  constexpr int LREP = SPW == 2 ? 64 : 1;
  // LDS: the dequant table first (LDS address 0, which the table reads rely
  // on), then two staging slots
  struct __attribute__((aligned(16))) Lds {
    uint32_t klut[256 * LREP];
    uint8_t slot0[SPW * MG * WB];
    uint8_t slot1[SPW * MG * WB];
  };
  __shared__ Lds sm;
  uint8_t* const slot0 = sm.slot0;
  uint8_t* const slot1 = sm.slot1;
  constexpr int NSLOT = 2;  // LDS slots per wave: one step computed, one in flight

  // dequant table: byte e -> fp16 values of its high nibble (low half) and
  // its low nibble (high half), built with the same table arithmetic as
  // dq8; LREP copies of each entry side by side (written 4 at a time)
  auto lut_val = [](int e) {
    uint32_t x[4];
    dq8((uint32_t)e * 0x01010101u, x);
    return (x[2] & 0xffffu) | (x[0] << 16);
  };
  if constexpr (LREP == 1) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x) sm.klut[i] = lut_val(i);
  } else {
    for (int i = threadIdx.x; i < 64 * LREP; i += blockDim.x) {
      const uint32_t val = lut_val(i / (LREP / 4));
      *reinterpret_cast<u32x4*>(&sm.klut[4 * i]) = u32x4{val, val, val, val};
    }
  }
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int q4 = lane >> 4, n = lane & 15;
  const uint32_t lane4 = (uint32_t)lane * 4;  // this lane's table copy (byte offset)
  // SPW splits per workgroup: waves [sub * G, (sub + 1) * G) serve split
  // SPW * (split group) + sub, so one workgroup fills a CU's wave slots and
  // its waves start together
  const int G = p.G;
  const int sub = SPW == 1 ? 0 : w / G;  // uniform
  const int hw = w - sub * G;            // kv head within the group
  const int nsg = (p.S + SPW - 1) / SPW;  // split groups per sequence
  int bid = blockIdx.x;
  const int hg = bid % p.HG;
  bid /= p.HG;
  const int s = (bid % nsg) * SPW + sub;
  const int b = bid / nsg;
  const int kvh = hg * G + hw;
  const int ratio = p.ratio;

  half8_t qb[KD], ql[QC ? 1 : KD];  // q' operands, filled once the first copy is in flight

  // s * q of this wave's heads, loaded first so that its latency overlaps
  // the page-table loads and the first copies: in load j < NQL, lane l holds
  // the 8 consecutive elements e = 512 j + 8 l .. + 7 (head e / PD, dim
  // e % PD).  Elements past the wave's heads read as zeros (empty range).
  // Larger head groups (ratio * PD > 512 * NQL) form q' through LDS below.
  constexpr int NQL = 2;
  const bool qreg = ratio * PD <= 512 * NQL;  // uniform
  float qx[NQL][8];
#if defined(__HIP_DEVICE_COMPILE__)
  {
    const _Float16* qbase = p.q + (int64_t)b * p.q_sb + (int64_t)kvh * ratio * p.q_sh;
    const int qrec = qreg ? (int)(((ratio - 1) * p.q_sh + PD) * 2) : 0;
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc((void*)qbase, (short)0, qrec, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsg = __builtin_amdgcn_make_buffer_rsrc(
        (void*)p.signs, (short)0, p.signs ? PD * 4 : 0, 0x00020000);
#pragma unroll
    for (int j = 0; j < NQL; j++) {
      const int e = 512 * j + 8 * lane;
      const int r = e / PD, d = e % PD;
      const u32x4 qv = __builtin_amdgcn_raw_buffer_load_b128(
          rq, (uint32_t)((r * p.q_sh + d) * 2), 0, 0);
      const u32x4 s0 = __builtin_amdgcn_raw_buffer_load_b128(rsg, (uint32_t)(d * 4), 0, 0);
      const u32x4 s1 = __builtin_amdgcn_raw_buffer_load_b128(rsg, (uint32_t)(d * 4 + 16), 0, 0);
      const uint32_t sw[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const float x = k & 1 ? hi_half(qv[k / 2]) : lo_half(qv[k / 2]);
        qx[j][k] = p.signs ? x * __uint_as_float(sw[k]) : x;
      }
    }
  }
#endif

  SoftmaxState<PD> st;
#pragma unroll
  for (int i = 0; i < NO; i++) st.O[i] = float4_t{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.mb = -INFINITY;
  st.lsum = 0.f;
  const float lpv = -__log2f(p.pv_scale);

  const int L = s < p.S ? p.seq_lens[b] : 0;  // a split past the last one is empty
  int c0 = s * p.cs;
  int c1 = min(c0 + p.cs, L);
  if (SPW == 2 && s - sub + 1 < p.S) {
    // The two wave groups of a workgroup do not progress at the same rate
    // (issue arbitration favours the older waves), so the token range of the
    // split pair is divided unevenly: the first group takes share0/256 of it,
    // rounded to whole 32-token steps.  Any partition merges to the same
    // attention.
    const int base = (s - sub) * p.cs;
    const int end = min(base + 2 * p.cs, p.seq_lens[b]);
    const int mid = min(end, base + ((max(end - base, 0) * p.share0 / 256 + 31) & ~31));
    c0 = sub ? mid : base;
    c1 = sub ? end : mid;
  }
  if (c0 < c1) {  // uniform over the workgroup
    constexpr int STEP = 2 * kTile;
    constexpr int TB = kTile * EBS;                // one tile of one slab (LDS)
    const int step0 = c0 / STEP, step1 = (c1 - 1) / STEP;
    const int tpp = p.block_size / kTile;  // tiles per page
    const int64_t tokstride = (int64_t)p.Hkv * EBS;
    const int ip = p.indptr[b];
    const uint8_t* kslab = p.ks + (int64_t)kvh * EBS;
    const uint8_t* vslab = p.vs + (int64_t)kvh * EBS;
    const int tile_last = (c1 - 1) / kTile;
    const int rec = (int)((kTile - 1) * tokstride + EBS);

    // tile offsets: lane i holds the byte offset inside a slab of tile
    // wtile + i (64 bit, as lo/hi halves) and tmask bit i says whether that
    // tile is present (within the split and on a page inside the cache).  A
    // window covers 32 steps (64 tiles) and is rebuilt between windows with
    // the copies drained.
    uint32_t tlo = 0, thi = 0;
    uint64_t tmask = 0;
    int wtile = 2 * step0;
    auto tile_ok = [&](int t) -> bool { return (tmask >> ((t - wtile) & 63)) & 1; };
    auto tile_base = [&](const uint8_t* slab, int t) -> const uint8_t* {
      const int j = (t - wtile) & 63;
      const uint64_t lo = (uint32_t)__builtin_amdgcn_readlane((int)tlo, j);
      const uint64_t hi = (uint32_t)__builtin_amdgcn_readlane((int)thi, j);
      return slab + (int64_t)((hi << 32) | lo);
    };

    // Copies of one region (16 tokens of one slab): the codes as CI
    // instructions of CW bytes per lane (lane-contiguous in LDS, token-major
    // with CB bytes per token), then the 16-byte entry tails (norm copies and
    // pad) as one 4-byte-per-lane instruction.  Every lane of every copy is
    // active, so the copies never sit under divergent control flow.
    constexpr int CB = PD / 2;                // code bytes per token
    constexpr int CW = PD == 64 ? 4 : 16;     // bytes per lane of a code copy
    constexpr int CI = kTile * CB / (64 * CW);  // code copies per region
    constexpr int CPT = CB / CW;              // lanes per token in a code copy
    uint32_t goff[CI];
#pragma unroll
    for (int i = 0; i < CI; i++) {
      const int c = 64 * i + lane;
      goff[i] = (uint32_t)((c / CPT) * tokstride + (c % CPT) * CW);
    }
    const uint32_t gtail = (uint32_t)((lane >> 2) * tokstride + CB + (lane & 3) * 4);
    // K of one step straight into registers: lane (token n, quarter q4)
    // loads its PD/8 code bytes of each tile and the K norm of token
    // 4*q4 + (lane & 3) of each tile (absent tiles read as zeros)
    struct KRegs {
      uint32_t k[2][KD];
      uint32_t nk[2];
    };
    const uint32_t kcoff = (uint32_t)(n * tokstride + q4 * (PD / 8));
    const uint32_t knoff = (uint32_t)((4 * q4 + (lane & 3)) * tokstride + CB);
    // K codes and norms of step k into kr (absent tiles read as zeros)
    // The loads are inline assembly: the compiler does not track them, so it
    // inserts no wait of its own; run() waits for them explicitly (vmcnt) and
    // then passes the registers through an empty asm so that no use can move
    // above that wait.
    auto stageK = [&](int k, KRegs& kr) {
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
      for (int T = 0; T < 2; T++) {
        const uint64_t base = (uint64_t)tile_base(kslab, 2 * k + T);
        const u32x4 rk = {(uint32_t)base, (uint32_t)(base >> 32) & 0xffffu,
                          (uint32_t)(tile_ok(2 * k + T) ? rec : 0), 0x00020000u};
        if constexpr (PD == 64) {
          u32x2 v;
          asm volatile("buffer_load_dwordx2 %0, %1, %2, 0 offen"
                       : "=v"(v)
                       : "v"(kcoff), "s"(rk)
                       : "memory");
          kr.k[T][0] = v[0];
          kr.k[T][1] = v[1];
        } else {
#pragma unroll
          for (int h = 0; h < KD / 4; h++) {
            u32x4 v;
            asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen offset:%3"
                         : "=v"(v)
                         : "v"(kcoff), "s"(rk), "i"(16 * h)
                         : "memory");
#pragma unroll
            for (int i = 0; i < 4; i++) kr.k[T][4 * h + i] = v[i];
          }
        }
        asm volatile("buffer_load_ushort %0, %1, %2, 0 offen"
                     : "=v"(kr.nk[T])
                     : "v"(knoff), "s"(rk)
                     : "memory");
      }
#else
      (void)k;
      (void)kr;
#endif
    };
    // V copies of step k into this wave's region of one slot (regions V t0,
    // V t1 of TB bytes each)
    auto stage = [&](int k, uint8_t* dst) {
#if defined(__HIP_DEVICE_COMPILE__)  // the LDS-copy builtin has no host form
#pragma unroll
      for (int r = 0; r < 2; r++) {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)tile_base(vslab, 2 * k + r), (short)0, tile_ok(2 * k + r) ? rec : 0,
            0x00020000);
#pragma unroll
        for (int i = 0; i < CI; i++)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (void*)(dst + r * TB + i * 64 * CW), CW,
                                                   goff[i], 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (void*)(dst + r * TB + kTile * CB), 4, gtail,
                                                 0, 0, 0);
      }
#else
      (void)k;
      (void)dst;
#endif
    };

    // per-lane LDS offsets inside a staged step of this wave
    const uint32_t voff = (uint32_t)((4 * q4) * CB + n * (PD / 32));
    const int slot = 16 / PACK;    // lanes per packed tile slot
    const int ptile = n / slot;    // tile of this lane's packed scores
    const int head = n % slot;     // head of this lane's packed scores
    const uint32_t noff = (uint32_t)(ptile * TB + kTile * CB + (4 * q4 + (lane & 3)) * 16);

    // math of one step; `kr` holds this step's K on entry and receives the
    // next step's K (loads issued once the scores no longer need it)
    auto compute = [&](int k, const StepData<PD>& d, KRegs& kr, bool knext) {
      const bool okT[2] = {tile_ok(2 * k), tile_ok(2 * k + 1)};
      // scores of both tiles (scheduling barriers keep the two tiles'
      // dequant temporaries from being live at the same time)
      float4_t acc[2];
      acc[0] = tile_scores<PD, QC, LREP>(kr.k[0], qb, ql, lane4);
      __builtin_amdgcn_sched_barrier(0);
      acc[1] = tile_scores<PD, QC, LREP>(kr.k[1], qb, ql, lane4);
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t nk01[2] = {kr.nk[0], kr.nk[1]};
      if (knext) stageK(k + 1, kr);
      constexpr int NV = 4 * (2 / PACK);  // score values per lane
      float sc[NV], nk[NV], nv[NV];
      bool valid[NV];
#pragma unroll
      for (int g = 0; g < 2 / PACK; g++) {
        const uint32_t nkv =
            (PACK == 2 ? (ptile ? nk01[1] : nk01[0]) : nk01[g]) | (d.nkv[g] << 16);
        const uint32_t nr[4] = {quad_bcast<0>(nkv), quad_bcast<1>(nkv), quad_bcast<2>(nkv),
                                quad_bcast<3>(nkv)};
#pragma unroll
        for (int r = 0; r < 4; r++) {
          nk[4 * g + r] = lo_half(nr[r]);
          nv[4 * g + r] = hi_half(nr[r]);
          if constexpr (PACK == 2) {
            // tile 0's scores in lanes 0..7 of each row, tile 1's in 8..15
            // (with QC both halves of a row hold the same sums)
            sc[r] = n < 8 ? acc[0][r] : acc[1][r];
          } else {
            sc[4 * g + r] = acc[g][r];
          }
        }
      }
      const int t_first = 2 * k * kTile;  // first token of this step
      const bool full = okT[0] && okT[1] && t_first >= c0 && t_first + 2 * kTile <= c1;
      if (!full) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
          const int T = PACK == 2 ? ptile : i / 4;
          const int t = (2 * k + T) * kTile + 4 * q4 + (i & 3);
          valid[i] = okT[T] && t >= c0 && t < c1;
        }
      }
      _Float16 pv[NV];
      softmax_step<PD, NV>(sc, nk, nv, full, valid, PACK == 2, head, ratio, lpv, st, pv);
      half8_t p8;
      if constexpr (PACK == 2) {
        half4_t p4 = {pv[0], pv[1], pv[2], pv[3]};
        const half4_t p4b = shl8(p4);
        p8 = half8_t{p4[0], p4[1], p4[2], p4[3], p4b[0], p4b[1], p4b[2], p4b[3]};
      } else {
        p8 = half8_t{pv[0], pv[1], pv[2], pv[3], pv[4], pv[5], pv[6], pv[7]};
      }
      step_pv<PD, LREP>(d.v[0], d.v[1], p8, st, lane4);
    };
    // one step: wait until its copy has landed (`later` = copy instructions
    // issued after it, which may stay in flight), read this wave's region of
    // `src` into registers, then the math
    // V copies per step; the K loads of step k + 1 are issued inside step
    // k, so when step k + 1 runs only the V copies of step k + 2 may still be
    // in flight behind it
    constexpr int NVCOPY = 2 * (CI + 1);
    KRegs kr;
    auto run = [&](int k, const uint8_t* src, int wend) {
      if (k + 1 <= wend) __builtin_amdgcn_s_waitcnt(vmcnt_imm(NVCOPY));
      else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
      for (int T = 0; T < 2; T++) {
#pragma unroll
        for (int i = 0; i < KD; i++) asm volatile("" : "+v"(kr.k[T][i]));
        asm volatile("" : "+v"(kr.nk[T]));
      }
#endif
      StepData<PD> d;
      uint32_t nv[2];
      read_v_asm<PD, PACK>(src, voff, noff, d, nv);
      d.nkv[0] = nv[0];
      d.nkv[1] = nv[1];
      compute(k, d, kr, k + 1 <= wend);
    };

    const size_t wofs = (size_t)w * WB;
    auto open_window = [&](int wstep) {
      wtile = 2 * wstep;
      const int t = wtile + lane;
      const int pg = (t <= tile_last) ? p.indices[ip + t / tpp] : -1;
      const bool ok = pg >= 0 && pg < p.num_blocks;
      const int64_t off = ok ? ((int64_t)pg * p.block_size + (t % tpp) * kTile) * tokstride : 0;
      tlo = (uint32_t)off;
      thi = (uint32_t)((uint64_t)off >> 32);
      tmask = __ballot(ok);
    };
    // steps wstep + 2j live in slot A (slot1), wstep + 2j + 1 in slot B
    // (slot0); one step is in flight while the other is computed.  The first
    // copy is issued before the q setup, which may use slot0 as scratch.
    uint8_t* const sA = slot1 + wofs;
    uint8_t* const sB = slot0 + wofs;
    open_window(step0);
    stage(step0, sA);
    stageK(step0, kr);
    // with q' formed in registers, slot0 is free: the second copy goes too
    bool staged1 = false;
    if (qreg && step0 + 1 <= min(step0 + 31, step1)) {
      stage(step0 + 1, sB);
      staged1 = true;
    }
    // ---- q' = FWHT(s*q)/sqrt(pd), scaled to log2 units and split into
    // fp16 hi + lo parts (q' = hi + lo to ~22 bits, so the scores keep
    // fp32-level accuracy even for heavy-tailed keys), in the MFMA B layout.
    const float qsc = (p.signs ? p.inv_sqrt_pd : 1.0f) * p.qk_scale;
    // element order of the K operand: the table yields dims 8c + e in order
    constexpr int ord[8] = {0, 1, 2, 3, 4, 5, 6, 7};
    const int hq = QC ? (n & 7) : n;  // q head of this lane's B column
    if (qreg) {
      // in registers: butterflies h = 1, 2, 4 inside a lane, h >= 8 between
      // lanes l and l ^ (h / 8); no LDS, no barrier
      if (p.signs) {
#pragma unroll
        for (int j = 0; j < NQL; j++) {
#pragma unroll
          for (int h = 1; h < 8; h <<= 1)
#pragma unroll
            for (int k = 0; k < 8; k++)
              if (!(k & h)) {
                const float a = qx[j][k], c = qx[j][k + h];
                qx[j][k] = a + c;
                qx[j][k + h] = a - c;
              }
#pragma unroll
          for (int h = 8; h < PD; h <<= 1) {
            const bool upper = lane & (h / 8);
#pragma unroll
            for (int k = 0; k < 8; k++) {
              const float pt = __shfl_xor(qx[j][k], h / 8);
              qx[j][k] = upper ? pt - qx[j][k] : qx[j][k] + pt;
            }
          }
        }
      }
      // packed fp16 hi / lo pairs in MFMA element order
      uint32_t ph[NQL][4], pl[NQL][4];
#pragma unroll
      for (int j = 0; j < NQL; j++)
#pragma unroll
        for (int wd = 0; wd < 4; wd++) {
          const float x0 = qx[j][ord[2 * wd]] * qsc, x1 = qx[j][ord[2 * wd + 1]] * qsc;
          const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
          const _Float16 l0 = (_Float16)(x0 - (float)h0), l1 = (_Float16)(x1 - (float)h1);
          ph[j][wd] = (uint32_t)__builtin_bit_cast(uint16_t, h0) |
                      ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
          pl[j][wd] = (uint32_t)__builtin_bit_cast(uint16_t, l0) |
                      ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
        }
      // B operand: column n takes head hq, dims q4 * PD/4 + 8c + ord[.] from
      // the lane holding those 8 elements
#pragma unroll
      for (int c = 0; c < KD; c++) {
        const int e = hq * PD + q4 * (PD / 4) + 8 * c;
        const int src = (e % 512) / 8, jsel = e / 512;
        u32x4 vh, vl;
#pragma unroll
        for (int wd = 0; wd < 4; wd++) {
          uint32_t h = (uint32_t)__shfl((int)ph[0][wd], src);
          uint32_t l = (uint32_t)__shfl((int)pl[0][wd], src);
#pragma unroll
          for (int j = 1; j < NQL; j++) {
            const uint32_t hj = (uint32_t)__shfl((int)ph[j][wd], src);
            const uint32_t lj = (uint32_t)__shfl((int)pl[j][wd], src);
            h = jsel == j ? hj : h;
            l = jsel == j ? lj : l;
          }
          if (hq >= ratio) h = l = 0u;
          vh[wd] = h;
          vl[wd] = l;
        }
        if constexpr (QC) {
          qb[c] = __builtin_bit_cast(half8_t, n < 8 ? vh : vl);
        } else {
          qb[c] = __builtin_bit_cast(half8_t, vh);
          ql[c] = __builtin_bit_cast(half8_t, vl);
        }
      }
    } else {
      // ---- q' = FWHT(s*q)/sqrt(pd) for this wave's `ratio` heads, on an LDS
      // scratch in slot0.  When it fits, the scratch is this wave's own region
      // of slot0: only this wave touches it and LDS operations of one wave
      // complete in order, so no workgroup barrier is needed.  Otherwise the
      // waves' scratches span slot0 and the workgroup synchronises.
      const bool qlocal = ratio * PD * 4 <= WB;  // uniform
      auto qsync = [&]() {
        if (qlocal) {
          __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
          __builtin_amdgcn_wave_barrier();
        } else {
          __syncthreads();
        }
      };
      float* const qs =
          reinterpret_cast<float*>(slot0 + (qlocal ? wofs : (size_t)w * ratio * PD * 4));
      for (int i = lane; i < ratio * PD; i += 64) {
        const int r = i / PD, d = i - r * PD;
        float x = (float)p.q[b * p.q_sb + (int64_t)(kvh * ratio + r) * p.q_sh + d];
        if (p.signs) x = x * p.signs[d];
        qs[i] = x;
      }
      qsync();
      if (p.signs) {
        for (int h = 1; h < PD; h <<= 1) {
          for (int i = lane; i < ratio * PD / 2; i += 64) {
            const int r = i / (PD / 2), j = i - r * (PD / 2);
            const int lo = r * PD + (j / h) * 2 * h + (j % h);
            const float a = qs[lo], c = qs[lo + h];
            qs[lo] = a + c;
            qs[lo + h] = a - c;
          }
          qsync();
        }
      }
      // q' (pre-scaled to log2 units) split into fp16 high and low parts
      // (q' = hi + lo to ~22 bits), so the scores keep fp32-level accuracy
      // even for heavy-tailed keys.
      {
#pragma unroll
        for (int c = 0; c < KD; c++) {
#pragma unroll
          for (int e = 0; e < 8; e++) {
            const int d = q4 * (PD / 4) + 8 * c + ord[e];
            const float x = (hq < ratio) ? qs[hq * PD + d] * qsc : 0.0f;
            const _Float16 hi = (_Float16)x;
            const _Float16 lo = (_Float16)(x - (float)hi);
            if constexpr (QC) {
              qb[c][e] = n < 8 ? hi : lo;
            } else {
              qb[c][e] = hi;
              ql[c][e] = lo;
            }
          }
        }
      }
      // the scratch is overwritten by the copies into slot0 below
      if (qlocal) {
#if defined(__HIP_DEVICE_COMPILE__)
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#endif
      } else {
        __syncthreads();
      }
    }

    for (int wstep = step0;;) {
      const int wend = min(wstep + 31, step1);
      if (wstep + 1 <= wend && !staged1) stage(wstep + 1, sB);
      staged1 = false;
      for (int k = wstep; k <= wend; k += NSLOT) {
        run(k, sA, wend);
        if (k + NSLOT <= wend) stage(k + NSLOT, sA);
        if (k + 1 > wend) break;
        run(k + 1, sB, wend);
        if (k + 1 + NSLOT <= wend) stage(k + 1 + NSLOT, sB);
      }
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // drain before the next window's page ids
      wstep += 32;
      if (wstep > step1) break;
      open_window(wstep);
      stage(wstep, sA);
      stageK(wstep, kr);
    }
  }

  // ---- two splits per workgroup: the second group hands its state to the
  // first through LDS (the staging slots are drained), the first merges it
  // and writes one partial for the pair; the second split's row is marked
  // empty.  Any partition of the tokens merges to the same attention.
  if constexpr (SPW == 2) {
    constexpr int NF = 4 * NO + 2;  // floats of state per lane
    float* const xs = reinterpret_cast<float*>(slot0) + (size_t)hw * 64 * NF;
    __syncthreads();  // every wave is past its last LDS read
    if (sub == 1) {
#pragma unroll
      for (int i = 0; i < NO; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) xs[(4 * i + r) * 64 + lane] = st.O[i][r];
      xs[4 * NO * 64 + lane] = st.mb;
      xs[(4 * NO + 1) * 64 + lane] = st.lsum;
    }
    __syncthreads();
    if (sub == 0) {
      const float mb1 = xs[4 * NO * 64 + lane];
      const float l1 = xs[(4 * NO + 1) * 64 + lane];
      const float mm = fmaxf(st.mb, mb1);
      const float a0 = st.mb == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(st.mb - mm);
      const float a1 = mb1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mb1 - mm);
#pragma unroll
      for (int i = 0; i < NO; i++)
#pragma unroll
        for (int r = 0; r < 4; r++)
          st.O[i][r] = a0 * st.O[i][r] + a1 * xs[(4 * i + r) * 64 + lane];
      st.lsum = a0 * st.lsum + a1 * l1;
      st.mb = mm;
    }
  }

  // ---- finish: O[i][r] = o[h = n][dim (4*q4 + r)*NO + i]
  float lt = st.lsum;
  if constexpr (PACK == 2) lt = lt + __int_as_float(__builtin_amdgcn_mov_dpp(
                                         __float_as_int(lt), 0x128, 0xf, 0xf, false));
  lt = xor32_sum(xor16_sum(lt));
  if (SPW == 2 && sub == 1) {
    if (n < ratio && q4 == 0 && s < p.S)
      p.plse[((int64_t)b * p.S + s) * p.Hq + kvh * ratio + n] = -INFINITY;
  } else if (n < ratio && s < p.S) {
    // o = pv_scale * O / lsum' (p' = p * pv_scale in both O and lsum')
    const float inv = lt > 0.f ? p.pv_scale / lt : 0.0f;
    const int64_t orow = ((int64_t)b * p.S + s) * p.Hq + kvh * ratio + n;
    float* out = p.po + orow * PD + q4 * (PD / 4);
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
      p.plse[orow] = lt > 0.f ? (st.mb + __log2f(lt)) * 0.69314718055994531f : -INFINITY;
  }
}
// LSE merge of the splits of one (sequence, q head), inverse rotation, fp16
// store.  256 threads: split weights are computed once into LDS, then
// 256/(PD/4) split groups each sum a strided subset of the splits for one
// float4 column, a tree in LDS adds the groups, and wave 0 runs the inverse
// FWHT across its 64 lanes.
template <int PD>
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ po,
                                                      const float* __restrict__ plse, int S_rows, int step,
                                                      int Hq, const float* __restrict__ signs,
                                                      float inv_sqrt_pd, _Float16* __restrict__ o) {
  constexpr int C = PD / 4;        // float4 columns
  constexpr int NG = 256 / C;      // split groups
  constexpr int V = PD / 64;       // dims per lane in the FWHT
  extern __shared__ float sm[];    // [S] weights or group maxima, then [NG][PD] sums + [NG] denominators
  __shared__ float red[8];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int b = blockIdx.x / Hq, h = blockIdx.x % Hq;
  // split j of sequence b is row row0 + j * rs (rows of the splits a partials
  // workgroup merged into its first row are skipped with step > 1)
  const int64_t row0 = (int64_t)b * S_rows * Hq + h;
  const int64_t rs = (int64_t)step * Hq;
  const int S = (S_rows + step - 1) / step;

  const int col = tid % C, grp = tid / C;
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
  float den = 0.f;
  constexpr int R = 16;  // splits per thread held in registers on the fast path
  if (S <= NG * R) {
    // one round trip: the LSEs and partial rows of this thread's splits
    // (grp, grp + NG, ...) are all loaded before any is used
    float l[R];
    float4_t v[R];
#pragma unroll
    for (int j = 0; j < R; j++) {
      const int s = grp + NG * j;
      l[j] = -INFINITY;
      v[j] = float4_t{0.f, 0.f, 0.f, 0.f};
      if (s < S) {
        l[j] = plse[row0 + (int64_t)s * rs];
        v[j] = *reinterpret_cast<const float4_t*>(po + (row0 + (int64_t)s * rs) * PD + col * 4);
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < R; j++) mx = fmaxf(mx, l[j]);
    // the groups hold disjoint splits: max over the groups through LDS
    if (col == 0) sm[grp] = mx;
    __syncthreads();
    mx = -INFINITY;
    for (int g = 0; g < NG; g++) mx = fmaxf(mx, sm[g]);
#pragma unroll
    for (int j = 0; j < R; j++) {
      const float wgt = (l[j] > -INFINITY && mx > -INFINITY) ? __expf(l[j] - mx) : 0.0f;
      den += wgt;
      acc += wgt != 0.0f ? wgt * v[j] : float4_t{0.f, 0.f, 0.f, 0.f};  // skipped rows may hold any bits
    }
    __syncthreads();  // the group maxima are read; LDS is reused below
  } else {
    float mx = -INFINITY;
    for (int s = tid; s < S; s += 256) mx = fmaxf(mx, plse[row0 + (int64_t)s * rs]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if (lane == 0) red[wv] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int s = tid; s < S; s += 256) {
      const float l = plse[row0 + (int64_t)s * rs];
      sm[s] = (l > -INFINITY && mx > -INFINITY) ? __expf(l - mx) : 0.0f;
    }
    __syncthreads();  // weights visible
    for (int s = grp; s < S; s += NG) {
      const float wgt = sm[s];
      den += wgt;
      if (wgt != 0.0f)
        acc += wgt * *reinterpret_cast<const float4_t*>(po + (row0 + (int64_t)s * rs) * PD + col * 4);
    }
    __syncthreads();  // weights no longer needed; reuse LDS for group sums
  }
  // den: each group summed its own splits (identical in all C lanes of the group)
  float* part = sm;
  *reinterpret_cast<float4_t*>(part + grp * PD + col * 4) = acc;
  if (col == 0) part[NG * PD + grp] = den;
  __syncthreads();
  if (wv == 0) {
    den = 0.f;
    for (int g = 0; g < NG; g++) den += part[NG * PD + g];
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

// Splits one partials workgroup serves: two (one 16-wave workgroup per CU)
// when q' is formed in registers (ratio * pd <= 1024) and pd >= 128, which
// keeps the workgroup free of barriers; head size 64 keeps three 8-wave
// workgroups per CU instead.  The pair's state is merged into the first
// split's row and the second row is marked empty.
int splits_per_workgroup(int ratio, int pd) { return (ratio * pd <= 1024 && pd >= 128) ? 2 : 1; }

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
  if ((uintptr_t)q % 16 || q_stride_b % 8 || q_stride_h % 8 || q_stride_h < padded_dim) {
    set_error("decode: q must be 16-byte aligned with strides multiple of 8 elements and "
              "q_stride_h >= padded_dim");
    return kEinval;
  }
  const int pd = padded_dim;
  const int ratio = num_qo_heads / num_kv_heads;
  // heads per workgroup: a divisor of num_kv_heads whose staged rows fit the
  // static LDS buffers (G*ebs <= ROW) and whose q scratch fits one buffer
  const int ebs_expected = pd == 64 ? 48 : (pd == 128 ? 80 : 144);
  if (ebs != ebs_expected) {
    set_error("decode: ebs %d does not match padded_dim %d (expected %d)", ebs, pd, ebs_expected);
    return kEinval;
  }
  // heads (waves) per workgroup: a divisor of num_kv_heads up to MAXG whose
  // q scratch fits the first slot
  const int maxg = pd == 256 ? 4 : 8;
  const size_t slot_bytes = (size_t)maxg * 2 * kTile * ebs_expected;
  int G = 0;
  for (int g = maxg; g >= 1; g--)
    if (num_kv_heads % g == 0 && (size_t)g * ratio * pd * sizeof(float) <= slot_bytes) {
      G = g;
      break;
    }
  if (G == 0) {
    set_error("decode: no workgroup shape for %d kv heads, ratio %d", num_kv_heads, ratio);
    return kEinval;
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
  // measured on MI355X at configs[2]: the first (older) group of a
  // two-split workgroup sustains ~3/4 of the pair's work in the same time
  p.share0 = 184;
  const int spw = splits_per_workgroup(ratio, pd);
  const int64_t blocks = (int64_t)batch * ((num_splits + spw - 1) / spw) * p.HG;
  if (blocks > 0x7fffffffLL) {
    set_error("decode: grid too large");
    return kEinval;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((unsigned)blocks), block(64 * G * spw);
  // scores of two tiles share one register set when ratio <= 8 (head size
  // 256 keeps one tile per set: two would exceed the register file)
  const bool pack2 = ratio <= 8 && pd <= 128;
  // q hi/lo parts share one B operand when the GQA ratio leaves 8 columns free
  const bool qc = ratio <= 8;
  // only the (head size, packing, split pairing) combinations these rules
  // reach are instantiated
#define TQ_LAUNCH(PDV, PK, QCV, SPWV) \
  hipLaunchKernelGGL((decode_partials_kernel<PDV, PK, QCV, SPWV>), grid, block, 0, st, p)
  switch (pd) {
    case 64:  // spw == 1
      if (pack2) TQ_LAUNCH(64, 2, true, 1);
      else TQ_LAUNCH(64, 1, false, 1);
      break;
    case 128:  // pack2 exactly when spw == 2
      if (pack2) TQ_LAUNCH(128, 2, true, 2);
      else TQ_LAUNCH(128, 1, false, 1);
      break;
    default:  // spw == 2 only when ratio <= 4
      if (spw == 2) TQ_LAUNCH(256, 1, true, 2);
      else if (qc) TQ_LAUNCH(256, 1, true, 1);
      else TQ_LAUNCH(256, 1, false, 1);
  }
#undef TQ_LAUNCH
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("decode: launch failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}

namespace tq {
static int combine_splits(const float* partition_o, const float* partition_lse, int step,
                                 int32_t batch, int32_t num_splits, int32_t num_qo_heads,
                                 int32_t padded_dim, const float* signs, void* o,
                                 tq_stream_t stream) {
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
  // weights of the splits, or the group sums [NG][pd] plus the group denominators
  const size_t lds = sizeof(float) * (size_t)(num_splits > 1024 + 64 ? num_splits : 1024 + 64);
  if (lds > 60 * 1024) {
    set_error("combine: num_splits %d too large", num_splits);
    return kEinval;
  }
  dim3 grid((unsigned)blocks), block(256);
  switch (pd) {
    case 64:
      hipLaunchKernelGGL(combine_kernel<64>, grid, block, lds, st, partition_o, partition_lse,
                         num_splits, step, num_qo_heads, signs, isq, out);
      break;
    case 128:
      hipLaunchKernelGGL(combine_kernel<128>, grid, block, lds, st, partition_o, partition_lse,
                         num_splits, step, num_qo_heads, signs, isq, out);
      break;
    default:
      hipLaunchKernelGGL(combine_kernel<256>, grid, block, lds, st, partition_o, partition_lse,
                         num_splits, step, num_qo_heads, signs, isq, out);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("combine: launch failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}

}  // namespace tq

extern "C" int tq_combine_splits(const float* partition_o, const float* partition_lse,
                                 int32_t batch, int32_t num_splits, int32_t num_qo_heads,
                                 int32_t padded_dim, const float* signs, void* o,
                                 tq_stream_t stream) {
  return tq::combine_splits(partition_o, partition_lse, 1, batch, num_splits, num_qo_heads,
                            padded_dim, signs, o, stream);
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
  // rows the partials kernel merged away are skipped
  return tq::combine_splits(partition_o, partition_lse,
                            tq::splits_per_workgroup(num_qo_heads / num_kv_heads, padded_dim),
                            batch, num_splits, num_qo_heads, padded_dim, signs, o, stream);
}
