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
//  * 4-bit -> fp16 dequant through a 256-entry LDS table (code byte -> the
//    fp16 values of its two nibbles), built once per workgroup from the odd
//    codebook (c[15-i] = -c[i]) with bit tricks and v_perm_b32 byte tables,
//    and held in 32 interleaved copies so that the lookups of a wave never
//    conflict on an LDS bank.
//  * The cache rows stream into LDS with direct-to-LDS 16-byte copies
//    (buffer_load ... lds), one workgroup-wide contiguous copy per 1 KB of
//    rows, through a ring of tile slots, so each cache line is requested once.
//  * The K norm scales the score; the V norm and 1/sqrt(pd) fold into the
//    probability, so dequantized operands are (scaled) codebook values.
//  * Accuracy: q' and the probabilities enter the MFMAs as fp16 hi + lo
//    pairs and the codebook tables are pre-scaled to fp16-friendly values,
//    keeping the result within ~1e-3 of fp32 math even for heavy-tailed keys.
//  * Online softmax in the exp2 domain with a lazy rescale (the running max
//    only moves when a tile exceeds it by more than 2^3), bounding p <= 8.
#include <math.h>

#include <mutex>
#include <type_traits>

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
  // > 0: the grid is two workgroups per CU and splits are served in pairs
  // (2j, 2j + 1) by blocks u and u + grid/2, which the dispatcher places on one
  // CU; the first-dispatched block takes the first pair_pct percent (rounded
  // up to 16 tokens) of the pair's tokens (it progresses faster while both
  // are resident)
  int pair_pct;
  // > 0: balanced plan.  The grid serves `units` work units per head group
  // (pairs of blocks when pair_pct > 0), and each unit covers U consecutive
  // tokens of one sequence, U being the smallest multiple of kPlanAlign with
  // sum_b ceil(seq_len_b / U) <= units, computed by every workgroup from
  // seq_lens on the device.  Partial rows are numbered by unit (two per unit
  // in pairs), so sequence b owns the contiguous rows split_out[b] ..
  // split_out[b + 1]; block 0 stores that table and U (split_out[B + 1]).
  int units;
  int32_t* split_out;
  float qk_scale;     // sm_scale * log2(e) / (sqrt(pd) * kCbScale)
  float inv_sqrt_pd;  // 1/sqrt(pd)
  float pv_scale;     // 1/(sqrt(pd) * kCbScale)
};

// Float max without NaN quieting: in IEEE mode fmaxf first canonicalizes
// both operands (two more VALU instructions); the scores are never
// signaling NaNs, so the plain instruction gives the same result.
__device__ __forceinline__ float vmax(float a, float b) {
#if defined(__HIP_DEVICE_COMPILE__)
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
#else
  return fmaxf(a, b);
#endif
}
__device__ __forceinline__ float vmax3(float a, float b, float c) {
#if defined(__HIP_DEVICE_COMPILE__)
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
#else
  return fmaxf(fmaxf(a, b), c);
#endif
}
// max(x, x of lane l ror 8 within its row): one DPP max (the s_nop covers
// the wait states of a DPP read after a VALU write of its source)
__device__ __forceinline__ float max_ror8(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  float r;
  asm("s_nop 1\n\tv_max_f32_dpp %0, %1, %1 row_ror:8 row_mask:0xf bank_mask:0xf"
      : "=v"(r)
      : "v"(x));
  return r;
#else
  return fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xf, 0xf,
                                                          false)));
#endif
}
// score * K norm, the norm an fp16 value in the low half of nr: one
// v_fma_mix (fp16 operand, fp32 math; +0 addend, which only differs from
// the product for a -0 score, and that feeds the same max and exp2)
__device__ __forceinline__ float mul_lo_half(float sc, uint32_t nr) {
#if defined(__HIP_DEVICE_COMPILE__)
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(nr), "v"(sc));
  return r;
#else
  return sc * (float)__builtin_bit_cast(_Float16, (uint16_t)(nr & 0xffffu));
#endif
}
__device__ __forceinline__ float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
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
// value of lane l ^ m (m = 1, 2, 4, 8 without LDS: DPP quad_perm, row
// half-mirror then quad reversal, row rotate by 8)
__device__ __forceinline__ float xor_lane(float x, int m) {
  const int v = __float_as_int(x);
  switch (m) {
    case 1: return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0xB1, 0xf, 0xf, false));
    case 2: return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0x4E, 0xf, 0xf, false));
    case 4: {
      const int t = __builtin_amdgcn_mov_dpp(v, 0x141, 0xf, 0xf, false);
      return __int_as_float(__builtin_amdgcn_mov_dpp(t, 0x1B, 0xf, 0xf, false));
    }
    case 8: return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0x128, 0xf, 0xf, false));
    default: return __shfl_xor(x, m);
  }
}
// LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* ptr) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)ptr;
}
// fp16 value held in the low / high half of a dword
__device__ __forceinline__ float lo_half(uint32_t v) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu));
}
__device__ __forceinline__ float hi_half(uint32_t v) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
}

// ---- balanced split plan ------------------------------------------------
constexpr int kPlanAlign = 2 * kTile;   // unit sizes are whole steps
constexpr int kPlanMaxBatch = 1024;     // sequences a balanced plan takes

__device__ __forceinline__ int xor_lane_i(int v, int m) {
  return __float_as_int(xor_lane(__int_as_float(v), m));
}
__device__ __forceinline__ int permlane_xor16_i(int v) {
  const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
  return (int)r[0] == v ? (int)r[1] : (int)r[0];
}
// sum / max over the 64 lanes (every lane gets the result): DPP lane xors
// inside rows of 16, then the 16- and 32-lane swaps
__device__ __forceinline__ int wave_sum_i(int v) {
  v += xor_lane_i(v, 1);
  v += xor_lane_i(v, 2);
  v += xor_lane_i(v, 4);
  v += xor_lane_i(v, 8);
  auto r = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
  v = (int)(r[0] + r[1]);
  r = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
  return (int)(r[0] + r[1]);
}
__device__ __forceinline__ int wave_max_i(int v) {
  v = max(v, xor_lane_i(v, 1));
  v = max(v, xor_lane_i(v, 2));
  v = max(v, xor_lane_i(v, 4));
  v = max(v, xor_lane_i(v, 8));
  auto r = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
  v = max((int)r[0], (int)r[1]);
  r = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
  return max((int)r[0], (int)r[1]);
}
// ceil(a / d) for a >= 0, d > 0, a + d < 2^31: below 2^24 a float estimate
// (off by at most one there) corrected both ways in integers; from 2^24 on
// (a sequence of 16M tokens or more) an integer division
__device__ __forceinline__ int ceil_div_est(int a, int d, float rd) {
  const int x = a + d - 1;
  if (x >= (1 << 24)) return x / d;
  int f = (int)((float)x * rd);
  f -= (f * d > x) ? 1 : 0;
  f += ((f + 1) * d <= x) ? 1 : 0;
  return f;
}

// The unit of a balanced plan a workgroup serves: sequence b (-1: none, the
// grid has more units than the plan uses), unit j of that sequence, its
// length L, page-table start ip, the sequence's first unit Pb and the unit
// size U in tokens.
struct PlanSlot {
  int b, j, L, Pb, U, ip;
};

// The plan from the sequence lengths, which `lens(i, lane)` returns for
// sequence 64 i + lane (0 past the batch) and `starts` likewise for the
// page-table starts; nreg = ceil(B / 64).  Every lane of a wave runs it and
// every field of the result is wave-uniform.  writer: this wave also stores
// the row table (rows = rowmul * units) and U.
template <typename LensFn, typename StartsFn>
__device__ __forceinline__ PlanSlot plan_slot(LensFn lens, StartsFn starts, int B, int nreg,
                                              int units, int u, int rowmul, int32_t* split_out,
                                              bool writer) {
  const int lane = threadIdx.x & 63;
  int tsum = 0, mx = 0, nz = 0;
  for (int i = 0; i < nreg; i++) {
    const int l = lens(i);
    tsum += l;
    mx = max(mx, l);
    nz += l > 0 ? 1 : 0;
  }
  tsum = __builtin_amdgcn_readfirstlane(wave_sum_i(tsum));
  mx = __builtin_amdgcn_readfirstlane(wave_max_i(mx));
  nz = __builtin_amdgcn_readfirstlane(wave_sum_i(nz));
  constexpr int A = kPlanAlign;
  if (nreg == 1 && nz == B && (int64_t)mx * B == (int64_t)tsum) {
    // every sequence has the same length L: sum_b ceil(L / U) <= units is
    // ceil(L / U) <= k = floor(units / B), i.e. U >= L / k, so the plan has
    // a closed form (no search, no scan before the first page-id loads)
    const int k = units / B;
    const int U = ((mx + k - 1) / k + A - 1) / A * A;
    const int c = (mx + U - 1) / U;  // units per sequence
    PlanSlot r = {-1, 0, 0, 0, U, 0};
    if (u < B * c) {
      r.b = u / c;
      r.j = u - r.b * c;
      r.Pb = r.b * c;
      r.L = mx;
      r.ip = __builtin_amdgcn_readlane(starts(0), r.b);
    }
    if (writer) {
      if (lane < B) split_out[lane] = lane * c * rowmul;
      if (lane == 0) {
        split_out[B] = B * c * rowmul;
        split_out[B + 1] = U;
      }
    }
    r.b = __builtin_amdgcn_readfirstlane(r.b);
    r.j = __builtin_amdgcn_readfirstlane(r.j);
    r.L = __builtin_amdgcn_readfirstlane(r.L);
    r.Pb = __builtin_amdgcn_readfirstlane(r.Pb);
    r.ip = __builtin_amdgcn_readfirstlane(r.ip);
    return r;
  }
  auto units_for = [&](int k) -> int {
    const int d = k * A;
    const float rd = 1.0f / (float)d;
    int c = 0;
    for (int i = 0; i < nreg; i++) c += ceil_div_est(lens(i), d, rd);
    return __builtin_amdgcn_readfirstlane(wave_sum_i(c));
  };
  // smallest feasible k in (lo, hi]: every k below tsum / (units * A) needs
  // more than `units` units; k = ceil(max_len / A) needs nz <= units, and so
  // does any k >= tsum / ((units - nz) * A) (at most one partial unit per
  // sequence)
  int hi = max(1, (mx + A - 1) / A);
  if (units > nz) hi = min(hi, max(1, (tsum + (units - nz) * A - 1) / ((units - nz) * A)));
  int lo = (tsum + units * A - 1) / (units * A) - 1;
  lo = max(0, min(lo, hi - 1));
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (units_for(mid) <= units) hi = mid; else lo = mid;
  }
  const int U = hi * A;
  const float rdU = 1.0f / (float)U;
  PlanSlot r = {-1, 0, 0, 0, U, 0};
  int carry = 0;
  for (int i = 0; i < nreg; i++) {
    const int l = lens(i);
    const int c = ceil_div_est(l, U, rdU);
    int incl = c;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(incl, off);
      if (lane >= off) incl += y;
    }
    incl += carry;
    const int excl = incl - c;
    const int bb = 64 * i + lane;
    if (writer && bb < B) split_out[bb] = excl * rowmul;
    const uint64_t hit = __ballot(c > 0 && excl <= u && u < incl);
    if (hit) {
      const int l0 = __builtin_ctzll(hit);
      r.b = 64 * i + l0;
      r.Pb = __builtin_amdgcn_readlane(excl, l0);
      r.j = u - r.Pb;
      r.L = __builtin_amdgcn_readlane(l, l0);
      r.ip = __builtin_amdgcn_readlane(starts(i), l0);
    }
    carry = __builtin_amdgcn_readlane(incl, 63);
  }
  if (writer && lane == 0) {
    split_out[B] = carry * rowmul;
    split_out[B + 1] = U;
  }
  // every field is wave-uniform; saying so keeps the addresses built from
  // them in scalar registers (buffer descriptors need them there)
  r.b = __builtin_amdgcn_readfirstlane(r.b);
  r.j = __builtin_amdgcn_readfirstlane(r.j);
  r.L = __builtin_amdgcn_readfirstlane(r.L);
  r.Pb = __builtin_amdgcn_readfirstlane(r.Pb);
  r.U = __builtin_amdgcn_readfirstlane(r.U);
  r.ip = __builtin_amdgcn_readfirstlane(r.ip);
  return r;
}

// Per-lane register geometry of the decode math for padded head size PD.
template <int PD>
struct DecodeGeom {
  static constexpr int KD = PD / 32;  // K dwords per lane per tile = QK MFMA pairs
  static constexpr int VB = PD / 32;  // V bytes per lane per token
  static constexpr int NO = PD / 16;  // PV MFMAs = output dim slots per lane
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

// The dequant table: 256 entries (entry e = fp16 values of the high and low
// nibble of code byte e), each held in LC copies side by side at the
// start of LDS (entry e, copy c at dword e * LC + c).  Lane l reads copy
// l mod LC; with 32 copies the 32 lanes the LDS serves per cycle always hit
// 32 distinct banks, whatever the codes, so a lookup never has a bank
// conflict.
//
// Copies of the table for a workgroup of G kv heads of head size PD.  32
// copies make every lookup conflict-free; 16 halve the table (lanes l and
// l + 16 may share a bank) so that more workgroups fit a CU.  Measured on
// configs[3] (B = 64 ragged): head size 256 with 2 kv heads 174 -> 158 us and
// head size 128 with 4 kv heads 170 -> 146 us with 16 copies; head size 64
// with 4 kv heads 97 -> 109 us (re-measured with the current kernel: head
// size 256 160.5 -> 150 us with 16 copies, head size 64 90 -> 109 us), so
// head size 64 keeps 32, as does the 8-head group of
// configs[2] (its two workgroups per CU are already bound by the ring); 8
// copies at head size 256, 2 kv heads, compiled for three waves per SIMD (168
// VGPRs, five workgroups per CU instead of four) measured 166.5 against
// 147 us: the lookups' bank conflicts cost more than the occupancy gains.
__host__ __device__ constexpr int lut_copies(int pd, int g) {
  return pd == 64 || (pd == 128 && g == 8) ? 32 : 16;
}
__host__ __device__ constexpr int lut_shift(int copies) { return copies == 32 ? 7 : 6; }

// LDS byte address of the table entry `byte k of w` for this lane (lanec =
// 4 * (lane mod copies), entries 2^SH bytes apart).
template <int SH>
__device__ __forceinline__ uint32_t lut_addr(uint32_t w, int k, uint32_t lanec) {
  return (((w >> (8 * k)) & 0xffu) << SH) | lanec;
}

// Table addresses from code bytes spread into 16-bit halves: lut_spread
// puts bytes 2i and 2i + 1 of w into the low and high halves of one register
// (v_perm), and lut_mad forms half * 2^SH + lanec in one v_mad_u32_u16
// (op_sel picks the half), so a pair of lookups costs three instructions
// instead of four.  lut_mad<SH, HI>(lut_spread(w, i), lanec) equals
// lut_addr<SH>(w, 2 * i + HI, lanec).
__device__ __forceinline__ uint32_t lut_spread(uint32_t w, int i) {
  return __builtin_amdgcn_perm(0u, w, i ? 0x0c030c02u : 0x0c010c00u);
}
template <int SH, int HI>
__device__ __forceinline__ uint32_t lut_mad(uint32_t h, uint32_t lanec) {
  uint32_t a;
#if defined(__HIP_DEVICE_COMPILE__)
  if constexpr (HI)
    asm("v_mad_u32_u16 %0, %1, %2, %3 op_sel:[1,0,0,0]" : "=v"(a) : "v"(h), "s"(1u << SH), "v"(lanec));
  else
    asm("v_mad_u32_u16 %0, %1, %2, %3" : "=v"(a) : "v"(h), "s"(1u << SH), "v"(lanec));
#else
  a = ((HI ? h >> 16 : h & 0xffffu) << SH) + lanec;
#endif
  return a;
}

// Eight table reads in place (each address register receives its entry):
// plain LDS loads of the table.  The table is a different field of the
// workgroup's LDS than the ring the direct-to-LDS copies write, so the
// compiler neither waits for the copies in flight before these loads nor
// orders them against the copies, and it interleaves them with the address
// arithmetic and the MFMAs (partial lgkmcnt waits).
__device__ __forceinline__ void lut_read8(uint32_t* a, const uint32_t* lut) {
#pragma unroll
  for (int i = 0; i < 8; i++)
    a[i] = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(lut) + a[i]);
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
template <int PD, bool QC, int SH, bool MERGE = true>
__device__ __forceinline__ float4_t tile_scores(const uint32_t* kw, const half8_t* qb,
                                                const half8_t* ql, uint32_t lanec,
                                                const uint32_t* lut) {
  constexpr int KD = PD / 32;
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < KD; c += 2) {
    // two K blocks per batch of 8 table reads and one wait
    uint32_t x[8];
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const uint32_t h = lut_spread(kw[c + u], i);
        x[4 * u + 2 * i] = lut_mad<SH, 0>(h, lanec);
        x[4 * u + 2 * i + 1] = lut_mad<SH, 1>(h, lanec);
      }
    lut_read8(x, lut);
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const half8_t kv8 = as_half8(x[4 * u], x[4 * u + 1], x[4 * u + 2], x[4 * u + 3]);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv8, qb[c + u], acc, 0, 0, 0);
      if constexpr (!QC)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv8, ql[c + u], acc, 0, 0, 0);
    }
  }
  if constexpr (QC && MERGE) {
#pragma unroll
    for (int r = 0; r < 4; r++) acc[r] = acc[r] + ror8(acc[r]);
  }
  return acc;
}

// PACK 2 scores of two tiles from their unmerged QC accumulators: lanes n < 8
// of each row get tile 0's hi + lo sums (lane n + 8 holds the lo part), lanes
// n >= 8 tile 1's (lane n - 8 holds the hi part): two DPP adds per value
// whose bank masks write one half of each row each.  The leading s_nops
// cover the wait states between the MFMAs that wrote a0 / a1 and their DPP
// read (inline assembly, so the compiler does not count them).
__device__ __forceinline__ float4_t pack_merge(float4_t a0, float4_t a1) {
  float4_t d;
#if defined(__HIP_DEVICE_COMPILE__)
  float d0, d1, d2, d3;
  asm volatile("s_nop 7\n\ts_nop 7\n\t"
               "v_add_f32_dpp %0, %4, %4 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
               "v_add_f32_dpp %0, %8, %8 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
               "v_add_f32_dpp %1, %5, %5 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
               "v_add_f32_dpp %1, %9, %9 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
               "v_add_f32_dpp %2, %6, %6 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
               "v_add_f32_dpp %2, %10, %10 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
               "v_add_f32_dpp %3, %7, %7 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
               "v_add_f32_dpp %3, %11, %11 row_ror:8 row_mask:0xf bank_mask:0xc"
               : "=&v"(d0), "=&v"(d1), "=&v"(d2), "=&v"(d3)
               : "v"(a0[0]), "v"(a0[1]), "v"(a0[2]), "v"(a0[3]), "v"(a1[0]), "v"(a1[1]),
                 "v"(a1[2]), "v"(a1[3]));
  d = float4_t{d0, d1, d2, d3};
#else
  d = a0 + a1;
#endif
  return d;
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
template <int PD, int SH>
__device__ __forceinline__ void step_pv(const uint32_t (*v0)[(PD / 32) >= 4 ? PD / 128 : 1],
                                        const uint32_t (*v1)[(PD / 32) >= 4 ? PD / 128 : 1],
                                        half8_t p, SoftmaxState<PD>& st, uint32_t lanec,
                                        const uint32_t* lut) {
  constexpr int VB = PD / 32;
  constexpr int VW = VB >= 4 ? VB / 4 : 1;
  // ix[T][pair][nibble][w]: pair 0 = tokens 0, 1; pair 1 = tokens 2, 3;
  // nibble 0 = low nibbles, 1 = high nibbles
  uint32_t ix[2][2][2][VW];
  uint32_t hs[2][2][2];  // two bytes of each index word, spread into 16-bit halves
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
    uint32_t x[8];
    if (j % 2 == 0) {
      // bytes j and j + 1 of every index word, spread into 16-bit halves
#pragma unroll
      for (int nb = 0; nb < 2; nb++)
#pragma unroll
        for (int T = 0; T < 2; T++)
#pragma unroll
          for (int pr = 0; pr < 2; pr++) hs[nb][T][pr] = lut_spread(ix[T][pr][nb][w], j / 2);
    }
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
#pragma unroll
      for (int T = 0; T < 2; T++)
#pragma unroll
        for (int pr = 0; pr < 2; pr++)
          x[4 * nb + 2 * T + pr] = j % 2 ? lut_mad<SH, 1>(hs[nb][T][pr], lanec)
                                         : lut_mad<SH, 0>(hs[nb][T][pr], lanec);
    lut_read8(x, lut);
    const half8_t lo8 = as_half8(x[0], x[1], x[2], x[3]);
    const half8_t hi8 = as_half8(x[4], x[5], x[6], x[7]);
    st.O[2 * k + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(lo8, p, st.O[2 * k + 1], 0, 0, 0);
    st.O[2 * k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(hi8, p, st.O[2 * k], 0, 0, 0);
  }
}

// This wave's share of one step (two tiles), read from LDS into registers.
template <int PD>
struct StepData {
  static constexpr int KD = PD / 32;
  static constexpr int VW = (PD / 32) >= 4 ? PD / 128 : 1;
  uint32_t k[2][KD];     // K codes of tiles 0 and 1: token l%16, dims of quarter q4
  uint32_t v[2][4][VW];  // V codes of tiles 0 and 1, tokens 4*q4 + j, bytes of slot l%16
  uint32_t nkv[2];       // norms (K low half, V high half) of the packed tokens, per group
};

// s_waitcnt immediate that waits until at most n vector-memory operations
// are outstanding (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] |
// vmcnt[5:4] in [15:14]; expcnt and lgkmcnt left at their maximum).
__host__ __device__ constexpr int vmcnt_imm(int n) {
  return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14);
}

// LDS staging geometry of one workgroup (G kv heads of one split).  A tile
// slot holds the 16 tokens of one tile for the workgroup's heads: the K slab
// region, then the V slab region, each SLAB bytes.  A region holds the 16
// token rows of CPT 16-byte chunks (G entries of EBS bytes) as copied from
// the cache, at a row stride of RCH chunks: CPT rounded up to an odd count,
// so that the 16 rows of one chunk column, and rows t and t + 4, fall into
// distinct bank groups (the pad chunk of a row receives a second copy of
// the row's last chunk).  NI 1 KB copies fill one region (the last may
// spill past the rows into the region's slack).  kRingSlots slots (two by
// default) form the ring.
#ifndef TQ_RING_SLOTS
#define TQ_RING_SLOTS 2
#endif
constexpr int kRingSlots = TQ_RING_SLOTS;  // tile slots in the LDS ring
// Cache policy of the ring copies: nt (non-temporal, bit 1 of the gfx950
// cache-policy field), since every cache line is read exactly once; measured
// 3-4 us faster per launch at configs[2] than the default policy.
[[maybe_unused]] constexpr int kCopyPolicy = 2;

template <int PD, int G>
struct RingGeom {
  static constexpr int EBS = PD == 64 ? 48 : (PD == 128 ? 80 : 144);  // entry bytes
  static constexpr int ECH = EBS / 16;                       // chunks per entry
  static constexpr int CPT = G * ECH;                         // chunks per token row
  static constexpr int RCH = CPT | 1;                         // row stride in chunks
  static constexpr int ROWB = RCH * 16;                       // row stride in bytes
  static constexpr int NI = (kTile * RCH + 63) / 64;          // copies per region
  static constexpr int SLAB = NI * 1024;                      // LDS bytes per region
  static constexpr int TS = 2 * SLAB;                         // LDS bytes per tile slot
  static constexpr int NIT = 2 * NI;                          // copies per tile
  static constexpr int NW_HI = (NIT + G - 1) / G;             // copies per tile, waves < NIT % G
  static constexpr int NW_LO = NIT / G;                       // copies per tile, other waves
  static constexpr int RING = kRingSlots * TS;
  static constexpr int LC = lut_copies(PD, G);               // table copies
  static constexpr int SH = lut_shift(LC);                    // log2 of an entry's bytes
  static constexpr int LUTB = 256 * 4 * LC;                   // table bytes
  static constexpr int LDS = LUTB + RING;                     // table + ring
};

// This wave's K codes, V codes and norms of the step's two tiles, read from
// the ring slots S0 (tile 0) and S1 (tile 1) into registers: inline assembly
// ending in lgkmcnt(0) (the compiler does not see these LDS reads, so it
// adds no wait for the copies in flight; the caller has waited for exactly
// the copies it reads).  oK / oV / oN: per-lane offsets inside a region of
// the K code chunk(s), the V code bytes of token 4*q4 (token 4*q4 + j is j
// rows further), and the entry tail (first norm copy) of token
// 4*q4 + (lane & 3); PACK 2 reads the norms
// of the lane's packed tile only, at oN (which then already includes the
// distance to that tile's slot from the lower of the two slots).
template <int PD, int G, int PACK>
__device__ __forceinline__ void read_step(const uint32_t* ka, uint32_t va, uint32_t vb,
                                          uint32_t na, uint32_t nb, StepData<PD>& d) {
#if defined(__HIP_DEVICE_COMPILE__)
  using RG = RingGeom<PD, G>;
  constexpr int R = RG::ROWB;
  constexpr int SL = RG::SLAB;
  uint32_t n0 = 0, n1 = 0, n2 = 0, n3 = 0;
// V codes of tokens 4*q4 + 0..3 of both tiles: rows R apart
#define TQ_V8(OP)                                \
  OP " %[a0], %[va]\n\t"                         \
  OP " %[a1], %[va] offset:%[r1]\n\t"            \
  OP " %[a2], %[va] offset:%[r2]\n\t"            \
  OP " %[a3], %[va] offset:%[r3]\n\t"            \
  OP " %[c0], %[vb]\n\t"                         \
  OP " %[c1], %[vb] offset:%[r1]\n\t"            \
  OP " %[c2], %[vb] offset:%[r2]\n\t"            \
  OP " %[c3], %[vb] offset:%[r3]\n\t"
#define TQ_VOUT                                                                          \
  [a0] "=&v"(a0), [a1] "=&v"(a1), [a2] "=&v"(a2), [a3] "=&v"(a3), [c0] "=&v"(c0),        \
  [c1] "=&v"(c1), [c2] "=&v"(c2), [c3] "=&v"(c3)
#define TQ_VIN [va] "v"(va), [vb] "v"(vb), [r1] "i"(R), [r2] "i"(2 * R), [r3] "i"(3 * R)
// norms: PACK 2 the lane's packed tile (K at na, V one region further); PACK 1
// both tiles (K t0 at na, K t1 at nb, V t0, V t1 one region further)
#define TQ_N2                                      \
  "ds_read_u16 %[n0], %[na]\n\t"                   \
  "ds_read_u16 %[n1], %[na] offset:%[sl]\n\t"
#define TQ_N1                                      \
  "ds_read_u16 %[n0], %[na]\n\t"                   \
  "ds_read_u16 %[n1], %[nb]\n\t"                   \
  "ds_read_u16 %[n2], %[na] offset:%[sl]\n\t"      \
  "ds_read_u16 %[n3], %[nb] offset:%[sl]\n\t"
  if constexpr (PD == 128 || PD == 64) {
    typedef typename std::conditional<PD == 128, u32x4, u32x2>::type KT;
    KT k0, k1;
    uint32_t a0, a1, a2, a3, c0, c1, c2, c3;
    if constexpr (PD == 128 && PACK == 2) {
      asm volatile("ds_read_b128 %[k0], %[ka0]\n\t"
                   "ds_read_b128 %[k1], %[ka1]\n\t"
                   TQ_V8("ds_read_b32") TQ_N2 "s_waitcnt lgkmcnt(0)"
                   : [k0] "=&v"(k0), [k1] "=&v"(k1), TQ_VOUT, [n0] "=&v"(n0), [n1] "=&v"(n1)
                   : [ka0] "v"(ka[0]), [ka1] "v"(ka[1]), TQ_VIN, [na] "v"(na), [sl] "i"(SL)
                   : "memory");
    } else if constexpr (PD == 128) {
      asm volatile("ds_read_b128 %[k0], %[ka0]\n\t"
                   "ds_read_b128 %[k1], %[ka1]\n\t"
                   TQ_V8("ds_read_b32") TQ_N1 "s_waitcnt lgkmcnt(0)"
                   : [k0] "=&v"(k0), [k1] "=&v"(k1), TQ_VOUT, [n0] "=&v"(n0), [n1] "=&v"(n1),
                     [n2] "=&v"(n2), [n3] "=&v"(n3)
                   : [ka0] "v"(ka[0]), [ka1] "v"(ka[1]), TQ_VIN, [na] "v"(na), [nb] "v"(nb),
                     [sl] "i"(SL)
                   : "memory");
    } else if constexpr (PACK == 2) {
      asm volatile("ds_read_b64 %[k0], %[ka0]\n\t"
                   "ds_read_b64 %[k1], %[ka1]\n\t"
                   TQ_V8("ds_read_u16") TQ_N2 "s_waitcnt lgkmcnt(0)"
                   : [k0] "=&v"(k0), [k1] "=&v"(k1), TQ_VOUT, [n0] "=&v"(n0), [n1] "=&v"(n1)
                   : [ka0] "v"(ka[0]), [ka1] "v"(ka[1]), TQ_VIN, [na] "v"(na), [sl] "i"(SL)
                   : "memory");
    } else {
      asm volatile("ds_read_b64 %[k0], %[ka0]\n\t"
                   "ds_read_b64 %[k1], %[ka1]\n\t"
                   TQ_V8("ds_read_u16") TQ_N1 "s_waitcnt lgkmcnt(0)"
                   : [k0] "=&v"(k0), [k1] "=&v"(k1), TQ_VOUT, [n0] "=&v"(n0), [n1] "=&v"(n1),
                     [n2] "=&v"(n2), [n3] "=&v"(n3)
                   : [ka0] "v"(ka[0]), [ka1] "v"(ka[1]), TQ_VIN, [na] "v"(na), [nb] "v"(nb),
                     [sl] "i"(SL)
                   : "memory");
    }
#pragma unroll
    for (int i = 0; i < PD / 32; i++) {
      d.k[0][i] = k0[i];
      d.k[1][i] = k1[i];
    }
    d.v[0][0][0] = a0; d.v[0][1][0] = a1; d.v[0][2][0] = a2; d.v[0][3][0] = a3;
    d.v[1][0][0] = c0; d.v[1][1][0] = c1; d.v[1][2][0] = c2; d.v[1][3][0] = c3;
  } else {
    static_assert(PD == 256 && PACK == 1, "head size 256 keeps one tile per score set");
    u32x4 k0, k1, k2, k3;
    u32x2 a0, a1, a2, a3, c0, c1, c2, c3;
    asm volatile("ds_read_b128 %[k0], %[ka0]\n\t"
                 "ds_read_b128 %[k1], %[ka0] offset:16\n\t"
                 "ds_read_b128 %[k2], %[ka1]\n\t"
                 "ds_read_b128 %[k3], %[ka1] offset:16\n\t"
                 TQ_V8("ds_read_b64") TQ_N1 "s_waitcnt lgkmcnt(0)"
                 : [k0] "=&v"(k0), [k1] "=&v"(k1), [k2] "=&v"(k2), [k3] "=&v"(k3), TQ_VOUT,
                   [n0] "=&v"(n0), [n1] "=&v"(n1), [n2] "=&v"(n2), [n3] "=&v"(n3)
                 : [ka0] "v"(ka[0]), [ka1] "v"(ka[1]), TQ_VIN, [na] "v"(na), [nb] "v"(nb),
                   [sl] "i"(SL)
                 : "memory");
#pragma unroll
    for (int i = 0; i < 4; i++) {
      d.k[0][i] = k0[i];
      d.k[0][4 + i] = k1[i];
      d.k[1][i] = k2[i];
      d.k[1][4 + i] = k3[i];
    }
    const u32x2 vva[4] = {a0, a1, a2, a3}, vvc[4] = {c0, c1, c2, c3};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      d.v[0][j][0] = vva[j][0]; d.v[0][j][1] = vva[j][1];
      d.v[1][j][0] = vvc[j][0]; d.v[1][j][1] = vvc[j][1];
    }
  }
#undef TQ_V8
#undef TQ_VOUT
#undef TQ_VIN
#undef TQ_N2
#undef TQ_N1
  d.nkv[0] = n0 | (PACK == 2 ? n1 : n2) << 16;
  d.nkv[1] = n1 | n3 << 16;  // PACK 1: tile 1
#else
  (void)ka; (void)va; (void)vb; (void)na; (void)nb; (void)d;
#endif
}

// fp16 pair (a * V norm of na, b * V norm of nb), the norms fp16 values in
// the high halves of na / nb: v_fma_mixlo writes the low half, v_fma_mixhi
// the high half (fp32 product, one rounding to fp16 each)
__device__ __forceinline__ uint32_t mix_pair(float a, uint32_t na, float b, uint32_t nb) {
  uint32_t r;
#if defined(__HIP_DEVICE_COMPILE__)
  asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixhi_f16 %0, %3, %4, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
      : "=&v"(r)
      : "v"(a), "v"(na), "v"(b), "v"(nb));
#else
  r = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(a * hi_half(na))) |
      ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(b * hi_half(nb))) << 16);
#endif
  return r;
}

// The fp16 remainders of two products: fp16(a * nv_a - h_a), h_a the low half
// of hw (mix_pair's result for a), and likewise for b with the high half;
// one fma with one rounding each, so hi + lo carries the fp32 product to
// about 22 bits
__device__ __forceinline__ uint32_t mix_pair_lo(float a, uint32_t na, float b, uint32_t nb,
                                                uint32_t hw) {
  uint32_t r;
#if defined(__HIP_DEVICE_COMPILE__)
  asm("v_fma_mixlo_f16 %0, %1, %2, -%5 op_sel:[0,1,0] op_sel_hi:[0,1,1]\n\t"
      "v_fma_mixhi_f16 %0, %3, %4, -%5 op_sel:[0,1,1] op_sel_hi:[0,1,1]"
      : "=&v"(r)
      : "v"(a), "v"(na), "v"(b), "v"(nb), "v"(hw));
#else
  const float ha = lo_half(hw), hb = hi_half(hw);
  r = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(a * hi_half(na) - ha)) |
      ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(b * hi_half(nb) - hb)) << 16);
#endif
  return r;
}

// Online softmax over the NV score values this lane holds for one step
// (PACK 2: 4 values, tile (l%16)/8, head l%8; PACK 1: 8 values, tile 0 then
// tile 1, head l%16; tokens 4*q4 + r), already scaled by the K norms.  nvr:
// the tokens' V norms (fp16, high halves).  valid: token masks, `full` when
// all are valid (uniform); hmask: the lanes of real heads (head < ratio).
// Writes p * nv as fp16 pairs to pw; the running
// max only moves when the step exceeds it by more than 2^3, so p <= 8.
template <int PD, int NV, bool LO = false>
__device__ __forceinline__ void softmax_step(float* sc, const uint32_t* nvr, bool full,
                                             const bool* valid, bool rot8, uint64_t hmask,
                                             float lpv, SoftmaxState<PD>& st, uint32_t* pw,
                                             uint32_t* pl = nullptr) {
  constexpr int NO = PD / 16;
  if (!full) {
#pragma unroll
    for (int r = 0; r < NV; r++) sc[r] = valid[r] ? sc[r] : -INFINITY;
  }
  float tmax = vmax(vmax3(sc[0], sc[1], sc[2]), sc[3]);
  if constexpr (NV == 8) tmax = vmax3(tmax, vmax3(sc[4], sc[5], sc[6]), sc[7]);
  if (rot8) tmax = max_ror8(tmax);
  tmax = xor16_max(tmax);
  tmax = xor32_max(tmax);
  const float m_new = vmax(st.m, tmax);
  // lanes of padding heads (head >= ratio) never move the max
  if ((__builtin_amdgcn_ballot_w64(m_new > st.m + 3.0f) & hmask) != 0) {
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
  float ls;
  if (full) {
    ls = (pr[0] + pr[1]) + (pr[2] + pr[3]);
    if constexpr (NV == 8) ls += (pr[4] + pr[5]) + (pr[6] + pr[7]);
#pragma unroll
    for (int r = 0; r < NV; r += 2) pw[r / 2] = mix_pair(pr[r], nvr[r], pr[r + 1], nvr[r + 1]);
    if constexpr (LO) {
#pragma unroll
      for (int r = 0; r < NV; r += 2)
        pl[r / 2] = mix_pair_lo(pr[r], nvr[r], pr[r + 1], nvr[r + 1], pw[r / 2]);
    }
  } else {
    // masked entries: p = 0, and their norm bits may be anything (0 * inf
    // is NaN), so their products are zeroed too
#pragma unroll
    for (int r = 0; r < NV; r++) pr[r] = valid[r] ? pr[r] : 0.0f;
    ls = (pr[0] + pr[1]) + (pr[2] + pr[3]);
    if constexpr (NV == 8) ls += (pr[4] + pr[5]) + (pr[6] + pr[7]);
#pragma unroll
    for (int r = 0; r < NV; r += 2) {
      const float x0 = valid[r] ? pr[r] * hi_half(nvr[r]) : 0.0f;
      const float x1 = valid[r + 1] ? pr[r + 1] * hi_half(nvr[r + 1]) : 0.0f;
      const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
      pw[r / 2] = (uint32_t)__builtin_bit_cast(uint16_t, h0) |
                  ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
      if constexpr (LO)
        pl[r / 2] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(x0 - (float)h0)) |
                    ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(x1 - (float)h1)) << 16);
    }
  }
  st.lsum += ls;
}

// Bring tile 1's packed probabilities (lanes 8..15 of each row) to lanes
// 0..7 (DPP row_shl:8), the B-operand position of the PV MFMA.
__device__ __forceinline__ uint32_t shl8(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x108, 0xf, 0xf, false);
}
// value of lane n ^ 8 within each row of 16 (DPP row_ror:8)
__device__ __forceinline__ uint32_t ror8u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xf, 0xf, false);
}

// Build option (-DTQ_PV_LO=1): the PV probabilities as fp16 hi + lo parts.
// With GQA ratio <= 8 (QC) the B operand's columns 8..15 carry no head, so
// they take the lo parts of heads 0..7 and the output adds column n + 8 to
// column n at the end; the products p * nv then enter the PV MFMAs to about
// 22 bits, as the reference's fp32 probabilities do.  Off by default:
// measured on the B = 64 ragged batches (Student-t keys) it lowers the rms
// error against the fp64 oracle by 16% (3.1e-4 -> 2.6e-4) but not the
// largest errors, which the fp16 partial rows and the fp16 output set, and
// costs 0.4 us per launch at configs[2] and 1.7% on the ragged batches.
#ifndef TQ_PV_LO
#define TQ_PV_LO 0
#endif
constexpr bool kPvLo = TQ_PV_LO != 0;

#ifndef TQ_DECODE_MATH
#define TQ_DECODE_MATH 2
#endif
// Split-KV partials.  Workgroup = (sequence b, split s, group hg of G kv
// heads), one wave per kv head.  The workgroup streams its heads' cache rows
// tile by tile (16 tokens x G entries of both slabs) into a ring of
// kRingSlots LDS tile slots with direct-to-LDS 16-byte copies: every copy
// instruction reads 1 KB of consecutive row bytes, so each cache line is
// requested once by one instruction.  A step is two tiles.  Per step: wait
// for the copies of the step's tiles (the waves share the copies, so each
// wave waits for its own and the barrier that follows makes all of them
// visible), barrier, each wave reads its own head's codes and norms into
// registers, barrier, then the copies of the tiles kRingSlots ahead are
// issued into the two slots just read, and the math runs while they are in
// flight.  Slot bases are runtime values (advanced by two slots per step).
// MATH: 2 = the kernel (TQ_DECODE_MATH, a build option for measurement
// builds only, sets the default); 1 and 0 are diagnostics of its data movement: 1 =
// the attention math compiled out (q' setup, table build and partial-row
// stores kept), 0 = the bare copy ring (page walk, copies, waits, barriers
// and slot reads only).
template <int PD, int G, int PACK, bool QC, bool PLAN, int MATH = TQ_DECODE_MATH>
__global__ __launch_bounds__(64 * G)
__attribute__((amdgpu_waves_per_eu(PD == 256 ? 2 : (PACK == 1 ? 3 : 4))))
void decode_partials_kernel(DecodeParams p) {
  using RG = RingGeom<PD, G>;
  constexpr int KD = PD / 32;
  constexpr int NO = PD / 16;
  constexpr int EBS = RG::EBS;
  constexpr int ECH = RG::ECH;
  constexpr int CPT = RG::CPT;
  constexpr int NI = RG::NI;
  constexpr bool PLO = QC && kPvLo && MATH >= 2;  // PV probabilities as hi + lo
  // LDS: the dequant table at address 0 (the table reads rely on it), then
  // the ring of tile slots
  struct __attribute__((aligned(16))) Lds {
    uint32_t klut[256 * RG::LC];
    uint8_t ring[RG::RING];
  };
  __shared__ Lds sm;

  // dequant table: byte e -> fp16 values of its high nibble (low half) and
  // its low nibble (high half), built with the same table arithmetic as dq8,
  // in RG::LC copies (written four at a time, as inline assembly: the
  // copies in flight into the ring do not touch it, which the compiler
  // cannot tell)
  auto init_table = [&]() {
    for (int i = threadIdx.x; i < 64 * RG::LC; i += 64 * G) {
      const int e = i / (RG::LC / 4);
      uint32_t x[4];
      dq8((uint32_t)e * 0x01010101u, x);
      [[maybe_unused]] const uint32_t val = (x[2] & 0xffffu) | (x[0] << 16);
#if defined(__HIP_DEVICE_COMPILE__)
      asm volatile("ds_write_b128 %0, %1" : : "v"(lds_addr(&sm.klut[4 * i])), "v"(u32x4{val, val, val, val}) : "memory");
#endif
    }
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#endif
  };

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int q4 = lane >> 4, n = lane & 15;
  const uint32_t lanec = (uint32_t)(lane & (RG::LC - 1)) * 4u;  // this lane's table copy
  const int half = gridDim.x >> 1;
  const int mem = p.pair_pct > 0 && (int)blockIdx.x >= half;
  int bid = blockIdx.x - mem * half;
  const int hg = bid % p.HG;
  bid /= p.HG;
  const int kvh = hg * G + w;
  const int ratio = p.ratio;
  // the token range [c0, c1) of sequence b this workgroup serves, and its
  // partial row
  int b, L, ip, c0, c1;
  int64_t row;
  if constexpr (PLAN) {
    const int rowmul = p.pair_pct > 0 ? 2 : 1;
    const bool writer = blockIdx.x == 0 && w == 0;
    PlanSlot ps;
    if (p.B <= 64) {
      // one sequence per lane: lengths and page-table starts in registers,
      // loaded in one round trip
      const bool in = lane < p.B;
      const int len = in ? max(p.seq_lens[lane], 0) : 0;
      const int ipl = in ? p.indptr[lane] : 0;
      ps = plan_slot([&](int) { return len; }, [&](int) { return ipl; }, p.B, 1, p.units, bid,
                     rowmul, p.split_out, writer);
    } else {
      // staged in LDS where the dequant table goes (built later): lengths,
      // then page-table starts, kPlanMaxBatch of each
      int* const st = reinterpret_cast<int*>(sm.klut);
      for (int i = threadIdx.x; i < kPlanMaxBatch; i += 64 * G) {
        st[i] = i < p.B ? max(p.seq_lens[i], 0) : 0;
        st[kPlanMaxBatch + i] = i < p.B ? p.indptr[i] : 0;
      }
      __syncthreads();
      ps = plan_slot([&](int i) { return st[64 * i + lane]; },
                     [&](int i) { return st[kPlanMaxBatch + 64 * i + lane]; }, p.B,
                     (p.B + 63) >> 6, p.units, bid, rowmul, p.split_out, writer);
      __syncthreads();  // the staging area is free again
    }
    if (ps.b < 0) return;  // unit beyond the plan: no row (uniform over the workgroup)
    b = ps.b;
    L = ps.L;
    ip = ps.ip;
    c0 = ps.j * ps.U;
    c1 = c0 + ps.U;
    if (p.pair_pct > 0) {
      const int first = min((ps.U * p.pair_pct / 100 + 15) & ~15, ps.U);
      c0 = mem ? c0 + first : c0;
      c1 = mem ? c1 : c0 + first;
      row = 2 * (int64_t)(ps.Pb + ps.j) + mem;
    } else {
      row = ps.Pb + ps.j;
    }
  } else {
    int s;
    if (p.pair_pct > 0) {
      const int pj = bid % (p.S >> 1);
      b = bid / (p.S >> 1);
      s = 2 * pj + mem;
    } else {
      s = bid % p.S;
      b = bid / p.S;
    }
    // sequence length and page-table start, loaded before anything else:
    // the first copies depend on them
    L = p.seq_lens[b];
    ip = p.indptr[b];
    c0 = s * p.cs;
    c1 = c0 + p.cs;
    if (p.pair_pct > 0) {
      const int base = (s & ~1) * p.cs;
      const int first = min((2 * p.cs * p.pair_pct / 100 + 15) & ~15, 2 * p.cs);
      c0 = (s & 1) ? base + first : base;
      c1 = (s & 1) ? base + 2 * p.cs : base + first;
    }
    row = (int64_t)b * p.S + s;
  }

  half8_t qb[KD], ql[QC ? 1 : KD];  // q' operands

  // s * q of this wave's heads, loaded first so that its latency overlaps
  // the page-table loads and the first copies: in load j < NQL, lane l holds
  // the 8 consecutive elements e = 512 j + 8 l .. + 7 (head e / PD, dim
  // e % PD).  Elements past the wave's heads read as zeros (empty range).
  // Larger head groups (ratio * PD > 512 * NQL) form q' through LDS below.
  // Four loads at head size 256 with at most two kv heads per workgroup
  // (ratio 8 there: 2048 elements), whose 8 KB hi / lo scratch per wave still
  // fits the table region; two elsewhere.  QLO: byte offset of the lo parts
  // in a wave's scratch (the hi parts come first).
  constexpr int NQL = PD == 256 && G <= 2 ? 4 : 2;
  constexpr int QLO = NQL * 1024;
  const bool qreg = ratio * PD <= 512 * NQL;  // uniform
  float qx[NQL][8];
  // sign bits of dims (8 lane) % PD .. + 7 (bit k: dim + k), for the inverse
  // rotation of the partial rows at the end (the same dims for every pass)
  [[maybe_unused]] uint32_t sgnbits = 0;
#if defined(__HIP_DEVICE_COMPILE__)
  if constexpr (MATH >= 1) {
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
      if (j == 0) {
#pragma unroll
        for (int k = 0; k < 8; k++) sgnbits |= (sw[k] >> 31) << k;
      }
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const float x = k & 1 ? hi_half(qv[k / 2]) : lo_half(qv[k / 2]);
        qx[j][k] = p.signs ? x * __uint_as_float(sw[k]) : x;
      }
    }
  }
#endif

#if defined(__HIP_DEVICE_COMPILE__)
  // both scalar loads complete here, in one round trip with the q loads in
  // flight (the compiler would otherwise sink the page-table start below the
  // branch on the split range and pay a second round trip)
  asm volatile("" : : "s"(L), "s"(ip));
#endif

  SoftmaxState<PD> st;
#pragma unroll
  for (int i = 0; i < NO; i++) st.O[i] = float4_t{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.mb = -INFINITY;
  st.lsum = 0.f;
  const float lpv = -__log2f(p.pv_scale);

  c0 = min(c0, L);
  c1 = min(c1, L);
  if (c0 < c1) {  // uniform over the workgroup
    constexpr int STEP = 2 * kTile;
    const int step0 = c0 / STEP, step1 = (c1 - 1) / STEP;
    const int tpp = p.block_size / kTile;  // tiles per page
    const int64_t tokstride = (int64_t)p.Hkv * EBS;
    [[maybe_unused]] const uint8_t* const kslab = p.ks;
    [[maybe_unused]] const uint8_t* const vslab = p.vs;
    const int tile_last = (c1 - 1) / kTile;
    const int tile_end = 2 * step1 + 1;  // last tile any step of this split reads
    [[maybe_unused]] const int rec = (int)(kTile * tokstride);

    // Tile window: lane i holds the byte offset inside a slab of tile
    // wtile + i (64 bit, as lo/hi halves) and tmask bit i says whether that
    // tile is present (within the split and on a page inside the cache).
    // When the copies reach the end of the window it slides by 32 tiles;
    // the page ids of the next 32 tiles are loaded one slide ahead (npg,
    // lanes 32..63).
    uint32_t tlo = 0, thi = 0;
    uint64_t tmask = 0;
    int wtile = 2 * step0;
    int npg = -1;
    auto page_of = [&](int t) -> int {
      return t <= tile_last ? p.indices[ip + t / tpp] : -1;
    };
    auto set_tile = [&](int t, int pg, bool& ok, uint32_t& lo, uint32_t& hi) {
      ok = pg >= 0 && pg < p.num_blocks;
      const int64_t off =
          ok ? ((int64_t)pg * p.block_size + (t % tpp) * kTile) * tokstride : 0;
      lo = (uint32_t)off;
      hi = (uint32_t)((uint64_t)off >> 32);
    };
    auto tile_ok = [&](int t) -> bool { return (tmask >> ((t - wtile) & 63)) & 1; };
    auto prefetch_pages = [&]() {
      npg = lane >= 32 ? page_of(wtile + 32 + lane) : -1;
    };
    {
      bool ok;
      set_tile(wtile + lane, page_of(wtile + lane), ok, tlo, thi);
      tmask = __ballot(ok);
      prefetch_pages();
    }
    auto slide = [&]() {
      bool ok;
      uint32_t lo, hi;
      set_tile(wtile + 32 + lane, npg, ok, lo, hi);
      const uint32_t lo_up = (uint32_t)__shfl((int)tlo, (lane + 32) & 63);
      const uint32_t hi_up = (uint32_t)__shfl((int)thi, (lane + 32) & 63);
      tlo = lane < 32 ? lo_up : lo;
      thi = lane < 32 ? hi_up : hi;
      tmask = (tmask >> 32) | (__ballot(ok && lane >= 32) & 0xffffffff00000000ull);
      wtile += 32;
      prefetch_pages();
    };

    // Copies: copy j of a tile (j < NI: K region, else V region; jj = j mod
    // NI) fills LDS chunks jj*64 + lane of the region.  Wave w issues copies
    // j = w, w + G, ...  Per-lane source offsets inside the tile's slab
    // (rows of tokstride bytes, the group's entries at hg*G*EBS):
    constexpr int NWMAX = RG::NW_HI;
    [[maybe_unused]] const int nmine = RG::NW_LO + (w < RG::NIT % G ? 1 : 0);  // uniform
    uint32_t goff[NWMAX];
#pragma unroll
    for (int i = 0; i < NWMAX; i++) {
      const int jj = (w + G * i) % NI;
      int pos = jj * 64 + lane;
      if (pos >= kTile * RG::RCH) pos = kTile * RG::RCH - 1;  // spill lanes reload a chunk
      const int t = pos / RG::RCH;
      const int c = min(pos % RG::RCH, CPT - 1);  // the pad chunk reloads the row's last
      goff[i] = (uint32_t)(t * tokstride + (int64_t)hg * G * EBS + c * 16);
    }
    auto issue = [&](int t, int slot) {
#if defined(__HIP_DEVICE_COMPILE__)  // the LDS-copy builtin has no host form
      const int jw = (t - wtile) & 63;
      const uint64_t off = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)thi, jw) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane((int)tlo, jw);
      const int nrec = tile_ok(t) ? rec : 0;
      const __amdgpu_buffer_rsrc_t rk =
          __builtin_amdgcn_make_buffer_rsrc((void*)(kslab + off), (short)0, nrec, 0x00020000);
      const __amdgpu_buffer_rsrc_t rv =
          __builtin_amdgcn_make_buffer_rsrc((void*)(vslab + off), (short)0, nrec, 0x00020000);
      uint8_t* const dst = sm.ring + slot * RG::TS;
#pragma unroll
      for (int i = 0; i < NWMAX; i++) {
        if (i < nmine) {
          const int j = w + G * i;
          const bool isv = j >= NI;
          const int jj = isv ? j - NI : j;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(isv ? rv : rk,
                                                   (void*)(dst + (isv ? RG::SLAB : 0) + jj * 1024),
                                                   16, goff[i], 0, 0, kCopyPolicy);
        }
      }
#else
      (void)t;
      (void)slot;
#endif
    };
    // wait until this wave's copies of every tile but the last `later`
    // issued ones have landed
    auto wait_copies = [&](int later) {
      const int nw = (RG::NW_HI != RG::NW_LO && w < RG::NIT % G) ? RG::NW_HI : RG::NW_LO;
      switch (later * nw) {
        case 0: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;
        case 1: __builtin_amdgcn_s_waitcnt(vmcnt_imm(1)); break;
        case 2: __builtin_amdgcn_s_waitcnt(vmcnt_imm(2)); break;
        case 3: __builtin_amdgcn_s_waitcnt(vmcnt_imm(3)); break;
        case 4: __builtin_amdgcn_s_waitcnt(vmcnt_imm(4)); break;
        case 5: __builtin_amdgcn_s_waitcnt(vmcnt_imm(5)); break;
        case 6: __builtin_amdgcn_s_waitcnt(vmcnt_imm(6)); break;
        case 7: __builtin_amdgcn_s_waitcnt(vmcnt_imm(7)); break;
        case 8: __builtin_amdgcn_s_waitcnt(vmcnt_imm(8)); break;
        case 9: __builtin_amdgcn_s_waitcnt(vmcnt_imm(9)); break;
        default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(10)); break;
      }
    };

    // per-lane LDS read offsets inside a region (see read_step)
    constexpr int ROWB = RG::ROWB;
    const int hb = w * ECH;  // first chunk of this wave's entry in a row
    uint32_t oK[1];
    if constexpr (PD == 128) {
      oK[0] = n * ROWB + (hb + q4) * 16;
    } else if constexpr (PD == 64) {
      oK[0] = n * ROWB + (hb + q4 / 2) * 16 + (q4 & 1) * 8;
    } else {
      oK[0] = n * ROWB + (hb + 2 * q4) * 16;  // two chunks: the second 16 bytes further
    }
    constexpr int VBY = PD / 32;  // V code bytes per lane per token
    const uint32_t oV = 4 * q4 * ROWB + hb * 16 + n * VBY;
    const int slotw = 16 / PACK;   // lanes per packed tile
    const int ptile = n / slotw;   // tile of this lane's packed scores
    const int head = n % slotw;    // head of this lane's packed scores
    const uint64_t hmask = __builtin_amdgcn_ballot_w64(head < ratio);  // lanes of real heads
    const uint32_t oN = (4 * q4 + (lane & 3)) * ROWB + (hb + PD / 32) * 16;

    // the q' scratch lives where the dequant table goes (the table is built
    // after it); with q' formed in registers it fits there (4 KB a wave), so
    // the first tiles go out before the q setup
    if (qreg) {
#pragma unroll
      for (int r = 0; r < kRingSlots; r++)
        if (2 * step0 + r <= tile_end) issue(2 * step0 + r, r);
    }

    // ---- q' = FWHT(s*q)/sqrt(pd), scaled to log2 units and split into
    // fp16 hi + lo parts (q' = hi + lo to ~22 bits, so the scores keep
    // fp32-level accuracy even for heavy-tailed keys), in the MFMA B layout.
    const float qsc = (p.signs ? p.inv_sqrt_pd : 1.0f) * p.qk_scale;
    const int hq = QC ? (n & 7) : n;  // q head of this lane's B column
    if constexpr (MATH == 0) {
      if (!qreg) {
#pragma unroll
        for (int r = 0; r < kRingSlots; r++)
          if (2 * step0 + r <= tile_end) issue(2 * step0 + r, r);
      }
    } else if (qreg) {
      // in registers: butterflies h = 1, 2, 4 inside a lane, h >= 8 between
      // lanes l and l ^ (h / 8) (DPP, one fma with a lane sign each)
      // the second 512 elements only exist when ratio * PD > 512
      const int nql = (ratio * PD + 511) / 512;  // loads holding real elements (uniform)
      if (p.signs) {
#pragma unroll
        for (int j = 0; j < NQL; j++) {
          if (j >= nql) break;
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
            const float sgn = (lane & (h / 8)) ? -1.0f : 1.0f;
#pragma unroll
            for (int k = 0; k < 8; k++) qx[j][k] = fmaf(sgn, qx[j][k], xor_lane(qx[j][k], h / 8));
          }
        }
      }
      // fp16 hi / lo parts through a per-wave LDS scratch (hi then lo, 1024
      // elements each) to the B layout: column n takes head hq, dims
      // q4 * PD/4 + 8c + 0..7.  Inline assembly: the scratch shares the ring
      // with the copy in flight, and the compiler would otherwise wait for it.
#if defined(__HIP_DEVICE_COMPILE__)
      const uint32_t qsb = lds_addr(sm.klut) + (uint32_t)w * (2u * QLO);
#pragma unroll
      for (int j = 0; j < NQL; j++) {
        if (j >= nql) break;  // those scratch elements are never read
        u32x4 vh, vl;
#pragma unroll
        for (int wd = 0; wd < 4; wd++) {
          const float x0 = qx[j][2 * wd] * qsc, x1 = qx[j][2 * wd + 1] * qsc;
          const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
          const _Float16 l0 = (_Float16)(x0 - (float)h0), l1 = (_Float16)(x1 - (float)h1);
          vh[wd] = (uint32_t)__builtin_bit_cast(uint16_t, h0) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
          vl[wd] = (uint32_t)__builtin_bit_cast(uint16_t, l0) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
        }
        const uint32_t a = qsb + (uint32_t)(512 * j + 8 * lane) * 2u;
        asm volatile("ds_write_b128 %0, %1\n\tds_write_b128 %0, %2 offset:%3"
                     :
                     : "v"(a), "v"(vh), "v"(vl), "i"(QLO)
                     : "memory");
      }
#pragma unroll
      for (int c = 0; c < KD; c++) {
        const uint32_t e = (uint32_t)(hq * PD + q4 * (PD / 4) + 8 * c);
        u32x4 vh, vl;
        if constexpr (QC) {
          // (columns of heads >= ratio read elements never written: zeroed)
          asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)"
                       : "=v"(vh)
                       : "v"(qsb + e * 2u + (n < 8 ? 0u : (uint32_t)QLO))
                       : "memory");
          if (hq >= ratio) vh = u32x4{0u, 0u, 0u, 0u};
          qb[c] = __builtin_bit_cast(half8_t, vh);
        } else {
          asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:%3\n\t"
                       "s_waitcnt lgkmcnt(0)"
                       : "=&v"(vh), "=&v"(vl)
                       : "v"(qsb + e * 2u), "i"(QLO)
                       : "memory");
          if (hq >= ratio) vh = vl = u32x4{0u, 0u, 0u, 0u};
          qb[c] = __builtin_bit_cast(half8_t, vh);
          ql[c] = __builtin_bit_cast(half8_t, vl);
        }
      }
#endif
      // once every wave has read its scratch, the table overwrites it
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      init_table();
    } else {
      // ---- q' = FWHT(s*q)/sqrt(pd) for this wave's `ratio` heads on an LDS
      // scratch from the table's place on (each wave its own region; the
      // launcher keeps G * ratio * PD floats within the table and the ring),
      // before any copy is issued.
      // LDS operations of one wave complete in order, so a wave barrier
      // orders the butterfly stages.
      float* const qs = reinterpret_cast<float*>(sm.klut) + (size_t)w * ratio * PD;
      auto qsync = [&]() {
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
      };
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
#pragma unroll
      for (int c = 0; c < KD; c++) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const int d = q4 * (PD / 4) + 8 * c + e;
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
      __syncthreads();  // every wave is done with its scratch: the copies may start
#pragma unroll
      for (int r = 0; r < kRingSlots; r++)
        if (2 * step0 + r <= tile_end) issue(2 * step0 + r, r);
      init_table();
    }

    // math of one step (tiles 2k, 2k + 1) from the registers in d
    auto compute = [&](int k, const StepData<PD>& d) {
      const bool okT[2] = {tile_ok(2 * k), tile_ok(2 * k + 1)};
      // scores of both tiles (scheduling barriers keep the two tiles'
      // dequant temporaries from being live at the same time)
      float4_t acc[2];
      constexpr bool PM = PACK == 2;  // packed merge of the two tiles' unmerged sums
      static_assert(PACK == 1 || QC, "two tiles per score set need the hi / lo columns");
      acc[0] = tile_scores<PD, QC, RG::SH, !PM>(d.k[0], qb, ql, lanec, sm.klut);
      __builtin_amdgcn_sched_barrier(0);
      acc[1] = tile_scores<PD, QC, RG::SH, !PM>(d.k[1], qb, ql, lanec, sm.klut);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (PM) acc[0] = pack_merge(acc[0], acc[1]);
      constexpr int NV = 4 * (2 / PACK);  // score values per lane
      float sc[NV];
      uint32_t nvr[NV];
      bool valid[NV];
#pragma unroll
      for (int g = 0; g < 2 / PACK; g++) {
        const uint32_t nkv = d.nkv[g];
        const uint32_t nr[4] = {quad_bcast<0>(nkv), quad_bcast<1>(nkv), quad_bcast<2>(nkv),
                                quad_bcast<3>(nkv)};
#pragma unroll
        for (int r = 0; r < 4; r++) {
          // tile 0's scores in lanes 0..7 of each row and tile 1's in 8..15
          // (PACK 2), times the K norm straight from its fp16 half
          const float a = PACK == 2 ? acc[0][r] : acc[g][r];
          sc[4 * g + r] = mul_lo_half(a, nr[r]);
          nvr[4 * g + r] = nr[r];
        }
      }
      const int t_first = 2 * k * kTile;  // first token of this step
      // (uniform; read back as a scalar so that it stays one)
      const bool full = __builtin_amdgcn_readfirstlane(
                            (okT[0] && okT[1] && t_first >= c0 && t_first + 2 * kTile <= c1)
                                ? 1 : 0) != 0;
      if (!full) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
          const int T = PACK == 2 ? ptile : i / 4;
          const int t = (2 * k + T) * kTile + 4 * q4 + (i & 3);
          valid[i] = okT[T] && t >= c0 && t < c1;
        }
      }
      uint32_t pw[NV / 2], pl[NV / 2];
      softmax_step<PD, NV, PLO>(sc, nvr, full, valid, PACK == 2, hmask, lpv, st, pw, pl);
      half8_t p8;
      if constexpr (PACK == 2 && PLO) {
        // lanes n < 8: hi parts of tile 0 (own) and tile 1 (lane n + 8);
        // lanes n >= 8: lo parts of tile 0 (lane n - 8) and tile 1 (own)
        const bool up = n >= 8;
        const uint32_t r0 = ror8u(up ? pw[0] : pl[0]), r1 = ror8u(up ? pw[1] : pl[1]);
        p8 = up ? as_half8(r0, r1, pl[0], pl[1]) : as_half8(pw[0], pw[1], r0, r1);
      } else if constexpr (PACK == 2) {
        p8 = as_half8(pw[0], pw[1], shl8(pw[0]), shl8(pw[1]));
      } else if constexpr (PLO) {
        // lanes n >= 8 hold the same scores as lane n - 8: their lo parts
        p8 = n >= 8 ? as_half8(pl[0], pl[1], pl[2], pl[3]) : as_half8(pw[0], pw[1], pw[2], pw[3]);
      } else {
        p8 = as_half8(pw[0], pw[1], pw[2], pw[3]);
      }
      step_pv<PD, RG::SH>(d.v[0], d.v[1], p8, st, lanec, sm.klut);
    };

    // one step: tiles 2k, 2k + 1 in ring slots s0, s1
    auto run = [&](int k, int s0, int s1) {
      // the tiles after 2k + 1 already issued may stay in flight
      wait_copies(max(0, min(kRingSlots - 2, tile_end - (2 * k + 1))));
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();  // every wave's copies of tiles 2k, 2k + 1 have landed
      __builtin_amdgcn_sched_barrier(0);
      StepData<PD> d;
      {
        const uint32_t b0 = RG::LUTB + s0 * RG::TS, b1 = RG::LUTB + s1 * RG::TS;  // K regions
        const uint32_t ka[2] = {oK[0] + b0, oK[0] + b1};
        const uint32_t na = oN + (PACK == 2 && ptile ? b1 : b0);
        read_step<PD, G, PACK>(ka, oV + b0 + RG::SLAB, oV + b1 + RG::SLAB, na, oN + b1, d);
      }
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();  // every wave has read the two slots
      __builtin_amdgcn_sched_barrier(0);
      // the next copies go into the two slots just read
      if (2 * k + kRingSlots <= tile_end) {
        if (2 * k + kRingSlots + 1 >= wtile + 64) slide();
        issue(2 * k + kRingSlots, s0);
        if (2 * k + kRingSlots + 1 <= tile_end) issue(2 * k + kRingSlots + 1, s1);
      }
      if constexpr (MATH >= 2) compute(k, d);
    };
    for (int k = step0, s0 = 0, s1 = 1; k <= step1; k++) {
      run(k, s0, s1);
      s0 = s0 + 2 >= kRingSlots ? s0 + 2 - kRingSlots : s0 + 2;  // tile t sits in slot
      s1 = s1 + 2 >= kRingSlots ? s1 + 2 - kRingSlots : s1 + 2;  // (t - 2 step0) mod slots
    }
  }

  if constexpr (MATH == 0) return;  // the bare ring stores nothing
  // ---- finish: O[i][r] = o[h = n][dim (4*q4 + r)*NO + i]
  if constexpr (PLO) {
    // column n + 8 accumulated the lo parts of head n's probabilities
#pragma unroll
    for (int i = 0; i < NO; i++)
#pragma unroll
      for (int r = 0; r < 4; r++)
        st.O[i][r] = st.O[i][r] + __uint_as_float(ror8u(__float_as_uint(st.O[i][r])));
  }
  float lt = st.lsum;
  if constexpr (PACK == 2) lt = lt + __int_as_float(__builtin_amdgcn_mov_dpp(
                                         __float_as_int(lt), 0x128, 0xf, 0xf, false));
  lt = xor32_sum(xor16_sum(lt));
  // The wave's partial rows (its `ratio` q heads, consecutive rows of
  // partition_o) are staged in LDS and written with whole-wave 1 KB stores:
  // written straight from the MFMA layout they take 16 lanes x 16 B per
  // store instruction at a 128-byte stride, and those scattered partial-line
  // writes slow the other workgroups' streaming reads (4-5 us per launch at
  // configs[2]).  After the barrier no wave reads the table or the ring any
  // more, so wave w stages at w * ratio * PD floats from the start of LDS.
  // The staging holds G * ratio * PD floats: within the table region when
  // ratio * PD <= 1024 (the assert), and within table + ring otherwise (the
  // launcher picks G so that the q scratch of that size fits, the same bound).
  static_assert(G * 2 * (PD == 256 && G <= 2 ? 4 : 2) * 1024 <= RG::LUTB,
                "the q' scratch of the waves exceeds the table region");
  __builtin_amdgcn_s_barrier();
  float* const stage = reinterpret_cast<float*>(&sm) + (size_t)w * ratio * PD;
  const int64_t orow0 = row * p.Hq + kvh * ratio;  // first row of this wave
  if (n < ratio) {
    // o = pv_scale * O / lsum' (p' = p * pv_scale in both O and lsum')
    const float inv = lt > 0.f ? p.pv_scale / lt : 0.0f;
    float* dst = stage + n * PD + q4 * (PD / 4);
#pragma unroll
    for (int r = 0; r < 4; r++) {
#pragma unroll
      for (int i = 0; i < NO; i += 4) {
        float4_t v = {st.O[i][r] * inv, st.O[i + 1][r] * inv, st.O[i + 2][r] * inv,
                      st.O[i + 3][r] * inv};
        *reinterpret_cast<float4_t*>(dst + r * NO + i) = v;
      }
    }
    // natural-log LSE: (m + log2(sum p)) * ln 2 = (mb + log2(lsum')) * ln 2
    if (q4 == 0)
      p.plse[orow0 + n] = lt > 0.f ? (st.mb + __log2f(lt)) * 0.69314718055994531f : -INFINITY;
  }
  // LDS operations of a wave complete in order: the reads below see the
  // writes above
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
  // Each row goes back to the original domain here, o = s * FWHT(o') /
  // sqrt(pd), per split as the reference's v5 kernel does
  // (flashinfer_decode_turboquant_v5_tc.cuh:712-765): the merge of the
  // splits is linear, so the combine then needs no rotation and no exchange
  // across its waves.  Lane l holds 8 consecutive dims of one row (PD / 8
  // lanes per row, whole rows per pass): butterflies 1, 2, 4 in-lane, the
  // rest between the row's lanes.  Rows are stored as fp16 (the combine
  // reads them so): half the bytes of fp32 rows, and their rounding
  // (relative 2^-11 on normalised outputs) is far inside the output
  // tolerance.
  _Float16* const out = reinterpret_cast<_Float16*>(p.po) + orow0 * PD;
  for (int e = 8 * lane; e < ratio * PD; e += 512) {
    const float4_t a = *reinterpret_cast<const float4_t*>(stage + e);
    const float4_t c = *reinterpret_cast<const float4_t*>(stage + e + 4);
    float x[8] = {a[0], a[1], a[2], a[3], c[0], c[1], c[2], c[3]};
    if constexpr (MATH >= 2) {
      if (p.signs) {  // uniform
#pragma unroll
        for (int hh = 1; hh < 8; hh <<= 1)
#pragma unroll
          for (int k = 0; k < 8; k++)
            if (!(k & hh)) {
              const float u = x[k], v = x[k + hh];
              x[k] = u + v;
              x[k + hh] = u - v;
            }
#pragma unroll
        for (int m = 1; m < PD / 8; m <<= 1) {
          const float sgn = (lane & m) ? -1.0f : 1.0f;  // upper lane: partner - own
#pragma unroll
          for (int k = 0; k < 8; k++) x[k] = __builtin_fmaf(sgn, x[k], xor_lane(x[k], m));
        }
#pragma unroll
        for (int k = 0; k < 8; k++)
          x[k] = __uint_as_float(__float_as_uint(x[k] * p.inv_sqrt_pd) ^
                                 (((sgnbits >> k) & 1u) << 31));
      }
    }
    const half8_t h = {(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3],
                       (_Float16)x[4], (_Float16)x[5], (_Float16)x[6], (_Float16)x[7]};
    *reinterpret_cast<half8_t*>(out + e) = h;
  }
}
// four fp16 partial-row values as fp32
__device__ __forceinline__ float4_t load_half4(const _Float16* src) {
  const half4_t h = *reinterpret_cast<const half4_t*>(src);
  return float4_t{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
}

// LSE merge of the splits of one (sequence, q head) and the fp16 store:
// o = sum_s e^(lse_s - M) o_s / sum_s e^(lse_s - M), splits with lse = -inf
// (no tokens) skipped.  The partial rows arrive in the original domain (the
// partials kernel applies the inverse rotation per split), so the four waves
// of a workgroup are independent: wave w merges dims [w PD/4, (w+1) PD/4),
// lane (c, g) the float4 column c of the wave's dims over the splits g,
// g + NG, ... (NG = 64 / (PD/16) split groups), with a running max per lane;
// the groups then meet through lane swaps (no LDS, no barrier), and the lanes
// of group 0 store.
template <int PD>
__global__ __launch_bounds__(256) void combine_kernel(const _Float16* __restrict__ po,
                                                      const float* __restrict__ plse, int S_fixed,
                                                      const int32_t* __restrict__ split_rows,
                                                      int Hq, _Float16* __restrict__ o) {
  constexpr int CW = PD / 16;      // float4 columns per wave (PD / 4 dims)
  constexpr int NG = 64 / CW;      // split groups per wave
  constexpr int R = 8;             // splits per lane per round trip
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int c = lane % CW, g = lane / CW;
  const int b = blockIdx.x / Hq, h = blockIdx.x % Hq;
  // the splits of sequence b are the partial rows r0 .. r0 + S - 1: b * S_fixed
  // onwards, or split_rows[b] .. split_rows[b + 1] (a balanced plan)
  int r0 = b * S_fixed, S = S_fixed;
  if (split_rows) {
    r0 = split_rows[b];
    S = split_rows[b + 1] - r0;
  }
  const int64_t row0 = (int64_t)r0 * Hq + h;
  const int col = wv * (PD / 4) + 4 * c;  // first dim of this lane's column
  float m = -INFINITY, den = 0.f;
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < S; s0 += NG * R) {
    // this round's LSEs and rows, all loaded before any is used
    float l[R];
    float4_t v[R];
#pragma unroll
    for (int j = 0; j < R; j++) {
      const int sj = s0 + g + NG * j;
      l[j] = -INFINITY;
      v[j] = float4_t{0.f, 0.f, 0.f, 0.f};
      if (sj < S) {
        const int64_t r = row0 + (int64_t)sj * Hq;
        l[j] = plse[r];
        v[j] = load_half4(po + r * PD + col);
      }
    }
    float mr = m;
#pragma unroll
    for (int j = 0; j < R; j++) mr = fmaxf(mr, l[j]);
    if (mr > -INFINITY) {
      const float sc = m > -INFINITY ? __expf(m - mr) : 0.0f;
      den *= sc;
      acc *= sc;
#pragma unroll
      for (int j = 0; j < R; j++) {
        const float wgt = l[j] > -INFINITY ? __expf(l[j] - mr) : 0.0f;
        den += wgt;
        // a skipped split's row may hold any bits: it adds nothing
        acc += wgt != 0.0f ? wgt * v[j] : float4_t{0.f, 0.f, 0.f, 0.f};
      }
      m = mr;
    }
  }
  // the split groups of a column: lanes c + CW g, g = 0 .. NG-1, met by lane
  // xors CW .. 32 (a common max first, then the rescaled sums)
  // (lane xor 4 / 8 by DPP, 16 / 32 by permlane swaps: no LDS round trips)
  auto xsum = [](float x, int d) {
    if (d == 16) return xor16_sum(x);
    if (d == 32) return xor32_sum(x);
    return x + xor_lane(x, d);
  };
  float mx = m;
#pragma unroll
  for (int d = CW; d < 64; d <<= 1) {
    if (d == 16) mx = xor16_max(mx);
    else if (d == 32) mx = xor32_max(mx);
    else mx = fmaxf(mx, xor_lane(mx, d));
  }
  const float sc = (m > -INFINITY) ? __expf(m - mx) : 0.0f;
  den *= sc;
  acc *= sc;
#pragma unroll
  for (int d = CW; d < 64; d <<= 1) {
    den = xsum(den, d);
#pragma unroll
    for (int k = 0; k < 4; k++) acc[k] = xsum(acc[k], d);
  }
  if (g == 0) {
    const float inv = den > 0.f ? 1.0f / den : 0.0f;
    const half4_t hv = {(_Float16)(acc[0] * inv), (_Float16)(acc[1] * inv),
                        (_Float16)(acc[2] * inv), (_Float16)(acc[3] * inv)};
    *reinterpret_cast<half4_t*>(o + ((int64_t)b * Hq + h) * PD + col) = hv;
  }
}

// LDS bytes of a partials workgroup of g kv heads (mirrors RingGeom).
int ring_lds_bytes(int pd, int g) {
  const int ech = (pd == 64 ? 48 : (pd == 128 ? 80 : 144)) / 16;
  const int rch = (g * ech) | 1;
  const int ni = (kTile * rch + 63) / 64;
  return 256 * 4 * lut_copies(pd, g) + kRingSlots * 2 * ni * 1024;
}

// Heads (waves) per partials workgroup: the largest of 8, 4, 2, 1 (at most 4
// for head size 256) that divides num_kv_heads and, when q' is formed in LDS
// (ratio * pd > 1024), whose q scratch fits the ring.
int decode_group_size(int pd, int hkv, int ratio) {
  const int maxg = pd == 256 ? 4 : 8;
  for (int g = maxg; g >= 1; g >>= 1)
    if (hkv % g == 0 &&
        (ratio * pd <= 1024 || (size_t)g * ratio * pd * 4 <= (size_t)ring_lds_bytes(pd, g)))
      return g;
  return 0;
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

// Occupancy facts of one kernel on the current device: CUs and resident
// workgroups per CU.  Queried once per (device, kernel) and cached, so a
// decode launch costs no device queries after the first.
struct Occupancy {
  int cus, per_cu;
};
Occupancy occupancy(const void* kernel, int threads) {
  struct Entry {
    int dev;
    const void* kernel;
    int threads;
    Occupancy occ;
  };
  // a fixed table (no allocation on any call): a few kernels per device
  constexpr int kEntries = 256;
  static std::mutex mu;
  static Entry cache[kEntries];
  static int used = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return {0, 0};
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < used; i++)
    if (cache[i].dev == dev && cache[i].kernel == kernel && cache[i].threads == threads)
      return cache[i].occ;
  Occupancy o = {0, 0};
  if (hipDeviceGetAttribute(&o.cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&o.per_cu, kernel, threads, 0) != hipSuccess)
    return {0, 0};
  if (used < kEntries) cache[used++] = {dev, kernel, threads, o};
  return o;
}

// Share of the first block of a split pair, in percent of the pair's tokens
// (rounded up to 16 tokens).  When the grid is exactly two resident
// workgroups on every CU, blocks u and u + grid/2 run side by side on one
// CU, and the one dispatched first finishes an equal range well before its
// partner (43 vs 61 us at 8 x 32k tokens, 8 kv heads, pd 128), which then
// runs alone on a half-empty CU.  Serving two token ranges from such a pair
// and giving the first block 62% of their tokens evens out the finish
// times.  Any other grid keeps equal ranges: there the pairing is not known
// and an uneven share would only lengthen the tail.
constexpr int kPairPct = 62;

typedef void (*PartialsFn)(DecodeParams);

// The partials instantiation for a geometry: scores of two tiles share one
// register set when ratio <= 8 (head size 256 keeps one tile per set: two
// would exceed the register file); q hi/lo parts share one B operand when
// the GQA ratio leaves 8 columns free.
template <bool PLAN>
PartialsFn partials_kernel_t(int pd, int G, int ratio) {
  const bool pack2 = ratio <= 8 && pd <= 128;
  const bool qc = ratio <= 8;
#define TQ_PICK_G(PDV, PK, QCV)                                                        \
  switch (G) {                                                                         \
    case 8: return &decode_partials_kernel<PDV, (PDV == 256 ? 4 : 8), PK, QCV, PLAN>; \
    case 4: return &decode_partials_kernel<PDV, 4, PK, QCV, PLAN>;                    \
    case 2: return &decode_partials_kernel<PDV, 2, PK, QCV, PLAN>;                    \
    default: return &decode_partials_kernel<PDV, 1, PK, QCV, PLAN>;                   \
  }
  switch (pd) {
    case 64:
      if (pack2) { TQ_PICK_G(64, 2, true) } else { TQ_PICK_G(64, 1, false) }
    case 128:
      if (pack2) { TQ_PICK_G(128, 2, true) } else { TQ_PICK_G(128, 1, false) }
    default:
      if (qc) { TQ_PICK_G(256, 1, true) } else { TQ_PICK_G(256, 1, false) }
  }
#undef TQ_PICK_G
}
PartialsFn partials_kernel(int pd, int G, int ratio, bool plan) {
  return plan ? partials_kernel_t<true>(pd, G, ratio) : partials_kernel_t<false>(pd, G, ratio);
}

// Checks shared by the partials launchers and the parameter block they fill
// (everything but the split layout).
int decode_setup(const void* q, int64_t q_stride_b, int64_t q_stride_h, const uint8_t* k_slab,
                 const uint8_t* v_slab, const int32_t* indices, const int32_t* indptr,
                 const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads,
                 int32_t num_kv_heads, int32_t padded_dim, int32_t block_size, int32_t ebs,
                 int64_t num_blocks, float sm_scale, const float* signs, float* partition_o,
                 float* partition_lse, DecodeParams& p) {
  int rc = check_geometry(padded_dim, num_qo_heads, num_kv_heads, block_size, ebs, "decode");
  if (rc) return rc;
  if (batch < 0) {
    set_error("decode: batch %d out of range", batch);
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
  const int ebs_expected = pd == 64 ? 48 : (pd == 128 ? 80 : 144);
  if (ebs != ebs_expected) {
    set_error("decode: ebs %d does not match padded_dim %d (expected %d)", ebs, pd, ebs_expected);
    return kEinval;
  }
  const int G = decode_group_size(pd, num_kv_heads, ratio);
  if (G == 0) {
    set_error("decode: no workgroup shape for %d kv heads, ratio %d", num_kv_heads, ratio);
    return kEinval;
  }
  p = DecodeParams{};
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
  p.G = G;
  p.HG = num_kv_heads / G;
  p.inv_sqrt_pd = 1.0f / sqrtf((float)pd);
  p.qk_scale = sm_scale * 1.4426950408889634f * p.inv_sqrt_pd / kCbScale;
  p.pv_scale = p.inv_sqrt_pd / kCbScale;
  return 0;
}

int launch_partials(PartialsFn fn, const DecodeParams& p, int64_t blocks, tq_stream_t stream) {
  if (blocks > 0x7fffffffLL) {
    set_error("decode: grid too large");
    return kEinval;
  }
  DecodeParams arg = p;
  void* args[] = {&arg};
  hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(fn), dim3((unsigned)blocks),
                                 dim3(64 * p.G), args, 0, reinterpret_cast<hipStream_t>(stream));
  if (e == hipSuccess) e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("decode: launch failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}

// The balanced grid for a batch: `units` work units per head group and
// whether they are served by block pairs.  The plan fills the resident
// workgroup slots once; a batch larger than that gets one unit per sequence.
struct BalancedGrid {
  int units, pair_pct;
  int64_t blocks;
  int rows;  // partial rows the plan may use
};
int balanced_grid(PartialsFn fn, const DecodeParams& p, int max_rows, BalancedGrid& g) {
  const Occupancy occ = occupancy(reinterpret_cast<const void*>(fn), 64 * p.G);
  if (occ.cus <= 0 || occ.per_cu <= 0) {
    set_error("decode: occupancy query failed");
    return kEinval;
  }
  g.pair_pct = 0;
  if (occ.per_cu == 2 && occ.cus % p.HG == 0 && occ.cus / p.HG >= p.B &&
      2 * (occ.cus / p.HG) <= max_rows) {
    g.units = occ.cus / p.HG;
    g.pair_pct = kPairPct;
    g.rows = 2 * g.units;
    g.blocks = (int64_t)2 * g.units * p.HG;
    return 0;
  }
  g.units = min(max(p.B, occ.cus * occ.per_cu / p.HG), max_rows);
  if (g.units < p.B) {
    set_error("decode: the partial workspace holds %d rows, fewer than the batch %d", max_rows,
              p.B);
    return kEinval;
  }
  g.rows = g.units;
  g.blocks = (int64_t)g.units * p.HG;
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
  if (num_splits < 1 || kv_chunk_size < 1) {
    set_error("decode: num_splits %d, kv_chunk_size %d out of range", num_splits,
              kv_chunk_size);
    return kEinval;
  }
  DecodeParams p;
  int rc = decode_setup(q, q_stride_b, q_stride_h, k_slab, v_slab, indices, indptr, seq_lens,
                        batch, num_qo_heads, num_kv_heads, padded_dim, block_size, ebs,
                        num_blocks, sm_scale, signs, partition_o, partition_lse, p);
  if (rc || batch == 0) return rc;
  p.S = num_splits;
  p.cs = kv_chunk_size;
  const int64_t blocks = (int64_t)batch * num_splits * p.HG;
  const PartialsFn fn = partials_kernel(padded_dim, p.G, p.ratio, false);
  const Occupancy occ = occupancy(reinterpret_cast<const void*>(fn), 64 * p.G);
  if (occ.per_cu == 2 && blocks == 2LL * occ.cus && num_splits % 2 == 0)
    p.pair_pct = kPairPct;
  return launch_partials(fn, p, blocks, stream);
}

namespace tq {
static int combine_splits(const float* partition_o, const float* partition_lse,
                          int32_t batch, int32_t num_splits, const int32_t* split_rows,
                          int32_t max_rows, int32_t num_qo_heads, int32_t padded_dim,
                          const float* signs, void* o, tq_stream_t stream) {
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
  _Float16* out = static_cast<_Float16*>(o);
  (void)signs;  // the partial rows come rotated back from the partials kernel
  (void)max_rows;
  dim3 grid((unsigned)blocks), block(256);
  const _Float16* prow = reinterpret_cast<const _Float16*>(partition_o);
  switch (pd) {
    case 64:
      hipLaunchKernelGGL(combine_kernel<64>, grid, block, 0, st, prow, partition_lse, num_splits,
                         split_rows, num_qo_heads, out);
      break;
    case 128:
      hipLaunchKernelGGL(combine_kernel<128>, grid, block, 0, st, prow, partition_lse, num_splits,
                         split_rows, num_qo_heads, out);
      break;
    default:
      hipLaunchKernelGGL(combine_kernel<256>, grid, block, 0, st, prow, partition_lse, num_splits,
                         split_rows, num_qo_heads, out);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("combine: launch failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}

// The partials kernel of a balanced decode alone; `rows` receives the rows
// the plan may use (for the combine's LDS sizing).
static int partials_balanced(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                             const uint8_t* k_slab, const uint8_t* v_slab,
                             const int32_t* indices, const int32_t* indptr,
                             const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads,
                             int32_t num_kv_heads, int32_t head_dim, int32_t padded_dim,
                             int32_t block_size, int32_t ebs, int64_t num_blocks, float sm_scale,
                             const float* signs, int32_t max_rows, float* partition_o,
                             float* partition_lse, int32_t* split_rows, tq_stream_t stream,
                             int* rows) {
  if (head_dim <= 0 || head_dim > padded_dim) {
    set_error("decode: head_dim %d exceeds padded_dim %d", head_dim, padded_dim);
    return kEinval;
  }
  DecodeParams p;
  int rc = decode_setup(q, q_stride_b, q_stride_h, k_slab, v_slab, indices, indptr, seq_lens,
                        batch, num_qo_heads, num_kv_heads, padded_dim, block_size, ebs,
                        num_blocks, sm_scale, signs, partition_o, partition_lse, p);
  if (rc || batch == 0) return rc;
  if (batch > kPlanMaxBatch) {
    set_error("decode: a balanced plan takes at most %d sequences, got %d", kPlanMaxBatch,
              batch);
    return kEinval;
  }
  if (!split_rows) {
    set_error("decode: null pointer");
    return kEinval;
  }
  const PartialsFn fn = partials_kernel(padded_dim, p.G, p.ratio, true);
  BalancedGrid g;
  rc = balanced_grid(fn, p, max_rows, g);
  if (rc) return rc;
  p.S = 1;
  p.cs = 1;
  p.units = g.units;
  p.pair_pct = g.pair_pct;
  p.split_out = split_rows;
  *rows = g.rows;
  return launch_partials(fn, p, g.blocks, stream);
}

// Balanced split: partials over a device-computed plan, then the combine
// over the row table the partials kernel wrote.
static int decode_balanced(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                           const uint8_t* k_slab, const uint8_t* v_slab, const int32_t* indices,
                           const int32_t* indptr, const int32_t* seq_lens, int32_t batch,
                           int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                           int32_t padded_dim, int32_t block_size, int32_t ebs,
                           int64_t num_blocks, float sm_scale, const float* signs,
                           int32_t max_rows, float* partition_o, float* partition_lse,
                           int32_t* split_rows, void* o, tq_stream_t stream) {
  if (!o) {
    set_error("decode: null pointer");
    return kEinval;
  }
  int rows = 0;
  const int rc = partials_balanced(q, q_stride_b, q_stride_h, k_slab, v_slab, indices, indptr,
                                   seq_lens, batch, num_qo_heads, num_kv_heads, head_dim,
                                   padded_dim, block_size, ebs, num_blocks, sm_scale, signs,
                                   max_rows, partition_o, partition_lse, split_rows, stream,
                                   &rows);
  if (rc || batch == 0) return rc;
  return combine_splits(partition_o, partition_lse, batch, 1, split_rows, rows,
                        num_qo_heads, padded_dim, signs, o, stream);
}

}  // namespace tq

extern "C" int tq_combine_splits(const float* partition_o, const float* partition_lse,
                                 int32_t batch, int32_t num_splits, int32_t num_qo_heads,
                                 int32_t padded_dim, const float* signs, void* o,
                                 tq_stream_t stream) {
  return tq::combine_splits(partition_o, partition_lse, batch, num_splits, nullptr, 0,
                            num_qo_heads, padded_dim, signs, o, stream);
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
  return tq::combine_splits(partition_o, partition_lse, batch, num_splits, nullptr, 0,
                            num_qo_heads, padded_dim, signs, o, stream);
}

extern "C" int tq_decode_paged_balanced(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                        const uint8_t* k_slab, const uint8_t* v_slab,
                                        const int32_t* indices, const int32_t* indptr,
                                        const int32_t* seq_lens, int32_t batch,
                                        int32_t num_qo_heads, int32_t num_kv_heads,
                                        int32_t head_dim, int32_t padded_dim,
                                        int32_t block_size, int32_t ebs, int64_t num_blocks,
                                        float sm_scale, const float* signs, int32_t max_rows,
                                        float* partition_o, float* partition_lse,
                                        int32_t* split_rows, void* o, tq_stream_t stream) {
  return tq::decode_balanced(q, q_stride_b, q_stride_h, k_slab, v_slab, indices, indptr,
                             seq_lens, batch, num_qo_heads, num_kv_heads, head_dim, padded_dim,
                             block_size, ebs, num_blocks, sm_scale, signs, max_rows,
                             partition_o, partition_lse, split_rows, o, stream);
}

namespace tq {
namespace {

// Workspace of tq_decode_paged_balanced_noalloc: the row table, the partial
// LSEs and the partial rows of one call, in a file-scope device array (one
// copy per GPU, held until the process ends).  In host code `scratch` names
// a host-side stand-in, never the device memory: host code uses only the
// per-device address from hipGetSymbolAddress.
constexpr size_t kScratchBytes = size_t(16) << 20;
__device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
int scratch_ptr(uint8_t** out) {
  static std::mutex mu;
  static uint8_t* ptrs[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("decode_noalloc: no usable current device");
    return e != hipSuccess ? (int)e : kEinval;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      set_error("decode_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                hipGetErrorString(e));
      return e != hipSuccess ? (int)e : kEinval;
    }
    ptrs[dev] = static_cast<uint8_t*>(ptr);
  }
  *out = ptrs[dev];
  return 0;
}

constexpr size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

}  // namespace
}  // namespace tq

extern "C" int tq_decode_paged_balanced_noalloc(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const uint8_t* k_slab,
    const uint8_t* v_slab, const int32_t* indices, const int32_t* indptr,
    const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t padded_dim, int32_t block_size, int32_t ebs, int64_t num_blocks,
    float sm_scale, const float* signs, void* o, tq_stream_t stream) {
  using namespace tq;
  if (batch < 0 || batch > kPlanMaxBatch || num_qo_heads <= 0 ||
      (padded_dim != 64 && padded_dim != 128 && padded_dim != 256)) {
    set_error("decode_noalloc: batch %d, num_qo_heads %d, padded_dim %d out of range", batch,
              num_qo_heads, padded_dim);
    return kEinval;
  }
  if (batch == 0) return 0;
  uint8_t* base = nullptr;
  int rc = scratch_ptr(&base);
  if (rc) return rc;
  // [row table: batch + 2 int32][lse: rows x Hq f32][partials: rows x Hq x pd f32]
  const size_t table = align256((size_t)(batch + 2) * 4);
  const size_t per_row = (size_t)num_qo_heads * 4 * (1 + (size_t)padded_dim);
  const size_t avail = kScratchBytes - table - 256;
  const int64_t fit = (int64_t)(avail / per_row);
  if (fit < batch) {
    set_error("decode_noalloc: %d sequences x %d heads x pd %d need %zu bytes of partials, "
              "more than the %zu-byte scratch (use tq_decode_paged_balanced with a workspace)",
              batch, num_qo_heads, padded_dim, (size_t)batch * per_row + table, kScratchBytes);
    return kEinval;
  }
  const int rows = (int)(fit < 0x7fffffff ? fit : 0x7fffffff);
  int32_t* split_rows = reinterpret_cast<int32_t*>(base);
  float* plse = reinterpret_cast<float*>(base + table);
  float* po = reinterpret_cast<float*>(base + table +
                                       align256((size_t)rows * num_qo_heads * 4));
  return tq::decode_balanced(q, q_stride_b, q_stride_h, k_slab, v_slab, indices, indptr,
                             seq_lens, batch, num_qo_heads, num_kv_heads, head_dim, padded_dim,
                             block_size, ebs, num_blocks, sm_scale, signs, rows, po, plse,
                             split_rows, o, stream);
}

// Diagnostic: the configs[2] partials kernel (head size 128, 8 kv heads per
// workgroup, static splits) with the step math compiled out: the same
// prologue, page walk, copy ring, waits, barriers and slot reads, zero
// partial rows.  Its time is what the data movement alone costs.
extern "C" int tq_diag_decode_stream(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                     const uint8_t* k_slab, const uint8_t* v_slab,
                                     const int32_t* indices, const int32_t* indptr,
                                     const int32_t* seq_lens, int32_t batch,
                                     int32_t num_qo_heads, int32_t num_kv_heads,
                                     int32_t padded_dim, int32_t block_size, int32_t ebs,
                                     int64_t num_blocks, float sm_scale, const float* signs,
                                     int32_t num_splits, int32_t kv_chunk_size,
                                     float* partition_o, float* partition_lse, int32_t mode,
                                     tq_stream_t stream) {
  using namespace tq;
  if (mode != 0 && mode != 1) {
    set_error("diag_decode_stream: mode %d is neither 0 (bare ring) nor 1 (no math)", mode);
    return kEinval;
  }
  if (num_splits < 1 || kv_chunk_size < 1) {
    set_error("diag_decode_stream: num_splits %d, kv_chunk_size %d out of range", num_splits,
              kv_chunk_size);
    return kEinval;
  }
  DecodeParams p;
  int rc = decode_setup(q, q_stride_b, q_stride_h, k_slab, v_slab, indices, indptr, seq_lens,
                        batch, num_qo_heads, num_kv_heads, padded_dim, block_size, ebs,
                        num_blocks, sm_scale, signs, partition_o, partition_lse, p);
  if (rc || batch == 0) return rc;
  if (padded_dim != 128 || p.G != 8 || p.ratio > 8) {
    set_error("diag_decode_stream: built for head size 128, 8 kv heads per workgroup, GQA "
              "ratio <= 8 only");
    return kEinval;
  }
  p.S = num_splits;
  p.cs = kv_chunk_size;
  const int64_t blocks = (int64_t)batch * num_splits * p.HG;
  const PartialsFn fn = mode == 0 ? &decode_partials_kernel<128, 8, 2, true, false, 0>
                                  : &decode_partials_kernel<128, 8, 2, true, false, 1>;
  const Occupancy occ = occupancy(reinterpret_cast<const void*>(fn), 64 * p.G);
  if (occ.per_cu == 2 && blocks == 2LL * occ.cus && num_splits % 2 == 0)
    p.pair_pct = kPairPct;
  return launch_partials(fn, p, blocks, stream);
}

namespace tq {
namespace {
// Streaming read of n 16-byte words with non-temporal loads, four per lane in
// flight per iteration, grid-strided; a lane stores the xor of the words it
// read only if it equals one constant, which keeps the loads.
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ src,
                                                          int64_t n, uint32_t* sink) {
  uint32_t acc = 0;
  const int64_t stride = (int64_t)gridDim.x * 1024;
  for (int64_t i = (int64_t)blockIdx.x * 1024 + threadIdx.x; i < n; i += stride) {
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; u++)
      v[u] = i + 256 * u < n ? __builtin_nontemporal_load(src + i + 256 * u) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < 4; u++) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  if (acc == 0x7e57c0deu) sink[0] = acc;
}
}  // namespace
}  // namespace tq

// Diagnostic: the HBM read rate a plain stream reaches (no page table, no
// LDS, no barriers), the reference point for the copy ring above.
extern "C" int tq_diag_stream_read(const void* src, int64_t bytes, uint32_t* sink,
                                   tq_stream_t stream) {
  using namespace tq;
  if (!src || !sink || bytes < 0 || bytes % 16 != 0 || ((uintptr_t)src & 15)) {
    set_error("diag_stream_read: need a 16-byte aligned source of a multiple of 16 bytes");
    return kEinval;
  }
  if (bytes == 0) return 0;
  hipLaunchKernelGGL(stream_read_kernel, dim3(2048), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const u32x4*>(src),
                     bytes / 16, sink);
  return (int)hipGetLastError();
}

extern "C" int tq_decode_partials_balanced(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const uint8_t* k_slab,
    const uint8_t* v_slab, const int32_t* indices, const int32_t* indptr,
    const int32_t* seq_lens, int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t padded_dim, int32_t block_size, int32_t ebs, int64_t num_blocks,
    float sm_scale, const float* signs, int32_t max_rows, float* partition_o,
    float* partition_lse, int32_t* split_rows, tq_stream_t stream) {
  int rows = 0;
  return tq::partials_balanced(q, q_stride_b, q_stride_h, k_slab, v_slab, indices, indptr,
                               seq_lens, batch, num_qo_heads, num_kv_heads, head_dim,
                               padded_dim, block_size, ebs, num_blocks, sm_scale, signs,
                               max_rows, partition_o, partition_lse, split_rows, stream, &rows);
}

extern "C" int tq_decode_balanced_rows(int32_t batch, int32_t num_qo_heads,
                                       int32_t num_kv_heads, int32_t padded_dim) {
  using namespace tq;
  const int ratio = num_kv_heads > 0 ? num_qo_heads / num_kv_heads : 0;
  const int G = num_kv_heads > 0 && num_qo_heads % num_kv_heads == 0 && ratio <= 16 &&
                        (padded_dim == 64 || padded_dim == 128 || padded_dim == 256)
                    ? decode_group_size(padded_dim, num_kv_heads, ratio)
                    : 0;
  if (G == 0 || batch < 0) {
    set_error("decode_balanced_rows: unsupported geometry");
    return kEinval;
  }
  const PartialsFn fn = partials_kernel(padded_dim, G, ratio, true);
  const Occupancy occ = occupancy(reinterpret_cast<const void*>(fn), 64 * G);
  if (occ.cus <= 0 || occ.per_cu <= 0) {
    set_error("decode_balanced_rows: occupancy query failed");
    return kEinval;
  }
  const int hg = num_kv_heads / G;
  return max(max(batch, occ.cus * occ.per_cu / hg), 2 * (occ.cus / hg));
}
