// tq_write.hip -- quantize-and-scatter of K/V rows into the packed paged cache.
//
// Same numbers as the reference scatter kernel
// (csrc/include/turboquant/quantize_write_kernel.cuh:332-431), which gives
// every vector 32 lanes of VEC = pd/32 consecutive dims: the fp32 sum of
// squares, its reduction tree, sqrt, reciprocal, sign flip, FWHT butterflies
// and the 1/sqrt(pd) scale happen in the same order and give the same bits.
// MI355X layout: 16 lanes per vector, each holding the dims of two of the
// reference's lanes (p and p + 16), so a wave64 carries four vectors and the
// per-vector work (index math, reduction, sqrt, divide, norm store) is
// shared by twice the dims; a 256-thread workgroup writes 16 consecutive
// (token, head) entries, i.e. whole cache rows.  One launch covers K and V.
#include <stdarg.h>
#include <stdio.h>

#include <type_traits>

#include <atomic>

#include "tq_common.h"

namespace tq {

namespace {

// Load VEC consecutive input elements as fp32 (exact for fp16/bf16).
template <int VEC>
__device__ __forceinline__ void load_row(const void* base, int64_t off, int dtype,
                                         int d0, int head_dim, bool vec_ok, float* x) {
  if (dtype == TQ_F16) {
    const _Float16* p = reinterpret_cast<const _Float16*>(base) + off + d0;
    if (vec_ok) {
      if constexpr (VEC == 2) {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        h2 v = *reinterpret_cast<const h2*>(p);
        x[0] = (float)v[0]; x[1] = (float)v[1];
      } else if constexpr (VEC == 4) {
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        h4 v = *reinterpret_cast<const h4*>(p);
#pragma unroll
        for (int i = 0; i < 4; i++) x[i] = (float)v[i];
      } else {
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        h8 v = *reinterpret_cast<const h8*>(p);
#pragma unroll
        for (int i = 0; i < 8; i++) x[i] = (float)v[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < VEC; i++) x[i] = (d0 + i < head_dim) ? (float)p[i] : 0.0f;
    }
  } else if (dtype == TQ_BF16) {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(base) + off + d0;
#pragma unroll
    for (int i = 0; i < VEC; i++)
      x[i] = (d0 + i < head_dim) ? __uint_as_float((uint32_t)p[i] << 16) : 0.0f;
  } else {
    const float* p = reinterpret_cast<const float*>(base) + off + d0;
#pragma unroll
    for (int i = 0; i < VEC; i++) x[i] = (d0 + i < head_dim) ? p[i] : 0.0f;
  }
}

// code = #{j : v >= b_j} over the 15 boundaries b_j = boundary_j * scale.
// The boundaries are symmetric with b_7 = 0, so for v >= 0 (this includes
// -0.0, as in the reference's `val >= b[mid]`) the code is 8 + #{k : v >= B_k},
// and for v < 0 or NaN it is 7 - #{k : |v| > B_k}, B_k = b_{7+k}.  On positive
// floats "a > B" is "bits(a) - 1 >= bits(B)" as integers, so one integer
// compare chain serves both sides.  Same result as the binary search of
// quantize_write_kernel.cuh:34-46 for every fp32 input.
__device__ __forceinline__ uint32_t bucketize(float v, const int32_t* bbits) {
  const bool pos = v >= 0.0f;
  int32_t a = (int32_t)(__float_as_uint(v) & 0x7fffffffu) - (pos ? 0 : 1);
  uint32_t k = 0;
#pragma unroll
  for (int j = 0; j < 7; j++) k += (a >= bbits[j]) ? 1u : 0u;
  return pos ? 8u + k : 7u - k;
}

// fp16 value in the low / high half of a dword, as fp32 (exact)
__device__ __forceinline__ float lo_half_f(uint32_t v) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu));
}
__device__ __forceinline__ float hi_half_f(uint32_t v) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
}

// Value of lane (lane ^ D) within each 32-lane half, without the LDS
// crossbar: DPP quad permutes for D = 1, 2, two masked row shifts for D = 4,
// a row rotate for D = 8 and the row swap of v_permlane16_swap for D = 16.
template <int D>
__device__ __forceinline__ float xor_lane(float x) {
  const int xi = __float_as_int(x);
  if constexpr (D == 1) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(xi, 0xb1, 0xf, 0xf, false));  // [1,0,3,2]
  } else if constexpr (D == 2) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(xi, 0x4e, 0xf, 0xf, false));  // [2,3,0,1]
  } else if constexpr (D == 4) {
    // banks 0, 2 (lanes 0-3, 8-11 of a row) take lane + 4; banks 1, 3 take lane - 4
    int r = __builtin_amdgcn_update_dpp(xi, xi, 0x104, 0xf, 0x5, false);  // row_shl:4
    r = __builtin_amdgcn_update_dpp(r, xi, 0x114, 0xf, 0xa, false);       // row_shr:4
    return __int_as_float(r);
  } else if constexpr (D == 8) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(xi, 0x128, 0xf, 0xf, false));  // row_ror:8
  } else {
    static_assert(D == 16, "xor distance");
    const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)xi, (uint32_t)xi, false, false);
    const bool odd_row = (threadIdx.x & 16) != 0;
    return __uint_as_float(odd_row ? r[0] : r[1]);
  }
}

// Quantize-and-scatter: 16 lanes per vector, 4 vectors per wave64, 16
// consecutive vectors (kv, token, head; head fastest, so the entries of one
// token's heads are written together) per 256-thread workgroup.  Physical
// lane p of a vector holds the dims of two lanes of the reference's 32-lane
// layout (quantize_write_kernel.cuh:332-431): lane p (dims VEC p .. +VEC) in
// x0 and lane p + 16 in x1.  The arithmetic is the reference's, in its
// order: per-lane FMA sums, the shfl_down tree 16, 8, 4, 2, 1 (its first
// level pairs x0 and x1 of one physical lane), IEEE sqrt and reciprocal,
// sign flip, FWHT stages h = 1 .. pd/2 in ascending order (the last one,
// between lanes p and p + 16, again inside one physical lane), 1/sqrt(pd),
// bucketize, pack.
template <int PD, bool VEC_OK>
__global__ __launch_bounds__(256) void write_kernel(
    uint8_t* __restrict__ k_slab, uint8_t* __restrict__ v_slab,
    const void* __restrict__ key, const void* __restrict__ value, int dtype,
    int64_t k_st, int64_t k_sh, int64_t v_st, int64_t v_sh,
    const float* __restrict__ signs, const int32_t* __restrict__ slots,
    uint32_t per_kv, int H, uint32_t hmul, int head_dim, int ebs, int64_t nslots,
    float scale) {
#pragma clang fp contract(off)
  constexpr int VEC = PD / 32;
  const int lane = threadIdx.x & 15;
  const uint32_t g = blockIdx.x * 16u + (threadIdx.x >> 4);
  if (g >= 2 * per_kv) return;  // a whole 16-lane group (one DPP row) leaves
  const int kv = g >= per_kv ? 1 : 0;
  const uint32_t rem = g - (kv ? per_kv : 0u);
  // t = rem / H by multiply-high (hmul = ceil(2^32 / H), exact for rem < 2^32 / H)
  const uint32_t t = H == 1 ? rem : __umulhi(rem, hmul);
  const int h = (int)(rem - t * (uint32_t)H);

  float x0[VEC], x1[VEC];
  const int da = lane * VEC, db = (lane + 16) * VEC;
  if (kv == 0) {
    load_row<VEC>(key, (int64_t)t * k_st + h * k_sh, dtype, da, head_dim, VEC_OK, x0);
    load_row<VEC>(key, (int64_t)t * k_st + h * k_sh, dtype, db, head_dim, VEC_OK, x1);
  } else {
    load_row<VEC>(value, (int64_t)t * v_st + h * v_sh, dtype, da, head_dim, VEC_OK, x0);
    load_row<VEC>(value, (int64_t)t * v_st + h * v_sh, dtype, db, head_dim, VEC_OK, x1);
  }
  const int32_t slot = slots[t];
  if (slot < 0 || (int64_t)slot >= nslots) return;  // whole 16-lane group together

  // 1. per-lane sums of squares, FMA-accumulated in dim order
  float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
  for (int i = 0; i < VEC; i++) {
    s0 = __builtin_fmaf(x0[i], x0[i], s0);
    s1 = __builtin_fmaf(x1[i], x1[i], s1);
  }
  // 2. the tree: level 16 in-lane, then 8, 4, 2, 1 across the 16 lanes;
  //    every lane ends with the bits the reference's lane 0 holds
  float ss = s0 + s1;
  ss = ss + xor_lane<8>(ss);
  ss = ss + xor_lane<4>(ss);
  ss = ss + xor_lane<2>(ss);
  ss = ss + xor_lane<1>(ss);
  // 3. IEEE sqrt and reciprocal
  const float l2 = __builtin_sqrtf(ss);
  const float inv = (l2 > 1e-8f) ? (1.0f / l2) : 0.0f;
  // 4. normalise, flip signs
#pragma unroll
  for (int i = 0; i < VEC; i++) {
    x0[i] = x0[i] * inv;
    x1[i] = x1[i] * inv;
  }
#pragma unroll
  for (int i = 0; i < VEC; i++) {
    x0[i] = x0[i] * signs[da + i];
    x1[i] = x1[i] * signs[db + i];
  }
  // 5. FWHT: in-lane stages h < VEC, cross-lane stages (lane xor 1..8), then
  //    the stage between lanes p and p + 16
#pragma unroll
  for (int hh = 1; hh < VEC; hh <<= 1) {
#pragma unroll
    for (int i = 0; i < VEC; i += 2 * hh) {
#pragma unroll
      for (int k = 0; k < hh; k++) {
        float a = x0[i + k], b = x0[i + k + hh];
        x0[i + k] = a + b;
        x0[i + k + hh] = a - b;
        a = x1[i + k];
        b = x1[i + k + hh];
        x1[i + k] = a + b;
        x1[i + k + hh] = a - b;
      }
    }
  }
  // butterfly partner + sign * own value: fma(+-1, v, p) rounds once, to the
  // same bits as v + p (lower lane) or p - v (upper lane)
  auto cross = [&](auto dist) {
    constexpr int D = decltype(dist)::value;
    const float sg = (lane & D) ? -1.0f : 1.0f;
#pragma unroll
    for (int i = 0; i < VEC; i++) {
      x0[i] = __builtin_fmaf(sg, x0[i], xor_lane<D>(x0[i]));
      x1[i] = __builtin_fmaf(sg, x1[i], xor_lane<D>(x1[i]));
    }
  };
  cross(std::integral_constant<int, 1>{});
  cross(std::integral_constant<int, 2>{});
  cross(std::integral_constant<int, 4>{});
  cross(std::integral_constant<int, 8>{});
#pragma unroll
  for (int i = 0; i < VEC; i++) {
    const float a = x0[i], b = x1[i];
    x0[i] = (a + b) * scale;
    x1[i] = (a - b) * scale;
  }

  // 6. bucketize against b_j * scale (fp32 products, as the reference forms them)
  int32_t bbits[7];
#pragma unroll
  for (int j = 0; j < 7; j++) bbits[j] = (int32_t)__float_as_uint(boundary_pos(j + 1) * scale);

  uint8_t* entry = (kv == 0 ? k_slab : v_slab) +
                   ((int64_t)slot * H + h) * (int64_t)ebs;  // slot*H == (block*bs+entry)*H
  // 7. pack: byte k = code[2k] << 4 | code[2k+1]
  uint32_t p0 = 0, p1 = 0;
#pragma unroll
  for (int i = 0; i < VEC; i += 2) {
    p0 |= ((bucketize(x0[i], bbits) << 4) | bucketize(x0[i + 1], bbits)) << (4 * i);
    p1 |= ((bucketize(x1[i], bbits) << 4) | bucketize(x1[i + 1], bbits)) << (4 * i);
  }
  uint8_t* d0p = entry + lane * (VEC / 2);
  uint8_t* d1p = entry + (lane + 16) * (VEC / 2);
  if constexpr (VEC == 2) {
    *d0p = (uint8_t)p0;
    *d1p = (uint8_t)p1;
  } else if constexpr (VEC == 4) {
    *reinterpret_cast<uint16_t*>(d0p) = (uint16_t)p0;
    *reinterpret_cast<uint16_t*>(d1p) = (uint16_t)p1;
  } else {
    *reinterpret_cast<uint32_t*>(d0p) = p0;
    *reinterpret_cast<uint32_t*>(d1p) = p1;
  }
  // 8. fp16(l2), round to nearest even, repeated pd/64 times after the codes
  if (lane == 0) {
    _Float16 nh = (_Float16)l2;
    uint32_t nb = (uint32_t)__builtin_bit_cast(uint16_t, nh);
    uint8_t* np = entry + PD / 2;
    if constexpr (PD == 64) {
      *reinterpret_cast<uint16_t*>(np) = (uint16_t)nb;
    } else if constexpr (PD == 128) {
      *reinterpret_cast<uint32_t*>(np) = nb | (nb << 16);
    } else {
      uint2 w;
      w.x = nb | (nb << 16);
      w.y = w.x;
      *reinterpret_cast<uint2*>(np) = w;
    }
  }
}

// ---------------------------------------------------------------------------
// fp16 fast path: 32 dims per lane, P = PD/32 lanes per vector.
//
// Lane p of a vector holds the 16-byte chunks j = p + P*i (i = 0..3), i.e.
// dims d = 8j + c (c = 0..7): bits 0-2 of d are in-lane, the next log2(P)
// bits pick the lane, the top two bits are in-lane again.  The reference's
// lane t holds dims [t*VEC, (t+1)*VEC) with VEC = PD/32, so this lane holds
// the reference lanes t = 8i + E*p + e (E = 8/VEC, e < E).  Both orders the
// reference fixes come out unchanged:
//  * sum-of-squares tree (shfl_down 16, 8, 4, 2, 1): levels 16 and 8 pair i
//    and i + 2, i and i + 1 (in-lane); levels 4, 2, 1 pair the low three
//    bits of t, which are lane bits (xor across lanes) from E up and in-lane
//    below, in the reference's level order;
//  * FWHT stages h = 1, 2, 4 (in-lane), h = 8 .. 4P (lane xor h/8), h = 8P
//    and 16P (in-lane), ascending.
// Every butterfly and every tree node is the same fp32 operation on the same
// two operands as in the reference (fp32 addition is commutative, negation
// is exact), so the bits are the same; only the lane that computes it and
// the sign it is held with differ.
//
// Instruction savings over the generic kernel:
//  * the sign flip is an XOR of the fp16 sign bits before conversion, and
//    the normalisation reads the fp16 value directly (v_fma_mix with a -0
//    addend, i.e. the exact product): (x*s)*inv == (x*inv)*s for s = +-1;
//  * a cross-lane butterfly is one fma with a DPP operand: lane l keeps
//    z_l + sg_l * z_partner (sg = -1 on the upper lane), which is the
//    reference's value times tau_l = +-1.  Negation commutes with the later
//    in-lane butterflies, so every lane ends with tau_l = (-1)^popcount(lane
//    bits) times the reference's values and folds tau_l into the 1/sqrt(pd)
//    scale, an fma with a +0 addend that also turns -0 into +0 (both give
//    code 8, as the reference's `val >= 0` does);
//  * bucketize is one LDS lookup: |v| (as ordered integer bits, minus one
//    for negative v so that `>=` becomes the reference's `>` on that side)
//    is clamped to the four binades that hold the seven positive
//    boundaries, and its exponent's low three bits plus its top three
//    mantissa bits index a 64-entry table of (boundary inside this
//    1/8-binade bin or none, 8 + boundaries below the bin).  Each bin holds
//    at most one boundary (the tests check this for every head size), so
//    code = (8 + below + (|v| >= boundary)) for v >= 0 and its 4-bit
//    complement for v < 0.
//  * vectors whose sum of squares is not finite (an inf or NaN input) give
//    NaN everywhere after the FWHT, i.e. code 0, as in the reference.
template <int PD>
struct FastGeom {
  // 16-byte chunks (8 dims) per lane: 4, and 2 at pd 64, where 4 would leave
  // a launch half the waves (measured 8.3 against 8.6 us for 8192 tokens x 8
  // heads; 1 chunk per lane: 9.7 us; 8 chunks per lane at pd 256: the same
  // as 4; 2 chunks per lane at pd 128: 15.7 against 14.5 us)
  static constexpr int CPL = PD == 64 ? 2 : 4;
  static constexpr int P = PD / (8 * CPL);     // lanes per vector (4, 4, 8)
  static constexpr int VEC = PD / 32;          // dims per reference lane
  static constexpr int E = 8 / VEC;            // reference lanes per chunk
  static constexpr int PE = P * E;             // reference lanes per chunk row (32 / CPL)
  static constexpr int VPW = 64 / P;           // vectors per wave
  static constexpr int VPB = 4 * VPW;          // vectors per 256-thread workgroup
};

// min(max(x, lo), hi) (unsigned) in one instruction
__device__ __forceinline__ uint32_t med3_u32(uint32_t x, uint32_t lo, uint32_t hi) {
  uint32_t r;
#if defined(__HIP_DEVICE_COMPILE__)
  asm("v_med3_u32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(lo), "v"(hi));
#else
  r = x < lo ? lo : (x > hi ? hi : x);
#endif
  return r;
}

// value of lane (lane ^ D), D in {1, 2}, as a DPP quad permute that the
// compiler can fold into the instruction using it
template <int D>
__device__ __forceinline__ float qxor(float x) {
  static_assert(D == 1 || D == 2, "quad distance");
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), D == 1 ? 0xb1 : 0x4e,
                                                    0xf, 0xf, true));
}
template <int D>
__device__ __forceinline__ float xor8(float x) {
  if constexpr (D <= 2) return qxor<D>(x);
  else return xor_lane<D>(x);
}

// x[k] += sg * x[k] of lane (lane ^ D), D in {1, 2}, for 8 registers: one
// v_fmac_f32 with a DPP quad-permuted operand each (one rounding, the same
// bits as x + partner or x - partner).  The leading s_nop covers the wait
// states a DPP read needs after a VALU write of its source.
template <int D>
__device__ __forceinline__ void fmac_qxor8(float* x, float sg) {
#if defined(__HIP_DEVICE_COMPILE__)
#define TQ_Q(I) "v_fmac_f32_dpp %" #I ", %" #I ", %8 quad_perm:" QP " row_mask:0xf bank_mask:0xf\n\t"
#define QP (D == 1 ? "[1,0,3,2]" : "[2,3,0,1]")
  if constexpr (D == 1) {
#undef QP
#define QP "[1,0,3,2]"
    asm volatile("s_nop 1\n\t" TQ_Q(0) TQ_Q(1) TQ_Q(2) TQ_Q(3) TQ_Q(4) TQ_Q(5) TQ_Q(6) TQ_Q(7)
                 : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]),
                   "+v"(x[6]), "+v"(x[7])
                 : "v"(sg));
  } else {
#undef QP
#define QP "[2,3,0,1]"
    asm volatile("s_nop 1\n\t" TQ_Q(0) TQ_Q(1) TQ_Q(2) TQ_Q(3) TQ_Q(4) TQ_Q(5) TQ_Q(6) TQ_Q(7)
                 : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]),
                   "+v"(x[6]), "+v"(x[7])
                 : "v"(sg));
  }
#undef QP
#undef TQ_Q
#else
  (void)x;
  (void)sg;
#endif
}

// r + r of lane (lane ^ D), D in {1, 2}: one v_add_f32 with a DPP operand
template <int D>
__device__ __forceinline__ float add_qxor(float r) {
#if defined(__HIP_DEVICE_COMPILE__)
  if constexpr (D == 1)
    asm volatile("s_nop 1\n\tv_add_f32_dpp %0, %0, %0 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf"
                 : "+v"(r));
  else
    asm volatile("s_nop 1\n\tv_add_f32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf"
                 : "+v"(r));
#endif
  return r;
}

template <int PD>
__global__ __launch_bounds__(256) void write_f16_kernel(
    uint8_t* __restrict__ k_slab, uint8_t* __restrict__ v_slab,
    const _Float16* __restrict__ key, const _Float16* __restrict__ value,
    int64_t k_st, int64_t k_sh, int64_t v_st, int64_t v_sh,
    const float* __restrict__ signs, const int32_t* __restrict__ slots,
    uint32_t per_kv, int H, uint32_t hmul, int ebs, int64_t nslots, float scale) {
#pragma clang fp contract(off)
  using FG = FastGeom<PD>;
  constexpr int P = FG::P, E = FG::E, VEC = FG::VEC, CPL = FG::CPL, PE = FG::PE;
  constexpr int ND = 8 * CPL;  // dims per lane
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(512))) uint32_t tbl[128];  // 64 x (2 * boundary, 8 + below)

  const int lane = threadIdx.x & 63;
  const int p = lane % P;
  const uint32_t g = blockIdx.x * (uint32_t)FG::VPB + (threadIdx.x >> 6) * FG::VPW + lane / P;
  const bool live = g < 2 * per_kv;

  // this vector's row: CPL chunks j = p + P*i, issued first (zeros past the end)
  const int kv = g >= per_kv ? 1 : 0;
  const uint32_t rem = g - (kv ? per_kv : 0u);
  const uint32_t t = H == 1 ? rem : __umulhi(rem, hmul);  // rem / H, exact (hmul = ceil(2^32/H))
  const int h = (int)(rem - t * (uint32_t)H);
  // lanes past the end read row 0 of K (no branch, no zero fill); they
  // store nothing (slot -1)
  u32x4 raw[CPL];
  const _Float16* row = !live ? key
                        : kv  ? value + (int64_t)t * v_st + (int64_t)h * v_sh
                              : key + (int64_t)t * k_st + (int64_t)h * k_sh;
#pragma unroll
  for (int i = 0; i < CPL; i++) raw[i] = *reinterpret_cast<const u32x4*>(row + 8 * (p + P * i));
  const int32_t slot = live ? slots[t] : -1;

  // boundaries b_k * scale (k = 1..7) as integer bits (positive floats order
  // as their bits); bin table over the four binades from the smallest one
  int32_t T[7];
#pragma unroll
  for (int k = 0; k < 7; k++) T[k] = (int32_t)__float_as_uint(boundary_pos(k + 1) * scale);
  const int32_t e0 = T[0] >> 23;
  const uint32_t lo2 = (uint32_t)e0 << 24;                // 2 * 2^e0 as bits
  const uint32_t hi2 = ((uint32_t)(e0 + 4) << 24) - 1u;   // just below 2 * 2^(e0 + 4)
  if (threadIdx.x < 64) {
    const int idx = threadIdx.x;
    const int e = e0 + (((idx >> 3) - e0) & 7);  // the exponent with these low bits
    uint32_t thr2 = 0xffffffffu, below = 8;
    if (e <= e0 + 3) {
      const int32_t start = (e << 23) | ((idx & 7) << 20), end = start + (1 << 20);
#pragma unroll
      for (int k = 0; k < 7; k++) {
        below += T[k] < start ? 1u : 0u;
        if (T[k] >= start && T[k] < end) thr2 = 2u * (uint32_t)T[k];
      }
    }
    tbl[2 * idx] = thr2;
    tbl[2 * idx + 1] = below;
  }

  // signed fp16 inputs: the sign bits of this lane's signs (+-1) flipped into
  // the halves (the top bytes of two floats go to bytes 1 and 3, then the
  // sign bits are kept)
  uint32_t hw[CPL][4];
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    const float4* sp = reinterpret_cast<const float4*>(signs + 8 * (p + P * i));
    const float4 s0 = sp[0], s1 = sp[1];
    const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const uint32_t sm = __builtin_amdgcn_perm(__float_as_uint(sv[2 * c + 1]),
                                                __float_as_uint(sv[2 * c]), 0x070c030cu);
      hw[i][c] = raw[i][c] ^ (sm & 0x80008000u);
    }
  }
  auto hv = [&](int i, int c) -> float {  // signed input dim 8j + c as fp32 (exact)
    return c & 1 ? hi_half_f(hw[i][c / 2]) : lo_half_f(hw[i][c / 2]);
  };

  // 1. per-reference-lane sums of squares, FMA in dim order
  float r[E];
  {
    float a[CPL][E];
#pragma unroll
    for (int i = 0; i < CPL; i++)
#pragma unroll
      for (int e = 0; e < E; e++) {
        float sacc = 0.0f;
#pragma unroll
        for (int c = 0; c < VEC; c++) {
          const float xv = hv(i, e * VEC + c);
          sacc = __builtin_fmaf(xv, xv, sacc);
        }
        a[i][e] = sacc;
      }
    // 2. the tree, levels 16 .. PE pair chunk rows i and i + L / PE (in-lane)
#pragma unroll
    for (int L = 16; L >= PE; L >>= 1)
#pragma unroll
      for (int i = 0; i < L / PE; i++)
#pragma unroll
        for (int e = 0; e < E; e++) a[i][e] = a[i][e] + a[i + L / PE][e];
#pragma unroll
    for (int e = 0; e < E; e++) r[e] = a[0][e];
  }
  // levels below PE: lane bits (xor across the vector's lanes) from E up,
  // in-lane below
  auto level = [&](auto lv) {
    constexpr int L = decltype(lv)::value;
    if constexpr (L < PE) {
      if constexpr (L >= E) {
#pragma unroll
        for (int e = 0; e < E; e++) {
          if constexpr (L / E <= 2) r[e] = add_qxor<L / E>(r[e]);
          else r[e] = r[e] + xor8<L / E>(r[e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < L; e++) r[e] = r[e] + r[e + L];
      }
    }
  };
  level(std::integral_constant<int, 16>{});
  level(std::integral_constant<int, 8>{});
  level(std::integral_constant<int, 4>{});
  level(std::integral_constant<int, 2>{});
  level(std::integral_constant<int, 1>{});
  const float ss = r[0];
  // 3. IEEE sqrt and reciprocal; normalise (exact products of the fp16 inputs)
  const float l2 = __builtin_sqrtf(ss);
  const float inv = (l2 > 1e-8f) ? (1.0f / l2) : 0.0f;
  const bool finite = ss <= 3.402823466e38f;  // false for inf and NaN
  float x[ND];  // x[8i + c] = dim 8(p + P i) + c, times tau
#pragma unroll
  for (int i = 0; i < CPL; i++)
#pragma unroll
    for (int c = 0; c < 8; c++) x[8 * i + c] = __builtin_fmaf(hv(i, c), inv, 0.0f);
  // 4. FWHT, ascending h: dim bits 0-2 in-lane, then the lane bits, then the
  //    chunk-row bits in-lane
#pragma unroll
  for (int hh = 1; hh < 8; hh <<= 1)
#pragma unroll
    for (int i = 0; i < CPL; i++)
#pragma unroll
      for (int c = 0; c < 8; c++)
        if (!(c & hh)) {
          const float u = x[8 * i + c], w = x[8 * i + c + hh];
          x[8 * i + c] = u + w;
          x[8 * i + c + hh] = u - w;
        }
  if constexpr (P >= 2) {
    const float sg = (lane & 1) ? -1.0f : 1.0f;
#pragma unroll
    for (int k = 0; k < ND; k += 8) fmac_qxor8<1>(x + k, sg);
  }
  if constexpr (P >= 4) {
    const float sg = (lane & 2) ? -1.0f : 1.0f;
#pragma unroll
    for (int k = 0; k < ND; k += 8) fmac_qxor8<2>(x + k, sg);
  }
  if constexpr (P >= 8) {
    const float sg = (lane & 4) ? -1.0f : 1.0f;
#pragma unroll
    for (int k = 0; k < ND; k++) x[k] = __builtin_fmaf(xor8<4>(x[k]), sg, x[k]);
  }
#pragma unroll
  for (int hi2 = 1; hi2 < CPL; hi2 <<= 1)
#pragma unroll
    for (int i = 0; i < CPL; i++)
      if (!(i & hi2))
#pragma unroll
        for (int c = 0; c < 8; c++) {
          const float u = x[8 * i + c], w = x[8 * (i + hi2) + c];
          x[8 * i + c] = u + w;
          x[8 * (i + hi2) + c] = u - w;
        }
  // 5. scale (with tau), bucketize through the bin table, pack
  const float ts = (__builtin_popcount(lane & (P - 1)) & 1) ? -scale : scale;
  __syncthreads();  // bin table ready
  uint32_t packed[CPL];
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    uint32_t wd = 0;
#pragma unroll
    for (int c = 0; c < 8; c++) {
      const uint32_t bits = __float_as_uint(__builtin_fmaf(x[8 * i + c], ts, 0.0f));
      const uint32_t m = (uint32_t)((int32_t)bits >> 31);  // all ones for v < 0
      // 2|v| as an unsigned integer (the sign bit shifts out), minus 2 if v < 0
      const uint32_t av2 = (bits + m) << 1;
      const uint32_t off = (med3_u32(av2, lo2, hi2) >> 18) & 0x1f8u;
      const uint32_t thr2 = tbl[off / 4], below8 = tbl[off / 4 + 1];
      uint32_t code = ((below8 + (av2 >= thr2 ? 1u : 0u)) ^ m) & 15u;  // one v_bitop3
#if defined(__HIP_DEVICE_COMPILE__)
      asm("" : "+v"(code));  // keeps the mask out of the pack (then one v_lshl_or)
#endif
      wd |= code << (c & 1 ? 8 * (c / 2) : 8 * (c / 2) + 4);
    }
    packed[i] = finite ? wd : 0u;
  }
  if (live && slot >= 0 && (int64_t)slot < nslots) {
    uint8_t* entry = (kv == 0 ? k_slab : v_slab) + ((int64_t)slot * H + h) * (int64_t)ebs;
#pragma unroll
    for (int i = 0; i < CPL; i++)
      *reinterpret_cast<uint32_t*>(entry + 4 * (p + P * i)) = packed[i];
    if (p == 0) {
      const uint32_t nb = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)l2);
      uint8_t* np = entry + PD / 2;
      if constexpr (PD == 64) {
        *reinterpret_cast<uint16_t*>(np) = (uint16_t)nb;
      } else if constexpr (PD == 128) {
        *reinterpret_cast<uint32_t*>(np) = nb | (nb << 16);
      } else {
        uint2 wq;
        wq.x = nb | (nb << 16);
        wq.y = wq.x;
        *reinterpret_cast<uint2*>(np) = wq;
      }
    }
  }
}

template <int PD>
hipError_t launch_write(bool vec_ok, dim3 grid, hipStream_t stream, uint8_t* ks, uint8_t* vs,
                        const void* key, const void* value, int dtype, int64_t k_st,
                        int64_t k_sh, int64_t v_st, int64_t v_sh, const float* signs,
                        const int32_t* slots, uint32_t per_kv, int H, uint32_t hmul, int hd,
                        int ebs, int64_t nslots, float scale) {
  if (vec_ok)
    hipLaunchKernelGGL((write_kernel<PD, true>), grid, dim3(256), 0, stream, ks, vs, key, value,
                       dtype, k_st, k_sh, v_st, v_sh, signs, slots, per_kv, H, hmul, hd, ebs,
                       nslots, scale);
  else
    hipLaunchKernelGGL((write_kernel<PD, false>), grid, dim3(256), 0, stream, ks, vs, key, value,
                       dtype, k_st, k_sh, v_st, v_sh, signs, slots, per_kv, H, hmul, hd, ebs,
                       nslots, scale);
  return hipGetLastError();
}

template <int PD>
hipError_t launch_write_f16(hipStream_t stream, uint8_t* ks, uint8_t* vs, const void* key,
                            const void* value, int64_t k_st, int64_t k_sh, int64_t v_st,
                            int64_t v_sh, const float* signs, const int32_t* slots,
                            uint32_t per_kv, int H, uint32_t hmul, int ebs, int64_t nslots,
                            float scale) {
  const int64_t blocks = (2 * (int64_t)per_kv + FastGeom<PD>::VPB - 1) / FastGeom<PD>::VPB;
  const unsigned grid = (unsigned)blocks;
  hipLaunchKernelGGL((write_f16_kernel<PD>), dim3(grid), dim3(256), 0, stream, ks, vs,
                     static_cast<const _Float16*>(key), static_cast<const _Float16*>(value), k_st,
                     k_sh, v_st, v_sh, signs, slots, per_kv, H, hmul, ebs, nslots, scale);
  return hipGetLastError();
}

}  // namespace

thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int device_cus() {
  constexpr int kMaxDev = 64;
  static std::atomic<int> cache[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 0;
  int c = cache[dev].load(std::memory_order_relaxed);
  if (c == 0 && hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
    cache[dev].store(c, std::memory_order_relaxed);
  return c;
}

}  // namespace tq

extern "C" const char* tq_last_error(void) { return tq::g_err; }
extern "C" int32_t tq_abi_version(void) { return 9; }

extern "C" int tq_quantize_write_kv_cache(void* k_slab, void* v_slab, const void* key,
                                          const void* value, int32_t in_dtype,
                                          int64_t k_stride_tok, int64_t k_stride_head,
                                          int64_t v_stride_tok, int64_t v_stride_head,
                                          const float* signs, const int32_t* slot_mapping,
                                          int64_t num_tokens, int32_t num_kv_heads,
                                          int32_t head_dim, int32_t padded_dim,
                                          int32_t block_size, int32_t ebs, int64_t num_blocks,
                                          tq_stream_t stream) {
  using namespace tq;
  const int pd = padded_dim;
  if (pd != 64 && pd != 128 && pd != 256) {
    set_error("quantize_write: padded_dim must be 64, 128 or 256, got %d", pd);
    return kEinval;
  }
  if (head_dim <= 0 || head_dim > pd || (pd > 64 && 2 * head_dim <= pd)) {
    set_error("quantize_write: head_dim %d does not pad to %d", head_dim, pd);
    return kEinval;
  }
  if (ebs % 16 != 0 || ebs < pd / 2 + 2 * (pd / 64)) {
    set_error("quantize_write: ebs %d must be a multiple of 16 and >= %d", ebs,
              pd / 2 + 2 * (pd / 64));
    return kEinval;
  }
  if (in_dtype != TQ_F32 && in_dtype != TQ_F16 && in_dtype != TQ_BF16) {
    set_error("quantize_write: unsupported input dtype %d", in_dtype);
    return kEinval;
  }
  if (num_kv_heads <= 0 || block_size <= 0 || num_tokens < 0 || num_blocks < 0) {
    set_error("quantize_write: bad sizes");
    return kEinval;
  }
  if (num_tokens == 0) return 0;
  if (!k_slab || !v_slab || !key || !value || !signs || !slot_mapping) {
    set_error("quantize_write: null pointer");
    return kEinval;
  }
  const int vec = pd / 32;
  const int esz = in_dtype == TQ_F32 ? 4 : 2;
  // vector loads need the full row, and every row start aligned to VEC elements
  bool vec_ok = in_dtype == TQ_F16 && head_dim == pd &&
                (k_stride_tok % vec == 0) && (k_stride_head % vec == 0) &&
                (v_stride_tok % vec == 0) && (v_stride_head % vec == 0) &&
                ((uintptr_t)key % (vec * esz) == 0) && ((uintptr_t)value % (vec * esz) == 0);
  // 16 vectors per workgroup; token = rem / H by multiply-high, exact while
  // num_tokens * H < 2^32 / H
  const int64_t per_kv = num_tokens * (int64_t)num_kv_heads;
  if (per_kv * num_kv_heads >= (int64_t)1 << 32 || 2 * per_kv >= (int64_t)1 << 32) {
    set_error("quantize_write: too many tokens (%lld x %d heads)", (long long)num_tokens,
              num_kv_heads);
    return kEinval;
  }
  const uint32_t hmul =
      num_kv_heads == 1 ? 0u : (uint32_t)((((uint64_t)1 << 32) + num_kv_heads - 1) / num_kv_heads);
  const int64_t blocks = (2 * per_kv + 15) / 16;
  const float scale = 1.0f / sqrtf((float)pd);
  const int64_t nslots = num_blocks * (int64_t)block_size;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((unsigned)blocks);
  uint8_t* ks = static_cast<uint8_t*>(k_slab);
  uint8_t* vs = static_cast<uint8_t*>(v_slab);
  hipError_t e;
  // fp16 rows of full width with 16-byte aligned chunks take the fast kernel
  const bool fast_ok = in_dtype == TQ_F16 && head_dim == pd && k_stride_tok % 8 == 0 &&
                       k_stride_head % 8 == 0 && v_stride_tok % 8 == 0 &&
                       v_stride_head % 8 == 0 && (uintptr_t)key % 16 == 0 &&
                       (uintptr_t)value % 16 == 0;
  if (fast_ok) {
    switch (pd) {
      case 64:
        e = launch_write_f16<64>(s, ks, vs, key, value, k_stride_tok, k_stride_head, v_stride_tok,
                                 v_stride_head, signs, slot_mapping, (uint32_t)per_kv,
                                 num_kv_heads, hmul, ebs, nslots, scale);
        break;
      case 128:
        e = launch_write_f16<128>(s, ks, vs, key, value, k_stride_tok, k_stride_head,
                                  v_stride_tok, v_stride_head, signs, slot_mapping,
                                  (uint32_t)per_kv, num_kv_heads, hmul, ebs, nslots, scale);
        break;
      default:
        e = launch_write_f16<256>(s, ks, vs, key, value, k_stride_tok, k_stride_head,
                                  v_stride_tok, v_stride_head, signs, slot_mapping,
                                  (uint32_t)per_kv, num_kv_heads, hmul, ebs, nslots, scale);
    }
    if (e != hipSuccess) {
      set_error("quantize_write: launch failed: %s", hipGetErrorString(e));
      return (int)e;
    }
    return 0;
  }
  switch (pd) {
    case 64:
      e = launch_write<64>(vec_ok, grid, s, ks, vs, key, value, in_dtype, k_stride_tok,
                           k_stride_head, v_stride_tok, v_stride_head, signs, slot_mapping,
                           (uint32_t)per_kv, num_kv_heads, hmul, head_dim, ebs, nslots, scale);
      break;
    case 128:
      e = launch_write<128>(vec_ok, grid, s, ks, vs, key, value, in_dtype, k_stride_tok,
                            k_stride_head, v_stride_tok, v_stride_head, signs, slot_mapping,
                            (uint32_t)per_kv, num_kv_heads, hmul, head_dim, ebs, nslots, scale);
      break;
    default:
      e = launch_write<256>(vec_ok, grid, s, ks, vs, key, value, in_dtype, k_stride_tok,
                            k_stride_head, v_stride_tok, v_stride_head, signs, slot_mapping,
                            (uint32_t)per_kv, num_kv_heads, hmul, head_dim, ebs, nslots, scale);
  }
  if (e != hipSuccess) {
    set_error("quantize_write: launch failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}
