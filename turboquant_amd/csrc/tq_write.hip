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

}  // namespace

thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

}  // namespace tq

extern "C" const char* tq_last_error(void) { return tq::g_err; }
extern "C" int32_t tq_abi_version(void) { return 1; }

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
