// tq_dequant.hip -- packed cache pages -> fp16 K/V rows in the original domain.
//
// Used by the prefill of a chunk whose sequence already has cached context:
// the context is read back from the quantized cache, as the decode reads it
// (dequantize-then-attend, turboquant/triton_decode_ref.py:89-131), and
// rotated back to the original domain so that it can be attended together
// with the chunk's fresh fp16 K/V.  Entry layout as written by
// quantize_write_kernel.cuh:332-431: pd/2 code bytes (dim 2k in the high
// nibble of byte k), then the fp16 norm.  Per vector:
//   y_d = c[code_d] * norm / sqrt(pd)       (the rotated-domain value)
//   x   = s * FWHT(y) / sqrt(pd)            (the inverse of the write's rotation)
// HBM-bound and off the decode path: one pass over the entries, L = pd/32
// lanes per vector (32 dims = 16 code bytes per lane, one 16-byte load, four
// 16-byte stores), the FWHT stages h >= 32 across lanes with shuffles.
#include <type_traits>

#include "tq_common.h"

namespace tq {
namespace {

__constant__ float kCodebook[16] = {
    -2.7326368f, -2.0693470f, -1.6180345f, -1.2562491f, -0.9423684f, -0.6567591f,
    -0.3880823f, -0.1284154f, 0.1284154f,  0.3880823f,  0.6567591f,  0.9423684f,
    1.2562491f,  1.6180345f,  2.0693470f,  2.7326368f};

// value of lane (lane ^ D) for D = 1, 2 (DPP quad permutes) and D = 4 (two
// masked row shifts: banks 0, 2 take lane + 4, banks 1, 3 lane - 4)
template <int D>
__device__ __forceinline__ float lane_xor(float x) {
  const int xi = __float_as_int(x);
  if constexpr (D == 1) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(xi, 0xb1, 0xf, 0xf, false));
  } else if constexpr (D == 2) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(xi, 0x4e, 0xf, 0xf, false));
  } else {
    static_assert(D == 4, "lane distance");
    int r = __builtin_amdgcn_update_dpp(xi, xi, 0x104, 0xf, 0x5, false);  // row_shl:4
    r = __builtin_amdgcn_update_dpp(r, xi, 0x114, 0xf, 0xa, false);       // row_shr:4
    return __int_as_float(r);
  }
}

constexpr int kVecsPerThread = 4;

template <int PD>
__global__ __launch_bounds__(256) void dequant_kernel(
    const uint8_t* __restrict__ k_slab, const uint8_t* __restrict__ v_slab,
    const int32_t* __restrict__ pages, int64_t num_tokens, int H, int head_dim,
    int block_size, int ebs, int64_t num_blocks, const float* __restrict__ signs,
    _Float16* __restrict__ out_k, _Float16* __restrict__ out_v, int64_t out_stride_tok,
    bool vec_store) {
  constexpr int L = PD / 32;  // lanes per vector, 32 dims (16 code bytes) each
  constexpr int VPB = 256 / L;
  constexpr int NV = kVecsPerThread;
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  __shared__ float cb[16];    // the codebook, indexed per lane
  if (threadIdx.x < 16) cb[threadIdx.x] = kCodebook[threadIdx.x];
  const int lane = threadIdx.x % L;
  const uint8_t* slab = blockIdx.y ? v_slab : k_slab;
  _Float16* out = blockIdx.y ? out_v : out_k;
  const int64_t nvec = num_tokens * H;

  // every load of the thread's NV vectors goes out before any math
  int64_t tv[NV];
  int hv[NV];
  int pg[NV];
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int64_t vec = ((int64_t)blockIdx.x * NV + j) * VPB + threadIdx.x / L;
    const bool live = vec < nvec;  // all L lanes of a vector agree
    tv[j] = live ? vec / H : -1;
    hv[j] = live ? (int)(vec % H) : 0;
    pg[j] = live ? pages[tv[j] / block_size] : -1;
  }
  u32x4 w[NV];
  float nrm[NV];
#pragma unroll
  for (int j = 0; j < NV; j++) {
    w[j] = u32x4{0u, 0u, 0u, 0u};
    nrm[j] = 0.0f;
    if (pg[j] >= 0 && pg[j] < num_blocks) {
      const uint8_t* e = slab + (((int64_t)pg[j] * block_size + tv[j] % block_size) * H + hv[j]) *
                                    (int64_t)ebs;
      w[j] = *reinterpret_cast<const u32x4*>(e + 16 * lane);
      nrm[j] = (float)__builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t*>(e + PD / 2));
    }
  }
  float sg[32];  // signs / sqrt(pd) of this lane's dims (or 1)
  {
    const float isq = 1.0f / __builtin_sqrtf((float)PD);
    if (signs) {
      const float4* sp = reinterpret_cast<const float4*>(signs + 32 * lane);
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float4 sv = sp[i];
        sg[4 * i] = sv.x * isq;
        sg[4 * i + 1] = sv.y * isq;
        sg[4 * i + 2] = sv.z * isq;
        sg[4 * i + 3] = sv.w * isq;
      }
    }
  }
  __syncthreads();  // codebook ready
  // packed full rows (row stride H * head_dim): a wave's 64 / L vectors are
  // 4 KB of consecutive output, staged in LDS and written with whole-wave
  // 1 KB stores instead of 16-byte pieces at a 64-byte stride
  __shared__ __attribute__((aligned(16))) _Float16 stage[VPB / (64 / L)][64 * 32];
  const bool packed = vec_store && out_stride_tok == (int64_t)H * head_dim;  // uniform
  const int wv = threadIdx.x >> 6;
#pragma unroll 1
  for (int j = 0; j < NV; j++) {
    if (!packed && tv[j] < 0) continue;  // whole vector (L lanes of one DPP row) together
    float y[32];  // dims 32 * lane + i
    const float sc = nrm[j] * (1.0f / __builtin_sqrtf((float)PD));
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const uint32_t b = (w[j][k / 4] >> (8 * (k % 4))) & 0xffu;
      y[2 * k] = cb[b >> 4] * sc;
      y[2 * k + 1] = cb[b & 15u] * sc;
    }
    if (signs) {
      // FWHT: stages 1 .. 16 in-lane, then across the vector's lanes
#pragma unroll
      for (int hh = 1; hh < 32; hh <<= 1)
#pragma unroll
        for (int i = 0; i < 32; i++)
          if (!(i & hh)) {
            const float a = y[i], b = y[i + hh];
            y[i] = a + b;
            y[i + hh] = a - b;
          }
      auto cross = [&](auto dist) {
        constexpr int D = decltype(dist)::value;
        const float s = (lane & D) ? -1.0f : 1.0f;  // upper lane: partner - own
#pragma unroll
        for (int i = 0; i < 32; i++) y[i] = __builtin_fmaf(y[i], s, lane_xor<D>(y[i]));
      };
      if constexpr (L >= 2) cross(std::integral_constant<int, 1>{});
      if constexpr (L >= 4) cross(std::integral_constant<int, 2>{});
      if constexpr (L >= 8) cross(std::integral_constant<int, 4>{});
#pragma unroll
      for (int i = 0; i < 32; i++) y[i] = y[i] * sg[i];
    }
    if (packed) {
      typedef _Float16 h8 __attribute__((ext_vector_type(8)));
      _Float16* st = &stage[wv][32 * (threadIdx.x & 63)];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        h8 o;
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = (_Float16)y[8 * c + i];
        *reinterpret_cast<h8*>(st + 8 * c) = o;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // the wave's vectors: vec0 .. vec0 + 64 / L - 1, the live ones first
      const int64_t vec0 = ((int64_t)blockIdx.x * NV + j) * VPB + (int64_t)wv * (64 / L);
      const int64_t live = nvec - vec0 < 64 / L ? nvec - vec0 : 64 / L;
      if (live > 0) {
        const int bytes = (int)live * head_dim * 2;
        uint8_t* const dst0 = reinterpret_cast<uint8_t*>(out + vec0 * head_dim);
        const uint8_t* const src0 = reinterpret_cast<const uint8_t*>(&stage[wv][0]);
        const int lb = 16 * (threadIdx.x & 63);
#pragma unroll
        for (int k = 0; k < 4; k++)
          if (lb + 1024 * k < bytes)
            *reinterpret_cast<u32x4*>(dst0 + lb + 1024 * k) =
                *reinterpret_cast<const u32x4*>(src0 + lb + 1024 * k);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();  // the next vectors rewrite the stage
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      continue;
    }
    _Float16* dst = out + tv[j] * out_stride_tok + (int64_t)hv[j] * head_dim + 32 * lane;
    if (vec_store) {  // 8 dims per 16-byte store
      typedef _Float16 h8 __attribute__((ext_vector_type(8)));
#pragma unroll
      for (int c = 0; c < 4; c++) {
        h8 o;
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = (_Float16)y[8 * c + i];
        *reinterpret_cast<h8*>(dst + 8 * c) = o;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 32; i++)
        if (32 * lane + i < head_dim) dst[i] = (_Float16)y[i];
    }
  }
}

}  // namespace
}  // namespace tq

extern "C" int tq_dequant_paged(const uint8_t* k_slab, const uint8_t* v_slab,
                                const int32_t* pages, int64_t num_tokens, int32_t num_kv_heads,
                                int32_t head_dim, int32_t padded_dim, int32_t block_size,
                                int32_t ebs, int64_t num_blocks, const float* signs,
                                void* out_k, void* out_v, int64_t out_stride_tok,
                                tq_stream_t stream) {
  using namespace tq;
  const int pd = padded_dim;
  if (pd != 64 && pd != 128 && pd != 256) {
    set_error("dequant: padded_dim must be 64, 128 or 256, got %d", pd);
    return kEinval;
  }
  if (head_dim <= 0 || head_dim > pd || num_kv_heads <= 0 || block_size <= 0 ||
      num_tokens < 0 || num_blocks < 0) {
    set_error("dequant: bad sizes");
    return kEinval;
  }
  if (ebs % 16 != 0 || ebs < pd / 2 + 2 * (pd / 64)) {
    set_error("dequant: ebs %d must be a multiple of 16 and >= %d", ebs, pd / 2 + 2 * (pd / 64));
    return kEinval;
  }
  if (out_stride_tok < (int64_t)num_kv_heads * head_dim) {
    set_error("dequant: out_stride_tok %lld < num_kv_heads * head_dim", (long long)out_stride_tok);
    return kEinval;
  }
  if (num_tokens == 0) return 0;
  if (!k_slab || !v_slab || !pages || !out_k || !out_v) {
    set_error("dequant: null pointer");
    return kEinval;
  }
  const int64_t vecs = num_tokens * num_kv_heads;
  const int per_block = kVecsPerThread * (256 / (pd / 32));
  const int64_t blocks = (vecs + per_block - 1) / per_block;
  if (blocks > 0x7fffffffLL) {
    set_error("dequant: too many tokens");
    return kEinval;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((unsigned)blocks, 2);
  // full rows with 16-byte aligned dims: vector stores
  const bool vec_store = head_dim == pd && out_stride_tok % 8 == 0 && head_dim % 8 == 0 &&
                         (uintptr_t)out_k % 16 == 0 && (uintptr_t)out_v % 16 == 0;
  _Float16* ok = static_cast<_Float16*>(out_k);
  _Float16* ov = static_cast<_Float16*>(out_v);
  switch (pd) {
    case 64:
      hipLaunchKernelGGL(dequant_kernel<64>, grid, dim3(256), 0, s, k_slab, v_slab, pages,
                         num_tokens, num_kv_heads, head_dim, block_size, ebs, num_blocks, signs,
                         ok, ov, out_stride_tok, vec_store);
      break;
    case 128:
      hipLaunchKernelGGL(dequant_kernel<128>, grid, dim3(256), 0, s, k_slab, v_slab, pages,
                         num_tokens, num_kv_heads, head_dim, block_size, ebs, num_blocks, signs,
                         ok, ov, out_stride_tok, vec_store);
      break;
    default:
      hipLaunchKernelGGL(dequant_kernel<256>, grid, dim3(256), 0, s, k_slab, v_slab, pages,
                         num_tokens, num_kv_heads, head_dim, block_size, ebs, num_blocks, signs,
                         ok, ov, out_stride_tok, vec_store);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("dequant: launch failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}
