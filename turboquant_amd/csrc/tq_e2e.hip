// tq_e2e.hip -- the layer glue of the end-to-end harness (turboquant_amd/e2e.py,
// configs[4]): a residual add fused with RMSNorm, the per-head q/k RMSNorm
// fused with rotate-half RoPE, and SiLU(g) * u.  In a vLLM deployment these
// are vLLM's own fused layer kernels; the harness needs them so that the
// model around the quantized attention runs as a server's would (one pass
// over each activation instead of one torch kernel per elementwise op, and
// ~11 fewer graph nodes per layer in the decode step).  fp16 tensors,
// fp32 arithmetic inside, one rounding to fp16 per output.
#include <cmath>

#include "tq_common.h"

namespace tq {
namespace {

constexpr int kGlueThreads = 256;

typedef _Float16 half8_g __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

// x[r] += y[r] (fp16 add, when y is given); h[r] = x[r] / rms(x[r]) * w
// (when h is given).  One workgroup per row of H <= 8192 dims, 8 per chunk.
__global__ __launch_bounds__(kGlueThreads) void add_rms_norm_kernel(
    _Float16* __restrict__ x, const _Float16* __restrict__ y, const _Float16* __restrict__ w,
    _Float16* __restrict__ h, int H, float eps) {
  constexpr int kMaxC = 4;  // chunks of 8 per thread (H <= 8192)
  __shared__ float part[kGlueThreads / 64];
  const int64_t row = blockIdx.x;
  const int nc = H / 8;
  half8_g s[kMaxC];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxC; i++) {
    const int c = threadIdx.x + kGlueThreads * i;
    if (c < nc) {
      half8_g a = *reinterpret_cast<const half8_g*>(x + row * H + 8 * c);
      if (y) {
        const half8_g b = *reinterpret_cast<const half8_g*>(y + row * H + 8 * c);
#pragma unroll
        for (int e = 0; e < 8; e++) a[e] = (_Float16)((float)a[e] + (float)b[e]);
        *reinterpret_cast<half8_g*>(x + row * H + 8 * c) = a;
      }
#pragma unroll
      for (int e = 0; e < 8; e++) ss = __builtin_fmaf((float)a[e], (float)a[e], ss);
      s[i] = a;
    }
  }
  if (!h) return;  // the add alone: no reduction, no barrier needed
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < kGlueThreads / 64; i++) tot += part[i];
  const float inv = rsqrtf(tot / (float)H + eps);
#pragma unroll
  for (int i = 0; i < kMaxC; i++) {
    const int c = threadIdx.x + kGlueThreads * i;
    if (c < nc) {
      const half8_g wv = *reinterpret_cast<const half8_g*>(w + 8 * c);
      half8_g o;
#pragma unroll
      for (int e = 0; e < 8; e++) o[e] = (_Float16)((float)s[i][e] * inv * (float)wv[e]);
      *reinterpret_cast<half8_g*>(h + row * H + 8 * c) = o;
    }
  }
}

// One wave per (token, head) of the q and k parts of a fused QKV row:
// RMSNorm over the head's D dims with the q or k weight, rounded to fp16,
// then rotate-half RoPE with the token's table row,
// out[i] = n[i] cos[i] + n[(i + D/2) mod D] sin_signed[i].  Lane l holds the
// D/64 consecutive dims l D/64 ..; the partner dims sit in lane l ^ 32.
template <int D>
__global__ __launch_bounds__(kGlueThreads) void qk_norm_rope_kernel(
    const _Float16* __restrict__ qkv, int64_t qkv_st, const _Float16* __restrict__ qw,
    const _Float16* __restrict__ kw, const _Float16* __restrict__ cosb,
    const _Float16* __restrict__ sinb, int64_t trows, const int64_t* __restrict__ pos,
    int64_t tokens, int hq, int hkv, float eps, _Float16* __restrict__ qo,
    _Float16* __restrict__ ko) {
  constexpr int V = D / 64;
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * (kGlueThreads / 64) + (threadIdx.x >> 6);
  const int nh = hq + hkv;
  if (r >= tokens * nh) return;  // whole waves leave together
  const int64_t t = r / nh;
  const int hd = (int)(r % nh);
  const bool isq = hd < hq;
  const _Float16* src = qkv + t * qkv_st + (int64_t)hd * D + V * lane;
  const _Float16* wt = (isq ? qw : kw) + V * lane;
  float a[V];
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < V; e++) {
    a[e] = (float)src[e];
    ss = __builtin_fmaf(a[e], a[e], ss);
  }
  ss = wave_sum(ss);
  const float inv = rsqrtf(ss / (float)D + eps);
  float n[V], pn[V];
#pragma unroll
  for (int e = 0; e < V; e++) n[e] = (float)(_Float16)(a[e] * inv * (float)wt[e]);
#pragma unroll
  for (int e = 0; e < V; e++) pn[e] = __shfl_xor(n[e], 32);
  const int64_t p = pos[t];
  _Float16* dst = isq ? qo + (t * hq + hd) * D + V * lane
                      : ko + (t * hkv + (hd - hq)) * D + V * lane;
  if (p < 0 || p >= trows) {  // no table row: NaN rows, no read past the tables
#pragma unroll
    for (int e = 0; e < V; e++) dst[e] = (_Float16)__builtin_nanf("");
    return;
  }
  const _Float16* cr = cosb + p * D + V * lane;
  const _Float16* sr = sinb + p * D + V * lane;
#pragma unroll
  for (int e = 0; e < V; e++)
    dst[e] = (_Float16)(__builtin_fmaf(pn[e], (float)sr[e], n[e] * (float)cr[e]));
}

// The same for any even head size D <= 256 (e.g. 96): lane l holds dims
// l, l + 64, ..; the RoPE partner comes through an LDS row per wave.
__global__ __launch_bounds__(kGlueThreads) void qk_norm_rope_any_kernel(
    const _Float16* __restrict__ qkv, int64_t qkv_st, const _Float16* __restrict__ qw,
    const _Float16* __restrict__ kw, const _Float16* __restrict__ cosb,
    const _Float16* __restrict__ sinb, int64_t trows, const int64_t* __restrict__ pos,
    int64_t tokens, int hq, int hkv, int D, float eps, _Float16* __restrict__ qo,
    _Float16* __restrict__ ko) {
  constexpr int kMaxV = 4;
  __shared__ float row[kGlueThreads / 64][256];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t r = (int64_t)blockIdx.x * (kGlueThreads / 64) + w;
  const int nh = hq + hkv;
  if (r >= tokens * nh) return;  // whole waves leave together; no block barrier below
  const int64_t t = r / nh;
  const int hd = (int)(r % nh);
  const bool isq = hd < hq;
  const _Float16* src = qkv + t * qkv_st + (int64_t)hd * D;
  const _Float16* wt = isq ? qw : kw;
  float a[kMaxV];
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < kMaxV; e++) {
    const int i = lane + 64 * e;
    a[e] = i < D ? (float)src[i] : 0.0f;
    ss = __builtin_fmaf(a[e], a[e], ss);
  }
  ss = wave_sum(ss);
  const float inv = rsqrtf(ss / (float)D + eps);
#pragma unroll
  for (int e = 0; e < kMaxV; e++) {
    const int i = lane + 64 * e;
    if (i < D) row[w][i] = (float)(_Float16)(a[e] * inv * (float)wt[i]);
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int64_t p = pos[t];
  _Float16* dst = isq ? qo + (t * hq + hd) * D : ko + (t * hkv + (hd - hq)) * D;
  const bool inside = p >= 0 && p < trows;  // else NaN rows, no read past the tables
#pragma unroll
  for (int e = 0; e < kMaxV; e++) {
    const int i = lane + 64 * e;
    if (i < D && !inside) {
      dst[i] = (_Float16)__builtin_nanf("");
    } else if (i < D) {
      const float n = row[w][i], pn = row[w][(i + D / 2) % D];
      dst[i] = (_Float16)(__builtin_fmaf(pn, (float)sinb[p * D + i], n * (float)cosb[p * D + i]));
    }
  }
}

// h[t, :] = silu(gu[t, :I]) * gu[t, I:], 8 dims per thread.
__global__ __launch_bounds__(kGlueThreads) void silu_mul_kernel(const _Float16* __restrict__ gu,
                                                                 _Float16* __restrict__ h,
                                                                 int64_t rows, int I) {
  const int64_t idx = (int64_t)blockIdx.x * kGlueThreads + threadIdx.x;
  const int per = I / 8;
  if (idx >= rows * per) return;
  const int64_t t = idx / per;
  const int c = (int)(idx % per);
  const half8_g g = *reinterpret_cast<const half8_g*>(gu + t * 2 * I + 8 * c);
  const half8_g u = *reinterpret_cast<const half8_g*>(gu + t * 2 * I + I + 8 * c);
  half8_g o;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const float gv = (float)g[e];
    o[e] = (_Float16)(gv / (1.0f + expf(-gv)) * (float)u[e]);
  }
  *reinterpret_cast<half8_g*>(h + t * I + 8 * c) = o;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace
}  // namespace tq

extern "C" int tq_e2e_add_rms_norm(void* x, const void* y, const void* w, void* h, int64_t rows,
                                   int32_t hidden, float eps, tq_stream_t stream) {
  if (rows < 0 || hidden <= 0 || hidden % 8 != 0 || hidden > 8 * 4 * tq::kGlueThreads) {
    tq::set_error("e2e_add_rms_norm: hidden %d must be a multiple of 8 up to 8192", hidden);
    return tq::kEinval;
  }
  if (rows == 0) return 0;
  if (!x || (!y && !h) || (h && !w)) {
    tq::set_error("e2e_add_rms_norm: null pointer");
    return tq::kEinval;
  }
  if (!tq::aligned16(x) || (y && !tq::aligned16(y)) || (h && (!tq::aligned16(h) ||
                                                               !tq::aligned16(w)))) {
    tq::set_error("e2e_add_rms_norm: rows must be 16-byte aligned");
    return tq::kEinval;
  }
  if (rows > 0x7fffffffLL) {
    tq::set_error("e2e_add_rms_norm: %lld rows out of range", (long long)rows);
    return tq::kEinval;
  }
  hipLaunchKernelGGL(tq::add_rms_norm_kernel, dim3((unsigned)rows), dim3(tq::kGlueThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<_Float16*>(x),
                     static_cast<const _Float16*>(y), static_cast<const _Float16*>(w),
                     static_cast<_Float16*>(h), hidden, eps);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) tq::set_error("e2e_add_rms_norm: launch failed: %s", hipGetErrorString(e));
  return (int)e;
}

extern "C" int tq_e2e_qk_norm_rope(const void* qkv, int64_t qkv_row_stride, const void* q_w,
                                   const void* k_w, const void* cos_table,
                                   const void* sin_table, int64_t table_rows,
                                   const int64_t* positions, int64_t tokens, int32_t q_heads,
                                   int32_t kv_heads,
                                   int32_t head_dim, float eps, void* q_out, void* k_out,
                                   tq_stream_t stream) {
  if (head_dim < 2 || head_dim > 256 || head_dim % 2 != 0) {
    tq::set_error("e2e_qk_norm_rope: head_dim %d unsupported (even, up to 256)", head_dim);
    return tq::kEinval;
  }
  if (tokens < 0 || q_heads <= 0 || kv_heads <= 0 || table_rows < 0 ||
      qkv_row_stride < (int64_t)(q_heads + 2 * kv_heads) * head_dim) {
    tq::set_error("e2e_qk_norm_rope: bad geometry");
    return tq::kEinval;
  }
  if (tokens == 0) return 0;
  if (!qkv || !q_w || !k_w || !cos_table || !sin_table || !positions || !q_out || !k_out) {
    tq::set_error("e2e_qk_norm_rope: null pointer");
    return tq::kEinval;
  }
  const int64_t waves = tokens * (q_heads + kv_heads);
  const int64_t blocks = (waves + tq::kGlueThreads / 64 - 1) / (tq::kGlueThreads / 64);
  if (blocks > 0x7fffffffLL) {
    tq::set_error("e2e_qk_norm_rope: %lld tokens out of range", (long long)tokens);
    return tq::kEinval;
  }
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define TQ_QKR(D)                                                                              \
  hipLaunchKernelGGL(tq::qk_norm_rope_kernel<D>, dim3((unsigned)blocks), dim3(tq::kGlueThreads), \
                     0, st, static_cast<const _Float16*>(qkv), qkv_row_stride,                   \
                     static_cast<const _Float16*>(q_w), static_cast<const _Float16*>(k_w),       \
                     static_cast<const _Float16*>(cos_table),                                    \
                     static_cast<const _Float16*>(sin_table), table_rows, positions, tokens,     \
                     q_heads, kv_heads, eps, static_cast<_Float16*>(q_out), static_cast<_Float16*>(k_out))
  if (head_dim == 64) TQ_QKR(64);
  else if (head_dim == 128) TQ_QKR(128);
  else if (head_dim == 256) TQ_QKR(256);
  else
    hipLaunchKernelGGL(tq::qk_norm_rope_any_kernel, dim3((unsigned)blocks),
                       dim3(tq::kGlueThreads), 0, st, static_cast<const _Float16*>(qkv),
                       qkv_row_stride, static_cast<const _Float16*>(q_w),
                       static_cast<const _Float16*>(k_w), static_cast<const _Float16*>(cos_table),
                       static_cast<const _Float16*>(sin_table), table_rows, positions, tokens,
                       q_heads, kv_heads, head_dim, eps, static_cast<_Float16*>(q_out),
                       static_cast<_Float16*>(k_out));
#undef TQ_QKR
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) tq::set_error("e2e_qk_norm_rope: launch failed: %s", hipGetErrorString(e));
  return (int)e;
}

extern "C" int tq_e2e_silu_mul(const void* gate_up, void* out, int64_t rows, int32_t inter,
                               tq_stream_t stream) {
  if (rows < 0 || inter <= 0 || inter % 8 != 0) {
    tq::set_error("e2e_silu_mul: intermediate size %d must be a multiple of 8", inter);
    return tq::kEinval;
  }
  if (rows == 0) return 0;
  if (!gate_up || !out) {
    tq::set_error("e2e_silu_mul: null pointer");
    return tq::kEinval;
  }
  if (!tq::aligned16(gate_up) || !tq::aligned16(out)) {
    tq::set_error("e2e_silu_mul: tensors must be 16-byte aligned");
    return tq::kEinval;
  }
  const int64_t threads = rows * (inter / 8);
  const int64_t blocks = (threads + tq::kGlueThreads - 1) / tq::kGlueThreads;
  if (blocks > 0x7fffffffLL) {
    tq::set_error("e2e_silu_mul: %lld rows out of range", (long long)rows);
    return tq::kEinval;
  }
  hipLaunchKernelGGL(tq::silu_mul_kernel, dim3((unsigned)blocks), dim3(tq::kGlueThreads), 0,
                     reinterpret_cast<hipStream_t>(stream),
                     static_cast<const _Float16*>(gate_up), static_cast<_Float16*>(out), rows,
                     inter);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) tq::set_error("e2e_silu_mul: launch failed: %s", hipGetErrorString(e));
  return (int)e;
}
