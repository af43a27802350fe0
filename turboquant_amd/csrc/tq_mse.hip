// tq_mse.hip -- the algorithm library's TurboQuantMSE (Algorithm 1 of
// arXiv:2504.19874) on the GPU: quantize fp32 vectors to b-bit Lloyd-Max
// codes (b = 1..4) packed low bits first, and dequantize them back.
//
// Semantics (reference turboquant/quantizer.py:63-118, with
// turboquant/hadamard.py:20-78 and turboquant/codebook.py:65-103):
//   quantize:   n = max(||x||, 1e-8); y = FWHT(s * pad(x / n)) / sqrt(pd);
//               code_d = #{j : boundary_j < y_d} (torch.bucketize: a value
//               equal to a boundary takes the lower code; NaN the top one);
//               byte k = sum_i code[k*per + i] << (i*b), per = 8 / b
//               (2 for b = 3).
//   dequantize: y_d = centroid[code_d]; x = (FWHT(y) / sqrt(pd) * s)[:dim] * n.
// The FWHT butterflies run in ascending stride, each stage (a + b, a - b),
// as the reference's, so the rotation carries the same fp32 bits; only the
// norm's summation order differs from torch's reduction (it can move a
// coordinate that sits within an ulp of a boundary).
//
// gfx950 layout: one wave64 per vector, lane l holding dims l*E .. l*E+E-1
// (E = pd / 64, pd = 64 .. 1024): stages of stride < E run in-lane, the
// others across lanes (lane xor h/E).  The codes go through LDS to be packed
// by bytes, so every bit width packs the same way.  The codebook sits in
// LDS.  HBM-bound: 4 dim + pd*b/8 + 4 bytes per vector.
#include <cmath>

#include "tq_common.h"

namespace tq {
namespace {

constexpr int kMseWaves = 4;  // vectors per workgroup

struct MseParams {
  const float* x;      // quantize in: [n, dim]
  uint8_t* packed;     // quantize out / dequantize in: [n, nbytes]
  float* norms;        // quantize out / dequantize in: [n]
  float* out;          // dequantize out: [n, dim]
  const float* signs;  // [pd]
  int64_t n;
  int dim, nbytes;
  float inv_sqrt_pd;
  float table[16];     // boundaries (quantize, levels - 1 used) or centroids
  int levels;
};

template <int E>
__device__ __forceinline__ void fwht_wave(float (&v)[E], int lane) {
#pragma unroll
  for (int h = 1; h < E; h <<= 1)
#pragma unroll
    for (int i = 0; i < E; i++)
      if ((i & h) == 0) {
        const float a = v[i], b = v[i + h];
        v[i] = a + b;
        v[i + h] = a - b;
      }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const bool lower = (lane & m) == 0;
#pragma unroll
    for (int i = 0; i < E; i++) {
      const float o = __shfl_xor(v[i], m);
      v[i] = lower ? v[i] + o : o - v[i];
    }
  }
}

template <int E, int BITS>
__global__ __launch_bounds__(64 * kMseWaves) void mse_quantize_kernel(MseParams p) {
  constexpr int PD = 64 * E;
  constexpr int PER = BITS == 3 ? 2 : 8 / BITS;
  __shared__ uint8_t codes[kMseWaves][PD];
  __shared__ float bnd[16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (threadIdx.x < 16) bnd[threadIdx.x] = p.table[threadIdx.x];
  __syncthreads();
  const int64_t row = (int64_t)blockIdx.x * kMseWaves + w;
  if (row >= p.n) return;
  const float* xr = p.x + row * p.dim;
  float v[E];
#pragma unroll
  for (int i = 0; i < E; i++) {
    const int d = lane * E + i;
    v[i] = d < p.dim ? xr[d] : 0.0f;
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < E; i++) ss = __builtin_fmaf(v[i], v[i], ss);
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m);
  const float sq = sqrtf(ss);
  const float nrm = sq < 1e-8f ? 1e-8f : sq;  // torch's clamp(min=1e-8), NaN kept
#pragma unroll
  for (int i = 0; i < E; i++) v[i] = (v[i] / nrm) * p.signs[lane * E + i];
  fwht_wave<E>(v, lane);
  const int nb = p.levels - 1;
#pragma unroll
  for (int i = 0; i < E; i++) {
    const float y = v[i] * p.inv_sqrt_pd;
    int c = 0;
    for (int j = 0; j < nb; j++) c += bnd[j] < y ? 1 : 0;
    if (y != y) c = nb;  // NaN: torch.bucketize's top index
    codes[w][lane * E + i] = (uint8_t)c;
  }
  if (lane == 0) p.norms[row] = nrm;
  // the wave's codes, written by every lane, are read by other lanes below
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
  __builtin_amdgcn_wave_barrier();
  uint8_t* pr = p.packed + row * p.nbytes;
  for (int k = lane; k < p.nbytes; k += 64) {
    uint32_t byte = 0;
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int d = k * PER + i;
      if (d < PD) byte |= (uint32_t)codes[w][d] << (i * BITS);
    }
    pr[k] = (uint8_t)byte;
  }
}

template <int E, int BITS>
__global__ __launch_bounds__(64 * kMseWaves) void mse_dequantize_kernel(MseParams p) {
  constexpr int PER = BITS == 3 ? 2 : 8 / BITS;
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  __shared__ float cen[16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (threadIdx.x < 16) cen[threadIdx.x] = p.table[threadIdx.x];
  __syncthreads();
  const int64_t row = (int64_t)blockIdx.x * kMseWaves + w;
  if (row >= p.n) return;
  const uint8_t* pr = p.packed + row * p.nbytes;
  float v[E];
#pragma unroll
  for (int i = 0; i < E; i++) {
    const int d = lane * E + i;
    const uint32_t c = ((uint32_t)pr[d / PER] >> ((d % PER) * BITS)) & kMask;
    v[i] = cen[c];
  }
  fwht_wave<E>(v, lane);
  const float nrm = p.norms[row];
  float* orow = p.out + row * p.dim;
#pragma unroll
  for (int i = 0; i < E; i++) {
    const int d = lane * E + i;
    if (d < p.dim) orow[d] = ((v[i] * p.inv_sqrt_pd) * p.signs[d]) * nrm;
  }
}

template <int E>
hipError_t launch_mse(bool quant, int bits, const MseParams& p, hipStream_t st) {
  const dim3 grid((unsigned)((p.n + kMseWaves - 1) / kMseWaves)), block(64 * kMseWaves);
#define TQ_MSE_CASE(B)                                                              \
  case B:                                                                           \
    if (quant)                                                                      \
      hipLaunchKernelGGL((mse_quantize_kernel<E, B>), grid, block, 0, st, p);       \
    else                                                                            \
      hipLaunchKernelGGL((mse_dequantize_kernel<E, B>), grid, block, 0, st, p);     \
    break;
  switch (bits) {
    TQ_MSE_CASE(1)
    TQ_MSE_CASE(2)
    TQ_MSE_CASE(3)
    TQ_MSE_CASE(4)
    default:
      return hipErrorInvalidValue;
  }
#undef TQ_MSE_CASE
  return hipGetLastError();
}

int mse_call(bool quant, const float* x, uint8_t* packed, float* norms, float* out,
             int64_t n, int32_t dim, int32_t padded_dim, int32_t bit_width, const float* signs,
             const float* table, tq_stream_t stream) {
  const char* what = quant ? "mse_quantize" : "mse_dequantize";
  if (bit_width < 1 || bit_width > 4) {
    set_error("%s: bit_width %d unsupported (1..4)", what, bit_width);
    return kEinval;
  }
  if (padded_dim < 64 || padded_dim > 1024 || (padded_dim & (padded_dim - 1)) != 0 ||
      dim < 1 || dim > padded_dim || 2 * dim <= padded_dim) {
    set_error("%s: padded_dim %d must be the power of two 64..1024 next to dim %d", what,
              padded_dim, dim);
    return kEinval;
  }
  if (n < 0 || n > ((int64_t)1 << 40)) {
    set_error("%s: vector count %lld out of range", what, (long long)n);
    return kEinval;
  }
  if (n == 0) return 0;
  if (!packed || !norms || !signs || !table || (quant ? !x : !out)) {
    set_error("%s: null pointer", what);
    return kEinval;
  }
  MseParams p;
  p.x = x;
  p.packed = packed;
  p.norms = norms;
  p.out = out;
  p.signs = signs;
  p.n = n;
  p.dim = dim;
  const int per = bit_width == 3 ? 2 : 8 / bit_width;
  p.nbytes = padded_dim / per;
  p.inv_sqrt_pd = (float)(1.0 / std::sqrt((double)padded_dim));
  p.levels = 1 << bit_width;
  for (int i = 0; i < 16; i++) p.table[i] = 0.0f;
  for (int i = 0; i < (quant ? p.levels - 1 : p.levels); i++) p.table[i] = table[i];
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  switch (padded_dim / 64) {
    case 1: e = launch_mse<1>(quant, bit_width, p, st); break;
    case 2: e = launch_mse<2>(quant, bit_width, p, st); break;
    case 4: e = launch_mse<4>(quant, bit_width, p, st); break;
    case 8: e = launch_mse<8>(quant, bit_width, p, st); break;
    default: e = launch_mse<16>(quant, bit_width, p, st); break;
  }
  if (e != hipSuccess) set_error("%s: launch failed: %s", what, hipGetErrorString(e));
  return (int)e;
}

}  // namespace
}  // namespace tq

extern "C" int tq_mse_quantize(const float* x, int64_t num_vectors, int32_t dim,
                               int32_t padded_dim, int32_t bit_width, const float* signs,
                               const float* boundaries, uint8_t* packed, float* norms,
                               tq_stream_t stream) {
  return tq::mse_call(true, x, packed, norms, nullptr, num_vectors, dim, padded_dim, bit_width,
                      signs, boundaries, stream);
}

extern "C" int tq_mse_dequantize(const uint8_t* packed, const float* norms, int64_t num_vectors,
                                 int32_t dim, int32_t padded_dim, int32_t bit_width,
                                 const float* signs, const float* centroids, float* out,
                                 tq_stream_t stream) {
  return tq::mse_call(false, nullptr, const_cast<uint8_t*>(packed), const_cast<float*>(norms),
                      out, num_vectors, dim, padded_dim, bit_width, signs, centroids, stream);
}
