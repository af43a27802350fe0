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
// as the reference's, so the rotation carries the same fp32 bits; x / n is
// correctly rounded (below); only the norm's summation order differs from
// torch's reduction (it can move a coordinate that sits within an ulp of a
// boundary).
//
// gfx950 layout: P lanes per vector (8, or pd / 32 from pd 512 up), each
// holding E = pd / P dims, so a wave serves 64 / P vectors: in the quantize
// kernel the E consecutive dims p E .., in the dequantize kernel NC = E / 8
// chunks of 8 consecutive dims, chunk i of lane p being dims 8 (p + P i) ..
// + 7 (the lanes of a vector then write neighbouring 32-byte pieces of its
// row).  FWHT stages of stride 1, 2, 4 run inside a chunk, strides 8 ..
// 4P across lanes as one fma with a DPP operand each, z + sg * partner with
// sg = -1 on the upper lane (a + b, or a - b negated: the same rounding; the
// sign is folded into the 1/sqrt(pd) scale, see tau_scale), and the larger
// strides between a lane's chunks.  The per-vector work (the
// norm's sqrt and its correctly rounded reciprocal) is shared by the P lanes
// and each lane's codes pack in its own registers.  HBM-bound in bytes:
// 4 dim + pd*b/8 + 4 per vector.
#include <atomic>
#include <cmath>
#include <cstring>

#include "tq_common.h"

namespace tq {
namespace {

constexpr int kMseThreads = 256;

struct MseParams {
  const float* x;      // quantize in: [n, dim]
  uint8_t* packed;     // quantize out / dequantize in: [n, nbytes]
  float* norms;        // quantize out / dequantize in: [n]
  float* out;          // dequantize out: [n, dim]
  const float* signs;  // [pd]
  float* resid;        // prod quantize out: unit residual [n, dim] (null: MSE only)
  float* rnorm;        // prod quantize out: residual norms [n]
  const float* add;    // prod dequantize in: S^T z rows [n, dim] (null: MSE only)
  const float* gamma;  // prod dequantize in: residual norms [n]
  float add_scale;     // sqrt(pi / 2) / dim
  int64_t n;
  int dim, nbytes;
  float inv_sqrt_pd;
  float table[16];     // boundaries (quantize, levels - 1 used) or centroids
  float cen[16];       // centroids for the prod quantize's read-back
  int levels;
  // quantize: the bin table of a symmetric codebook (see bin_code), when
  // use_bins; else the binary search over `table`
  int use_bins, bin_base;
  uint32_t bin_b[64], bin_n[64];
};

template <int PD>
struct MseGeom {
  static constexpr int P = PD <= 256 ? 8 : PD / 32;  // lanes per vector
  static constexpr int E = PD / P;                   // dims per lane (8 .. 32)
  static constexpr int VPB = kMseThreads / P;        // vectors per workgroup
};

// value of lane l ^ m: DPP moves for m = 1, 2, 4, 8 (quad permutes; row
// half-mirror then quad reversal; row rotate by 8), ds_bpermute otherwise
__device__ __forceinline__ float lane_xor(float v, int m) {
  const int x = __float_as_int(v);
  switch (m) {
    case 1: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xf, 0xf, false));
    case 2: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xf, 0xf, false));
    case 4: {
      const int t = __builtin_amdgcn_mov_dpp(x, 0x141, 0xf, 0xf, false);
      return __int_as_float(__builtin_amdgcn_mov_dpp(t, 0x1B, 0xf, 0xf, false));
    }
    case 8: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x128, 0xf, 0xf, false));
    default: return __shfl_xor(v, m);
  }
}

// x[k] += sg * (x[k] of lane l ^ M) for 8 registers, M in {1, 2, 8}: one
// v_fmac_f32 with a DPP operand each (quad permute, or row rotate by 8),
// one rounding.  The leading s_nop covers the wait states a DPP read needs
// after a VALU write of its source; no instruction of the batch reads a
// register another one writes.
template <int M>
__device__ __forceinline__ void fmac_xor8(float* x, float sg) {
  static_assert(M == 1 || M == 2 || M == 8, "DPP distance");
#if defined(__HIP_DEVICE_COMPILE__)
#define TQ_F(I, CTL) "v_fmac_f32_dpp %" #I ", %" #I ", %8 " CTL " row_mask:0xf bank_mask:0xf\n\t"
#define TQ_F8(CTL)                                                                          \
  asm volatile("s_nop 1\n\t" TQ_F(0, CTL) TQ_F(1, CTL) TQ_F(2, CTL) TQ_F(3, CTL)           \
                   TQ_F(4, CTL) TQ_F(5, CTL) TQ_F(6, CTL) TQ_F(7, CTL)                       \
               : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]),     \
                 "+v"(x[6]), "+v"(x[7])                                                      \
               : "v"(sg))
  if constexpr (M == 1) TQ_F8("quad_perm:[1,0,3,2]");
  else if constexpr (M == 2) TQ_F8("quad_perm:[2,3,0,1]");
  else TQ_F8("row_ror:8");
#undef TQ_F8
#undef TQ_F
#else
  for (int k = 0; k < 8; k++) x[k] = __builtin_fmaf(lane_xor(x[k], M), sg, x[k]);
#endif
}

// one cross-lane stage over E registers: v += sg * v of lane l ^ m
template <int E>
__device__ __forceinline__ void fmac_xor(float (&v)[E], int m, float sg) {
  static_assert(E % 8 == 0, "registers in batches of 8");
#pragma unroll
  for (int b = 0; b < E; b += 8) {
    if (m == 1) fmac_xor8<1>(v + b, sg);
    else if (m == 2) fmac_xor8<2>(v + b, sg);
    else if (m == 8) fmac_xor8<8>(v + b, sg);
    else {
#pragma unroll
      for (int k = 0; k < 8; k++) v[b + k] = __builtin_fmaf(lane_xor(v[b + k], m), sg, v[b + k]);
    }
  }
}

// Walsh-Hadamard transform (unnormalised, ascending stride) of the PD dims
// the P lanes of a vector hold: v[8 i + c] = dim 8 (p + P i) + c.
template <int E, int P>
__device__ __forceinline__ void fwht_group(float (&v)[E], int p) {
#pragma unroll
  for (int h = 1; h < 8; h <<= 1)
#pragma unroll
    for (int i = 0; i < E; i++)
      if ((i & h) == 0) {
        const float a = v[i], b = v[i + h];
        v[i] = a + b;
        v[i + h] = a - b;
      }
#pragma unroll
  for (int m = 1; m < P; m <<= 1) {
    const float sg = (p & m) ? -1.0f : 1.0f;  // own + sg * partner: one v_fmac with DPP
    fmac_xor<E>(v, m, sg);
  }
#pragma unroll
  for (int h = 8; h < E; h <<= 1)  // chunk index bits: stride 8 P h / 8
#pragma unroll
    for (int i = 0; i < E; i++)
      if ((i & h) == 0) {
        const float a = v[i], b = v[i + h];
        v[i] = a + b;
        v[i + h] = a - b;
      }
}

// The same transform with lane p holding the E consecutive dims p E .. p E +
// E - 1 (the quantize kernel's layout): strides 1 .. E/2 in-lane, E .. 4P
// across lanes.
template <int E, int P>
__device__ __forceinline__ void fwht_contig(float (&v)[E], int p) {
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
  for (int m = 1; m < P; m <<= 1) {
    const float sg = (p & m) ? -1.0f : 1.0f;
    fmac_xor<E>(v, m, sg);
  }
}

// Both transforms leave lane p with tau_p times the reference's values, tau_p
// = (-1)^popcount(p): a cross-lane stage keeps own + sg * partner, which on
// the upper lane is own - partner = -(partner - own), the reference's value
// negated (exactly); lanes paired in a stage share tau from the earlier
// stages, and negation commutes with the in-lane stages.  The scale 1/sqrt(pd)
// then takes tau: (tau v) * (tau s) == v * s bit for bit.
template <int P>
__device__ __forceinline__ float tau_scale(float inv_sqrt_pd, int p) {
  return (__builtin_popcount(p & (P - 1)) & 1) ? -inv_sqrt_pd : inv_sqrt_pd;
}

// fp32 value with the sign of a +-1 sign value folded in (exact: s * v)
__device__ __forceinline__ float apply_sign(float v, float s) {
  return __uint_as_float(__float_as_uint(v) ^ (__float_as_uint(s) & 0x80000000u));
}

// code = #{j : b_j < y} (torch.bucketize; NaN takes the top code) by a
// binary search over the sorted boundaries in LDS: BITS dependent LDS reads.
template <int BITS>
__device__ __forceinline__ int search_code(float y, const float* bnd) {
  int c = 0;
#pragma unroll
  for (int s = BITS - 1; s >= 0; s--) {
    const int cand = c + (1 << s);
    c = bnd[cand - 1] < y ? cand : c;
  }
  return y != y ? (1 << BITS) - 1 : c;
}

// The same code from one LDS lookup, for a codebook symmetric about a middle
// boundary 0 (b[M-1+k] == -b[M-1-k], M = 2^(BITS-1)).  With a = |y| as
// integer bits (positive floats order as their bits), bin = clamp((a >> 20)
// - base, 0, 63) is a 1/8-binade bin; the host builds the table so that each
// bin holds at most one positive boundary B (bits; all ones if none) and
// below = M + #{positive boundaries under the bin}, bins 0..7 lying under the
// smallest positive boundary and bin 63 over the largest.  For y > 0 (and
// NaN, which lands in bin 63): code = below + (a > B).  For y <= 0, code =
// (M - 1) - #{P <= |y|} = (2M - 1) - (below + (a >= B)), and a >= B is
// a + 1 > B.
template <int BITS>
__device__ __forceinline__ int bin_code(float y, const uint2* bins, int base) {
  constexpr uint32_t kTop = (1u << BITS) - 1u;
  const uint32_t a = __float_as_uint(y) & 0x7fffffffu;
  const bool pos = !(y <= 0.0f);
  const int bin = min(max((int)(a >> 20) - base, 0), 63);
  const uint2 e = bins[bin];
  const uint32_t t = e.y + ((pos ? a : a + 1u) > e.x ? 1u : 0u);
  return (int)(pos ? t : kTop - t);
}

// Quantize: lane p of a vector holds its E consecutive dims p E .. p E + E - 1
// (whole 16-byte pieces per load, and its E / per code bytes contiguous for
// the stores); measured faster here than the dequantize kernel's chunk
// layout (127 against 161 us on 1M x 128 at 4 bits).
//
// With RES (TurboQuantProd's first stage, reference quantizer.py:137-143) the
// row also reads its codes back as the dequantize kernel does (centroids,
// the same ascending-stride FWHT, scale, sign, norm: the same fp32 bits),
// forms the residual r = x - x_hat over the first dim dims, its norm
// rn = max(||r||, 1e-8) (stored) and r / rn correctly rounded, left in v
// (0 beyond dim).  Every lane of the workgroup runs this, live or not (the
// lane exchanges need the whole vector group); only live rows store.
template <int PD>
__device__ __forceinline__ void load_row(const MseParams& p, int64_t row, int sub,
                                         float (&v)[MseGeom<PD>::E]) {
  constexpr int E = MseGeom<PD>::E;
  const bool live = row < p.n;
  const int d0 = sub * E;
  if (live && p.dim == PD) {
    const float4* src = reinterpret_cast<const float4*>(p.x + row * PD + d0);
#pragma unroll
    for (int i = 0; i < E / 4; i++) {
      const float4 f = src[i];
      v[4 * i] = f.x;
      v[4 * i + 1] = f.y;
      v[4 * i + 2] = f.z;
      v[4 * i + 3] = f.w;
    }
  } else {
    const float* src = p.x + (live ? row : 0) * p.dim;
#pragma unroll
    for (int i = 0; i < E; i++) v[i] = (live && d0 + i < p.dim) ? src[d0 + i] : 0.0f;
  }
}

// v holds the row as load_row leaves it
template <int PD, int BITS, bool RES>
__device__ __forceinline__ void quantize_row(const MseParams& p, const float* bnd,
                                             const uint2* bins, const float* cen, int64_t row,
                                             int sub, float (&v)[MseGeom<PD>::E]) {
#pragma clang fp contract(off)
  using MG = MseGeom<PD>;
  constexpr int P = MG::P, E = MG::E;
  constexpr int PER = BITS == 3 ? 2 : 8 / BITS;  // codes per byte
  constexpr int NB = E / PER;                    // packed bytes per lane
  const bool live = row < p.n;
  const int d0 = sub * E;
  float xo[RES ? E : 1];
  if constexpr (RES) {
#pragma unroll
    for (int i = 0; i < E; i++) xo[i] = v[i];
  }
  // ||x||: the lane's squares in dim order, then across the vector's lanes
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < E; i++) ss = __builtin_fmaf(v[i], v[i], ss);
#pragma unroll
  for (int m = 1; m < P; m <<= 1) ss += lane_xor(ss, m);
  const float sq = sqrtf(ss);
  const float nrm = sq < 1e-8f ? 1e-8f : sq;  // torch's clamp(min=1e-8), NaN kept
  // x / n correctly rounded without a division per element: with y the
  // correctly rounded 1/n, q = RN(x y) and the exact remainder r = x - q n
  // (one fma), RN(q + r y) is the correctly rounded quotient (Markstein's
  // theorem, IBM J. Res. Dev. 34(1), 1990), for every finite x here (|x / n|
  // <= 1, no overflow; x = 0 gives +-0 as x / n does)
  const float yr = 1.0f / nrm;
  float sgn[E];  // the lane's signs, float4 loads (signs is 16-byte aligned)
#pragma unroll
  for (int i = 0; i < E / 4; i++) {
    const float4 f = reinterpret_cast<const float4*>(p.signs + d0)[i];
    sgn[4 * i] = f.x;
    sgn[4 * i + 1] = f.y;
    sgn[4 * i + 2] = f.z;
    sgn[4 * i + 3] = f.w;
  }
#pragma unroll
  for (int i = 0; i < E; i++) {
    const float q = v[i] * yr;
    const float r = __builtin_fmaf(-q, nrm, v[i]);
    v[i] = apply_sign(__builtin_fmaf(r, yr, q), sgn[i]);
  }
  fwht_contig<E, P>(v, sub);
  const float ts = tau_scale<P>(p.inv_sqrt_pd, sub);  // v holds tau * FWHT
  // code = #{j : b_j < y}
  uint32_t word[(NB + 3) / 4] = {};
  auto encode = [&](auto code_of) {
#pragma unroll
    for (int i = 0; i < E; i++) {
      const int c = code_of(v[i] * ts);
      const int byte = i / PER, slot = i % PER;
      word[byte / 4] |= (uint32_t)c << (8 * (byte % 4) + BITS * slot);
      if constexpr (RES) v[i] = cen[c];
    }
  };
  if (p.use_bins)
    encode([&](float y) { return bin_code<BITS>(y, bins, p.bin_base); });
  else
    encode([&](float y) { return search_code<BITS>(y, bnd); });
  if constexpr (RES) {
    fwht_contig<E, P>(v, sub);
    float rs = 0.0f;
#pragma unroll
    for (int i = 0; i < E; i++) {
      const float xh = apply_sign(v[i] * ts, sgn[i]) * nrm;
      v[i] = d0 + i < p.dim ? xo[i] - xh : 0.0f;
      rs = __builtin_fmaf(v[i], v[i], rs);
    }
#pragma unroll
    for (int m = 1; m < P; m <<= 1) rs += lane_xor(rs, m);
    const float rq = sqrtf(rs);
    const float rn = rq < 1e-8f ? 1e-8f : rq;
    const float ry = 1.0f / rn;
#pragma unroll
    for (int i = 0; i < E; i++) {  // r / rn correctly rounded, as x / n above
      const float q = v[i] * ry;
      const float r = __builtin_fmaf(-q, rn, v[i]);
      v[i] = __builtin_fmaf(r, ry, q);
    }
    if (live && sub == 0) p.rnorm[row] = rn;
  }
  if (!live) return;
  if (sub == 0) p.norms[row] = nrm;
  uint8_t* dst = p.packed + row * p.nbytes + sub * NB;
  if constexpr (NB == 1) {
    *dst = (uint8_t)word[0];
  } else if constexpr (NB == 2) {
    *reinterpret_cast<uint16_t*>(dst) = (uint16_t)word[0];
  } else {
#pragma unroll
    for (int k = 0; k < NB / 4; k++) reinterpret_cast<uint32_t*>(dst)[k] = word[k];
  }
}

template <int PD, int BITS, bool RES>
__global__ __launch_bounds__(kMseThreads) void mse_quantize_kernel(MseParams p) {
  using MG = MseGeom<PD>;
  constexpr int P = MG::P, E = MG::E;
  __shared__ float bnd[16];
  __shared__ float cen[16];
  __shared__ uint2 bins[64];
  if (threadIdx.x < 16) bnd[threadIdx.x] = p.table[threadIdx.x];
  if (RES && threadIdx.x >= 16 && threadIdx.x < 32) cen[threadIdx.x - 16] = p.cen[threadIdx.x - 16];
  if (threadIdx.x >= 64 && threadIdx.x < 128)
    bins[threadIdx.x - 64] = uint2{p.bin_b[threadIdx.x - 64], p.bin_n[threadIdx.x - 64]};
  __syncthreads();
  const int lane = threadIdx.x & 63, sub = lane % P;
  const int64_t row = (int64_t)blockIdx.x * MG::VPB + threadIdx.x / P;
  float v[E];
  load_row<PD>(p, row, sub, v);
  quantize_row<PD, BITS, RES>(p, bnd, bins, cen, row, sub, v);
  if constexpr (RES) {
    if (row >= p.n) return;
    const int d0 = sub * E;
    float* rrow = p.resid + row * p.dim;
    if (p.dim == PD) {
#pragma unroll
      for (int i = 0; i < E / 4; i++)
        reinterpret_cast<float4*>(rrow + d0)[i] =
            float4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
    } else {
#pragma unroll
      for (int i = 0; i < E; i++)
        if (d0 + i < p.dim) rrow[d0 + i] = v[i];
    }
  }
}

// Dequantize of one row in the chunk layout (lane p: chunks of 8 dims at
// 8 (p + P i)).  With ADD (TurboQuantProd's dequantize, reference
// quantizer.py:145-158 and qjl.py:46-63) each output gains the QJL term
// arow[d] * (add_scale * gamma) in torch's order: the row's weight first,
// then the product, then the sum; arow may point to global memory or LDS.
// a row's code words (chunk layout) and norm
template <int PD, int BITS>
struct RowCodes {
  uint32_t word[MseGeom<PD>::E / 8];
  float nrm;
};

template <int PD, int BITS>
__device__ __forceinline__ RowCodes<PD, BITS> load_codes(const MseParams& p, int64_t row,
                                                         int sub) {
  using MG = MseGeom<PD>;
  constexpr int P = MG::P, NC = MG::E / 8;
  constexpr int PER = BITS == 3 ? 2 : 8 / BITS;
  constexpr int CB = 8 / PER;
  RowCodes<PD, BITS> rc;
#pragma unroll
  for (int i = 0; i < NC; i++) rc.word[i] = 0u;
  rc.nrm = 0.0f;
  if (row < p.n) {
#pragma unroll
    for (int i = 0; i < NC; i++) {
      const uint8_t* src = p.packed + row * p.nbytes + (sub + P * i) * CB;
      if constexpr (CB == 1) rc.word[i] = *src;
      else if constexpr (CB == 2) rc.word[i] = *reinterpret_cast<const uint16_t*>(src);
      else rc.word[i] = *reinterpret_cast<const uint32_t*>(src);
    }
    rc.nrm = p.norms[row];
  }
  return rc;
}

template <int PD, int BITS, bool ADD>
__device__ __forceinline__ void dequantize_row(const MseParams& p, const float* cen, int64_t row,
                                               int sub, const float* arow,
                                               const RowCodes<PD, BITS>& rc,
                                               float* stage = nullptr) {
#pragma clang fp contract(off)
  using MG = MseGeom<PD>;
  constexpr int P = MG::P, E = MG::E, NC = E / 8;
  constexpr int PER = BITS == 3 ? 2 : 8 / BITS;
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  const bool live = row < p.n;
  const uint32_t* word = rc.word;
  const float nrm = rc.nrm;
  float v[E];
#pragma unroll
  for (int i = 0; i < E; i++) {
    const int k = i % 8;
    v[i] = cen[(word[i / 8] >> (8 * (k / PER) + BITS * (k % PER))) & kMask];
  }
  fwht_group<E, P>(v, sub);
  const float ts = tau_scale<P>(p.inv_sqrt_pd, sub);  // v holds tau * FWHT
  if (!live) return;
  float* orow = p.out + row * p.dim;
  const float wq = ADD ? p.add_scale * p.gamma[row] : 0.0f;
  // the signs of the lane's chunks, two float4 loads per chunk
  float sg[E];
#pragma unroll
  for (int i = 0; i < NC; i++) {
    const float4* sp = reinterpret_cast<const float4*>(p.signs + 8 * (sub + P * i));
    const float4 a = sp[0], b = sp[1];
    sg[8 * i] = a.x;
    sg[8 * i + 1] = a.y;
    sg[8 * i + 2] = a.z;
    sg[8 * i + 3] = a.w;
    sg[8 * i + 4] = b.x;
    sg[8 * i + 5] = b.y;
    sg[8 * i + 6] = b.z;
    sg[8 * i + 7] = b.w;
  }
  auto val = [&](int i) {
    const int d = 8 * (sub + P * (i / 8)) + i % 8;
    const float xm = apply_sign(v[i] * ts, sg[i]) * nrm;
    if constexpr (ADD) return xm + arow[d] * wq;
    else return xm;
  };
  if (p.dim == PD) {
    // into the row's LDS stage (the caller writes it out coalesced), or HBM
    float* const dst = stage ? stage : orow;
#pragma unroll
    for (int i = 0; i < NC; i++) {
      float4* o4 = reinterpret_cast<float4*>(dst + 8 * (sub + P * i));
      o4[0] = float4{val(8 * i), val(8 * i + 1), val(8 * i + 2), val(8 * i + 3)};
      o4[1] = float4{val(8 * i + 4), val(8 * i + 5), val(8 * i + 6), val(8 * i + 7)};
    }
  } else {
#pragma unroll
    for (int i = 0; i < E; i++) {
      const int d = 8 * (sub + P * (i / 8)) + i % 8;
      if (d < p.dim) orow[d] = val(i);
    }
  }
}

// Full-width rows (dim == pd) go out through an LDS stage per wave: the
// wave's 64 / P rows are consecutive in memory, so each store instruction
// writes 1 KB of consecutive bytes (64 lanes x 16 B) instead of 16-byte
// pieces at a 32-byte stride that leave every line half-written.
template <int PD, int BITS, bool ADD>
__global__ __launch_bounds__(kMseThreads) void mse_dequantize_kernel(MseParams p) {
  using MG = MseGeom<PD>;
  constexpr int P = MG::P, VW = 64 / P;  // vectors per wave
  __shared__ float cen[16];
  __shared__ __attribute__((aligned(16))) float stg[kMseThreads / 64][VW * PD];
  if (threadIdx.x < 16) cen[threadIdx.x] = p.table[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int sub = lane % P, vw = lane / P;
  const int64_t row = (int64_t)blockIdx.x * MG::VPB + threadIdx.x / P;
  const bool staged = p.dim == PD;  // uniform
  dequantize_row<PD, BITS, ADD>(p, cen, row, sub,
                                ADD && row < p.n ? p.add + row * p.dim : nullptr,
                                load_codes<PD, BITS>(p, row, sub),
                                staged ? &stg[w][vw * PD] : nullptr);
  if (!staged) return;
  // LDS operations of one wave complete in order; the wave barrier keeps the
  // compiler from moving the reads above the writes
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int64_t row0 = (int64_t)blockIdx.x * MG::VPB + (int64_t)w * VW;
  const int64_t rows = p.n - row0 < VW ? p.n - row0 : VW;
  if (rows <= 0) return;
  const int total = (int)rows * PD;  // floats of the wave's live rows
  float* const dst = p.out + row0 * PD;
#pragma unroll
  for (int k = 4 * lane; k < VW * PD; k += 256)
    if (k < total) *reinterpret_cast<float4*>(dst + k) = *reinterpret_cast<const float4*>(&stg[w][k]);
}

// --------------------------------------------------------------------------
// TurboQuantProd with the QJL projections on the matrix cores (padded size 64
// or 128, so dim <= 128).  The d x d Gaussian matrix S enters as fp16 hi + lo
// halves (S = hi + lo to 22 bits, zero-padded to PD x PD); every product
// S r runs as v_mfma_f32_16x16x32_f16 with fp32 accumulation:
//   quantize:   sign(S r) = sign(hi rh + hi rl + lo rh), r = rh + rl the unit
//               residual split the same way (the dropped lo rl term and the
//               splits' rounding are ~2^-22 of |S_j| |r|, so a sign differs
//               from an fp32 GEMM's only where that GEMM's own rounding could
//               flip it);
//   dequantize: z S = z hi + z lo (z = +-1 exact in fp16).
// Persistent workgroups: each wave loads its 16-row blocks of S (or S^T) into
// registers once and then serves batches of 32 vectors.  C^T = S R^T per
// batch: A = S rows (lane: row l % 16, dims 8 (l / 16) ..), B = the batch's
// vectors from LDS (lane: vector l % 16, the same dims), D = lane: vector
// l % 16, outputs 4 (l / 16) + e.
// --------------------------------------------------------------------------
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct QjlParams {
  const _Float16* s_hi;  // [PD][PD] row-major: quantize S, dequantize S^T
  const _Float16* s_lo;
  int8_t* z;             // quantize out: +-1 [n][dim]
  const int8_t* zin;     // dequantize in: +-1 [n][dim]
  int64_t nbatch;        // ceil(n / 32)
};

template <int PD>
struct QjlGeom {
  static constexpr int NRB = PD / 64;  // 16-row blocks of S per wave (4 waves)
  static constexpr int NKS = PD / 32;  // k-steps of 32 dims
  static constexpr int RS = PD + 8;    // LDS row stride in halves (16-byte pad)
};

template <int PD>
__device__ __forceinline__ void load_s_frags(const QjlParams& q, int w, int lane,
                                             half8_t (&ah)[QjlGeom<PD>::NRB][QjlGeom<PD>::NKS],
                                             half8_t (&al)[QjlGeom<PD>::NRB][QjlGeom<PD>::NKS]) {
  using QG = QjlGeom<PD>;
#pragma unroll
  for (int rb = 0; rb < QG::NRB; rb++)
#pragma unroll
    for (int ks = 0; ks < QG::NKS; ks++) {
      const int64_t off =
          (int64_t)(16 * (QG::NRB * w + rb) + (lane & 15)) * PD + 32 * ks + 8 * (lane >> 4);
      ah[rb][ks] = *reinterpret_cast<const half8_t*>(q.s_hi + off);
      al[rb][ks] = *reinterpret_cast<const half8_t*>(q.s_lo + off);
    }
}

template <int PD, int BITS>
__global__ __launch_bounds__(kMseThreads) void prod_qjl_quantize_kernel(MseParams p, QjlParams q) {
  using MG = MseGeom<PD>;
  using QG = QjlGeom<PD>;
  constexpr int P = MG::P, E = MG::E, RS = QG::RS;
  static_assert(MG::VPB == 32 && (PD == 64 || PD == 128), "32 vectors of <= 128 dims per batch");
  __shared__ float bnd[16];
  __shared__ float cen[16];
  __shared__ uint2 bins[64];
  __shared__ __attribute__((aligned(16))) _Float16 rh[32 * RS];
  __shared__ __attribute__((aligned(16))) _Float16 rl[32 * RS];
  if (threadIdx.x < 16) bnd[threadIdx.x] = p.table[threadIdx.x];
  if (threadIdx.x >= 16 && threadIdx.x < 32) cen[threadIdx.x - 16] = p.cen[threadIdx.x - 16];
  if (threadIdx.x >= 64 && threadIdx.x < 128)
    bins[threadIdx.x - 64] = uint2{p.bin_b[threadIdx.x - 64], p.bin_n[threadIdx.x - 64]};
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, sub = lane % P, vl = threadIdx.x / P;
  half8_t ah[QG::NRB][QG::NKS], al[QG::NRB][QG::NKS];
  load_s_frags<PD>(q, w, lane, ah, al);
  float xn[E];  // the next batch's rows, loaded while this batch computes
  load_row<PD>(p, (int64_t)blockIdx.x * 32 + vl, sub, xn);
  __syncthreads();
  for (int64_t bt = blockIdx.x; bt < q.nbatch; bt += gridDim.x) {
    float v[E];
#pragma unroll
    for (int i = 0; i < E; i++) v[i] = xn[i];
    if (bt + gridDim.x < q.nbatch) load_row<PD>(p, (bt + gridDim.x) * 32 + vl, sub, xn);
    quantize_row<PD, BITS, true>(p, bnd, bins, cen, bt * 32 + vl, sub, v);
    // the unit residual as fp16 hi + lo (v - hi is exact in fp32)
#pragma unroll
    for (int c = 0; c < E / 8; c++) {
      half8_t h, l;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        h[e] = (_Float16)v[8 * c + e];
        l[e] = (_Float16)(v[8 * c + e] - (float)h[e]);
      }
      *reinterpret_cast<half8_t*>(rh + vl * RS + sub * E + 8 * c) = h;
      *reinterpret_cast<half8_t*>(rl + vl * RS + sub * E + 8 * c) = l;
    }
    __syncthreads();
#pragma unroll
    for (int cb = 0; cb < 2; cb++) {
      f32x4 acc[QG::NRB];
#pragma unroll
      for (int rb = 0; rb < QG::NRB; rb++) acc[rb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < QG::NKS; ks++) {
        const int o = (16 * cb + (lane & 15)) * RS + 32 * ks + 8 * (lane >> 4);
        const half8_t bh = *reinterpret_cast<const half8_t*>(rh + o);
        const half8_t bl = *reinterpret_cast<const half8_t*>(rl + o);
#pragma unroll
        for (int rb = 0; rb < QG::NRB; rb++) {
          acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[rb][ks], bh, acc[rb], 0, 0, 0);
          acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[rb][ks], bl, acc[rb], 0, 0, 0);
          acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[rb][ks], bh, acc[rb], 0, 0, 0);
        }
      }
      const int64_t vec = bt * 32 + 16 * cb + (lane & 15);
      if (vec < p.n) {
        int8_t* zrow = q.z + vec * p.dim;
#pragma unroll
        for (int rb = 0; rb < QG::NRB; rb++) {
          const int j = 16 * (QG::NRB * w + rb) + 4 * (lane >> 4);
          uint32_t pk = 0;
#pragma unroll
          for (int e = 0; e < 4; e++)  // +1 for >= 0 (sign() with 0 -> +1), else -1
            pk |= (acc[rb][e] >= 0.0f ? 0x01u : 0xffu) << (8 * e);
          if ((p.dim & 3) == 0) {
            if (j < p.dim) *reinterpret_cast<uint32_t*>(zrow + j) = pk;
          } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
              if (j + e < p.dim) zrow[j + e] = (int8_t)(pk >> (8 * e));
          }
        }
      }
    }
    __syncthreads();  // the next batch rewrites the tile
  }
}

template <int PD, int BITS>
__global__ __launch_bounds__(kMseThreads) void prod_qjl_dequantize_kernel(MseParams p,
                                                                          QjlParams q) {
  using MG = MseGeom<PD>;
  using QG = QjlGeom<PD>;
  constexpr int P = MG::P, TS = PD + 4;  // fp32 term tile row stride
  static_assert(MG::VPB == 32 && (PD == 64 || PD == 128), "32 vectors of <= 128 dims per batch");
  __shared__ float cen[16];
  __shared__ __attribute__((aligned(16))) float term[32 * TS];
  if (threadIdx.x < 16) cen[threadIdx.x] = p.table[threadIdx.x];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, sub = lane % P, vl = threadIdx.x / P;
  half8_t ah[QG::NRB][QG::NKS], al[QG::NRB][QG::NKS];
  load_s_frags<PD>(q, w, lane, ah, al);  // S^T rows
  // the QJL signs of a batch as B fragments: lane (vector l % 16 of column
  // block cb, dims 32 ks + 8 (l / 16) ..) holds 8 signs, 0 past dim or n
  auto load_z = [&](int64_t bt, uint2 (&zb)[2][QG::NKS]) {
#pragma unroll
    for (int cb = 0; cb < 2; cb++) {
      const int64_t vec = bt * 32 + 16 * cb + (lane & 15);
      const bool vlive = vec < p.n;
#pragma unroll
      for (int ks = 0; ks < QG::NKS; ks++) {
        const int k0 = 32 * ks + 8 * (lane >> 4);
        const int8_t* zp = q.zin + (vlive ? vec : 0) * p.dim + k0;
        if (vlive && (p.dim & 7) == 0 && k0 < p.dim) {
          zb[cb][ks] = *reinterpret_cast<const uint2*>(zp);
        } else {
          uint32_t lo = 0, hi = 0;
#pragma unroll
          for (int e = 0; e < 8; e++) {
            const uint32_t byte = (vlive && k0 + e < p.dim) ? (uint8_t)zp[e] : 0u;
            if (e < 4) lo |= byte << (8 * e);
            else hi |= byte << (8 * (e - 4));
          }
          zb[cb][ks] = uint2{lo, hi};
        }
      }
    }
  };
  uint2 zn[2][QG::NKS];
  load_z(blockIdx.x, zn);
  RowCodes<PD, BITS> cn = load_codes<PD, BITS>(p, (int64_t)blockIdx.x * 32 + vl, sub);
  __syncthreads();
  for (int64_t bt = blockIdx.x; bt < q.nbatch; bt += gridDim.x) {
    uint2 zc[2][QG::NKS];
#pragma unroll
    for (int cb = 0; cb < 2; cb++)
#pragma unroll
      for (int ks = 0; ks < QG::NKS; ks++) zc[cb][ks] = zn[cb][ks];
    const RowCodes<PD, BITS> cc = cn;
    if (bt + gridDim.x < q.nbatch) {  // the next batch's inputs, in flight meanwhile
      load_z(bt + gridDim.x, zn);
      cn = load_codes<PD, BITS>(p, (bt + gridDim.x) * 32 + vl, sub);
    }
#pragma unroll
    for (int cb = 0; cb < 2; cb++) {
      f32x4 acc[QG::NRB];
#pragma unroll
      for (int rb = 0; rb < QG::NRB; rb++) acc[rb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < QG::NKS; ks++) {
        half8_t b;
#pragma unroll
        for (int e = 0; e < 8; e++)
          b[e] = (_Float16)(int8_t)((e < 4 ? zc[cb][ks].x : zc[cb][ks].y) >> (8 * (e & 3)));
#pragma unroll
        for (int rb = 0; rb < QG::NRB; rb++) {
          acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[rb][ks], b, acc[rb], 0, 0, 0);
          acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[rb][ks], b, acc[rb], 0, 0, 0);
        }
      }
#pragma unroll
      for (int rb = 0; rb < QG::NRB; rb++) {
        const int j = 16 * (QG::NRB * w + rb) + 4 * (lane >> 4);
        *reinterpret_cast<f32x4*>(term + (16 * cb + (lane & 15)) * TS + j) = acc[rb];
      }
    }
    __syncthreads();
    const int64_t row = bt * 32 + vl;
    // full-width rows: each lane overwrites its own dims of the term row with
    // the output, and the wave writes its 8 consecutive rows out coalesced
    const bool staged = p.dim == PD;  // uniform
    dequantize_row<PD, BITS, true>(p, cen, row, sub, term + vl * TS, cc,
                                   staged ? term + vl * TS : nullptr);
    if (staged) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      constexpr int VW = 64 / P;
      const int64_t row0 = bt * 32 + (int64_t)w * VW;
      const int64_t rows = p.n - row0 < VW ? p.n - row0 : VW;
      if (rows > 0) {
        const int total = (int)rows * PD;
        float* const dst = p.out + row0 * PD;
#pragma unroll
        for (int k = 4 * lane; k < VW * PD; k += 256)
          if (k < total)
            *reinterpret_cast<float4*>(dst + k) = *reinterpret_cast<const float4*>(
                term + (w * VW + k / PD) * TS + k % PD);
      }
    }
    __syncthreads();  // the next batch rewrites the tile
  }
}

template <int PD>
hipError_t launch_mse(bool quant, int bits, const MseParams& p, hipStream_t st) {
  const dim3 grid((unsigned)((p.n + MseGeom<PD>::VPB - 1) / MseGeom<PD>::VPB));
  const dim3 block(kMseThreads);
#define TQ_MSE_CASE(B)                                                                   \
  case B:                                                                                \
    if (quant && p.resid)                                                                \
      hipLaunchKernelGGL((mse_quantize_kernel<PD, B, true>), grid, block, 0, st, p);     \
    else if (quant)                                                                      \
      hipLaunchKernelGGL((mse_quantize_kernel<PD, B, false>), grid, block, 0, st, p);    \
    else if (p.add)                                                                      \
      hipLaunchKernelGGL((mse_dequantize_kernel<PD, B, true>), grid, block, 0, st, p);   \
    else                                                                                 \
      hipLaunchKernelGGL((mse_dequantize_kernel<PD, B, false>), grid, block, 0, st, p);  \
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

// The bin table of bin_code for the 2^bits - 1 sorted boundaries b, when the
// codebook is symmetric about a middle 0 and every 1/8-binade bin holds at
// most one positive boundary (the Lloyd-Max codebooks of 1..4 bits do);
// returns false (binary search) otherwise.
std::atomic<int> g_force_search{0};  // tq_diag_mse_bucketize

bool build_bins(const float* b, int bits, MseParams& p) {
  if (g_force_search.load(std::memory_order_relaxed)) return false;
  const int M = 1 << (bits - 1);
  auto fbits = [](float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
  };
  if (fbits(b[M - 1]) & 0x7fffffffu) return false;  // middle boundary +-0
  for (int k = 1; k < M; k++)
    if (!(b[M - 1 + k] > 0.0f) || fbits(b[M - 1 + k]) != (fbits(b[M - 1 - k]) ^ 0x80000000u))
      return false;
  if (M == 1) {
    p.bin_base = 0;
    for (int i = 0; i < 64; i++) {
      p.bin_b[i] = 0xffffffffu;
      p.bin_n[i] = 1;
    }
    p.use_bins = 1;
    return true;
  }
  const int base = (int)(fbits(b[M]) >> 20) - 8;
  if (base < 0) return false;
  for (int i = 0; i < 64; i++) {
    const uint64_t lo = (uint64_t)(base + i) << 20, hi = (uint64_t)(base + i + 1) << 20;
    int below = 0, inside = 0;
    uint32_t bb = 0xffffffffu;
    for (int k = 1; k < M; k++) {
      const uint64_t u = fbits(b[M - 1 + k]);
      if (u < lo) {
        below++;
      } else if (u < hi) {
        inside++;
        bb = (uint32_t)u;
      }
    }
    if (inside > 1 || (i == 0 && below > 0) || (i == 63 && below + inside != M - 1))
      return false;
    if (i == 63 && inside) return false;  // the top bin holds every larger |y|
    p.bin_b[i] = bb;
    p.bin_n[i] = (uint32_t)(M + below);
  }
  p.bin_base = base;
  p.use_bins = 1;
  return true;
}

// The extra operands of the prod variants (all null for the MSE entry points)
struct ProdArgs {
  const float* centroids = nullptr;  // quantize: read-back table
  float* resid = nullptr;
  float* rnorm = nullptr;
  const float* add = nullptr;  // dequantize
  const float* gamma = nullptr;
  float add_scale = 0.0f;
};

int mse_call(bool quant, const float* x, uint8_t* packed, float* norms, float* out,
             int64_t n, int32_t dim, int32_t padded_dim, int32_t bit_width, const float* signs,
             const float* table, tq_stream_t stream, const char* what,
             const ProdArgs& pa = ProdArgs()) {
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
  const bool prod_q = pa.resid || pa.rnorm || pa.centroids;
  const bool prod_d = pa.add || pa.gamma;
  if ((prod_q && !(pa.resid && pa.rnorm && pa.centroids)) || (prod_d && !(pa.add && pa.gamma))) {
    set_error("%s: null pointer", what);
    return kEinval;
  }
  // full-width rows are read / written as float4, packed rows as dwords
  const uintptr_t al = (uintptr_t)(quant ? (const void*)x : (const void*)out) |
                       (uintptr_t)packed | (uintptr_t)pa.resid | (uintptr_t)signs;
  if ((al & 15) != 0) {
    set_error("%s: x / out, packed and signs must be 16-byte aligned", what);
    return kEinval;
  }
  const int per = bit_width == 3 ? 2 : 8 / bit_width;
  MseParams p;
  p.x = x;
  p.packed = packed;
  p.norms = norms;
  p.out = out;
  p.signs = signs;
  p.resid = pa.resid;
  p.rnorm = pa.rnorm;
  p.add = pa.add;
  p.gamma = pa.gamma;
  p.add_scale = pa.add_scale;
  p.n = n;
  p.dim = dim;
  p.nbytes = padded_dim / per;
  p.inv_sqrt_pd = (float)(1.0 / std::sqrt((double)padded_dim));
  p.levels = 1 << bit_width;
  for (int i = 0; i < 16; i++) p.table[i] = 0.0f;
  for (int i = 0; i < (quant ? p.levels - 1 : p.levels); i++) p.table[i] = table[i];
  for (int i = 0; i < 16; i++) p.cen[i] = (pa.centroids && i < p.levels) ? pa.centroids[i] : 0.0f;
  p.use_bins = 0;
  p.bin_base = 0;
  if (quant) build_bins(table, bit_width, p);
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  switch (padded_dim) {
    case 64: e = launch_mse<64>(quant, bit_width, p, st); break;
    case 128: e = launch_mse<128>(quant, bit_width, p, st); break;
    case 256: e = launch_mse<256>(quant, bit_width, p, st); break;
    case 512: e = launch_mse<512>(quant, bit_width, p, st); break;
    default: e = launch_mse<1024>(quant, bit_width, p, st); break;
  }
  if (e != hipSuccess) set_error("%s: launch failed: %s", what, hipGetErrorString(e));
  return (int)e;
}


// TurboQuantProd with the QJL projections fused (padded size 64 or 128).
int prod_qjl_call(bool quant, const float* x, uint8_t* packed, float* norms, float* out,
                  int64_t n, int32_t dim, int32_t padded_dim, int32_t bits, const float* signs,
                  const float* table, const float* centroids, const _Float16* s_hi,
                  const _Float16* s_lo, int8_t* z, const int8_t* zin, float* rnorm,
                  const float* gamma, tq_stream_t stream) {
  const char* what = quant ? "prod_quantize_qjl" : "prod_dequantize_qjl";
  if (padded_dim != 64 && padded_dim != 128) {
    set_error("%s: padded_dim %d unsupported (64 or 128; larger sizes take the BLAS path)", what,
              padded_dim);
    return kEinval;
  }
  if (bits < 1 || bits > 4) {
    set_error("%s: bit_width %d unsupported (1..4)", what, bits);
    return kEinval;
  }
  if (dim < 1 || dim > padded_dim || 2 * dim <= padded_dim) {
    set_error("%s: padded_dim %d must be the power of two next to dim %d", what, padded_dim, dim);
    return kEinval;
  }
  if (n < 0 || n > ((int64_t)1 << 40)) {
    set_error("%s: vector count %lld out of range", what, (long long)n);
    return kEinval;
  }
  if (!packed || !norms || !signs || !table || !s_hi || !s_lo ||
      (quant ? (!x || !centroids || !z || !rnorm) : (!out || !zin || !gamma))) {
    set_error("%s: null pointer", what);
    return kEinval;
  }
  if (n == 0) return 0;
  const uintptr_t al = (uintptr_t)(quant ? (const void*)x : (const void*)out) |
                       (uintptr_t)packed | (uintptr_t)s_hi | (uintptr_t)s_lo | (uintptr_t)signs;
  if ((al & 15) != 0) {
    set_error("%s: x / out, packed, signs and the S halves must be 16-byte aligned", what);
    return kEinval;
  }
  if ((((uintptr_t)z | (uintptr_t)zin) & 7) != 0) {
    set_error("%s: qjl_signs must be 8-byte aligned", what);
    return kEinval;
  }
  const int per = bits == 3 ? 2 : 8 / bits;
  MseParams p;
  p.x = x;
  p.packed = packed;
  p.norms = norms;
  p.out = out;
  p.signs = signs;
  p.resid = nullptr;
  p.rnorm = rnorm;
  p.add = nullptr;
  p.gamma = gamma;
  p.add_scale = (float)(std::sqrt(M_PI / 2.0) / dim);
  p.n = n;
  p.dim = dim;
  p.nbytes = padded_dim / per;
  p.inv_sqrt_pd = (float)(1.0 / std::sqrt((double)padded_dim));
  p.levels = 1 << bits;
  for (int i = 0; i < 16; i++) {
    p.table[i] = i < (quant ? p.levels - 1 : p.levels) ? table[i] : 0.0f;
    p.cen[i] = (centroids && i < p.levels) ? centroids[i] : 0.0f;
  }
  p.use_bins = 0;
  p.bin_base = 0;
  if (quant) build_bins(table, bits, p);
  QjlParams q;
  q.s_hi = s_hi;
  q.s_lo = s_lo;
  q.z = z;
  q.zin = zin;
  q.nbatch = (n + 31) / 32;
  // persistent: the resident workgroups of the whole chip, each loading its
  // S blocks once (occupancy queried per kernel, once)
  const int cus = device_cus();
  const dim3 block(kMseThreads);
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  auto grid_for = [&](const void* fn, std::atomic<int>& per_cu) {
    int b = per_cu.load(std::memory_order_relaxed);
    if (b == 0) {
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, fn, kMseThreads, 0) != hipSuccess ||
          b < 1)
        b = 1;
      per_cu.store(b, std::memory_order_relaxed);
    }
    const int64_t cap = (int64_t)(cus > 0 ? cus : 256) * b;
    return dim3((unsigned)(q.nbatch < cap ? q.nbatch : cap));
  };
#define TQ_QJL_CASE(PD, B)                                                                      \
  if (padded_dim == PD && bits == B) {                                                         \
    static std::atomic<int> occ_q{0}, occ_d{0};                                                \
    if (quant)                                                                                 \
      hipLaunchKernelGGL((prod_qjl_quantize_kernel<PD, B>),                                    \
                         grid_for((const void*)prod_qjl_quantize_kernel<PD, B>, occ_q), block, \
                         0, st, p, q);                                                         \
    else                                                                                       \
      hipLaunchKernelGGL((prod_qjl_dequantize_kernel<PD, B>),                                  \
                         grid_for((const void*)prod_qjl_dequantize_kernel<PD, B>, occ_d),      \
                         block, 0, st, p, q);                                                  \
  }
  TQ_QJL_CASE(64, 1)
  TQ_QJL_CASE(64, 2)
  TQ_QJL_CASE(64, 3)
  TQ_QJL_CASE(64, 4)
  TQ_QJL_CASE(128, 1)
  TQ_QJL_CASE(128, 2)
  TQ_QJL_CASE(128, 3)
  TQ_QJL_CASE(128, 4)
#undef TQ_QJL_CASE
  const hipError_t e = hipGetLastError();
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
                      signs, boundaries, stream, "mse_quantize");
}

extern "C" int tq_mse_dequantize(const uint8_t* packed, const float* norms, int64_t num_vectors,
                                 int32_t dim, int32_t padded_dim, int32_t bit_width,
                                 const float* signs, const float* centroids, float* out,
                                 tq_stream_t stream) {
  return tq::mse_call(false, nullptr, const_cast<uint8_t*>(packed), const_cast<float*>(norms),
                      out, num_vectors, dim, padded_dim, bit_width, signs, centroids, stream,
                      "mse_dequantize");
}

extern "C" int tq_prod_quantize(const float* x, int64_t num_vectors, int32_t dim,
                                int32_t padded_dim, int32_t mse_bit_width, const float* signs,
                                const float* boundaries, const float* centroids, uint8_t* packed,
                                float* norms, float* residual_unit, float* residual_norms,
                                tq_stream_t stream) {
  tq::ProdArgs pa;
  pa.centroids = centroids;
  pa.resid = residual_unit;
  pa.rnorm = residual_norms;
  if (!centroids || !residual_unit || !residual_norms) {
    tq::set_error("prod_quantize: null pointer");
    return tq::kEinval;
  }
  return tq::mse_call(true, x, packed, norms, nullptr, num_vectors, dim, padded_dim,
                      mse_bit_width, signs, boundaries, stream, "prod_quantize", pa);
}

extern "C" int tq_prod_dequantize(const uint8_t* packed, const float* norms,
                                  const float* qjl_term, const float* residual_norms,
                                  int64_t num_vectors, int32_t dim, int32_t padded_dim,
                                  int32_t mse_bit_width, const float* signs,
                                  const float* centroids, float* out, tq_stream_t stream) {
  tq::ProdArgs pa;
  pa.add = qjl_term;
  pa.gamma = residual_norms;
  pa.add_scale = (float)(std::sqrt(M_PI / 2.0) / dim);
  if (!qjl_term || !residual_norms) {
    tq::set_error("prod_dequantize: null pointer");
    return tq::kEinval;
  }
  return tq::mse_call(false, nullptr, const_cast<uint8_t*>(packed), const_cast<float*>(norms),
                      out, num_vectors, dim, padded_dim, mse_bit_width, signs, centroids, stream,
                      "prod_dequantize", pa);
}

extern "C" int tq_prod_quantize_qjl(const float* x, int64_t num_vectors, int32_t dim,
                                    int32_t padded_dim, int32_t mse_bit_width, const float* signs,
                                    const float* boundaries, const float* centroids,
                                    const void* s_hi, const void* s_lo, uint8_t* packed,
                                    float* norms, int8_t* qjl_signs, float* residual_norms,
                                    tq_stream_t stream) {
  return tq::prod_qjl_call(true, x, packed, norms, nullptr, num_vectors, dim, padded_dim,
                           mse_bit_width, signs, boundaries, centroids,
                           static_cast<const _Float16*>(s_hi), static_cast<const _Float16*>(s_lo),
                           qjl_signs, nullptr, residual_norms, nullptr, stream);
}

extern "C" int tq_prod_dequantize_qjl(const uint8_t* packed, const float* norms,
                                      const int8_t* qjl_signs, const float* residual_norms,
                                      int64_t num_vectors, int32_t dim, int32_t padded_dim,
                                      int32_t mse_bit_width, const float* signs,
                                      const float* centroids, const void* st_hi,
                                      const void* st_lo, float* out, tq_stream_t stream) {
  return tq::prod_qjl_call(false, nullptr, const_cast<uint8_t*>(packed),
                           const_cast<float*>(norms), out, num_vectors, dim, padded_dim,
                           mse_bit_width, signs, centroids, nullptr,
                           static_cast<const _Float16*>(st_hi), static_cast<const _Float16*>(st_lo),
                           nullptr, qjl_signs, nullptr, residual_norms, stream);
}

extern "C" int tq_diag_mse_bucketize(int32_t force_search) {
  tq::g_force_search.store(force_search ? 1 : 0, std::memory_order_relaxed);
  return 0;
}
