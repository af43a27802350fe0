/*
 * tq_oracle.c -- CPU restatement of TurboQuant's quantized paged-KV hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * kernels in turboquant_amd/csrc.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product path never does.
 *
 * What it restates (citations are into the reference tree):
 *   - write:  csrc/include/turboquant/quantize_write_kernel.cuh:332-431
 *             (quantize_write_hadamard_scatter_kernel, canonical fp32 op
 *             order of a 32-lane warp holding VEC = pd/32 dims per lane),
 *             host constants csrc/src/quantize_write_binding.cu:207-269,
 *             boundaries quantize_write_kernel.cuh:22-28,
 *             bucketize quantize_write_kernel.cuh:34-46.
 *   - decode: dequantize-then-attend, turboquant/triton_decode_ref.py:89-131
 *             and :264-299, in the rotated domain with the forward rotation
 *             of q and inverse rotation of o as in
 *             csrc/include/flashinfer_decode_turboquant_v5_tc.cuh:206-275 and
 *             :712-765; page walk as in v5_tc.cuh:331-340; codebook
 *             csrc/include/turboquant/page_turbo.cuh:18-23.
 *
 * Build: -O2 -ffp-contract=off (no implicit FMA); the one FMA the canonical
 * order has (the per-lane sum of squares) is written as fmaf().
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define TQ_EXPORT __attribute__((visibility("default")))

/* 16-level Lloyd-Max centroids for N(0,1) (page_turbo.cuh:18-23). */
static const float kCodebook[16] = {
    -2.7326368f, -2.0693470f, -1.6180345f, -1.2562491f,
    -0.9423684f, -0.6567591f, -0.3880823f, -0.1284154f,
     0.1284154f,  0.3880823f,  0.6567591f,  0.9423684f,
     1.2562491f,  1.6180345f,  2.0693470f,  2.7326368f,
};

/* 15 midpoints, as fp32 literals (quantize_write_kernel.cuh:22-28). */
static const float kBoundaries[15] = {
    -2.4009919259139040f, -1.8436907609368955f, -1.4371417912897455f,
    -1.0993087223329937f, -0.7995637494657970f, -0.5224207238480534f,
    -0.2582488430577470f,  0.0000000000000000f,  0.2582488430577470f,
     0.5224207238480534f,  0.7995637494657970f,  1.0993087223329937f,
     1.4371417912897455f,  1.8436907609368955f,  2.4009919259139040f,
};

/* ---------------------------------------------------------------- fp16 -- */

TQ_EXPORT float tq_oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0x1f) {
        bits = sign | 0x7f800000u | (m << 13);
    } else if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else { /* subnormal: m * 2^-24 */
            float f = (float)m * 5.9604644775390625e-08f;
            memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* fp32 -> fp16, round to nearest even (the conversion __float2half does). */
TQ_EXPORT uint16_t tq_oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
    if (a >= 0x477ff000u) /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7c00u);
    if (a < 0x38800000u) { /* below 2^-14: fp16 subnormal or zero */
        if (a < 0x33000000u) /* <= 2^-25 rounds to zero (tie goes to even 0) */
            return (uint16_t)sign;
        uint32_t e = a >> 23;
        uint32_t m = (a & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e;
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((((a >> 23) - 112u) << 10) | ((a & 0x7fffffu) >> 13));
    uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

/* ----------------------------------------------------------- constants -- */

/* 1/sqrt(pd) as the kernels use it.  Exact for 64 and 256; for 128 it is the
 * correctly rounded value 0x3DB504F3 (also what 1.0f/sqrtf(128.0f) gives). */
TQ_EXPORT float tq_oracle_inv_sqrt_pd(int pd) {
    return 1.0f / sqrtf((float)pd);
}

TQ_EXPORT const float* tq_oracle_codebook(void) { return kCodebook; }
TQ_EXPORT const float* tq_oracle_boundaries(void) { return kBoundaries; }

/* Binary search over the 15 scaled boundaries; `val >= b[mid]` goes up, so a
 * value exactly on a boundary takes the upper code (quantize_write_kernel.cuh:34-46). */
TQ_EXPORT int tq_oracle_bucketize(float val, const float* b) {
    int lo = 0, hi = 15;
    for (int i = 0; i < 4; i++) {
        int mid = (lo + hi) >> 1;
        if (mid < 15 && val >= b[mid]) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

/* In-order FWHT butterflies (a+b, a-b) for h = 1, 2, 4, ... (unnormalised). */
TQ_EXPORT void tq_oracle_fwht_f32(float* v, int n) {
    for (int h = 1; h < n; h <<= 1)
        for (int i = 0; i < n; i += 2 * h)
            for (int k = 0; k < h; k++) {
                float a = v[i + k], b = v[i + k + h];
                v[i + k] = a + b;
                v[i + k + h] = a - b;
            }
}

/* ---------------------------------------------------------------- write -- */

/*
 * Quantize one vector in the canonical order of
 * quantize_write_kernel.cuh:332-431 (32 lanes, lane t holds dims t*VEC+i):
 *   1. per-lane ss = fma(x,x,ss) over i ascending,
 *   2. shfl_down tree 16,8,4,2,1 (lane 0 result),
 *   3. l2 = sqrtf(ss), inv = l2 > 1e-8 ? 1/l2 : 0,
 *   4. v = x*inv, v *= sign, FWHT (h ascending), v *= 1/sqrt(pd),
 *   5. code = bucketize(v, b*1/sqrt(pd)), byte k = code[2k]<<4 | code[2k+1],
 *   6. fp16(l2) (round to nearest even) repeated pd/64 times after the codes.
 * x: head_dim floats.  out: qbytes + 2*dc bytes.
 */
TQ_EXPORT void tq_oracle_quantize_vec(const float* x, int head_dim, int pd,
                                      const float* signs, uint8_t* out) {
    float v[256];
    const int VEC = pd / 32;
    for (int d = 0; d < pd; d++) v[d] = d < head_dim ? x[d] : 0.0f;

    float part[32];
    for (int t = 0; t < 32; t++) {
        float ss = 0.0f;
        for (int i = 0; i < VEC; i++) {
            float val = v[t * VEC + i];
            ss = fmaf(val, val, ss);
        }
        part[t] = ss;
    }
    for (int off = 16; off > 0; off >>= 1)
        for (int t = 0; t < off; t++) part[t] = part[t] + part[t + off];
    float l2 = sqrtf(part[0]);
    float inv = (l2 > 1e-8f) ? (1.0f / l2) : 0.0f;

    for (int d = 0; d < pd; d++) v[d] = v[d] * inv;
    for (int d = 0; d < pd; d++) v[d] = v[d] * signs[d];
    tq_oracle_fwht_f32(v, pd);
    const float sc = tq_oracle_inv_sqrt_pd(pd);
    for (int d = 0; d < pd; d++) v[d] = v[d] * sc;

    float bs[15];
    for (int j = 0; j < 15; j++) bs[j] = kBoundaries[j] * sc;

    for (int k = 0; k < pd / 2; k++) {
        int c0 = tq_oracle_bucketize(v[2 * k], bs);
        int c1 = tq_oracle_bucketize(v[2 * k + 1], bs);
        out[k] = (uint8_t)((c0 << 4) | (c1 & 0x0f));
    }
    uint16_t nh = tq_oracle_f32_to_f16(l2);
    const int dc = pd / 64;
    for (int c = 0; c < dc; c++) {
        out[pd / 2 + 2 * c] = (uint8_t)(nh & 0xff);
        out[pd / 2 + 2 * c + 1] = (uint8_t)(nh >> 8);
    }
}

/*
 * Scatter-quantize K and V into the paged cache slabs
 * (quantize_write_binding.cu:207-269 + scatter kernel).  key/value are fp16
 * bit patterns with element (t, h, d) at t*stride_tok + h*stride_head + d.
 * Slots < 0 or >= num_blocks*block_size are skipped.  Pad bytes untouched.
 */
TQ_EXPORT int tq_oracle_write_kv_cache(uint8_t* k_slab, uint8_t* v_slab,
                                       const uint16_t* key, const uint16_t* value,
                                       int64_t k_stride_tok, int64_t k_stride_head,
                                       int64_t v_stride_tok, int64_t v_stride_head,
                                       const float* signs, const int32_t* slots,
                                       int64_t num_tokens, int num_kv_heads,
                                       int head_dim, int pd, int block_size,
                                       int ebs, int64_t num_blocks) {
    if (pd != 64 && pd != 128 && pd != 256) return -22;
    if (head_dim > pd || head_dim <= 0) return -22;
    const int qbytes = pd / 2;
    if (ebs < qbytes + 2 * (pd / 64)) return -22;
    float x[256];
    uint8_t entry[144];
    const int64_t nslots = num_blocks * (int64_t)block_size;
#pragma omp parallel for private(x, entry) schedule(static)
    for (int64_t t = 0; t < num_tokens; t++) {
        int32_t slot = slots[t];
        if (slot < 0 || slot >= nslots) continue;
        int64_t blk = slot / block_size, ent = slot % block_size;
        for (int h = 0; h < num_kv_heads; h++) {
            size_t off = (size_t)(((blk * block_size + ent) * num_kv_heads + h) * ebs);
            for (int kv = 0; kv < 2; kv++) {
                const uint16_t* src = kv == 0 ? key + t * k_stride_tok + h * k_stride_head
                                              : value + t * v_stride_tok + h * v_stride_head;
                for (int d = 0; d < head_dim; d++) x[d] = tq_oracle_f16_to_f32(src[d]);
                tq_oracle_quantize_vec(x, head_dim, pd, signs, entry);
                memcpy((kv == 0 ? k_slab : v_slab) + off, entry, (size_t)(qbytes + 2 * (pd / 64)));
            }
        }
    }
    return 0;
}

/* --------------------------------------------------------------- decode -- */

/* Dequantize one cache entry to the rotated domain:
 * x[d] = codebook[code_d] * (1/sqrt(pd) * norm[d/64])  (v5_tc.cuh:60-92, 356-387). */
static void dequant_entry(const uint8_t* e, int pd, float* out) {
    const float sc = tq_oracle_inv_sqrt_pd(pd);
    for (int d = 0; d < pd; d++) {
        uint8_t byte = e[d / 2];
        int code = (d & 1) ? (byte & 0x0f) : (byte >> 4);
        int chunk = d / 64;
        uint16_t nh = (uint16_t)(e[pd / 2 + 2 * chunk] | (e[pd / 2 + 2 * chunk + 1] << 8));
        float ns = sc * tq_oracle_f16_to_f32(nh);
        out[d] = kCodebook[code] * ns;
    }
}

/*
 * Dequantize-then-attend over the paged cache, one decode token per sequence.
 * q: fp16 bits [B, Hq, pd] at q + b*q_stride_b + h*q_stride_h.
 * Rotated-domain math: q' = FWHT(s*q)/sqrt(pd), scores = q'.K^ * sm_scale,
 * softmax, o' = P V^, o = s * FWHT(o')/sqrt(pd).  signs == NULL: no rotation.
 * Sequence b's token t lives in page indices[indptr[b] + t/block_size],
 * entry t % block_size.  Accumulation in double; out: fp32 [B, Hq, pd].
 * A sequence with seq_len 0 yields zeros.
 */
TQ_EXPORT int tq_oracle_decode(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h,
                               const uint8_t* k_slab, const uint8_t* v_slab,
                               const int32_t* indices, const int32_t* indptr,
                               const int32_t* seq_lens, int batch, int num_qo_heads,
                               int num_kv_heads, int pd, int block_size, int ebs,
                               float sm_scale, const float* signs, float* out) {
    if (pd != 64 && pd != 128 && pd != 256) return -22;
    if (num_kv_heads <= 0 || num_qo_heads % num_kv_heads) return -22;
    const int ratio = num_qo_heads / num_kv_heads;
    const float sc = tq_oracle_inv_sqrt_pd(pd);
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int b = 0; b < batch; b++) {
        for (int kvh = 0; kvh < num_kv_heads; kvh++) {
            const int L = seq_lens[b];
            float qr[16][256];
            double acc[16][256];
            double mx[16], den[16];
            for (int r = 0; r < ratio && r < 16; r++) {
                const uint16_t* qp = q + b * q_stride_b + (int64_t)(kvh * ratio + r) * q_stride_h;
                for (int d = 0; d < pd; d++) qr[r][d] = tq_oracle_f16_to_f32(qp[d]);
                if (signs) {
                    for (int d = 0; d < pd; d++) qr[r][d] = qr[r][d] * signs[d];
                    tq_oracle_fwht_f32(qr[r], pd);
                    for (int d = 0; d < pd; d++) qr[r][d] = qr[r][d] * sc;
                }
                for (int d = 0; d < pd; d++) acc[r][d] = 0.0;
                mx[r] = -INFINITY;
                den[r] = 0.0;
            }
            float kd[256], vd[256];
            for (int t = 0; t < L; t++) {
                int32_t page = indices[indptr[b] + t / block_size];
                int ent = t % block_size;
                size_t off = (size_t)(((int64_t)page * block_size + ent) * num_kv_heads + kvh) * (size_t)ebs;
                dequant_entry(k_slab + off, pd, kd);
                dequant_entry(v_slab + off, pd, vd);
                for (int r = 0; r < ratio; r++) {
                    double s = 0.0;
                    for (int d = 0; d < pd; d++) s += (double)qr[r][d] * (double)kd[d];
                    s *= (double)sm_scale;
                    /* online softmax in double (exact-math equivalent of softmax) */
                    if (s > mx[r]) {
                        double a = exp(mx[r] - s);
                        for (int d = 0; d < pd; d++) acc[r][d] *= a;
                        den[r] *= a;
                        mx[r] = s;
                    }
                    double p = exp(s - mx[r]);
                    den[r] += p;
                    for (int d = 0; d < pd; d++) acc[r][d] += p * (double)vd[d];
                }
            }
            for (int r = 0; r < ratio; r++) {
                float o[256];
                for (int d = 0; d < pd; d++) o[d] = den[r] > 0.0 ? (float)(acc[r][d] / den[r]) : 0.0f;
                if (signs) {
                    tq_oracle_fwht_f32(o, pd);
                    for (int d = 0; d < pd; d++) o[d] = o[d] * sc * signs[d];
                }
                float* op = out + ((int64_t)b * num_qo_heads + kvh * ratio + r) * pd;
                memcpy(op, o, sizeof(float) * (size_t)pd);
            }
        }
    }
    return 0;
}
