/*
 * Scalar C restatement of the integer / bit-exact parts of the bitcache path.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (via ctypes) to cross-check the
 * numpy oracle in oracle/oracle.py.  It is written independently of the numpy
 * code: it simulates the reference kernels' 128-thread block literally (per
 * "thread" strided accumulation, then the shared-memory tree) and carries its
 * own IEEE binary16 conversions instead of relying on numpy's.
 *
 * Built with -ffp-contract=off and without fast-math so every float operation
 * is a single IEEE-754 binary32 operation, as written.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define NTHREADS 128 /* blockDim.x of the reference encode kernels (src/binary_encode.cu:72) */

/* ---- IEEE binary16 <-> binary32 ---------------------------------------- */
float orc_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400) == 0);
            man &= 0x3ff;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* round-to-nearest-even float -> half (what __float2half does) */
uint16_t orc_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xff;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff) { /* inf / nan */
        if (man) return (uint16_t)(sign | 0x7e00u);
        return (uint16_t)(sign | 0x7c00u);
    }
    int e = (int)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
    if (e <= 0) {                                      /* subnormal or zero */
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        int shift = 14 - e; /* 24-bit mantissa -> (10 + e)-bit */
        uint32_t hm = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t hm = man >> 13;
    uint32_t rem = man & 0x1fffu;
    uint16_t h = (uint16_t)(sign | ((uint32_t)e << 10) | hm);
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1))) h++; /* may carry into exponent: correct */
    return h;
}

/* ---- block simulation of the encode reduction -------------------------- */
/* src/binary_encode.cu:31-53: per-thread strided |x| sum, then tree. */
static float block_abs_sum(const float* v, int d) {
    float partial[NTHREADS];
    for (int t = 0; t < NTHREADS; t++) {
        float local = 0.0f;
        for (int i = t; i < d; i += NTHREADS) local += fabsf(v[i]);
        partial[t] = local;
    }
    for (int stride = NTHREADS / 2; stride > 0; stride >>= 1)
        for (int t = 0; t < stride; t++) partial[t] += partial[t + stride];
    return partial[0];
}

/* src/residual.cu:30-53: per-thread fmaxf from 0.0f, then fmaxf tree. */
static float block_abs_max(const float* r, int d) {
    float partial[NTHREADS];
    for (int t = 0; t < NTHREADS; t++) {
        float local = 0.0f;
        for (int i = t; i < d; i += NTHREADS) local = fmaxf(local, fabsf(r[i]));
        partial[t] = local;
    }
    for (int stride = NTHREADS / 2; stride > 0; stride >>= 1)
        for (int t = 0; t < stride; t++) partial[t] = fmaxf(partial[t], partial[t + stride]);
    return partial[0];
}

/* __float2int_rn: round half to even; NaN -> 0; saturating. */
static int f2i_rn(float v) {
    if (v != v) return 0;
    if (v >= 2147483520.0f) return 2147483647;
    if (v <= -2147483648.0f) return (-2147483647 - 1);
    return (int)nearbyintf(v);
}

/* binary_encode_kernel (src/binary_encode.cu:8-60) for n vectors. */
void orc_binary_encode(const uint16_t* x, int n, int d, uint32_t* words, uint16_t* scale16,
                       float* mean32) {
    float v[256];
    int nw = d / 32;
    for (int k = 0; k < n; k++) {
        for (int i = 0; i < d; i++) v[i] = orc_half_to_float(x[(long)k * d + i]);
        for (int w = 0; w < nw; w++) words[(long)k * nw + w] = 0u;
        for (int i = 0; i < d; i++)
            if (v[i] >= 0.0f) words[(long)k * nw + i / 32] |= 1u << (i % 32);
        float mean = block_abs_sum(v, d) / (float)d;
        mean32[k] = mean;
        scale16[k] = orc_float_to_half(mean);
    }
}

/* residual_encode_kernel (src/residual.cu:9-78) given bits and the scale
 * the residual is taken against (fp16-rounded for the two-step path, fp32 mean
 * for online_encode_token, src/online_encode.cu:74,88). */
void orc_residual_encode(const uint16_t* x, const uint32_t* words, const float* s, int n, int d,
                         int8_t* codes, uint16_t* rscale16) {
    float r[256];
    int nw = d / 32;
    for (int k = 0; k < n; k++) {
        float sb = s[k];
        for (int i = 0; i < d; i++) {
            int bit = (words[(long)k * nw + i / 32] >> (i % 32)) & 1u;
            float rec = bit ? sb : -sb;
            r[i] = orc_half_to_float(x[(long)k * d + i]) - rec;
        }
        float absmax = block_abs_max(r, d);
        float inv = (absmax > 0.0f) ? (7.0f / absmax) : 0.0f;
        rscale16[k] = orc_float_to_half(absmax);
        for (int i = 0; i < d; i++) {
            int q = f2i_rn(r[i] * inv);
            q = q < -7 ? -7 : (q > 7 ? 7 : q);
            codes[(long)k * d + i] = (int8_t)q;
        }
    }
}

/* pack_sign_bits + sequential scale_q (src/xnor_dot.cuh:36-52;
 * src/compensated_attention.cu:58-67). */
void orc_query_prep(const uint16_t* q, int nq, int d, uint32_t* qwords, float* scale_q) {
    int nw = d / 32;
    for (int k = 0; k < nq; k++) {
        float acc = 0.0f;
        for (int w = 0; w < nw; w++) qwords[(long)k * nw + w] = 0u;
        for (int i = 0; i < d; i++) {
            float v = orc_half_to_float(q[(long)k * d + i]);
            if (v >= 0.0f) qwords[(long)k * nw + i / 32] |= 1u << (i % 32);
            acc += fabsf(v);
        }
        scale_q[k] = acc / (float)d;
    }
}

/* Tree-order scale_q of compute_head_entropy_kernel (src/adaptive_precision.cu:46-59). */
void orc_query_prep_tree(const uint16_t* q, int nq, int d, uint32_t* qwords, float* scale_q) {
    float v[256];
    for (int k = 0; k < nq; k++) {
        for (int i = 0; i < d; i++) v[i] = orc_half_to_float(q[(long)k * d + i]);
        int nw = d / 32;
        for (int w = 0; w < nw; w++) qwords[(long)k * nw + w] = 0u;
        for (int i = 0; i < d; i++)
            if (v[i] >= 0.0f) qwords[(long)k * nw + i / 32] |= 1u << (i % 32);
        scale_q[k] = block_abs_sum(v, d) / (float)d;
    }
}

/* xnor_dot (src/xnor_dot.cuh:14-31) for S keys of one query; also popcounts. */
void orc_xnor_scores(const uint32_t* qw, float scale_q, const uint32_t* kw, const uint16_t* ks,
                     int S, int d, int32_t* pc_out, float* xdot_out) {
    int nw = d / 32;
    for (int s = 0; s < S; s++) {
        int pc = 0;
        for (int w = 0; w < nw; w++) pc += __builtin_popcount(~(qw[w] ^ kw[(long)s * nw + w]));
        pc_out[s] = pc;
        float sk = orc_half_to_float(ks[s]);
        xdot_out[s] = scale_q * sk * (float)(2 * pc - d);
    }
}

/* compute_head_entropy_kernel's final combination for one head, two passes
 * over already computed (no 1/sqrt(d)) scores (src/adaptive_precision.cu:65-129). */
float orc_entropy(const float* score, int S) {
    float M = -1e30f;
    for (int s = 0; s < S; s++) M = fmaxf(M, score[s]);
    float Z = 0.0f, W = 0.0f;
    for (int s = 0; s < S; s++) {
        float e = expf(score[s] - M);
        Z += e;
        W += e * score[s];
    }
    float logZ = logf(Z) + M;
    return logZ - W / fmaxf(Z, 1e-12f);
}

int orc_abi_version(void) { return 1; }
