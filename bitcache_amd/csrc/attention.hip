// Split-KV decode attention over the compressed cache (binary, compensated and
// adaptive top-k), per-key binary scores, head entropy, the exact fp16
// attention baseline and the split combine.
//
// Work decomposition (one launch): grid.x = key split, grid.y = (b, kv head,
// query-head group).  A 256-thread workgroup (4 wave64) owns one contiguous key
// range of one kv head and G query heads that read that kv head (GQA: every
// key tile is fetched once for all G heads).  Waves take 64-key tiles
// round-robin.  Per tile:
//   score phase  lane = key.  Popcount of the 64-bit sign words against the
//                query's signs, the INT4 residual dot via v_dot2_f32_f16 on
//                nibbles turned into fp16 pairs (see residual_dot_pairs), online
//                softmax in the log2 domain with a wave max per tile.
//   value phase  lane = (32-dim slice c, key subgroup r).  Each lane decodes
//                the sign word and 4 dwords of codes of its keys and
//                accumulates w*sv*sign + w*(rs/7)*n in fp32 registers.
// The workgroup folds its 4 waves into one (m, l, acc[D]) partial per query
// head in the workspace; attn_combine_kernel merges the splits.
#include <math.h>
#include <stdlib.h>

#include <mutex>
#include <vector>

#include "attn.h"

using bc::AttnArgs;
using bc::kLog2e;
using bc::MODE_BINARY;
using bc::MODE_COMP;
using bc::MODE_ADAPTIVE;
using bc::MODE_MIXED;

namespace {

template <int D>
struct QPrep {
    // per query head, in LDS
    uint32_t signs[D / 32];
    uint32_t pairs[D / 8][4];  // fp16 pairs (q[8w+t], q[8w+4+t]) for the nibble dot
    float scale_q;             // sequential mean |q| (src/compensated_attention.cu:65-67)
    float offset;              // 1032 * sum(q): removed from the magic-number dot
};

// Residual dot sum_i q_i * n_i for one key whose codes are D/8 dwords.
// Each dword holds 8 nibbles (element 8w+t in bits 4t..4t+3).  XOR 0x8 turns
// a two's-complement nibble n into u = n + 8 in [0, 15]; OR-ing u into the
// mantissa of fp16 1024.0 (0x6400) gives the exact fp16 value 1024 + u, two
// elements per dword, so v_dot2_f32_f16 accumulates q*(1032 + n).  The
// constant 1032*sum(q) is subtracted once per key.
template <int D>
__device__ __forceinline__ float residual_dot_pairs(const uint32_t* codes, const QPrep<D>& qp) {
    float acc = 0.0f;
#pragma unroll
    for (int w = 0; w < D / 8; w++) {
        const uint32_t x = codes[w] ^ 0x88888888u;
        const uint4 qv = *(const uint4*)qp.pairs[w];
        const uint32_t p0 = (x & 0x000F000Fu) | 0x64006400u;
        const uint32_t p1 = ((x >> 4) & 0x000F000Fu) | 0x64006400u;
        const uint32_t p2 = ((x >> 8) & 0x000F000Fu) | 0x64006400u;
        const uint32_t p3 = ((x >> 12) & 0x000F000Fu) | 0x64006400u;
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, qv.x), __builtin_bit_cast(h2, p0), acc, false);
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, qv.y), __builtin_bit_cast(h2, p1), acc, false);
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, qv.z), __builtin_bit_cast(h2, p2), acc, false);
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, qv.w), __builtin_bit_cast(h2, p3), acc, false);
    }
    return acc - qp.offset;
}

// Fill QPrep for G query heads from global Q (all 256 threads participate).
template <int D, int G>
__device__ void prep_queries(const uint16_t* qbase, QPrep<D>* qp, float* qf_scratch) {
    const int tid = threadIdx.x;
    for (int i = tid; i < G * D; i += blockDim.x) qf_scratch[i] = h2f(qbase[i]);
    __syncthreads();
    for (int i = tid; i < G * (D / 32); i += blockDim.x) {
        const int g = i / (D / 32), w = i % (D / 32);
        uint32_t bits = 0;
        for (int b = 0; b < 32; b++) bits |= (qf_scratch[g * D + 32 * w + b] >= 0.0f ? 1u : 0u) << b;
        qp[g].signs[w] = bits;
    }
    for (int i = tid; i < G * (D / 8) * 4; i += blockDim.x) {
        const int g = i / (D / 2), r = i % (D / 2), w = r / 4, t = r % 4;
        const uint32_t lo = qbase[g * D + 8 * w + t];
        const uint32_t hi = qbase[g * D + 8 * w + 4 + t];
        qp[g].pairs[w][t] = lo | (hi << 16);
    }
    if (tid < G) {
        // sequential fp32 order (element 0 first); the reads are independent
        float acc = 0.0f, sum = 0.0f;
#pragma unroll 32
        for (int i = 0; i < D; i++) {
            acc += fabsf(qf_scratch[tid * D + i]);
            sum += qf_scratch[tid * D + i];
        }
        qp[tid].scale_q = acc / (float)D;
        qp[tid].offset = 1032.0f * sum;
    }
    __syncthreads();
}

template <int D, int G, int MODE>
__global__ __launch_bounds__(256) void attn_split_kernel(AttnArgs a) {
    constexpr int NW = D / 32;            // sign words per key
    constexpr int LPK = D / 32;           // value-phase lanes per key (32 dims each)
    constexpr int R = 64 / LPK;           // key subgroups in the value phase
    constexpr int KPL = (64 + R - 1) / R; // keys per value lane per tile
    constexpr bool RES = MODE != MODE_BINARY;
    // every key's residual data is read (compensated, and per-head modes)
    constexpr bool ALLRES = MODE == MODE_COMP || MODE == MODE_MIXED;

    __shared__ QPrep<D> qp[G];
    __shared__ float qf[G * D];
    __shared__ float2 wl[4][G][64];       // per wave: (2*w*sv, w*rs/7) of each key
    __shared__ uint32_t sel_lds[4][64];   // adaptive: per key bitmask over g
    __shared__ float red[4][64][33];      // value-lane partials (padded)
    __shared__ float wsum[4][G][D];
    __shared__ float wm[4][G], wlsum[4][G];

    const int split = blockIdx.x;
    const int nqg = (a.Hq / a.Hkv) / G;
    // per-head modes: this launch's query-head groups come from its list
    int y = blockIdx.y;
    if constexpr (MODE == MODE_BINARY || MODE == MODE_MIXED) {
        if (a.group_list != nullptr) {
            if (y >= *a.group_count) return;
            y = a.group_list[y];
        }
    }
    const int qg = y % nqg;
    const int bkv = y / nqg;  // b * Hkv + kvh
    const int b = bkv / a.Hkv;
    const int kvh = bkv % a.Hkv;
    const int hq0 = kvh * (a.Hq / a.Hkv) + qg * G;
    const int bhq0 = b * a.Hq + hq0;

    prep_queries<D, G>(a.q + (int64_t)bhq0 * D, qp, qf);

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int key_begin = split * a.chunk;
    const int key_end = min(a.S, key_begin + a.chunk);
    const int64_t kv_base = (int64_t)bkv * a.kv_stride;
    const float isd2 = (1.0f / sqrtf((float)D)) * kLog2e;

    // value-lane coordinates
    const int vc = lane % LPK;
    const int vr = lane / LPK;

    float m[G], lsum[G], off[G];
    float acc[G][32];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -INFINITY;
        lsum[g] = 0.0f;
        off[g] = 0.0f;
#pragma unroll
        for (int k = 0; k < 32; k++) acc[g][k] = 0.0f;
    }

    uint32_t thresh[G];
    int cutoff[G];
    if constexpr (MODE == MODE_ADAPTIVE) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            thresh[g] = a.thresh[bhq0 + g];
            cutoff[g] = a.cutoff[bhq0 + g];
        }
    }
    // per-head modes: which heads of the group add their residual
    bool hm[G];
#pragma unroll
    for (int g = 0; g < G; g++) hm[g] = MODE != MODE_MIXED || a.head_mode[bhq0 + g] != 0;

    for (int t0 = key_begin + wave * 64; t0 < key_end; t0 += 4 * 64) {
        // ---------------- issue value loads (independent of scores)
        uint4 vcodes[KPL];
        uint32_t vsigns[KPL];
#pragma unroll
        for (int k = 0; k < KPL; k++) {
            const int sl = vr + R * k;
            const int s = t0 + sl;
            vcodes[k] = make_uint4(0, 0, 0, 0);
            vsigns[k] = 0;
            if (vr < R && sl < 64 && s < key_end) {
                const int64_t vi = kv_base + s;
                vsigns[k] = ((const uint32_t*)(a.vb.signs + vi * (D / 8)))[vc];
                if constexpr (ALLRES)
                    vcodes[k] = ((const uint4*)(a.vr.codes + vi * (D / 2)))[vc];
            }
        }

        // ---------------- score phase: lane = key
        const int s = t0 + lane;
        const bool valid = s < key_end;
        const int64_t ki = kv_base + (valid ? s : t0);
        const SignWords<D> ks = load_signs<D>(a.kb.signs + ki * (D / 8));
        const float sk = h2f(a.kb.scales[ki]);
        const float svv = h2f(a.vb.scales[ki]);
        float rsk = 0.0f, rsv = 0.0f;
        uint32_t kcodes[D / 8];
        if constexpr (ALLRES) {
            rsk = h2f(a.kr.scales[ki]);
            rsv = h2f(a.vr.scales[ki]);
            const uint4* cp = (const uint4*)(a.kr.codes + ki * (D / 2));
#pragma unroll
            for (int i = 0; i < D / 32; i++) {
                const uint4 c = cp[i];
                kcodes[4 * i] = c.x; kcodes[4 * i + 1] = c.y; kcodes[4 * i + 2] = c.z; kcodes[4 * i + 3] = c.w;
            }
        }

        float sc[G];
        uint32_t selmask = 0;
#pragma unroll
        for (int g = 0; g < G; g++) {
            int pc = 0;
#pragma unroll
            for (int w = 0; w < NW; w++) pc += __builtin_popcount(~(qp[g].signs[w] ^ ks.w[w]));
            const float mq = (float)(2 * pc - D);
            // (scale_q * scale_k) * (2pc - d)   (src/xnor_dot.cuh:30)
            const float xdot = (qp[g].scale_q * sk) * mq;
            if constexpr (MODE == MODE_ADAPTIVE) {
                // above the threshold, or equal to it up to the cutoff index
                const uint32_t key = ordered_key(sk * mq);
                const bool sel = key > thresh[g] || (key == thresh[g] && s <= cutoff[g]);
                selmask |= (sel && valid) ? (1u << g) : 0u;
            }
            sc[g] = xdot;
        }

        if constexpr (MODE == MODE_ADAPTIVE) {
            if (selmask) {
                rsk = h2f(a.kr.scales[ki]);
                rsv = h2f(a.vr.scales[ki]);
                const uint4* cp = (const uint4*)(a.kr.codes + ki * (D / 2));
#pragma unroll
                for (int i = 0; i < D / 32; i++) {
                    const uint4 c = cp[i];
                    kcodes[4 * i] = c.x; kcodes[4 * i + 1] = c.y; kcodes[4 * i + 2] = c.z; kcodes[4 * i + 3] = c.w;
                }
            }
            sel_lds[wave][lane] = selmask;
            if (a.selected != nullptr && valid) {
#pragma unroll
                for (int g = 0; g < G; g++)
                    a.selected[(int64_t)(bhq0 + g) * a.S + s] = (selmask >> g) & 1u;
            }
        }

#pragma unroll
        for (int g = 0; g < G; g++) {
            float score = sc[g];
            if constexpr (ALLRES) {
                if (hm[g]) {
                    const float rdot = residual_dot_pairs<D>(kcodes, qp[g]) * (rsk / 7.0f);
                    score = score + rdot;
                }
            } else if constexpr (MODE == MODE_ADAPTIVE) {
                if ((selmask >> g) & 1u) {
                    const float rdot = residual_dot_pairs<D>(kcodes, qp[g]) * (rsk / 7.0f);
                    score = score + rdot;
                }
            }
            float s2 = valid ? score * isd2 : -INFINITY;
            const float mt = wave_max(s2);
            const float mn = fmaxf(m[g], mt);
            if (mn > m[g]) {
                const float alpha = exp2f(m[g] - mn);
                lsum[g] *= alpha;
                off[g] *= alpha;
#pragma unroll
                for (int k = 0; k < 32; k++) acc[g][k] *= alpha;
                m[g] = mn;
            }
            const float p = valid ? exp2f(s2 - mn) : 0.0f;
            lsum[g] += p;
            float rv = 0.0f;
            if constexpr (ALLRES) rv = hm[g] ? p * (rsv / 7.0f) : 0.0f;
            if constexpr (MODE == MODE_ADAPTIVE) rv = ((selmask >> g) & 1u) ? p * (rsv / 7.0f) : 0.0f;
            wl[wave][g][lane] = make_float2(2.0f * p * svv, rv);
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");

        // ---------------- value phase: lane = (slice vc, subgroup vr)
#pragma unroll
        for (int k = 0; k < KPL; k++) {
            const int sl = vr + R * k;
            const int sv_ = t0 + sl;
            if (!(vr < R && sl < 64 && sv_ < key_end)) continue;
            uint4 codes = vcodes[k];
            if constexpr (MODE == MODE_ADAPTIVE) {
                if (sel_lds[wave][sl] != 0u) {
                    const int64_t vi = kv_base + sv_;
                    codes = ((const uint4*)(a.vr.codes + vi * (D / 2)))[vc];
                }
            }
            const uint32_t sb = vsigns[k];
            float fb[32];
#pragma unroll
            for (int e = 0; e < 32; e++) fb[e] = (float)((sb >> e) & 1u);
            float fu[32];
            if constexpr (RES) {
                const uint32_t cw[4] = {codes.x, codes.y, codes.z, codes.w};
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    const uint32_t x = cw[w] ^ 0x88888888u;
                    const uint32_t lo = x & 0x0F0F0F0Fu;
                    const uint32_t hi = (x >> 4) & 0x0F0F0F0Fu;
                    fu[8 * w + 0] = (float)((lo >> 0) & 0xFFu);
                    fu[8 * w + 2] = (float)((lo >> 8) & 0xFFu);
                    fu[8 * w + 4] = (float)((lo >> 16) & 0xFFu);
                    fu[8 * w + 6] = (float)((lo >> 24) & 0xFFu);
                    fu[8 * w + 1] = (float)((hi >> 0) & 0xFFu);
                    fu[8 * w + 3] = (float)((hi >> 8) & 0xFFu);
                    fu[8 * w + 5] = (float)((hi >> 16) & 0xFFu);
                    fu[8 * w + 7] = (float)((hi >> 24) & 0xFFu);
                }
            }
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float2 wv = wl[wave][g][sl];
                // acc += 2*w*sv*bit - w*sv  +  w*rs/7*u - 8*w*rs/7
                off[g] += 0.5f * wv.x;
#pragma unroll
                for (int e = 0; e < 32; e++) acc[g][e] = fmaf(wv.x, fb[e], acc[g][e]);
                if constexpr (RES) {
                    off[g] += 8.0f * wv.y;
#pragma unroll
                    for (int e = 0; e < 32; e++) acc[g][e] = fmaf(wv.y, fu[e], acc[g][e]);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    }

    // ---------------- fold the workgroup into one partial per query head
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float l_w = wave_sum(lsum[g]);
        if (lane == 0) {
            wm[wave][g] = m[g];
            wlsum[wave][g] = l_w;
        }
#pragma unroll
        for (int e = 0; e < 32; e++) red[wave][lane][e] = acc[g][e] - off[g];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // lane j sums over subgroups for dims j, j + 64, ...
        for (int i = lane; i < D; i += 64) {
            const int c = i / 32, e = i % 32;
            float sum = 0.0f;
            for (int r = 0; r < R; r++) sum += red[wave][r * LPK + c][e];
            wsum[wave][g][i] = sum;
        }
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    for (int i = threadIdx.x; i < G * D; i += blockDim.x) {
        const int g = i / D, d = i % D;
        float M = -INFINITY;
        for (int w = 0; w < 4; w++) M = fmaxf(M, wm[w][g]);
        float accv = 0.0f, lv = 0.0f;
        if (M != -INFINITY) {
            for (int w = 0; w < 4; w++) {
                const float f = (wm[w][g] == -INFINITY) ? 0.0f : exp2f(wm[w][g] - M);
                accv += f * wsum[w][g][d];
                lv += f * wlsum[w][g];
            }
        }
        float* dst = a.ws + ((int64_t)(bhq0 + g) * a.n_splits + split) * (D + 2);
        dst[2 + d] = accv;
        if (d == 0) {
            dst[0] = M;
            dst[1] = lv;
        }
    }
}

// Merge split partials: out = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).
// Same normalisation as the reference (acc * (l > 0 ? 1/l : 0), fp16 store,
// src/compensated_attention.cu:104-108).
// Merge of the split partials of one (b, query head) per block: the maximum,
// weights f_s = 2^(m_s - M) and the total sum are reduced over the splits in
// parallel; then P = 256 / D thread groups each sum a residue class of the
// splits for every dimension, and the groups are added.
constexpr int kMaxSplits = 2048;

__device__ __forceinline__ float block_reduce(float v, bool is_max, float* red) {
    v = is_max ? wave_max(v) : wave_sum(v);
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < nw; w++) r = is_max ? fmaxf(r, red[w]) : r + red[w];
    return r;
}

template <int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* ws, uint16_t* out,
                                                           int n_splits) {
    constexpr int P = 256 / D > 0 ? 256 / D : 1;
    __shared__ float fsh[kMaxSplits];
    __shared__ float red[256];
    const int bh = blockIdx.x, tid = threadIdx.x;
    const float* p = ws + (int64_t)bh * n_splits * (D + 2);
    float m = -INFINITY;
    for (int s = tid; s < n_splits; s += blockDim.x) m = fmaxf(m, p[(int64_t)s * (D + 2)]);
    const float M = block_reduce(m, true, red);
    float l = 0.0f;
    for (int s = tid; s < n_splits; s += blockDim.x) {
        const float ms = p[(int64_t)s * (D + 2)];
        const float f = (ms == -INFINITY) ? 0.0f : exp2f(ms - M);
        fsh[s] = f;
        l += f * p[(int64_t)s * (D + 2) + 1];
    }
    const float L = block_reduce(l, false, red);  // its barriers also publish fsh
    const int part = tid / D, d = tid % D;
    float acc = 0.0f;
    if (part < P) {
#pragma unroll 4
        for (int s = part; s < n_splits; s += P) acc += fsh[s] * p[(int64_t)s * (D + 2) + 2 + d];
    }
    __syncthreads();
    red[tid] = acc;
    __syncthreads();
    if (tid < D) {
        float tot = red[tid];
        for (int q = 1; q < P; q++) tot += red[q * D + tid];
        out[(int64_t)bh * D + tid] = f2h(L > 0.0f ? tot * (1.0f / L) : 0.0f);
    }
}

// ---------------------------------------------------------------- fp16 reference
// Exact attention over dense fp16 K/V [B, Hkv, S, D] with fp32 accumulation,
// the same split / online-softmax structure and partial format as the
// compressed kernels.  A key row (2D bytes) is read by LPR = D/8 lanes, 16
// bytes each, in a slot of LP lanes (LPR rounded up to a power of two; the
// lanes past LPR load nothing and add zeros), so every load instruction
// covers whole rows; a wave takes NR such loads of K and of V per tile
// (TK = NR * 64/LP <= 64 keys).
// q.k: 4 v_dot2_f32_f16 per lane and a sum over the row's lanes (DPP);
// softmax with lane = key; p*v: 8 mixed-precision FMAs per lane, reduced over
// the rows of the tile once at the end.
template <int LPR>
__device__ __forceinline__ float row_sum_f(float v) {
    if constexpr (LPR == 4) {
        v += dpp_f<0x4E>(v);
        v += dpp_f<0xB1>(v);
    } else if constexpr (LPR == 8) {
        v += dpp_f<0x141>(v);   // half mirror
        v += dpp_f<0x4E>(v);
        v += dpp_f<0xB1>(v);
    } else {
        v += dpp_f<0x128>(v);
        v += dpp_f<0x124>(v);
        v += dpp_f<0x122>(v);
        v += dpp_f<0x121>(v);
        if constexpr (LPR == 32) v += swz_f<0x401F>(v);
    }
    return v;
}

template <int D, int G>
__global__ __launch_bounds__(256) void ref_split_kernel(const uint16_t* q, const uint16_t* K,
                                                       const uint16_t* V, int Hq, int Hkv, int S,
                                                       int n_splits, int chunk, float* ws) {
    constexpr int LPR = D / 8;           // lanes holding a key row
    constexpr int LP = LPR <= 4 ? 4 : (LPR <= 8 ? 8 : (LPR <= 16 ? 16 : 32));   // lane slot per row
    constexpr int RPI = 64 / LP;         // rows per load instruction
    constexpr int NR = 8 * RPI <= 64 ? 8 : 64 / RPI;   // loads of K (and of V) per tile
    constexpr int TK = NR * RPI;         // keys per tile (at most 64: lane = key below)
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    __shared__ float sc[4][G][64];
    __shared__ float red[4][RPI][D];
    __shared__ float wsum[4][G][D];
    __shared__ float wm[4][G], wlsum[4][G];

    const int split = blockIdx.x;
    const int nqg = (Hq / Hkv) / G;
    const int qg = blockIdx.y % nqg;
    const int bkv = blockIdx.y / nqg;
    const int b = bkv / Hkv, kvh = bkv % Hkv;
    const int hq0 = kvh * (Hq / Hkv) + qg * G;
    const int bhq0 = b * Hq + hq0;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int row = lane / LP, part = lane % LP;
    const bool act = part < LPR;         // (a lane past the row's 16-byte pieces)
    const int key_begin = split * chunk, key_end = min(S, key_begin + chunk);
    const int64_t base = (int64_t)bkv * S;
    const float isd2 = (1.0f / sqrtf((float)D)) * kLog2e;

    h2 qp[G][4];   // this lane's 8 query dims (part*8 ..) per head
#pragma unroll
    for (int g = 0; g < G; g++) {
        const uint4 w = act ? ((const uint4*)(q + (int64_t)(bhq0 + g) * D))[part] : make_uint4(0, 0, 0, 0);
        qp[g][0] = __builtin_bit_cast(h2, w.x);
        qp[g][1] = __builtin_bit_cast(h2, w.y);
        qp[g][2] = __builtin_bit_cast(h2, w.z);
        qp[g][3] = __builtin_bit_cast(h2, w.w);
    }
    float m[G], lp[G], acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -INFINITY;
        lp[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = 0.0f;
    }
    for (int t0 = key_begin + wave * TK; t0 < key_end; t0 += 4 * TK) {
        uint4 kr[NR], vr[NR];
#pragma unroll
        for (int i = 0; i < NR; i++) {
            const int key = t0 + i * RPI + row;
            const int64_t ki = base + (key < key_end ? key : t0);
            // nontemporal: each instruction reads whole rows once
            const bc_v4u z = {0u, 0u, 0u, 0u};
            const bc_v4u kv = act ? __builtin_nontemporal_load((const bc_v4u*)(K + ki * D) + part) : z;
            const bc_v4u vv = act ? __builtin_nontemporal_load((const bc_v4u*)(V + ki * D) + part) : z;
            kr[i] = make_uint4(kv[0], kv[1], kv[2], kv[3]);
            vr[i] = make_uint4(vv[0], vv[1], vv[2], vv[3]);
        }
        // scores -> LDS (lane = key)
#pragma unroll
        for (int i = 0; i < NR; i++) {
            const bool valid = t0 + i * RPI + row < key_end;
#pragma unroll
            for (int g = 0; g < G; g++) {
                float d = 0.0f;
                d = __builtin_amdgcn_fdot2(qp[g][0], __builtin_bit_cast(h2, kr[i].x), d, false);
                d = __builtin_amdgcn_fdot2(qp[g][1], __builtin_bit_cast(h2, kr[i].y), d, false);
                d = __builtin_amdgcn_fdot2(qp[g][2], __builtin_bit_cast(h2, kr[i].z), d, false);
                d = __builtin_amdgcn_fdot2(qp[g][3], __builtin_bit_cast(h2, kr[i].w), d, false);
                d = row_sum_f<LP>(d);
                if (part == 0) sc[wave][g][i * RPI + row] = valid ? d * isd2 : -INFINITY;
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // online softmax over the tile (lane = key; lanes >= TK hold no key)
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float s2 = lane < TK ? sc[wave][g][lane] : -INFINITY;
            const float mn = fmaxf(m[g], wave_max(s2));
            if (mn > m[g]) {
                const float alpha = exp2f(m[g] - mn);
                lp[g] *= alpha;
#pragma unroll
                for (int e = 0; e < 8; e++) acc[g][e] *= alpha;
                m[g] = mn;
            }
            const float p = s2 == -INFINITY ? 0.0f : exp2f(s2 - mn);
            lp[g] += p;
            if (lane < TK) sc[wave][g][lane] = p;
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // p * v: this lane's 8 dims of the keys of its row
#pragma unroll
        for (int i = 0; i < NR; i++) {
            const uint32_t vw[4] = {vr[i].x, vr[i].y, vr[i].z, vr[i].w};
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float p = sc[wave][g][i * RPI + row];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const h2 hv = __builtin_bit_cast(h2, vw[e]);
                    acc[g][2 * e] = fmaf(p, (float)hv.x, acc[g][2 * e]);
                    acc[g][2 * e + 1] = fmaf(p, (float)hv.y, acc[g][2 * e + 1]);
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
    }
    // per wave: sum the rows, then combine the 4 waves
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float l_w = wave_sum(lp[g]);
        if (lane == 0) {
            wm[wave][g] = m[g];
            wlsum[wave][g] = l_w;
        }
#pragma unroll
        for (int e = 0; e < 8; e++)
            if (act) red[wave][row][part * 8 + e] = acc[g][e];
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        for (int i = lane; i < D; i += 64) {
            float sum = 0.0f;
            for (int r = 0; r < RPI; r++) sum += red[wave][r][i];
            wsum[wave][g][i] = sum;
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    for (int i = threadIdx.x; i < G * D; i += blockDim.x) {
        const int g = i / D, d = i % D;
        float M = -INFINITY;
        for (int w = 0; w < 4; w++) M = fmaxf(M, wm[w][g]);
        float accv = 0.0f, lv = 0.0f;
        if (M != -INFINITY) {
            for (int w = 0; w < 4; w++) {
                const float f = (wm[w][g] == -INFINITY) ? 0.0f : exp2f(wm[w][g] - M);
                accv += f * wsum[w][g][d];
                lv += f * wlsum[w][g];
            }
        }
        float* dst = ws + ((int64_t)(bhq0 + g) * n_splits + split) * (D + 2);
        dst[2 + d] = accv;
        if (d == 0) {
            dst[0] = M;
            dst[1] = lv;
        }
    }
}

// ---------------------------------------------------------------- binary scores
// One workgroup per (key chunk, b, kv head, batch of up to kScoreHeads query
// heads of the group): each key's sign row and scale are read once and scored
// against every head of the batch, one lane per key, kScoreUnroll keys in
// flight per lane.  Exact fp32 score (scale_q*scale_k)*(2pc-d) * (1/sqrt(d)).
constexpr int kScoreHeads = 16;
constexpr int kScoreUnroll = 4;

template <int D>
__global__ __launch_bounds__(256) void scores_kernel(const uint16_t* q, BinPlanes kb, float* scores,
                                                    int32_t* pcs, int Hq, int Hkv, int S,
                                                    int kv_stride, int chunk, int n_hb) {
    constexpr int W = D / 32;
    __shared__ float qf[kScoreHeads][D];
    __shared__ uint32_t qs[kScoreHeads][W];
    __shared__ float sq[kScoreHeads];
    const int G = Hq / Hkv;
    const int hb = blockIdx.y % n_hb, bkv = blockIdx.y / n_hb;
    const int b = bkv / Hkv, kvh = bkv % Hkv;
    const int h0 = kvh * G + hb * kScoreHeads;                 // first query head of the batch
    const int nh = min(kScoreHeads, G - hb * kScoreHeads);
    const uint16_t* qb = q + ((int64_t)b * Hq + h0) * D;
    for (int i = threadIdx.x; i < nh * D; i += blockDim.x) qf[i / D][i % D] = h2f(qb[i]);
    __syncthreads();
    for (int i = threadIdx.x; i < nh * W; i += blockDim.x) {
        const int h = i / W, w = i % W;
        uint32_t bits = 0;
        for (int j = 0; j < 32; j++) bits |= (qf[h][32 * w + j] >= 0.0f ? 1u : 0u) << j;
        qs[h][w] = bits;
    }
    if (threadIdx.x < nh) {
        float acc = 0.0f;
        for (int i = 0; i < D; i++) acc += fabsf(qf[threadIdx.x][i]);  // sequential (src/compensated_attention.cu:65-67)
        sq[threadIdx.x] = acc / (float)D;
    }
    __syncthreads();
    const float isd = 1.0f / sqrtf((float)D);
    const int64_t base = (int64_t)bkv * kv_stride;
    const int k0 = blockIdx.x * chunk, k1 = min(S, k0 + chunk);
    for (int s0 = k0; s0 < k1; s0 += kScoreUnroll * 256) {
        SignWords<D> ks[kScoreUnroll];
        float sk[kScoreUnroll];
#pragma unroll
        for (int u = 0; u < kScoreUnroll; u++) {
            const int s = s0 + u * 256 + (int)threadIdx.x;
            const int64_t ki = base + (s < k1 ? s : k0);        // in range; unused past k1
            ks[u] = load_signs<D, true>(kb.signs + ki * (D / 8));
            sk[u] = h2f(kb.scales[ki]);
        }
#pragma unroll
        for (int u = 0; u < kScoreUnroll; u++) {
            const int s = s0 + u * 256 + (int)threadIdx.x;
            if (s >= k1) continue;
            for (int h = 0; h < nh; h++) {
                int pc = 0;
#pragma unroll
                for (int w = 0; w < W; w++) pc += __builtin_popcount(~(qs[h][w] ^ ks[u].w[w]));
                const int64_t o = ((int64_t)b * Hq + h0 + h) * S + s;
                if (scores) scores[o] = ((sq[h] * sk[u]) * (float)(2 * pc - D)) * isd;
                if (pcs) pcs[o] = pc;
            }
        }
    }
}

// ---------------------------------------------------------------- entropy
// src/adaptive_precision.cu:13-130.  Tree-order scale_q (thread t of 128
// holds |q_t| + |q_{t+128}|, tree s = 64..1), scores without 1/sqrt(d),
// H = (log Z + M) - W / max(Z, 1e-12) with an online (M, Z, W) per thread,
// merged over the block.  A block of T threads takes key chunk blockIdx.y of
// (b, h) = blockIdx.x: with one chunk per head it writes H (T = 1024, the
// entry points without a workspace); with several it writes its (M, Z, W) to
// the workspace and entropy_merge_kernel finishes each head (T = 256, about
// eight blocks per CU: one block per head cannot draw a CU's share of HBM).
constexpr int kEntropyThreads = 1024;
constexpr int kEntPartThreads = 256;
template <int D, int T>
__global__ __launch_bounds__(T) void entropy_kernel(const uint16_t* q, BinPlanes kb, float* out,
                                                    float* ws, int Hq, int Hkv, int S,
                                                    int kv_stride, int chunk) {
    constexpr int NW = T / 64;
    __shared__ float part[128];
    __shared__ uint32_t qs[D / 32];
    __shared__ float sm[NW], sz[NW], sw[NW];
    const int bh = blockIdx.x, c = blockIdx.y;
    const uint16_t* qb = q + (int64_t)bh * D;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid < 128) {
        float local = 0.0f;
        for (int i = tid; i < D; i += 128) local += fabsf(h2f(qb[i]));
        part[tid] = local;
    }
    if (tid < D / 32) {
        uint32_t bits = 0;
        for (int i = 0; i < 32; i++) bits |= (h2f(qb[32 * tid + i]) >= 0.0f ? 1u : 0u) << i;
        qs[tid] = bits;
    }
    __syncthreads();
    for (int st = 64; st > 0; st >>= 1) {
        if (tid < st) part[tid] += part[tid + st];
        __syncthreads();
    }
    const float sq = part[0] / (float)D;
    // query head h of batch b reads kv head h / (Hq / Hkv) of that batch
    const int b = bh / Hq, kvh = (bh % Hq) / (Hq / Hkv);
    const int64_t base = ((int64_t)b * Hkv + kvh) * kv_stride;
    const int k0 = c * chunk, k1 = min(S, k0 + chunk);
    // online (M, Z, W) per thread over keys k0 + tid, + T, ...; four keys'
    // loads in flight per thread
    constexpr int U = 4;
    float M = -1e30f, Z = 0.0f, W = 0.0f;
    for (int s0 = k0 + tid; s0 < k1; s0 += U * T) {
        SignWords<D> ks[U];
        float skv[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int s = s0 + u * T;
            const int64_t i = base + (s < k1 ? s : s0);
            ks[u] = load_signs<D, true>(kb.signs + i * (D / 8));
            skv[u] = h2f(kb.scales[i]);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (s0 + u * T >= k1) break;
            int pc = 0;
#pragma unroll
            for (int w = 0; w < D / 32; w++) pc += __builtin_popcount(~(qs[w] ^ ks[u].w[w]));
            const float sc = sq * skv[u] * (float)(2 * pc - D);
            if (sc > M) {
                const float f = expf(M - sc);
                Z *= f;
                W *= f;
                M = sc;
            }
            const float e = expf(sc - M);
            Z += e;
            W += e * sc;
        }
    }
    // merge: (M, Z, W) of two key sets is (max, Z1 f1 + Z2 f2, W1 f1 + W2 f2)
    // with f_i = e^(M_i - max); a butterfly over each wave, then the waves
    for (int off = 32; off >= 1; off >>= 1) {
        const float m2 = __shfl_xor(M, off, 64), z2 = __shfl_xor(Z, off, 64), w2 = __shfl_xor(W, off, 64);
        const float mm = fmaxf(M, m2);
        const float f1 = expf(M - mm), f2 = expf(m2 - mm);
        Z = Z * f1 + z2 * f2;
        W = W * f1 + w2 * f2;
        M = mm;
    }
    if (lane == 0) {
        sm[wave] = M;
        sz[wave] = Z;
        sw[wave] = W;
    }
    __syncthreads();
    if (tid == 0) {
        float gm = -1e30f;
        for (int i = 0; i < NW; i++) gm = fmaxf(gm, sm[i]);
        float z = 0.0f, w = 0.0f;
        for (int i = 0; i < NW; i++) {
            const float f = expf(sm[i] - gm);
            z += sz[i] * f;
            w += sw[i] * f;
        }
        if (ws != nullptr) {
            float* p = ws + ((int64_t)bh * gridDim.y + c) * 3;
            p[0] = gm;
            p[1] = z;
            p[2] = w;
        } else {
            out[bh] = (logf(z) + gm) - w / fmaxf(z, 1e-12f);
        }
    }
}

// H per (b, h) from its nchunk (M, Z, W) partials (one thread per head)
__global__ void entropy_merge_kernel(const float* ws, float* out, int n, int nchunk) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float* p = ws + (int64_t)i * nchunk * 3;
    float gm = -1e30f;
    for (int c = 0; c < nchunk; c++) gm = fmaxf(gm, p[3 * c]);
    float z = 0.0f, w = 0.0f;
    for (int c = 0; c < nchunk; c++) {
        const float f = expf(p[3 * c] - gm);
        z += p[3 * c + 1] * f;
        w += p[3 * c + 2] * f;
    }
    out[i] = (logf(z) + gm) - w / fmaxf(z, 1e-12f);
}

// Query-head groups of per-head modes, compacted in order: group y (heads
// b*Hq + hq0 .. + G - 1 of grid row y, as the attention kernels map it) goes
// to the binary list when all its heads have mode 0, else to the mixed list.
// One block; lists[0], lists[1] = the counts, the lists from word 64 on.
constexpr int kListThreads = 1024;
constexpr size_t kListHeader = 256;   // bytes before the lists (the two counts)
__global__ __launch_bounds__(kListThreads) void mode_groups_kernel(const uint8_t* head_mode,
                                                                   int32_t* lists, int groups,
                                                                   int nqg, int Hq, int Hkv,
                                                                   int G) {
    __shared__ int wb[kListThreads / 64], wm_[kListThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int32_t* bin_list = lists + kListHeader / sizeof(int32_t);
    int32_t* mix_list = bin_list + groups;
    int nb = 0, nm = 0;   // entries written so far (uniform)
    for (int y0 = 0; y0 < groups; y0 += kListThreads) {
        const int y = y0 + tid;
        bool live = y < groups, res = false;
        if (live) {
            const int qg = y % nqg, bkv = y / nqg;
            const int b = bkv / Hkv, kvh = bkv % Hkv;
            const int bhq0 = b * Hq + kvh * (Hq / Hkv) + qg * G;
            for (int g = 0; g < G; g++) res |= head_mode[bhq0 + g] != 0;
        }
        const uint64_t mb = __ballot(live && !res), mm = __ballot(live && res);
        const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
        if (lane == 0) {
            wb[wave] = __popcll(mb);
            wm_[wave] = __popcll(mm);
        }
        __syncthreads();
        int ob = nb, om = nm;
        for (int w = 0; w < wave; w++) {
            ob += wb[w];
            om += wm_[w];
        }
        if (live && !res) bin_list[ob + __popcll(mb & below)] = y;
        if (live && res) mix_list[om + __popcll(mm & below)] = y;
        for (int w = 0; w < kListThreads / 64; w++) {
            nb += wb[w];
            nm += wm_[w];
        }
        __syncthreads();
    }
    if (tid == 0) {
        lists[0] = nb;
        lists[1] = nm;
    }
}

__global__ void select_kernel(const float* e, uint8_t* modes, int n, float thr) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) modes[i] = e[i] >= thr ? 0 : 1;  // src/adaptive_precision.cu:133-144
}

// ---------------------------------------------------------------- host side
int pick_g(int group) {
    if (group % 8 == 0) return 8;
    if (group % 4 == 0) return 4;
    if (group % 2 == 0) return 2;
    return 1;
}

struct SplitPlan {
    int n_splits, chunk, G;
};

// Key splits per (b, query-head group).  per_cu > 0: the launch is modelled
// as rounds of `per_cu` resident workgroups per CU, a split count s costing
// rounds(s) * (tiles per split + 2), the 2 standing for a workgroup's fixed
// prologue/epilogue/combine cost in tiles; the cheapest s wins (the fewer
// splits on a tie), so a launch that fits is one round of equal workgroups
// and no CU idles at its tail (measured faster on the c2, c4 and c5 shapes).
// per_cu = 0: about 8 workgroups per CU, i.e. several rounds that balance
// per-CU speed differences of a long bandwidth-bound launch (measured faster
// on the 64K-context MHA compensated step); a launch too small for two such
// rounds fills one round of 3 workgroups per CU.
// `cu` is the device's CU count (0: the current device's).
SplitPlan plan_splits(int batch, int hq, int hkv, int S, int per_cu, int cu = 0) {
    SplitPlan p;
    p.G = pick_g(hq / hkv);
    const int64_t groups = (int64_t)batch * hkv * ((hq / hkv) / p.G);
    const int tiles = (S + 63) / 64;
    if (cu <= 0) cu = bc::device_cu_count();
    int max_split = tiles / 8;                   // at least 8 tiles (2 per wave) per split
    if (max_split > kMaxSplits) max_split = kMaxSplits;   // the combine kernel's weight table
    if (max_split < 1) max_split = 1;
    int want = 1;
    if (groups > 0 && tiles > 0 && per_cu > 0) {
        const int64_t slots = (int64_t)per_cu * cu;
        // beyond 4 rounds' worth of splits nothing improves
        const int64_t lim = 4 * slots / groups + 1;
        const int hi = lim < max_split ? (int)lim : max_split;
        double best = 0.0;
        for (int sp = 1; sp <= hi; sp++) {
            const int per = (tiles + sp - 1) / sp;
            const int n = (tiles + per - 1) / per;
            if (n != sp) continue;               // (the same plan as a smaller count)
            const int64_t rounds = (groups * n + slots - 1) / slots;
            const double t = (double)rounds * (per + 2);
            if (sp == 1 || t < best * 0.999) {
                best = t;
                want = sp;
            }
        }
    } else if (groups > 0) {
        want = (int)((8 * cu + groups - 1) / groups);
        if (want > max_split) want = max_split;
        if (groups * want < 6LL * cu) {
            const int64_t one_round = (3LL * cu) / groups;
            want = one_round < max_split ? (int)one_round : max_split;
        }
    }
    static const int forced = [] {
        const char* e = getenv("BITCACHE_SPLITS");
        return e ? atoi(e) : 0;
    }();
    if (forced > 0) want = forced < tiles ? forced : tiles;   // tuning override
    if (want > kMaxSplits) want = kMaxSplits;
    if (want < 1) want = 1;
    const int tiles_per = (tiles + want - 1) / want;
    p.chunk = tiles_per * 64;
    p.n_splits = tiles == 0 ? 1 : (tiles + tiles_per - 1) / tiles_per;
    return p;
}

// The split policy of a full attention call (plan_splits' per_cu): MHA
// compensated attention several rounds; binary, GQA compensated and adaptive
// attention one round of what fits of their kernel, at most three workgroups
// per CU (the adaptive kernel's LDS allows two at d = 128), binary attention
// at most two (its tiles are short, so a workgroup's fixed prologue and
// epilogue weigh more than the latency hiding of a third: c2 54.5 -> 52.9 us).
//
// kMaxPerCu bounds every policy: ws_bytes sizes the workspace over the plans
// of per_cu = 0 .. kMaxPerCu, so a policy above it would launch more splits
// than the workspace holds.
constexpr int kMaxPerCu = 4;
int plan_per_cu(int mode, int D, int G) {
    if ((mode == MODE_COMP || mode == MODE_MIXED) && G == 1) return 0;
    // (MHA binary 2, GQA binary 4, the other modes 3: measured)
    int cap = mode == MODE_BINARY ? (G == 1 ? 2 : 4) : 3;
    if (cap > kMaxPerCu) cap = kMaxPerCu;
    const int n = bc::mfma_wgs_per_cu(mode, D, G);
    return n <= 0 ? cap : (n < cap ? n : cap);
}
// the policy of the split-phase entry points (bc_attention_partial and
// bc_attention_combine, which does not know the mode), and of the fp16
// reference kernel
constexpr int kPlanFixed = 0;

// Binary MHA attention (d = 64, 128, 256: the matrix-core head dims) with one
// head per CU: one workgroup of kWideWaves waves per head takes all its keys
// (wave w the tiles w, w + 8, ...), merges its waves and writes the output,
// so the call writes no partials and launches no merge.  Measured on the
// 256-head, 32K-key binary step: d = 128 52.8-56.0 -> 47.0-48.1 us (the 4-wave
// plan: two workgroups per CU and the merge launch; 16-wave workgroups
// 50.4-51.0 us), d = 256 101.2-103.2 -> 96.8-97.3 us, d = 64 42.6-46.4 ->
// 42.4-43.0 us.  With two or more heads
// per CU the split plans already launch no merge and the wide plan measured
// within noise of them (-4% to +2%), so it is left to one round.  Contexts up
// to kWideMaxKeys (each wave's sums cover at most 16K keys, as in the split
// plans).  The compensated kernel gains nothing this way (one round of
// 12-wave workgroups at 64K keys: kernel 425 against 406 us, step 430 against
// 428 us), so it keeps its split plans.  BITCACHE_WIDE=0 turns this off
// (tuning).
constexpr int kWideWaves = 8;
constexpr int kWideMaxKeys = 131072;
bool wide_plan(int mode, int D, int G, int64_t groups, int S, int cu) {
    static const bool off = [] {
        const char* e = getenv("BITCACHE_WIDE");
        return e != nullptr && atoi(e) == 0;
    }();
    return !off && mode == MODE_BINARY && G == 1 && (D == 64 || D == 128 || D == 256) && S > 0 &&
           S <= kWideMaxKeys && cu > 0 && groups == cu;
}

// BITCACHE_VALU_ATTENTION=1 selects the VALU split kernel for every head dim
bool valu_forced() {
    static const bool forced = [] {
        const char* e = getenv("BITCACHE_VALU_ATTENTION");
        return e != nullptr && e[0] == '1';
    }();
    return forced;
}

// bytes of the split partials a plan writes: one (max, sum, acc[D]) fp32
// record per (b, query head, split)
size_t plan_bytes(int batch, int hq, const SplitPlan& p, int D) {
    return (size_t)batch * hq * p.n_splits * (D + 2) * sizeof(float);
}

// Per-head modes: after a plan's partials (at the next 256-byte boundary)
// the workspace holds the two group lists of the mode launches: a 256-byte
// header with the binary and mixed counts, then the binary groups' indices,
// then the mixed groups' (int32, `groups` each).
size_t list_offset(size_t partial_bytes) { return (partial_bytes + 255) & ~(size_t)255; }
size_t list_bytes(int64_t groups) { return kListHeader + 2 * (size_t)groups * sizeof(int32_t); }

// workspace of the split partials: the largest plan of any policy
// plan_per_cu can return (per_cu = 0 .. kMaxPerCu), and the group lists
size_t ws_bytes(int batch, int hq, int hkv, int S, int D, int cu = 0) {
    size_t n = plan_bytes(batch, hq, plan_splits(batch, hq, hkv, S, 0, cu), D);
    for (int per_cu = 1; per_cu <= kMaxPerCu; per_cu++) {
        const size_t b = plan_bytes(batch, hq, plan_splits(batch, hq, hkv, S, per_cu, cu), D);
        n = b > n ? b : n;
    }
    const int G = pick_g(hq / hkv);
    return list_offset(n) + list_bytes((int64_t)batch * hkv * ((hq / hkv) / G));
}

int validate_heads(int batch, int n_heads, int n_kv_heads, int seq_len, int kv_stride, int d) {
    BC_REQUIRE(bc::head_dim_ok(d), BC_ERR_UNSUPPORTED,
               "head_dim must be a multiple of 32 in [32, 256], got %d", d);
    BC_REQUIRE(batch >= 0 && n_heads >= 0 && n_kv_heads > 0 && seq_len >= 0, BC_ERR_INVALID_ARGUMENT,
               "invalid dims batch=%d n_heads=%d n_kv_heads=%d seq_len=%d", batch, n_heads,
               n_kv_heads, seq_len);
    BC_REQUIRE(n_heads % n_kv_heads == 0, BC_ERR_INVALID_ARGUMENT,
               "n_heads (%d) must be a multiple of n_kv_heads (%d)", n_heads, n_kv_heads);
    BC_REQUIRE(kv_stride >= seq_len, BC_ERR_INVALID_ARGUMENT, "kv_stride (%d) < seq_len (%d)",
               kv_stride, seq_len);
    return BC_OK;
}

template <int D, int G>
void launch_split(int mode, const AttnArgs& a, dim3 grid, hipStream_t st) {
    if (mode == MODE_BINARY)
        hipLaunchKernelGGL((attn_split_kernel<D, G, MODE_BINARY>), grid, dim3(256), 0, st, a);
    else if (mode == MODE_COMP)
        hipLaunchKernelGGL((attn_split_kernel<D, G, MODE_COMP>), grid, dim3(256), 0, st, a);
    else if (mode == MODE_MIXED)
        hipLaunchKernelGGL((attn_split_kernel<D, G, MODE_MIXED>), grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((attn_split_kernel<D, G, MODE_ADAPTIVE>), grid, dim3(256), 0, st, a);
}

template <int D>
void launch_split_g(int mode, int G, const AttnArgs& a, dim3 grid, hipStream_t st) {
    switch (G) {
        case 8: launch_split<D, 8>(mode, a, grid, st); break;
        case 4: launch_split<D, 4>(mode, a, grid, st); break;
        case 2: launch_split<D, 2>(mode, a, grid, st); break;
        default: launch_split<D, 1>(mode, a, grid, st); break;
    }
}

template <int D>
void launch_combine(const float* ws, uint16_t* out, int bh, int n_splits, hipStream_t st) {
    hipLaunchKernelGGL((attn_combine_kernel<D>), dim3(bh), dim3(256), 0, st, ws, out, n_splits);
}

#define BC_DISPATCH_D(d, FN, ...)                                           \
    switch (d) {                                                            \
        case 32: FN<32>(__VA_ARGS__); break;                                \
        case 64: FN<64>(__VA_ARGS__); break;                                \
        case 96: FN<96>(__VA_ARGS__); break;                                \
        case 128: FN<128>(__VA_ARGS__); break;                              \
        case 160: FN<160>(__VA_ARGS__); break;                              \
        case 192: FN<192>(__VA_ARGS__); break;                              \
        case 224: FN<224>(__VA_ARGS__); break;                              \
        case 256: FN<256>(__VA_ARGS__); break;                              \
        default: return bc::set_error(BC_ERR_UNSUPPORTED, "head_dim %d", d); \
    }

}  // namespace

namespace bc {

// Phase 1 (split partials into the workspace) and phase 2 (combine).  Shared
// by the public entry points and the adaptive driver (adaptive.hip).
int run_partial(int mode, const void* q, const void* k_bin, const void* k_res, const void* v_bin,
                const void* v_res, int batch, int n_heads, int n_kv_heads, int seq_len,
                int kv_stride, int head_dim, void* workspace, size_t workspace_bytes,
                hipStream_t st, const uint32_t* thresh, const int32_t* cutoff,
                uint8_t* selected, const void* pcs, int per_cu, const AppendArgs* app = nullptr,
                const uint8_t* head_mode = nullptr, void* direct_out = nullptr,
                bool* wrote_out = nullptr) {
    if (wrote_out) *wrote_out = false;
    int v = validate_heads(batch, n_heads, n_kv_heads, seq_len, kv_stride, head_dim);
    if (v != BC_OK) return v;
    if ((int64_t)batch * n_heads == 0) return BC_OK;
    BC_REQUIRE(q && k_bin && v_bin, BC_ERR_INVALID_ARGUMENT, "null pointer");
    BC_REQUIRE(mode == MODE_BINARY || (k_res && v_res), BC_ERR_INVALID_ARGUMENT,
               "residual blobs required");
    const size_t need_ws = ws_bytes(batch, n_heads, n_kv_heads, seq_len, head_dim);
    BC_REQUIRE(workspace != nullptr && workspace_bytes >= need_ws, BC_ERR_WORKSPACE,
               "workspace of %zu bytes required, got %zu", need_ws, workspace_bytes);
    const SplitPlan p = plan_splits(batch, n_heads, n_kv_heads, seq_len, per_cu);
    const int64_t groups = (int64_t)batch * n_kv_heads * ((n_heads / n_kv_heads) / p.G);
    // (the bound the launch needs: the partials of the plan it runs, and for
    // per-head modes the group lists after them)
    const size_t plan_ws = plan_bytes(batch, n_heads, p, head_dim);
    const size_t plan_need =
        mode == MODE_MIXED ? list_offset(plan_ws) + list_bytes(groups) : plan_ws;
    BC_REQUIRE(workspace_bytes >= plan_need, BC_ERR_WORKSPACE,
               "the split plan writes %zu bytes of partials and lists, workspace holds %zu",
               plan_need, workspace_bytes);
    const int64_t cap = (int64_t)batch * n_kv_heads * kv_stride;
    AttnArgs a{};
    a.q = (const uint16_t*)q;
    a.kb = bin_planes(k_bin, cap, head_dim);
    a.vb = bin_planes(v_bin, cap, head_dim);
    if (k_res) a.kr = res_planes(k_res, cap, head_dim);
    if (v_res) a.vr = res_planes(v_res, cap, head_dim);
    a.B = batch;
    a.Hq = n_heads;
    a.Hkv = n_kv_heads;
    a.S = seq_len;
    a.kv_stride = kv_stride;
    a.n_splits = p.n_splits;
    a.chunk = p.chunk;
    a.ws = (float*)workspace;
    a.thresh = thresh;
    a.cutoff = cutoff;
    a.selected = selected;
    a.pcs = pcs;
    a.head_mode = head_mode;
    if (app != nullptr) {
        a.app_k = (const uint16_t*)app->k;
        a.app_v = (const uint16_t*)app->v;
        a.app_slot = app->slot;
    }
    const dim3 grid(p.n_splits, batch * n_kv_heads * ((n_heads / n_kv_heads) / p.G));
    // matrix-core value phase for head_dim 64/128/256; the VALU kernel covers the
    // other head dims (and is selectable with BITCACHE_VALU_ATTENTION=1).  With
    // one split per group the matrix-core kernel normalises and writes the
    // output itself (no merge launch).
    if (direct_out != nullptr && p.n_splits == 1) a.out = (uint16_t*)direct_out;
    // Per-head modes: the groups whose heads are all binary go to the binary
    // kernel, which reads none of their residual bytes, the others to the
    // mixed kernel.  A compaction launch lists each kind in order, and each
    // mode launch's grid row y takes the y-th group of its list, so a
    // launch's live workgroups come first in dispatch order and spread over
    // the CUs evenly (rows past its count return at once).
    int32_t* lists = nullptr;
    if (mode == MODE_MIXED) {
        lists = (int32_t*)((uint8_t*)workspace + list_offset(plan_ws));
        hipLaunchKernelGGL(mode_groups_kernel, dim3(1), dim3(kListThreads), 0, st, head_mode,
                           lists, (int)groups, (n_heads / n_kv_heads) / p.G, n_heads, n_kv_heads,
                           p.G);
        const int rc = bc::check_launch("per-head mode groups");
        if (rc != BC_OK) return rc;
        a.group_list = lists + kListHeader / sizeof(int32_t);
        a.group_count = lists;
    }
    const bool mfma = !valu_forced() && bc::mfma_split_ok(head_dim, a.chunk) &&
                      (head_dim == 64 || head_dim == 128 || head_dim == 256);
    // one wide workgroup per head (wide_plan): no partials, no merge launch
    if (mfma && direct_out != nullptr && app == nullptr &&
        wide_plan(mode, head_dim, p.G, groups, seq_len, bc::device_cu_count())) {
        AttnArgs w = a;
        w.n_splits = 1;
        w.chunk = (seq_len + 63) / 64 * 64;
        w.out = (uint16_t*)direct_out;
        if (bc::mfma_split_ok(head_dim, w.chunk) &&
            bc::launch_mfma_split(mode, head_dim, 1, w, dim3(1, (unsigned)groups), st, kWideWaves)) {
            if (wrote_out) *wrote_out = true;
            return bc::check_launch("attention (wide workgroups)");
        }
    }
    if (mode == MODE_MIXED) {
        if (mfma) {
            BC_REQUIRE(bc::launch_mfma_split(MODE_BINARY, head_dim, p.G, a, grid, st),
                       BC_ERR_UNSUPPORTED, "head_dim %d", head_dim);
        } else {
            a.out = nullptr;
            BC_DISPATCH_D(head_dim, launch_split_g, MODE_BINARY, p.G, a, grid, st);
        }
        const int rc = bc::check_launch("attention split (binary heads)");
        if (rc != BC_OK) return rc;
        a.group_list = lists + kListHeader / sizeof(int32_t) + groups;
        a.group_count = lists + 1;
    }
    if (mfma && bc::launch_mfma_split(mode, head_dim, p.G, a, grid, st)) {
        if (wrote_out) *wrote_out = a.out != nullptr;
        return bc::check_launch("attention split (mfma)");
    }
    a.out = nullptr;
    // (the VALU kernel does not append; the append entry point checks first)
    BC_REQUIRE(app == nullptr, BC_ERR_UNSUPPORTED, "in-place append needs the MFMA kernel");
    BC_DISPATCH_D(head_dim, launch_split_g, mode, p.G, a, grid, st);
    return bc::check_launch("attention split");
}

int run_combine(int per_cu, const void* workspace, void* out, int batch, int n_heads, int n_kv_heads,
                int seq_len, int head_dim, hipStream_t st) {
    int v = validate_heads(batch, n_heads, n_kv_heads, seq_len, seq_len, head_dim);
    if (v != BC_OK) return v;
    if ((int64_t)batch * n_heads == 0) return BC_OK;
    BC_REQUIRE(workspace && out, BC_ERR_INVALID_ARGUMENT, "null pointer");
    const SplitPlan p = plan_splits(batch, n_heads, n_kv_heads, seq_len, per_cu);
    BC_DISPATCH_D(head_dim, launch_combine, (const float*)workspace, (uint16_t*)out,
                  batch * n_heads, p.n_splits, st);
    return bc::check_launch("attention combine");
}

int run_attention(int mode, const void* q, const void* k_bin, const void* k_res, const void* v_bin,
                  const void* v_res, void* out, int batch, int n_heads, int n_kv_heads,
                  int seq_len, int kv_stride, int head_dim, void* workspace,
                  size_t workspace_bytes, hipStream_t st, const uint32_t* thresh,
                  const int32_t* cutoff, uint8_t* selected, const void* pcs, const AppendArgs* app,
                  const uint8_t* head_mode) {
    const int per_cu = head_dim > 0 && n_kv_heads > 0
                           ? plan_per_cu(mode, head_dim, pick_g(n_heads / n_kv_heads)) : kPlanFixed;
    BC_REQUIRE(out != nullptr || (int64_t)batch * n_heads == 0, BC_ERR_INVALID_ARGUMENT,
               "null output");
    bool wrote = false;
    int rc = run_partial(mode, q, k_bin, k_res, v_bin, v_res, batch, n_heads, n_kv_heads, seq_len,
                         kv_stride, head_dim, workspace, workspace_bytes, st, thresh, cutoff,
                         selected, pcs, per_cu, app, head_mode, out, &wrote);
    if (rc != BC_OK || wrote) return rc;
    return run_combine(per_cu, workspace, out, batch, n_heads, n_kv_heads, seq_len, head_dim, st);
}

size_t attention_ws_bytes(int batch, int n_heads, int n_kv_heads, int seq_len, int d) {
    return ws_bytes(batch, n_heads, n_kv_heads, seq_len, d);
}

}  // namespace bc

extern "C" int bc_attention_workspace_size(int batch, int n_heads, int n_kv_heads, int seq_len,
                                           int head_dim, size_t* bytes) {
    int v = validate_heads(batch, n_heads, n_kv_heads, seq_len, seq_len, head_dim);
    if (v != BC_OK) return v;
    BC_REQUIRE(bytes != nullptr, BC_ERR_INVALID_ARGUMENT, "null bytes");
    *bytes = ws_bytes(batch, n_heads, n_kv_heads, seq_len, head_dim);
    return BC_OK;
}

extern "C" int bc_attention_split_plan(int mode, int batch, int n_heads, int n_kv_heads,
                                       int seq_len, int head_dim, int cu_count, int* n_splits,
                                       size_t* partial_bytes, size_t* workspace_bytes) {
    int v = validate_heads(batch, n_heads, n_kv_heads, seq_len, seq_len, head_dim);
    if (v != BC_OK) return v;
    BC_REQUIRE(mode >= MODE_BINARY && mode <= MODE_MIXED, BC_ERR_INVALID_ARGUMENT,
               "unknown attention mode %d", mode);
    BC_REQUIRE(cu_count >= 0, BC_ERR_INVALID_ARGUMENT, "cu_count %d < 0", cu_count);
    BC_REQUIRE(n_splits && partial_bytes && workspace_bytes, BC_ERR_INVALID_ARGUMENT,
               "null output");
    const int per_cu = plan_per_cu(mode, head_dim, pick_g(n_heads / n_kv_heads));
    SplitPlan p = plan_splits(batch, n_heads, n_kv_heads, seq_len, per_cu, cu_count);
    const int64_t groups = (int64_t)batch * n_kv_heads * ((n_heads / n_kv_heads) / p.G);
    if (wide_plan(mode, head_dim, p.G, groups, seq_len, cu_count > 0 ? cu_count : bc::device_cu_count())) {
        // (one wide workgroup per head; no partials are written)
        p.n_splits = 1;
        p.chunk = (seq_len + 63) / 64 * 64;
    }
    *n_splits = p.n_splits;
    *partial_bytes = plan_bytes(batch, n_heads, p, head_dim);
    *workspace_bytes = ws_bytes(batch, n_heads, n_kv_heads, seq_len, head_dim, cu_count);
    return BC_OK;
}

extern "C" int bc_attention_partial(const void* q, const void* k_bin, const void* k_res,
                                    const void* v_bin, const void* v_res, int batch, int n_heads,
                                    int n_kv_heads, int seq_len, int kv_stride, int head_dim,
                                    void* workspace, size_t workspace_bytes, void* stream) {
    BC_REQUIRE((k_res == nullptr) == (v_res == nullptr), BC_ERR_INVALID_ARGUMENT,
               "k_res and v_res must both be given or both be null");
    return bc::run_partial(k_res ? MODE_COMP : MODE_BINARY, q, k_bin, k_res, v_bin, v_res, batch,
                           n_heads, n_kv_heads, seq_len, kv_stride, head_dim, workspace,
                           workspace_bytes, (hipStream_t)stream, nullptr, nullptr, nullptr, nullptr,
                           kPlanFixed);
}

extern "C" int bc_attention_combine(const void* workspace, void* out, int batch, int n_heads,
                                    int n_kv_heads, int seq_len, int head_dim, void* stream) {
    // (the partials of bc_attention_partial, planned with the same fixed policy)
    return bc::run_combine(kPlanFixed, workspace, out, batch, n_heads, n_kv_heads, seq_len, head_dim,
                           (hipStream_t)stream);
}

extern "C" int bc_binary_attention(const void* q, const void* k_bin, const void* v_bin, void* out,
                                   int batch, int n_heads, int seq_len, int head_dim,
                                   void* workspace, size_t workspace_bytes, void* stream) {
    return bc::run_attention(MODE_BINARY, q, k_bin, nullptr, v_bin, nullptr, out, batch, n_heads,
                             n_heads, seq_len, seq_len, head_dim, workspace, workspace_bytes,
                             (hipStream_t)stream, nullptr, nullptr, nullptr, nullptr);
}

extern "C" int bc_compensated_attention(const void* q, const void* k_bin, const void* k_res,
                                        const void* v_bin, const void* v_res, void* out, int batch,
                                        int n_heads, int seq_len, int head_dim, void* workspace,
                                        size_t workspace_bytes, void* stream) {
    return bc::run_attention(MODE_COMP, q, k_bin, k_res, v_bin, v_res, out, batch, n_heads,
                             n_heads, seq_len, seq_len, head_dim, workspace, workspace_bytes,
                             (hipStream_t)stream, nullptr, nullptr, nullptr, nullptr);
}

extern "C" int bc_attention_gqa(const void* q, const void* k_bin, const void* k_res,
                                const void* v_bin, const void* v_res, void* out, int batch,
                                int n_heads, int n_kv_heads, int seq_len, int kv_stride,
                                int head_dim, void* workspace, size_t workspace_bytes,
                                void* stream) {
    BC_REQUIRE((k_res == nullptr) == (v_res == nullptr), BC_ERR_INVALID_ARGUMENT,
               "k_res and v_res must both be given or both be null");
    return bc::run_attention(k_res ? MODE_COMP : MODE_BINARY, q, k_bin, k_res, v_bin, v_res, out,
                             batch, n_heads, n_kv_heads, seq_len, kv_stride, head_dim, workspace,
                             workspace_bytes, (hipStream_t)stream, nullptr, nullptr, nullptr, nullptr);
}

// ---------------------------------------------------------------- allocation-free attention
// bc_attention_gqa_noalloc keeps its split partials in `scratch`, a file-scope
// device array (one copy per GPU, held until the process ends) of
// kNoAllocScratchBytes.  Host code never passes the array's name to a kernel
// (on the host it is a stand-in, not a device address): each device's
// address comes from hipGetSymbolAddress on that device's first call and is
// kept per device.  Calls that overlap on one GPU share the array and race.
// Every split partial is written by its workgroup before the combine reads
// it, so nothing needs clearing between calls.
constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

static std::mutex g_scratch_mutex;
static std::vector<void*> g_scratch_ptrs;   // per device ordinal

static int scratch_address(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return bc::set_error(BC_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if ((int)g_scratch_ptrs.size() <= dev) g_scratch_ptrs.resize(dev + 1, nullptr);
    if (g_scratch_ptrs[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr)
            return bc::set_error(BC_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        g_scratch_ptrs[dev] = p;
    }
    *out = g_scratch_ptrs[dev];
    return BC_OK;
}

extern "C" int bc_attention_gqa_noalloc(const void* q, const void* k_bin, const void* k_res,
                                        const void* v_bin, const void* v_res, void* out, int batch,
                                        int n_heads, int n_kv_heads, int seq_len, int kv_stride,
                                        int head_dim, void* stream) {
    int v = validate_heads(batch, n_heads, n_kv_heads, seq_len, kv_stride, head_dim);
    if (v != BC_OK) return v;
    const size_t need = ws_bytes(batch, n_heads, n_kv_heads, seq_len, head_dim);
    BC_REQUIRE(need <= kNoAllocScratchBytes, BC_ERR_WORKSPACE,
               "this shape needs %zu bytes of split partials; the allocation-free entry point "
               "holds at most %zu (use bc_attention_gqa with a caller workspace)",
               need, kNoAllocScratchBytes);
    void* ws = nullptr;
    const int rc = scratch_address(&ws);
    if (rc != BC_OK) return rc;
    return bc_attention_gqa(q, k_bin, k_res, v_bin, v_res, out, batch, n_heads, n_kv_heads, seq_len,
                            kv_stride, head_dim, ws, kNoAllocScratchBytes, stream);
}

// One decode step on a ring cache: the new token's K and V vectors go to
// position current_len % max_seq of every (b, kv head) row (the slot rule of
// src/online_encode.cu:139, bitcache/__init__.py:112-113), then the query
// attends over the min(current_len + 1, max_seq) filled positions.  The same
// bytes and outputs as bc_online_encode_kv followed by bc_attention_gqa; in one
// launch when the MFMA kernel runs with one query-head group per kv head (the
// workgroup whose keys hold the slot encodes the token before reading them),
// otherwise as those two calls.
extern "C" int bc_append_attention(const void* q, const void* k_new, const void* v_new, void* k_bin,
                                   void* k_res, void* v_bin, void* v_res, void* out, int batch,
                                   int n_heads, int n_kv_heads, int head_dim, int64_t current_len,
                                   int max_seq, void* workspace, size_t workspace_bytes,
                                   void* stream) {
    BC_REQUIRE((k_res == nullptr) == (v_res == nullptr), BC_ERR_INVALID_ARGUMENT,
               "k_res and v_res must both be given or both be null");
    BC_REQUIRE(max_seq > 0 && current_len >= 0, BC_ERR_INVALID_ARGUMENT,
               "invalid ring: max_seq=%d current_len=%lld", max_seq, (long long)current_len);
    int v = validate_heads(batch, n_heads, n_kv_heads, max_seq, max_seq, head_dim);
    if (v != BC_OK) return v;
    if ((int64_t)batch * n_heads == 0) return BC_OK;
    BC_REQUIRE(q && k_new && v_new && k_bin && v_bin && out, BC_ERR_INVALID_ARGUMENT, "null pointer");
    const int seq_len = current_len + 1 < max_seq ? (int)(current_len + 1) : max_seq;
    // (checked before the token is written, so a failed step leaves the cache as it was)
    const size_t need_ws = ws_bytes(batch, n_heads, n_kv_heads, seq_len, head_dim);
    BC_REQUIRE(workspace != nullptr && workspace_bytes >= need_ws, BC_ERR_WORKSPACE,
               "workspace of %zu bytes required, got %zu", need_ws, workspace_bytes);
    const int mode = k_res ? MODE_COMP : MODE_BINARY;
    const int group = n_heads / n_kv_heads;
    const SplitPlan p = plan_splits(batch, n_heads, n_kv_heads, seq_len,
                                    plan_per_cu(mode, head_dim, pick_g(group)));
    hipStream_t st = (hipStream_t)stream;
    if (valu_forced() || pick_g(group) != group || !bc::mfma_split_ok(head_dim, p.chunk)) {
        const int rc = bc_online_encode_kv(k_new, v_new, k_bin, k_res, v_bin, v_res, batch,
                                           n_kv_heads, head_dim, current_len, max_seq, stream);
        if (rc != BC_OK) return rc;
        return bc::run_attention(mode, q, k_bin, k_res, v_bin, v_res, out, batch, n_heads, n_kv_heads,
                                 seq_len, max_seq, head_dim, workspace, workspace_bytes, st, nullptr,
                                 nullptr, nullptr, nullptr);
    }
    const bc::AppendArgs app{k_new, v_new, (int)(current_len % max_seq)};
    return bc::run_attention(mode, q, k_bin, k_res, v_bin, v_res, out, batch, n_heads, n_kv_heads,
                             seq_len, max_seq, head_dim, workspace, workspace_bytes, st, nullptr,
                             nullptr, nullptr, nullptr, &app);
}

// Per-head mode dispatch (the reference's adaptive-precision intent,
// src/adaptive_precision.cuh:6-49, examples/generation_demo.py:129-141): head
// (b, h) is attended in binary mode where modes[b*n_heads + h] == 0 (as
// bc_adaptive_select writes for a high-entropy head) and in compensated mode
// otherwise, in one launch over the compensated cache.
extern "C" int bc_head_mode_attention(const void* q, const void* k_bin, const void* k_res,
                                      const void* v_bin, const void* v_res, const uint8_t* modes,
                                      void* out, int batch, int n_heads, int n_kv_heads, int seq_len,
                                      int kv_stride, int head_dim, void* workspace,
                                      size_t workspace_bytes, void* stream) {
    BC_REQUIRE(k_res && v_res, BC_ERR_INVALID_ARGUMENT, "residual blobs required");
    BC_REQUIRE(modes != nullptr || (int64_t)batch * n_heads == 0, BC_ERR_INVALID_ARGUMENT,
               "null modes");
    return bc::run_attention(MODE_MIXED, q, k_bin, k_res, v_bin, v_res, out, batch, n_heads,
                             n_kv_heads, seq_len, kv_stride, head_dim, workspace, workspace_bytes,
                             (hipStream_t)stream, nullptr, nullptr, nullptr, nullptr, nullptr, modes);
}

template <int D>
static void launch_scores(const void* q, BinPlanes kb, float* scores, int32_t* pcs, int batch,
                          int hq, int hkv, int S, int stride, hipStream_t st) {
    // about 8 workgroups per CU, each a chunk of at least 1024 keys
    const int n_hb = (hq / hkv + kScoreHeads - 1) / kScoreHeads;
    const int64_t rows = (int64_t)batch * hkv * n_hb;
    const int64_t want = (8LL * bc::device_cu_count() + rows - 1) / rows;
    const int64_t most = ((int64_t)S + 1023) / 1024;
    const int n_chunks = (int)(want < most ? (want < 1 ? 1 : want) : most);
    const int chunk = (S + n_chunks - 1) / n_chunks;
    hipLaunchKernelGGL((scores_kernel<D>), dim3(n_chunks, (unsigned)rows), dim3(256), 0, st,
                       (const uint16_t*)q, kb, scores, pcs, hq, hkv, S, stride, chunk, n_hb);
}

extern "C" int bc_binary_scores(const void* q, const void* k_bin, float* scores,
                                int32_t* popcounts, int batch, int n_heads, int n_kv_heads,
                                int seq_len, int kv_stride, int head_dim, void* stream) {
    int v = validate_heads(batch, n_heads, n_kv_heads, seq_len, kv_stride, head_dim);
    if (v != BC_OK) return v;
    if ((int64_t)batch * n_heads * seq_len == 0) return BC_OK;
    BC_REQUIRE(q && k_bin, BC_ERR_INVALID_ARGUMENT, "null pointer");
    const int64_t cap = (int64_t)batch * n_kv_heads * kv_stride;
    BinPlanes kb = bin_planes(k_bin, cap, head_dim);
    BC_DISPATCH_D(head_dim, launch_scores, q, kb, scores, popcounts, batch, n_heads, n_kv_heads,
                  seq_len, kv_stride, (hipStream_t)stream);
    return bc::check_launch("binary scores");
}

// key chunks per (b, query head) of the entropy pass: about eight 256-thread
// blocks per CU over all heads, at least 4096 keys per chunk; one chunk means
// the single-block kernel (no workspace)
static int entropy_chunks(int batch, int hq, int S) {
    const int64_t heads = (int64_t)batch * hq;
    if (heads <= 0 || S <= 0) return 1;
    int64_t n = (8LL * bc::device_cu_count() + heads - 1) / heads;
    const int64_t most = ((int64_t)S + 4095) / 4096;
    if (n > most) n = most;
    return n < 1 ? 1 : (int)n;
}

static size_t entropy_ws_bytes(int batch, int hq, int S) {
    const int n = entropy_chunks(batch, hq, S);
    return n <= 1 ? 0 : (size_t)batch * hq * n * 3 * sizeof(float);
}

template <int D>
static void launch_entropy(const void* q, BinPlanes kb, float* out, float* ws, int batch, int hq,
                           int hkv, int S, int stride, hipStream_t st) {
    const int n = ws != nullptr ? entropy_chunks(batch, hq, S) : 1;
    if (n <= 1) {
        hipLaunchKernelGGL((entropy_kernel<D, kEntropyThreads>), dim3(batch * hq, 1),
                           dim3(kEntropyThreads), 0, st, (const uint16_t*)q, kb, out,
                           (float*)nullptr, hq, hkv, S, stride, S);
        return;
    }
    const int chunk = (S + n - 1) / n;
    hipLaunchKernelGGL((entropy_kernel<D, kEntPartThreads>), dim3(batch * hq, n),
                       dim3(kEntPartThreads), 0, st, (const uint16_t*)q, kb, out, ws, hq, hkv, S,
                       stride, chunk);
    const int heads = batch * hq;
    hipLaunchKernelGGL(entropy_merge_kernel, dim3((heads + 255) / 256), dim3(256), 0, st,
                       (const float*)ws, out, heads, n);
}

extern "C" int bc_entropy_workspace_size(int batch, int n_heads, int seq_len, size_t* bytes) {
    BC_REQUIRE(batch >= 0 && n_heads >= 0 && seq_len >= 0, BC_ERR_INVALID_ARGUMENT,
               "invalid dims batch=%d n_heads=%d seq_len=%d", batch, n_heads, seq_len);
    BC_REQUIRE(bytes != nullptr, BC_ERR_INVALID_ARGUMENT, "null bytes");
    *bytes = entropy_ws_bytes(batch, n_heads, seq_len);
    return BC_OK;
}

extern "C" int bc_compute_head_entropy_ws(const void* q, const void* k_bin, float* entropy,
                                          int batch, int n_heads, int n_kv_heads, int seq_len,
                                          int kv_stride, int head_dim, void* workspace,
                                          size_t workspace_bytes, void* stream) {
    int v = validate_heads(batch, n_heads, n_kv_heads, seq_len, kv_stride, head_dim);
    if (v != BC_OK) return v;
    if ((int64_t)batch * n_heads == 0) return BC_OK;
    BC_REQUIRE(q && k_bin && entropy, BC_ERR_INVALID_ARGUMENT, "null pointer");
    const size_t need = entropy_ws_bytes(batch, n_heads, seq_len);
    BC_REQUIRE(workspace == nullptr || workspace_bytes >= need, BC_ERR_WORKSPACE,
               "workspace of %zu bytes required, got %zu", need, workspace_bytes);
    const int64_t cap = (int64_t)batch * n_kv_heads * kv_stride;
    BinPlanes kb = bin_planes(k_bin, cap, head_dim);
    float* ws = need > 0 ? (float*)workspace : nullptr;
    BC_DISPATCH_D(head_dim, launch_entropy, q, kb, entropy, ws, batch, n_heads, n_kv_heads,
                  seq_len, kv_stride, (hipStream_t)stream);
    return bc::check_launch("entropy");
}

extern "C" int bc_compute_head_entropy_gqa(const void* q, const void* k_bin, float* entropy,
                                           int batch, int n_heads, int n_kv_heads, int seq_len,
                                           int kv_stride, int head_dim, void* stream) {
    return bc_compute_head_entropy_ws(q, k_bin, entropy, batch, n_heads, n_kv_heads, seq_len,
                                      kv_stride, head_dim, nullptr, 0, stream);
}

extern "C" int bc_compute_head_entropy(const void* q, const void* k_bin, float* entropy,
                                       int batch, int n_heads, int seq_len, int head_dim,
                                       void* stream) {
    return bc_compute_head_entropy_gqa(q, k_bin, entropy, batch, n_heads, n_heads > 0 ? n_heads : 1,
                                       seq_len, seq_len, head_dim, stream);
}

extern "C" int bc_adaptive_select(const float* entropy, uint8_t* modes, int batch, int n_heads,
                                  float threshold, void* stream) {
    BC_REQUIRE(batch >= 0 && n_heads >= 0, BC_ERR_INVALID_ARGUMENT, "negative dims");
    const int n = batch * n_heads;
    if (n == 0) return BC_OK;
    BC_REQUIRE(entropy && modes, BC_ERR_INVALID_ARGUMENT, "null pointer");
    hipLaunchKernelGGL(select_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       entropy, modes, n, threshold);
    return bc::check_launch("adaptive select");
}

template <int D>
static void launch_ref(int G, const void* q, const void* k, const void* v, int hq, int hkv, int S,
                       int ns, int chunk, float* ws, dim3 grid, hipStream_t st) {
    const uint16_t *qq = (const uint16_t*)q, *kk = (const uint16_t*)k, *vv = (const uint16_t*)v;
    switch (G) {
        case 8: hipLaunchKernelGGL((ref_split_kernel<D, 8>), grid, dim3(256), 0, st, qq, kk, vv, hq, hkv, S, ns, chunk, ws); break;
        case 4: hipLaunchKernelGGL((ref_split_kernel<D, 4>), grid, dim3(256), 0, st, qq, kk, vv, hq, hkv, S, ns, chunk, ws); break;
        case 2: hipLaunchKernelGGL((ref_split_kernel<D, 2>), grid, dim3(256), 0, st, qq, kk, vv, hq, hkv, S, ns, chunk, ws); break;
        default: hipLaunchKernelGGL((ref_split_kernel<D, 1>), grid, dim3(256), 0, st, qq, kk, vv, hq, hkv, S, ns, chunk, ws); break;
    }
}

extern "C" int bc_reference_attention(const void* q, const void* k, const void* v, void* out,
                                      int batch, int n_heads, int n_kv_heads, int seq_len,
                                      int head_dim, void* workspace, size_t workspace_bytes,
                                      void* stream) {
    int vv = validate_heads(batch, n_heads, n_kv_heads, seq_len, seq_len, head_dim);
    if (vv != BC_OK) return vv;
    if ((int64_t)batch * n_heads == 0) return BC_OK;
    BC_REQUIRE(q && k && v && out, BC_ERR_INVALID_ARGUMENT, "null pointer");
    const size_t need_ws = ws_bytes(batch, n_heads, n_kv_heads, seq_len, head_dim);
    BC_REQUIRE(workspace != nullptr && workspace_bytes >= need_ws, BC_ERR_WORKSPACE,
               "workspace of %zu bytes required, got %zu", need_ws, workspace_bytes);
    const SplitPlan p = plan_splits(batch, n_heads, n_kv_heads, seq_len, kPlanFixed);
    const dim3 grid(p.n_splits, batch * n_kv_heads * ((n_heads / n_kv_heads) / p.G));
    hipStream_t st = (hipStream_t)stream;
    BC_DISPATCH_D(head_dim, launch_ref, p.G, q, k, v, n_heads, n_kv_heads, seq_len, p.n_splits,
                  p.chunk, (float*)workspace, grid, st);
    int rc = bc::check_launch("reference attention");
    if (rc != BC_OK) return rc;
    BC_DISPATCH_D(head_dim, launch_combine, (const float*)workspace, (uint16_t*)out,
                  batch * n_heads, p.n_splits, st);
    return bc::check_launch("reference combine");
}
