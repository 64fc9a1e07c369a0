// Split-KV decode attention with the value phase on the matrix cores (gfx950).
//
// Same work decomposition and partial format as attn_split_kernel
// (attention.hip): grid.x = key split, grid.y = (b, kv head, query-head
// group), 4 wave64 per workgroup, 64-key tiles round-robin over the waves.
//
// Score phase (lane = key): XNOR popcount of the sign words, and the INT4
// residual dot with v_dot8_i32_i4 directly on the stored two's-complement
// nibbles against the query quantised to 16-bit fixed point and split into
// four balanced int4 digits (q_int = d0 + 16 d1 + 256 d2 + 4096 d3).
//
// Value phase: out[e] = sum_s a_s*(2*bit_se - 1) + b_s*(u_se - 8) with
// a = p*sv, b = p*rs/7, u = n + 8.  The V tile (sign bytes and code bytes of
// 64 keys) is copied global->LDS with direct loads, then ds_read_b64_tr_b4
// transposes 16 keys x 16 nibbles per 16-lane group so that each lane holds
// 16 keys of one dimension.  Nibbles (u) and sign bits become exact fp16
// subnormals (value * 2^-24) with one shift + one mask per pair, and
// v_mfma_f32_16x16x32_f16 accumulates dims x weight-columns, where the weight
// columns are (hi, lo) fp16 splits of a and b for each query head of the
// group.  The fp32 accumulators are rescaled on running-max changes.
#include <math.h>

#include "attn.h"

using bc::AttnArgs;
using bc::kLog2e;
using bc::MODE_ADAPTIVE;
using bc::MODE_BINARY;
using bc::MODE_COMP;

namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef int v2i_t __attribute__((ext_vector_type(2)));
#define LDS_PTR(T, p) ((__attribute__((address_space(3))) T*)(p))

template <int D, int G>
struct QDigits {
    uint32_t signs[G][D / 32];
    int4 digits[G][D / 8];        // .x..w = balanced int4 digits 0..3 of elements 8w..8w+7 (nibble k = element 8w+k)
    float scale_q[G];             // sequential mean |q| (src/compensated_attention.cu:65-67)
    float dq[G];                  // fixed-point step of q_int
};

// Per-wave LDS: V staging (codes then signs) and the (hi, lo) fp16 weight
// columns; the epilogue reuses it for [2 parts][G][D] partial sums + G offsets.
template <int D, int G>
struct WaveLds {
    static constexpr int kCodeBytes = 64 * D / 2;
    static constexpr int kSignBytes = 64 * D / 8;
    static constexpr int kWeightBytes = 2 * 16 * 64 * 2;  // [part][col][slot] fp16
    static constexpr int kMain = kCodeBytes + kSignBytes + kWeightBytes;
    static constexpr int kEpi = ((2 * G * D + G) * 4 + 15) / 16 * 16;
    static constexpr int kBytes = kMain > kEpi ? kMain : kEpi;
};

__device__ __forceinline__ uint16_t f2h_bits(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float h_bits2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// slot position of key k (0..63) inside the weight columns: for MFMA half mh of
// group g4, slots (2t, 2t+1) hold keys (t, t+4) of the 8-key run.
__device__ __forceinline__ int slot_of(int k) {
    const int g4 = k >> 4, mh = (k >> 3) & 1, r = k & 7;
    return 16 * g4 + 8 * mh + ((r & 3) << 1) + (r >> 2);
}

template <int D, int G>
__device__ void prep_digits(const uint16_t* qbase, QDigits<D, G>& qd, float* qf) {
    const int tid = threadIdx.x;
    for (int i = tid; i < G * D; i += blockDim.x) qf[i] = h2f(qbase[i]);
    __syncthreads();
    if (tid < G) {
        float acc = 0.0f, mx = 0.0f;
        for (int i = 0; i < D; i++) {
            acc += fabsf(qf[tid * D + i]);
            mx = fmaxf(mx, fabsf(qf[tid * D + i]));
        }
        qd.scale_q[tid] = acc / (float)D;
        // |q_int| <= 30583 keeps the top digit in [-8, 7]
        qd.dq[tid] = mx > 0.0f ? mx / 30583.0f : 1.0f;
    }
    for (int i = tid; i < G * (D / 32); i += blockDim.x) {
        const int g = i / (D / 32), w = i % (D / 32);
        uint32_t bits = 0;
        for (int b = 0; b < 32; b++) bits |= (qf[g * D + 32 * w + b] >= 0.0f ? 1u : 0u) << b;
        qd.signs[g][w] = bits;
    }
    __syncthreads();
    for (int i = tid; i < G * (D / 8); i += blockDim.x) {
        const int g = i / (D / 8), w = i % (D / 8);
        uint32_t dg[4] = {0u, 0u, 0u, 0u};
        for (int k = 0; k < 8; k++) {
            int t = (int)__builtin_rintf(qf[g * D + 8 * w + k] / qd.dq[g]);
            for (int j = 0; j < 4; j++) {
                const int d = ((t + 8) & 15) - 8;
                dg[j] |= ((uint32_t)d & 0xFu) << (4 * k);
                t = (t - d) >> 4;
            }
        }
        qd.digits[g][w] = make_int4((int)dg[0], (int)dg[1], (int)dg[2], (int)dg[3]);
    }
    __syncthreads();
}

// Resident waves per SIMD the register allocation targets: two for small
// query groups (memory latency is hidden by the second wave), one otherwise.
template <int D, int G>
struct Occupancy {
    static constexpr int kWaves = (G <= 2 && D <= 128) ? 2 : 1;
};

template <int D, int G, int MODE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(Occupancy<D, G>::kWaves)))
void attn_mfma_kernel(AttnArgs a) {
    constexpr int NB = D / 16;   // nibble dim-blocks (16 dims each)
    constexpr int NH = D / 64;   // sign blocks (64 dims each)
    constexpr int CW = D / 8;    // code dwords per key
    constexpr bool RES = MODE != MODE_BINARY;
    constexpr int SB = D / 8;    // sign bytes per key
    using WL = WaveLds<D, G>;

    __shared__ QDigits<D, G> qd;
    __shared__ float qf[G * D];
    __shared__ __attribute__((aligned(16))) uint8_t wave_lds[4][WL::kBytes];
    __shared__ float wm[4][G], wlsum[4][G], wsc[4];

    const int split = blockIdx.x;
    const int nqg = (a.Hq / a.Hkv) / G;
    const int qg = blockIdx.y % nqg;
    const int bkv = blockIdx.y / nqg;
    const int b = bkv / a.Hkv, kvh = bkv % a.Hkv;
    const int hq0 = kvh * (a.Hq / a.Hkv) + qg * G;
    const int bhq0 = b * a.Hq + hq0;

    prep_digits<D, G>(a.q + (int64_t)bhq0 * D, qd, qf);

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int g4 = lane >> 4, lj = lane & 15;
    const int key_begin = split * a.chunk;
    const int key_end = min(a.S, key_begin + a.chunk);
    const int64_t kv_base = (int64_t)bkv * a.kv_stride;
    const float isd2 = (1.0f / sqrtf((float)D)) * kLog2e;

    uint8_t* my = wave_lds[wave];
    uint8_t* st_codes = my;                              // [D/32 chunks][64 keys][16 B]
    uint8_t* st_signs = my + WL::kCodeBytes;             // SB >= 16: [SB/16][64][16 B]; SB == 8: [64][8 B]
    uint16_t* wts = (uint16_t*)(my + WL::kCodeBytes + WL::kSignBytes);  // [2][16][64]

    // weight column owned by this lane in the MFMA B operand, and its head
    const int my_col = lj;
    const int my_head = my_col >> 1;

    float m[G], lsum[G], off[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -INFINITY;
        lsum[g] = 0.0f;
        off[g] = 0.0f;
    }
    f4_t cs[NH][4];   // sign part: [block][p] rows = dims 64h + 4m + p
    f4_t cn[NB];      // residual part: rows = dims 16db + m
#pragma unroll
    for (int h = 0; h < NH; h++)
#pragma unroll
        for (int p = 0; p < 4; p++) cs[h][p] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < NB; d++) cn[d] = f4_t{0.f, 0.f, 0.f, 0.f};

    // weights enter the MFMAs as w * 2^wexp (fp16 hi + lo), wexp chosen so the
    // largest weight sits near 2^14: no overflow, and weights down to ~2^-38 of
    // the largest keep their contribution (undone exactly in the epilogue)
    int wexp = 0;
    bool have_wexp = false;

    uint32_t thresh[G];
    int need[G];
    if constexpr (MODE == MODE_ADAPTIVE) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            thresh[g] = a.thresh[bhq0 + g];
            need[g] = a.need[bhq0 + g];
        }
    }

    // query digits: one head -> scalar registers for the whole loop (uniform
    // operands of v_dot8); several heads -> re-read from LDS every tile
    int sdig[G == 1 ? CW : 1][4];
    if constexpr (G == 1) {
#pragma unroll
        for (int w = 0; w < CW; w++) {
            const int4 dg = qd.digits[0][w];
            sdig[w][0] = __builtin_amdgcn_readfirstlane(dg.x);
            sdig[w][1] = __builtin_amdgcn_readfirstlane(dg.y);
            sdig[w][2] = __builtin_amdgcn_readfirstlane(dg.z);
            sdig[w][3] = __builtin_amdgcn_readfirstlane(dg.w);
        }
    }

    for (int t0 = key_begin + wave * 64; t0 < key_end; t0 += 4 * 64) {
        const int s = t0 + lane;
        const bool valid = s < key_end;
        const int64_t ki = kv_base + (valid ? s : t0);

        // ---------------- V tile: global -> LDS
        if constexpr (SB >= 16) {
            if (valid) {  // lane = key: 16-byte chunks land at chunk*1024 + 16*lane
                const uint8_t* vs = a.vb.signs + ki * SB;
#pragma unroll
                for (int c = 0; c < SB / 16; c++)
                    __builtin_amdgcn_global_load_lds(
                        (const __attribute__((address_space(1))) void*)(vs + 16 * c),
                        LDS_PTR(void, st_signs + c * 1024), 16, 0, 0);
            }
        } else {
            // 8-byte sign rows: lane l < 32 copies keys 2l and 2l+1 (16 bytes; a
            // second key past the range reads the blob's own next bytes and gets
            // weight 0)
            if (lane < 32 && t0 + 2 * lane < key_end)
                __builtin_amdgcn_global_load_lds(
                    (const __attribute__((address_space(1))) void*)(a.vb.signs +
                                                                    (kv_base + t0 + 2 * lane) * SB),
                    LDS_PTR(void, st_signs), 16, 0, 0);
        }
        if constexpr (MODE == MODE_COMP) {
            if (valid) {
                const uint8_t* vc = a.vr.codes + ki * (D / 2);
#pragma unroll
                for (int c = 0; c < D / 32; c++)
                    __builtin_amdgcn_global_load_lds(
                        (const __attribute__((address_space(1))) void*)(vc + 16 * c),
                        LDS_PTR(void, st_codes + c * 1024), 16, 0, 0);
            }
        }

        // ---------------- score phase (lane = key)
        const SignWords<D> ks = load_signs<D>(a.kb.signs + ki * (D / 8));
        const float sk = h2f(a.kb.scales[ki]);
        const float svv = h2f(a.vb.scales[ki]);
        float rsk = 0.0f, rsv = 0.0f;
        uint32_t kc[CW];
        if constexpr (MODE == MODE_COMP) {
            rsk = h2f(a.kr.scales[ki]);
            rsv = h2f(a.vr.scales[ki]);
            const uint4* cp = (const uint4*)(a.kr.codes + ki * (D / 2));
#pragma unroll
            for (int i = 0; i < CW / 4; i++) {
                const uint4 c = cp[i];
                kc[4 * i] = c.x; kc[4 * i + 1] = c.y; kc[4 * i + 2] = c.z; kc[4 * i + 3] = c.w;
            }
        }

        float xd[G];
        uint32_t selmask = 0;
#pragma unroll
        for (int g = 0; g < G; g++) {
            int pc = 0;
#pragma unroll
            for (int w = 0; w < D / 32; w++) pc += __builtin_popcount(~(qd.signs[g][w] ^ ks.w[w]));
            const float mq = (float)(2 * pc - D);
            xd[g] = (qd.scale_q[g] * sk) * mq;  // (scale_q * scale_k) * (2pc - d)  (src/xnor_dot.cuh:179)
            if constexpr (MODE == MODE_ADAPTIVE) {
                const uint32_t key = ordered_key(sk * mq);
                const uint64_t tie = __ballot(valid && key == thresh[g]);
                bool sel = key > thresh[g];
                if (key == thresh[g] && need[g] > 0) {
                    const int before = __builtin_popcountll(tie & ((1ull << lane) - 1ull));
                    sel = (a.tie_prefix[(int64_t)(bhq0 + g) * a.n_tiles + (t0 >> 6)] + before) < need[g];
                }
                selmask |= (sel && valid) ? (1u << g) : 0u;
            }
        }
        if constexpr (MODE == MODE_ADAPTIVE) {
            if (selmask) {
                rsk = h2f(a.kr.scales[ki]);
                rsv = h2f(a.vr.scales[ki]);
                const uint4* cp = (const uint4*)(a.kr.codes + ki * (D / 2));
#pragma unroll
                for (int i = 0; i < CW / 4; i++) {
                    const uint4 c = cp[i];
                    kc[4 * i] = c.x; kc[4 * i + 1] = c.y; kc[4 * i + 2] = c.z; kc[4 * i + 3] = c.w;
                }
                const uint8_t* vc = a.vr.codes + ki * (D / 2);
#pragma unroll
                for (int c = 0; c < D / 32; c++)
                    __builtin_amdgcn_global_load_lds(
                        (const __attribute__((address_space(1))) void*)(vc + 16 * c),
                        LDS_PTR(void, st_codes + c * 1024), 16, 0, 0);
            }
            if (a.selected != nullptr && valid) {
#pragma unroll
                for (int g = 0; g < G; g++)
                    a.selected[(int64_t)(bhq0 + g) * a.S + s] = (selmask >> g) & 1u;
            }
        }

        // residual dot on the raw int4 codes: sum_i q_int_i * n_i per head
        int racc[G];
#pragma unroll
        for (int g = 0; g < G; g++) racc[g] = 0;
        if constexpr (RES) {
            bool any_res = MODE == MODE_COMP;
            if constexpr (MODE == MODE_ADAPTIVE) any_res = selmask != 0u;
            if (any_res) {
                if constexpr (G == 1) {
                    int s0 = 0, s1 = 0, s2 = 0, s3 = 0;
#pragma unroll
                    for (int w = 0; w < CW; w++) {
                        s0 = __builtin_amdgcn_sdot8(sdig[w][0], (int)kc[w], s0, false);
                        s1 = __builtin_amdgcn_sdot8(sdig[w][1], (int)kc[w], s1, false);
                        s2 = __builtin_amdgcn_sdot8(sdig[w][2], (int)kc[w], s2, false);
                        s3 = __builtin_amdgcn_sdot8(sdig[w][3], (int)kc[w], s3, false);
                    }
                    racc[0] = s0 + 16 * s1 + 256 * s2 + 4096 * s3;
                } else {
                    int sa[G][4];
#pragma unroll
                    for (int g = 0; g < G; g++) sa[g][0] = sa[g][1] = sa[g][2] = sa[g][3] = 0;
                    // an opaque zero makes the digit reads loop-variant, so they are
                    // not hoisted out of the tile loop (64 registers per head)
                    int z;
                    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
                    // code dword outer, head inner: each head's digit quad is one
                    // 16-byte LDS read right before its four v_dot8
#pragma unroll
                    for (int w = 0; w < CW; w++) {
#pragma unroll
                        for (int g = 0; g < G; g++) {
                            const int4 dg = qd.digits[g][w + z];
                            sa[g][0] = __builtin_amdgcn_sdot8(dg.x, (int)kc[w], sa[g][0], false);
                            sa[g][1] = __builtin_amdgcn_sdot8(dg.y, (int)kc[w], sa[g][1], false);
                            sa[g][2] = __builtin_amdgcn_sdot8(dg.z, (int)kc[w], sa[g][2], false);
                            sa[g][3] = __builtin_amdgcn_sdot8(dg.w, (int)kc[w], sa[g][3], false);
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
#pragma unroll
                    for (int g = 0; g < G; g++)
                        racc[g] = sa[g][0] + 16 * sa[g][1] + 256 * sa[g][2] + 4096 * sa[g][3];
                }
            }
        }
        float sc[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            float score = xd[g];
            bool use_res = MODE == MODE_COMP;
            if constexpr (MODE == MODE_ADAPTIVE) use_res = (selmask >> g) & 1u;
            if (RES && use_res) score = score + (float)racc[g] * (qd.dq[g] * (rsk * (1.0f / 7.0f)));
            sc[g] = valid ? score * isd2 : -INFINITY;
        }

        // ---------------- weight scale for this tile (p <= 1, so w <= max(2 sv, rs/7))
        {
            float wb = valid ? fmaxf(2.0f * svv, rsv * (1.0f / 7.0f)) : 0.0f;
            wb = wave_max(wb);
            if (wb > 0.0f && wb < INFINITY) {
                const int e = 14 - (int)ceilf(log2f(wb));
                if (!have_wexp) {
                    wexp = e;
                    have_wexp = true;
                } else if (e < wexp) {
                    // a larger weight than planned: bring the accumulated sums down
                    const float f = ldexpf(1.0f, e - wexp);
#pragma unroll
                    for (int h = 0; h < NH; h++)
#pragma unroll
                        for (int p = 0; p < 4; p++) cs[h][p] *= f;
#pragma unroll
                    for (int d = 0; d < NB; d++) cn[d] *= f;
#pragma unroll
                    for (int g = 0; g < G; g++) off[g] *= f;
                    wexp = e;
                }
            }
        }

        // ---------------- online softmax, weights for the value MFMAs
        float lane_alpha = 1.0f;
        bool any_rescale = false;
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float mt = wave_max(sc[g]);
            const float mn = fmaxf(m[g], mt);
            if (mn > m[g]) {
                const float alpha = exp2f(m[g] - mn);
                lsum[g] *= alpha;
                off[g] *= alpha;
                if (my_head == g) lane_alpha = alpha;
                any_rescale = true;
                m[g] = mn;
            }
            const float p = valid ? exp2f(sc[g] - mn) : 0.0f;
            lsum[g] += p;
            const float a2 = ldexpf(2.0f * p * svv, wexp);
            float bv = 0.0f;
            if constexpr (MODE == MODE_COMP) bv = ldexpf(p * (rsv * (1.0f / 7.0f)), wexp);
            if constexpr (MODE == MODE_ADAPTIVE)
                bv = ((selmask >> g) & 1u) ? ldexpf(p * (rsv * (1.0f / 7.0f)), wexp) : 0.0f;
            const uint16_t a2h = f2h_bits(a2);
            const uint16_t a2l = f2h_bits(a2 - h_bits2f(a2h));
            const uint16_t bh = f2h_bits(bv);
            const uint16_t bl = f2h_bits(bv - h_bits2f(bh));
            // offset removed at the end: sum_s (a_s + 8 b_s) with the weights as rounded
            off[g] += 0.5f * (h_bits2f(a2h) + h_bits2f(a2l)) + 8.0f * (h_bits2f(bh) + h_bits2f(bl));
            const int sl = slot_of(lane);
            wts[(0 * 16 + 2 * g) * 64 + sl] = a2h;
            wts[(0 * 16 + 2 * g + 1) * 64 + sl] = a2l;
            wts[(1 * 16 + 2 * g) * 64 + sl] = bh;
            wts[(1 * 16 + 2 * g + 1) * 64 + sl] = bl;
        }
        if (any_rescale) {
            if (my_head >= G) lane_alpha = 1.0f;
#pragma unroll
            for (int h = 0; h < NH; h++)
#pragma unroll
                for (int p = 0; p < 4; p++) cs[h][p] *= lane_alpha;
#pragma unroll
            for (int d = 0; d < NB; d++) cn[d] *= lane_alpha;
        }

        // V tile and weights must be in LDS before the transposed reads
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");

        // B operands: (hi, lo) weight columns; unused columns are zero
        h8_t bsig[2], bres[2];
#pragma unroll
        for (int mh = 0; mh < 2; mh++) {
            if (my_col < 2 * G) {
                bsig[mh] = *(const h8_t*)&wts[(0 * 16 + my_col) * 64 + 16 * g4 + 8 * mh];
                bres[mh] = *(const h8_t*)&wts[(1 * 16 + my_col) * 64 + 16 * g4 + 8 * mh];
            } else {
                bsig[mh] = h8_t{0, 0, 0, 0, 0, 0, 0, 0};
                bres[mh] = bsig[mh];
            }
        }

        // ---------------- sign part: rows = dims 64h + 4*lj + p
        const int row_key = 16 * g4 + lj;  // this lane addresses row (key) lj of its group
#pragma unroll
        for (int h = 0; h < NH; h++) {
            const uint8_t* rp = (SB >= 16) ? st_signs + (h >> 1) * 1024 + 16 * row_key + 8 * (h & 1)
                                           : st_signs + 8 * row_key;
            const v2i_t w = __builtin_amdgcn_ds_read_tr4_b64_v2i32(LDS_PTR(v2i_t, rp));
#pragma unroll
            for (int mh = 0; mh < 2; mh++) {
                const uint32_t x = (uint32_t)(mh ? w.y : w.x);
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    uint32_t pw[4];
#pragma unroll
                    for (int k = 0; k < 4; k++) pw[k] = (x >> (4 * k + p)) & 0x00010001u;
                    const h8_t av = __builtin_bit_cast(h8_t, pw);
                    cs[h][p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bsig[mh], cs[h][p], 0, 0, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }

        // ---------------- residual part: rows = dims 16db + lj
        if constexpr (RES) {
            bool any_sel = true;
            if constexpr (MODE == MODE_ADAPTIVE) any_sel = __ballot(selmask != 0u) != 0ull;
            if (any_sel) {
#pragma unroll
                for (int db = 0; db < NB; db++) {
                    const uint8_t* rp = st_codes + (db >> 1) * 1024 + 16 * row_key + 8 * (db & 1);
                    const v2i_t w = __builtin_amdgcn_ds_read_tr4_b64_v2i32(LDS_PTR(v2i_t, rp));
#pragma unroll
                    for (int mh = 0; mh < 2; mh++) {
                        const uint32_t x = (uint32_t)(mh ? w.y : w.x) ^ 0x88888888u;
                        uint32_t pw[4];
#pragma unroll
                        for (int k = 0; k < 4; k++) pw[k] = (x >> (4 * k)) & 0x000F000Fu;
                        const h8_t av = __builtin_bit_cast(h8_t, pw);
                        cn[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bres[mh], cn[db], 0, 0, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
        // all LDS reads of this tile retire before the next tile's loads land
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_wave_barrier();
    }

    // ---------------- epilogue: per wave, per head: acc[e] = ((cs + cn) * 2^24 - off) * 2^-wexp
    float* accw = (float*)my;  // [2 parts][G][D] floats + G offsets
    const float two24 = 16777216.0f;
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float l_w = wave_sum(lsum[g]);
        const float o_w = wave_sum(off[g]);
        if (lane == 0) {
            wm[wave][g] = m[g];
            wlsum[wave][g] = l_w;
            wsc[wave] = ldexpf(1.0f, -wexp);
            accw[2 * G * D + g] = o_w;  // stash after the arrays
        }
    }
    // hi + lo columns are adjacent lanes (col 2g, 2g+1)
#pragma unroll
    for (int h = 0; h < NH; h++)
#pragma unroll
        for (int p = 0; p < 4; p++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float v = cs[h][p][i] + __shfl_xor(cs[h][p][i], 1, 64);
                if (my_col < 2 * G && (my_col & 1) == 0) {
                    const int dim = 64 * h + 4 * (4 * g4 + i) + p;
                    accw[(0 * G + my_head) * D + dim] = v;
                }
            }
    if constexpr (RES) {
#pragma unroll
        for (int d = 0; d < NB; d++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float v = cn[d][i] + __shfl_xor(cn[d][i], 1, 64);
                if (my_col < 2 * G && (my_col & 1) == 0) {
                    const int dim = 16 * d + 4 * g4 + i;
                    accw[(1 * G + my_head) * D + dim] = v;
                }
            }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < G * D; i += blockDim.x) {
        const int g = i / D, e = i % D;
        float M = -INFINITY;
        for (int w = 0; w < 4; w++) M = fmaxf(M, wm[w][g]);
        float accv = 0.0f, lv = 0.0f;
        if (M != -INFINITY) {
            for (int w = 0; w < 4; w++) {
                if (wm[w][g] == -INFINITY) continue;
                const float f = exp2f(wm[w][g] - M);
                const float* aw = (const float*)wave_lds[w];
                float v = aw[(0 * G + g) * D + e];
                if (RES) v += aw[(1 * G + g) * D + e];
                v = (v * two24 - aw[2 * G * D + g]) * wsc[w];
                accv += f * v;
                lv += f * wlsum[w][g];
            }
        }
        float* dst = a.ws + ((int64_t)(bhq0 + g) * a.n_splits + split) * (D + 2);
        dst[2 + e] = accv;
        if (e == 0) {
            dst[0] = M;
            dst[1] = lv;
        }
    }
}

template <int D, int G>
void launch_dg(int mode, const AttnArgs& a, dim3 grid, hipStream_t st) {
    if (mode == MODE_BINARY)
        hipLaunchKernelGGL((attn_mfma_kernel<D, G, MODE_BINARY>), grid, dim3(256), 0, st, a);
    else if (mode == MODE_COMP)
        hipLaunchKernelGGL((attn_mfma_kernel<D, G, MODE_COMP>), grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((attn_mfma_kernel<D, G, MODE_ADAPTIVE>), grid, dim3(256), 0, st, a);
}

template <int D>
void launch_d(int mode, int G, const AttnArgs& a, dim3 grid, hipStream_t st) {
    switch (G) {
        case 8: launch_dg<D, 8>(mode, a, grid, st); break;
        case 4: launch_dg<D, 4>(mode, a, grid, st); break;
        case 2: launch_dg<D, 2>(mode, a, grid, st); break;
        default: launch_dg<D, 1>(mode, a, grid, st); break;
    }
}

}  // namespace

namespace bc {

bool launch_mfma_split(int mode, int D, int G, const AttnArgs& a, dim3 grid, hipStream_t st) {
    switch (D) {
        case 64: launch_d<64>(mode, G, a, grid, st); return true;
        case 128: launch_d<128>(mode, G, a, grid, st); return true;
        case 256: launch_d<256>(mode, G, a, grid, st); return true;
        default: return false;
    }
}

}  // namespace bc
