// Split-KV decode attention with the value phase on the matrix cores (gfx950).
//
// Same work decomposition and partial format as attn_split_kernel
// (attention.hip): grid.x = key split, grid.y = (b, kv head, query-head
// group), 4 wave64 per workgroup, 64-key tiles round-robin over the waves.
//
// Score phase (lane = key): XNOR popcount of the sign words, and the INT4
// residual dot directly on the stored two's-complement nibbles against the
// query in 24-bit fixed point: six balanced int4 digits for v_dot8_i32_i4
// (MHA) or three balanced int8 planes for an int8 MFMA (GQA groups), of which
// a tile uses the top 16 bits unless a key's residual scale makes it a
// precise tile.
//
// Value phase: out[e] = sum_s a_s*(2*bit_se - 1) + b_s*(u_se - 8) with
// a = p*sv, b = p*rs/7, u = n + 8.  The V tile (sign bytes and code bytes of
// 64 keys) is copied to LDS with direct buffer loads, then ds_read_b64_tr_b4
// transposes 16 keys x 16 nibbles per 16-lane group so that each lane holds
// 16 keys of one dimension.  fp16 path: nibbles (u) and sign bits become
// exact fp16 subnormals (value * 2^(j-24) for bit position j < 10) with one
// mask per pair of keys, left in place (the power of two is folded into the
// weights of odd keys and into the accumulator of bit p), and
// v_mfma_f32_16x16x32_f16 accumulates dims x weight-columns, where the weight
// columns are (hi, lo) fp16 splits of a and b for each query head of the
// group; the fp32 accumulators are rescaled on running-max changes.  int8
// path (the sign part of binary and adaptive attention, groups up to 4):
// sign bits in place as int8 elements, four keys per mask, weights as
// balanced 8-bit digit columns, exact int32 sums flushed into a float bank on
// rescales (see I8 below).
#include <math.h>

#include "attn.h"
#include "encode_row.h"

#include <map>
#include <mutex>
#include <tuple>

using bc::AttnArgs;
using bc::kLog2e;
using bc::MODE_ADAPTIVE;
using bc::MODE_BINARY;
using bc::MODE_COMP;
using bc::MODE_MIXED;

namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef int v2i_t __attribute__((ext_vector_type(2)));
typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef unsigned int v4u_t __attribute__((ext_vector_type(4)));
typedef unsigned int v2u_t __attribute__((ext_vector_type(2)));
#define LDS_PTR(T, p) ((__attribute__((address_space(3))) T*)(p))

// Word 3 of a gfx9 buffer resource for raw byte-addressed loads (32-bit data
// format, no swizzle; with stride 0 a load past num_records returns zeros).
constexpr int kBufWord3 = 0x00020000;

// D/8 sign bytes at byte offset off of a buffer, as D/32 words.
template <int D, int AUX>
__device__ __forceinline__ SignWords<D> buf_signs(__amdgpu_buffer_rsrc_t r, int off) {
    SignWords<D> s;
    if constexpr (D % 128 == 0) {
#pragma unroll
        for (int i = 0; i < D / 128; i++) {
            const v4u_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * i, 0, AUX);
            s.w[4 * i + 0] = v[0]; s.w[4 * i + 1] = v[1]; s.w[4 * i + 2] = v[2]; s.w[4 * i + 3] = v[3];
        }
    } else {
        static_assert(D % 64 == 0, "sign rows of 8-byte multiples");
#pragma unroll
        for (int i = 0; i < D / 64; i++) {
            const v2u_t v = __builtin_amdgcn_raw_buffer_load_b64(r, off + 8 * i, 0, AUX);
            s.w[2 * i + 0] = v[0]; s.w[2 * i + 1] = v[1];
        }
    }
    return s;
}

// The query of the INT4 residual dot as 24-bit fixed point:
// q_int = rint(q / step), step = max|q| / kQIntMax, written as six balanced
// int4 digits (q_int = sum_j d_j 16^j, d_j in [-8, 7]) or three balanced int8
// planes (q_int = p0 + 256 p1 + 65536 p2).  A tile's dots use the top 16 bits
// (digits 2..5, planes 1..2: q_int / 256 within 0.53, i.e. 16-bit fixed point
// of step 256*step) unless a key of the tile could see a score error above
// kPrecNats from it; then the low digits / plane are added (an fp32-level
// error).  kQIntMax leaves room below 7*(16^6 - 1)/15 = 7829367, the largest
// six-digit value, for the rounding of q / step.
constexpr float kQIntMax = 7800000.0f;
constexpr float kPrecNats = 1.0f / 2048.0f;

template <int D, int G>
struct QDigits {
    uint32_t signs[G][D / 32];
    int4 digits[G][D / 8];        // .x..w = balanced int4 digits 2..5 of q_int of elements 8w..8w+7 (nibble k = element 8w+k)
    int2 digits_lo[G][D / 8];     // digits 0..1
    // int8 MFMA B operands of the K residual dot (GQA groups, d >= 128):
    // [piece][half][lane] (see the kernel): planes 1, 2 (and plane 0 where
    // the columns hold it), and plane 0 for groups of more than 5 heads
    int4 bq[(G > 1 && D >= 128) ? D / 128 : 1][2][(G > 1 && D >= 128) ? 64 : 1];
    int4 bq_lo[(G > 5 && D >= 128) ? D / 128 : 1][2][(G > 5 && D >= 128) ? 64 : 1];
    float scale_q[G];             // sequential mean |q| (src/compensated_attention.cu:65-67)
    float dq[G];                  // step of the top 16 bits: 256 * step of q_int
    // bound on a key's score error (nats) from the top-16-bit dot, per unit of
    // its residual scale: 0.53 * max_g dq * D / sqrt(D)
    float prec_bound;
};

// Per-wave LDS, one __shared__ array per role (the compiler tracks LDS
// direct loads per array, so reading staging buffer i or the weights does not
// wait for the direct loads still landing in buffer i+1): V staging buffers
// (tile i is consumed while tile i+1 lands), each the tile's code bytes then
// its sign bytes; the (hi, lo) fp16 weight columns [part][2G][72 slots]; the
// K-side residual dots [64 keys][G] of GQA groups.  The epilogue reduces heads
// in batches through staging buffer 0.  Binary attention stages no codes.
template <int D, int G, bool RES>
struct WaveLds {
    static constexpr int kCodeBytes = RES ? 64 * D / 2 : 0;
    // D = 64: 8-byte sign rows are copied two keys per lane by all 64 lanes
    // (lanes 32..63 repeat lanes 0..31 into the second half), hence 1 KB
    static constexpr int kSignBytes = 64 * D / 8 > 1024 ? 64 * D / 8 : 1024;
    static constexpr int kStage = kCodeBytes + kSignBytes;
    // weight columns of 72 slots (64 used): the 16 lanes of a row group read
    // 16-byte runs of 16 columns without LDS bank conflicts
    static constexpr int kColSlots = 72;
    static constexpr int kWeightBytes = 2 * 2 * G * kColSlots * 2;
    static constexpr int kRdInts = (G > 1 && RES) ? 64 * G : 4;
    // epilogue: heads per pass through staging buffer 0 ([parts][heads][D] floats)
    static constexpr int kEpiHeads = kStage / ((RES ? 2 : 1) * D * 4) < G ? kStage / ((RES ? 2 : 1) * D * 4) : G;
    static_assert(kEpiHeads >= 1, "staging buffer holds one head's partial sums");
};

// K-side data of one 64-key tile held in registers: sign words and scales of
// the lane's own key, and the lane's code pieces (see the kernel).
template <int D>
struct KRegs {
    SignWords<D> ks;              // (adaptive mode: the stored popcounts instead)
    uint32_t pcw[4];              // adaptive: the G popcounts of the lane's key
    uint32_t kc[D / 8];           // (adaptive mode: gathered later, selected keys)
    uint16_t sk, svv, rsk, rsv;   // raw fp16 scales (converted at use, so the
                                  // loads of the next tile are not waited on)
    uint32_t sel;                 // adaptive: bit g = head g selected the lane's key
};

// Eight INT4 codes of two dwords as the int8 MFMA operand 16*n (signed): low
// nibbles shifted up, high nibbles masked in place.
__device__ __forceinline__ v4i_t codes_i8(uint32_t x0, uint32_t x1) {
    return v4i_t{(int)((x0 << 4) & 0xF0F0F0F0u), (int)(x0 & 0xF0F0F0F0u), (int)((x1 << 4) & 0xF0F0F0F0u),
                 (int)(x1 & 0xF0F0F0F0u)};
}

// x through an empty asm: the compiler cannot split or re-associate it
__device__ __forceinline__ int opaque_int(int x) {
    asm volatile("" : "+v"(x));
    return x;
}

__device__ __forceinline__ uint16_t f2h_bits(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float h_bits2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// slot position of key k (0..63) inside the weight columns: for MFMA half mh of
// group g4, slots (2t, 2t+1) hold keys (t, t+4) of the 8-key run.
__device__ __forceinline__ int slot_of(int k) {
    const int g4 = k >> 4, mh = (k >> 3) & 1, r = k & 7;
    return 16 * g4 + 8 * mh + ((r & 3) << 1) + (r >> 2);
}

// Slot of key k in the int8 weight columns: the 16 K-slots of lane group g4
// in the 16x16x64 int8 MFMA are the keys of that group's transposed sign
// read in register order, i.e. even then odd nibbles of its first word
// (keys 16g4 + 0..7), then of its second (keys 16g4 + 8..15).
__device__ __forceinline__ int slot8_of(int k) {
    const int g4 = k >> 4, hw = (k >> 3) & 1, r = k & 7;
    return 16 * g4 + 8 * hw + 4 * (r & 1) + (r >> 1);
}

// Adaptive mode packs the keys of a tile that some head selected into
// positions 0..n-1 of its residual data.  Position j sits in V staging row
// res_row(j): rows 16g + 0..7 feed MFMA half 0 and rows 16g + 8..15 half 1, so
// positions 0..31 are exactly the rows of half 0.  res_pos is the inverse.
__device__ __forceinline__ int res_row(int j) { return 16 * ((j >> 3) & 3) + 8 * (j >> 5) + (j & 7); }
__device__ __forceinline__ int res_pos(int row) { return 32 * ((row >> 3) & 1) + 8 * (row >> 4) + (row & 7); }
__device__ __forceinline__ int mbcnt64(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Workgroup barrier for data exchanged through LDS only: this wave's LDS
// stores have completed (lgkmcnt), the compiler moves no memory access across
// it, and loads in flight (the first tile's, some into other LDS arrays) stay
// in flight.  A __syncthreads() would also wait for every direct-to-LDS load.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Query preparation of one workgroup (NT threads), spread over all threads:
// the query as floats and its sign words (a wave ballot per 64 elements);
// scale_q (sequential fp32 order, element 0 first) and the fixed-point step
// per head; q_int = rint(q / step) per element (in place of the floats); then
// the balanced int4 digit words (one (word, digit) pair per thread) and the
// int8 MFMA operand words (the fixed-point parts only for residual modes).
template <int D, int G, bool KMF, bool RES, int NT, int NQ>
__device__ void prep_digits(const uint16_t (&qpre)[NQ], QDigits<D, G>& qd, float* qf) {
    static_assert((G * D) % 64 == 0, "whole waves of query elements");
    const int tid = threadIdx.x, lane = tid & 63;
    uint32_t* signs = &qd.signs[0][0];   // [G * D / 32] words, bit b of word i = element 32i + b
    __shared__ float gmax[G * D / 64];   // max |q| of each 64-element group
    // the three int8 planes of q_int per element (int8 MFMA operands)
    __shared__ __attribute__((aligned(8))) uint8_t pbytes[KMF ? 3 : 1][KMF ? G * D : 8];
    // floats, sign words (wave ballots) and each wave's max |q| (its 64
    // elements lie in one head); element tid + NT j was loaded into qpre[j]
#pragma unroll
    for (int j = 0; j < NQ; j++) {
        const int i = tid + NT * j;
        if (i >= G * D) break;   // (whole waves)
        const float x = h2f(qpre[j]);
        qf[i] = x;
        const uint64_t bits = __ballot(x >= 0.0f);
        const float wm = wave_max(fabsf(x));
        if (lane == 0) {
            signs[i / 32] = (uint32_t)bits;
            signs[i / 32 + 1] = (uint32_t)(bits >> 32);
            gmax[i / 64] = wm;
        }
    }
    lds_barrier();
    if (tid < G) {
        // sequential fp32 order (element 0 first), eight float4 reads in
        // flight at a time
        float acc = 0.0f;
        const float4* q4 = (const float4*)&qf[tid * D];
#pragma unroll
        for (int c0 = 0; c0 < D / 4; c0 += 8) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = q4[c0 + u];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                acc += fabsf(v[u].x); acc += fabsf(v[u].y); acc += fabsf(v[u].z); acc += fabsf(v[u].w);
            }
        }
        qd.scale_q[tid] = acc / (float)D;
        float mx = 0.0f;
#pragma unroll
        for (int k = 0; k < D / 64; k++) mx = fmaxf(mx, gmax[tid * (D / 64) + k]);
        qd.dq[tid] = mx > 0.0f ? 256.0f * (mx / kQIntMax) : 256.0f;
    }
    lds_barrier();
    // binary attention needs only the sign words and scale_q
    if constexpr (!RES) return;
    if (tid == 0) {
        float m = 0.0f;
        for (int g = 0; g < G; g++) m = fmaxf(m, qd.dq[g]);
        qd.prec_bound = 0.53f * m * sqrtf((float)D);
    }
    // q_int over the floats (each thread converts the elements it reads) and
    // its balanced int8 planes, q_int = p0 + 256 p1 + 65536 p2, p_i in [-128, 127]
    int* qint = (int*)qf;
    for (int i = tid; i < G * D; i += NT) {
        const int t = (int)__builtin_rintf(qf[i] / (qd.dq[i / D] * (1.0f / 256.0f)));
        qint[i] = t;
        if constexpr (KMF) {
            const int p0 = ((t + 128) & 255) - 128;
            const int t1 = (t - p0) >> 8;
            const int p1 = ((t1 + 128) & 255) - 128;
            pbytes[0][i] = (uint8_t)p0;
            pbytes[1][i] = (uint8_t)p1;
            pbytes[2][i] = (uint8_t)((t1 - p1) >> 8);
        }
    }
    lds_barrier();
    // digit j of the 8 elements of word w: nibble k = element 8w + k (balanced
    // base 16: t = sum_j d_j 16^j, d_j in [-8, 7]).  Four threads per word
    // (a DPP quad), two elements each; the quad ORs its nibbles together.
    static_assert((G * D / 2) % 4 == 0, "whole quads per digit word");
    for (int e = tid; e < G * (D / 2); e += NT) {
        const int gw = e >> 2, q = e & 3, g = gw / (D / 8), w = gw % (D / 8);
        uint32_t word[6];
#pragma unroll
        for (int j = 0; j < 6; j++) word[j] = 0u;
#pragma unroll
        for (int k = 2 * q; k < 2 * q + 2; k++) {
            int t = qint[g * D + 8 * w + k];
#pragma unroll
            for (int j = 0; j < 6; j++) {
                const int d = ((t + 8) & 15) - 8;
                word[j] |= ((uint32_t)d & 0xFu) << (4 * k);
                t = (t - d) >> 4;
            }
        }
#pragma unroll
        for (int j = 0; j < 6; j++) {
            word[j] |= dpp_u<0xB1>(word[j]);   // quad 1,0,3,2
            word[j] |= dpp_u<0x4E>(word[j]);   // quad 2,3,0,1
        }
        if (q == 0) {
            qd.digits[g][w] = make_int4((int)word[2], (int)word[3], (int)word[4], (int)word[5]);
            qd.digits_lo[g][w] = make_int2((int)word[0], (int)word[1]);
        }
    }
    if constexpr (KMF) {
        // B operand words: column c = 2g + p (c < 2G) holds plane p + 1 of
        // head g, column 2G + g plane 0 of head g when 3G <= 16 (bq_lo column
        // 2g otherwise); slot s = 4r + j of lane group q for piece pc and half
        // h holds dim 32 (q + 4 pc) + 8 (2h + r/2) + 2j + r%2, where the
        // unpacked codes put it: words r = 2rr, 2rr + 1 are the even and odd
        // bytes of the 8 plane bytes at dim 32 (q + 4 pc) + 8 (2h + rr)
        constexpr int NPC = D / 128;
        constexpr bool LO_COLS = 3 * G <= 16;
        for (int e = tid; e < NPC * 2 * 64; e += NT) {
            const int pc = e / 128, h = (e / 64) & 1, ln = e & 63;
            const int col = ln & 15, qg4 = ln >> 4;
            int gv = 0, pv = -1;   // the lane's column: plane pv of head gv (pv < 0: zeros)
            if (col < 2 * G) {
                gv = col >> 1;
                pv = (col & 1) ? 2 : 1;
            } else if (LO_COLS && col < 3 * G) {
                gv = col - 2 * G;
                pv = 0;
            }
            const bool lo_col = !LO_COLS && col < 2 * G && !(col & 1);
            int wd[4] = {0, 0, 0, 0}, wl[4] = {0, 0, 0, 0};
#pragma unroll
            for (int rr = 0; rr < 2; rr++) {
                const int at = gv * D + 32 * (qg4 + 4 * pc) + 8 * (2 * h + rr);
                if (pv >= 0) {
                    const bc_v2u x = *(const bc_v2u*)&pbytes[pv][at];
                    wd[2 * rr] = (int)__builtin_amdgcn_perm(x[1], x[0], 0x06040200u);
                    wd[2 * rr + 1] = (int)__builtin_amdgcn_perm(x[1], x[0], 0x07050301u);
                }
                if (lo_col) {
                    const bc_v2u x = *(const bc_v2u*)&pbytes[0][at];
                    wl[2 * rr] = (int)__builtin_amdgcn_perm(x[1], x[0], 0x06040200u);
                    wl[2 * rr + 1] = (int)__builtin_amdgcn_perm(x[1], x[0], 0x07050301u);
                }
            }
            qd.bq[pc][h][ln] = make_int4(wd[0], wd[1], wd[2], wd[3]);
            if constexpr (!LO_COLS) qd.bq_lo[pc][h][ln] = make_int4(wl[0], wl[1], wl[2], wl[3]);
        }
    }
    lds_barrier();
}

// Build-time switches; each default is the measured fastest on MI355X:
//   BC_MHA_WAVES   waves/SIMD the MHA compensated kernel's registers target (3)
//   BC_BIN_WAVES   the same for binary attention of groups up to 2 (5)
//   BC_ADAPT_WAVES the same for adaptive attention up to d = 128 (2; its LDS
//                  holds two workgroups per CU at d = 128)
//   BC_LIN_K / BC_LIN_V  code tiles read as linear KiB runs (1) instead of per key
//   BC_MHA_PIPE / BC_ADAPT_PIPE / BC_GQA_PIPE  one-tile prefetch with two staging
//                  buffers for MHA (1), adaptive (1) and GQA compensated (0: one
//                  buffer keeps a third workgroup per CU) kernels
//   BC_NT_AUX      cache policy of the loads that cover whole KiB runs (K and V
//                  sign rows, the linear V code tile, the K code blocks of GQA
//                  groups, linear K code rows): 2 = nontemporal (8-11% faster;
//                  lines that several loads share keep the default policy)
//   BC_NT_SCALES   cache policy of the 2-byte scale loads (0: default)
#ifndef BC_MHA_WAVES
#define BC_MHA_WAVES 3
#endif
#ifndef BC_LIN_K
#define BC_LIN_K 1
#endif
#ifndef BC_LIN_V
#define BC_LIN_V 1
#endif
#ifndef BC_MHA_PIPE
#define BC_MHA_PIPE 1
#endif
#ifndef BC_ADAPT_PIPE
#define BC_ADAPT_PIPE 1
#endif
#ifndef BC_GQA_PIPE
#define BC_GQA_PIPE 0
#endif
#ifndef BC_BIN_WAVES
#define BC_BIN_WAVES 5
#endif
#ifndef BC_NT_AUX
#define BC_NT_AUX 2
#endif
#ifndef BC_NT_SCALES
#define BC_NT_SCALES 0
#endif
#ifndef BC_ADAPT_WAVES
#define BC_ADAPT_WAVES 2
#endif
template <int D, int G, int MODE>
struct Occupancy {
    static constexpr int kWaves =
        MODE == MODE_BINARY     ? (D <= 128 ? (G <= 2 ? BC_BIN_WAVES : 3) : 2)
        : MODE == MODE_ADAPTIVE ? (D <= 128 ? BC_ADAPT_WAVES : 1)
        : (G == 1 && D <= 128)  ? BC_MHA_WAVES
                                : (D <= 128 ? (G <= 4 && !BC_GQA_PIPE ? 3 : 2) : 1);
};

// Sum of v over the Q consecutive lanes that share one key row (DPP, no LDS).
template <int Q>
__device__ __forceinline__ int row_group_sum(int v) {
    if constexpr (Q >= 2) v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);   // quad_perm [1,0,3,2]
    if constexpr (Q >= 4) v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);   // quad_perm [2,3,0,1]
    if constexpr (Q >= 8) v += __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true);  // row_half_mirror
    return v;
}

// NW waves per workgroup (4, or 8 to 16 for a wide workgroup that takes all
// keys of its group: one split, no merge launch); wave w takes tiles w, w + NW,
// w + 2 NW, ... of the key range, and the epilogue merges the NW waves.
template <int D, int G, int MODE, int NW = 4>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(Occupancy<D, G, MODE>::kWaves)))
void attn_mfma_kernel(AttnArgs a) {
    constexpr int NB = D / 16;   // nibble dim-blocks (16 dims each)
    constexpr int NH = D / 64;   // sign blocks (64 dims each)
    constexpr int CW = D / 8;    // code dwords per key
    constexpr bool RES = MODE != MODE_BINARY;
    constexpr int SB = D / 8;    // sign bytes per key
    constexpr int CB = D / 2;    // code bytes per key
    // Code loads.  Per key (lane = key): lane l reads its key's row in 16-byte
    // pieces, so one load touches 64 rows.  Linear: load round i, lane l takes
    // the 16 bytes at i*1024 + 16*l of the tile (contiguous KiB), i.e. piece
    // l%Q of key i*(64/Q) + l/Q; for K this needs a Q-lane reduction of the
    // partial dots.  The adaptive mode gathers only selected keys' codes and
    // always works per key.
    // GQA groups (d >= 128): the K residual dots of all G heads come from one
    // set of int8 MFMAs (keys x dims times dims x (head, digit plane)); the
    // lane holds 16-byte code pieces of 16 keys instead of one key's row
    constexpr bool KMF = G > 1 && RES && D >= 128;
    constexpr int NPC = D / 128;  // 16-byte pieces per lane per 16-key block
    // every key's residual data is read (compensated, and mixed per-head modes)
    constexpr bool ALLRES = MODE == MODE_COMP || MODE == MODE_MIXED;
    constexpr bool LIN_K = (BC_LIN_K || G > 1) && ALLRES && !KMF;
    constexpr bool LIN_V = BC_LIN_V && ALLRES;
    constexpr int Q = D / 32;    // 16-byte pieces per code row
    // Vector-memory operations issued per prefetched tile, counted at their
    // fewest (a load moves at most 16 bytes; planes are separate loads), so
    // waiting down to this many outstanding operations completes everything
    // issued before the prefetch and never less.
    constexpr int kSignDma = SB >= 16 ? SB / 16 : 1;
    constexpr int kVDma = kSignDma + (ALLRES ? Q : 0);
    constexpr int kKLoads = (SB + 15) / 16 + (RES ? 4 + Q : 2);
    constexpr int kPrefetchOps = kVDma + kKLoads;
    static_assert(kPrefetchOps + kVDma < 64, "vmcnt holds 6 bits");
    // GQA groups in compensated mode run without the one-tile prefetch: one
    // staging buffer and one K register set leave room for a third workgroup
    // per CU (measured faster); adaptive mode keeps it
    constexpr bool PIPE = (G == 1 && BC_MHA_PIPE) || (MODE == MODE_ADAPTIVE && BC_ADAPT_PIPE) || BC_GQA_PIPE;
    using WL = WaveLds<D, G, RES>;
    // Binary and adaptive modes, groups up to 4: the sign-part value MFMAs
    // run on int8 operands (the residual part keeps fp16).  The sign bits
    // enter in place (element 2^p for bit p of a nibble, four keys per AND
    // instead of two fp16 elements) and each weight as an integer below 2^22
    // in three balanced 8-bit digit columns (columns 4g + plane, the fourth
    // unused), summed exactly in int32 accumulators.  A rescale (running max
    // or weight plan) flushes those sums, scaled, into a per-wave float bank
    // in LDS and restarts them at zero (flush8).
    constexpr bool I8 = (MODE == MODE_BINARY || MODE == MODE_ADAPTIVE) && G <= 4;
    constexpr int kW8Stride = 80;   // bytes per int8 weight column (64 slots + pad)

    __shared__ QDigits<D, G> qd;
    __shared__ __attribute__((aligned(16))) float qf[G * D];
    __shared__ __attribute__((aligned(16))) uint8_t lds_st0[NW][WL::kStage];
    __shared__ __attribute__((aligned(16))) uint8_t lds_st1[NW][PIPE ? WL::kStage : 16];
    __shared__ __attribute__((aligned(16))) uint16_t lds_wts[NW][(I8 && !RES) ? 8 : WL::kWeightBytes / 2];
    __shared__ __attribute__((aligned(16))) int8_t lds_w8[NW][I8 ? 4 * G * kW8Stride : 16];
    // (int8 path) per wave and head, the float sums of the keys before the
    // last rescale, [head][D] in the epilogue's dim order
    __shared__ __attribute__((aligned(16))) float lds_bank[NW][I8 ? G * D : 4];
    __shared__ __attribute__((aligned(16))) int lds_rd[NW][WL::kRdInts];
    __shared__ __attribute__((aligned(16))) int lds_rdlo[NW][(KMF && 3 * G <= 16) ? WL::kRdInts : 1];
    __shared__ float wofs[NW][G];
    __shared__ float wm[NW][G], wlsum[NW][G], wsc[NW];

    const int split = blockIdx.x;
    const int nqg = (a.Hq / a.Hkv) / G;
    // per-head modes: this launch's query-head groups come from its list
    int grow = blockIdx.y;
    if constexpr (MODE == MODE_BINARY || MODE == MODE_MIXED) {
        if (a.group_list != nullptr) {
            if (grow >= *a.group_count) return;
            grow = a.group_list[grow];
        }
    }
    const int qg = grow % nqg;
    const int bkv = grow / nqg;
    const int b = bkv / a.Hkv, kvh = bkv % a.Hkv;
    const int hq0 = kvh * (a.Hq / a.Hkv) + qg * G;
    const int bhq0 = b * a.Hq + hq0;

    // the wave index is uniform: readfirstlane lets the compiler keep the tile
    // loop in scalar registers (a uniform loop, not an exec-masked one)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int g4 = lane >> 4, lj = lane & 15;
    const int key_begin = split * a.chunk;
    const int key_end = min(a.S, key_begin + a.chunk);
    const int64_t kv_base = (int64_t)bkv * a.kv_stride;
    const float isd2 = (1.0f / sqrtf((float)D)) * kLog2e;
    // the key whose score this lane computes (tile-relative)
    const int kown = LIN_K ? (lane % Q) * (64 / Q) + lane / Q : lane;
    const int quarter = lane % Q;
    // V code tiles of compensated mode (linear rows of CB bytes): the 16-byte
    // pieces of row k are stored at piece ^ vsw(k), vsw(k) = (k*CB/256) mod Q,
    // so the rows that one transposed read covers spread over the LDS banks;
    // the copy permutes the pieces within each row (same cache lines).  A
    // lane's transposed reads cover row = lane.
    const int vsw = ((lane * CB) >> 8) & (Q - 1);

    // Buffer resources over this workgroup's key range [key_begin, key_end)
    // of each plane: offsets are 32-bit and tile-relative, and a load of a key
    // past the range returns zeros (its weight is 0), so no lane clamps its
    // address and every lane issues the same loads (the wait counts stay exact)
    const int nk = max(key_end - key_begin, 0);   // (an empty split issues no loads)
    auto rsrc = [&](const void* plane, int rb) {
        return __builtin_amdgcn_make_buffer_rsrc(
            (void*)((const uint8_t*)plane + (kv_base + key_begin) * rb), (short)0, nk * rb, kBufWord3);
    };
    const __amdgpu_buffer_rsrc_t r_ks = rsrc(a.kb.signs, SB), r_vs = rsrc(a.vb.signs, SB);
    const __amdgpu_buffer_rsrc_t r_ksc = rsrc(a.kb.scales, 2), r_vsc = rsrc(a.vb.scales, 2);
    const __amdgpu_buffer_rsrc_t r_kc = rsrc(a.kr.codes, CB), r_vc = rsrc(a.vr.codes, CB);
    const __amdgpu_buffer_rsrc_t r_krs = rsrc(a.kr.scales, 2), r_vrs = rsrc(a.vr.scales, 2);
    // adaptive: stored popcounts of this group, one pack of G per key
    using Pack = bc::PcPack<bc::PcT<D>, G>;
    constexpr int kPack = (int)sizeof(Pack);
    static_assert(kPack <= 16, "one load per pack");
    const __amdgpu_buffer_rsrc_t r_pc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const Pack*)a.pcs + (int64_t)bhq0 / G * bc::pcs_stride(a.S) + key_begin), (short)0, nk * kPack, kBufWord3);
    // an offset past every range (the host keeps each range's bytes below
    // 2^31 - 4096): such a load returns zeros and moves no data
    constexpr int kOob = 0x7FFFF000;

    // ---------------- loads of one tile: K side into registers, V side to LDS
    auto load_k = [&](KRegs<D>& r, int t0) {
        const int tr = t0 - key_begin;      // tile offset in the range (keys)
        const int kk = tr + kown;
        if constexpr (MODE == MODE_ADAPTIVE) {
            // popcounts and the two binary scales; residual data is gathered
            // once the tile's selection is known
            if constexpr (kPack == 1) {
                r.pcw[0] = __builtin_amdgcn_raw_buffer_load_b8(r_pc, kk, 0, 0);
            } else if constexpr (kPack == 2) {
                r.pcw[0] = __builtin_amdgcn_raw_buffer_load_b16(r_pc, kk * 2, 0, 0);
            } else if constexpr (kPack == 4) {
                r.pcw[0] = __builtin_amdgcn_raw_buffer_load_b32(r_pc, kk * 4, 0, 0);
            } else if constexpr (kPack == 8) {
                const v2u_t v = __builtin_amdgcn_raw_buffer_load_b64(r_pc, kk * 8, 0, 0);
                r.pcw[0] = v[0]; r.pcw[1] = v[1];
            } else {
                const v4u_t v = __builtin_amdgcn_raw_buffer_load_b128(r_pc, kk * 16, 0, 0);
                r.pcw[0] = v[0]; r.pcw[1] = v[1]; r.pcw[2] = v[2]; r.pcw[3] = v[3];
            }
            r.sk = __builtin_amdgcn_raw_buffer_load_b16(r_ksc, kk * 2, 0, 0);
            r.svv = __builtin_amdgcn_raw_buffer_load_b16(r_vsc, kk * 2, 0, 0);
            r.rsk = 0;
            r.rsv = 0;
            return;
        }
        r.ks = buf_signs<D, BC_NT_AUX>(r_ks, kk * SB);
        r.sk = __builtin_amdgcn_raw_buffer_load_b16(r_ksc, kk * 2, 0, BC_NT_SCALES);
        r.svv = __builtin_amdgcn_raw_buffer_load_b16(r_vsc, kk * 2, 0, BC_NT_SCALES);
        r.rsk = 0;
        r.rsv = 0;
        // residual scales and K codes of every key (adaptive mode too: the
        // selection is known only after the scores, and these loads are the
        // ones worth prefetching; V codes are gathered for selected keys)
        if constexpr (RES) {
            r.rsk = __builtin_amdgcn_raw_buffer_load_b16(r_krs, kk * 2, 0, BC_NT_SCALES);
            r.rsv = __builtin_amdgcn_raw_buffer_load_b16(r_vrs, kk * 2, 0, BC_NT_SCALES);
            if constexpr (KMF) {
                // key block kb: key 16kb + l%16, 16-byte piece l/16 + 4pc of its row
                const int base = (tr + (lane & 15)) * CB + 16 * (lane >> 4);
#pragma unroll
                for (int kb = 0; kb < 4; kb++)
#pragma unroll
                    for (int pc = 0; pc < NPC; pc++) {
                        const v4u_t c = __builtin_amdgcn_raw_buffer_load_b128(r_kc, base + 16 * kb * CB + 64 * pc, 0, BC_NT_AUX);
                        const int i = kb * NPC + pc;
                        r.kc[4 * i] = c[0]; r.kc[4 * i + 1] = c[1]; r.kc[4 * i + 2] = c[2]; r.kc[4 * i + 3] = c[3];
                    }
            } else {
                // per key: the lane's own row; linear: piece i*1024 + 16l of the tile
                const int base = LIN_K ? tr * CB + 16 * lane : kk * CB;
#pragma unroll
                for (int i = 0; i < Q; i++) {
                    const v4u_t c = __builtin_amdgcn_raw_buffer_load_b128(r_kc, base + (LIN_K ? i * 1024 : 16 * i), 0,
                                                                          LIN_K ? BC_NT_AUX : 0);
                    r.kc[4 * i] = c[0]; r.kc[4 * i + 1] = c[1]; r.kc[4 * i + 2] = c[2]; r.kc[4 * i + 3] = c[3];
                }
            }
        }
    };
    // V tile to LDS: key k's sign row at k*SB; its code row at k*CB (linear,
    // pieces swizzled as above) or piece c at c*1024 + 16k (per key)
    auto issue_v = [&](int buf, int t0) {
        const int tr = t0 - key_begin;
        uint8_t* st_codes = buf ? lds_st1[wave] : lds_st0[wave];
        uint8_t* st_signs = st_codes + WL::kCodeBytes;
        if constexpr (SB >= 16) {
#pragma unroll
            for (int c = 0; c < SB / 16; c++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(r_vs, LDS_PTR(void, st_signs + c * 1024), 16,
                                                         tr * SB + 16 * lane + c * 1024, 0, 0, BC_NT_AUX);
        } else {
            // 8-byte rows: one KiB load covers 128 rows, so lanes 32..63 repeat
            // lanes 0..31 (into bytes 512..1023)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r_vs, LDS_PTR(void, st_signs), 16,
                                                     tr * SB + 16 * (lane & 31), 0, 0, 0);
        }
        if constexpr (ALLRES) {
#pragma unroll
            for (int c = 0; c < Q; c++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    r_vc, LDS_PTR(void, st_codes + c * 1024), 16,
                    LIN_V ? tr * CB + c * 1024 + 16 * (lane ^ ((4 * c + (lane >> 4)) & (Q - 1)))
                          : (tr + lane) * CB + 16 * c, 0, 0, LIN_V ? BC_NT_AUX : 0);
        }
    };

    // The query's elements are loaded first, then the wave's first tile
    // (except in adaptive mode, whose first tile needs the selection, and in
    // the workgroup that appends a token), and the query preparation runs
    // while that tile is in flight: it waits only for the older query loads,
    // and its barriers wait for LDS traffic only.
    constexpr int NT = NW * 64;
    constexpr int NQ = (G * D + NT - 1) / NT;
    uint16_t qpre[NQ];
    {
        const uint16_t* qb = a.q + (int64_t)bhq0 * D;
#pragma unroll
        for (int j = 0; j < NQ; j++) {
            const int i = (int)threadIdx.x + NT * j;
            qpre[j] = i < G * D ? qb[i] : (uint16_t)0;
        }
    }
    const bool app_here = a.app_k != nullptr && a.app_slot >= key_begin && a.app_slot < key_end;
    int t = key_begin + wave * 64;
    const bool early = MODE != MODE_ADAPTIVE && !app_here && t < key_end;
    KRegs<D> ka, kb;
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (MODE != MODE_ADAPTIVE) {
        // without a first tile to fetch, the same loads address keys past the
        // range (a split holds fewer than 2^23 keys): zeros, no traffic, and
        // the same instructions on every path, so that the preparation's
        // wait for the query counts them exactly
        const int t_first = early ? t : key_begin + (1 << 23) + 1024;
        load_k(ka, t_first);
        issue_v(0, t_first);
    }
    __builtin_amdgcn_sched_barrier(0);
    prep_digits<D, G, KMF, RES, NT>(qpre, qd, qf);

    // In-place append: the workgroup whose key range holds the new token's slot
    // encodes the token's K and V vectors into the cache first (wave 0, lane
    // groups 0 and 1, online-encode semantics: the residual against the fp32
    // mean).  Its stores complete before the barrier, so its own tile loads see
    // them; no other workgroup reads the slot's cache lines (key ranges are
    // whole 64-key tiles, and the host appends only with one query-head group
    // per kv head), and later launches see them as after a separate encode.
    if constexpr (MODE != MODE_ADAPTIVE) {
        if (a.app_k != nullptr && a.app_slot >= key_begin && a.app_slot < key_end) {
            if (wave == 0) {
                constexpr int L = D / 8;
                const int grp = lane / L, j = lane % L;
                const bool is_v = grp == 1;
                const uint16_t* src = (is_v ? a.app_v : a.app_k) + (int64_t)bkv * D;
                const BinPlanes& bp = is_v ? a.vb : a.kb;
                const ResPlanes& rp = is_v ? a.vr : a.kr;
                // (the attention arguments hold the cache planes read-only)
                const bc::EncodeDst dst{(uint8_t*)bp.signs, (uint16_t*)bp.scales,
                                        RES ? (uint8_t*)rp.codes : nullptr, RES ? (uint16_t*)rp.scales : nullptr};
                bc::encode_row<D, RES ? bc::ENC_FUSED_FP32 : bc::ENC_BINARY>(src, j, grp < 2, dst,
                                                                            kv_base + a.app_slot);
                __builtin_amdgcn_s_waitcnt(0);
            }
            __syncthreads();
        }
    }

    // weight column owned by this lane in the MFMA B operand, and its head
    const int my_col = lj;
    // (int8 path: the sign part's columns are 4 per head, the residual
    // part's 2 per head as in the fp16 layout)
    const int my_head = I8 ? my_col >> 2 : my_col >> 1;
    const int my_rhead = my_col >> 1;
    const int bcol = my_col < 2 * G ? my_col : (my_col & 1);

    // weight columns [2 parts][2G cols][72 slots]: this lane's store slot in
    // column 0, and its B-operand read position in column bcol.  The lane
    // offsets go through an opaque copy so that every access is one constant
    // offset from a base that the compiler ties to lds_wts (accesses it cannot
    // tie to one array wait for all direct loads in flight, the prefetch too)
    uint16_t* wsl = &lds_wts[0][0] + opaque_int(wave * (WL::kWeightBytes / 2) + slot_of(kown));
    const uint16_t* wrd = &lds_wts[0][0] + opaque_int(wave * (WL::kWeightBytes / 2) + bcol * WL::kColSlots + 16 * g4);
    // int8 weight columns [4G cols][80 bytes]: this lane's digit bytes at its
    // key's slot of column 0, and its B-operand read (16 bytes of column
    // my_col; lanes of unused columns read column 0 again)
    int8_t* w8st = &lds_w8[0][0] + opaque_int(wave * (I8 ? 4 * G * kW8Stride : 16) + (I8 ? slot8_of(kown) : 0));
    const int8_t* w8rd = &lds_w8[0][0] + opaque_int(wave * (I8 ? 4 * G * kW8Stride : 16) +
                                                    (I8 ? (my_col < 4 * G ? my_col : 0) * kW8Stride + 16 * g4 : 0));
    int* rdl = lds_rd[wave];          // [64 keys][G] residual dots
    int* rdlo = lds_rdlo[wave];       // their plane-0 parts (precise tiles)

    // softmax reference per head, lowered lazily: weights p = 2^(s - m) stay
    // <= 2^kTau, and the accumulators are rescaled only when a score passes
    // m + kTau (the result does not depend on m).  The int8 path's fixed-point
    // weights give up kTau of their 22 bits to this headroom: 4 there.
    constexpr int kTauI = I8 ? 4 : 8;
    constexpr float kTau = (float)kTauI;
    float m[G], mlim[G], lsum[G], off[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -INFINITY;
        mlim[g] = -INFINITY;
        lsum[g] = 0.0f;
        off[g] = 0.0f;
    }
    f4_t cs[I8 ? 1 : NH][4];   // sign part: [block][p] rows = dims 64h + 4m + p
    v4i_t ci[I8 ? NH : 1][4];  // (int8 path) the same, per digit column
    f4_t cn[NB];      // residual part: rows = dims 16db + m
#pragma unroll
    for (int h = 0; h < (I8 ? 1 : NH); h++)
#pragma unroll
        for (int p = 0; p < 4; p++) cs[h][p] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h = 0; h < (I8 ? NH : 1); h++)
#pragma unroll
        for (int p = 0; p < 4; p++) ci[h][p] = v4i_t{0, 0, 0, 0};
#pragma unroll
    for (int d = 0; d < NB; d++) cn[d] = f4_t{0.f, 0.f, 0.f, 0.f};

    // (int8 path) a head's digit columns 4g + 0..2 are one lane quad; its
    // first lane owns the head's rows in the bank.  flush8: bank = (bank +
    // d0 + 256 d1 + 65536 d2) * f per element, the integer sums restart at 0
    const bool owner8 = I8 && my_col < 4 * G && (my_col & 3) == 0;
    float* bank = &lds_bank[0][0] + opaque_int(wave * (I8 ? G * D : 4) + (I8 ? (my_col >> 2) * D : 0));
    bool banked = false;   // (wave-uniform) the bank holds values
    bool live8 = false;    // (wave-uniform) the integer sums hold values
    auto flush8 = [&](float f) {
#pragma unroll
        for (int h = 0; h < NH; h++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float t[4];
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    const float v0 = (float)ci[h][p][i];
                    t[p] = v0 + 256.0f * dpp_f<0x39>(v0) + 65536.0f * dpp_f<0x4E>(v0);
                    ci[h][p][i] = 0;
                }
                if (owner8) {
                    float4* bp = (float4*)&bank[64 * h + 4 * (4 * g4 + i)];
                    float4 b = banked ? *bp : make_float4(0.f, 0.f, 0.f, 0.f);
                    *bp = make_float4((b.x + t[0]) * f, (b.y + t[1]) * f, (b.z + t[2]) * f, (b.w + t[3]) * f);
                }
            }
        banked = true;
    };

    // weights enter the MFMAs as w * 2^wexp (fp16 hi + lo), wexp chosen so the
    // largest possible weight sits near 2^14 (int8 path: integers up to 2^22):
    // no overflow, and weights down to ~2^-30 of the largest keep their
    // contribution (fp16; undone exactly in the epilogue)
    constexpr int kWTop = I8 ? 22 : 14;
    int wexp = 0;
    bool have_wexp = false;
    float wlim = 0.0f;

    uint32_t thresh[G];
    int cutoff[G];
    float thr_floor[G], thr_value[G];   // the threshold as float bounds
    if constexpr (MODE == MODE_ADAPTIVE) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            thresh[g] = a.thresh[bhq0 + g];
            cutoff[g] = a.cutoff[bhq0 + g];
            thr_floor[g] = key_floor(thresh[g]);
            thr_value[g] = key_value(thresh[g]);
        }
    }
    // mixed mode: which heads of the group add their residual
    bool hmode[G];
#pragma unroll
    for (int g = 0; g < G; g++) hmode[g] = true;
    if constexpr (MODE == MODE_MIXED) {
#pragma unroll
        for (int g = 0; g < G; g++) hmode[g] = a.head_mode[bhq0 + g] != 0;
    }

    // query digits of a single head in scalar registers for the whole loop
    // (uniform operands of v_dot8) when codes are read per key, and the int8
    // MFMA B operands of the K residual dot (loop invariant)
    int sdig[(G == 1 && RES && !LIN_K) ? CW : 1][4];
    v4i_t bq[KMF ? NPC : 1][2];
    if constexpr (G == 1 && RES && !LIN_K) {
#pragma unroll
        for (int w = 0; w < CW; w++) {
            const int4 dg = qd.digits[0][w];
            sdig[w][0] = __builtin_amdgcn_readfirstlane(dg.x);
            sdig[w][1] = __builtin_amdgcn_readfirstlane(dg.y);
            sdig[w][2] = __builtin_amdgcn_readfirstlane(dg.z);
            sdig[w][3] = __builtin_amdgcn_readfirstlane(dg.w);
        }
    }
    if constexpr (KMF) {
#pragma unroll
        for (int pc = 0; pc < NPC; pc++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int4 w = qd.bq[pc][h][lane];
                bq[pc][h] = v4i_t{w.x, w.y, w.z, w.w};
            }
    }

    // ---------------- adaptive mode: a tile's selection, from its stored
    // popcounts and K scales, and the loads of its residual data: the residual
    // scales per key (lane = key), the K codes and V codes of the selected keys
    // at their compacted positions (K codes to registers, V codes to staging
    // buffer buf with the V signs).  Unselected keys and the positions past
    // the selected ones load from past the range (zeros, no traffic), so the
    // loads issue without branches.
    auto gather = [&](KRegs<D>& r, int t0, int buf) {
        const int s = t0 + kown;
        const bool valid = s < key_end;
        const float sk = h2f(r.sk);
        uint32_t selmask = 0;
        // selected: above the threshold, or equal to it at an index up to the
        // cutoff (ties are taken lowest index first); compared as exact float
        // scores unless a lane of the wave has a non-finite scale
        const bool fast = __ballot(!finite_scale(sk)) == 0ull;
        const float sk2 = 2.0f * sk, nd = -(float)D * sk;
#pragma unroll
        for (int g = 0; g < G; g++) {
            constexpr int bits = 8 * (int)sizeof(bc::PcT<D>);
            constexpr int per_word = 32 / bits;
            const int pc = (int)((r.pcw[g / per_word] >> (bits * (g % per_word))) & ((1u << bits) - 1u));
            bool above, tie;
            if (fast) {
                const float sc = fmaf((float)pc, sk2, nd);
                above = sc > thr_floor[g];
                tie = sc == thr_value[g];
            } else {
                const uint32_t key = ordered_key(sk * (float)(2 * pc - D));
                above = key > thresh[g];
                tie = key == thresh[g];
            }
            const bool sel = above || (tie && s <= cutoff[g]);
            selmask |= (sel && valid) ? (1u << g) : 0u;
        }
        r.sel = selmask;
        issue_v(buf, t0);
        uint8_t* st_codes = buf ? lds_st1[wave] : lds_st0[wave];
        const uint64_t selany = __ballot(selmask != 0u);
        const int nsel = __builtin_popcountll(selany);
        const int tr = t0 - key_begin;
        const bool mine = selmask != 0u;
        const int kk = tr + kown;
        // compacted positions: key s goes to position mbcnt (selected) or to
        // n + its rank among the others; key_at = the key at position lane
        const int mb = mbcnt64(selany);
        const int key_at = __builtin_amdgcn_ds_permute(4 * (mine ? mb : nsel + lane - mb), lane);
        r.rsk = __builtin_amdgcn_raw_buffer_load_b16(r_krs, mine ? kk * 2 : kOob, 0, 0);
        r.rsv = __builtin_amdgcn_raw_buffer_load_b16(r_vrs, mine ? kk * 2 : kOob, 0, 0);
        if constexpr (KMF) {
            // key block kb: position 16kb + l%16, 16-byte piece l/16 + 4pc of
            // its key's row
#pragma unroll
            for (int kb = 0; kb < 4; kb++) {
                const int j = 16 * kb + lj;
                const int key = __builtin_amdgcn_ds_bpermute(4 * j, key_at);
                const int base = j < nsel ? (tr + key) * CB + 16 * g4 : kOob;
#pragma unroll
                for (int pc = 0; pc < NPC; pc++) {
                    const v4u_t c = __builtin_amdgcn_raw_buffer_load_b128(r_kc, base + 64 * pc, 0, 0);
                    const int i = kb * NPC + pc;
                    r.kc[4 * i] = c[0]; r.kc[4 * i + 1] = c[1]; r.kc[4 * i + 2] = c[2]; r.kc[4 * i + 3] = c[3];
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < Q; i++) {
                const v4u_t c = __builtin_amdgcn_raw_buffer_load_b128(r_kc, mine ? kk * CB + 16 * i : kOob, 0, 0);
                r.kc[4 * i] = c[0]; r.kc[4 * i + 1] = c[1]; r.kc[4 * i + 2] = c[2]; r.kc[4 * i + 3] = c[3];
            }
        }
        // V codes: staging row lane holds position res_pos(lane)
        const int jv = res_pos(lane);
        const int vkey = __builtin_amdgcn_ds_bpermute(4 * jv, key_at);
#pragma unroll
        for (int c = 0; c < Q; c++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r_vc, LDS_PTR(void, st_codes + c * 1024), 16,
                                                     jv < nsel ? (tr + vkey) * CB + 16 * c : kOob, 0, 0, 0);
    };

    // ---------------- one tile: scores, online softmax, value MFMAs
    auto process = [&](const KRegs<D>& r, int t0, int buf) {
        uint8_t* st_codes = buf ? lds_st1[wave] : lds_st0[wave];
        uint8_t* st_signs = st_codes + WL::kCodeBytes;
        const int s = t0 + kown;
        const bool valid = s < key_end;
        // this tile's K registers: the younger operations are this tile's V
        // loads and the whole next-tile prefetch.  An explicit count keeps the
        // compiler from draining the queue (with direct-to-LDS loads pending it
        // would wait for zero).
        if constexpr (MODE != MODE_ADAPTIVE && PIPE) {
            constexpr int n = kVDma + kPrefetchOps;
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt((n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8));
            __builtin_amdgcn_sched_barrier(0);
        }
        const float sk = h2f(r.sk), svv = h2f(r.svv);
        float rsk = h2f(r.rsk), rsv = h2f(r.rsv);
        uint32_t kc[CW];
        if constexpr (RES) {
#pragma unroll
            for (int w = 0; w < CW; w++) kc[w] = r.kc[w];
        }

        float xd[G];
        uint32_t selmask = 0;
#pragma unroll
        for (int g = 0; g < G; g++) {
            int pc = 0;
            if constexpr (MODE == MODE_ADAPTIVE) {
                // stored by the selection passes (same popcount as below)
                constexpr int bits = 8 * (int)sizeof(bc::PcT<D>);
                constexpr int per_word = 32 / bits;
                pc = (int)((r.pcw[g / per_word] >> (bits * (g % per_word))) & ((1u << bits) - 1u));
            } else {
#pragma unroll
                for (int w = 0; w < D / 32; w++) pc += __builtin_popcount(~(qd.signs[g][w] ^ r.ks.w[w]));
            }
            const float mq = (float)(2 * pc - D);
            xd[g] = (qd.scale_q[g] * sk) * mq;  // (scale_q * scale_k) * (2pc - d)  (src/xnor_dot.cuh:30)
        }
        // adaptive: the tile's compacted residual positions (as in gather):
        // nsel selected keys, the lane's key at position rpos
        int nsel = 64, rpos = kown;
        if constexpr (MODE == MODE_ADAPTIVE) {
            selmask = r.sel;
            const uint64_t selany = __ballot(selmask != 0u);
            const int mb = mbcnt64(selany);
            nsel = __builtin_popcountll(selany);
            rpos = selmask != 0u ? mb : nsel + lane - mb;
        }
        if constexpr (MODE == MODE_ADAPTIVE) {
            if (a.selected != nullptr && valid) {
#pragma unroll
                for (int g = 0; g < G; g++)
                    a.selected[(int64_t)(bhq0 + g) * a.S + s] = (selmask >> g) & 1u;
            }
        }

        // residual dot on the raw int4 codes: sum_i q_int_i * n_i per head, in
        // units of the top-16-bit step dq (racc, exact integers; in a precise
        // tile the float bits of that plus the low digits' part / 256)
        int racc[G];
#pragma unroll
        for (int g = 0; g < G; g++) racc[g] = 0;
        // precise tile: some key's score could move by more than kPrecNats
        // from the top 16 bits alone (uniform over the wave)
        const bool prec = RES && __ballot(rsk * qd.prec_bound > kPrecNats) != 0ull;
        if constexpr (KMF) {
          // key blocks holding codes: all four, or (adaptive) the blocks of
          // the nsel compacted positions
          const int nkb = (nsel + 15) >> 4;
          if (nkb > 0) {
            // codes as int8 16*n (signed): low nibbles via x << 4, high nibbles in
            // place; each half of a piece is one 16x16x64 MFMA of (head, digit
            // plane) rows x 64 dims times 64 dims x 16 keys (columns of keys whose
            // codes were not loaded are never used)
            // Lane l holds rows 4(l/16) + i = (head 2(l/16) + i/2, plane i%2 + 1)
            // of position 16kb + l%16: both planes of a head sit in one lane, and
            // q_int dot * 16 / 256 = plane1 + 256 plane2 goes to rdl[position][head].
            // Plane 0 of a precise tile (q_int dot * 16 = 65536 plane2 +
            // 256 plane1 + plane0): groups of more than 5 heads take it from a
            // second B operand (LDS) into the same lanes and store the float
            // bits of the sum; smaller groups have it in rows 2G + g (below)
            constexpr bool LO_COLS = 3 * G <= 16;
            v4i_t acc[4];
#pragma unroll
            for (int kb = 0; kb < 4; kb++) {
                if (kb >= nkb) break;
                acc[kb] = v4i_t{0, 0, 0, 0};
                v4i_t accl = v4i_t{0, 0, 0, 0};
#pragma unroll
                for (int pc = 0; pc < NPC; pc++)
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const v4i_t av = codes_i8(kc[4 * (kb * NPC + pc) + 2 * h], kc[4 * (kb * NPC + pc) + 2 * h + 1]);
                        acc[kb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bq[pc][h], av, acc[kb], 0, 0, 0);
                        if (!LO_COLS && prec) {
                            const int4 w = qd.bq_lo[pc][h][lane];
                            accl = __builtin_amdgcn_mfma_i32_16x16x64_i8(v4i_t{w.x, w.y, w.z, w.w}, av, accl, 0, 0, 0);
                        }
                    }
                if (lane < 8 * G) {
                    int2 v = make_int2(acc[kb][0] + 256 * acc[kb][1], acc[kb][2] + 256 * acc[kb][3]);
                    if (!LO_COLS && prec)
                        v = make_int2(__builtin_bit_cast(int, (float)v.x + (float)accl[0] * (1.0f / 256.0f)),
                                      __builtin_bit_cast(int, (float)v.y + (float)accl[2] * (1.0f / 256.0f)));
                    *(int2*)&rdl[(16 * kb + lj) * G + 2 * g4] = v;
                }
            }
            if (LO_COLS && prec && g4 == G / 2) {
                // plane 0 (q_int dot * 16 = 65536 plane2 + 256 plane1 + plane0)
                // to rdlo[position][head]: rows 2G + g of the same MFMAs (lane
                // group G/2, i = g)
#pragma unroll
                for (int kb = 0; kb < 4; kb++) {
                    if (kb >= nkb) break;
#pragma unroll
                    for (int g = 0; g < (LO_COLS ? G : 1); g++) rdlo[(16 * kb + lj) * G + g] = acc[kb][g];
                }
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            // kept x16: the factor is folded into the score's scale below
            // (lanes past the written positions read values they never use)
            if constexpr (G % 4 == 0) {
#pragma unroll
                for (int g = 0; g < G; g += 4) {
                    const int4 v = *(const int4*)&rdl[rpos * G + g];
                    racc[g] = v.x; racc[g + 1] = v.y; racc[g + 2] = v.z; racc[g + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int g = 0; g < G; g++) racc[g] = rdl[rpos * G + g];
            }
            if (LO_COLS && prec) {
#pragma unroll
                for (int g = 0; g < G; g++)
                    racc[g] = __builtin_bit_cast(int, (float)racc[g] + (float)rdlo[rpos * G + g] * (1.0f / 256.0f));
            }
          }
        } else if constexpr (LIN_K) {
            // round i: this lane holds 32 dims (quarter) of key i*(64/Q) + l/Q;
            // partial dots are summed over the Q lanes of the row, and the lane
            // whose own key it is keeps the total
            int z;
            asm volatile("v_mov_b32 %0, 0" : "=v"(z));  // keeps digit reads per tile (not hoisted)
#pragma unroll
            for (int i = 0; i < Q; i++) {
#pragma unroll
                for (int g = 0; g < G; g++) {
                    int s0 = 0, s1 = 0, s2 = 0, s3 = 0;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int4 dg = qd.digits[g][4 * quarter + j + z];
                        const int x = (int)kc[4 * i + j];
                        s0 = __builtin_amdgcn_sdot8(dg.x, x, s0, false);
                        s1 = __builtin_amdgcn_sdot8(dg.y, x, s1, false);
                        s2 = __builtin_amdgcn_sdot8(dg.z, x, s2, false);
                        s3 = __builtin_amdgcn_sdot8(dg.w, x, s3, false);
                    }
                    int tot = row_group_sum<Q>(s0 + 16 * s1 + 256 * s2 + 4096 * s3);
                    if (G > 1 && prec) {
                        // digits 0..1: the dot becomes tot + lo / 256 (float bits)
                        int l0 = 0, l1 = 0;
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const int2 dl = qd.digits_lo[g][4 * quarter + j + z];
                            const int x = (int)kc[4 * i + j];
                            l0 = __builtin_amdgcn_sdot8(dl.x, x, l0, false);
                            l1 = __builtin_amdgcn_sdot8(dl.y, x, l1, false);
                        }
                        const int totl = row_group_sum<Q>(l0 + 16 * l1);
                        tot = __builtin_bit_cast(int, (float)tot + (float)totl * (1.0f / 256.0f));
                    }
                    racc[g] = quarter == i ? tot : racc[g];
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            if (G == 1 && prec) {
                // (a single head: a separate pass keeps the register peak of
                // the main loop) digits 0..1: the dot becomes racc + lo / 256
#pragma unroll
                for (int i = 0; i < Q; i++) {
#pragma unroll
                    for (int g = 0; g < G; g++) {
                        int l0 = 0, l1 = 0;
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const int2 dl = qd.digits_lo[g][4 * quarter + j + z];
                            const int x = (int)kc[4 * i + j];
                            l0 = __builtin_amdgcn_sdot8(dl.x, x, l0, false);
                            l1 = __builtin_amdgcn_sdot8(dl.y, x, l1, false);
                        }
                        const int totl = row_group_sum<Q>(l0 + 16 * l1);
                        if (quarter == i)
                            racc[g] = __builtin_bit_cast(int, (float)racc[g] + (float)totl * (1.0f / 256.0f));
                    }
                }
            }
        } else if constexpr (G == 1 && RES && !LIN_K) {
            {
                int s0 = 0, s1 = 0, s2 = 0, s3 = 0;
#pragma unroll
                for (int w = 0; w < CW; w++) {
                    s0 = __builtin_amdgcn_sdot8(sdig[w][0], (int)kc[w], s0, false);
                    s1 = __builtin_amdgcn_sdot8(sdig[w][1], (int)kc[w], s1, false);
                    s2 = __builtin_amdgcn_sdot8(sdig[w][2], (int)kc[w], s2, false);
                    s3 = __builtin_amdgcn_sdot8(sdig[w][3], (int)kc[w], s3, false);
                }
                racc[0] = s0 + 16 * s1 + 256 * s2 + 4096 * s3;
                if (prec) {
                    int l0 = 0, l1 = 0;
#pragma unroll
                    for (int w = 0; w < CW; w++) {
                        const int2 dl = qd.digits_lo[0][w];
                        l0 = __builtin_amdgcn_sdot8(dl.x, (int)kc[w], l0, false);
                        l1 = __builtin_amdgcn_sdot8(dl.y, (int)kc[w], l1, false);
                    }
                    racc[0] = __builtin_bit_cast(int, (float)racc[0] + (float)(l0 + 16 * l1) * (1.0f / 256.0f));
                }
            }
        } else if constexpr (RES) {
            bool any_res = ALLRES;
            if constexpr (MODE == MODE_ADAPTIVE) any_res = selmask != 0u;
            if (any_res) {
                int sa[G][4];
#pragma unroll
                for (int g = 0; g < G; g++) sa[g][0] = sa[g][1] = sa[g][2] = sa[g][3] = 0;
                int z;
                asm volatile("v_mov_b32 %0, 0" : "=v"(z));
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
                if (prec) {
#pragma unroll
                    for (int g = 0; g < G; g++) {
                        int l0 = 0, l1 = 0;
#pragma unroll
                        for (int w = 0; w < CW; w++) {
                            const int2 dl = qd.digits_lo[g][w + z];
                            l0 = __builtin_amdgcn_sdot8(dl.x, (int)kc[w], l0, false);
                            l1 = __builtin_amdgcn_sdot8(dl.y, (int)kc[w], l1, false);
                        }
                        racc[g] = __builtin_bit_cast(int, (float)racc[g] + (float)(l0 + 16 * l1) * (1.0f / 256.0f));
                    }
                }
            }
        }
        float sc[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            float score = xd[g];
            bool use_res = MODE == MODE_COMP;
            if constexpr (MODE == MODE_ADAPTIVE) use_res = (selmask >> g) & 1u;
            if constexpr (MODE == MODE_MIXED) use_res = hmode[g];
            // the dot in units of dq (the matrix-core dots come x16, an exact
            // power of two; in a precise tile they are float bits already)
            const float rd = prec ? __builtin_bit_cast(float, racc[g]) : (float)racc[g];
            if (RES && use_res)
                score = score + rd * (qd.dq[g] * (rsk * (KMF ? 1.0f / 112.0f : 1.0f / 7.0f)));
            sc[g] = valid ? score * isd2 : -INFINITY;
        }

        // weight scale: weights are p * wb * 2^wexp with p <= 2^kTau, so the
        // plan holds while every wb <= wlim = 2^(kWTop - kTau - wexp); it is
        // redone (one wave max) only when a key exceeds it, and then only lowered
        float wfac = 1.0f;   // (int8 path) the factor that lowering applies
        {
            const float wb = valid ? fmaxf(2.0f * svv, rsv * (1.0f / 7.0f)) : 0.0f;
            if (__ballot(wb > wlim) != 0ull) {
                const float wmx = wave_max(wb);
                if (wmx < INFINITY) {
                    const int e = kWTop - kTauI - (int)ceilf(log2f(wmx));
                    if (have_wexp) {
                        // a larger weight than planned (e < wexp): bring the sums down
                        const float f = ldexpf(1.0f, e - wexp);
                        if constexpr (I8) {
                            wfac = f;   // applied by the flush below
                        } else {
#pragma unroll
                            for (int h = 0; h < NH; h++)
#pragma unroll
                                for (int p = 0; p < 4; p++) cs[h][p] *= f;
                        }
#pragma unroll
                        for (int d = 0; d < NB; d++) cn[d] *= f;
#pragma unroll
                        for (int g = 0; g < G; g++) off[g] *= f;
                    }
                    wexp = e;
                    have_wexp = true;
                    wlim = ldexpf(1.0f, kWTop - kTauI - wexp);
                }
            }
        }

        // online softmax; (hi, lo) fp16 weights to LDS in MFMA slot order
        float lane_alpha = 1.0f;
        float lane_ralpha = 1.0f;   // (int8 path) the residual part's head
        bool any_rescale = false;
        // the value operands of odd rows come out 16x larger (see the MFMA
        // loops below): their weights carry 1/16 so that every product is exact
        // (the residual row of a key is its compacted position's row, of the
        // parity of rpos); the int8 sign elements carry no such factor
        const float kfac = (!I8 && (kown & 1)) ? 0.0625f : 1.0f;
        const float kfac_res = (rpos & 1) ? 0.0625f : 1.0f;
        // per-key factors shared by the heads: sign weight a2 = p * fa, residual
        // weight b = p * fb, and the offset sum_s (a_s + 8 b_s) grows by p * fo
        const float fa = ldexpf(2.0f * svv * kfac, wexp);
        // (int8 path: the fp16 residual weights stay below 2^14 at 2^(wexp - 8))
        const float fb = RES ? ldexpf(rsv * (1.0f / 7.0f) * kfac_res, wexp - (kWTop - 14)) : 0.0f;
        const float fo_bin = ldexpf(svv, wexp);
        const float fo_res = RES ? ldexpf(svv + rsv * (8.0f / 7.0f), wexp) : fo_bin;
        // residual weights go to the slot of the key's residual position
        // (adaptive: compacted; unselected keys write zeros to the positions
        // past nsel, so every slot a residual MFMA reads is written)
        uint16_t* wres = wsl;
        if constexpr (MODE == MODE_ADAPTIVE)
            wres = &lds_wts[0][0] + opaque_int(wave * (WL::kWeightBytes / 2) + slot_of(res_row(rpos)));
#pragma unroll
        for (int g = 0; g < G; g++) {
            // the reference m[g] moves only when a score passes m[g] + kTau
            if (__ballot(sc[g] > mlim[g]) != 0ull) {
                const float mn = fmaxf(m[g], wave_max(sc[g]));
                const float alpha = __builtin_amdgcn_exp2f(m[g] - mn);   // 0 when m was -inf
                lsum[g] *= alpha;
                off[g] *= alpha;
                if (my_head == g) lane_alpha = alpha;
                if (I8 && my_rhead == g) lane_ralpha = alpha;
                any_rescale = true;
                m[g] = mn;
                mlim[g] = mn + kTau;
            }
            const float p = valid ? __builtin_amdgcn_exp2f(sc[g] - m[g]) : 0.0f;
            lsum[g] += p;
            const float a2 = p * fa;
            float bv = 0.0f, fo = fo_bin;
            if constexpr (MODE == MODE_COMP) {
                bv = p * fb;
                fo = fo_res;
            }
            if constexpr (MODE == MODE_MIXED) {
                bv = hmode[g] ? p * fb : 0.0f;
                fo = hmode[g] ? fo_res : fo_bin;
            }
            if constexpr (MODE == MODE_ADAPTIVE) {
                const bool selg = (selmask >> g) & 1u;
                bv = selg ? p * fb : 0.0f;
                fo = selg ? fo_res : fo_bin;
            }
            // offset removed at the end, from the unrounded weights: the (hi, lo)
            // pairs carry ~22 bits (int8 path: rounding to integers up to
            // 2^22), so the difference is a zero-mean ~2^-22 term
            off[g] = fmaf(p, fo, off[g]);
            if constexpr (I8) {
                // w = rint(a2) <= 2^22 from the low mantissa bits of
                // a2 + 1.5 * 2^23, as balanced digits d0 + 256 d1 + 65536 d2:
                // the bytes of w, of (w + 128) >> 8 and of (w + 32896) >> 16
                const uint32_t wb3 = __builtin_bit_cast(uint32_t, a2 + 12582912.0f);
                int8_t* ws = w8st + 4 * g * kW8Stride;
                ws[0] = (int8_t)wb3;
                ws[kW8Stride] = (int8_t)((wb3 + 128u) >> 8);
                ws[2 * kW8Stride] = (int8_t)((wb3 - 4161408u) >> 16);   // (0x4B400000 - 0x400000 + 32896)
            } else {
                const uint16_t a2h = f2h_bits(a2);
                const uint16_t a2l = f2h_bits(a2 - h_bits2f(a2h));
                wsl[(0 * 2 * G + 2 * g) * WL::kColSlots] = a2h;
                wsl[(0 * 2 * G + 2 * g + 1) * WL::kColSlots] = a2l;
            }
            if constexpr (RES) {
                const uint16_t bh = f2h_bits(bv);
                const uint16_t bl = f2h_bits(bv - h_bits2f(bh));
                wres[(1 * 2 * G + 2 * g) * WL::kColSlots] = bh;
                wres[(1 * 2 * G + 2 * g + 1) * WL::kColSlots] = bl;
            }
        }
        if constexpr (I8) {
            // the integer sums so far move to the float bank, scaled by this
            // tile's factors (rare: the weight plan was lowered or a score
            // passed m + kTau)
            if (live8 && (any_rescale || wfac != 1.0f)) {
                if (my_head >= G) lane_alpha = 1.0f;
                flush8(lane_alpha * wfac);
            }
            if (RES && any_rescale) {
                if (my_rhead >= G) lane_ralpha = 1.0f;
#pragma unroll
                for (int d = 0; d < NB; d++) cn[d] *= lane_ralpha;
            }
        } else if (any_rescale) {
            if (my_head >= G) lane_alpha = 1.0f;
#pragma unroll
            for (int h = 0; h < NH; h++)
#pragma unroll
                for (int p = 0; p < 4; p++) cs[h][p] *= lane_alpha;
#pragma unroll
            for (int d = 0; d < NB; d++) cn[d] *= lane_alpha;
        }

        // this tile's V data must be in LDS: everything but the next tile's
        // loads (the youngest kPrefetchOps vector-memory operations) completes
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (MODE != MODE_ADAPTIVE && PIPE) {
            constexpr int n = kPrefetchOps;
            __builtin_amdgcn_s_waitcnt((n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8));
        } else if constexpr (MODE != MODE_ADAPTIVE) {
            __builtin_amdgcn_s_waitcnt(0);
        }
        // (adaptive mode: the compiler waits for this staging buffer's loads)
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the weight stores above
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");

        // B operands: (hi, lo) weight columns; lanes of unused columns read
        // columns 0/1 again (their output columns are never read back)
        h8_t bsig[2], bres[2];
        v4i_t b8 = v4i_t{0, 0, 0, 0};
        if constexpr (I8) {
            b8 = *(const v4i_t*)w8rd;
            if constexpr (RES) {
#pragma unroll
                for (int mh = 0; mh < 2; mh++) bres[mh] = *(const h8_t*)&wrd[(1 * 2 * G) * WL::kColSlots + 8 * mh];
            }
        } else {
#pragma unroll
            for (int mh = 0; mh < 2; mh++) {
                bsig[mh] = *(const h8_t*)&wrd[(0 * 2 * G) * WL::kColSlots + 8 * mh];
                if constexpr (RES) bres[mh] = *(const h8_t*)&wrd[(1 * 2 * G) * WL::kColSlots + 8 * mh];
                else bres[mh] = bsig[mh];
            }
        }

        // all transposed reads of the tile first (they retire in order while
        // the MFMAs of earlier blocks run)
        const int row_key = 16 * g4 + lj;  // this lane addresses row (key) lj of its group
        // MFMA halves that hold residual positions (adaptive: ceil(nsel / 32))
        const int nmh = (nsel + 31) >> 5;
        v2i_t wsg[NH];
#pragma unroll
        for (int h = 0; h < NH; h++)
            wsg[h] = __builtin_amdgcn_ds_read_tr4_b64_v2i32(LDS_PTR(v2i_t, st_signs + SB * row_key + 8 * h));
        v2i_t wrs[RES ? NB : 1];
        if constexpr (RES) {
            if (nmh > 0) {
#pragma unroll
                for (int db = 0; db < NB; db++) {
                    const uint8_t* rp = LIN_V ? st_codes + CB * row_key + 16 * ((db >> 1) ^ vsw) + 8 * (db & 1)
                                              : st_codes + (db >> 1) * 1024 + 16 * row_key + 8 * (db & 1);
                    wrs[db] = __builtin_amdgcn_ds_read_tr4_b64_v2i32(LDS_PTR(v2i_t, rp));
                }
            }
        }

        // sign part: rows = dims 64h + 4*lj + p
        if constexpr (I8) {
            // int8: the lane's 16 keys (first word keys 0..7, second 8..15,
            // nibble r = key r) as bytes holding bit p of their nibble in
            // place (element 2^p): even nibbles from the word, odd ones from
            // the word >> 4, one AND per four keys; all 64 keys in one MFMA
#pragma unroll
            for (int h = 0; h < NH; h++) {
                const uint32_t x = (uint32_t)wsg[h].x, y = (uint32_t)wsg[h].y;
                const uint32_t x4 = x >> 4, y4 = y >> 4;
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    const uint32_t msk = 0x01010101u << p;
                    const v4i_t av = v4i_t{(int)(x & msk), (int)(x4 & msk), (int)(y & msk), (int)(y4 & msk)};
                    ci[h][p] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b8, ci[h][p], 0, 0, 0);
                }
            }
            live8 = true;
        }
#pragma unroll
        for (int h = 0; h < (I8 ? 0 : NH); h++) {
#pragma unroll
            for (int mh = 0; mh < 2; mh++) {
                // x holds nibble r of key r (r = 0..3) and of key r + 4 (bits
                // 16 + 4r): pair word k keeps bit p of keys k and k + 4 in place,
                // an fp16 subnormal 2^(4(k&1) + p - 24); keys 2, 3 via x >> 8
                const uint32_t x = (uint32_t)(mh ? wsg[h].y : wsg[h].x);
                const uint32_t y = x >> 8;
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    uint32_t pw[4];
                    pw[0] = x & (0x00010001u << p);
                    pw[1] = x & (0x00100010u << p);
                    pw[2] = y & (0x00010001u << p);
                    pw[3] = y & (0x00100010u << p);
                    const h8_t av = __builtin_bit_cast(h8_t, pw);
                    cs[h][p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bsig[mh], cs[h][p], 0, 0, 0);
                }
            }
        }

        // residual part: rows = dims 16db + lj
        auto res_mfma = [&](int db, int mh) {
            // u = n + 8 in place: keys k, k + 4 at 4(k&1) (odd keys 16x)
            const uint32_t x = (uint32_t)(mh ? wrs[db].y : wrs[db].x) ^ 0x88888888u;
            const uint32_t y = x >> 8;
            uint32_t pw[4];
            pw[0] = x & 0x000F000Fu;
            pw[1] = x & 0x00F000F0u;
            pw[2] = y & 0x000F000Fu;
            pw[3] = y & 0x00F000F0u;
            const h8_t av = __builtin_bit_cast(h8_t, pw);
            cn[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bres[mh], cn[db], 0, 0, 0);
        };
        if constexpr (MODE == MODE_ADAPTIVE) {
            // half 0 when any key is selected, half 1 only past 32 of them
#pragma unroll
            for (int mh = 0; mh < 2; mh++) {
                if (mh >= nmh) break;
#pragma unroll
                for (int db = 0; db < NB; db++) res_mfma(db, mh);
            }
        } else if constexpr (RES) {
#pragma unroll
            for (int db = 0; db < NB; db++) {
                res_mfma(db, 0);
                res_mfma(db, 1);
            }
        }
        // the staging buffer is refilled two tiles later: its reads retire here
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
    };

    // ---------------- software-pipelined tile loop: tile i+1 loads in flight
    // while tile i computes (two register sets, two LDS staging buffers).  The
    // prefetch after a wave's last tile addresses the tile past the range: its
    // loads return zeros and move no data, and no load sits behind a branch.  Every iteration of the two-tile
    // loop starts with no load in flight: the compiler follows direct loads to
    // LDS per staging buffer only within an iteration (across the back edge it
    // would wait for all of them at the first staging-buffer read), so the
    // prefetch issued before an iteration's second tile lands by its end.
    if constexpr (MODE == MODE_ADAPTIVE) {
        // popcounts and binary scales two tiles ahead, selection and residual
        // gathers one tile ahead; each iteration (two tiles) starts with no
        // load in flight and every load has a tile of compute to land
        if (t < key_end) {
            KRegs<D> ra, rb, rc, rd;
            load_k(ra, t);
            load_k(rb, t + NW * 64);
            gather(ra, t, 0);
            __builtin_amdgcn_s_waitcnt(0);
            for (;;) {
                const int t1 = t + NW * 64;
                gather(rb, t1, 1);
                load_k(rc, t + 2 * NW * 64);
                load_k(rd, t + 3 * NW * 64);
                process(ra, t, 0);
                if (t1 >= key_end) break;
                // ra is free: it takes the popcounts and scales of tile t + 512
                // and receives that tile's residual gathers
                ra.pcw[0] = rc.pcw[0]; ra.pcw[1] = rc.pcw[1]; ra.pcw[2] = rc.pcw[2]; ra.pcw[3] = rc.pcw[3];
                ra.sk = rc.sk;
                ra.svv = rc.svv;
                gather(ra, t + 2 * NW * 64, 0);
                process(rb, t1, 1);
                t += 2 * NW * 64;
                if (t >= key_end) break;
                __builtin_amdgcn_s_waitcnt(0);
                rb.pcw[0] = rd.pcw[0]; rb.pcw[1] = rd.pcw[1]; rb.pcw[2] = rd.pcw[2]; rb.pcw[3] = rd.pcw[3];
                rb.sk = rd.sk;
                rb.svv = rd.svv;
            }
            __builtin_amdgcn_s_waitcnt(0);
            __builtin_amdgcn_wave_barrier();
        }
    } else if (!PIPE) {
        bool issued = early;   // (the first tile's loads went out before the preparation)
        for (; t < key_end; t += NW * 64) {
            if (!issued) {
                load_k(ka, t);
                issue_v(0, t);
            }
            issued = false;
            process(ka, t, 0);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_wave_barrier();
    } else if (t < key_end) {
        if (!early) {
            load_k(ka, t);
            issue_v(0, t);
        }
        __builtin_amdgcn_s_waitcnt(0);
        for (;;) {
            int tp = t + NW * 64;
            load_k(kb, tp);
            issue_v(1, tp);
            process(ka, t, 0);
            t += NW * 64;
            if (t >= key_end) break;
            tp = t + NW * 64;
            load_k(ka, tp);
            issue_v(0, tp);
            process(kb, t, 1);
            t += NW * 64;
            if (t >= key_end) break;
            __builtin_amdgcn_s_waitcnt(0);
        }
        // the last prefetch still writes LDS that the epilogue reuses
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_wave_barrier();
    }

    // ---------------- epilogue: per wave, per head: acc[e] = ((cs + cn) * unit - off) * 2^-wexp,
    // then the four waves' partials are merged.  Heads pass through staging
    // buffer 0 kEpiHeads at a time ([parts][kEpiHeads][D] floats per wave).
    constexpr int HP = WL::kEpiHeads;
    const float two24 = 16777216.0f;
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float l_w = wave_sum(lsum[g]);
        const float o_w = wave_sum(off[g]);
        if (lane == 0) {
            wm[wave][g] = m[g];
            wlsum[wave][g] = l_w;
            wofs[wave][g] = o_w;
        }
    }
    if (lane == 0) wsc[wave] = ldexpf(1.0f, -wexp);
    // per head: the maximum M over the waves, each wave's factor
    // 2^(m_w - M) * 2^-wexp_w (0 for a wave without keys) and the total l
    // (published by the first barrier of the head batches below)
    __shared__ float mfac[NW][G], hsum[2][G];
    __syncthreads();
    if (threadIdx.x < G) {
        const int g = threadIdx.x;
        float M = -INFINITY;
        for (int w = 0; w < NW; w++) M = fmaxf(M, wm[w][g]);
        float lv = 0.0f;
        for (int w = 0; w < NW; w++) {
            const bool live = M != -INFINITY && wm[w][g] != -INFINITY;
            const float f = live ? exp2f(wm[w][g] - M) : 0.0f;
            mfac[w][g] = f * wsc[w];
            if (live) lv += f * wlsum[w][g];
        }
        hsum[0][g] = M;
        hsum[1][g] = lv;
    }
    float* accw = (float*)lds_st0[wave];
    // hi + lo columns are adjacent lanes (col 2g, 2g+1); the even lane writes.
    // int8 path: the digit columns 4g + 0..2 of a head are one lane quad; its
    // first lane writes
    const bool writer = I8 ? (my_col < 4 * G && (my_col & 3) == 0) : (my_col < 2 * G && (my_col & 1) == 0);
    // the sign part's unit: 2^-24 (fp16 subnormal elements) or 1 (int8)
    const float sunit = I8 ? 1.0f : two24;
    for (int g0 = 0; g0 < G; g0 += HP) {
        const int hs = my_head - g0;   // this lane's head slot in the batch
        const bool wr = writer && hs >= 0 && hs < HP;
        // the residual part's writer (fp16 column layout in both paths)
        const int rhs = my_rhead - g0;
        const bool rwr = my_col < 2 * G && (my_col & 1) == 0 && rhs >= 0 && rhs < HP;
        if (g0 > 0) __syncthreads();   // the previous batch has been read
        // hi + lo: the neighbour lane's column by DPP (quad_perm [1,0,3,2]),
        // all sums first, then the stores under one branch
        float sv[I8 ? 1 : NH][4][4];
        float nv[RES ? NB : 1][4];
        if constexpr (I8) {
            // digits d0 + 256 d1 + 65536 d2 from lanes +0, +1, +2 of the quad
            // (quad_perm [1,2,3,0] and [2,3,0,1]); one 64-dim block at a time
            // (accumulator p carries 2^p: bit p read in place)
#pragma unroll
            for (int h = 0; h < NH; h++) {
#pragma unroll
                for (int p = 0; p < 4; p++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float v0 = (float)ci[h][p][i];
                        sv[0][p][i] = v0 + 256.0f * dpp_f<0x39>(v0) + 65536.0f * dpp_f<0x4E>(v0);
                    }
                if (wr) {
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        // plus the banked sums of the keys before the last rescale
                        float4 b = make_float4(0.f, 0.f, 0.f, 0.f);
                        if (banked) b = *(const float4*)&bank[64 * h + 4 * (4 * g4 + i)];
                        const float bb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                        for (int p = 0; p < 4; p++)
                            accw[(0 * HP + hs) * D + 64 * h + 4 * (4 * g4 + i) + p] =
                                (sv[0][p][i] + bb[p]) * (1.0f / (float)(1 << p));
                    }
                }
            }
        } else {
#pragma unroll
            for (int h = 0; h < NH; h++)
#pragma unroll
                for (int p = 0; p < 4; p++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        // accumulator p carries 2^p (bit p read in place)
                        sv[h][p][i] = (cs[h][p][i] + dpp_f<0xB1>(cs[h][p][i])) * (1.0f / (float)(1 << p));
        }
        if constexpr (RES) {
#pragma unroll
            for (int d = 0; d < NB; d++)
#pragma unroll
                for (int i = 0; i < 4; i++) nv[d][i] = cn[d][i] + dpp_f<0xB1>(cn[d][i]);
        }
        if (wr) {
#pragma unroll
            for (int h = 0; h < (I8 ? 0 : NH); h++)
#pragma unroll
                for (int p = 0; p < 4; p++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        accw[(0 * HP + hs) * D + 64 * h + 4 * (4 * g4 + i) + p] = sv[I8 ? 0 : h][p][i];
        }
        if constexpr (RES) {
            // (int8 path: the residual part's units of 2^-24, its weights
            // 2^-8 of the sign weights' scale, become the sign part's units)
            if (rwr) {
#pragma unroll
                for (int d = 0; d < NB; d++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        accw[(1 * HP + rhs) * D + 16 * d + 4 * g4 + i] = I8 ? nv[d][i] * (two24 * 256.0f) : nv[d][i];
            }
        }
        __syncthreads();
        const int nh = min(HP, G - g0);
        for (int i = threadIdx.x; i < nh * D; i += blockDim.x) {
            const int hs2 = i / D, e = i % D, g = g0 + hs2;
            float accv = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; w++) {
                const float* aw = (const float*)lds_st0[w];
                float v = aw[(0 * HP + hs2) * D + e];
                if (RES) v += aw[(1 * HP + hs2) * D + e];
                const float f = mfac[w][g];
                accv += f == 0.0f ? 0.0f : (v * sunit - wofs[w][g]) * f;
            }
            if (a.out != nullptr) {
                // one split: the output itself, normalised as the merge of a
                // single partial would (factor 1, sum l)
                const float L = hsum[1][g];
                a.out[(int64_t)(bhq0 + g) * D + e] = f2h(L > 0.0f ? accv * (1.0f / L) : 0.0f);
            } else {
                float* dst = a.ws + ((int64_t)(bhq0 + g) * a.n_splits + split) * (D + 2);
                dst[2 + e] = accv;
                if (e == 0) {
                    dst[0] = hsum[0][g];
                    dst[1] = hsum[1][g];
                }
            }
        }
    }
}

// Wide workgroups (one split per group, the output written directly): MHA
// binary attention at d = 64, 128, 256 with 8 waves; false for any other
// request.
bool launch_wide(int mode, int D, int G, const AttnArgs& a, dim3 grid, hipStream_t st, int nw) {
    if (mode != MODE_BINARY || G != 1 || nw != 8) return false;
    switch (D) {
        case 64: hipLaunchKernelGGL((attn_mfma_kernel<64, 1, MODE_BINARY, 8>), grid, dim3(8 * 64), 0, st, a); return true;
        case 128: hipLaunchKernelGGL((attn_mfma_kernel<128, 1, MODE_BINARY, 8>), grid, dim3(8 * 64), 0, st, a); return true;
        case 256: hipLaunchKernelGGL((attn_mfma_kernel<256, 1, MODE_BINARY, 8>), grid, dim3(8 * 64), 0, st, a); return true;
        default: return false;
    }
}

template <int D, int G>
void launch_dg(int mode, const AttnArgs& a, dim3 grid, hipStream_t st) {
    if (mode == MODE_BINARY)
        hipLaunchKernelGGL((attn_mfma_kernel<D, G, MODE_BINARY>), grid, dim3(256), 0, st, a);
    else if (mode == MODE_COMP)
        hipLaunchKernelGGL((attn_mfma_kernel<D, G, MODE_COMP>), grid, dim3(256), 0, st, a);
    else if (mode == MODE_MIXED)
        hipLaunchKernelGGL((attn_mfma_kernel<D, G, MODE_MIXED>), grid, dim3(256), 0, st, a);
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

template <int D, int G>
int occupancy_dg(int mode) {
    int n = 0;
    hipError_t e;
    if (mode == MODE_BINARY)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, attn_mfma_kernel<D, G, MODE_BINARY>, 256, 0);
    else if (mode == MODE_COMP)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, attn_mfma_kernel<D, G, MODE_COMP>, 256, 0);
    else if (mode == MODE_MIXED)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, attn_mfma_kernel<D, G, MODE_MIXED>, 256, 0);
    else
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, attn_mfma_kernel<D, G, MODE_ADAPTIVE>, 256, 0);
    return e == hipSuccess ? n : 0;
}

template <int D>
int occupancy_d(int mode, int G) {
    switch (G) {
        case 8: return occupancy_dg<D, 8>(mode);
        case 4: return occupancy_dg<D, 4>(mode);
        case 2: return occupancy_dg<D, 2>(mode);
        default: return occupancy_dg<D, 1>(mode);
    }
}

}  // namespace

namespace bc {

int mfma_wgs_per_cu(int mode, int D, int G) {
    static std::mutex mu;
    static std::map<std::tuple<int, int, int, int>, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    const auto key = std::make_tuple(dev, mode, D, G);
    std::lock_guard<std::mutex> lock(mu);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int n = 0;
    switch (D) {
        case 64: n = occupancy_d<64>(mode, G); break;
        case 128: n = occupancy_d<128>(mode, G); break;
        case 256: n = occupancy_d<256>(mode, G); break;
        default: n = 0;
    }
    cache[key] = n;
    return n;
}

bool mfma_split_ok(int D, int64_t chunk) {
    if (D != 64 && D != 128 && D != 256) return false;
    // buffer offsets are 32-bit and relative to a split's key range; the
    // prefetches reach up to 17 tiles (1088 keys) past its end.  The int8
    // value path adds at most 2^16 per tile to an int32 accumulator: a wave
    // takes at most 2^15 tiles (a split below 2^23 keys)
    return (chunk + 2048) * (D / 2) + 4096 < ((int64_t)1 << 31) && chunk < ((int64_t)1 << 23);
}

bool launch_mfma_split(int mode, int D, int G, const AttnArgs& a, dim3 grid, hipStream_t st, int nw) {
    if (!mfma_split_ok(D, a.chunk)) return false;
    // adaptive mode reads the popcounts stored by the selection passes
    if (mode == MODE_ADAPTIVE && a.pcs == nullptr) return false;
    if (nw != 4) return launch_wide(mode, D, G, a, grid, st, nw);
    switch (D) {
        case 64: launch_d<64>(mode, G, a, grid, st); return true;
        case 128: launch_d<128>(mode, G, a, grid, st); return true;
        case 256: launch_d<256>(mode, G, a, grid, st); return true;
        default: return false;
    }
}

}  // namespace bc
