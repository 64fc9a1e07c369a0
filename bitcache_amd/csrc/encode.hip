// Encode kernels: fp16 vectors -> sign bits + fp16 mean-|x| scale (+ INT4 residual).
//
// One wave64 encodes one vector.  Lane l holds elements l + 64k (k < D/64),
// which makes the sign words two (or one) wave ballots and lets the scale be
// reduced in exactly the reference's fp32 order: the reference block has 128
// threads, thread t summing |x_t| + |x_{t+128}| (src/binary_encode.cu:31-41),
// followed by a shared-memory tree p[t] += p[t+s], s = 64..1 (:44-50).  Lane l
// plays threads l and l+64; the s = 64 step is an in-lane add and the s = 32..1
// steps are an xor butterfly whose lane-0 value follows the tree's association
// exactly (fp32 addition is commutative).
#include <math.h>

#include <mutex>

#include "common.h"
#include "encode_row.h"

namespace {
using bc::ENC_BINARY;
using bc::ENC_FUSED_FP16;
using bc::ENC_FUSED_FP32;
using bc::ENC_RESIDUAL_ONLY;
using bc::ENC_TRAFFIC;
using bc::EncodeDst;
using bc::quant7;

// Unsigned 32-bit division by an invariant divisor 1 <= d <= 2^31 (the
// round-up method of Granlund and Montgomery, "Division by invariant integers
// using multiplication", 1994): with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1, n / d = (mulhi(m, n) + n) >> l for every
// 32-bit n (the sum taken in 64 bits).
struct FastDiv {
    uint32_t d, m;
    int l;
};

FastDiv make_fastdiv(uint32_t d) {
    FastDiv f{d, 0u, 0};
    while ((1ull << f.l) < d) f.l++;
    f.m = (uint32_t)(((1ull << 32) * ((1ull << f.l) - d)) / d + 1ull);
    return f;
}

__device__ __forceinline__ uint32_t fast_div(uint32_t n, const FastDiv& f) {
    return (uint32_t)(((uint64_t)__umulhi(n, f.m) + n) >> f.l);
}

// Source vector v of a job is element (b, s, h) of a [rows / H, S, H] grid in
// source order, v = (b S + s) H + h, and lands in destination vector
// (b H + h) * row_stride + row_offset + s.  [rows, seq, d] sources are H = 1
// (rows of S consecutive positions), [batch, seq, heads, d] sources H = heads,
// one token per row S = 1.
struct EncodeJob {
    const uint16_t* src;          // [n, D] fp16
    uint8_t* sign_plane;          // destination binary planes (ENC_RESIDUAL_ONLY: source)
    uint16_t* scale_plane;
    uint8_t* code_plane;          // destination residual planes (may be null)
    uint16_t* rscale_plane;
    int64_t n;                    // vectors in this job (< 2^31)
    FastDiv H, S;
    int64_t row_stride, row_offset;
};

__device__ __forceinline__ int64_t dest_index(const EncodeJob& J, int64_t v) {
    const uint32_t u = (uint32_t)v;
    const uint32_t i = fast_div(u, J.H);          // b S + s
    const uint32_t h = u - i * J.H.d;
    const uint32_t b = fast_div(i, J.S);
    const uint32_t s = i - b * J.S.d;
    return (int64_t)(b * J.H.d + h) * J.row_stride + J.row_offset + s;
}

template <int D, int MODE>
__global__ __launch_bounds__(256) void encode_kernel(EncodeJob j0, EncodeJob j1) {
    constexpr int K = (D + 63) / 64;  // elements per lane
    const int lane = threadIdx.x & 63;
    const int64_t total = j0.n + j1.n;
    const int64_t nwaves = (int64_t)gridDim.x * (blockDim.x / 64);
    for (int64_t gv = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6); gv < total;
         gv += nwaves) {
        const bool second = gv >= j0.n;
        const EncodeJob& J = second ? j1 : j0;
        const int64_t v = second ? gv - j0.n : gv;
        const int64_t dv = dest_index(J, v);

        float x[K];
        bool active[K];
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int e = lane + 64 * k;
            active[k] = e < D;
            x[k] = active[k] ? h2f(J.src[v * D + e]) : 0.0f;
        }

        float scale_for_residual;
        uint64_t bits[K];
        if constexpr (MODE == ENC_RESIDUAL_ONLY) {
            const uint32_t* sp = (const uint32_t*)(J.sign_plane + dv * (D / 8));
#pragma unroll
            for (int k = 0; k < K; k++) {
                const uint64_t lo = sp[2 * k];
                const uint64_t hi = (2 * k + 1 < D / 32) ? sp[2 * k + 1] : 0u;
                bits[k] = lo | (hi << 32);
            }
            scale_for_residual = h2f(J.scale_plane[dv]);
        } else {
#pragma unroll
            for (int k = 0; k < K; k++) {
                // x >= 0.0f: +-0 -> 1, NaN -> 0 (src/binary_encode.cu:36)
                bits[k] = __ballot(active[k] && x[k] >= 0.0f);
            }
            // tree-order abs sum (see file comment).  Lane l is thread l (elements
            // l, l+128) and thread l+64 (elements l+64, l+192); absent elements
            // are 0 and adding them is exact.
            float pA = 0.0f + fabsf(x[0]);
            if constexpr (K > 2) pA = pA + fabsf(x[2]);
            float pB = 0.0f;
            if constexpr (K > 1) pB = pB + fabsf(x[1]);
            if constexpr (K > 3) pB = pB + fabsf(x[3]);
            float p = pA + pB;
#pragma unroll
            for (int s = 32; s > 0; s >>= 1) p = p + __shfl_xor(p, s, 64);
            const float total_abs =
                __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, p)));
            const float mean = total_abs / (float)D;
            if (lane == 0) J.scale_plane[dv] = f2h(mean);
            // sign words: D/32 little-endian uint32 words per vector
            uint32_t* sp = (uint32_t*)(J.sign_plane + dv * (D / 8));
            if (lane < D / 32) {
                uint64_t w = bits[0];
#pragma unroll
                for (int k = 1; k < K; k++) w = ((lane >> 1) == k) ? bits[k] : w;
                sp[lane] = (lane & 1) ? (uint32_t)(w >> 32) : (uint32_t)w;
            }
            if constexpr (MODE == ENC_FUSED_FP16) scale_for_residual = h2f(f2h(mean));
            else scale_for_residual = mean;
        }

        if constexpr (MODE != ENC_BINARY) {
            if (J.code_plane == nullptr) continue;
            const float s = scale_for_residual;
            float r[K];
            float m = 0.0f;
#pragma unroll
            for (int k = 0; k < K; k++) {
                const bool b = (bits[k] >> lane) & 1ull;
                r[k] = x[k] - (b ? s : -s);
                if (active[k]) m = fmaxf(m, fabsf(r[k]));
            }
            // fmaxf ignores NaN and is order independent: a butterfly gives the
            // reference's absmax (src/residual.cu:30-53) in every lane.
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
            const float absmax = m;
            const float inv = absmax > 0.0f ? 7.0f / absmax : 0.0f;
            if (lane == 0) J.rscale_plane[dv] = f2h(absmax);
            uint8_t* cp = J.code_plane + dv * (D / 2);
#pragma unroll
            for (int k = 0; k < K; k++) {
                // element e = lane + 64k; element 2j -> low nibble of byte j
                uint32_t c = (uint32_t)quant7(r[k] * inv) & 0xFu;
                uint32_t byte = c | (__shfl_xor(c, 1, 64) << 4);          // valid on even lanes
                uint32_t half = byte | (__shfl_xor(byte, 2, 64) << 8);     // lanes % 4 == 0
                uint32_t word = half | (__shfl_xor(half, 4, 64) << 16);    // lanes % 8 == 0
                const int e = lane + 64 * k;
                if ((lane & 7) == 0 && e < D) ((uint32_t*)cp)[e >> 3] = word;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Two-slice row encoder for d in {64, 128, 256}: P = d/16 lanes per vector,
// lane j (0 <= j < P) of its group holding slice A = elements 8j..8j+7 and
// slice B = elements d/2 + 8j..d/2 + 8j + 7 (two 16-byte loads).  The
// reference's first reduction level pairs t with t + d/2 (for d = 256 the
// per-thread |x_t| + |x_{t+128}| of src/binary_encode.cu:31-41, for d = 128
// the s = 64 step of :44-50, for d = 64 the s = 32 step after an s = 64 step
// that adds +0.0), so it is one in-lane add per element pair with no lane
// idle; the levels s = d/4 .. 8 pair lane j with lane j + s/8 (DPP row_shl)
// and s = 4, 2, 1 are in-lane, the reference tree's association exactly.
// Half as many lanes per vector as a one-slice layout halves the per-vector
// work (lane reductions, the division, the stores) per element.
//
// Quantisation fast path: when every x of the wave's vectors is finite (the
// abs sum is finite exactly then: |x| <= 65504 and d <= 256) and 7 / absmax
// is finite, |y| = |r * inv| <= 7 (1 + 2^-24)^2 < 7.5 because |r| <= absmax,
// so the clamp to [-7, 7] of src/residual.cu:67-72 never applies and
// __float2int_rn(y) is y + 12582920.0f rounded to an integer (ulp 1 there;
// 12582920 = 1.5 * 2^23 + 8 is even, so ties go to even as in rint): the
// low byte of its bits is rint(y) + 8 in [1, 15] with a clear high nibble,
// and nibble pairs are (c1 << 4) | c0 in the low byte, gathered with byte
// permutes; xor 0x8 per nibble turns the offset code into two's complement.
// Any other wave takes quant7 per element.
//
// |a| + |b| and x - (+-s) take the fp16 elements straight into v_fma_mix
// (fma(a, 1, b) is the single-rounded sum, equal to the fp32 add of the
// exactly converted halves); `one` is an fp16 1.0 the compiler cannot fold,
// so it keeps the fma rather than rewriting it to convert + add.
template <int D, int MODE>
__device__ __forceinline__ void encode_two_slices(const bc_v4u ra, const bc_v4u rb, int j, bool live,
                                                  const EncodeDst& dst, int64_t dv, _Float16 one) {
    static_assert(D == 64 || D == 128 || D == 256, "two-slice encoder: d in {64, 128, 256}");
    constexpr int P = D / 16;
    if constexpr (MODE == ENC_TRAFFIC) {
        // the fused encoder's loads and stores with no arithmetic
        const uint32_t x = ra[0] ^ rb[1], y = ra[1] ^ rb[0];
        if (live) {
            uint8_t* srow = dst.sign_plane + dv * (D / 8);
            if ((j & 3) == 0) {
                ((uint32_t*)srow)[j >> 2] = x;
                ((uint32_t*)(srow + P))[j >> 2] = y;
            }
            uint32_t* crow = (uint32_t*)(dst.code_plane + dv * (D / 2));
            crow[j] = ra[2] ^ rb[3];
            crow[P + j] = ra[3] ^ rb[2];
            if (j == 0) {
                dst.scale_plane[dv] = (uint16_t)x;
                dst.rscale_plane[dv] = (uint16_t)y;
            }
        }
        return;
    }
    // swizzle (and-mask mode) that broadcasts lane 0 of each P-lane group
    constexpr int BCAST = P == 4 ? 0x1C : (P == 8 ? 0x18 : 0x10);
    _Float16 xa[8], xb[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        xa[k] = __builtin_bit_cast(_Float16, (uint16_t)(ra[k >> 1] >> (16 * (k & 1))));
        xb[k] = __builtin_bit_cast(_Float16, (uint16_t)(rb[k >> 1] >> (16 * (k & 1))));
    }
    const float onef = (float)one;
    bool pa[8], pb[8];      // x >= 0: +-0 -> 1, NaN -> 0 (src/binary_encode.cu:36)
    uint32_t byte_a = 0, byte_b = 0;
    float s;
    float total_abs = 0.0f;
    if constexpr (MODE == ENC_RESIDUAL_ONLY) {
        const uint8_t* sp = dst.sign_plane + dv * (D / 8);
        byte_a = sp[j];
        byte_b = sp[P + j];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            pa[k] = (byte_a >> k) & 1u;
            pb[k] = (byte_b >> k) & 1u;
        }
        s = h2f(dst.scale_plane[dv]);
    } else {
#pragma unroll
        for (int k = 0; k < 8; k++) {
            pa[k] = xa[k] >= (_Float16)0.0f;
            pb[k] = xb[k] >= (_Float16)0.0f;
            byte_a |= (pa[k] ? 1u : 0u) << k;
            byte_b |= (pb[k] ? 1u : 0u) << k;
        }
        float p[8];
#pragma unroll
        for (int k = 0; k < 8; k++)
            p[k] = __builtin_fmaf((float)__builtin_fabsf16(xa[k]), onef, (float)__builtin_fabsf16(xb[k]));
        if constexpr (P == 16) {
#pragma unroll
            for (int k = 0; k < 8; k++) p[k] = p[k] + dpp_f<0x108>(p[k]);   // s = 64
        }
        if constexpr (P >= 8) {
#pragma unroll
            for (int k = 0; k < 8; k++) p[k] = p[k] + dpp_f<0x104>(p[k]);   // s = 32
        }
#pragma unroll
        for (int k = 0; k < 8; k++) p[k] = p[k] + dpp_f<0x102>(p[k]);       // s = 16
#pragma unroll
        for (int k = 0; k < 8; k++) p[k] = p[k] + dpp_f<0x101>(p[k]);       // s = 8
#pragma unroll
        for (int k = 0; k < 4; k++) p[k] = p[k] + p[k + 4];                  // s = 4
        p[0] = p[0] + p[2];
        p[1] = p[1] + p[3];                                                   // s = 2
        p[0] = p[0] + p[1];                                                   // s = 1
        total_abs = swz_f<BCAST>(p[0]);
        const float mean = total_abs / (float)D;
        if constexpr (MODE == ENC_FUSED_FP16) s = h2f(f2h(mean));
        else s = mean;
        // sign bytes: A of lanes j..j+3 -> row dword j/4, B -> dword P/4 + j/4
        const uint32_t v = byte_a | (byte_b << 16);
        const uint32_t u = v | (dpp_u<0x101>(v) << 8);      // A, B bytes of lanes j, j+1
        const uint32_t w = dpp_u<0x102>(u);                  // the same for lanes j+2, j+3
        if (live) {
            uint8_t* srow = dst.sign_plane + dv * (D / 8);
            if ((j & 3) == 0) {
                ((uint32_t*)srow)[j >> 2] = __builtin_amdgcn_perm(w, u, 0x05040100u);
                ((uint32_t*)(srow + P))[j >> 2] = __builtin_amdgcn_perm(w, u, 0x07060302u);
            }
            if (j == 0) dst.scale_plane[dv] = f2h(mean);
        }
    }

    if constexpr (MODE != ENC_BINARY) {
        if (dst.code_plane == nullptr) return;
        float r_a[8], r_b[8];
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            r_a[k] = __builtin_fmaf((float)xa[k], onef, pa[k] ? -s : s);
            r_b[k] = __builtin_fmaf((float)xb[k], onef, pb[k] ? -s : s);
            m = fmaxf(m, fabsf(r_a[k]));
            m = fmaxf(m, fabsf(r_b[k]));
        }
        // fmaxf ignores NaN and is order independent (src/residual.cu:30-53);
        // m is a non-negative float, never NaN, and for those the integer
        // order of the bits is the float order: lanes merge with integer max
        uint32_t mb = __builtin_bit_cast(uint32_t, m);
        if constexpr (P == 4) {
            mb = max(mb, dpp_u<0xB1>(mb));    // quad 1,0,3,2
            mb = max(mb, dpp_u<0x4E>(mb));    // quad 2,3,0,1
        } else if constexpr (P == 8) {
            mb = max(mb, dpp_u<0x141>(mb));   // half mirror
            mb = max(mb, dpp_u<0x4E>(mb));
            mb = max(mb, dpp_u<0xB1>(mb));
        } else {
            mb = max(mb, dpp_u<0x128>(mb));   // row rotations
            mb = max(mb, dpp_u<0x124>(mb));
            mb = max(mb, dpp_u<0x122>(mb));
            mb = max(mb, dpp_u<0x121>(mb));
        }
        const float absmax = __builtin_bit_cast(float, mb);
        const float inv = absmax > 0.0f ? 7.0f / absmax : 0.0f;
        float y_a[8], y_b[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            y_a[k] = r_a[k] * inv;
            y_b[k] = r_b[k] * inv;
        }
        bool finite;
        if constexpr (MODE == ENC_RESIDUAL_ONLY) {
            // the packed fp16 sum of the elements is finite only if each is
            typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
            h2_t hs = __builtin_bit_cast(h2_t, ra[0]);
#pragma unroll
            for (int i = 1; i < 4; i++) hs = hs + __builtin_bit_cast(h2_t, ra[i]);
#pragma unroll
            for (int i = 0; i < 4; i++) hs = hs + __builtin_bit_cast(h2_t, rb[i]);
            finite = __builtin_isfinite(hs[0]) && __builtin_isfinite(hs[1]) && __builtin_isfinite(s) &&
                     __builtin_isfinite(inv);
        } else {
            finite = __builtin_isfinite(total_abs) && __builtin_isfinite(inv);
        }
        uint32_t word_a, word_b;
        if (__ballot(!finite) == 0ull) {
            auto pack = [](const float* y) -> uint32_t {
                uint32_t c[8];
#pragma unroll
                for (int k = 0; k < 8; k++) c[k] = __builtin_bit_cast(uint32_t, y[k] + 12582920.0f);
                const uint32_t p0 = (c[1] << 4) | c[0], p1 = (c[3] << 4) | c[2];
                const uint32_t p2 = (c[5] << 4) | c[4], p3 = (c[7] << 4) | c[6];
                const uint32_t t0 = __builtin_amdgcn_perm(p1, p0, 0x0C0C0400u);   // p0.b0, p1.b0
                const uint32_t t1 = __builtin_amdgcn_perm(p3, p2, 0x0C0C0400u);   // p2.b0, p3.b0
                return __builtin_amdgcn_perm(t1, t0, 0x05040100u) ^ 0x88888888u;
            };
            word_a = pack(y_a);
            word_b = pack(y_b);
        } else {
            word_a = word_b = 0;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                word_a |= ((uint32_t)quant7(y_a[k]) & 0xFu) << (4 * k);
                word_b |= ((uint32_t)quant7(y_b[k]) & 0xFu) << (4 * k);
            }
        }
        if (live) {
            uint32_t* crow = (uint32_t*)(dst.code_plane + dv * (D / 2));
            crow[j] = word_a;
            crow[P + j] = word_b;
            if (j == 0) dst.rscale_plane[dv] = f2h(absmax);
        }
    }
}

// Row-parallel encoder for d in {64, 128, 256}: 64/P vectors per wave
// iteration (encode_two_slices), coalesced loads and stores, all reductions
// on DPP / swizzle lane moves.  Same results as encode_kernel.
template <int D, int MODE>
__global__ __launch_bounds__(256) void encode_rows_kernel(EncodeJob j0, EncodeJob j1, int lg_run) {
    static_assert(D == 64 || D == 128 || D == 256, "row encoder: d in {64, 128, 256}");
    constexpr int L = D / 16;       // lanes per vector
    constexpr int VPW = 64 / L;     // vectors per wave
    const int lane = threadIdx.x & 63;
    const int sub = lane / L, j = lane % L;
    // (readfirstlane: the wave index is uniform, so the loop below runs on
    // scalar registers and its branches are uniform)
    const int64_t wave_id = (int64_t)blockIdx.x * (blockDim.x >> 6) +
                            __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t nwaves = (int64_t)gridDim.x * (blockDim.x >> 6);
    // the next iteration's slice is loaded before this one is encoded, so
    // each wave keeps two 16-byte loads per lane in flight
#pragma unroll 1
    for (int jb = 0; jb < 2; jb++) {
        const EncodeJob& J = jb ? j1 : j0;
        // the second job starts at the other half of the waves (jobs of a
        // few runs then run side by side)
        int64_t wid = wave_id;
        if (jb) {
            wid += nwaves / 2;
            if (wid >= nwaves) wid -= nwaves;
        }
        // (jobs hold fewer than 2^31 vectors: 32-bit vector indices)
        auto vec_of = [&](int64_t b) -> int64_t {
            return (int64_t)min((uint32_t)b + (uint32_t)sub, (uint32_t)J.n - 1u);
        };
        // destination of this lane's vector b + sub: when the wave's VPW
        // vectors sit in one row (H = 1: consecutive positions) or in one
        // (batch, position) (consecutive heads), one scalar index computation
        // for the wave, else per lane
        auto dest_for = [&](int64_t b) -> int64_t {
            const uint32_t u = (uint32_t)b;
            const uint32_t i = fast_div(u, J.H);
            const uint32_t h = u - i * J.H.d;
            const uint32_t bb = fast_div(i, J.S);
            const uint32_t s = i - bb * J.S.d;
            const bool run = b + VPW <= J.n && (J.H.d == 1 ? s + VPW <= J.S.d : h + VPW <= J.H.d);
            if (run)
                return (int64_t)(bb * J.H.d + h) * J.row_stride + J.row_offset + s +
                       (int64_t)sub * (J.H.d == 1 ? 1 : J.row_stride);
            return dest_index(J, vec_of(b));
        };
        const EncodeDst dst{J.sign_plane, J.scale_plane, J.code_plane, J.rscale_plane};
        // each wave encodes runs of 2^lg_run x VPW consecutive vectors (runs
        // of 16 write the cache lines of the scale and sign planes whole from
        // one wave, i.e. one L2, rather than in pieces from several XCDs;
        // small jobs take runs of 1 to spread over the waves).  Iteration t of
        // the wave starts at ((t >> lg) nwaves + wid) VPW 2^lg + (t mod 2^lg) VPW,
        // stepped incrementally: +VPW inside a run, +jump to the next run.
        const int run = 1 << lg_run;
        const int64_t jump = (int64_t)VPW + (nwaves - 1) * ((int64_t)run * VPW);
        auto step = [&](int64_t b, int& pos) -> int64_t {
            if (++pos == run) {
                pos = 0;
                return b + jump;
            }
            return b + VPW;
        };
        // fp16 1.0 hidden from constant folding (see encode_two_slices)
        _Float16 one = (_Float16)1.0f;
        asm volatile("" : "+v"(one));
        // slices A and B of this lane's vector (nontemporal: each wave's
        // vectors are one contiguous run read once)
        auto load = [&](int64_t b, bc_v4u& a, bc_v4u& bb) {
            const bc_v4u* p = (const bc_v4u*)(J.src + vec_of(b) * D) + j;
            a = __builtin_nontemporal_load(p);
            bb = __builtin_nontemporal_load(p + D / 16);
        };
        // two register sets used in turn (a copy between them would wait for
        // the load in flight); the prefetch is issued unconditionally (past
        // the last iteration it reloads the current slices) so that the wait
        // before each encode leaves it in flight
        int64_t base = wid * ((int64_t)run * VPW);
        if (base >= J.n) continue;
        int pos = 0;   // (wave-uniform: base, pos and nb run on scalar registers)
        bc_v4u ra, rb, qa, qb;
        load(base, ra, rb);
        for (;;) {
            int64_t nb = step(base, pos);
            bool more = nb < J.n;
            load(more ? nb : base, qa, qb);
            encode_two_slices<D, MODE>(ra, rb, j, base + sub < J.n, dst, dest_for(base), one);
            if (!more) break;
            base = nb;
            nb = step(base, pos);
            more = nb < J.n;
            load(more ? nb : base, ra, rb);
            encode_two_slices<D, MODE>(qa, qb, j, base + sub < J.n, dst, dest_for(base), one);
            if (!more) break;
            base = nb;
        }
    }
}

int grid_for(int64_t nvec) {
    const int64_t want = (nvec + 3) / 4;
    const int64_t cap = (int64_t)bc::device_cu_count() * 32;
    return (int)(want < cap ? (want < 1 ? 1 : want) : cap);
}

// Blocks per CU of the row encoder: 3 (12 waves per CU) measured fastest for
// its mixed read / write stream (2: 1.27 ms, 3: 1.17 ms, 4: 1.19 ms, 16:
// 1.21 ms for 16.8M vectors of d = 128); more waves in flight add contention
// in the memory system, fewer leave the loads' latency exposed.
constexpr int kEncodeBlocksPerCU = 3;

// 256-thread blocks of `kernel` resident per CU (occupancy query, once per
// kernel; at least 1)
template <int MODE>
int resident_blocks(int d, void (*kernel)(EncodeJob, EncodeJob, int)) {
    static std::mutex mu;
    static int cached[3] = {0, 0, 0};
    const int slot = d == 64 ? 0 : (d == 128 ? 1 : 2);
    std::lock_guard<std::mutex> lock(mu);
    if (cached[slot] == 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, 256, 0) != hipSuccess || n < 1) n = 1;
        cached[slot] = n;
    }
    return cached[slot];
}

template <int MODE>
int launch_encode(int d, const EncodeJob& a, const EncodeJob& b, hipStream_t st) {
    if (d == 64 || d == 128 || d == 256) {
        // row encoder: 64/P vectors per wave, 4 waves per block, grid-stride
        // over at most kEncodeBlocksPerCU blocks per CU, all resident at once
        // (a grid of several rounds ends with a round at low occupancy)
        auto kernel = d == 64 ? encode_rows_kernel<64, MODE>
                              : (d == 128 ? encode_rows_kernel<128, MODE> : encode_rows_kernel<256, MODE>);
        const int per_cu = resident_blocks<MODE>(d, kernel);
        const int64_t cap =
            (int64_t)bc::device_cu_count() * (per_cu < kEncodeBlocksPerCU ? per_cu : kEncodeBlocksPerCU);
        // a grid of one iteration per wave if that fits, else the resident
        // blocks with runs of up to 16 iterations (at most a quarter of each
        // wave's, a power of two)
        const int64_t vpw = 64 / (d / 16);
        const int64_t one_pass = (a.n + b.n + 4 * vpw - 1) / (4 * vpw);
        const int grid = (int)(one_pass < cap ? (one_pass < 1 ? 1 : one_pass) : cap);
        const int64_t per_wave = (a.n + b.n + (int64_t)grid * 4 * vpw - 1) / ((int64_t)grid * 4 * vpw);
        int lg_run = 0;
        while (lg_run < 4 && (int64_t)(2 << lg_run) * 4 <= per_wave) lg_run++;
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), 0, st, a, b, lg_run);
        return bc::check_launch("encode");
    }
    if constexpr (MODE == ENC_TRAFFIC) {
        return bc::set_error(BC_ERR_UNSUPPORTED, "traffic probe: head_dim %d unsupported", d);
    } else {
        const int grid = grid_for(a.n + b.n);
        switch (d) {
#define BC_CASE(DD)                                                                           \
    case DD:                                                                                  \
        hipLaunchKernelGGL((encode_kernel<DD, MODE>), dim3(grid), dim3(256), 0, st, a, b);     \
        break;
            BC_CASE(32) BC_CASE(64) BC_CASE(96) BC_CASE(128) BC_CASE(160) BC_CASE(192) BC_CASE(224)
            BC_CASE(256)
#undef BC_CASE
            default:
                return bc::set_error(BC_ERR_UNSUPPORTED, "head_dim %d unsupported", d);
        }
        return bc::check_launch("encode");
    }
}

EncodeJob make_job(const void* src, void* bin, void* res, int64_t n, int64_t cap, int d,
                   int64_t heads, int64_t seq, int64_t row_stride, int64_t row_offset) {
    EncodeJob j{};
    j.src = (const uint16_t*)src;
    j.sign_plane = (uint8_t*)bin;
    j.scale_plane = (uint16_t*)((uint8_t*)bin + cap * (d / 8));
    if (res) {
        j.code_plane = (uint8_t*)res;
        j.rscale_plane = (uint16_t*)((uint8_t*)res + cap * (d / 2));
    }
    j.n = n;
    j.H = make_fastdiv((uint32_t)heads);
    j.S = make_fastdiv((uint32_t)seq);
    j.row_stride = row_stride;
    j.row_offset = row_offset;
    return j;
}

}  // namespace

extern "C" int bc_binary_encode(const void* src, void* binary_blob, int64_t n_vecs, int head_dim,
                                void* stream) {
    BC_REQUIRE(bc::head_dim_ok(head_dim), BC_ERR_UNSUPPORTED,
               "head_dim must be a multiple of 32 in [32, 256], got %d", head_dim);
    BC_REQUIRE(n_vecs >= 0, BC_ERR_INVALID_ARGUMENT, "n_vecs < 0");
    if (n_vecs == 0) return BC_OK;
    BC_REQUIRE(src && binary_blob, BC_ERR_INVALID_ARGUMENT, "null pointer");
    BC_REQUIRE(n_vecs <= INT32_MAX, BC_ERR_INVALID_ARGUMENT, "n_vecs above 2^31 - 1");
    EncodeJob a = make_job(src, binary_blob, nullptr, n_vecs, n_vecs, head_dim, 1, 1, 1, 0);
    EncodeJob b{};
    return launch_encode<ENC_BINARY>(head_dim, a, b, (hipStream_t)stream);
}

extern "C" int bc_residual_encode(const void* src, const void* binary_blob, void* residual_blob,
                                  int64_t n_vecs, int head_dim, void* stream) {
    BC_REQUIRE(bc::head_dim_ok(head_dim), BC_ERR_UNSUPPORTED,
               "head_dim must be a multiple of 32 in [32, 256], got %d", head_dim);
    BC_REQUIRE(n_vecs >= 0, BC_ERR_INVALID_ARGUMENT, "n_vecs < 0");
    if (n_vecs == 0) return BC_OK;
    BC_REQUIRE(src && binary_blob && residual_blob, BC_ERR_INVALID_ARGUMENT, "null pointer");
    BC_REQUIRE(n_vecs <= INT32_MAX, BC_ERR_INVALID_ARGUMENT, "n_vecs above 2^31 - 1");
    EncodeJob a = make_job(src, (void*)binary_blob, residual_blob, n_vecs, n_vecs, head_dim, 1, 1, 1, 0);
    EncodeJob b{};
    return launch_encode<ENC_RESIDUAL_ONLY>(head_dim, a, b, (hipStream_t)stream);
}

extern "C" int bc_encode_fused(const void* src, void* binary_blob, void* residual_blob,
                               int64_t n_vecs, int head_dim, int scale_mode, void* stream) {
    BC_REQUIRE(bc::head_dim_ok(head_dim), BC_ERR_UNSUPPORTED,
               "head_dim must be a multiple of 32 in [32, 256], got %d", head_dim);
    BC_REQUIRE(n_vecs >= 0, BC_ERR_INVALID_ARGUMENT, "n_vecs < 0");
    BC_REQUIRE(scale_mode == 0 || scale_mode == 1, BC_ERR_INVALID_ARGUMENT,
               "scale_mode must be 0 or 1");
    if (n_vecs == 0) return BC_OK;
    BC_REQUIRE(src && binary_blob, BC_ERR_INVALID_ARGUMENT, "null pointer");
    BC_REQUIRE(n_vecs <= INT32_MAX, BC_ERR_INVALID_ARGUMENT, "n_vecs above 2^31 - 1");
    EncodeJob a = make_job(src, binary_blob, residual_blob, n_vecs, n_vecs, head_dim, 1, 1, 1, 0);
    EncodeJob b{};
    if (!residual_blob) return launch_encode<ENC_BINARY>(head_dim, a, b, (hipStream_t)stream);
    if (scale_mode == 0) return launch_encode<ENC_FUSED_FP16>(head_dim, a, b, (hipStream_t)stream);
    return launch_encode<ENC_FUSED_FP32>(head_dim, a, b, (hipStream_t)stream);
}

extern "C" int bc_encode_traffic_probe(const void* src, void* binary_blob, void* residual_blob,
                                       int64_t n_vecs, int head_dim, void* stream) {
    BC_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256, BC_ERR_UNSUPPORTED,
               "traffic probe: head_dim must be 64, 128 or 256, got %d", head_dim);
    BC_REQUIRE(n_vecs >= 0, BC_ERR_INVALID_ARGUMENT, "n_vecs < 0");
    if (n_vecs == 0) return BC_OK;
    BC_REQUIRE(src && binary_blob && residual_blob, BC_ERR_INVALID_ARGUMENT, "null pointer");
    BC_REQUIRE(n_vecs <= INT32_MAX, BC_ERR_INVALID_ARGUMENT, "n_vecs above 2^31 - 1");
    EncodeJob a = make_job(src, binary_blob, residual_blob, n_vecs, n_vecs, head_dim, 1, 1, 1, 0);
    EncodeJob b{};
    return launch_encode<ENC_TRAFFIC>(head_dim, a, b, (hipStream_t)stream);
}

static int online_common(const void* k, const void* v, void* k_bin, void* k_res, void* v_bin,
                         void* v_res, int batch, int n_heads, int head_dim, int64_t current_len,
                         int max_seq, void* stream) {
    BC_REQUIRE(bc::head_dim_ok(head_dim), BC_ERR_UNSUPPORTED,
               "head_dim must be a multiple of 32 in [32, 256], got %d", head_dim);
    BC_REQUIRE(batch >= 0 && n_heads >= 0, BC_ERR_INVALID_ARGUMENT, "negative batch/n_heads");
    BC_REQUIRE(max_seq > 0, BC_ERR_INVALID_ARGUMENT, "max_seq must be > 0");
    BC_REQUIRE(current_len >= 0, BC_ERR_INVALID_ARGUMENT, "current_len must be >= 0");
    const int64_t bh = (int64_t)batch * n_heads;
    if (bh == 0) return BC_OK;
    BC_REQUIRE(k && k_bin, BC_ERR_INVALID_ARGUMENT, "null pointer");
    BC_REQUIRE(!v || v_bin, BC_ERR_INVALID_ARGUMENT, "null V cache");
    const int64_t cap = bh * max_seq;
    const int64_t slot = current_len % max_seq;  // src/online_encode.cu:139
    // binary-only caches (null residual) take the residual-free path
    const bool res = k_res != nullptr && (!v || v_res != nullptr);
    BC_REQUIRE(bh <= INT32_MAX, BC_ERR_INVALID_ARGUMENT, "batch * n_heads above 2^31 - 1");
    EncodeJob a = make_job(k, k_bin, res ? k_res : nullptr, bh, cap, head_dim, 1, 1, max_seq, slot);
    EncodeJob b{};
    if (v) b = make_job(v, v_bin, res ? v_res : nullptr, bh, cap, head_dim, 1, 1, max_seq, slot);
    if (!res && (k_res || (v && v_res))) {
        // mixed: one side has a residual cache, the other not -> two launches
        EncodeJob e{};
        EncodeJob ak = make_job(k, k_bin, k_res, bh, cap, head_dim, 1, 1, max_seq, slot);
        int st = k_res ? launch_encode<ENC_FUSED_FP32>(head_dim, ak, e, (hipStream_t)stream)
                       : launch_encode<ENC_BINARY>(head_dim, ak, e, (hipStream_t)stream);
        if (st != BC_OK || !v) return st;
        EncodeJob av = make_job(v, v_bin, v_res, bh, cap, head_dim, 1, 1, max_seq, slot);
        return v_res ? launch_encode<ENC_FUSED_FP32>(head_dim, av, e, (hipStream_t)stream)
                     : launch_encode<ENC_BINARY>(head_dim, av, e, (hipStream_t)stream);
    }
    if (res) return launch_encode<ENC_FUSED_FP32>(head_dim, a, b, (hipStream_t)stream);
    return launch_encode<ENC_BINARY>(head_dim, a, b, (hipStream_t)stream);
}

extern "C" int bc_online_encode_token(const void* kv, void* binary_cache, void* residual_cache,
                                      int batch, int n_heads, int head_dim, int64_t current_len,
                                      int max_seq, void* stream) {
    return online_common(kv, nullptr, binary_cache, residual_cache, nullptr, nullptr, batch,
                         n_heads, head_dim, current_len, max_seq, stream);
}

extern "C" int bc_online_encode_kv(const void* k, const void* v, void* k_bin, void* k_res,
                                   void* v_bin, void* v_res, int batch, int n_heads, int head_dim,
                                   int64_t current_len, int max_seq, void* stream) {
    BC_REQUIRE(v != nullptr, BC_ERR_INVALID_ARGUMENT, "null V");
    return online_common(k, v, k_bin, k_res, v_bin, v_res, batch, n_heads, head_dim, current_len,
                         max_seq, stream);
}

static int encode_into_cache(const void* src, void* binary_cache, void* residual_cache,
                             int64_t rows, int64_t heads, int seq, int head_dim, int start_pos,
                             int max_seq, int scale_mode, void* stream) {
    BC_REQUIRE(bc::head_dim_ok(head_dim), BC_ERR_UNSUPPORTED,
               "head_dim must be a multiple of 32 in [32, 256], got %d", head_dim);
    BC_REQUIRE(rows >= 0 && heads > 0 && rows % heads == 0 && seq >= 0 && start_pos >= 0 &&
                   max_seq > 0,
               BC_ERR_INVALID_ARGUMENT, "invalid dims");
    BC_REQUIRE((int64_t)start_pos + seq <= max_seq, BC_ERR_INVALID_ARGUMENT,
               "start_pos + seq (%d) exceeds max_seq (%d)", start_pos + seq, max_seq);
    BC_REQUIRE(scale_mode == 0 || scale_mode == 1, BC_ERR_INVALID_ARGUMENT,
               "scale_mode must be 0 or 1");
    if (rows * seq == 0) return BC_OK;
    BC_REQUIRE(rows * seq <= INT32_MAX, BC_ERR_INVALID_ARGUMENT, "more than 2^31 - 1 vectors");
    BC_REQUIRE(src && binary_cache, BC_ERR_INVALID_ARGUMENT, "null pointer");
    const int64_t cap = rows * max_seq;
    EncodeJob a = make_job(src, binary_cache, residual_cache, rows * seq, cap, head_dim, heads, seq,
                           max_seq, start_pos);
    EncodeJob b{};
    hipStream_t st = (hipStream_t)stream;
    if (!residual_cache) return launch_encode<ENC_BINARY>(head_dim, a, b, st);
    if (scale_mode == 0) return launch_encode<ENC_FUSED_FP16>(head_dim, a, b, st);
    return launch_encode<ENC_FUSED_FP32>(head_dim, a, b, st);
}

extern "C" int bc_encode_into_cache(const void* src, void* binary_cache, void* residual_cache,
                                    int64_t rows, int seq, int head_dim, int start_pos,
                                    int max_seq, int scale_mode, void* stream) {
    return encode_into_cache(src, binary_cache, residual_cache, rows, 1, seq, head_dim, start_pos,
                             max_seq, scale_mode, stream);
}

extern "C" int bc_encode_into_cache_bshd(const void* src, void* binary_cache, void* residual_cache,
                                         int batch, int seq, int n_heads, int head_dim,
                                         int start_pos, int max_seq, int scale_mode, void* stream) {
    BC_REQUIRE(batch >= 0 && n_heads > 0, BC_ERR_INVALID_ARGUMENT, "invalid batch / n_heads");
    return encode_into_cache(src, binary_cache, residual_cache, (int64_t)batch * n_heads, n_heads,
                             seq, head_dim, start_pos, max_seq, scale_mode, stream);
}
