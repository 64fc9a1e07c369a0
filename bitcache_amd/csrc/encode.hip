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

#include "common.h"
#include "encode_row.h"

namespace {
using bc::ENC_BINARY;
using bc::ENC_FUSED_FP16;
using bc::ENC_FUSED_FP32;
using bc::ENC_RESIDUAL_ONLY;
using bc::EncodeDst;
using bc::encode_row;
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
// Row-parallel encoder for d in {64, 128, 256}: L = d/8 lanes per vector, each
// lane holding 8 consecutive elements (one 16-byte load), so a wave encodes
// 64/L vectors at once with coalesced loads and stores and all reductions on
// DPP / swizzle lane moves (encode_row in encode_row.h).  Same arithmetic as
// encode_kernel.
template <int D, int MODE>
__global__ __launch_bounds__(256) void encode_rows_kernel(EncodeJob j0, EncodeJob j1) {
    static_assert(D == 64 || D == 128 || D == 256, "row encoder: d in {64, 128, 256}");
    constexpr int L = D / 8;        // lanes per vector
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
        // each wave encodes runs of kRun * VPW consecutive vectors, so that the
        // cache lines of the scale and sign planes are written whole by one
        // wave (one L2) rather than in pieces from several XCDs
        constexpr int64_t kRun = 16;
        auto base_of = [&](int64_t t) {
            return ((t / kRun) * nwaves + wave_id) * (kRun * VPW) + (t % kRun) * VPW;
        };
        // two register sets used in turn (a copy between them would wait for
        // the load in flight); the prefetch is issued unconditionally (past
        // the last iteration it reloads the current slice) so that the wait
        // before each encode leaves it in flight
        int64_t t = 0;
        int64_t base = base_of(0);
        if (base >= J.n) continue;
        bc_v4u ra = bc::load_row_slice(J.src + vec_of(base) * D, j), rb;
        for (;;) {
            int64_t nb = base_of(t + 1);
            bool more = nb < J.n;   // (wave-uniform)
            rb = bc::load_row_slice(J.src + vec_of(more ? nb : base) * D, j);
            bc::encode_row_slice<D, MODE>(ra, j, base + sub < J.n, dst, dest_for(base));
            if (!more) break;
            base = nb;
            nb = base_of(t + 2);
            more = nb < J.n;
            ra = bc::load_row_slice(J.src + vec_of(more ? nb : base) * D, j);
            bc::encode_row_slice<D, MODE>(rb, j, base + sub < J.n, dst, dest_for(base));
            if (!more) break;
            base = nb;
            t += 2;
        }
    }
}

int grid_for(int64_t nvec) {
    const int64_t want = (nvec + 3) / 4;
    const int64_t cap = (int64_t)bc::device_cu_count() * 32;
    return (int)(want < cap ? (want < 1 ? 1 : want) : cap);
}

template <int MODE>
int launch_encode(int d, const EncodeJob& a, const EncodeJob& b, hipStream_t st) {
    if (d == 64 || d == 128 || d == 256) {
        // row encoder: 64/L vectors per wave, 4 waves per block, runs of 16
        // wave iterations, grid-stride
        const int64_t vpb = 4 * (64 / (d / 8)) * 16;
        const int64_t want = (a.n + b.n + vpb - 1) / vpb;
        const int64_t cap = (int64_t)bc::device_cu_count() * 16;
        const int grid = (int)(want < cap ? (want < 1 ? 1 : want) : cap);
        if (d == 64)
            hipLaunchKernelGGL((encode_rows_kernel<64, MODE>), dim3(grid), dim3(256), 0, st, a, b);
        else if (d == 128)
            hipLaunchKernelGGL((encode_rows_kernel<128, MODE>), dim3(grid), dim3(256), 0, st, a, b);
        else
            hipLaunchKernelGGL((encode_rows_kernel<256, MODE>), dim3(grid), dim3(256), 0, st, a, b);
        return bc::check_launch("encode");
    }
    const int grid = grid_for(a.n + b.n);
    switch (d) {
#define BC_CASE(DD)                                                                       \
    case DD:                                                                              \
        hipLaunchKernelGGL((encode_kernel<DD, MODE>), dim3(grid), dim3(256), 0, st, a, b); \
        break;
        BC_CASE(32) BC_CASE(64) BC_CASE(96) BC_CASE(128) BC_CASE(160) BC_CASE(192) BC_CASE(224)
        BC_CASE(256)
#undef BC_CASE
        default:
            return bc::set_error(BC_ERR_UNSUPPORTED, "head_dim %d unsupported", d);
    }
    return bc::check_launch("encode");
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
