// Adaptive precision: exact top-k residual selection per (b, query head).
//
// The ranking key of key s is scale_k * (2*popcount - d) (exact in fp32),
// mapped to an order-preserving uint32 (ordered_key).  The k-th largest key T
// and the tie cutoff come from four launches:
//   1. hist_kernel: the popcounts of every key from the K sign planes, stored
//      (one byte per query head and key, two for d = 256: the later launches
//      and the attention pass read them instead of the d/8-byte sign rows),
//      and per key chunk a histogram of the keys' top 13 bits (16-bit counts;
//      only its 64-word blocks holding a count are stored, with a mask of
//      them: scores fill a few binades, so most blocks are empty);
//   2. pick_kernel: per (b, head), sums the chunk histograms and picks the
//      bucket (top-13-bit digit) holding the k-th largest key; `remain` keys
//      are still to be taken from it;
//   3. collect_kernel: lists the keys of that bucket (about 1% of a head's
//      keys at k = S/10 on Gaussian data), each as one 32-bit entry holding
//      key bits 18..6 and the index in its chunk;
//   4. final_kernel: per (b, head), an exact radix select of the remain-th
//      largest listed key (T; `need` keys equal to T are taken), then the
//      need-th smallest index among the listed keys equal to T (ties are
//      taken lowest index first) as the cutoff.
// The attention kernel selects key > T, or key == T at an index <= cutoff.
//
// Why key bits 18..6 identify a listed key: with a finite fp16 scale the
// score is an exact fp32 product of an 11-bit significand and an even integer
// of magnitude <= 256 (at most 18 significant bits), so its low 6 bits are
// zero, as are those of +-inf and +0.  The ordered key therefore ends in six
// 0 bits when bit 31 is set (scores >= +0) and in six 1 bits otherwise (the
// key of a negative score is the complement; NaN ranks as -inf).  Listed keys
// share bits 31..19 (the bucket), which fixes the rest.
//
// Scores are compared as exact floats against bounds derived from the key
// prefix (see key_floor), which order like the keys; a wave holding a
// non-finite scale compares the keys themselves.
//
// Workspace: chunk histograms [B*Hq][hsplit][8192] u16 | their block masks
//   [B*Hq][hsplit] u64 | prefix [B*Hq] u32
//   | remain [B*Hq] i32 | cutoff [B*Hq] i32 | popcounts [B*Hq/G][pcs_stride(S)][G]
//   | bucket lists [B*Hq][nsplit][4 waves][wcap] u32 | list counts [B*Hq][nsplit][4] u32
//   | attention partials.
#include "attn.h"

namespace {
using bc::PcPack;
using bc::PcT;

constexpr int kBins = 2048;             // radix rounds of the final select
constexpr int kTopBits = 13;            // the first digit (bucket): key bits 31..19
constexpr int kTopShift = 32 - kTopBits;
constexpr int kTopBins = 1 << kTopBits; // counted as 16-bit halves of 32-bit words
constexpr uint32_t kTopMask = ~0u << kTopShift;
constexpr int kLowBits = kTopShift - 6; // listed key bits 18..6
constexpr int kHistThreads = 512;
constexpr int kMaxHistTiles = 1023;     // 64-key tiles per histogram chunk (counts < 2^16)
constexpr int kMaxSplit = 1024;       // key chunks per head
constexpr int kMaxChunk = 65536;      // keys per chunk (16-bit indices in the lists)
constexpr int kFinalThreads = 512;
constexpr int kStageCap = 6144;       // bucket entries the final select holds in LDS
                                      // (more: re-read from the lists each round)
static_assert(kStageCap % kFinalThreads == 0 && kFinalThreads <= kBins, "final select sizes");

struct SelArgs {
    const uint16_t* q;
    BinPlanes kb;
    int Hq, Hkv, S, kv_stride;
    int hsplit, hchunk;  // key chunks of the histogram pass (hchunk <= 64 * kMaxHistTiles)
    int nsplit, chunk;   // key chunks of the collect pass (chunk: a multiple of 64, <= kMaxChunk)
    int wcap;            // list entries per (head, chunk, wave)
    uint32_t* hist;      // [B*Hq][hsplit][kTopBins / 2] each key chunk's top-digit histogram
                         // (bin b: half b & 1 of word b >> 1); only the 64-word blocks
                         // whose bit is set in hmask are stored (the others are 0)
    uint64_t* hmask;     // [B*Hq][hsplit] bit k: block k (words 64k .. 64k + 63) holds a count
    uint32_t* prefix;    // [B*Hq] bucket digit << kTopShift, then the threshold T
    int32_t* remain;     // [B*Hq] keys still to take from the bucket, then at T
    int32_t* cutoff;     // [B*Hq]
    void* pcs;           // [B*Hq/G][pcs_stride(S)][G] popcounts (PcT<D>)
    uint32_t* lists;     // [B*Hq][nsplit][4][wcap] bucket entries
    uint32_t* counts;    // [B*Hq][nsplit][4] entries per list region
    int oct;             // K scales load eight keys at a time (kv_stride % 8 == 0,
                         // 16-byte aligned scale plane)
};

template <int D, int G>
__device__ void load_q_signs(const uint16_t* qb, uint32_t (*qs)[D / 32]) {
    for (int i = threadIdx.x; i < G * (D / 32); i += blockDim.x) {
        const int g = i / (D / 32), w = i % (D / 32);
        uint32_t bits = 0;
        for (int b = 0; b < 32; b++) bits |= (h2f(qb[g * D + 32 * w + b]) >= 0.0f ? 1u : 0u) << b;
        qs[g][w] = bits;
    }
}

template <int D>
__device__ __forceinline__ int popc_of(const uint32_t* qs, const SignWords<D>& ks) {
    int pc = 0;
#pragma unroll
    for (int w = 0; w < D / 32; w++) pc += __builtin_popcount(~(qs[w] ^ ks.w[w]));
    return pc;
}

template <int D>
__device__ __forceinline__ uint32_t key_of_pc(int pc, float sk) {
    return ordered_key(sk * (float)(2 * pc - D));
}

// Every key of a chunk: the popcounts of the G heads of the group (stored)
// and each head's histogram of the top 13 key bits, 16-bit counts two to a
// word (a chunk holds fewer than 2^16 keys), stored whole for the chunk
// (plain coalesced stores; the pick sums the chunks).
// grid: (hsplit, B*Hkv*(group/G)); block kHistThreads.
template <int D, int G>
__global__ __launch_bounds__(kHistThreads) void hist_kernel(SelArgs a) {
    __shared__ uint32_t qs[G][D / 32];
    __shared__ __attribute__((aligned(16))) uint32_t h[G][kTopBins / 2];
    const int nqg = (a.Hq / a.Hkv) / G;
    const int qg = blockIdx.y % nqg, bkv = blockIdx.y / nqg;
    const int b = bkv / a.Hkv, kvh = bkv % a.Hkv;
    const int bhq0 = b * a.Hq + kvh * (a.Hq / a.Hkv) + qg * G;
    load_q_signs<D, G>(a.q + (int64_t)bhq0 * D, qs);
    for (int i = threadIdx.x; i < G * kTopBins / 2; i += blockDim.x) (&h[0][0])[i] = 0u;
    __syncthreads();
    const int64_t base = (int64_t)bkv * a.kv_stride;
    const int k0 = blockIdx.x * a.hchunk, k1 = min(a.S, k0 + a.hchunk);
    using P = PcT<D>;
    using Pack = PcPack<P, G>;
    Pack* pcs = (Pack*)a.pcs + (int64_t)bhq0 / G * bc::pcs_stride(a.S);   // this group's packs
    auto bump = [&](int g, uint32_t key) {
        const uint32_t bin = key >> kTopShift;
        atomicAdd(&h[g][bin >> 1], 1u << ((bin & 1u) << 4));
    };
    auto count = [&](const Pack& pk, float sk) {
        // (a wave with a non-finite scale takes the key path for all its lanes)
        if (__ballot(!finite_scale(sk)) == 0ull) {
            const float sk2 = 2.0f * sk, nd = -(float)D * sk;
#pragma unroll
            for (int g = 0; g < G; g++) bump(g, ordered_bits(fmaf((float)pk.v[g], sk2, nd)));
        } else {
#pragma unroll
            for (int g = 0; g < G; g++) bump(g, key_of_pc<D>((int)pk.v[g], sk));
        }
    };
    // Two register stages of UP keys per thread: the loads of the next stage
    // are in flight while a stage is counted.
    constexpr int UP = D >= 256 ? 2 : 4;
    constexpr int step = UP * kHistThreads;
    struct Stage {
        SignWords<D> ks[UP];
        uint16_t sk[UP];
    };
    auto load = [&](Stage& st, int s) {
#pragma unroll
        for (int u = 0; u < UP; u++) {
            const int ss = s + u * kHistThreads;
            const int64_t i = base + (ss < k1 ? ss : k0);
            st.ks[u] = load_signs<D, true>(a.kb.signs + i * (D / 8));
            st.sk[u] = a.kb.scales[i];
        }
    };
    auto run = [&](const Stage& st, int s) {
#pragma unroll
        for (int u = 0; u < UP; u++) {
            const int ss = s + u * kHistThreads;
            if (ss >= k1) break;
            Pack pk;
#pragma unroll
            for (int g = 0; g < G; g++) pk.v[g] = (P)popc_of<D>(qs[g], st.ks[u]);
            pcs[ss] = pk;
            count(pk, h2f(st.sk[u]));
        }
    };
    if (k0 + (int)threadIdx.x < k1) {
        Stage sa, sb;
        int s = k0 + threadIdx.x;
        load(sa, s);
        for (;;) {
            load(sb, s + step);
            run(sa, s);
            s += step;
            if (s >= k1) break;
            load(sa, s + step);
            run(sb, s);
            s += step;
            if (s >= k1) break;
        }
    }
    __syncthreads();
    // Per head: thread t holds words 8t .. 8t + 7 (block t / 8); a block is
    // stored, as whole lines, when one of its words holds a count, and the
    // head's mask of such blocks goes with it (the pick reads only those)
    static_assert(kTopBins / 2 == 8 * kHistThreads && kTopBins / 2 / 64 == 64, "one 64-bit block mask per head");
    __shared__ uint32_t bm[G][kHistThreads / 64];   // per head and wave: its 8 blocks' bits
    const int wv = threadIdx.x >> 6, ln = threadIdx.x & 63;
#pragma unroll
    for (int g = 0; g < G; g++) {
        const bc_v4u x0 = *(const bc_v4u*)&h[g][8 * threadIdx.x];
        const bc_v4u x1 = *(const bc_v4u*)&h[g][8 * threadIdx.x + 4];
        const bool nz = (x0[0] | x0[1] | x0[2] | x0[3] | x1[0] | x1[1] | x1[2] | x1[3]) != 0u;
        const uint64_t lanes = __ballot(nz);   // lanes 8k .. 8k + 7: block 8 wv + k
        if (ln == 0) {
            uint32_t bits = 0u;
#pragma unroll
            for (int k = 0; k < 8; k++) bits |= ((lanes >> (8 * k)) & 0xFFull) != 0ull ? (1u << k) : 0u;
            bm[g][wv] = bits;
        }
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; g++) {
        const int64_t row = (int64_t)(bhq0 + g) * a.hsplit + blockIdx.x;
        const int blk = threadIdx.x >> 3;   // 0 .. 63
        if ((bm[g][blk >> 3] >> (blk & 7)) & 1u) {
            bc_v4u* dst = (bc_v4u*)(a.hist + row * (kTopBins / 2) + 8 * threadIdx.x);
            dst[0] = *(const bc_v4u*)&h[g][8 * threadIdx.x];
            dst[1] = *(const bc_v4u*)&h[g][8 * threadIdx.x + 4];
        }
        if (threadIdx.x == 0) {
            uint64_t m = 0ull;
#pragma unroll
            for (int w = 0; w < kHistThreads / 64; w++) m |= (uint64_t)bm[g][w] << (8 * w);
            a.hmask[row] = m;
        }
    }
}

// One block per (b, query head): sum the chunk histograms and pick the bucket
// (top-13-bit digit) holding the top_k-th largest key:
// prefix = digit << kTopShift, remain = top_k - (keys above the bucket).
// Thread t sums bins [kTopBins - 32 (t + 1), kTopBins - 32 t) of every chunk
// in registers, so the threads in order hold descending bin groups.
__global__ __launch_bounds__(256) void pick_kernel(SelArgs a, int top_k) {
    constexpr int kPer = kTopBins / 256;   // bins per thread
    __shared__ uint32_t part[256];
    const int bhq = blockIdx.x;
    const uint32_t* h = a.hist + (int64_t)bhq * a.hsplit * (kTopBins / 2);
    const uint64_t* hm = a.hmask + (int64_t)bhq * a.hsplit;
    const int b0 = kTopBins - kPer * ((int)threadIdx.x + 1);
    const int blk = (b0 / 2) / 64;   // this thread's 16 words lie in one 64-word block
    static_assert(kPer == 32, "16 words per thread, within one block");
    uint32_t cnt[kPer];
#pragma unroll
    for (int j = 0; j < kPer; j++) cnt[j] = 0u;
    for (int c = 0; c < a.hsplit; c++) {
        if (((hm[c] >> blk) & 1ull) == 0ull) continue;   // (a block never stored: all zero)
        const bc_v4u* src = (const bc_v4u*)(h + (int64_t)c * (kTopBins / 2) + b0 / 2);
#pragma unroll
        for (int v = 0; v < kPer / 8; v++) {
            const bc_v4u x = src[v];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                cnt[8 * v + 2 * e] += x[e] & 0xFFFFu;
                cnt[8 * v + 2 * e + 1] += x[e] >> 16;
            }
        }
    }
    uint32_t local = 0;
#pragma unroll
    for (int j = 0; j < kPer; j++) local += cnt[j];
    part[threadIdx.x] = local;
    __syncthreads();
    const int remain = top_k;
    if (remain <= 0) {
        if (threadIdx.x == 0) {
            a.prefix[bhq] = 0xFFFFFFFFu;  // nothing selected: no key exceeds it, no tie taken
            a.remain[bhq] = 0;
        }
        return;
    }
    // inclusive prefix over the 256 partial counts (Hillis-Steele in LDS)
    uint32_t incl = local;
    for (int off = 1; off < 256; off <<= 1) {
        const uint32_t add = threadIdx.x >= off ? part[threadIdx.x - off] : 0u;
        __syncthreads();
        incl += add;
        part[threadIdx.x] = incl;
        __syncthreads();
    }
    const uint32_t excl = incl - local;
    if (threadIdx.x == 255 && incl < (uint32_t)remain) {
        // fewer keys than remain: select everything
        a.prefix[bhq] = 0u;
        a.remain[bhq] = 0;
    }
    if (excl < (uint32_t)remain && incl >= (uint32_t)remain) {
        // this thread's bins hold the remain-th largest key: from its top bin down
        uint32_t above = excl;
        int digit = b0;
        bool found = false;
#pragma unroll
        for (int j = kPer - 1; j >= 0; j--) {
            if (!found) {
                if (above + cnt[j] >= (uint32_t)remain) {
                    digit = b0 + j;
                    found = true;
                } else {
                    above += cnt[j];
                }
            }
        }
        a.prefix[bhq] = (uint32_t)digit << kTopShift;
        a.remain[bhq] = remain - (int)above;
    }
}

// List regions: each (head, chunk) has one region of wcap entries per wave
// of the collecting workgroup; a wave sees at most 64 lanes x ceil(octets /
// 256) octets of its chunk (plain path: 64 x ceil(keys / 256) keys), which is
// at most 512 * ceil(chunk / 2048) keys, and never more than the chunk.
inline int list_wave_cap(int chunk) {
    const int c = 512 * ((chunk + 2047) / 2048);
    return c < chunk ? c : chunk;
}

// Orders a wave's LDS writes before its later LDS reads of other lanes' data.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The bucket lists: every key of the chunk whose top 13 bits are the picked
// bucket of a head goes into that head's list as
// (key bits 18..6) << 16 | (index - chunk start).  A wave gathers the entries
// of a row of 512 keys in its LDS area (ballot counts, no atomics), then
// appends them to its own list region with whole-wave stores, so a row costs
// one store per head instead of one per key step and head; it stores its
// region counts at the end.  Every lane of a wave runs the same trip count
// (lanes past the chunk take no key).
// OCT: the eight-key loads (SelArgs::oct); one path per instance keeps the
// loop's code within the instruction cache.
// grid: (nsplit, B*Hkv*(group/G)); block 256.
template <int D, int G, bool OCT>
__global__ __launch_bounds__(256) void collect_kernel(SelArgs a) {
    constexpr int kRow = 512;   // keys of a wave's row (64 lanes x 8)
    __shared__ uint32_t stg[4][G][kRow];
    const int nqg = (a.Hq / a.Hkv) / G;
    const int qg = blockIdx.y % nqg, bkv = blockIdx.y / nqg;
    const int b = bkv / a.Hkv, kvh = bkv % a.Hkv;
    const int bhq0 = b * a.Hq + kvh * (a.Hq / a.Hkv) + qg * G;
    const int wave = threadIdx.x >> 6;
    const int64_t base = (int64_t)bkv * a.kv_stride;
    const int k0 = blockIdx.x * a.chunk, k1 = min(a.S, k0 + a.chunk);
    using P = PcT<D>;
    using Pack = PcPack<P, G>;
    const Pack* pcs = (const Pack*)a.pcs + (int64_t)bhq0 / G * bc::pcs_stride(a.S);
    // the bucket as a key range [klo, khi] and, for scores of a finite scale,
    // as the float range (flo, fhi]
    uint32_t klo[G], khi[G];
    float flo[G], fhi[G];
    bool live[G];
    uint32_t* lst[G];
    uint32_t off[G];   // entries in the wave's list region
    uint32_t rc[G];    // entries of the current row in LDS
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int g = 0; g < G; g++) {
        const int bhq = bhq0 + g;
        live[g] = a.remain[bhq] > 0;
        klo[g] = a.prefix[bhq] & kTopMask;
        khi[g] = klo[g] | ~kTopMask;
        flo[g] = klo[g] == 0u ? -INFINITY : key_floor(klo[g] - 1u);
        fhi[g] = key_floor(khi[g]);
        lst[g] = a.lists + (((int64_t)bhq * a.nsplit + blockIdx.x) * 4 + wave) * a.wcap;
        off[g] = 0u;
        rc[g] = 0u;
    }
    // one key: the popcounts pc[g] of the G heads, the K scale, the index
    auto take = [&](const int* pc, float sk, int s, bool valid) {
        bool mt[G];
        uint32_t key[G];
        if (__ballot(valid && !finite_scale(sk)) == 0ull) {
            const float sk2 = 2.0f * sk, nd = -(float)D * sk;
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float sc = fmaf((float)pc[g], sk2, nd);
                mt[g] = valid && live[g] && sc > flo[g] && sc <= fhi[g];
                key[g] = ordered_bits(sc);
            }
        } else {
#pragma unroll
            for (int g = 0; g < G; g++) {
                key[g] = key_of_pc<D>(pc[g], sk);
                mt[g] = valid && live[g] && key[g] >= klo[g] && key[g] <= khi[g];
            }
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            const uint64_t m = __ballot(mt[g]);
            if (m != 0ull) {
                if (mt[g]) {
                    const uint32_t below =
                        __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
                    stg[wave][g][rc[g] + below] = (((key[g] >> 6) & ((1u << kLowBits) - 1u)) << 16) | (uint32_t)(s - k0);
                }
                rc[g] += (uint32_t)__builtin_popcountll(m);
            }
        }
    };
    // the row's entries from LDS to the list regions
    auto flush = [&]() {
        wave_lds_sync();
#pragma unroll
        for (int g = 0; g < G; g++) {
            for (uint32_t i = lane; i < rc[g]; i += 64) lst[g][off[g] + i] = stg[wave][g][i];
            off[g] += rc[g];
            rc[g] = 0u;
        }
        wave_lds_sync();
    };
    if constexpr (OCT) {
        // eight consecutive keys per lane and load: their packs (whole 16-byte
        // loads where they fill one) and their K scales (16 bytes); two
        // register stages of UP octets, the next stage's loads in flight
        // while a stage is taken (one copy of the stage body: the next stage
        // moves into the current one)
        constexpr int kOct = 8 * (int)sizeof(Pack);   // pack bytes of eight keys
        constexpr int NW = kOct / 4;
        constexpr int UP = kOct >= 64 ? 1 : 2;         // octets per lane and stage
        constexpr int step = UP * 256;                 // octets per block and stage
        const int o0 = k0 / 8, o1 = (k1 + 7) / 8;
        const uint16_t* scales = a.kb.scales + base;
        struct Stage {
            uint32_t pw[UP][NW];
            bc_v4u sc[UP];
        };
        auto load = [&](Stage& st, int o) {
#pragma unroll
            for (int u = 0; u < UP; u++) {
                const int oo = o + u * 256;
                const int oc = oo < o1 ? oo : o0;
                const uint32_t* src = (const uint32_t*)(pcs + 8 * oc);
                if constexpr (kOct >= 16) {
#pragma unroll
                    for (int v = 0; v < kOct / 16; v++) {
                        const bc_v4u x = ((const bc_v4u*)src)[v];
                        st.pw[u][4 * v] = x[0]; st.pw[u][4 * v + 1] = x[1];
                        st.pw[u][4 * v + 2] = x[2]; st.pw[u][4 * v + 3] = x[3];
                    }
                } else {
                    const bc_v2u x = *(const bc_v2u*)src;
                    st.pw[u][0] = x[0]; st.pw[u][1] = x[1];
                }
                st.sc[u] = *(const bc_v4u*)(scales + 8 * oc);
            }
        };
        // the fast path's bounds: a head without a bucket (live false) gets
        // an empty range
        float flo_f[G];
#pragma unroll
        for (int g = 0; g < G; g++) flo_f[g] = live[g] ? flo[g] : INFINITY;
        auto pc_of = [&](const Stage& st, int u, int j, int g) {
            constexpr int pb = (int)sizeof(P);
            const int byte = (j * G + g) * pb;
            return (st.pw[u][byte / 4] >> (8 * (byte % 4))) & ((1u << (8 * pb)) - 1u);
        };
        auto run = [&](const Stage& st, int o) {
#pragma unroll
            for (int u = 0; u < UP; u++) {
                const int oo = o + u * 256;
                float sk[8];
                bool nonfinite = false;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const uint32_t sw = st.sc[u][j >> 1];
                    sk[j] = h2f((uint16_t)((j & 1) ? (sw >> 16) : (sw & 0xFFFFu)));
                    const bool valid = oo < o1 && 8 * oo + j < k1;
                    nonfinite |= valid && !finite_scale(sk[j]);
                }
                if (__ballot(nonfinite) == 0ull) {
                    // every scale of the wave's octets is finite: exact float
                    // scores against the bucket's float range; a key past the
                    // chunk gets a NaN scale, so its compares fail
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const int s = 8 * oo + j;
                        const float skj = (oo < o1 && s < k1) ? sk[j] : __builtin_nanf("");
                        const float sk2 = 2.0f * skj, nd = -(float)D * skj;
#pragma unroll
                        for (int g = 0; g < G; g++) {
                            const float sc = fmaf((float)pc_of(st, u, j, g), sk2, nd);
                            const bool in = sc > flo_f[g] && sc <= fhi[g];
                            // the same test as the two compares' lane masks
                            // ANDed (a ballot of `in` would first copy the
                            // flag through a vector register: two more VALU
                            // instructions per key and head)
                            const uint64_t m = __builtin_amdgcn_fcmpf(sc, flo_f[g], 2 /* ordered > */) &
                                               __builtin_amdgcn_fcmpf(sc, fhi[g], 5 /* ordered <= */);
                            if (m != 0ull) {
                                if (in) {
                                    const uint32_t below = __builtin_amdgcn_mbcnt_hi(
                                        (uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
                                    stg[wave][g][rc[g] + below] =
                                        (((ordered_bits(sc) >> 6) & ((1u << kLowBits) - 1u)) << 16) | (uint32_t)(s - k0);
                                }
                                rc[g] += (uint32_t)__builtin_popcountll(m);
                            }
                        }
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const int s = 8 * oo + j;
                        int pc[G];
#pragma unroll
                        for (int g = 0; g < G; g++) pc[g] = (int)pc_of(st, u, j, g);
                        take(pc, sk[j], s, oo < o1 && s < k1);
                    }
                }
                flush();
            }
        };
        Stage cur, nxt;
        int o = o0 + threadIdx.x;      // this lane's octet of the stage
        int ow = o0 + 64 * wave;       // the wave's first octet of the stage (uniform)
        load(cur, o);
        for (;;) {
            load(nxt, o + step);
            run(cur, o);
            o += step;
            ow += step;
            if (ow >= o1) break;
            cur = nxt;
        }
    } else {
        // sixteen keys per thread per iteration
        constexpr int U = 16;
        for (int sw = k0 + 64 * wave; sw < k1; sw += U * 256) {   // the wave's first key (uniform)
            const int s = sw - 64 * wave + (int)threadIdx.x;
            Pack pk[U];
            float sk[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int ss = s + u * 256;
                const int sc = ss < k1 ? ss : k0;
                pk[u] = pcs[sc];
                sk[u] = h2f(a.kb.scales[base + sc]);
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int ss = s + u * 256;
                int pc[G];
#pragma unroll
                for (int g = 0; g < G; g++) pc[g] = (int)pk[u].v[g];
                take(pc, sk[u], ss, ss < k1);
                if (u % 8 == 7) flush();   // (a row: 8 keys per lane)
            }
        }
    }
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int g = 0; g < G; g++)
            a.counts[((int64_t)(bhq0 + g) * a.nsplit + blockIdx.x) * 4 + wave] = off[g];
    }
}

// Inclusive sum of v over the block's NT threads (wsum: LDS [NT / 64]).
template <int NT>
__device__ uint32_t block_incl_sum(uint32_t v, uint32_t* wsum) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t up = __shfl_up(v, off, 64);
        if (lane >= off) v += up;
    }
    if (lane == 63) wsum[wave] = v;
    __syncthreads();
    uint32_t base = 0;
    for (int w = 0; w < wave; w++) base += wsum[w];
    __syncthreads();   // (wsum is free again)
    return v + base;
}

// Given the histogram cnt[nb] of the elements' digits, the digit d of the
// r-th largest element (1 <= r <= total): count(digit > d) < r <=
// count(digit >= d).  Every thread gets d and count(digit > d).
template <int NT>
__device__ void block_pick(const uint32_t* cnt, int nb, uint32_t r, uint32_t* wsum, uint32_t* res, int& digit,
                           uint32_t& above) {
    const int per = (nb + NT - 1) / NT;   // consecutive bins per thread, descending
    uint32_t local = 0;
    for (int j = 0; j < per; j++) {
        const int d = nb - 1 - ((int)threadIdx.x * per + j);
        if (d >= 0) local += cnt[d];
    }
    if (threadIdx.x == 0) {
        res[0] = 0u;   // (r beyond the total: digit 0, nothing above)
        res[1] = 0u;
    }
    const uint32_t incl = block_incl_sum<NT>(local, wsum);
    const uint32_t excl = incl - local;
    if (excl < r && incl >= r) {
        uint32_t ab = excl;
        int dg = 0;
        for (int j = 0; j < per; j++) {
            const int d = nb - 1 - ((int)threadIdx.x * per + j);
            if (d < 0) break;
            if (ab + cnt[d] >= r) {
                dg = d;
                break;
            }
            ab += cnt[d];
        }
        res[0] = (uint32_t)dg;
        res[1] = ab;
    }
    __syncthreads();
    digit = (int)res[0];
    above = res[1];
    __syncthreads();   // (res is free again)
}

// One block per (b, query head): the exact threshold and tie cutoff from the
// head's bucket list.  The list regions are read in one flat index space
// (region = chunk * 4 + wave); when the bucket fits in LDS it is staged there
// once, else every round re-reads it.
__global__ __launch_bounds__(kFinalThreads) void final_kernel(SelArgs a) {
    constexpr int NT = kFinalThreads;
    __shared__ uint32_t s_k[kStageCap];        // key bits 18..6
    __shared__ uint32_t s_i[kStageCap];        // key index
    __shared__ uint32_t cnt[kBins];
    __shared__ uint32_t rpre[4 * kMaxSplit + 1];
    __shared__ uint32_t wsum[NT / 64];
    __shared__ uint32_t res[2];
    const int bhq = blockIdx.x;
    const int r0 = a.remain[bhq];
    if (r0 <= 0) {
        // k = 0, or every key taken: the prefix already says which; no ties
        if (threadIdx.x == 0) a.cutoff[bhq] = -1;
        return;
    }
    const uint32_t P0 = a.prefix[bhq];
    const int nreg = 4 * a.nsplit;
    const uint32_t* counts = a.counts + (int64_t)bhq * nreg;
    const uint32_t* lists = a.lists + (int64_t)bhq * nreg * a.wcap;
    {
        // exclusive prefix of the region counts
        constexpr int kPer = 4 * kMaxSplit / NT;
        uint32_t c[kPer];
        uint32_t local = 0;
#pragma unroll
        for (int j = 0; j < kPer; j++) {
            const int r = (int)threadIdx.x * kPer + j;
            c[j] = r < nreg ? counts[r] : 0u;
            local += c[j];
        }
        const uint32_t incl = block_incl_sum<NT>(local, wsum);
        uint32_t run = incl - local;
#pragma unroll
        for (int j = 0; j < kPer; j++) {
            const int r = (int)threadIdx.x * kPer + j;
            if (r < nreg) rpre[r] = run;
            run += c[j];
        }
        if (threadIdx.x == NT - 1) rpre[nreg] = incl;
        __syncthreads();
    }
    const uint32_t n = rpre[nreg];
    // entry i of the flat list: its region is the last r with rpre[r] <= i;
    // returns (key bits 18..6) and the key index
    auto fetch = [&](uint32_t i, uint32_t& k15, uint32_t& idx) {
        int lo = 0, hi = nreg - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (rpre[mid] <= i) lo = mid;
            else hi = mid - 1;
        }
        const uint32_t e = lists[(int64_t)lo * a.wcap + (i - rpre[lo])];
        k15 = e >> 16;
        idx = (uint32_t)(lo >> 2) * (uint32_t)a.chunk + (e & 0xFFFFu);
    };
    constexpr int U = 8;   // entries per thread with their loads in flight together
    const bool staged = n <= (uint32_t)kStageCap;
    if (staged) {
        // each thread a run of E <= kStageCap / NT consecutive entries: the
        // region of its first entry by binary search, then walking forward
        // (the next region's start kept in a register), so the loads issue
        // back to back
        constexpr int EM = kStageCap / NT;
        const uint32_t E = (n + NT - 1) / NT;
        const uint32_t i0 = threadIdx.x * E;
        if (i0 < n) {
            int rg = 0;
            {
                int hi = nreg - 1;
                while (rg < hi) {
                    const int mid = (rg + hi + 1) >> 1;
                    if (rpre[mid] <= i0) rg = mid;
                    else hi = mid - 1;
                }
            }
            uint32_t nxt = rpre[rg + 1];
            uint32_t e[EM];
            int rgs[EM];
#pragma unroll
            for (int u = 0; u < EM; u++) {
                const uint32_t i = i0 + u;
                if ((uint32_t)u < E && i < n) {
                    while (i >= nxt) {   // (past the last entry of region rg; empty regions skipped)
                        rg++;
                        nxt = rpre[rg + 1];
                    }
                    rgs[u] = rg;
                    e[u] = lists[(int64_t)rg * a.wcap + (i - rpre[rg])];
                }
            }
#pragma unroll
            for (int u = 0; u < EM; u++) {
                const uint32_t i = i0 + u;
                if ((uint32_t)u < E && i < n) {
                    s_k[i] = e[u] >> 16;
                    s_i[i] = (uint32_t)(rgs[u] >> 2) * (uint32_t)a.chunk + (e[u] & 0xFFFFu);
                }
            }
        }
        __syncthreads();
    }
    // fn(key bits 18..6, index) for every entry of the bucket
    auto each = [&](auto&& fn) {
        if (staged) {
            for (uint32_t i = threadIdx.x; i < n; i += NT) fn(s_k[i], s_i[i]);
        } else {
            for (uint32_t i0 = 0; i0 < n; i0 += NT * U) {
                uint32_t k[U], x[U];
#pragma unroll
                for (int u = 0; u < U; u++) {
                    const uint32_t i = i0 + u * NT + threadIdx.x;
                    if (i < n) fetch(i, k[u], x[u]);
                }
#pragma unroll
                for (int u = 0; u < U; u++) {
                    const uint32_t i = i0 + u * NT + threadIdx.x;
                    if (i < n) fn(k[u], x[u]);
                }
            }
        }
    };
    // The r-th largest of val(k, x) < 2^vbits (vbits <= 31) over the entries
    // with part(k, x), by radix rounds of up to 11 bits from the top.  On
    // return r is what remains of it at that value (the number of entries
    // equal to it to take) and t the number of such entries.
    auto select = [&](uint32_t& r, int vbits, auto&& val, auto&& part, uint32_t& t) -> uint32_t {
        uint32_t pref = 0;
        int hi = vbits;   // value bits above hi are decided
        int d = 0;
        while (hi > 0) {
            const int nbits = hi >= 11 ? 11 : hi;
            const int shift = hi - nbits;
            const int nb = 1 << nbits;
            for (int i = threadIdx.x; i < nb; i += NT) cnt[i] = 0u;
            __syncthreads();
            each([&](uint32_t k, uint32_t x) {
                if (!part(k, x)) return;
                const uint32_t v = val(k, x);
                if ((v >> hi) == (pref >> hi)) atomicAdd(&cnt[(v >> shift) & (uint32_t)(nb - 1)], 1u);
            });
            __syncthreads();
            uint32_t above;
            block_pick<NT>(cnt, nb, r, wsum, res, d, above);
            pref |= (uint32_t)d << shift;
            r -= above;
            hi = shift;
        }
        t = cnt[d];
        __syncthreads();   // (cnt is free again)
        return pref;
    };
    uint32_t r = (uint32_t)r0, t = 0;
    const uint32_t kT = select(
        r, kLowBits, [](uint32_t k, uint32_t) { return k; }, [](uint32_t, uint32_t) { return true; }, t);
    const uint32_t T = (P0 & kTopMask) | (kT << 6) | ((P0 & 0x80000000u) ? 0u : 0x3Fu);
    const uint32_t need = r;   // 1 <= need <= t
    int cutoff;
    if (need >= t) {
        // every key equal to T is taken: the cutoff is the largest such index
        if (threadIdx.x == 0) res[0] = 0u;
        __syncthreads();
        each([&](uint32_t k, uint32_t x) {
            if (k == kT) atomicMax(&res[0], x);
        });
        __syncthreads();
        cutoff = (int)res[0];
    } else if (t <= (uint32_t)NT) {
        // a few ties: their indices compacted in LDS (cnt is free); the one
        // with need - 1 smaller indices is the cutoff
        if (threadIdx.x == 0) res[0] = 0u;
        __syncthreads();
        each([&](uint32_t k, uint32_t x) {
            if (k == kT) cnt[atomicAdd(&res[0], 1u)] = x;
        });
        __syncthreads();
        if (threadIdx.x < t) {
            const uint32_t x = cnt[threadIdx.x];
            uint32_t below = 0;
            for (uint32_t j = 0; j < t; j++) below += cnt[j] < x ? 1u : 0u;
            if (below == need - 1) res[1] = x;
        }
        __syncthreads();
        cutoff = (int)res[1];
    } else {
        // many ties: the need-th smallest index is the need-th largest of
        // 0x7FFFFFFF - index
        uint32_t rr = need, tt = 0;
        const uint32_t v = select(
            rr, 31, [](uint32_t, uint32_t x) { return 0x7FFFFFFFu - x; },
            [kT](uint32_t k, uint32_t) { return k == kT; }, tt);
        cutoff = (int)(0x7FFFFFFFu - v);
    }
    if (threadIdx.x == 0) {
        a.prefix[bhq] = T;
        a.remain[bhq] = (int)need;
        a.cutoff[bhq] = cutoff;
    }
}

int pick_g(int group) {
    if (group % 8 == 0) return 8;
    if (group % 4 == 0) return 4;
    if (group % 2 == 0) return 2;
    return 1;
}

struct Chunks {
    int nsplit, chunk;     // collect pass
    int hsplit, hchunk;    // histogram pass
};

// key chunks of the collect pass: ~4 workgroups per CU over all groups, at
// most kMaxSplit chunks of at most kMaxChunk keys; of the histogram pass:
// ~2 workgroups (of kHistThreads) per CU, at most kMaxHistTiles tiles each
Chunks chunks_for(int batch, int hq, int hkv, int S) {
    const int G = pick_g(hq / hkv);
    const int groups = batch * hkv * ((hq / hkv) / G);
    const int tiles = (S + 63) / 64;
    auto split = [&](int per_cu, int most, int max_tiles, int& n, int& chunk) {
        int ns = (per_cu * bc::device_cu_count() + groups - 1) / (groups > 0 ? groups : 1);
        if (ns > most) ns = most;
        const int min_split = (tiles + max_tiles - 1) / max_tiles;
        if (ns < min_split) ns = min_split;
        if (ns > tiles) ns = tiles;
        if (ns < 1) ns = 1;
        const int tiles_per = (tiles + ns - 1) / ns > 0 ? (tiles + ns - 1) / ns : 1;
        chunk = tiles_per * 64;
        n = (tiles + tiles_per - 1) / tiles_per;
        if (n < 1) n = 1;
    };
    Chunks c;
    split(4, kMaxSplit, kMaxChunk / 64, c.nsplit, c.chunk);
    split(2, 1 << 30, kMaxHistTiles, c.hsplit, c.hchunk);
    return c;
}

struct Layout {
    size_t hist, hmask, prefix, remain, cutoff, pcs, lists, counts, attn, total;
};

Layout layout(int batch, int hq, int hkv, int S, int d) {
    Layout L;
    const size_t bh = (size_t)batch * hq;
    const Chunks c = chunks_for(batch, hq, hkv, S);
    const size_t regions = bh * (size_t)c.nsplit * 4;
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    L.hist = 0;
    L.hmask = al(L.hist + bh * (size_t)c.hsplit * (kTopBins / 2) * 4);
    L.prefix = al(L.hmask + bh * (size_t)c.hsplit * 8);
    L.remain = al(L.prefix + bh * 4);
    L.cutoff = al(L.remain + bh * 4);
    L.pcs = al(L.cutoff + bh * 4);
    L.lists = al(L.pcs + bh * (size_t)bc::pcs_stride(S) * (d > 255 ? 2 : 1));
    L.counts = al(L.lists + regions * (size_t)list_wave_cap(c.chunk) * 4);
    L.attn = al(L.counts + regions * 4);
    L.total = L.attn + bc::attention_ws_bytes(batch, hq, hkv, S, d);
    return L;
}

template <int D, int G>
void run_select(const SelArgs& a, int groups, int bh, int top_k, hipStream_t st) {
    const dim3 grid(a.nsplit, groups);
    hipLaunchKernelGGL((hist_kernel<D, G>), dim3(a.hsplit, groups), dim3(kHistThreads), 0, st, a);
    hipLaunchKernelGGL(pick_kernel, dim3(bh), dim3(256), 0, st, a, top_k);
    if (a.oct)
        hipLaunchKernelGGL((collect_kernel<D, G, true>), grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((collect_kernel<D, G, false>), grid, dim3(256), 0, st, a);
    hipLaunchKernelGGL(final_kernel, dim3(bh), dim3(kFinalThreads), 0, st, a);
}

template <int D>
void run_select_g(int G, const SelArgs& a, int groups, int bh, int top_k, hipStream_t st) {
    switch (G) {
        case 8: run_select<D, 8>(a, groups, bh, top_k, st); break;
        case 4: run_select<D, 4>(a, groups, bh, top_k, st); break;
        case 2: run_select<D, 2>(a, groups, bh, top_k, st); break;
        default: run_select<D, 1>(a, groups, bh, top_k, st); break;
    }
}

}  // namespace

extern "C" int bc_adaptive_attention_workspace_size(int batch, int n_heads, int n_kv_heads,
                                                    int seq_len, int head_dim, size_t* bytes) {
    BC_REQUIRE(bc::head_dim_ok(head_dim), BC_ERR_UNSUPPORTED, "head_dim %d unsupported", head_dim);
    BC_REQUIRE(batch >= 0 && n_heads >= 0 && n_kv_heads > 0 && seq_len >= 0 &&
                   n_heads % n_kv_heads == 0,
               BC_ERR_INVALID_ARGUMENT, "invalid dims");
    BC_REQUIRE(bytes != nullptr, BC_ERR_INVALID_ARGUMENT, "null bytes");
    BC_REQUIRE(seq_len <= kMaxSplit * kMaxChunk, BC_ERR_UNSUPPORTED,
               "adaptive attention: seq_len %d above %d", seq_len, kMaxSplit * kMaxChunk);
    *bytes = layout(batch, n_heads, n_kv_heads, seq_len, head_dim).total;
    return BC_OK;
}

extern "C" int bc_adaptive_attention(const void* q, const void* k_bin, const void* k_res,
                                     const void* v_bin, const void* v_res, void* out,
                                     uint8_t* selected, int batch, int n_heads, int n_kv_heads,
                                     int seq_len, int kv_stride, int head_dim, int top_k,
                                     void* workspace, size_t workspace_bytes, void* stream) {
    BC_REQUIRE(bc::head_dim_ok(head_dim), BC_ERR_UNSUPPORTED, "head_dim %d unsupported", head_dim);
    BC_REQUIRE(batch >= 0 && n_heads >= 0 && n_kv_heads > 0 && seq_len >= 0 &&
                   n_heads % n_kv_heads == 0 && kv_stride >= seq_len,
               BC_ERR_INVALID_ARGUMENT, "invalid dims");
    BC_REQUIRE(top_k >= 0, BC_ERR_INVALID_ARGUMENT, "top_k must be >= 0");
    BC_REQUIRE(seq_len <= kMaxSplit * kMaxChunk, BC_ERR_UNSUPPORTED,
               "adaptive attention: seq_len %d above %d", seq_len, kMaxSplit * kMaxChunk);
    if ((int64_t)batch * n_heads == 0) return BC_OK;
    BC_REQUIRE(q && k_bin && k_res && v_bin && v_res && out, BC_ERR_INVALID_ARGUMENT,
               "null pointer");
    const Layout L = layout(batch, n_heads, n_kv_heads, seq_len, head_dim);
    BC_REQUIRE(workspace != nullptr && workspace_bytes >= L.total, BC_ERR_WORKSPACE,
               "workspace of %zu bytes required, got %zu", L.total, workspace_bytes);
    hipStream_t st = (hipStream_t)stream;
    uint8_t* ws = (uint8_t*)workspace;
    const int bh = batch * n_heads;
    const int64_t cap = (int64_t)batch * n_kv_heads * kv_stride;
    SelArgs a{};
    a.q = (const uint16_t*)q;
    a.kb = bin_planes(k_bin, cap, head_dim);
    a.Hq = n_heads;
    a.Hkv = n_kv_heads;
    a.S = seq_len;
    a.kv_stride = kv_stride;
    a.hist = (uint32_t*)(ws + L.hist);
    a.hmask = (uint64_t*)(ws + L.hmask);
    a.prefix = (uint32_t*)(ws + L.prefix);
    a.remain = (int32_t*)(ws + L.remain);
    a.cutoff = (int32_t*)(ws + L.cutoff);
    a.pcs = ws + L.pcs;
    a.lists = (uint32_t*)(ws + L.lists);
    a.counts = (uint32_t*)(ws + L.counts);
    a.oct = kv_stride % 8 == 0 && ((uintptr_t)a.kb.scales % 16) == 0;
    const int G = pick_g(n_heads / n_kv_heads);
    const int groups = batch * n_kv_heads * ((n_heads / n_kv_heads) / G);
    const Chunks c = chunks_for(batch, n_heads, n_kv_heads, seq_len);
    a.nsplit = c.nsplit;
    a.chunk = c.chunk;
    a.hsplit = c.hsplit;
    a.hchunk = c.hchunk;
    a.wcap = list_wave_cap(c.chunk);
    const int k = top_k > seq_len ? seq_len : top_k;
    switch (head_dim) {
        case 32: run_select_g<32>(G, a, groups, bh, k, st); break;
        case 64: run_select_g<64>(G, a, groups, bh, k, st); break;
        case 96: run_select_g<96>(G, a, groups, bh, k, st); break;
        case 128: run_select_g<128>(G, a, groups, bh, k, st); break;
        case 160: run_select_g<160>(G, a, groups, bh, k, st); break;
        case 192: run_select_g<192>(G, a, groups, bh, k, st); break;
        case 224: run_select_g<224>(G, a, groups, bh, k, st); break;
        case 256: run_select_g<256>(G, a, groups, bh, k, st); break;
        default: return bc::set_error(BC_ERR_UNSUPPORTED, "head_dim %d", head_dim);
    }
    int rc = bc::check_launch("adaptive select");
    if (rc != BC_OK) return rc;
    return bc::run_attention(2, q, k_bin, k_res, v_bin, v_res, out, batch, n_heads, n_kv_heads,
                             seq_len, kv_stride, head_dim, ws + L.attn, workspace_bytes - L.attn,
                             st, a.prefix, a.cutoff, selected, a.pcs);
}
