// Adaptive precision: exact top-k residual selection per (b, query head).
//
// The ranking key of key s is scale_k * (2*popcount - d) (exact in fp32),
// mapped to an order-preserving uint32 u.  The k-th largest u is found by a
// radix select over three digits (bits 31..21, 20..10, 9..0): each pass
// histograms the digit of the keys that still match the prefix found so far
// (one LDS histogram per key chunk, stored whole), and a one-block scan per
// (b, head) sums the chunks and picks the digit where the running count from
// the top reaches k.  After the third pass the threshold T and the number
// `need` of keys equal to T that are still to be taken are exact.  Ties at T
// are taken in key order, i.e. up to a cutoff key index: the third pass's
// chunk histograms locate the chunk holding the need-th tie; one block per
// (b, head) then scans only that chunk for the cutoff index.  The attention
// kernel selects key > T, or key == T at an index <= cutoff.  Passes, tie
// scan and attention compare exact float scores against bounds derived from
// the key prefix (see key_floor), which order like the keys.
//
// The first pass computes the popcounts from the K sign planes and stores
// them (one byte per query head and key; two for d = 256), so the later
// passes, the tie scan and the attention pass read those instead of the
// d/8-byte sign rows.
//
// Workspace: chunk histograms [B*Hq][nsplit][2048] u32 | prefix [B*Hq] u32
//            | remain [B*Hq] i32 | cutoff [B*Hq] i32 | popcounts [B*Hq/G][pcs_stride(S)][G] | attention partials.
#include "attn.h"

namespace {
using bc::PcPack;
using bc::PcT;

constexpr int kBins = 2048;

struct SelArgs {
    const uint16_t* q;
    BinPlanes kb;
    int Hq, Hkv, S, kv_stride;
    int nsplit, chunk;   // key chunks of the histogram passes
    uint32_t* hist;      // [B*Hq][nsplit][2048] each key chunk's histogram of a pass
    uint32_t* prefix;    // [B*Hq]
    int32_t* remain;     // [B*Hq]
    int32_t* cutoff;     // [B*Hq]
    void* pcs;           // [B*Hq/G][pcs_stride(S)][G] popcounts (PcT<D>)
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

// Histogram of digit `pass` over keys matching prefix[bhq] in the higher digits.
// grid: (splits, B*Hkv*(group/G)); block 256; each thread strides over keys.
template <int D, int G>
__global__ __launch_bounds__(256) void hist_kernel(SelArgs a, int pass, int chunk) {
    __shared__ uint32_t qs[G][D / 32];
    __shared__ uint32_t h[G][kBins];
    const int nqg = (a.Hq / a.Hkv) / G;
    const int qg = blockIdx.y % nqg, bkv = blockIdx.y / nqg;
    const int b = bkv / a.Hkv, kvh = bkv % a.Hkv;
    const int bhq0 = b * a.Hq + kvh * (a.Hq / a.Hkv) + qg * G;
    if (pass == 0) load_q_signs<D, G>(a.q + (int64_t)bhq0 * D, qs);
    for (int i = threadIdx.x; i < G * kBins; i += blockDim.x) (&h[0][0])[i] = 0u;
    __syncthreads();
    const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
    const uint32_t dmask = pass == 2 ? 0x3FFu : 0x7FFu;
    const int pbits = pass == 0 ? 0 : (pass == 1 ? 11 : 22);
    uint32_t pref[G];
#pragma unroll
    for (int g = 0; g < G; g++) pref[g] = pass == 0 ? 0u : a.prefix[bhq0 + g];
    const int64_t base = (int64_t)bkv * a.kv_stride;
    const int k0 = blockIdx.x * chunk, k1 = min(a.S, k0 + chunk);
    using P = PcT<D>;
    using Pack = PcPack<P, G>;
    Pack* pcs = (Pack*)a.pcs + (int64_t)bhq0 / G * bc::pcs_stride(a.S);   // this group's packs
    // the prefix found so far as a key range [klo, khi] and, for scores of a
    // finite scale, as the float range (flo, fhi]
    uint32_t klo[G], khi[G];
    float flo[G], fhi[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const uint32_t low = pbits == 0 ? 0xFFFFFFFFu : (0xFFFFFFFFu >> pbits);
        klo[g] = pref[g] & ~low;
        khi[g] = klo[g] | low;
        flo[g] = klo[g] == 0u ? -INFINITY : key_floor(klo[g] - 1u);
        fhi[g] = key_floor(khi[g]);
    }
    // one key: the popcounts pc[g] of the G heads and the K scale
    auto count_key = [&](const int* pc, float sk, bool all) {
        // (a wave with a non-finite scale takes the key path for all its lanes)
        if (__ballot(!finite_scale(sk)) == 0ull) {
            const float sk2 = 2.0f * sk, nd = -(float)D * sk;
            float sc[G];
            bool mt[G];
            bool any = false;
#pragma unroll
            for (int g = 0; g < G; g++) {
                sc[g] = fmaf((float)pc[g], sk2, nd);
                mt[g] = all || (sc[g] > flo[g] && sc[g] <= fhi[g]);
                any = any || mt[g];
            }
            // (later passes: most waves have no match for a key, and skip it)
            if (all || __ballot(any) != 0ull) {
#pragma unroll
                for (int g = 0; g < G; g++)
                    if (mt[g]) atomicAdd(&h[g][(ordered_bits(sc[g]) >> shift) & dmask], 1u);
            }
        } else {
#pragma unroll
            for (int g = 0; g < G; g++) {
                const uint32_t key = key_of_pc<D>(pc[g], sk);
                if (key >= klo[g] && key <= khi[g]) atomicAdd(&h[g][(key >> shift) & dmask], 1u);
            }
        }
    };
    auto count = [&](const Pack& pk, float sk, bool all) {
        int pc[G];
#pragma unroll
        for (int g = 0; g < G; g++) pc[g] = (int)pk.v[g];
        count_key(pc, sk, all);
    };
    if (pass == 0) {
        // popcounts from the sign rows, stored for the later passes.  Two
        // register stages of UP keys per thread: the loads of the next stage
        // are in flight while a stage is counted.
        constexpr int UP = D >= 256 ? 2 : 4;
        constexpr int step = UP * 256;
        struct Stage {
            SignWords<D> ks[UP];
            uint16_t sk[UP];
        };
        auto load = [&](Stage& st, int s) {
#pragma unroll
            for (int u = 0; u < UP; u++) {
                const int ss = s + u * 256;
                const int64_t i = base + (ss < k1 ? ss : k0);
                st.ks[u] = load_signs<D, true>(a.kb.signs + i * (D / 8));
                st.sk[u] = a.kb.scales[i];
            }
        };
        auto run = [&](const Stage& st, int s) {
#pragma unroll
            for (int u = 0; u < UP; u++) {
                const int ss = s + u * 256;
                if (ss >= k1) break;
                Pack pk;
#pragma unroll
                for (int g = 0; g < G; g++) pk.v[g] = (P)popc_of<D>(qs[g], st.ks[u]);
                pcs[ss] = pk;
                count(pk, h2f(st.sk[u]), true);
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
    } else if (a.oct) {
        // stored popcounts, eight consecutive keys per lane and load: their
        // packs (8 G-head packs, whole 16-byte loads where they fill one) and
        // their K scales (16 bytes).  Two register stages of UP octets: the
        // loads of the next stage are in flight while a stage is counted.
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
        auto run = [&](const Stage& st, int o) {
#pragma unroll
            for (int u = 0; u < UP; u++) {
                const int oo = o + u * 256;
                if (oo >= o1) break;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    if (8 * oo + j >= k1) break;   // (only the range's last octet is partial)
                    const uint32_t sw = st.sc[u][j >> 1];
                    const float sk = h2f((uint16_t)((j & 1) ? (sw >> 16) : (sw & 0xFFFFu)));
                    int pc[G];
#pragma unroll
                    for (int g = 0; g < G; g++) {
                        constexpr int pb = (int)sizeof(P);
                        const int byte = (j * G + g) * pb;
                        pc[g] = (int)((st.pw[u][byte / 4] >> (8 * (byte % 4))) & ((1u << (8 * pb)) - 1u));
                    }
                    count_key(pc, sk, false);
                }
            }
        };
        Stage sa, sb;
        int o = o0 + threadIdx.x;
        load(sa, o);
        for (;;) {
            load(sb, o + step);
            run(sa, o);
            o += step;
            if (o >= o1) break;
            load(sa, o + step);
            run(sb, o);
            o += step;
            if (o >= o1) break;
        }
    } else {
        // stored popcounts: sixteen keys per thread per iteration
        constexpr int U = 16;
        for (int s = k0 + threadIdx.x; s < k1; s += U * blockDim.x) {
            Pack pk[U];
            float sk[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int ss = s + u * blockDim.x;
                const int sc = ss < k1 ? ss : s;
                pk[u] = pcs[sc];
                sk[u] = h2f(a.kb.scales[base + sc]);
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (s + u * (int)blockDim.x >= k1) break;
                count(pk[u], sk[u], false);
            }
        }
    }
    __syncthreads();
    // this chunk's histogram, stored whole (plain coalesced stores; the pick
    // sums the chunks, and the last pass's chunk histograms locate the ties)
    const int nb = pass == 2 ? 1024 : kBins;
    for (int i = threadIdx.x; i < G * nb; i += blockDim.x) {
        const int g = i / nb, bin = i % nb;
        a.hist[((int64_t)(bhq0 + g) * a.nsplit + blockIdx.x) * kBins + bin] = h[g][bin];
    }
}

// One block per (b, query head): sum the chunk histograms of the pass and
// pick the digit holding the remain-th largest key; extend the prefix.
__global__ __launch_bounds__(256) void pick_kernel(SelArgs a, int pass, int top_k) {
    __shared__ uint32_t cnt[kBins];
    __shared__ uint32_t part[256];
    const int bhq = blockIdx.x;
    const uint32_t* h = a.hist + (int64_t)bhq * a.nsplit * kBins;
    const int nbins = pass == 2 ? 1024 : 2048;
    const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
    {
        // eight consecutive bins per thread (the last pass stores 1024)
        const int b0 = threadIdx.x * 8;
        uint32_t sum[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
        if (b0 < nbins) {
            for (int c = 0; c < a.nsplit; c++) {
                const bc_v4u x = *(const bc_v4u*)(h + (int64_t)c * kBins + b0);
                const bc_v4u y = *(const bc_v4u*)(h + (int64_t)c * kBins + b0 + 4);
                sum[0] += x[0]; sum[1] += x[1]; sum[2] += x[2]; sum[3] += x[3];
                sum[4] += y[0]; sum[5] += y[1]; sum[6] += y[2]; sum[7] += y[3];
            }
        }
#pragma unroll
        for (int j = 0; j < 8; j++) cnt[b0 + j] = sum[j];
    }
    __syncthreads();
    int remain = pass == 0 ? top_k : a.remain[bhq];
    uint32_t prefix = pass == 0 ? 0u : a.prefix[bhq];
    // per-thread counts of 8 consecutive bins (descending digits)
    const int per = kBins / 256;
    uint32_t local = 0;
    for (int j = 0; j < per; j++) {
        const int d = nbins - 1 - (threadIdx.x * per + j);
        if (d >= 0) local += cnt[d];
    }
    part[threadIdx.x] = local;
    __syncthreads();
    if (remain <= 0) {
        if (threadIdx.x == 0 && pass == 0) {
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
        // fewer matching keys than remain: select everything
        a.prefix[bhq] = 0u;
        a.remain[bhq] = 0;
    }
    if (excl < (uint32_t)remain && incl >= (uint32_t)remain) {
        // this thread's 8 bins hold the remain-th largest key
        uint32_t above = excl;
        int digit = 0;
        for (int j = 0; j < per; j++) {
            const int d = nbins - 1 - (threadIdx.x * per + j);
            if (d < 0) break;
            if (above + cnt[d] >= (uint32_t)remain) {
                digit = d;
                break;
            }
            above += cnt[d];
        }
        a.prefix[bhq] = prefix | ((uint32_t)digit << shift);
        a.remain[bhq] = remain - (int)above;
    }
}

// Cutoff index of the ties at the final threshold T: one block per (b, query
// head).  The chunk histograms give the chunk holding the need-th tie; that
// chunk is scanned from the stored popcounts and K scales (see below).
template <int D, int G>
__global__ __launch_bounds__(256) void tie_locate_kernel(SelArgs a) {
    __shared__ int sh_chunk, sh_rank, sh_total;
    __shared__ uint64_t tmask[64][4];   // [stripe][wave] tie ballots of a window
    using Pack = PcPack<PcT<D>, G>;
    const int bhq = blockIdx.x;
    const int b = bhq / a.Hq, h = bhq % a.Hq;
    const int kvh = h / (a.Hq / a.Hkv);
    const int g = bhq % G;   // head slot in its group (groups are G consecutive heads)
    const int need = a.remain[bhq];
    if (need <= 0) {
        if (threadIdx.x == 0) a.cutoff[bhq] = -1;
        return;
    }
    const uint32_t T = a.prefix[bhq];
    const float tv = key_value(T);   // the score of key T (finite scales)
    if (threadIdx.x == 0) {
        const uint32_t* ch = a.hist + (int64_t)bhq * a.nsplit * kBins + (T & 0x3FFu);
        int cum = 0, c = 0;
        for (; c < a.nsplit - 1; c++) {
            const int t = (int)ch[(int64_t)c * kBins];
            if (cum + t >= need) break;
            cum += t;
        }
        sh_chunk = c;
        sh_rank = need - cum;   // the rank-th tie (from 1) of chunk c is the last one taken
    }
    __syncthreads();
    const int64_t base = ((int64_t)b * a.Hkv + kvh) * a.kv_stride;
    const Pack* pcs = (const Pack*)a.pcs + (int64_t)(bhq - g) / G * bc::pcs_stride(a.S);
    const int k0 = sh_chunk * a.chunk, k1 = min(a.S, k0 + a.chunk);
    // windows of 64 stripes of 256 keys, read coalesced (all loads of 16
    // stripes issued first); a wave ballot per stripe records the ties; one
    // wave prefix-sums the 64 stripe counts, finds the stripe holding the
    // rank-th tie, and picks the key from that stripe's per-wave masks
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int rank = sh_rank;
    for (int w0 = k0; w0 < k1; w0 += 256 * 64) {
        for (int b0 = 0; b0 < 64; b0 += 16) {
            int pcv[16];
            float skv[16];
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const int sv = w0 + (b0 + u) * 256 + (int)threadIdx.x;
                const int sc = sv < k1 ? sv : k0;
                pcv[u] = (int)pcs[sc].v[g];
                skv[u] = h2f(a.kb.scales[base + sc]);
            }
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const int sv = w0 + (b0 + u) * 256 + (int)threadIdx.x;
                const float sk = skv[u];
                bool tie;
                if (__ballot(!finite_scale(sk)) == 0ull) tie = fmaf((float)pcv[u], 2.0f * sk, -(float)D * sk) == tv;
                else tie = key_of_pc<D>(pcv[u], sk) == T;
                const uint64_t m = __ballot(sv < k1 && tie);
                if (lane == 0) tmask[b0 + u][wave] = m;
            }
        }
        __syncthreads();
        if (wave == 0) {
            const int j = lane;   // stripe
            const uint32_t c = (uint32_t)(__builtin_popcountll(tmask[j][0]) + __builtin_popcountll(tmask[j][1]) +
                                          __builtin_popcountll(tmask[j][2]) + __builtin_popcountll(tmask[j][3]));
            uint32_t incl = c;
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t up = __shfl_up(incl, off, 64);
                if (lane >= off) incl += up;
            }
            const uint32_t excl = incl - c;
            if (excl < (uint32_t)rank && incl >= (uint32_t)rank) {
                uint32_t r = (uint32_t)rank - excl;
                for (int w = 0; w < 4; w++) {
                    const uint64_t m = tmask[j][w];
                    const uint32_t cw = (uint32_t)__builtin_popcountll(m);
                    if (r <= cw) {
                        for (int i = 0; i < 64; i++) {
                            if (((m >> i) & 1ull) && --r == 0) {
                                a.cutoff[bhq] = w0 + j * 256 + w * 64 + i;
                                break;
                            }
                        }
                        break;
                    }
                    r -= cw;
                }
            }
            if (lane == 63) sh_total = (int)incl;
        }
        __syncthreads();
        if (sh_total >= rank) break;   // found in this window
        rank -= sh_total;
    }
}

int pick_g(int group) {
    if (group % 8 == 0) return 8;
    if (group % 4 == 0) return 4;
    if (group % 2 == 0) return 2;
    return 1;
}

struct Chunks {
    int nsplit, chunk;
};

// key chunks of the histogram passes: ~4 workgroups per CU over all groups
Chunks chunks_for(int batch, int hq, int hkv, int S) {
    const int G = pick_g(hq / hkv);
    const int groups = batch * hkv * ((hq / hkv) / G);
    const int tiles = (S + 63) / 64;
    int nsplit = (4 * bc::device_cu_count() + groups - 1) / (groups > 0 ? groups : 1);
    if (nsplit > tiles) nsplit = tiles;
    if (nsplit < 1) nsplit = 1;
    const int tiles_per = (tiles + nsplit - 1) / nsplit > 0 ? (tiles + nsplit - 1) / nsplit : 1;
    Chunks c;
    c.chunk = tiles_per * 64;
    c.nsplit = (tiles + tiles_per - 1) / tiles_per;
    if (c.nsplit < 1) c.nsplit = 1;
    return c;
}

struct Layout {
    size_t hist, prefix, remain, cutoff, pcs, attn, total;
};

Layout layout(int batch, int hq, int hkv, int S, int d) {
    Layout L;
    const size_t bh = (size_t)batch * hq;
    const Chunks c = chunks_for(batch, hq, hkv, S);
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    L.hist = 0;
    L.prefix = al(L.hist + bh * (size_t)c.nsplit * kBins * 4);
    L.remain = al(L.prefix + bh * 4);
    L.cutoff = al(L.remain + bh * 4);
    L.pcs = al(L.cutoff + bh * 4);
    L.attn = al(L.pcs + bh * (size_t)bc::pcs_stride(S) * (d > 255 ? 2 : 1));
    L.total = L.attn + bc::attention_ws_bytes(batch, hq, hkv, S, d);
    return L;
}

template <int D, int G>
void run_passes(const SelArgs& a, int splits_y, int chunk, int nsplit, int bh, int top_k,
                hipStream_t st) {
    const dim3 grid(nsplit, splits_y);
    for (int pass = 0; pass < 3; pass++) {
        hipLaunchKernelGGL((hist_kernel<D, G>), grid, dim3(256), 0, st, a, pass, chunk);
        hipLaunchKernelGGL(pick_kernel, dim3(bh), dim3(256), 0, st, a, pass, top_k);
    }
    hipLaunchKernelGGL((tie_locate_kernel<D, G>), dim3(bh), dim3(256), 0, st, a);
}

template <int D>
void run_passes_g(int G, const SelArgs& a, int groups, int chunk, int nsplit, int bh, int top_k,
                  hipStream_t st) {
    switch (G) {
        case 8: run_passes<D, 8>(a, groups, chunk, nsplit, bh, top_k, st); break;
        case 4: run_passes<D, 4>(a, groups, chunk, nsplit, bh, top_k, st); break;
        case 2: run_passes<D, 2>(a, groups, chunk, nsplit, bh, top_k, st); break;
        default: run_passes<D, 1>(a, groups, chunk, nsplit, bh, top_k, st); break;
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
    a.prefix = (uint32_t*)(ws + L.prefix);
    a.remain = (int32_t*)(ws + L.remain);
    a.cutoff = (int32_t*)(ws + L.cutoff);
    a.pcs = ws + L.pcs;
    a.oct = kv_stride % 8 == 0 && ((uintptr_t)a.kb.scales % 16) == 0;
    const int G = pick_g(n_heads / n_kv_heads);
    const int groups = batch * n_kv_heads * ((n_heads / n_kv_heads) / G);
    const Chunks c = chunks_for(batch, n_heads, n_kv_heads, seq_len);
    const int nsplit = c.nsplit, chunk = c.chunk;
    a.nsplit = nsplit;
    a.chunk = chunk;
    const int k = top_k > seq_len ? seq_len : top_k;
    switch (head_dim) {
        case 32: run_passes_g<32>(G, a, groups, chunk, nsplit, bh, k, st); break;
        case 64: run_passes_g<64>(G, a, groups, chunk, nsplit, bh, k, st); break;
        case 96: run_passes_g<96>(G, a, groups, chunk, nsplit, bh, k, st); break;
        case 128: run_passes_g<128>(G, a, groups, chunk, nsplit, bh, k, st); break;
        case 160: run_passes_g<160>(G, a, groups, chunk, nsplit, bh, k, st); break;
        case 192: run_passes_g<192>(G, a, groups, chunk, nsplit, bh, k, st); break;
        case 224: run_passes_g<224>(G, a, groups, chunk, nsplit, bh, k, st); break;
        case 256: run_passes_g<256>(G, a, groups, chunk, nsplit, bh, k, st); break;
        default: return bc::set_error(BC_ERR_UNSUPPORTED, "head_dim %d", head_dim);
    }
    int rc = bc::check_launch("adaptive select");
    if (rc != BC_OK) return rc;
    return bc::run_attention(2, q, k_bin, k_res, v_bin, v_res, out, batch, n_heads, n_kv_heads,
                             seq_len, kv_stride, head_dim, ws + L.attn, workspace_bytes - L.attn,
                             st, a.prefix, a.cutoff, selected, a.pcs);
}
