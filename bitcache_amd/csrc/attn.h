// Shared declarations of the split-KV attention kernels (attention.hip,
// attention_mfma.hip).
#pragma once

#include "common.h"

namespace bc {

constexpr float kLog2e = 1.4426950408889634f;

enum AttnMode : int { MODE_BINARY = 0, MODE_COMP = 1, MODE_ADAPTIVE = 2 };

struct AttnArgs {
    const uint16_t* q;  // [B, Hq, D] fp16
    BinPlanes kb, vb;
    ResPlanes kr, vr;
    int B, Hq, Hkv, S, kv_stride;
    int n_splits, chunk;  // chunk: keys per split (multiple of 64)
    float* ws;            // [B*Hq][n_splits][D + 2]: m (log2 domain), l, acc[D]
    // adaptive selection (MODE_ADAPTIVE)
    const uint32_t* thresh;      // [B*Hq] ordered key threshold
    const int32_t* cutoff;       // [B*Hq] keys equal to the threshold are taken up to
                                 // this key index (-1: none)
    uint8_t* selected;           // optional [B, Hq, S]
    const void* pcs;             // adaptive: [B*Hq/G][pcs_stride(S)] PcPack<PcT<D>, G>
                                 // popcounts of the selection passes (G = the kernel's
                                 // head group)
};

// Packs per row of the stored popcounts: S rounded up to 16, so that every
// row starts 16-byte aligned and eight-key runs load whole.
__host__ __device__ inline int pcs_stride(int S) { return (S + 15) & ~15; }

// Stored popcount of one (query head, key): 8 bits, 16 for d = 256 (popcount
// up to 256).  A pack holds the G heads of a query-head group for one key.
template <bool WIDE> struct PcSel { typedef uint8_t type; };
template <> struct PcSel<true> { typedef uint16_t type; };
template <int D> using PcT = typename PcSel<(D > 255)>::type;
template <typename P, int G>
struct __attribute__((aligned(G * sizeof(P)))) PcPack {
    P v[G];
};

// MFMA value-phase kernels (attention_mfma.hip): true if (D, G, mode) is
// handled there and the launch was issued.
bool launch_mfma_split(int mode, int D, int G, const AttnArgs& a, dim3 grid, hipStream_t st);
// Resident workgroups per CU of the MFMA kernel of (mode, D, G) on the current
// device (0 when no MFMA kernel handles it).
int mfma_wgs_per_cu(int mode, int D, int G);
}  // namespace bc
