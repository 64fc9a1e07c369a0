// Shared declarations of the split-KV attention kernels (attention.hip,
// attention_mfma.hip).
#pragma once

#include "common.h"

namespace bc {

constexpr float kLog2e = 1.4426950408889634f;

// MODE_MIXED: compensated data flow, each (b, query head) adding its residual
// (score and value) or not as head_mode says: per-head binary / compensated
// dispatch in one launch.
enum AttnMode : int { MODE_BINARY = 0, MODE_COMP = 1, MODE_ADAPTIVE = 2, MODE_MIXED = 3 };

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
    // in-place append (binary and compensated modes, one query-head group per
    // kv head): the new K and V vectors [B*Hkv, D] fp16 are encoded into cache
    // position app_slot of every (b, kv head) row before the row is attended
    // (null: no append)
    const uint16_t* app_k;
    const uint16_t* app_v;
    int app_slot;
    // MODE_MIXED: [B*Hq] 0 = binary attention for that head, else compensated
    const uint8_t* head_mode;
    // per-head modes run as two launches (binary kernel, mixed kernel), each
    // over the query-head groups of its kind: grid row y takes group
    // group_list[y] while y < *group_count, and returns otherwise (lists in
    // the workspace, written by a compaction launch; null: row y is group y)
    const int32_t* group_list;
    const int32_t* group_count;
    // one split per group (n_splits == 1): when set, the kernel writes the
    // normalised output [B, Hq, D] fp16 here instead of its partial, and no
    // merge launch follows
    uint16_t* out;
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
bool launch_mfma_split(int mode, int D, int G, const AttnArgs& a, dim3 grid, hipStream_t st, int nw = 4);
// True if the MFMA kernels handle head_dim D with splits of `chunk` keys.
bool mfma_split_ok(int D, int64_t chunk);
// Resident workgroups per CU of the MFMA kernel of (mode, D, G) on the current
// device (0 when no MFMA kernel handles it).
int mfma_wgs_per_cu(int mode, int D, int G);

// New K/V token encoded into cache position `slot` by the attention launch
// itself (see AttnArgs::app_k).
struct AppendArgs {
    const void* k;   // [B*Hkv, D] fp16
    const void* v;
    int slot;
};

// Split partials + combine (attention.hip), shared by the public entry points
// and the adaptive driver (adaptive.hip).  app: append the token first (the
// caller has checked that the MFMA kernel runs with one query-head group per
// kv head).
int run_attention(int mode, const void* q, const void* k_bin, const void* k_res, const void* v_bin,
                  const void* v_res, void* out, int batch, int n_heads, int n_kv_heads,
                  int seq_len, int kv_stride, int head_dim, void* workspace,
                  size_t workspace_bytes, hipStream_t st, const uint32_t* thresh,
                  const int32_t* cutoff, uint8_t* selected, const void* pcs,
                  const AppendArgs* app = nullptr, const uint8_t* head_mode = nullptr);
size_t attention_ws_bytes(int batch, int n_heads, int n_kv_heads, int seq_len, int d);
}  // namespace bc
