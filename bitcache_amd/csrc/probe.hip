// Measurement aid: the HBM read ceiling of a plain streaming read on this
// device, for reading the attention kernels' bandwidth against what the
// memory system delivers rather than against the data-sheet peak alone.
//
// bc_mix_probe does the same for a stream of 3 bytes read per byte written
// (whole-line 16-byte-per-lane stores): the ceiling of the encoders' mix.
//
// Each workgroup reads one contiguous slab with 16-byte nontemporal loads
// (eight in flight per lane), the access policy the attention kernels use for
// their whole-KiB runs, and XOR-reduces it into one word (so the loads stay
// live; one word per wave goes to out).  Four workgroups per CU.
#include <hip/hip_runtime.h>

#include "common.h"

namespace {

typedef unsigned int u4_t __attribute__((ext_vector_type(4)));
constexpr int kReadUnroll = 8;
constexpr int kReadWgsPerCu = 4;

__global__ __launch_bounds__(256) void read_probe_kernel(const u4_t* __restrict__ src, int64_t n_u4, uint32_t* out) {
    const int64_t per = (n_u4 + gridDim.x - 1) / gridDim.x;
    const int64_t lo = (int64_t)blockIdx.x * per;
    const int64_t hi = lo + per < n_u4 ? lo + per : n_u4;
    u4_t acc = {0u, 0u, 0u, 0u};
    for (int64_t i = lo + threadIdx.x; i < hi; i += 256 * kReadUnroll) {
        u4_t v[kReadUnroll];
#pragma unroll
        for (int u = 0; u < kReadUnroll; u++) {
            const int64_t j = i + (int64_t)u * 256;
            v[u] = j < hi ? __builtin_nontemporal_load(src + j) : u4_t{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < kReadUnroll; u++) acc ^= v[u];
    }
    // one word per wave: the XOR of its lanes' words
    uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
    r ^= __shfl_xor(r, 32);
    r ^= __shfl_xor(r, 16);
    r ^= __shfl_xor(r, 8);
    r ^= __shfl_xor(r, 4);
    r ^= __shfl_xor(r, 2);
    r ^= __shfl_xor(r, 1);
    if ((threadIdx.x & 63) == 0) out[4 * blockIdx.x + (threadIdx.x >> 6)] = r;
}

// Mixed stream: per iteration each lane reads three 16-byte words (three
// coalesced KiB per wave) and writes their XOR (one whole-line KiB per wave):
// 3 bytes read per byte written, about the encoders' 256 B in / 84 B out.
template <bool NT_STORE>
__global__ __launch_bounds__(256) void mix_probe_kernel(const u4_t* __restrict__ src, u4_t* __restrict__ dst,
                                                        int64_t n_out, int64_t per) {
    // per and n_out are multiples of 256 words: every block below starts at a
    // multiple of 256 and lies wholly inside [lo, hi), so its three input
    // blocks lie inside src's 3 * n_out words
    const int64_t lo = (int64_t)blockIdx.x * per;
    const int64_t hi = lo + per < n_out ? lo + per : n_out;
    constexpr int U = 2;
    for (int64_t i0 = lo; i0 < hi; i0 += 256 * U) {
        u4_t v[U][3];
#pragma unroll
        for (int u = 0; u < U; u++) {
            // output words [i0 + 256u, +256) come from input words 3 * (that block)
            const int64_t blk = i0 + 256 * u;
            const int64_t j = blk + threadIdx.x;
#pragma unroll
            for (int r = 0; r < 3; r++)
                v[u][r] = j < hi ? __builtin_nontemporal_load(src + 3 * blk + 256 * r + threadIdx.x)
                                 : u4_t{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t j = i0 + 256 * u + threadIdx.x;
            if (j < hi) {
                const u4_t w = v[u][0] ^ v[u][1] ^ v[u][2];
                if (NT_STORE) __builtin_nontemporal_store(w, dst + j);
                else dst[j] = w;
            }
        }
    }
}

}  // namespace

extern "C" int bc_mix_probe(const void* src, void* dst, int64_t n_write_bytes, int nt_store, void* stream) {
    BC_REQUIRE(n_write_bytes >= 0 && n_write_bytes % 16 == 0, BC_ERR_INVALID_ARGUMENT,
               "mix probe: n_write_bytes must be a non-negative multiple of 16, got %lld",
               (long long)n_write_bytes);
    if (n_write_bytes == 0) return BC_OK;
    BC_REQUIRE(src && dst, BC_ERR_INVALID_ARGUMENT, "null pointer");
    BC_REQUIRE(((uintptr_t)src & 15) == 0 && ((uintptr_t)dst & 15) == 0, BC_ERR_INVALID_ARGUMENT,
               "mix probe: src and dst must be 16-byte aligned");
    const int64_t n_out = n_write_bytes / 16;
    int wgs = bc::device_cu_count() * kReadWgsPerCu;
    // whole 256-word blocks per workgroup, so that every read stays in src
    const int64_t blocks = n_out / 256;
    BC_REQUIRE(n_out % 256 == 0, BC_ERR_INVALID_ARGUMENT,
               "mix probe: n_write_bytes must be a multiple of 4096");
    if (wgs > blocks) wgs = (int)blocks;
    // each workgroup's range is whole blocks: round the per-workgroup share up
    const int64_t per_blocks = (blocks + wgs - 1) / wgs;
    wgs = (int)((blocks + per_blocks - 1) / per_blocks);
    if (nt_store)
        hipLaunchKernelGGL(mix_probe_kernel<true>, dim3(wgs), dim3(256), 0, (hipStream_t)stream,
                           (const u4_t*)src, (u4_t*)dst, n_out, per_blocks * 256);
    else
        hipLaunchKernelGGL(mix_probe_kernel<false>, dim3(wgs), dim3(256), 0, (hipStream_t)stream,
                           (const u4_t*)src, (u4_t*)dst, n_out, per_blocks * 256);
    return bc::check_launch("mix_probe_kernel");
}

extern "C" int bc_read_probe(const void* src, int64_t n_bytes, void* out, void* stream) {
    BC_REQUIRE(n_bytes >= 0 && n_bytes % 16 == 0, BC_ERR_INVALID_ARGUMENT,
               "read probe: n_bytes must be a non-negative multiple of 16, got %lld", (long long)n_bytes);
    if (n_bytes == 0) return BC_OK;
    BC_REQUIRE(src && out, BC_ERR_INVALID_ARGUMENT, "null pointer");
    BC_REQUIRE(((uintptr_t)src & 15) == 0, BC_ERR_INVALID_ARGUMENT, "read probe: src must be 16-byte aligned");
    int wgs = bc::device_cu_count() * kReadWgsPerCu;
    if (wgs > BC_READ_PROBE_MAX_WGS) wgs = BC_READ_PROBE_MAX_WGS;
    const int64_t n_u4 = n_bytes / 16;
    if (wgs > n_u4) wgs = (int)n_u4;
    hipLaunchKernelGGL(read_probe_kernel, dim3(wgs), dim3(256), 0, (hipStream_t)stream, (const u4_t*)src, n_u4,
                       (uint32_t*)out);
    return bc::check_launch("read_probe_kernel");
}
