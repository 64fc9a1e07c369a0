// Conversion between the dense planar blobs and the reference's array-of-structs
// bytes (BinaryVec = u32 words[8] + fp16 scale + 2 pad bytes, 36 B;
// ResidualVec = u8 nibbles[128] + fp16 scale, 130 B; src/binary_encode.cuh:13-18,
// src/residual.cuh:11-16).  One thread per output byte: trivially coalesced on
// the output side; the input side reads small contiguous runs.
#include "common.h"

namespace {

constexpr int kBinVec = 36, kResVec = 130;

__global__ void bin_to_ref(const uint8_t* blob, uint8_t* aos, int64_t n, int d) {
    const uint8_t* scales = blob + n * (d / 8);
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n * kBinVec;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t v = i / kBinVec;
        const int o = (int)(i % kBinVec);
        uint8_t b = 0;
        if (o < d / 8) b = blob[v * (d / 8) + o];
        else if (o == 32 || o == 33) b = scales[2 * v + (o - 32)];
        aos[i] = b;
    }
}

__global__ void bin_from_ref(const uint8_t* aos, uint8_t* blob, int64_t n, int d) {
    const int64_t sb = n * (d / 8);
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < sb + 2 * n;
         i += (int64_t)gridDim.x * blockDim.x) {
        if (i < sb) {
            const int64_t v = i / (d / 8);
            blob[i] = aos[v * kBinVec + (i % (d / 8))];
        } else {
            const int64_t j = i - sb;
            blob[i] = aos[(j / 2) * kBinVec + 32 + (j % 2)];
        }
    }
}

__global__ void res_to_ref(const uint8_t* blob, uint8_t* aos, int64_t n, int d) {
    const uint8_t* scales = blob + n * (d / 2);
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n * kResVec;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t v = i / kResVec;
        const int o = (int)(i % kResVec);
        uint8_t b = 0;
        if (o < d / 2) b = blob[v * (d / 2) + o];
        else if (o == 128 || o == 129) b = scales[2 * v + (o - 128)];
        aos[i] = b;
    }
}

__global__ void res_from_ref(const uint8_t* aos, uint8_t* blob, int64_t n, int d) {
    const int64_t sb = n * (d / 2);
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < sb + 2 * n;
         i += (int64_t)gridDim.x * blockDim.x) {
        if (i < sb) {
            const int64_t v = i / (d / 2);
            blob[i] = aos[v * kResVec + (i % (d / 2))];
        } else {
            const int64_t j = i - sb;
            blob[i] = aos[(j / 2) * kResVec + 128 + (j % 2)];
        }
    }
}

int grid_bytes(int64_t n) {
    int64_t g = (n + 255) / 256;
    return (int)(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

}  // namespace

#define BC_CONV_CHECK()                                                                        \
    BC_REQUIRE(bc::head_dim_ok(head_dim), BC_ERR_UNSUPPORTED, "head_dim %d unsupported", head_dim); \
    BC_REQUIRE(n >= 0, BC_ERR_INVALID_ARGUMENT, "n < 0");                                       \
    if (n == 0) return BC_OK;

extern "C" int bc_binary_to_reference(const void* blob, void* ref_aos, int64_t n, int head_dim,
                                      void* stream) {
    BC_CONV_CHECK();
    BC_REQUIRE(blob && ref_aos, BC_ERR_INVALID_ARGUMENT, "null pointer");
    hipLaunchKernelGGL(bin_to_ref, dim3(grid_bytes(n * kBinVec)), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)blob, (uint8_t*)ref_aos, n, head_dim);
    return bc::check_launch("binary_to_reference");
}

extern "C" int bc_binary_from_reference(const void* ref_aos, void* blob, int64_t n, int head_dim,
                                        void* stream) {
    BC_CONV_CHECK();
    BC_REQUIRE(blob && ref_aos, BC_ERR_INVALID_ARGUMENT, "null pointer");
    hipLaunchKernelGGL(bin_from_ref, dim3(grid_bytes(n * (head_dim / 8 + 2))), dim3(256), 0,
                       (hipStream_t)stream, (const uint8_t*)ref_aos, (uint8_t*)blob, n, head_dim);
    return bc::check_launch("binary_from_reference");
}

extern "C" int bc_residual_to_reference(const void* blob, void* ref_aos, int64_t n, int head_dim,
                                        void* stream) {
    BC_CONV_CHECK();
    BC_REQUIRE(blob && ref_aos, BC_ERR_INVALID_ARGUMENT, "null pointer");
    hipLaunchKernelGGL(res_to_ref, dim3(grid_bytes(n * kResVec)), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)blob, (uint8_t*)ref_aos, n, head_dim);
    return bc::check_launch("residual_to_reference");
}

extern "C" int bc_residual_from_reference(const void* ref_aos, void* blob, int64_t n,
                                          int head_dim, void* stream) {
    BC_CONV_CHECK();
    BC_REQUIRE(blob && ref_aos, BC_ERR_INVALID_ARGUMENT, "null pointer");
    hipLaunchKernelGGL(res_from_ref, dim3(grid_bytes(n * (head_dim / 2 + 2))), dim3(256), 0,
                       (hipStream_t)stream, (const uint8_t*)ref_aos, (uint8_t*)blob, n, head_dim);
    return bc::check_launch("residual_from_reference");
}
