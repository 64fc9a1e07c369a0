// One vector of the row encoder, shared by the encode kernels (encode.hip) and
// the attention kernel's in-place append (attention_mfma.hip).
//
// d in {64, 128, 256}: L = d/8 lanes per vector, lane j (0 <= j < L) of its
// L-lane group holding elements 8j..8j+7 (one 16-byte load); a wave holds
// 64/L such groups, lane = group * L + j, and every lane of the wave calls
// encode_row (the reductions are DPP / swizzle moves within the group).  The
// scale sum follows the reference tree exactly: element t = 8j + k sits in
// lane j, so the tree levels s = 64..8 (src/binary_encode.cu:44-50) pair lane
// j with lane j + s/8 (row_shl) and the levels s = 4, 2, 1 are in-lane; d = 256
// first adds |x_{t+128}| from the lane 16 above (the reference's per-thread
// loop, :31-41), d = 64 skips the s = 64 level (it adds +0.0).
#pragma once

#include "common.h"

namespace bc {

enum EncodeMode : int {
    ENC_BINARY = 0,         // bits + scale
    ENC_FUSED_FP16 = 1,     // bits + scale + residual against the fp16 scale (two-step semantics)
    ENC_FUSED_FP32 = 2,     // bits + scale + residual against the fp32 mean (online semantics)
    ENC_RESIDUAL_ONLY = 3,  // residual against bits + fp16 scale read from a binary blob
    ENC_TRAFFIC = 4,        // the fused encoder's loads and stores, no arithmetic (memory floor)
};

// Planes of a destination blob pair (code_plane may be null: binary only).
struct EncodeDst {
    uint8_t* sign_plane;    // ENC_RESIDUAL_ONLY: read, not written
    uint16_t* scale_plane;
    uint8_t* code_plane;
    uint16_t* rscale_plane;
};

// __float2int_rn followed by the [-7, 7] clamp of src/residual.cu:67-72; NaN -> 0.
__device__ __forceinline__ int quant7(float v) {
    if (!(v == v)) return 0;
    float c = fminf(fmaxf(v, -7.0f), 7.0f);
    return (int)__builtin_rintf(c);
}

// This lane's 16-byte slice (elements 8j..8j+7) of the fp16 vector at vec:
// nontemporal, the wave's vectors are one contiguous run read once.
__device__ __forceinline__ bc_v4u load_row_slice(const uint16_t* vec, int j) {
    return __builtin_nontemporal_load((const bc_v4u*)vec + j);
}

// Encode the d-element fp16 vector whose slice this lane holds (raw, from
// load_row_slice) into vector slot dv of dst; lanes with live = false compute
// along (their group's reductions) but store nothing.
template <int D, int MODE>
__device__ __forceinline__ void encode_row_slice(const bc_v4u raw, int j, bool live, const EncodeDst& dst,
                                                 int64_t dv) {
    static_assert(D == 64 || D == 128 || D == 256, "row encoder: d in {64, 128, 256}");
    constexpr int L = D / 8;        // lanes per vector
    // swizzle pattern that broadcasts lane 0 of each L-lane group (and-mask mode)
    constexpr int BCAST = L == 8 ? 0x18 : (L == 16 ? 0x10 : 0x00);
    const uint32_t hw[4] = {raw[0], raw[1], raw[2], raw[3]};
    float x[8];
#pragma unroll
    for (int k = 0; k < 8; k++) x[k] = h2f((uint16_t)(hw[k >> 1] >> (16 * (k & 1))));

    uint32_t byte = 0;
    float s;
    float mean = 0.0f;
    if constexpr (MODE == ENC_RESIDUAL_ONLY) {
        byte = dst.sign_plane[dv * (D / 8) + j];
        s = h2f(dst.scale_plane[dv]);
    } else {
#pragma unroll
        for (int k = 0; k < 8; k++) byte |= (x[k] >= 0.0f ? 1u : 0u) << k;  // +-0 -> 1, NaN -> 0
        // (the first level takes |x| of both operands as source modifiers)
        float p[8];
        if constexpr (D == 256) {
#pragma unroll
            for (int k = 0; k < 8; k++) p[k] = fabsf(x[k]) + fabsf(swz_f<0x401F>(x[k]));  // + |x_{t+128}|
#pragma unroll
            for (int k = 0; k < 8; k++) p[k] = p[k] + dpp_f<0x108>(p[k]);   // s = 64
#pragma unroll
            for (int k = 0; k < 8; k++) p[k] = p[k] + dpp_f<0x104>(p[k]);   // s = 32
        } else if constexpr (D == 128) {
#pragma unroll
            for (int k = 0; k < 8; k++) p[k] = fabsf(x[k]) + fabsf(dpp_f<0x108>(x[k]));   // s = 64
#pragma unroll
            for (int k = 0; k < 8; k++) p[k] = p[k] + dpp_f<0x104>(p[k]);   // s = 32
        } else {
#pragma unroll
            for (int k = 0; k < 8; k++) p[k] = fabsf(x[k]) + fabsf(dpp_f<0x104>(x[k]));   // s = 32
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
        const float total_abs = swz_f<BCAST>(p[0]);
        mean = total_abs / (float)D;
        if constexpr (MODE == ENC_FUSED_FP16) s = h2f(f2h(mean));
        else s = mean;
        // sign bytes of 4 lanes -> one little-endian word
        const uint32_t w = byte | (dpp_u<0x101>(byte) << 8) | (dpp_u<0x102>(byte) << 16) |
                           (dpp_u<0x103>(byte) << 24);
        if (live) {
            if ((j & 3) == 0) ((uint32_t*)(dst.sign_plane + dv * (D / 8)))[j >> 2] = w;
            if (j == 0) dst.scale_plane[dv] = f2h(mean);
        }
    }

    if constexpr (MODE != ENC_BINARY) {
        if (dst.code_plane == nullptr) return;
        float r[8];
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            r[k] = x[k] - (((byte >> k) & 1u) ? s : -s);
            m = fmaxf(m, fabsf(r[k]));
        }
        // fmaxf ignores NaN and is order independent (src/residual.cu:30-53).
        // m is a non-negative float, never NaN (the chain starts at 0 and
        // fmaxf drops NaN operands), and for those the integer order of the
        // bits is the float order: the lanes merge with integer max
        uint32_t mb = __builtin_bit_cast(uint32_t, m);
        if constexpr (L == 8) {
            mb = max(mb, dpp_u<0x141>(mb));   // half mirror
            mb = max(mb, dpp_u<0x4E>(mb));    // quad 2,3,0,1
            mb = max(mb, dpp_u<0xB1>(mb));    // quad 1,0,3,2
        } else {
            mb = max(mb, dpp_u<0x128>(mb));   // row rotations
            mb = max(mb, dpp_u<0x124>(mb));
            mb = max(mb, dpp_u<0x122>(mb));
            mb = max(mb, dpp_u<0x121>(mb));
            if constexpr (L == 32)
                mb = max(mb, (uint32_t)__builtin_amdgcn_ds_swizzle((int)mb, 0x401F));
        }
        const float absmax = __builtin_bit_cast(float, mb);
        const float inv = absmax > 0.0f ? 7.0f / absmax : 0.0f;
        float y[8];
#pragma unroll
        for (int k = 0; k < 8; k++) y[k] = r[k] * inv;
        // Every y is finite (and within 7(1 + 2^-23) in magnitude, since
        // |r| <= absmax) when every x is finite and inv is finite: the x are
        // then finite, so are s and r.  The packed fp16 sum of the eight x is
        // finite only if each x is (an overflow merely sends the lanes to the
        // exact path).
        typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
        const h2_t hs = (__builtin_bit_cast(h2_t, hw[0]) + __builtin_bit_cast(h2_t, hw[1])) +
                        (__builtin_bit_cast(h2_t, hw[2]) + __builtin_bit_cast(h2_t, hw[3]));
        const bool finite = __builtin_isfinite(hs[0]) && __builtin_isfinite(hs[1]) &&
                            __builtin_isfinite(inv);
        uint32_t word = 0;
        if (__ballot(!finite) == 0ull) {
            // clamp to [-7, 7], then round half to even by adding 1.5 * 2^23
            // (unit in the last place 1): the low nibble of the sum's bits
            // is the code in two's complement, as quant7 gives it
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float c = __builtin_amdgcn_fmed3f(y[k], -7.0f, 7.0f) + 12582912.0f;
                word |= (__builtin_bit_cast(uint32_t, c) & 0xFu) << (4 * k);
            }
        } else {
#pragma unroll
            for (int k = 0; k < 8; k++) word |= ((uint32_t)quant7(y[k]) & 0xFu) << (4 * k);
        }
        if (live) {
            ((uint32_t*)(dst.code_plane + dv * (D / 2)))[j] = word;
            if (j == 0) dst.rscale_plane[dv] = f2h(absmax);
        }
    }
}

template <int D, int MODE>
__device__ __forceinline__ void encode_row(const uint16_t* vec, int j, bool live, const EncodeDst& dst,
                                           int64_t dv) {
    encode_row_slice<D, MODE>(load_row_slice(vec, j), j, live, dst, dv);
}

}  // namespace bc
