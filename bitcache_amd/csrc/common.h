// Shared device/host helpers for the bitcache gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bitcache.h"

#define BC_WAVE 64
#define BC_MAX_HEAD_DIM 256

// ---------------------------------------------------------------- error state
namespace bc {

int set_error(int status, const char* fmt, ...);
int check_launch(const char* what);

inline bool head_dim_ok(int d) { return d >= 32 && d <= BC_MAX_HEAD_DIM && (d % 32) == 0; }

// CU count of the current device (cached per device).
int device_cu_count();

}  // namespace bc

#define BC_REQUIRE(cond, status, ...)                   \
    do {                                                \
        if (!(cond)) return bc::set_error(status, __VA_ARGS__); \
    } while (0)

// ---------------------------------------------------------------- blob layout
// Dense planar blob of capacity n vectors (see include/bitcache.h).
struct BinPlanes {
    const uint8_t* signs;    // n * d/8 bytes
    const uint16_t* scales;  // n fp16
};
struct ResPlanes {
    const uint8_t* codes;    // n * d/2 bytes
    const uint16_t* scales;  // n fp16
};

__host__ __device__ inline BinPlanes bin_planes(const void* blob, int64_t cap, int d) {
    const uint8_t* p = (const uint8_t*)blob;
    return BinPlanes{p, (const uint16_t*)(p + cap * (d / 8))};
}
__host__ __device__ inline ResPlanes res_planes(const void* blob, int64_t cap, int d) {
    const uint8_t* p = (const uint8_t*)blob;
    return ResPlanes{p, (const uint16_t*)(p + cap * (d / 2))};
}

// ---------------------------------------------------------------- device helpers
__device__ __forceinline__ float h2f(uint16_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, h);
    return (float)v;
}
// round-to-nearest-even fp32 -> fp16 (v_cvt_f16_f32 in the default rounding mode)
__device__ __forceinline__ uint16_t f2h(float f) {
    _Float16 v = (_Float16)f;
    return __builtin_bit_cast(uint16_t, v);
}

// Lane moves without LDS traffic: DPP (row_shl / row_ror / quad_perm /
// mirrors, within 16-lane rows) and ds_swizzle (within 32-lane halves).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                  0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}
template <int PAT>
__device__ __forceinline__ float swz_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), PAT));
}

// Wave-wide max / sum, every lane gets the result: row rotations, then the
// two rows of each half (swizzle xor 16), then the two halves (readlane).
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0x128>(v));
    v = fmaxf(v, dpp_f<0x124>(v));
    v = fmaxf(v, dpp_f<0x122>(v));
    v = fmaxf(v, dpp_f<0x121>(v));
    v = fmaxf(v, swz_f<0x401F>(v));
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    return fmaxf(a, b);
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0x128>(v);
    v += dpp_f<0x124>(v);
    v += dpp_f<0x122>(v);
    v += dpp_f<0x121>(v);
    v += swz_f<0x401F>(v);
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    return a + b;
}
__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// Sign-word loaders: D/8 bytes per vector, returned as D/32 uint32 words.
template <int D>
struct SignWords {
    uint32_t w[D / 32];
};
typedef unsigned int bc_v4u __attribute__((ext_vector_type(4)));
typedef unsigned int bc_v2u __attribute__((ext_vector_type(2)));

// NT: nontemporal loads (for streams read once, whole lines per instruction)
template <int D, bool NT = false>
__device__ __forceinline__ SignWords<D> load_signs(const uint8_t* p) {
    // D/8 bytes at a D/8-byte aligned address: 16-byte loads where the stride allows
    SignWords<D> s;
    if constexpr (D % 128 == 0) {
#pragma unroll
        for (int i = 0; i < D / 128; i++) {
            const bc_v4u v = NT ? __builtin_nontemporal_load((const bc_v4u*)p + i) : ((const bc_v4u*)p)[i];
            s.w[4 * i + 0] = v[0]; s.w[4 * i + 1] = v[1]; s.w[4 * i + 2] = v[2]; s.w[4 * i + 3] = v[3];
        }
    } else if constexpr (D % 64 == 0) {
#pragma unroll
        for (int i = 0; i < D / 64; i++) {
            const bc_v2u v = NT ? __builtin_nontemporal_load((const bc_v2u*)p + i) : ((const bc_v2u*)p)[i];
            s.w[2 * i + 0] = v[0]; s.w[2 * i + 1] = v[1];
        }
    } else {
#pragma unroll
        for (int i = 0; i < D / 32; i++)
            s.w[i] = NT ? __builtin_nontemporal_load((const uint32_t*)p + i) : ((const uint32_t*)p)[i];
    }
    return s;
}

// Order-preserving map of an fp32 key to uint32 (larger float -> larger uint).
// -0 is folded into +0 and NaN into -inf before the map.
__device__ __forceinline__ uint32_t ordered_key(float f) {
    f = f + 0.0f;
    if (!(f == f)) f = -INFINITY;
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Ranking scores of the top-k selection in the float domain.  For a finite
// scale, fma(pc, 2 scale, -d scale) is exactly scale * (2pc - d) (at most 20
// significant bits), never -0 and never NaN; on such scores the order of
// ordered_key() is the float order, so a bound on keys is a float bound:
//   ordered_key(s) <= T  <=>  s <= key_floor(T)
//   ordered_key(s) == T  <=>  s == key_value(T)   (NaN: no such score)
// key_floor(T) is the largest float that is not -0 or NaN whose key is <= T
// (-inf when there is none, since every such score is finite).
__host__ __device__ inline float key_floor(uint32_t T) {
    if (T >= 0xFF800000u) return INFINITY;    // the key of +inf, or a NaN's
    if (T < 0x007FFFFFu) return -INFINITY;    // below the key of -inf (NaNs)
    const uint32_t bits = (T & 0x80000000u) ? (T & 0x7FFFFFFFu) : ~T;
    // -0 never occurs: the next float below it
    return __builtin_bit_cast(float, bits == 0x80000000u ? 0x80000001u : bits);
}
__host__ __device__ inline float key_value(uint32_t T) {
    if (T > 0xFF800000u || T < 0x007FFFFFu || T == 0x7FFFFFFFu) return __builtin_nanf("");
    return __builtin_bit_cast(float, (T & 0x80000000u) ? (T & 0x7FFFFFFFu) : ~T);
}
// ordered_key() of a score that is not NaN or -0 (no folding needed)
__device__ __forceinline__ uint32_t ordered_bits(float s) {
    const uint32_t u = __builtin_bit_cast(uint32_t, s);
    return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
}
__device__ __forceinline__ bool finite_scale(float sk) { return __builtin_fabsf(sk) < INFINITY; }

