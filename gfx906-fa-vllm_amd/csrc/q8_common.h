// q8_common.h - device helpers shared by the gfx950 Q8_0 kernels.
//
// Wave64 throughout.  Cross-lane work uses DPP inside 16-lane rows and the
// gfx950 permlane16/32 swaps across rows; nothing here goes through LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gfx906_fa_amd.h"

namespace gfa {

constexpr int QK = 32;          // values per Q8_0 block
constexpr int QBYTES = 34;      // fp16 scale + 32 int8
constexpr int SUBPAGE = 16;     // tokens per planar sub-page
constexpr int SUBPAGE_BYTES = 2176;
constexpr int SCALE_OFF = 2048; // scale table offset inside a sub-page

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
    return __uint_as_float(b << 16);
}

__device__ __forceinline__ float half_bits_to_f32(uint32_t b) {
    half_t h = __builtin_bit_cast(half_t, (uint16_t)b);
    return (float)h;
}

// Element load from an fp32 / fp16 / bf16 array, exact widening to fp32.
template <int DT>
__device__ __forceinline__ float load_as_f32(const void *p, int64_t i) {
    if constexpr (DT == GFA_DTYPE_F32) {
        return static_cast<const float *>(p)[i];
    } else if constexpr (DT == GFA_DTYPE_F16) {
        return half_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
    } else {
        return bf16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
    }
}

// Two consecutive elements (i, i+1); i even and the base 4-byte aligned for
// the 16-bit types.
template <int DT>
__device__ __forceinline__ void load2_as_f32(const void *p, int64_t i, float &a, float &b) {
    if constexpr (DT == GFA_DTYPE_F32) {
        const float2 v = *reinterpret_cast<const float2 *>(static_cast<const float *>(p) + i);
        a = v.x;
        b = v.y;
    } else {
        const uint32_t w = *reinterpret_cast<const uint32_t *>(static_cast<const uint16_t *>(p) + i);
        if constexpr (DT == GFA_DTYPE_F16) {
            a = half_bits_to_f32(w & 0xFFFFu);
            b = half_bits_to_f32(w >> 16);
        } else {
            a = bf16_bits_to_f32(w & 0xFFFFu);
            b = bf16_bits_to_f32(w >> 16);
        }
    }
}

// DPP controls (GFX9 encoding).
constexpr int DPP_QUAD_XOR1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// max over the 16 lanes of a DPP row; every lane of the row gets the result.
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_f32<DPP_QUAD_XOR1>(v));
    v = fmaxf(v, dpp_f32<DPP_QUAD_XOR2>(v));
    v = fmaxf(v, dpp_f32<DPP_ROW_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f32<DPP_ROW_MIRROR>(v));
    return v;
}

// Combine lane i with lane i^16 and lane i^32 (the four 16-lane rows).
__device__ __forceinline__ float xrow_max(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float xrow_sum(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Q8_0 closed form for the two values (a, b) a lane holds of a 32-value
// block spread over one 16-lane DPP row (extension/gfx906_fa_quant.cu:45-85):
//   amax = max|x|; d = amax/127.f; id = d > 0 ? 1.f/d : 0;
//   q = clamp((int)rintf(x*id), -128, 127).
// Division and reciprocal are IEEE correctly rounded (no fast-math in this
// build); rintf rounds half to even; (int) of +-inf saturates and of NaN is 0
// on this hardware, matching the reference kernel's conversion.
struct Q8Pair {
    int8_t qa, qb;
    float d;
};

__device__ __forceinline__ Q8Pair q8_quantize_pair(float a, float b) {
    float amax = row16_max(fmaxf(fabsf(a), fabsf(b)));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    int qa = (int)rintf(a * id);
    int qb = (int)rintf(b * id);
    qa = qa < -128 ? -128 : (qa > 127 ? 127 : qa);
    qb = qb < -128 ? -128 : (qb > 127 ? 127 : qb);
    Q8Pair r;
    r.qa = (int8_t)qa;
    r.qb = (int8_t)qb;
    r.d = d;
    return r;
}

__device__ __forceinline__ uint16_t f32_to_half_bits(float d) {
    half_t h = (half_t)d;  // v_cvt_f16_f32, round to nearest even
    return __builtin_bit_cast(uint16_t, h);
}

// Stores the Q8_0 K and V values a lane holds of one token row (columns
// d0 = 2*lane and d0+1, from q8_quantize_pair) into a planar K and V
// sub-page at token tt, plus the block scales from the first lane of each
// 16-lane row:
//   K ints  at (b/2)*1024 + (4tt + g)*16 + (b%2)*8 + d%8   (b = d/32, g = (d%32)/8)
//   V ints  at (m/4)*1024 + ((tt/4)*16 + d%16)*16 + (m%4)*4 + tt%4   (m = d/16)
//   scales  K at 2048 + (4tt + b)*2, V at 2048 + ((tt/4)*4 + b)*8 + (tt%4)*2
__device__ __forceinline__ void planar_store_pair(uint8_t *ksub, uint8_t *vsub, int tt, int lane,
                                                  const Q8Pair &rk, const Q8Pair &rv) {
    const int d0 = 2 * lane;
    const int b = lane >> 4;
    const int kpos = (b >> 1) * 1024 + (4 * tt + ((d0 >> 3) & 3)) * 16 + (b & 1) * 8 + (d0 & 7);
    *reinterpret_cast<uint16_t *>(ksub + kpos) = (uint16_t)((uint8_t)rk.qa | ((uint16_t)(uint8_t)rk.qb << 8));
    const int m = d0 >> 4;
    const int vrow = (m >> 2) * 1024 + ((tt >> 2) * 16) * 16 + (m & 3) * 4 + (tt & 3);
    vsub[vrow + (d0 & 15) * 16] = (uint8_t)rv.qa;
    vsub[vrow + ((d0 + 1) & 15) * 16] = (uint8_t)rv.qb;
    if ((lane & 15) == 0) {
        *reinterpret_cast<uint16_t *>(ksub + SCALE_OFF + (4 * tt + b) * 2) = f32_to_half_bits(rk.d);
        *reinterpret_cast<uint16_t *>(vsub + SCALE_OFF + ((tt >> 2) * 4 + b) * 8 + (tt & 3) * 2) =
            f32_to_half_bits(rv.d);
    }
}

// 4 int8 (one dword) -> 4 exact fp16 values as two packed pairs.
// u = q ^ 0x80 is q + 128 as an unsigned byte; fp16 bits 0x6400|u encode
// 1024 + u exactly, and subtracting 1152 leaves q exactly.
__device__ __forceinline__ void i8x4_to_f16x4(uint32_t w, half2_t &lo, half2_t &hi) {
    const uint32_t u = w ^ 0x80808080u;
    // v_perm_b32: selector bytes 0..3 pick from src1, 4..7 from src0.
    const uint32_t plo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // [u0,64,u1,64]
    const uint32_t phi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // [u2,64,u3,64]
    const half2_t bias = {(half_t)-1152.0f, (half_t)-1152.0f};
    lo = __builtin_bit_cast(half2_t, plo) + bias;
    hi = __builtin_bit_cast(half2_t, phi) + bias;
}

// 8 int8 (two dwords) -> half8 exact.
__device__ __forceinline__ half8_t i8x8_to_half8(uint32_t w0, uint32_t w1) {
    half2_t a, b, c, d;
    i8x4_to_f16x4(w0, a, b);
    i8x4_to_f16x4(w1, c, d);
    half8_t r;
    r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
    r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
    return r;
}

}  // namespace gfa
