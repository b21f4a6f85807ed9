// q8_rope.hip - fused rotary embedding + Q8_0 K/V cache write for gfx950.
//
// One launch does what the unfused path does in two (the rotary-embedding op
// on query and key, then gfx906_fa_amd_cache_write_kv): it rotates query and
// key in place and quantizes the rotated key and the value into the planar
// Q8_0 cache at slot_mapping.  The reference backend declares no such fusion
// (extension/gfx906_fa_backend.py:444-445 returns False).
//
// Rotary semantics are those of vLLM's rotary embedding (the native torch
// form and the device kernel agree): cos and sin are taken from
// cos_sin_cache[position] (cos in columns [0, rot/2), sin in [rot/2, rot))
// and converted to the model dtype, then for each rotated pair (x, y)
//     x' = x*cos - y*sin,  y' = y*cos + x*sin
// with every product, difference and sum rounded to the model dtype (fp16 /
// bf16), i.e. computed in fp32 and rounded after each operation.  Pairs are
// (i, i + rot/2) in the neox style and (2i, 2i+1) otherwise; dims >= rot are
// left as they are.  The quantized key is the rotated key as stored, so the
// fused op is bit-identical to rotating, storing and then writing the cache.
//
// Work mapping: a wave takes 32 of one token's rows (query heads, then key
// heads), four at a time, one per 16-lane row of the wave, 8 values (16
// bytes) per lane; the lane's cos / sin are loaded once for all of them.  A
// Q8_0 block (32 values) is one lane quad, so its amax is two DPP steps; the
// neox partner of a lane's 8 values sits in the same 16-lane row (one
// ds_bpermute per dword).
#include <cstdio>

#include "q8_common.h"

using namespace gfa;

// No floating-point contraction anywhere in this file: every product, sum and
// difference of the rotation is rounded on its own (a fused multiply-add
// would skip the product's rounding).
#pragma clang fp contract(off)

namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// model-dtype element bits -> fp32 (exact)
template <int DT>
__device__ __forceinline__ float el_to_f32(uint32_t bits) {
    if constexpr (DT == GFA_DTYPE_F16) return half_bits_to_f32(bits);
    else return bf16_bits_to_f32(bits);
}

// fp32 -> model dtype, round to nearest even (finite inputs)
template <int DT>
__device__ __forceinline__ uint32_t f32_to_el(float v) {
    if constexpr (DT == GFA_DTYPE_F16) {
        return f32_to_half_bits(v);
    } else {
        const uint32_t u = __float_as_uint(v);
        return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
    }
}

// one rounding to the model dtype, back in fp32
template <int DT>
__device__ __forceinline__ float rnd(float v) {
    return el_to_f32<DT>(f32_to_el<DT>(v));
}

// x*y, x-y, x+y of model-dtype values, rounded to the model dtype.  fp16
// uses the IEEE fp16 operations (a fp32 operation rounded to fp16 gives the
// same value, fp32 having more than 2*11+2 bits, and the fp16 instruction
// keeps the sign of a zero product, which a multiply selected as an fma
// with +0 would lose); bf16 rounds the fp32 result.
template <int DT>
struct RoundedOps {
    static __device__ __forceinline__ float mul(float x, float y) { return rnd<DT>(x * y); }
    static __device__ __forceinline__ float sub(float x, float y) { return rnd<DT>(x - y); }
    static __device__ __forceinline__ float add(float x, float y) { return rnd<DT>(x + y); }
};
template <>
struct RoundedOps<GFA_DTYPE_F16> {
    static __device__ __forceinline__ float mul(float x, float y) { return (float)((half_t)x * (half_t)y); }
    static __device__ __forceinline__ float sub(float x, float y) { return (float)((half_t)x - (half_t)y); }
    static __device__ __forceinline__ float add(float x, float y) { return (float)((half_t)x + (half_t)y); }
};

// 8 consecutive values of a 16-byte aligned row chunk as fp32
template <int DT>
__device__ __forceinline__ void load8(const void *p, float (&v)[8]) {
    const u32x4_t w = *reinterpret_cast<const u32x4_t *>(p);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        v[2 * e] = el_to_f32<DT>(w[e] & 0xFFFFu);
        v[2 * e + 1] = el_to_f32<DT>(w[e] >> 16);
    }
}

template <int DT>
__device__ __forceinline__ void store8(void *p, const float (&v)[8]) {
    u32x4_t w;
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = f32_to_el<DT>(v[2 * e]) | (f32_to_el<DT>(v[2 * e + 1]) << 16);
    *reinterpret_cast<u32x4_t *>(p) = w;
}

// n (4 or 8) consecutive cos or sin values of the cache row, converted to
// the model dtype (the native form's cos.to(x.dtype)); 8-byte aligned
template <int DT, int CSDT, int N>
__device__ __forceinline__ void load_cs(const void *row, int col, float (&v)[8]) {
    if constexpr (CSDT == GFA_DTYPE_F32) {
        const float *p = static_cast<const float *>(row) + col;
#pragma unroll
        for (int e = 0; e < N; e += 2) {
            const float2 f = *reinterpret_cast<const float2 *>(p + e);
            v[e] = rnd<DT>(f.x);
            v[e + 1] = rnd<DT>(f.y);
        }
    } else {
        const uint16_t *p = static_cast<const uint16_t *>(row) + col;
#pragma unroll
        for (int e = 0; e < N; e += 2) {
            const uint32_t w = *reinterpret_cast<const uint32_t *>(p + e);
            // a cache in the other 16-bit type is rounded to the model dtype
            v[e] = rnd<DT>(el_to_f32<CSDT>(w & 0xFFFFu));
            v[e + 1] = rnd<DT>(el_to_f32<CSDT>(w >> 16));
        }
    }
}

// The lane's cos / sin for its 8 columns d0..d0+7 (the same for every head
// of a token): neox - the pair index of column d is d mod rot/2; GPT-J - the
// lane's 4 pairs are d0/2 .. d0/2+3.
template <int DT, int CSDT, bool NEOX>
__device__ __forceinline__ void load_lane_cs(const void *csrow, int d0, int rot, float (&c)[8], float (&s)[8]) {
    const int half = rot >> 1;
    if (d0 >= rot) return;
    if constexpr (NEOX) {
        const int col = d0 < half ? d0 : d0 - half;
        load_cs<DT, CSDT, 8>(csrow, col, c);
        load_cs<DT, CSDT, 8>(csrow, half + col, s);
    } else {
        load_cs<DT, CSDT, 4>(csrow, d0 >> 1, c);
        load_cs<DT, CSDT, 4>(csrow, half + (d0 >> 1), s);
    }
}

// Rotates the lane's 8 values v (row columns d0..d0+7) in place.  Every
// lane of the 16-lane row takes part (the neox partner exchange).
template <int DT, bool NEOX>
__device__ __forceinline__ void rope8(float (&v)[8], const float (&c)[8], const float (&s)[8], int d0,
                                      int rot, int lane) {
    using M = RoundedOps<DT>;
    const int half = rot >> 1;
    if constexpr (NEOX) {
        // partner columns d0 +- half live 16-lane-row locally at lane +- half/8
        const int src = d0 < half ? lane + (half >> 3) : (d0 < rot ? lane - (half >> 3) : lane);
        uint32_t pw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            pw[e] = (uint32_t)__shfl((int)(f32_to_el<DT>(v[2 * e]) | (f32_to_el<DT>(v[2 * e + 1]) << 16)), src);
        if (d0 >= rot) return;  // uniform over the lane's 8 values (rot % 16 == 0)
        const bool xpart = d0 < half;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float p = el_to_f32<DT>(e & 1 ? pw[e >> 1] >> 16 : pw[e >> 1] & 0xFFFFu);
            if (xpart) v[e] = M::sub(M::mul(v[e], c[e]), M::mul(p, s[e]));  // x' = x c - y s
            else v[e] = M::add(M::mul(v[e], c[e]), M::mul(p, s[e]));        // y' = y c + x s
        }
    } else {
        if (d0 >= rot) return;  // rot % 8 == 0: the lane's 4 pairs are all rotated or all not
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float x = v[2 * j], y = v[2 * j + 1];
            v[2 * j] = M::sub(M::mul(x, c[j]), M::mul(y, s[j]));
            v[2 * j + 1] = M::add(M::mul(y, c[j]), M::mul(x, s[j]));
        }
    }
}

// Q8_0 closed form over the lane quad's 32 values (8 per lane), packed as
// two dwords of int8; returns the block scale d.
__device__ __forceinline__ float quant8(const float (&v)[8], uint32_t &lo, uint32_t &hi) {
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
    amax = fmaxf(amax, dpp_f32<DPP_QUAD_XOR1>(amax));
    amax = fmaxf(amax, dpp_f32<DPP_QUAD_XOR2>(amax));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    lo = hi = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        int qi = (int)rintf(v[e] * id);
        qi = qi < -128 ? -128 : (qi > 127 ? 127 : qi);
        if (e < 4) lo |= (uint32_t)(uint8_t)qi << (8 * e);
        else hi |= (uint32_t)(uint8_t)qi << (8 * (e - 4));
    }
    return d;
}

struct RopeArgs {
    void *q;
    void *k;
    const void *v;
    const int64_t *pos;
    const void *cs;
    const int64_t *slot;
    uint8_t *kc, *vc;
    int64_t qts, qhs, kts, khs, vts, vhs, cs_stride, cbs, chs;
    int64_t num_tokens;
    int Hq, Hkv, rot, block_size, max_pos, nchunk;
};

#ifndef GFA_ROPE_ITERS
#define GFA_ROPE_ITERS 8
#endif
constexpr int ROPE_ITERS = GFA_ROPE_ITERS;  // row quads per wave: 8 x 4 = 32 rows

// Wave (token t, chunk c) takes the token's rows 32c .. 32c+31 of the list
// [Hq query heads, Hkv key heads]: iteration it, lane row g -> row
// 32c + 4it + g (32 rows per wave measured 4 % faster than 16 and 56).
// At least 4 waves per SIMD: left to itself the compiler gives the fp16
// instantiations 234-238 VGPRs (one wave per SIMD, half the bf16 rate); at
// this bound both dtypes fit 104-114 with no spills.
template <int DT, int CSDT, bool NEOX>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void q8_rope_cache_write_kernel(RopeArgs a) {
    const int64_t wave = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int i = lane & 15, g = lane >> 4;
    const int d0 = 8 * i;
    const int64_t t = wave / a.nchunk;
    if (t >= a.num_tokens) return;  // uniform over the wave
    const int c0 = 4 * ROPE_ITERS * (int)(wave - t * a.nchunk);
    const int R = a.Hq + a.Hkv;
    // the rows of every iteration are loaded first (they depend on nothing),
    // then the position, the slot and the lane's cos / sin
    u32x4_t xw[ROPE_ITERS], vw[ROPE_ITERS];
#pragma unroll
    for (int it = 0; it < ROPE_ITERS; ++it) {
        xw[it] = u32x4_t{0, 0, 0, 0};
        vw[it] = u32x4_t{0, 0, 0, 0};
        const int row = c0 + 4 * it + g;
        if (row < a.Hq) {
            xw[it] = *reinterpret_cast<const u32x4_t *>(static_cast<const uint16_t *>(a.q) + t * a.qts +
                                                      (int64_t)row * a.qhs + d0);
        } else if (row < R) {
            const int h = row - a.Hq;
            xw[it] = *reinterpret_cast<const u32x4_t *>(static_cast<const uint16_t *>(a.k) + t * a.kts +
                                                      (int64_t)h * a.khs + d0);
            vw[it] = *reinterpret_cast<const u32x4_t *>(static_cast<const uint16_t *>(a.v) + t * a.vts +
                                                      (int64_t)h * a.vhs + d0);
        }
    }
    const int64_t pos = a.pos[t];
    const int64_t slot = a.slot[t];
    const bool in_range = pos >= 0 && pos < a.max_pos;  // others stay unrotated
    float cs_c[8], cs_s[8];
    if (in_range) {
        const void *csrow = static_cast<const char *>(a.cs) + pos * a.cs_stride * (CSDT == GFA_DTYPE_F32 ? 4 : 2);
        load_lane_cs<DT, CSDT, NEOX>(csrow, d0, a.rot, cs_c, cs_s);
    }
#pragma unroll
    for (int it = 0; it < ROPE_ITERS; ++it) {
        if (c0 + 4 * it >= R) break;  // uniform: no row of this iteration exists
        const int row = c0 + 4 * it + g;
        const bool active = row < R;  // the same for the 16 lanes of a row
        const bool is_q = row < a.Hq;
        float x[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[2 * e] = el_to_f32<DT>(xw[it][e] & 0xFFFFu);
            x[2 * e + 1] = el_to_f32<DT>(xw[it][e] >> 16);
        }
        if (in_range) {
            rope8<DT, NEOX>(x, cs_c, cs_s, d0, a.rot, lane);
            if (active && d0 < a.rot) {
                uint16_t *dst = is_q ? static_cast<uint16_t *>(a.q) + t * a.qts + (int64_t)row * a.qhs + d0
                                     : static_cast<uint16_t *>(a.k) + t * a.kts + (int64_t)(row - a.Hq) * a.khs + d0;
                store8<DT>(dst, x);
            }
        }
        if (!active || is_q) continue;

        // the rotated key and the value as Q8_0 into the planar sub-page of slot
        float vv[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            vv[2 * e] = el_to_f32<DT>(vw[it][e] & 0xFFFFu);
            vv[2 * e + 1] = el_to_f32<DT>(vw[it][e] >> 16);
        }
        uint32_t klo, khi, vlo, vhi;
        const float dk = quant8(x, klo, khi);
        const float dv = quant8(vv, vlo, vhi);
        if (slot < 0) continue;
        const int h = row - a.Hq;
        const int64_t page = slot / a.block_size;
        const int off = (int)(slot - page * a.block_size);
        const int sp = off >> 4, tt = off & 15;
        const int64_t base = page * a.cbs + (int64_t)h * a.chs + (int64_t)sp * SUBPAGE_BYTES;
        const int b = d0 >> 5, kg = (d0 >> 3) & 3;
        *reinterpret_cast<u32x2 *>(a.kc + base + (b >> 1) * 1024 + (4 * tt + kg) * 16 + (b & 1) * 8) =
            u32x2{klo, khi};
        const int m = d0 >> 4;
        uint8_t *vrow = a.vc + base + (m >> 2) * 1024 + (tt >> 2) * 256 + (tt & 3) + (m & 3) * 4 + (d0 & 15) * 16;
#pragma unroll
        for (int e = 0; e < 8; ++e) vrow[e * 16] = (uint8_t)((e < 4 ? vlo : vhi) >> (8 * (e & 3)));
        if ((i & 3) == 0) {
            *reinterpret_cast<uint16_t *>(a.kc + base + SCALE_OFF + (4 * tt + b) * 2) = f32_to_half_bits(dk);
            *reinterpret_cast<uint16_t *>(a.vc + base + SCALE_OFF + ((tt >> 2) * 4 + b) * 8 + (tt & 3) * 2) =
                f32_to_half_bits(dv);
        }
    }
}

template <int DT, int CSDT>
void launch_rope(const RopeArgs &a, bool neox, unsigned grid, hipStream_t stream) {
    if (neox) q8_rope_cache_write_kernel<DT, CSDT, true><<<grid, 256, 0, stream>>>(a);
    else q8_rope_cache_write_kernel<DT, CSDT, false><<<grid, 256, 0, stream>>>(a);
}

}  // namespace

extern "C" hipError_t gfx906_fa_amd_rope_cache_write_kv(
    void *query, void *key, const void *value, int dtype, const int64_t *positions,
    const void *cos_sin_cache, int cos_sin_dtype, int64_t cos_sin_stride, int max_position,
    int rot_dim, int is_neox, const int64_t *slot_mapping, uint8_t *k_cache, uint8_t *v_cache,
    int num_tokens, int num_heads, int num_kv_heads, int head_size, int block_size,
    int64_t query_token_stride, int64_t query_head_stride, int64_t key_token_stride,
    int64_t key_head_stride, int64_t value_token_stride, int64_t value_head_stride,
    int64_t cache_block_stride, int64_t cache_head_stride, hipStream_t stream) {
    if (head_size != 128 || block_size <= 0 || block_size % SUBPAGE != 0 || num_heads <= 0 ||
        num_kv_heads <= 0 || num_tokens < 0 || (dtype != GFA_DTYPE_F16 && dtype != GFA_DTYPE_BF16) ||
        cos_sin_dtype < 0 || cos_sin_dtype > 2 || max_position <= 0) {
        fprintf(stderr,
                "[gfx906_fa_amd] rope_cache_write_kv: need head_size 128, block_size %% 16 == 0, "
                "fp16/bf16 query/key/value, max_position > 0 (got head_size=%d block_size=%d dtype=%d)\n",
                head_size, block_size, dtype);
        return hipErrorInvalidValue;
    }
    if (rot_dim <= 0 || rot_dim > head_size || rot_dim % (is_neox ? 16 : 8) != 0 ||
        cos_sin_stride < rot_dim) {
        fprintf(stderr,
                "[gfx906_fa_amd] rope_cache_write_kv: rot_dim=%d must be in (0, 128], a multiple of %d, "
                "and <= the cos_sin row stride (%lld)\n",
                rot_dim, is_neox ? 16 : 8, (long long)cos_sin_stride);
        return hipErrorInvalidValue;
    }
    // 16-byte row chunks for query / key / value, 8-byte cos / sin pairs and
    // cache stores
    const uint64_t e16 = (uint64_t)(query_token_stride | query_head_stride | key_token_stride |
                                    key_head_stride | value_token_stride | value_head_stride);
    const int cs_esz = cos_sin_dtype == GFA_DTYPE_F32 ? 4 : 2;
    if ((((uintptr_t)query | (uintptr_t)key | (uintptr_t)value) & 15u) || (e16 & 7u) ||
        (((uintptr_t)cos_sin_cache | (uint64_t)(cos_sin_stride * cs_esz)) & 7u) ||
        (((uintptr_t)k_cache | (uintptr_t)v_cache | (uint64_t)cache_block_stride |
          (uint64_t)cache_head_stride) & 7u)) {
        fprintf(stderr,
                "[gfx906_fa_amd] rope_cache_write_kv: query/key/value rows must start 16-byte aligned "
                "(bases 16-aligned, strides multiples of 8 elements), cos_sin rows and the cache 8-aligned\n");
        return hipErrorInvalidValue;
    }
    if (num_tokens == 0) return hipSuccess;
    RopeArgs a;
    a.q = query;
    a.k = key;
    a.v = value;
    a.pos = positions;
    a.cs = cos_sin_cache;
    a.slot = slot_mapping;
    a.kc = k_cache;
    a.vc = v_cache;
    a.qts = query_token_stride;
    a.qhs = query_head_stride;
    a.kts = key_token_stride;
    a.khs = key_head_stride;
    a.vts = value_token_stride;
    a.vhs = value_head_stride;
    a.cs_stride = cos_sin_stride;
    a.cbs = cache_block_stride;
    a.chs = cache_head_stride;
    a.num_tokens = num_tokens;
    a.nchunk = (num_heads + num_kv_heads + 4 * ROPE_ITERS - 1) / (4 * ROPE_ITERS);
    a.Hq = num_heads;
    a.Hkv = num_kv_heads;
    a.rot = rot_dim;
    a.block_size = block_size;
    a.max_pos = max_position;
    const int64_t waves = (int64_t)num_tokens * a.nchunk;
    const int64_t blocks = (waves + 3) / 4;
    if (blocks > 0x7FFFFFFF) {
        fprintf(stderr, "[gfx906_fa_amd] rope_cache_write_kv: too many rows\n");
        return hipErrorInvalidValue;
    }
    const unsigned grid = (unsigned)blocks;
    const bool neox = is_neox != 0;
#define GFA_ROPE_CS(DT)                                                     \
    switch (cos_sin_dtype) {                                                \
        case GFA_DTYPE_F32: launch_rope<DT, GFA_DTYPE_F32>(a, neox, grid, stream); break; \
        case GFA_DTYPE_F16: launch_rope<DT, GFA_DTYPE_F16>(a, neox, grid, stream); break; \
        default: launch_rope<DT, GFA_DTYPE_BF16>(a, neox, grid, stream); break;           \
    }
    if (dtype == GFA_DTYPE_F16) {
        GFA_ROPE_CS(GFA_DTYPE_F16)
    } else {
        GFA_ROPE_CS(GFA_DTYPE_BF16)
    }
#undef GFA_ROPE_CS
    return hipGetLastError();
}
