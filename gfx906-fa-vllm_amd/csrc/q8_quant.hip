// q8_quant.hip - Q8_0 quantize and paged cache-write kernels for gfx950.
//
// Work mapping: a Q8_0 block of 32 values lives on one 16-lane DPP row, two
// values per lane, so one wave64 quantizes 4 blocks (one D=128 row) with the
// amax reduction entirely in DPP (no LDS, no barriers).
//
//   q8_dense_kernel          rows [N, D] -> AoS rows          (reference:
//                            extension/gfx906_fa_quant.cu:100-129)
//   q8_reshape_cache_kernel  key rows -> AoS paged cache     (reference:
//                            extension/gfx906_fa_quant.cu:150-200)
//   q8_cache_write_kv_kernel key AND value rows -> planar paged cache (the
//                            backend's hot-path write; no reference kernel
//                            writes V, extension/gfx906_fa.cpp:322-326)
#include <cstdio>

#include "q8_common.h"

using namespace gfa;

namespace {

// ---------------------------------------------------------------------------
// Dense: blocks are consecutive (row-major [N, D] with D % 32 == 0), so the
// input is a flat array of nblk = N*D/32 blocks and the output a flat array of
// nblk 34-byte blocks.  One 16-lane row per block, lane owns values 2i, 2i+1.
template <int DT>
__global__ __launch_bounds__(256) void q8_dense_kernel(const void *__restrict__ x,
                                                      uint8_t *__restrict__ y, int64_t nblk) {
    const int lane16 = threadIdx.x & 15;
    const int64_t blk = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 4;
    // every lane of a 16-lane row shares blk, so rows retire together (the
    // DPP reduction only mixes lanes of the same row).
    if (blk >= nblk) return;
    float a, b;
    load2_as_f32<DT>(x, blk * QK + 2 * lane16, a, b);
    const Q8Pair r = q8_quantize_pair(a, b);
    uint8_t *o = y + blk * QBYTES;
    // 34*blk + 2 + 2*lane16 is even: 16-bit stores are aligned.
    *reinterpret_cast<uint16_t *>(o + 2 + 2 * lane16) =
        (uint16_t)((uint8_t)r.qa | ((uint16_t)(uint8_t)r.qb << 8));
    if (lane16 == 0) *reinterpret_cast<uint16_t *>(o) = f32_to_half_bits(r.d);
}

// ---------------------------------------------------------------------------
// AoS paged write with arbitrary strides (reference contract).  One wave per
// (token, kv-head); each of the 4 DPP rows takes one block per iteration.
// Stores are bytewise so any byte stride works.
template <int DT>
__global__ __launch_bounds__(256) void q8_reshape_cache_kernel(
    const void *__restrict__ key, const int64_t *__restrict__ slot_mapping,
    uint8_t *__restrict__ cache, int num_tokens, int num_kv_heads, int head_size,
    int block_size, int64_t kts, int64_t khs, int64_t cbs, int64_t cts, int64_t chs) {
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (wave >= num_tokens * num_kv_heads) return;
    const int t = wave / num_kv_heads;
    const int h = wave - t * num_kv_heads;
    const int64_t slot = slot_mapping[t];
    if (slot < 0) return;
    const int64_t blk = slot / block_size;
    const int64_t off = slot - blk * block_size;
    const int64_t xb = (int64_t)t * kts + (int64_t)h * khs;
    uint8_t *row = cache + blk * cbs + off * cts + (int64_t)h * chs;
    const int nb = head_size / QK;
    const int lane16 = lane & 15;
    for (int b0 = 0; b0 < nb; b0 += 4) {
        const int b = b0 + (lane >> 4);
        if (b < nb) {  // uniform across the 16-lane row
            const float a = load_as_f32<DT>(key, xb + b * QK + 2 * lane16);
            const float c = load_as_f32<DT>(key, xb + b * QK + 2 * lane16 + 1);
            const Q8Pair r = q8_quantize_pair(a, c);
            uint8_t *o = row + b * QBYTES;
            o[2 + 2 * lane16] = (uint8_t)r.qa;
            o[3 + 2 * lane16] = (uint8_t)r.qb;
            if (lane16 == 0) {
                const uint16_t hb = f32_to_half_bits(r.d);
                o[0] = (uint8_t)(hb & 0xFF);
                o[1] = (uint8_t)(hb >> 8);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Planar K+V write (D = 128).  One wave per (token, kv-head): lane l holds
// dims 2l, 2l+1 of K and of V; block b = l/16 is the lane's DPP row.
//   K ints : u16 store at kpos(t, 2l)   (2l, 2l+1 share an 8-group)
//            kpos(t, d) = (b/2)*1024 + (4t+g)*16 + (b%2)*8 + d%8, b = d/32, g = (d%32)/8
//   V ints : byte stores at vpos(t, 2l), vpos(t, 2l+1)
//            vpos(t, d) = (m/4)*1024 + ((t/4)*16 + d%16)*16 + (m%4)*4 + t%4, m = d/16
//   scales : lane 16b writes fp16 scale[t][b] of K (at 2048 + (4t+b)*2) and
//            of V (at 2048 + ((t/4)*4+b)*8 + (t%4)*2)
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void q8_cache_write_kv_kernel(
    const void *__restrict__ key, const void *__restrict__ value,
    const int64_t *__restrict__ slot_mapping, uint8_t *__restrict__ kc,
    uint8_t *__restrict__ vc, int num_tokens, int num_kv_heads, int block_size,
    int64_t kts, int64_t khs, int64_t vts, int64_t vhs, int64_t cbs, int64_t chs) {
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (wave >= num_tokens * num_kv_heads) return;
    const int t = wave / num_kv_heads;
    const int h = wave - t * num_kv_heads;
    // the row's values are loaded before the slot test (they are valid input
    // rows either way), so the slot and value loads share one memory round trip
    const int d0 = 2 * lane;
    float ka, kb, va, vb;
    if constexpr (VEC) {
        load2_as_f32<DT>(key, (int64_t)t * kts + (int64_t)h * khs + d0, ka, kb);
        load2_as_f32<DT>(value, (int64_t)t * vts + (int64_t)h * vhs + d0, va, vb);
    } else {
        ka = load_as_f32<DT>(key, (int64_t)t * kts + (int64_t)h * khs + d0);
        kb = load_as_f32<DT>(key, (int64_t)t * kts + (int64_t)h * khs + d0 + 1);
        va = load_as_f32<DT>(value, (int64_t)t * vts + (int64_t)h * vhs + d0);
        vb = load_as_f32<DT>(value, (int64_t)t * vts + (int64_t)h * vhs + d0 + 1);
    }
    const int64_t slot = slot_mapping[t];
    if (slot < 0) return;
    const int64_t page = slot / block_size;
    const int off = (int)(slot - page * block_size);
    const int sp = off >> 4, tt = off & 15;
    const int64_t base = page * cbs + (int64_t)h * chs + (int64_t)sp * SUBPAGE_BYTES;
    const Q8Pair rk = q8_quantize_pair(ka, kb);
    const Q8Pair rv = q8_quantize_pair(va, vb);
    planar_store_pair(kc + base, vc + base, tt, lane, rk, rv);
}

// ---------------------------------------------------------------------------
// Planar K+V write, block per lane (D = 128).  One wave per (16 consecutive
// tokens, kv-head): lane l takes token t0 + l%16 and Q8_0 block b = l/16, so
// the 32 values of a block sit in one lane and amax needs no cross-lane
// reduction; the per-element arithmetic is the closed form of
// q8_quantize_pair.  Each lane writes its own slot (any slot mapping; slot <
// 0 or a token past the end writes nothing):
//   K ints : four 8-byte stores, kpos(tt, 32b + 8g) for g = 0..3
//   V ints : 32 byte stores at vpos(tt, 32b + e)
//   scales : one fp16 each (K at 2048 + (4tt+b)*2, V at 2048 + ((tt/4)*4+b)*8 + (tt%4)*2)
// (tt = slot % 16 is the token's place in its sub-page.)  Needs the cache
// bases and strides 8-byte aligned.
template <int DT, bool VEC>
__device__ __forceinline__ void load_block32(const void *x, int64_t off, float (&v)[QK]) {
    if constexpr (VEC && DT != GFA_DTYPE_F32) {
        const u32x4 *p = reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(x) + off);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const u32x4 w = p[c];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t we = w[e];
                if constexpr (DT == GFA_DTYPE_F16) {
                    v[8 * c + 2 * e] = half_bits_to_f32(we & 0xFFFFu);
                    v[8 * c + 2 * e + 1] = half_bits_to_f32(we >> 16);
                } else {
                    v[8 * c + 2 * e] = bf16_bits_to_f32(we & 0xFFFFu);
                    v[8 * c + 2 * e + 1] = bf16_bits_to_f32(we >> 16);
                }
            }
        }
    } else if constexpr (VEC) {
        const float4_t *p = reinterpret_cast<const float4_t *>(static_cast<const float *>(x) + off);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const float4_t w = p[c];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * c + e] = w[e];
        }
    } else {
#pragma unroll
        for (int e = 0; e < QK; ++e) v[e] = load_as_f32<DT>(x, off + e);
    }
}

// the Q8_0 closed form over one lane's 32 values (see q8_quantize_pair)
__device__ __forceinline__ float quantize_block32(const float (&v)[QK], int8_t (&q)[QK]) {
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < QK; ++e) amax = fmaxf(amax, fabsf(v[e]));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
    for (int e = 0; e < QK; ++e) {
        int qi = (int)rintf(v[e] * id);
        qi = qi < -128 ? -128 : (qi > 127 ? 127 : qi);
        q[e] = (int8_t)qi;
    }
    return d;
}

template <int DT, bool VEC>
__global__ __launch_bounds__(256) void q8_cache_write_kv_blk_kernel(
    const void *__restrict__ key, const void *__restrict__ value,
    const int64_t *__restrict__ slot_mapping, uint8_t *__restrict__ kc,
    uint8_t *__restrict__ vc, int num_tokens, int num_kv_heads, int block_size,
    int64_t kts, int64_t khs, int64_t vts, int64_t vhs, int64_t cbs, int64_t chs) {
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t grp = wave / num_kv_heads;
    const int h = (int)(wave - grp * num_kv_heads);
    const int64_t t = 16 * grp + (lane & 15);
    const int b = lane >> 4;
    if (t >= num_tokens) return;  // per lane: nothing below is shared
    const int64_t slot = slot_mapping[t];
    if (slot < 0) return;
    const int64_t page = slot / block_size;
    const int off = (int)(slot - page * block_size);
    const int sp = off >> 4, tt = off & 15;
    const int64_t base = page * cbs + (int64_t)h * chs + (int64_t)sp * SUBPAGE_BYTES;

    float v[QK];
    int8_t q[QK];
    // K: four 8-byte runs (d = 32b + 8g .. +7) and the block scale
    load_block32<DT, VEC>(key, t * kts + (int64_t)h * khs + QK * b, v);
    float d = quantize_block32(v, q);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            lo |= (uint32_t)(uint8_t)q[8 * g + e] << (8 * e);
            hi |= (uint32_t)(uint8_t)q[8 * g + 4 + e] << (8 * e);
        }
        const int kpos = (b >> 1) * 1024 + (4 * tt + g) * 16 + (b & 1) * 8;
        *reinterpret_cast<u32x2 *>(kc + base + kpos) = u32x2{lo, hi};
    }
    *reinterpret_cast<uint16_t *>(kc + base + SCALE_OFF + (4 * tt + b) * 2) = f32_to_half_bits(d);
    // V: byte stores into the transposed (4 tokens per dword) layout
    load_block32<DT, VEC>(value, t * vts + (int64_t)h * vhs + QK * b, v);
    d = quantize_block32(v, q);
    uint8_t *vrow = vc + base + (b >> 1) * 1024 + (tt >> 2) * 256 + (tt & 3);
#pragma unroll
    for (int e = 0; e < QK; ++e) {
        const int m = 2 * b + (e >> 4);  // d / 16
        vrow[(e & 15) * 16 + (m & 3) * 4] = (uint8_t)q[e];
    }
    *reinterpret_cast<uint16_t *>(vc + base + SCALE_OFF + ((tt >> 2) * 4 + b) * 8 + (tt & 3) * 2) =
        f32_to_half_bits(d);
}

#ifndef GFA_WRITE_ROW_KERNEL_MAX
#define GFA_WRITE_ROW_KERNEL_MAX 4096  // (token, kv-head) rows
#endif

bool bad_dtype(int dt) { return dt != GFA_DTYPE_F32 && dt != GFA_DTYPE_F16 && dt != GFA_DTYPE_BF16; }

}  // namespace

extern "C" const char *gfx906_fa_amd_version(void) { return "gfx906_fa_amd 0.1 gfx950"; }

extern "C" hipError_t gfx906_fa_amd_quantize_q8_0(const void *x, int x_dtype, uint8_t *y,
                                                  int64_t N, int D, hipStream_t stream) {
    if (D <= 0 || D % QK != 0 || N < 0 || bad_dtype(x_dtype)) {
        fprintf(stderr, "[gfx906_fa_amd] quantize_q8_0: need D %% 32 == 0 (D=%d), N >= 0, dtype 0/1/2\n", D);
        return hipErrorInvalidValue;
    }
    if (N == 0) return hipSuccess;
    const int64_t nblk = N * (D / QK);
    const int64_t threads = nblk * 16;
    const unsigned grid = (unsigned)((threads + 255) / 256);
    switch (x_dtype) {
        case GFA_DTYPE_F32: q8_dense_kernel<GFA_DTYPE_F32><<<grid, 256, 0, stream>>>(x, y, nblk); break;
        case GFA_DTYPE_F16: q8_dense_kernel<GFA_DTYPE_F16><<<grid, 256, 0, stream>>>(x, y, nblk); break;
        default: q8_dense_kernel<GFA_DTYPE_BF16><<<grid, 256, 0, stream>>>(x, y, nblk); break;
    }
    return hipGetLastError();
}

extern "C" hipError_t launch_quantize_q8_0_dense(const void *x, uint8_t *y, int N, int D,
                                                 hipStream_t stream) {
    return gfx906_fa_amd_quantize_q8_0(x, GFA_DTYPE_F16, y, N, D, stream);
}

extern "C" hipError_t gfx906_fa_amd_reshape_and_cache_q8(
    const void *key, int key_dtype, const int64_t *slot_mapping, uint8_t *k_cache_q8,
    int num_tokens, int num_kv_heads, int head_size, int block_size, int64_t kts, int64_t khs,
    int64_t cbs, int64_t cts, int64_t chs, hipStream_t stream) {
    if (head_size <= 0 || head_size % QK != 0 || block_size <= 0 || bad_dtype(key_dtype) ||
        num_kv_heads <= 0 || num_tokens < 0) {
        fprintf(stderr, "[gfx906_fa_amd] reshape_and_cache_q8: bad arguments (head_size=%d, block_size=%d)\n",
                head_size, block_size);
        return hipErrorInvalidValue;
    }
    if (num_tokens == 0) return hipSuccess;
    const int64_t waves = (int64_t)num_tokens * num_kv_heads;
    const unsigned grid = (unsigned)((waves + 3) / 4);
#define GFA_LAUNCH_RC(DT)                                                                   \
    q8_reshape_cache_kernel<DT><<<grid, 256, 0, stream>>>(key, slot_mapping, k_cache_q8,   \
                                                         num_tokens, num_kv_heads,          \
                                                         head_size, block_size, kts, khs,   \
                                                         cbs, cts, chs)
    switch (key_dtype) {
        case GFA_DTYPE_F32: GFA_LAUNCH_RC(GFA_DTYPE_F32); break;
        case GFA_DTYPE_F16: GFA_LAUNCH_RC(GFA_DTYPE_F16); break;
        default: GFA_LAUNCH_RC(GFA_DTYPE_BF16); break;
    }
#undef GFA_LAUNCH_RC
    return hipGetLastError();
}

extern "C" hipError_t launch_reshape_and_cache_q8(const void *key, const int64_t *slot_mapping,
                                                  uint8_t *k_cache_q8, int num_tokens,
                                                  int num_kv_heads, int head_size,
                                                  int block_size, int64_t kts, int64_t khs,
                                                  int64_t cbs, int64_t cts, int64_t chs,
                                                  hipStream_t stream) {
    return gfx906_fa_amd_reshape_and_cache_q8(key, GFA_DTYPE_F16, slot_mapping, k_cache_q8,
                                              num_tokens, num_kv_heads, head_size, block_size,
                                              kts, khs, cbs, cts, chs, stream);
}

extern "C" hipError_t gfx906_fa_amd_cache_write_kv(
    const void *key, const void *value, int dtype, const int64_t *slot_mapping, uint8_t *k_cache,
    uint8_t *v_cache, int num_tokens, int num_kv_heads, int head_size, int block_size,
    int64_t kts, int64_t khs, int64_t vts, int64_t vhs, int64_t cbs, int64_t chs,
    hipStream_t stream) {
    if (head_size != 128 || block_size <= 0 || block_size % SUBPAGE != 0 || bad_dtype(dtype) ||
        num_kv_heads <= 0 || num_tokens < 0) {
        fprintf(stderr,
                "[gfx906_fa_amd] cache_write_kv: need head_size == 128 (got %d) and block_size %% 16 == 0 (got %d)\n",
                head_size, block_size);
        return hipErrorInvalidValue;
    }
    if (((uintptr_t)k_cache | (uintptr_t)v_cache | (uint64_t)cbs | (uint64_t)chs) & 1u) {
        fprintf(stderr, "[gfx906_fa_amd] cache_write_kv: cache bases and strides must be even\n");
        return hipErrorInvalidValue;
    }
    if (num_tokens == 0) return hipSuccess;
    const int esz = dtype == GFA_DTYPE_F32 ? 4 : 2;
    const bool vec = (((uintptr_t)key | (uintptr_t)value) % (2 * esz) == 0) && (kts % 2 == 0) &&
                     (khs % 2 == 0) && (vts % 2 == 0) && (vhs % 2 == 0);
    // Small batches (decode steps) take the wave-per-row kernel: its serial
    // work per lane is one pair of values, so a handful of rows finishes in
    // the latency of its loads; the block-per-lane kernel's 32-value serial
    // quantize only pays once there are enough rows to fill the device.
    const bool few_rows = (int64_t)num_tokens * num_kv_heads <= GFA_WRITE_ROW_KERNEL_MAX;
    if (!few_rows && (((uintptr_t)k_cache | (uintptr_t)v_cache | (uint64_t)cbs | (uint64_t)chs) & 7u) == 0) {
        // block per lane: vector loads need 16-byte aligned rows of 32 values
        const bool vec16 = (((uintptr_t)key | (uintptr_t)value) % 16 == 0) &&
                           ((kts * esz) % 16 == 0) && ((khs * esz) % 16 == 0) &&
                           ((vts * esz) % 16 == 0) && ((vhs * esz) % 16 == 0);
        const int64_t waves = (int64_t)((num_tokens + 15) / 16) * num_kv_heads;
        const unsigned grid = (unsigned)((waves + 3) / 4);
#define GFA_LAUNCH_BLK(DT, V)                                                                    \
    q8_cache_write_kv_blk_kernel<DT, V><<<grid, 256, 0, stream>>>(key, value, slot_mapping,     \
                                                                 k_cache, v_cache, num_tokens,   \
                                                                 num_kv_heads, block_size, kts,  \
                                                                 khs, vts, vhs, cbs, chs)
        if (vec16) {
            switch (dtype) {
                case GFA_DTYPE_F32: GFA_LAUNCH_BLK(GFA_DTYPE_F32, true); break;
                case GFA_DTYPE_F16: GFA_LAUNCH_BLK(GFA_DTYPE_F16, true); break;
                default: GFA_LAUNCH_BLK(GFA_DTYPE_BF16, true); break;
            }
        } else {
            switch (dtype) {
                case GFA_DTYPE_F32: GFA_LAUNCH_BLK(GFA_DTYPE_F32, false); break;
                case GFA_DTYPE_F16: GFA_LAUNCH_BLK(GFA_DTYPE_F16, false); break;
                default: GFA_LAUNCH_BLK(GFA_DTYPE_BF16, false); break;
            }
        }
#undef GFA_LAUNCH_BLK
        return hipGetLastError();
    }
    const int64_t waves = (int64_t)num_tokens * num_kv_heads;
    const unsigned grid = (unsigned)((waves + 3) / 4);
#define GFA_LAUNCH_KV(DT, V)                                                                 \
    q8_cache_write_kv_kernel<DT, V><<<grid, 256, 0, stream>>>(key, value, slot_mapping,     \
                                                             k_cache, v_cache, num_tokens,   \
                                                             num_kv_heads, block_size, kts,  \
                                                             khs, vts, vhs, cbs, chs)
    if (vec) {
        switch (dtype) {
            case GFA_DTYPE_F32: GFA_LAUNCH_KV(GFA_DTYPE_F32, true); break;
            case GFA_DTYPE_F16: GFA_LAUNCH_KV(GFA_DTYPE_F16, true); break;
            default: GFA_LAUNCH_KV(GFA_DTYPE_BF16, true); break;
        }
    } else {
        switch (dtype) {
            case GFA_DTYPE_F32: GFA_LAUNCH_KV(GFA_DTYPE_F32, false); break;
            case GFA_DTYPE_F16: GFA_LAUNCH_KV(GFA_DTYPE_F16, false); break;
            default: GFA_LAUNCH_KV(GFA_DTYPE_BF16, false); break;
        }
    }
#undef GFA_LAUNCH_KV
    return hipGetLastError();
}
