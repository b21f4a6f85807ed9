// q8_pack.hip - contiguous -> planar repacking for the flat attention entry
// (the op module's forward(), the reference's contiguous path
// extension/gfx906_fa.cpp:120-265 over K_q8 [B, Hkv, Skv, 136] and fp16
// V [B, Hkv, Skv, D]).
//
//   pack_k_kernel    AoS Q8_0 K rows -> planar Q8 K sub-pages (a byte
//                    permutation: the same Q8_0 blocks, placed for the MFMA
//                    operand loads)
//   pack_v16_kernel  fp16 V rows -> planar fp16 V sub-pages (4096 B per 16
//                    tokens; element (t, d) at
//                    2048*(d/64) + 32*(16*(t/4) + d%16) + 8*((d/16)%4) + 2*(t%4),
//                    i.e. the 32 bytes a lane of the prefill kernel moves
//                    into its transposed V tile are contiguous)
// Tokens past Skv (up to the 16-token sub-page boundary) are written as
// zeros.  Rows r index the [B*Hkv] (sequence, kv-head) pairs.
#include <cstdio>

#include "q8_common.h"

using namespace gfa;

namespace {

__device__ __forceinline__ int kpos(int t, int d) {
    const int b = d >> 5, g = (d & 31) >> 3;
    return (b >> 1) * 1024 + (4 * t + g) * 16 + (b & 1) * 8 + (d & 7);
}

// one thread per (row, token, byte of the 136-byte AoS row)
__global__ __launch_bounds__(256) void pack_k_kernel(const uint8_t *__restrict__ k_aos,
                                                     uint8_t *__restrict__ k_pl, int64_t total,
                                                     int Skv, int Skv_pad) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int c = (int)(i % 136);
    const int64_t rt = i / 136;
    const int t = (int)(rt % Skv_pad);
    const int64_t r = rt / Skv_pad;
    const uint8_t v = t < Skv ? k_aos[(r * Skv + t) * 136 + c] : (uint8_t)0;
    const int b = c / 34, o = c - 34 * b, tt = t & 15;
    const int pos = o < 2 ? SCALE_OFF + (4 * tt + b) * 2 + o : kpos(tt, 32 * b + o - 2);
    k_pl[(r * (Skv_pad / 16) + t / 16) * SUBPAGE_BYTES + pos] = v;
}

// one thread per (row, token, d)
__global__ __launch_bounds__(256) void pack_v16_kernel(const uint16_t *__restrict__ v,
                                                       uint16_t *__restrict__ v_pl, int64_t total,
                                                       int Skv, int Skv_pad) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int d = (int)(i & 127);
    const int64_t rt = i >> 7;
    const int t = (int)(rt % Skv_pad);
    const int64_t r = rt / Skv_pad;
    const uint16_t x = t < Skv ? v[(r * Skv + t) * 128 + d] : (uint16_t)0;
    const int tt = t & 15;
    const int byte = 2048 * (d >> 6) + 32 * (16 * (tt >> 2) + (d & 15)) + 8 * ((d >> 4) & 3) + 2 * (tt & 3);
    v_pl[((r * (Skv_pad / 16) + t / 16) * 4096 + byte) >> 1] = x;
}

}  // namespace

extern "C" hipError_t gfx906_fa_amd_pack_flat_kv(const uint8_t *k_aos, const void *v_f16,
                                                 uint8_t *k_planar, void *v_planar, int rows,
                                                 int Skv, int head_size, hipStream_t stream) {
    if (rows <= 0 || Skv <= 0) return hipSuccess;
    if (head_size != 128) {
        fprintf(stderr, "[gfx906_fa_amd] pack_flat_kv: head_size=%d unsupported (only 128)\n", head_size);
        return hipErrorInvalidValue;
    }
    const int Skv_pad = (Skv + 15) & ~15;
    const int64_t nk = (int64_t)rows * Skv_pad * 136;
    const int64_t nv = (int64_t)rows * Skv_pad * 128;
    pack_k_kernel<<<(unsigned)((nk + 255) / 256), 256, 0, stream>>>(k_aos, k_planar, nk, Skv, Skv_pad);
    pack_v16_kernel<<<(unsigned)((nv + 255) / 256), 256, 0, stream>>>(
        static_cast<const uint16_t *>(v_f16), static_cast<uint16_t *>(v_planar), nv, Skv, Skv_pad);
    return hipGetLastError();
}
