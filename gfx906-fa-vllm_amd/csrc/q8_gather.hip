// q8_gather.hip - paged -> contiguous gather kernels for gfx950.
//
// Contract (extension/gfx906_fa_gather.cu:190-357, the reference's default
// v2 kernel): for s < B, h < Hkv, t < Sk with lb = t / bs and
// pb = lb < max_blocks ? block_table[s][lb] : -1, a token is valid iff
// t < seq_lens[s] and pb >= 0.  Valid: copy the K row and the V row.
// Invalid: zero the V row, leave the K row untouched.
//
//   gather_rows_kernel    AoS rows of arbitrary byte size (K q8 + V fp16 of the
//                         reference, or K q8 + V q8)
//   gather_planar_kernel  planar K+V sub-pages -> AoS K and V rows
#include <cstdio>

#include "q8_common.h"

using namespace gfa;

namespace {

// One workgroup per (sequence, kv-head, 16-token slab).  Rows are copied in
// W-byte words (W = 8 when every row address is 8-byte aligned, else 1).
template <typename WORD>
__global__ __launch_bounds__(256) void gather_rows_kernel(
    const uint8_t *__restrict__ kc, const uint8_t *__restrict__ vc,
    const int32_t *__restrict__ block_table, const int32_t *__restrict__ seq_lens,
    uint8_t *__restrict__ k_out, uint8_t *__restrict__ v_out, int num_kv_heads, int Sk,
    int k_row, int v_row, int block_size, int max_blocks, int64_t kbs, int64_t kts, int64_t khs,
    int64_t vbs, int64_t vts, int64_t vhs) {
    const int s = blockIdx.z;
    const int h = blockIdx.y;
    const int t0 = blockIdx.x * 16;
    const int sl = seq_lens[s];
    const int kw = k_row / (int)sizeof(WORD);
    const int vw = v_row / (int)sizeof(WORD);
    const int64_t obase = ((int64_t)s * num_kv_heads + h) * Sk;
    // V rows (copy or zero) and K rows (copy only), flattened over the slab.
    const int nv = 16 * vw, nk = 16 * kw;
    for (int i = threadIdx.x; i < nv + nk; i += blockDim.x) {
        const bool isv = i < nv;
        const int j = isv ? i : i - nv;
        const int words = isv ? vw : kw;
        const int tl = j / words;
        const int w = j - tl * words;
        const int t = t0 + tl;
        if (t >= Sk) continue;
        const int lb = t / block_size;
        const int pb = lb < max_blocks ? block_table[(int64_t)s * max_blocks + lb] : -1;
        const bool valid = t < sl && pb >= 0;
        const int off = t - lb * block_size;
        if (isv) {
            WORD val = 0;
            if (valid)
                val = reinterpret_cast<const WORD *>(vc + pb * vbs + off * vts + h * vhs)[w];
            reinterpret_cast<WORD *>(v_out + (obase + t) * v_row)[w] = val;
        } else if (valid) {
            reinterpret_cast<WORD *>(k_out + (obase + t) * k_row)[w] =
                reinterpret_cast<const WORD *>(kc + pb * kbs + off * kts + h * khs)[w];
        }
    }
}

// One workgroup (256 threads) per (sequence, kv-head, 16-token sub-page).
// Each thread emits 4-byte words of the AoS rows: 16 tokens x 34 words per
// plane.  Output rows are 136 bytes, so word stores are 4-byte aligned.
__global__ __launch_bounds__(256) void gather_planar_kernel(
    const uint8_t *__restrict__ kc, const uint8_t *__restrict__ vc,
    const int32_t *__restrict__ block_table, const int32_t *__restrict__ seq_lens,
    uint8_t *__restrict__ k_out, uint8_t *__restrict__ v_out, int num_kv_heads, int Sk,
    int block_size, int max_blocks, int64_t cbs, int64_t chs) {
    const int s = blockIdx.z;
    const int h = blockIdx.y;
    const int t0 = blockIdx.x * 16;
    const int sl = seq_lens[s];
    const int lb = t0 / block_size;  // a 16-token sub-page never straddles pages
    const int pb = lb < max_blocks ? block_table[(int64_t)s * max_blocks + lb] : -1;
    const int sp = (t0 - lb * block_size) >> 4;
    const int64_t src = (pb >= 0 ? (int64_t)pb * cbs : 0) + (int64_t)h * chs + (int64_t)sp * SUBPAGE_BYTES;
    const int64_t obase = ((int64_t)s * num_kv_heads + h) * Sk;
    for (int i = threadIdx.x; i < 2 * 16 * 34; i += blockDim.x) {
        const int plane = i / (16 * 34);
        const int j = i - plane * 16 * 34;
        const int tl = j / 34;
        const int w = j - tl * 34;
        const int t = t0 + tl;
        if (t >= Sk) continue;
        const bool valid = t < sl && pb >= 0;
        uint8_t *dst = (plane ? v_out : k_out) + (obase + t) * 136 + 4 * w;
        if (!valid) {
            if (plane) *reinterpret_cast<uint32_t *>(dst) = 0u;
            continue;
        }
        const uint8_t *sub = (plane ? vc : kc) + src;
        uint32_t word = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int p = 4 * w + k;          // byte position inside the AoS row
            const int b = p / 34;
            const int r = p - b * 34;
            uint8_t byte;
            if (r < 2) {
                byte = sub[(plane ? SCALE_OFF + ((tl >> 2) * 4 + b) * 8 + (tl & 3) * 2
                                  : SCALE_OFF + (4 * tl + b) * 2) + r];
            } else {
                const int d = 32 * b + (r - 2);
                const int pos = plane ? ((d >> 6) * 1024 + ((tl >> 2) * 16 + (d & 15)) * 16 +
                                         ((d >> 4) & 3) * 4 + (tl & 3))
                                      : ((d >> 6) * 1024 + (4 * tl + ((d >> 3) & 3)) * 16 +
                                         ((d >> 5) & 1) * 8 + (d & 7));
                byte = sub[pos];
            }
            word |= (uint32_t)byte << (8 * k);
        }
        *reinterpret_cast<uint32_t *>(dst) = word;
    }
}

}  // namespace

extern "C" hipError_t gfx906_fa_amd_gather_rows(
    const uint8_t *k_cache, const uint8_t *v_cache, const int32_t *block_table,
    const int32_t *seq_lens, uint8_t *k_out, uint8_t *v_out, int num_seqs, int num_kv_heads,
    int Sk, int k_row_bytes, int v_row_bytes, int block_size, int max_blocks_per_seq,
    int64_t kbs, int64_t kts, int64_t khs, int64_t vbs, int64_t vts, int64_t vhs,
    hipStream_t stream) {
    if (num_seqs == 0 || num_kv_heads == 0 || Sk == 0) return hipSuccess;
    if (num_seqs < 0 || num_kv_heads < 0 || Sk < 0 || block_size <= 0 || k_row_bytes <= 0 ||
        v_row_bytes <= 0 || max_blocks_per_seq < 0) {
        fprintf(stderr, "[gfx906_fa_amd] gather: bad arguments\n");
        return hipErrorInvalidValue;
    }
    const bool w8 = ((((uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)k_out |
                       (uintptr_t)v_out) | (uint64_t)kbs | (uint64_t)kts | (uint64_t)khs |
                      (uint64_t)vbs | (uint64_t)vts | (uint64_t)vhs | (uint64_t)k_row_bytes |
                      (uint64_t)v_row_bytes) & 7u) == 0;
    dim3 grid((Sk + 15) / 16, num_kv_heads, num_seqs);
    if (w8) {
        gather_rows_kernel<uint64_t><<<grid, 256, 0, stream>>>(
            k_cache, v_cache, block_table, seq_lens, k_out, v_out, num_kv_heads, Sk, k_row_bytes,
            v_row_bytes, block_size, max_blocks_per_seq, kbs, kts, khs, vbs, vts, vhs);
    } else {
        gather_rows_kernel<uint8_t><<<grid, 256, 0, stream>>>(
            k_cache, v_cache, block_table, seq_lens, k_out, v_out, num_kv_heads, Sk, k_row_bytes,
            v_row_bytes, block_size, max_blocks_per_seq, kbs, kts, khs, vbs, vts, vhs);
    }
    return hipGetLastError();
}

extern "C" hipError_t launch_gather_paged_kv_q8(
    const uint8_t *key_cache_q8, const void *value_cache, const int32_t *block_table,
    const int32_t *seq_lens, uint8_t *k_out, void *v_out, int num_seqs, int num_kv_heads, int Sk,
    int D, int bytes_per_row, int block_size, int max_blocks_per_seq, int64_t cache_block_stride,
    int64_t cache_token_stride, int64_t cache_head_stride_q8, int64_t v_cache_block_stride,
    int64_t v_cache_token_stride, int64_t v_cache_head_stride, hipStream_t stream) {
    if (num_seqs == 0 || num_kv_heads == 0 || Sk == 0) return hipSuccess;
    if (D % 32 != 0) {
        fprintf(stderr, "[gfx906_fa_amd] gather_paged_kv_q8: D=%d must be a multiple of 32\n", D);
        return hipErrorInvalidValue;
    }
    // V strides are in fp16 elements in this contract.
    return gfx906_fa_amd_gather_rows(key_cache_q8, static_cast<const uint8_t *>(value_cache),
                                     block_table, seq_lens, k_out, static_cast<uint8_t *>(v_out),
                                     num_seqs, num_kv_heads, Sk, bytes_per_row, D * 2, block_size,
                                     max_blocks_per_seq, cache_block_stride, cache_token_stride,
                                     cache_head_stride_q8, v_cache_block_stride * 2,
                                     v_cache_token_stride * 2, v_cache_head_stride * 2, stream);
}

extern "C" hipError_t gfx906_fa_amd_gather_planar(
    const uint8_t *k_cache, const uint8_t *v_cache, const int32_t *block_table,
    const int32_t *seq_lens, uint8_t *k_out, uint8_t *v_out, int num_seqs, int num_kv_heads,
    int Sk, int head_size, int block_size, int max_blocks_per_seq, int64_t cbs, int64_t chs,
    hipStream_t stream) {
    if (num_seqs == 0 || num_kv_heads == 0 || Sk == 0) return hipSuccess;
    if (head_size != 128 || block_size <= 0 || block_size % 16 != 0 || num_seqs < 0 ||
        num_kv_heads < 0 || Sk < 0 || ((uintptr_t)k_out | (uintptr_t)v_out) % 4 != 0) {
        fprintf(stderr, "[gfx906_fa_amd] gather_planar: need head_size 128, block_size %% 16 == 0, 4-byte aligned outputs\n");
        return hipErrorInvalidValue;
    }
    dim3 grid((Sk + 15) / 16, num_kv_heads, num_seqs);
    gather_planar_kernel<<<grid, 256, 0, stream>>>(k_cache, v_cache, block_table, seq_lens, k_out,
                                                   v_out, num_kv_heads, Sk, block_size,
                                                   max_blocks_per_seq, cbs, chs);
    return hipGetLastError();
}
