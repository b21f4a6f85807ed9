// q8_gather.hip - paged -> contiguous gather kernels for gfx950.
//
// Contract (extension/gfx906_fa_gather.cu:190-357, the reference's default
// v2 kernel): for s < B, h < Hkv, t < Sk with lb = t / bs and
// pb = lb < max_blocks ? block_table[s][lb] : -1, a token is valid iff
// t < seq_lens[s] and pb >= 0.  Valid: copy the K row and the V row.
// Invalid: zero the V row, leave the K row untouched.
//
//   gather_rows16_kernel  AoS rows (K q8 + V fp16 of the reference, or K q8 +
//                         V q8) in 16-byte chunks; gather_rows_kernel is the
//                         per-word form for other block sizes / alignments
//   gather_planar16_kernel planar K+V sub-pages -> AoS K and V rows through LDS;
//                         gather_planar_kernel is the direct per-word form
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

// Fast path: block_size % 16 == 0, Sk % 16 == 0, 8-byte aligned rows and
// strides, 16-byte aligned outputs.  One workgroup (128 threads) per (sequence, kv-head,
// 16-token slab): the slab lies in one page, so its page id is read once.
// The slab's output is 16 * (k_row + v_row) contiguous bytes in two runs (its
// K rows, its V rows), each a whole number of 16-byte chunks.  A thread moves
// one chunk at a time: two 8-byte loads (a Q8_0 row is 8-byte but not 16-byte
// aligned, so a chunk can span two rows) and one 16-byte store, or 8-byte
// stores where a K chunk touches a token whose K row must stay untouched.
__global__ __launch_bounds__(128) void gather_rows16_kernel(
    const uint8_t *__restrict__ kc, const uint8_t *__restrict__ vc,
    const int32_t *__restrict__ block_table, const int32_t *__restrict__ seq_lens,
    uint8_t *__restrict__ k_out, uint8_t *__restrict__ v_out, int num_kv_heads, int Sk,
    int k_row, int v_row, int block_size, int max_blocks, int64_t kbs, int64_t kts, int64_t khs,
    int64_t vbs, int64_t vts, int64_t vhs) {
    const int s = blockIdx.z;
    const int h = blockIdx.y;
    const int t0 = blockIdx.x * 16;
    const int ntok = min(16, Sk - t0);
    const int sl = seq_lens[s];
    const int lb = t0 / block_size;
    const int pb = lb < max_blocks ? block_table[(int64_t)s * max_blocks + lb] : -1;
    const int off0 = t0 - lb * block_size;
    const int nvalid = pb >= 0 ? max(0, min(ntok, sl - t0)) : 0;  // tokens t0 .. t0+nvalid-1 valid
    const int64_t orow = ((int64_t)s * num_kv_heads + h) * Sk + t0;
    const uint8_t *kpage = kc + (int64_t)max(pb, 0) * kbs + (int64_t)off0 * kts + (int64_t)h * khs;
    const uint8_t *vpage = vc + (int64_t)max(pb, 0) * vbs + (int64_t)off0 * vts + (int64_t)h * vhs;
    auto load8 = [](const uint8_t *p) { return *reinterpret_cast<const uint64_t *>(p); };
    // V: copy valid rows, zero the rest
    {
        uint8_t *dst = v_out + orow * v_row;
        const int nch = ntok * v_row / 16;
        for (int c = threadIdx.x; c < nch; c += blockDim.x) {
            const int o = 16 * c;
            const int ta = o / v_row, ra = o - ta * v_row;
            const int tb = (o + 8) / v_row, rb = o + 8 - tb * v_row;
            const uint64_t a = ta < nvalid ? load8(vpage + ta * vts + ra) : 0;
            const uint64_t b = tb < nvalid ? load8(vpage + tb * vts + rb) : 0;
            *reinterpret_cast<u32x4 *>(dst + o) = u32x4{(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b,
                                                        (uint32_t)(b >> 32)};
        }
    }
    // K: copy valid rows only
    {
        uint8_t *dst = k_out + orow * k_row;
        const int nch = nvalid * k_row / 16;  // whole chunks inside the valid rows
        for (int c = threadIdx.x; c < nch; c += blockDim.x) {
            const int o = 16 * c;
            const int ta = o / k_row, ra = o - ta * k_row;
            const int tb = (o + 8) / k_row, rb = o + 8 - tb * k_row;
            const uint64_t a = load8(kpage + ta * kts + ra);
            const uint64_t b = load8(kpage + tb * kts + rb);
            *reinterpret_cast<u32x4 *>(dst + o) = u32x4{(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b,
                                                        (uint32_t)(b >> 32)};
        }
        // an 8-byte tail of the valid rows that a 16-byte chunk would overrun
        if (threadIdx.x == 0 && (nvalid * k_row) % 16 != 0) {
            const int o = nvalid * k_row - 8;
            const int ta = o / k_row, ra = o - ta * k_row;
            *reinterpret_cast<uint64_t *>(dst + o) = load8(kpage + ta * kts + ra);
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

// Planar -> AoS through LDS (Sk % 16 == 0, 16-byte aligned outputs): one
// workgroup of exactly 128 threads per (sequence, kv-head, 16-token sub-page).  The K
// and V sub-pages (2 x 2176 B) come in with 16-byte loads, the AoS rows are
// assembled in LDS from the staged bytes (the byte permutation of the planar
// layout), and the 16 rows of each plane (2176 contiguous output bytes) go
// out with 16-byte stores: all V rows (zeroed past the valid tokens), the K
// rows of valid tokens only (an 8-byte tail where their bytes end mid-chunk).
__global__ __launch_bounds__(128) void gather_planar16_kernel(
    const uint8_t *__restrict__ kc, const uint8_t *__restrict__ vc,
    const int32_t *__restrict__ block_table, const int32_t *__restrict__ seq_lens,
    uint8_t *__restrict__ k_out, uint8_t *__restrict__ v_out, int num_kv_heads, int Sk,
    int block_size, int max_blocks, int64_t cbs, int64_t chs) {
    __shared__ __attribute__((aligned(16))) uint8_t stage[2][SUBPAGE_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t rows[2][16 * 136];
    const int s = blockIdx.z;
    const int h = blockIdx.y;
    const int t0 = blockIdx.x * 16;
    const int sl = seq_lens[s];
    const int lb = t0 / block_size;  // a 16-token sub-page never straddles pages
    const int pb = lb < max_blocks ? block_table[(int64_t)s * max_blocks + lb] : -1;
    const int sp = (t0 - lb * block_size) >> 4;
    const int nvalid = pb >= 0 ? max(0, min(16, sl - t0)) : 0;
    const int64_t orow = ((int64_t)s * num_kv_heads + h) * Sk + t0;
    if (nvalid > 0) {
        const int64_t src = (int64_t)pb * cbs + (int64_t)h * chs + (int64_t)sp * SUBPAGE_BYTES;
        for (int i = threadIdx.x; i < 2 * SUBPAGE_BYTES / 16; i += blockDim.x) {
            const int plane = i >= SUBPAGE_BYTES / 16;
            const int c = i - plane * (SUBPAGE_BYTES / 16);
            *reinterpret_cast<u32x4 *>(&stage[plane][16 * c]) =
                *reinterpret_cast<const u32x4 *>((plane ? vc : kc) + src + 16 * c);
        }
    }
    __syncthreads();
    // One thread per (plane, token tl, Q8_0 block b): the 34 AoS bytes
    // (fp16 scale, 32 ints) assembled in registers and written to the row in
    // LDS as 17 halfwords (34b is only 2-byte aligned).  K ints of (tl, b) are
    // four 8-byte runs of the planar sub-page; V ints are one byte each (V is
    // stored token-minor, four tokens per 4-byte word).
    {
        const int plane = threadIdx.x >> 6;
        const int tl = (threadIdx.x >> 2) & 15;
        const int b = threadIdx.x & 3;
        const uint8_t *sub = stage[plane];
        uint16_t hw[17];
        if (tl < nvalid) {
            hw[0] = plane ? *reinterpret_cast<const uint16_t *>(sub + SCALE_OFF + ((tl >> 2) * 4 + b) * 8 + (tl & 3) * 2)
                          : *reinterpret_cast<const uint16_t *>(sub + SCALE_OFF + (4 * tl + b) * 2);
            uint32_t q[8];  // the 32 ints, little-endian in d
            if (plane == 0) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {  // d = 32b + 8r .. +7
                    const u32x2 v = *reinterpret_cast<const u32x2 *>(sub + (b >> 1) * 1024 + (4 * tl + r) * 16 + (b & 1) * 8);
                    q[2 * r] = v[0];
                    q[2 * r + 1] = v[1];
                }
            } else {
#pragma unroll
                for (int w = 0; w < 8; ++w) {
                    uint32_t x = 0;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int d = 32 * b + 4 * w + k;
                        const uint32_t byte = sub[(d >> 6) * 1024 + ((tl >> 2) * 16 + (d & 15)) * 16 +
                                                  ((d >> 4) & 3) * 4 + (tl & 3)];
                        x |= byte << (8 * k);
                    }
                    q[w] = x;
                }
            }
#pragma unroll
            for (int k = 0; k < 16; ++k) hw[1 + k] = (uint16_t)(q[k >> 1] >> (16 * (k & 1)));
        } else {
#pragma unroll
            for (int k = 0; k < 17; ++k) hw[k] = 0;
        }
        uint16_t *row = reinterpret_cast<uint16_t *>(&rows[plane][136 * tl + 34 * b]);
#pragma unroll
        for (int k = 0; k < 17; ++k) row[k] = hw[k];
    }
    __syncthreads();
    {   // V: all 16 rows
        uint8_t *dst = v_out + orow * 136;
        for (int c = threadIdx.x; c < 16 * 136 / 16; c += blockDim.x)
            *reinterpret_cast<u32x4 *>(dst + 16 * c) = *reinterpret_cast<const u32x4 *>(&rows[1][16 * c]);
    }
    {   // K: the valid rows only
        uint8_t *dst = k_out + orow * 136;
        const int nb = nvalid * 136;
        for (int c = threadIdx.x; c < nb / 16; c += blockDim.x)
            *reinterpret_cast<u32x4 *>(dst + 16 * c) = *reinterpret_cast<const u32x4 *>(&rows[0][16 * c]);
        if (threadIdx.x == 0 && nb % 16 != 0)
            *reinterpret_cast<uint64_t *>(dst + nb - 8) = *reinterpret_cast<const uint64_t *>(&rows[0][nb - 8]);
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
    if (w8 && block_size % 16 == 0 && Sk % 16 == 0 && (((uintptr_t)k_out | (uintptr_t)v_out) & 15u) == 0) {
        gather_rows16_kernel<<<grid, 128, 0, stream>>>(
            k_cache, v_cache, block_table, seq_lens, k_out, v_out, num_kv_heads, Sk, k_row_bytes,
            v_row_bytes, block_size, max_blocks_per_seq, kbs, kts, khs, vbs, vts, vhs);
    } else if (w8) {
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
    if (Sk % 16 == 0 && (((uintptr_t)k_out | (uintptr_t)v_out) & 15u) == 0)
        gather_planar16_kernel<<<grid, 128, 0, stream>>>(k_cache, v_cache, block_table, seq_lens, k_out,
                                                         v_out, num_kv_heads, Sk, block_size,
                                                         max_blocks_per_seq, cbs, chs);
    else
        gather_planar_kernel<<<grid, 256, 0, stream>>>(k_cache, v_cache, block_table, seq_lens, k_out,
                                                       v_out, num_kv_heads, Sk, block_size,
                                                       max_blocks_per_seq, cbs, chs);
    return hipGetLastError();
}
