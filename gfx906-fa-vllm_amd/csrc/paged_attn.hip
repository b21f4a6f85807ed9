// paged_attn.hip - direct-paged Q8_0 attention for gfx950 (decode, chunked
// prefill, mixed batches, speculative verify).
//
// Semantics follow the reference's paged FA (kernel/fattn-q8-paged.cuh:381-641,
// causal rule kernel/fattn-q8.cuh:646-653, GQA map kernel/fattn-q8.cuh:898-901,
// kv cutoff extension/gfx906_fa.cpp:595-604) with dequantize-then-fp32 math.
//
// Formulation (wave64, v_mfma_f32_16x16x32_f16), everything transposed so a
// lane owns one query row:
//   S^T[16 tok x 16 rows] = K[16 tok x 32 d] . Q^T[32 d x 16 rows]   (per Q8 block)
//   O^T[16 d x 16 rows]  += V^T[16 d x 32 tok] . P'^T[32 tok x 16 rows]
// Lane l = 16*g + i: row (column of S^T / O^T) i, token group / d group g.
// K int8 values enter the MFMA exactly (int8 -> fp16 is exact); each Q8 block
// gets its own MFMA and its fp16 scale multiplies the fp32 product.  V int8
// values also enter exactly; the V scale d_v[t][b] is folded into P
// (P'_b[t] = p[t] * d_v[t][b]) for the MFMAs of d-block b.  Softmax statistics
// and O accumulate in fp32.
//
// The planar page layout (include/gfx906_fa_amd.h) makes every operand an
// aligned 16-byte load straight from HBM: per 16-token sub-page a lane loads
// 32 B of K ints, 32 B of K scales, 32 B of V ints, 32 B of V scales.
//
// Query rows are GQA-packed: rows of one kv-head are r = j*G + gq (token j,
// q-head h*G + gq), so one K/V stream serves all G query heads.
//
//   attn_decode_kernel   rows <= 16*NRG per (seq, kv-head); KV split across
//                        the grid (split-K) and across the NW waves of a
//                        workgroup (merged in LDS); partials merged by
//                        attn_combine_kernel when a sequence has > 1 split.
//   attn_prefill_kernel  rows > 32: each wave owns 64 rows and streams the
//                        causal KV range; no cross-wave state.
#include <cstdio>

#include "q8_common.h"

using namespace gfa;

namespace {

constexpr float LOG2E = 1.4426950408889634f;
constexpr int DEC_DEPTH = 3;   // decode sub-page ring depth
constexpr int DEC_NW = 4;      // decode waves per workgroup (split the KV range)
constexpr int PF_NW = 4;       // prefill waves per workgroup
constexpr int PF_NRG = 2;      // prefill 16-row groups per wave
constexpr int ROWS_CAP = 32;   // decode partial slots per (seq, kv-head)

struct AttnParams {
    const void *q;
    int64_t q_ts, q_hs;
    const uint8_t *kc, *vc;
    int64_t cbs, chs;
    const int32_t *bt;
    int64_t bt_stride;
    const int32_t *seq_lens, *qsl, *q_abs;
    int causal;
    int Hkv, G, block_size;
    float scale_log2e;
    void *out;
    int64_t o_ts, o_hs;
    float *ws_o, *ws_ml;
    int split_len, max_splits;
    int dec_rows_max;  // rows handled by the decode kernel
};

__device__ __forceinline__ float4_t mfma16(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float hlo(uint32_t w) { return half_bits_to_f32(w & 0xFFFFu); }
__device__ __forceinline__ float hhi(uint32_t w) { return half_bits_to_f32(w >> 16); }

template <int QDT>
__device__ __forceinline__ half8_t load_q8(const void *q, int64_t off) {
    half8_t r;
    if constexpr (QDT == GFA_DTYPE_F16) {
        const uint16_t *p = static_cast<const uint16_t *>(q) + off;
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = __builtin_bit_cast(half_t, p[e]);
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = (half_t)load_as_f32<QDT>(q, off + e);
    }
    return r;
}

template <int ODT>
__device__ __forceinline__ void store_out(void *out, int64_t off, float v) {
    if constexpr (ODT == GFA_DTYPE_F32) {
        static_cast<float *>(out)[off] = v;
    } else if constexpr (ODT == GFA_DTYPE_F16) {
        static_cast<half_t *>(out)[off] = (half_t)v;
    } else {
        // fp32 -> bf16, round to nearest even (inputs are finite here)
        const uint32_t u = __float_as_uint(v);
        const uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
        static_cast<uint16_t *>(out)[off] = (uint16_t)r;
    }
}

// Raw operand registers for one 16-token sub-page.
struct SubPage {
    u32x4 kq[2], ks[2], vq[2], vs[2];
};

template <bool NT>
__device__ __forceinline__ void load_subpage(SubPage &sp, const uint8_t *kb, const uint8_t *vb,
                                             int i16, int g) {
    const u32x4 *k0 = reinterpret_cast<const u32x4 *>(kb + i16 * 128 + 32 * g);
    const u32x4 *ks = reinterpret_cast<const u32x4 *>(kb + SCALE_OFF + 32 * g);
    const u32x4 *v0 = reinterpret_cast<const u32x4 *>(vb + (16 * g + i16) * 32);
    const u32x4 *vs = reinterpret_cast<const u32x4 *>(vb + SCALE_OFF + 32 * g);
    if constexpr (NT) {  // each KV byte is read once: keep it out of the caches
        sp.kq[0] = __builtin_nontemporal_load(k0);
        sp.kq[1] = __builtin_nontemporal_load(k0 + 1);
        sp.vq[0] = __builtin_nontemporal_load(v0);
        sp.vq[1] = __builtin_nontemporal_load(v0 + 1);
    } else {
        sp.kq[0] = k0[0];
        sp.kq[1] = k0[1];
        sp.vq[0] = v0[0];
        sp.vq[1] = v0[1];
    }
    sp.ks[0] = ks[0];
    sp.ks[1] = ks[1];
    sp.vs[0] = vs[0];
    sp.vs[1] = vs[1];
}

__device__ __forceinline__ uint32_t dw(const u32x4 (&v)[2], int i) { return v[i >> 2][i & 3]; }

// Per-wave online-softmax state for NRG groups of 16 rows.  m is in scaled
// log2 units (score * scale * log2 e).
template <int NRG>
struct WaveAcc {
    float4_t o[NRG][8];
    float m[NRG];
    float l[NRG];
};

template <int NRG>
__device__ __forceinline__ void acc_init(WaveAcc<NRG> &a) {
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
        a.m[rg] = -INFINITY;
        a.l[rg] = 0.0f;
#pragma unroll
        for (int mm = 0; mm < 8; ++mm) a.o[rg][mm] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
}

// Lazy rescaling: the running max m only moves when a row's new max exceeds
// it by more than LAZY_TAU (log2 units), so O and l are rescaled rarely.
// p <= 2^LAZY_TAU keeps p * d_v within fp16 range for any fp16 V
// (d_v <= 65504/127) and for bf16 V with |v| < 1.3e5.
constexpr float LAZY_TAU = 6.0f;

__device__ __forceinline__ float4_t mfma16k16(half4_t a, half4_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// One 16-token sub-page starting at tok0.
//   QK: 4 x mfma 16x16x32 (one per Q8 block), K scales on the fp32 products.
//   PV: 8 x mfma 16x16x16 (one per 16 d); lane (i, g) feeds tokens 4g..4g+3,
//       the same tokens its S^T fragment holds, so P needs no shuffles.
// mask (wave-uniform): apply kv_end and the per-row causal bounds lim[rg].
template <int NRG>
__device__ __forceinline__ void attend_subpage(WaveAcc<NRG> &acc, const SubPage &sp,
                                               const half8_t (&qf)[NRG][4], int tok0, int kv_end,
                                               const int (&lim)[NRG], float c, int g, bool mask) {
    half8_t ka[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) ka[b] = i8x8_to_half8(dw(sp.kq, 2 * b), dw(sp.kq, 2 * b + 1));
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
        float4_t cb[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) cb[b] = mfma16(ka[b], qf[rg][b], float4_t{0.f, 0.f, 0.f, 0.f});
        float sv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // K scales of token 4g+i: blocks (0,1), (2,3)
            const uint32_t s01 = dw(sp.ks, 2 * i), s23 = dw(sp.ks, 2 * i + 1);
            float v = cb[0][i] * hlo(s01);
            v = fmaf(cb[1][i], hhi(s01), v);
            v = fmaf(cb[2][i], hlo(s23), v);
            sv[i] = fmaf(cb[3][i], hhi(s23), v);
        }
        if (mask) {  // uniform: only partial / causal-diagonal sub-pages
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = tok0 + 4 * g + i;
                sv[i] = (key < kv_end && key <= lim[rg]) ? sv[i] : -INFINITY;
            }
        }
        float mt = xrow_max(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]))) * c;
        const bool need = mt > acc.m[rg] + LAZY_TAU;
        if (__builtin_amdgcn_ballot_w64(need)) {  // wave-uniform, rare after warm-up
            const float mn = need ? mt : acc.m[rg];
            // 0 when m was -inf (nothing accumulated yet); 1 for rows that keep m
            const float alpha = need ? __builtin_amdgcn_exp2f(acc.m[rg] - mn) : 1.0f;
            acc.m[rg] = mn;
            acc.l[rg] *= alpha;
#pragma unroll
            for (int mm = 0; mm < 8; ++mm) acc.o[rg][mm] *= alpha;
        }
        const float nms = acc.m[rg] == -INFINITY ? 0.0f : -acc.m[rg];
        float pr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) pr[i] = __builtin_amdgcn_exp2f(fmaf(sv[i], c, nms));
        acc.l[rg] += (pr[0] + pr[1]) + (pr[2] + pr[3]);
        // P'_b[i] = p[i] * d_v[4g + i][b] in packed fp16: the V scale table keeps
        // the four tokens of a lane group adjacent per block, so dword 2b holds
        // the scales of tokens (4g, 4g+1) and dword 2b+1 those of (4g+2, 4g+3).
        const half2_t p01 = {(half_t)pr[0], (half_t)pr[1]};
        const half2_t p23 = {(half_t)pr[2], (half_t)pr[3]};
        half4_t pb[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const half2_t a = p01 * __builtin_bit_cast(half2_t, dw(sp.vs, 2 * b));
            const half2_t c2 = p23 * __builtin_bit_cast(half2_t, dw(sp.vs, 2 * b + 1));
            pb[b] = half4_t{a[0], a[1], c2[0], c2[1]};
        }
#pragma unroll
        for (int mm = 0; mm < 8; ++mm) {
            half2_t lo, hi;
            i8x4_to_f16x4(dw(sp.vq, mm), lo, hi);
            const half4_t va = {lo[0], lo[1], hi[0], hi[1]};
            acc.o[rg][mm] = mfma16k16(va, pb[mm >> 1], acc.o[rg][mm]);
        }
    }
}

// Loads the Q^T fragments and per-row causal bounds for rows row0 + 16*rg + i16.
template <int NRG, int QDT>
__device__ __forceinline__ void load_rows(const AttnParams &p, int h, int q0, int nrows, int row0,
                                          int sl, int qa, int i16, int g, half8_t (&qf)[NRG][4],
                                          int (&lim)[NRG]) {
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
        const int r = row0 + 16 * rg + i16;
        if (r < nrows) {
            const int j = r / p.G;
            const int hq = h * p.G + (r - j * p.G);
            const int64_t qoff = (int64_t)(q0 + j) * p.q_ts + (int64_t)hq * p.q_hs;
#pragma unroll
            for (int b = 0; b < 4; ++b) qf[rg][b] = load_q8<QDT>(p.q, qoff + 32 * b + 8 * g);
            lim[rg] = p.causal ? min(sl - 1, qa + j) : sl - 1;
        } else {
#pragma unroll
            for (int b = 0; b < 4; ++b) qf[rg][b] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
            lim[rg] = INT32_MAX;  // padding rows never limit the unmasked test
        }
    }
}

// Streams the keys [wb, we) (wb a multiple of 16) through the wave, two
// sub-pages per k-step, with register ping-pong prefetch one k-step ahead.
// Page ids come from a lane-distributed copy of the block table (lane i holds
// the page of sub-page 64*chunk + i), refreshed one chunk ahead, so no load in
// the loop depends on another load.
template <int NRG, bool NT, int DEPTH>
__device__ __forceinline__ void stream_range(WaveAcc<NRG> &acc, const AttnParams &p, int s, int h,
                                             int wb, int we, const half8_t (&qf)[NRG][4],
                                             const int (&lim)[NRG], int lane, int i16, int g) {
    const int nsub = (we - wb + 15) >> 4;
    if (nsub <= 0) return;
    const int32_t *btrow = p.bt + (int64_t)s * p.bt_stride;
    const uint8_t *kbase = p.kc + (int64_t)h * p.chs;
    const uint8_t *vbase = p.vc + (int64_t)h * p.chs;
    const int bs = p.block_size;
    auto load_pg = [&](int chunk) -> int {
        const int j = 64 * chunk + lane;
        return j < nsub ? btrow[(wb + 16 * j) / bs] : 0;
    };
    int pg_cur = load_pg(0);
    int pg_nxt = nsub > 64 ? load_pg(1) : 0;
    int chunk = 0;
    // smallest causal bound over the wave's real rows: a k-step entirely below
    // it (and below we) needs no mask
    int lim_min = lim[0];
#pragma unroll
    for (int rg = 1; rg < NRG; ++rg) lim_min = min(lim_min, lim[rg]);
    {
        // wave-wide min (exact in fp32: bounds are clamped to 2^24)
        const float f = (float)min(lim_min, 1 << 24);
        lim_min = __builtin_amdgcn_readfirstlane((int)(-row16_max(xrow_max(-f))));
    }
    const float c = p.scale_log2e;

    auto fetch = [&](SubPage &sp, int j) {
        if (j < nsub) {
            if ((j >> 6) != chunk) {  // advance the page-id window (uniform)
                chunk = j >> 6;
                pg_cur = pg_nxt;
                pg_nxt = 64 * (chunk + 1) < nsub ? load_pg(chunk + 1) : 0;
            }
            const int tb = wb + 16 * j;
            const int64_t page = __builtin_amdgcn_readlane(pg_cur, j & 63);
            const int64_t off = page * p.cbs + (int64_t)((tb % bs) >> 4) * SUBPAGE_BYTES;
            load_subpage<NT>(sp, kbase + off, vbase + off, i16, g);
        }
    };
    // ring of DEPTH sub-page buffers: DEPTH-1 sub-pages in flight while one computes
    SubPage buf[DEPTH];
#pragma unroll
    for (int u = 0; u < DEPTH - 1; ++u) fetch(buf[u], u);
    for (int base = 0; base < nsub; base += DEPTH) {
#pragma unroll
        for (int u = 0; u < DEPTH; ++u) {
            const int j = base + u;
            if (j >= nsub) break;
            fetch(buf[(u + DEPTH - 1) % DEPTH], j + DEPTH - 1);
            const int tok0 = wb + 16 * j;
            attend_subpage<NRG>(acc, buf[u], qf, tok0, we, lim, c, g,
                                !(tok0 + 16 <= we && tok0 + 15 <= lim_min));
        }
    }
}

// ---------------------------------------------------------------------------
// Decode / verify kernel.  grid (max_splits, Hkv, num_seqs), block 64*NW.
template <int NRG, int NW, int QDT, int ODT>
__global__ __launch_bounds__(64 * NW) void attn_decode_kernel(AttnParams p) {
    const int s = blockIdx.z, h = blockIdx.y, split = blockIdx.x;
    const int q0 = p.qsl[s];
    const int nq = p.qsl[s + 1] - q0;
    const int nrows = nq * p.G;
    if (nq <= 0 || nrows > p.dec_rows_max) return;
    const int sl = p.seq_lens[s];
    const int qa = p.q_abs ? p.q_abs[s] : sl - nq;
    const int kv_lim = p.causal ? min(sl, max(qa + nq, 0)) : sl;
    // never more splits than the workspace holds; the last one takes the rest
    const int nsplit = min(max(1, (kv_lim + p.split_len - 1) / p.split_len), p.max_splits);
    if (split >= nsplit) return;
    const int kv_begin = split * p.split_len;
    const int kv_end = split == nsplit - 1 ? kv_lim : min(kv_lim, kv_begin + p.split_len);

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int i16 = lane & 15, g = lane >> 4;
    half8_t qf[NRG][4];
    int lim[NRG];
    load_rows<NRG, QDT>(p, h, q0, nrows, 0, sl, qa, i16, g, qf, lim);

    WaveAcc<NRG> acc;
    acc_init(acc);
    // wave w streams a contiguous quarter of the split (whole k-steps)
    const int chunk = ((kv_end - kv_begin + NW - 1) / NW + 31) & ~31;
    const int wb = min(kv_end, kv_begin + w * chunk);
    const int we = min(kv_end, wb + chunk);
    stream_range<NRG, true, DEC_DEPTH>(acc, p, s, h, wb, we, qf, lim, lane, i16, g);
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) acc.l[rg] = xrow_sum(acc.l[rg]);

    constexpr int R = 16 * NRG;
    __shared__ float sm_o[NW][R][128 + 4];
    __shared__ float sm_m[NW][R], sm_l[NW][R];
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
        const int r = 16 * rg + i16;
        if (g == 0) {
            sm_m[w][r] = acc.m[rg];
            sm_l[w][r] = acc.l[rg];
        }
#pragma unroll
        for (int mm = 0; mm < 8; ++mm)
#pragma unroll
            for (int i = 0; i < 4; ++i) sm_o[w][r][16 * mm + 4 * g + i] = acc.o[rg][mm][i];
    }
    __syncthreads();

    // merge the NW waves; thread -> (row, 4 consecutive d)
    for (int it = threadIdx.x; it < R * 32; it += 64 * NW) {
        const int r = it >> 5, d0 = (it & 31) * 4;
        if (r >= nrows) continue;
        float mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < NW; ++k) mx = fmaxf(mx, sm_m[k][r]);
        const float ms = mx == -INFINITY ? 0.0f : mx;
        float l = 0.f, o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
#pragma unroll
        for (int k = 0; k < NW; ++k) {
            const float wk = __builtin_amdgcn_exp2f(sm_m[k][r] - ms);
            l = fmaf(sm_l[k][r], wk, l);
            o0 = fmaf(sm_o[k][r][d0 + 0], wk, o0);
            o1 = fmaf(sm_o[k][r][d0 + 1], wk, o1);
            o2 = fmaf(sm_o[k][r][d0 + 2], wk, o2);
            o3 = fmaf(sm_o[k][r][d0 + 3], wk, o3);
        }
        if (nsplit == 1) {
            const int j = r / p.G;
            const int hq = h * p.G + (r - j * p.G);
            const int64_t ob = (int64_t)(q0 + j) * p.o_ts + (int64_t)hq * p.o_hs + d0;
            const float inv = l > 0.f ? 1.0f / l : 0.0f;
            store_out<ODT>(p.out, ob + 0, o0 * inv);
            store_out<ODT>(p.out, ob + 1, o1 * inv);
            store_out<ODT>(p.out, ob + 2, o2 * inv);
            store_out<ODT>(p.out, ob + 3, o3 * inv);
        } else {
            const int64_t slot = (((int64_t)s * p.Hkv + h) * ROWS_CAP + r) * p.max_splits + split;
            *reinterpret_cast<float4_t *>(p.ws_o + slot * 128 + d0) = float4_t{o0, o1, o2, o3};
            if (d0 == 0) {
                p.ws_ml[2 * slot] = mx;
                p.ws_ml[2 * slot + 1] = l;
            }
        }
    }
}

// Merge split partials.  grid (Hkv, num_seqs), block 256: thread -> (row, 4 d).
template <int ODT>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnParams p) {
    const int s = blockIdx.y, h = blockIdx.x;
    const int q0 = p.qsl[s];
    const int nq = p.qsl[s + 1] - q0;
    const int nrows = nq * p.G;
    if (nq <= 0 || nrows > p.dec_rows_max) return;
    const int sl = p.seq_lens[s];
    const int qa = p.q_abs ? p.q_abs[s] : sl - nq;
    const int kv_lim = p.causal ? min(sl, max(qa + nq, 0)) : sl;
    const int nsplit = min(max(1, (kv_lim + p.split_len - 1) / p.split_len), p.max_splits);
    if (nsplit == 1) return;
    for (int it = threadIdx.x; it < ROWS_CAP * 32; it += 256) {
        const int r = it >> 5, d0 = (it & 31) * 4;
        if (r >= nrows) continue;
        const int64_t slot0 = (((int64_t)s * p.Hkv + h) * ROWS_CAP + r) * p.max_splits;
        float mx = -INFINITY;
        for (int k = 0; k < nsplit; ++k) mx = fmaxf(mx, p.ws_ml[2 * (slot0 + k)]);
        const float ms = mx == -INFINITY ? 0.0f : mx;
        float l = 0.f;
        float4_t o = {0.f, 0.f, 0.f, 0.f};
        for (int k = 0; k < nsplit; ++k) {
            const float wk = __builtin_amdgcn_exp2f(p.ws_ml[2 * (slot0 + k)] - ms);
            l = fmaf(p.ws_ml[2 * (slot0 + k) + 1], wk, l);
            const float4_t ok = *reinterpret_cast<const float4_t *>(p.ws_o + (slot0 + k) * 128 + d0);
            o += ok * wk;
        }
        const int j = r / p.G;
        const int hq = h * p.G + (r - j * p.G);
        const int64_t ob = (int64_t)(q0 + j) * p.o_ts + (int64_t)hq * p.o_hs + d0;
        const float inv = l > 0.f ? 1.0f / l : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) store_out<ODT>(p.out, ob + i, o[i] * inv);
    }
}

// ---------------------------------------------------------------------------
// Prefill kernel.  grid (row_tiles, Hkv, num_seqs), block 64*NW; wave w of
// workgroup x owns rows [64*(NW*x + w), +64) of (seq, kv-head).
template <int NW, int QDT, int ODT>
__global__ __launch_bounds__(64 * NW) void attn_prefill_kernel(AttnParams p) {
    constexpr int NRG = PF_NRG;
    const int s = blockIdx.z, h = blockIdx.y;
    const int q0 = p.qsl[s];
    const int nq = p.qsl[s + 1] - q0;
    const int nrows = nq * p.G;
    if (nq <= 0 || nrows <= p.dec_rows_max) return;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int row0 = 16 * NRG * (NW * blockIdx.x + w);
    if (row0 >= nrows) return;  // whole wave; no barriers in this kernel
    const int i16 = lane & 15, g = lane >> 4;
    const int sl = p.seq_lens[s];
    const int qa = p.q_abs ? p.q_abs[s] : sl - nq;
    const int jlast = (min(row0 + 16 * NRG, nrows) - 1) / p.G;
    const int kv_end = p.causal ? min(sl, max(qa + jlast + 1, 0)) : sl;

    half8_t qf[NRG][4];
    int lim[NRG];
    load_rows<NRG, QDT>(p, h, q0, nrows, row0, sl, qa, i16, g, qf, lim);
    WaveAcc<NRG> acc;
    acc_init(acc);
    stream_range<NRG, false, 2>(acc, p, s, h, 0, kv_end, qf, lim, lane, i16, g);
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
        const float l = xrow_sum(acc.l[rg]);
        const int r = row0 + 16 * rg + i16;
        if (r >= nrows) continue;
        const int j = r / p.G;
        const int hq = h * p.G + (r - j * p.G);
        const int64_t ob = (int64_t)(q0 + j) * p.o_ts + (int64_t)hq * p.o_hs;
        const float inv = l > 0.f ? 1.0f / l : 0.0f;
#pragma unroll
        for (int mm = 0; mm < 8; ++mm)
#pragma unroll
            for (int i = 0; i < 4; ++i) store_out<ODT>(p.out, ob + 16 * mm + 4 * g + i, acc.o[rg][mm][i] * inv);
    }
}

// ---------------------------------------------------------------------------
// Host-side plan.  Deterministic in the call's scalar arguments so that
// workspace_size() and the launch agree.
struct Plan {
    int dec_rows_max;   // 16 or 32
    int dec_nrg;        // 1 or 2
    int split_len;      // tokens per split, multiple of 32*DEC_NW
    int max_splits;
    bool need_prefill;
    size_t ws_o_floats, ws_ml_floats;
};


Plan make_plan(int num_seqs, int num_heads, int num_kv_heads, int max_query_len, int max_seq_len) {
    Plan pl;
    const int G = num_heads / num_kv_heads;
    const int max_rows = max_query_len * G;
    pl.dec_nrg = (max_rows <= 16) ? 1 : 2;
    pl.dec_rows_max = 16 * pl.dec_nrg;
    pl.need_prefill = max_rows > pl.dec_rows_max;
    // Split-K: aim for ~2048 (seq, kv-head, split) workgroups at the longest
    // context, keep each split >= 64 tokens per decode row so the partials
    // stay a few percent of the KV bytes, and round to whole k-steps.
    const int step = 32 * DEC_NW;
    int64_t target = ((int64_t)num_seqs * num_kv_heads * (int64_t)max(max_seq_len, 1)) / 2048;
    int64_t minlen = 64LL * pl.dec_rows_max;
    int64_t sl = max(target, minlen);
    sl = ((sl + step - 1) / step) * step;
    if (sl > (1 << 30)) sl = 1 << 30;
    pl.split_len = (int)sl;
    pl.max_splits = max(1, (max_seq_len + pl.split_len - 1) / pl.split_len);
    if (pl.max_splits > 1) {
        pl.ws_o_floats = (size_t)num_seqs * num_kv_heads * ROWS_CAP * pl.max_splits * 128;
        pl.ws_ml_floats = (size_t)num_seqs * num_kv_heads * ROWS_CAP * pl.max_splits * 2;
    } else {
        pl.ws_o_floats = pl.ws_ml_floats = 0;
    }
    return pl;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

template <int QDT, int ODT>
hipError_t launch_all(const AttnParams &p0, const Plan &pl, int num_seqs, int num_kv_heads,
                      int max_query_len, hipStream_t stream) {
    AttnParams p = p0;
    dim3 dgrid(pl.max_splits, num_kv_heads, num_seqs);
    if (pl.dec_nrg == 1)
        attn_decode_kernel<1, DEC_NW, QDT, ODT><<<dgrid, 64 * DEC_NW, 0, stream>>>(p);
    else
        attn_decode_kernel<2, DEC_NW, QDT, ODT><<<dgrid, 64 * DEC_NW, 0, stream>>>(p);
    if (pl.max_splits > 1)
        attn_combine_kernel<ODT><<<dim3(num_kv_heads, num_seqs), 256, 0, stream>>>(p);
    if (pl.need_prefill) {
        const int rows = max_query_len * p.G;
        const int tiles = (rows + 16 * PF_NRG * PF_NW - 1) / (16 * PF_NRG * PF_NW);
        attn_prefill_kernel<PF_NW, QDT, ODT><<<dim3(tiles, num_kv_heads, num_seqs), 64 * PF_NW, 0, stream>>>(p);
    }
    return hipGetLastError();
}

}  // namespace

extern "C" size_t gfx906_fa_amd_paged_attention_workspace_size(int num_seqs, int num_tokens,
                                                               int num_heads, int num_kv_heads,
                                                               int head_size, int max_query_len,
                                                               int max_seq_len) {
    (void)num_tokens;
    (void)head_size;
    if (num_seqs <= 0 || num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads) return 0;
    const Plan pl = make_plan(num_seqs, num_heads, num_kv_heads, max(max_query_len, 1), max_seq_len);
    if (pl.max_splits <= 1) return 0;
    return align256(pl.ws_o_floats * 4) + align256(pl.ws_ml_floats * 4);
}

extern "C" hipError_t gfx906_fa_amd_paged_attention(
    const void *q, int q_dtype, int64_t q_token_stride, int64_t q_head_stride,
    const uint8_t *k_cache, const uint8_t *v_cache, int64_t cache_block_stride,
    int64_t cache_head_stride, const int32_t *block_table, int64_t block_table_stride,
    const int32_t *seq_lens, const int32_t *query_start_loc, const int32_t *q_abs_offset,
    int causal, int num_seqs, int num_tokens, int num_heads, int num_kv_heads, int head_size,
    int block_size, int max_query_len, int max_seq_len, float scale, void *out, int out_dtype,
    int64_t out_token_stride, int64_t out_head_stride, void *workspace, size_t workspace_bytes,
    hipStream_t stream) {
    if (num_seqs == 0 || num_tokens == 0) return hipSuccess;
    if (head_size != 128) {
        fprintf(stderr, "[gfx906_fa_amd] paged_attention: head_size=%d unsupported (only 128)\n", head_size);
        return hipErrorInvalidValue;
    }
    if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0) {
        fprintf(stderr, "[gfx906_fa_amd] paged_attention: num_heads=%d not divisible by num_kv_heads=%d\n",
                num_heads, num_kv_heads);
        return hipErrorInvalidValue;
    }
    if (block_size <= 0 || block_size % 16 != 0) {
        fprintf(stderr, "[gfx906_fa_amd] paged_attention: block_size=%d must be a multiple of 16\n", block_size);
        return hipErrorInvalidValue;
    }
    if ((((uintptr_t)k_cache | (uintptr_t)v_cache) | (uint64_t)cache_block_stride |
         (uint64_t)cache_head_stride) & 15u) {
        fprintf(stderr, "[gfx906_fa_amd] paged_attention: cache bases and strides must be 16-byte aligned\n");
        return hipErrorInvalidValue;
    }
    if (q_dtype < 0 || q_dtype > 2 || out_dtype < 0 || out_dtype > 2 || num_seqs < 0 ||
        max_query_len < 0 || max_seq_len < 0) {
        fprintf(stderr, "[gfx906_fa_amd] paged_attention: bad dtype or size\n");
        return hipErrorInvalidValue;
    }
    const int G = num_heads / num_kv_heads;
    const Plan pl = make_plan(num_seqs, num_heads, num_kv_heads, max(max_query_len, 1), max_seq_len);
    const size_t need = pl.max_splits > 1 ? align256(pl.ws_o_floats * 4) + align256(pl.ws_ml_floats * 4) : 0;
    if (need > 0 && (workspace == nullptr || workspace_bytes < need || ((uintptr_t)workspace & 255u))) {
        fprintf(stderr, "[gfx906_fa_amd] paged_attention: workspace of %zu bytes (256-aligned) required, got %zu\n",
                need, workspace_bytes);
        return hipErrorInvalidValue;
    }
    AttnParams p;
    p.q = q;
    p.q_ts = q_token_stride;
    p.q_hs = q_head_stride;
    p.kc = k_cache;
    p.vc = v_cache;
    p.cbs = cache_block_stride;
    p.chs = cache_head_stride;
    p.bt = block_table;
    p.bt_stride = block_table_stride;
    p.seq_lens = seq_lens;
    p.qsl = query_start_loc;
    p.q_abs = q_abs_offset;
    p.causal = causal ? 1 : 0;
    p.Hkv = num_kv_heads;
    p.G = G;
    p.block_size = block_size;
    p.scale_log2e = scale * LOG2E;
    p.out = out;
    p.o_ts = out_token_stride;
    p.o_hs = out_head_stride;
    p.ws_o = need ? static_cast<float *>(workspace) : nullptr;
    p.ws_ml = need ? reinterpret_cast<float *>(static_cast<char *>(workspace) + align256(pl.ws_o_floats * 4)) : nullptr;
    p.split_len = pl.split_len;
    p.max_splits = pl.max_splits;
    p.dec_rows_max = pl.dec_rows_max;

#define GFA_DISPATCH_O(QDT)                                                                    \
    switch (out_dtype) {                                                                       \
        case GFA_DTYPE_F32: return launch_all<QDT, GFA_DTYPE_F32>(p, pl, num_seqs, num_kv_heads, max_query_len, stream); \
        case GFA_DTYPE_F16: return launch_all<QDT, GFA_DTYPE_F16>(p, pl, num_seqs, num_kv_heads, max_query_len, stream); \
        default: return launch_all<QDT, GFA_DTYPE_BF16>(p, pl, num_seqs, num_kv_heads, max_query_len, stream); \
    }
    switch (q_dtype) {
        case GFA_DTYPE_F32: GFA_DISPATCH_O(GFA_DTYPE_F32);
        case GFA_DTYPE_F16: GFA_DISPATCH_O(GFA_DTYPE_F16);
        default: GFA_DISPATCH_O(GFA_DTYPE_BF16);
    }
#undef GFA_DISPATCH_O
}
