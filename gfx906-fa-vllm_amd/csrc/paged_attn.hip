// paged_attn.hip - direct-paged Q8_0 attention for gfx950 (decode, chunked
// prefill, mixed batches, speculative verify).
//
// Semantics follow the reference's paged FA (kernel/fattn-q8-paged.cuh:381-641,
// causal rule kernel/fattn-q8.cuh:646-653, GQA map kernel/fattn-q8.cuh:898-901,
// kv cutoff extension/gfx906_fa.cpp:595-604) with dequantize-then-fp32 math.
//
// Formulation (wave64, fp16 MFMA, fp32 accumulation), transposed so a lane
// owns one query row:
//   S^T[16 tok x 16 rows] = K[16 tok x 32 d] . Q^T[32 d x 16 rows]
//       one v_mfma_f32_16x16x32_f16 per Q8 block of d
//   O^T[16 d x 16 rows]  += V^T[16 d x 16 tok] . P'^T[16 tok x 16 rows]
//       one v_mfma_f32_16x16x16_f16 per 16 d
// Lane l = 16*g + i: row i (column of S^T / O^T), token group / d group g.
// A lane dequantizes the K values of its own token to fp16 once per sub-page
// (K^ = q * d_k, one rounding), and the four MFMAs of the row group
// accumulate into one chain.  V int8 values enter the MFMA exactly;
// the V scale d_v[t][b] is folded into P (P'_b[t] = p[t] * d_v[t][b], fp16)
// for the MFMAs of d-block b.  Softmax statistics and O accumulate in fp32.
//
// The planar page layout (include/gfx906_fa_amd.h) makes every operand an
// aligned 16-byte load straight from HBM, each wave-wide load instruction
// covering 1 KB contiguous: per 16-token sub-page a lane loads 32 B of K
// ints, 32 B of K scales, 32 B of V ints and 32 B of V scales.
//
// Query rows are GQA-packed: rows of one kv-head are r = j*G + gq (token j,
// q-head h*G + gq), so one K/V stream serves all G query heads.
//
//   attn_decode_kernel   sequences with n_q*G <= 64 rows (decode, verify):
//                        stream-K over all KV sub-pages, equal share per wave;
//                        16-, 32- or 48-row tiles per wave, 64 rows in two
//                        32-row chunks
//   attn_prefill_kernel  sequences with more rows: 128-row workgroups share
//                        K/V tiles dequantized to fp16 in LDS; 32x32x16 MFMA
#include <atomic>
#include <cstdio>
#include <mutex>
#include <type_traits>

#include "q8_common.h"

using namespace gfa;

namespace {

constexpr float LOG2E = 1.4426950408889634f;
// Tuning knobs (compile-time; defaults measured on MI355X).
#ifndef GFA_DEC_DEPTH
#define GFA_DEC_DEPTH 2
#endif
#ifndef GFA_DEC_NT
#define GFA_DEC_NT 1
#endif
#ifndef GFA_DEC_WPE
#define GFA_DEC_WPE 3
#endif
constexpr int DEC_DEPTH = GFA_DEC_DEPTH;  // decode sub-page ring depth (DEPTH-1 in flight)

struct AttnParams {
    const void *q;
    int64_t q_ts, q_hs;
    const uint8_t *kc, *vc;
    int64_t cbs, chs;    // K (and Q8 V) plane strides in bytes: page, kv-head
    int64_t vcbs, vchs;  // V plane strides (equal to cbs, chs for a Q8 V plane)
    const uint16_t *mask;             // optional additive fp16 mask [B][n_q][mask_cols]
    int64_t mask_bs, mask_rs;         // its batch and row strides (elements)
    int mask_cols;                    // keys it covers
    int mask_vec;                     // rows 8-byte aligned, mask_cols % 4 == 0: 4 keys per load
    const int32_t *bt;
    int64_t bt_stride;
    const int32_t *seq_lens, *qsl, *q_abs;
    int causal;
    int Hkv, G, block_size;
    float scale_log2e;
    float pf_qmul, pf_kmul;  // prefill: Q * 2^-e and K^ * (c * 2^e), c = scale_log2e (qmul * kmul = c)
    void *out;
    int64_t o_ts, o_hs;
    float *ws_ml, *ws_o;  // partial (m, l) and O per slot row
    int64_t *ws_hdr;      // decode plan published for the combine kernel: U, nwg
    int *ws_pre;          // per-sequence exclusive prefix of decode sub-pages
    int num_seqs, nwg;    // nwg: decode workgroups (the grid)
    int dec_rows_lo;      // a decode launch takes sequences with dec_rows_lo < n_q*G
    int dec_rows_max;     //   <= dec_rows_max; the prefill kernel takes n_q*G > dec_rows_max
                          //   (in a decode launch also the rows of its partial slots)
    // prefill work list (heaviest first) built by prefill_plan_kernel: item i
    // is key tiles [pf_kt0[i], pf_kt1[i]) of row tile pf_rt[i] of sequence
    // pf_seq[i], *pf_count items; pf_slot[i] >= 0: a piece of a split row
    // tile, whose partial (m, l, O) goes to partial slot pf_slot[i] (merged
    // by attn_prefill_combine_kernel), else the piece is the whole row tile
    // and writes the output.  nullptr: the prefill grid is
    // (row tiles * Hkv, num_seqs) instead, with no split.
    int *pf_seq, *pf_rt, *pf_kt0, *pf_kt1, *pf_slot, *pf_count;
    int pf_rows;        // query rows per prefill row tile: PF_ROWS, or PF_ROWS / 2 (KS = 2 tiles)
    int pf_items_max;   // row tiles, at most
    int pf_grid_items;  // work-list capacity (the grid): row tiles + extra pieces
    int pf_ncu;         // CUs the split targets
    int pf_split_max;   // split row tiles, at most
    int pf_slots_max;   // partial slots per kv head
    int *pf_split;      // split row tiles: (sequence, row tile, first slot, pieces) each
    float *pf_ml, *pf_o;  // partials: [slot][Hkv][pf_rows] x (m, l) and x 128
    // Dequantized tile images (work-list launches only; nullptr: none): the
    // fp16 K^ and V^T of 64-key tile kt of prefill sequence s for kv-head h,
    // byte for byte the prefill kernel's LDS stages, at image
    // (pf_tbase[s] + kt) * Hkv + h of pf_tiles, written once per call by
    // prefill_tiles_kernel when every image fits pf_tiles_cap bytes and the
    // row tiles read each key tile PF_IMG_REUSE times on average (the plan
    // kernel decides: pf_count[2], pf_count[3] = image tiles per kv-head);
    // the prefill workgroups then copy them into LDS instead of dequantizing
    // every tile themselves.
    uint8_t *pf_tiles;
    int *pf_tbase;      // per sequence (num_seqs + 1): first image tile
    int64_t pf_tiles_cap;
    // Fused cache write of the step's new tokens (decode kernels only; nullptr:
    // none).  Row qsl[s] + j of new_k / new_v (the query dtype) holds the key /
    // value of position seq_lens[s] - n_q + j, written at slot new_slot[row].
    const void *new_k, *new_v;
    int64_t nk_ts, nk_hs, nv_ts, nv_hs;  // element strides
    const int64_t *new_slot;
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
    u32x4 kq[2];
    u32x2 ks;  // the four block scales of the lane's token i16
    u32x4 vq[2], vs[2];
};

// Per-lane byte offsets of a lane's operands inside a 2176-byte sub-page.
struct LaneOffsets {
    uint32_t kq, ks, vq, vs;
};

__device__ __forceinline__ LaneOffsets lane_offsets(int i16, int g) {
    LaneOffsets o;
    o.kq = (4 * i16 + g) * 16;          // K ints of token i16, group g: +0 and +1024
    o.ks = SCALE_OFF + 8 * i16;         // K scales of token i16, blocks 0..3
    o.vq = (16 * g + i16) * 16;         // V ints, d = 16m + i16, tokens 4g..4g+3: +0 and +1024
    o.vs = SCALE_OFF + 32 * g;          // V scales of tokens 4g..4g+3
    return o;
}

// kb / vb are wave-uniform sub-page bases; lane offsets are 32-bit, so the
// loads use the scalar-base + vector-offset addressing form.
template <bool NT>
__device__ __forceinline__ void load_subpage(SubPage &sp, const uint8_t *kb, const uint8_t *vb,
                                             const LaneOffsets &lo) {
    const u32x4 *k0 = reinterpret_cast<const u32x4 *>(kb + lo.kq);
    const u32x2 *ks = reinterpret_cast<const u32x2 *>(kb + lo.ks);
    const u32x4 *v0 = reinterpret_cast<const u32x4 *>(vb + lo.vq);
    const u32x4 *vs = reinterpret_cast<const u32x4 *>(vb + lo.vs);
    if constexpr (NT) {  // each KV byte is read once: keep it out of the caches
        sp.kq[0] = __builtin_nontemporal_load(k0);
        sp.kq[1] = __builtin_nontemporal_load(k0 + 64);
        sp.vq[0] = __builtin_nontemporal_load(v0);
        sp.vq[1] = __builtin_nontemporal_load(v0 + 64);
    } else {
        sp.kq[0] = k0[0];
        sp.kq[1] = k0[64];
        sp.vq[0] = v0[0];
        sp.vq[1] = v0[64];
    }
    sp.ks = ks[0];
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

// Max of three as the IEEE 754-2019 maximum (NaN-propagating): the compiler
// forms v_maximum3_f32 and, unlike fmaxf on MFMA results, needs no
// canonicalizing v_max_f32 x, x first (a 32-value tree: 16 instructions,
// against 18).  Not inline assembly: the compiler's wait states between an
// MFMA and a VALU read of its result do not cover instructions inside asm
// statements.
__device__ __forceinline__ float max3f(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}
// Max of a lane's four scores the same way: v_maximum + v_maximum3 (fmaxf
// needs two canonicalizing moves and two maxes).
__device__ __forceinline__ float max4f(const float (&v)[4]) {
    return max3f(v[0], v[1], __builtin_elementwise_maximum(v[2], v[3]));
}

__device__ __forceinline__ float4_t mfma16k16(half4_t a, half4_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// One 16-token sub-page starting at tok0.
//   QK: 4 x mfma 16x16x32 (one per Q8 block) in one accumulator chain over
//       K^ = fp16(q * d_k): each lane dequantizes the 32 values of its own
//       token i16 once (v_pk_mul_f16, one rounding), for all row groups.
//   PV: 8 x mfma 16x16x16 (one per 16 d); lane (i, g) feeds tokens 4g..4g+3,
//       the same tokens its S^T fragment holds, so P needs no shuffles.
// mask (wave-uniform): apply kv_end and the per-row causal bounds lim[rg].
template <int NRG>
__device__ __forceinline__ void attend_subpage(WaveAcc<NRG> &acc, const SubPage &sp,
                                               const half8_t (&qf)[NRG][4], int tok0, int kv_end,
                                               const int (&lim)[NRG], float c, int g, bool mask) {
    half8_t ka[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const uint32_t sw = sp.ks[b >> 1];
        const half_t d = __builtin_bit_cast(half2_t, sw)[b & 1];
        const half8_t dd = {d, d, d, d, d, d, d, d};
        ka[b] = i8x8_to_half8(dw(sp.kq, 2 * b), dw(sp.kq, 2 * b + 1)) * dd;
    }
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
        float4_t sacc = mfma16(ka[0], qf[rg][0], float4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int b = 1; b < 4; ++b) sacc = mfma16(ka[b], qf[rg][b], sacc);
        float sv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = sacc[i];  // token 4g + i
        if (mask) {  // uniform: only partial / causal-diagonal sub-pages
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = tok0 + 4 * g + i;
                sv[i] = (key < kv_end && key <= lim[rg]) ? sv[i] : -INFINITY;
            }
        }
        // The lane's max over its 4 keys; a row's max is the largest of its
        // four lanes' (i16 + 16 g), so no lane above m + LAZY_TAU means no row
        // is, and the cross-lane step runs only when some row may rescale.
        const float ml = max4f(sv) * c;
        if (__builtin_amdgcn_ballot_w64(ml > acc.m[rg] + LAZY_TAU)) {  // wave-uniform, rare after warm-up
            const float mt = xrow_max(ml);
            const bool need = mt > acc.m[rg] + LAZY_TAU;
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
// the page of sub-page 64*chunk + i, and the sub-page's index in that page),
// refreshed one chunk ahead, so no load in the loop depends on another load
// and a sub-page's address is scalar arithmetic (no division per sub-page).
// j0 / jstep: the wave takes sub-pages j0, j0 + jstep, ... of the range (the
// waves of a workgroup interleave over one range).
template <int NRG, bool NT, int DEPTH>
__device__ __forceinline__ void stream_range(WaveAcc<NRG> &acc, const AttnParams &p, int s, int h,
                                             int wb, int we, const half8_t (&qf)[NRG][4],
                                             const int (&lim)[NRG], int lane, int i16, int g,
                                             int j0 = 0, int jstep = 1) {
    const int nall = (we - wb + 15) >> 4;
    const int nsub = nall > j0 ? (nall - j0 + jstep - 1) / jstep : 0;  // this wave's sub-pages
    if (nsub <= 0) return;
    const int32_t *btrow = p.bt + (int64_t)s * p.bt_stride;
    const uint8_t *kbase = p.kc + (int64_t)h * p.chs;
    const uint8_t *vbase = p.vc + (int64_t)h * p.chs;
    const int spp = p.block_size >> 4;  // sub-pages per page
    auto load_pg = [&](int chunk, int &spi) -> int {
        const int j = 64 * chunk + lane;
        const int sp = (wb >> 4) + j0 + jstep * j;  // the sub-page's index in the sequence
        const int pi = sp / spp;
        spi = sp - pi * spp;
        return j < nsub ? btrow[pi] : 0;
    };
    int ps_cur = 0, ps_nxt = 0;
    int pg_cur = load_pg(0, ps_cur);
    int pg_nxt = nsub > 64 ? load_pg(1, ps_nxt) : 0;
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
    const LaneOffsets lo = lane_offsets(i16, g);

    auto fetch = [&](SubPage &sp, int j) {
        if (j < nsub) {
            if ((j >> 6) != chunk) {  // advance the page-id window (uniform)
                chunk = j >> 6;
                pg_cur = pg_nxt;
                ps_cur = ps_nxt;
                pg_nxt = 64 * (chunk + 1) < nsub ? load_pg(chunk + 1, ps_nxt) : 0;
            }
            const int64_t page = __builtin_amdgcn_readlane(pg_cur, j & 63);
            const int spi = __builtin_amdgcn_readlane(ps_cur, j & 63);
            const int64_t off = page * p.cbs + (int64_t)spi * SUBPAGE_BYTES;
            load_subpage<NT>(sp, kbase + off, vbase + off, lo);
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
            if (j < nsub) {  // uniform
                fetch(buf[(u + DEPTH - 1) % DEPTH], j + DEPTH - 1);
                const int tok0 = wb + 16 * (j0 + jstep * j);
                attend_subpage<NRG>(acc, buf[u], qf, tok0, we, lim, c, g,
                                    !(tok0 + 16 <= we && tok0 + 15 <= lim_min));
            }
        }
    }
}

// One 16-byte-per-lane copy from global memory straight into LDS
// (global_load_lds_dwordx4: lane i writes lds + 16 i), issued from inline
// assembly.  The compiler counts an LDS DMA issued through its builtin as
// both a global and an LDS access: while one is in flight it waits for every
// LDS read at once (lgkmcnt(0)) and drains the copies at barriers, which
// takes away the overlap the copies are for.  Issued here, the copies are
// invisible to it, and the caller waits for them itself (vmcnt; loads
// complete in order, so any later vector-memory instruction only makes such
// a wait stricter).  M0 holds the LDS address; its previous value is put
// back.  An LDS DMA may not read M0 in the instruction right after an SALU
// write of it (the compiler puts a wait state there for its own copies):
// s_nop 0.  NT: the nontemporal hint (bytes read once; as the register
// path's K/V loads).
template <bool NT>
__device__ __forceinline__ void lds_dma16(const void *src, uint32_t lds) {
    uint32_t saved;
    if constexpr (NT)
        asm volatile("s_mov_b32 %0, m0\n\t"
                     "s_mov_b32 m0, %2\n\t"
                     "s_nop 0\n\t"
                     "global_load_lds_dwordx4 %1, off nt\n\t"
                     "s_mov_b32 m0, %0"
                     : "=&s"(saved)
                     : "v"(src), "s"(lds)
                     : "memory");
    else
        asm volatile("s_mov_b32 %0, m0\n\t"
                     "s_mov_b32 m0, %2\n\t"
                     "s_nop 0\n\t"
                     "global_load_lds_dwordx4 %1, off\n\t"
                     "s_mov_b32 m0, %0"
                     : "=&s"(saved)
                     : "v"(src), "s"(lds)
                     : "memory");
}

constexpr int cmax(int a, int b) { return a > b ? a : b; }
constexpr int DEC_RING_SLOT = 2 * SUBPAGE_BYTES;     // K then V sub-page
#ifndef GFA_DEC_RING
#define GFA_DEC_RING 3
#endif
constexpr int DEC_RING = GFA_DEC_RING;               // LDS ring slots per wave (verify tiles)
constexpr int DEC_RING_DMA = 6;                      // copies per sub-page and wave
static_assert(SUBPAGE_BYTES == 2 * 1024 + 128, "two full copies and an 8-lane one per sub-page");

// stream_range with the sub-pages staged through a per-wave LDS ring of
// DEPTH slots (ring: this wave's LDS, DEPTH * DEC_RING_SLOT bytes): sub-page
// j + DEPTH - 1 is copied into slot (j + DEPTH - 1) % DEPTH while sub-page j
// is computed, so DEPTH - 1 sub-pages are in flight per wave with no
// registers held for them.  The slot a copy fills was read into registers
// (and consumed) in the previous step.
template <int NRG, int DEPTH>
__device__ __forceinline__ void stream_range_lds(WaveAcc<NRG> &acc, const AttnParams &p, int s, int h,
                                                 int wb, int we, const half8_t (&qf)[NRG][4],
                                                 const int (&lim)[NRG], int lane, int i16, int g, int j0,
                                                 int jstep, uint8_t *ring) {
    const int nall = (we - wb + 15) >> 4;
    const int nsub = nall > j0 ? (nall - j0 + jstep - 1) / jstep : 0;  // this wave's sub-pages
    if (nsub <= 0) return;
    const int32_t *btrow = p.bt + (int64_t)s * p.bt_stride;
    const uint8_t *kbase = p.kc + (int64_t)h * p.chs;
    const uint8_t *vbase = p.vc + (int64_t)h * p.chs;
    const int spp = p.block_size >> 4;  // sub-pages per page
    auto load_pg = [&](int chunk, int &spi) -> int {
        const int j = 64 * chunk + lane;
        const int sp = (wb >> 4) + j0 + jstep * j;  // the sub-page's index in the sequence
        const int pi = sp / spp;
        spi = sp - pi * spp;
        return j < nsub ? btrow[pi] : 0;
    };
    // A window load is waited for where it is issued (once per 64
    // sub-pages): the compiler does not see the ring's copies, so a window
    // register still pending at its v_readlane would take a vmcnt(0) there,
    // draining every copy in flight.
    auto ready = [](int &v) __attribute__((always_inline)) { asm volatile("" : "+v"(v)); };
    int ps_cur = 0, ps_nxt = 0;
    int pg_cur = load_pg(0, ps_cur);
    int pg_nxt = nsub > 64 ? load_pg(1, ps_nxt) : 0;
    ready(pg_cur);
    ready(pg_nxt);
    int chunk = 0;
    int lim_min = lim[0];
#pragma unroll
    for (int rg = 1; rg < NRG; ++rg) lim_min = min(lim_min, lim[rg]);
    {
        const float f = (float)min(lim_min, 1 << 24);
        lim_min = __builtin_amdgcn_readfirstlane((int)(-row16_max(xrow_max(-f))));
    }
    const float c = p.scale_log2e;
    const LaneOffsets lo = lane_offsets(i16, g);
    const uint32_t ring_lds =
        __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)ring);

    // copies of sub-page j into slot sl: exactly DEC_RING_DMA per wave
    auto fetch = [&](int j, int sl) __attribute__((always_inline)) {
        if (j < nsub) {  // uniform
            if ((j >> 6) != chunk) {  // advance the page-id window (uniform)
                chunk = j >> 6;
                pg_cur = pg_nxt;
                ps_cur = ps_nxt;
                pg_nxt = 64 * (chunk + 1) < nsub ? load_pg(chunk + 1, ps_nxt) : 0;
                ready(pg_nxt);
            }
            const int64_t page = __builtin_amdgcn_readlane(pg_cur, j & 63);
            const int spi = __builtin_amdgcn_readlane(ps_cur, j & 63);
            const int64_t off = page * p.cbs + (int64_t)spi * SUBPAGE_BYTES;
            const uint8_t *kb = kbase + off + 16 * lane, *vb = vbase + off + 16 * lane;
            const uint32_t dk = ring_lds + sl * DEC_RING_SLOT, dv = dk + SUBPAGE_BYTES;
            constexpr bool NT = GFA_DEC_NT != 0;
            lds_dma16<NT>(kb, dk);
            lds_dma16<NT>(kb + 1024, dk + 1024);
            lds_dma16<NT>(vb, dv);
            lds_dma16<NT>(vb + 1024, dv + 1024);
            if (lane < 8) {  // the last 128 bytes of each
                lds_dma16<NT>(kb + 2048, dk + 2048);
                lds_dma16<NT>(vb + 2048, dv + 2048);
            }
        }
    };
    // sub-page j has landed: the copies of the DEPTH - 1 later sub-pages may
    // still be in flight (all of them issued), else wait for every copy
    auto landed = [&](int j) __attribute__((always_inline)) {
        static_assert(DEC_RING_DMA * (DEPTH - 1) <= 63, "vmcnt immediate");
        if (j + DEPTH - 1 < nsub) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DEC_RING_DMA * (DEPTH - 1)) : "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    };
#pragma unroll
    for (int u = 0; u < DEPTH - 1; ++u) fetch(u, u);
    for (int base = 0; base < nsub; base += DEPTH) {
#pragma unroll
        for (int u = 0; u < DEPTH; ++u) {
            const int j = base + u;
            if (j < nsub) {  // uniform
                // the previous step's reads of the slot refilled next have
                // completed (their values were consumed, but the compiler may
                // place the last uses after this point)
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                fetch(j + DEPTH - 1, (u + DEPTH - 1) % DEPTH);
                landed(j);
                const uint8_t *sb = ring + u * DEC_RING_SLOT;
                SubPage sp;
                sp.kq[0] = *reinterpret_cast<const u32x4 *>(sb + lo.kq);
                sp.kq[1] = *reinterpret_cast<const u32x4 *>(sb + lo.kq + 1024);
                sp.ks = *reinterpret_cast<const u32x2 *>(sb + lo.ks);
                sp.vq[0] = *reinterpret_cast<const u32x4 *>(sb + SUBPAGE_BYTES + lo.vq);
                sp.vq[1] = *reinterpret_cast<const u32x4 *>(sb + SUBPAGE_BYTES + lo.vq + 1024);
                sp.vs[0] = *reinterpret_cast<const u32x4 *>(sb + SUBPAGE_BYTES + lo.vs);
                sp.vs[1] = *reinterpret_cast<const u32x4 *>(sb + SUBPAGE_BYTES + lo.vs + 16);
                const int tok0 = wb + 16 * (j0 + jstep * j);
                attend_subpage<NRG>(acc, sp, qf, tok0, we, lim, c, g,
                                    !(tok0 + 16 <= we && tok0 + 15 <= lim_min));
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // (every copy was waited for above)
}

// ---------------------------------------------------------------------------
// Decode / speculative-verify kernel (stream-K over workgroups).
//
// Work units are the 16-token sub-pages of every (sequence, kv-head) segment
// whose query rows fit one decode tile (n_q * G <= 16*NRG), ordered
// sequence-major, kv-head minor.  The grid holds the resident workgroups;
// workgroup w streams the contiguous unit range [U*w/nwg, U*(w+1)/nwg), so
// every workgroup gets the same number of bytes whatever the context
// lengths.  Its four waves interleave over each piece (wave k takes
// sub-pages k, k+4, ...) and merge their softmax states in LDS at the end of
// the piece.  A range covers whole segments (written out directly) plus at
// most one partial piece at each end, stored in the workgroup's two
// workspace slots and merged by attn_combine_kernel.
//
// Register budget: one row group runs GFA_DEC_WPE waves per SIMD; two row
// groups (speculative verify) need twice the accumulators and run 2.
// One new (token, kv-head) row of the fused cache write: input row `row` of
// new_k / new_v quantized to Q8_0 (two values per lane, a block per 16-lane
// DPP row, the closed form of the cache-write kernel) and stored at
// new_slot[row] (< 0: nothing).  The whole wave takes part.
template <int DT>
__device__ __forceinline__ void write_new_token(const AttnParams &p, int h, int64_t row, int lane) {
    const int d0 = 2 * lane;
    float ka, kb, va, vb;
    load2_as_f32<DT>(p.new_k, row * p.nk_ts + (int64_t)h * p.nk_hs + d0, ka, kb);
    load2_as_f32<DT>(p.new_v, row * p.nv_ts + (int64_t)h * p.nv_hs + d0, va, vb);
    const int64_t slot = p.new_slot[row];
    if (slot < 0) return;  // uniform
    const Q8Pair rk = q8_quantize_pair(ka, kb);
    const Q8Pair rv = q8_quantize_pair(va, vb);
    const int64_t page = slot / p.block_size;
    const int off = (int)(slot - page * p.block_size);
    const int64_t sub = (int64_t)(off >> 4) * SUBPAGE_BYTES;
    planar_store_pair(const_cast<uint8_t *>(p.kc) + page * p.cbs + (int64_t)h * p.chs + sub,
                      const_cast<uint8_t *>(p.vc) + page * p.vcbs + (int64_t)h * p.vchs + sub, off & 15, lane,
                      rk, rv);
}

constexpr int DEC_NW = 4;          // waves per decode workgroup
constexpr int DEC_CHUNK_ROWS = 64; // rows the two-row-group launch takes, in 32-row chunks
#ifndef GFA_DEC_MIN_UNITS
#define GFA_DEC_MIN_UNITS 16
#endif
constexpr int DEC_MIN_UNITS = GFA_DEC_MIN_UNITS;  // sub-pages per decode workgroup, at least

#ifndef GFA_DEC_DEPTH2
#define GFA_DEC_DEPTH2 2
#endif
#ifndef GFA_DEC_WPE2
#define GFA_DEC_WPE2 2
#endif
template <int NRG>
struct DecCfg {
    static constexpr int depth = NRG == 1 ? DEC_DEPTH : GFA_DEC_DEPTH2;
    static constexpr int wpe = NRG == 1 ? GFA_DEC_WPE : GFA_DEC_WPE2;
};

struct SegInfo {
    int q0, nq, sl, qa, kv_lim, nsub;
};

// Per-sequence decode segment: nsub sub-pages of keys (at least one, so a
// sequence with no visible key still gets its zero output written), or 0 when
// the sequence belongs to the prefill kernel.
__device__ __forceinline__ SegInfo seg_info(const AttnParams &p, int s) {
    SegInfo si;
    si.q0 = p.qsl[s];
    si.nq = p.qsl[s + 1] - si.q0;
    si.sl = p.seq_lens[s];
    si.qa = p.q_abs ? p.q_abs[s] : si.sl - si.nq;
    si.kv_lim = p.causal ? min(si.sl, max(si.qa + si.nq, 0)) : si.sl;
    const bool dec = si.nq > 0 && si.nq * p.G > p.dec_rows_lo && si.nq * p.G <= p.dec_rows_max;
    si.nsub = dec ? max((si.kv_lim + 15) >> 4, 1) : 0;
    return si;
}

__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(v, o);
        if (lane >= o) v += t;
    }
    return v;
}

__device__ __forceinline__ int64_t uniform64(int64_t v) {
    return ((int64_t)__builtin_amdgcn_readfirstlane((int)(v >> 32)) << 32) |
           (uint32_t)__builtin_amdgcn_readfirstlane((int)(v & 0xFFFFFFFF));
}

// Total decode units U and the number of participating workgroups: at least
// DEC_MIN_UNITS units per range, or one workgroup per segment where segments
// are shorter than that (each piece a workgroup streams costs a Q load and a
// cross-wave merge, so many short pieces in one range serialize), and at
// most the resident workgroups.  Every range is non-empty: each counted
// segment holds at least one unit.  Wave-level, uniform.
__device__ __forceinline__ void dec_total(const AttnParams &p, int lane, int64_t &U, int &nwg) {
    int64_t tot = 0;
    int nseg = 0;
    for (int base = 0; base < p.num_seqs; base += 64) {
        const int si = base + lane;
        const int n = si < p.num_seqs ? seg_info(p, si).nsub : 0;
        tot += __shfl(wave_incl_scan(n, lane), 63);
        nseg += __builtin_popcountll(__ballot(n > 0));
    }
    U = uniform64(tot * p.Hkv);
    const int64_t want = max(U / DEC_MIN_UNITS, (int64_t)nseg * p.Hkv);
    nwg = (int)max((int64_t)1, min((int64_t)p.nwg, want));
}

__device__ __forceinline__ int64_t range_start(int64_t U, int k, int n) { return U * k / n; }
// the workgroup whose range holds unit u
__device__ __forceinline__ int range_of(int64_t U, int64_t u, int n) { return (int)(((u + 1) * n - 1) / U); }

// CHUNK: sequences may have more rows than one tile (up to dec_rows_max):
// each piece is streamed once per R-row chunk.  A separate instantiation, so
// the launches that never need it keep their register allocation.
// Waves per decode workgroup.  The 32-row class in one row chunk (verify
// tiles) runs one 8-wave workgroup per CU (137 KB of LDS: eight ring slices)
// instead of two 4-wave ones: half the pieces, and one cross-wave merge per
// CU.  Measured on three boxes: 6/1, 8 x (131072 + 5) 1.4-4 % faster, 48/8
// within -0.8..+0.5 %.  The 16- and 48-row classes measured slower that way
// (the fused cache write of a decode step; 14 spilled VGPRs), and the
// two-chunk mode pairs its waves two by two.
constexpr int dec_nw(int nrg, bool chunk) { return nrg == 2 && !chunk ? 8 : DEC_NW; }

template <int NRG, int QDT, int ODT, bool CHUNK = false>
__global__ __launch_bounds__(64 * dec_nw(NRG, CHUNK))
__attribute__((amdgpu_waves_per_eu(DecCfg<NRG>::wpe, DecCfg<NRG>::wpe))) void attn_decode_kernel(AttnParams p) {
    constexpr int NW = dec_nw(NRG, CHUNK);  // waves in this workgroup
    static_assert((NW & (NW - 1)) == 0, "sub-pages are dealt to the waves by js & (NW - 1)");
    constexpr int R = 16 * NRG;  // rows per slot
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i16 = lane & 15, g = lane >> 4;
    const int B = p.num_seqs, Hkv = p.Hkv;
    const int w = blockIdx.x;

    // Batches of up to 64 sequences (uniform): lane i loads sequence i's
    // metadata once, and the plan, the segment search and the segment's own
    // fields all come from those registers - one memory round trip where the
    // general path below takes three before the first K/V load.
    const bool small = B <= 64;
    SegInfo lsi = seg_info(p, small ? min(lane, B - 1) : 0);
    const int ln = small && lane < B ? lsi.nsub : 0;
    const int lincl = wave_incl_scan(ln, lane);
    int64_t U;
    int nwg;
    if (small) {
        const int64_t tot = __shfl(lincl, 63);
        const int nseg = __builtin_popcountll(__ballot(ln > 0));
        U = uniform64(tot * Hkv);
        const int64_t want = max(U / DEC_MIN_UNITS, (int64_t)nseg * Hkv);
        nwg = (int)max((int64_t)1, min((int64_t)p.nwg, want));
    } else {
        dec_total(p, lane, U, nwg);
    }
    if (w == 0 && wv == 0) {
        // publish the plan for attn_combine_kernel: U, nwg, per-sequence
        // exclusive prefix of decode sub-pages
        if (small) {
            if (lane < B) p.ws_pre[lane] = lincl - ln;
        } else {
            int64_t run = 0;
            for (int base = 0; base < B; base += 64) {
                const int sj = base + lane;
                const int n = sj < B ? seg_info(p, sj).nsub : 0;
                const int incl = wave_incl_scan(n, lane);
                if (sj < B) p.ws_pre[sj] = (int)run + incl - n;
                run += __shfl(incl, 63);
            }
        }
        if (lane == 0) {
            p.ws_hdr[0] = U;
            p.ws_hdr[1] = nwg;
        }
    }
    if (w >= nwg || U == 0) return;  // uniform over the workgroup
    const int64_t u0 = range_start(U, w, nwg), u1 = range_start(U, w + 1, nwg);
    // locate the sequence holding u0 (Ps = sub-pages of the sequences before s)
    int s = 0;
    int64_t Ps = 0;
    SegInfo si;
    if (small) {
        const uint64_t bal = __ballot((int64_t)lincl * Hkv > u0);  // non-empty: u0 < U
        s = __builtin_ctzll(bal);
        Ps = __builtin_amdgcn_readlane(lincl - ln, s);
        si.q0 = __builtin_amdgcn_readlane(lsi.q0, s);
        si.nq = __builtin_amdgcn_readlane(lsi.nq, s);
        si.sl = __builtin_amdgcn_readlane(lsi.sl, s);
        si.qa = __builtin_amdgcn_readlane(lsi.qa, s);
        si.kv_lim = __builtin_amdgcn_readlane(lsi.kv_lim, s);
        si.nsub = __builtin_amdgcn_readlane(lsi.nsub, s);
    } else {
        for (int base = 0; base < B; base += 64) {
            const int sidx = base + lane;
            const int n = sidx < B ? seg_info(p, sidx).nsub : 0;
            const int incl = wave_incl_scan(n, lane);
            const int ctot = __shfl(incl, 63);
            if ((Ps + ctot) * Hkv > u0) {
                const uint64_t bal = __ballot((Ps + incl) * Hkv > u0);
                const int i = __builtin_ctzll(bal);
                s = base + i;
                Ps += __shfl(incl - n, i);
                break;
            }
            Ps += ctot;
        }
        s = __builtin_amdgcn_readfirstlane(s);
        Ps = uniform64(Ps);
        si = seg_info(p, s);
    }

    if (p.new_k) {
        // Fused cache write, before any streaming: the walk of the main loop
        // below over this workgroup's pieces.  The step's new tokens (positions
        // sl - n_q .. sl - 1, input rows q0 ..) that lie in a piece's
        // sub-pages are quantized and stored by the wave that will stream
        // their sub-page (wave (js - a) % NW takes sub-page js of piece
        // [a, b)), so each new (token, kv-head) is written by the wave that
        // reads it in this launch (by both, in the two-chunk mode), and that
        // wave's later loads follow its own stores in program order.
        int64_t uu = u0, Pw = Ps;
        int sw = s;
        SegInfo sv = si;
        while (uu < u1) {
            const int64_t off = uu - Pw * Hkv;
            const int hh = (int)(off / sv.nsub);
            const int a = (int)(off - (int64_t)hh * sv.nsub);
            const int b = (int)min((int64_t)sv.nsub, a + (u1 - uu));
            const int lo = sv.sl - sv.nq;
            // two row chunks at once (see rows_pass below): sub-page js is
            // streamed by the two waves with (js - a) % 2 == wv % 2, and both
            // write its new tokens (the same bytes), each before its own loads
            const bool dual = CHUNK && sv.nq * p.G > R;
            for (int js = max(a, lo >> 4); js < b; ++js) {  // uniform
                if (dual ? (((js - a) & 1) != (wv & 1)) : (((js - a) & (NW - 1)) != wv)) continue;
                const int t_hi = min(16 * js + 16, sv.sl);
                for (int pos = max(16 * js, lo); pos < t_hi; ++pos)
                    write_new_token<QDT>(p, hh, sv.q0 + (pos - lo), lane);
            }
            uu += b - a;
            if (uu < u1 && b == sv.nsub && hh == Hkv - 1) {
                Pw += sv.nsub;
                do {
                    ++sw;
                    sv = seg_info(p, sw);
                } while (sv.nsub == 0 && sw + 1 < B);
            }
        }
        // the stores above and this wave's loads of the same sub-pages below
        // (other lanes of the same wave): a wavefront's memory operations are
        // performed in order, so this fence costs no instruction; it keeps
        // the compiler from moving the loads above the stores
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    }

    // per wave: its merge rows (32 at most: 48-row tiles merge in two
    // passes), or (verify tiles) its LDS ring while it streams; rows past R
    // only lengthen the slice for the ring
    constexpr int RA = NRG >= 2 ? cmax(R < 32 ? R : 32, (DEC_RING * DEC_RING_SLOT + 4 * 132 - 1) / (4 * 132)) : R;
    __shared__ float sm_o[NW][RA][128 + 4];
    __shared__ float sm_m[NW][R], sm_l[NW][R];
    int64_t u = u0;
    bool first = true;
    while (u < u1) {
        const int64_t off = u - Ps * Hkv;
        const int h = (int)(off / si.nsub);
        const int a = (int)(off - (int64_t)h * si.nsub);
        const int b = (int)min((int64_t)si.nsub, a + (u1 - u));
        const int nrows = si.nq * p.G;

        // CHUNK: rows beyond one tile (up to 64: a verify step of 6 tokens at
        // 6 q-heads per kv-head is 36 rows) are taken in two R-row chunks at
        // once: waves 0, 1 hold rows 0..R-1 and waves 2, 3 rows R..2R-1, each
        // pair interleaving the piece's sub-pages the same way, so a sub-page
        // is fetched by two waves of the CU close together and the second
        // fetch is served by the caches, not HBM.  Otherwise the four waves
        // interleave over the piece for one row tile.
        // rc: this wave's first row; j0 / jstep: its sub-pages of the piece;
        // wpc: waves per chunk (their states are merged).
        auto rows_pass = [&](int rc, int j0, int jstep, int wpc) {
        half8_t qf[NRG][4];
        int lim[NRG];
        load_rows<NRG, QDT>(p, h, si.q0, nrows, rc, si.sl, si.qa, i16, g, qf, lim);
        WaveAcc<NRG> acc;
        acc_init(acc);
        if constexpr (NRG >= 2) {  // verify tiles: sub-pages staged through this wave's sm_o slice
            static_assert(sizeof(sm_o[0]) >= DEC_RING * DEC_RING_SLOT, "ring fits the wave's slice");
            stream_range_lds<NRG, DEC_RING>(acc, p, s, h, 16 * a, min(16 * b, si.kv_lim), qf, lim, lane, i16,
                                            g, j0, jstep, reinterpret_cast<uint8_t *>(&sm_o[wv][0][0]));
        } else {
            stream_range<NRG, GFA_DEC_NT != 0, DecCfg<NRG>::depth>(acc, p, s, h, 16 * a,
                                                                     min(16 * b, si.kv_lim), qf, lim,
                                                                     lane, i16, g, j0, jstep);
        }
        // ---- merge the chunk's waves' states in LDS ------------------------
        // in passes of 32 rows (row groups 2*ps, 2*ps + 1): a wave's LDS
        // slice holds 32 rows, so 48-row tiles take two passes
        constexpr int NPASS = (R + 31) / 32;
        static_assert(!CHUNK || NPASS == 1, "two-chunk tiles merge in one pass");
        const bool whole = a == 0 && b == si.nsub;
        const int slot = 2 * w + (first ? 0 : 1);
        const int rows_c = CHUNK ? nrows : min(nrows, R);
#pragma unroll
        for (int ps = 0; ps < NPASS; ++ps) {
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg) {
            if ((rg >> 1) != ps) continue;
            const float l = xrow_sum(acc.l[rg]);
            const int r = 16 * rg + i16;
            if (g == 0) {
                sm_m[wv][r] = acc.m[rg];
                sm_l[wv][r] = l;
            }
#pragma unroll
            for (int mm = 0; mm < 8; ++mm)
                *reinterpret_cast<float4_t *>(&sm_o[wv][r - 32 * ps][16 * mm + 4 * g]) = acc.o[rg][mm];
        }
        __syncthreads();
        const int r_hi = NPASS == 1 ? rows_c : min(rows_c, 32 * ps + 32);
        for (int it = threadIdx.x + 32 * 32 * ps; it < r_hi * 32; it += 64 * NW) {
            const int r = it >> 5, d0 = (it & 31) * 4;
            const int ch = CHUNK ? r / R : 0;   // the row's chunk: waves ch*wpc .. ch*wpc + wpc - 1
            const int rl = r - ch * R;          // its row inside the chunk
            const int ro = rl - 32 * ps;        // its row in the LDS slices
            const int k0 = ch * wpc;
            float mx = -INFINITY;
            for (int k = k0; k < k0 + wpc; ++k) mx = fmaxf(mx, sm_m[k][rl]);
            const float ms = mx == -INFINITY ? 0.0f : mx;
            float l = 0.f;
            float4_t o = {0.f, 0.f, 0.f, 0.f};
            for (int k = k0; k < k0 + wpc; ++k) {
                const float wk = __builtin_amdgcn_exp2f(sm_m[k][rl] - ms);
                l = fmaf(sm_l[k][rl], wk, l);
                o += *reinterpret_cast<const float4_t *>(&sm_o[k][ro][d0]) * wk;
            }
            if (whole) {
                const int j = r / p.G;
                const int hq = h * p.G + (r - j * p.G);
                const int64_t ob = (int64_t)(si.q0 + j) * p.o_ts + (int64_t)hq * p.o_hs + d0;
                const float inv = l > 0.f ? 1.0f / l : 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) store_out<ODT>(p.out, ob + i, o[i] * inv);
            } else {
                const int64_t row = (int64_t)slot * (CHUNK ? p.dec_rows_max : R) + r;
                *reinterpret_cast<float4_t *>(p.ws_o + row * 128 + d0) = o;
                if (d0 == 0) {
                    p.ws_ml[2 * row] = mx;
                    p.ws_ml[2 * row + 1] = l;
                }
            }
        }
        __syncthreads();  // LDS reused by the next pass or piece
        }
        };
        static_assert((NW == 4 || !CHUNK) && DEC_CHUNK_ROWS <= 2 * 32, "two row chunks of two waves each");
        if (CHUNK && nrows > R) {  // uniform: rows R..nrows-1 (nrows <= 2R) in the second chunk
            rows_pass(R * (wv >> 1), wv & 1, 2, NW / 2);
        } else {
            rows_pass(0, wv, NW, NW);
        }
        u += b - a;
        first = false;
        if (u < u1 && b == si.nsub && h == Hkv - 1) {  // next sequence with decode work
            Ps += si.nsub;
            do {
                ++s;
                si = seg_info(p, s);
            } while (si.nsub == 0 && s + 1 < B);
        }
    }
}

// Merge pass over split segments, from the plan the decode kernel published
// (U, nwg, per-sequence prefix).  grid (num_seqs, Hkv, 16*NRG rows), block
// 256: workgroup (s, h, r) merges row r of segment (s, h) when the segment
// was split.  Thread t owns d-chunk t%32 (4 d) and pieces k = wf + t/32,
// wf + t/32 + 8, ... (one-pass online merge, independent loads); the 8
// partial states per d-chunk are then merged through LDS.  Piece k
// (workgroup k) sits in slot 2k+1 when the segment starts inside k's range
// (it is k's last piece), else in slot 2k.  (A last-arriver merge inside the
// decode kernel needs agent-scope release / acquire fences around a
// per-segment counter; on this part those write back and invalidate the
// XCD's L2 and made the decode pass 3.5x slower, so the merge stays a
// second, tiny launch.)
template <int NRG, int ODT>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnParams p) {
    constexpr int R = 16 * NRG;
    const int s = blockIdx.x, h = blockIdx.y, r = blockIdx.z;
    // the plan words are read together with the sequence's metadata (one
    // memory round trip instead of two: they are needed only when the
    // segment turns out to be split)
    const int64_t U = p.ws_hdr[0];
    const int nwg = (int)p.ws_hdr[1];
    const int pre = p.ws_pre[s];
    const SegInfo si = seg_info(p, s);
    if (si.nsub == 0 || r >= si.nq * p.G) return;
    if (U == 0) return;
    const int64_t S0 = (int64_t)pre * p.Hkv + (int64_t)h * si.nsub;
    const int wf = range_of(U, S0, nwg), wl = range_of(U, S0 + si.nsub - 1, nwg);
    if (wf == wl && range_start(U, wf, nwg) <= S0 && range_start(U, wf + 1, nwg) >= S0 + si.nsub)
        return;  // whole segment in one workgroup: already written
    const int t = threadIdx.x, dc = t & 31, sub = t >> 5;
    const int d0 = 4 * dc;
    float m = -INFINITY, l = 0.f;
    float4_t o = {0.f, 0.f, 0.f, 0.f};
    // group `sub` merges pieces wf + sub, wf + sub + 8, ... in order; the loads
    // of CU of them are issued before they are merged (in flight together)
#ifndef GFA_COMB_CU
#define GFA_COMB_CU 8
#endif
    constexpr int CU = GFA_COMB_CU;
    for (int k0 = wf + sub; k0 <= wl; k0 += 8 * CU) {
        float2_t mlk[CU];
        float4_t ok[CU];
#pragma unroll
        for (int i = 0; i < CU; ++i) {
            const int k = k0 + 8 * i;
            if (k <= wl) {
                const int sk = (k == wf && range_start(U, k, nwg) < S0) ? 2 * k + 1 : 2 * k;
                const int64_t row = (int64_t)sk * p.dec_rows_max + r;
                mlk[i] = *reinterpret_cast<const float2_t *>(p.ws_ml + 2 * row);
                ok[i] = *reinterpret_cast<const float4_t *>(p.ws_o + row * 128 + d0);
            }
        }
#pragma unroll
        for (int i = 0; i < CU; ++i) {
            if (k0 + 8 * i > wl) break;
            const float mk = mlk[i][0], lk = mlk[i][1];
            const float mn = fmaxf(m, mk);
            const float ms = mn == -INFINITY ? 0.0f : mn;
            const float a = __builtin_amdgcn_exp2f(m - ms), c = __builtin_amdgcn_exp2f(mk - ms);
            l = l * a + lk * c;
            o = o * a + ok[i] * c;
            m = mn;
        }
    }
    __shared__ float sm[8][32][6];
    sm[sub][dc][0] = m;
    sm[sub][dc][1] = l;
#pragma unroll
    for (int i = 0; i < 4; ++i) sm[sub][dc][2 + i] = o[i];
    __syncthreads();
    if (sub != 0) return;
#pragma unroll
    for (int q = 1; q < 8; ++q) {
        const float mk = sm[q][dc][0], lk = sm[q][dc][1];
        const float mn = fmaxf(m, mk);
        const float ms = mn == -INFINITY ? 0.0f : mn;
        const float a = __builtin_amdgcn_exp2f(m - ms), c = __builtin_amdgcn_exp2f(mk - ms);
        l = l * a + lk * c;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = o[i] * a + sm[q][dc][2 + i] * c;
        m = mn;
    }
    const int j = r / p.G;
    const int hq = h * p.G + (r - j * p.G);
    const int64_t ob = (int64_t)(si.q0 + j) * p.o_ts + (int64_t)hq * p.o_hs + d0;
    const float inv = l > 0.f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) store_out<ODT>(p.out, ob + i, o[i] * inv);
}

// The same merge for segments of few pieces (a batch whose resident
// workgroups are few per segment), and for the second decode class of a
// mixed batch with many segments (mostly empty there; a per-row grid would
// be mostly workgroups that find nothing): one workgroup per (sequence,
// kv-head), thread t takes d-chunk t % 32 of rows t / 32, t / 32 + 8, ...
// and merges the segment's pieces in order, the loads of up to 8 of them in
// flight.
template <int ODT>
__global__ __launch_bounds__(256) void attn_combine_few_kernel(AttnParams p) {
    const int s = blockIdx.x, h = blockIdx.y;
    const int64_t U = p.ws_hdr[0];
    const int nwg = (int)p.ws_hdr[1];
    const int pre = p.ws_pre[s];
    const SegInfo si = seg_info(p, s);
    if (si.nsub == 0 || U == 0) return;
    const int64_t S0 = (int64_t)pre * p.Hkv + (int64_t)h * si.nsub;
    const int wf = range_of(U, S0, nwg), wl = range_of(U, S0 + si.nsub - 1, nwg);
    if (wf == wl && range_start(U, wf, nwg) <= S0 && range_start(U, wf + 1, nwg) >= S0 + si.nsub)
        return;  // whole segment in one workgroup: already written
    const int rows = si.nq * p.G;
    const int dc = threadIdx.x & 31, d0 = 4 * dc;
    constexpr int CU = 8;
    for (int r = threadIdx.x >> 5; r < rows; r += 8) {
        float m = -INFINITY, l = 0.f;
        float4_t o = {0.f, 0.f, 0.f, 0.f};
        for (int k0 = wf; k0 <= wl; k0 += CU) {
            float2_t mlk[CU];
            float4_t ok[CU];
#pragma unroll
            for (int i = 0; i < CU; ++i) {
                const int k = k0 + i;
                if (k <= wl) {
                    const int sk = (k == wf && range_start(U, k, nwg) < S0) ? 2 * k + 1 : 2 * k;
                    const int64_t row = (int64_t)sk * p.dec_rows_max + r;
                    mlk[i] = *reinterpret_cast<const float2_t *>(p.ws_ml + 2 * row);
                    ok[i] = *reinterpret_cast<const float4_t *>(p.ws_o + row * 128 + d0);
                }
            }
#pragma unroll
            for (int i = 0; i < CU; ++i) {
                if (k0 + i > wl) break;
                const float mk = mlk[i][0], lk = mlk[i][1];
                const float mn = fmaxf(m, mk);
                const float ms = mn == -INFINITY ? 0.0f : mn;
                const float a = __builtin_amdgcn_exp2f(m - ms), c = __builtin_amdgcn_exp2f(mk - ms);
                l = l * a + lk * c;
                o = o * a + ok[i] * c;
                m = mn;
            }
        }
        const int j = r / p.G;
        const int hq = h * p.G + (r - j * p.G);
        const int64_t ob = (int64_t)(si.q0 + j) * p.o_ts + (int64_t)hq * p.o_hs + d0;
        const float inv = l > 0.f ? 1.0f / l : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) store_out<ODT>(p.out, ob + i, o[i] * inv);
    }
}

// ---------------------------------------------------------------------------
// Prefill kernel: sequences with more than dec_rows_max packed rows.
//
// Workgroup = 12 waves over 256 consecutive packed rows of one (sequence,
// kv-head).  K/V stream through LDS in 64-key tiles (four 16-token
// sub-pages), dequantized ONCE per workgroup to fp16 (K^ = q * d_k,
// V^ = q * d_v, each rounded to fp16).  The waves have two roles:
//   consumers (waves 0-7, two per SIMD): 32 query rows each; per tile
//     S'^T[64 keys x 32 rows] = K^ . Q^T - m   16 x v_mfma_f32_32x32x16_f16
//     O^T[128 d x 32 rows]   += V^T . P^T      16 x v_mfma_f32_32x32x16_f16
//     with Q (pre-scaled by scale*log2 e) held in registers for the whole
//     kernel and the running row max m fed in as the accumulator input;
//   producers (waves 8-11, one per SIMD): wave 8 + i fetches sub-page i of
//     every tile from HBM, PF_PDEPTH tiles ahead, and dequantizes it into
//     the LDS stage the consumers read next - or, when the plan wrote the
//     launch's tile images (each tile dequantized once into the workspace by
//     prefill_tiles_kernel), copies a quarter of each image straight into
//     LDS (global_load_lds).
// A consumer's only LDS traffic is its MFMA operand reads, so the waits in
// front of its MFMAs never queue behind dequant stores (LDS instructions of
// one wave complete in order), and the dequant VALU work issues from a wave
// of its own beside the two consumers' MFMAs.  Tile t sits in LDS stage
// t % 3.  The two consumer waves of a SIMD run half a tile apart (two
// barriers per tile, the half-steps below); the producers write K^ of tile
// t in half-step 2t - 2 and V^T in 2t - 1.
// 32x32x16 operand layout (lane l, h = l/32): A[i = l%32][k = 8h+e],
// B[k = 8h+e][j = l%32], D[i = 8(r/4)+4h+r%4][j = l%32] for register r.  A
// lane's S^T registers 8s..8s+7 are then exactly the keys its P^T operand
// needs for PV step s when the contraction order inside each 16 keys swaps
// key bits 2 and 3; V^T is stored in LDS in that order.
//
// LDS tile (per stage):
//   K^   [64 keys][272 B]  (128 fp16 + 16 B pad)
//   V^T  [128 d][144 B]    (64 fp16 in contraction order + 16 B pad)
// The pads make every ds_read_b128 of the MFMA operands and every dequant
// store bank-conflict free with plain (immediate-offset) addressing.
// Keys at or past the workgroup's kv_end are masked to -inf in S; the V
// scales are made finite during dequantization so their P = 0 products stay
// 0 whatever those cache bytes hold.
//
// grid (row_tiles * Hkv, num_seqs): blockIdx.x % Hkv is the kv-head (one head
// per XCD when Hkv = 8: the XCD's L2 serves that head's K/V to all its
// workgroups) and row tiles run last-first, heaviest causal ranges first.
//
// Key-interleaved 128-row tile (KS = 2).  With few rows per kv-head most of a
// 256-row tile's consumer waves idle and a key tile costs a whole
// QK -> softmax -> PV chain of one wave per SIMD, as long as a full tile.
// The KS = 2 form gives consumer waves w and w + 4 the same 32 rows: group A
// (waves 0-3) takes the even key tiles, group B (waves 4-7) the odd ones, so
// one tile is consumed per half-step (A's QK beside B's softmax + PV on each
// SIMD, and the reverse in the next half-step) and the producers dequantize a
// whole tile (K^ of tile h + 1, V^T of tile h) per half-step h into two LDS
// stages (tile t: stage t % 2, so group A always reads stage 0 and group B
// stage 1).  The two partial states of each row merge through LDS at the
// end: each wave of a pair sends the partner the half of O^T it will not
// store.
constexpr int PF_CWAVES = 8;                  // consumer waves (32 rows each)
constexpr int PF_PWAVES = 4;                  // producer waves (one sub-page of each tile)
constexpr int PF_WAVES = PF_CWAVES + PF_PWAVES;
constexpr int PF_ROWS = 32 * PF_CWAVES;       // rows per tile (KS = 1); KS = 2 tiles hold PF_ROWS / 2
constexpr int PF_TK = 64;                     // keys per LDS tile
constexpr int PF_NSP = PF_TK / 16;            // sub-pages per tile
static_assert(PF_NSP == PF_PWAVES, "one producer wave per sub-page");
constexpr int PF_NST = PF_TK / 32;            // 32-key S subtiles per tile
#ifndef GFA_PF_PDEPTH
#define GFA_PF_PDEPTH 4
#endif
constexpr int PF_PDEPTH = GFA_PF_PDEPTH;      // producer register ring: tiles fetched ahead + 1
static_assert(PF_PDEPTH == 2 || PF_PDEPTH == 4, "ring depth: even, unrolled");
constexpr int PF_KPITCH = 272;
constexpr int PF_VPITCH = 2 * PF_TK + 16;
constexpr int PF_KBYTES = PF_TK * PF_KPITCH;
constexpr int PF_VBYTES = 128 * PF_VPITCH;
constexpr int PF_IMG_BYTES = PF_KBYTES + PF_VBYTES;  // one tile image: K^ stage, then V^T stage
constexpr int PF_NSTAGE = 3;                           // LDS stages of K^ and of V^T (tile t: stage t % 3)
#ifndef GFA_PF_IMG_REUSE
#define GFA_PF_IMG_REUSE 32
#endif
constexpr int PF_IMG_REUSE = GFA_PF_IMG_REUSE;         // reads per tile image, on average, at least
// a tile image is copied into LDS as four equal shares, one per producer
// wave, each 4 x 1 KB plus a partial 1 KB row (64 lanes x 16 bytes per copy)
constexpr int PF_KSHARE = PF_KBYTES / PF_PWAVES, PF_VSHARE = PF_VBYTES / PF_PWAVES;
static_assert(PF_KSHARE % 16 == 0 && PF_VSHARE % 16 == 0 && PF_KSHARE / 1024 == 4 && PF_VSHARE / 1024 == 4 &&
                  PF_KSHARE % 1024 != 0 && PF_VSHARE % 1024 != 0,
              "five copies per wave and stage");

typedef float float16v_t __attribute__((ext_vector_type(16)));
typedef uint64_t u64x8_t __attribute__((ext_vector_type(8)));
struct PHalf8 {
    half2_t h[4];
};

__device__ __forceinline__ float16v_t mfma32(half8_t a, half8_t b, float16v_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Max over the 32 values of two S accumulators as a tree of depth 4 (a
// running fmaxf chain is 16 dependent steps deep).
__device__ __forceinline__ float tile_max32(const float16v_t &x, const float16v_t &y) {
    float b[11];
#pragma unroll
    for (int i = 0; i < 5; ++i) b[i] = max3f(x[3 * i], x[3 * i + 1], x[3 * i + 2]);
    b[5] = max3f(x[15], y[0], y[1]);
#pragma unroll
    for (int i = 0; i < 4; ++i) b[6 + i] = max3f(y[2 + 3 * i], y[3 + 3 * i], y[4 + 3 * i]);
    b[10] = y[14];
    const float c0 = max3f(b[0], b[1], b[2]), c1 = max3f(b[3], b[4], b[5]);
    const float c2 = max3f(b[6], b[7], b[8]), c3 = max3f(b[9], b[10], y[15]);
    return max3f(max3f(c0, c1, c2), c3, c3);
}

// Raw bytes of one half (hf = 0, 1) of a sub-page as a lane holds them:
// the Q8_0 blocks 2hf and 2hf+1 of K and of V.
//   K: token t = l%16, group g = l/16: k = ints of d = 8g + 32b + (0..7),
//      b = 2hf, 2hf+1 (chunk hf*64 + 4t+g); ks = the two scales (t, b).
//   V: token quad T = l/16, i = l%16: v = ints of tokens 4T..4T+3 at
//      d = i + 16m, m = 4hf..4hf+3 (chunk hf*64 + l); vs = their scales.
struct PfRaw {
    u32x4 k, v, vs;
    uint32_t ks;
};

// VF16: V is a planar fp16 sub-page (4096 B; element (t, d) at
// 2048*(d/64) + 32*(16*(t/4) + d%16) + 8*((d/16)%4) + 2*(t%4)), so the lane's
// 16 fp16 values (4 d x 4 tokens) are the 32 bytes at 2048*hf + 32*lane:
// v = the first 16, vs = the second 16.
template <bool VF16>
__device__ __forceinline__ void pf_fetch(PfRaw &r, const uint8_t *kb, const uint8_t *vb, int lane, int hf) {
    const int t = lane & 15, g = lane >> 4;
    r.k = *reinterpret_cast<const u32x4 *>(kb + hf * 1024 + (4 * t + g) * 16);
    r.ks = *reinterpret_cast<const uint32_t *>(kb + SCALE_OFF + 8 * t + 4 * hf);
    if constexpr (VF16) {
        const u32x4 *v = reinterpret_cast<const u32x4 *>(vb + hf * 2048 + lane * 32);
        r.v = v[0];
        r.vs = v[1];
    } else {
        r.v = *reinterpret_cast<const u32x4 *>(vb + hf * 1024 + lane * 16);
        r.vs = *reinterpret_cast<const u32x4 *>(vb + SCALE_OFF + 32 * g + 16 * hf);
    }
}

// v * s for exact fp16 v and an fp32 s: each product formed in fp32 and
// rounded to fp16 once (v_fma_mix).
__device__ __forceinline__ half8_t scale8_f32(half8_t v, float s) {
    half8_t r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (half_t)fmaf((float)v[e], s, 0.0f);
    return r;
}

// fp16 pair with Inf / NaN replaced by +-65504 (v_pk_max/min_f16 return the
// non-NaN operand).
__device__ __forceinline__ half2_t finite2(half2_t x) {
    const half2_t hi = {(half_t)65504.0f, (half_t)65504.0f};
    return __builtin_elementwise_min(__builtin_elementwise_max(x, -hi), hi);
}

// Dequantizes the lane's raw half sub-page into the LDS stages (sub-page sp
// of the tile): K^ rows into kst, V^T columns into vst.  TAIL (the last tile
// of the range, the only one that can hold keys past kv_end): bytes of tokens
// past the valid range are dequantized as they are - their scores are masked
// to -inf (P = 0) - and the V scales are made finite so that 0 * V^ stays 0.
// K^ carries the part kmul = c * 2^e of the softmax scale c = scale * log2 e
// (Q carries the exact power of two 2^-e): K^ = fp16(q * (d * kmul)), the
// product formed in fp32 and rounded once.  Pre-scaling Q by c in fp16 would
// add a second rounding to every score; this keeps fp16 / bf16 Q exact.
__device__ __forceinline__ void pf_dequant_k(const PfRaw &r, uint8_t *kst, int sp, int lane, int hf,
                                             float kmul) {
    const int t = lane & 15, g = lane >> 4;
    // (vector elements are copied to scalars before __builtin_bit_cast: a
    // bit_cast of an ext_vector element lvalue reads element 0 with this clang)
    const half2_t ks = __builtin_bit_cast(half2_t, r.ks);
    const float s0 = (float)ks[0] * kmul, s1 = (float)ks[1] * kmul;
    const uint32_t k0 = r.k[0], k1 = r.k[1], k2 = r.k[2], k3 = r.k[3];
    // K^: row 16sp + t, d chunks 4b + g (8 fp16 each)
    uint8_t *krow = kst + (16 * sp + t) * PF_KPITCH + 16 * g + 128 * hf;
    *reinterpret_cast<half8_t *>(krow) = scale8_f32(i8x8_to_half8(k0, k1), s0);
    *reinterpret_cast<half8_t *>(krow + 64) = scale8_f32(i8x8_to_half8(k2, k3), s1);
}

template <bool TAIL, bool VF16>
__device__ __forceinline__ void pf_dequant_v(const PfRaw &r, uint8_t *vst, int sp, int lane, int hf) {
    const int i = lane & 15, T = lane >> 4;
    const uint32_t vq[4] = {r.v[0], r.v[1], r.v[2], r.v[3]};
    const uint32_t vsw[4] = {r.vs[0], r.vs[1], r.vs[2], r.vs[3]};
    // V^T: rows d = i + 16m; the 4 tokens 4T..4T+3 of sub-page sp sit at
    // contraction position 16sp + 8(T&1) + 4(T>>1) (key bits 2 and 3 swapped)
    uint8_t *vcol = vst + (i + 64 * hf) * PF_VPITCH + 2 * (16 * sp + 8 * (T & 1) + 4 * (T >> 1));
    if constexpr (VF16) {  // already fp16: 4 tokens of d = i + 16(4hf + mm) per 8 bytes
#pragma unroll
        for (int mm = 0; mm < 4; ++mm) {
            const uint32_t lo = mm < 2 ? vq[2 * mm] : vsw[2 * mm - 4];
            const uint32_t hi = mm < 2 ? vq[2 * mm + 1] : vsw[2 * mm - 3];
            *reinterpret_cast<u32x2 *>(vcol + 16 * mm * PF_VPITCH) = u32x2{lo, hi};
        }
        return;
    }
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
        const int b = mm >> 1;  // block 2hf + b: scale dwords 2b (tokens 0,1), 2b+1 (2,3)
        half2_t s01 = __builtin_bit_cast(half2_t, vsw[2 * b]);
        half2_t s23 = __builtin_bit_cast(half2_t, vsw[2 * b + 1]);
        if (TAIL) {
            s01 = finite2(s01);
            s23 = finite2(s23);
        }
        half2_t lo, hi;
        i8x4_to_f16x4(vq[mm], lo, hi);
        lo *= s01;
        hi *= s23;
        *reinterpret_cast<half4_t *>(vcol + 16 * mm * PF_VPITCH) = half4_t{lo[0], lo[1], hi[0], hi[1]};
    }
}

template <int QDT, int ODT, bool VF16, bool MASK, int KS = 1>
__global__ __launch_bounds__(64 * PF_WAVES)
__attribute__((amdgpu_waves_per_eu(3, 3))) void attn_prefill_kernel(AttnParams p) {
    static_assert(KS == 1 || KS == 2, "256-row tiles, or 128-row key-interleaved tiles");
    constexpr int ROWS = PF_ROWS / KS;               // query rows per tile
    constexpr int NSTAGE = KS == 1 ? PF_NSTAGE : 2;  // LDS stages of K^ and of V^T (tile t: t % NSTAGE)
    __shared__ __attribute__((aligned(16))) uint8_t lds[NSTAGE * (PF_KBYTES + PF_VBYTES)];
    uint8_t *const ldsk = lds;
    uint8_t *const ldsv = lds + NSTAGE * PF_KBYTES;
    const int Hkv = p.Hkv;
    const int h = blockIdx.x % Hkv;
    int s, rt, kt0 = 0, kt1 = INT32_MAX, slot = -1;
    if (p.pf_seq) {  // the sorted work list (uniform)
        const int item = blockIdx.x / Hkv;
        if (item >= p.pf_count[0]) return;
        s = p.pf_seq[item];
        rt = p.pf_rt[item];
        kt0 = p.pf_kt0[item];
        kt1 = p.pf_kt1[item];
        slot = p.pf_slot[item];
    } else {         // row tiles last-first within each sequence
        s = blockIdx.y;
        rt = (gridDim.x / Hkv) - 1 - (int)(blockIdx.x / Hkv);
    }
    const int q0 = p.qsl[s];
    const int nq = p.qsl[s + 1] - q0;
    const int nrows = nq * p.G;
    if (nq <= 0 || nrows <= p.dec_rows_max) return;  // uniform over the workgroup
    const int row0 = ROWS * rt;
    if (row0 >= nrows) return;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int sl = p.seq_lens[s];
    const int qa = p.q_abs ? p.q_abs[s] : sl - nq;
    const int jlast = (min(row0 + ROWS, nrows) - 1) / p.G;
    const int kv_end = p.causal ? min(sl, max(qa + jlast + 1, 0)) : sl;
    // key tiles [ktb, ktb + ntk) of the row tile's (kv_end + PF_TK - 1) / PF_TK;
    // the loops below count tiles from 0 and add ktb where they need a key index
    const int ntk_all = (kv_end + PF_TK - 1) / PF_TK;
    const int ktb = min(kt0, ntk_all);
    const int ntk = min(kt1, ntk_all) - ktb;
    using Even = std::integral_constant<bool, false>;
    using Odd = std::integral_constant<bool, true>;

    if (w >= PF_CWAVES) {
        // ---- producer: sub-page wsp of every tile, both halves ----------
        // Page ids come from two lane-distributed windows of 64 tiles (lane i
        // of pw0 / pw1: the page of this wave's sub-page in tile cbase + i /
        // cbase + 64 + i).  Tile t sits in ring slot t % PF_PDEPTH from its
        // fetch until its dequant, one iteration before the consumers read it.
        const int wsp = w - PF_CWAVES;
        // (no images for KS = 2 tiles: the host never passes them there)
        if (KS == 1 && p.pf_tiles != nullptr && p.pf_count[2] != 0) {  // uniform
            // The tiles are dequantized images in the workspace.  Copy batch
            // b (K^ of tile b/2 for even b, V^T for odd b) goes from the image
            // straight into its LDS stage in half-step b - 4 and has landed by
            // the end of half-step b - 1, before the barrier that opens the
            // consumers' first read of it.  The stage it fills was last read
            // in half-step b - 5 (tile b/2 - 3).  Each wave copies one quarter
            // of a stage per batch: exactly five copies, so "batch h + 1 has
            // landed" at the end of half-step h is vmcnt(15) (the three later
            // batches may still be in flight), or vmcnt(0) near the end, where
            // fewer batches follow.
            const int64_t istride = (int64_t)Hkv * PF_IMG_BYTES;
            const uint8_t *img0 = p.pf_tiles + ((int64_t)(p.pf_tbase[s] + ktb) * Hkv + h) * PF_IMG_BYTES;
            auto copy = [&](int b) __attribute__((always_inline)) {
                const int t = b >> 1;
                if (t >= ntk) return;  // uniform
                const bool isv = b & 1;
                const int share = isv ? PF_VSHARE : PF_KSHARE;
                const uint8_t *src = img0 + t * istride + (isv ? PF_KBYTES : 0) + wsp * share;
                uint8_t *dst = (isv ? ldsv + (t % PF_NSTAGE) * PF_VBYTES : ldsk + (t % PF_NSTAGE) * PF_KBYTES) +
                               wsp * share;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    __builtin_amdgcn_global_load_lds(src + i * 1024 + lane * 16,
                                                     (__attribute__((address_space(3))) void *)(dst + i * 1024), 16, 0, 0);
                if (16 * lane < share - 4096)  // the partial row
                    __builtin_amdgcn_global_load_lds(src + 4096 + lane * 16,
                                                     (__attribute__((address_space(3))) void *)(dst + 4096), 16, 0, 0);
            };
            // the end of half-step h (h = -1: before the first barrier)
            auto landed = [&](int h) __attribute__((always_inline)) {
                if (h + 4 < 2 * ntk) __builtin_amdgcn_s_waitcnt(0x0F7F);  // vmcnt(15)
                else __builtin_amdgcn_s_waitcnt(0x0F70);                  // vmcnt(0)
            };
#pragma unroll
            for (int b = 0; b < 4; ++b) copy(b);
            landed(-1);
            __syncthreads();
            for (int hs = 0; hs <= 2 * ntk; ++hs) {  // half-steps 0 .. 2 ntk
                copy(hs + 4);
                landed(hs);
                __syncthreads();
            }
            return;
        }
        const int32_t *btrow = p.bt + (int64_t)s * p.bt_stride;
        const int bs = p.block_size;
        const int last_sp = max((kv_end - 1) >> 4, 0);  // last sub-page with a valid key
        const int spb = PF_NSP * ktb + wsp;
        auto sp_of = [&](int kt) { return min(PF_NSP * kt + spb, last_sp); };
        auto load_pg = [&](int c) -> int {
            const int kt = 64 * c + lane;
            return kt < ntk ? btrow[(16 * sp_of(kt)) / bs] : 0;
        };
        // Waits for a window load right where it is issued (once per 64
        // tiles): a window register still pending in the loop would make
        // every v_readlane of it wait for all loads in flight (vmcnt counts in
        // order), the K/V fetches included.
        auto ready = [](int &v) { asm volatile("" : "+v"(v)); };
        const uint8_t *kplane = p.kc + (int64_t)h * p.chs;
        const uint8_t *vplane = p.vc + (int64_t)h * p.vchs;
        constexpr int VSUB = VF16 ? 4096 : SUBPAGE_BYTES;  // V bytes per 16-token sub-page
        int pw0 = 0, pw1 = 0, cbase = 0;
        struct PfRawT {
            PfRaw h[2];
        };
        PfRawT ring[PF_PDEPTH];
        // Fetch of tile t (uniform, t < cbase + 128).  Tiles past the range
        // read page 0 at the last valid sub-page's offset (their bytes are
        // never dequantized into a stage that is read).  The steady-state
        // loop fetches unconditionally: with the same number of loads on
        // every path the compiler's vmcnt waits cover only the tile being
        // dequantized, not the PF_PDEPTH - 1 tiles still in flight.
        auto fetch = [&](PfRawT &rw, int t) __attribute__((always_inline)) {
            const int rel = t - cbase;  // 0..127, uniform
            const int pa = __builtin_amdgcn_readlane(pw0, rel & 63);
            const int pb = __builtin_amdgcn_readlane(pw1, rel & 63);
            const int64_t page = rel < 64 ? pa : pb;
            const int64_t spi = ((16 * sp_of(t)) % bs) >> 4;
            const uint8_t *kb = kplane + page * p.cbs + spi * SUBPAGE_BYTES;
            const uint8_t *vb = vplane + page * p.vcbs + spi * VSUB;
            pf_fetch<VF16>(rw.h[0], kb, vb, lane, 0);
            pf_fetch<VF16>(rw.h[1], kb, vb, lane, 1);
        };
        // keeps the fetches of tiles up to kt + 2 * PF_PDEPTH inside the
        // windows: called at kt = 0 mod PF_PDEPTH (uniform), before the
        // group of PF_PDEPTH half-step pairs that fetch those tiles
        auto slide = [&](int kt) __attribute__((always_inline)) {
            if (kt - cbase >= 64) {
                cbase += 64;
                pw0 = pw1;
                pw1 = cbase + 64 < ntk ? load_pg(cbase / 64 + 1) : 0;
                ready(pw1);
            }
        };
        // dequantizes the K (or V) half of tile t (in the ring) into stage t % NSTAGE
        auto dequant_k = [&](const PfRawT &rw, int t) __attribute__((always_inline)) {
            uint8_t *kst = ldsk + (t % NSTAGE) * PF_KBYTES;
            pf_dequant_k(rw.h[0], kst, wsp, lane, 0, p.pf_kmul);
            pf_dequant_k(rw.h[1], kst, wsp, lane, 1, p.pf_kmul);
        };
        auto dequant_v = [&](const PfRawT &rw, int t, auto tail) __attribute__((always_inline)) {
            uint8_t *vst = ldsv + (t % NSTAGE) * PF_VBYTES;
            constexpr bool T = decltype(tail)::value;
            pf_dequant_v<T, VF16>(rw.h[0], vst, wsp, lane, 0);
            pf_dequant_v<T, VF16>(rw.h[1], vst, wsp, lane, 1);
        };
        using NoTail = std::integral_constant<bool, false>;
        using IsTail = std::integral_constant<bool, true>;
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1 % PF_PDEPTH>;
        using S2 = std::integral_constant<int, 2 % PF_PDEPTH>;
        using S3 = std::integral_constant<int, 3 % PF_PDEPTH>;
        if constexpr (KS == 2) {
            // Half-steps h = 0 .. ntk (a barrier each, after the prologue's):
            // K^ of tile h + 1 and V^T of tile h are written in half-step h
            // (K^ of tile 0 in the prologue).  The K stage (h + 1) % 2 was
            // last read by the QK of tile h - 1 and the V stage h % 2 by the
            // softmax + PV of tile h - 2, both in half-step h - 1.  After V^T
            // of tile h its ring slot takes tile h + PF_PDEPTH.
            static_assert(KS != 2 || PF_PDEPTH == 4, "the KS = 2 producer loop is unrolled for a 4-deep ring");
            if (ntk > 0) {
                pw0 = load_pg(0);
                pw1 = ntk > 64 ? load_pg(1) : 0;
                ready(pw0);
                ready(pw1);
#pragma unroll
                for (int i = 0; i < PF_PDEPTH; ++i) fetch(ring[i], i);
                dequant_k(ring[0], 0);
            }
            __syncthreads();
            // a half-step h < ntk - 1: tile h + 1 in slot SK, tile h in slot SV
            auto hs2 = [&](int hh, auto sv_c, auto sk_c) __attribute__((always_inline)) {
                constexpr int SV = decltype(sv_c)::value, SK = decltype(sk_c)::value;
                dequant_k(ring[SK], hh + 1);
                dequant_v(ring[SV], hh, NoTail{});
                fetch(ring[SV], hh + PF_PDEPTH);
                __syncthreads();
            };
            int hh = 0;
            for (; hh + PF_PDEPTH <= ntk - 1; hh += PF_PDEPTH) {
                slide(hh);
                hs2(hh, S0{}, S1{});
                hs2(hh + 1, S1{}, S2{});
                hs2(hh + 2, S2{}, S3{});
                hs2(hh + 3, S3{}, S0{});
            }
            slide(hh);
            const int rem = ntk - 1 - hh;  // half-steps left before the tail one: 0 .. 3 (uniform)
            if (rem >= 1) hs2(hh, S0{}, S1{});
            if (rem >= 2) hs2(hh + 1, S1{}, S2{});
            if (rem >= 3) hs2(hh + 2, S2{}, S3{});
            if (ntk >= 1) {  // half-step ntk - 1: V^T of the tail tile, from slot (ntk - 1) % 4
                const int tl = ntk - 1;
                switch (tl % PF_PDEPTH) {
                case 0: dequant_v(ring[0], tl, IsTail{}); break;
                case 1: dequant_v(ring[1 % PF_PDEPTH], tl, IsTail{}); break;
                case 2: dequant_v(ring[2 % PF_PDEPTH], tl, IsTail{}); break;
                default: dequant_v(ring[3 % PF_PDEPTH], tl, IsTail{}); break;
                }
                __syncthreads();
            }
            __syncthreads();  // half-step ntk: no producer work
            __syncthreads();  // the consumers' merge exchange
            return;
        }
        if (ntk > 0) {
            pw0 = load_pg(0);
            pw1 = ntk > 64 ? load_pg(1) : 0;
            ready(pw0);
            ready(pw1);
#pragma unroll
            for (int i = 0; i < PF_PDEPTH; ++i) fetch(ring[i], i);
            dequant_k(ring[0], 0);
            if (ntk == 1) dequant_v(ring[0], 0, IsTail{});
            else dequant_v(ring[0], 0, NoTail{});
            fetch(ring[0], PF_PDEPTH);
        }
        __syncthreads();
        // Half-steps h = 0 .. 2 ntk (a barrier each): K^ of tile t is written in
        // h = 2t - 2 and V^ in h = 2t - 1, one half-step before consumer group
        // A reads them (the stage each overwrites was last read in the
        // half-step before).  After V^ of tile t its ring slot takes tile
        // t + PF_PDEPTH.
        auto hstep = [&](int t, auto slot_c) __attribute__((always_inline)) {
            constexpr int SL = decltype(slot_c)::value;  // t % PF_PDEPTH
            dequant_k(ring[SL], t);
            __syncthreads();
            dequant_v(ring[SL], t, NoTail{});
            fetch(ring[SL], t + PF_PDEPTH);
            __syncthreads();
        };
        // tiles 1 .. ntk - 2 (full), then the tail tile ntk - 1
        int t = 1;
        for (; t + PF_PDEPTH <= ntk - 1; t += PF_PDEPTH) {
            slide(t - 1);
            hstep(t, S1{});
            hstep(t + 1, S2{});
            if constexpr (PF_PDEPTH == 4) {
                hstep(t + 2, S3{});
                hstep(t + 3, S0{});
            }
        }
        slide(t - 1);
        const int rem = ntk - 1 - t;  // 0 .. PF_PDEPTH - 1 (uniform)
        if (rem >= 1) hstep(t, S1{});
        if constexpr (PF_PDEPTH == 4) {
            if (rem >= 2) hstep(t + 1, S2{});
            if (rem >= 3) hstep(t + 2, S3{});
        }
        if (ntk >= 2) {  // tile ntk - 1 from slot (ntk - 1) % PF_PDEPTH
            const int tl = ntk - 1;
            switch (tl % PF_PDEPTH) {
            case 0: dequant_k(ring[0], tl); __syncthreads(); dequant_v(ring[0], tl, IsTail{}); break;
            case 1: dequant_k(ring[1 % PF_PDEPTH], tl); __syncthreads(); dequant_v(ring[1 % PF_PDEPTH], tl, IsTail{}); break;
            case 2: dequant_k(ring[2 % PF_PDEPTH], tl); __syncthreads(); dequant_v(ring[2 % PF_PDEPTH], tl, IsTail{}); break;
            default: dequant_k(ring[3 % PF_PDEPTH], tl); __syncthreads(); dequant_v(ring[3 % PF_PDEPTH], tl, IsTail{}); break;
            }
            __syncthreads();
        }
        // the half-steps 2 ntk - 2 .. 2 ntk hold no producer work
        for (int i = ntk >= 1 ? 3 : 1; i > 0; --i) __syncthreads();
        return;
    }

    // ---- consumer: 32 query rows ----------------------------------------
    const int hb = lane >> 5;
    // the wave's 32-row chunk of the tile and its group (A: 0, B: 1)
    const int cw = KS == 1 ? w : w % (PF_CWAVES / 2);
    const int grp = w / (PF_CWAVES / 2);
    // this lane's query row, its causal bound and its Q^T fragments
    const int r = row0 + 32 * cw + (lane & 31);
    const bool rvalid = r < nrows;
    const int j = rvalid ? r / p.G : 0;
    const int hq = h * p.G + (rvalid ? r - j * p.G : 0);
    const int lim = rvalid ? (p.causal ? min(sl - 1, qa + j) : sl - 1) : INT32_MAX;
    const bool wact = row0 + 32 * cw < nrows;  // uniform over the wave (and its KS = 2 partner)
    if (!wact) {
        // all 32 rows past the sequence's rows (its last row tile): keep the
        // workgroup's barrier count
        for (int i = 0; i < (KS == 1 ? 2 * ntk + 2 : ntk + 3); ++i) __syncthreads();
        return;
    }
    half8_t qf[8];
    {
        const float c = p.pf_qmul;  // a power of two: exact for fp16 / bf16 Q
        const int64_t qoff = (int64_t)(q0 + j) * p.q_ts + (int64_t)hq * p.q_hs + 8 * hb;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {  // (row j = 0 stands in for rows past nrows: a valid address)
                const float v = load_as_f32<QDT>(p.q, qoff + 16 * kk + e);
                qf[kk][e] = rvalid ? (half_t)(v * c) : (half_t)0.0f;
            }
        }
    }
    int lim_min;  // smallest bound over the wave's rows: tiles below it need no mask
    {
        const float f = (float)min(lim, 1 << 24);
        lim_min = __builtin_amdgcn_readfirstlane((int)(-row16_max(xrow_max(-f))));
    }

    float16v_t o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] = 0.0f;
    // Running max m (log2 units) enters the S MFMA chain as its accumulator
    // input (-m in all 16 registers), so S' = S - m comes out of the matrix
    // core directly.  has_m: a visible key has been seen (m valid).
    float m_use = 0.0f, l_run = 0.0f;
    bool has_m = false;
    bool all_m = false;  // wave-uniform: every lane's has_m

    // lane-constant LDS offsets of the MFMA operands
    const int kread = (lane & 31) * PF_KPITCH + 16 * hb;  // + 32*st*KPITCH + 32*kk
    const int vread = (lane & 31) * PF_VPITCH + 16 * hb;  // + 32*dt*VPITCH + 16*(4st+2sg)

    // The two consumer waves of a SIMD run half a tile apart: group A (waves
    // 0-3) computes S' of tile kt in half-step 2kt and its softmax + PV in
    // half-step 2kt + 1; group B (waves 4-7) one half-step later.  Each
    // half-step a SIMD then holds one wave's QK MFMAs and the other's
    // exponentials and PV MFMAs.
    float16v_t sacc[PF_NST];  // S' of the tile between its two half-steps
    // S'^T = K^ . Q^T - m for the 32-key subtiles of the tile (stage kst)
    auto qk = [&](const uint8_t *kst) __attribute__((always_inline)) {
        // -m in all 16 accumulator registers, the srcC of the first MFMA of
        // both chains.  Each 64-bit pair passes through an empty asm so that
        // the compiler copies it with one v_mov_b64 (7 moves, against 15
        // v_mov_b32 for a plain splat).  Empty asm statements count as no
        // wait states, so the VALU-write -> MFMA-read gap is still enforced.
        float16v_t msp;
        {
            const uint64_t pr = ((uint64_t)__float_as_uint(-m_use) << 32) | __float_as_uint(-m_use);
            u64x8_t sp;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                uint64_t t = pr;
                asm volatile("" : "+v"(t));
                sp[e] = t;
            }
            msp = __builtin_bit_cast(float16v_t, sp);
        }
#pragma unroll
        for (int st = 0; st < PF_NST; ++st) {
            sacc[st] = msp;
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                const half8_t a = *reinterpret_cast<const half8_t *>(kst + kread + 32 * st * PF_KPITCH + 32 * kk);
                sacc[st] = mfma32(a, qf[kk], sacc[st]);
            }
        }
        // Schedule of this block: the K^ operand reads run two ahead of the
        // MFMAs (read, read, then MFMA / read pairs), in the registers of
        // the two in flight.  The compiler's own order waited for each pair
        // before its two MFMAs.  One box: cfg3 11.48 -> 11.20 ms, cfg4 5.93
        // -> 5.83 ms; three ahead: cfg3 11.22 ms, cfg4 5.90 ms.
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS reads
#pragma unroll
        for (int i = 0; i < 8 * PF_NST - 1; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    };
    // softmax and O += P V^ over tile kt (stage vst)
    auto sv = [&](int kt, const uint8_t *vst) __attribute__((always_inline)) {
        const int kbase_t = PF_TK * (kt + ktb);
        if constexpr (MASK) {  // S' += mask[s][j][key] (natural log units -> log2)
            const uint16_t *mrow = p.mask + (int64_t)s * p.mask_bs + (int64_t)j * p.mask_rs;
            if (p.mask_vec) {  // uniform: the lane's keys come in runs of 4 (register e = 4q + i)
#pragma unroll
                for (int st = 0; st < PF_NST; ++st)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int key = kbase_t + 32 * st + 8 * q + 4 * hb;  // a multiple of 4
                        uint2 w = {0u, 0u};
                        if (key < p.mask_cols) w = *reinterpret_cast<const uint2 *>(mrow + key);
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const uint16_t hb16 = (uint16_t)((i < 2 ? w.x : w.y) >> (16 * (i & 1)));
                            sacc[st][4 * q + i] = fmaf(half_bits_to_f32(hb16), LOG2E, sacc[st][4 * q + i]);
                        }
                    }
            } else {
#pragma unroll
                for (int st = 0; st < PF_NST; ++st)
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int key = kbase_t + 32 * st + 8 * (e >> 2) + 4 * hb + (e & 3);
                        const float mv = key < p.mask_cols ? half_bits_to_f32(mrow[key]) : 0.0f;
                        sacc[st][e] = fmaf(mv, LOG2E, sacc[st][e]);
                    }
            }
        }
        if (kbase_t + PF_TK - 1 > lim_min) {  // uniform: tile crosses some row's bound
#pragma unroll
            for (int st = 0; st < PF_NST; ++st)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int key = kbase_t + 32 * st + 8 * (e >> 2) + 4 * hb + (e & 3);
                    sacc[st][e] = key <= lim ? sacc[st][e] : -INFINITY;
                }
        }
        // The lane's own max over its 32 keys, as a tree of depth 4.  A row's
        // max is the larger of its two lanes', so
        // "every lane <= LAZY_TAU once every row has m" is exactly the case in
        // which the rescale below would change nothing: that test needs no
        // cross-lane step.
        float mx = tile_max32(sacc[0], sacc[1]);
        if (!all_m || __builtin_amdgcn_ballot_w64(mx > LAZY_TAU)) {  // wave-uniform, rare after the first tile
            auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
            mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
            // lazy rescale: move m only when the tile max exceeds it by > LAZY_TAU
            // (or on the first visible key of the row)
            const bool need = has_m ? mx > LAZY_TAU : mx > -INFINITY;
            if (__builtin_amdgcn_ballot_w64(need)) {
                const float delta = need ? mx : 0.0f;
                const float alpha = (need && has_m) ? __builtin_amdgcn_exp2f(-delta) : 1.0f;
                m_use += delta;
                has_m = has_m || need;
                l_run *= alpha;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
#pragma unroll
                for (int st = 0; st < PF_NST; ++st) sacc[st] -= delta;
            }
            all_m = __builtin_amdgcn_ballot_w64(!has_m) == 0;
        }
        // Row sum of the fp16-rounded p with v_dot2 (the same values the PV
        // MFMAs consume).
        const half2_t ones = {(half_t)1.0f, (half_t)1.0f};
        float tsum = 0.0f;
#pragma unroll
        for (int st = 0; st < PF_NST; ++st) {
#pragma unroll
            for (int sg = 0; sg < 2; ++sg) {
                PHalf8 pk;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float p0 = __builtin_amdgcn_exp2f(sacc[st][8 * sg + 2 * e]);
                    const float p1 = __builtin_amdgcn_exp2f(sacc[st][8 * sg + 2 * e + 1]);
                    pk.h[e] = half2_t{(half_t)p0, (half_t)p1};
                    tsum = __builtin_amdgcn_fdot2(pk.h[e], ones, tsum, false);
                }
                const half8_t pb = __builtin_bit_cast(half8_t, pk);
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    const half8_t a = *reinterpret_cast<const half8_t *>(
                        vst + vread + 32 * dt * PF_VPITCH + 16 * (4 * st + 2 * sg));
                    o[dt] = mfma32(a, pb, o[dt]);
                }
            }
        }
        l_run += tsum;
    };
    __syncthreads();  // the producers' first tile
    if constexpr (KS == 1) {
        if (grp) __syncthreads();  // half-step 0
        for (int kt = 0, stg = 0; kt < ntk; ++kt, stg = stg == NSTAGE - 1 ? 0 : stg + 1) {
            qk(ldsk + stg * PF_KBYTES);
            __syncthreads();
            sv(kt, ldsv + stg * PF_VBYTES);
            __syncthreads();
        }
        if (!grp) __syncthreads();  // half-step 2 ntk (group B's last softmax)
    } else {
        // group A: the even tiles (QK in half-step kt, softmax + PV in kt + 1)
        // from stage 0; group B: the odd tiles from stage 1.  Both then pad
        // to the ntk + 2 barriers of the producers' half-steps.
        if (grp) __syncthreads();  // half-step 0
        const uint8_t *kst = ldsk + grp * PF_KBYTES;
        const uint8_t *vst = ldsv + grp * PF_VBYTES;
        for (int kt = grp; kt < ntk; kt += 2) {
            qk(kst);
            __syncthreads();
            sv(kt, vst);
            __syncthreads();
        }
        if ((ntk & 1) == grp) __syncthreads();
    }

    // normalise and store: register e of d-tile dt is d = 32dt + 8(e/4) + 4hb + e%4
    auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
    float l = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    float mrow = has_m ? m_use : -INFINITY;
    using D0 = std::integral_constant<int, 0>;
    using D2 = std::integral_constant<int, 2>;
    if constexpr (KS == 2) {
        // Merge the pair's partial states through LDS (the stages are free:
        // every read of them ended before the last barrier).  Group A stores
        // d-tiles 0-1 and sends 2-3, group B the reverse; both send (m, l).
        // Layout [group][chunk][8 float4][64 lanes]: a wave's 16-byte stores
        // and loads are lane-contiguous.
        float4_t *xo = reinterpret_cast<float4_t *>(lds);
        float2_t *xml = reinterpret_cast<float2_t *>(lds + 2 * 4 * 8 * 64 * 16);
        static_assert(2 * 4 * 8 * 64 * 16 + 2 * 4 * 64 * 8 <= NSTAGE * (PF_KBYTES + PF_VBYTES), "merge fits the stages");
        float4_t *mine = xo + (grp * 4 + cw) * 8 * 64 + lane;
        auto send = [&](auto dtb) __attribute__((always_inline)) {
            constexpr int DB = decltype(dtb)::value;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4)
                    mine[(4 * i + q4) * 64] = float4_t{o[DB + i][4 * q4], o[DB + i][4 * q4 + 1], o[DB + i][4 * q4 + 2],
                                                       o[DB + i][4 * q4 + 3]};
        };
        if (grp == 0) send(D2{});
        else send(D0{});
        xml[(grp * 4 + cw) * 64 + lane] = float2_t{mrow, l};
        __syncthreads();
        const float4_t *theirs = xo + ((1 - grp) * 4 + cw) * 8 * 64 + lane;
        const float2_t mlp = xml[((1 - grp) * 4 + cw) * 64 + lane];
        const float M = fmaxf(mrow, mlp[0]);
        const bool none = M == -INFINITY;  // neither half saw a key of this row
        const float a = none ? 0.0f : __builtin_amdgcn_exp2f(mrow - M);
        const float b = none ? 0.0f : __builtin_amdgcn_exp2f(mlp[0] - M);
        auto merge = [&](auto dtb) __attribute__((always_inline)) {
            constexpr int DB = decltype(dtb)::value;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const float4_t t = theirs[(4 * i + q4) * 64];
#pragma unroll
                    for (int k = 0; k < 4; ++k) o[DB + i][4 * q4 + k] = fmaf(o[DB + i][4 * q4 + k], a, t[k] * b);
                }
        };
        if (grp == 0) merge(D0{});
        else merge(D2{});
        l = fmaf(l, a, mlp[1] * b);
        mrow = M;
    }
    // stores d-tiles DB .. DB + ND - 1 of the wave's rows
    auto store_tiles = [&](auto dtb, auto ndt) __attribute__((always_inline)) {
        constexpr int DB = decltype(dtb)::value, ND = decltype(ndt)::value;
        if (slot >= 0) {  // a piece of a split row tile: unnormalised O, m (log2), l
            const int rl = 32 * cw + (lane & 31);
            if (!rvalid) return;  // the combine reads the sequence's rows only
            const int64_t reg = (int64_t)slot * Hkv + h;
            float *po = p.pf_o + (reg * ROWS + rl) * 128 + 4 * hb;
#pragma unroll
            for (int dt = DB; dt < DB + ND; ++dt)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4)
                    *reinterpret_cast<float4_t *>(po + 32 * dt + 8 * q4) =
                        float4_t{o[dt][4 * q4], o[dt][4 * q4 + 1], o[dt][4 * q4 + 2], o[dt][4 * q4 + 3]};
            if (DB == 0 && hb == 0) {
                float *pm = p.pf_ml + (reg * ROWS + rl) * 2;
                pm[0] = mrow;
                pm[1] = l;
            }
        } else if (rvalid) {
            const float inv = l > 0.f ? 1.0f / l : 0.0f;
            const int64_t ob = (int64_t)(q0 + j) * p.o_ts + (int64_t)hq * p.o_hs + 4 * hb;
#pragma unroll
            for (int dt = DB; dt < DB + ND; ++dt)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    store_out<ODT>(p.out, ob + 32 * dt + 8 * (e >> 2) + (e & 3), o[dt][e] * inv);
        }
    };
    if constexpr (KS == 1) store_tiles(D0{}, std::integral_constant<int, 4>{});
    else if (grp == 0) store_tiles(D0{}, D2{});
    else store_tiles(D2{}, D2{});
}

// ---------------------------------------------------------------------------
// Prefill work list.  One workgroup enumerates every (sequence, row tile)
// of prefill work and counting-sorts the items by the number of 64-key tiles
// their causal range spans, heaviest first, so that the prefill grid
// dispatches the longest workgroups first whatever the order of the
// sequences in the batch (a mixed batch otherwise ends on a tail of its
// longest-context chunk running on part of the device).
constexpr int PL_THREADS = 1024;
constexpr int PL_MAX_SEQS = 8192;  // larger batches keep the 2-D grid
constexpr int PL_BUCKETS = 4096;   // key tiles per item, clamped (256K keys)
#ifndef GFA_PF_SPLIT_MIN
#define GFA_PF_SPLIT_MIN 16
#endif
constexpr int PF_SPLIT_MIN = GFA_PF_SPLIT_MIN;  // a split row tile's pieces: at least this many tiles
#ifndef GFA_PFC_WGS_PER_CU
#define GFA_PFC_WGS_PER_CU 4  // split-merge workgroups per CU (more loads in flight)
#endif

// The plan's workgroup-wide ordering point.  On one wave (NT = 64) it needs
// no barrier: a wave's LDS instructions complete in the order it issues
// them, and the wave-scope fence keeps the compiler from moving LDS accesses
// across it.  (A workgroup barrier would also wait for the wave's global
// stores to complete, which the plan never needs.)
template <int NT>
__device__ __forceinline__ void pl_sync() {
    if constexpr (NT == 64) {
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    } else {
        __syncthreads();
    }
}

template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// sum over the wave, every lane receives it: butterflies within each 16-lane
// DPP row, then across the four rows with the permlane swaps
__device__ __forceinline__ int pl_wave_sum32(int v) {
    v += dpp_i32<DPP_QUAD_XOR1>(v);
    v += dpp_i32<DPP_QUAD_XOR2>(v);
    v += dpp_i32<DPP_ROW_HALF_MIRROR>(v);
    v += dpp_i32<DPP_ROW_MIRROR>(v);
    const auto a = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
    v = (int)(a[0] + a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    return (int)(b[0] + b[1]);
}

// exclusive scan of v over the workgroup; *total receives the sum (a scan
// inside each wave, then the waves' totals through tmp)
template <int NT>
__device__ __forceinline__ int pl_block_scan(int v, int *tmp, int *total) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off);
        if (lane >= off) x += y;
    }
    if constexpr (NT == 64) {
        *total = __builtin_amdgcn_readlane(x, 63);
        return x - v;
    }
    __syncthreads();  // tmp[] of a previous call has been read
    if (lane == 63) tmp[wv] = x;
    __syncthreads();
    int before = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) {
        const int t = tmp[i];
        before += i < wv ? t : 0;
        tot += t;
    }
    *total = tot;
    return before + x - v;
}

// floor(a / b) for a >= 0, b >= 1.  Below 2^22 from the float quotient,
// which is then within 1 of it, and one correction each way (the compiler's
// integer division is a long instruction sequence).
__device__ __forceinline__ int pl_div(int a, int b) {
    if (a >= (1 << 22)) return a / b;
    int q = (int)((float)a * __builtin_amdgcn_rcpf((float)b));
    const int r = a - q * b;
    q += r < 0 ? -1 : (r >= b ? 1 : 0);
    return q;
}

// A sequence's scalars as the plan reads them.
struct PlSeq {
    int nq, sl, qa;
};

__device__ __forceinline__ PlSeq pl_seq(const AttnParams &p, int s) {
    PlSeq q;
    q.nq = p.qsl[s + 1] - p.qsl[s];
    q.sl = p.seq_lens[s];
    q.qa = p.q_abs ? p.q_abs[s] : q.sl - q.nq;
    return q;
}

// prefill row tiles of a sequence (0 for decode sequences)
__device__ __forceinline__ int pl_tiles(const AttnParams &p, const PlSeq &q) {
    const int nrows = q.nq * p.G;
    return (q.nq > 0 && nrows > p.dec_rows_max) ? pl_div(nrows + p.pf_rows - 1, p.pf_rows) : 0;
}

// 64-key tiles row tile rt of a sequence attends (the prefill kernel's ntk_all)
__device__ __forceinline__ int pl_ntk(const AttnParams &p, const PlSeq &q, int rt) {
    const int nrows = q.nq * p.G;
    const int jlast = pl_div(min(p.pf_rows * (rt + 1), nrows) - 1, p.G);
    const int kv_end = p.causal ? min(q.sl, max(q.qa + jlast + 1, 0)) : q.sl;
    return (kv_end + PF_TK - 1) / PF_TK;
}

__device__ __forceinline__ int pl_bucket(int tiles) { return min(tiles, PL_BUCKETS - 1); }

// sum of v over the workgroup (every thread receives it)
template <int NT>
__device__ __forceinline__ long long pl_block_sum(long long v, long long *red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    if constexpr (NT == 64) return uniform64(v);  // (in scalar registers: the plan's control flow is uniform)
    __syncthreads();  // red[] of a previous call has been read
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    long long t = 0;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) t += red[i];
    return t;
}

// max of v over the workgroup (every thread receives it)
template <int NT>
__device__ __forceinline__ long long pl_block_max(long long v, long long *red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = max(v, (long long)__shfl_xor(v, off));
    if constexpr (NT == 64) return uniform64(v);
    __syncthreads();  // red[] of a previous call has been read
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    long long t = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) t = max(t, red[i]);
    return t;
}

// Pieces row tile of w key tiles is cut into when pieces hold at most tsplit
// tiles; piece c of k covers tiles [c*w/k, (c+1)*w/k).
__device__ __forceinline__ int pl_pieces(int w, int tsplit) { return w > tsplit ? pl_div(w + tsplit - 1, tsplit) : 1; }

template <int NT>
__global__ __launch_bounds__(NT) void prefill_plan_kernel(AttnParams p) {
    __shared__ int s_pre[PL_MAX_SEQS + 1];  // exclusive prefix of row tiles per sequence
    __shared__ int s_bk[PL_BUCKETS];        // bucket counts, then write cursors
    __shared__ int s_tmp[NT / 64];
    __shared__ long long s_red[NT / 64];
    __shared__ int s_w[NT];  // key tiles of row tile i (launches of <= NT row tiles)
    __shared__ PlSeq s_seq[NT];  // the sequences' scalars (launches of <= NT sequences)
    __shared__ int s_nsplit, s_nslot;
    const int B = p.num_seqs, tid = threadIdx.x;
    int carry = 0;
    // image tiles of a prefill sequence: the key tiles of its last row tile
    // (the longest causal range); a sequence past 2^20 of them (64M keys)
    // leaves the whole call without images
    constexpr int IMG_SEQ_MAX = 1 << 20;
    long long icarry = 0;
    int ibig = 0;
    for (int base = 0; base < B; base += NT) {
        const int sq = base + tid;
        PlSeq qs = {0, 0, 0};
        if (sq < B) qs = pl_seq(p, sq);  // one round of loads
        if (B <= NT) s_seq[tid] = qs;
        const int v = sq < B ? pl_tiles(p, qs) : 0;
        int tot;
        const int ex = pl_block_scan<NT>(v, s_tmp, &tot);
        if (sq < B) s_pre[sq] = carry + ex;
        carry += tot;
        int vt = v > 0 ? pl_ntk(p, qs, v - 1) : 0;
        ibig |= vt > IMG_SEQ_MAX;
        vt = min(vt, IMG_SEQ_MAX);
        int itot;
        const int iex = pl_block_scan<NT>(vt, s_tmp, &itot);
        if (p.pf_tbase != nullptr && sq < B) p.pf_tbase[sq] = (int)min(icarry + iex, (long long)INT32_MAX);
        icarry += itot;
    }
    const bool img_big = pl_block_max<NT>(ibig, s_red) != 0;
    if (tid == 0) {
        s_pre[B] = carry;
        s_nsplit = 0;
        s_nslot = 0;
        if (p.pf_tbase != nullptr) p.pf_tbase[B] = (int)min(icarry, (long long)INT32_MAX);
    }
    pl_sync<NT>();
    const int n = min(carry, p.pf_items_max);
    auto seq_of = [&](int sq) { return B <= NT ? s_seq[sq] : pl_seq(p, sq); };
    // item i -> (sequence, row tile): the last sequence whose prefix is <= i
    auto locate = [&](int i, int &sq, int &rt) {
        int lo = 0, hi = B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (s_pre[mid] <= i) lo = mid;
            else hi = mid - 1;
        }
        sq = lo;
        rt = i - s_pre[lo];
    };
    // Split: a row tile longer than tsplit key tiles is cut into pieces of at
    // most tsplit.  tsplit starts at one CU's share of the launch's key tiles
    // (all row tiles x kv heads over pf_ncu; at least PF_SPLIT_MIN): split row
    // tiles then number < pf_ncu / Hkv, their pieces < 2 pf_ncu / Hkv, and the
    // extra work items < pf_ncu / Hkv.
    // With few row tiles (n <= 2m, m = pf_ncu / Hkv: one or two rounds of
    // workgroups) the rounds decide the time instead: a few workgroups over a
    // multiple of the CU count start another round.  tsplit then rises to the
    // smallest value whose pieces fit R rounds (sum of pieces <= R m): R = 1
    // for n < m, else one round more than the unsplit row tiles take, kept
    // only if R rounds of tsplit beat the unsplit rounds of the longest row
    // tile by 10 %.  Pieces then number <= 3m and split row tiles <= 2m.
    // Past the workspace's bounds (impossible by these sums) nothing is split.
    long long wsum = 0, wmx = 0;
    for (int i = tid; i < n; i += NT) {
        int sq, rt;
        locate(i, sq, rt);
        const int w = pl_ntk(p, seq_of(sq), rt);
        if (n <= NT) s_w[i] = w;
        wsum += w;
        wmx = max(wmx, (long long)w);
    }
    // (the block reductions below order these stores before their reads)
    auto ntk_of = [&](int i, int sq, int rt) { return n <= NT ? s_w[i] : pl_ntk(p, seq_of(sq), rt); };
    const long long W = pl_block_sum<NT>(wsum, s_red);
    const long long wmax = pl_block_max<NT>(wmx, s_red);  // the longest row tile
    long long tl = max((W * p.Hkv + p.pf_ncu - 1) / p.pf_ncu, (long long)PF_SPLIT_MIN);
    const int m = p.pf_ncu / p.Hkv;
    bool proven = false;  // the bisection's sums bound the plan: no check pass
    if (m > 0 && n > 0 && n <= 2 * m && n <= NT && p.pf_slots_max > 0) {
        int wt = 0;  // thread t holds row tile t's key tiles
        if (tid < n) wt = s_w[tid];
        const int rounds0 = (n + m - 1) / m;       // unsplit, all row tiles alike
        const int R = n < m ? 1 : rounds0 + 1;
        const long long cap = (long long)R * m;   // > n
        // pieces(tsplit) is non-increasing, >= W / tsplit, and at hi sums to
        // <= W / hi + n <= cap
        long long lo = max((W + cap - 1) / cap, (long long)PF_SPLIT_MIN);
        long long hi = max(lo, (W + (cap - n) - 1) / (cap - n));
        while (lo < hi) {
            const long long mid = (lo + hi) >> 1;
            long long P;
            if constexpr (NT == 64) {  // 32-bit DPP sum; counts above 2^24 only need to exceed cap
                const int k = tid < n ? pl_pieces(wt, (int)min(mid, (long long)INT32_MAX)) : 0;
                P = __builtin_amdgcn_readfirstlane(pl_wave_sum32(min(k, 1 << 24)));
            } else {
                P = pl_block_sum<NT>(tid < n ? pl_pieces(wt, (int)min(mid, (long long)INT32_MAX)) : 0, s_red);
            }
            if (P <= cap) hi = mid;
            else lo = mid + 1;
        }
        if (R == 1 || 10 * R * lo < 9LL * rounds0 * wmax) {
            tl = lo;
            proven = true;  // pieces <= R m <= 3m, split row tiles <= n <= 2m
        }
    }
    int tsplit = (p.pf_slots_max > 0 && tl < wmax) ? (int)tl : INT32_MAX;  // else nothing is cut
    if (tsplit < INT32_MAX && !proven) {
        long long ex = 0, sl = 0, ns = 0;
        for (int i = tid; i < n; i += NT) {
            int sq, rt;
            locate(i, sq, rt);
            const int k = pl_pieces(ntk_of(i, sq, rt), tsplit);
            if (k > 1) {
                ex += k - 1;
                sl += k;
                ns += 1;
            }
        }
        ex = pl_block_sum<NT>(ex, s_red);
        sl = pl_block_sum<NT>(sl, s_red);
        ns = pl_block_sum<NT>(ns, s_red);
        if (n + ex > p.pf_grid_items || sl > p.pf_slots_max || ns > p.pf_split_max) tsplit = INT32_MAX;
    }
    // buckets that can hold an item: an unsplit row tile has at most
    // min(wmax, tsplit) key tiles, and so has a piece of a split one
    const int nb = (int)min(min(wmax, (long long)tsplit), (long long)PL_BUCKETS - 1) + 1;
    for (int b = tid; b < nb; b += NT) s_bk[b] = 0;
    pl_sync<NT>();
    for (int i = tid; i < n; i += NT) {
        int sq, rt;
        locate(i, sq, rt);
        const int w = ntk_of(i, sq, rt);
        const int k = pl_pieces(w, tsplit);
        if (k == 1) {
            atomicAdd(&s_bk[pl_bucket(w)], 1);
        } else {  // w % k pieces of w / k + 1 tiles, the others of w / k
            const int q = pl_div(w, k), big = w - q * k;
            if (big) atomicAdd(&s_bk[pl_bucket(q + 1)], big);
            atomicAdd(&s_bk[pl_bucket(q)], k - big);
        }
    }
    pl_sync<NT>();
    // write cursors in descending bucket order: thread t owns the per
    // buckets nb-1-per*t .. nb-per-per*t (those >= 0)
    int total;
    {
        const int per = (nb + NT - 1) / NT;
        int loc = 0;
        for (int k = 0; k < per; ++k) {
            const int b = nb - 1 - (per * tid + k);
            if (b >= 0) loc += s_bk[b];
        }
        int run = pl_block_scan<NT>(loc, s_tmp, &total);
        for (int k = 0; k < per; ++k) {
            const int b = nb - 1 - (per * tid + k);
            if (b >= 0) {
                const int c = s_bk[b];
                s_bk[b] = run;
                run += c;
            }
        }
    }
    pl_sync<NT>();
    for (int i = tid; i < n; i += NT) {
        int sq, rt;
        locate(i, sq, rt);
        const int w = ntk_of(i, sq, rt);
        const int k = pl_pieces(w, tsplit);
        int slot0 = -1;
        if (k > 1) {
            slot0 = atomicAdd(&s_nslot, k);
            int *e = p.pf_split + 4 * atomicAdd(&s_nsplit, 1);
            e[0] = sq;
            e[1] = rt;
            e[2] = slot0;
            e[3] = k;
        }
        // piece c: tiles [c w / k, (c + 1) w / k), stepped without a division:
        // (c + 1) w = (a + q) k + (rem + rw) for a = c w / k, rem = c w % k
        const int q = pl_div(w, k), rw = w - q * k;
        int b = 0, rem = 0;
        for (int c = 0; c < k; ++c) {
            const int a = b;
            rem += rw;
            b = a + q + (rem >= k ? 1 : 0);
            rem -= rem >= k ? k : 0;
            const int pos = atomicAdd(&s_bk[pl_bucket(b - a)], 1);
            p.pf_seq[pos] = sq;
            p.pf_rt[pos] = rt;
            p.pf_kt0[pos] = a;
            p.pf_kt1[pos] = k > 1 ? b : INT32_MAX;
            p.pf_slot[pos] = k > 1 ? slot0 + c : -1;
        }
    }
    pl_sync<NT>();
    if (tid == 0) {
        p.pf_count[0] = total;
        p.pf_count[1] = s_nsplit;
        // the tile images: all of them in the workspace's image region, or
        // none; and only where the row tiles read each tile PF_IMG_REUSE times
        // on average (writing an image costs about what that many workgroups
        // save by copying it instead of dequantizing)
        const bool fit = p.pf_tiles != nullptr && !img_big && icarry <= INT32_MAX &&
                         icarry <= p.pf_tiles_cap / ((long long)p.Hkv * PF_IMG_BYTES) &&
                         W >= (long long)PF_IMG_REUSE * icarry;
        p.pf_count[2] = fit ? 1 : 0;
        p.pf_count[3] = fit ? (int)icarry : 0;
    }
}

// Writes the dequantized tile images of a work-list launch (when the plan
// kernel chose them): image (tbase[s] + kt) * Hkv + h holds K^ and V^T of
// keys 64 kt .. 64 kt + 63 of sequence s, kv-head h, exactly as the prefill
// producers would dequantize them into LDS (the same functions, so the same
// bytes).  Sub-pages past the sequence's last key read its last valid
// sub-page, and the V scales are made finite in every tile: keys past a row
// tile's causal bound are masked to P = 0, which must meet finite V^.
// Persistent grid; a workgroup's four waves dequantize the four sub-pages of
// one image into LDS, then write it out in whole 16-byte rows per lane.
template <bool VF16>
__global__ __launch_bounds__(64 * PF_NSP) void prefill_tiles_kernel(AttnParams p) {
    __shared__ __attribute__((aligned(16))) uint8_t img_lds[PF_IMG_BYTES];
    if (p.pf_tiles == nullptr || p.pf_count[2] == 0) return;  // uniform
    const int64_t n = (int64_t)p.pf_count[3] * p.Hkv;
    const int lane = threadIdx.x & 63;
    const int wsp = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int B = p.num_seqs, Hkv = p.Hkv, bs = p.block_size;
    constexpr int VSUB = VF16 ? 4096 : SUBPAGE_BYTES;
    for (int64_t i = blockIdx.x; i < n; i += gridDim.x) {
        const int tix = (int)(i / Hkv), h = (int)(i - (int64_t)tix * Hkv);
        // its sequence: the last s < B with tbase[s] <= tix (sequences with no
        // images share their successor's base), a 64-way search per step
        int lo = 0, hi = B;
        while (hi - lo > 1) {
            const int step = (hi - lo + 63) >> 6;
            const int idx = lo + lane * step;
            const bool le = idx < hi && p.pf_tbase[idx] <= tix;
            const uint64_t bal = __ballot(le);  // a prefix of the lanes, lane 0 included
            const int k = 63 - __builtin_clzll(bal);
            lo += k * step;
            hi = min(hi, lo + step);
        }
        const int s = __builtin_amdgcn_readfirstlane(lo);
        const int kt = tix - p.pf_tbase[s];
        const int nq = p.qsl[s + 1] - p.qsl[s];
        const int sl = p.seq_lens[s];
        const int qa = p.q_abs ? p.q_abs[s] : sl - nq;
        const int kv_lim = p.causal ? min(sl, max(qa + nq, 0)) : sl;
        const int sp = min(PF_NSP * kt + wsp, max((kv_lim - 1) >> 4, 0));
        const int64_t page = p.bt[(int64_t)s * p.bt_stride + (16 * sp) / bs];
        const int64_t spi = ((16 * sp) % bs) >> 4;
        const uint8_t *kb = p.kc + (int64_t)h * p.chs + page * p.cbs + spi * SUBPAGE_BYTES;
        const uint8_t *vb = p.vc + (int64_t)h * p.vchs + page * p.vcbs + spi * VSUB;
        PfRaw r0, r1;
        pf_fetch<VF16>(r0, kb, vb, lane, 0);
        pf_fetch<VF16>(r1, kb, vb, lane, 1);
        __syncthreads();  // the previous image has been written out
        pf_dequant_k(r0, img_lds, wsp, lane, 0, p.pf_kmul);
        pf_dequant_k(r1, img_lds, wsp, lane, 1, p.pf_kmul);
        pf_dequant_v<true, VF16>(r0, img_lds + PF_KBYTES, wsp, lane, 0);
        pf_dequant_v<true, VF16>(r1, img_lds + PF_KBYTES, wsp, lane, 1);
        __syncthreads();
        uint8_t *img = p.pf_tiles + i * PF_IMG_BYTES;
        for (int o = 16 * threadIdx.x; o < PF_IMG_BYTES; o += 16 * 64 * PF_NSP)
            *reinterpret_cast<u32x4 *>(img + o) = *reinterpret_cast<const u32x4 *>(img_lds + o);
    }
}

// Merges the pieces of each split row tile: per row, an online merge of the
// pieces' (m, l, O) - the running sums rescaled to the largest m so far - and
// O divided by l at the end (0 for a row no piece saw a key of).  A unit is 16
// rows of one (split row tile, kv head): 32 lanes per row, four d each, two
// rows per thread.  A thread issues the loads of both rows for four pieces
// before merging them, so they are in flight together.
template <int ODT>
__global__ __launch_bounds__(256) void attn_prefill_combine_kernel(AttnParams p) {
    constexpr int RPU = 16, U = 4;
    const int nsplit = p.pf_count[1];
    const int prows = p.pf_rows;
    const int units = nsplit * p.Hkv * (prows / RPU);
    const int rr = threadIdx.x >> 5, d = 4 * (threadIdx.x & 31);
    const int64_t rstep = (int64_t)p.Hkv * prows;  // piece c -> c + 1
    for (int u = blockIdx.x; u < units; u += gridDim.x) {
        const int h = u % p.Hkv;
        const int t = u / p.Hkv;
        const int rg = t % (prows / RPU);
        const int *e = p.pf_split + 4 * (t / (prows / RPU));
        const int s = e[0], rt = e[1], slot0 = e[2], k = e[3];
        const int q0 = p.qsl[s];
        const int nrows = (p.qsl[s + 1] - q0) * p.G;
        float M[2], L[2];
        float4_t acc[2];
        int64_t reg0[2];
        bool ok[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int rl = RPU * rg + rr + 8 * i;  // row inside the tile
            ok[i] = prows * rt + rl < nrows;
            reg0[i] = ((int64_t)slot0 * p.Hkv + h) * prows + rl;
            M[i] = -INFINITY;
            L[i] = 0.f;
            acc[i] = float4_t{0.f, 0.f, 0.f, 0.f};
        }
        for (int c0 = 0; c0 < k; c0 += U) {
            float2_t ml[2][U];
            float4_t oc[2][U];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < U; ++j) {
                    const int64_t reg = reg0[i] + (c0 + j) * rstep;
                    const bool in = ok[i] && c0 + j < k;
                    ml[i][j] = in ? *reinterpret_cast<const float2_t *>(p.pf_ml + reg * 2) : float2_t{-INFINITY, 0.f};
                    oc[i][j] = in ? *reinterpret_cast<const float4_t *>(p.pf_o + reg * 128 + d)
                                  : float4_t{0.f, 0.f, 0.f, 0.f};
                }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < U; ++j) {
                    const float mc = ml[i][j][0];
                    if (mc > -INFINITY) {
                        const float mn = fmaxf(M[i], mc);
                        const float a = __builtin_amdgcn_exp2f(M[i] - mn);  // 0 while M is -inf
                        const float b = __builtin_amdgcn_exp2f(mc - mn);
                        L[i] = fmaf(L[i], a, b * ml[i][j][1]);
                        acc[i] = acc[i] * a + b * oc[i][j];
                        M[i] = mn;
                    }
                }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if (!ok[i]) continue;
            const int r = prows * rt + RPU * rg + rr + 8 * i;
            const float inv = L[i] > 0.f ? 1.0f / L[i] : 0.0f;
            const int j = r / p.G;
            const int hq = h * p.G + (r - j * p.G);
            const int64_t ob = (int64_t)(q0 + j) * p.o_ts + (int64_t)hq * p.o_hs + d;
#pragma unroll
            for (int x = 0; x < 4; ++x) store_out<ODT>(p.out, ob + x, acc[i][x] * inv);
        }
    }
}

// ---------------------------------------------------------------------------
// Contiguous decode: the op module's forward() for rows (Sq * G per kv-head)
// that fit one 16-row group, with no mask.  It reads the reference's
// contiguous layouts as they are (extension/gfx906_fa.cpp:120-265): K as
// AoS Q8_0 rows [B][Hkv][Skv][136 B], V as fp16 rows [B][Hkv][Skv][128], so
// no repacking pass runs.  A segment is one (batch, kv-head); its 16-token
// sub-pages are cut into P equal pieces, one single-wave workgroup each
// (grid B * Hkv * P).  A piece streams its sub-pages through a 3-slot LDS
// ring, two sub-pages ahead (global_load_lds copies: 2176 B of K rows, 4096
// B of V rows), and computes as the decode kernel's one-row-group tile:
//   S^T = K^ . Q^T   4 x mfma 16x16x32, K^ = fp16(q * d_k) per lane from its
//                    token's AoS row (8 int8 of block b at 34b + 2 + 8g);
//   O^T += V^T . P^T 8 x mfma 16x16x16, V exact in fp16 (lane (i, g) reads
//                    d = 16m + i of tokens 4g..4g+3), P unscaled.
// With P = 1 the piece writes the normalized output, else (m, l, O) for
// flat_combine_kernel.  A segment's K rows start 8 bytes past a 16-byte
// boundary when seg * Skv is odd (136-byte rows, a 16-byte aligned tensor):
// the copies then start at the boundary below (koff = 8), and the K region
// of a slot has room for the extra bytes.  A segment's last sub-page is read
// with guarded dword loads (zeros past Skv), so no copy reads past a
// segment's rows (nor, for the first segment, before them: koff = 0).
constexpr int FD_KROWS = 16 * 136;             // K rows of a sub-page
constexpr int FD_KREG = FD_KROWS + 16;         // their slot region (koff + rows, 16-byte multiple)
constexpr int FD_SLOT = FD_KREG + 16 * 256;    // then the V rows
constexpr int FD_RING = 3;
constexpr int FD_DMA = 7;                      // copies per sub-page: K 2 + 1 partial, V 4
constexpr int FD_ROW = 132;                    // partial row: m, l, 2 pad, O[128] (floats)
static_assert(FD_KROWS == 2 * 1024 + 128 && FD_KREG == 2 * 1024 + 9 * 16, "K: two full copies, 8 or 9 lanes");

struct FlatParams {
    const void *q;
    int64_t q_ts, q_hs;
    const uint8_t *k;       // AoS Q8_0 rows, [B * Hkv * Skv][136]
    const uint8_t *v;       // fp16 rows, [B * Hkv * Skv][256 B]
    const int32_t *kv_len;  // [B]: keys each batch row sees (clamped to [0, Skv])
    const int32_t *q_abs;   // [B] or nullptr: row j sees keys <= q_abs[b] + j
    int B, Hkv, G, Sq, Skv, P, nsp;
    float c;                // scale * log2 e
    float *out;             // fp32 [B * Sq][Hq][128]
    int64_t o_ts, o_hs;
    float *ws;              // partials [segment][piece][Sq * G rows][FD_ROW]
};

__device__ __forceinline__ uint32_t lds32(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }

template <int QDT>
__global__ __launch_bounds__(64) void flat_decode_kernel(FlatParams p) {
    __shared__ __attribute__((aligned(16))) uint8_t ring[FD_RING * FD_SLOT];
    const int lane = threadIdx.x, i16 = lane & 15, g = lane >> 4;
    const int seg = blockIdx.x / p.P, pc = blockIdx.x - seg * p.P;
    const int b = seg / p.Hkv, h = seg - b * p.Hkv;
    const int kvl = min(max(p.kv_len[b], 0), p.Skv);
    const int s0 = (int)((int64_t)pc * p.nsp / p.P);
    const int s1 = min((int)((int64_t)(pc + 1) * p.nsp / p.P), (kvl + 15) >> 4);
    const int n = max(s1 - s0, 0);
    const int nrows = p.Sq * p.G;
    // the lane's query row i16 (token i16 / G, q-head h * G + i16 % G)
    half8_t qf[4];
    int lim = INT32_MAX;
    const int jr = i16 / p.G;
    const int hq = h * p.G + (i16 - jr * p.G);
    if (i16 < nrows) {
        const int64_t qoff = (int64_t)(b * p.Sq + jr) * p.q_ts + (int64_t)hq * p.q_hs + 8 * g;
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) qf[bb] = load_q8<QDT>(p.q, qoff + 32 * bb);
        lim = p.q_abs ? min(kvl - 1, p.q_abs[b] + jr) : kvl - 1;
    } else {
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) qf[bb] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
    }
    int lim_min;
    {
        const float f = (float)min(lim, 1 << 24);
        lim_min = __builtin_amdgcn_readfirstlane((int)(-row16_max(xrow_max(-f))));
    }
    float4_t o[8];
#pragma unroll
    for (int mm = 0; mm < 8; ++mm) o[mm] = float4_t{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;
    const float c = p.c;
    const int64_t rows0 = (int64_t)seg * p.Skv;  // the segment's first row
    const uint8_t *kseg = p.k + rows0 * 136;
    const uint8_t *vseg = p.v + rows0 * 256;
    const int koff = (int)(rows0 & 1) * 8;       // kseg is 8 bytes past a 16-byte boundary for odd rows0
    const int last_sp = p.nsp - 1;               // the segment's last sub-page (guarded loads)
    const uint32_t ring_lds =
        __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)ring);

    // sub-page j of the piece into slot sl (K rows at koff, V rows at
    // FD_KREG): FD_DMA copies, or for the segment's last sub-page guarded
    // dword loads stored to LDS, after which every earlier copy has landed
    // too (loads complete in order)
    auto fetch = [&](int j, int sl) __attribute__((always_inline)) {
        if (j >= n) return;  // uniform
        const int sp = s0 + j, tok0 = 16 * sp;
        const uint32_t dk = ring_lds + sl * FD_SLOT, dv = dk + FD_KREG;
        if (sp != last_sp) {  // uniform: 16 rows, and the 16-byte runs copied stay inside the segment
            const uint8_t *kb = kseg + (int64_t)tok0 * 136 - koff + 16 * lane;
            const uint8_t *vb = vseg + (int64_t)tok0 * 256 + 16 * lane;
            lds_dma16<true>(kb, dk);
            lds_dma16<true>(kb + 1024, dk + 1024);
            lds_dma16<true>(vb, dv);
            lds_dma16<true>(vb + 1024, dv + 1024);
            lds_dma16<true>(vb + 2048, dv + 2048);
            lds_dma16<true>(vb + 3072, dv + 3072);
            if (16 * lane < FD_KROWS + koff - 2048) lds_dma16<true>(kb + 2048, dk + 2048);
        } else {
            const int nt = min(p.Skv - tok0, 16);  // valid rows
            const uint32_t *ksrc = reinterpret_cast<const uint32_t *>(kseg + (int64_t)tok0 * 136);
            const uint32_t *vsrc = reinterpret_cast<const uint32_t *>(vseg + (int64_t)tok0 * 256);
            uint32_t *kd = reinterpret_cast<uint32_t *>(ring + sl * FD_SLOT + koff);
            uint32_t *vd = reinterpret_cast<uint32_t *>(ring + sl * FD_SLOT + FD_KREG);
            for (int i = lane; i < FD_KROWS / 4; i += 64) kd[i] = i < nt * 34 ? ksrc[i] : 0u;
            for (int i = lane; i < 16 * 64; i += 64) vd[i] = i < nt * 64 ? vsrc[i] : 0u;
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        }
    };
    auto landed = [&](int j) __attribute__((always_inline)) {
        static_assert(FD_DMA * (FD_RING - 1) <= 63, "vmcnt immediate");
        if (j + FD_RING - 1 < n) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(FD_DMA * (FD_RING - 1)) : "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    };
    // one sub-page from slot sb (tokens tok0 .. tok0 + 15)
    auto attend = [&](const uint8_t *sb, int tok0) __attribute__((always_inline)) {
        half8_t ka[4];
        const uint8_t *krow = sb + koff + i16 * 136;
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
            const uint8_t *blk = krow + 34 * bb;  // 4-byte aligned for even bb, else 2 past
            uint32_t w0, w1, dsc;
            if ((bb & 1) == 0) {  // ints at blk + 2 + 8g: 2 bytes past a dword
                const uint32_t d0 = lds32(blk + 8 * g), d1 = lds32(blk + 8 * g + 4), d2 = lds32(blk + 8 * g + 8);
                w0 = __builtin_amdgcn_alignbyte(d1, d0, 2);
                w1 = __builtin_amdgcn_alignbyte(d2, d1, 2);
                dsc = lds32(blk) & 0xFFFFu;
            } else {              // ints at blk + 2 + 8g: dword aligned
                w0 = lds32(blk + 2 + 8 * g);
                w1 = lds32(blk + 6 + 8 * g);
                dsc = lds32(blk - 2) >> 16;
            }
            const half_t d = __builtin_bit_cast(half_t, (uint16_t)dsc);
            const half8_t dd = {d, d, d, d, d, d, d, d};
            ka[bb] = i8x8_to_half8(w0, w1) * dd;
        }
        float4_t sacc = mfma16(ka[0], qf[0], float4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int bb = 1; bb < 4; ++bb) sacc = mfma16(ka[bb], qf[bb], sacc);
        float sv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = sacc[i];  // token tok0 + 4g + i
        if (!(tok0 + 16 <= kvl && tok0 + 15 <= lim_min)) {  // uniform
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = tok0 + 4 * g + i;
                sv[i] = (key < kvl && key <= lim) ? sv[i] : -INFINITY;
            }
        }
        // lane-local test first; the row's max (over lanes i16 + 16 g) only
        // when some lane may rescale
        const float ml = max4f(sv) * c;
        if (__builtin_amdgcn_ballot_w64(ml > m + LAZY_TAU)) {  // wave-uniform, rare after warm-up
            const float mt = xrow_max(ml);
            const bool need = mt > m + LAZY_TAU;
            const float mn = need ? mt : m;
            const float alpha = need ? __builtin_amdgcn_exp2f(m - mn) : 1.0f;
            m = mn;
            l *= alpha;
#pragma unroll
            for (int mm = 0; mm < 8; ++mm) o[mm] *= alpha;
        }
        const float nms = m == -INFINITY ? 0.0f : -m;
        float pr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) pr[i] = __builtin_amdgcn_exp2f(fmaf(sv[i], c, nms));
        l += (pr[0] + pr[1]) + (pr[2] + pr[3]);
        const half4_t pb = {(half_t)pr[0], (half_t)pr[1], (half_t)pr[2], (half_t)pr[3]};
        const uint16_t *vt = reinterpret_cast<const uint16_t *>(sb + FD_KREG) + (4 * g) * 128 + i16;
#pragma unroll
        for (int mm = 0; mm < 8; ++mm) {
            half4_t va;
#pragma unroll
            for (int e = 0; e < 4; ++e) va[e] = __builtin_bit_cast(half_t, vt[e * 128 + 16 * mm]);
            o[mm] = mfma16k16(va, pb, o[mm]);
        }
    };
#pragma unroll
    for (int u = 0; u < FD_RING - 1; ++u) fetch(u, u);
    for (int base = 0; base < n; base += FD_RING) {
#pragma unroll
        for (int u = 0; u < FD_RING; ++u) {
            const int j = base + u;
            if (j < n) {  // uniform
                // the previous step's reads of the slot refilled next have completed
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                fetch(j + FD_RING - 1, (u + FD_RING - 1) % FD_RING);
                landed(j);
                attend(ring + u * FD_SLOT, 16 * (s0 + j));
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    l = xrow_sum(l);
    if (i16 >= nrows) return;
    if (p.P == 1) {  // the whole segment: normalized output
        const float inv = l > 0.f ? 1.0f / l : 0.0f;
        float *ob = p.out + (int64_t)(b * p.Sq + jr) * p.o_ts + (int64_t)hq * p.o_hs + 4 * g;
#pragma unroll
        for (int mm = 0; mm < 8; ++mm) *reinterpret_cast<float4_t *>(ob + 16 * mm) = o[mm] * inv;
    } else {
        float *row = p.ws + (((int64_t)seg * p.P + pc) * nrows + i16) * FD_ROW;
        if (g == 0) *reinterpret_cast<float2_t *>(row) = float2_t{m, l};
#pragma unroll
        for (int mm = 0; mm < 8; ++mm) *reinterpret_cast<float4_t *>(row + 4 + 16 * mm + 4 * g) = o[mm];
    }
}

// Merges the P pieces of each (segment, row): grid (B * Hkv, Sq * G, FC_DS),
// 1024 threads; workgroup z takes 128 / FC_DS of the d.  Thread t owns the
// 4-d chunk t % FC_DCH of them and pieces t / FC_DCH + FC_GROUPS k (one-pass
// online merge, eight pieces' loads in flight: 8 FC_GROUPS pieces per round
// trip); the FC_GROUPS partial states per chunk then merge in a tree through
// LDS.  (A segment is often cut into hundreds of pieces for few rows, so the
// merge is latency-bound: with 256 threads and four loads in flight, 512
// pieces took 14 us; one 1024-thread workgroup per row, 7.7 us under the
// kernel tracer.  The quarter split takes a B = 1, 8/4, 128K-key forward
// from 44.2 to 42.0 us.)
#ifndef GFA_FC_DS
#define GFA_FC_DS 4
#endif
constexpr int FC_THREADS = 1024, FC_DS = GFA_FC_DS, FC_DCH = 32 / FC_DS, FC_GROUPS = FC_THREADS / FC_DCH, FC_U = 8;
__global__ __launch_bounds__(FC_THREADS) void flat_combine_kernel(FlatParams p) {
    __shared__ float sm_m[FC_GROUPS], sm_l[FC_GROUPS];
    __shared__ float4_t sm_o[FC_GROUPS][FC_DCH];
    const int seg = blockIdx.x, r = blockIdx.y;
    const int nrows = p.Sq * p.G;
    const int t = threadIdx.x, grp = t / FC_DCH, dc = t % FC_DCH, d0 = 4 * (blockIdx.z * FC_DCH + dc);
    float M = -INFINITY, L = 0.f;
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
    const float *base = p.ws + ((int64_t)seg * p.P * nrows + r) * FD_ROW;
    const int64_t pstep = (int64_t)nrows * FD_ROW;  // piece k -> k + 1
    for (int k0 = grp; k0 < p.P; k0 += FC_GROUPS * FC_U) {
        float2_t ml[FC_U];
        float4_t oc[FC_U];
#pragma unroll
        for (int u = 0; u < FC_U; ++u) {
            const int k = k0 + FC_GROUPS * u;
            const float *row = base + k * pstep;
            ml[u] = k < p.P ? *reinterpret_cast<const float2_t *>(row) : float2_t{-INFINITY, 0.f};
            oc[u] = k < p.P ? *reinterpret_cast<const float4_t *>(row + 4 + d0) : float4_t{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < FC_U; ++u) {
            const float mc = ml[u][0];
            if (mc > -INFINITY) {
                const float mn = fmaxf(M, mc);
                const float a = __builtin_amdgcn_exp2f(M - mn);  // 0 while M is -inf
                const float bw = __builtin_amdgcn_exp2f(mc - mn);
                L = fmaf(L, a, bw * ml[u][1]);
                acc = acc * a + bw * oc[u];
                M = mn;
            }
        }
    }
    // tree merge of the groups' states through LDS
#pragma unroll
    for (int half = FC_GROUPS / 2; half >= 1; half >>= 1) {
        if (grp >= half && grp < 2 * half) {
            if (dc == 0) {
                sm_m[grp] = M;
                sm_l[grp] = L;
            }
            sm_o[grp][dc] = acc;
        }
        __syncthreads();
        if (grp < half) {
            const float m2 = sm_m[grp + half];
            const float mn = fmaxf(M, m2);
            const float a = mn == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - mn);
            const float b = mn == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m2 - mn);
            L = fmaf(L, a, sm_l[grp + half] * b);
            acc = acc * a + sm_o[grp + half][dc] * b;
            M = mn;
        }
        __syncthreads();
    }
    if (grp != 0) return;
    const int b = seg / p.Hkv, h = seg - b * p.Hkv;
    const int j = r / p.G, hq = h * p.G + (r - j * p.G);
    const float inv = L > 0.f ? 1.0f / L : 0.0f;
    *reinterpret_cast<float4_t *>(p.out + (int64_t)(b * p.Sq + j) * p.o_ts + (int64_t)hq * p.o_hs + d0) = acc * inv;
}

// ---------------------------------------------------------------------------
// Host-side plan.  Deterministic in the call's scalar arguments and the
// device's CU count, so that workspace_size() and the launch agree.
//
// Decode work is split by packed rows per sequence into classes, each with
// its own stream-K plan, workspace region and combine: n_q*G <= 16 runs the
// one-row-group kernel (three waves per SIMD), 16 < n_q*G <= 32 the
// two-row-group kernel (speculative verify), and up to 64 rows its chunked
// instantiation (32 rows per pass, 64-row partial slots; only when the
// batch's max_query_len * G exceeds 32).  A batch whose sequences all have
// max_query_len tokens (num_tokens == num_seqs * max_query_len) needs at
// most one class, and a uniform prefill batch none; a class launched alone
// takes every row count up to its bound.  Sequences above the largest bound
// go to the prefill kernel, which handles any row count.
struct DecClass {
    int nrg;            // row groups per decode wave (1, 2 or 3)
    int rows_lo, rows_hi;
    int nwg;            // decode workgroups (resident workgroups of the device)
    size_t off_hdr, off_pre, off_ml, off_o;  // workspace layout
};

#ifndef GFA_COMB_FEW
#define GFA_COMB_FEW 8          // resident decode workgroups per segment, at most
#endif
#ifndef GFA_DEC_ROWS48_UNITS
#define GFA_DEC_ROWS48_UNITS 8  // sub-pages per decode workgroup from which 33-48 rows take 48-row tiles
#endif
#ifndef GFA_COMB_SEGS
#define GFA_COMB_SEGS 64        // segments from which a mixed batch's verify class merges per segment
#endif
#ifndef GFA_COMB_FEW_KEYS
#define GFA_COMB_FEW_KEYS 1024  // longest context for the per-segment merge
#endif
#ifndef GFA_PF_KS2_MAX_ROWS
#define GFA_PF_KS2_MAX_ROWS 128  // most rows per kv-head for which 128-row (KS = 2) prefill tiles are chosen
#endif
struct Plan {
    DecClass dc[3];
    int ndc;            // decode classes launched (0..3)
    int dec_rows_max;   // largest decode row bound (0: every sequence is prefill)
    bool need_prefill;
    int pf_rows;        // rows per prefill row tile: PF_ROWS (KS = 1) or PF_ROWS / 2 (KS = 2)
    int pf_items_max;   // bound on prefill row tiles (0: no work list)
    int pf_split_max;   // split row tiles, at most
    int pf_slots_max;   // partial slots per kv head
    int pf_grid_items;  // work-list capacity: the prefill grid over Hkv
    size_t off_items, off_split, off_pml, off_po, off_tbase;
    size_t bytes;       // the regions a call needs; the tile images follow at `bytes`
    size_t img_bytes;   // room the tile images of the call's shape can take (capped)
    bool comb_short;    // contexts of at most GFA_COMB_FEW_KEYS keys (combine choice)
};

// Workspace room for the prefill tile images, at most (bytes).  A call whose
// images do not fit the workspace it is given dequantizes in the prefill
// workgroups instead.
#ifndef GFA_PF_IMG_CAP_MB
#define GFA_PF_IMG_CAP_MB 1024
#endif
constexpr size_t PF_IMG_CAP = (size_t)GFA_PF_IMG_CAP_MB << 20;

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Splits the softmax scale c between Q and K^ for the prefill kernel:
// Q * 2^-e (exact) and K^ * (c * 2^e), with e chosen so that c * 2^e is in
// [0.5, 1): K^ = fp16(q * d_k * kmul) stays at or below the dequantized key
// q * d_k, so it is finite wherever the decode kernel's fp16(q * d_k) is
// (a kmul up to 2 would overflow keys above 65504 / kmul, 32.8K at worst).
void set_prefill_scale(AttnParams &p) {
    int e = 0;
    (void)frexpf(p.scale_log2e, &e);  // c = m * 2^e, m in [0.5, 1)
    e = max(-60, min(60, -e));
    p.pf_qmul = ldexpf(1.0f, -e);
    p.pf_kmul = ldexpf(p.scale_log2e, e);
}

// CUs of the current device, queried once per device.  Threads may race on
// the first query of a device; they store the same value, and the relaxed
// atomics make that race well defined.  256 (MI355X) when no device is
// visible, so plans and workspace sizes computed on a host without a GPU
// match the target part.
int device_cus() {
    static std::atomic<int> cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

void plan_add_class(Plan &pl, int nrg, int lo, int hi) {
    DecClass &c = pl.dc[pl.ndc++];
    c.nrg = nrg;
    c.rows_lo = lo;
    c.rows_hi = hi;
    c.nwg = device_cus() * 4 * (nrg == 1 ? DecCfg<1>::wpe : DecCfg<2>::wpe) / DEC_NW;
}

// Prefill work-list bounds and the workspace layout, once the decode classes
// are chosen.  Every region grows monotonically with num_seqs, num_tokens and
// the classes' row bounds (the workspace bound below relies on it).
// pf_seqs: the sequences the row-tile count assumes; force_pf: lay out the
// work list even where a call would keep the 2-D prefill grid (bound only).
// allow_split: reserve the partial slots of row tiles split over the keys
// (without them the plan kernel leaves every row tile whole).
// max_seq_len < 0: unknown (the image room is then the cap).
void plan_finish(Plan &pl, int num_seqs, int64_t num_tokens, int G, int num_kv_heads, bool force_pf,
                 bool allow_split, int64_t max_seq_len, int64_t max_query_len) {
    pl.dec_rows_max = pl.ndc ? pl.dc[pl.ndc - 1].rows_hi : 0;
    // row tiles over all sequences <= sum ceil(n_q * G / R) <= T*G/R + B (R = pf_rows)
    const int pf_seqs = min(num_seqs, PL_MAX_SEQS);
    const int64_t items = (max(num_tokens, (int64_t)0) * G + pl.pf_rows - 1) / pl.pf_rows + pf_seqs;
    // a split row tile holds more than pf_ncu / Hkv of the launch's key tiles:
    // fewer than ceil(CUs / Hkv) of them, with fewer than twice that many pieces
    // (a few row tiles, n <= 2 ceil(CUs / Hkv), may instead be cut into up to
    // three rounds of workgroups: <= 3 ceil(CUs / Hkv) pieces in all)
    const int64_t split = (device_cus() + num_kv_heads - 1) / num_kv_heads;
    const bool pf = force_pf || (pl.need_prefill && num_seqs <= PL_MAX_SEQS &&
                                 (items + 3 * split) * num_kv_heads < INT32_MAX);
    const int64_t grid_items = pf ? max(items + split, 3 * split) : 0;
    pl.pf_items_max = pf ? (int)min(items, (int64_t)INT32_MAX) : 0;
    pl.pf_split_max = pf && allow_split ? (int)(2 * split) : 0;
    pl.pf_slots_max = pf && allow_split ? (int)(3 * split) : 0;
    pl.pf_grid_items = (int)min(grid_items, (int64_t)INT32_MAX);
    size_t off = 0;
    for (int k = 0; k < pl.ndc; ++k) {
        DecClass &c = pl.dc[k];
        const size_t rc = (size_t)c.rows_hi;  // rows per partial slot
        c.off_hdr = off;
        c.off_pre = off + 256;
        c.off_ml = c.off_pre + align256((size_t)num_seqs * sizeof(int));
        c.off_o = c.off_ml + align256((size_t)2 * c.nwg * rc * 2 * sizeof(float));
        off = c.off_o + align256((size_t)2 * c.nwg * rc * 128 * sizeof(float));
    }
    pl.off_items = off;
    // work list: a 256-byte header (item count, split row tile count), the
    // five item arrays, the split list, then the partials of the split pieces
    // (slots of the call's tile rows)
    pl.off_split = pl.off_items + 256 + align256((size_t)5 * grid_items * sizeof(int));
    // partial slots of the call's tile rows (a bound over every call: PF_ROWS)
    const size_t prow = (size_t)pl.pf_slots_max * num_kv_heads * (force_pf ? PF_ROWS : pl.pf_rows);
    pl.off_pml = pl.off_split + align256((size_t)4 * pl.pf_split_max * sizeof(int));
    pl.off_po = pl.off_pml + align256(prow * 2 * sizeof(float));
    // the per-sequence first image tile, then (optional) the images: every
    // prefill sequence (n_q * G above the largest decode bound) at
    // max_seq_len keys
    pl.off_tbase = pl.off_po + align256(prow * 128 * sizeof(float));
    pl.bytes = max(pl.off_tbase + (pf ? align256((size_t)(num_seqs + 1) * sizeof(int)) : 0), (size_t)256);
    // (no image room where no sequence can have PF_IMG_REUSE row tiles: the
    // launch then never writes images, see the call's image pointer)
    pl.img_bytes = 0;
    if (pf && (max(max_query_len, (int64_t)0) * G + PF_ROWS - 1) / PF_ROWS >= PF_IMG_REUSE) {
        const int64_t nq_min = pl.dec_rows_max / max(G, 1) + 1;  // a prefill sequence's query tokens, at least
        const int64_t npf = max((int64_t)1, min((int64_t)num_seqs, max(num_tokens, (int64_t)0) / nq_min));
        const double want = max_seq_len < 0 ? (double)PF_IMG_CAP
                                            : (double)npf * (double)((max_seq_len + PF_TK - 1) / PF_TK) *
                                                  num_kv_heads * PF_IMG_BYTES;
        pl.img_bytes = want >= (double)PF_IMG_CAP ? PF_IMG_CAP : align256((size_t)want);
    }
}

Plan make_plan(int num_seqs, int num_tokens, int num_heads, int num_kv_heads, int max_query_len,
               int64_t max_seq_len, bool allow_split = true) {
    Plan pl{};
    const int G = num_heads / num_kv_heads;
    const int max_rows = max_query_len * G;
    const bool uniform = (int64_t)num_tokens == (int64_t)num_seqs * max_query_len;
    pl.ndc = 0;
    // tiles of 16, 32 or 48 rows per wave (one, two or three row groups);
    // up to DEC_CHUNK_ROWS rows the two-row-group class takes in 32-row
    // chunks.  A 48-row tile streams each sub-page once for all its rows
    // and dequantizes it once; two 32-row chunks stream and dequantize it
    // twice (6/1 heads, 8 x (131072 + 6): 69.5 against 88.5 us).
    // Below about 8 sub-pages per workgroup (short contexts, few segments)
    // the 48-row tile's fixed costs (a two-pass merge, spilled registers)
    // outweigh the second chunk it saves: 8 x (2000 + 6) at 6/1 measured
    // 21.1 against 19.7 us, 32 x (1000 + 6) at 48/8 39.8 against 41.5 us.
    const int64_t units_est = (int64_t)num_seqs * num_kv_heads * ((max(max_seq_len, (int64_t)1) + 15) / 16);
    const bool rows48 = max_rows > 32 && max_rows <= 48 &&
                        units_est >= (int64_t)GFA_DEC_ROWS48_UNITS * device_cus() * 4 * DecCfg<2>::wpe / DEC_NW;
    const int hi2 = max_rows <= 32 ? 32 : DEC_CHUNK_ROWS;
    if (max_rows <= 16) {
        plan_add_class(pl, 1, 0, 16);
    } else if (uniform) {
        if (rows48) plan_add_class(pl, 3, 0, 48);
        else if (max_rows <= DEC_CHUNK_ROWS) plan_add_class(pl, 2, 0, hi2);
    } else {
        // mixed row counts: each sequence takes the smallest tile that
        // holds its rows (one launch pair per class)
        if (G <= 16) plan_add_class(pl, 1, 0, 16);
        if (rows48) {
            if (G <= 32) plan_add_class(pl, 2, pl.ndc ? 16 : 0, 32);
            plan_add_class(pl, 3, pl.ndc ? pl.dc[pl.ndc - 1].rows_hi : 0, 48);
        } else if (G <= DEC_CHUNK_ROWS) {
            plan_add_class(pl, 2, pl.ndc ? 16 : 0, hi2);
        }
    }
    pl.need_prefill = max_rows > (pl.ndc ? pl.dc[pl.ndc - 1].rows_hi : 0);
    // Prefill tile rows: 128-row key-interleaved (KS = 2) tiles when the
    // longest prefill sequence has at most 128 rows per kv-head.  There a
    // 256-row tile fills at most half its consumer waves and costs about as
    // much per key tile as a full one.  Measured on one box (48/8, fp16 out):
    // 8 x (32768 + 12) 201 -> 193 us, 32 x (4096 + 12) 104.6 -> 98.2 us,
    // 8 x (32768 + 16) at 64/8 222 -> 216 us.  With more rows the extra row
    // tiles cost more than the padding they save: 1 x (65536 + 50) (300
    // rows, three 128-row tiles against two of 256) 148.5 -> 152.7 us,
    // 1 x (131072 + 64) (384 rows) 261 -> 275 us.
    pl.pf_rows = max_rows <= GFA_PF_KS2_MAX_ROWS ? PF_ROWS / 2 : PF_ROWS;
    plan_finish(pl, num_seqs, num_tokens, G, num_kv_heads, false, allow_split, max_seq_len, max_query_len);
    pl.comb_short = max_seq_len <= GFA_COMB_FEW_KEYS;
    return pl;
}

// A plan whose every workspace region is at least that of any make_plan()
// call with num_seqs <= max_num_seqs and num_tokens <= max_num_tokens (any
// max_query_len, any mix of decode and prefill sequences): each decode class
// a call can have, at its largest row bound (16 rows; 48 for the three-row-
// group class; 64 for the two-row-group class, which also covers a call's
// 32-row class), and a prefill work list sized for max_num_tokens.
// plan_finish's regions are monotone in all of these, and the decode
// regions a call lays out sum to at most those laid out here.
Plan bound_plan(int max_num_seqs, int64_t max_num_tokens, int num_heads, int num_kv_heads, bool allow_split,
                int64_t max_seq_len = -1) {
    Plan pl{};
    const int G = num_heads / num_kv_heads;
    pl.ndc = 0;
    if (G <= 16) plan_add_class(pl, 1, 0, 16);
    if (G <= 48) plan_add_class(pl, 3, pl.ndc ? 16 : 0, 48);
    if (G <= DEC_CHUNK_ROWS) plan_add_class(pl, 2, pl.ndc ? pl.dc[pl.ndc - 1].rows_hi : 0, DEC_CHUNK_ROWS);
    pl.need_prefill = true;
    pl.pf_rows = PF_ROWS / 2;  // the smaller tile: the most row tiles
    plan_finish(pl, max_num_seqs, max_num_tokens, G, num_kv_heads, true, allow_split, max_seq_len, max_num_tokens);
    return pl;
}

template <int QDT, int ODT>
hipError_t launch_all(const AttnParams &p0, const Plan &pl, char *ws, int num_seqs, int num_kv_heads,
                      int max_query_len, hipStream_t stream) {
    AttnParams p = p0;
    p.dec_rows_lo = 0;
    p.dec_rows_max = pl.dec_rows_max;
    if (pl.need_prefill && p.pf_seq) {
        // one wave for small batches: its scans and reductions need no
        // barriers across 16 waves (8 x (32768 + 12) at 48/8: 18.6 us with
        // 1024 threads)
        if (num_seqs <= 64 && pl.pf_items_max <= 64) prefill_plan_kernel<64><<<1, 64, 0, stream>>>(p);
        else prefill_plan_kernel<PL_THREADS><<<1, PL_THREADS, 0, stream>>>(p);
    }
    for (int k = 0; k < pl.ndc; ++k) {
        const DecClass &c = pl.dc[k];
        AttnParams pd = p;
        pd.dec_rows_lo = c.rows_lo;
        pd.dec_rows_max = c.rows_hi;
        pd.nwg = c.nwg;
        pd.ws_hdr = reinterpret_cast<int64_t *>(ws + c.off_hdr);
        pd.ws_pre = reinterpret_cast<int *>(ws + c.off_pre);
        pd.ws_ml = reinterpret_cast<float *>(ws + c.off_ml);
        pd.ws_o = reinterpret_cast<float *>(ws + c.off_o);
        // combine rows: a split segment has at most min(max_query_len * G, slot) rows
        const int crow = max(1, min(max_query_len * p.G, c.rows_hi));
        if (c.nrg == 1) {
            attn_decode_kernel<1, QDT, ODT><<<c.nwg, 64 * DEC_NW, 0, stream>>>(pd);
            // short contexts with few pieces per segment at most (resident
            // workgroups over segments): one merging workgroup per segment.
            // There the merge launch is mostly workgroups that find their
            // segment whole (32 x 32 keys, 48/8: 6.7 against 7.9 us per
            // call); with long contexts the per-row launch measured faster.
            if (pl.comb_short && (int64_t)c.nwg <= (int64_t)GFA_COMB_FEW * num_seqs * num_kv_heads)
                attn_combine_few_kernel<ODT><<<dim3(num_seqs, num_kv_heads), 256, 0, stream>>>(pd);
            else
                attn_combine_kernel<1, ODT><<<dim3(num_seqs, num_kv_heads, crow), 256, 0, stream>>>(pd);
        } else if (c.nrg == 3) {
            attn_decode_kernel<3, QDT, ODT><<<c.nwg, 64 * DEC_NW, 0, stream>>>(pd);
            attn_combine_kernel<3, ODT><<<dim3(num_seqs, num_kv_heads, crow), 256, 0, stream>>>(pd);
        } else {
            if (c.rows_hi > 32) attn_decode_kernel<2, QDT, ODT, true><<<c.nwg, 64 * DEC_NW, 0, stream>>>(pd);
            else {  // one 8-wave workgroup where the plan sized two 4-wave ones
                constexpr int nw = dec_nw(2, false);
                pd.nwg = c.nwg * DEC_NW / nw;
                attn_decode_kernel<2, QDT, ODT><<<pd.nwg, 64 * nw, 0, stream>>>(pd);
            }
            if (c.rows_lo > 0 && (int64_t)num_seqs * num_kv_heads >= GFA_COMB_SEGS)
                attn_combine_few_kernel<ODT><<<dim3(num_seqs, num_kv_heads), 256, 0, stream>>>(pd);
            else
                attn_combine_kernel<2, ODT><<<dim3(num_seqs, num_kv_heads, crow), 256, 0, stream>>>(pd);
        }
    }
    if (pl.need_prefill) {
        // the tile images, after the decode launches (their write-back then
        // overlaps the MFMA-bound prefill, not the HBM-bound decode); returns
        // at once when the plan chose none
        if (p.pf_seq && p.pf_tiles) prefill_tiles_kernel<false><<<device_cus() * 4, 64 * PF_NSP, 0, stream>>>(p);
        const int rows = max_query_len * p.G;
        const int tiles = (rows + pl.pf_rows - 1) / pl.pf_rows;
        const dim3 grid = p.pf_seq ? dim3(pl.pf_grid_items * num_kv_heads) : dim3(tiles * num_kv_heads, num_seqs);
        if (pl.pf_rows == PF_ROWS) attn_prefill_kernel<QDT, ODT, false, false><<<grid, 64 * PF_WAVES, 0, stream>>>(p);
        else attn_prefill_kernel<QDT, ODT, false, false, 2><<<grid, 64 * PF_WAVES, 0, stream>>>(p);
        if (p.pf_seq && pl.pf_split_max)  // returns at once when the plan split nothing
            attn_prefill_combine_kernel<ODT><<<device_cus() * GFA_PFC_WGS_PER_CU, 256, 0, stream>>>(p);
    }
    return hipGetLastError();
}

}  // namespace

extern "C" size_t gfx906_fa_amd_paged_attention_workspace_size(int num_seqs, int num_tokens,
                                                               int num_heads, int num_kv_heads,
                                                               int head_size, int max_query_len,
                                                               int max_seq_len) {
    (void)head_size;
    if (num_seqs <= 0 || num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads) return 0;
    const Plan pl = make_plan(num_seqs, num_tokens, num_heads, num_kv_heads, max(max_query_len, 1), max(max_seq_len, 1));
    return pl.bytes + pl.img_bytes;
}

extern "C" size_t gfx906_fa_amd_paged_attention_workspace_bound(int max_num_seqs, int64_t max_num_tokens,
                                                                int num_heads, int num_kv_heads,
                                                                int head_size) {
    (void)head_size;
    if (max_num_seqs <= 0 || max_num_tokens < 0 || num_kv_heads <= 0 || num_heads <= 0 ||
        num_heads % num_kv_heads)
        return 0;
    const Plan pl = bound_plan(max_num_seqs, max_num_tokens, num_heads, num_kv_heads, true);
    return pl.bytes + pl.img_bytes;
}

extern "C" int gfx906_fa_amd_paged_attention_workspace_bound_info(int max_num_seqs, int64_t max_num_tokens,
                                                                  int num_heads, int num_kv_heads, int head_size,
                                                                  int64_t max_seq_len, int64_t *info, int info_len) {
    (void)head_size;
    if (info == nullptr || max_num_seqs <= 0 || max_num_tokens < 0 || num_kv_heads <= 0 || num_heads <= 0 ||
        num_heads % num_kv_heads)
        return -1;
    const Plan pl = bound_plan(max_num_seqs, max_num_tokens, num_heads, num_kv_heads, true,
                               max_seq_len > 0 ? max_seq_len : -1);
    const int64_t v[] = {(int64_t)pl.bytes, (int64_t)pl.img_bytes};
    const int n = (int)(sizeof(v) / sizeof(v[0]));
    for (int i = 0; i < n && i < info_len; ++i) info[i] = v[i];
    return n;
}

extern "C" int gfx906_fa_amd_device_cus(void) { return device_cus(); }

extern "C" int gfx906_fa_amd_paged_attention_plan_info(int num_seqs, int num_tokens, int num_heads,
                                                       int num_kv_heads, int head_size, int max_query_len,
                                                       int max_seq_len, int64_t *info, int info_len) {
    (void)head_size;
    if (info == nullptr || num_seqs <= 0 || num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads)
        return -1;
    const Plan pl = make_plan(num_seqs, num_tokens, num_heads, num_kv_heads, max(max_query_len, 1), max(max_seq_len, 1));
    const int64_t v[] = {(int64_t)(pl.bytes + pl.img_bytes), pl.ndc, pl.dec_rows_max, pl.need_prefill ? 1 : 0,
                         pl.pf_items_max, pl.pf_grid_items, pl.pf_split_max, pl.pf_slots_max,
                         pl.pf_items_max ? (int64_t)pl.off_items : -1, device_cus(), (int64_t)pl.bytes,
                         (int64_t)pl.img_bytes, pl.need_prefill ? pl.pf_rows : 0};
    const int n = (int)(sizeof(v) / sizeof(v[0]));
    for (int i = 0; i < n && i < info_len; ++i) info[i] = v[i];
    return n;
}

namespace {

// Scratch of gfx906_fa_amd_paged_attention_noalloc: the workspace of every
// call on a device, one copy per device (each device that runs this code
// object holds it until the process ends).  No initial contents are needed:
// each call writes what it reads.  In host code `scratch` names a host-side
// stand-in; its device address comes from hipGetSymbolAddress, once per
// device, with that device current.
static __device__ __align__(256) uint8_t scratch[GFX906_FA_AMD_SCRATCH_BYTES];

hipError_t scratch_address(void **out) {
    static std::atomic<void *> addr[64];
    static std::mutex mu;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    void *a = addr[dev].load(std::memory_order_acquire);
    if (a == nullptr) {
        std::lock_guard<std::mutex> lock(mu);
        a = addr[dev].load(std::memory_order_relaxed);
        if (a == nullptr) {
            e = hipGetSymbolAddress(&a, HIP_SYMBOL(scratch));
            if (e != hipSuccess || a == nullptr) {
                fprintf(stderr, "[gfx906_fa_amd] paged_attention_noalloc: hipGetSymbolAddress(scratch) failed (%d)\n",
                        (int)e);
                return e != hipSuccess ? e : hipErrorInvalidSymbol;
            }
            addr[dev].store(a, std::memory_order_release);
        }
    }
    *out = a;
    return hipSuccess;
}

}  // namespace

extern "C" hipError_t gfx906_fa_amd_noalloc_scratch_copy(void *dst, size_t offset, size_t bytes, hipStream_t stream) {
    if (dst == nullptr || offset > GFX906_FA_AMD_SCRATCH_BYTES || bytes > GFX906_FA_AMD_SCRATCH_BYTES - offset) {
        fprintf(stderr, "[gfx906_fa_amd] noalloc_scratch_copy: range past the %zu-byte scratch\n",
                (size_t)GFX906_FA_AMD_SCRATCH_BYTES);
        return hipErrorInvalidValue;
    }
    if (bytes == 0) return hipSuccess;
    void *a = nullptr;
    const hipError_t e = scratch_address(&a);
    if (e != hipSuccess) return e;
    return hipMemcpyAsync(dst, static_cast<char *>(a) + offset, bytes, hipMemcpyDeviceToDevice, stream);
}

namespace {

// The step's new K/V rows for the fused cache write (element strides).
struct NewKV {
    const void *key, *value;
    int dtype;
    int64_t kts, khs, vts, vhs;
    const int64_t *slot_mapping;
};

hipError_t paged_attention_impl(
    const void *q, int q_dtype, int64_t q_token_stride, int64_t q_head_stride,
    const uint8_t *k_cache, const uint8_t *v_cache, int64_t cache_block_stride,
    int64_t cache_head_stride, const int32_t *block_table, int64_t block_table_stride,
    const int32_t *seq_lens, const int32_t *query_start_loc, const int32_t *q_abs_offset,
    int causal, int num_seqs, int num_tokens, int num_heads, int num_kv_heads, int head_size,
    int block_size, int max_query_len, int max_seq_len, float scale, void *out, int out_dtype,
    int64_t out_token_stride, int64_t out_head_stride, void *workspace, size_t workspace_bytes,
    const NewKV *nkv, hipStream_t stream, bool noalloc = false) {
    if (nkv && num_tokens > 0) {
        const uint64_t align = nkv->dtype == GFA_DTYPE_F32 ? 8 : 4;  // two values per lane
        if (nkv->dtype != q_dtype ||
            (((uintptr_t)nkv->key | (uintptr_t)nkv->value) & (align - 1)) ||
            ((uint64_t)(nkv->kts | nkv->khs | nkv->vts | nkv->vhs) & 1u)) {
            fprintf(stderr,
                    "[gfx906_fa_amd] paged_attention_kv_write: new key/value must have the query dtype, "
                    "%d-byte aligned bases and even element strides\n", (int)align);
            return hipErrorInvalidValue;
        }
    }
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
    Plan pl = make_plan(num_seqs, num_tokens, num_heads, num_kv_heads, max(max_query_len, 1), max(max_seq_len, 1));
    if (noalloc) {
        // the library's scratch array instead of a caller workspace; a plan
        // whose split-prefill partials do not fit leaves row tiles unsplit
        if (pl.bytes > GFX906_FA_AMD_SCRATCH_BYTES)
            pl = make_plan(num_seqs, num_tokens, num_heads, num_kv_heads, max(max_query_len, 1),
                           max(max_seq_len, 1), false);
        if (pl.bytes > GFX906_FA_AMD_SCRATCH_BYTES) {
            fprintf(stderr,
                    "[gfx906_fa_amd] paged_attention_noalloc: this batch needs %zu bytes of scratch, more than "
                    "the library's %zu (use gfx906_fa_amd_paged_attention with a workspace)\n",
                    pl.bytes, (size_t)GFX906_FA_AMD_SCRATCH_BYTES);
            return hipErrorInvalidValue;
        }
        const hipError_t e = scratch_address(&workspace);
        if (e != hipSuccess) return e;
        workspace_bytes = GFX906_FA_AMD_SCRATCH_BYTES;
    }
    if (workspace == nullptr || workspace_bytes < pl.bytes || ((uintptr_t)workspace & 255u)) {
        fprintf(stderr, "[gfx906_fa_amd] paged_attention: workspace of %zu bytes (256-aligned) required, got %zu\n",
                pl.bytes, workspace_bytes);
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
    p.vcbs = cache_block_stride;
    p.vchs = cache_head_stride;
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
    set_prefill_scale(p);
    p.out = out;
    p.o_ts = out_token_stride;
    p.o_hs = out_head_stride;
    char *ws = static_cast<char *>(workspace);
    p.num_seqs = num_seqs;
    p.pf_rows = pl.pf_rows;
    p.pf_items_max = pl.pf_items_max;
    p.pf_grid_items = pl.pf_grid_items;
    p.pf_ncu = device_cus();
    p.pf_split_max = pl.pf_split_max;
    p.pf_slots_max = pl.pf_slots_max;
    const int ni = pl.pf_grid_items;
    p.pf_count = pl.pf_items_max ? reinterpret_cast<int *>(ws + pl.off_items) : nullptr;
    p.pf_seq = pl.pf_items_max ? reinterpret_cast<int *>(ws + pl.off_items + 256) : nullptr;
    p.pf_rt = pl.pf_items_max ? p.pf_seq + ni : nullptr;
    p.pf_kt0 = pl.pf_items_max ? p.pf_seq + 2 * ni : nullptr;
    p.pf_kt1 = pl.pf_items_max ? p.pf_seq + 3 * ni : nullptr;
    p.pf_slot = pl.pf_items_max ? p.pf_seq + 4 * ni : nullptr;
    p.pf_split = pl.pf_items_max ? reinterpret_cast<int *>(ws + pl.off_split) : nullptr;
    p.pf_ml = pl.pf_items_max ? reinterpret_cast<float *>(ws + pl.off_pml) : nullptr;
    p.pf_o = pl.pf_items_max ? reinterpret_cast<float *>(ws + pl.off_po) : nullptr;
    // tile images: whatever room the workspace has past the call's regions.
    // None when no sequence can have PF_IMG_REUSE row tiles: the row tiles
    // then read each key tile fewer times than that on average (a sequence's
    // row tiles each read at most the key tiles of its last), so the plan
    // would decline them, and the pre-pass launch is skipped.
    p.pf_tbase = pl.pf_items_max ? reinterpret_cast<int *>(ws + pl.off_tbase) : nullptr;
    const size_t img_room = workspace_bytes > pl.bytes ? workspace_bytes - pl.bytes : 0;
    const bool img_reuse = pl.pf_rows == PF_ROWS && ((int64_t)max_query_len * G + PF_ROWS - 1) / PF_ROWS >= PF_IMG_REUSE;
    p.pf_tiles = (pl.pf_items_max && img_reuse && img_room >= (size_t)PF_IMG_BYTES)
                     ? reinterpret_cast<uint8_t *>(ws + pl.bytes)
                     : nullptr;
    p.pf_tiles_cap = p.pf_tiles ? (int64_t)img_room : 0;
    // decode workspace pointers are set per decode class in launch_all
    p.ws_hdr = nullptr;
    p.ws_pre = nullptr;
    p.ws_ml = nullptr;
    p.ws_o = nullptr;
    p.nwg = 0;
    p.new_k = p.new_v = nullptr;
    p.nk_ts = p.nk_hs = p.nv_ts = p.nv_hs = 0;
    p.new_slot = nullptr;
    if (nkv) {
        if (q_abs_offset == nullptr && !pl.need_prefill) {
            // every sequence is decode-shaped: its new tokens are the last n_q
            // positions, written by the decode wave that streams their sub-page
            p.new_k = nkv->key;
            p.new_v = nkv->value;
            p.nk_ts = nkv->kts;
            p.nk_hs = nkv->khs;
            p.nv_ts = nkv->vts;
            p.nv_hs = nkv->vhs;
            p.new_slot = nkv->slot_mapping;
        } else {
            // prefill rows read new tokens from many workgroups: write first
            const hipError_t e = gfx906_fa_amd_cache_write_kv(
                nkv->key, nkv->value, nkv->dtype, nkv->slot_mapping, const_cast<uint8_t *>(k_cache),
                const_cast<uint8_t *>(v_cache), num_tokens, num_kv_heads, head_size, block_size, nkv->kts,
                nkv->khs, nkv->vts, nkv->vhs, cache_block_stride, cache_head_stride, stream);
            if (e != hipSuccess) return e;
        }
    }

#define GFA_DISPATCH_O(QDT)                                                                    \
    switch (out_dtype) {                                                                       \
        case GFA_DTYPE_F32: return launch_all<QDT, GFA_DTYPE_F32>(p, pl, ws, num_seqs, num_kv_heads, max_query_len, stream); \
        case GFA_DTYPE_F16: return launch_all<QDT, GFA_DTYPE_F16>(p, pl, ws, num_seqs, num_kv_heads, max_query_len, stream); \
        default: return launch_all<QDT, GFA_DTYPE_BF16>(p, pl, ws, num_seqs, num_kv_heads, max_query_len, stream); \
    }
    switch (q_dtype) {
        case GFA_DTYPE_F32: GFA_DISPATCH_O(GFA_DTYPE_F32);
        case GFA_DTYPE_F16: GFA_DISPATCH_O(GFA_DTYPE_F16);
        default: GFA_DISPATCH_O(GFA_DTYPE_BF16);
    }
#undef GFA_DISPATCH_O
}

}  // namespace

extern "C" hipError_t gfx906_fa_amd_paged_attention(
    const void *q, int q_dtype, int64_t q_token_stride, int64_t q_head_stride,
    const uint8_t *k_cache, const uint8_t *v_cache, int64_t cache_block_stride,
    int64_t cache_head_stride, const int32_t *block_table, int64_t block_table_stride,
    const int32_t *seq_lens, const int32_t *query_start_loc, const int32_t *q_abs_offset,
    int causal, int num_seqs, int num_tokens, int num_heads, int num_kv_heads, int head_size,
    int block_size, int max_query_len, int max_seq_len, float scale, void *out, int out_dtype,
    int64_t out_token_stride, int64_t out_head_stride, void *workspace, size_t workspace_bytes,
    hipStream_t stream) {
    return paged_attention_impl(q, q_dtype, q_token_stride, q_head_stride, k_cache, v_cache,
                                cache_block_stride, cache_head_stride, block_table, block_table_stride,
                                seq_lens, query_start_loc, q_abs_offset, causal, num_seqs, num_tokens,
                                num_heads, num_kv_heads, head_size, block_size, max_query_len, max_seq_len,
                                scale, out, out_dtype, out_token_stride, out_head_stride, workspace,
                                workspace_bytes, nullptr, stream);
}

extern "C" hipError_t gfx906_fa_amd_paged_attention_noalloc(
    const void *q, int q_dtype, int64_t q_token_stride, int64_t q_head_stride,
    const uint8_t *k_cache, const uint8_t *v_cache, int64_t cache_block_stride,
    int64_t cache_head_stride, const int32_t *block_table, int64_t block_table_stride,
    const int32_t *seq_lens, const int32_t *query_start_loc, const int32_t *q_abs_offset,
    int causal, int num_seqs, int num_tokens, int num_heads, int num_kv_heads, int head_size,
    int block_size, int max_query_len, int max_seq_len, float scale, void *out, int out_dtype,
    int64_t out_token_stride, int64_t out_head_stride, hipStream_t stream) {
    return paged_attention_impl(q, q_dtype, q_token_stride, q_head_stride, k_cache, v_cache,
                                cache_block_stride, cache_head_stride, block_table, block_table_stride,
                                seq_lens, query_start_loc, q_abs_offset, causal, num_seqs, num_tokens,
                                num_heads, num_kv_heads, head_size, block_size, max_query_len, max_seq_len,
                                scale, out, out_dtype, out_token_stride, out_head_stride, nullptr, 0,
                                nullptr, stream, true);
}

extern "C" hipError_t gfx906_fa_amd_paged_attention_kv_write(
    const void *q, int q_dtype, int64_t q_token_stride, int64_t q_head_stride,
    const uint8_t *k_cache, const uint8_t *v_cache, int64_t cache_block_stride,
    int64_t cache_head_stride, const int32_t *block_table, int64_t block_table_stride,
    const int32_t *seq_lens, const int32_t *query_start_loc, const int32_t *q_abs_offset,
    int causal, int num_seqs, int num_tokens, int num_heads, int num_kv_heads, int head_size,
    int block_size, int max_query_len, int max_seq_len, float scale, void *out, int out_dtype,
    int64_t out_token_stride, int64_t out_head_stride, void *workspace, size_t workspace_bytes,
    const void *key, const void *value, int kv_dtype, int64_t key_token_stride,
    int64_t key_head_stride, int64_t value_token_stride, int64_t value_head_stride,
    const int64_t *slot_mapping, hipStream_t stream) {
    if (key == nullptr || value == nullptr || slot_mapping == nullptr) {
        fprintf(stderr, "[gfx906_fa_amd] paged_attention_kv_write: key, value and slot_mapping are required\n");
        return hipErrorInvalidValue;
    }
    const NewKV nkv{key, value, kv_dtype, key_token_stride, key_head_stride, value_token_stride,
                    value_head_stride, slot_mapping};
    return paged_attention_impl(q, q_dtype, q_token_stride, q_head_stride, k_cache, v_cache,
                                cache_block_stride, cache_head_stride, block_table, block_table_stride,
                                seq_lens, query_start_loc, q_abs_offset, causal, num_seqs, num_tokens,
                                num_heads, num_kv_heads, head_size, block_size, max_query_len, max_seq_len,
                                scale, out, out_dtype, out_token_stride, out_head_stride, workspace,
                                workspace_bytes, &nkv, stream);
}

namespace {

// Pieces per segment of the contiguous decode: enough single-wave
// workgroups to fill the device (8 per CU), each at least FD_MIN_SUB
// sub-pages (its fixed costs - Q load, ring fill, partial write - stay
// small against its stream).
#ifndef GFA_FD_MIN_SUB
#define GFA_FD_MIN_SUB 8
#endif
int flat_pieces(int nseg, int nsp) {
    const int64_t target = (int64_t)device_cus() * 8;
    const int64_t want = (target + nseg - 1) / max(nseg, 1);
    const int64_t most = max(nsp / GFA_FD_MIN_SUB, 1);
    return (int)max((int64_t)1, min(want, most));
}

}  // namespace

extern "C" size_t gfx906_fa_amd_flat_decode_workspace_size(int batch, int seq_q, int num_heads, int num_kv_heads,
                                                          int seq_kv) {
    if (batch <= 0 || seq_q <= 0 || num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads || seq_kv <= 0)
        return 256;
    const int nseg = batch * num_kv_heads, nsp = (seq_kv + 15) / 16;
    const int P = flat_pieces(nseg, nsp);
    const size_t rows = (size_t)seq_q * (num_heads / num_kv_heads);
    return P > 1 ? align256((size_t)nseg * P * rows * FD_ROW * sizeof(float)) : 256;
}

extern "C" hipError_t gfx906_fa_amd_flat_decode(
    const void *q, int q_dtype, int64_t q_token_stride, int64_t q_head_stride, const uint8_t *k_q8,
    const void *v_f16, const int32_t *kv_len, const int32_t *q_abs_offset, int batch, int seq_q, int num_heads,
    int num_kv_heads, int seq_kv, int head_size, float scale, float *out, int64_t out_token_stride,
    int64_t out_head_stride, void *workspace, size_t workspace_bytes, hipStream_t stream) {
    if (batch == 0 || seq_q == 0 || seq_kv == 0) return hipSuccess;
    const int G = (num_kv_heads > 0 && num_heads > 0) ? num_heads / num_kv_heads : 0;
    if (head_size != 128 || G <= 0 || num_heads % num_kv_heads || batch < 0 || seq_q < 0 || seq_kv < 0 ||
        (int64_t)seq_q * G > 16 || q_dtype < 0 || q_dtype > 2 || kv_len == nullptr) {
        fprintf(stderr, "[gfx906_fa_amd] flat_decode: unsupported configuration (head_size=%d heads=%d/%d seq_q=%d: "
                        "seq_q * heads/kv_heads must be <= 16; kv_len required)\n",
                head_size, num_heads, num_kv_heads, seq_q);
        return hipErrorInvalidValue;
    }
    if (((uintptr_t)k_q8 | (uintptr_t)v_f16) & 15u) {
        fprintf(stderr, "[gfx906_fa_amd] flat_decode: K and V bases must be 16-byte aligned\n");
        return hipErrorInvalidValue;
    }
    const size_t need = gfx906_fa_amd_flat_decode_workspace_size(batch, seq_q, num_heads, num_kv_heads, seq_kv);
    const int nseg = batch * num_kv_heads, nsp = (seq_kv + 15) / 16;
    const int P = flat_pieces(nseg, nsp);
    if (P > 1 && (workspace == nullptr || workspace_bytes < need || ((uintptr_t)workspace & 15u))) {
        fprintf(stderr, "[gfx906_fa_amd] flat_decode: workspace of %zu bytes required, got %zu\n", need,
                workspace_bytes);
        return hipErrorInvalidValue;
    }
    FlatParams p;
    p.q = q;
    p.q_ts = q_token_stride;
    p.q_hs = q_head_stride;
    p.k = k_q8;
    p.v = static_cast<const uint8_t *>(v_f16);
    p.kv_len = kv_len;
    p.q_abs = q_abs_offset;
    p.B = batch;
    p.Hkv = num_kv_heads;
    p.G = G;
    p.Sq = seq_q;
    p.Skv = seq_kv;
    p.P = P;
    p.nsp = nsp;
    p.c = scale * LOG2E;
    p.out = out;
    p.o_ts = out_token_stride;
    p.o_hs = out_head_stride;
    p.ws = static_cast<float *>(workspace);
    const int64_t grid = (int64_t)nseg * P;
    switch (q_dtype) {
        case GFA_DTYPE_F32: flat_decode_kernel<GFA_DTYPE_F32><<<(unsigned)grid, 64, 0, stream>>>(p); break;
        case GFA_DTYPE_F16: flat_decode_kernel<GFA_DTYPE_F16><<<(unsigned)grid, 64, 0, stream>>>(p); break;
        default: flat_decode_kernel<GFA_DTYPE_BF16><<<(unsigned)grid, 64, 0, stream>>>(p); break;
    }
    if (P > 1) flat_combine_kernel<<<dim3(nseg, seq_q * G, FC_DS), FC_THREADS, 0, stream>>>(p);
    return hipGetLastError();
}

extern "C" hipError_t gfx906_fa_amd_paged_attention_tiled(
    const void *q, int q_dtype, int64_t q_token_stride, int64_t q_head_stride,
    const uint8_t *k_cache, const void *v_cache, int v_format, int64_t k_block_stride,
    int64_t k_head_stride, int64_t v_block_stride, int64_t v_head_stride,
    const int32_t *block_table, int64_t block_table_stride, const int32_t *seq_lens,
    const int32_t *query_start_loc, const int32_t *q_abs_offset, int causal,
    const void *mask, int64_t mask_batch_stride, int64_t mask_row_stride, int mask_cols,
    int num_seqs, int num_tokens, int num_heads, int num_kv_heads, int head_size,
    int block_size, int max_query_len, float scale, float *out, int64_t out_token_stride,
    int64_t out_head_stride, hipStream_t stream) {
    if (num_seqs == 0 || num_tokens == 0) return hipSuccess;
    if (head_size != 128 || num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0 ||
        block_size <= 0 || block_size % 16 != 0 || q_dtype < 0 || q_dtype > 2 ||
        (v_format != 0 && v_format != 1) || max_query_len < 0 || (mask && mask_cols < 0)) {
        fprintf(stderr, "[gfx906_fa_amd] paged_attention_tiled: unsupported configuration "
                        "(head_size=%d heads=%d/%d block_size=%d v_format=%d)\n",
                head_size, num_heads, num_kv_heads, block_size, v_format);
        return hipErrorInvalidValue;
    }
    if ((((uintptr_t)k_cache | (uintptr_t)v_cache) | (uint64_t)k_block_stride |
         (uint64_t)k_head_stride | (uint64_t)v_block_stride | (uint64_t)v_head_stride) & 15u) {
        fprintf(stderr, "[gfx906_fa_amd] paged_attention_tiled: cache bases and strides must be 16-byte aligned\n");
        return hipErrorInvalidValue;
    }
    AttnParams p = {};
    p.q = q;
    p.q_ts = q_token_stride;
    p.q_hs = q_head_stride;
    p.kc = k_cache;
    p.vc = static_cast<const uint8_t *>(v_cache);
    p.cbs = k_block_stride;
    p.chs = k_head_stride;
    p.vcbs = v_block_stride;
    p.vchs = v_head_stride;
    p.bt = block_table;
    p.bt_stride = block_table_stride;
    p.seq_lens = seq_lens;
    p.qsl = query_start_loc;
    p.q_abs = q_abs_offset;
    p.causal = causal ? 1 : 0;
    p.mask = static_cast<const uint16_t *>(mask);
    p.mask_bs = mask_batch_stride;
    p.mask_rs = mask_row_stride;
    p.mask_cols = mask_cols;
    p.mask_vec = mask != nullptr && ((uintptr_t)mask & 7) == 0 && (mask_batch_stride & 3) == 0 &&
                 (mask_row_stride & 3) == 0 && (mask_cols & 3) == 0;
    p.Hkv = num_kv_heads;
    p.G = num_heads / num_kv_heads;
    p.block_size = block_size;
    p.scale_log2e = scale * LOG2E;
    set_prefill_scale(p);
    p.out = out;
    p.o_ts = out_token_stride;
    p.o_hs = out_head_stride;
    p.num_seqs = num_seqs;
    p.pf_rows = PF_ROWS;
    p.dec_rows_max = 0;  // every sequence through the tiled kernel
    const int rows = max(max_query_len, 1) * p.G;
    const dim3 grid(((rows + PF_ROWS - 1) / PF_ROWS) * num_kv_heads, num_seqs);
    const dim3 block(64 * PF_WAVES);
#define GFA_TILED(QDT)                                                                                      \
    if (v_format == 1) {                                                                                    \
        if (mask) attn_prefill_kernel<QDT, GFA_DTYPE_F32, true, true><<<grid, block, 0, stream>>>(p);       \
        else attn_prefill_kernel<QDT, GFA_DTYPE_F32, true, false><<<grid, block, 0, stream>>>(p);           \
    } else {                                                                                                \
        if (mask) attn_prefill_kernel<QDT, GFA_DTYPE_F32, false, true><<<grid, block, 0, stream>>>(p);      \
        else attn_prefill_kernel<QDT, GFA_DTYPE_F32, false, false><<<grid, block, 0, stream>>>(p);          \
    }
    switch (q_dtype) {
        case GFA_DTYPE_F32: GFA_TILED(GFA_DTYPE_F32); break;
        case GFA_DTYPE_F16: GFA_TILED(GFA_DTYPE_F16); break;
        default: GFA_TILED(GFA_DTYPE_BF16); break;
    }
#undef GFA_TILED
    return hipGetLastError();
}
