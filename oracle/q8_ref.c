/* CPU restatement (plain C) of the Q8_0 quantizer, the paged cache write and
 * the paged gather of the reference.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ and bench.py's cpu_baseline leg
 * as a checker, never by the product path.
 *
 * Restates:
 *   q8_ref_quantize_block   extension/gfx906_fa_quant.cu:45-85
 *   q8_ref_quantize_rows    extension/gfx906_fa_quant.cu:100-129
 *   q8_ref_reshape_and_cache extension/gfx906_fa_quant.cu:150-200
 *   q8_ref_gather           extension/gfx906_fa_gather.cu:190-357 (v2)
 *
 * Built with plain IEEE single-precision arithmetic (no -ffast-math): the
 * closed form needs correctly rounded division and round-half-even rint.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* float -> IEEE binary16 bits, round to nearest even (the semantics of the
 * GPU's v_cvt_f16_f32 with default rounding). */
static uint16_t f32_to_f16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t mant = x & 0x007FFFFFu;
    int32_t exp = (int32_t)((x >> 23) & 0xFF);
    if (exp == 0xFF) { /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0u));
    }
    int32_t e = exp - 127 + 15;
    if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u); /* overflow -> inf */
    if (e <= 0) {
        /* subnormal half (or zero) */
        if (e < -10) return (uint16_t)sign;
        mant |= 0x00800000u;
        int shift = 14 - e;             /* 24-bit mantissa -> 10-bit at e */
        uint32_t half_m = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half_m & 1u))) half_m++;
        return (uint16_t)(sign | half_m);
    }
    uint32_t half_m = mant >> 13;
    uint32_t rem = mant & 0x1FFFu;
    uint32_t h = sign | ((uint32_t)e << 10) | half_m;
    if (rem > 0x1000u || (rem == 0x1000u && (half_m & 1u))) h++; /* may carry into exp: ok */
    return (uint16_t)h;
}

/* AMD v_cvt_i32_f32 semantics: NaN -> 0, saturate; then clamp to int8. */
static int8_t rint_to_i8(float v) {
    if (v != v) return 0;
    float r = rintf(v);
    if (r < -128.0f) r = -128.0f;
    if (r > 127.0f) r = 127.0f;
    return (int8_t)(int)r;
}

/* One 32-element block: writes d (fp16 bits) and 32 int8. */
void q8_ref_quantize_block(const float *x, uint16_t *d_out, int8_t *q_out) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
        float a = fabsf(x[i]);
        amax = fmaxf(amax, a);
    }
    volatile float d = amax / 127.0f;
    volatile float id = d > 0.0f ? 1.0f / d : 0.0f;
    for (int i = 0; i < 32; ++i) {
        volatile float p = x[i] * id;
        q_out[i] = rint_to_i8(p);
    }
    *d_out = f32_to_f16_rne(d);
}

static float f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FF, x;
    if (e == 0) {
        if (m == 0) { x = sign; }
        else {
            int sh = 0;
            while (!(m & 0x400)) { m <<= 1; ++sh; }
            m &= 0x3FF;
            x = sign | ((uint32_t)(127 - 15 - sh + 1) << 23) | (m << 13);
        }
    } else if (e == 0x1F) {
        x = sign | 0x7F800000u | (m << 13);
    } else {
        x = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static float bf16_to_f32(uint16_t b) {
    uint32_t x = (uint32_t)b << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* in_dtype: 1 = fp16 bits, 2 = bf16 bits, 0 = fp32. */
static float load_elem(const void *x, int64_t i, int in_dtype) {
    if (in_dtype == 0) return ((const float *)x)[i];
    uint16_t b = ((const uint16_t *)x)[i];
    return in_dtype == 1 ? f16_to_f32(b) : bf16_to_f32(b);
}

/* Dense rows: x [N, D] -> y [N, D/32*34] block_q8_0 bytes. */
void q8_ref_quantize_rows(const void *x, int in_dtype, uint8_t *y, int64_t N, int D) {
    const int nb = D / 32;
    float buf[32];
    for (int64_t r = 0; r < N; ++r) {
        for (int b = 0; b < nb; ++b) {
            for (int i = 0; i < 32; ++i) buf[i] = load_elem(x, r * D + b * 32 + i, in_dtype);
            uint16_t d;
            int8_t q[32];
            q8_ref_quantize_block(buf, &d, q);
            uint8_t *o = y + (r * nb + b) * 34;
            o[0] = (uint8_t)(d & 0xFF);
            o[1] = (uint8_t)(d >> 8);
            memcpy(o + 2, q, 32);
        }
    }
}

/* reshape_and_cache_q8: key strides in elements, cache strides in bytes. */
void q8_ref_reshape_and_cache(const void *key, int in_dtype, const int64_t *slot_mapping,
                              uint8_t *cache, int num_tokens, int Hkv, int D, int block_size,
                              int64_t key_token_stride, int64_t key_head_stride,
                              int64_t cache_block_stride, int64_t cache_token_stride,
                              int64_t cache_head_stride) {
    const int nb = D / 32;
    float buf[32];
    for (int t = 0; t < num_tokens; ++t) {
        int64_t slot = slot_mapping[t];
        if (slot < 0) continue;
        int64_t blk = slot / block_size, off = slot % block_size;
        for (int h = 0; h < Hkv; ++h) {
            int64_t xb = (int64_t)t * key_token_stride + (int64_t)h * key_head_stride;
            uint8_t *row = cache + blk * cache_block_stride + off * cache_token_stride + h * cache_head_stride;
            for (int b = 0; b < nb; ++b) {
                for (int i = 0; i < 32; ++i) buf[i] = load_elem(key, xb + b * 32 + i, in_dtype);
                uint16_t d;
                int8_t q[32];
                q8_ref_quantize_block(buf, &d, q);
                row[b * 34 + 0] = (uint8_t)(d & 0xFF);
                row[b * 34 + 1] = (uint8_t)(d >> 8);
                memcpy(row + b * 34 + 2, q, 32);
            }
        }
    }
}

/* Gather (v2 contract): K rows of k_row_bytes, V rows of v_row_bytes.
 * Valid token: copy both.  Invalid: zero V, leave K. */
void q8_ref_gather(const uint8_t *k_cache, const uint8_t *v_cache, const int32_t *block_table,
                   const int32_t *seq_lens, uint8_t *k_out, uint8_t *v_out,
                   int num_seqs, int Hkv, int Sk, int k_row_bytes, int v_row_bytes,
                   int block_size, int max_blocks,
                   int64_t kc_block, int64_t kc_token, int64_t kc_head,
                   int64_t vc_block, int64_t vc_token, int64_t vc_head) {
    for (int s = 0; s < num_seqs; ++s) {
        int sl = seq_lens[s];
        for (int h = 0; h < Hkv; ++h) {
            for (int t = 0; t < Sk; ++t) {
                int lb = t / block_size;
                int pb = lb < max_blocks ? block_table[(int64_t)s * max_blocks + lb] : -1;
                uint8_t *kd = k_out + (((int64_t)s * Hkv + h) * Sk + t) * k_row_bytes;
                uint8_t *vd = v_out + (((int64_t)s * Hkv + h) * Sk + t) * v_row_bytes;
                if (t < sl && pb >= 0) {
                    int off = t % block_size;
                    memcpy(kd, k_cache + pb * kc_block + off * kc_token + h * kc_head, k_row_bytes);
                    memcpy(vd, v_cache + pb * vc_block + off * vc_token + h * vc_head, v_row_bytes);
                } else {
                    memset(vd, 0, v_row_bytes);
                }
            }
        }
    }
}
