/*
 * si_oracle.c -- CPU parity oracle (TEST INFRASTRUCTURE ONLY, see si_oracle.h).
 *
 * Restates the reference's portable scalar path with a runtime shape.  Build
 * flags follow the reference Makefile:7 (-O2 -std=c11 -ffp-contract=off), so
 * every float operation rounds exactly where the reference's does: no fused
 * multiply-add, C left-to-right evaluation, the same libm calls.
 */
#define _GNU_SOURCE
#include "si_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static __attribute__((noreturn)) void or_die(const char *what) {
    /* qwen_one_layer.c:26-28: errors are fail-stop. */
    fprintf(stderr, "oracle error: %s\n", what);
    exit(1);
}

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* ------------------------------------------------------------------------
 * IEEE binary16 <-> binary32 (qwen_one_layer.c:42-86).
 * Widening is exact.  Narrowing is round-to-nearest-even with gradual
 * underflow; any NaN becomes sign|0x7e00 and overflow becomes sign|inf.
 * ---------------------------------------------------------------------- */
float or_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in binary32 */
        float v = (float)m * 0x1p-24f;
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t or_f32_to_f16(float x) {
    const uint32_t b = f2u(x);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    const uint32_t a = b & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {
        /* below 2^-14: result is k * 2^-24; |x|*2^24 is exact, RNE to int */
        float k = nearbyintf(u2f(a) * 0x1p24f);
        return (uint16_t)(sign | (uint16_t)k);
    }
    /* normal: rebias the exponent (127 -> 15) and round 23 -> 10 bits, RNE;
     * a mantissa carry correctly bumps the exponent. */
    uint32_t r = a - 0x38000000u;
    r += 0x0fffu + ((r >> 13) & 1u);
    return (uint16_t)(sign | (r >> 13));
}

void or_f32_to_f16_array(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = or_f32_to_f16(src[i]);
}

void or_f16_to_f32_array(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = or_f16_to_f32(src[i]);
}

/* ------------------------------------------------------------------------
 * xorshift32 RNG (qwen_one_layer.c:88-96), used by the reference's own
 * validation cases.  Uniform values k/32767.5 - 1 for k in 0..65535.
 * ---------------------------------------------------------------------- */
static uint32_t or_state = 0x5217ac8bu;

void or_rng_seed(uint32_t seed) { or_state = seed; }

uint32_t or_rng_u32(void) {
    uint32_t s = or_state;
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    or_state = s;
    return s;
}

float or_rng_float(void) {
    return (float)(or_rng_u32() & 0xffffu) * (1.0f / 32767.5f) - 1.0f;
}

void or_rng_fill(float *dst, size_t n, float scale) {
    for (size_t i = 0; i < n; ++i) dst[i] = or_rng_float() * scale;
}

/* ------------------------------------------------------------------------
 * Q8_0 activation quantization (qwen_one_layer.c:98-116).
 * d = amax/127 (binary32, correctly rounded); the stored scale is fp16(d) but
 * the reciprocal is taken from the unrounded d; values round half-even
 * (lrintf) and clamp to [-127, 127].
 * ---------------------------------------------------------------------- */
void or_quantize_q8(const float *src, or_block_q8_0 *dst, int count) {
    if (count % OR_QK) or_die("Q8 quantization length must be multiple of 32");
    const int nb = count / OR_QK;
    for (int b = 0; b < nb; ++b) {
        const float *x = src + (size_t)b * OR_QK;
        float amax = 0.0f;
        for (int j = 0; j < OR_QK; ++j) {
            const float a = fabsf(x[j]);
            if (a > amax) amax = a;
        }
        const float d = amax / 127.0f;
        dst[b].d = or_f32_to_f16(d);
        const float inv = (d == 0.0f) ? 0.0f : 1.0f / d;
        for (int j = 0; j < OR_QK; ++j) {
            long q = lrintf(x[j] * inv);
            q = q > 127 ? 127 : q;
            q = q < -127 ? -127 : q;
            dst[b].qs[j] = (int8_t)q;
        }
    }
}

/* ------------------------------------------------------------------------
 * One Q4_0 block x one Q8_0 block (qwen_one_layer.c:118-146, scalar branch).
 * Byte j of the packed nibbles holds element j (low) and j+16 (high); the
 * stored value is nibble-8.  Exact int32, |result| <= 32*8*127.
 * ---------------------------------------------------------------------- */
int32_t or_dot_32_q4q8(const uint8_t *w, const int8_t *a) {
    const uint8_t *qs = w + 2; /* skip the fp16 scale */
    int32_t acc = 0;
    for (int j = 0; j < 16; ++j) {
        const int lo = (int)(qs[j] & 0x0f) - 8;
        const int hi = (int)(qs[j] >> 4) - 8;
        acc += lo * a[j];
        acc += hi * a[j + 16];
    }
    return acc;
}

static inline uint16_t q4_scale_bits(const uint8_t *blk) {
    return (uint16_t)((uint16_t)blk[0] | ((uint16_t)blk[1] << 8));
}

void or_block_dots(const uint8_t *w, const or_block_q8_0 *x, int inputs,
                   int outputs, int32_t *dots) {
    const int nb = inputs / OR_QK;
    for (int r = 0; r < outputs; ++r)
        for (int b = 0; b < nb; ++b)
            dots[(size_t)r * nb + b] =
                or_dot_32_q4q8(w + ((size_t)r * nb + b) * OR_Q4_BYTES, x[b].qs);
}

/* ------------------------------------------------------------------------
 * Row-major Q4_0 x Q8_0 mat-vec (qwen_one_layer.c:148-162).
 * y = bias (or 0); then for blocks 0..K/32-1 in order:
 *   y = y + ((float)dot * fp16(w.d)) * fp16(x.d)
 * ---------------------------------------------------------------------- */
void or_matvec_q4q8(const uint8_t *w, const or_block_q8_0 *x, int inputs,
                    int outputs, const float *bias, float *out) {
    const int nb = inputs / OR_QK;
    for (int r = 0; r < outputs; ++r) {
        const uint8_t *row = w + (size_t)r * nb * OR_Q4_BYTES;
        float y = bias ? bias[r] : 0.0f;
        for (int b = 0; b < nb; ++b) {
            const uint8_t *blk = row + (size_t)b * OR_Q4_BYTES;
            const int32_t dot = or_dot_32_q4q8(blk, x[b].qs);
            const float term = (float)dot * or_f16_to_f32(q4_scale_bits(blk)) *
                               or_f16_to_f32(x[b].d);
            y = y + term;
        }
        out[r] = y;
    }
}

/* ------------------------------------------------------------------------
 * RMSNorm (qwen_one_layer.c:164-169): sum of squares in binary64, in order;
 * inv = 1/sqrt(float(sum/n) + eps); out = (x*inv)*gain.
 * ---------------------------------------------------------------------- */
void or_rmsnorm(const float *in, const float *w, float *out, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) ss += (double)in[i] * in[i];
    const float inv = 1.0f / sqrtf((float)(ss / n) + eps);
    for (int i = 0; i < n; ++i) out[i] = in[i] * inv * (w ? w[i] : 1.0f);
}

/* ------------------------------------------------------------------------
 * RoPE, rotate-half pairing (i, i+hdim/2) (qwen_one_layer.c:172-183).
 * theta_i = pos / base^(2i/hdim); a' = a*c - b*s, b' = b*c + a*s.
 * ---------------------------------------------------------------------- */
void or_rope_table(int pos0, int npos, int hdim, float base, float *cos_out,
                   float *sin_out) {
    const int half = hdim / 2;
    for (int p = 0; p < npos; ++p) {
        for (int i = 0; i < half; ++i) {
            const float theta = (float)(pos0 + p) / powf(base, (float)(2 * i) / (float)hdim);
            cos_out[(size_t)p * half + i] = cosf(theta);
            sin_out[(size_t)p * half + i] = sinf(theta);
        }
    }
}

void or_rope(float *heads, int nheads, int hdim, int position, float base) {
    const int half = hdim / 2;
    for (int h = 0; h < nheads; ++h) {
        float *v = heads + (size_t)h * hdim;
        for (int i = 0; i < half; ++i) {
            const float theta = (float)position / powf(base, (float)(2 * i) / (float)hdim);
            const float c = cosf(theta), s = sinf(theta);
            const float a = v[i], b = v[i + half];
            v[i] = a * c - b * s;
            v[i + half] = b * c + a * s;
        }
    }
}

/* ------------------------------------------------------------------------
 * Streaming (online-softmax) GQA attention (attention_kernels.h:80-164).
 * KV layout [ctx][kvheads][hdim] fp16; head h reads group h/(qheads/kvheads).
 * Scores are sequential fp32 dots scaled after the sum; one exp per token:
 *   new max:  alpha = exp(m - s); l = l*alpha + 1; o = o*alpha + v; m = s
 *   else:     beta  = exp(s - m); l += beta;       o += beta*v
 * ---------------------------------------------------------------------- */
void or_attention_flash(const or_shape_t *s, const float *q, const uint16_t *kc,
                        const uint16_t *vc, int context, float *out) {
    const int D = s->hdim;
    const float scale = 1.0f / sqrtf((float)D);
    const size_t stride = (size_t)s->kvheads * D;
    const int per_group = s->qheads / s->kvheads;
    for (int h = 0; h < s->qheads; ++h) {
        const int g = h / per_group;
        const float *qh = q + (size_t)h * D;
        float *o = out + (size_t)h * D;
        if (context <= 0) {
            memset(o, 0, (size_t)D * sizeof(float));
            continue;
        }
        float m = 0.0f, l = 1.0f;
        for (int t = 0; t < context; ++t) {
            const uint16_t *k = kc + (size_t)t * stride + (size_t)g * D;
            const uint16_t *v = vc + (size_t)t * stride + (size_t)g * D;
            float sc = 0.0f;
            for (int d = 0; d < D; ++d) sc += qh[d] * or_f16_to_f32(k[d]);
            if (t == 0) {
                m = sc * scale;
                l = 1.0f;
                for (int d = 0; d < D; ++d) o[d] = or_f16_to_f32(v[d]);
                continue;
            }
            sc *= scale;
            if (sc > m) {
                const float alpha = expf(m - sc);
                l = l * alpha + 1.0f;
                for (int d = 0; d < D; ++d) o[d] = o[d] * alpha + or_f16_to_f32(v[d]);
                m = sc;
            } else {
                const float beta = expf(sc - m);
                l += beta;
                for (int d = 0; d < D; ++d) o[d] += beta * or_f16_to_f32(v[d]);
            }
        }
        const float inv = 1.0f / l;
        for (int d = 0; d < D; ++d) o[d] *= inv;
    }
}

/* Materialized-score attention (attention_kernels.h:33-78): scores
 * [qheads][context], max / exp / sum / normalize, then a separate V pass. */
void or_attention_standard(const or_shape_t *s, const float *q, const uint16_t *kc,
                           const uint16_t *vc, int context, float *out,
                           float *scores) {
    const int D = s->hdim;
    const float inv_sqrt = 1.0f / sqrtf((float)D);
    const size_t stride = (size_t)s->kvheads * D;
    const int per_group = s->qheads / s->kvheads;
    for (int h = 0; h < s->qheads; ++h) {
        const int g = h / per_group;
        const float *qh = q + (size_t)h * D;
        float *row = scores + (size_t)h * context;
        for (int t = 0; t < context; ++t) {
            const uint16_t *k = kc + (size_t)t * stride + (size_t)g * D;
            float dot = 0.0f;
            for (int d = 0; d < D; ++d) dot += qh[d] * or_f16_to_f32(k[d]);
            row[t] = dot * inv_sqrt;
        }
    }
    for (int h = 0; h < s->qheads; ++h) {
        float *row = scores + (size_t)h * context;
        float m = -INFINITY;
        for (int t = 0; t < context; ++t) m = fmaxf(m, row[t]);
        float sum = 0.0f;
        for (int t = 0; t < context; ++t) {
            row[t] = expf(row[t] - m);
            sum += row[t];
        }
        const float inv = 1.0f / sum;
        for (int t = 0; t < context; ++t) row[t] *= inv;
    }
    for (int h = 0; h < s->qheads; ++h) {
        const int g = h / per_group;
        const float *row = scores + (size_t)h * context;
        float *o = out + (size_t)h * D;
        memset(o, 0, (size_t)D * sizeof(float));
        for (int t = 0; t < context; ++t) {
            const uint16_t *v = vc + (size_t)t * stride + (size_t)g * D;
            const float p = row[t];
            for (int d = 0; d < D; ++d) o[d] += p * or_f16_to_f32(v[d]);
        }
    }
}

/* Build-defined SwiGLU (Qwen2 MLP): silu(g) = g / (1 + exp(-g)); out = silu(g)*u. */
void or_swiglu(const float *gate, const float *up, float *out, int n) {
    for (int i = 0; i < n; ++i) {
        const float g = gate[i];
        const float silu = g / (1.0f + expf(-g));
        out[i] = silu * up[i];
    }
}

static void check_shape(const or_shape_t *s) {
    if (s->hidden % OR_QK || s->qheads <= 0 || s->kvheads <= 0 ||
        s->qheads % s->kvheads || s->hdim % 2 || (s->qheads * s->hdim) % OR_QK ||
        (s->ffn && s->ffn % OR_QK))
        or_die("invalid shape");
}

/* Attention sublayer of one token (qwen_one_layer.c:237-281):
 * RMSNorm -> Q8 -> Q,K,V (+bias) -> RoPE at context-1 -> fp16 K/V append at
 * row context-1 -> attention over the fp16 cache -> Q8 -> W_O (no bias). */
static void attn_sublayer(const or_shape_t *s, const or_layer_t *l, const float *x,
                          uint16_t *kc, uint16_t *vc, int context, float *out,
                          int method, float *scores, or_capture_t *cap) {
    const int H = s->hidden, D = s->hdim;
    const int QD = s->qheads * D, KVD = s->kvheads * D;
    float *normed = malloc(sizeof(float) * H);
    or_block_q8_0 *xq = malloc(sizeof(or_block_q8_0) * (H / OR_QK));
    float *q = malloc(sizeof(float) * QD);
    float *k = malloc(sizeof(float) * KVD);
    float *v = malloc(sizeof(float) * KVD);
    float *att = malloc(sizeof(float) * QD);
    or_block_q8_0 *aq = malloc(sizeof(or_block_q8_0) * (QD / OR_QK));
    float *own_scores = NULL;
    if (!normed || !xq || !q || !k || !v || !att || !aq) or_die("oom");
    if (method == OR_ATTENTION_STANDARD && !scores) {
        own_scores = malloc(sizeof(float) * (size_t)s->qheads * context);
        if (!own_scores) or_die("oom");
        scores = own_scores;
    }

    or_rmsnorm(x, l->norm, normed, H, s->rms_eps);
    or_quantize_q8(normed, xq, H);
    or_matvec_q4q8(l->wq, xq, H, QD, l->bq, q);
    or_matvec_q4q8(l->wk, xq, H, KVD, l->bk, k);
    or_matvec_q4q8(l->wv, xq, H, KVD, l->bv, v);
    or_rope(q, s->qheads, D, context - 1, s->rope_base);
    or_rope(k, s->kvheads, D, context - 1, s->rope_base);
    const size_t row = (size_t)(context - 1) * KVD;
    for (int i = 0; i < KVD; ++i) {
        kc[row + i] = or_f32_to_f16(k[i]);
        vc[row + i] = or_f32_to_f16(v[i]);
    }
    if (method == OR_ATTENTION_FLASH)
        or_attention_flash(s, q, kc, vc, context, att);
    else
        or_attention_standard(s, q, kc, vc, context, att, scores);
    or_quantize_q8(att, aq, QD);
    or_matvec_q4q8(l->wo, aq, QD, H, NULL, out);

    if (cap) {
        if (cap->normed) memcpy(cap->normed, normed, sizeof(float) * H);
        if (cap->xq) memcpy(cap->xq, xq, sizeof(or_block_q8_0) * (H / OR_QK));
        if (cap->q) memcpy(cap->q, q, sizeof(float) * QD);
        if (cap->k) memcpy(cap->k, k, sizeof(float) * KVD);
        if (cap->v) memcpy(cap->v, v, sizeof(float) * KVD);
        if (cap->attn) memcpy(cap->attn, att, sizeof(float) * QD);
        if (cap->attq) memcpy(cap->attq, aq, sizeof(or_block_q8_0) * (QD / OR_QK));
        if (cap->attn_out) memcpy(cap->attn_out, out, sizeof(float) * H);
    }
    free(normed); free(xq); free(q); free(k); free(v); free(att); free(aq);
    free(own_scores);
}

void or_run_layer(const or_shape_t *s, const or_layer_t *l, const float *x,
                  uint16_t *kc, uint16_t *vc, int context, float *out,
                  int method, float *scores, or_capture_t *cap) {
    check_shape(s);
    if (context < 1) or_die("context must be >= 1");
    attn_sublayer(s, l, x, kc, vc, context, out, method, scores, cap);
}

/* Build-defined second half of a Qwen2 decoder layer:
 * h = x + attn_out; n2 = RMSNorm(h, post_norm); a = SwiGLU(W_gate.Q8(n2),
 * W_up.Q8(n2)); out = h + W_down.Q8(a).  Every projection is the same
 * Q4_0 x Q8_0 mat-vec as the reference's. */
static void ffn_half(const or_shape_t *s, const or_layer_t *l, const float *x,
                     const float *attn_out, float *out, or_capture_t *cap) {
    const int H = s->hidden, F = s->ffn;
    float *h = malloc(sizeof(float) * H);
    float *n2 = malloc(sizeof(float) * H);
    or_block_q8_0 *xq2 = malloc(sizeof(or_block_q8_0) * (H / OR_QK));
    float *g = malloc(sizeof(float) * F);
    float *u = malloc(sizeof(float) * F);
    float *a = malloc(sizeof(float) * F);
    or_block_q8_0 *aq = malloc(sizeof(or_block_q8_0) * (F / OR_QK));
    float *y = malloc(sizeof(float) * H);
    if (!h || !n2 || !xq2 || !g || !u || !a || !aq || !y) or_die("oom");
    for (int i = 0; i < H; ++i) h[i] = x[i] + attn_out[i];
    or_rmsnorm(h, l->post_norm, n2, H, s->rms_eps);
    or_quantize_q8(n2, xq2, H);
    or_matvec_q4q8(l->wgate, xq2, H, F, NULL, g);
    or_matvec_q4q8(l->wup, xq2, H, F, NULL, u);
    or_swiglu(g, u, a, F);
    or_quantize_q8(a, aq, F);
    or_matvec_q4q8(l->wdown, aq, F, H, NULL, y);
    for (int i = 0; i < H; ++i) out[i] = h[i] + y[i];
    if (cap) {
        if (cap->h) memcpy(cap->h, h, sizeof(float) * H);
        if (cap->normed2) memcpy(cap->normed2, n2, sizeof(float) * H);
        if (cap->xq2) memcpy(cap->xq2, xq2, sizeof(or_block_q8_0) * (H / OR_QK));
        if (cap->gate) memcpy(cap->gate, g, sizeof(float) * F);
        if (cap->up) memcpy(cap->up, u, sizeof(float) * F);
        if (cap->act) memcpy(cap->act, a, sizeof(float) * F);
        if (cap->actq) memcpy(cap->actq, aq, sizeof(or_block_q8_0) * (F / OR_QK));
        if (cap->ffn_out) memcpy(cap->ffn_out, y, sizeof(float) * H);
    }
    free(h); free(n2); free(xq2); free(g); free(u); free(a); free(aq); free(y);
}

void or_layer_decode(const or_shape_t *s, const or_layer_t *l, const float *x,
                     uint16_t *kc, uint16_t *vc, int context, float *out,
                     or_capture_t *cap) {
    check_shape(s);
    if (s->ffn <= 0) or_die("full layer needs ffn > 0");
    if (context < 1) or_die("context must be >= 1");
    float *ao = malloc(sizeof(float) * s->hidden);
    if (!ao) or_die("oom");
    attn_sublayer(s, l, x, kc, vc, context, ao, OR_ATTENTION_FLASH, NULL, cap);
    ffn_half(s, l, x, ao, out, cap);
    free(ao);
}

/* Causal prefill (prefill_weight_stationary.h:183-311 order): phase 1 writes
 * RoPE'd fp16 K and V for every token at rows prefix+t; phase 2 gives token t
 * Q, attention with context prefix+t+1, Q8 and W_O (then the FFN half when
 * full != 0).  Validated in the reference as equal to sequential decode
 * (bench_ai_dma_prefill.c:104-129). */
void or_layer_prefill(const or_shape_t *s, const or_layer_t *l, const float *x,
                      int ntok, int prefix, uint16_t *kc, uint16_t *vc,
                      const int *rows, int nrows, int full, float *out) {
    check_shape(s);
    if (ntok < 1 || prefix < 0) or_die("invalid prefill size");
    if (full && s->ffn <= 0) or_die("full layer needs ffn > 0");
    const int H = s->hidden, D = s->hdim;
    const int QD = s->qheads * D, KVD = s->kvheads * D;
    float *normed = malloc(sizeof(float) * H);
    or_block_q8_0 *xq = malloc(sizeof(or_block_q8_0) * (size_t)ntok * (H / OR_QK));
    float *k = malloc(sizeof(float) * KVD);
    float *v = malloc(sizeof(float) * KVD);
    float *q = malloc(sizeof(float) * QD);
    float *att = malloc(sizeof(float) * QD);
    or_block_q8_0 *aq = malloc(sizeof(or_block_q8_0) * (QD / OR_QK));
    float *ao = malloc(sizeof(float) * H);
    if (!normed || !xq || !k || !v || !q || !att || !aq || !ao) or_die("oom");

    for (int t = 0; t < ntok; ++t) {
        or_block_q8_0 *xt = xq + (size_t)t * (H / OR_QK);
        or_rmsnorm(x + (size_t)t * H, l->norm, normed, H, s->rms_eps);
        or_quantize_q8(normed, xt, H);
        or_matvec_q4q8(l->wk, xt, H, KVD, l->bk, k);
        or_matvec_q4q8(l->wv, xt, H, KVD, l->bv, v);
        or_rope(k, s->kvheads, D, prefix + t, s->rope_base);
        const size_t row = (size_t)(prefix + t) * KVD;
        for (int i = 0; i < KVD; ++i) {
            kc[row + i] = or_f32_to_f16(k[i]);
            vc[row + i] = or_f32_to_f16(v[i]);
        }
    }
    const int count = rows ? nrows : ntok;
    for (int r = 0; r < count; ++r) {
        const int t = rows ? rows[r] : r;
        if (t < 0 || t >= ntok) or_die("prefill row out of range");
        const or_block_q8_0 *xt = xq + (size_t)t * (H / OR_QK);
        or_matvec_q4q8(l->wq, xt, H, QD, l->bq, q);
        or_rope(q, s->qheads, D, prefix + t, s->rope_base);
        or_attention_flash(s, q, kc, vc, prefix + t + 1, att);
        or_quantize_q8(att, aq, QD);
        float *dst = out + (size_t)r * H;
        if (full) {
            or_matvec_q4q8(l->wo, aq, QD, H, NULL, ao);
            ffn_half(s, l, x + (size_t)t * H, ao, dst, NULL);
        } else {
            or_matvec_q4q8(l->wo, aq, QD, H, NULL, dst);
        }
    }
    free(normed); free(xq); free(k); free(v); free(q); free(att); free(aq); free(ao);
}

/* ------------------------------------------------------------------------
 * Q4_0 weight quantizer: ggml's published quantize_row_q4_0_ref.  The
 * reference consumes pre-quantized GGUF bytes (extract_weights.py:4-5), so
 * this is not pinned by it; it is pinned by invariants in the tests.
 * Per 32-block: m = the signed value of largest magnitude, d = m / -8,
 * nibble = min(15, trunc(x/d + 8.5)); byte j = nib(j) | nib(j+16) << 4.
 * ---------------------------------------------------------------------- */
void or_quantize_q4_0(const float *src, uint8_t *dst, int count) {
    if (count % OR_QK) or_die("Q4_0 length must be multiple of 32");
    for (int b = 0; b < count / OR_QK; ++b) {
        const float *x = src + (size_t)b * OR_QK;
        uint8_t *blk = dst + (size_t)b * OR_Q4_BYTES;
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < OR_QK; ++j) {
            if (amax < fabsf(x[j])) { amax = fabsf(x[j]); mx = x[j]; }
        }
        const float d = mx / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t hb = or_f32_to_f16(d);
        blk[0] = (uint8_t)(hb & 0xff);
        blk[1] = (uint8_t)(hb >> 8);
        for (int j = 0; j < 16; ++j) {
            int n0 = (int8_t)(x[j] * id + 8.5f);
            int n1 = (int8_t)(x[j + 16] * id + 8.5f);
            n0 = n0 > 15 ? 15 : n0;
            n1 = n1 > 15 ? 15 : n1;
            blk[2 + j] = (uint8_t)(n0 | (n1 << 4));
        }
    }
}

void or_dequantize_q4_0(const uint8_t *src, float *dst, int count) {
    for (int b = 0; b < count / OR_QK; ++b) {
        const uint8_t *blk = src + (size_t)b * OR_Q4_BYTES;
        const float d = or_f16_to_f32(q4_scale_bits(blk));
        for (int j = 0; j < 16; ++j) {
            dst[(size_t)b * OR_QK + j] = (float)((blk[2 + j] & 0x0f) - 8) * d;
            dst[(size_t)b * OR_QK + j + 16] = (float)((blk[2 + j] >> 4) - 8) * d;
        }
    }
}

/* ---- Column-SoA tiles (repack_weights.py) and the legacy fused decode path
 *      (fused_layer.h:169-455).  Written for hdim 128: a tile holds 256
 *      outputs, i.e. two query heads, or the 128 K and 128 V outputs of one KV
 *      group; query heads pair up within their KV group; W_O splits into
 *      256-row output tiles. ---- */

#define OR_COL_GROUP 5120 /* fused_layer.h:33: 32 columns x 128 B + 256 fp32 scales */

static void check_colsoa_shape(const or_shape_t *s) {
    check_shape(s);
    if (s->hdim != 128 || (s->qheads / s->kvheads) % 2 || s->hidden % 256)
        or_die("column-SoA tiles need hdim 128, paired query heads and hidden % 256 == 0");
}

size_t or_colsoa_bytes(const or_shape_t *s, int which) {
    const size_t nb = (size_t)s->hidden / OR_QK, pairs = (size_t)s->qheads / 2;
    switch (which) {
        case 0: return pairs * nb * OR_COL_GROUP;                           /* q.colsoa  */
        case 1: return (size_t)s->kvheads * nb * OR_COL_GROUP;              /* kv.colsoa */
        default: return pairs * ((size_t)s->hidden / 256) * 8 * OR_COL_GROUP; /* o.colsoa */
    }
}

/* repack_weights.py:39-52 (nibble, scale_f32): element `col` of row `row`
 * of a row-major Q4_0 matrix with `cols` inputs. */
static unsigned q4_nibble(const uint8_t *w, int cols, int row, int col) {
    const uint8_t *blk = w + ((size_t)row * (cols / OR_QK) + col / OR_QK) * OR_Q4_BYTES;
    const int k = col % OR_QK;
    const uint8_t byte = blk[2 + k % 16];
    return k < 16 ? (byte & 15u) : (unsigned)(byte >> 4);
}

/* repack_weights.py:55-76 (pack_tile): nblocks groups from input block b0;
 * low nibbles = rows lo_row..lo_row+127 of lo, high = hi_row.. of hi. */
static void pack_tile(uint8_t *dst, const uint8_t *lo, const uint8_t *hi, int cols, int lo_row,
                      int hi_row, int b0, int nblocks) {
    for (int b = 0; b < nblocks; ++b) {
        uint8_t *g = dst + (size_t)b * OR_COL_GROUP;
        const int blk = b0 + b;
        for (int k = 0; k < OR_QK; ++k)
            for (int j = 0; j < 128; ++j)
                g[k * 128 + j] = (uint8_t)(q4_nibble(lo, cols, lo_row + j, blk * OR_QK + k) |
                                           q4_nibble(hi, cols, hi_row + j, blk * OR_QK + k) << 4);
        for (int j = 0; j < 256; ++j) {
            const uint8_t *src = j < 128 ? lo : hi;
            const int row = j < 128 ? lo_row + j : hi_row + j - 128;
            const uint8_t *e = src + ((size_t)row * (cols / OR_QK) + blk) * OR_Q4_BYTES;
            const float sc = or_f16_to_f32((uint16_t)(e[0] | e[1] << 8));
            memcpy(g + 4096 + 4 * j, &sc, 4);
        }
    }
}

/* repack_weights.py:96-120: q tiles per head pair, kv tiles per KV group
 * (K rows low, V rows high), o tiles per input head pair x 256-row output
 * tile (8 blocks each). */
void or_colsoa_repack(const or_shape_t *s, const uint8_t *wq, const uint8_t *wk,
                      const uint8_t *wv, const uint8_t *wo, uint8_t *q, uint8_t *kv,
                      uint8_t *o) {
    check_colsoa_shape(s);
    const int H = s->hidden, QD = s->qheads * s->hdim, nb = H / OR_QK, pairs = s->qheads / 2;
    const size_t tile = (size_t)nb * OR_COL_GROUP, sub = 8 * (size_t)OR_COL_GROUP;
    for (int p = 0; p < pairs; ++p) pack_tile(q + p * tile, wq, wq, H, p * 256, p * 256 + 128, 0, nb);
    for (int g = 0; g < s->kvheads; ++g)
        pack_tile(kv + g * tile, wk, wv, H, g * 128, g * 128, 0, nb);
    for (int p = 0; p < pairs; ++p)
        for (int y = 0; y < H / 256; ++y)
            pack_tile(o + ((size_t)p * (H / 256) + y) * sub, wo, wo, QD, y * 256, y * 256 + 128,
                      p * 8, 8);
}

/* fused_column_matvec, scalar path (fused_layer.h:220-244). */
void or_fused_column_matvec(const uint8_t *tile, const or_block_q8_0 *x, int nblocks,
                            const float *bias_lo, const float *bias_hi, float *out, int add) {
    if (!add)
        for (int j = 0; j < 128; ++j) {
            out[j] = bias_lo ? bias_lo[j] : 0.0f;
            out[j + 128] = bias_hi ? bias_hi[j] : 0.0f;
        }
    for (int b = 0; b < nblocks; ++b) {
        const uint8_t *g = tile + (size_t)b * OR_COL_GROUP;
        int32_t acc[256];
        memset(acc, 0, sizeof acc);
        for (int k = 0; k < OR_QK; ++k) {
            const int a = x[b].qs[k];
            for (int j = 0; j < 128; ++j) {
                const uint8_t w = g[k * 128 + j];
                acc[j] += ((int)(w & 15) - 8) * a;
                acc[j + 128] += ((int)(w >> 4) - 8) * a;
            }
        }
        const float dx = or_f16_to_f32(x[b].d);
        for (int j = 0; j < 256; ++j) {
            float sc;
            memcpy(&sc, g + 4096 + 4 * j, 4);
            out[j] += ((float)acc[j] * sc) * dx;
        }
    }
}

/* fused_attention_pair, scalar path (fused_layer.h:251-355): query heads
 * 2h' and 2h'+1 of qpair against KV group `group`; the one-exp-per-token
 * recurrence of attention_flash. */
void or_attention_pair(const or_shape_t *s, const float *qpair, const uint16_t *kc,
                       const uint16_t *vc, int context, int group, float *opair) {
    const int D = s->hdim;
    const float inv_dim = 1.0f / sqrtf((float)D);
    const size_t stride = (size_t)s->kvheads * D;
    float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.0f, 0.0f};
    memset(opair, 0, sizeof(float) * 2 * D);
    for (int t = 0; t < context; ++t) {
        const uint16_t *k = kc + (size_t)t * stride + (size_t)group * D;
        const uint16_t *v = vc + (size_t)t * stride + (size_t)group * D;
        for (int h = 0; h < 2; ++h) {
            const float *qh = qpair + h * D;
            float *o = opair + h * D;
            float sc = 0.0f;
            for (int d = 0; d < D; ++d) sc += qh[d] * or_f16_to_f32(k[d]);
            sc *= inv_dim;
            if (t == 0) {
                m[h] = sc;
                l[h] = 1.0f;
                for (int d = 0; d < D; ++d) o[d] = or_f16_to_f32(v[d]);
            } else if (sc > m[h]) {
                const float alpha = expf(m[h] - sc);
                l[h] = l[h] * alpha + 1.0f;
                for (int d = 0; d < D; ++d) o[d] = o[d] * alpha + or_f16_to_f32(v[d]);
                m[h] = sc;
            } else {
                const float beta = expf(sc - m[h]);
                l[h] += beta;
                for (int d = 0; d < D; ++d) o[d] += beta * or_f16_to_f32(v[d]);
            }
        }
    }
    for (int h = 0; h < 2; ++h)
        for (int d = 0; d < D; ++d) opair[h * D + d] *= 1.0f / l[h];
}

/* run_layer_legacy_fused (fused_layer.h:397-455) with attention_wo_fused
 * (:361-390): per KV group the K/V tile (+bias), RoPE of K, fp16 append;
 * per head pair the Q tile (+bias), RoPE, pair attention, Q8 of its 256
 * values and the W_O partial added into the zeroed output, tile by tile.
 * Captures (fp32 [qheads*hdim], Q8 [qheads*hdim/32]) may be NULL. */
void or_run_layer_legacy_fused(const or_shape_t *s, const or_layer_t *l, const uint8_t *qt,
                               const uint8_t *kvt, const uint8_t *ot, const float *x,
                               uint16_t *kc, uint16_t *vc, int context, float *out,
                               float *attn_capture, or_block_q8_0 *q8_capture) {
    check_colsoa_shape(s);
    if (context < 1) or_die("context must be >= 1");
    const int H = s->hidden, D = s->hdim, KVD = s->kvheads * D, nb = H / OR_QK;
    const int ppg = s->qheads / s->kvheads / 2, ytiles = H / 256;
    const size_t tile = (size_t)nb * OR_COL_GROUP, sub = 8 * (size_t)OR_COL_GROUP;
    float *normed = malloc(sizeof(float) * H);
    or_block_q8_0 *inq8 = malloc(sizeof(or_block_q8_0) * nb);
    if (!normed || !inq8) or_die("oom");
    or_rmsnorm(x, l->norm, normed, H, s->rms_eps);
    or_quantize_q8(normed, inq8, H);
    memset(out, 0, sizeof(float) * H);
    for (int g = 0; g < s->kvheads; ++g) {
        float kvpair[256];
        or_fused_column_matvec(kvt + g * tile, inq8, nb, l->bk ? l->bk + g * D : NULL,
                               l->bv ? l->bv + g * D : NULL, kvpair, 0);
        or_rope(kvpair, 1, D, context - 1, s->rope_base);
        const size_t off = (size_t)(context - 1) * KVD + (size_t)g * D;
        for (int d = 0; d < D; ++d) {
            kc[off + d] = or_f32_to_f16(kvpair[d]);
            vc[off + d] = or_f32_to_f16(kvpair[d + D]);
        }
        for (int p = 0; p < ppg; ++p) {
            const int pair = g * ppg + p;
            float qpair[256], opair[256];
            or_block_q8_0 oq[8];
            const float *bq = l->bq ? l->bq + (size_t)pair * 256 : NULL;
            or_fused_column_matvec(qt + pair * tile, inq8, nb, bq, bq ? bq + 128 : NULL, qpair,
                                   0);
            or_rope(qpair, 2, D, context - 1, s->rope_base);
            or_attention_pair(s, qpair, kc, vc, context, g, opair);
            if (attn_capture) memcpy(attn_capture + (size_t)pair * 256, opair, sizeof opair);
            or_quantize_q8(opair, oq, 256);
            if (q8_capture) memcpy(q8_capture + (size_t)pair * 8, oq, sizeof oq);
            for (int y = 0; y < ytiles; ++y)
                or_fused_column_matvec(ot + ((size_t)pair * ytiles + y) * sub, oq, 8, NULL, NULL,
                                       out + y * 256, 1);
        }
    }
    free(normed);
    free(inq8);
}
