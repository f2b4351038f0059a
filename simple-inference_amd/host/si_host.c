/*
 * si_host.c -- C11 host mirror of the reference entry points over the
 * MI355X C ABI (include/si_host.h documents every difference).
 */
#define _GNU_SOURCE
#include "si_host.h"

#include <errno.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

/* qwen_one_layer.c:26-28: errors are fail-stop. */
static void die(const char *message) {
    fprintf(stderr, "error: %s\n", message);
    exit(1);
}

static void check(int rc, const char *what) {
    if (rc != SI_OK) {
        fprintf(stderr, "error: %s: %s\n", what, si_last_error());
        exit(1);
    }
}

static void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) {
        fprintf(stderr, "error: %s: %s\n", what, hipGetErrorString(e));
        exit(1);
    }
}

/* load_file (qwen_one_layer.c:188-208): exact size check, optional files
 * may be absent (ENOENT), anything else is fatal. */
static void *load_file(const char *dir, const char *name, size_t expected, int optional) {
    char path[1024];
    int n = snprintf(path, sizeof path, "%s/%s", dir, name);
    if (n < 0 || (size_t)n >= sizeof path) die("Weights directory path too long");
    FILE *f = fopen(path, "rb");
    if (!f) {
        if (optional && errno == ENOENT) return NULL;
        perror(path);
        exit(1);
    }
    if (fseek(f, 0, SEEK_END) != 0 || ftell(f) != (long)expected || fseek(f, 0, SEEK_SET) != 0) {
        fprintf(stderr, "Wrong size for %s (expected %zu bytes)\n", path, expected);
        exit(1);
    }
    void *buf = malloc(expected);
    if (!buf) die("Out of memory loading weights");
    if (fread(buf, 1, expected, f) != expected) die("Failed to read weight file");
    fclose(f);
    return buf;
}

si_model_t *si_model_from_host(const si_shape_t *shape, const si_layer_host_t *w,
                               int max_tokens, int max_pos) {
    si_model_t *m = calloc(1, sizeof *m);
    if (!m) die("Out of memory");
    m->shape = *shape;
    m->max_tokens = max_tokens;
    m->max_pos = max_pos;
    check(si_layer_create(shape, w, max_tokens, max_pos, &m->layer), "si_layer_create");
    m->attn_ws_bytes = si_attention_workspace(shape, 1, max_pos);
    hip_check(hipMalloc(&m->attn_ws, m->attn_ws_bytes), "hipMalloc(attention workspace)");
    check(si_layer_set_timing(m->layer, 1), "si_layer_set_timing");
    return m;
}

si_model_t *load_layer(const si_shape_t *s, const char *dir, int max_tokens, int max_pos) {
    const size_t H = (size_t)s->hidden, QD = (size_t)s->qheads * s->hdim;
    const size_t KVD = (size_t)s->kvheads * s->hdim, F = (size_t)s->ffn;
    si_layer_host_t w;
    memset(&w, 0, sizeof w);
    /* qwen_one_layer.c:212-219 with runtime sizes */
    w.wq = load_file(dir, "q.q4_0", QD * H / 32 * 18, 0);
    w.wk = load_file(dir, "k.q4_0", KVD * H / 32 * 18, 0);
    w.wv = load_file(dir, "v.q4_0", KVD * H / 32 * 18, 0);
    w.wo = load_file(dir, "o.q4_0", H * QD / 32 * 18, 0);
    w.norm = load_file(dir, "norm.f32", H * sizeof(float), 1);
    w.bq = load_file(dir, "q_bias.f32", QD * sizeof(float), 1);
    w.bk = load_file(dir, "k_bias.f32", KVD * sizeof(float), 1);
    w.bv = load_file(dir, "v_bias.f32", KVD * sizeof(float), 1);
    if (F) {
        w.post_norm = load_file(dir, "post_norm.f32", H * sizeof(float), 1);
        w.wgate = load_file(dir, "gate.q4_0", F * H / 32 * 18, 1);
        w.wup = load_file(dir, "up.q4_0", F * H / 32 * 18, 1);
        w.wdown = load_file(dir, "down.q4_0", H * F / 32 * 18, 1);
    }
    si_model_t *m = si_model_from_host(s, &w, max_tokens, max_pos);
    free((void *)w.wq); free((void *)w.wk); free((void *)w.wv); free((void *)w.wo);
    free((void *)w.norm); free((void *)w.bq); free((void *)w.bk); free((void *)w.bv);
    free((void *)w.post_norm); free((void *)w.wgate); free((void *)w.wup);
    free((void *)w.wdown);
    return m;
}

void free_layer(si_model_t *m) {
    if (!m) return;
    si_layer_destroy(m->layer);
    if (m->attn_ws) (void)hipFree(m->attn_ws);
    free(m);
}

/* Maps the device phases onto the reference's nine (qwen_one_layer.c:323-334). */
static phase_t phases_to_ref(const si_model_t *l, const float *ms) {
    phase_t p;
    memset(&p, 0, sizeof p);
    const float qd = (float)(l->shape.qheads * l->shape.hdim);
    const float kvd = (float)(l->shape.kvheads * l->shape.hdim);
    const float qkv = ms[SI_PHASE_QKV] * 1e-3f;
    p.rms = ms[SI_PHASE_RMS_Q8] * 1e-3f;       /* RMSNorm + Q8 fused */
    p.q8_input = 0.0f;
    p.q_proj = qkv * qd / (qd + 2 * kvd);
    p.k_proj = qkv * kvd / (qd + 2 * kvd);
    p.v_proj = qkv * kvd / (qd + 2 * kvd);
    p.rope_cache = ms[SI_PHASE_ROPE_KV] * 1e-3f;
    p.attention = ms[SI_PHASE_ATTENTION_Q8] * 1e-3f; /* attention + Q8 fused */
    p.q8_output = 0.0f;
    p.out_proj = ms[SI_PHASE_OUT_PROJ] * 1e-3f;
    return p;
}

/* Planar Q8 (device) -> block_q8_0 records (host). */
static void capture_q8(const si_model_t *l, block_q8_0 *dst) {
    const int qd = l->shape.qheads * l->shape.hdim, nb = qd / 32;
    int8_t *qs = malloc((size_t)qd);
    uint16_t *d = malloc((size_t)nb * sizeof(uint16_t));
    if (!qs || !d) die("Out of memory");
    hip_check(hipMemcpy(qs, si_layer_buffer(l->layer, SI_BUF_ATTQ_QS), (size_t)qd,
                        hipMemcpyDeviceToHost), "capture q8");
    hip_check(hipMemcpy(d, si_layer_buffer(l->layer, SI_BUF_ATTQ_D), (size_t)nb * 2,
                        hipMemcpyDeviceToHost), "capture q8 scales");
    for (int b = 0; b < nb; ++b) {
        dst[b].d = d[b];
        memcpy(dst[b].qs, qs + (size_t)b * 32, 32);
    }
    free(qs);
    free(d);
}

static phase_t decode(const si_model_t *l, const float *x, uint16_t *kc, uint16_t *vc,
                      int context, float *output, int flags, float *attn_copy,
                      block_q8_0 *q8_copy) {
    if (context < 1 || context > l->max_pos) die("Context must be 1..max_pos");
    check(si_layer_decode(l->layer, x, kc, vc, context, output, flags, l->stream),
          "si_layer_decode");
    float ms[SI_PHASE_COUNT];
    check(si_layer_phase_ms(l->layer, ms), "si_layer_phase_ms");
    phase_t p = phases_to_ref(l, ms);
    if (attn_copy)
        hip_check(hipMemcpy(attn_copy, si_layer_buffer(l->layer, SI_BUF_ATTN),
                            sizeof(float) * l->shape.qheads * l->shape.hdim,
                            hipMemcpyDeviceToHost), "capture attention");
    if (q8_copy) capture_q8(l, q8_copy);
    return p;
}

phase_t run_layer(const si_model_t *l, const float *x, uint16_t *kc, uint16_t *vc, int context,
                  float *output, attention_method_t method, float *scores, float *attn_copy,
                  block_q8_0 *q8_copy) {
    /* the standard method materializes its scores in the layer's own
     * [qheads][max_pos] device buffer; the caller's scores are not needed */
    (void)scores;
    if (method != ATTENTION_STANDARD && method != ATTENTION_FLASH) die("Unknown attention method");
    const int flags = SI_LAYER_ATTN_ONLY | (method == ATTENTION_STANDARD ? SI_LAYER_ATTN_STANDARD : 0);
    return decode(l, x, kc, vc, context, output, flags, attn_copy, q8_copy);
}

fused_stats_t run_layer_fused(const si_model_t *l, const float *x, uint16_t *kc, uint16_t *vc,
                              int context, float *output, float *attn_capture,
                              block_q8_0 *q8_capture) {
    fused_stats_t st;
    st.phase = decode(l, x, kc, vc, context, output, SI_LAYER_ATTN_ONLY, attn_capture, q8_capture);
    st.tcm_stage = 0.0;
    return st;
}

phase_t run_layer_full(const si_model_t *l, const float *x, uint16_t *kc, uint16_t *vc,
                       int context, float *output) {
    return decode(l, x, kc, vc, context, output, SI_LAYER_FULL, NULL, NULL);
}

void pf_run_batch(const si_model_t *l, const float *x, int ntok, int prefix, uint16_t *kc,
                  uint16_t *vc, float *output, int full) {
    /* prefill_weight_stationary.h:187 */
    if (ntok < 1 || ntok > l->max_tokens || prefix < 0 || prefix + ntok > l->max_pos)
        die("Invalid prefill configuration");
    check(si_layer_prefill(l->layer, x, ntok, prefix, kc, vc, output,
                           full ? SI_LAYER_FULL : SI_LAYER_ATTN_ONLY, l->stream),
          "si_layer_prefill");
    hip_check(hipStreamSynchronize((hipStream_t)l->stream), "prefill");
}

void attention_flash(const si_model_t *l, const float *q, const uint16_t *kc, const uint16_t *vc,
                     int context, float *out) {
    if (context <= 0) {
        /* attention_kernels.h:95-98: empty context gives zero output */
        hip_check(hipMemsetAsync(out, 0, sizeof(float) * l->shape.qheads * l->shape.hdim,
                                 (hipStream_t)l->stream), "attention_flash");
        return;
    }
    if (context > l->max_pos) die("Context exceeds max_pos");
    check(si_attention(&l->shape, q, 1, kc, vc, 0, NULL, context, 0, context, out, NULL, NULL,
                       NULL, l->attn_ws, l->attn_ws_bytes, l->stream),
          "si_attention");
}

void attention_compute(const si_model_t *l, attention_method_t method, const float *q,
                       const uint16_t *kc, const uint16_t *vc, int context, float *out,
                       float *score_workspace) {
    if (method != ATTENTION_STANDARD && method != ATTENTION_FLASH) die("Unknown attention method");
    if (method == ATTENTION_FLASH) {
        attention_flash(l, q, kc, vc, context, out);
        return;
    }
    /* attention_kernels.h:33-78; score_workspace: device [qheads][context] */
    if (context < 0) context = 0;
    if (context > 0 && !score_workspace) die("Standard attention needs a score workspace");
    check(si_attention_standard(&l->shape, q, kc, vc, context, out, score_workspace, l->stream),
          "si_attention_standard");
}

void quantize_q8(const float *src, block_q8_0 *dst, int count) {
    if (count % 32) die("Q8 quantization length must be multiple of 32"); /* :99 */
    check(si_quantize_q8(src, dst, count, NULL), "si_quantize_q8");
}

void si_quantize_q4_0_host(const float *src, uint8_t *dst, int count) {
    if (count % 32) die("Q4_0 length must be multiple of 32");
    for (int b = 0; b < count / 32; ++b) {
        const float *x = src + (size_t)b * 32;
        uint8_t *blk = dst + (size_t)b * 18;
        float amax = 0.0f, m = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float a = fabsf(x[j]);
            if (amax < a) {
                amax = a;
                m = x[j];
            }
        }
        const float d = m / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        /* fp16(d), round to nearest even (the F16C conversion ggml uses) */
        uint32_t bits;
        memcpy(&bits, &d, 4);
        const uint32_t sign = (bits >> 16) & 0x8000u, a = bits & 0x7fffffffu;
        uint16_t h;
        if (a >= 0x7f800000u) h = (uint16_t)(sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
        else if (a >= 0x477ff000u) h = (uint16_t)(sign | 0x7c00u);
        else if (a < 0x38800000u) {
            float av;
            memcpy(&av, &a, 4);
            h = (uint16_t)(sign | (uint16_t)nearbyintf(av * 0x1p24f));
        } else {
            uint32_t r = a - 0x38000000u;
            r += 0x0fffu + ((r >> 13) & 1u);
            h = (uint16_t)(sign | (r >> 13));
        }
        blk[0] = (uint8_t)(h & 0xff);
        blk[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 16; ++j) {
            int lo = (int8_t)(x[j] * id + 8.5f);
            int hi = (int8_t)(x[j + 16] * id + 8.5f);
            lo = lo > 15 ? 15 : lo;
            hi = hi > 15 ? 15 : hi;
            blk[2 + j] = (uint8_t)(lo | (hi << 4));
        }
    }
}
