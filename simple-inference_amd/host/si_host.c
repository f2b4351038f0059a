/*
 * si_host.c -- C11 host mirror of the reference entry points over the
 * MI355X C ABI (include/si_host.h documents every difference).
 */
#define _GNU_SOURCE
#include "si_host.h"

#include <errno.h>
#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

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

static void *dev_alloc(size_t bytes, const char *what) {
    void *p = NULL;
    hip_check(hipMalloc(&p, bytes ? bytes : 1), what);
    return p;
}

static double wall_seconds(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* A weight file of exactly `want` bytes under dir, read whole into host
 * memory.  A missing optional file gives NULL; a missing required file, a
 * size mismatch or a read error ends the process (the loading contract of
 * qwen_one_layer.c:188-208). */
static void *read_weight_file(const char *dir, const char *name, size_t want, int optional) {
    char *path = NULL;
    if (asprintf(&path, "%s/%s", dir, name) < 0) die("Out of memory building a weight path");
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        if (optional && errno == ENOENT) {
            free(path);
            return NULL;
        }
        fprintf(stderr, "error: cannot open %s: %s\n", path, strerror(errno));
        exit(1);
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode) || (size_t)st.st_size != want) {
        fprintf(stderr, "error: %s holds %lld bytes; this shape needs exactly %zu\n", path,
                (long long)st.st_size, want);
        exit(1);
    }
    unsigned char *buf = malloc(want ? want : 1);
    if (!buf) die("Out of memory reading weights");
    for (size_t got = 0; got < want;) {
        const ssize_t r = read(fd, buf + got, want - got);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) {
            fprintf(stderr, "error: short read of %s\n", path);
            exit(1);
        }
        got += (size_t)r;
    }
    close(fd);
    free(path);
    return buf;
}

static float *upload_opt(const float *src, size_t n) {
    if (!src) return NULL;
    float *d = dev_alloc(n * sizeof(float), "hipMalloc(layer vector)");
    hip_check(hipMemcpy(d, src, n * sizeof(float), hipMemcpyHostToDevice), "upload vector");
    return d;
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
    const size_t pair_ws = si_attention_group_workspace(shape, 2, max_pos);
    if (pair_ws > m->attn_ws_bytes) m->attn_ws_bytes = pair_ws;
    m->attn_ws = dev_alloc(m->attn_ws_bytes, "hipMalloc(attention workspace)");
    /* RoPE angle tables for rope() and the column-SoA path */
    const size_t te = (size_t)max_pos * (shape->hdim / 2);
    float *c = malloc(te * sizeof(float)), *sn = malloc(te * sizeof(float));
    if (!c || !sn) die("Out of memory");
    check(si_rope_table(max_pos, shape->hdim, shape->rope_base, c, sn), "si_rope_table");
    m->rope_cos = upload_opt(c, te);
    m->rope_sin = upload_opt(sn, te);
    free(c);
    free(sn);
    const size_t QD = (size_t)shape->qheads * shape->hdim, KVD = (size_t)shape->kvheads * shape->hdim;
    m->norm = upload_opt(w->norm, (size_t)shape->hidden);
    m->bq = upload_opt(w->bq, QD);
    m->bk = upload_opt(w->bk, KVD);
    m->bv = upload_opt(w->bv, KVD);
    check(si_layer_set_timing(m->layer, 1), "si_layer_set_timing");
    return m;
}

si_model_t *load_layer(const si_shape_t *s, const char *dir, int max_tokens, int max_pos) {
    const size_t H = (size_t)s->hidden, QD = (size_t)s->qheads * s->hdim;
    const size_t KVD = (size_t)s->kvheads * s->hdim, F = (size_t)s->ffn;
    const size_t f32 = sizeof(float);
    /* the files of qwen_one_layer.c:212-219 at the runtime shape, then the
     * build-defined FFN's */
    struct {
        const char *name;
        size_t bytes;
        int optional;
    } const files[12] = {
        {"q.q4_0", QD * H / 32 * 18, 0},      {"k.q4_0", KVD * H / 32 * 18, 0},
        {"v.q4_0", KVD * H / 32 * 18, 0},     {"o.q4_0", H * QD / 32 * 18, 0},
        {"norm.f32", H * f32, 1},             {"q_bias.f32", QD * f32, 1},
        {"k_bias.f32", KVD * f32, 1},         {"v_bias.f32", KVD * f32, 1},
        {"post_norm.f32", H * f32, 1},        {"gate.q4_0", F * H / 32 * 18, 1},
        {"up.q4_0", F * H / 32 * 18, 1},      {"down.q4_0", H * F / 32 * 18, 1},
    };
    void *data[12] = {0};
    const int nfiles = F ? 12 : 8;
    for (int i = 0; i < nfiles; ++i)
        data[i] = read_weight_file(dir, files[i].name, files[i].bytes, files[i].optional);
    si_layer_host_t w = {
        .wq = data[0], .wk = data[1], .wv = data[2], .wo = data[3],
        .norm = data[4], .bq = data[5], .bk = data[6], .bv = data[7],
        .post_norm = data[8], .wgate = data[9], .wup = data[10], .wdown = data[11],
    };
    si_model_t *m = si_model_from_host(s, &w, max_tokens, max_pos);
    for (int i = 0; i < 12; ++i) free(data[i]);
    return m;
}

void free_layer(si_model_t *m) {
    if (!m) return;
    si_layer_destroy(m->layer);
    void *dev[] = {m->attn_ws, m->rope_cos, m->rope_sin, m->norm, m->bq, m->bk, m->bv};
    for (size_t i = 0; i < sizeof dev / sizeof dev[0]; ++i)
        if (dev[i]) (void)hipFree(dev[i]);
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
    /* the attention row and its Q8 stay in the layer's buffers only when asked for */
    if (attn_copy || q8_copy) flags |= SI_LAYER_CAPTURE;
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

fused_stats_t run_layer_fused(const si_model_t *l, const fused_weights_t *fw, const float *x,
                              uint16_t *kc, uint16_t *vc, int context, float *output,
                              float *attn_capture, block_q8_0 *q8_capture) {
    (void)fw; /* the fused kernels read the layer's own repack of the same weights */
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

void matvec_q4q8(const uint8_t *weights, const block_q8_0 *input, int inputs, int outputs,
                 const float *bias, float *out) {
    if (inputs <= 0 || inputs % 32 || outputs < 0) die("matvec_q4q8: bad size");
    check(si_matvec_q4q8_rowmajor(weights, input, inputs, outputs, bias, out, NULL),
          "si_matvec_q4q8_rowmajor");
}

void rmsnorm(const si_model_t *l, const float *input, const float *weight, float *out) {
    check(si_rmsnorm(input, weight, 1, l->shape.hidden, l->shape.rms_eps, out, l->stream),
          "si_rmsnorm");
}

void rope(const si_model_t *l, float *heads, int nheads, int position) {
    if (position < 0 || position >= l->max_pos) die("rope: position outside the layer's tables");
    check(si_rope(&l->shape, heads, nheads, position, l->rope_cos, l->rope_sin, l->max_pos,
                  l->stream),
          "si_rope");
}

/* ------------------------------------------------------------------ */
/* Column-SoA tiles and the legacy fused path (fused_layer.h)          */
/* ------------------------------------------------------------------ */

#define COL_GROUP 5120u /* 32 columns x 128 packed bytes + 256 fp32 scales */

static int colsoa_shape(const si_shape_t *s) {
    return s->hdim == 128 && s->kvheads > 0 && s->qheads % s->kvheads == 0 &&
           (s->qheads / s->kvheads) % 2 == 0 && s->hidden > 0 && s->hidden % 256 == 0;
}

size_t si_colsoa_bytes(const si_shape_t *s, int which) {
    if (!s || !colsoa_shape(s)) return 0;
    const size_t blocks = (size_t)s->hidden / 32, pairs = (size_t)s->qheads / 2;
    if (which == 0) return pairs * blocks * COL_GROUP;
    if (which == 1) return (size_t)s->kvheads * blocks * COL_GROUP;
    if (which == 2) return pairs * ((size_t)s->hidden / 256) * 8 * COL_GROUP;
    return 0;
}

/* Nibble of input `col` of row `row` in a row-major Q4_0 matrix. */
static unsigned nibble_at(const uint8_t *w, int ncols, int row, int col) {
    const uint8_t *blk = w + ((size_t)row * (ncols / 32) + col / 32) * 18;
    const int e = col % 32;
    return e < 16 ? (blk[2 + e] & 15u) : (unsigned)(blk[2 + e - 16] >> 4);
}

/* One tile: `nblocks` groups from input block b0 whose low nibbles are rows
 * lo..lo+127 of wlo and high nibbles rows hi..hi+127 of whi, followed per
 * group by the 256 scales widened to fp32 (exact). */
static void colsoa_tile(uint8_t *dst, const uint8_t *wlo, const uint8_t *whi, int ncols, int lo,
                        int hi, int b0, int nblocks) {
    for (int b = 0; b < nblocks; ++b) {
        uint8_t *grp = dst + (size_t)b * COL_GROUP;
        for (int k = 0; k < 32; ++k) {
            const int col = (b0 + b) * 32 + k;
            for (int j = 0; j < 128; ++j)
                grp[k * 128 + j] =
                    (uint8_t)(nibble_at(wlo, ncols, lo + j, col) | nibble_at(whi, ncols, hi + j, col) << 4);
        }
        float *sc = (float *)(void *)(grp + 4096);
        for (int half = 0; half < 2; ++half)
            for (int j = 0; j < 128; ++j) {
                const uint8_t *w = half ? whi : wlo;
                const int row = (half ? hi : lo) + j;
                const uint8_t *blk = w + ((size_t)row * (ncols / 32) + b0 + b) * 18;
                const uint16_t h = (uint16_t)(blk[0] | blk[1] << 8);
                float v;
                /* binary16 -> binary32 is exact: rebuild the value */
                const int e = (h >> 10) & 31, m = h & 1023;
                if (e == 0) v = ldexpf((float)m, -24);
                else if (e == 31) v = m ? NAN : INFINITY;
                else v = ldexpf((float)(m | 1024), e - 25);
                sc[half * 128 + j] = (h & 0x8000u) ? -v : v;
            }
    }
}

void si_colsoa_repack_host(const si_shape_t *s, const si_layer_host_t *w, uint8_t *q,
                           uint8_t *kv, uint8_t *o) {
    if (!colsoa_shape(s)) die("Column-SoA tiles need hdim 128, paired heads, hidden % 256 == 0");
    const int H = s->hidden, QD = s->qheads * s->hdim, nb = H / 32;
    const size_t tile = (size_t)nb * COL_GROUP, sub = 8 * (size_t)COL_GROUP;
    for (int p = 0; p < s->qheads / 2; ++p)
        colsoa_tile(q + p * tile, w->wq, w->wq, H, 256 * p, 256 * p + 128, 0, nb);
    for (int g = 0; g < s->kvheads; ++g)
        colsoa_tile(kv + g * tile, w->wk, w->wv, H, 128 * g, 128 * g, 0, nb);
    const int yt = H / 256;
    for (int p = 0; p < s->qheads / 2; ++p)
        for (int y = 0; y < yt; ++y)
            colsoa_tile(o + ((size_t)p * yt + y) * sub, w->wo, w->wo, QD, 256 * y, 256 * y + 128,
                        8 * p, 8);
}

static fused_weights_t fused_alloc(const si_model_t *l) {
    const si_shape_t *s = &l->shape;
    if (!colsoa_shape(s)) die("This shape has no column-SoA layout (needs hdim 128)");
    fused_weights_t fw;
    memset(&fw, 0, sizeof fw);
    fw.q_bytes = si_colsoa_bytes(s, 0);
    fw.kv_bytes = si_colsoa_bytes(s, 1);
    fw.o_bytes = si_colsoa_bytes(s, 2);
    fw.q = dev_alloc(fw.q_bytes, "hipMalloc(q tiles)");
    fw.kv = dev_alloc(fw.kv_bytes, "hipMalloc(kv tiles)");
    fw.o = dev_alloc(fw.o_bytes, "hipMalloc(o tiles)");
    fw.normed = dev_alloc(sizeof(float) * (size_t)s->hidden, "hipMalloc");
    fw.kvpair = dev_alloc(sizeof(float) * 256, "hipMalloc");
    fw.qpair = dev_alloc(sizeof(float) * 256, "hipMalloc");
    fw.opair = dev_alloc(sizeof(float) * 256, "hipMalloc");
    fw.inq8 = dev_alloc(sizeof(block_q8_0) * (size_t)(s->hidden / 32), "hipMalloc");
    fw.oq = dev_alloc(sizeof(block_q8_0) * 8, "hipMalloc");
    return fw;
}

fused_weights_t si_fused_weights_from_host(const si_model_t *l, const uint8_t *q,
                                           const uint8_t *kv, const uint8_t *o) {
    fused_weights_t fw = fused_alloc(l);
    hip_check(hipMemcpy(fw.q, q, fw.q_bytes, hipMemcpyHostToDevice), "upload q tiles");
    hip_check(hipMemcpy(fw.kv, kv, fw.kv_bytes, hipMemcpyHostToDevice), "upload kv tiles");
    hip_check(hipMemcpy(fw.o, o, fw.o_bytes, hipMemcpyHostToDevice), "upload o tiles");
    return fw;
}

fused_weights_t fused_weights_load(const si_model_t *l, const char *dir, int use_tcm, int block) {
    (void)block;
    if (use_tcm) die("FUSED_TCM requested, but the GPU has no scratchpad to stage tiles in");
    const si_shape_t *s = &l->shape;
    if (!colsoa_shape(s)) die("This shape has no column-SoA layout (needs hdim 128)");
    uint8_t *q = read_weight_file(dir, "q.colsoa", si_colsoa_bytes(s, 0), 0);
    uint8_t *kv = read_weight_file(dir, "kv.colsoa", si_colsoa_bytes(s, 1), 0);
    uint8_t *o = read_weight_file(dir, "o.colsoa", si_colsoa_bytes(s, 2), 0);
    fused_weights_t fw = si_fused_weights_from_host(l, q, kv, o);
    free(q);
    free(kv);
    free(o);
    return fw;
}

void fused_weights_free(fused_weights_t *fw) {
    void *dev[] = {fw->q, fw->kv, fw->o, fw->normed, fw->kvpair, fw->qpair, fw->opair,
                   fw->inq8, fw->oq};
    for (size_t i = 0; i < sizeof dev / sizeof dev[0]; ++i)
        if (dev[i]) (void)hipFree(dev[i]);
    memset(fw, 0, sizeof *fw);
}

void fused_column_matvec(const uint8_t *tile, const block_q8_0 *x, int nblocks,
                         const float *bias_lo, const float *bias_hi, float *output, int add) {
    check(si_colsoa_matvec(tile, 1, x, nblocks, bias_lo, bias_hi, output, add, NULL),
          "si_colsoa_matvec");
}

void fused_attention_pair(const si_model_t *l, const float *qpair, const uint16_t *kc,
                          const uint16_t *vc, int context, int group, float *opair) {
    if (context < 1 || context > l->max_pos) die("Context must be 1..max_pos");
    check(si_attention_group(&l->shape, qpair, 2, group, kc, vc, context, opair, l->attn_ws,
                             l->attn_ws_bytes, l->stream),
          "si_attention_group");
}

/* Runs on the layer's stream; returns the stage's wall time after it ends. */
static double finish(const si_model_t *l, double t0) {
    hip_check(hipStreamSynchronize((hipStream_t)l->stream), "stage");
    return wall_seconds() - t0;
}

void attention_wo_fused(const si_model_t *l, const fused_weights_t *fw, const float *qpair,
                        const uint16_t *kc, const uint16_t *vc, int context, int group, int pair,
                        float *output_y, fused_stats_t *stats, float *attention_capture,
                        block_q8_0 *quantized_capture) {
    const int H = l->shape.hidden;
    double t = wall_seconds();
    fused_attention_pair(l, qpair, kc, vc, context, group, fw->opair);
    stats->phase.attention += (float)finish(l, t);
    if (attention_capture)
        hip_check(hipMemcpy(attention_capture + (size_t)pair * 256, fw->opair,
                            256 * sizeof(float), hipMemcpyDeviceToHost), "attention capture");
    t = wall_seconds();
    check(si_quantize_q8(fw->opair, fw->oq, 256, l->stream), "si_quantize_q8");
    stats->phase.q8_output += (float)finish(l, t);
    if (quantized_capture)
        hip_check(hipMemcpy(quantized_capture + (size_t)pair * 8, fw->oq, 8 * sizeof(block_q8_0),
                            hipMemcpyDeviceToHost), "Q8 capture");
    /* the pair's 256 input columns of W_O: H/256 output tiles of 8 blocks */
    t = wall_seconds();
    check(si_colsoa_matvec(fw->o + (size_t)pair * (H / 256) * 8 * COL_GROUP, H / 256, fw->oq, 8,
                           NULL, NULL, output_y, 1, l->stream),
          "si_colsoa_matvec");
    stats->phase.out_proj += (float)finish(l, t);
}

fused_stats_t run_layer_legacy_fused(const si_model_t *l, const fused_weights_t *fw,
                                     const float *x, uint16_t *kc, uint16_t *vc, int context,
                                     float *output, float *attn_capture,
                                     block_q8_0 *q8_capture) {
    const si_shape_t *s = &l->shape;
    if (!colsoa_shape(s)) die("This shape has no column-SoA layout (needs hdim 128)");
    if (context < 1 || context > l->max_pos) die("Context must be 1..max_pos");
    const int H = s->hidden, D = s->hdim, KVD = s->kvheads * D, nb = H / 32;
    const int pairs_per_group = s->qheads / s->kvheads / 2;
    const size_t tile = (size_t)nb * COL_GROUP;
    hipStream_t st = (hipStream_t)l->stream;
    fused_stats_t stats;
    memset(&stats, 0, sizeof stats);

    double t = wall_seconds();
    check(si_rmsnorm(x, l->norm, 1, H, s->rms_eps, fw->normed, st), "si_rmsnorm");
    stats.phase.rms = (float)finish(l, t);
    t = wall_seconds();
    check(si_quantize_q8(fw->normed, fw->inq8, H, st), "si_quantize_q8");
    stats.phase.q8_input = (float)finish(l, t);
    hip_check(hipMemsetAsync(output, 0, sizeof(float) * H, st), "zero output");

    for (int g = 0; g < s->kvheads; ++g) {
        t = wall_seconds();
        check(si_colsoa_matvec(fw->kv + g * tile, 1, fw->inq8, nb, l->bk ? l->bk + g * D : NULL,
                               l->bv ? l->bv + g * D : NULL, fw->kvpair, 0, st),
              "si_colsoa_matvec");
        const double kv_time = finish(l, t);
        stats.phase.k_proj += (float)(kv_time * 0.5);
        stats.phase.v_proj += (float)(kv_time * 0.5);
        /* RoPE of the K half, fp16 K and V rows at context-1 */
        t = wall_seconds();
        check(si_rope(s, fw->kvpair, 1, context - 1, l->rope_cos, l->rope_sin, l->max_pos, st),
              "si_rope");
        const size_t row = (size_t)(context - 1) * KVD + (size_t)g * D;
        check(si_f32_to_f16(fw->kvpair, kc + row, D, st), "si_f32_to_f16");
        check(si_f32_to_f16(fw->kvpair + D, vc + row, D, st), "si_f32_to_f16");
        stats.phase.rope_cache += (float)finish(l, t);
        for (int p = 0; p < pairs_per_group; ++p) {
            const int pair = g * pairs_per_group + p;
            const float *bq = l->bq ? l->bq + (size_t)pair * 256 : NULL;
            t = wall_seconds();
            check(si_colsoa_matvec(fw->q + pair * tile, 1, fw->inq8, nb, bq, bq ? bq + 128 : NULL,
                                   fw->qpair, 0, st),
                  "si_colsoa_matvec");
            stats.phase.q_proj += (float)finish(l, t);
            t = wall_seconds();
            check(si_rope(s, fw->qpair, 2, context - 1, l->rope_cos, l->rope_sin, l->max_pos, st),
                  "si_rope");
            stats.phase.rope_cache += (float)finish(l, t);
            attention_wo_fused(l, fw, fw->qpair, kc, vc, context, g, pair, output, &stats,
                               attn_capture, q8_capture);
        }
    }
    return stats;
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
