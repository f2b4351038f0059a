/*
 * si_qwen_layer.c -- the reference's one-layer command line
 * (qwen_one_layer.c:596-713) on the MI355X, over the host mirror
 * (include/si_host.h).
 *
 *   si_qwen_layer <weights_dir|synthetic> [context=256] [repeat=1]
 *                 [standard|flash|compare|fused|fused-compare|reference|soa-staged|soa-fused]
 *
 * Same arguments, limits, synthetic inputs and reports as the reference:
 *   - standard / flash / reference: one method, the nine-phase table
 *     (report, qwen_one_layer.c:310-409); reference is flash, as there;
 *   - compare: both methods on the same tensors, alternating order, the
 *     table with both columns plus attention / Q8 / output agreement
 *     (report_compare, :421-511);
 *   - fused / soa-staged / soa-fused: the fused decode kernels, summary
 *     line (:687-701); there is no scratchpad staging on the GPU, so the
 *     staged variants run the same kernels;
 *   - fused-compare: staged flash vs fused (report_fusion, :526-594).
 * The shape comes from SI_SHAPE (0.5b, 1.5b, 7b; default 1.5b, the
 * reference's compile-time shape, defines.h:16-25).  weights_dir holds the
 * files load_layer reads; "synthetic" generates seeded Q4_0 weights instead.
 * Times are GPU event times of each phase; fused phases read 0 and are
 * reported inside the phase they run in (include/si_host.h).
 */
#define _GNU_SOURCE
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "si_host.h"

static void die(const char *message) {
    fprintf(stderr, "error: %s\n", message);
    exit(1);
}

static void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) {
        fprintf(stderr, "error: %s: %s\n", what, hipGetErrorString(e));
        exit(1);
    }
}

/* The reference's synthetic input stream (qwen_one_layer.c:88-96):
 * xorshift32 from 0x5217ac8b, 16 low bits scaled to [-1, 1]. */
static uint32_t g_rng = 0x5217ac8bu;
static float next_uniform(void) {
    uint32_t v = g_rng;
    v ^= v << 13;
    v ^= v >> 17;
    v ^= v << 5;
    g_rng = v;
    return (float)(v & 0xffffu) * (1.0f / 32767.5f) - 1.0f;
}

/* IEEE binary32 -> binary16, round to nearest even (qwen_one_layer.c:61-86). */
static uint16_t to_half(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    const uint32_t sign = (b >> 16) & 0x8000u, a = b & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (a < 0x38800000u) {
        float v;
        memcpy(&v, &a, 4);
        return (uint16_t)(sign | (uint16_t)nearbyintf(v * 0x1p24f));
    }
    uint32_t r = a - 0x38000000u;
    r += 0x0fffu + ((r >> 13) & 1u);
    return (uint16_t)(sign | (r >> 13));
}

static int shape_named(const char *name, si_shape_t *s) {
    memset(s, 0, sizeof *s);
    s->rope_base = 1e6f;
    s->rms_eps = 1e-6f;
    if (!strcmp(name, "0.5b")) {
        s->hidden = 896; s->qheads = 14; s->kvheads = 2; s->hdim = 64;
    } else if (!strcmp(name, "1.5b")) {
        s->hidden = 1536; s->qheads = 12; s->kvheads = 2; s->hdim = 128;
    } else if (!strcmp(name, "7b")) {
        s->hidden = 3584; s->qheads = 28; s->kvheads = 4; s->hdim = 128;
    } else {
        return 0;
    }
    return 1; /* attention sublayer only: ffn 0, as the reference's layer_t */
}

/* Seeded synthetic attention weights (no files): Q4_0 of uniform values in
 * +-0.05, norm gains 1 +- 0.1, biases +-0.02, from a stream separate from
 * the inputs'. */
static si_model_t *synthetic_layer(const si_shape_t *s, int max_pos) {
    const size_t H = (size_t)s->hidden, QD = (size_t)s->qheads * s->hdim;
    const size_t KVD = (size_t)s->kvheads * s->hdim;
    const uint32_t saved = g_rng;
    g_rng = 0x0badf00du;
    uint8_t *w[4];
    const size_t rows[4] = {QD, KVD, KVD, H}, cols[4] = {H, H, H, QD};
    for (int i = 0; i < 4; ++i) {
        const size_t n = rows[i] * cols[i];
        float *f = malloc(n * sizeof(float));
        w[i] = malloc(n / 32 * 18);
        if (!f || !w[i]) die("Out of memory generating synthetic weights");
        for (size_t j = 0; j < n; ++j) f[j] = next_uniform() * 0.05f;
        si_quantize_q4_0_host(f, w[i], (int)n);
        free(f);
    }
    float *norm = malloc(H * sizeof(float)), *bq = malloc(QD * sizeof(float));
    float *bk = malloc(KVD * sizeof(float)), *bv = malloc(KVD * sizeof(float));
    if (!norm || !bq || !bk || !bv) die("Out of memory generating synthetic weights");
    for (size_t j = 0; j < H; ++j) norm[j] = 1.0f + 0.1f * next_uniform();
    for (size_t j = 0; j < QD; ++j) bq[j] = 0.02f * next_uniform();
    for (size_t j = 0; j < KVD; ++j) bk[j] = 0.02f * next_uniform();
    for (size_t j = 0; j < KVD; ++j) bv[j] = 0.02f * next_uniform();
    si_layer_host_t h;
    memset(&h, 0, sizeof h);
    h.wq = w[0]; h.wk = w[1]; h.wv = w[2]; h.wo = w[3];
    h.norm = norm; h.bq = bq; h.bk = bk; h.bv = bv;
    si_model_t *m = si_model_from_host(s, &h, 1, max_pos);
    for (int i = 0; i < 4; ++i) free(w[i]);
    free(norm); free(bq); free(bk); free(bv);
    g_rng = saved;
    return m;
}

/* Binary KiB/MiB footprints (qwen_one_layer.c:288-302). */
static void fmt_bytes(size_t bytes, char *out, size_t n) {
    if (bytes >= 1024u * 1024u)
        snprintf(out, n, "%.2f MiB", (double)bytes / (1024.0 * 1024.0));
    else if (bytes >= 1024u)
        snprintf(out, n, "%.2f KiB", (double)bytes / 1024.0);
    else
        snprintf(out, n, "%zu B", bytes);
}

static void label(char *out, size_t n, const char *what, size_t bytes) {
    char b[32];
    fmt_bytes(bytes, b, sizeof b);
    snprintf(out, n, "%s %s", what, b);
}

static void add_phase(phase_t *sum, phase_t p) {
    sum->rms += p.rms;
    sum->q8_input += p.q8_input;
    sum->q_proj += p.q_proj;
    sum->k_proj += p.k_proj;
    sum->v_proj += p.v_proj;
    sum->rope_cache += p.rope_cache;
    sum->attention += p.attention;
    sum->q8_output += p.q8_output;
    sum->out_proj += p.out_proj;
}

static void as_array(const phase_t *p, double t[9]) {
    t[0] = p->rms; t[1] = p->q8_input; t[2] = p->q_proj;
    t[3] = p->k_proj; t[4] = p->v_proj; t[5] = p->rope_cache;
    t[6] = p->attention; t[7] = p->q8_output; t[8] = p->out_proj;
}

/* The nine rows' output shapes and data footprints for a runtime shape. */
typedef struct {
    char result[9][32];
    char data[9][36];
} rows_t;

static void row_labels(const si_model_t *l, int context, rows_t *r) {
    const si_shape_t *s = &l->shape;
    const size_t H = (size_t)s->hidden, QD = (size_t)s->qheads * s->hdim;
    const size_t KVD = (size_t)s->kvheads * s->hdim;
    snprintf(r->result[0], 32, "FP32 [%d]", (int)H);
    snprintf(r->result[1], 32, "Q8_0 [%d blocks]", (int)(H / 32));
    snprintf(r->result[2], 32, "FP32 [%d x %d]", s->qheads, s->hdim);
    snprintf(r->result[3], 32, "FP32 [%d x %d]", s->kvheads, s->hdim);
    snprintf(r->result[4], 32, "FP32 [%d x %d]", s->kvheads, s->hdim);
    snprintf(r->result[5], 32, "KV cache update");
    snprintf(r->result[6], 32, "FP32 [%d x %d]", s->qheads, s->hdim);
    snprintf(r->result[7], 32, "Q8_0 [%d blocks]", (int)(QD / 32));
    snprintf(r->result[8], 32, "FP32 [%d]", (int)H);
    label(r->data[0], 36, "Norm", H * sizeof(float));
    label(r->data[1], 36, "Q8 buffer", H / 32 * 34);
    label(r->data[2], 36, "Wq Q4_0", QD * H / 32 * 18);
    label(r->data[3], 36, "Wk Q4_0", KVD * H / 32 * 18);
    label(r->data[4], 36, "Wv Q4_0", KVD * H / 32 * 18);
    label(r->data[5], 36, "New K+V", KVD * 2 * 2);
    label(r->data[6], 36, "KV cache", (size_t)context * KVD * 2 * 2);
    label(r->data[7], 36, "Q8 buffer", QD / 32 * 34);
    label(r->data[8], 36, "Wo Q4_0", H * QD / 32 * 18);
}

static const char *const OPS[9] = {"RMSNorm", "Quantize input", "Q projection",
                                   "K projection", "V projection", "RoPE + KV append",
                                   "GQA attention", "Quantize attention", "Output projection"};
static const char *const RULE =
    "-----------------------------------------------------------------------------------"
    "-----------------------------------";

static double checksum(const float *y, int n, const char *what) {
    double c = 0.0;
    for (int i = 0; i < n; ++i) {
        if (!isfinite(y[i])) die(what);
        c += (double)y[i];
    }
    return c;
}

/* report (qwen_one_layer.c:310-409) */
static void report(const phase_t *p, const si_model_t *l, const char *shape, int context,
                   int repeat, const float *out, attention_method_t method) {
    rows_t r;
    row_labels(l, context, &r);
    double t[9], total = 0.0;
    as_array(p, t);
    for (int i = 0; i < 9; ++i) total += t[i];
    const int H = l->shape.hidden;
    const double sum = checksum(out, H, "Non-finite projection output");
    printf("\nQwen2 %s | one attention sublayer (decode) | MI355X\n", shape);
    printf("Attention: %s | Context: %d tokens | Repeats: %d\n",
           method == ATTENTION_FLASH ? "flash" : "standard", context, repeat);
    printf("Weights: Q4_0  |  Matvec activations: Q8_0  |  KV cache: FP16\n");
    printf("Timings are GPU event times; they exclude loading, synthetic inputs and setup.\n\n");
    puts(RULE);
    printf(" %3s  %-22s  %-18s  %-22s %10s %10s %7s\n", "#", "Operation (in order)", "Output",
           "Weights / data", "ms/run", "ms total", "Share");
    puts(RULE);
    for (int i = 0; i < 9; ++i) {
        const char *op = i == 6 ? (method == ATTENTION_FLASH ? "GQA online (flash)"
                                                              : "GQA score/softmax")
                                : OPS[i];
        printf(" %3d  %-22s  %-18s  %-22s %10.3f %10.3f %6.1f%%\n", i + 1, op, r.result[i],
               r.data[i], t[i] * 1000.0 / repeat, t[i] * 1000.0,
               total > 0 ? 100.0 * t[i] / total : 0.0);
    }
    puts(RULE);
    printf("      %-22s  %-18s  %-22s %10.3f %10.3f %6.1f%%\n", "TOTAL (timed)", "", "",
           total * 1000.0 / repeat, total * 1000.0, 100.0);
    const double proj = t[2] + t[3] + t[4], window = t[6] + t[7] + t[8];
    printf("\nQKV projections: %.3f ms/run (%.1f%% of timed work)\n", proj * 1000.0 / repeat,
           total > 0 ? proj * 100.0 / total : 0.0);
    printf("Fusion target (attention + quantize + W_O): %.3f ms/run (%.1f%%)\n",
           window * 1000.0 / repeat, total > 0 ? window * 100.0 / total : 0.0);
    printf("Output checksum: %.9g  |  First 4: [%.6g, %.6g, %.6g, %.6g]\n", sum, out[0], out[1],
           out[2], out[3]);
    puts("Note: data sizes are footprints, not measured memory traffic; fused phases read 0\n"
         "      and are timed inside the phase they run in.\n");
}

/* report_compare (qwen_one_layer.c:421-511) */
static void report_compare(const phase_t *st, const phase_t *fl, const si_model_t *l,
                           const char *shape, int context, int repeat, const float *out_st,
                           const float *out_fl, const float *att_st, const float *att_fl,
                           const block_q8_0 *q8_st, const block_q8_0 *q8_fl) {
    rows_t r;
    row_labels(l, context, &r);
    double a[9], b[9], ta = 0.0, tb = 0.0;
    as_array(st, a);
    as_array(fl, b);
    printf("\nQwen2 %s | single attention sublayer | STANDARD vs FLASH | MI355X\n", shape);
    printf("Context: %d | Repeats: %d per mode\n", context, repeat);
    puts("Weights Q4_0 | Activations Q8_0 | KV FP16 | Same tensors and W_O kernel");
    puts("FLASH = fused streaming online-softmax kernels; STANDARD = materialized QK scores.");
    puts("Timings exclude model loading, synthetic setup, captures and output comparison.\n");
    puts(RULE);
    printf(" %3s  %-21s %-18s %-21s %12s %12s %10s\n", "#", "Operation", "Output",
           "Weights/data", "Std ms/run", "Flash ms/run", "Speedup");
    puts(RULE);
    for (int i = 0; i < 9; ++i) {
        ta += a[i];
        tb += b[i];
        const double ams = a[i] * 1000.0 / repeat, bms = b[i] * 1000.0 / repeat;
        printf(" %3d  %-21s %-18s %-21s %12.3f %12.3f %9.3fx\n", i + 1, OPS[i], r.result[i],
               r.data[i], ams, bms, bms > 0 ? ams / bms : 0.0);
    }
    puts(RULE);
    printf("      %-21s %-18s %-21s %12.3f %12.3f %9.3fx\n", "TOTAL (timed)", "", "",
           ta * 1000.0 / repeat, tb * 1000.0 / repeat, tb > 0 ? ta / tb : 0.0);
    const double fa = (a[6] + a[7] + a[8]) * 1000.0 / repeat;
    const double fb = (b[6] + b[7] + b[8]) * 1000.0 / repeat;
    printf("      %-21s %-18s %-21s %12.3f %12.3f %9.3fx\n", "Future fusion region",
           "attention + Q8 + W_O", "", fa, fb, fb > 0 ? fa / fb : 0.0);

    const int H = l->shape.hidden, QD = l->shape.qheads * l->shape.hdim;
    double att_abs = 0.0, att_rel = 0.0, out_abs = 0.0, out_rel = 0.0;
    for (int i = 0; i < QD; ++i) {
        if (!isfinite(att_st[i]) || !isfinite(att_fl[i]))
            die("Non-finite output in attention comparison");
        const double d = fabs((double)att_st[i] - att_fl[i]);
        const double m = fmax(fabs((double)att_st[i]), fabs((double)att_fl[i]));
        if (d > att_abs) att_abs = d;
        if (m > 1e-6 && d / m > att_rel) att_rel = d / m;
    }
    for (int i = 0; i < H; ++i) {
        const double d = fabs((double)out_st[i] - out_fl[i]);
        const double m = fmax(fabs((double)out_st[i]), fabs((double)out_fl[i]));
        if (d > out_abs) out_abs = d;
        if (m > 1e-6 && d / m > out_rel) out_rel = d / m;
    }
    const double cs = checksum(out_st, H, "Non-finite output in attention comparison");
    const double cf = checksum(out_fl, H, "Non-finite output in attention comparison");
    int changed = 0;
    for (int i = 0; i < QD / 32; ++i)
        changed += memcmp(&q8_st[i], &q8_fl[i], sizeof(block_q8_0)) != 0;
    printf("\nCorrectness (same projected inputs; FP32 rounding may differ):\n");
    printf("  Attention O[%d]: max_abs=%.7g, max_rel=%.7g\n", QD, att_abs, att_rel);
    printf("  Quantized attention: %d / %d Q8_0 blocks differ\n", changed, QD / 32);
    printf("  Final W_O result:   max_abs=%.7g, max_rel=%.7g\n", out_abs, out_rel);
    printf("  Output checksums: standard=%.9g, flash=%.9g\n", cs, cf);
    if (att_abs > 1e-3 || changed > 0)
        puts("  NOTE: The online and standard reductions have different rounding; check Q8 "
             "differences before interpreting projection speedup.");
    puts("\nMode order alternates on successive repeats to reduce first-run bias.\n");
}

/* report_fusion (qwen_one_layer.c:526-594) */
static void report_fusion(const phase_t *base, const fused_stats_t *fused, const char *shape,
                          int context, int repeat, const float *y_ref, const float *y_fused,
                          const float *att_ref, const float *att_fused,
                          const block_q8_0 *q8_ref, const block_q8_0 *q8_fused, int H, int QD) {
    static const char *const names[9] = {"RMSNorm", "Quantize X", "Wq", "Wk", "Wv",
                                         "RoPE + KV append", "Online attention (GQA)",
                                         "Quantize O", "W_o"};
    double a[9], b[9], ta = 0.0, tb = 0.0;
    as_array(base, a);
    as_array(&fused->phase, b);
    for (int i = 0; i < 9; ++i) {
        ta += a[i];
        tb += b[i];
    }
    printf("\nQwen2 %s | STAGED FLASH vs FUSED DECODE KERNELS | MI355X\n", shape);
    printf("One token | context=%d | repeats=%d/mode\n", context, repeat);
    puts("All weights remain 4-bit Q4_0; activations Q8_0; KV FP16.");
    puts("--------------------------------------------------------------------------");
    printf(" %-24s %15s %15s %10s\n", "Operation", "Baseline ms", "Fused ms", "Speedup");
    puts("--------------------------------------------------------------------------");
    for (int i = 0; i < 9; ++i) {
        if (i == 4) continue; /* K and V are reported together */
        const double av = (a[i] + (i == 3 ? a[4] : 0)) * 1000.0 / repeat;
        const double fv = (b[i] + (i == 3 ? b[4] : 0)) * 1000.0 / repeat;
        printf(" %-24s %15.3f %15.3f %9.3fx\n", i == 3 ? "Wk + Wv (interleaved)" : names[i],
               av, fv, fv > 0 ? av / fv : 0.0);
    }
    puts("--------------------------------------------------------------------------");
    printf(" %-24s %15.3f %15.3f %9.3fx\n", "Compute only", ta * 1000 / repeat,
           tb * 1000 / repeat, tb > 0 ? ta / tb : 0.0);
    printf(" %-24s %15s %15.3f\n", "Staging (none on GPU)", "-", fused->tcm_stage * 1000 / repeat);
    const double aw = (a[6] + a[7] + a[8]) * 1000 / repeat, bw = (b[6] + b[7] + b[8]) * 1000 / repeat;
    printf(" %-24s %15.3f %15.3f %9.3fx\n", "Attention + Q8 + W_o", aw, bw, bw > 0 ? aw / bw : 0.0);
    double max_att = 0, max_y = 0, max_rel = 0;
    for (int i = 0; i < QD; ++i) {
        const double da = fabs((double)att_ref[i] - att_fused[i]);
        if (da > max_att) max_att = da;
    }
    for (int i = 0; i < H; ++i) {
        const double dy = fabs((double)y_ref[i] - y_fused[i]);
        const double m = fmax(fabs((double)y_ref[i]), fabs((double)y_fused[i]));
        if (dy > max_y) max_y = dy;
        if (m > 1e-6 && dy / m > max_rel) max_rel = dy / m;
    }
    int q8diff = 0;
    for (int i = 0; i < QD / 32; ++i)
        q8diff += memcmp(&q8_ref[i], &q8_fused[i], sizeof(block_q8_0)) != 0;
    printf("\nCorrectness: attention max_abs=%.8g, Q8 blocks different=%d/%d\n", max_att, q8diff,
           QD / 32);
    printf("             output max_abs=%.8g, output max_rel=%.8g\n", max_y, max_rel);
    printf("             checksum baseline=%.10g fused=%.10g\n",
           checksum(y_ref, H, "Non-finite fused output"),
           checksum(y_fused, H, "Non-finite fused output"));
    puts("On the GPU the staged flash layer already runs the fused decode kernels.\n");
}

int main(int argc, char **argv) {
    if (argc < 2 || argc > 5) {
        fprintf(stderr,
                "Usage: %s <weights_directory|synthetic> [context=256] [repeat=1] "
                "[standard|flash|compare|fused|fused-compare|reference|soa-staged|soa-fused]\n"
                "       (shape from SI_SHAPE: 0.5b, 1.5b or 7b; default 1.5b)\n",
                argv[0]);
        return 2;
    }
    char *end = NULL;
    const long context = argc >= 3 ? strtol(argv[2], &end, 10) : 256;
    if (argc >= 3 && *end) die("Invalid context argument");
    const long repeat = argc >= 4 ? strtol(argv[3], &end, 10) : 1;
    if (argc >= 4 && *end) die("Invalid repeat argument");
    if (context < 1 || context > 32768 || repeat < 1 || repeat > 100000)
        die("Context must be 1..32768 and repeat 1..100000");
    const char *mode = argc >= 5 ? argv[4] : "compare";
    const int compare = !strcmp(mode, "compare");
    const int fused_compare = !strcmp(mode, "fused-compare");
    const int fused_mode = !strcmp(mode, "fused") || fused_compare ||
                           !strcmp(mode, "soa-fused") || !strcmp(mode, "soa-staged");
    const int single = !strcmp(mode, "standard") || !strcmp(mode, "flash") ||
                       !strcmp(mode, "reference");
    if (!compare && !fused_mode && !single)
        die("Attention mode must be standard, flash, compare, fused, fused-compare, reference, "
            "soa-staged or soa-fused");
    const attention_method_t selected =
        !strcmp(mode, "standard") ? ATTENTION_STANDARD : ATTENTION_FLASH;

    const char *shape_name = getenv("SI_SHAPE") ? getenv("SI_SHAPE") : "1.5b";
    si_shape_t shape;
    if (!shape_named(shape_name, &shape)) die("SI_SHAPE must be 0.5b, 1.5b or 7b");
    const int ctx = (int)context, reps = (int)repeat;
    si_model_t *l = !strcmp(argv[1], "synthetic") ? synthetic_layer(&shape, ctx)
                                                  : load_layer(&shape, argv[1], 1, ctx);
    const int H = shape.hidden, QD = shape.qheads * shape.hdim, KVD = shape.kvheads * shape.hdim;

    /* synthetic inputs in the reference's order (qwen_one_layer.c:641-642) */
    float *input = malloc((size_t)H * sizeof(float));
    uint16_t *kh = calloc((size_t)ctx * KVD, sizeof(uint16_t));
    uint16_t *vh = calloc((size_t)ctx * KVD, sizeof(uint16_t));
    if (!input || !kh || !vh) die("Out of memory creating synthetic inputs");
    for (int i = 0; i < H; ++i) input[i] = next_uniform();
    for (size_t i = 0, n = (size_t)(ctx - 1) * KVD; i < n; ++i) {
        kh[i] = to_half(next_uniform() * 0.25f);
        vh[i] = to_half(next_uniform() * 0.25f);
    }
    float *x, *out[2];
    uint16_t *kc, *vc;
    hip_check(hipMalloc((void **)&x, (size_t)H * sizeof(float)), "hipMalloc");
    hip_check(hipMalloc((void **)&out[0], (size_t)H * sizeof(float)), "hipMalloc");
    hip_check(hipMalloc((void **)&out[1], (size_t)H * sizeof(float)), "hipMalloc");
    hip_check(hipMalloc((void **)&kc, (size_t)ctx * KVD * 2), "hipMalloc");
    hip_check(hipMalloc((void **)&vc, (size_t)ctx * KVD * 2), "hipMalloc");
    hip_check(hipMemcpy(x, input, (size_t)H * sizeof(float), hipMemcpyHostToDevice), "copy");
    hip_check(hipMemcpy(kc, kh, (size_t)ctx * KVD * 2, hipMemcpyHostToDevice), "copy");
    hip_check(hipMemcpy(vc, vh, (size_t)ctx * KVD * 2, hipMemcpyHostToDevice), "copy");

    float *y[2], *att[2];
    block_q8_0 *q8[2];
    for (int i = 0; i < 2; ++i) {
        y[i] = malloc((size_t)H * sizeof(float));
        att[i] = malloc((size_t)QD * sizeof(float));
        q8[i] = malloc((size_t)(QD / 32) * sizeof(block_q8_0));
        if (!y[i] || !att[i] || !q8[i]) die("Out of memory for comparison buffers");
    }
    phase_t sums[2];
    memset(sums, 0, sizeof sums);
    if (fused_compare) {
        /* staged flash and fused, alternating, captures in an untimed replay */
        fused_stats_t fs;
        memset(&fs, 0, sizeof fs);
        for (int i = 0; i < 4; ++i) {
            if (i == 0 || i == 3)
                (void)run_layer(l, x, kc, vc, ctx, out[0], ATTENTION_FLASH, NULL, NULL, NULL);
            else
                (void)run_layer_fused(l, x, kc, vc, ctx, out[1], NULL, NULL);
        }
        for (int r = 0; r < reps; ++r)
            for (int j = 0; j < 2; ++j) {
                const int which = (r & 1) ? 1 - j : j;
                if (which == 0) {
                    add_phase(&sums[0],
                              run_layer(l, x, kc, vc, ctx, out[0], ATTENTION_FLASH, NULL, NULL,
                                        NULL));
                } else {
                    const fused_stats_t f = run_layer_fused(l, x, kc, vc, ctx, out[1], NULL, NULL);
                    add_phase(&fs.phase, f.phase);
                    fs.tcm_stage += f.tcm_stage;
                }
            }
        (void)run_layer(l, x, kc, vc, ctx, out[0], ATTENTION_FLASH, NULL, att[0], q8[0]);
        (void)run_layer_fused(l, x, kc, vc, ctx, out[1], att[1], q8[1]);
        for (int i = 0; i < 2; ++i)
            hip_check(hipMemcpy(y[i], out[i], (size_t)H * sizeof(float), hipMemcpyDeviceToHost),
                      "copy");
        report_fusion(&sums[0], &fs, shape_name, ctx, reps, y[0], y[1], att[0], att[1], q8[0],
                      q8[1], H, QD);
    } else if (fused_mode) {
        fused_stats_t fs;
        memset(&fs, 0, sizeof fs);
        for (int r = 0; r < reps; ++r) {
            const fused_stats_t f = run_layer_fused(l, x, kc, vc, ctx, out[0], NULL, NULL);
            add_phase(&fs.phase, f.phase);
        }
        hip_check(hipMemcpy(y[0], out[0], (size_t)H * sizeof(float), hipMemcpyDeviceToHost),
                  "copy");
        double t[9], total = 0.0;
        as_array(&fs.phase, t);
        for (int i = 0; i < 9; ++i) total += t[i];
        printf("%s one-token | context=%d repeats=%d | MI355X fused decode kernels\n",
               !strcmp(mode, "soa-staged") ? "SOA STAGED" : "REGISTER FUSED", ctx, reps);
        printf("Compute %.3f ms/token, staging %.3f ms/token, all %.3f ms/token\n",
               total * 1e3 / reps, 0.0, total * 1e3 / reps);
        printf("Output checksum %.10g | first four %.6g %.6g %.6g %.6g\n",
               checksum(y[0], H, "Non-finite fused output"), y[0][0], y[0][1], y[0][2], y[0][3]);
    } else if (compare) {
        /* alternating-order warmup, excluded from the measurements (:714-719) */
        for (int i = 0; i < 4; ++i) {
            const int m = (i == 0 || i == 3) ? ATTENTION_STANDARD : ATTENTION_FLASH;
            (void)run_layer(l, x, kc, vc, ctx, out[m], (attention_method_t)m, NULL, NULL, NULL);
        }
        for (int r = 0; r < reps; ++r)
            for (int j = 0; j < 2; ++j) {
                const int m = (r & 1) == 0 ? j : 1 - j;
                add_phase(&sums[m], run_layer(l, x, kc, vc, ctx, out[m], (attention_method_t)m,
                                              NULL, att[m], q8[m]));
            }
        for (int i = 0; i < 2; ++i)
            hip_check(hipMemcpy(y[i], out[i], (size_t)H * sizeof(float), hipMemcpyDeviceToHost),
                      "copy");
        report_compare(&sums[0], &sums[1], l, shape_name, ctx, reps, y[0], y[1], att[0], att[1],
                       q8[0], q8[1]);
    } else {
        for (int r = 0; r < reps; ++r)
            add_phase(&sums[0], run_layer(l, x, kc, vc, ctx, out[0], selected, NULL, NULL, NULL));
        hip_check(hipMemcpy(y[0], out[0], (size_t)H * sizeof(float), hipMemcpyDeviceToHost),
                  "copy");
        report(&sums[0], l, shape_name, ctx, reps, y[0], selected);
    }
    for (int i = 0; i < 2; ++i) {
        free(y[i]);
        free(att[i]);
        free(q8[i]);
        (void)hipFree(out[i]);
    }
    (void)hipFree(x);
    (void)hipFree(kc);
    (void)hipFree(vc);
    free(input);
    free(kh);
    free(vh);
    free_layer(l);
    return 0;
}
