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
 *   - fused / soa-staged / soa-fused: run_layer_legacy_fused on the
 *     reference's column-SoA tiles (q.colsoa, kv.colsoa, o.colsoa, as
 *     repack_weights.py writes them; fused_weights_load, :650) when the
 *     weights directory holds them, or on tiles built from the synthetic
 *     weights; for a shape with no column-SoA layout (hdim 64, odd heads per
 *     group) or a directory without the files, the fused decode kernels.
 *     Summary line (:687-701); there is no scratchpad staging on the GPU, so
 *     the staged variant runs the same path;
 *   - fused-compare: staged flash vs that fused path, alternating order
 *     (report_fusion, :526-594).
 * The shape comes from SI_SHAPE (0.5b, 1.5b, 7b; default 1.5b, the
 * reference's compile-time shape, defines.h:16-25).  weights_dir holds the
 * files load_layer reads; "synthetic" generates seeded Q4_0 weights instead.
 * Times are GPU event times of each phase; fused phases read 0 and are
 * reported inside the phase they run in (include/si_host.h).
 */
#define _GNU_SOURCE
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

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
/* The synthetic layer; when fw is not NULL and the shape has a column-SoA
 * layout, also its column-SoA tiles (*have_fw = 1). */
static si_model_t *synthetic_layer(const si_shape_t *s, int max_pos, fused_weights_t *fw,
                                   int *have_fw) {
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
    if (fw && have_fw && si_colsoa_bytes(s, 0) > 0) {
        uint8_t *t[3];
        for (int i = 0; i < 3; ++i)
            if (!(t[i] = malloc(si_colsoa_bytes(s, i))))
                die("Out of memory building column-SoA tiles");
        si_colsoa_repack_host(s, &h, t[0], t[1], t[2]);
        *fw = si_fused_weights_from_host(m, t[0], t[1], t[2]);
        *have_fw = 1;
        for (int i = 0; i < 3; ++i) free(t[i]);
    }
    for (int i = 0; i < 4; ++i) free(w[i]);
    free(norm); free(bq); free(bk); free(bv);
    g_rng = saved;
    return m;
}

/* "<what> <size>" with the size in the largest binary unit up to MiB that
 * keeps it at 1 or more, two decimals past bytes (the tables' footprint
 * column). */
static void footprint(char *out, size_t n, const char *what, size_t bytes) {
    static const char *const unit[] = {"B", "KiB", "MiB"};
    double v = (double)bytes;
    int u = 0;
    while (u < 2 && v >= 1024.0) {
        v /= 1024.0;
        ++u;
    }
    if (u == 0)
        snprintf(out, n, "%s %zu B", what, bytes);
    else
        snprintf(out, n, "%s %.2f %s", what, v, unit[u]);
}

/* phase_t's nine fields in report order, so the tables and sums loop over
 * them instead of naming each one. */
static const size_t PHASE_FIELD[9] = {
    offsetof(phase_t, rms),        offsetof(phase_t, q8_input),  offsetof(phase_t, q_proj),
    offsetof(phase_t, k_proj),     offsetof(phase_t, v_proj),    offsetof(phase_t, rope_cache),
    offsetof(phase_t, attention),  offsetof(phase_t, q8_output), offsetof(phase_t, out_proj),
};

static double phase_value(const phase_t *p, int i) {
    float v;
    memcpy(&v, (const char *)p + PHASE_FIELD[i], sizeof v);
    return v;
}

static void phase_accumulate(phase_t *into, const phase_t *from) {
    for (int i = 0; i < 9; ++i) {
        float v;
        memcpy(&v, (const char *)into + PHASE_FIELD[i], sizeof v);
        v += (float)phase_value(from, i);
        memcpy((char *)into + PHASE_FIELD[i], &v, sizeof v);
    }
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
    const struct {
        const char *what;
        size_t bytes;
    } data[9] = {
        {"Norm", H * sizeof(float)},          {"Q8 buffer", H / 32 * 34},
        {"Wq Q4_0", QD * H / 32 * 18},        {"Wk Q4_0", KVD * H / 32 * 18},
        {"Wv Q4_0", KVD * H / 32 * 18},       {"New K+V", KVD * 2 * 2},
        {"KV cache", (size_t)context * KVD * 2 * 2}, {"Q8 buffer", QD / 32 * 34},
        {"Wo Q4_0", H * QD / 32 * 18},
    };
    for (int i = 0; i < 9; ++i) footprint(r->data[i], sizeof r->data[i], data[i].what, data[i].bytes);
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
    for (int i = 0; i < 9; ++i) total += t[i] = phase_value(p, i);
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
    for (int i = 0; i < 9; ++i) {
        a[i] = phase_value(st, i);
        b[i] = phase_value(fl, i);
    }
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
                          const block_q8_0 *q8_ref, const block_q8_0 *q8_fused, int H, int QD,
                          int legacy) {
    static const char *const names[9] = {"RMSNorm", "Quantize X", "Wq", "Wk", "Wv",
                                         "RoPE + KV append", "Online attention (GQA)",
                                         "Quantize O", "W_o"};
    double a[9], b[9], ta = 0.0, tb = 0.0;
    for (int i = 0; i < 9; ++i) {
        ta += a[i] = phase_value(base, i);
        tb += b[i] = phase_value(&fused->phase, i);
    }
    printf("\nQwen2 %s | STAGED FLASH vs %s | MI355X\n", shape,
           legacy ? "COLUMN-SoA FUSED (run_layer_legacy_fused)" : "FUSED DECODE KERNELS");
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
    puts(legacy ? "Fused path: the column-SoA tiles, per head pair, W_O accumulated per pair.\n"
                : "On the GPU the staged flash layer already runs the fused decode kernels.\n");
}

/* Whether dir holds the three column-SoA tile files fused_weights_load
 * reads. */
static int has_colsoa_files(const char *dir) {
    static const char *const names[3] = {"q.colsoa", "kv.colsoa", "o.colsoa"};
    char path[4096];
    for (int i = 0; i < 3; ++i) {
        if (snprintf(path, sizeof path, "%s/%s", dir, names[i]) >= (int)sizeof path) return 0;
        if (access(path, R_OK) != 0) return 0;
    }
    return 1;
}

/* ---- command line ---------------------------------------------------- */

typedef enum { RUN_SINGLE, RUN_COMPARE, RUN_FUSED, RUN_FUSED_COMPARE } run_kind_t;

/* The reference's modes (qwen_one_layer.c:610-629).  On the GPU the staged
 * and register-fused variants run the same fused path (no scratchpad). */
static const struct {
    const char *name;
    run_kind_t kind;
    attention_method_t method;
    const char *banner;
} MODES[] = {
    {"standard", RUN_SINGLE, ATTENTION_STANDARD, NULL},
    {"flash", RUN_SINGLE, ATTENTION_FLASH, NULL},
    {"reference", RUN_SINGLE, ATTENTION_FLASH, NULL},
    {"compare", RUN_COMPARE, ATTENTION_FLASH, NULL},
    {"fused", RUN_FUSED, ATTENTION_FLASH, "REGISTER FUSED"},
    {"soa-fused", RUN_FUSED, ATTENTION_FLASH, "REGISTER FUSED"},
    {"soa-staged", RUN_FUSED, ATTENTION_FLASH, "SOA STAGED"},
    {"fused-compare", RUN_FUSED_COMPARE, ATTENTION_FLASH, NULL},
};
#define NMODES ((int)(sizeof MODES / sizeof MODES[0]))

typedef struct {
    const char *source; /* weights directory or "synthetic" */
    int context, repeat, mode;
} cli_t;

/* A decimal argument; `complaint` when characters follow the number. */
static long decimal_arg(const char *text, const char *complaint) {
    char *rest = NULL;
    const long v = strtol(text, &rest, 10);
    if (*rest) die(complaint);
    return v;
}

static cli_t parse_cli(int argc, char **argv) {
    if (argc < 2 || argc > 5) {
        fprintf(stderr,
                "Usage: %s <weights_directory|synthetic> [context=256] [repeat=1] "
                "[standard|flash|compare|fused|fused-compare|reference|soa-staged|soa-fused]\n"
                "       (shape from SI_SHAPE: 0.5b, 1.5b or 7b; default 1.5b)\n",
                argv[0]);
        exit(2);
    }
    cli_t c = {argv[1], 256, 1, -1};
    const long context = argc > 2 ? decimal_arg(argv[2], "Invalid context argument") : 256;
    const long repeat = argc > 3 ? decimal_arg(argv[3], "Invalid repeat argument") : 1;
    if (context < 1 || context > 32768 || repeat < 1 || repeat > 100000)
        die("Context must be 1..32768 and repeat 1..100000");
    c.context = (int)context;
    c.repeat = (int)repeat;
    const char *mode = argc > 4 ? argv[4] : "compare";
    for (int i = 0; i < NMODES && c.mode < 0; ++i)
        if (!strcmp(MODES[i].name, mode)) c.mode = i;
    if (c.mode < 0)
        die("Attention mode must be standard, flash, compare, fused, fused-compare, reference, "
            "soa-staged or soa-fused");
    return c;
}

/* Everything one layer call needs; slot 0/1 name the two paths a
 * comparison alternates (their own outputs and captures). */
typedef struct {
    const si_model_t *l;
    float *x;
    uint16_t *kc, *vc;
    int context;
    float *out[2];              /* device */
    float *att[2];              /* host captures, or NULL */
    block_q8_0 *q8[2];
    attention_method_t method[2];
    int fused[2];               /* slot runs the fused path */
    const fused_weights_t *fw;  /* column-SoA tiles: run_layer_legacy_fused; NULL: run_layer_fused */
} bench_t;

static phase_t run_slot(const bench_t *b, int slot) {
    if (b->fused[slot] && b->fw)
        return run_layer_legacy_fused(b->l, b->fw, b->x, b->kc, b->vc, b->context,
                                      b->out[slot], b->att[slot], b->q8[slot])
            .phase;
    if (b->fused[slot])
        return run_layer_fused(b->l, NULL, b->x, b->kc, b->vc, b->context, b->out[slot],
                               b->att[slot], b->q8[slot])
            .phase;
    return run_layer(b->l, b->x, b->kc, b->vc, b->context, b->out[slot], b->method[slot], NULL,
                     b->att[slot], b->q8[slot]);
}

/* `rounds` rounds over the first `nslots` slots, the slot order reversed on
 * every other round so neither path always runs first; phases are summed
 * per slot into sums unless it is NULL (warm-up). */
static void interleave(const bench_t *b, int nslots, int rounds, phase_t *sums) {
    for (int r = 0; r < rounds; ++r)
        for (int k = 0; k < nslots; ++k) {
            const int slot = (r & 1) ? nslots - 1 - k : k;
            const phase_t p = run_slot(b, slot);
            if (sums) phase_accumulate(&sums[slot], &p);
        }
}

static void to_host(float *dst, const float *src, int n) {
    hip_check(hipMemcpy(dst, src, (size_t)n * sizeof(float), hipMemcpyDeviceToHost), "copy");
}

int main(int argc, char **argv) {
    const cli_t cli = parse_cli(argc, argv);
    const char *shape_name = getenv("SI_SHAPE") ? getenv("SI_SHAPE") : "1.5b";
    si_shape_t shape;
    if (!shape_named(shape_name, &shape)) die("SI_SHAPE must be 0.5b, 1.5b or 7b");
    const int ctx = cli.context, reps = cli.repeat;
    const run_kind_t kind = MODES[cli.mode].kind;
    const int fused_kind = kind == RUN_FUSED || kind == RUN_FUSED_COMPARE;
    const int synthetic = !strcmp(cli.source, "synthetic");
    fused_weights_t fw;
    int have_fw = 0;
    memset(&fw, 0, sizeof fw);
    si_model_t *l = synthetic ? synthetic_layer(&shape, ctx, fused_kind ? &fw : NULL, &have_fw)
                              : load_layer(&shape, cli.source, 1, ctx);
    if (fused_kind && !synthetic && si_colsoa_bytes(&shape, 0) > 0 &&
        has_colsoa_files(cli.source)) {
        /* qwen_one_layer.c:647-650: FUSED_TCM / TCM_BLOCK as the reference
         * reads them (a TCM request is refused: the GPU has no scratchpad) */
        const char *tcm = getenv("FUSED_TCM"), *blk = getenv("TCM_BLOCK");
        fw = fused_weights_load(l, cli.source, tcm && atoi(tcm) != 0, blk ? atoi(blk) : 0);
        have_fw = 1;
    }
    const int H = shape.hidden, QD = shape.qheads * shape.hdim, KVD = shape.kvheads * shape.hdim;
    const size_t kv_elems = (size_t)ctx * KVD;

    /* the synthetic token, then the cache history, from the reference's
     * input stream in its order (qwen_one_layer.c:641-642) */
    float *token = malloc((size_t)H * sizeof(float));
    uint16_t *hist[2] = {calloc(kv_elems, 2), calloc(kv_elems, 2)};
    if (!token || !hist[0] || !hist[1]) die("Out of memory creating synthetic inputs");
    for (int i = 0; i < H; ++i) token[i] = next_uniform();
    const size_t hist_elems = kv_elems - KVD; /* rows 0..context-2 */
    for (size_t i = 0; i < hist_elems; ++i) {
        hist[0][i] = to_half(next_uniform() * 0.25f);
        hist[1][i] = to_half(next_uniform() * 0.25f);
    }

    bench_t b;
    memset(&b, 0, sizeof b);
    b.l = l;
    b.context = ctx;
    b.fw = have_fw ? &fw : NULL;
    hip_check(hipMalloc((void **)&b.x, (size_t)H * sizeof(float)), "hipMalloc");
    hip_check(hipMalloc((void **)&b.kc, kv_elems * 2), "hipMalloc");
    hip_check(hipMalloc((void **)&b.vc, kv_elems * 2), "hipMalloc");
    hip_check(hipMemcpy(b.x, token, (size_t)H * sizeof(float), hipMemcpyHostToDevice), "copy");
    hip_check(hipMemcpy(b.kc, hist[0], kv_elems * 2, hipMemcpyHostToDevice), "copy");
    hip_check(hipMemcpy(b.vc, hist[1], kv_elems * 2, hipMemcpyHostToDevice), "copy");
    float *y[2], *att[2];
    block_q8_0 *q8[2];
    for (int s = 0; s < 2; ++s) {
        hip_check(hipMalloc((void **)&b.out[s], (size_t)H * sizeof(float)), "hipMalloc");
        y[s] = malloc((size_t)H * sizeof(float));
        att[s] = malloc((size_t)QD * sizeof(float));
        q8[s] = malloc((size_t)(QD / 32) * sizeof(block_q8_0));
        if (!y[s] || !att[s] || !q8[s]) die("Out of memory for comparison buffers");
    }

    phase_t sums[2];
    memset(sums, 0, sizeof sums);
    if (kind == RUN_COMPARE || kind == RUN_FUSED_COMPARE) {
        /* slot 0: the staged path (standard, or flash against the fused
         * kernels); slot 1: flash or fused */
        b.method[0] = kind == RUN_COMPARE ? ATTENTION_STANDARD : ATTENTION_FLASH;
        b.method[1] = ATTENTION_FLASH;
        b.fused[1] = kind == RUN_FUSED_COMPARE;
        interleave(&b, 2, 2, NULL); /* warm-up, untimed */
        if (kind == RUN_COMPARE) {
            b.att[0] = att[0], b.att[1] = att[1], b.q8[0] = q8[0], b.q8[1] = q8[1];
            interleave(&b, 2, reps, sums);
        } else {
            interleave(&b, 2, reps, sums); /* timed without captures */
            b.att[0] = att[0], b.att[1] = att[1], b.q8[0] = q8[0], b.q8[1] = q8[1];
            interleave(&b, 2, 1, NULL);    /* one captured replay of each */
        }
        to_host(y[0], b.out[0], H);
        to_host(y[1], b.out[1], H);
        if (kind == RUN_COMPARE) {
            report_compare(&sums[0], &sums[1], l, shape_name, ctx, reps, y[0], y[1], att[0],
                           att[1], q8[0], q8[1]);
        } else {
            fused_stats_t fs;
            memset(&fs, 0, sizeof fs);
            fs.phase = sums[1];
            report_fusion(&sums[0], &fs, shape_name, ctx, reps, y[0], y[1], att[0], att[1],
                          q8[0], q8[1], H, QD, have_fw);
        }
    } else {
        b.method[0] = MODES[cli.mode].method;
        b.fused[0] = kind == RUN_FUSED;
        interleave(&b, 1, reps, sums);
        to_host(y[0], b.out[0], H);
        if (kind == RUN_SINGLE) {
            report(&sums[0], l, shape_name, ctx, reps, y[0], b.method[0]);
        } else {
            double total = 0.0;
            for (int i = 0; i < 9; ++i) total += phase_value(&sums[0], i);
            printf("%s one-token | context=%d repeats=%d | MI355X %s\n",
                   MODES[cli.mode].banner, ctx, reps,
                   have_fw ? "column-SoA tiles (run_layer_legacy_fused)"
                           : "fused decode kernels");
            printf("Compute %.3f ms/token, staging %.3f ms/token, all %.3f ms/token\n",
                   total * 1e3 / reps, 0.0, total * 1e3 / reps);
            printf("Output checksum %.10g | first four %.6g %.6g %.6g %.6g\n",
                   checksum(y[0], H, "Non-finite fused output"), y[0][0], y[0][1], y[0][2],
                   y[0][3]);
        }
    }
    for (int s = 0; s < 2; ++s) {
        free(y[s]);
        free(att[s]);
        free(q8[s]);
        (void)hipFree(b.out[s]);
    }
    if (have_fw) fused_weights_free(&fw);
    (void)hipFree(b.x);
    (void)hipFree(b.kc);
    (void)hipFree(b.vc);
    free(token);
    free(hist[0]);
    free(hist[1]);
    free_layer(l);
    return 0;
}
