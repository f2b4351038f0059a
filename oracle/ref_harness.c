/*
 * ref_harness.c -- builds the reference's OWN portable scalar path into
 * oracle/_ref/libsi_ref.so so the oracle can be checked against it.
 *
 * TEST INFRASTRUCTURE ONLY.  The reference source is not copied: it is
 * compiled where it lies (-I /root/reference), with the reference's flags
 * (Makefile:7, :21: -O2 -std=c11 -ffp-contract=off -DUSE_RVV=0), using the
 * reference's own reuse idiom of renaming main and including the single
 * translation unit (verify_fused_projections.c:17-19).  The wrappers below
 * only give the reference's static functions exported names.
 *
 * The reference fixes its shapes at compile time (defines.h:16-25: hidden
 * 1536, 12 q-heads, 2 kv-heads, head_dim 128), so shape-dependent functions
 * are checked at that shape only; quantize/dot/matvec/f16 take sizes.
 */
#define main si_reference_cli_main_unused
#include "qwen_one_layer.c"
#undef main

int si_ref_hidden(void) { return HIDDEN; }
int si_ref_qheads(void) { return QHEADS; }
int si_ref_kvheads(void) { return KVHEADS; }
int si_ref_hdim(void) { return HDIM; }

float si_ref_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t si_ref_f32_to_f16(float x) { return f32_to_f16(x); }

void si_ref_f32_to_f16_array(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = f32_to_f16(src[i]);
}
void si_ref_f16_to_f32_array(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = f16_to_f32(src[i]);
}

void si_ref_rng_seed(uint32_t s) { rng_state = s; }
float si_ref_random_float(void) { return random_float(); }
void si_ref_fill_kv_history(uint16_t *kc, uint16_t *vc, int context) {
    fill_kv_history(kc, vc, context);
}

void si_ref_quantize_q8(const float *src, block_q8_0 *dst, int count) {
    quantize_q8(src, dst, count);
}
int32_t si_ref_dot_32_q4q8(const uint8_t *w, const int8_t *a) { return dot_32_q4q8(w, a); }
void si_ref_matvec_q4q8(const uint8_t *w, const block_q8_0 *x, int inputs,
                        int outputs, const float *bias, float *out) {
    matvec_q4q8(w, x, inputs, outputs, bias, out);
}
void si_ref_rmsnorm(const float *in, const float *w, float *out) { rmsnorm(in, w, out); }
void si_ref_rope(float *heads, int nheads, int position) { rope(heads, nheads, position); }
void si_ref_attention_flash(const float *q, const uint16_t *kc, const uint16_t *vc,
                            int context, float *out) {
    attention_flash(q, kc, vc, context, out);
}
void si_ref_attention_standard(const float *q, const uint16_t *kc, const uint16_t *vc,
                               int context, float *out, float *scores) {
    attention_standard(q, kc, vc, context, out, scores);
}

/* run_layer (qwen_one_layer.c:237-281) with the layer passed as pointers. */
void si_ref_run_layer(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv,
                      const uint8_t *wo, const float *norm, const float *bq,
                      const float *bk, const float *bv, const float *x,
                      uint16_t *kc, uint16_t *vc, int context, float *out,
                      int method, float *scores, float *attn_copy,
                      block_q8_0 *q8_copy) {
    layer_t l;
    l.wq = (uint8_t *)wq; l.wk = (uint8_t *)wk; l.wv = (uint8_t *)wv; l.wo = (uint8_t *)wo;
    l.norm = (float *)norm; l.bq = (float *)bq; l.bk = (float *)bk; l.bv = (float *)bv;
    (void)run_layer(&l, x, kc, vc, context, out, (attention_method_t)method,
                    scores, attn_copy, q8_copy);
}

/* The column-SoA path (fused_layer.h), portable build. */
void si_ref_fused_column_matvec(const uint8_t *tile, const block_q8_0 *x, int nblocks,
                                const float *bias_lo, const float *bias_hi, float *out,
                                int add) {
    fused_column_matvec(tile, x, nblocks, bias_lo, bias_hi, out, add);
}
void si_ref_fused_attention_pair(const float *qpair, const uint16_t *kc, const uint16_t *vc,
                                 int context, int group, float *opair) {
    fused_attention_pair(qpair, kc, vc, context, group, opair);
}
/* run_layer_fused (register_fusion.h:344-411): in the portable build it is
 * run_layer_legacy_fused (fused_layer.h:397-455) over q/kv/o column-SoA
 * tiles held in memory (no TCM). */
void si_ref_run_layer_fused(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv,
                            const uint8_t *wo, const float *norm, const float *bq,
                            const float *bk, const float *bv, const uint8_t *qt,
                            const uint8_t *kvt, const uint8_t *ot, const float *x, uint16_t *kc,
                            uint16_t *vc, int context, float *out, float *attn_capture,
                            block_q8_0 *q8_capture) {
    layer_t l;
    l.wq = (uint8_t *)wq; l.wk = (uint8_t *)wk; l.wv = (uint8_t *)wv; l.wo = (uint8_t *)wo;
    l.norm = (float *)norm; l.bq = (float *)bq; l.bk = (float *)bk; l.bv = (float *)bv;
    fused_weights_t fw;
    memset(&fw, 0, sizeof fw);
    fw.q = (uint8_t *)qt; fw.kv = (uint8_t *)kvt; fw.o = (uint8_t *)ot;
    fw.tcm_fd = -1;
    (void)run_layer_fused(&l, &fw, x, kc, vc, context, out, attn_capture, q8_capture);
}
