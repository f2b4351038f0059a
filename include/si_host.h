/*
 * si_host.h -- C11 host mirror of the reference's layer and kernel entry
 * points, running on the MI355X through include/si_abi.h.
 *
 * Same names, argument meaning and error behaviour as the reference:
 *   - run_layer           qwen_one_layer.c:237-281
 *   - run_layer_fused     register_fusion.h:344-411 (same math on the GPU)
 *   - pf_run_batch        prefill_weight_stationary.h:183-311
 *   - attention_compute   attention_kernels.h:166-173
 *   - attention_flash     attention_kernels.h:80-164
 *   - quantize_q8         qwen_one_layer.c:98-116
 *   - load_layer / free_layer  qwen_one_layer.c:188-226
 * Differences, all forced by the device boundary:
 *   - shapes are runtime (si_shape_t) and travel inside si_model_t, which
 *     replaces the compile-time macros of defines.h:16-25;
 *   - activations, KV caches and outputs are DEVICE pointers (the caller
 *     owns them, as in the reference); weights are uploaded once by
 *     load_layer;
 *   - errors still never return: they print and exit(1) like die()
 *     (qwen_one_layer.c:26-28);
 *   - timings (phase_t) are GPU event times in seconds.  The decode kernels
 *     fuse RMSNorm + Q8 into the Q/K/V projection, RoPE + K/V append into
 *     attention and the attention output's Q8 into W_O: a fused phase is
 *     reported under the projection or attention it runs in, the others
 *     read 0.  The fused Q/K/V time is apportioned by output rows, as
 *     fused_layer.h:424-426 splits its fused K/V time.
 */
#ifndef SI_HOST_H
#define SI_HOST_H

#include <stdint.h>

#include "si_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* defines.h:27-28 */
typedef struct { uint16_t d; int8_t qs[32]; } block_q8_0;

/* defines.h:35-37 */
typedef struct {
    float rms, q8_input, q_proj, k_proj, v_proj, rope_cache, attention, q8_output, out_proj;
} phase_t;

/* fused_layer.h:68-71 */
typedef struct {
    phase_t phase;
    double tcm_stage; /* no scratchpad staging on the GPU: always 0 */
} fused_stats_t;

/* attention_kernels.h:24-27 */
typedef enum { ATTENTION_STANDARD = 0, ATTENTION_FLASH = 1 } attention_method_t;

/* A loaded layer: shape + device weights + stream (replaces layer_t and
 * fused_weights_t, defines.h:30-33, fused_layer.h:60-66). */
typedef struct {
    si_shape_t shape;
    si_layer_t *layer;
    void *stream;      /* hipStream_t; NULL = default stream */
    int max_tokens;
    int max_pos;
    void *attn_ws;     /* device workspace for attention_compute/_flash */
    size_t attn_ws_bytes;
} si_model_t;

/* load_layer (qwen_one_layer.c:210-221): reads q.q4_0 k.q4_0 v.q4_0 o.q4_0
 * and the optional norm.f32 q_bias.f32 k_bias.f32 v_bias.f32 from dir with
 * the reference's exact size checks, plus the build-defined FFN files
 * post_norm.f32 gate.q4_0 up.q4_0 down.q4_0 when present. */
si_model_t *load_layer(const si_shape_t *shape, const char *dir, int max_tokens, int max_pos);

/* Same, from host tensors already in memory. */
si_model_t *si_model_from_host(const si_shape_t *shape, const si_layer_host_t *w,
                               int max_tokens, int max_pos);
void free_layer(si_model_t *m);

/* qwen_one_layer.c:237-281 with device x/kc/vc/output.  ATTENTION_FLASH runs
 * the fused streaming kernels; ATTENTION_STANDARD the staged order with the
 * three-stage textbook attention (SI_LAYER_ATTN_STANDARD), whose scores live
 * in the layer's own device buffer, so scores is unused.  attn_copy (fp32 [qheads*hdim])
 * and q8_copy (block_q8_0 [qheads*hdim/32]) are HOST buffers or NULL,
 * filled after the timed work as the reference's captures are (:277-279). */
phase_t run_layer(const si_model_t *l, const float *x, uint16_t *kc, uint16_t *vc,
                  int context, float *output, attention_method_t method, float *scores,
                  float *attn_copy, block_q8_0 *q8_copy);

/* register_fusion.h:344-411: identical result contract to run_layer. */
fused_stats_t run_layer_fused(const si_model_t *l, const float *x, uint16_t *kc,
                              uint16_t *vc, int context, float *output, float *attn_capture,
                              block_q8_0 *q8_capture);

/* Full build-defined Qwen2 layer (attention + residual + post-norm + SwiGLU
 * FFN + residual) for one token. */
phase_t run_layer_full(const si_model_t *l, const float *x, uint16_t *kc, uint16_t *vc,
                       int context, float *output);

/* pf_run_batch (prefill_weight_stationary.h:183-311): x [ntok][hidden]
 * device, K/V appended at prefix..prefix+ntok-1, output [ntok][hidden].
 * full != 0 runs the build-defined full layer per token. */
void pf_run_batch(const si_model_t *l, const float *x, int ntok, int prefix, uint16_t *kc,
                  uint16_t *vc, float *output, int full);

/* attention_kernels.h:80-164 / :166-173 for one token (device q/kc/vc/out;
 * score_workspace: device fp32 [qheads][context], used by ATTENTION_STANDARD). */
void attention_flash(const si_model_t *l, const float *q, const uint16_t *kc,
                     const uint16_t *vc, int context, float *out);
void attention_compute(const si_model_t *l, attention_method_t method, const float *q,
                       const uint16_t *kc, const uint16_t *vc, int context, float *out,
                       float *score_workspace);

/* qwen_one_layer.c:98-116 on device buffers (dst: block_q8_0 records). */
void quantize_q8(const float *src, block_q8_0 *dst, int count);

/* ------------------------------------------------------------------ */
/* Paged KV bookkeeping and a multi-layer decode stack (si_kvpages.c). */
/* No counterpart in the reference (one layer, one contiguous cache,   */
/* qwen_one_layer.c:237-281): the step after a single layer.           */
/* ------------------------------------------------------------------ */

/* A pool of npages pages of page_size positions (a power of two) and the
 * page lists of up to max_seqs sequences of up to max_pages pages each.
 * Free pages are handed out lowest id first and reused after
 * si_kv_seq_free.  Misuse (unknown sequence, shrinking) dies. */
typedef struct si_kv_pages si_kv_pages_t;
si_kv_pages_t *si_kv_pages_create(int npages, int page_size, int max_seqs, int max_pages);
void si_kv_pages_destroy(si_kv_pages_t *p);
/* a new empty sequence: its id, or -1 when every slot is taken */
int si_kv_seq_add(si_kv_pages_t *p);
/* pages for len positions: 0, or -1 (nothing taken) when the pool or the
 * sequence's max_pages cannot hold them */
int si_kv_seq_grow(si_kv_pages_t *p, int seq, int len);
void si_kv_seq_free(si_kv_pages_t *p, int seq);
int si_kv_seq_len(const si_kv_pages_t *p, int seq);
int si_kv_pages_free(const si_kv_pages_t *p);
/* host [max_seqs][max_pages] page ids by sequence id (unused entries 0) */
const int *si_kv_page_table(const si_kv_pages_t *p);

/* nlayers full layers (or attention sublayers with ffn 0) sharing one
 * workspace, each with its own K and V page pool (npages pages of
 * page_size rows), one page table for all of them. */
typedef struct si_stack si_stack_t;
si_stack_t *si_stack_create(const si_shape_t *s, const si_layer_host_t *layers, int nlayers,
                            int max_seqs, int max_ctx, int npages, int page_size);
void si_stack_destroy(si_stack_t *st);
si_kv_pages_t *si_stack_pages(si_stack_t *st);
uint16_t *si_stack_k_pool(si_stack_t *st, int layer);
uint16_t *si_stack_v_pool(si_stack_t *st, int layer);
si_layer_t *si_stack_layer(si_stack_t *st, int layer);
const int *si_stack_dev_table(const si_stack_t *st);
const int *si_stack_dev_ctx(const si_stack_t *st);
/* sequences of the last successful si_stack_prepare (0: none, or it failed) */
int si_stack_nseq(const si_stack_t *st);
/* Grows each of the nseq distinct sequences seqs[] by one position (the
 * token about to be decoded) and uploads their page lists and contexts in
 * batch order (synchronous copies, after waiting for the stream of the
 * previous si_stack_decode, whose kernels read them).  -1 when the pool is exhausted (the
 * lengths are left as before; pages already taken stay with their
 * sequences, and si_stack_decode dies until a later prepare succeeds),
 * else 0. */
int si_stack_prepare(si_stack_t *st, const int *seqs, int nseq);
/* x [nseq][hidden] (device) through every layer -> out [nseq][hidden]: the
 * residual stream of a decode step; kernel launches only (capturable). */
void si_stack_decode(si_stack_t *st, const float *x, float *out, int flags, void *stream);

/* Offline weight preparation (host memory): ggml's Q4_0 rule, the format
 * extract_weights.py copies from GGUF.  Per 32 values: d = m/-8 for the
 * signed value m of largest magnitude, nibble = min(15, trunc(x/d + 8.5)). */
void si_quantize_q4_0_host(const float *src, uint8_t *dst, int count);

#ifdef __cplusplus
}
#endif
#endif
