/*
 * si_host.h -- C11 host mirror of the reference's layer and kernel entry
 * points, running on the MI355X through include/si_abi.h.
 *
 * Same names, argument meaning and error behaviour as the reference:
 *   - run_layer           qwen_one_layer.c:237-281
 *   - run_layer_fused     register_fusion.h:344-411 (same math on the GPU)
 *   - run_layer_legacy_fused, attention_wo_fused, fused_attention_pair,
 *     fused_column_matvec    fused_layer.h:169-455 (column-SoA tiles)
 *   - fused_weights_load / fused_weights_free  fused_layer.h:131-146
 *   - pf_run_batch        prefill_weight_stationary.h:183-311
 *   - attention_compute   attention_kernels.h:166-173
 *   - attention_flash     attention_kernels.h:80-164
 *   - matvec_q4q8         qwen_one_layer.c:148-162
 *   - rmsnorm, rope       qwen_one_layer.c:164-183
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
 *   - functions whose size the reference takes from defines.h (rmsnorm,
 *     rope, the pair attention) take the loaded layer, whose runtime shape,
 *     RoPE tables and stream they use;
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
    float *rope_cos, *rope_sin;  /* device [max_pos][hdim/2] (si_rope_table) */
    float *norm, *bq, *bk, *bv;  /* device copies (NULL = identity / zero), for
                                    the column-SoA path */
} si_model_t;

/* fused_layer.h:60-66: the column-SoA weights repack_weights.py writes
 * (q.colsoa, kv.colsoa, o.colsoa), on the device, plus the device scratch
 * of the legacy fused path.  There is no scratchpad (TCM) on the GPU.  The
 * layout needs hdim 128 (a tile is one query-head pair, or one KV group's
 * 128 K and 128 V rows), an even number of query heads per KV group and
 * hidden a multiple of 256 (W_O output tiles); si_colsoa_bytes is 0 for
 * other shapes. */
typedef struct {
    uint8_t *q, *kv, *o;
    size_t q_bytes, kv_bytes, o_bytes;
    float *normed, *kvpair, *qpair, *opair;
    block_q8_0 *inq8, *oq;
} fused_weights_t;

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

/* register_fusion.h:344-411: identical result contract to run_layer, run by
 * the fused decode kernels on the layer's own repacked weights (the GPU's
 * counterpart of the register-resident path).  fw (the same weights as
 * column-SoA tiles) may be NULL; run_layer_legacy_fused is the path that
 * reads it. */
fused_stats_t run_layer_fused(const si_model_t *l, const fused_weights_t *fw, const float *x,
                              uint16_t *kc, uint16_t *vc, int context, float *output,
                              float *attn_capture, block_q8_0 *q8_capture);

/* fused_layer.h:397-455 on the device, over the column-SoA tiles of fw:
 * per KV group the K/V tile (+bias), RoPE of K and the fp16 append at row
 * context-1; per head pair the Q tile (+bias), RoPE, the pair's attention,
 * Q8 of its 256 values and the W_O partial added into the zeroed output.
 * Captures are HOST buffers or NULL.  Phase times are host wall-clock
 * seconds around each synchronized stage. */
fused_stats_t run_layer_legacy_fused(const si_model_t *l, const fused_weights_t *fw,
                                     const float *x, uint16_t *kc, uint16_t *vc, int context,
                                     float *output, float *attn_capture,
                                     block_q8_0 *q8_capture);

/* fused_layer.h:361-390: fused_attention_pair of qpair (device, the pair's
 * two rotated query heads), quantize_q8 of the 256 outputs, and the pair's
 * W_O tiles of fw added into output_y (device [hidden]).  The captures
 * (HOST, or NULL) receive the pair's slice at pair*256 / pair*8. */
void attention_wo_fused(const si_model_t *l, const fused_weights_t *fw, const float *qpair,
                        const uint16_t *kc, const uint16_t *vc, int context, int group, int pair,
                        float *output_y, fused_stats_t *stats, float *attention_capture,
                        block_q8_0 *quantized_capture);

/* fused_layer.h:251-355: attention of two query heads (qpair [2][hdim],
 * device) over KV group `group` of the device caches into opair. */
void fused_attention_pair(const si_model_t *l, const float *qpair, const uint16_t *kc,
                          const uint16_t *vc, int context, int group, float *opair);

/* fused_layer.h:169-245 on device buffers: one column-SoA tile of nblocks
 * groups against nblocks block_q8_0 records into output[256]; add = 0
 * starts from bias_lo/bias_hi (128 each, NULL = 0), add != 0 accumulates. */
void fused_column_matvec(const uint8_t *tile, const block_q8_0 *x, int nblocks,
                         const float *bias_lo, const float *bias_hi, float *output, int add);

/* fused_layer.h:131-139: reads q.colsoa, kv.colsoa and o.colsoa from dir
 * (exact sizes for the layer's shape) onto the device.  use_tcm must be 0:
 * there is no scratchpad to stage tiles in. */
fused_weights_t fused_weights_load(const si_model_t *l, const char *dir, int use_tcm, int block);
/* Same from column-SoA tiles in host memory. */
fused_weights_t si_fused_weights_from_host(const si_model_t *l, const uint8_t *q,
                                           const uint8_t *kv, const uint8_t *o);
void fused_weights_free(fused_weights_t *fw);

/* Bytes of q.colsoa (which 0), kv.colsoa (1) or o.colsoa (2) for a shape;
 * 0 when the shape has no column-SoA layout. */
size_t si_colsoa_bytes(const si_shape_t *s, int which);
/* repack_weights.py:55-120 in C: the three column-SoA files from the
 * row-major Q4_0 matrices of w (host memory; sizes from si_colsoa_bytes). */
void si_colsoa_repack_host(const si_shape_t *s, const si_layer_host_t *w, uint8_t *q,
                           uint8_t *kv, uint8_t *o);

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

/* qwen_one_layer.c:148-162 on device buffers: weights row-major Q4_0
 * [outputs][inputs/32], input block_q8_0 [inputs/32], bias [outputs] or
 * NULL; the reference's block order and roundings (bit-exact). */
void matvec_q4q8(const uint8_t *weights, const block_q8_0 *input, int inputs, int outputs,
                 const float *bias, float *out);

/* qwen_one_layer.c:164-169: out = rmsnorm(input) * weight (NULL = 1) over
 * the layer's hidden size, device buffers. */
void rmsnorm(const si_model_t *l, const float *input, const float *weight, float *out);

/* qwen_one_layer.c:172-183: rotates nheads heads of hdim values (device) in
 * place at `position` (0..max_pos-1), angles from the layer's tables. */
void rope(const si_model_t *l, float *heads, int nheads, int position);

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
