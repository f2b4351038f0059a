/*
 * si_oracle.h -- CPU parity oracle for the one-Qwen-layer hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load this library, and only as the checker or
 * as the timed CPU baseline.  The product path (simple-inference_amd/) never
 * links or calls it.
 *
 * It restates the reference's portable scalar C path (USE_RVV=0) with the
 * compile-time shape macros turned into a runtime shape, following the same
 * operation order so that results are bit-identical to the reference at the
 * shapes the reference compiles for (pinned in tests against oracle/_ref,
 * the reference's own sources compiled unchanged).  Each function names the
 * reference lines it restates.
 *
 * Functions that have no counterpart in the reference (the SwiGLU FFN, the
 * residual/post-attention norm composition and the Q4_0 weight quantizer)
 * are build-defined; they are pinned by closed-form and brute-force tests,
 * not by the reference.
 */
#ifndef SI_ORACLE_H
#define SI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_QK 32
#define OR_Q4_BYTES 18 /* defines.h:22 */
#define OR_Q8_BYTES 34 /* defines.h:23 */

/* defines.h:27-28: one Q8_0 block, fp16 scale bits then 32 int8 values. */
typedef struct {
    uint16_t d;
    int8_t qs[OR_QK];
} or_block_q8_0;

/* defines.h:16-25 as runtime values. */
typedef struct {
    int hidden;   /* HIDDEN */
    int qheads;   /* QHEADS */
    int kvheads;  /* KVHEADS */
    int hdim;     /* HDIM */
    int ffn;      /* FFN width (build-defined; 0 = attention sublayer only) */
    float rope_base; /* ROPE_BASE */
    float rms_eps;   /* RMS_EPS */
} or_shape_t;

/* defines.h:30-33 (layer_t) plus the build-defined FFN tensors.
 * Q4_0 matrices are the reference's row-major [rows][K/32] 18-byte blocks.
 * NULL norm = identity gain, NULL bias = zero (qwen_one_layer.c:168,:154). */
typedef struct {
    const uint8_t *wq, *wk, *wv, *wo;
    const float *norm, *bq, *bk, *bv;
    const float *post_norm;                 /* build-defined */
    const uint8_t *wgate, *wup, *wdown;     /* build-defined */
} or_layer_t;

/* Optional intermediate captures of one decoded token (any may be NULL). */
typedef struct {
    float *normed;        /* [hidden]                     */
    or_block_q8_0 *xq;    /* [hidden/32]                  */
    float *q;             /* [qheads*hdim] after RoPE     */
    float *k;             /* [kvheads*hdim] after RoPE    */
    float *v;             /* [kvheads*hdim]               */
    float *attn;          /* [qheads*hdim]                */
    or_block_q8_0 *attq;  /* [qheads*hdim/32]             */
    float *attn_out;      /* [hidden]  W_O output         */
    float *h;             /* [hidden]  residual 1         */
    float *normed2;       /* [hidden]                     */
    or_block_q8_0 *xq2;   /* [hidden/32]                  */
    float *gate, *up;     /* [ffn]                        */
    float *act;           /* [ffn]  silu(gate)*up         */
    or_block_q8_0 *actq;  /* [ffn/32]                     */
    float *ffn_out;       /* [hidden]                     */
} or_capture_t;

enum { OR_ATTENTION_STANDARD = 0, OR_ATTENTION_FLASH = 1 }; /* attention_kernels.h:24-27 */

/* ---- numerics (qwen_one_layer.c:42-86) ---- */
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float x);
void or_f32_to_f16_array(const float *src, uint16_t *dst, size_t n);
void or_f16_to_f32_array(const uint16_t *src, float *dst, size_t n);

/* ---- reference RNG (qwen_one_layer.c:88-96) ---- */
void or_rng_seed(uint32_t seed);
uint32_t or_rng_u32(void);
float or_rng_float(void);
void or_rng_fill(float *dst, size_t n, float scale);

/* ---- kernels ---- */
void or_quantize_q8(const float *src, or_block_q8_0 *dst, int count);   /* :98-116  */
int32_t or_dot_32_q4q8(const uint8_t *w, const int8_t *a);               /* :118-146 */
void or_block_dots(const uint8_t *w, const or_block_q8_0 *x, int inputs,
                   int outputs, int32_t *dots);                          /* per-block :154-157 */
void or_matvec_q4q8(const uint8_t *w, const or_block_q8_0 *x, int inputs,
                    int outputs, const float *bias, float *out);         /* :148-162 */
void or_rmsnorm(const float *in, const float *w, float *out, int n, float eps); /* :164-169 */
void or_rope(float *heads, int nheads, int hdim, int position, float base);     /* :172-183 */
void or_rope_table(int pos0, int npos, int hdim, float base, float *cos_out, float *sin_out);
void or_attention_flash(const or_shape_t *s, const float *q, const uint16_t *kc,
                        const uint16_t *vc, int context, float *out);   /* attention_kernels.h:80-164 */
void or_attention_standard(const or_shape_t *s, const float *q, const uint16_t *kc,
                           const uint16_t *vc, int context, float *out,
                           float *scores);                              /* attention_kernels.h:33-78 */
void or_swiglu(const float *gate, const float *up, float *out, int n);  /* build-defined */

/* qwen_one_layer.c:237-281: attention sublayer, output = W_O . Q8(attn). */
void or_run_layer(const or_shape_t *s, const or_layer_t *l, const float *x,
                  uint16_t *kc, uint16_t *vc, int context, float *out,
                  int method, float *scores, or_capture_t *cap);

/* Build-defined full layer: attention sublayer, residual, post-attention
 * RMSNorm, SwiGLU FFN, residual.  Needs s->ffn > 0. */
void or_layer_decode(const or_shape_t *s, const or_layer_t *l, const float *x,
                     uint16_t *kc, uint16_t *vc, int context, float *out,
                     or_capture_t *cap);

/* Causal prefill contract (prefill_weight_stationary.h:173-311): K/V of all
 * ntok tokens first (rows prefix..prefix+ntok-1), then token t attends with
 * context prefix+t+1.  Full-layer outputs are produced only for the rows
 * listed (rows==NULL: all rows, out is [ntok][hidden]; else out is
 * [nrows][hidden]).  full==0 runs the attention sublayer only. */
void or_layer_prefill(const or_shape_t *s, const or_layer_t *l, const float *x,
                      int ntok, int prefix, uint16_t *kc, uint16_t *vc,
                      const int *rows, int nrows, int full, float *out);

/* ggml Q4_0 quantizer (quantize_row_q4_0_ref), build-side weight preparation. */
/* ---- column-SoA tiles and the legacy fused path (hdim 128 shapes) ---- */
size_t or_colsoa_bytes(const or_shape_t *s, int which);   /* 0 q, 1 kv, 2 o */
void or_colsoa_repack(const or_shape_t *s, const uint8_t *wq, const uint8_t *wk,
                      const uint8_t *wv, const uint8_t *wo, uint8_t *q, uint8_t *kv,
                      uint8_t *o);                            /* repack_weights.py:55-120 */
void or_fused_column_matvec(const uint8_t *tile, const or_block_q8_0 *x, int nblocks,
                            const float *bias_lo, const float *bias_hi, float *out,
                            int add);                         /* fused_layer.h:169-245 */
void or_attention_pair(const or_shape_t *s, const float *qpair, const uint16_t *kc,
                       const uint16_t *vc, int context, int group,
                       float *opair);                         /* fused_layer.h:251-355 */
void or_run_layer_legacy_fused(const or_shape_t *s, const or_layer_t *l, const uint8_t *qt,
                               const uint8_t *kvt, const uint8_t *ot, const float *x,
                               uint16_t *kc, uint16_t *vc, int context, float *out,
                               float *attn_capture,
                               or_block_q8_0 *q8_capture);    /* fused_layer.h:361-455 */

void or_quantize_q4_0(const float *src, uint8_t *dst, int count);
void or_dequantize_q4_0(const uint8_t *src, float *dst, int count);

#ifdef __cplusplus
}
#endif
#endif
