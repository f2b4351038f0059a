/*
 * si_abi.h -- C ABI of the MI355X (gfx950) one-Qwen-layer hot path.
 *
 * The reference is one C translation unit of static functions over raw
 * pointers with compile-time shapes (qwen_one_layer.c, attention_kernels.h,
 * fused_layer.h).  This ABI replaces its hot-path functions with HIP kernels:
 *
 *   - plain C types only: device pointers, sizes, an opaque stream handle
 *     (a hipStream_t passed as void*; NULL = the default stream);
 *   - the caller owns every buffer (as in the reference); nothing here
 *     allocates device memory except the layer and workspace create calls;
 *   - shapes are runtime values (si_shape_t) instead of defines.h:16-25;
 *   - every call returns 0 on success or an SI_ERR_* code, with a message in
 *     si_last_error(); the reference's die() (qwen_one_layer.c:26-28) is the
 *     host mirror's job (include/si_host.h);
 *   - calls only enqueue work on the stream; none synchronizes the host.
 *
 * Device data formats
 *   Q4_0 weights (the reference's row-major [N][K/32] 18-byte blocks,
 *   repack_weights.py:43-52) are repacked losslessly once (si_q4_repack) into
 *       qs : uint8  [K/32][N][16]   byte j = element j | element j+16 << 4
 *       d  : uint16 [N/tile][K/32][tile]  fp16 scale bits, tile-major
 *   so a wavefront reads consecutive rows of one block as one contiguous run
 *   of 16 B each, and the scales of a workgroup's `tile` rows form one run
 *   per block that no other workgroup reads.  tile is 8, 16, 32 or 64
 *   (si_q4_tile gives the mat-vec's choice for a shape); d holds
 *   si_q4_scale_count(n, k, tile) entries (N rounded up to the tile).
 *   Q8_0 activations are planar:
 *       qs : int8   [M][K]          d : uint16 [M][K/32]
 *       s  : int16  [M][K/32]       sum of the block's 32 int8 values
 *   (s lets the Q4_0 offset of 8 be applied once per block:
 *    sum((n-8)*a) = sum(n*a) - 8*sum(a), an exact integer identity).
 *   The KV cache is the reference's fp16 [ctx][kvheads][hdim] K and V arrays
 *   (attention_kernels.h:43-44, :101-105).
 */
#ifndef SI_ABI_H
#define SI_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    SI_OK = 0,
    SI_ERR_ARG = 1,    /* invalid size, shape or pointer */
    SI_ERR_HIP = 2,    /* a HIP runtime call failed */
    SI_ERR_STATE = 3,  /* object not ready / wrong mode */
    SI_ERR_NOMEM = 4   /* device allocation failed (create only) */
};

/* Message of the last failing call on this host thread. */
const char *si_last_error(void);

/* Per-dispatch kernel timing, for benchmarks and profiles.  Between start
 * and stop, each kernel launch of this library whose kernel name contains
 * one of the '|'-separated alternatives of `filter` (e.g. "k_dec_attn<" or
 * "k_dec_|k_matvec<") gets HIP events attached to the dispatch itself
 * (hipExtLaunchKernelGGL), for up to `capacity` launches; launches under
 * stream capture are not timed.  stop waits for the recorded launches and
 * writes their durations in milliseconds, in launch order, to ms[0 ..
 * *count - 1]; timing_name(i) is then the i-th timed launch's kernel (its
 * demangled name without namespace and parameters, e.g.
 * "k_dec_attn<64, 8, false, false, 1>"), valid until the next start.  Process-wide; not for concurrent use.  The
 * reference times whole phases on the host instead (phase_t,
 * qwen_one_layer.c:245-276). */
int si_kernel_timing_start(const char *filter, int capacity);
int si_kernel_timing_stop(float *ms, int capacity, int *count);
const char *si_kernel_timing_name(int i);

/* Measurement only, no counterpart in the reference: one streaming pass
 * over `bytes` (a multiple of 16, buf 16-byte aligned) of device memory
 * with 16-byte loads, `depth` (4, 8 or 16) per thread in flight, the buffer
 * cut into at most `workgroups` (1..65536) contiguous slices of 256-thread
 * workgroups; workgroup i writes one word of a checksum to sink[i] (the
 * XOR of all sink words equals the XOR of the buffer's 32-bit words; at
 * most `workgroups` words are written).  Its rate at a kernel's traffic
 * size is the plain-read ceiling that kernel's HBM fraction is compared
 * against. */
int si_stream_read(const void *buf, size_t bytes, uint32_t *sink, int workgroups, int depth,
                   void *stream);

/* defines.h:16-25 (HIDDEN, QHEADS, KVHEADS, HDIM, ROPE_BASE, RMS_EPS) as
 * runtime values; ffn is the build-defined SwiGLU width (0 = none). */
typedef struct si_shape {
    int hidden;
    int qheads;
    int kvheads;
    int hdim;
    int ffn;
    float rope_base;
    float rms_eps;
} si_shape_t;

/* ------------------------------------------------------------------ */
/* Formats                                                             */
/* ------------------------------------------------------------------ */

/* Lossless row-major Q4_0 -> device repack.  Replaces the role of
 * repack_weights.py:43-52 (a lossless target-specific relayout). */
int si_q4_repack(const uint8_t *src_rowmajor, int n, int k, int tile, uint8_t *qs,
                 uint16_t *d, void *stream);
/* Scale tile the mat-vec uses for an n x k matrix (its rows per workgroup). */
int si_q4_tile(int n, int k);
/* Entries of the scale array d for an n x k matrix with a given tile. */
size_t si_q4_scale_count(int n, int k, int tile);
/* Inverse of si_q4_repack (round-trip check, repack_weights.py:126-137). */
int si_q4_unpack(const uint8_t *qs, const uint16_t *d, int n, int k, int tile,
                 uint8_t *dst_rowmajor, void *stream);

/* ------------------------------------------------------------------ */
/* Primitive kernels (one per reference function)                      */
/* ------------------------------------------------------------------ */

/* quantize_q8 (qwen_one_layer.c:98-116): count fp32 values -> count/32
 * block_q8_0 records of 34 bytes (defines.h:27-28), bit-exact. */
int si_quantize_q8(const float *src, void *dst_blocks, int count, void *stream);

/* quantize_q8 over rows x k values into the planar format (bit-exact). */
int si_quantize_q8_rows(const float *src, int rows, int k, int8_t *qs,
                        uint16_t *d, int16_t *s, void *stream);

/* rmsnorm (qwen_one_layer.c:164-169) then quantize_q8, per row.  gain may be
 * NULL (identity, :168); normed (fp32 copy) may be NULL. */
int si_rmsnorm_q8(const float *x, const float *gain, int rows, int n, float eps,
                  float *normed, int8_t *qs, uint16_t *d, int16_t *s, void *stream);

/* Per-(row, block) int32 Q4_0 x Q8_0 dots, dots[n][k/32] (dot_32_q4q8,
 * qwen_one_layer.c:118-146).  Test entry point for the integer core. */
int si_q4q8_block_dots(const uint8_t *wqs, const uint16_t *wd, int n, int k,
                       const int8_t *xqs, const int16_t *xs, int32_t *dots,
                       void *stream);

/* flags of si_matvec_q4q8 / si_gemm_q4q8 / si_gemm_gateup_q8.
 * SI_GEMM_F16 (si_gemm_gateup_q8 only, not with SI_GEMM_EXACT, no K split):
 * the same results bit for bit from f16 matrix-core products of the
 * integer-valued operands (one fused multiply-add per output and block in
 * place of a conversion and one); slower than the default int8 formulation
 * at the layer shapes measured on MI355X, kept as the measured alternative.
 * SI_GEMM_TILED_A (si_gemm_q4q8: m <= 512; si_gemm_gateup_q8: m <= 64; alone):
 * xqs and xd hold the activations
 * operand-tiled (si_q8_tile), streamed next to the weights block by block.
 * si_gemm_q4q8: one pass over any K (no workspace); the same sums as the
 * default within fp32 summation order (K is spread over 12 wavefronts
 * instead of 16).  si_gemm_gateup_q8 (k <= 3840): the same results as the
 * default bit for bit.
 * SI_GEMM_F6 (alone; si_gemm_gateup_q8: shapes whose plan needs no K split):
 * the exact fp6 formulation the layer's prefill GEMMs use past 512 rows.
 * Each Q8 value q = 16 (q >> 4) + (q & 15) and each weight (nibble - 8) are
 * fp6 e2m3 codes of half the value; one scaled fp6 matrix instruction per
 * 32 x 32 tile and block gives the block's integer dot exactly, as a float
 * (no conversion in the epilogue).  The call converts both operands into
 * the workspace first, which must be si_gemm_f6_workspace(m, n, k) bytes
 * (gate|up: n = 2f), 256-byte aligned.  The sums are those of the default
 * tile kernel's plan (bit for bit where the default runs it: more than 512
 * rows, or a shape the streaming kernel does not take).  No reference
 * counterpart: a device formulation of matvec_q4q8 (qwen_one_layer.c:148-162). */
enum { SI_GEMM_EXACT = 1, SI_GEMM_F16 = 2, SI_GEMM_TILED_A = 4, SI_GEMM_F6 = 8 };

/* Operand-tiled Q8_0 (the activation operand of SI_GEMM_TILED_A): rows in
 * panels of 32 (the last padded: ceil(m/32) panels); block b of panel p is
 * 1 KB at tq + (p * k/32 + b) * 1024, laid out [half g][row j][16 bytes],
 * half g of row j holding the block's bytes 8g..8g+7 then 16+8g..16+8g+7;
 * scales td[(p * k/32 + b) * 32 + j].  si_q8_tile writes it from planar
 * qs [m][k] / d [m][k/32] (padding rows: zero).  No reference counterpart:
 * a device layout of block_q8_0 (defines.h:27-28) for the matrix cores. */
int si_q8_tile(const int8_t *qs, const uint16_t *d, int m, int k, int8_t *tq, uint16_t *td,
               void *stream);

/* matvec_q4q8 (qwen_one_layer.c:148-162), one activation row:
 *   out[r] = residual[r] + (bias[r] + sum_b ((float)dot_b * w.d) * x.d)
 * bias and residual may be NULL; wqs and xqs 16-byte aligned.  With
 * flags & SI_GEMM_EXACT the blocks of a row are accumulated in order with
 * the reference's rounding (bit-exact); otherwise K is spread over the
 * threads of a workgroup and the partial sums are added in a fixed order
 * (deterministic, within fp32 rounding of the reference).  A workgroup
 * owns `tile` rows (at most 64), the tile the weights were repacked with. */
int si_matvec_q4q8(const uint8_t *wqs, const uint16_t *wd, int tile, int n, int k,
                   const int8_t *xqs, const uint16_t *xd, const int16_t *xs,
                   const float *bias, const float *residual, float *out,
                   int flags, void *stream);

/* matvec_q4q8 applied to m activation rows (prefill / batched decode):
 * out[i][r] (row stride ldo; residual uses the same stride) =
 * residual + (bias + sum over blocks).  int8 matrix-core tiles compute every
 * per-block int32 dot exactly.  With flags & SI_GEMM_EXACT the fp32
 * epilogue reproduces the reference's rounding sequence (bit-exact with
 * matvec_q4q8); otherwise each block adds dot * (x.d * w.d) in one fused
 * multiply-add, the scale product exact in fp32 (within fp32 rounding of
 * the reference).  A grid too small for the chip splits K: that needs
 * si_gemm_workspace(m, n, k) bytes of workspace (NULL or smaller: no split);
 * the split sums are added in a fixed order (deterministic). */
int si_gemm_q4q8(const uint8_t *wqs, const uint16_t *wd, int tile, int n, int k,
                 const int8_t *xqs, const uint16_t *xd, int m,
                 const float *bias, const float *residual, float *out, int ldo,
                 int flags, void *workspace, size_t ws_bytes, void *stream);
size_t si_gemm_workspace(int m, int n, int k);
/* Workspace bytes of si_gemm_q4q8 / si_gemm_gateup_q8 with SI_GEMM_F6 (the
 * converted operands and the K-split partials).  No reference counterpart. */
size_t si_gemm_f6_workspace(int m, int n, int k);

/* The FFN gate|up projection of m activation rows with SwiGLU and Q8_0:
 * gu = [gate | up] = matvec_q4q8 of each row (qwen_one_layer.c:148-162)
 * against the 2f x k matrix [gate rows; up rows], act = silu(gate)*up,
 * quantize_q8(act) (:98-116) into planar qs/d/bsum ([m][f], [m][f/32]).
 * gu ([m][2f] fp32) is written when given; it is required only where it is
 * the intermediate: SI_GEMM_EXACT, or a plan that splits K (si_gemm_workspace
 * (m, 2f, k) > 0) given less workspace than that.  act and bsum may be NULL.
 * wqs, xqs, qs and act are 16-byte aligned.
 * flags: SI_GEMM_EXACT as for si_gemm_q4q8, SI_GEMM_F16, or SI_GEMM_F6. */
int si_gemm_gateup_q8(const uint8_t *wqs, const uint16_t *wd, int tile, int f, int k,
                      const int8_t *xqs, const uint16_t *xd, int m, float *gu, float *act,
                      int8_t *qs, uint16_t *d, int16_t *bsum, int flags, void *workspace,
                      size_t ws_bytes, void *stream);

/* The decode FFN front half for one row, fused: rmsnorm(h, gain)
 * (qwen_one_layer.c:164-169) -> quantize_q8 (:98-116) -> gate and up
 * projections (matvec_q4q8, :148-162) -> act = silu(gate)*up ->
 * quantize_q8(act) into planar qs/d/bsum (f values; act, the fp32 copy,
 * may be NULL).  wqs/wd: the 2f x hidden matrix [gate rows; up rows]
 * repacked with tile 32 (each workgroup pairs 32 gate with 32 up rows).
 * flags: SI_GEMM_EXACT for the reference's block order and roundings. */
int si_ffn_gateup_q8(const float *h, const float *gain, int hidden, float eps,
                     const uint8_t *wqs, const uint16_t *wd, int tile, int f, float *act,
                     int8_t *qs, uint16_t *d, int16_t *bsum, int flags, void *stream);

/* RoPE (qwen_one_layer.c:172-183) + fp16 K/V append (:262-266) for ntok
 * rows of the fused projection output qkv[t] = [q | k | v]
 * (qheads*hdim + 2*kvheads*hdim floats, row stride ldqkv).  Token t is at
 * position ctx_dev[t]-1 when ctx_dev (device ints) is given, else
 * pos0 + t*pos_step (1 for a prefill batch, 0 for one position per row).
 * Writes rotated q to q_out[t] (qheads*hdim), K/V rows into kc/vc
 * (+ t*kv_seq_stride elements when kv_seq_stride != 0, i.e. one cache per
 * sequence; kv_seq_stride == 0 means one shared cache; a multiple of 8).
 * rope_cos/rope_sin: [max_pos][hdim/2] tables (si_rope_table); rows whose
 * position falls outside 0..max_pos-1 are skipped. */
int si_rope_kv_append(const si_shape_t *s, const float *qkv, int ldqkv, int ntok,
                      int pos0, int pos_step, int max_pos, const int *ctx_dev,
                      const float *rope_cos,
                      const float *rope_sin, float *q_out, uint16_t *kc,
                      uint16_t *vc, size_t kv_seq_stride, void *stream);

/* Host-side RoPE table, theta = pos / powf(base, 2i/hdim) with libm
 * cosf/sinf exactly as qwen_one_layer.c:176-177; [npos][hdim/2] each. */
int si_rope_table(int npos, int hdim, float base, float *cos_host, float *sin_host);

/* attention_flash (attention_kernels.h:80-164) for nq queries, GQA.
 * q: [nq][qheads*hdim] fp32.  Query i attends to positions [0, ctx_i) of
 * cache kc/vc + i*kv_seq_stride, where ctx_i = ctx_dev[i] if ctx_dev != NULL,
 * else ctx0 + i*ctx_step (decode: ctx_step 0; causal prefill: ctx_step 1).
 * Contexts above max_ctx are clamped to it; a context <= 0 gives zeros
 * (attention_kernels.h:95-98).  Output attn fp32 [nq][qheads*hdim] and its
 * Q8_0 quantization (planar, optional: pass NULL qs to skip).
 * workspace: si_attention_workspace bytes. */
int si_attention(const si_shape_t *s, const float *q, int nq, const uint16_t *kc,
                 const uint16_t *vc, size_t kv_seq_stride, const int *ctx_dev,
                 int ctx0, int ctx_step, int max_ctx, float *attn, int8_t *qs,
                 uint16_t *d, int16_t *bsum, void *workspace, size_t workspace_bytes,
                 void *stream);
size_t si_attention_workspace(const si_shape_t *s, int nq, int max_ctx);

/* si_attention without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * partial states live in one fixed buffer of SI_ATTENTION_STATIC_MAX bytes
 * per GPU inside the library (held until the process ends); the call
 * allocates nothing and returns SI_ERR_ARG when
 * si_attention_workspace(s, nq, max_ctx) exceeds that size.  Every call on
 * a GPU shares its buffer: calls that overlap on one GPU (other streams or
 * host threads) race; calls ordered on one stream do not.  Results are
 * bit-identical to si_attention's on the same inputs. */
#define SI_ATTENTION_STATIC_MAX (16u << 20)
int si_attention_static(const si_shape_t *s, const float *q, int nq, const uint16_t *kc,
                        const uint16_t *vc, size_t kv_seq_stride, const int *ctx_dev, int ctx0,
                        int ctx_step, int max_ctx, float *attn, int8_t *qs, uint16_t *d,
                        int16_t *bsum, void *stream);

/* attention_standard (attention_kernels.h:33-78) for one query: scores
 * [qheads][context] fp32 (device, caller-owned like the reference's
 * score_workspace) receive the scaled Q.K products (the reference's bits:
 * sequential sum over the head dimension), are normalised in place by a
 * softmax, and weight V into out [qheads][hdim].  kc/vc are [context][kvheads]
 * [hdim] fp16, both 16-byte aligned.  context 0 gives a zero output. */
int si_attention_standard(const si_shape_t *s, const float *q, const uint16_t *kc,
                          const uint16_t *vc, int context, float *out, float *scores,
                          void *stream);

/* Build-defined SwiGLU + quantize_q8: act = silu(gate)*up with
 * silu(g) = g/(1+expf(-g)); gate = gu[r][0..f), up = gu[r][f..2f). */
int si_swiglu_q8(const float *gu, int rows, int f, float *act, int8_t *qs,
                 uint16_t *d, int16_t *s, void *stream);

/* h = x + y (residual) then rmsnorm + quantize_q8 of h. */
int si_residual_rmsnorm_q8(const float *x, const float *y, const float *gain,
                           int rows, int n, float eps, float *h, float *normed,
                           int8_t *qs, uint16_t *d, int16_t *s, void *stream);

/* ------------------------------------------------------------------ */
/* The reference's own formats (behind the host mirror's drop-ins)     */
/* ------------------------------------------------------------------ */

/* f32_to_f16 / f16_to_f32 (qwen_one_layer.c:42-86) over n device values:
 * round to nearest even with subnormals, NaN -> sign|0x7e00, overflow ->
 * sign|inf; the widening is exact (bit-exact both ways). */
int si_f32_to_f16(const float *src, uint16_t *dst, size_t n, void *stream);
int si_f16_to_f32(const uint16_t *src, float *dst, size_t n, void *stream);

/* matvec_q4q8 (qwen_one_layer.c:148-162) on the reference's formats:
 * w row-major Q4_0 ([outputs][inputs/32] 18-byte blocks), x block_q8_0
 * records ([inputs/32] x 34 bytes, defines.h:27-28), both 2-byte aligned;
 * out[r] = bias[r] (0 when NULL) + sum over blocks in order of
 * ((float)dot * w.d) * x.d, the reference's roundings (bit-exact). */
int si_matvec_q4q8_rowmajor(const uint8_t *w, const void *x_blocks, int inputs, int outputs,
                            const float *bias, float *out, void *stream);

/* fused_column_matvec (fused_layer.h:169-245) over ntiles consecutive
 * column-SoA tiles of nblocks 5120-byte groups (the layout
 * repack_weights.py writes: per input block 32 columns x 128 packed bytes,
 * low nibble = output j, high = output j+128, then 256 fp32 scales).  Tile
 * t writes out[t*256 .. t*256+255]: with add == 0 it starts from
 * bias_lo[t*256 + j] / bias_hi[t*256 + j] (0 when NULL), with add != 0 from
 * the current out values; each block adds ((float)sum * scale) * x.d
 * (bit-exact).  x_blocks: nblocks block_q8_0 records; tiles 4-byte aligned. */
int si_colsoa_matvec(const uint8_t *tiles, int ntiles, const void *x_blocks, int nblocks,
                     const float *bias_lo, const float *bias_hi, float *out, int add,
                     void *stream);

/* rmsnorm (qwen_one_layer.c:164-169) of rows x n values, without the Q8
 * step: out = (x * inv) * gain (gain NULL = 1). */
int si_rmsnorm(const float *x, const float *gain, int rows, int n, float eps, float *out,
               void *stream);

/* rope (qwen_one_layer.c:172-183) in place on nheads heads of s->hdim
 * values at `position`, with si_rope_table cos/sin tables of max_pos rows
 * on the device (bit-exact). */
int si_rope(const si_shape_t *s, float *heads, int nheads, int position, const float *rope_cos,
            const float *rope_sin, int max_pos, void *stream);

/* attention_flash (attention_kernels.h:80-164) for nheads query heads that
 * share KV group `group` of s's cache layout (fused_attention_pair,
 * fused_layer.h:251-355, is nheads = 2): q [nheads][hdim], kc/vc the
 * [context][kvheads][hdim] fp16 caches, out [nheads][hdim].  workspace:
 * si_attention_group_workspace bytes. */
int si_attention_group(const si_shape_t *s, const float *q, int nheads, int group,
                       const uint16_t *kc, const uint16_t *vc, int context, float *out,
                       void *workspace, size_t ws_bytes, void *stream);
size_t si_attention_group_workspace(const si_shape_t *s, int nheads, int context);

/* ------------------------------------------------------------------ */
/* Layer level (run_layer / run_layer_fused / pf_run_batch)            */
/* ------------------------------------------------------------------ */

/* Host-side layer tensors in the reference's file formats
 * (qwen_one_layer.c:210-221): row-major Q4_0 matrices, optional fp32
 * norm/bias vectors (NULL = identity/zero).  post_norm, wgate, wup, wdown
 * are the build-defined FFN (all NULL = attention sublayer only). */
typedef struct si_layer_host {
    const uint8_t *wq, *wk, *wv, *wo;
    const float *norm, *bq, *bk, *bv;
    const float *post_norm;
    const uint8_t *wgate, *wup, *wdown;
} si_layer_host_t;

typedef struct si_layer si_layer_t; /* opaque: device weights + a workspace */
typedef struct si_workspace si_workspace_t; /* opaque: activations, partials, RoPE */

/* A workspace: activation buffers for up to max_tokens rows per call,
 * attention partials and RoPE tables for max_pos positions: the intermediate
 * vectors run_layer keeps on its stack (qwen_one_layer.c:242-243).  Layers of
 * one model may share one; calls on layers sharing a workspace must not run
 * concurrently.  The memory is released when the workspace handle and every
 * layer using it are gone. */
int si_workspace_create(const si_shape_t *s, int max_tokens, int max_pos,
                        si_workspace_t **out);
int si_workspace_destroy(si_workspace_t *ws);

/* Uploads and repacks the weights (load_layer, qwen_one_layer.c:210-221,
 * plus the build's FFN weights).  si_layer_create also creates a private
 * workspace; si_layer_create_in uses a shared one.  With the workspace calls,
 * the only calls that allocate device memory. */
int si_layer_create(const si_shape_t *s, const si_layer_host_t *w, int max_tokens,
                    int max_pos, si_layer_t **out);
int si_layer_create_in(si_workspace_t *ws, const si_layer_host_t *w, si_layer_t **out);
int si_layer_destroy(si_layer_t *l);

enum {
    SI_LAYER_FULL = 0,      /* attention + residual + norm + SwiGLU FFN + residual */
    SI_LAYER_ATTN_ONLY = 1, /* reference run_layer: out = W_O . Q8(attn)          */
    SI_LAYER_EXACT = 2,     /* reference rounding in every projection (bit-exact Q/K/V,
                               O, gate/up, down given identical inputs): mat-vecs
                               without K splits, GEMMs with the exact epilogue */
    SI_LAYER_ATTN_STANDARD = 4, /* si_layer_decode only: the reference's staged order
                               with ATTENTION_STANDARD (qwen_one_layer.c:260-275):
                               RoPE + K/V append, si_attention_standard into the
                               layer's [qheads][max_pos] score buffer, Q8, W_O */
    SI_LAYER_CAPTURE = 8    /* also store the intermediates no later stage reads
                               (si_layer_buffer: NORMED, NORMED2, GU, ACT, the
                               decode's XQ, XQ2, Q, ATTN, ATTQ, ATTN_OUT); without it
                               those buffers are not written, as the reference's
                               NULL captures (qwen_one_layer.c:278-279) */
};

/* run_layer (qwen_one_layer.c:237-281) for one token at position context-1:
 * x [hidden] -> out [hidden]; appends K/V at row context-1 of kc/vc. */
int si_layer_decode(si_layer_t *l, const float *x, uint16_t *kc, uint16_t *vc,
                    int context, float *out, int flags, void *stream);

/* Batched decode: nseq independent sequences, one new token each.
 * x, out: [nseq][hidden]; sequence i's cache is kc/vc + i*kv_seq_stride,
 * its new token sits at position ctx_dev[i]-1 (device int array; NULL = all
 * context).  max_ctx bounds every context. */
int si_layer_decode_batch(si_layer_t *l, const float *x, int nseq, uint16_t *kc,
                          uint16_t *vc, size_t kv_seq_stride, const int *ctx_dev,
                          int context, int max_ctx, float *out, int flags,
                          void *stream);

/* Paged KV cache (no counterpart in the reference, which keeps one
 * contiguous [ctx][kvheads][hdim] cache per layer, qwen_one_layer.c:262-266;
 * this is the step after a single layer: many sequences of unequal length
 * sharing one pool).  A pool holds npages pages of page_size (a power of
 * two) fp16 rows of kvheads*hdim values, K and V in separate pools.
 * pages (device int [nseq][max_pages]) maps sequence i's position p to pool
 * row pages[i*max_pages + p/page_size]*page_size + p%page_size; page ids
 * outside [0, npages) are clamped (they cannot address outside the pool).
 * The pool bytes are npages*page_size*kvheads*hdim*2 each.
 *
 * si_layer_decode_batch over a paged cache: sequence i's new token sits at
 * position ctx_dev[i]-1 (NULL = all context); its K/V row is appended
 * through the table, then attention reads the sequence's rows through it.
 * Prefill and single-token decode keep contiguous caches. */
int si_layer_decode_paged(si_layer_t *l, const float *x, int nseq, uint16_t *k_pool,
                          uint16_t *v_pool, int npages, int page_size, const int *pages,
                          int max_pages, const int *ctx_dev, int context, int max_ctx,
                          float *out, int flags, void *stream);

/* si_attention for nq decode queries over a paged cache (ctx_dev required):
 * the same kernels as the contiguous form, so the result is bit-identical to
 * si_attention on the same rows laid out contiguously. */
int si_attention_paged(const si_shape_t *s, const float *q, int nq, const uint16_t *k_pool,
                       const uint16_t *v_pool, int npages, int page_size, const int *pages,
                       int max_pages, const int *ctx_dev, int max_ctx, float *attn, int8_t *qs,
                       uint16_t *d, int16_t *bsum, void *workspace, size_t workspace_bytes,
                       void *stream);

/* pf_run_batch (prefill_weight_stationary.h:183-311): causal prefill of
 * ntok tokens after prefix cached positions.  Appends K/V rows
 * prefix..prefix+ntok-1; token t attends with context prefix+t+1. */
int si_layer_prefill(si_layer_t *l, const float *x, int ntok, int prefix,
                     uint16_t *kc, uint16_t *vc, float *out, int flags, void *stream);

/* Device pointers to a layer's intermediates of the last call, for parity
 * checks and captures (run_layer's attn_copy/q8_copy, :278-279). */
enum {
    SI_BUF_NORMED = 0,  /* fp32 [rows][hidden]                  */
    SI_BUF_XQ_QS, SI_BUF_XQ_D, SI_BUF_XQ_S,
    SI_BUF_QKV,         /* fp32 [rows][qd + 2 kvd] (pre-RoPE)   */
    SI_BUF_Q,           /* fp32 [rows][qd] rotated q            */
    SI_BUF_ATTN,        /* fp32 [rows][qd]                      */
    SI_BUF_ATTQ_QS, SI_BUF_ATTQ_D, SI_BUF_ATTQ_S,
    SI_BUF_ATTN_OUT,    /* fp32 [rows][hidden] W_O output       */
    SI_BUF_H,           /* fp32 [rows][hidden] residual 1       */
    SI_BUF_NORMED2,
    SI_BUF_XQ2_QS, SI_BUF_XQ2_D, SI_BUF_XQ2_S,
    SI_BUF_GU,          /* fp32 [rows][2 ffn] gate | up         */
    SI_BUF_ACT,         /* fp32 [rows][ffn]                     */
    SI_BUF_ACTQ_QS, SI_BUF_ACTQ_D, SI_BUF_ACTQ_S,
    SI_BUF_ACTQ_TQ,     /* act Q8_0 operand-tiled: calls of 2..512 rows whose  */
    SI_BUF_ACTQ_TD,     /* down projection streamed it (else not written)     */
    SI_BUF_COUNT
};
void *si_layer_buffer(si_layer_t *l, int which);

/* Per-phase GPU timing of layer calls (hipEvents between stages), the
 * device analogue of phase_t (defines.h:35-37, qwen_one_layer.c:245-276).
 * RMSNorm+Q8, attention+Q8, SwiGLU+Q8 are single fused kernels. */
enum {
    SI_PHASE_RMS_Q8 = 0,
    SI_PHASE_QKV,
    SI_PHASE_ROPE_KV,
    SI_PHASE_ATTENTION_Q8,
    SI_PHASE_OUT_PROJ,
    SI_PHASE_POST_NORM_Q8,
    SI_PHASE_GATE_UP,
    SI_PHASE_SWIGLU_Q8,
    SI_PHASE_DOWN,
    SI_PHASE_COUNT
};
int si_layer_set_timing(si_layer_t *l, int enable);
/* Milliseconds per phase of the last timed call; waits for it to finish. */
int si_layer_phase_ms(si_layer_t *l, float *ms);

/* Device weights of a created layer, for kernel-level benchmarks:
 * which = 0 QKV (fused rows q|k|v), 1 O, 2 gate|up, 3 down. */
int si_layer_weights(si_layer_t *l, int which, const uint8_t **qs,
                     const uint16_t **d, int *tile, int *n, int *k);

#ifdef __cplusplus
}
#endif
#endif /* SI_ABI_H */
