// si_kernels.hpp -- launcher prototypes shared by the HIP translation units.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <atomic>
#include <stdint.h>
namespace si {
// Per-dispatch kernel timing (si_kernel_timing_start / _stop): when it is on
// and the kernel's name contains the filter, hands out a pair of events for
// hipExtLaunchKernelGGL to attach to the dispatch itself.
bool kernel_timing_events(const void *kernel, hipStream_t st, hipEvent_t *start,
                          hipEvent_t *stop);
// Read on every launch from any host thread (relaxed: the events it guards
// are handed out under the timing mutex); written under that mutex.
extern std::atomic<bool> g_kernel_timing_on;
}  // namespace si

// Every kernel launch of the library goes through SI_LAUNCH (same arguments
// as hipLaunchKernelGGL; K parenthesised when it holds commas).
#define SI_LAUNCH(K, G, B, S, ST, ...)                                                 \
    do {                                                                             \
        hipEvent_t si_ev0_, si_ev1_;                                                 \
        if (::si::g_kernel_timing_on.load(std::memory_order_relaxed) &&             \
            ::si::kernel_timing_events((const void *)(K), ST, &si_ev0_, &si_ev1_))   \
            hipExtLaunchKernelGGL(K, G, B, S, ST, si_ev0_, si_ev1_, 0, __VA_ARGS__);  \
        else                                                                         \
            hipLaunchKernelGGL(K, G, B, S, ST, __VA_ARGS__);                         \
    } while (0)

namespace si {
void launch_quantize_q8_aos(const float *src, void *dst, int count, hipStream_t st);
void launch_quantize_q8_rows(const float *src, int rows, int k, int8_t *qs, uint16_t *d,
                             int16_t *s, hipStream_t st);
// tq/td (optional): the Q8_0 output operand-tiled as well (q8_tiled_byte);
// x6 (optional): as the fp6 GEMM's activation codes as well (launch_q8_to_x6's
// layout, m = rows)
void launch_rmsnorm_q8(const float *x, const float *y, const float *gain, int rows, int n,
                       float eps, float *h, float *normed, int8_t *qs, uint16_t *d, int16_t *s,
                       hipStream_t st, int8_t *tq = nullptr, uint16_t *td = nullptr,
                       uint8_t *x6 = nullptr);
void launch_swiglu_q8(const float *gu, int rows, int f, float *act, int8_t *qs, uint16_t *d,
                      int16_t *s, hipStream_t st, int8_t *tq = nullptr, uint16_t *td = nullptr);
void launch_q4_repack(const uint8_t *src, int n, int k, int tile, uint8_t *qs, uint16_t *d,
                      hipStream_t st);
void launch_q4_unpack(const uint8_t *qs, const uint16_t *d, int n, int k, int tile,
                      uint8_t *dst, hipStream_t st);
// pre (optional): the value before the residual is added
void launch_matvec(const int8_t *xqs, const uint16_t *xd, const int16_t *xs, int k,
                   const uint8_t *wqs, const uint16_t *wd, int tile, int n, const float *bias,
                   const float *residual, float *out, bool exact, hipStream_t st,
                   float *pre = nullptr);
void launch_block_dots(const uint8_t *wqs, int n, int k, const int8_t *xqs, const int16_t *xs,
                       int32_t *dots, hipStream_t st);
// The GEMM of launch_gemm_q4q8 without bias or residual; when the plan
// splits K, the split partial sums stay in workspace as [splits][m][n] for
// the caller to reduce and the number of splits is returned, else 0 (out
// holds the product).
int launch_gemm_q4q8_parts(const uint8_t *wqs, const uint16_t *wd, int tile, int n, int k,
                           const int8_t *xqs, const uint16_t *xd, int m, float *out, bool exact,
                           void *workspace, size_t ws_bytes, hipStream_t st);
// out[m][n] = sum of part[s][m][n] in split order.
void launch_gemm_reduce(const float *part, int splits, int m, int n, float *out, hipStream_t st);
// launch_rmsnorm_q8 with y = the split-order sum of part[splits][rows][n],
// written to y_out as well.
void launch_rmsnorm_q8_parts(const float *x, const float *part, int splits, const float *gain,
                             int rows, int n, float eps, float *y_out, float *h, float *normed,
                             int8_t *qs, uint16_t *d, int16_t *s, hipStream_t st,
                             int8_t *tq = nullptr, uint16_t *td = nullptr, uint8_t *x6 = nullptr);
void launch_gemm_q4q8(const uint8_t *wqs, const uint16_t *wd, int tile, int n, int k,
                      const int8_t *xqs, const uint16_t *xd, int m, const float *bias,
                      const float *residual, float *out, int ldo, bool exact, void *workspace,
                      size_t ws_bytes, hipStream_t st);
// planar Q8_0 (qs [m][k], d [m][k/32]) -> operand-tiled (q8_tiled_byte)
void launch_q8_tile(const int8_t *qs, const uint16_t *d, int m, int k, int8_t *tq, uint16_t *td,
                    hipStream_t st);
// launch_gemm_q4q8 (no K split, not exact) with the activations operand-
// tiled (q8_tiled_byte: tq [ceil(m/32)][k/32] KB, td [ceil(m/32)][k/32][32]);
// m <= 64.
void launch_gemm_q4q8_tiled(const uint8_t *wqs, const uint16_t *wd, int tile, int n, int k,
                            const int8_t *tq, const uint16_t *td, int m, const float *bias,
                            const float *residual, float *out, int ldo, hipStream_t st);
// f16: k_gemm_h16 (the f16 formulation) where the plan runs one fused pass.
// tq/td (optional): the Q8_0 output operand-tiled as well.  txq/txd
// (optional): the same activations as xqs/xd operand-tiled, streamed instead
// of staged where gemm_gateup_streams() holds for the call.
void launch_gemm_gateup_q8(const uint8_t *wqs, const uint16_t *wd, int tile, int f, int k,
                           const int8_t *xqs, const uint16_t *xd, int m, float *gu, float *act,
                           int8_t *qs, uint16_t *d, int16_t *s, bool exact, void *workspace,
                           size_t ws_bytes, hipStream_t st, bool f16 = false,
                           int8_t *tq = nullptr, uint16_t *td = nullptr,
                           const int8_t *txq = nullptr, const uint16_t *txd = nullptr);
// Whether launch_gemm_gateup_q8 streams txq/txd (default flags) for m rows,
// f features, K = k.
bool gemm_gateup_streams(int m, int f, int k);
// Whether launch_gemm_q4q8_tiled is the one-tile kernel's plan for m x n x k
// (the default path would take k_gemm_bd too); it takes any m <= 512.
bool gemm_streams(int m, int n, int k);
size_t gemm_workspace_bytes(int m, int n, int k);
// workspace launch_gemm_gateup_q8 uses for f features (0: never splits K)
size_t gemm_gateup_workspace_bytes(int m, int f, int k);
}  // namespace si
namespace si {
// A paged KV cache: sequence i's position p lives in pool row
// pages[i*max_pages + p/page_size]*page_size + p%page_size (page_size =
// 1 << shift).  Page ids are device data, clamped to [0, npages) so a bad
// table cannot address outside the pool.  pages == nullptr: contiguous
// caches, sequence i at i*kv_seq_stride.
struct KvPages {
    const int *pages = nullptr;
    int max_pages = 0, shift = 0, npages = 0;
    // element offset of the row; PAGED fixed at compile time (the tuned
    // kernels are instantiated for both layouts)
    template <bool PAGED>
    __device__ __forceinline__ size_t at(int seq, int pos, size_t kv_seq_stride, int kvd) const {
        if constexpr (!PAGED) {
            return (size_t)seq * kv_seq_stride + (size_t)pos * kvd;
        } else {
            int pg = pages[(size_t)seq * max_pages + min(pos >> shift, max_pages - 1)];
            pg = min(max(pg, 0), npages - 1);
            return (((size_t)pg << shift) | (size_t)(pos & ((1 << shift) - 1))) * kvd;
        }
    }
    __device__ __forceinline__ size_t row(int seq, int pos, size_t kv_seq_stride,
                                          int kvd) const {
        return pages ? at<true>(seq, pos, kv_seq_stride, kvd)
                     : at<false>(seq, pos, kv_seq_stride, kvd);
    }
};
// k_gemm_bd MODE 2 (the fused Q|K|V projection of a prefill) over weights
// whose output rows are permuted per head as [e, hdim/2 + e] for e = 0 ..
// hdim/2 - 1 (rope_perm_row), so a rotation pair sits in two neighbouring
// lanes of one tile: RoPE of q and k at token t's position pos0 + t, q to
// q_out, k and v as fp16 into the caches at row t * kv_seq_stride + pos *
// kvd (contiguous layout); out (optional) gets the unrotated q|k|v in the
// original column order
struct RopeOut {
    const float *rc, *rs;  // [pos][hdim / 2] cos, sin
    float *q_out;          // [m][qd]
    uint16_t *kc, *vc;
    size_t kv_seq_stride;
    int pos0, max_pos, hdim, qd, kvd;
};
// The prefill Q|K|V projection + bias with the RoPE and the K/V append in
// its epilogue (k_gemm_bd MODE 2, LDS-staged activations), over weights and
// bias whose output rows are in rope_perm_row order: false (nothing
// launched) unless the staged one-tile kernel runs the shape in one K range
// (more than 64 and up to 512 rows); the caller then projects and runs
// k_rope_kv.
bool launch_gemm_qkv_rope(const uint8_t *wqs, const uint16_t *wd, int tile, int n, int k,
                          const int8_t *xqs, const uint16_t *xd, int m, const float *bias_perm,
                          float *out, const RopeOut &ro, hipStream_t st);
// The fp6 formulation of the fast-path GEMM (k_gemm_f6): the weights once as
// w6 fp6 codes (n * nb * 24 bytes) + d6 [nb][n] fp16 scales (logical gate|up
// row order when gu_f > 0), each Q8 activation as x6 (m * nb * 48 bytes: hi
// and lo codes).  launch_gemm_f6 has gemm_core's plan, splits and reduce
// (want_part: the split count, partials left in the workspace); with gu_f > 0
// it is the fused gate|up + SwiGLU + Q8 pass (out: the optional gate|up, ldo
// 2 gu_f; atq/atd, optional: the Q8 also operand-tiled), and returns -1
// (nothing launched) when that plan needs a K split.
void launch_q8_to_x6(const int8_t *qs, int m, int nb, uint8_t *x6, hipStream_t st);
size_t gemm_f6_partial_bytes(int m, int n, int k);  // launch_gemm_f6's K-split partials
void launch_q4_to_w6(const uint8_t *qs, const uint16_t *d, int n, int nb, int tile, int gu_f,
                     uint8_t *w6, uint16_t *d6, hipStream_t st);
int launch_gemm_f6(const uint8_t *w6, const uint16_t *d6, int n, int k, const uint8_t *x6,
                   const uint16_t *xd, int m, const float *bias, const float *residual,
                   float *out, int ldo, void *workspace, size_t ws_bytes, bool want_part,
                   int gu_f, float *act, int8_t *aqs, uint16_t *ad, int16_t *as, hipStream_t st,
                   int8_t *atq = nullptr, uint16_t *atd = nullptr);
// Original output row of row pr of the RoPE-permuted Q|K|V weights: per head
// of hdim rows, [e, hdim/2 + e] for e = 0 .. hdim/2 - 1.
inline int rope_perm_row(int pr, int hdim) {
    const int head = pr / hdim, within = pr % hdim;
    return head * hdim + (within >> 1) + (within & 1) * (hdim >> 1);
}
void launch_rope_kv(const float *qkv, int ldqkv, int ntok, int qheads, int kvheads, int hdim,
                    int pos0, int pos_step, int max_pos, const int *ctx_dev, const float *rc,
                    const float *rs, float *q_out, uint16_t *kc, uint16_t *vc,
                    size_t kv_seq_stride, hipStream_t st, KvPages pg = KvPages());
int attn_nsplit(int kvheads, int nq, int max_ctx);
size_t attn_workspace_bytes(int qheads, int hdim, int kvheads, int nq, int max_ctx);
bool attn_supported(int qheads, int kvheads, int hdim);
// three-stage textbook attention for one query (scores: [qheads][ctx] fp32)
bool attn_standard_supported(int qheads, int kvheads, int hdim);
void launch_attn_standard(const float *q, int qheads, int kvheads, int hdim, const uint16_t *kc,
                          const uint16_t *vc, int ctx, float *out, float *scores, hipStream_t st);
void launch_attention(const float *q, int nq, int qheads, int kvheads, int hdim,
                      const uint16_t *kc, const uint16_t *vc, size_t kv_seq_stride,
                      const int *ctx_dev, int ctx0, int ctx_step, int max_ctx, float *attn,
                      int8_t *qs, uint16_t *d, int16_t *bsum, void *workspace,
                      hipStream_t st, KvPages pg = KvPages(), int kv_row = 0);
bool attn_prefill_supported(int qheads, int kvheads, int hdim);
size_t attn_prefill_workspace_bytes(int qheads, int hdim, int ntok);
void launch_attn_prefill(const float *q, int ntok, int qheads, int kvheads, int hdim, int pos0,
                         const uint16_t *kc, const uint16_t *vc, float *attn, int8_t *qs,
                         uint16_t *qd, int16_t *bsum, void *workspace, size_t ws_bytes,
                         hipStream_t st);
}  // namespace si
namespace si {
// fused decode kernels (si_decode.hip)
void launch_dec_qkv(const float *x, const float *gain, int hidden, float eps, const uint8_t *wqs,
                    const uint16_t *wd, int tile, int n, const float *bias, float *cap_normed,
                    int8_t *cap_qs, uint16_t *cap_d, int16_t *cap_s, float *qkv, bool exact,
                    hipStream_t st);
void launch_dec_wo(const float *pm, const float *pl, const float *po, int ns, int qheads,
                   int hdim, const uint8_t *wqs, const uint16_t *wd, int tile, int n,
                   const float *residual, float *cap_attn, int8_t *cap_qs, uint16_t *cap_d,
                   int16_t *cap_s, float *cap_y, float *out, bool exact, hipStream_t st);
void launch_dec_gateup(const float *h, const float *gain, int hidden, float eps,
                       const uint8_t *wqs, const uint16_t *wd, int tile, int f,
                       float *cap_normed,
                       int8_t *cap_qs, uint16_t *cap_d, int16_t *cap_s, float *gu, float *act,
                       int8_t *aqs, uint16_t *ad, int16_t *as, bool exact, hipStream_t st);
int dec_attn_chunks(int qheads, int kvheads, int hdim, int nq, int max_ctx);
// The layer input, RMSNorm gain and fused Q|K|V matrix (+bias) of the
// single-token decode kernel that projects and attends in one launch.
struct DecQkvIn {
    const float *x = nullptr, *gain = nullptr;
    int hidden = 0;
    float eps = 0.0f;
    const uint8_t *wqs = nullptr;
    const uint16_t *wd = nullptr;
    int tile = 0, n = 0;
    const float *bias = nullptr;
    // optional captures: the normalised row and its Q8, the q|k|v row
    float *cap_normed = nullptr;
    int8_t *cap_qs = nullptr;
    uint16_t *cap_d = nullptr;
    int16_t *cap_s = nullptr;
    float *cap_qkv = nullptr;
};
bool dec_qkv_attn_ok(int hidden, int qheads, int kvheads, int hdim, int ctx);
void launch_dec_qkv_attn(const DecQkvIn &fq, int qheads, int kvheads, int hdim, const float *rc,
                         const float *rs, uint16_t *kc, uint16_t *vc, int ctx, int ns,
                         float *q_cap, void *workspace, hipStream_t st);
size_t dec_attn_workspace_bytes(int qheads, int hdim, int kvheads, int nq, int max_ctx);
void launch_dec_attn(const float *qkv, int ldqkv, int nq, int qheads, int kvheads, int hdim,
                     const float *rc, const float *rs, uint16_t *kc, uint16_t *vc,
                     size_t kv_seq_stride, const int *ctx_dev, int ctx0, int max_ctx,
                     float *q_cap, int ns, void *workspace, float *attn, int8_t *aqs,
                     uint16_t *ad, int16_t *as, hipStream_t st, KvPages pg = KvPages());
// tq/td (optional): the Q8_0 also operand-tiled (q8_tiled_byte; qs required)
void launch_attn_combine(int nq, int qheads, int hdim, int nsplit, const void *workspace,
                         float *attn, int8_t *qs, uint16_t *d, int16_t *bsum, hipStream_t st,
                         int8_t *tq = nullptr, uint16_t *td = nullptr);
// Kernels over the reference's own formats (si_mirror.hip): row-major Q4_0
// with block_q8_0 records, column-SoA tiles, stand-alone rmsnorm and rope.
void launch_matvec_rowmajor(const uint8_t *w, const void *x, int inputs, int outputs,
                            const float *bias, float *out, hipStream_t st);
void launch_colsoa_matvec(const uint8_t *tiles, int ntiles, const void *x, int nblocks,
                          const float *bias_lo, const float *bias_hi, float *out, int add,
                          hipStream_t st);
void launch_rmsnorm(const float *x, const float *gain, int rows, int n, float eps, float *out,
                    hipStream_t st);
void launch_rope_inplace(float *heads, int nheads, int hdim, int position, const float *rc,
                         const float *rs, hipStream_t st);
void launch_f16_convert(const void *src, void *dst, size_t n, bool to_half, hipStream_t st);
// one streaming pass over bytes (a multiple of 16) of buf (si_stream.hip)
void launch_stream_read(const void *buf, size_t bytes, uint32_t *sink, int workgroups,
                        int depth, hipStream_t st);
}  // namespace si
