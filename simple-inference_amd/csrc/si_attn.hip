// si_attn.hip -- RoPE + fp16 K/V append, and GQA attention over the fp16
// cache for decode, batched decode and causal prefill.
//
// RoPE (qwen_one_layer.c:172-183) uses cos/sin tables computed on the host
// with the reference's libm calls (as register_fusion.h:364-369 does), so
// the rotation  a' = a*c - b*s,  b' = b*c + a*s  and the fp16 narrowing of
// the new K/V rows are bit-exact given identical projections.
//
// Attention (attention_flash, attention_kernels.h:80-164) is split over the
// context ("flash-decoding"): each workgroup owns one query, one KV group
// (all qheads/kvheads query heads that share it, so every K/V byte is read
// once per query) and one context chunk, runs the scores and the weighted
// V sum on the fp16 matrix cores with an online softmax, and leaves
// (max, sum, unnormalised output) partials; a second kernel merges the
// chunks, normalises and quantizes the result to Q8_0 (the reference's next
// step, qwen_one_layer.c:272).
#include "si_device.hpp"
#include "si_kernels.hpp"

namespace si {

// grid (ntok, qheads + kvheads), block hdim/2: one thread per rotation pair.
__global__ void k_rope_kv(const float *__restrict__ qkv, int ldqkv, int qheads, int kvheads,
                          int hdim, int pos0, int pos_step, int max_pos,
                          const int *__restrict__ ctx_dev,
                          const float *__restrict__ rc, const float *__restrict__ rs,
                          float *__restrict__ q_out, uint16_t *__restrict__ kc,
                          uint16_t *__restrict__ vc, size_t kv_seq_stride) {
    const int t = blockIdx.x, h = blockIdx.y, i = threadIdx.x;
    const int half = hdim >> 1;
    const int pos = ctx_dev ? ctx_dev[t] - 1 : pos0 + t * pos_step;
    if (pos < 0 || pos >= max_pos) return;  // device-supplied contexts are not host-checked
    const float c = rc[(size_t)pos * half + i], s = rs[(size_t)pos * half + i];
    const float *row = qkv + (size_t)t * ldqkv;
    const int qd = qheads * hdim, kvd = kvheads * hdim;
    if (h < qheads) {
        const float a = row[h * hdim + i], b = row[h * hdim + i + half];
        float *qo = q_out + (size_t)t * qd + h * hdim;
        qo[i] = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s));
        qo[i + half] = __fadd_rn(__fmul_rn(b, c), __fmul_rn(a, s));
    } else {
        const int g = h - qheads;
        const float a = row[qd + g * hdim + i], b = row[qd + g * hdim + i + half];
        const float ka = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s));
        const float kb = __fadd_rn(__fmul_rn(b, c), __fmul_rn(a, s));
        const size_t base = (size_t)t * kv_seq_stride + (size_t)pos * kvd + (size_t)g * hdim;
        kc[base + i] = f2h(ka);
        kc[base + i + half] = f2h(kb);
        vc[base + i] = f2h(row[qd + kvd + g * hdim + i]);
        vc[base + i + half] = f2h(row[qd + kvd + g * hdim + i + half]);
    }
}

void launch_rope_kv(const float *qkv, int ldqkv, int ntok, int qheads, int kvheads, int hdim,
                    int pos0, int pos_step, int max_pos, const int *ctx_dev, const float *rc,
                    const float *rs, float *q_out, uint16_t *kc, uint16_t *vc,
                    size_t kv_seq_stride, hipStream_t st) {
    if (ntok <= 0) return;
    hipLaunchKernelGGL(k_rope_kv, dim3(ntok, qheads + kvheads), dim3(hdim / 2), 0, st, qkv,
                       ldqkv, qheads, kvheads, hdim, pos0, pos_step, max_pos, ctx_dev, rc, rs,
                       q_out, kc, vc, kv_seq_stride);
}

constexpr int ATT_MAXPER = 16;  // query heads per KV group (the 16 MFMA columns)

// grid (qheads, nq), block hdim: merge chunks, normalise, quantize to Q8_0.
__global__ void k_attn_combine(int qheads, int hdim, int nsplit, const float *__restrict__ ws_m,
                               const float *__restrict__ ws_l, const float *__restrict__ ws_o,
                               float *__restrict__ attn, int8_t *__restrict__ qs,
                               uint16_t *__restrict__ d, int16_t *__restrict__ bsum) {
    const int h = blockIdx.x, qi = blockIdx.y, jj = threadIdx.x;
    const size_t base = ((size_t)qi * qheads + h) * nsplit;
    float mx = -INFINITY;
    for (int s = 0; s < nsplit; ++s) mx = fmaxf(mx, ws_m[base + s]);
    float l = 0.0f, acc = 0.0f;
    for (int s = 0; s < nsplit; ++s) {
        const float w = expf(ws_m[base + s] - mx);  // empty chunk: m = -inf -> 0
        l = fmaf(ws_l[base + s], w, l);
        acc = fmaf(ws_o[(base + s) * hdim + jj], w, acc);
    }
    // context <= 0 (only possible through ctx_dev): zero output, as
    // attention_kernels.h:95-98 does
    const float y = mx == -INFINITY ? 0.0f : acc * (1.0f / l);
    const size_t off = (size_t)qi * qheads * hdim + (size_t)h * hdim + jj;
    attn[off] = y;
    if (qs) {
        uint16_t dbits;
        int sum;
        const int q = quant_block_lane(y, dbits, sum);
        qs[off] = (int8_t)q;
        if ((jj & 31) == 0) {
            const size_t bi = off / SI_QK;
            d[bi] = dbits;
            if (bsum) bsum[bi] = (int16_t)sum;
        }
    }
}

// ===========================================================================
// Matrix-core decode attention.
//
// One workgroup owns (query, KV group, context chunk); its 4 wavefronts take
// every 4th 16-position tile of the chunk.  Per tile a wavefront computes
//     S^T[pos][head] = K[pos][:] . Q[head][:]        (v_mfma_f32_16x16x32_f16)
// with the GQA group's query heads as the 16 MFMA columns (padded), then an
// online-softmax update per head, then
//     O^T[d][head] += V^T[d][pos] . P[pos][head]     (v_mfma_f32_16x16x16_f16)
// K is read straight from HBM as the MFMA A operand (16 B per lane); V rows
// are staged through LDS and read transposed (the MFMA reduction runs over
// positions).  Q and P are fp32 values split into fp16 hi + lo halves
// (x = hi + lo to 22 bits), each product done twice, so the result keeps
// fp32-level accuracy although the matrix cores take fp16.  Each wavefront's
// (max, sum, unnormalised O) is one partial; k_attn_combine merges them.
//
// Layouts (16x16 tiles): MFMA output element (i, j) is held by lane
// j + 16*(i/4), register i%4.  The A/B operands give lane l row/column l%16
// and the k-slice (l/16); A and B use the same k-slice per lane, so any
// consistent assignment of reduction indices to slices is exact.
// ===========================================================================
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int MA_TILE = 16;            // positions per wavefront tile
constexpr int MA_SUPER = 4 * MA_TILE;  // positions per workgroup step
constexpr int MA_VPAD = 16;            // halves of LDS row padding (bank spread)

__device__ __forceinline__ void split_hi_lo(float x, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

template <int D>
__global__ void __launch_bounds__(256) k_attn_decode_mfma(
    const float *__restrict__ q, int qheads, int kvheads, const uint16_t *__restrict__ kc,
    const uint16_t *__restrict__ vc, size_t kv_seq_stride, const int *__restrict__ ctx_dev,
    int ctx0, int ctx_step, int max_ctx, int chunk, float scale, float *__restrict__ ws_m,
    float *__restrict__ ws_l, float *__restrict__ ws_o) {
    constexpr int KS = D / 32;  // k-steps of the score MFMA
    constexpr int DT = D / 16;  // d-tiles of the PV MFMA
    constexpr int VROW = D + MA_VPAD;
    __shared__ __attribute__((aligned(16))) _Float16 v_lds[MA_SUPER * VROW];

    const int sp = blockIdx.x, g = blockIdx.y, qi = blockIdx.z;
    const int nsplit4 = gridDim.x * 4;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int per = qheads / kvheads;
    int ctx = ctx_dev ? ctx_dev[qi] : ctx0 + qi * ctx_step;
    ctx = min(ctx, max_ctx);
    const int p0 = sp * chunk;
    const int p1 = min(ctx, p0 + chunk);
    const int kvd = kvheads * D;
    const uint16_t *kbase = kc + (size_t)qi * kv_seq_stride + (size_t)g * D;
    const uint16_t *vbase = vc + (size_t)qi * kv_seq_stride + (size_t)g * D;

    // Q^T as the B operand: lane holds Q[head = col][d = 8*grp + 32*ks + 0..7]
    h8 qh[KS], ql[KS];
    {
        const bool hv = col < per;
        const float *qrow = q + (size_t)qi * qheads * D + (size_t)(g * per + (hv ? col : 0)) * D;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = hv ? qrow[32 * ks + 8 * grp + e] : 0.0f;
                _Float16 hi, lo;
                split_hi_lo(x, hi, lo);
                qh[ks][e] = hi;
                ql[ks][e] = lo;
            }
    }
    float m = -INFINITY, lsum = 0.0f;  // running state of head `col`
    f4 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = (f4){0.f, 0.f, 0.f, 0.f};

    for (int s0 = p0; s0 < p1; s0 += MA_SUPER) {
        // stage the step's V rows (clamped to valid rows) into LDS
        constexpr int CHUNKS = MA_SUPER * D / 8;  // 16-byte pieces
#pragma unroll
        for (int c = tid; c < CHUNKS; c += 256) {
            const int r = c / (D / 8), e = (c % (D / 8)) * 8;
            const int pos = min(s0 + r, p1 - 1);
            const uint4 v8 = *(const uint4 *)(vbase + (size_t)pos * kvd + e);
            *(uint4 *)(&v_lds[r * VROW + e]) = v8;
        }
        __syncthreads();
        const int t0 = s0 + MA_TILE * wave;
        if (t0 < p1) {
            // scores: A = K rows (pos = t0 + col), k-slice grp
            const int kpos = min(t0 + col, p1 - 1);
            const uint16_t *krow = kbase + (size_t)kpos * kvd + 8 * grp;
            f4 sacc = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const uint4 kraw = *(const uint4 *)(krow + 32 * ks);
                const h8 ka = __builtin_bit_cast(h8, kraw);
                sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[ks], sacc, 0, 0, 0);
                sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[ks], sacc, 0, 0, 0);
            }
            // lane holds S^T[pos = t0 + 4*grp + r][head = col]
            float s[4];
            float mx = -INFINITY;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int pos = t0 + 4 * grp + r;
                s[r] = pos < p1 ? sacc[r] * scale : -INFINITY;
                mx = fmaxf(mx, s[r]);
            }
            mx = fmaxf(mx, swap16_f(mx));
            mx = fmaxf(mx, swap32_f(mx));
            const float mnew = fmaxf(m, mx);
            const float alpha = expf(m - mnew);  // 0 while m is -inf
            float p[4], ps = 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                p[r] = expf(s[r] - mnew);
                ps += p[r];
            }
            ps += swap16_f(ps);
            ps += swap32_f(ps);
            lsum = lsum * alpha + ps;
            m = mnew;
            h4 ph, pl;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                _Float16 hi, lo;
                split_hi_lo(p[r], hi, lo);
                ph[r] = hi;
                pl[r] = lo;
            }
            // PV: A = V^T[d = 16*dt + col][pos = 4*grp + r] from this wave's LDS rows
            const _Float16 *vw = &v_lds[(MA_TILE * wave + 4 * grp) * VROW + col];
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                h4 va;
#pragma unroll
                for (int r = 0; r < 4; ++r) va[r] = vw[r * VROW + 16 * dt];
                f4 acc = o[dt] * alpha;
                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(va, ph, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pl, acc, 0, 0, 0);
                o[dt] = acc;
            }
        }
        __syncthreads();  // V rows are overwritten by the next step
    }
    // this wavefront's partial: split index sp*4 + wave
    if (col < per) {
        const int h = g * per + col;
        const size_t pi = ((size_t)qi * qheads + h) * nsplit4 + sp * 4 + wave;
        if (grp == 0) {
            ws_m[pi] = m;
            ws_l[pi] = lsum;
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r) ws_o[pi * D + 16 * dt + 4 * grp + r] = o[dt][r];
    }
}

// Context chunks per (query, KV group): enough workgroups to cover the chip
// (>= ~512) while every chunk keeps at least one 64-position step.
int attn_nsplit(int kvheads, int nq, int max_ctx) {
    const int base = kvheads * nq;
    int ns = (512 + base - 1) / base;
    const int maxs = (max_ctx + MA_SUPER - 1) / MA_SUPER;
    if (ns > maxs) ns = maxs;
    return ns < 1 ? 1 : ns;
}

size_t attn_workspace_bytes(int qheads, int hdim, int kvheads, int nq, int max_ctx) {
    const int ns = attn_nsplit(kvheads, nq, max_ctx) * 4;  // one partial per wavefront
    return (size_t)nq * qheads * ns * (hdim + 2) * sizeof(float);
}

bool attn_supported(int qheads, int kvheads, int hdim) {
    return kvheads > 0 && qheads % kvheads == 0 && qheads / kvheads <= ATT_MAXPER &&
           (hdim == 32 || hdim == 64 || hdim == 96 || hdim == 128);
}

void launch_attention(const float *q, int nq, int qheads, int kvheads, int hdim,
                      const uint16_t *kc, const uint16_t *vc, size_t kv_seq_stride,
                      const int *ctx_dev, int ctx0, int ctx_step, int max_ctx, float *attn,
                      int8_t *qs, uint16_t *d, int16_t *bsum, void *workspace,
                      hipStream_t st) {
    if (nq <= 0) return;
    const int ns = attn_nsplit(kvheads, nq, max_ctx);
    int chunk = (max_ctx + ns - 1) / ns;
    chunk = (chunk + MA_SUPER - 1) / MA_SUPER * MA_SUPER;
    const int ns4 = ns * 4;
    float *ws_m = (float *)workspace;
    float *ws_l = ws_m + (size_t)nq * qheads * ns4;
    float *ws_o = ws_l + (size_t)nq * qheads * ns4;
    const float scale = 1.0f / sqrtf((float)hdim);  // attention_kernels.h:86
    const dim3 grid(ns, kvheads, nq);
#define SI_ATTN_LAUNCH(DIM)                                                                  \
    hipLaunchKernelGGL(k_attn_decode_mfma<DIM>, grid, dim3(256), 0, st, q, qheads, kvheads, kc, \
                       vc, kv_seq_stride, ctx_dev, ctx0, ctx_step, max_ctx, chunk, scale, ws_m, \
                       ws_l, ws_o)
    switch (hdim) {
        case 32: SI_ATTN_LAUNCH(32); break;
        case 64: SI_ATTN_LAUNCH(64); break;
        case 96: SI_ATTN_LAUNCH(96); break;
        default: SI_ATTN_LAUNCH(128); break;
    }
#undef SI_ATTN_LAUNCH
    hipLaunchKernelGGL(k_attn_combine, dim3(qheads, nq), dim3(hdim), 0, st, qheads, hdim, ns4,
                       ws_m, ws_l, ws_o, attn, qs, d, bsum);
}

// Merge of nsplit partials laid out as [nq][qheads][nsplit] (m, l) and
// [nq][qheads][nsplit][hdim] (o) in one workspace.
void launch_attn_combine(int nq, int qheads, int hdim, int nsplit, const void *workspace,
                         float *attn, int8_t *qs, uint16_t *d, int16_t *bsum, hipStream_t st) {
    const float *ws_m = (const float *)workspace;
    const float *ws_l = ws_m + (size_t)nq * qheads * nsplit;
    const float *ws_o = ws_l + (size_t)nq * qheads * nsplit;
    hipLaunchKernelGGL(k_attn_combine, dim3(qheads, nq), dim3(hdim), 0, st, qheads, hdim, nsplit,
                       ws_m, ws_l, ws_o, attn, qs, d, bsum);
}

// Test entry: one 16x16 tile with each of the two f16 matrix-core shapes,
// operands placed with the lane layouts above, output scattered back to
// row-major with the assumed output layout.  A [16][32], B [32][16] halves.
__global__ void k_debug_mfma_f16(const _Float16 *A, const _Float16 *B, float *D32, float *D16) {
    const int lane = threadIdx.x, col = lane & 15, grp = lane >> 4;
    h8 a8, b8;
    for (int e = 0; e < 8; ++e) {
        a8[e] = A[col * 32 + 8 * grp + e];
        b8[e] = B[(8 * grp + e) * 16 + col];
    }
    f4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a8, b8, (f4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    for (int r = 0; r < 4; ++r) D32[(4 * grp + r) * 16 + col] = d[r];
    h4 a4, b4;
    for (int e = 0; e < 4; ++e) {
        a4[e] = A[col * 32 + 4 * grp + e];
        b4[e] = B[(4 * grp + e) * 16 + col];
    }
    f4 d2 = __builtin_amdgcn_mfma_f32_16x16x16f16(a4, b4, (f4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    for (int r = 0; r < 4; ++r) D16[(4 * grp + r) * 16 + col] = d2[r];
}

void launch_debug_mfma_f16(const void *A, const void *B, float *D32, float *D16, hipStream_t st) {
    hipLaunchKernelGGL(k_debug_mfma_f16, dim3(1), dim3(64), 0, st, (const _Float16 *)A,
                       (const _Float16 *)B, D32, D16);
}

}  // namespace si
