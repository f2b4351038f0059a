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
// once per query) and one context chunk, streams 256-position tiles with an
// online softmax, and leaves (max, sum, unnormalised output) partials; a
// second kernel merges the chunks, normalises and quantizes the result to
// Q8_0 (the reference's next step, qwen_one_layer.c:272).
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

constexpr int ATT_TILE = 256;  // positions per tile (= threads per workgroup)
constexpr int ATT_MAXPER = 8;  // query heads per KV group supported
constexpr int ATT_MAXD = 128;  // head dim supported

// grid (nsplit, kvheads, nq), block 256.
__global__ void __launch_bounds__(256) k_attn_partial(
    const float *__restrict__ q, int qheads, int kvheads, int hdim,
    const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc, size_t kv_seq_stride,
    const int *__restrict__ ctx_dev, int ctx0, int ctx_step, int max_ctx, int chunk, float scale,
    float *__restrict__ ws_m, float *__restrict__ ws_l, float *__restrict__ ws_o) {
    __shared__ float q_s[ATT_MAXPER * ATT_MAXD];
    __shared__ float p_s[ATT_MAXPER][ATT_TILE];
    __shared__ float m_s[ATT_MAXPER], l_s[ATT_MAXPER], a_s[ATT_MAXPER];

    const int sp = blockIdx.x, g = blockIdx.y, qi = blockIdx.z;
    const int nsplit = gridDim.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int per = qheads / kvheads;
    int ctx = ctx_dev ? ctx_dev[qi] : ctx0 + qi * ctx_step;
    ctx = min(ctx, max_ctx);  // device-supplied contexts are not host-checked
    const int p0 = sp * chunk;
    const int p1 = min(ctx, p0 + chunk);
    const int kvd = kvheads * hdim;
    const uint16_t *kbase = kc + (size_t)qi * kv_seq_stride + (size_t)g * hdim;
    const uint16_t *vbase = vc + (size_t)qi * kv_seq_stride + (size_t)g * hdim;

    for (int i = tid; i < per * hdim; i += 256)
        q_s[i] = q[(size_t)qi * qheads * hdim + (size_t)g * per * hdim + i];
    if (tid < per) {
        m_s[tid] = -INFINITY;
        l_s[tid] = 0.0f;
    }
    // outputs owned by this thread: o_idx = tid + 256*r over per*hdim
    float o[4] = {0.f, 0.f, 0.f, 0.f};
    __syncthreads();

    for (int t0 = p0; t0 < p1; t0 += ATT_TILE) {
        const int p = t0 + tid;
        // scores for position p, all heads of the group
        float sc[ATT_MAXPER];
#pragma unroll
        for (int hh = 0; hh < ATT_MAXPER; ++hh) sc[hh] = 0.0f;
        if (p < p1) {
            const uint16_t *kr = kbase + (size_t)p * kvd;
            for (int d0 = 0; d0 < hdim; d0 += 8) {
                const uint4 kv8 = *(const uint4 *)(kr + d0);
                const uint32_t kw[4] = {kv8.x, kv8.y, kv8.z, kv8.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float kf = h2f_fast((uint16_t)(kw[e >> 1] >> (16 * (e & 1))));
#pragma unroll
                    for (int hh = 0; hh < ATT_MAXPER; ++hh)
                        if (hh < per) sc[hh] = fmaf(q_s[hh * hdim + d0 + e], kf, sc[hh]);
                }
            }
        }
#pragma unroll
        for (int hh = 0; hh < ATT_MAXPER; ++hh)
            if (hh < per) p_s[hh][tid] = p < p1 ? sc[hh] * scale : -INFINITY;
        __syncthreads();
        // per-head online-softmax update (one wavefront per head)
        for (int hh = wave; hh < per; hh += 4) {
            float mx = -INFINITY;
            for (int i = lane; i < ATT_TILE; i += 64) mx = fmaxf(mx, p_s[hh][i]);
            mx = wave_max(mx);
            const float mold = m_s[hh];
            const float mnew = fmaxf(mold, mx);
            float sum = 0.0f;
            for (int i = lane; i < ATT_TILE; i += 64) {
                const float e = expf(p_s[hh][i] - mnew);
                p_s[hh][i] = e;
                sum += e;
            }
            sum = wave_sum(sum);
            if (lane == 0) {
                const float alpha = expf(mold - mnew);  // 0 on the first tile
                a_s[hh] = alpha;
                l_s[hh] = l_s[hh] * alpha + sum;
                m_s[hh] = mnew;
            }
        }
        __syncthreads();
        const int np = min(ATT_TILE, p1 - t0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int oi = tid + 256 * r;
            if (oi < per * hdim) {
                const int hh = oi / hdim, jj = oi - hh * hdim;
                float acc = o[r] * a_s[hh];
                const uint16_t *vr = vbase + (size_t)t0 * kvd + jj;
                for (int t = 0; t < np; ++t)
                    acc = fmaf(p_s[hh][t], h2f_fast(vr[(size_t)t * kvd]), acc);
                o[r] = acc;
            }
        }
        __syncthreads();
    }
    // partials: [qi][h][sp]
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int oi = tid + 256 * r;
        if (oi < per * hdim) {
            const int hh = oi / hdim, jj = oi - hh * hdim;
            const int h = g * per + hh;
            ws_o[(((size_t)qi * qheads + h) * nsplit + sp) * hdim + jj] = o[r];
        }
    }
    if (tid < per) {
        const int h = g * per + tid;
        ws_m[((size_t)qi * qheads + h) * nsplit + sp] = m_s[tid];
        ws_l[((size_t)qi * qheads + h) * nsplit + sp] = l_s[tid];
    }
}

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

int attn_nsplit(int kvheads, int nq, int max_ctx) {
    // aim for >= ~512 workgroups, chunks of at least one 256-position tile
    const int base = kvheads * nq;
    int ns = (512 + base - 1) / base;
    const int maxs = (max_ctx + ATT_TILE - 1) / ATT_TILE;
    if (ns > maxs) ns = maxs;
    if (ns < 1) ns = 1;
    return ns;
}

size_t attn_workspace_bytes(int qheads, int hdim, int kvheads, int nq, int max_ctx) {
    const int ns = attn_nsplit(kvheads, nq, max_ctx);
    return (size_t)nq * qheads * ns * (hdim + 2) * sizeof(float);
}

bool attn_supported(int qheads, int kvheads, int hdim) {
    return kvheads > 0 && qheads % kvheads == 0 && qheads / kvheads <= ATT_MAXPER &&
           hdim <= ATT_MAXD && hdim % 32 == 0 && hdim >= 32;
}

void launch_attention(const float *q, int nq, int qheads, int kvheads, int hdim,
                      const uint16_t *kc, const uint16_t *vc, size_t kv_seq_stride,
                      const int *ctx_dev, int ctx0, int ctx_step, int max_ctx, float *attn,
                      int8_t *qs, uint16_t *d, int16_t *bsum, void *workspace,
                      hipStream_t st) {
    if (nq <= 0) return;
    const int ns = attn_nsplit(kvheads, nq, max_ctx);
    int chunk = (max_ctx + ns - 1) / ns;
    chunk = (chunk + ATT_TILE - 1) / ATT_TILE * ATT_TILE;
    float *ws_m = (float *)workspace;
    float *ws_l = ws_m + (size_t)nq * qheads * ns;
    float *ws_o = ws_l + (size_t)nq * qheads * ns;
    const float scale = 1.0f / sqrtf((float)hdim);  // attention_kernels.h:86
    hipLaunchKernelGGL(k_attn_partial, dim3(ns, kvheads, nq), dim3(256), 0, st, q, qheads,
                       kvheads, hdim, kc, vc, kv_seq_stride, ctx_dev, ctx0, ctx_step, max_ctx,
                       chunk, scale, ws_m, ws_l, ws_o);
    hipLaunchKernelGGL(k_attn_combine, dim3(qheads, nq), dim3(hdim), 0, st, qheads, hdim, ns,
                       ws_m, ws_l, ws_o, attn, qs, d, bsum);
}

}  // namespace si
