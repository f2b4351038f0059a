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

// grid (ntok, ceil((qheads + kvheads) * hdim/2 / 256)), block 256: one
// thread per rotation pair (head h = j / (hdim/2), pair i = j % (hdim/2) of
// token t), so a workgroup covers several heads of a token (half-wavefront
// workgroups per head had left most lanes idle).  With a page table
// (pg.pages != nullptr) token t's K/V row goes to the pool row of sequence
// t's position pos (kv_seq_stride unused).
constexpr int ROPE_T = 256;
__global__ void __launch_bounds__(ROPE_T) k_rope_kv(
    const float *__restrict__ qkv, int ldqkv, int qheads, int kvheads, int hdim, int pos0,
    int pos_step, int max_pos, const int *__restrict__ ctx_dev, const float *__restrict__ rc,
    const float *__restrict__ rs, float *__restrict__ q_out, uint16_t *__restrict__ kc,
    uint16_t *__restrict__ vc, size_t kv_seq_stride, KvPages pg) {
    const int t = blockIdx.x;
    const int half = hdim >> 1;
    const int j = blockIdx.y * ROPE_T + threadIdx.x;
    if (j >= (qheads + kvheads) * half) return;
    const int h = j / half, i = j - h * half;
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
        const size_t base = pg.row(t, pos, kv_seq_stride, kvd) + (size_t)g * hdim;
        kc[base + i] = f2h(ka);
        kc[base + i + half] = f2h(kb);
        vc[base + i] = f2h(row[qd + kvd + g * hdim + i]);
        vc[base + i + half] = f2h(row[qd + kvd + g * hdim + i + half]);
    }
}

void launch_rope_kv(const float *qkv, int ldqkv, int ntok, int qheads, int kvheads, int hdim,
                    int pos0, int pos_step, int max_pos, const int *ctx_dev, const float *rc,
                    const float *rs, float *q_out, uint16_t *kc, uint16_t *vc,
                    size_t kv_seq_stride, hipStream_t st, KvPages pg) {
    if (ntok <= 0) return;
    const int pairs = (qheads + kvheads) * (hdim / 2);
    SI_LAUNCH(k_rope_kv, dim3(ntok, (pairs + ROPE_T - 1) / ROPE_T), dim3(ROPE_T), 0, st, qkv,
              ldqkv, qheads, kvheads, hdim, pos0, pos_step, max_pos, ctx_dev, rc, rs,
              q_out, kc, vc, kv_seq_stride, pg);
}

constexpr int ATT_MAXPER = 16;  // query heads per KV group (the 16 MFMA columns)

// grid (qheads, nq), block hdim: merge chunks, normalise, quantize to Q8_0
// (tq/td, optional: the Q8_0 also operand-tiled, q8_tiled_byte).
__global__ void k_attn_combine(int qheads, int hdim, int nsplit, const float *__restrict__ ws_m,
                               const float *__restrict__ ws_l, const float *__restrict__ ws_o,
                               float *__restrict__ attn, int8_t *__restrict__ qs,
                               uint16_t *__restrict__ d, int16_t *__restrict__ bsum,
                               int8_t *__restrict__ tq, uint16_t *__restrict__ td) {
    const int h = blockIdx.x, qi = blockIdx.y, jj = threadIdx.x;
    const size_t base = ((size_t)qi * qheads + h) * nsplit;
    // unrolled: the loads of 8 splits are in flight together
    float mx = -INFINITY;
#pragma unroll 8
    for (int s = 0; s < nsplit; ++s) mx = fmaxf(mx, ws_m[base + s]);
    float l = 0.0f, acc = 0.0f;
#pragma unroll 8
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
        if (tq) {
            const int qd = qheads * hdim;
            const size_t pb = (size_t)(qi >> 5) * (qd / SI_QK) + (h * hdim + jj) / SI_QK;
            tq[q8_tiled_byte(pb, qi & 31, jj & 31)] = (int8_t)q;
            if ((jj & 31) == 0) td[pb * 32 + (qi & 31)] = dbits;
        }
    }
}

// Block-wide max or sum of one value per thread (blockDim.x a multiple of
// 64, at most 1024): wave reduction, then the wave results in wave order.
__device__ __forceinline__ float block_reduce_1024(float v, float *red, bool is_max) {
    // wave reduction, then the 16 wave results in a fixed order
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(v, off, 64);
        v = is_max ? fmaxf(v, o) : v + o;
    }
    const int wave = threadIdx.x >> 6;
    __syncthreads();  // red[] may still be read from the previous reduction
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
    return r;
}

// k_attn_combine for many partials (>= 32 per head): grid (qheads, nq),
// block P*hdim, P = 1024/hdim.  The max is taken block-wide; thread
// (group, column) merges the partials s = group, group + P, ... and the P
// group sums are added in group order, so the loads of P partials are in
// flight at once instead of one after another.
__global__ __launch_bounds__(1024) void k_attn_combine_wide(
    int qheads, int hdim, int nsplit, const float *__restrict__ ws_m,
    const float *__restrict__ ws_l, const float *__restrict__ ws_o, float *__restrict__ attn,
    int8_t *__restrict__ qs, uint16_t *__restrict__ d, int16_t *__restrict__ bsum,
    int8_t *__restrict__ tq, uint16_t *__restrict__ td) {
    __shared__ float red_o[1024];
    __shared__ float red_l[32];
    __shared__ float red_m[16];
    const int h = blockIdx.x, qi = blockIdx.y, tid = threadIdx.x;
    const int P = blockDim.x / hdim, grp = tid / hdim, jj = tid % hdim;
    const size_t base = ((size_t)qi * qheads + h) * nsplit;
    float mx = -INFINITY;
    for (int s = tid; s < nsplit; s += blockDim.x) mx = fmaxf(mx, ws_m[base + s]);
    mx = block_reduce_1024(mx, red_m, true);
    float l = 0.0f, acc = 0.0f;
#pragma unroll 4
    for (int s = grp; s < nsplit; s += P) {
        const float w = expf(ws_m[base + s] - mx);  // empty chunk: m = -inf -> 0
        l = fmaf(ws_l[base + s], w, l);
        acc = fmaf(ws_o[(base + s) * hdim + jj], w, acc);
    }
    red_o[tid] = acc;
    if (jj == 0) red_l[grp] = l;
    __syncthreads();
    if (tid >= hdim) return;  // no barrier below
    float a = red_o[jj], lt = red_l[0];
    for (int g = 1; g < P; ++g) {
        a += red_o[g * hdim + jj];
        lt += red_l[g];
    }
    const float y = mx == -INFINITY ? 0.0f : a * (1.0f / lt);
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
        if (tq) {
            const int qd = qheads * hdim;
            const size_t pb = (size_t)(qi >> 5) * (qd / SI_QK) + (h * hdim + jj) / SI_QK;
            tq[q8_tiled_byte(pb, qi & 31, jj & 31)] = (int8_t)q;
            if ((jj & 31) == 0) td[pb * 32 + (qi & 31)] = dbits;
        }
    }
}

// Either combine kernel by partial count.
static void combine(int qheads, int hdim, int nq, int nsplit, const float *ws_m,
                    const float *ws_l, const float *ws_o, float *attn, int8_t *qs, uint16_t *d,
                    int16_t *bsum, hipStream_t st, int8_t *tq = nullptr, uint16_t *td = nullptr) {
    if (nsplit >= 32)
        SI_LAUNCH(k_attn_combine_wide, dim3(qheads, nq), dim3(1024 / hdim * hdim), 0, st,
                  qheads, hdim, nsplit, ws_m, ws_l, ws_o, attn, qs, d, bsum, tq, td);
    else
        SI_LAUNCH(k_attn_combine, dim3(qheads, nq), dim3(hdim), 0, st, qheads, hdim,
                  nsplit, ws_m, ws_l, ws_o, attn, qs, d, bsum, tq, td);
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
// fp32-level accuracy although the matrix cores take fp16.  The 4 wavefronts'
// (max, sum, unnormalised O) are merged in LDS into one partial per
// workgroup; k_attn_combine merges the chunks.
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
    float *__restrict__ ws_l, float *__restrict__ ws_o, KvPages pg, int kv_row) {
    constexpr int KS = D / 32;  // k-steps of the score MFMA
    constexpr int DT = D / 16;  // d-tiles of the PV MFMA
    constexpr int VROW = D + MA_VPAD;
    __shared__ __attribute__((aligned(16))) _Float16 v_lds[MA_SUPER * VROW];

    const int sp = blockIdx.x, g = blockIdx.y, qi = blockIdx.z;
    const int nsplit = gridDim.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int per = qheads / kvheads;
    int ctx = ctx_dev ? ctx_dev[qi] : ctx0 + qi * ctx_step;
    ctx = min(ctx, max_ctx);
    const int p0 = sp * chunk;
    const int p1 = min(ctx, p0 + chunk);
    const int kvd = kv_row;  // elements per cache row (kvheads * D unless a caller
                             // passes one KV group of a wider cache)
    const uint16_t *kbase = kc + (size_t)g * D;  // + pg.row(qi, pos, ...) per row
    const uint16_t *vbase = vc + (size_t)g * D;

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
            const uint4 v8 = *(const uint4 *)(vbase + pg.row(qi, pos, kv_seq_stride, kvd) + e);
            *(uint4 *)(&v_lds[r * VROW + e]) = v8;
        }
        __syncthreads();
        const int t0 = s0 + MA_TILE * wave;
        if (t0 < p1) {
            // scores: A = K rows (pos = t0 + col), k-slice grp
            const int kpos = min(t0 + col, p1 - 1);
            const uint16_t *krow = kbase + pg.row(qi, kpos, kv_seq_stride, kvd) + 8 * grp;
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
    // merge the 4 wavefronts' states into the workgroup's partial (split
    // index sp): each wave rescales its sums to the common max, and the
    // scaled outputs are added in wave order through LDS
    __shared__ float mrg_m[4][16], mrg_l[4][16];
    __shared__ float mrg_o[16 * D];
    if (grp == 0) {
        mrg_m[wave][col] = m;
        mrg_l[wave][col] = lsum;
    }
    __syncthreads();
    const float mall = fmaxf(fmaxf(mrg_m[0][col], mrg_m[1][col]), fmaxf(mrg_m[2][col], mrg_m[3][col]));
    const float w = m == -INFINITY ? 0.0f : expf(m - mall);  // a wave with no positions adds 0
    for (int k = 0; k < 4; ++k) {
        if (wave == k)
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int idx = col * D + 16 * dt + 4 * grp + r;
                    const float v = o[dt][r] * w;
                    mrg_o[idx] = k == 0 ? v : mrg_o[idx] + v;
                }
        __syncthreads();
    }
    const size_t pbase = ((size_t)qi * qheads + (size_t)g * per) * nsplit + sp;  // head col 0
    if (wave == 0 && grp == 0 && col < per) {
        float l = 0.0f;
        for (int k = 0; k < 4; ++k)
            if (mrg_m[k][col] != -INFINITY) l += mrg_l[k][col] * expf(mrg_m[k][col] - mall);
        ws_m[pbase + (size_t)col * nsplit] = mall;
        ws_l[pbase + (size_t)col * nsplit] = l;
    }
    for (int idx = tid; idx < per * D; idx += 256)
        ws_o[(pbase + (size_t)(idx / D) * nsplit) * D + idx % D] = mrg_o[idx];
}

// ===========================================================================
// Causal prefill attention (flash attention over 32 x 32 tiles).
//
// One workgroup owns one KV group, 32 consecutive query tokens and NW of
// the group's query heads (blockIdx.z picks which NW); wavefront w computes
// one head for those tokens, so each K/V tile staged in LDS serves NW heads.
// Fewer heads per workgroup give more, shorter workgroups where the tokens
// alone would not fill the CUs.  Per 32-position K/V tile a
// wavefront computes
//     S^T[pos][tok] = K[pos][:] . Q[tok][:]          (v_mfma_f32_32x32x16_f16)
// (Q split into fp16 hi + lo halves, each product done twice, for fp32-level
// scores), applies the causal mask and the online softmax per token (a
// token's 32 scores sit in one lane and its partner lane ^ 32), then
//     O^T[d][tok] += V^T[d][pos] . P^T[pos][tok]     (v_mfma_f32_32x32x16_f16)
// The running max and sum of a token then live in the lanes that hold its O^T
// column, so the rescale is a per-lane multiply.  P is split into fp16 hi +
// lo halves like Q (an fp16-only P moves outputs by ~1e-3 relative, enough
// to break the prefill == sequential decode agreement the reference tests).
// V is staged transposed so the A operand of the PV product is two 8-byte
// LDS reads per lane.  The epilogue normalises, stores fp32 and quantizes
// every 32-dim block to Q8_0 (qwen_one_layer.c:272) in registers.
//
// 32x32 layouts: output (i, j) is held by lane j + 32*((i/4)%2), register
// (i%4) + 4*(i/8); operand lane l supplies row (or column) l%32 and k-slice
// l/32.  A and B use the same k assignment, so any consistent assignment of
// reduction indices to (slice, element) is exact.
// ===========================================================================
typedef float f16v __attribute__((ext_vector_type(16)));
typedef int pf_v4i __attribute__((ext_vector_type(4)));

constexpr int PF_T = 32;      // query tokens per workgroup, positions per K/V tile
constexpr int PF_KPAD = 8;    // halves of padding per K row
constexpr int PF_VPAD = 4;    // halves of padding per V^T row (18-dword rows)

// Causal balance: query tiles qsplit..nqt-1 (nsplit of them) run as two
// workgroups each, over K/V tiles [0, cap) and [cap, end); their partial
// states go to ws_* as [token - 32*qsplit][head][2] and k_attn_combine
// merges them.
struct PrefillSplit {
    int nqt, qsplit, nsplit, cap;
    float *ws_m, *ws_l, *ws_o;
};

template <int D, int NW>
struct PrefillLds {
    static constexpr int KROW = D + PF_KPAD, VROW = PF_T + PF_VPAD;
    static constexpr size_t bytes() { return (size_t)(PF_T * KROW + D * VROW) * 2; }
};

template <int D, int NW>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2))) k_attn_prefill(
    const float *__restrict__ q, int ntok, int qheads, int kvheads, int pos0,
    const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc, float scale,
    float *__restrict__ attn, int8_t *__restrict__ qs, uint16_t *__restrict__ qd,
    int16_t *__restrict__ bsum, PrefillSplit sp) {
    using Lds = PrefillLds<D, NW>;
    constexpr int NT = NW * 64, KS = D / 16, DT = D / 32;
    constexpr int KPIECES = PF_T * D / 8;        // 16-byte K pieces per tile
    constexpr int VITEMS = (PF_T / 2) * (D / 8); // (position pair, 8 dims) per tile
    constexpr int KPT = (KPIECES + NT - 1) / NT, VPT = (VITEMS + NT - 1) / NT;
    extern __shared__ __attribute__((aligned(16))) uint8_t pf_sm[];
    _Float16 *k_l = (_Float16 *)pf_sm;                  // [PF_T][KROW]
    _Float16 *vt_l = k_l + PF_T * Lds::KROW;            // [D][VROW]

    // work unit of this workgroup, longest first: the first K/V halves of
    // the split query tiles, then their second halves interleaved with the
    // unsplit tiles (unit -1: whole range, 0: [0, cap), 1: [cap, end)).
    // Odd head subsets take the units in reverse order: the workgroups that
    // share a CU (dispatched a whole subset apart) then pair a long query
    // tile with a short one (7B, 2048 tokens: 150 -> 118 us).
    int qt, unit;
    {
        const int b = (blockIdx.z & 1) ? gridDim.x - 1 - blockIdx.x : blockIdx.x;
        const int S = sp.nsplit, Q0 = sp.qsplit;
        if (b < S) {
            qt = sp.nqt - 1 - b;
            unit = 0;
        } else {
            const int bp = b - S, m2 = min(S, Q0);
            if (bp < 2 * m2) {
                const int k = bp >> 1;
                qt = (bp & 1) ? Q0 - 1 - k : sp.nqt - 1 - k;
                unit = (bp & 1) ? -1 : 1;
            } else {
                const int r = m2 + (bp - 2 * m2);
                qt = S > Q0 ? sp.nqt - 1 - r : Q0 - 1 - r;
                unit = S > Q0 ? 1 : -1;
            }
        }
    }
    const int g = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int t = lane & 31, hh = lane >> 5;
    const int per = qheads / kvheads;
    const int hw = blockIdx.z * NW + w;  // head within the group
    const bool active = hw < per;
    const int h = g * per + (active ? hw : 0);
    const int tq = qt * PF_T + t;  // this lane's query token
    const int ptq = pos0 + tq;     // its position: it sees cache rows 0..ptq
    const int kvd = kvheads * D;
    const int last = min(pos0 + qt * PF_T + PF_T - 1, pos0 + ntok - 1);  // last cache row used
    const int it0 = unit == 1 ? sp.cap : 0;
    const int it1 = unit == 0 ? sp.cap : last / PF_T + 1;

    // Q^T as the B operand of the score MFMA: column tok = t, k-slice hh
    h8 qh[KS], ql[KS];
    {
        const bool ok = active && tq < ntok;
        const float *qrow = q + ((size_t)(ok ? tq : 0) * qheads + h) * D;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const float4 a = *(const float4 *)(qrow + 16 * ks + 8 * hh);
            const float4 b = *(const float4 *)(qrow + 16 * ks + 8 * hh + 4);
            const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                _Float16 hi, lo;
                split_hi_lo(ok ? x[e] : 0.0f, hi, lo);
                qh[ks][e] = hi;
                ql[ks][e] = lo;
            }
        }
    }

    // register staging of one K/V tile (rows clamped to `last`; the clamped
    // duplicates lie past every token's causal limit and are masked)
    // clang vectors, not uint4 structs: arrays of those stay in registers
    pf_v4i rk[KPT], rv[VPT][2];
    auto load_tile = [&](int kv0) {
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int c = min(tid + NT * i, KPIECES - 1);
            const int r = c / (D / 8), e8 = c % (D / 8);
            const int pos = min(kv0 + r, last);
            rk[i] = *(const pf_v4i *)(kc + (size_t)pos * kvd + (size_t)g * D + 8 * e8);
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int c = min(tid + NT * i, VITEMS - 1);
            const int pr = c % (PF_T / 2), e8 = c / (PF_T / 2);
            const int p0 = min(kv0 + 2 * pr, last), p1 = min(kv0 + 2 * pr + 1, last);
            rv[i][0] = *(const pf_v4i *)(vc + (size_t)p0 * kvd + (size_t)g * D + 8 * e8);
            rv[i][1] = *(const pf_v4i *)(vc + (size_t)p1 * kvd + (size_t)g * D + 8 * e8);
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int c = tid + NT * i;
            if (KPIECES % NT == 0 || c < KPIECES) {
                const int r = c / (D / 8), e8 = c % (D / 8);
                *(pf_v4i *)(k_l + r * Lds::KROW + 8 * e8) = rk[i];
            }
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int c = tid + NT * i;
            if (VITEMS % NT == 0 || c < VITEMS) {
                // position pairs fastest: with 18-dword V^T rows the 64
                // lanes' 4-byte writes hit 64 distinct banks
                const int pr = c % (PF_T / 2), e8 = c / (PF_T / 2);
                const uint32_t a[4] = {(uint32_t)rv[i][0][0], (uint32_t)rv[i][0][1],
                                       (uint32_t)rv[i][0][2], (uint32_t)rv[i][0][3]};
                const uint32_t b[4] = {(uint32_t)rv[i][1][0], (uint32_t)rv[i][1][1],
                                       (uint32_t)rv[i][1][2], (uint32_t)rv[i][1][3]};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    // dims 8*e8 + 2j (low halves) and + 2j + 1 (high halves)
                    const uint32_t lo = __builtin_amdgcn_perm(b[j], a[j], 0x05040100u);
                    const uint32_t hi = __builtin_amdgcn_perm(b[j], a[j], 0x07060302u);
                    *(uint32_t *)(vt_l + (8 * e8 + 2 * j) * Lds::VROW + 2 * pr) = lo;
                    *(uint32_t *)(vt_l + (8 * e8 + 2 * j + 1) * Lds::VROW + 2 * pr) = hi;
                }
            }
        }
    };

    float m = -INFINITY, lsum = 0.0f;  // softmax state of token t (same in both halves)
    f16v o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = (f16v){};

    load_tile(it0 * PF_T);
    for (int it = it0; it < it1; ++it) {
        const int kv0 = it * PF_T;
        store_tile();
        __syncthreads();
        // next tile in flight, unconditionally (the last iteration re-reads
        // its own rows): a conditional load keeps the staging registers in
        // scratch memory and waits for every load
        load_tile(min(kv0 + PF_T, (it1 - 1) * PF_T));
        if (active) {
            // scores S^T[pos = kv0 + i][tok = t]
            f16v sh = (f16v){}, sl = (f16v){};  // two independent MFMA chains
            const _Float16 *krow = k_l + t * Lds::KROW + 8 * hh;  // A row pos = lane % 32
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const h8 ka = *(const h8 *)(krow + 16 * ks);
                sh = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qh[ks], sh, 0, 0, 0);
                sl = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, ql[ks], sl, 0, 0, 0);
            }
            const f16v sacc = sh + sl;
            float sv[16];
            float mx = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int pos = kv0 + 8 * (r >> 2) + 4 * hh + (r & 3);
                sv[r] = pos <= ptq ? sacc[r] * scale : -INFINITY;
                mx = fmaxf(mx, sv[r]);
            }
            mx = fmaxf(mx, swap32_f(mx));
            const float mnew = fmaxf(m, mx);
            // a second K/V half can be entirely past a token's causal limit:
            // its state stays (-inf, 0, 0) instead of turning NaN
            const float mref = mnew == -INFINITY ? 0.0f : mnew;
            const float alpha = __expf(m - mref);
            float ps = 0.0f;
            h8 pbh[2], pbl[2];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float pr = __expf(sv[r] - mref);
                ps += pr;
                _Float16 hi, lo;
                split_hi_lo(pr, hi, lo);
                pbh[r >> 3][r & 7] = hi;
                pbl[r >> 3][r & 7] = lo;
            }
            ps += swap32_f(ps);
            lsum = fmaf(lsum, alpha, ps);
            m = mnew;
            // O^T[d][tok] += V^T[d][pos] P^T[pos][tok]; k-step s2 covers
            // positions 16*s2 + 8*(e/4) + 4*hh + e%4 (e = element 0..7), the
            // positions of registers 8*s2 + e of the score output
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                f16v acc = o[dt] * alpha;
                const _Float16 *vrow = vt_l + (32 * dt + t) * Lds::VROW + 4 * hh;
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2) {
                    const h4 v0 = *(const h4 *)(vrow + 16 * s2);
                    const h4 v1 = *(const h4 *)(vrow + 16 * s2 + 8);
                    const h8 va = (h8){v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pbh[s2], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pbl[s2], acc, 0, 0, 0);
                }
                o[dt] = acc;
            }
        }
        __syncthreads();  // the tile's LDS is rewritten next
    }

    if (!active || tq >= ntok) return;
    // lane holds O[tok][32*dt + 8*(r/4) + 4*hh + r%4] in o[dt][r]
    if (unit >= 0) {  // a half of a split tile: (max, sum, unnormalised O) for the merge
        const size_t pi = ((size_t)(tq - sp.qsplit * PF_T) * qheads + h) * 2 + unit;
        if (hh == 0) {
            sp.ws_m[pi] = m;
            sp.ws_l[pi] = lsum;
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
                *(float4 *)(sp.ws_o + pi * D + 32 * dt + 8 * r4 + 4 * hh) =
                    make_float4(o[dt][4 * r4], o[dt][4 * r4 + 1], o[dt][4 * r4 + 2],
                                o[dt][4 * r4 + 3]);
        return;
    }
    const float inv = 1.0f / lsum;
    const size_t rowoff = ((size_t)tq * qheads + h) * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
        float y[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) y[r] = o[dt][r] * inv;
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
            *(float4 *)(attn + rowoff + 32 * dt + 8 * r4 + 4 * hh) =
                make_float4(y[4 * r4], y[4 * r4 + 1], y[4 * r4 + 2], y[4 * r4 + 3]);
        if (qs) {
            int qv[16];
            uint16_t dbits;
            int sum;
            quant_block_pair16(y, qv, dbits, sum);
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
                *(uint32_t *)(qs + rowoff + 32 * dt + 8 * r4 + 4 * hh) =
                    (uint32_t)(qv[4 * r4] & 0xff) | (uint32_t)(qv[4 * r4 + 1] & 0xff) << 8 |
                    (uint32_t)(qv[4 * r4 + 2] & 0xff) << 16 | (uint32_t)(qv[4 * r4 + 3] & 0xff) << 24;
            if (hh == 0) {
                const size_t bi = (rowoff + 32 * dt) / SI_QK;
                qd[bi] = dbits;
                if (bsum) bsum[bi] = (int16_t)sum;
            }
        }
    }
}

// Causal prefill of ntok tokens at positions pos0.. of one sequence whose
// cache rows 0..pos0+ntok-1 are in place (RoPE'd K, V).
bool attn_prefill_supported(int qheads, int kvheads, int hdim) {
    return kvheads > 0 && qheads % kvheads == 0 && qheads / kvheads <= 16 &&
           (hdim == 32 || hdim == 64 || hdim == 96 || hdim == 128);
}

// Split plan of a causal prefill: when the tiles do not fill the CUs, a
// query tile whose K/V range exceeds half of the longest one is cut in two
// (more workgroups, each at most half the longest range).  A grid that
// already fills the chip is not split: measured at 7B / 2048 tokens (256
// workgroups), the split ran slower (164 + 19 us merge vs 148 us).
static PrefillSplit prefill_split(int ntok, int pos0, int kvheads) {
    PrefillSplit p{};
    p.nqt = (ntok + PF_T - 1) / PF_T;
    auto tiles = [&](int qt) { return min(pos0 + qt * PF_T + PF_T - 1, pos0 + ntok - 1) / PF_T + 1; };
    const int longest = tiles(p.nqt - 1);
    p.cap = (longest + 1) / 2;
    p.qsplit = p.nqt;
    if (longest >= 4 && p.nqt * kvheads < 256)  // short ranges or a full grid: unsplit
        while (p.qsplit > 0 && tiles(p.qsplit - 1) > p.cap) --p.qsplit;
    p.nsplit = p.nqt - p.qsplit;
    return p;
}

size_t attn_prefill_workspace_bytes(int qheads, int hdim, int ntok) {
    return (size_t)ntok * qheads * 2 * (hdim + 2) * sizeof(float);
}

void launch_attn_prefill(const float *q, int ntok, int qheads, int kvheads, int hdim, int pos0,
                         const uint16_t *kc, const uint16_t *vc, float *attn, int8_t *qs,
                         uint16_t *qd, int16_t *bsum, void *workspace, size_t ws_bytes,
                         hipStream_t st) {
    if (ntok <= 0) return;
    const int per = qheads / kvheads;
    PrefillSplit sp = prefill_split(ntok, pos0, kvheads);
    const int rows_split = ntok - sp.qsplit * PF_T;
    if (sp.nsplit > 0 &&
        (!workspace || ws_bytes < attn_prefill_workspace_bytes(qheads, hdim, rows_split))) {
        sp.qsplit = sp.nqt;  // no room for the partial states: unsplit
        sp.nsplit = 0;
    }
    if (sp.nsplit > 0) {
        const size_t np = (size_t)rows_split * qheads * 2;
        sp.ws_m = (float *)workspace;
        sp.ws_l = sp.ws_m + np;
        sp.ws_o = sp.ws_l + np;
    }
    // heads per workgroup: up to 8 (a wider group takes several
    // workgroups), halved while the grid has fewer than ~2 workgroups per CU
    // (down to 2 heads for hdim >= 96, whose one-wavefront workgroups would
    // spill registers)
    const int units = 2 * sp.nsplit + sp.qsplit;
    const int nw_min = hdim >= 96 ? 2 : 1;
    int nw = 8;
    while (nw > nw_min && (size_t)units * kvheads * ((per + nw - 1) / nw) < 512) nw /= 2;
    const dim3 grid(units, kvheads, (per + nw - 1) / nw);
    const float scale = 1.0f / sqrtf((float)hdim);  // attention_kernels.h:86
#define PF_CALL(DIM, NW)                                                                      \
    SI_LAUNCH((k_attn_prefill<DIM, NW>), grid, dim3(NW * 64),                                 \
              (PrefillLds<DIM, NW>::bytes()), st, q, ntok, qheads, kvheads, pos0, kc,         \
              vc, scale, attn, qs, qd, bsum, sp)
#define PF_DIM(DIM)                     \
    switch (nw) {                       \
        case 1: PF_CALL(DIM, 1); break; \
        case 2: PF_CALL(DIM, 2); break; \
        case 4: PF_CALL(DIM, 4); break; \
        default: PF_CALL(DIM, 8);       \
    }
    switch (hdim) {
        case 32: PF_DIM(32); break;
        case 64: PF_DIM(64); break;
        case 96: PF_DIM(96); break;
        default: PF_DIM(128); break;
    }
#undef PF_DIM
#undef PF_CALL
    if (sp.nsplit > 0) {
        const size_t t0 = (size_t)sp.qsplit * PF_T, qd_ = (size_t)qheads * hdim;
        SI_LAUNCH(k_attn_combine, dim3(qheads, rows_split), dim3(hdim), 0, st, qheads,
                  hdim, 2, sp.ws_m, sp.ws_l, sp.ws_o, attn + t0 * qd_,
                  qs ? qs + t0 * qd_ : nullptr, qs ? qd + t0 * qd_ / SI_QK : nullptr,
                  bsum ? bsum + t0 * qd_ / SI_QK : nullptr, (int8_t *)nullptr,
                  (uint16_t *)nullptr);
    }
}

// Context chunks per (query, KV group): enough workgroups to cover the chip
// (>= ~512) while every chunk keeps at least one 64-position step.
int attn_nsplit(int kvheads, int nq, int max_ctx) {
    const int base = kvheads * nq;
    int ns = (512 + base - 1) / base;
    // down to one workgroup step per chunk: the many partials this leaves
    // for a single query go to the wide combine kernel (7B, ctx 4096, cold
    // cache, before the in-workgroup merge: 4-step chunks 22.9 us, 1-step
    // 19.9 us)
    const int maxs = (max_ctx + MA_SUPER - 1) / MA_SUPER;
    if (ns > maxs) ns = maxs;
    return ns < 1 ? 1 : ns;
}

size_t attn_workspace_bytes(int qheads, int hdim, int kvheads, int nq, int max_ctx) {
    const int ns = attn_nsplit(kvheads, nq, max_ctx);  // one partial per workgroup
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
                      hipStream_t st, KvPages pg, int kv_row) {
    if (nq <= 0) return;
    if (kv_row <= 0) kv_row = kvheads * hdim;
    const int ns = attn_nsplit(kvheads, nq, max_ctx);
    int chunk = (max_ctx + ns - 1) / ns;
    chunk = (chunk + MA_SUPER - 1) / MA_SUPER * MA_SUPER;
    float *ws_m = (float *)workspace;
    float *ws_l = ws_m + (size_t)nq * qheads * ns;
    float *ws_o = ws_l + (size_t)nq * qheads * ns;
    const float scale = 1.0f / sqrtf((float)hdim);  // attention_kernels.h:86
    const dim3 grid(ns, kvheads, nq);
#define SI_ATTN_LAUNCH(DIM)                                                                  \
    SI_LAUNCH(k_attn_decode_mfma<DIM>, grid, dim3(256), 0, st, q, qheads, kvheads, kc,       \
              vc, kv_seq_stride, ctx_dev, ctx0, ctx_step, max_ctx, chunk, scale, ws_m,       \
              ws_l, ws_o, pg, kv_row)
    switch (hdim) {
        case 32: SI_ATTN_LAUNCH(32); break;
        case 64: SI_ATTN_LAUNCH(64); break;
        case 96: SI_ATTN_LAUNCH(96); break;
        default: SI_ATTN_LAUNCH(128); break;
    }
#undef SI_ATTN_LAUNCH
    combine(qheads, hdim, nq, ns, ws_m, ws_l, ws_o, attn, qs, d, bsum, st);
}

// Merge of nsplit partials laid out as [nq][qheads][nsplit] (m, l) and
// [nq][qheads][nsplit][hdim] (o) in one workspace.
void launch_attn_combine(int nq, int qheads, int hdim, int nsplit, const void *workspace,
                         float *attn, int8_t *qs, uint16_t *d, int16_t *bsum, hipStream_t st,
                         int8_t *tq, uint16_t *td) {
    const float *ws_m = (const float *)workspace;
    const float *ws_l = ws_m + (size_t)nq * qheads * nsplit;
    const float *ws_o = ws_l + (size_t)nq * qheads * nsplit;
    combine(qheads, hdim, nq, nsplit, ws_m, ws_l, ws_o, attn, qs, d, bsum, st, tq, td);
}

// ---------------------------------------------------------------------------
// Textbook attention in three stages (attention_standard,
// attention_kernels.h:33-78): the fp32 scores of every (head, position) are
// materialized in a [qheads][context] buffer, normalised in place, then
// weighted into V.  It is the comparison mode of the decode layer; the
// streaming kernels above are the fast path.

// Stage 1, grid (ceil(ctx/64), kvheads), block 256: a workgroup stages the
// K rows of 64 positions of one KV group in LDS (coalesced 16-byte loads,
// each K byte read once per group) and computes the scores of all the
// group's query heads for them: thread (slot, r) owns position t0 + r and
// heads slot, slot + 4, ...  Each dot product is summed in head-dimension
// order with separate multiply and add (the reference's loop under
// -ffp-contract=off), then scaled by 1/sqrt(hdim): the scores match the
// reference's bits.
template <int D>
__global__ __launch_bounds__(256) void k_std_scores(const float *__restrict__ q,
                                                    const uint16_t *__restrict__ kc, int qheads,
                                                    int kvheads, int ctx, float inv,
                                                    float *__restrict__ scores) {
    __shared__ float ks[64][D + 1];  // +1: the dot loop's column reads hit distinct banks
    __shared__ float qsh[ATT_MAXPER][D];
    constexpr int CPR = D / 8;  // 16-byte chunks per K row
    const int g = blockIdx.y, G = qheads / kvheads, t0 = blockIdx.x * 64, tid = threadIdx.x;
    for (int i = tid; i < G * D; i += 256) qsh[i / D][i % D] = q[(size_t)g * G * D + i];
    for (int i = tid; i < 64 * CPR; i += 256) {
        const int r = i / CPR, c = i % CPR;
        const int t = min(t0 + r, ctx - 1);  // rows past the context are loaded, never used
        const uint4 u = *(const uint4 *)(kc + ((size_t)t * kvheads + g) * D + c * 8);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) ks[r][c * 8 + e] = h2f((uint16_t)(w[e >> 1] >> (16 * (e & 1))));
    }
    __syncthreads();
    const int r = tid & 63, slot = tid >> 6, t = t0 + r;
    if (t >= ctx) return;
    for (int j = slot; j < G; j += 4) {
        float dot = 0.0f;
#pragma unroll 16
        for (int d = 0; d < D; ++d) dot = __fadd_rn(dot, __fmul_rn(qsh[j][d], ks[r][d]));
        scores[(size_t)(g * G + j) * ctx + t] = __fmul_rn(dot, inv);
    }
}

// Stage 2, grid qheads, block 1024: max, exp(s - max) written in place with
// their sum, then multiplied by 1/sum (attention_kernels.h:50-62).
__global__ __launch_bounds__(1024) void k_std_softmax(float *__restrict__ scores, int ctx) {
    __shared__ float red[16];
    float *row = scores + (size_t)blockIdx.x * ctx;
    float m = -INFINITY;
    for (int t = threadIdx.x; t < ctx; t += 1024) m = fmaxf(m, row[t]);
    m = block_reduce_1024(m, red, true);
    float sum = 0.0f;
    for (int t = threadIdx.x; t < ctx; t += 1024) {
        const float e = expf(row[t] - m);
        row[t] = e;
        sum += e;
    }
    const float inv = 1.0f / block_reduce_1024(sum, red, false);
    for (int t = threadIdx.x; t < ctx; t += 1024) row[t] *= inv;
}

// Stage 3, 8 * ceil(qheads * hdim/8 / 8) workgroups of 1024 threads: a
// workgroup owns the 8 output columns 8c..8c+7 of one head (one 16-byte V
// load per position).  Workgroups are dealt to the 8 XCDs in turn (linear
// id % 8), so (head, c) pairs are numbered head-major and each XCD takes a
// contiguous range: the column workgroups of a head, and the heads of a KV
// group, then share their V cache lines in one XCD's L2.
// thread i sums p[t] v[t] over t = i, i + 1024, ... (four loads in flight),
// then the 1024 partial sums are added in a fixed order
// (attention_kernels.h:64-77 up to the summation order).  The normalised
// scores stay in place.
__global__ __launch_bounds__(1024) void k_std_pv(const float *__restrict__ scores,
                                                 const uint16_t *__restrict__ vc, int qheads,
                                                 int kvheads, int hdim, int ctx,
                                                 float *__restrict__ out) {
    __shared__ float red[16][8];
    const int cpr = hdim / 8, npair = qheads * cpr, per_xcd = (npair + 7) / 8;
    const int pair = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (pair >= npair) return;  // whole workgroup: no barrier is skipped
    const int h = pair / cpr, c = pair % cpr, g = h / (qheads / kvheads), tid = threadIdx.x;
    const float *p = scores + (size_t)h * ctx;
    const size_t rstride = (size_t)kvheads * hdim / 8;  // uint4 per cache row
    const uint4 *v = (const uint4 *)vc + (size_t)g * (hdim / 8) + c;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    auto add = [&](const uint4 u, float pt) {
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
            acc[e] = __fadd_rn(acc[e], __fmul_rn(pt, h2f((uint16_t)(w[e >> 1] >> (16 * (e & 1))))));
    };
    int t = tid;
    for (; t + 3 * 1024 < ctx; t += 4 * 1024) {
        uint4 u[4];
        float pt[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            u[k] = v[(size_t)(t + k * 1024) * rstride];
            pt[k] = p[t + k * 1024];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) add(u[k], pt[k]);
    }
    for (; t < ctx; t += 1024) add(v[(size_t)t * rstride], p[t]);
    // fixed-order reduction: butterfly within each wavefront, then the 16
    // wavefront sums in wave order
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += __shfl_xor(acc[e], off, 64);
    if ((tid & 63) == 0)
#pragma unroll
        for (int e = 0; e < 8; ++e) red[tid >> 6][e] = acc[e];
    __syncthreads();
    if (tid < 8) {
        float r = red[0][tid];
        for (int w = 1; w < 16; ++w) r += red[w][tid];
        out[(size_t)h * hdim + c * 8 + tid] = r;
    }
}

bool attn_standard_supported(int qheads, int kvheads, int hdim) {
    return kvheads >= 1 && qheads % kvheads == 0 && qheads / kvheads <= ATT_MAXPER &&
           (hdim == 32 || hdim == 64 || hdim == 96 || hdim == 128);
}

void launch_attn_standard(const float *q, int qheads, int kvheads, int hdim, const uint16_t *kc,
                          const uint16_t *vc, int ctx, float *out, float *scores,
                          hipStream_t st) {
    const float inv = 1.0f / sqrtf((float)hdim);
    if (ctx > 0) {
        const dim3 grid((ctx + 63) / 64, kvheads);
        switch (hdim) {  // the head dimensions check_shape admits
        case 32: SI_LAUNCH(k_std_scores<32>, grid, dim3(256), 0, st, q, kc, qheads, kvheads, ctx, inv, scores); break;
        case 64: SI_LAUNCH(k_std_scores<64>, grid, dim3(256), 0, st, q, kc, qheads, kvheads, ctx, inv, scores); break;
        case 96: SI_LAUNCH(k_std_scores<96>, grid, dim3(256), 0, st, q, kc, qheads, kvheads, ctx, inv, scores); break;
        default: SI_LAUNCH(k_std_scores<128>, grid, dim3(256), 0, st, q, kc, qheads, kvheads, ctx, inv, scores); break;
        }
        SI_LAUNCH(k_std_softmax, dim3(qheads), dim3(1024), 0, st, scores, ctx);
    }
    // context 0 leaves the output zero (attention_kernels.h:70)
    const int npair = qheads * (hdim / 8);
    SI_LAUNCH(k_std_pv, dim3(8 * ((npair + 7) / 8)), dim3(1024), 0, st, scores, vc,
              qheads, kvheads, hdim, ctx, out);
}

}  // namespace si
