// si_decode.hip -- decode layer (one new token per sequence) in five fused
// kernels.
//
// A decode layer is latency-bound at small shapes (8.9 MB of weights and KV
// for the 0.5B layer stream in ~1.1 us at HBM peak, while a kernel boundary
// costs ~2 us) and HBM-bound at 7B.  The reference's staged run_layer
// (qwen_one_layer.c:237-281: RMSNorm, Q8, Q/K/V, RoPE + KV append,
// attention, Q8, W_O) plus the build-defined FFN runs as:
//
//   1 k_dec_qkv    RMSNorm -> Q8 (recomputed by every workgroup into LDS),
//                  Q|K|V mat-vec (+bias)                         -> qkv fp32
//   2 k_dec_attn   RoPE of q and of the new K row, fp16 K/V append, matrix-
//                  core attention over a context chunk           -> partials
//   3 k_dec_wo     merge of the attention partials, Q8, W_O mat-vec
//                  (+ residual x)                                -> h
//   4 k_dec_gateup post-attention RMSNorm -> Q8, gate|up mat-vec,
//                  SwiGLU -> Q8                                  -> act Q8
//   5 k_matvec     down mat-vec + residual h                     -> out
//                  (si_gemv.hip)
//
// A small layer (dec_qkv_attn_ok) runs 1 and 2 as one kernel,
// k_dec_attn<..., FQ = true>: each (chunk, query head) workgroup projects
// its head's q and its group's k and v itself.
//
// The mat-vec core is GemvRows (si_gemv.hpp); with SI_LAYER_EXACT every
// projection runs its bit-exact instantiation.
#include "si_device.hpp"
#include "si_gemv.hpp"
#include "si_kernels.hpp"

namespace si {

// blocks per load batch of the fused decode mat-vecs (0.5B layer: 25.5 us
// at 8, 24.8 at 2, 24.1 at 4)
constexpr int DEC_U = 4;

// ---------------------------------------------------------------------------
// Activation prologues: the row a workgroup's mat-vec consumes, built in LDS.
// ---------------------------------------------------------------------------
struct Q8Lds {
    int8_t *qs;
    uint16_t *d;
    int16_t *s;
};

// quantize_q8 of one block held by one thread (bit-exact, same rules as
// quant_block_lane).
__device__ __forceinline__ void quant_block_serial(const float (&v)[32], uint32_t (&q)[8],
                                                   uint16_t &dbits, int &bsum) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));  // NaN ignored
    const float d = __fdiv_rn(amax, 127.0f);
    dbits = f2h(d);
    const float inv = (d == 0.0f) ? 0.0f : __fdiv_rn(1.0f, d);
    int sum = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = 0;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const float y = __fmul_rn(v[j], inv);
        int qq;
        if (!(fabsf(y) <= 3.0e38f)) {
            qq = -127;  // NaN or +-inf: lrintf gives LONG_MIN on x86-64
        } else {
            qq = (int)rintf(fminf(fmaxf(y, -200.0f), 200.0f));
            qq = qq > 127 ? 127 : (qq < -127 ? -127 : qq);
        }
        sum += qq;
        q[j >> 2] |= (uint32_t)(qq & 0xff) << (8 * (j & 3));
    }
    bsum = sum;
}

// RMSNorm (qwen_one_layer.c:164-169) then quantize_q8 (:98-116) of one
// activation row into LDS.  Thread t owns 4 consecutive values (t + T*i
// groups of 4), so a Q8 block is 8 consecutive lanes and its max and sum
// are three DPP steps.  The sum of squares is taken in binary64 (4 values
// per lane, then a fixed tree); the Q8 blocks are bit-exact given the
// normalised values.  Two steps so a kernel can order its memory requests
// as it consumes them (loads retire in issue order): load() requests the
// thread's x and gain values (its first NI groups of 4: the whole row up
// to 4*NI*T values), the kernel then requests its weights, and run() waits
// only for x and gain.  Values past 4*NI*T are loaded by run() itself, and
// those wait behind the weights.  Workgroup 0 stores the captures.
template <int T>
struct NormQ8Prologue {
    // groups of 4 held per thread: rows of up to 4096 values at T >= 256
    static constexpr int NI = T >= 256 ? (1024 + T - 1) / T : 4;
    const float *x, *gain;
    int n;
    float4 v[NI], g[NI];

    __device__ __forceinline__ NormQ8Prologue(const float *__restrict__ x_,
                                              const float *__restrict__ gain_, int n_)
        : x(x_), gain(gain_), n(n_) {}

    __device__ __forceinline__ void load4(int e4, float4 &xv, float4 &gv) const {
        xv = *(const float4 *)(x + 4 * e4);
        gv = gain ? *(const float4 *)(gain + 4 * e4) : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    }
    __device__ __forceinline__ void load() {  // branch-free (clamped index)
#pragma unroll
        for (int u = 0; u < NI; ++u) load4(min((int)threadIdx.x + u * T, n / 4 - 1), v[u], g[u]);
    }

    __device__ void run(float eps, Q8Lds xq, double *dscr, float *__restrict__ cap_normed,
                        int8_t *__restrict__ cap_qs, uint16_t *__restrict__ cap_d,
                        int16_t *__restrict__ cap_s) {
        const int t = threadIdx.x;
        const int n4 = n / 4;
        auto sq = [](float4 a) {
            return (double)a.x * a.x + (double)a.y * a.y + (double)a.z * a.z + (double)a.w * a.w;
        };
        double ss = 0.0;
#pragma unroll
        for (int u = 0; u < NI; ++u)
            if (t + u * T < n4) ss += sq(v[u]);
        for (int e4 = t + NI * T; e4 < n4; e4 += T) {  // rows past 4*NI*T values
            float4 xv, gv;
            load4(e4, xv, gv);
            ss += sq(xv);
        }
        ss = wave_sum_d(ss);
        if ((t & 63) == 0) dscr[t >> 6] = ss;
        __syncthreads();
        double tot = 0.0;
#pragma unroll
        for (int w = 0; w < T / 64; ++w) tot += dscr[w];
        const float inv = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn((float)(tot / (double)n), eps)));
        const bool cap = blockIdx.x == 0;
        auto emit = [&](int e4, float4 xv, float4 gv) {
            const float y[4] = {__fmul_rn(__fmul_rn(xv.x, inv), gv.x),
                                __fmul_rn(__fmul_rn(xv.y, inv), gv.y),
                                __fmul_rn(__fmul_rn(xv.z, inv), gv.z),
                                __fmul_rn(__fmul_rn(xv.w, inv), gv.w)};
            uint16_t dbits;
            int bsum;
            const uint32_t q = quant_block_oct(y, dbits, bsum);
            *(uint32_t *)(xq.qs + 4 * e4) = q;
            const int blk = e4 >> 3;
            if ((e4 & 7) == 0) {
                xq.d[blk] = dbits;
                xq.s[blk] = (int16_t)bsum;
            }
            if (cap) {
                if (cap_normed) *(float4 *)(cap_normed + 4 * e4) = make_float4(y[0], y[1], y[2], y[3]);
                if (cap_qs) *(uint32_t *)(cap_qs + 4 * e4) = q;
                if ((e4 & 7) == 0) {
                    if (cap_d) cap_d[blk] = dbits;
                    if (cap_s) cap_s[blk] = (int16_t)bsum;
                }
            }
        };
        // whole 8-lane groups in or out (n4 % 8 == 0)
#pragma unroll
        for (int u = 0; u < NI; ++u)
            if (t + u * T < n4) emit(t + u * T, v[u], g[u]);
        for (int e4 = t + NI * T; e4 < n4; e4 += T) {
            float4 xv, gv;
            load4(e4, xv, gv);
            emit(e4, xv, gv);
        }
        __syncthreads();
    }
};

// LDS carve-up for the kernels that build their activation row in LDS:
// [dscr: 16 doubles][red][y: R floats][xf: k floats + extra][d][s][qs]
template <int R, int T>
struct DecLds {
    double *dscr;
    float *red, *y, *xf;
    Q8Lds xq;
    static constexpr size_t bytes(int k, bool with_xf, int extra_floats) {
        return 16 * 8 + (size_t)red_floats<R, T>() * 4 + R * 4 + (with_xf ? (size_t)k * 4 : 0) +
               (size_t)extra_floats * 4 + (size_t)(k / 32) * 4 + 16 + k;
    }
    // Offsets are counted from the (16-byte aligned) base, never through an
    // integer round trip of the pointer: the compiler then keeps the LDS
    // address space and emits ds_* accesses (a generic pointer gives flat
    // accesses, which count as memory loads in the wait counters, so waits
    // for LDS would also wait for every global load in flight).
    __device__ DecLds(char *p, int k, bool with_xf, int extra_floats) {
        size_t o = 0;
        dscr = (double *)(p + o);
        o += 16 * 8;
        red = (float *)(p + o);
        o += red_floats<R, T>() * 4;
        y = (float *)(p + o);
        o += R * 4;
        xf = (float *)(p + o);
        o += (with_xf ? (size_t)k * 4 : 0) + (size_t)extra_floats * 4;
        xq.d = (uint16_t *)(p + o);
        o += (k / 32) * 2;
        xq.s = (int16_t *)(p + o);
        o += (k / 32) * 2;
        o = (o + 15) & ~(size_t)15;
        xq.qs = (int8_t *)(p + o);
    }
};

// ---------------------------------------------------------------------------
// 1: RMSNorm -> Q8 -> Q|K|V (+bias) -> qkv fp32
// ---------------------------------------------------------------------------
template <int R, int T, bool EXACT>
__global__ void __launch_bounds__(T) k_dec_qkv(
    const float *__restrict__ x, const float *__restrict__ gain, int hidden, float eps,
    const uint8_t *__restrict__ wqs, const uint16_t *__restrict__ wd, int tile, int n,
    const float *__restrict__ bias, float *__restrict__ cap_normed, int8_t *__restrict__ cap_qs,
    uint16_t *__restrict__ cap_d, int16_t *__restrict__ cap_s, float *__restrict__ qkv) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    DecLds<R, T> L(smem, hidden, false, 0);
    const int tile0 = blockIdx.x * R;
    const int t = threadIdx.x;
    const int row = tile0 + (t % R);
    NormQ8Prologue<T> pro(x, gain, hidden);
    pro.load();  // requested in the order they are consumed
    const float b0 = bias ? bias[min(row, n - 1)] : 0.0f;
    GemvRows<R, T, EXACT, RowIdentity, DEC_U> g(wqs, wd, tile, n, n, hidden / SI_QK, tile0,
                                         RowIdentity{});
    g.start();  // weights in flight while the activation row is built
    pro.run(eps, L.xq, L.dscr, cap_normed, cap_qs, cap_d, cap_s);
    const float y = g.finish(Q8Row{L.xq.qs, L.xq.d, L.xq.s}, EXACT ? b0 : 0.0f, L.red);
    if (t < R && row < n) qkv[row] = EXACT ? y : y + b0;
}

// ---------------------------------------------------------------------------
// 3: merge attention partials -> attn fp32 -> Q8 -> W_O mat-vec (+ residual)
// ---------------------------------------------------------------------------
// Partials per (head, chunk s): running max m, sum l, unnormalised o[D].
// attn[h][d] = sum_s o_s[d] e^(m_s - M) * (1 / sum_s l_s e^(m_s - M)),
// M = max_s m_s; a head with no context (M = -inf) gives 0
// (attention_kernels.h:95-98).
template <int R, int T, bool EXACT>
__global__ void __launch_bounds__(T) k_dec_wo(
    const float *__restrict__ pm, const float *__restrict__ pl, const float *__restrict__ po,
    int ns, int qheads, int hdim, const uint8_t *__restrict__ wqs,
    const uint16_t *__restrict__ wd, int tile, int n, const float *__restrict__ residual,
    float *__restrict__ cap_attn, int8_t *__restrict__ cap_qs, uint16_t *__restrict__ cap_d,
    int16_t *__restrict__ cap_s, float *__restrict__ cap_y, float *__restrict__ out) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int qd = qheads * hdim;
    DecLds<R, T> L(smem, qd, false, 0);
    const int tile0 = blockIdx.x * R;
    const int t = threadIdx.x;
    const bool cap = blockIdx.x == 0;
    // the residual is requested first: read after the sums it would add a
    // memory round trip to the end of the kernel
    const float r0 = residual ? residual[min(tile0 + (t % R), n - 1)] : 0.0f;
    GemvRows<R, T, EXACT, RowIdentity, DEC_U> g(wqs, wd, tile, n, n, qd / SI_QK, tile0,
                                         RowIdentity{});
    // Thread t merges the 4 consecutive elements 4*e4.. (e4 = t + T*i), 8
    // chunks at a time, with the online rule (m, l, o) <- (M',
    // l e^(m-M') + l_s e^(m_s-M'), o e^(m-M') + o_s e^(m_s-M')), then
    // quantizes: 8 consecutive lanes hold one Q8_0 block of the output
    // (qwen_one_layer.c:272).  The first group of partials is requested
    // before the weights, which then load while the merge runs.  A
    // wavefront with no elements in this round loads and merges nothing.
    constexpr int SC = 8;
    bool started = false;
    const int qd4 = qd / 4;
    for (int e40 = 0; e40 < qd4; e40 += T) {
        const int e4 = e40 + t;
        const bool eok = e4 < qd4;
        const bool wact = e40 + (t & ~63) < qd4;  // wavefront-uniform
        const int ec = 4 * min(e4, qd4 - 1);
        const int h = ec / hdim, d = ec - h * hdim;
        float M = -INFINITY, Ls = 0.0f;
        float A[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int s0 = 0; s0 < ns; s0 += SC) {
            float om[SC], ol[SC];
            float4 oo[SC];
            if (wact) {
#pragma unroll
                for (int u = 0; u < SC; ++u) {  // clamped index
                    const size_t pi = (size_t)h * ns + min(s0 + u, ns - 1);
                    om[u] = pm[pi];
                    ol[u] = pl[pi];
                    oo[u] = *(const float4 *)(po + pi * hdim + d);
                }
            }
            if (!started) {
                g.start();
                started = true;
            }
            if (!wact) continue;
#pragma unroll
            for (int u = 0; u < SC; ++u) {
                if (s0 + u >= ns || om[u] == -INFINITY) continue;  // empty chunk
                const float mn = fmaxf(M, om[u]);
                // hardware exp2, as in the attention's own online softmax
                const float a = M == -INFINITY ? 0.0f : __expf(M - mn);
                const float bw = __expf(om[u] - mn);
                A[0] = fmaf(oo[u].x, bw, A[0] * a);
                A[1] = fmaf(oo[u].y, bw, A[1] * a);
                A[2] = fmaf(oo[u].z, bw, A[2] * a);
                A[3] = fmaf(oo[u].w, bw, A[3] * a);
                Ls = fmaf(ol[u], bw, Ls * a);
                M = mn;
            }
        }
        if (e40 + (t & ~7) < qd4) {  // whole 8-lane groups
            // normalise (attention_kernels.h:163); no context gives 0 (:95-98)
            const float r = M == -INFINITY ? 0.0f : 1.0f / Ls;
            const float y[4] = {A[0] * r, A[1] * r, A[2] * r, A[3] * r};
            uint16_t dbits;
            int bsum;
            const uint32_t q = quant_block_oct(y, dbits, bsum);
            if (eok) {
                *(uint32_t *)(L.xq.qs + 4 * e4) = q;
                if ((e4 & 7) == 0) {
                    L.xq.d[e4 >> 3] = dbits;
                    L.xq.s[e4 >> 3] = (int16_t)bsum;
                }
                if (cap) {
                    if (cap_attn) *(float4 *)(cap_attn + 4 * e4) = make_float4(y[0], y[1], y[2], y[3]);
                    if (cap_qs) *(uint32_t *)(cap_qs + 4 * e4) = q;
                    if ((e4 & 7) == 0) {
                        if (cap_d) cap_d[e4 >> 3] = dbits;
                        if (cap_s) cap_s[e4 >> 3] = (int16_t)bsum;
                    }
                }
            }
        }
    }
    __syncthreads();
    const float y = g.finish(Q8Row{L.xq.qs, L.xq.d, L.xq.s}, 0.0f, L.red);
    const int row = tile0 + t;
    if (t < R && row < n) {
        if (cap_y) cap_y[row] = y;
        out[row] = residual ? __fadd_rn(r0, y) : y;
    }
}

// ---------------------------------------------------------------------------
// 4: post-attention RMSNorm -> Q8 -> gate|up -> SwiGLU -> Q8
// ---------------------------------------------------------------------------
template <int R, int T, bool EXACT>
__global__ void __launch_bounds__(T) k_dec_gateup(
    const float *__restrict__ h, const float *__restrict__ gain, int hidden, float eps,
    const uint8_t *__restrict__ wqs, const uint16_t *__restrict__ wd, int tile, int f,
    float *__restrict__ cap_normed, int8_t *__restrict__ cap_qs, uint16_t *__restrict__ cap_d,
    int16_t *__restrict__ cap_s, float *__restrict__ gu, float *__restrict__ act,
    int8_t *__restrict__ aqs, uint16_t *__restrict__ ad, int16_t *__restrict__ as) {
    static_assert(R % 64 == 0, "gate|up rows pair within a wavefront");
    extern __shared__ __attribute__((aligned(16))) char smem[];
    DecLds<R, T> L(smem, hidden, false, 0);
    const int tile0 = blockIdx.x * R;
    const int t = threadIdx.x;
    NormQ8Prologue<T> pro(h, gain, hidden);
    pro.load();  // requested in the order they are consumed
    GemvRows<R, T, EXACT, RowGateUp, DEC_U> g(wqs, wd, tile, 2 * f, 2 * f, hidden / SI_QK, tile0,
                                       RowGateUp{f});
    g.start();  // weights in flight while the activation row is built
    pro.run(eps, L.xq, L.dscr, cap_normed, cap_qs, cap_d, cap_s);
    const float y = g.finish(Q8Row{L.xq.qs, L.xq.d, L.xq.s}, 0.0f, L.red);
    if (t < R) L.y[t] = y;
    __syncthreads();
    if (t >= R) return;
    const int lrow = tile0 + t;  // logical row (f is a multiple of 32: whole wavefronts)
    if (lrow >= 2 * f) return;
    const int j = 32 * (lrow >> 6) + (lrow & 31);
    if (gu) gu[(lrow & 32) ? f + j : j] = y;
    if (t & 32) return;  // lanes 0..31 of each wavefront hold the gate rows
    // SwiGLU (silu(g) = g / (1 + e^-g), then * u) and quantize_q8 of the block
    const float gv = y, u = L.y[t + 32];
    const float a = __fmul_rn(__fdiv_rn(gv, __fadd_rn(1.0f, expf(-gv))), u);
    uint16_t dbits;
    int bsum;
    const int q = quant_block_lane(a, dbits, bsum);
    if (act) act[j] = a;
    aqs[j] = (int8_t)q;
    if ((t & 31) == 0) {
        ad[j / SI_QK] = dbits;
        as[j / SI_QK] = (int16_t)bsum;
    }
}

// ===========================================================================
// 2: decode attention with RoPE and the K/V append folded in.
//
// Workgroup (chunk sp, KV group g, sequence qi), NW wavefronts.  The new
// token sits at position p = ctx - 1.  Every workgroup rotates the group's
// query heads itself (RoPE, qwen_one_layer.c:260-261); the workgroup whose
// chunk holds p also rotates the group's K row, narrows K and V to fp16 and
// appends them to the cache (:262-266), and uses those fp16 values for
// position p (the reference reads the new row back from the fp16 cache).
//
// Wavefront w takes the 16-position tiles w, w + NW, ... of the chunk:
//   S^T[pos][head] = K[pos][:] . Q[head][:]      v_mfma_f32_16x16x32_f16
//   online softmax per head (one head per MFMA column)
//   O^T[d][head] += V^T[d][pos] . P[pos][head]   v_mfma_f32_16x16x16f16
// fp32 Q and P enter the fp16 matrix cores as hi + lo halves, so products
// keep fp32-level accuracy.  K tiles are MFMA A operands loaded straight
// from HBM; V tiles pass through the wavefront's own LDS rows to be read
// transposed.  The next tile's K and V loads are issued before the current
// tile is computed.  The wavefronts' (m, l, o) are merged in LDS into one
// partial per workgroup; with FINAL (single chunk) the workgroup normalises
// and quantizes the output itself.
// MFMA 16x16 output element (i, j): lane j + 16*(i/4), register i%4.
// ===========================================================================
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int DA_TILE = 16;
constexpr int DA_VPAD = 8;  // halves of padding per LDS V row

__device__ __forceinline__ void hi_lo(float x, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

template <int D, int NW>
struct AttnLds {
    static constexpr int VROW = D + DA_VPAD;
    static constexpr size_t v_bytes = (size_t)NW * DA_TILE * VROW * 2;
    static constexpr size_t merge_bytes(int per) {
        return ((size_t)NW * per * (D + 3) + 2 * per) * 4;
    }
    static constexpr size_t raw_bytes(int per) { return (size_t)(per * D + 3 * D) * 4; }
    static constexpr size_t bytes(int per) {
        size_t m = merge_bytes(per);
        if (raw_bytes(per) > m) m = raw_bytes(per);
        return 2 * D * 2 + (v_bytes > m ? v_bytes : m);
    }
};

// LDS of the fused QKV prologue (FQ), after the attention's own: the
// norm's scratch, the three mat-vecs' partial sums, the normalised Q8 row.
template <int D, int NW>
struct FqLds {
    static constexpr int RED = red_floats<D, NW * 64>();
    static constexpr size_t bytes(int hidden) {
        return 16 * 8 + (size_t)3 * RED * 4 + (size_t)(hidden / 32) * 4 + 16 + hidden;
    }
};

// DEPTH: K/V tiles in flight per wavefront; 1 when every wavefront has at
// most one tile (single queries: more chunks, a shorter chain), else 2 (3
// measured no faster).  FQ: single-token decode with the Q|K|V projection
// inside (a workgroup per (chunk, query head): RMSNorm -> Q8 of the layer
// input, then the head's q rows and its group's k and v rows of the fused
// matrix, + bias), for a small model whose 3*hdim rows a workgroup streams
// quickly; the k_dec_qkv launch and the q|k|v round trip through memory
// disappear, at the price of every chunk recomputing its head's rows.
template <int D, int NW, bool FINAL, bool PAGED, int DEPTH, bool FQ = false>
__global__ void __launch_bounds__(NW * 64) k_dec_attn(
    const float *__restrict__ qkv, int ldqkv, int qheads, int kvheads,
    const float *__restrict__ rc, const float *__restrict__ rs, uint16_t *__restrict__ kc,
    uint16_t *__restrict__ vc, size_t kv_seq_stride, const int *__restrict__ ctx_dev, int ctx0,
    int max_ctx, int chunk, float scale, float *__restrict__ q_cap, float *__restrict__ ws_m,
    float *__restrict__ ws_l, float *__restrict__ ws_o, float *__restrict__ attn,
    int8_t *__restrict__ aqs, uint16_t *__restrict__ ad, int16_t *__restrict__ as, KvPages pg,
    DecQkvIn fq) {
    constexpr int KS = D / 32, DT = D / 16, HALF = D / 2;
    constexpr int VROW = AttnLds<D, NW>::VROW;
    constexpr int VL = DA_TILE * D / (64 * 8);  // 16-byte V pieces per lane per tile
    extern __shared__ __attribute__((aligned(16))) char smem[];
    uint16_t *newk = (uint16_t *)smem;  // fp16 K and V rows of the new token
    uint16_t *newv = newk + D;
    char *big = smem + 2 * D * 2;
    _Float16 *vbuf = (_Float16 *)big;

    const int sp = blockIdx.x, qi = FQ ? 0 : blockIdx.z, ns = gridDim.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int per = qheads / kvheads;
    // this workgroup's query heads: hbase .. hbase + nh - 1, of group g
    const int g = FQ ? (int)blockIdx.y / per : (int)blockIdx.y;
    const int nh = FQ ? 1 : per;
    const int hbase = FQ ? (int)blockIdx.y : g * per;
    const int qd = qheads * D, kvd = kvheads * D;
    int ctx = ctx_dev ? ctx_dev[qi] : ctx0;
    ctx = min(ctx, max_ctx);
    const int pnew = ctx - 1;  // < 0: empty context (device-supplied only)
    const int p0 = sp * chunk;
    const int p1 = min(ctx, p0 + chunk);
    const bool owner = pnew >= p0 && pnew < p1;
    const float *row = qkv + (size_t)qi * ldqkv;
    const float *cr = rc + (size_t)max(pnew, 0) * HALF;
    const float *sr = rs + (size_t)max(pnew, 0) * HALF;
    // cache row of position p: pg.at<PAGED>(qi, p, ...) (contiguous or paged)
    const uint16_t *kbase = kc + (size_t)g * D;
    const uint16_t *vbase = vc + (size_t)g * D;
    _Float16 *vw = vbuf + (size_t)wave * DA_TILE * VROW;

    // K pieces of the lane's row (pos = t0 + col), V pieces of the tile
    // (branch-free: positions past the chunk re-read its last row, or row 0
    // for an empty context; such rows are masked out of the scores)
    auto load_k = [&](int t0, uint4(&kr)[KS]) {
        const int pos = max(min(t0 + col, p1 - 1), 0);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            kr[ks] = *(const uint4 *)(kbase + pg.template at<PAGED>(qi, pos, kv_seq_stride, kvd) + 32 * ks + 8 * grp);
    };
    auto load_v = [&](int t0, uint4(&vr)[VL]) {
#pragma unroll
        for (int j = 0; j < VL; ++j) {
            const int c = lane + 64 * j;
            const int r = c / (D / 8), e = (c % (D / 8)) * 8;
            vr[j] = *(const uint4 *)(vbase + pg.template at<PAGED>(qi, max(min(t0 + r, p1 - 1), 0), kv_seq_stride, kvd) + e);
        }
    };
    // The new token's row is taken from LDS (its cache row may not be
    // written yet: the global value read for it is discarded).  Applied when
    // a tile is consumed, so prefetched loads stay in flight until then.
    auto sel = [](bool c, uint4 a, uint4 b) {
        return make_uint4(c ? a.x : b.x, c ? a.y : b.y, c ? a.z : b.z, c ? a.w : b.w);
    };
    auto fix = [&](int t0, uint4(&kr)[KS], uint4(&vr)[VL]) {
        const int pos = min(t0 + col, p1 - 1);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            kr[ks] = sel(pos == pnew, *(const uint4 *)(newk + 32 * ks + 8 * grp), kr[ks]);
#pragma unroll
        for (int j = 0; j < VL; ++j) {
            const int c = lane + 64 * j;
            const int r = c / (D / 8), e = (c % (D / 8)) * 8;
            vr[j] = sel(min(t0 + r, p1 - 1) == pnew, *(const uint4 *)(newv + e), vr[j]);
        }
    };

    // Requests in the order they are consumed (loads retire in issue order):
    // 1. the group's raw q rows, the raw K and V rows of the new token and
    //    the RoPE row at its position, one or a few floats per thread;
    float *qraw = (float *)big;   // [nh][D]; these LDS rows are reused for
    float *kraw = qraw + nh * D;  // the V tiles once Q is in registers
    float *vraw = kraw + D;
    float *csr = vraw + D;        // [HALF] cos, then [HALF] sin
    constexpr int STEP = DA_TILE * NW;
    int t0 = p0 + DA_TILE * wave;
    uint4 kr[DEPTH][KS], vr[DEPTH][VL];
    if constexpr (FQ) {
        // 1. the layer input and gain, the rows' weights, bias and RoPE
        //    row, 2. the first K and V tiles; then the Q8 row in LDS and
        //    the three mat-vecs (their sums meet in separate LDS areas)
        constexpr int NT = NW * 64;
        using F = FqLds<D, NW>;
        char *fx = smem + ((AttnLds<D, NW>::bytes(1) + 15) & ~(size_t)15);
        double *dscr = (double *)fx;
        float *red = (float *)(fx + 16 * 8);
        const int nb = fq.hidden / SI_QK;
        Q8Lds xq;
        xq.d = (uint16_t *)(red + 3 * F::RED);
        xq.s = (int16_t *)(xq.d + nb);
        xq.qs = (int8_t *)(xq.s + nb + (8 - (2 * nb) % 8) % 8);  // 16-byte aligned
        NormQ8Prologue<NT> pro(fq.x, fq.gain, fq.hidden);
        pro.load();
        GemvRows<D, NT, false, RowIdentity, DEC_U> wq(fq.wqs, fq.wd, fq.tile, fq.n, fq.n, nb,
                                                     hbase * D, RowIdentity{});
        GemvRows<D, NT, false, RowIdentity, DEC_U> wk(fq.wqs, fq.wd, fq.tile, fq.n, fq.n, nb,
                                                     qd + g * D, RowIdentity{});
        GemvRows<D, NT, false, RowIdentity, DEC_U> wv(fq.wqs, fq.wd, fq.tile, fq.n, fq.n, nb,
                                                     qd + kvd + g * D, RowIdentity{});
        wq.start();
        wk.start();
        wv.start();
        const int e = min(tid, D - 1);
        const float cs = e < HALF ? cr[e] : sr[e - HALF];
        float bq = 0.0f, bk = 0.0f, bv = 0.0f;
        if (fq.bias) {
            bq = fq.bias[hbase * D + e];
            bk = fq.bias[qd + g * D + e];
            bv = fq.bias[qd + kvd + g * D + e];
        }
#pragma unroll
        for (int b = 0; b < DEPTH; ++b) {
            load_k(t0 + b * STEP, kr[b]);
            load_v(t0 + b * STEP, vr[b]);
        }
        const bool c0 = blockIdx.y == 0;  // (workgroup (0, 0) writes the row captures)
        pro.run(fq.eps, xq, dscr, c0 ? fq.cap_normed : nullptr, c0 ? fq.cap_qs : nullptr,
                c0 ? fq.cap_d : nullptr, c0 ? fq.cap_s : nullptr);
        const Q8Row xr{xq.qs, xq.d, xq.s};
        const float yq = wq.finish(xr, 0.0f, red) + bq;
        const float yk = wk.finish(xr, 0.0f, red + F::RED) + bk;
        const float yv = wv.finish(xr, 0.0f, red + 2 * F::RED) + bv;
        if (tid < D) {
            qraw[tid] = yq;
            kraw[tid] = yk;
            vraw[tid] = yv;
            csr[tid] = cs;
            if (fq.cap_qkv && sp == 0) {
                fq.cap_qkv[hbase * D + tid] = yq;
                if (hbase == g * per) {
                    fq.cap_qkv[qd + g * D + tid] = yk;
                    fq.cap_qkv[qd + kvd + g * D + tid] = yv;
                }
            }
        }
    } else {
        const int nraw = per * D + 3 * D;
        constexpr int RAWPT = (16 * D + 3 * D + NW * 64 - 1) / (NW * 64);
        float rv[RAWPT];
#pragma unroll
        for (int u = 0; u < RAWPT; ++u) {  // branch-free: clamped index
            const int i = min(tid + u * NW * 64, nraw - 1);
            {
                const float *src;
                if (i < per * D)
                    src = row + (size_t)g * per * D + i;
                else if (i < per * D + D)
                    src = row + qd + g * D + (i - per * D);
                else if (i < per * D + 2 * D)
                    src = row + qd + kvd + g * D + (i - per * D - D);
                else {
                    const int j = i - per * D - 2 * D;
                    src = j < HALF ? cr + j : sr + (j - HALF);
                }
                rv[u] = *src;
            }
        }
        // 2. the wavefront's first DEPTH K and V tiles (that many in flight
        //    throughout)
#pragma unroll
        for (int b = 0; b < DEPTH; ++b) {
            load_k(t0 + b * STEP, kr[b]);
            load_v(t0 + b * STEP, vr[b]);
        }
#pragma unroll
        for (int u = 0; u < RAWPT; ++u) {
            const int i = tid + u * NW * 64;
            if (i < nraw) qraw[i] = rv[u];
        }
    }
    __syncthreads();
    // rotate-half RoPE (qwen_one_layer.c:172-183) of element dd of a head row
    auto rot = [&](const float *v, int dd) {
        const int i = dd < HALF ? dd : dd - HALF;
        const float a = v[i], b = v[i + HALF], c = csr[i], s = csr[HALF + i];
        return dd < HALF ? __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s))
                         : __fadd_rn(__fmul_rn(b, c), __fmul_rn(a, s));
    };
    if (owner) {  // the new token's K (rotated) and V rows, fp16, into the cache
        for (int dd = tid; dd < D; dd += NW * 64) {
            const uint16_t kh = f2h(rot(kraw, dd));
            const uint16_t vh = f2h(vraw[dd]);
            newk[dd] = kh;
            newv[dd] = vh;
            kc[pg.template at<PAGED>(qi, pnew, kv_seq_stride, kvd) + g * D + dd] = kh;
            vc[pg.template at<PAGED>(qi, pnew, kv_seq_stride, kvd) + g * D + dd] = vh;
        }
    }
    // Q^T as the B operand: lane holds Q[head col][d = 32*ks + 8*grp + e],
    // rotated from 8 consecutive pairs read as 16-byte LDS vectors
    h8 qh[KS], ql[KS];
    {
        const bool hv = col < nh && pnew >= 0;
        const int hc = col < nh ? col : 0;
        const bool capq = q_cap && sp == 0 && wave == 0 && hv;
        const float *qh_row = qraw + hc * D;
        auto ld8 = [](const float *p, float (&v)[8]) {
            const float4 a = *(const float4 *)p, b = *(const float4 *)(p + 4);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        };
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int d0 = 32 * ks + 8 * grp;
            const int i0 = d0 < HALF ? d0 : d0 - HALF;
            float a[8], b[8], c[8], sn[8], v[8];
            ld8(qh_row + i0, a);
            ld8(qh_row + i0 + HALF, b);
            ld8(csr + i0, c);
            ld8(csr + HALF + i0, sn);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                v[e] = !hv ? 0.0f
                           : (d0 < HALF ? __fsub_rn(__fmul_rn(a[e], c[e]), __fmul_rn(b[e], sn[e]))
                                        : __fadd_rn(__fmul_rn(b[e], c[e]), __fmul_rn(a[e], sn[e])));
                _Float16 hi, lo;
                hi_lo(v[e], hi, lo);
                qh[ks][e] = hi;
                ql[ks][e] = lo;
            }
            if (capq) {
                float *qc = q_cap + (size_t)qi * qd + (size_t)(hbase + hc) * D + d0;
                *(float4 *)qc = make_float4(v[0], v[1], v[2], v[3]);
                *(float4 *)(qc + 4) = make_float4(v[4], v[5], v[6], v[7]);
            }
        }
    }
    __syncthreads();  // newk/newv visible; the raw rows are no longer read

    float m = -INFINITY, lsum = 0.0f;
    f4 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = (f4){0.f, 0.f, 0.f, 0.f};

    // one 16-position tile: scores, online softmax, weighted V sum
    auto tile = [&](int t0, uint4(&kr)[KS], uint4(&vr)[VL]) {
        // only the owner chunk's tile holding the new row (or clamped onto
        // it) needs the LDS copy (wave-uniform test)
        if (owner && t0 + DA_TILE > pnew) fix(t0, kr, vr);
        // stage V rows into this wavefront's LDS rows
#pragma unroll
        for (int j = 0; j < VL; ++j) {
            const int c = lane + 64 * j;
            const int r = c / (D / 8), e = (c % (D / 8)) * 8;
            *(uint4 *)(vw + r * VROW + e) = vr[j];
        }
        h8 ka[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) ka[ks] = __builtin_bit_cast(h8, kr[ks]);
        f4 sacc = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[ks], qh[ks], sacc, 0, 0, 0);
            sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[ks], ql[ks], sacc, 0, 0, 0);
        }
        // lane holds S^T[pos = t0 + 4*grp + r][head col]
        float s[4], mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            s[r] = (t0 + 4 * grp + r < p1) ? sacc[r] * scale : -INFINITY;
            mx = fmaxf(mx, s[r]);
        }
        mx = fmaxf(mx, swap16_f(mx));
        mx = fmaxf(mx, swap32_f(mx));
        const float mnew = fmaxf(m, mx);
        // hardware exp2 (relative error ~1e-6 here, far inside the 2e-3
        // attention tolerance); mnew is finite from the first tile on
        const float alpha = __expf(m - mnew);  // 0 while m is -inf
        float p[4], ps = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            p[r] = __expf(s[r] - mnew);
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
            hi_lo(p[r], hi, lo);
            ph[r] = hi;
            pl[r] = lo;
        }
        // the V rows written above by other lanes of this wavefront
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // A = V^T[d = 16*dt + col][pos = 4*grp + r], gathered by the
        // transposing read: lane (col, grp) points at V row 4*grp + col/4,
        // dims 16*dt + 4*(col%4) .. +3
        const _Float16 *vsrc = vw + (4 * grp + (col >> 2)) * VROW + 4 * (col & 3);
        // rescale only when some column's running max moved (alpha == 1
        // exactly otherwise: exp of 0), a wavefront-uniform branch
        if (__ballot(alpha != 1.0f)) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const h4 va = __builtin_bit_cast(h4, lds_read_tr16(vsrc + 16 * dt));
            f4 acc = o[dt];
            acc = __builtin_amdgcn_mfma_f32_16x16x16f16(va, ph, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pl, acc, 0, 0, 0);
            o[dt] = acc;
        }
        // V rows are read before the next tile overwrites them
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    // tiles t0, t0 + STEP, ... rotate through the DEPTH register sets; each
    // set is refilled DEPTH tiles ahead once consumed (past the chunk:
    // clamped, unused).  With DEPTH 2 every set of a round is consumed, also
    // when its tile lies past the chunk (all scores masked: the state is
    // unchanged): a conditional exit between the sets makes the compiler
    // wait for every load in flight at the loop head.  With DEPTH 1 nothing
    // else is in flight, so the refill is skipped past the chunk (a
    // wavefront-uniform test).
    for (; t0 < p1; t0 += DEPTH * STEP) {
#pragma unroll
        for (int b = 0; b < DEPTH; ++b) {
            const int tb = t0 + b * STEP;
            tile(tb, kr[b], vr[b]);
            if (DEPTH > 1 || tb + STEP < p1) {
                load_k(tb + DEPTH * STEP, kr[b]);
                load_v(tb + DEPTH * STEP, vr[b]);
            }
        }
    }

    // merge the NW wavefront states in LDS (reusing the V rows)
    __syncthreads();
    float *mm = (float *)big;  // [NW][nh]
    float *ml = mm + NW * nh;  // [NW][nh]
    float *mo = ml + NW * nh;  // [NW][nh][D]
    if (col < nh) {
        if (grp == 0) {
            mm[wave * nh + col] = m;
            ml[wave * nh + col] = lsum;
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)  // rows 4*grp .. 4*grp + 3: one 16-byte write
            *(f4 *)(mo + ((size_t)wave * nh + col) * D + 16 * dt + 4 * grp) = o[dt];
    }
    __syncthreads();
    // 4 consecutive elements per thread; 8 lanes = 32 elements = one Q8_0
    // block of one head (D is a multiple of 32).  Each thread forms its
    // head's M = max over wavefronts, the factors e^(m_w - M) and the total
    // l itself (broadcast LDS reads; no further barrier).
    const int nel4 = nh * D / 4;
    for (int e40 = 0; e40 < nel4; e40 += NW * 64) {
        const int e4 = e40 + tid;
        const bool ok = e4 < nel4;
        const int ec = 4 * min(e4, nel4 - 1);
        const int hc = ec / D, dd = ec - hc * D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, mm[w * nh + hc]);
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, ltot = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float4 ov = *(const float4 *)(mo + ((size_t)w * nh + hc) * D + dd);
            // hardware exp2, as in the tile loop; an empty wavefront gives 0
            const float f = M == -INFINITY ? 0.0f : __expf(mm[w * nh + hc] - M);
            ltot = fmaf(ml[w * nh + hc], f, ltot);
            acc[0] = fmaf(ov.x, f, acc[0]);
            acc[1] = fmaf(ov.y, f, acc[1]);
            acc[2] = fmaf(ov.z, f, acc[2]);
            acc[3] = fmaf(ov.w, f, acc[3]);
        }
        const int h = hbase + hc;
        if (!FINAL) {
            if (ok) {
                const size_t pi = ((size_t)qi * qheads + h) * ns + sp;
                if (dd == 0) {
                    ws_m[pi] = M;
                    ws_l[pi] = ltot;
                }
                *(float4 *)(ws_o + pi * D + dd) = make_float4(acc[0], acc[1], acc[2], acc[3]);
            }
        } else if (e40 + (tid & ~7) < nel4) {
            // normalise (attention_kernels.h:163; no context: 0, :95-98) and
            // quantize_q8
            const float r = M == -INFINITY ? 0.0f : 1.0f / ltot;
            const float y[4] = {acc[0] * r, acc[1] * r, acc[2] * r, acc[3] * r};
            uint16_t dbits;
            int bsum;
            const uint32_t q = quant_block_oct(y, dbits, bsum);
            if (ok) {
                const size_t off = (size_t)qi * qd + (size_t)h * D + dd;
                *(float4 *)(attn + off) = make_float4(y[0], y[1], y[2], y[3]);
                *(uint32_t *)(aqs + off) = q;
                if ((e4 & 7) == 0) {
                    ad[off / SI_QK] = dbits;
                    if (as) as[off / SI_QK] = (int16_t)bsum;
                }
            }
        }
    }
}

// ===========================================================================
// Decode attention over whole cache rows (kvheads <= 4).
//
// One workgroup of 4 wavefronts owns (query, context chunk) and every KV
// group: wavefront w serves group w % G over every (4/G)-th 16-position tile
// of the chunk.  Per step the workgroup stages 16*(4/G) whole cache rows
// (every group, K and V) in LDS with row-contiguous loads, then each
// wavefront runs k_dec_attn's MFMA scores, online softmax and PV on its
// group's columns (V^T operands by the transposing LDS read).  Reading
// whole rows is the point: one group's 2*hdim-byte slice of each row
// streams at ~4.0 TB/s, whole rows at ~6.4 TB/s (7B, 64 x 4096 cache,
// measured).  The new token's K/V row is substituted in LDS.
// ===========================================================================
template <int D, int G>
struct RowsLds {
    static constexpr int NWG = 4 / G;            // wavefronts per group
    static constexpr int ROWS = DA_TILE * NWG;  // positions per step
    static constexpr int RW = G * D + 8;        // halves per LDS row (padded)
    // K and V rows of a step, twice: steps alternate between the two copies
    static constexpr size_t tile_bytes = (size_t)2 * 2 * ROWS * RW * 2;
    static constexpr size_t raw_bytes(int per) {
        return (size_t)(G * per * D + 2 * G * D + D) * 4;
    }
    static constexpr size_t merge_bytes(int per) {  // NWG states per group + factors
        return (size_t)G * (NWG * per * (D + 2) + per * (NWG + 2)) * 4;
    }
    static constexpr size_t bytes(int per) {
        size_t m = tile_bytes;
        if (raw_bytes(per) > m) m = raw_bytes(per);
        if (merge_bytes(per) > m) m = merge_bytes(per);
        return (size_t)2 * G * D * 2 + m;  // new K|V row (fp16) + the shared region
    }
};

template <int D, int G, bool FINAL, bool PAGED>
__global__ void __launch_bounds__(256) k_dec_attn_rows(
    const float *__restrict__ qkv, int ldqkv, int qheads, const float *__restrict__ rc,
    const float *__restrict__ rs, uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
    size_t kv_seq_stride, const int *__restrict__ ctx_dev, int ctx0, int max_ctx, int chunk,
    float scale, float *__restrict__ q_cap, float *__restrict__ ws_m, float *__restrict__ ws_l,
    float *__restrict__ ws_o, float *__restrict__ attn, int8_t *__restrict__ aqs,
    uint16_t *__restrict__ ad, int16_t *__restrict__ as, KvPages pg) {
    using L = RowsLds<D, G>;
    constexpr int KS = D / 32, DT = D / 16, HALF = D / 2, NWG = L::NWG, ROWS = L::ROWS;
    constexpr int RW = L::RW, KVD = G * D;
    constexpr int RP = KVD / 8;                     // 16-byte pieces per row
    constexpr int PT = ROWS * RP / 256;             // pieces per thread per step (K; same for V)
    static_assert(ROWS * RP % 256 == 0, "whole pieces per thread");
    extern __shared__ __attribute__((aligned(16))) char smem[];
    uint16_t *newk = (uint16_t *)smem;  // [G*D] fp16 K row of the new token (RoPE'd)
    uint16_t *newv = newk + KVD;        // [G*D] its V row
    char *big = smem + 2 * KVD * 2;
    // [2][K, V][ROWS][RW]: even steps stage their rows in copy 0, odd steps
    // in copy 1, so a step's staging never overwrites rows another
    // wavefront may still be reading (one barrier per step)
    _Float16 *kt0 = (_Float16 *)big;
    _Float16 *vt0 = kt0 + ROWS * RW;
    _Float16 *kt1 = vt0 + ROWS * RW;
    _Float16 *vt1 = kt1 + ROWS * RW;

    const int sp = blockIdx.x, qi = blockIdx.y, ns = gridDim.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int g = wave % G, wj = wave / G;  // group, tile slot within the step
    const int per = qheads / G;
    const int qd = qheads * D;
    int ctx = ctx_dev ? ctx_dev[qi] : ctx0;
    ctx = min(ctx, max_ctx);
    const int pnew = ctx - 1;  // < 0: empty context (device-supplied only)
    const int p0 = sp * chunk;
    const int p1 = min(ctx, p0 + chunk);
    // rows the loads may touch: known at launch, so the first loads need not
    // wait for ctx_dev (the cache holds max_ctx rows per sequence)
    const int pmax = min(max_ctx, p0 + chunk);
    const bool owner = pnew >= p0 && pnew < p1;
    const float *row = qkv + (size_t)qi * ldqkv;
    const float *cr = rc + (size_t)max(pnew, 0) * HALF;
    const float *sr = rs + (size_t)max(pnew, 0) * HALF;
    // cache row of position p: pg.at<PAGED>(qi, p, ...) (contiguous or paged)

    // 1. the fused q|k|v row (q of every head, then the new token's raw K
    //    and V rows) and the RoPE cos|sin row at its position, as float4
    //    pieces with clamped indices (no branches)
    float *qraw = (float *)big;        // [G*per][D]
    float *kraw = qraw + G * per * D;  // [G][D]
    float *vraw = kraw + KVD;          // [G][D]
    float *csr = vraw + KVD;           // [HALF] cos, [HALF] sin
    const int nrow4 = (qd + 2 * KVD) / 4;
    constexpr int ROW4PT = ((16 + 2) * G * D / 4 + 255) / 256;  // per <= 16
    float4 rv[ROW4PT];
#pragma unroll
    for (int u = 0; u < ROW4PT; ++u)
        rv[u] = ((const float4 *)row)[min(tid + u * 256, nrow4 - 1)];
    float4 csv;
    {
        const int t = min(tid, D / 4 - 1);
        const float4 *cp = t < HALF / 4 ? (const float4 *)cr + t : (const float4 *)sr + (t - HALF / 4);
        csv = *cp;
    }
    // 2. the first two steps' whole rows (positions clamped into the chunk,
    //    or row 0 for an empty context; such rows are masked out of the
    //    scores): two register buffers keep two steps of loads in flight
    uint4 ak[PT], av[PT], bk[PT], bv[PT];
    auto load_step = [&](uint4 (&rk)[PT], uint4 (&rvv)[PT], int ps) {
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const int c = (wave * PT + i) * 64 + lane;  // a wavefront's pieces are contiguous
            const int r = c / RP, e = (c % RP) * 8;
            const size_t ro = pg.template at<PAGED>(qi, max(min(ps + r, pmax - 1), 0), kv_seq_stride, KVD);
            rk[i] = *(const uint4 *)(kc + ro + e);
            rvv[i] = *(const uint4 *)(vc + ro + e);
        }
    };
    load_step(ak, av, p0);
    // issue order A then B, as in the loop (interleaved loads here would make
    // the compiler's wait counts for the loop conservative)
    __builtin_amdgcn_sched_barrier(0);
    load_step(bk, bv, p0 + ROWS);
    // unconditional stores at the clamped index (duplicates write equal
    // values): a guarded store lets the compiler sink its load behind the
    // K/V loads above and wait for all of them
#pragma unroll
    for (int u = 0; u < ROW4PT; ++u) ((float4 *)qraw)[min(tid + u * 256, nrow4 - 1)] = rv[u];
    ((float4 *)csr)[min(tid, D / 4 - 1)] = csv;
    __syncthreads();
    // rotate-half RoPE (qwen_one_layer.c:172-183) of element dd of a head row
    auto rot = [&](const float *v, int dd) {
        const int i = dd < HALF ? dd : dd - HALF;
        const float a = v[i], b = v[i + HALF], c = csr[i], s = csr[HALF + i];
        return dd < HALF ? __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s))
                         : __fadd_rn(__fmul_rn(b, c), __fmul_rn(a, s));
    };
    // the new token's K (rotated) and V rows in fp16, for every group (a
    // constant trip count: a loop with stores and no loads makes the
    // compiler drain every load in flight before it)
#pragma unroll
    for (int u = 0; u < (KVD + 255) / 256; ++u) {
        const int i = tid + 256 * u;
        if (i >= KVD) break;
        const uint16_t kh = f2h(rot(kraw + (i / D) * D, i % D));
        const uint16_t vh = f2h(vraw[i]);
        newk[i] = kh;
        newv[i] = vh;
        if (owner) {
            kc[pg.template at<PAGED>(qi, pnew, kv_seq_stride, KVD) + i] = kh;
            vc[pg.template at<PAGED>(qi, pnew, kv_seq_stride, KVD) + i] = vh;
        }
    }
    // Q^T of this wavefront's group as the B operand: lane holds
    // Q[head col][d = 32*ks + 8*grp + e]
    h8 qh[KS], ql[KS];
    {
        const bool hv = col < per && pnew >= 0;
        const int hc = col < per ? col : 0;
        const bool capq = q_cap && sp == 0 && wj == 0 && hv;
        const float *qh_row = qraw + (size_t)(g * per + hc) * D;
        auto ld8 = [](const float *p, float (&v)[8]) {
            const float4 a = *(const float4 *)p, b = *(const float4 *)(p + 4);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        };
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int d0 = 32 * ks + 8 * grp;
            const int i0 = d0 < HALF ? d0 : d0 - HALF;
            float a[8], b[8], c[8], sn[8], v[8];
            ld8(qh_row + i0, a);
            ld8(qh_row + i0 + HALF, b);
            ld8(csr + i0, c);
            ld8(csr + HALF + i0, sn);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                v[e] = !hv ? 0.0f
                           : (d0 < HALF ? __fsub_rn(__fmul_rn(a[e], c[e]), __fmul_rn(b[e], sn[e]))
                                        : __fadd_rn(__fmul_rn(b[e], c[e]), __fmul_rn(a[e], sn[e])));
                _Float16 hi, lo;
                hi_lo(v[e], hi, lo);
                qh[ks][e] = hi;
                ql[ks][e] = lo;
            }
            if (capq) {
                float *qc = q_cap + (size_t)qi * qd + (size_t)(g * per + hc) * D + d0;
                *(float4 *)qc = make_float4(v[0], v[1], v[2], v[3]);
                *(float4 *)(qc + 4) = make_float4(v[4], v[5], v[6], v[7]);
            }
        }
    }
    __syncthreads();  // newk/newv visible; the raw rows are no longer read

    float m = -INFINITY, lsum = 0.0f;
    f4 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = (f4){0.f, 0.f, 0.f, 0.f};
    const int nsteps = (p1 - p0 + ROWS - 1) / ROWS;  // 0 for an empty chunk
    auto step = [&](uint4 (&rk)[PT], uint4 (&rvv)[PT], int st, _Float16 *kt, _Float16 *vt) {
        const int ps = p0 + st * ROWS;
        const bool tail = ps + ROWS > p1;  // workgroup-uniform
        // stage the step's rows; V rows past the context as zeros (their
        // scores are masked); the new token's row from LDS, since its cache
        // row may not be written yet
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const int c = (wave * PT + i) * 64 + lane;
            const int r = c / RP, e = (c % RP) * 8;
            uint4 kv = rk[i], vv = rvv[i];
            if (tail) {  // rows past the context may hold any bits (NaN * 0 = NaN)
                const bool live = ps + r < p1;
                vv.x = live ? vv.x : 0u; vv.y = live ? vv.y : 0u;
                vv.z = live ? vv.z : 0u; vv.w = live ? vv.w : 0u;
            }
            if (owner) {  // workgroup-uniform
                const bool isnew = ps + r == pnew;
                const uint4 nk = *(const uint4 *)(newk + e), nv = *(const uint4 *)(newv + e);
                // per component: a select of whole uint4 values becomes a
                // select of stack addresses (scratch traffic)
                kv.x = isnew ? nk.x : kv.x; kv.y = isnew ? nk.y : kv.y;
                kv.z = isnew ? nk.z : kv.z; kv.w = isnew ? nk.w : kv.w;
                vv.x = isnew ? nv.x : vv.x; vv.y = isnew ? nv.y : vv.y;
                vv.z = isnew ? nv.z : vv.z; vv.w = isnew ? nv.w : vv.w;
            }
            *(uint4 *)(kt + r * RW + e) = kv;
            *(uint4 *)(vt + r * RW + e) = vv;
        }
        __syncthreads();
        // the step after next, unconditionally: clamped positions stay in
        // the chunk, and a branch here would make the compiler wait for both
        // buffers at every step
        load_step(rk, rvv, ps + 2 * ROWS);
        // this wavefront's tile: rows 16*wj .. +15 of the step, group g
        const int t0 = ps + DA_TILE * wj;
        h8 ka[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            ka[ks] = *(const h8 *)(kt + (DA_TILE * wj + col) * RW + g * D + 32 * ks + 8 * grp);
        f4 sacc = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[ks], qh[ks], sacc, 0, 0, 0);
            sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[ks], ql[ks], sacc, 0, 0, 0);
        }
        // lane holds S^T[pos = t0 + 4*grp + r][head col]
        float s[4], mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            s[r] = (t0 + 4 * grp + r < p1) ? sacc[r] * scale : -INFINITY;
            mx = fmaxf(mx, s[r]);
        }
        mx = fmaxf(mx, swap16_f(mx));
        mx = fmaxf(mx, swap32_f(mx));
        const float mnew = fmaxf(m, mx);
        // a tile past the chunk end leaves the state as it is (no NaN)
        const float mref = mnew == -INFINITY ? 0.0f : mnew;
        const float alpha = __expf(m - mref);
        float p[4], ps_ = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            p[r] = __expf(s[r] - mref);
            ps_ += p[r];
        }
        ps_ += swap16_f(ps_);
        ps_ += swap32_f(ps_);
        lsum = lsum * alpha + ps_;
        m = mnew;
        h4 ph, pl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            _Float16 hi, lo;
            hi_lo(p[r], hi, lo);
            ph[r] = hi;
            pl[r] = lo;
        }
        // A = V^T[d = g*D + 16*dt + col][pos = 4*grp + r] by the transposing
        // read: lane (col, grp) points at row 16*wj + 4*grp + col/4
        const _Float16 *vsrc = vt + (DA_TILE * wj + 4 * grp + (col >> 2)) * RW + g * D + 4 * (col & 3);
        // rescale only when some column's running max moved (alpha == 1
        // exactly otherwise: exp of 0), a wavefront-uniform branch
        if (__ballot(alpha != 1.0f)) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const h4 va = __builtin_bit_cast(h4, lds_read_tr16(vsrc + 16 * dt));
            f4 acc = o[dt];
            acc = __builtin_amdgcn_mfma_f32_16x16x16f16(va, ph, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pl, acc, 0, 0, 0);
            o[dt] = acc;
        }
        // no barrier: the next step stages the other copy, and the step
        // after it rewrites this one only once every wavefront has passed
        // the next step's barrier, i.e. finished reading this step's rows
    };
    // steps in pairs (workgroup-uniform); the second step of the last pair
    // of an odd count lies past the chunk, is masked out entirely and
    // leaves the softmax state as it is
    for (int st = 0; st < nsteps; st += 2) {
        step(ak, av, st, kt0, vt0);
        step(bk, bv, st + 1, kt1, vt1);
    }
    __syncthreads();  // the rows' LDS is reused below

    if constexpr (NWG == 1 && !FINAL) {
        // one wavefront per group: its state is the chunk's partial, written
        // from registers (lane (col, grp) holds O^T[16*dt + 4*grp + r][col])
        if (col < per) {
            const size_t pi = ((size_t)qi * qheads + g * per + col) * ns + sp;
            if (grp == 0) {
                ws_m[pi] = m;
                ws_l[pi] = lsum;
            }
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
                *(float4 *)(ws_o + pi * D + 16 * dt + 4 * grp) =
                    make_float4(o[dt][0], o[dt][1], o[dt][2], o[dt][3]);
        }
        return;
    }
    // merge the NWG wavefront states of each group in LDS (reusing the rows)
    float *mm = (float *)big;                   // [G][NWG][per]
    float *ml = mm + G * NWG * per;             // [G][NWG][per]
    float *mo = ml + G * NWG * per;             // [G][NWG][per][D]
    float *sc = mo + (size_t)G * NWG * per * D;  // [G][per][NWG]
    float *ltot = sc + G * per * NWG;           // [G][per]
    float *mtot = ltot + G * per;               // [G][per]
    if (col < per) {
        const int si = (g * NWG + wj) * per + col;
        if (grp == 0) {
            mm[si] = m;
            ml[si] = lsum;
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r) mo[(size_t)si * D + 16 * dt + 4 * grp + r] = o[dt][r];
    }
    __syncthreads();
    if (tid < G * per) {
        const int gg = tid / per, hc = tid % per;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NWG; ++w) M = fmaxf(M, mm[(gg * NWG + w) * per + hc]);
        float l = 0.0f;
#pragma unroll
        for (int w = 0; w < NWG; ++w) {
            const float f = M == -INFINITY ? 0.0f : expf(mm[(gg * NWG + w) * per + hc] - M);
            sc[tid * NWG + w] = f;
            l = fmaf(ml[(gg * NWG + w) * per + hc], f, l);
        }
        ltot[tid] = l;
        mtot[tid] = M;
    }
    __syncthreads();
    // 4 consecutive elements per thread; 8 lanes = 32 elements = one Q8_0
    // block of one head (D is a multiple of 32); heads in global order
    const int nel4 = qd / 4;
    for (int e40 = 0; e40 < nel4; e40 += 256) {
        const int e4 = e40 + tid;
        const bool ok = e4 < nel4;
        const int ec = 4 * min(e4, nel4 - 1);
        const int h = ec / D, dd = ec - h * D;  // h = gg * per + hc
        const int gg = h / per, hc = h - gg * per;
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int w = 0; w < NWG; ++w) {
            const float4 ov = *(const float4 *)(mo + ((size_t)(gg * NWG + w) * per + hc) * D + dd);
            const float f = sc[h * NWG + w];
            acc[0] = fmaf(ov.x, f, acc[0]);
            acc[1] = fmaf(ov.y, f, acc[1]);
            acc[2] = fmaf(ov.z, f, acc[2]);
            acc[3] = fmaf(ov.w, f, acc[3]);
        }
        if (!FINAL) {
            if (ok) {
                const size_t pi = ((size_t)qi * qheads + h) * ns + sp;
                if (dd == 0) {
                    ws_m[pi] = mtot[h];
                    ws_l[pi] = ltot[h];
                }
                *(float4 *)(ws_o + pi * D + dd) = make_float4(acc[0], acc[1], acc[2], acc[3]);
            }
        } else if (e40 + (tid & ~7) < nel4) {
            // normalise (attention_kernels.h:163; no context: 0, :95-98) and
            // quantize_q8
            const float r = mtot[h] == -INFINITY ? 0.0f : 1.0f / ltot[h];
            const float y[4] = {acc[0] * r, acc[1] * r, acc[2] * r, acc[3] * r};
            uint16_t dbits;
            int bsum;
            const uint32_t q = quant_block_oct(y, dbits, bsum);
            if (ok) {
                const size_t off = (size_t)qi * qd + (size_t)h * D + dd;
                *(float4 *)(attn + off) = make_float4(y[0], y[1], y[2], y[3]);
                *(uint32_t *)(aqs + off) = q;
                if ((e4 & 7) == 0) {
                    ad[off / SI_QK] = dbits;
                    if (as) as[off / SI_QK] = (int16_t)bsum;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// launch policy
// ---------------------------------------------------------------------------
void launch_dec_qkv(const float *x, const float *gain, int hidden, float eps, const uint8_t *wqs,
                    const uint16_t *wd, int tile, int n, const float *bias, float *cap_normed,
                    int8_t *cap_qs, uint16_t *cap_d, int16_t *cap_s, float *qkv, bool exact,
                    hipStream_t st) {
#define CALL(R, T, E)                                                                            \
    SI_LAUNCH((k_dec_qkv<R, T, E>), dim3((n + R - 1) / R), dim3(T),                              \
              (DecLds<R, T>::bytes(hidden, false, 0)), st, x, gain, hidden, eps, wqs,            \
              wd, tile, n, bias, cap_normed, cap_qs, cap_d, cap_s, qkv)
    if (exact) {
        CALL(64, 64, true);
    } else {
        const int r = tile < 64 ? tile : 64;
        SI_GEMV_SWITCH(r, dec_threads(r, hidden / SI_QK), CALL)
    }
#undef CALL
}

void launch_dec_wo(const float *pm, const float *pl, const float *po, int ns, int qheads,
                   int hdim, const uint8_t *wqs, const uint16_t *wd, int tile, int n,
                   const float *residual, float *cap_attn, int8_t *cap_qs, uint16_t *cap_d,
                   int16_t *cap_s, float *cap_y, float *out, bool exact, hipStream_t st) {
    const int qd = qheads * hdim;
#define CALL(R, T, E)                                                                            \
    SI_LAUNCH((k_dec_wo<R, T, E>), dim3((n + R - 1) / R), dim3(T),                               \
              (DecLds<R, T>::bytes(qd, false, 0)), st, pm, pl, po, ns,                           \
              qheads, hdim, wqs, wd, tile, n, residual, cap_attn, cap_qs, cap_d, cap_s,          \
              cap_y, out)
    if (exact) {
        CALL(64, 64, true);
    } else {
        const int r = tile < 64 ? tile : 64;
        SI_GEMV_SWITCH(r, dec_threads(r, qd / SI_QK), CALL)
    }
#undef CALL
}

// gate|up: 64 logical rows per workgroup (32 gate + 32 up rows, one scale
// tile of 32 each), 8 K lanes per row when K has >= 8 blocks.
void launch_dec_gateup(const float *h, const float *gain, int hidden, float eps,
                       const uint8_t *wqs, const uint16_t *wd, int tile, int f,
                       float *cap_normed, int8_t *cap_qs, uint16_t *cap_d, int16_t *cap_s,
                       float *gu, float *act, int8_t *aqs, uint16_t *ad, int16_t *as, bool exact,
                       hipStream_t st) {
    const int n = 2 * f;
#define CALL(R, T, E)                                                                            \
    SI_LAUNCH((k_dec_gateup<R, T, E>), dim3((n + R - 1) / R), dim3(T),                           \
              (DecLds<R, T>::bytes(hidden, false, 0)), st, h, gain, hidden, eps, wqs,            \
              wd, tile, f, cap_normed, cap_qs, cap_d, cap_s, gu, act, aqs, ad, as)
    if (exact) {
        CALL(64, 64, true);
    } else if (hidden / SI_QK >= 8) {
        CALL(64, 512, false);
    } else {
        CALL(64, 256, false);
    }
#undef CALL
}

// Decode attention: DA_NW wavefronts per workgroup; chunks so that every
// wavefront has about two 16-position tiles, at most 32 chunks, and no more
// than ~1024 workgroups in total.
constexpr int DA_NW = 8;

// LDS of a whole-row workgroup (two copies of a step's K and V rows):
// two workgroups still fit a CU's 160 KB
constexpr size_t ROWS_LDS_MAX = 80 * 1024;

// The whole-row kernel serves batches (>= 8 queries: one query is latency
// bound and k_dec_attn's shorter chain wins) of 1, 2 or 4 KV groups of up to
// 16 query heads.
static bool dec_rows_ok(int qheads, int kvheads, int hdim, int nq) {
    if (nq < 8 || !(kvheads == 1 || kvheads == 2 || kvheads == 4)) return false;
    if (qheads % kvheads || qheads / kvheads > 16) return false;
    const int per = qheads / kvheads;
    size_t b = 0;
#define RB(DIM)                                                             \
    b = kvheads == 1 ? RowsLds<DIM, 1>::bytes(per)                          \
                     : kvheads == 2 ? RowsLds<DIM, 2>::bytes(per) : RowsLds<DIM, 4>::bytes(per)
    switch (hdim) {
        case 32: RB(32); break;
        case 64: RB(64); break;
        case 96: RB(96); break;
        case 128: RB(128); break;
        default: return false;
    }
#undef RB
    return b <= ROWS_LDS_MAX;
}

// A single query over more than 128 tiles (2048 positions) takes 4
// wavefronts per workgroup and up to 64 chunks of one tile per wavefront:
// twice the workgroups of 8-wavefront chunks, whose 32-chunk cap left half
// the CUs idle (7B, context 4096: attention 8.5-8.9 -> 7.2-7.4 us, the
// layer 52.1 -> 51.3 us with the larger merge).
static bool dec_long_single(int nq, int max_ctx) {
    return nq == 1 && (max_ctx + DA_TILE - 1) / DA_TILE > 128;
}

int dec_attn_chunks(int qheads, int kvheads, int hdim, int nq, int max_ctx) {
    if (dec_rows_ok(qheads, kvheads, hdim, nq)) {
        // >= 4 steps of 16*(4/kvheads) positions per chunk (fewer partials
        // for the consumer to merge), <= ~512 workgroups (2 per CU), <= 32
        // chunks
        const int rows = DA_TILE * (4 / kvheads);
        int ns = (max_ctx + 4 * rows - 1) / (4 * rows);
        const int cap = (512 + nq - 1) / nq;
        if (ns > cap) ns = cap;
        if (ns > 32) ns = 32;
        return ns < 1 ? 1 : ns;
    }
    const int tiles = (max_ctx + DA_TILE - 1) / DA_TILE;
    if (dec_long_single(nq, max_ctx)) {
        const int ns = (tiles + 3) / 4;
        return ns > 64 ? 64 : ns;
    }
    if (nq == 1) {
        // one query is latency bound: one tile per wavefront (the shortest
        // chain), up to 32 chunks
        const int ns = (tiles + DA_NW - 1) / DA_NW;
        return ns < 1 ? 1 : (ns > 32 ? 32 : ns);
    }
    int ns = (tiles + 2 * DA_NW - 1) / (2 * DA_NW);
    // enough workgroups to cover the CUs once; a context split beyond that
    // only adds pipeline ramps and partial sums (7B, 64 x 4096: 131 -> 118 us)
    if (ns * kvheads * nq > 256) ns = (256 + kvheads * nq - 1) / (kvheads * nq);
    if (ns > 32) ns = 32;
    return ns < 1 ? 1 : ns;
}

size_t dec_attn_workspace_bytes(int qheads, int hdim, int kvheads, int nq, int max_ctx) {
    const int ns = dec_attn_chunks(qheads, kvheads, hdim, nq, max_ctx);
    return (size_t)nq * qheads * ns * (hdim + 2) * sizeof(float);
}

template <bool PAGED>
static void dec_attn_impl(const float *qkv, int ldqkv, int nq, int qheads, int kvheads, int hdim,
                          const float *rc, const float *rs, uint16_t *kc, uint16_t *vc,
                          size_t kv_seq_stride, const int *ctx_dev, int ctx0, int max_ctx,
                          float *q_cap, int ns, void *workspace, float *attn, int8_t *aqs,
                          uint16_t *ad, int16_t *as, hipStream_t st, KvPages pg) {
    if (nq <= 0) return;
    int chunk = (max_ctx + ns - 1) / ns;
    chunk = (chunk + DA_TILE - 1) / DA_TILE * DA_TILE;
    float *ws_m = (float *)workspace;
    float *ws_l = ws_m + (size_t)nq * qheads * ns;
    float *ws_o = ws_l + (size_t)nq * qheads * ns;
    const float scale = 1.0f / sqrtf((float)hdim);  // attention_kernels.h:86
    const int per = qheads / kvheads;
    const bool fin = attn != nullptr;
    if (dec_rows_ok(qheads, kvheads, hdim, nq)) {
#define RCALL(DIM, GG, FIN)                                                                       \
    do {                                                                                          \
        static bool big_lds = false;                                                              \
        if (!big_lds) {                                                                           \
            /* past 64 KB of dynamic LDS; a failure surfaces as the launch's error */            \
            (void)hipFuncSetAttribute((const void *)k_dec_attn_rows<DIM, GG, FIN, PAGED>,         \
                                      hipFuncAttributeMaxDynamicSharedMemorySize,                 \
                                      (int)ROWS_LDS_MAX);                                         \
            big_lds = true;                                                                       \
        }                                                                                         \
        SI_LAUNCH((k_dec_attn_rows<DIM, GG, FIN, PAGED>), dim3(ns, nq), dim3(256),                \
                  (RowsLds<DIM, GG>::bytes(per)), st, qkv, ldqkv, qheads, rc, rs, kc, vc,         \
                  kv_seq_stride, ctx_dev, ctx0, max_ctx, chunk, scale, q_cap, ws_m, ws_l,         \
                  ws_o, attn, aqs, ad, as, pg);                                                   \
    } while (0)
#define RCALLG(DIM)                                                \
    if (kvheads == 1) {                                            \
        if (fin) RCALL(DIM, 1, true); else RCALL(DIM, 1, false);   \
    } else if (kvheads == 2) {                                     \
        if (fin) RCALL(DIM, 2, true); else RCALL(DIM, 2, false);   \
    } else {                                                       \
        if (fin) RCALL(DIM, 4, true); else RCALL(DIM, 4, false);   \
    }
        switch (hdim) {
            case 32: RCALLG(32); break;
            case 64: RCALLG(64); break;
            case 96: RCALLG(96); break;
            default: RCALLG(128); break;
        }
#undef RCALLG
#undef RCALL
        return;
    }
    const dim3 grid(ns, kvheads, nq);
#define CALL(DIM, NW, FIN, DEP)                                                                \
    SI_LAUNCH((k_dec_attn<DIM, NW, FIN, PAGED, DEP>), grid, dim3(NW * 64),                     \
              (AttnLds<DIM, NW>::bytes(per)), st, qkv, ldqkv, qheads, kvheads, rc, rs,         \
              kc, vc, kv_seq_stride, ctx_dev, ctx0, max_ctx, chunk, scale, q_cap,              \
              ws_m, ws_l, ws_o, attn, aqs, ad, as, pg, DecQkvIn{})
#define CALLN(DIM, NW, FIN)                                             \
    if (chunk <= DA_TILE * NW) {                                        \
        CALL(DIM, NW, FIN, 1);                                          \
    } else {                                                            \
        CALL(DIM, NW, FIN, 2);                                          \
    }
    // 8 wavefronts unless the merge buffers of a wide GQA group exceed 64
    // KiB or a single query spans many chunks (dec_long_single); one K/V
    // tile in flight per wavefront when each has at most one (chunk <= 16 *
    // NW positions)
    const bool long1 = dec_long_single(nq, max_ctx);
#define CALLD(DIM)                                           \
    if (AttnLds<DIM, DA_NW>::bytes(per) <= 65536 && !long1) { \
        if (fin) {                                           \
            CALLN(DIM, DA_NW, true);                         \
        } else {                                             \
            CALLN(DIM, DA_NW, false);                        \
        }                                                    \
    } else if (fin) {                                        \
        CALLN(DIM, 4, true);                                 \
    } else {                                                 \
        CALLN(DIM, 4, false);                                \
    }
    switch (hdim) {
        case 32: CALLD(32); break;
        case 64: CALLD(64); break;
        case 96: CALLD(96); break;
        default: CALLD(128); break;
    }
#undef CALLD
#undef CALLN
#undef CALL
}

// Single-token decode with the Q|K|V projection inside the attention
// (k_dec_attn<..., FQ>): worth it while a workgroup's 3*hdim weight rows
// stream in well under a kernel boundary (0.5B: 97 KB); 7B's 384 rows of
// 3584 values (774 KB) would take one CU several microseconds.  Past 2048
// positions the context splits into up to 64 chunks sized for 4-wavefront
// workgroups; every chunk would re-project its head's rows, so such
// contexts take the staged pair (k_dec_qkv, then k_dec_attn).
bool dec_qkv_attn_ok(int hidden, int qheads, int kvheads, int hdim, int ctx) {
    if (dec_long_single(1, ctx)) return false;
    if (kvheads <= 0 || qheads % kvheads || qheads / kvheads > 16) return false;
    if (hdim != 64 && hdim != 128) return false;
    if (hidden % SI_QK) return false;
    return (size_t)3 * hdim * (hidden / SI_QK) * 18 <= 128 * 1024;
}

void launch_dec_qkv_attn(const DecQkvIn &fq, int qheads, int kvheads, int hdim, const float *rc,
                         const float *rs, uint16_t *kc, uint16_t *vc, int ctx, int ns,
                         float *q_cap, void *workspace, hipStream_t st) {
    int chunk = (ctx + ns - 1) / ns;
    chunk = (chunk + DA_TILE - 1) / DA_TILE * DA_TILE;
    float *ws_m = (float *)workspace;
    float *ws_l = ws_m + (size_t)qheads * ns;
    float *ws_o = ws_l + (size_t)qheads * ns;
    const float scale = 1.0f / sqrtf((float)hdim);  // attention_kernels.h:86
    const dim3 grid(ns, qheads, 1);
#define FQCALL(DIM, DEP)                                                                       \
    SI_LAUNCH((k_dec_attn<DIM, DA_NW, false, false, DEP, true>), grid, dim3(DA_NW * 64),       \
              ((AttnLds<DIM, DA_NW>::bytes(1) + 15) / 16 * 16 +                                \
               FqLds<DIM, DA_NW>::bytes(fq.hidden)),                                           \
              st, nullptr, 0, qheads, kvheads, rc, rs, kc, vc, (size_t)0, nullptr, ctx, ctx,   \
              chunk, scale, q_cap, ws_m, ws_l, ws_o, nullptr, nullptr, nullptr, nullptr,       \
              KvPages(), fq)
    const bool one = chunk <= DA_TILE * DA_NW;
    if (hdim == 64) {
        if (one) FQCALL(64, 1); else FQCALL(64, 2);
    } else {
        if (one) FQCALL(128, 1); else FQCALL(128, 2);
    }
#undef FQCALL
}

void launch_dec_attn(const float *qkv, int ldqkv, int nq, int qheads, int kvheads, int hdim,
                     const float *rc, const float *rs, uint16_t *kc, uint16_t *vc,
                     size_t kv_seq_stride, const int *ctx_dev, int ctx0, int max_ctx,
                     float *q_cap, int ns, void *workspace, float *attn, int8_t *aqs,
                     uint16_t *ad, int16_t *as, hipStream_t st, KvPages pg) {
    if (pg.pages)
        dec_attn_impl<true>(qkv, ldqkv, nq, qheads, kvheads, hdim, rc, rs, kc, vc, kv_seq_stride,
                            ctx_dev, ctx0, max_ctx, q_cap, ns, workspace, attn, aqs, ad, as, st,
                            pg);
    else
        dec_attn_impl<false>(qkv, ldqkv, nq, qheads, kvheads, hdim, rc, rs, kc, vc,
                             kv_seq_stride, ctx_dev, ctx0, max_ctx, q_cap, ns, workspace, attn,
                             aqs, ad, as, st, pg);
}

}  // namespace si
