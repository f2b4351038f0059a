// si_quant.hip -- elementwise/normalisation kernels of the hot path, each
// ending in the bit-exact Q8_0 quantizer (qwen_one_layer.c:98-116):
//   quantize_q8 (AoS drop-in and planar), RMSNorm->Q8, residual+RMSNorm->Q8,
//   SwiGLU->Q8, and the lossless Q4_0 repack.
// All are HBM-streaming: one pass over the fp32 input, one write of the
// int8 payload (+2 B scale, +2 B block sum per 32 values).
#include "si_device.hpp"
#include "si_kernels.hpp"

namespace si {

// One Q8 block per half wavefront; blocks of 256 threads = 8 blocks.
__global__ void __launch_bounds__(256) k_quantize_q8_aos(const float *__restrict__ src,
                                                         uint8_t *__restrict__ dst, int nblocks) {
    const int blk = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int j = threadIdx.x & 31;
    if (blk >= nblocks) return;  // whole half-waves exit together
    const float x = src[(size_t)blk * SI_QK + j];
    uint16_t dbits;
    int bsum;
    const int q = quant_block_lane(x, dbits, bsum);
    uint8_t *rec = dst + (size_t)blk * 34;  // block_q8_0: {uint16 d; int8 qs[32]}
    rec[2 + j] = (uint8_t)(int8_t)q;
    if (j == 0) {
        rec[0] = (uint8_t)(dbits & 0xff);
        rec[1] = (uint8_t)(dbits >> 8);
    }
}

__global__ void __launch_bounds__(256) k_quantize_q8_rows(const float *__restrict__ src, int k,
                                                          int nblocks_row, int total_blocks,
                                                          int8_t *__restrict__ qs,
                                                          uint16_t *__restrict__ d,
                                                          int16_t *__restrict__ s) {
    const int blk = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int j = threadIdx.x & 31;
    if (blk >= total_blocks) return;
    const int r = blk / nblocks_row, b = blk - r * nblocks_row;
    const size_t off = (size_t)r * k + (size_t)b * SI_QK + j;
    uint16_t dbits;
    int bsum;
    const int q = quant_block_lane(src[off], dbits, bsum);
    qs[off] = (int8_t)q;
    if (j == 0) {
        d[blk] = dbits;
        if (s) s[blk] = (int16_t)bsum;
    }
}

// Quantizes n values held in LDS (row r) into the planar Q8 layout.
__device__ __forceinline__ void quantize_lds_row(const float *row_lds, int n, int r,
                                                 int8_t *__restrict__ qs,
                                                 uint16_t *__restrict__ d,
                                                 int16_t *__restrict__ s) {
    const int nb = n / SI_QK;
    const int hw = threadIdx.x >> 5, j = threadIdx.x & 31;
    const int nhw = blockDim.x >> 5;
    for (int b = hw; b < nb; b += nhw) {
        uint16_t dbits;
        int bsum;
        const int q = quant_block_lane(row_lds[b * SI_QK + j], dbits, bsum);
        qs[(size_t)r * n + b * SI_QK + j] = (int8_t)q;
        if (j == 0) {
            d[(size_t)r * nb + b] = dbits;
            if (s) s[(size_t)r * nb + b] = (int16_t)bsum;
        }
    }
}

// Block-wide double sum over blockDim.x / 64 wavefronts (scratch: one per
// wavefront), added in wavefront order.
__device__ __forceinline__ double block_sum_d(double v, double *scratch) {
    v = wave_sum_d(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) scratch[w] = v;
    __syncthreads();
    double t = 0.0;
    const int nw = blockDim.x >> 6;
    for (int i = 0; i < nw; ++i) t += scratch[i];
    return t;
}

// RMSNorm (qwen_one_layer.c:164-169): squares summed in binary64,
// inv = 1/sqrt(float(ss/n) + eps) correctly rounded, out = (x*inv)*gain.
// The binary64 partial sums are combined as a tree, not in index order;
// the float result equals the reference's except when the binary64 sum
// lands within a few ulp of a binary32 rounding boundary.
// Optionally first forms h = x + y (residual) and stores it.
template <bool RESIDUAL>
__global__ void __launch_bounds__(256) k_rmsnorm_q8(const float *__restrict__ x,
                                                    const float *__restrict__ y,
                                                    const float *__restrict__ gain, int n,
                                                    float eps, float *__restrict__ h_out,
                                                    float *__restrict__ normed,
                                                    int8_t *__restrict__ qs,
                                                    uint16_t *__restrict__ d,
                                                    int16_t *__restrict__ s) {
    extern __shared__ float lds[];  // n floats
    __shared__ double red[8];
    const int r = blockIdx.x;
    const float *xr = x + (size_t)r * n;
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float v = xr[i];
        if (RESIDUAL) {
            v = __fadd_rn(v, y[(size_t)r * n + i]);
            h_out[(size_t)r * n + i] = v;
        }
        lds[i] = v;
        ss += (double)v * (double)v;
    }
    const double tot = block_sum_d(ss, red);
    const float ms = (float)(tot / (double)n);
    const float inv = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(ms, eps)));
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float v = __fmul_rn(lds[i], inv);
        v = __fmul_rn(v, gain ? gain[i] : 1.0f);
        lds[i] = v;
        if (normed) normed[(size_t)r * n + i] = v;
    }
    __syncthreads();
    quantize_lds_row(lds, n, r, qs, d, s);
}

// The same RMSNorm + Q8_0 with the row held in registers: thread t owns the
// float4 chunks t + T*i (i < NPT) of its workgroup's row, so 8 consecutive
// threads hold one 32-value block and quantize it with quant_block_oct.  One
// pass over global memory, no LDS staging; needs 16-byte aligned rows.
// PARTS (with RESIDUAL): y is the split-order sum of y[sp * rows * n + ...]
// for sp < splits (a K-split GEMM's partials), also written to y_out.
// tq/td (optional): the Q8_0 row written operand-tiled as well
// (q8_tiled_byte; a thread's 4 values are 4 consecutive bytes there too).
// x6 (optional): the row's fp6 GEMM codes as well (f6_store_oct, m =
// gridDim.x rows).
// T threads per row: 1024 for a few long rows (each thread's serial share
// of the quantization shrinks), 256 otherwise.
template <bool RESIDUAL, int NPT, bool PARTS = false, int T = 256>
__global__ void __launch_bounds__(T) k_rmsnorm_q8_v4(const float *__restrict__ x,
                                                       const float *__restrict__ y,
                                                       const float *__restrict__ gain, int n,
                                                       float eps, float *__restrict__ h_out,
                                                       float *__restrict__ normed,
                                                       int8_t *__restrict__ qs,
                                                       uint16_t *__restrict__ d,
                                                       int16_t *__restrict__ s, int splits = 1,
                                                       float *__restrict__ y_out = nullptr,
                                                       int8_t *__restrict__ tq = nullptr,
                                                       uint16_t *__restrict__ td = nullptr,
                                                       uint8_t *__restrict__ x6 = nullptr) {
    __shared__ double red[T / 64];
    const int r = blockIdx.x, tid = threadIdx.x, n4 = n / 4;
    const size_t base = (size_t)r * n;
    float v[NPT][4];
    // the gain is read with the row, not after the reduction
    float4 gv[NPT];
#pragma unroll
    for (int i = 0; i < NPT; ++i)
        gv[i] = gain ? *(const float4 *)(gain + 4 * min(tid + T * i, n4 - 1))
                     : make_float4(1.f, 1.f, 1.f, 1.f);
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
        const int c = min(tid + T * i, n4 - 1);  // clamped: branch-free loads
        float4 a = *(const float4 *)(x + base + 4 * c);
        if (RESIDUAL) {
            float4 b = *(const float4 *)(y + base + 4 * c);
            if (PARTS) {
                // groups of 8 splits, loads branch-free (clamped split,
                // selected out of the sum) so a group is in flight together
                const size_t ps = (size_t)gridDim.x * n;
                for (int s0 = 1; s0 < splits; s0 += 8) {
                    float4 p[8];
#pragma unroll
                    for (int k = 0; k < 8; ++k)
                        p[k] = *(const float4 *)(y + min(s0 + k, splits - 1) * ps + base + 4 * c);
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        const bool on = s0 + k < splits;
                        b.x = on ? b.x + p[k].x : b.x;
                        b.y = on ? b.y + p[k].y : b.y;
                        b.z = on ? b.z + p[k].z : b.z;
                        b.w = on ? b.w + p[k].w : b.w;
                    }
                }
                if (tid + T * i < n4) *(float4 *)(y_out + base + 4 * c) = b;
            }
            a = make_float4(__fadd_rn(a.x, b.x), __fadd_rn(a.y, b.y), __fadd_rn(a.z, b.z),
                            __fadd_rn(a.w, b.w));
        }
        v[i][0] = a.x; v[i][1] = a.y; v[i][2] = a.z; v[i][3] = a.w;
        if (tid + T * i < n4) {
            if (RESIDUAL) *(float4 *)(h_out + base + 4 * c) = a;
#pragma unroll
            for (int k = 0; k < 4; ++k) ss += (double)v[i][k] * (double)v[i][k];
        }
    }
    const double tot = block_sum_d(ss, red);
    const float ms = (float)(tot / (double)n);
    const float inv = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(ms, eps)));
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
        const int c = tid + T * i;
        if (c < n4) {  // whole 8-thread groups (n is a multiple of 32)
            const float g4[4] = {gv[i].x, gv[i].y, gv[i].z, gv[i].w};
            float o[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = __fmul_rn(__fmul_rn(v[i][k], inv), g4[k]);
            if (normed) *(float4 *)(normed + base + 4 * c) = make_float4(o[0], o[1], o[2], o[3]);
            uint16_t dbits;
            int bsum;
            const uint32_t packed = quant_block_oct(o, dbits, bsum);
            *(uint32_t *)(qs + base + 4 * c) = packed;
            if ((tid & 7) == 0) {
                const size_t bi = (base + 4 * c) / SI_QK;
                d[bi] = dbits;
                if (s) s[bi] = (int16_t)bsum;
            }
            if (tq) {
                const size_t pb = (size_t)(r >> 5) * (n / SI_QK) + (4 * c) / SI_QK;
                *(uint32_t *)(tq + q8_tiled_byte(pb, r & 31, (4 * c) % SI_QK)) = packed;
                if ((tid & 7) == 0) td[pb * 32 + (r & 31)] = dbits;
            }
            if (x6) f6_store_oct(packed, x6, gridDim.x, r, (4 * c) / SI_QK);
        }
    }
}

// Build-defined SwiGLU then quantize_q8: a = (g / (1 + expf(-g))) * u
// (tq/td, optional: the Q8_0 also operand-tiled, q8_tiled_byte).
__global__ void __launch_bounds__(256) k_swiglu_q8(const float *__restrict__ gu, int f,
                                                   int nb_row, int total_blocks,
                                                   float *__restrict__ act,
                                                   int8_t *__restrict__ qs,
                                                   uint16_t *__restrict__ d,
                                                   int16_t *__restrict__ s,
                                                   int8_t *__restrict__ tq,
                                                   uint16_t *__restrict__ td) {
    const int blk = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int j = threadIdx.x & 31;
    if (blk >= total_blocks) return;
    const int r = blk / nb_row, b = blk - r * nb_row;
    const float *row = gu + (size_t)r * 2 * f;
    const float g = row[b * SI_QK + j];
    const float u = row[f + b * SI_QK + j];
    const float silu = __fdiv_rn(g, __fadd_rn(1.0f, expf(-g)));
    const float a = __fmul_rn(silu, u);
    const size_t off = (size_t)r * f + (size_t)b * SI_QK + j;
    if (act) act[off] = a;
    uint16_t dbits;
    int bsum;
    const int q = quant_block_lane(a, dbits, bsum);
    qs[off] = (int8_t)q;
    if (j == 0) {
        d[blk] = dbits;
        if (s) s[blk] = (int16_t)bsum;
    }
    if (tq) {
        const size_t pb = (size_t)(r >> 5) * nb_row + b;
        tq[q8_tiled_byte(pb, r & 31, j)] = (int8_t)q;
        if (j == 0) td[pb * 32 + (r & 31)] = dbits;
    }
}

// Row-major 18-byte Q4_0 blocks -> [K/32][N][16] nibbles + [K/32][N] scales.
__global__ void k_q4_repack(const uint8_t *__restrict__ src, int n, int nb, int tile,
                            uint8_t *__restrict__ qs, uint16_t *__restrict__ d) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // i = b*n + row
    if (i >= (size_t)n * nb) return;
    const int b = (int)(i / n), row = (int)(i - (size_t)b * n);
    const uint8_t *blk = src + ((size_t)row * nb + b) * 18;
    d[q4_scale_index(row, b, nb, tile)] = (uint16_t)(blk[0] | (blk[1] << 8));
    uint32_t w[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
        w[t] = (uint32_t)blk[2 + 4 * t] | ((uint32_t)blk[3 + 4 * t] << 8) |
               ((uint32_t)blk[4 + 4 * t] << 16) | ((uint32_t)blk[5 + 4 * t] << 24);
    *(uint4 *)(qs + i * 16) = make_uint4(w[0], w[1], w[2], w[3]);
}

__global__ void k_q4_unpack(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ d,
                            int n, int nb, int tile, uint8_t *__restrict__ dst) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)n * nb) return;
    const int b = (int)(i / n), row = (int)(i - (size_t)b * n);
    uint8_t *blk = dst + ((size_t)row * nb + b) * 18;
    const uint16_t dv = d[q4_scale_index(row, b, nb, tile)];
    blk[0] = (uint8_t)(dv & 0xff);
    blk[1] = (uint8_t)(dv >> 8);
    for (int t = 0; t < 16; ++t) blk[2 + t] = qs[i * 16 + t];
}

// ----------------------------------------------------------------------
// launchers
// ----------------------------------------------------------------------
void launch_quantize_q8_aos(const float *src, void *dst, int count, hipStream_t st) {
    const int nb = count / SI_QK;
    if (nb == 0) return;
    SI_LAUNCH(k_quantize_q8_aos, dim3((nb + 7) / 8), dim3(256), 0, st, src,
              (uint8_t *)dst, nb);
}

void launch_quantize_q8_rows(const float *src, int rows, int k, int8_t *qs, uint16_t *d,
                             int16_t *s, hipStream_t st) {
    const int nbr = k / SI_QK, tot = nbr * rows;
    if (tot == 0) return;
    SI_LAUNCH(k_quantize_q8_rows, dim3((tot + 7) / 8), dim3(256), 0, st, src, k, nbr,
              tot, qs, d, s);
}

void launch_rmsnorm_q8_parts(const float *x, const float *part, int splits, const float *gain,
                             int rows, int n, float eps, float *y_out, float *h, float *normed,
                             int8_t *qs, uint16_t *d, int16_t *s, hipStream_t st, int8_t *tq,
                             uint16_t *td, uint8_t *x6) {
    if (rows == 0) return;
    const auto al = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    const int n4 = n / 4;
    if (!(n4 <= 2048 && al(x) && al(part) && al(y_out) && al(h) && al(normed) && al(gain) &&
          al(qs))) {
        launch_gemm_reduce(part, splits, rows, n, y_out, st);
        launch_rmsnorm_q8(x, y_out, gain, rows, n, eps, h, normed, qs, d, s, st, tq, td, x6);
        return;
    }
#define RMS_P(NPT)                                                                              \
    SI_LAUNCH((k_rmsnorm_q8_v4<true, NPT, true>), dim3(rows), dim3(256), 0, st, x, part,        \
              gain, n, eps, h, normed, qs, d, s, splits, y_out, tq, td, x6)
    if (n4 <= 256) RMS_P(1);
    else if (n4 <= 512) RMS_P(2);
    else if (n4 <= 1024) RMS_P(4);
    else RMS_P(8);
#undef RMS_P
}

void launch_rmsnorm_q8(const float *x, const float *y, const float *gain, int rows, int n,
                       float eps, float *h, float *normed, int8_t *qs, uint16_t *d, int16_t *s,
                       hipStream_t st, int8_t *tq, uint16_t *td, uint8_t *x6) {
    if (rows == 0) return;
    const auto al = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    const int n4 = n / 4;
    if (n4 <= 2048 && al(x) && al(y) && al(h) && al(normed) && al(gain) && al(qs)) {
        // a few long rows (batched decode): 1024 threads per row
        const bool wide = rows <= 128 && n4 > 256;
        const int npt = wide ? (n4 <= 1024 ? 1 : 2)
                             : n4 <= 256 ? 1 : n4 <= 512 ? 2 : n4 <= 1024 ? 4 : 8;
#define RMS_V4(RES, NPT, T)                                                                       \
    SI_LAUNCH((k_rmsnorm_q8_v4<RES, NPT, false, T>), dim3(rows), dim3(T), 0, st, x, y, gain, n,   \
              eps, h, normed, qs, d, s, 1, (float *)nullptr, tq, td, x6)
#define RMS_V4N(RES)                             \
    if (wide) {                                  \
        if (npt == 1) RMS_V4(RES, 1, 1024);      \
        else RMS_V4(RES, 2, 1024);               \
    } else {                                     \
        switch (npt) {                           \
            case 1: RMS_V4(RES, 1, 256); break;  \
            case 2: RMS_V4(RES, 2, 256); break;  \
            case 4: RMS_V4(RES, 4, 256); break;  \
            default: RMS_V4(RES, 8, 256); break; \
        }                                        \
    }
        if (y) {
            RMS_V4N(true);
        } else {
            RMS_V4N(false);
        }
#undef RMS_V4N
#undef RMS_V4
        return;
    }
    const size_t lds = (size_t)n * sizeof(float);
    if (y)
        SI_LAUNCH(k_rmsnorm_q8<true>, dim3(rows), dim3(256), lds, st, x, y, gain, n,
                  eps, h, normed, qs, d, s);
    else
        SI_LAUNCH(k_rmsnorm_q8<false>, dim3(rows), dim3(256), lds, st, x, y, gain, n,
                  eps, h, normed, qs, d, s);
    if (tq) launch_q8_tile(qs, d, rows, n, tq, td, st);  // this path writes planar only
    if (x6) launch_q8_to_x6(qs, rows, n / SI_QK, x6, st);
}

void launch_swiglu_q8(const float *gu, int rows, int f, float *act, int8_t *qs, uint16_t *d,
                      int16_t *s, hipStream_t st, int8_t *tq, uint16_t *td) {
    const int nbr = f / SI_QK, tot = nbr * rows;
    if (tot == 0) return;
    SI_LAUNCH(k_swiglu_q8, dim3((tot + 7) / 8), dim3(256), 0, st, gu, f, nbr, tot, act,
              qs, d, s, tq, td);
}

void launch_q4_repack(const uint8_t *src, int n, int k, int tile, uint8_t *qs, uint16_t *d,
                      hipStream_t st) {
    const size_t tot = (size_t)n * (k / SI_QK);
    if (!tot) return;
    SI_LAUNCH(k_q4_repack, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st, src,
              n, k / SI_QK, tile, qs, d);
}

void launch_q4_unpack(const uint8_t *qs, const uint16_t *d, int n, int k, int tile,
                      uint8_t *dst, hipStream_t st) {
    const size_t tot = (size_t)n * (k / SI_QK);
    if (!tot) return;
    SI_LAUNCH(k_q4_unpack, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st, qs,
              d, n, k / SI_QK, tile, dst);
}

// Planar Q8_0 -> operand-tiled (q8_tiled_byte): one thread per (row of
// the padded panels, block); padding rows get zeros.
__global__ void __launch_bounds__(256) k_q8_tile(const int8_t *__restrict__ qs,
                                                 const uint16_t *__restrict__ d, int m, int nb,
                                                 int8_t *__restrict__ tq, uint16_t *__restrict__ td,
                                                 int total) {
    const int t = blockIdx.x * 256 + threadIdx.x;  // row-major over (row, block)
    if (t >= total) return;
    const int r = t / nb, b = t - r * nb;
    int4 lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};  // bytes 0..15 and 16..31 of the block
    uint16_t sc = 0;
    if (r < m) {
        const int4 *src = (const int4 *)(qs + ((size_t)r * nb + b) * SI_QK);
        lo = src[0];
        hi = src[1];
        sc = d[(size_t)r * nb + b];
    }
    const size_t pb = (size_t)(r >> 5) * nb + b;
    int8_t *dst = tq + q8_tiled_byte(pb, r & 31, 0);
    *(int4 *)dst = (int4){lo.x, lo.y, hi.x, hi.y};          // half 0: bytes 0..7, 16..23
    *(int4 *)(dst + 512) = (int4){lo.z, lo.w, hi.z, hi.w};  // half 1: bytes 8..15, 24..31
    td[pb * 32 + (r & 31)] = sc;
}

void launch_q8_tile(const int8_t *qs, const uint16_t *d, int m, int k, int8_t *tq, uint16_t *td,
                    hipStream_t st) {
    const int nb = k / SI_QK, total = (m + 31) / 32 * 32 * nb;
    if (total == 0) return;
    SI_LAUNCH(k_q8_tile, dim3((total + 255) / 256), dim3(256), 0, st, qs, d, m, nb, tq, td,
              total);
}

}  // namespace si
