// si_mirror.hip -- kernels over the reference's own data formats, behind the
// host mirror's drop-in entry points (include/si_host.h):
//   - the row-major Q4_0 matrix and block_q8_0 records of matvec_q4q8
//     (qwen_one_layer.c:148-162);
//   - the column-SoA tiles of fused_column_matvec (fused_layer.h:169-245;
//     layout of repack_weights.py:1-20);
//   - a stand-alone rmsnorm (qwen_one_layer.c:164-169) and an in-place rope
//     (:172-183).
// Each follows the reference's summation order and roundings (separate
// multiply and add, as the reference compiles under -ffp-contract=off), so
// the projections and rotations are the reference's bits.  The timed hot
// path reads the repacked formats of si_gemv / si_gemm instead.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "si_device.hpp"
#include "si_kernels.hpp"

namespace si {

// ---------------------------------------------------------------------------
// matvec_q4q8 over row-major Q4_0 (18-byte blocks: fp16 scale, 16 nibble
// bytes) and block_q8_0 records (34 bytes: fp16 scale, 32 int8).  Both are
// 2-byte aligned at every block, so blocks are read as 16-bit words.
//
// One 64-lane workgroup per row.  Lane l forms the scaled block products
// p_b = ((float)dot_b * w.d) * x.d of blocks b = l, l + 64, ... of a chunk of
// MV_CHUNK blocks into LDS; lane 0 then adds them to the row sum in block
// order, the reference's sequence of roundings (:153-159).
// ---------------------------------------------------------------------------
constexpr int MV_CHUNK = 512;

__global__ void __launch_bounds__(64)
    k_matvec_rowmajor(const uint16_t *__restrict__ w, const uint16_t *__restrict__ x, int nblocks,
                      const float *__restrict__ bias, float *__restrict__ out) {
    __shared__ float prod[MV_CHUNK];
    const int lane = threadIdx.x, row = blockIdx.x;
    const uint16_t *wrow = w + (size_t)row * nblocks * 9;  // 9 words per block
    float sum = bias ? bias[row] : 0.0f;
    for (int c0 = 0; c0 < nblocks; c0 += MV_CHUNK) {
        const int cn = min(MV_CHUNK, nblocks - c0);
        for (int i = lane; i < cn; i += 64) {
            const int b = c0 + i;
            const uint16_t *wb = wrow + (size_t)b * 9;
            const uint16_t *xb = x + (size_t)b * 17;  // 17 words per record
            int dot = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                // nibble bytes 2j, 2j+1: elements 2j, 2j+1 (low) and
                // 2j+16, 2j+17 (high) against a[2j..2j+1], a[2j+16..2j+17]
                const uint32_t q2 = wb[1 + j];
                const uint32_t a2 = xb[1 + j], c2 = xb[9 + j];
                const int a0 = (int8_t)(a2 & 0xff), a1 = (int8_t)(a2 >> 8);
                const int c0v = (int8_t)(c2 & 0xff), c1v = (int8_t)(c2 >> 8);
                dot += ((int)(q2 & 15) - 8) * a0 + ((int)((q2 >> 4) & 15) - 8) * c0v;
                dot += ((int)((q2 >> 8) & 15) - 8) * a1 + ((int)(q2 >> 12) - 8) * c1v;
            }
            prod[i] = __fmul_rn(__fmul_rn((float)dot, h2f(wb[0])), h2f(xb[0]));
        }
        __syncthreads();
        if (lane == 0)
            for (int i = 0; i < cn; ++i) sum = __fadd_rn(sum, prod[i]);
        __syncthreads();  // prod is rewritten by the next chunk
    }
    if (lane == 0) out[row] = sum;
}

void launch_matvec_rowmajor(const uint8_t *w, const void *x, int inputs, int outputs,
                            const float *bias, float *out, hipStream_t st) {
    if (outputs <= 0) return;
    SI_LAUNCH(k_matvec_rowmajor, dim3(outputs), dim3(64), 0, st, (const uint16_t *)w,
              (const uint16_t *)x, inputs / SI_QK, bias, out);
}

// ---------------------------------------------------------------------------
// fused_column_matvec (fused_layer.h:220-244) over ntiles consecutive tiles
// of nblocks 5120-byte groups: per input block, 32 packed columns of 128
// bytes (byte j: low nibble = output j, high nibble = output j + 128) and
// 256 fp32 scales by output.  Thread j of workgroup t owns output j of tile
// t: out[t*256 + j] starts from the bias (bias_lo/bias_hi + t*256, absent =
// 0) or, with add, from its current value, then adds
// ((float)sum_b * scale_j) * x_b.d block by block.
// ---------------------------------------------------------------------------
constexpr int COLSOA_GROUP = 5120;

__global__ void __launch_bounds__(256)
    k_colsoa_matvec(const uint8_t *__restrict__ tiles, const uint16_t *__restrict__ x, int nblocks,
                    const float *__restrict__ bias_lo, const float *__restrict__ bias_hi,
                    float *__restrict__ out, int add) {
    __shared__ int xs[32];
    const int t = blockIdx.x, j = threadIdx.x;
    const bool high = j >= 128;
    const int col = j & 127;
    float y;
    if (add) y = out[(size_t)t * 256 + j];
    else {
        const float *b = high ? bias_hi : bias_lo;
        y = b ? b[(size_t)t * 256 + col] : 0.0f;
    }
    const uint8_t *tile = tiles + (size_t)t * nblocks * COLSOA_GROUP;
    for (int blk = 0; blk < nblocks; ++blk) {
        const uint16_t *xb = x + (size_t)blk * 17;
        __syncthreads();  // the previous block's values are consumed
        if (j < 16) {
            const uint32_t a2 = xb[1 + j];
            xs[2 * j] = (int8_t)(a2 & 0xff);
            xs[2 * j + 1] = (int8_t)(a2 >> 8);
        }
        __syncthreads();
        const uint8_t *group = tile + (size_t)blk * COLSOA_GROUP;
        int sum = 0;
#pragma unroll 8
        for (int k = 0; k < 32; ++k) {
            const uint32_t wv = group[k * 128 + col];
            const int nib = high ? (int)(wv >> 4) : (int)(wv & 15);
            sum += (nib - 8) * xs[k];
        }
        const float scale = ((const float *)(group + 4096))[j];
        y = __fadd_rn(y, __fmul_rn(__fmul_rn((float)sum, scale), h2f(xb[0])));
    }
    out[(size_t)t * 256 + j] = y;
}

void launch_colsoa_matvec(const uint8_t *tiles, int ntiles, const void *x, int nblocks,
                          const float *bias_lo, const float *bias_hi, float *out, int add,
                          hipStream_t st) {
    if (ntiles <= 0) return;
    SI_LAUNCH(k_colsoa_matvec, dim3(ntiles), dim3(256), 0, st, tiles,
              (const uint16_t *)x, nblocks, bias_lo, bias_hi, out, add);
}

// ---------------------------------------------------------------------------
// rmsnorm (qwen_one_layer.c:164-169) of rows of n values: the squares summed
// in binary64 (exact products; partial sums combined as a tree, so the float
// result equals the reference's except when the binary64 sum falls within a
// few ulp of a binary32 rounding boundary), inv = 1/sqrtf((float)(ss/n) +
// eps) correctly rounded, out = (x * inv) * gain.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
    k_rmsnorm(const float *__restrict__ x, const float *__restrict__ gain, int n, float eps,
              float *__restrict__ out) {
    __shared__ double red[4];
    const size_t base = (size_t)blockIdx.x * n;
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) {
        const double v = (double)x[base + i];
        ss += v * v;
    }
    ss = wave_sum_d(ss);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    const double tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn((float)(tot / (double)n), eps)));
    for (int i = threadIdx.x; i < n; i += 256)
        out[base + i] = __fmul_rn(__fmul_rn(x[base + i], inv), gain ? gain[i] : 1.0f);
}

void launch_rmsnorm(const float *x, const float *gain, int rows, int n, float eps, float *out,
                    hipStream_t st) {
    if (rows <= 0) return;
    SI_LAUNCH(k_rmsnorm, dim3(rows), dim3(256), 0, st, x, gain, n, eps, out);
}

// ---------------------------------------------------------------------------
// rope (qwen_one_layer.c:172-183) in place: pairs (i, i + hdim/2) of each of
// nheads heads rotated by the host table's angle at `position`
// (cos/sin [max_pos][hdim/2], libm values as the reference computes them).
// ---------------------------------------------------------------------------
__global__ void k_rope_inplace(float *__restrict__ heads, int nheads, int hdim, int position,
                               const float *__restrict__ rc, const float *__restrict__ rs) {
    const int half = hdim / 2;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= nheads * half) return;
    const int h = idx / half, i = idx - h * half;
    float *v = heads + (size_t)h * hdim;
    const float c = rc[(size_t)position * half + i], s = rs[(size_t)position * half + i];
    const float first = v[i], second = v[i + half];
    v[i] = __fsub_rn(__fmul_rn(first, c), __fmul_rn(second, s));
    v[i + half] = __fadd_rn(__fmul_rn(second, c), __fmul_rn(first, s));
}

void launch_rope_inplace(float *heads, int nheads, int hdim, int position, const float *rc,
                         const float *rs, hipStream_t st) {
    const int n = nheads * (hdim / 2);
    if (n <= 0) return;
    SI_LAUNCH(k_rope_inplace, dim3((n + 255) / 256), dim3(256), 0, st, heads, nheads,
              hdim, position, rc, rs);
}

// f32_to_f16 / f16_to_f32 (qwen_one_layer.c:42-86) elementwise.
// Grid-stride loops over a capped grid: any n the 64-bit size allows maps
// onto at most F16_MAX_BLOCKS workgroups (a 1-D grid is limited to 2^32
// threads).
constexpr unsigned F16_MAX_BLOCKS = 8192;
__global__ void k_f32_to_f16(const float *__restrict__ src, uint16_t *__restrict__ dst,
                             size_t n) {
    const size_t step = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step)
        dst[i] = f2h(src[i]);
}
__global__ void k_f16_to_f32(const uint16_t *__restrict__ src, float *__restrict__ dst,
                             size_t n) {
    const size_t step = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step)
        dst[i] = h2f(src[i]);
}

void launch_f16_convert(const void *src, void *dst, size_t n, bool to_half, hipStream_t st) {
    if (n == 0) return;
    const size_t blocks = (n + 255) / 256;
    const dim3 grid((unsigned)(blocks < F16_MAX_BLOCKS ? blocks : F16_MAX_BLOCKS));
    if (to_half)
        SI_LAUNCH(k_f32_to_f16, grid, dim3(256), 0, st, (const float *)src,
                  (uint16_t *)dst, n);
    else
        SI_LAUNCH(k_f16_to_f32, grid, dim3(256), 0, st, (const uint16_t *)src,
                  (float *)dst, n);
}

}  // namespace si
