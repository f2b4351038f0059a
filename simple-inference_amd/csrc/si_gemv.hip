// si_gemv.hip -- decode-time Q4_0 x Q8_0 mat-vec (one activation row).
//
// Replaces matvec_q4q8 (qwen_one_layer.c:148-162) and the column-SoA
// fused_column_matvec (fused_layer.h:169-245).  The RVV design put output
// neurons on vector lanes; on CDNA4 the same idea maps to "one lane = one
// output row": with the block-major weight layout [K/32][N][16 B] a
// wavefront's 64 lanes read 64 consecutive rows of one block as a single
// 1 KiB coalesced line (16 B per lane), plus 128 B of fp16 scales.  The
// activation block is wavefront-uniform and comes through scalar loads.
//
// Per block and lane: unpack 32 nibbles with 8 AND/shift ops, 8 v_dot4
// int8 dots, subtract 8*sum(a) (the Q4_0 offset), then the reference's
// fp32 epilogue  acc = acc + ((float)dot * w.d) * x.d  with explicit
// round-to-nearest ops, so a row accumulated over all its blocks in order
// reproduces the reference bit for bit.  K may be split into ranges for
// parallelism; partial sums are then combined in range order.
//
// HBM roofline: 18 B/block/row of weights dominate (activations and
// outputs are < 1 %), so the kernel is bound by 8 TB/s.
#include "si_device.hpp"
#include "si_kernels.hpp"

namespace si {

// Integer dot of one Q4_0 block (16 nibble bytes in w) with one Q8_0 block
// (32 int8 in a), via raw nibbles 0..15 and the exact offset correction.
__device__ __forceinline__ int q4q8_block_dot(const uint4 w, const int4 alo, const int4 ahi,
                                              int asum) {
    const uint32_t m = 0x0f0f0f0fu;
    int acc = 0;
    acc = sdot4((int)(w.x & m), alo.x, acc);
    acc = sdot4((int)(w.y & m), alo.y, acc);
    acc = sdot4((int)(w.z & m), alo.z, acc);
    acc = sdot4((int)(w.w & m), alo.w, acc);
    acc = sdot4((int)((w.x >> 4) & m), ahi.x, acc);
    acc = sdot4((int)((w.y >> 4) & m), ahi.y, acc);
    acc = sdot4((int)((w.z >> 4) & m), ahi.z, acc);
    acc = sdot4((int)((w.w >> 4) & m), ahi.w, acc);
    return acc - 8 * asum;
}

// grid: x = row tiles of 64 (one wavefront, lane = row), y = K ranges.
//
// With several K ranges, each workgroup stores its 64 partial sums, then the
// last workgroup of the row tile to arrive (device-scope counter) adds the
// ranges in order and writes the row; it resets the counter, so the kernel
// leaves the counters zero for the next launch.
template <int U>
__global__ void __launch_bounds__(64) k_gemv_q4q8(
    const uint8_t *__restrict__ wqs, const uint16_t *__restrict__ wd, int n, int nb,
    const int8_t *__restrict__ xqs, const uint16_t *__restrict__ xd,
    const int16_t *__restrict__ xs, const float *__restrict__ bias,
    const float *__restrict__ residual, float *__restrict__ out, int bps,
    float *__restrict__ partial, unsigned int *__restrict__ counters) {
    const int row = blockIdx.x * 64 + threadIdx.x;
    const int split = blockIdx.y;
    const int b0 = split * bps;
    const int b1 = min(nb, b0 + bps);
    const bool live = row < n;
    const int r = live ? row : n - 1;  // dead lanes load a valid row
    float acc = (split == 0 && bias) ? bias[r] : 0.0f;

    int b = b0;
    for (; b + U <= b1; b += U) {
        uint4 w[U];
        uint16_t ws[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            w[u] = *(const uint4 *)(wqs + ((size_t)(b + u) * n + r) * 16);
            ws[u] = wd[(size_t)(b + u) * n + r];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int8_t *xb = xqs + (size_t)(b + u) * SI_QK;
            const int4 alo = *(const int4 *)xb;
            const int4 ahi = *(const int4 *)(xb + 16);
            const int dot = q4q8_block_dot(w[u], alo, ahi, xs[b + u]);
            const float t = __fmul_rn(__fmul_rn((float)dot, h2f(ws[u])), h2f(xd[b + u]));
            acc = __fadd_rn(acc, t);
        }
    }
    for (; b < b1; ++b) {
        const uint4 w = *(const uint4 *)(wqs + ((size_t)b * n + r) * 16);
        const uint16_t ws = wd[(size_t)b * n + r];
        const int8_t *xb = xqs + (size_t)b * SI_QK;
        const int dot = q4q8_block_dot(w, *(const int4 *)xb, *(const int4 *)(xb + 16), xs[b]);
        const float t = __fmul_rn(__fmul_rn((float)dot, h2f(ws)), h2f(xd[b]));
        acc = __fadd_rn(acc, t);
    }
    const int splits = gridDim.y;
    if (splits == 1) {
        if (live) out[row] = residual ? __fadd_rn(residual[row], acc) : acc;
        return;
    }
    if (live) partial[(size_t)split * n + row] = acc;
    __threadfence();  // partials visible device-wide before the arrival count
    unsigned int prev = 0;
    if (threadIdx.x == 0) prev = atomicAdd(&counters[blockIdx.x], 1u);
    prev = __shfl(prev, 0, 64);
    if (prev != (unsigned int)(splits - 1)) return;
    __threadfence();  // acquire the other workgroups' partials
    if (live) {
        float y = partial[row];
        for (int sp = 1; sp < splits; ++sp) y = __fadd_rn(y, partial[(size_t)sp * n + row]);
        out[row] = residual ? __fadd_rn(residual[row], y) : y;
    }
    if (threadIdx.x == 0) atomicExch(&counters[blockIdx.x], 0u);
}

// dots[row][b] for every (row, block): the integer core, exposed for tests.
__global__ void __launch_bounds__(64) k_block_dots(const uint8_t *__restrict__ wqs, int n, int nb,
                                                   const int8_t *__restrict__ xqs,
                                                   const int16_t *__restrict__ xs,
                                                   int32_t *__restrict__ dots) {
    const int row = blockIdx.x * 64 + threadIdx.x;
    const int b = blockIdx.y;
    if (row >= n) return;
    const uint4 w = *(const uint4 *)(wqs + ((size_t)b * n + row) * 16);
    const int8_t *xb = xqs + (size_t)b * SI_QK;
    dots[(size_t)row * nb + b] =
        q4q8_block_dot(w, *(const int4 *)xb, *(const int4 *)(xb + 16), xs[b]);
}

// Workspace: a fixed block of arrival counters first (so one workspace can
// serve mat-vecs of different shapes: partial sums never overlap counters),
// then splits * n partial sums.
constexpr size_t GEMV_COUNTERS = 4096;  // row tiles: n <= 262144

size_t gemv_workspace_bytes(int n, int k, int splits) {
    splits = gemv_effective_splits(k, splits);
    if (splits == 1) return 0;
    return GEMV_COUNTERS * sizeof(unsigned int) + (size_t)splits * n * sizeof(float);
}

void launch_gemv_q4q8(const uint8_t *wqs, const uint16_t *wd, int n, int k, const int8_t *xqs,
                      const uint16_t *xd, const int16_t *xs, const float *bias,
                      const float *residual, float *out, int splits, void *workspace,
                      hipStream_t st) {
    const int nb = k / SI_QK;
    splits = gemv_effective_splits(k, splits);
    unsigned int *counters = splits > 1 ? (unsigned int *)workspace : nullptr;
    float *partial = splits > 1 ? (float *)(counters + GEMV_COUNTERS) : nullptr;
    const int bps = (nb + splits - 1) / splits;
    const dim3 grid((n + 63) / 64, splits);
    hipLaunchKernelGGL(k_gemv_q4q8<4>, grid, dim3(64), 0, st, wqs, wd, n, nb, xqs, xd, xs, bias,
                       residual, out, bps, partial, counters);
}

int gemv_effective_splits(int k, int splits) {
    const int nb = k / SI_QK;
    if (splits < 1) splits = 1;
    if (splits > nb) splits = nb;
    const int bps = (nb + splits - 1) / splits;
    return (nb + bps - 1) / bps;
}

void launch_block_dots(const uint8_t *wqs, int n, int k, const int8_t *xqs, const int16_t *xs,
                       int32_t *dots, hipStream_t st) {
    const int nb = k / SI_QK;
    hipLaunchKernelGGL(k_block_dots, dim3((n + 63) / 64, nb), dim3(64), 0, st, wqs, n, nb, xqs,
                       xs, dots);
}

}  // namespace si
