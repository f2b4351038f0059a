// si_gemv.hip -- stand-alone Q4_0 x Q8_0 mat-vec (matvec_q4q8,
// qwen_one_layer.c:148-162) over one activation row in global memory, used
// for the decode layer's down projection and by si_matvec_q4q8; and the
// per-block int32 dot test entry (dot_32_q4q8, :118-146).
//
// HBM roofline: 18 B per (row, block) of weights dominate; the activation
// (34 B per block, read once per workgroup from L2) and the outputs are
// under 2 % of the traffic at R >= 8 rows per workgroup.
#include "si_device.hpp"
#include "si_gemv.hpp"
#include "si_kernels.hpp"

namespace si {

// out = residual + (bias + W.x); bias and residual may be null.  The
// activation row is staged in LDS once per workgroup (every thread reads
// its blocks from there).
template <int R, int T>
constexpr size_t matvec_lds_bytes(int k) {
    return (((size_t)red_floats<R, T>() * 4 + (size_t)(k / SI_QK) * 4 + 15) & ~(size_t)15) + k;
}

template <int R, int T, bool EXACT>
__global__ void __launch_bounds__(T) k_matvec(
    const int8_t *__restrict__ xqs, const uint16_t *__restrict__ xd,
    const int16_t *__restrict__ xs, int k, const uint8_t *__restrict__ wqs,
    const uint16_t *__restrict__ wd, int tile, int n, const float *__restrict__ bias,
    const float *__restrict__ residual, float *__restrict__ out, float *__restrict__ pre) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int nb = k / SI_QK;
    float *red = (float *)smem;
    uint16_t *ld = (uint16_t *)(smem + red_floats<R, T>() * 4);
    int16_t *ls = (int16_t *)(ld + nb);
    int8_t *lq = (int8_t *)(smem + ((red_floats<R, T>() * 4 + nb * 4 + 15) & ~15));  // 16 B aligned
    const int tile0 = blockIdx.x * R;
    const int t = threadIdx.x;
    // The activation row is requested first (loads retire in issue order),
    // then the weights, which stay in flight while the row goes to LDS.
    constexpr int XQ = 4, XD = 2;  // pieces per thread held in registers
    int4 xr[XQ];
    uint16_t dr[XD];
    int16_t sr[XD];
#pragma unroll
    for (int u = 0; u < XQ; ++u)  // branch-free: clamped index
        xr[u] = ((const int4 *)xqs)[min(t + u * T, k / 16 - 1)];
#pragma unroll
    for (int u = 0; u < XD; ++u) {
        dr[u] = xd[min(t + u * T, nb - 1)];
        sr[u] = xs[min(t + u * T, nb - 1)];
    }
    GemvRows<R, T, EXACT, RowIdentity> g(wqs, wd, tile, n, n, nb, tile0, RowIdentity{});
    g.start();
    // Stored at the same clamped index, unconditionally (threads past the
    // row rewrite its last piece with the value it already holds): a store
    // under a branch lets the compiler sink the load into the branch, behind
    // the weight loads, and wait for all of them.
#pragma unroll
    for (int u = 0; u < XQ; ++u) ((int4 *)lq)[min(t + u * T, k / 16 - 1)] = xr[u];
#pragma unroll
    for (int u = 0; u < XD; ++u) {
        ld[min(t + u * T, nb - 1)] = dr[u];
        ls[min(t + u * T, nb - 1)] = sr[u];
    }
    for (int i = t + XQ * T; i < k / 16; i += T) ((int4 *)lq)[i] = ((const int4 *)xqs)[i];
    for (int i = t + XD * T; i < nb; i += T) {
        ld[i] = xd[i];
        ls[i] = xs[i];
    }
    // bias and residual requested before the weights are consumed: a load
    // after the sums would wait a whole memory round trip at the end
    const int row = tile0 + (t % R);
    const float b0 = bias ? bias[min(row, n - 1)] : 0.0f;
    const float r0 = residual ? residual[min(row, n - 1)] : 0.0f;
    __syncthreads();
    const float y = g.finish(Q8Row{lq, ld, ls}, EXACT ? b0 : 0.0f, red);
    if (t < R && row < n) {
        const float v = EXACT ? y : y + b0;
        if (pre) pre[row] = v;
        out[row] = residual ? __fadd_rn(r0, v) : v;
    }
}

void launch_matvec(const int8_t *xqs, const uint16_t *xd, const int16_t *xs, int k,
                   const uint8_t *wqs, const uint16_t *wd, int tile, int n, const float *bias,
                   const float *residual, float *out, bool exact, hipStream_t st, float *pre) {
    if (n <= 0) return;
#define CALL(R, T, E)                                                                        \
    SI_LAUNCH((k_matvec<R, T, E>), dim3((n + R - 1) / R), dim3(T),                           \
              (matvec_lds_bytes<R, T>(k)), st, xqs, xd, xs, k, wqs, wd, tile, n, bias,       \
              residual, out, pre)
    if (exact) {
        CALL(64, 64, true);
    } else {
        // R = the scale tile (up to 64 rows per workgroup)
        const int r = tile < 64 ? tile : 64;
        SI_GEMV_SWITCH(r, gemv_threads(r, k / SI_QK), CALL)
    }
#undef CALL
}

__global__ void __launch_bounds__(64) k_block_dots(const uint8_t *__restrict__ wqs, int n, int nb,
                                                   const int8_t *__restrict__ xqs,
                                                   const int16_t *__restrict__ xs,
                                                   int32_t *__restrict__ dots) {
    const int row = blockIdx.x * 64 + threadIdx.x;
    const int b = blockIdx.y;
    if (row >= n) return;
    const uint4 w = *(const uint4 *)(wqs + ((size_t)b * n + row) * 16);
    const int8_t *xb = xqs + (size_t)b * SI_QK;
    dots[(size_t)row * nb + b] = dot_q4_q8(w, *(const int4 *)xb, *(const int4 *)(xb + 16), xs[b]);
}

void launch_block_dots(const uint8_t *wqs, int n, int k, const int8_t *xqs, const int16_t *xs,
                       int32_t *dots, hipStream_t st) {
    const int nb = k / SI_QK;
    SI_LAUNCH(k_block_dots, dim3((n + 63) / 64, nb), dim3(64), 0, st, wqs, n, nb, xqs,
              xs, dots);
}

}  // namespace si
