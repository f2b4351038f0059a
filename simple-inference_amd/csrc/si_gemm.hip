// si_gemm.hip -- Q4_0 x Q8_0 GEMM for M > 1 activation rows (prefill,
// batched decode): matvec_q4q8 (qwen_one_layer.c:148-162) applied to every
// row, the reference's weight-stationary prefill idea (each weight tile is
// brought on chip once per batch, prefill_weight_stationary.h:1-20) realised
// as LDS tiles shared by all activation rows of a workgroup.
//
// One 32-wide K block of Q4_0 x Q8_0 is exactly one v_mfma_i32_32x32x32_i8:
// the int8 matrix core produces the per-block int32 dots exactly, then the
// fp32 epilogue applies both fp16 block scales:
//     acc[m][n] += (float)dot * (x.d[m] * w.d[n])
// The weights are staged once per tile as signed int8 (nibble - 8) so the
// matrix core needs no offset correction.
//
// MFMA operand layout (32x32x32 i8): lane l supplies 16 int8 of row l%32 for
// k-half l/32 of both A and B; output element (i, j) of a 32x32 tile lives in
// lane j + 32*((i/4)%2), register (i%4) + 4*(i/8).  Because A and B use the
// same k split, any consistent assignment of the 32 block elements to the two
// k halves gives the exact dot; Q4_0's own split (low nibbles = elements
// 0..15, high = 16..31) is used directly.
#include "si_device.hpp"
#include "si_kernels.hpp"

namespace si {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// nibbles 0..15 packed in bytes -> signed int8 (nibble - 8) per byte,
// without borrows between bytes: ((x | 0x80) - 8) ^ 0x80.
__device__ __forceinline__ uint32_t nib_to_s8(uint32_t x) {
    return ((x | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

constexpr int BM = 64;    // activation rows per workgroup
constexpr int BN = 128;   // weight rows per workgroup (4 wavefronts x 32)
constexpr int AST = 48;   // LDS row stride (bytes) of the A tile, padded
constexpr int BST = 48;   // LDS row stride (bytes) of the B tile, padded

// EXACT: the reference's rounding sequence per block, y = bias, then in block
// order y = y + ((float)dot * w.d) * x.d (qwen_one_layer.c:153-159), so each
// output equals matvec_q4q8 bit for bit.  Otherwise one fused multiply-add
// per block with the scale product x.d*w.d and the bias added at the end.
template <bool EXACT>
__global__ void __launch_bounds__(256) k_gemm_q4q8(
    const uint8_t *__restrict__ wqs, const uint16_t *__restrict__ wd, int tile, int n, int nb,
    const int8_t *__restrict__ xqs, const uint16_t *__restrict__ xd, int m,
    const float *__restrict__ bias, const float *__restrict__ residual,
    float *__restrict__ out, int ldo) {
    __shared__ __attribute__((aligned(16))) uint8_t a_lds[BM * AST];
    __shared__ __attribute__((aligned(16))) uint8_t b_lds[BN * BST];
    __shared__ float dx_lds[BM];
    __shared__ float dw_lds[BN];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int k = nb * SI_QK;

    // global -> register staging assignment
    // A: 64 rows x 32 B = 128 x 16 B (threads 0..127)
    // B: 128 rows x 16 B nibbles (threads 128..255)
    const int a_row = (tid & 127) >> 1, a_half = tid & 1;
    const int a_grow = min(m0 + a_row, m - 1);
    const int b_row = tid & 127;
    const int b_grow = min(n0 + b_row, n - 1);

    const int j = lane & 31, g = lane >> 5;
    const int col = n0 + wave * 32 + j;
    const float bias0 = (EXACT && bias) ? bias[min(col, n - 1)] : 0.0f;
    float acc[2][16];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[t][v] = bias0;

    uint4 stage;
    float sscale = 0.0f;
    auto load_block = [&](int b) {
        if (tid < 128) {
            stage = *(const uint4 *)(xqs + (size_t)a_grow * k + (size_t)b * SI_QK + a_half * 16);
            if (a_half == 0) sscale = h2f(xd[(size_t)a_grow * nb + b]);
        } else {
            stage = *(const uint4 *)(wqs + ((size_t)b * n + b_grow) * 16);
            sscale = h2f(wd[q4_scale_index(b_grow, b, nb, tile)]);
        }
    };
    auto store_block = [&]() {
        if (tid < 128) {
            *(uint4 *)(a_lds + a_row * AST + a_half * 16) = stage;
            if (a_half == 0) dx_lds[a_row] = sscale;
        } else {
            const uint32_t w[4] = {stage.x, stage.y, stage.z, stage.w};
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                lo[t] = nib_to_s8(w[t] & 0x0f0f0f0fu);
                hi[t] = nib_to_s8((w[t] >> 4) & 0x0f0f0f0fu);
            }
            *(uint4 *)(b_lds + b_row * BST) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            *(uint4 *)(b_lds + b_row * BST + 16) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            dw_lds[b_row] = sscale;
        }
    };

    load_block(0);
    for (int b = 0; b < nb; ++b) {
        __syncthreads();  // previous block's LDS reads are done
        store_block();
        __syncthreads();
        if (b + 1 < nb) load_block(b + 1);

        const v4i bop = *(const v4i *)(b_lds + (wave * 32 + j) * BST + g * 16);
        const float dwv = dw_lds[wave * 32 + j];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const v4i aop = *(const v4i *)(a_lds + (t * 32 + j) * AST + g * 16);
            v16i z = {};
            const v16i dot = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop, z, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int mi = t * 32 + 8 * (v >> 2) + 4 * g + (v & 3);
                if (EXACT)
                    acc[t][v] = __fadd_rn(acc[t][v],
                                          __fmul_rn(__fmul_rn((float)dot[v], dwv), dx_lds[mi]));
                else
                    acc[t][v] = fmaf((float)dot[v], dx_lds[mi] * dwv, acc[t][v]);
            }
        }
    }

    if (col >= n) return;
    const float bv = (!EXACT && bias) ? bias[col] : 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int row = m0 + t * 32 + 8 * (v >> 2) + 4 * g + (v & 3);
            if (row < m) {
                float y = EXACT ? acc[t][v] : acc[t][v] + bv;
                if (residual) y = __fadd_rn(residual[(size_t)row * ldo + col], y);
                out[(size_t)row * ldo + col] = y;
            }
        }
}

void launch_gemm_q4q8(const uint8_t *wqs, const uint16_t *wd, int tile, int n, int k,
                      const int8_t *xqs,
                      const uint16_t *xd, int m, const float *bias, const float *residual,
                      float *out, int ldo, bool exact, hipStream_t st) {
    if (m <= 0 || n <= 0) return;
    const dim3 grid((n + BN - 1) / BN, (m + BM - 1) / BM);
    if (exact)
        hipLaunchKernelGGL(k_gemm_q4q8<true>, grid, dim3(256), 0, st, wqs, wd, tile, n, k / SI_QK, xqs,
                           xd, m, bias, residual, out, ldo);
    else
        hipLaunchKernelGGL(k_gemm_q4q8<false>, grid, dim3(256), 0, st, wqs, wd, tile, n, k / SI_QK, xqs,
                           xd, m, bias, residual, out, ldo);
}

}  // namespace si
