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
// The weights are staged once per tile as signed int8 (nibble - 8, or
// 16*(nibble - 8) on the fast paths) so the matrix core needs no offset
// correction.
//
// MFMA operand layout (32x32x32 i8): lane l supplies 16 int8 of row l%32 for
// k-half l/32 of both A and B; output element (i, j) of a 32x32 tile lives in
// lane j + 32*((i/4)%2), register (i%4) + 4*(i/8).  Because A and B use the
// same k split, any consistent assignment of the 32 block elements to the two
// k halves gives the exact dot; Q4_0's own split (low nibbles = elements
// 0..15, high = 16..31) is used directly.
#include "si_device.hpp"
#include "si_kernels.hpp"

#include <algorithm>

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

// ===========================================================================
// Fast path (everything but SI_GEMM_EXACT).
//
// The VALU epilogue bounds this GEMM: each (m, n, 32-wide block) needs an
// int->float conversion and an FMA with the scale product dx*dw, and the
// VALU retires 16 lanes per clock per SIMD against 1024 int8 MACs for the
// matrix core.  So everything else is moved off the VALU:
//   * the scale product of a 32x32 output tile is one f16 MFMA
//     (v_mfma_f32_32x32x8_f16 with dx as the only nonzero column of A and
//     dw as the only nonzero row of B: an outer product, exact in fp32);
//   * the epilogue is then cvt + fma per output and block, the fp32 FMA
//     rounding once where the reference rounds twice;
//   * operands stream through LDS stages of G_KB blocks, the next stage's
//     global loads in flight in registers while the current one is used;
//     two blocks per stage keep the kernel under 168 VGPRs (3 waves per
//     SIMD), which hides more latency than deeper stages do;
//   * MFMA results are written to VGPRs (-amdgpu-mfma-vgpr-form), so the
//     epilogue reads them without a v_accvgpr_read per element;
//   * the weights are staged as 16*(nibble - 8), three ALU ops per nibble
//     word (see k_gemm_bd): the sums come out 16x, exactly, and are scaled
//     by 1/16 in the epilogue.
// Counters on the 7B gate|up GEMM (2048 x 37888 x 3584): the VALU is ~90%
// busy, 73% of its instructions are the cvt + fma epilogue, the matrix
// pipe ~33% (i8 and f16 MFMA 32 cycles each per 32x32 tile and block).
// Tiles: WM x WN wavefronts, each TM x TN MFMA tiles of 32x32, so the
// workgroup covers BM = 32*WM*TM rows by BN = 32*WN*TN columns.  A grid too
// small for the chip splits K over gridDim.z; the split partial sums go to
// a workspace and k_gemm_reduce adds them in split order (deterministic).
// ===========================================================================
typedef _Float16 gh4 __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));

constexpr int G_KB = 2;   // K blocks per LDS stage (deeper stages cost occupancy)
constexpr int G_ST = 48;  // LDS bytes per (row, block): 32 data + 16 padding
constexpr int F6_BYTES = 24;  // 32 six-bit codes
typedef int v8i __attribute__((ext_vector_type(8)));

template <int WM, int WN, int TM, int TN>
struct GemmCfg {
    static constexpr int BM = 32 * WM * TM, BN = 32 * WN * TN;
    static constexpr int A_PIECES = BM * G_KB * 2;  // 16-byte pieces per stage
    static constexpr int B_PIECES = BN * G_KB;      // 16-byte nibble pieces per stage
    static constexpr int A_PT = (A_PIECES + 255) / 256, B_PT = (B_PIECES + 255) / 256;
    static constexpr int SX_PT = (BM * G_KB + 255) / 256, SW_PT = (BN * G_KB + 255) / 256;
    // scales as 8-byte {fp16 bits, 0} entries: x.d [G_KB][BM]; w.d [G_KB][BN],
    // 8 entries of padding, then a zero copy of the same shape that lanes
    // 32..63 read (16 banks away from the real one)
    static constexpr int SW_TWIN = G_KB * BN + 8;
    static constexpr size_t lds_bytes() {
        return (size_t)G_KB * (BM + BN) * G_ST + (size_t)(G_KB * BM + SW_TWIN + G_KB * BN) * 8;
    }
};

// Gate|up fusion order: logical rows alternate 32 gate rows (physical
// 0..f-1) and the 32 up rows of the same features (physical f..2f-1), so a
// wavefront's two 32-column tiles hold gate and up of the same 32 features.
__device__ __forceinline__ int gate_up_row(int r, int f) {
    const int j = 32 * (r >> 6) + (r & 31);
    return (r & 32) ? f + j : j;
}

// Outputs of the fused SwiGLU + Q8_0 epilogue.
struct GateUpOut {
    int f;
    float *act;     // optional fp32 SwiGLU output [m][f]
    int8_t *qs;     // Q8_0 of the SwiGLU output, planar [m][f]
    uint16_t *d;    // [m][f/32] fp16 scale bits
    int16_t *s;     // optional [m][f/32] block sums
    int8_t *tq;     // optional: the same Q8_0 operand-tiled (q8_tiled_qs)
    uint16_t *td;   // with tq: its scales (q8_tiled_d)
};


// Register staging of one LDS stage of k_gemm_fast.  Each thread's byte
// offsets inside a stage are fixed (rows clamped once); a stage moves the
// buffer bases, scalar work, so a stage costs no per-load VALU address math.
// Blocks past the split (read, never used) stay in bounds or read as zero.
template <int BM, int BN, int A_PT, int B_PT, int SX_PT, int SW_PT>
struct GemmStage {
    v4i ra[A_PT], rb[B_PT];  // clang vectors: kept in registers
    uint16_t rsx[SX_PT], rsw[SW_PT];
    uint32_t oa[A_PT], ob[B_PT], osx[SX_PT], osw[SW_PT];

    // gu_f > 0: logical weight row r is physical row gate_up_row(r, gu_f)
    __device__ __forceinline__ void init(int tile, int n, int nb, int m, int m0, int n0,
                                         int gu_f) {
        const int tid = threadIdx.x, k = nb * SI_QK;
        constexpr int A_PIECES = BM * G_KB * 2, B_PIECES = BN * G_KB;
#pragma unroll
        for (int i = 0; i < A_PT; ++i) {
            const int p = min(tid + 256 * i, A_PIECES - 1);
            const int row = p / (G_KB * 2), blk = (p >> 1) % G_KB, half = p & 1;
            oa[i] = (uint32_t)(min(m0 + row, m - 1) * k + blk * SI_QK + half * 16);
        }
#pragma unroll
        for (int i = 0; i < B_PT; ++i) {
            const int p = min(tid + 256 * i, B_PIECES - 1);
            const int row = p / G_KB, blk = p % G_KB;
            const int lr = min(n0 + row, n - 1);
            ob[i] = (uint32_t)((blk * n + (gu_f ? gate_up_row(lr, gu_f) : lr)) * 16);
        }
#pragma unroll
        for (int i = 0; i < SX_PT; ++i) {
            const int p = min(tid + 256 * i, BM * G_KB - 1);
            const int row = p / G_KB, blk = p % G_KB;
            osx[i] = (uint32_t)((min(m0 + row, m - 1) * nb + blk) * 2);
        }
#pragma unroll
        for (int i = 0; i < SW_PT; ++i) {
            const int p = min(tid + 256 * i, BN * G_KB - 1);
            const int row = p / G_KB, blk = p % G_KB;
            const int lr = min(n0 + row, n - 1);
            osw[i] = (uint32_t)(q4_scale_index(gu_f ? gate_up_row(lr, gu_f) : lr, blk, nb, tile) * 2);
        }
    }

    // stage starting at block bs (< nb)
    __device__ __forceinline__ void load(const uint8_t *__restrict__ wqs,
                                         const uint16_t *__restrict__ wd, int tile, int n, int nb,
                                         const int8_t *__restrict__ xqs,
                                         const uint16_t *__restrict__ xd, int m, int bs) {
        const uint32_t k = (uint32_t)nb * SI_QK;
        const __amdgpu_buffer_rsrc_t ra_s = buf_rsrc(xqs + (size_t)bs * SI_QK,
                                                     (uint32_t)m * k - (uint32_t)bs * SI_QK);
        const __amdgpu_buffer_rsrc_t rb_s = buf_rsrc(wqs + (size_t)bs * n * 16,
                                                     (uint32_t)(nb - bs) * (uint32_t)n * 16);
        const __amdgpu_buffer_rsrc_t rx_s = buf_rsrc(xd + bs, ((uint32_t)m * nb - bs) * 2);
        const uint32_t wcount = (uint32_t)q4_scale_count(n, nb, tile);
        const __amdgpu_buffer_rsrc_t rw_s = buf_rsrc(wd + (size_t)bs * tile,
                                                     (wcount - (uint32_t)bs * tile) * 2);
#pragma unroll
        for (int i = 0; i < A_PT; ++i) ra[i] = __builtin_amdgcn_raw_buffer_load_b128(ra_s, oa[i], 0, 0);
#pragma unroll
        for (int i = 0; i < B_PT; ++i) rb[i] = __builtin_amdgcn_raw_buffer_load_b128(rb_s, ob[i], 0, 0);
#pragma unroll
        for (int i = 0; i < SX_PT; ++i) rsx[i] = __builtin_amdgcn_raw_buffer_load_b16(rx_s, osx[i], 0, 0);
#pragma unroll
        for (int i = 0; i < SW_PT; ++i) rsw[i] = __builtin_amdgcn_raw_buffer_load_b16(rw_s, osw[i], 0, 0);
    }

    __device__ __forceinline__ void store(uint8_t *a_l, uint8_t *b_l, v2u *sx_l, v2u *sw_l,
                                          int buf) const {
        const int tid = threadIdx.x;
        constexpr int A_PIECES = BM * G_KB * 2, B_PIECES = BN * G_KB;
#pragma unroll
        for (int i = 0; i < A_PT; ++i) {
            const int p = tid + 256 * i;
            if (A_PIECES % 256 == 0 || p < A_PIECES) {
                const int row = p / (G_KB * 2), blk = (p >> 1) % G_KB, half = p & 1;
                *(v4i *)(a_l + (((size_t)buf * G_KB + blk) * BM + row) * G_ST + half * 16) = ra[i];
            }
        }
#pragma unroll
        for (int i = 0; i < B_PT; ++i) {
            const int p = tid + 256 * i;
            if (B_PIECES % 256 == 0 || p < B_PIECES) {
                const int row = p / G_KB, blk = p % G_KB;
                const uint32_t w[4] = {(uint32_t)rb[i][0], (uint32_t)rb[i][1], (uint32_t)rb[i][2],
                                       (uint32_t)rb[i][3]};
                // 16*(nibble - 8) as int8: (n ^ 8) in the byte's top nibble
                // (the dots come out 16x, exactly; k_gemm_fast rescales)
                uint32_t lo[4], hi[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    lo[t] = ((w[t] << 4) ^ 0x80808080u) & 0xf0f0f0f0u;
                    hi[t] = (w[t] ^ 0x80808080u) & 0xf0f0f0f0u;
                }
                uint8_t *dst = b_l + (((size_t)buf * G_KB + blk) * BN + row) * G_ST;
                *(uint4 *)dst = make_uint4(lo[0], lo[1], lo[2], lo[3]);
                *(uint4 *)(dst + 16) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            }
        }
#pragma unroll
        for (int i = 0; i < SX_PT; ++i) {
            const int p = tid + 256 * i;
            if ((BM * G_KB) % 256 == 0 || p < BM * G_KB) {
                const int row = p / G_KB, blk = p % G_KB;
                sx_l[((size_t)buf * G_KB + blk) * BM + row] = (v2u){(unsigned)rsx[i], 0u};
            }
        }
#pragma unroll
        for (int i = 0; i < SW_PT; ++i) {
            const int p = tid + 256 * i;
            if ((BN * G_KB) % 256 == 0 || p < BN * G_KB) {
                const int row = p / G_KB, blk = p % G_KB;
                sw_l[((size_t)buf * G_KB + blk) * BN + row] = (v2u){(unsigned)rsw[i], 0u};
            }
        }
    }
};

// FUSE: the weights are a gate|up pair (n = 2f, the physical rows gate then
// up), read in gate_up_row order; the epilogue writes the gate|up outputs in
// physical order to out (optional) and SwiGLU + Q8_0 (k_swiglu_q8's rules)
// to go.  Needs TN == 2 and one K split.
// Epilogue of the fast-path tile kernels for a wavefront's TM x TN tiles of
// 32 x 32 sums acc, each scaled by os on the way out (exact: a power of two).
// FUSE: gate|up SwiGLU + Q8_0 through the wavefront's 32 x GEMM_EPI_FT floats
// at tl_base (free LDS, after the last barrier); otherwise bias + residual into
// out, or the K split's partials into part.
constexpr int GEMM_EPI_FT = 36;  // floats per LDS row of the transposition (16-byte aligned)
template <int WM, int WN, int TM, int TN, bool FUSE>
__device__ __forceinline__ void gemm_tile_epilogue(
    const float (&acc)[TM][TN][16], float os, float *tl_base, int m, int n, int m0, int n0,
    const float *__restrict__ bias, const float *__restrict__ residual, float *__restrict__ out,
    int ldo, float *__restrict__ part, const GateUpOut &go) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int j = lane & 31, g = lane >> 5;
    // output (i, j) of a 32x32 tile: lane j + 32*((i/4)%2), register (i%4) + 4*(i/8)
    if (FUSE) {
        const int f = go.f;
        const int fb = (n0 + wn * 64) / 2;  // the wavefront's 32 features: one Q8 block
        const bool fok = fb < f;            // the block is all in or all out
        // SwiGLU exactly as k_swiglu_q8 per output; then each row's block is
        // read back row-wise from this wavefront's LDS area, lanes l and
        // l ^ 32 holding features 0..15 and 16..31 of row l & 31, and
        // quantized with the same rules (quant_block_pair16): one scale
        // division per block instead of one per output, no half-wave
        // reductions per register, 16-byte stores
        constexpr int FT = GEMM_EPI_FT;
        float *tl = tl_base + wave * (32 * FT);
        const int rr = lane & 31, hh = lane >> 5;
#pragma unroll
        for (int a = 0; a < TM; ++a) {
            const int r0 = m0 + (wm * TM + a) * 32;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int i = 8 * (v >> 2) + 4 * g + (v & 3);
                const float gv = acc[a][0][v] * os, uv = acc[a][TN - 1][v] * os;
                const float silu = __fdiv_rn(gv, __fadd_rn(1.0f, expf(-gv)));
                tl[i * FT + j] = __fmul_rn(silu, uv);
                if (out && r0 + i < m && fok) {
                    out[(size_t)(r0 + i) * ldo + fb + j] = gv;
                    out[(size_t)(r0 + i) * ldo + f + fb + j] = uv;
                }
            }
            // the wavefront's own area: its LDS accesses complete in order
            __builtin_amdgcn_wave_barrier();
            float x[16];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float4 p = *(const float4 *)(tl + rr * FT + 16 * hh + 4 * t);
                x[4 * t] = p.x;
                x[4 * t + 1] = p.y;
                x[4 * t + 2] = p.z;
                x[4 * t + 3] = p.w;
            }
            __builtin_amdgcn_wave_barrier();  // the next tile rewrites the area
            int q[16];
            uint16_t dbits;
            int bsum;
            quant_block_pair16(x, q, dbits, bsum);
            const int row = r0 + rr;
            if (row < m && fok) {
                const size_t o = (size_t)row * f + fb + 16 * hh;
                if (go.act)
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        *(float4 *)(go.act + o + 4 * t) =
                            make_float4(x[4 * t], x[4 * t + 1], x[4 * t + 2], x[4 * t + 3]);
                uint32_t pk[4];
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    pk[t] = (uint32_t)(q[4 * t] & 0xff) | (uint32_t)(q[4 * t + 1] & 0xff) << 8 |
                            (uint32_t)(q[4 * t + 2] & 0xff) << 16 | (uint32_t)q[4 * t + 3] << 24;
                *(uint4 *)(go.qs + o) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
                if (hh == 0) {
                    go.d[o / SI_QK] = dbits;
                    if (go.s) go.s[o / SI_QK] = (int16_t)bsum;
                }
                if (go.tq) {
                    // bytes 16hh..16hh+7 and +8..+15 of the row's block: the
                    // first 8 of halves 0 and 1 at position 8hh
                    const size_t pb = (size_t)(row >> 5) * (f / SI_QK) + fb / SI_QK;
                    int8_t *tb = go.tq + q8_tiled_byte(pb, row & 31, 16 * hh);
                    *(uint2 *)tb = make_uint2(pk[0], pk[1]);
                    *(uint2 *)(tb + 512) = make_uint2(pk[2], pk[3]);
                    if (hh == 0) go.td[pb * 32 + (row & 31)] = dbits;
                }
            }
        }
        return;
    }
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int col = n0 + (wn * TN + b) * 32 + j;
            if (col >= n) continue;
            const float bv = (part == nullptr && bias) ? bias[col] : 0.0f;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = m0 + (wm * TM + a) * 32 + 8 * (v >> 2) + 4 * g + (v & 3);
                if (row >= m) continue;
                if (part) {
                    part[((size_t)blockIdx.z * m + row) * n + col] = acc[a][b][v] * os;
                } else {
                    float y = acc[a][b][v] * os + bv;
                    if (residual) y = __fadd_rn(residual[(size_t)row * ldo + col], y);
                    out[(size_t)row * ldo + col] = y;
                }
            }
        }
}

template <int WM, int WN, int TM, int TN, bool FUSE>
__global__ void __launch_bounds__(256) k_gemm_fast(
    const uint8_t *__restrict__ wqs, const uint16_t *__restrict__ wd, int tile, int n, int nb,
    const int8_t *__restrict__ xqs, const uint16_t *__restrict__ xd, int m,
    const float *__restrict__ bias, const float *__restrict__ residual, float *__restrict__ out,
    int ldo, float *__restrict__ part, int bps, GateUpOut go) {
    static_assert(!FUSE || TN == 2, "gate|up fusion pairs two column tiles per wavefront");
    using C = GemmCfg<WM, WN, TM, TN>;
    constexpr int BM = C::BM, BN = C::BN;
    extern __shared__ __attribute__((aligned(16))) uint8_t gsm[];
    uint8_t *a_l = gsm;                                   // [G_KB][BM][G_ST]
    uint8_t *b_l = a_l + G_KB * BM * G_ST;                // [G_KB][BN][G_ST]
    // fp16 scale bits zero-extended to 64 bits: an LDS read is then a
    // ready f16x4 MFMA operand {scale, 0, 0, 0}
    v2u *sx_l = (v2u *)(b_l + G_KB * BN * G_ST);  // [G_KB][BM]
    v2u *sw_l = sx_l + G_KB * BM;                 // [G_KB][BN], pad, zero copy

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int j = lane & 31, g = lane >> 5;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int b_begin = blockIdx.z * bps, b_end = min(nb, b_begin + bps);

#pragma unroll
    for (int i = 0; i < (G_KB * BN + 255) / 256; ++i)  // the zero copy (before the first barrier)
        if ((G_KB * BN) % 256 == 0 || tid + 256 * i < G_KB * BN)
            sw_l[C::SW_TWIN + tid + 256 * i] = (v2u){0u, 0u};
    GemmStage<BM, BN, C::A_PT, C::B_PT, C::SX_PT, C::SW_PT> stg;
    float acc[TM][TN][16];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;

    const int nstage = (b_end - b_begin + G_KB - 1) / G_KB;
    stg.init(tile, n, nb, m, m0, n0, FUSE ? go.f : 0);
    stg.load(wqs, wd, tile, n, nb, xqs, xd, m, b_begin);
    // One LDS stage: the next stage's global loads are in flight in registers
    // while this one is consumed; the trailing barrier frees the LDS.
    for (int st = 0; st < nstage; ++st) {
        const int buf = 0;
        stg.store(a_l, b_l, sx_l, sw_l, buf);
        __syncthreads();
        const int bs = b_begin + st * G_KB;
        // next stage in flight (branch-free: the last iteration re-reads
        // its own stage and never stores it)
        stg.load(wqs, wd, tile, n, nb, xqs, xd, m, min(bs + G_KB, b_begin + (nstage - 1) * G_KB));
#pragma unroll
        for (int blk = 0; blk < G_KB; ++blk) {
            if (bs + blk >= b_end) break;
            const uint8_t *ab = a_l + ((size_t)buf * G_KB + blk) * BM * G_ST;
            const uint8_t *bb = b_l + ((size_t)buf * G_KB + blk) * BN * G_ST;
            const v2u *sxb = sx_l + ((size_t)buf * G_KB + blk) * BM;
            const v2u *swb = sw_l + ((size_t)buf * G_KB + blk) * BN;
            v4i aop[TM], bop[TN];
            gh4 asc[TM], bsc[TN];
            // scale-product operands: A carries x.d at k = 0 (lanes 0..31)
            // and k = 4 (lanes 32..63), B carries w.d at k = 0 and, from the
            // zero copy, 0 at k = 4, so the product is x.d[row] * w.d[col]
            // with no per-lane select
            const v2u *swl = swb + g * C::SW_TWIN;
#pragma unroll
            for (int a = 0; a < TM; ++a) {
                const int r = (wm * TM + a) * 32 + j;
                aop[a] = *(const v4i *)(ab + r * G_ST + g * 16);
                asc[a] = __builtin_bit_cast(gh4, sxb[r]);
            }
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                const int c = (wn * TN + b) * 32 + j;
                bop[b] = *(const v4i *)(bb + c * G_ST + g * 16);
                bsc[b] = __builtin_bit_cast(gh4, swl[c]);
            }
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TN; ++b) {
                    v16i z = {};
                    const v16i dot = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop[a], bop[b], z, 0, 0, 0);
                    v16f zf = {};
                    const v16f sc = __builtin_amdgcn_mfma_f32_32x32x8f16(asc[a], bsc[b], zf, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[a][b][v] = fmaf((float)dot[v], sc[v], acc[a][b][v]);
                }
        }
        __syncthreads();  // the stage's LDS is rewritten next
    }

    static_assert(4 * 32 * GEMM_EPI_FT * 4 <= C::lds_bytes(), "the transposition fits the stage LDS");
    gemm_tile_epilogue<WM, WN, TM, TN, FUSE>(acc, 0.0625f, (float *)gsm, m, n, m0, n0, bias,
                                             residual, out, ldo, part, go);
}

// ===========================================================================
// Fast path, fp6 formulation (k_gemm_f6): the same sums as k_gemm_fast bit for
// bit, with one VALU operation per output and block instead of two.
//
// The weights are w6 + d6 [nb][n] (launch_q4_to_w6: fp6 e2m3 codes of
// (nibble - 8) / 2, logical row order, gate|up included) and each Q8
// activation x6 (launch_q8_to_x6: q = 16 hi + lo, hi = q >> 4 in -8..7,
// lo = q & 15, codes of hi / 2 and lo / 2).  A row's 32 codes are 24 bytes,
// kept as a 16-byte and an 8-byte part: a region of R rows (w6: one block,
// n rows; x6: one block's hi or lo codes, m rows) is [R][16] then [R][8],
// w6 [nb] regions, x6 [nb][2].  One
// v_mfma_scale_f32_32x32x64_f8f6f4 takes a block's 32 hi codes in k 0..31
// (lanes 0..31, block scale 2^5) and its 32 lo codes in k 32..63 (lanes
// 32..63, scale 2^1) against the weight codes twice (scale 2^1): every
// product is an integer of magnitude <= 1016 and every partial sum (<= 32512)
// is exact in fp32, so the block dot arrives exactly, as a float, and the
// epilogue is k_gemm_fast's fma without the conversion; the nibble unpack is
// gone too.  The matrix instruction issues at the i8 one's rate (~36 cycles
// per 32 x 32 x 64, measured on MI355X).
//
// Staging: a stage (G_KB blocks) is copied global -> LDS by buffer loads
// that write LDS directly (no staging registers), into two static buffers
// used in turn; the copy of stage s + 1 is issued right after the barrier
// that opens stage s and waited for (vmcnt(0)) before the next barrier, so it
// overlaps a whole stage of matrix work, with one barrier per stage.  The
// grid runs M tiles fastest (workgroups sharing a weight tile run together).
// One lane's operand: 32 six-bit codes, bytes 0..15 at p16 (16-byte aligned)
// and 16..23 at p8; the instruction reads six registers.
__device__ __forceinline__ v8i f6_operand(const uint8_t *p16, const uint8_t *p8) {
    const uint4 a = *(const uint4 *)p16;
    const uint2 b = *(const uint2 *)p8;
    return (v8i){(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, 0, 0};
}

typedef __attribute__((address_space(3))) void lds_void;

// One wavefront copy global -> LDS: lane l's 16 bytes at voff of r land at
// lds + 16 l; a 2-byte copy lands zero-extended in the dword at lds + 4 l
// (measured on MI355X); lds wavefront-uniform.
__device__ __forceinline__ void lds_copy16(__amdgpu_buffer_rsrc_t r, uint8_t *lds, uint32_t voff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 16, voff, 0, 0, 0);
}
__device__ __forceinline__ void lds_copy2(__amdgpu_buffer_rsrc_t r, uint8_t *lds, uint32_t voff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 2, voff, 0, 0, 0);
}

// this wavefront's copies into LDS complete, its LDS writes too, then the
// workgroup barrier (no memory fence: the fence of __syncthreads would also
// wait for the next stage's copies already in flight)
__device__ __forceinline__ void f6_stage_sync() {
    __builtin_amdgcn_s_waitcnt(0x3070);  // vmcnt(0) lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int WM, int WN, int TM, int TN, bool FUSE>
__global__ void __launch_bounds__(256, 3) k_gemm_f6(
    const uint8_t *__restrict__ w6, const uint16_t *__restrict__ d6, int n, int nb,
    const uint8_t *__restrict__ x6, const uint16_t *__restrict__ xd, int m,
    const float *__restrict__ bias, const float *__restrict__ residual, float *__restrict__ out,
    int ldo, float *__restrict__ part, int bps, GateUpOut go) {
    static_assert(!FUSE || TN == 2, "gate|up fusion pairs two column tiles per wavefront");
    static_assert(WM * WN == 4, "four wavefronts");
    using C = GemmCfg<WM, WN, TM, TN>;
    constexpr int BM = C::BM, BN = C::BN;
    // a stage buffer: activations [G_KB][2] regions of BM rows, weights
    // [G_KB] regions of BN rows (each [rows][16] then [rows][8]), scales x.d
    // [G_KB][BM] and w.d [G_KB][BN] (fp16 bits zero-extended to a dword: the
    // low register of the scale-product operand)
    constexpr int A_BYTES = G_KB * 2 * BM * F6_BYTES, B_BYTES = G_KB * BN * F6_BYTES;
    constexpr int SX_OFF = A_BYTES + B_BYTES, SW_OFF = SX_OFF + G_KB * BM * 4;
    constexpr int STAGE = SW_OFF + G_KB * BN * 4;
    // wavefront copy instructions per stage: 64 lanes x 16 bytes (operands),
    // 64 lanes x 2 bytes into dwords (scales); instruction q goes to
    // wavefront q % 4
    constexpr int AR = BM * F6_BYTES / 16, BR = BN * F6_BYTES / 16;  // 16-byte pieces per region
    constexpr int A_WI = G_KB * 2 * AR / 64, B_WI = G_KB * BR / 64;
    constexpr int SX_WI = G_KB * BM / 64, SW_WI = G_KB * BN / 64;
    static_assert(G_KB * 2 * AR % 64 == 0 && G_KB * BR % 64 == 0, "whole copy instructions");
    constexpr int A_PW = (A_WI + 3) / 4, B_PW = (B_WI + 3) / 4;
    constexpr int SX_PW = (SX_WI + 3) / 4, SW_PW = (SW_WI + 3) / 4;
    // sb0 also holds the gate|up epilogue's transposition
    constexpr int EPI = 4 * 32 * GEMM_EPI_FT * 4;
    __shared__ __attribute__((aligned(16))) uint8_t sb0[STAGE > EPI ? STAGE : EPI];
    __shared__ __attribute__((aligned(16))) uint8_t sb1[STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int j = lane & 31, g = lane >> 5;
    const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
    const int b_begin = blockIdx.z * bps, b_end = min(nb, b_begin + bps);
    const int f6_sa = g ? 128 : 132;  // hi codes 2^5 (16 x the codes' 2^1), lo 2^1

    // stage-relative source offsets of this lane's copies
    uint32_t oa[A_PW], ob[B_PW], osx[SX_PW], osw[SW_PW];
    // piece q of a region's stage slice: rows' 16-byte parts (q < rows),
    // then their 8-byte parts, in LDS at 16 q either way
#pragma unroll
    for (int i = 0; i < A_PW; ++i) {
        const int p = (4 * i + wave) * 64 + lane, reg = p / AR, q = p % AR;
        oa[i] = (uint32_t)(reg * m * F6_BYTES +
                           (q < BM ? m0 * 16 + q * 16 : m * 16 + m0 * 8 + (q - BM) * 16));
    }
#pragma unroll
    for (int i = 0; i < B_PW; ++i) {
        const int p = (4 * i + wave) * 64 + lane, blk = p / BR, q = p % BR;
        ob[i] = (uint32_t)(blk * n * F6_BYTES +
                           (q < BN ? n0 * 16 + q * 16 : n * 16 + n0 * 8 + (q - BN) * 16));
    }
#pragma unroll
    for (int i = 0; i < SX_PW; ++i) {
        const int e = (4 * i + wave) * 64 + lane, blk = e / BM, row = e % BM;
        osx[i] = (uint32_t)((min(m0 + row, m - 1) * nb + blk) * 2);
    }
#pragma unroll
    for (int i = 0; i < SW_PW; ++i) {
        const int e = (4 * i + wave) * 64 + lane, blk = e / BN, c = e % BN;
        osw[i] = (uint32_t)((blk * n + min(n0 + c, n - 1)) * 2);
    }
    // copy the stage starting at block bs into buf: past row m or n a piece
    // reads the next region or, past the array, zero (buffer bounds); such
    // rows and columns reach only outputs that are never stored
    const int wu = __builtin_amdgcn_readfirstlane(wave);  // scalar copy addresses
    const auto issue = [&](uint8_t *buf, int bs) {
        const uint32_t left = (uint32_t)(nb - bs);
        const __amdgpu_buffer_rsrc_t ra_s =
            buf_rsrc(x6 + (size_t)bs * 2 * m * F6_BYTES, left * 2 * (uint32_t)m * F6_BYTES);
        const __amdgpu_buffer_rsrc_t rb_s =
            buf_rsrc(w6 + (size_t)bs * n * F6_BYTES, left * (uint32_t)n * F6_BYTES);
        const __amdgpu_buffer_rsrc_t rx_s = buf_rsrc(xd + bs, ((uint32_t)m * nb - bs) * 2);
        const __amdgpu_buffer_rsrc_t rw_s = buf_rsrc(d6 + (size_t)bs * n, left * (uint32_t)n * 2);
#pragma unroll
        for (int i = 0; i < A_PW; ++i)
            if (A_WI % 4 == 0 || 4 * i + wu < A_WI)
                lds_copy16(ra_s, buf + 1024 * (4 * i + wu), oa[i]);
#pragma unroll
        for (int i = 0; i < B_PW; ++i)
            if (B_WI % 4 == 0 || 4 * i + wu < B_WI)
                lds_copy16(rb_s, buf + A_BYTES + 1024 * (4 * i + wu), ob[i]);
#pragma unroll
        for (int i = 0; i < SX_PW; ++i)
            if (SX_WI % 4 == 0 || 4 * i + wu < SX_WI)
                lds_copy2(rx_s, buf + SX_OFF + 256 * (4 * i + wu), osx[i]);
#pragma unroll
        for (int i = 0; i < SW_PW; ++i)
            if (SW_WI % 4 == 0 || 4 * i + wu < SW_WI)
                lds_copy2(rw_s, buf + SW_OFF + 256 * (4 * i + wu), osw[i]);
    };

    float acc[TM][TN][16];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;

    // per-lane LDS offsets inside a stage buffer (each access is then the
    // buffer's static address + a constant + one of these): the lane's hi
    // (lanes 0..31) or lo (32..63) activation row, weight row, scales
    const int ra = wm * TM * 32 + j, rb = wn * TN * 32 + j;
    const int a16 = g * BM * F6_BYTES + ra * 16, a8 = g * BM * F6_BYTES + BM * 16 + ra * 8;
    const int b16 = A_BYTES + rb * 16, b8 = A_BYTES + BN * 16 + rb * 8;
    const int sx_off = SX_OFF + ra * 4, sw_off = SW_OFF + rb * 4;
    const auto compute = [&](const uint8_t *buf, int bs) {
#pragma unroll
        for (int blk = 0; blk < G_KB; ++blk) {
            if (bs + blk >= b_end) break;
            // scale-product operands {x.d, 0, 0, 0} and {w.d, 0, 0, 0}: x.d at
            // k = 0 and 4, w.d at k = 0 only (lanes 32..63 take zero)
            v8i aop[TM], bop[TN];
            gh4 asc[TM], bsc[TN];
#pragma unroll
            for (int a = 0; a < TM; ++a) {
                aop[a] = f6_operand(buf + a16 + blk * 2 * BM * F6_BYTES + a * 32 * 16,
                                    buf + a8 + blk * 2 * BM * F6_BYTES + a * 32 * 8);
                // keeps each operand's two reads its own (merged reads of two
                // tiles' 8-byte parts cost register copies)
                __builtin_amdgcn_sched_barrier(0);
                const unsigned xs = *(const uint32_t *)(buf + sx_off + (blk * BM + a * 32) * 4);
                asc[a] = __builtin_bit_cast(gh4, (v2u){xs, 0u});
            }
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                bop[b] = f6_operand(buf + b16 + blk * BN * F6_BYTES + b * 32 * 16,
                                    buf + b8 + blk * BN * F6_BYTES + b * 32 * 8);
                __builtin_amdgcn_sched_barrier(0);
                const unsigned ws = *(const uint32_t *)(buf + sw_off + (blk * BN + b * 32) * 4);
                bsc[b] = __builtin_bit_cast(gh4, (v2u){g ? 0u : ws, 0u});
            }
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TN; ++b) {
                    v16f zf = {};
                    const v16f dot = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        aop[a], bop[b], zf, 2, 2, 0, f6_sa, 0, 128);
                    const v16f sc = __builtin_amdgcn_mfma_f32_32x32x8f16(asc[a], bsc[b], zf, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[a][b][v] = fmaf(dot[v], sc[v], acc[a][b][v]);
                }
        }
    };

    // the two buffers in turn, unrolled so each access names its buffer
    const int nstage = (b_end - b_begin + G_KB - 1) / G_KB;
    if (nstage > 0) issue(sb0, b_begin);
    for (int st = 0; st < nstage; st += 2) {
        f6_stage_sync();  // stage st in sb0; everyone is done with sb1
        if (st + 1 < nstage) issue(sb1, b_begin + (st + 1) * G_KB);
        compute(sb0, b_begin + st * G_KB);
        if (st + 1 >= nstage) break;
        f6_stage_sync();  // stage st + 1 in sb1; everyone is done with sb0
        if (st + 2 < nstage) issue(sb0, b_begin + (st + 2) * G_KB);
        compute(sb1, b_begin + (st + 1) * G_KB);
    }
    __syncthreads();  // no copy in flight; every wavefront is done reading
    gemm_tile_epilogue<WM, WN, TM, TN, FUSE>(acc, 1.0f, (float *)sb0, m, n, m0, n0, bias,
                                             residual, out, ldo, part, go);
}

// ===========================================================================
// Fast path, f16 formulation (k_gemm_h16): the same products as k_gemm_fast
// with one VALU operation per (row, column, block) instead of two.
//
// A Q8_0 value (-127..127) and a Q4_0 value (nibble - 8, -8..7) are exact
// fp16 numbers, their products (|p| <= 1016) exact in fp32 and every partial
// sum of a 32-wide block (|s| <= 32512 < 2^24) too, so two
// v_mfma_f32_32x32x16_f16 over the block's 32 values give the block's
// int32 dot exactly, already in fp32: the epilogue is the one fma by the
// scale product (itself one f16 MFMA, as in k_gemm_fast), no conversion.
// The results equal k_gemm_fast's bit for bit (same blocks in the same
// order through the same fma; k_gemm_fast's 16x operands scale every term
// by a power of two, which commutes with rounding).
//
// The operands are converted once per LDS stage, by all threads of the
// workgroup while the stage is written to LDS, so each converted value
// serves a whole tile of outputs:
//   int8 b -> fp16: the byte b ^ 0x80 = b + 128 as the low byte of the half
//     0x64xx is 1024 + b + 128 (one v_perm_b32 per pair), minus 1152 (one
//     v_pk_add_f16 per pair), exact;
//   nibble n -> fp16 n - 8: 0x6400 | n is 1024 + n, minus 1032, likewise.
// LDS rows hold a block's 32 halves in element order, 80 bytes apart; two
// stage buffers, the next stage converted and written while this one is
// consumed, one barrier per stage.
// Measured on the 7B gate|up GEMM (2048 x 37888 x 3584), bit-identical to
// k_gemm_fast: 951-965 us for 128 x 256 workgroup tiles (8 wavefronts of
// 2 x 2 MFMA tiles; 1121-1410 us for the other tilings tried) against
// 745-822 us for k_gemm_fast.  Counters: the conversions are gone but the
// operand conversion adds about as many VALU instructions back (42 per
// thread per stage at 128 x 128), the matrix pipe works 1.5x the cycles
// (two f16 MFMAs per block instead of one i8), LDS traffic doubles, and
// neither pipe passes ~60 % busy (waits on LDS and barriers), so the
// default path keeps the int8 formulation; SI_GEMM_F16 selects this one.
// ===========================================================================
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));

constexpr int H_KB = 2;   // K blocks per LDS stage
constexpr int H_ST = 80;  // LDS bytes per (row, block): 32 halves + 16 bytes of padding

// four int8 (one dword) -> four fp16, element order (two dwords)
__device__ __forceinline__ void s8x4_to_h(uint32_t x, uint32_t &p0, uint32_t &p1) {
    const uint32_t u = x ^ 0x80808080u;
    const h2v bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    p0 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v, __builtin_amdgcn_perm(
                                                                0x64646464u, u, 0x04010400u)) +
                                          bias);
    p1 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v, __builtin_amdgcn_perm(
                                                                0x64646464u, u, 0x04030402u)) +
                                          bias);
}
// four nibbles, one per byte (bits 0..3) -> four fp16 (nibble - 8)
__device__ __forceinline__ void n4x4_to_h(uint32_t x, uint32_t &p0, uint32_t &p1) {
    const h2v bias = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    p0 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v, __builtin_amdgcn_perm(
                                                                0x64646464u, x, 0x04010400u)) +
                                          bias);
    p1 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v, __builtin_amdgcn_perm(
                                                                0x64646464u, x, 0x04030402u)) +
                                          bias);
}

template <int WM, int WN, int TM, int TN>
struct H16Cfg {
    static constexpr int NT = 64 * WM * WN;  // threads
    static constexpr int BM = 32 * WM * TM, BN = 32 * WN * TN;
    static constexpr int A_PIECES = BM * H_KB * 2;  // 16 int8 per piece
    static constexpr int B_PIECES = BN * H_KB;      // 32 nibbles per piece
    static constexpr int A_PT = (A_PIECES + NT - 1) / NT, B_PT = (B_PIECES + NT - 1) / NT;
    static constexpr int SX_PT = (BM * H_KB + NT - 1) / NT, SW_PT = (BN * H_KB + NT - 1) / NT;
    static constexpr int SW_TWIN = H_KB * BN + 8;  // as GemmCfg: w.d, padding, a zero copy
    // one stage buffer: operands, then scales
    static constexpr size_t buf_bytes() {
        return (size_t)H_KB * (BM + BN) * H_ST + (size_t)(H_KB * BM + SW_TWIN + H_KB * BN) * 8;
    }
    // two stage buffers: the next stage is written while this one is used
    static constexpr size_t lds_bytes() { return 2 * buf_bytes(); }
};

// Register staging of one stage (GemmStage's scheme for NT threads), the
// operands converted to fp16 on their way into LDS.
template <typename C>
struct H16Stage {
    v4i ra[C::A_PT], rb[C::B_PT];
    uint16_t rsx[C::SX_PT], rsw[C::SW_PT];
    uint32_t oa[C::A_PT], ob[C::B_PT], osx[C::SX_PT], osw[C::SW_PT];

    __device__ __forceinline__ void init(int tile, int n, int nb, int m, int m0, int n0,
                                         int gu_f) {
        const int tid = threadIdx.x, k = nb * SI_QK;
#pragma unroll
        for (int i = 0; i < C::A_PT; ++i) {
            const int p = min(tid + C::NT * i, C::A_PIECES - 1);
            const int row = p / (H_KB * 2), blk = (p >> 1) % H_KB, half = p & 1;
            oa[i] = (uint32_t)(min(m0 + row, m - 1) * k + blk * SI_QK + half * 16);
        }
#pragma unroll
        for (int i = 0; i < C::B_PT; ++i) {
            const int p = min(tid + C::NT * i, C::B_PIECES - 1);
            const int row = p / H_KB, blk = p % H_KB;
            const int lr = min(n0 + row, n - 1);
            ob[i] = (uint32_t)((blk * n + (gu_f ? gate_up_row(lr, gu_f) : lr)) * 16);
        }
#pragma unroll
        for (int i = 0; i < C::SX_PT; ++i) {
            const int p = min(tid + C::NT * i, C::BM * H_KB - 1);
            const int row = p / H_KB, blk = p % H_KB;
            osx[i] = (uint32_t)((min(m0 + row, m - 1) * nb + blk) * 2);
        }
#pragma unroll
        for (int i = 0; i < C::SW_PT; ++i) {
            const int p = min(tid + C::NT * i, C::BN * H_KB - 1);
            const int row = p / H_KB, blk = p % H_KB;
            const int lr = min(n0 + row, n - 1);
            osw[i] = (uint32_t)(q4_scale_index(gu_f ? gate_up_row(lr, gu_f) : lr, blk, nb, tile) *
                                2);
        }
    }

    __device__ __forceinline__ void load(const uint8_t *__restrict__ wqs,
                                         const uint16_t *__restrict__ wd, int tile, int n, int nb,
                                         const int8_t *__restrict__ xqs,
                                         const uint16_t *__restrict__ xd, int m, int bs) {
        const uint32_t k = (uint32_t)nb * SI_QK;
        const __amdgpu_buffer_rsrc_t ra_s = buf_rsrc(xqs + (size_t)bs * SI_QK,
                                                     (uint32_t)m * k - (uint32_t)bs * SI_QK);
        const __amdgpu_buffer_rsrc_t rb_s = buf_rsrc(wqs + (size_t)bs * n * 16,
                                                     (uint32_t)(nb - bs) * (uint32_t)n * 16);
        const __amdgpu_buffer_rsrc_t rx_s = buf_rsrc(xd + bs, ((uint32_t)m * nb - bs) * 2);
        const uint32_t wcount = (uint32_t)q4_scale_count(n, nb, tile);
        const __amdgpu_buffer_rsrc_t rw_s = buf_rsrc(wd + (size_t)bs * tile,
                                                     (wcount - (uint32_t)bs * tile) * 2);
#pragma unroll
        for (int i = 0; i < C::A_PT; ++i)
            ra[i] = __builtin_amdgcn_raw_buffer_load_b128(ra_s, oa[i], 0, 0);
#pragma unroll
        for (int i = 0; i < C::B_PT; ++i)
            rb[i] = __builtin_amdgcn_raw_buffer_load_b128(rb_s, ob[i], 0, 0);
#pragma unroll
        for (int i = 0; i < C::SX_PT; ++i)
            rsx[i] = __builtin_amdgcn_raw_buffer_load_b16(rx_s, osx[i], 0, 0);
#pragma unroll
        for (int i = 0; i < C::SW_PT; ++i)
            rsw[i] = __builtin_amdgcn_raw_buffer_load_b16(rw_s, osw[i], 0, 0);
    }

    __device__ __forceinline__ void store(uint8_t *a_l, uint8_t *b_l, v2u *sx_l,
                                          v2u *sw_l) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < C::A_PT; ++i) {
            const int p = tid + C::NT * i;
            if (C::A_PIECES % C::NT == 0 || p < C::A_PIECES) {
                const int row = p / (H_KB * 2), blk = (p >> 1) % H_KB, half = p & 1;
                uint32_t h[8];
#pragma unroll
                for (int t = 0; t < 4; ++t) s8x4_to_h((uint32_t)ra[i][t], h[2 * t], h[2 * t + 1]);
                uint8_t *dst = a_l + ((size_t)blk * C::BM + row) * H_ST + half * 32;
                *(uint4 *)dst = make_uint4(h[0], h[1], h[2], h[3]);
                *(uint4 *)(dst + 16) = make_uint4(h[4], h[5], h[6], h[7]);
            }
        }
#pragma unroll
        for (int i = 0; i < C::B_PT; ++i) {
            const int p = tid + C::NT * i;
            if (C::B_PIECES % C::NT == 0 || p < C::B_PIECES) {
                const int row = p / H_KB, blk = p % H_KB;
                // byte t holds element t (low nibble) and t + 16 (high)
                uint32_t lo[8], hi[8];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint32_t w = (uint32_t)rb[i][t];
                    n4x4_to_h(w & 0x0f0f0f0fu, lo[2 * t], lo[2 * t + 1]);
                    n4x4_to_h((w >> 4) & 0x0f0f0f0fu, hi[2 * t], hi[2 * t + 1]);
                }
                uint8_t *dst = b_l + ((size_t)blk * C::BN + row) * H_ST;
                *(uint4 *)dst = make_uint4(lo[0], lo[1], lo[2], lo[3]);
                *(uint4 *)(dst + 16) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
                *(uint4 *)(dst + 32) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
                *(uint4 *)(dst + 48) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
            }
        }
#pragma unroll
        for (int i = 0; i < C::SX_PT; ++i) {
            const int p = tid + C::NT * i;
            if ((C::BM * H_KB) % C::NT == 0 || p < C::BM * H_KB) {
                const int row = p / H_KB, blk = p % H_KB;
                sx_l[(size_t)blk * C::BM + row] = (v2u){(unsigned)rsx[i], 0u};
            }
        }
#pragma unroll
        for (int i = 0; i < C::SW_PT; ++i) {
            const int p = tid + C::NT * i;
            if ((C::BN * H_KB) % C::NT == 0 || p < C::BN * H_KB) {
                const int row = p / H_KB, blk = p % H_KB;
                sw_l[(size_t)blk * C::BN + row] = (v2u){(unsigned)rsw[i], 0u};
            }
        }
    }
};

// Same interface and epilogues as k_gemm_fast (FUSE: gate|up SwiGLU + Q8).
template <int WM, int WN, int TM, int TN, bool FUSE>
__global__ void __launch_bounds__(64 * WM * WN) k_gemm_h16(
    const uint8_t *__restrict__ wqs, const uint16_t *__restrict__ wd, int tile, int n, int nb,
    const int8_t *__restrict__ xqs, const uint16_t *__restrict__ xd, int m,
    const float *__restrict__ bias, const float *__restrict__ residual, float *__restrict__ out,
    int ldo, float *__restrict__ part, int bps, GateUpOut go) {
    static_assert(!FUSE || TN == 2, "gate|up fusion pairs two column tiles per wavefront");
    using C = H16Cfg<WM, WN, TM, TN>;
    constexpr int BM = C::BM, BN = C::BN, NT = C::NT;
    extern __shared__ __attribute__((aligned(16))) uint8_t hsm[];
    // stage buffer q (0, 1): operands [H_KB][BM][H_ST], [H_KB][BN][H_ST],
    // scales [H_KB][BM], [H_KB][BN], pad, zero copy
    auto a_of = [&](int q) { return hsm + (size_t)q * C::buf_bytes(); };
    auto b_of = [&](int q) { return a_of(q) + H_KB * BM * H_ST; };
    auto sx_of = [&](int q) { return (v2u *)(b_of(q) + H_KB * BN * H_ST); };
    auto sw_of = [&](int q) { return sx_of(q) + H_KB * BM; };

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int j = lane & 31, g = lane >> 5;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int b_begin = blockIdx.z * bps, b_end = min(nb, b_begin + bps);

#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int i = 0; i < (H_KB * BN + NT - 1) / NT; ++i)  // the zero copies
            if ((H_KB * BN) % NT == 0 || tid + NT * i < H_KB * BN)
                sw_of(q)[C::SW_TWIN + tid + NT * i] = (v2u){0u, 0u};
    H16Stage<C> stg;
    float acc[TM][TN][16];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;

    const int nstage = (b_end - b_begin + H_KB - 1) / H_KB;
    const int last = b_begin + (nstage - 1) * H_KB;  // first block of the last stage
    stg.init(tile, n, nb, m, m0, n0, FUSE ? go.f : 0);
    stg.load(wqs, wd, tile, n, nb, xqs, xd, m, b_begin);
    stg.store(a_of(0), b_of(0), sx_of(0), sw_of(0));
    __syncthreads();
    // stage st+1 in registers, then written to the other buffer while stage
    // st is consumed; one barrier per stage (branch-free loads: past the
    // last stage the last one is re-read and never stored)
    stg.load(wqs, wd, tile, n, nb, xqs, xd, m, min(b_begin + H_KB, last));
    for (int st = 0; st < nstage; ++st) {
        const int cur = st & 1;
        if (st + 1 < nstage) {
            stg.store(a_of(cur ^ 1), b_of(cur ^ 1), sx_of(cur ^ 1), sw_of(cur ^ 1));
            stg.load(wqs, wd, tile, n, nb, xqs, xd, m, min(b_begin + (st + 2) * H_KB, last));
        }
        const int bs = b_begin + st * H_KB;
#pragma unroll
        for (int blk = 0; blk < H_KB; ++blk) {
            if (bs + blk >= b_end) break;
            const uint8_t *ab = a_of(cur) + (size_t)blk * BM * H_ST;
            const uint8_t *bb = b_of(cur) + (size_t)blk * BN * H_ST;
            const v2u *sxb = sx_of(cur) + (size_t)blk * BM;
            const v2u *swl = sw_of(cur) + (size_t)blk * BN + g * C::SW_TWIN;
            h8v aop[TM][2], bop[TN][2];
            gh4 asc[TM], bsc[TN];
            // lane (j, g) of MFMA step s supplies elements 16 s + 8 g .. +7
            // of row (A) / column (B) j, in both operands
#pragma unroll
            for (int a = 0; a < TM; ++a) {
                const int r = (wm * TM + a) * 32 + j;
#pragma unroll
                for (int s = 0; s < 2; ++s)
                    aop[a][s] = *(const h8v *)(ab + r * H_ST + 32 * s + 16 * g);
                asc[a] = __builtin_bit_cast(gh4, sxb[r]);
            }
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                const int c = (wn * TN + b) * 32 + j;
#pragma unroll
                for (int s = 0; s < 2; ++s)
                    bop[b][s] = *(const h8v *)(bb + c * H_ST + 32 * s + 16 * g);
                bsc[b] = __builtin_bit_cast(gh4, swl[c]);
            }
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TN; ++b) {
                    v16f dot = {};
                    dot = __builtin_amdgcn_mfma_f32_32x32x16_f16(aop[a][0], bop[b][0], dot, 0, 0, 0);
                    dot = __builtin_amdgcn_mfma_f32_32x32x16_f16(aop[a][1], bop[b][1], dot, 0, 0, 0);
                    v16f zf = {};
                    const v16f sc = __builtin_amdgcn_mfma_f32_32x32x8f16(asc[a], bsc[b], zf, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[a][b][v] = fmaf(dot[v], sc[v], acc[a][b][v]);
                }
        }
        // the stage written above is complete, and this one's reads are
        // done before it is rewritten two stages on
        __syncthreads();
    }

    // output (i, j) of a 32x32 tile: lane j + 32*((i/4)%2), register (i%4) + 4*(i/8)
    if (FUSE) {
        const int f = go.f;
        const int fb = (n0 + wn * 64) / 2;  // the wavefront's 32 features: one Q8 block
        const bool fok = fb < f;
        constexpr int FT = 36;  // floats per LDS row (16-byte aligned rows)
        static_assert((size_t)(NT / 64) * 32 * FT * 4 <= C::lds_bytes(),
                      "the transposition fits the stage LDS");
        float *tl = (float *)hsm + wave * (32 * FT);  // after the last barrier: free
        const int rr = lane & 31, hh = lane >> 5;
#pragma unroll
        for (int a = 0; a < TM; ++a) {
            const int r0 = m0 + (wm * TM + a) * 32;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int i = 8 * (v >> 2) + 4 * g + (v & 3);
                const float gv = acc[a][0][v], uv = acc[a][TN - 1][v];
                const float silu = __fdiv_rn(gv, __fadd_rn(1.0f, expf(-gv)));
                tl[i * FT + j] = __fmul_rn(silu, uv);
                if (out && r0 + i < m && fok) {
                    out[(size_t)(r0 + i) * ldo + fb + j] = gv;
                    out[(size_t)(r0 + i) * ldo + f + fb + j] = uv;
                }
            }
            __builtin_amdgcn_wave_barrier();
            float x[16];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float4 p = *(const float4 *)(tl + rr * FT + 16 * hh + 4 * t);
                x[4 * t] = p.x;
                x[4 * t + 1] = p.y;
                x[4 * t + 2] = p.z;
                x[4 * t + 3] = p.w;
            }
            __builtin_amdgcn_wave_barrier();
            int q[16];
            uint16_t dbits;
            int bsum;
            quant_block_pair16(x, q, dbits, bsum);
            const int row = r0 + rr;
            if (row < m && fok) {
                const size_t o = (size_t)row * f + fb + 16 * hh;
                if (go.act)
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        *(float4 *)(go.act + o + 4 * t) =
                            make_float4(x[4 * t], x[4 * t + 1], x[4 * t + 2], x[4 * t + 3]);
                uint32_t pk[4];
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    pk[t] = (uint32_t)(q[4 * t] & 0xff) | (uint32_t)(q[4 * t + 1] & 0xff) << 8 |
                            (uint32_t)(q[4 * t + 2] & 0xff) << 16 | (uint32_t)q[4 * t + 3] << 24;
                *(uint4 *)(go.qs + o) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
                if (hh == 0) {
                    go.d[o / SI_QK] = dbits;
                    if (go.s) go.s[o / SI_QK] = (int16_t)bsum;
                }
                if (go.tq) {
                    // bytes 16hh..16hh+7 and +8..+15 of the row's block: the
                    // first 8 of halves 0 and 1 at position 8hh
                    const size_t pb = (size_t)(row >> 5) * (f / SI_QK) + fb / SI_QK;
                    int8_t *tb = go.tq + q8_tiled_byte(pb, row & 31, 16 * hh);
                    *(uint2 *)tb = make_uint2(pk[0], pk[1]);
                    *(uint2 *)(tb + 512) = make_uint2(pk[2], pk[3]);
                    if (hh == 0) go.td[pb * 32 + (row & 31)] = dbits;
                }
            }
        }
        return;
    }
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int col = n0 + (wn * TN + b) * 32 + j;
            if (col >= n) continue;
            const float bv = (part == nullptr && bias) ? bias[col] : 0.0f;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = m0 + (wm * TM + a) * 32 + 8 * (v >> 2) + 4 * g + (v & 3);
                if (row >= m) continue;
                if (part) {
                    part[((size_t)blockIdx.z * m + row) * n + col] = acc[a][b][v];
                } else {
                    float y = acc[a][b][v] + bv;
                    if (residual) y = __fadd_rn(residual[(size_t)row * ldo + col], y);
                    out[(size_t)row * ldo + col] = y;
                }
            }
        }
}

// ---------------------------------------------------------------------
// Batched-decode GEMM (m <= 64 activation rows; also the short-K one-tile
// projections of prefill up to 512 rows, bd_takes).
//
// At this size each output costs two VALU operations per K block (the
// exact int32 dot converted, then one fused multiply-add by the fp32 scale
// product) against a fraction of one matrix-core instruction, so the
// kernel is built to keep the vector ALUs issuing:
//   * a workgroup holds 32 activation rows of one K range (at most
//     BD_MAX_CB blocks) in LDS for its whole life, filled once with
//     coalesced loads, in MFMA operand order;
//   * its W wavefronts (8, 12 or 16: 2-4 per SIMD) share that range block by
//     block (wavefront w takes blocks w, w + W, ...) and stream their
//     weights straight into registers P blocks ahead, with no barrier in
//     the K loop, over a persistent walk of the workgroup's column tiles:
//     the prefetch runs on across tiles;
//   * at the end of a tile the partial sums meet in LDS and are added in a
//     fixed order (deterministic); wavefront w < 8 finishes output
//     registers 2w and 2w + 1 of the 16 of every lane.
// The 32-row halves of a set of tiles run on the same XCD (blockIdx % 8),
// so the later halves' weight reads hit that XCD's L2.  Longer K is
// split into ranges whose partials [c][m][n] are summed afterwards, as
// k_gemm_fast's are.
//
// Operands: lane (j, g) of the 32x32x32 i8 MFMA supplies half g of a block
// as elements 8g..8g+7 and 16+8g..16+8g+7 (A and B agree, so the MFMA gives
// the block's exact integer dot): for Q4_0 these are both nibbles of bytes
// 8g..8g+7, one 8-byte load.  Nibble n becomes the int8 16*(n - 8): n ^ 8
// is the 4-bit two's complement of n - 8, so in a byte's top nibble it
// reads as 16*(n - 8).  The dots come out 16x, exactly (|16 dot| < 2^20),
// and fma(16 dot, s, 16 acc) is 16 times fma(dot, s, acc) bit for bit (a
// power-of-two scale commutes with rounding), so the sums are scaled by
// 1/16, exactly, once at the end.
//
// LDS: block b of the activations is 1 KB, [half g][slot][16 B], row i in
// slot i ^ 2(b & 3): a fill instruction's 8 rows x 4 blocks then spread
// over the banks, and the 32 lanes of a half read one 512-byte run.
//
// MODE 0 (TN = 1): out = residual + (acc + bias) (both optional), or the
// partials.  MODE 1 (TN = 2, gate|up, one K range): tile u pairs the gate
// rows 32u..32u+31 with the up rows f+32u..; SwiGLU + Q8_0 epilogue as
// k_gemm_fast's, optionally also written operand-tiled.
//
// DA (one K range of any length): the activations arrive
// operand-tiled (q8_tiled_qs / q8_tiled_d): a block of a 32-row panel is one
// contiguous 1 KB run in exactly the order the MFMA lanes take it, so each
// stage loads its block's activations with one 16-byte load per lane next to
// its weights, and there is no fill, no LDS copy of the rows and no K-range
// limit (one pass, no partials).  Read from the planar layout the same loads
// would touch 32 cache lines each (one per row); through the LDS fill they
// cost a serial phase per workgroup and, for long K, the K split.
//
// PIPE (one tile): block i's two matrix-core products are issued before
// block i-1's epilogue runs, which consumes the products issued one step
// earlier (two register sets by the parity of the unrolled step), so each
// wavefront has its products in flight while it converts and accumulates;
// the blocks are still accumulated in the same order (same bits).
constexpr int BD_RED = 8 * 16 * 64 * 4;                    // 8 partial 32x32 fp32 tiles
constexpr int BD_LDS_MAX = 160 * 1024;                     // LDS of a gfx950 CU
// x.d row stride in halves for a K range of cb blocks: an odd number of
// dwords, so the 32 rows' values of one block sit in 32 different banks
__host__ __device__ constexpr int bd_xst(int cb) { return 2 * (((cb + 1) >> 1) | 1); }
// LDS of a K range of cb blocks: Q8 rows (a multiple of 4 blocks), x.d
// rows, partial tiles
__host__ __device__ constexpr size_t bd_lds(int cb) {
    return (size_t)((cb + 3) & ~3) * 1024 + 64 * (size_t)bd_xst(cb) + BD_RED;
}
constexpr int BD_MAX_CB = 120;
static_assert(bd_lds(BD_MAX_CB) <= BD_LDS_MAX, "a K range fits a CU's LDS");

typedef unsigned gv2u __attribute__((vector_size(8)));  // an 8-byte buffer load's value
typedef int v2i __attribute__((ext_vector_type(2)));

template <int TN>
struct BdStage {
    gv2u w[TN];       // nibble bytes 8g..8g+7 of weight row j of tile u
    uint16_t ws[TN];  // w.d fp16 bits (lanes 32..63: 0); widened where used, so
                      // that nothing waits for the load before then
    v4i a;            // streamed activations: this lane's 16 operand bytes
    uint16_t xs;      // streamed activations: x.d of row j
};

// A workgroup barrier ordering LDS only: __syncthreads() also orders global
// memory, which waits for every global load in flight (here the weight
// prefetch); the partial sums and the fill need the LDS half alone.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Workgroup id -> (row half h, K range c, slot s) with the halves of one
// (c, s) on one XCD; q >= C * S: no work.
__device__ __forceinline__ void bd_place(int id, int H, int S, int &h, int &q, int &c, int &s) {
    const int x = id & 7, r = id >> 3;
    h = r % H;
    q = (r / H) * 8 + x;
    c = q / S;
    s = q - c * S;
}

template <int TN, int P, int MODE, int BD_W, bool DA, bool PIPE = false>
__global__ void __launch_bounds__(64 * BD_W) k_gemm_bd(
    const uint8_t *__restrict__ wqs, const uint16_t *__restrict__ wd, int tile, int n, int nb,
    const int8_t *__restrict__ xqs, const uint16_t *__restrict__ xd, int m,
    const float *__restrict__ bias, const float *__restrict__ residual, float *__restrict__ out,
    int ldo, float *__restrict__ part, int H, int C, int S, int cb, int units, GateUpOut go,
    RopeOut ro) {
    static_assert(MODE == 1 ? TN == 2 : TN == 1, "MODE 0 and 2 take one tile, gate|up two");
    static_assert(BD_W >= 8 && BD_W <= 16 && BD_W % 4 == 0, "8, 12 or 16 wavefronts");
    static_assert(!PIPE || (TN == 1 && P % 2 == 0), "pipelined: one tile, an even unroll");
    constexpr int BD_T = 64 * BD_W;                              // threads
    constexpr int BD_FILL = (BD_MAX_CB * 64 + BD_T - 1) / BD_T;  // 16-byte fill pieces per thread
    constexpr int BD_XFILL = (32 * 128 + BD_T - 1) / BD_T;       // x.d fill values per thread
    extern __shared__ __attribute__((aligned(16))) uint8_t bd_sm[];
    const int tid = threadIdx.x, lane = tid & 63;
    // the wavefront index as a scalar: block numbers derived from it are
    // the buffer loads' scalar offsets
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 31, g = lane >> 5;
    int h, q, c, s;
    bd_place(blockIdx.x, H, S, h, q, c, s);
    if (q >= C * S) return;  // the whole workgroup
    const int m0 = 32 * h, b0 = c * cb, len = min(nb, b0 + cb) - b0;
    const int k = nb * SI_QK;
    const int cb4 = DA ? 0 : (cb + 3) & ~3;
    uint8_t *a_l = bd_sm;  // [cb4][2][32][16 B]
    const int xst = bd_xst(cb);  // x.d row stride (halves)
    uint16_t *x_l = (uint16_t *)(bd_sm + (size_t)cb4 * 1024);  // [32][xst]
    // [8][16][64] floats (streamed activations: the only LDS)
    float4 *red = (float4 *)(DA ? bd_sm : bd_sm + bd_lds(cb) - BD_RED);

    // ---- the tiles of this workgroup: units s, s + S, ...
    const int per = (len + BD_W - 1) / BD_W;  // blocks per wavefront per tile (some may be past len)
    const int nu = s < units ? (units - 1 - s) / S + 1 : 0;
    const int total = nu * per;
    if (total <= 0) return;  // no tile here: the whole workgroup
    const int ltile = __builtin_ctz((unsigned)tile);
    const __amdgpu_buffer_rsrc_t rb = buf_rsrc(wqs, (uint32_t)nb * n * 16);
    // streamed activations: panel h's block b at (h nb + b) KB; lane (j, g)
    // reads 16 bytes at g * 512 + j * 16 of it, its x.d at (h nb + b) * 64 + 2 j
    const __amdgpu_buffer_rsrc_t rta = buf_rsrc(xqs, DA ? (uint32_t)H * nb * 1024 : 0u);
    const __amdgpu_buffer_rsrc_t rtx = buf_rsrc(xd, DA ? (uint32_t)H * nb * 64 : 0u);
    const uint32_t vta = (uint32_t)h * nb * 1024 + g * 512 + j * 16;
    const uint32_t vtx = ((uint32_t)h * nb * 32 + j) * 2;
    const __amdgpu_buffer_rsrc_t rw =
        buf_rsrc(wd, __builtin_amdgcn_readfirstlane((int)q4_scale_count(n, nb, tile) * 2));
    // first column of tile u of unit iu (scalar)
    auto col0 = [&](int iu, int u) {
        const int unit = s + S * iu;
        return MODE == 1 ? (u ? go.f : 0) + 32 * unit : 32 * unit;
    };
    // the load pointer: (unit lu, step lk), its lanes' byte offsets
    int lu = 0, lk = 0, lu_set = -1;
    uint32_t vob[TN], vow[TN];
    auto set_unit = [&](int iu) {
#pragma unroll
        for (int u = 0; u < TN; ++u) {
            const int cc = min(col0(iu, u) + j, n - 1);  // past n: any valid row
            vob[u] = (uint32_t)cc * 16 + 8 * g;
            vow[u] = g ? 0x80000000u
                       : (uint32_t)(((cc >> ltile) * nb << ltile) + (cc & (tile - 1))) * 2;
        }
    };
    // Streamed activations (one K range, b0 = 0, len = nb): the scalar
    // offsets of block b = BD_W lk + wave advance by a constant per step.
    // They are not clamped: a block past nb reads as zero (past the buffer)
    // or as another panel's block, and only steps whose block is in range
    // use their loads (the pipelined step gives the others zero scales).
    uint32_t oa = 0, ox = 0, ow = 0, os = 0;
    auto da_reset = [&]() {
        const uint32_t b = (uint32_t)(b0 + wave);
        oa = b * 1024;
        ox = b * 64;
        ow = b * (uint32_t)n * 16;
        os = (b << ltile) * 2;
    };
    if (DA) da_reset();
    auto load = [&](BdStage<TN> &st) {
        const int iu = min(lu, nu - 1);  // past the end: a valid block again
        if (iu != lu_set) {
            set_unit(iu);
            lu_set = iu;
        }
        if constexpr (DA) {
            st.a = __builtin_amdgcn_raw_buffer_load_b128(rta, vta, oa, 0);
            st.xs = __builtin_amdgcn_raw_buffer_load_b16(rtx, vtx, ox, 0);
#pragma unroll
            for (int u = 0; u < TN; ++u) {
                st.w[u] = __builtin_amdgcn_raw_buffer_load_b64(rb, vob[u], ow, 0);
                st.ws[u] = __builtin_amdgcn_raw_buffer_load_b16(rw, vow[u], os, 0);
            }
            oa += BD_W * 1024;
            ox += BD_W * 64;
            ow += (uint32_t)BD_W * n * 16;
            os += (uint32_t)(BD_W << ltile) * 2;
        } else {
            const int b = b0 + min(BD_W * lk + wave, len - 1);
#pragma unroll
            for (int u = 0; u < TN; ++u) {
                st.w[u] = __builtin_amdgcn_raw_buffer_load_b64(rb, vob[u], b * n * 16, 0);
                st.ws[u] = __builtin_amdgcn_raw_buffer_load_b16(rw, vow[u], (b << ltile) * 2, 0);
            }
        }
        if (++lk == per) {
            lk = 0;
            ++lu;
            if (DA) da_reset();
        }
    };

    // bias and residual of up to two tiles are read before the K loop: a
    // load in the epilogue would wait for every weight load in flight
    float pb[2] = {0.0f, 0.0f}, pr[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
    const bool pre = MODE == 0 && nu <= 2 && (bias || residual) && wave < 8;
    if (pre) {
#pragma unroll
        for (int iu = 0; iu < 2; ++iu) {
            if (iu >= nu) break;
            const int col = min(col0(iu, 0) + j, n - 1);
            if (bias) pb[iu] = bias[col];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int row = min(m0 + 8 * (wave >> 1) + 4 * g + 2 * (wave & 1) + i, m - 1);
                if (residual) pr[iu][i] = residual[(size_t)row * ldo + col];
            }
        }
    }

    // ---- fill: the K range's 32 rows (clamped to m - 1) and their x.d.
    // Loads retire in issue order: the fill's loads go first, then the
    // first P blocks of weights, and the fill waits for its own loads only,
    // while the weights stream in behind them.  (Streamed activations: no
    // fill.)
    v4i fv[DA ? 1 : BD_FILL];
    uint32_t xv[DA ? 1 : BD_XFILL];
    if constexpr (!DA) {
    const __amdgpu_buffer_rsrc_t ra = buf_rsrc(xqs, (uint32_t)m * k);
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(xd, (uint32_t)m * nb * 2);
    // Q8: 8 threads read a row's 128 bytes (4 blocks), 8 rows per 64
    // threads; a wavefront's pieces are 4 whole blocks, so whether they are
    // stored is decided per wavefront (pieces past len read zero)
#pragma unroll
    for (int i = 0; i < BD_FILL; ++i) {
        const int p = tid + BD_T * i, t8 = p & 7, ri = (p >> 3) & 31;
        const int b = 4 * (p >> 8) + (t8 >> 1);
        const int row = min(m0 + ri, m - 1);
        const uint32_t off = b < len ? (uint32_t)row * k + (uint32_t)(b0 + b) * SI_QK + (t8 & 1) * 16
                                     : 0x80000000u;  // past the end: zero, no access
        fv[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0);
    }
    // x.d: 128 threads per row, consecutive blocks
#pragma unroll
    for (int i = 0; i < BD_XFILL; ++i) {
        const int e = tid + BD_T * i, ri = e >> 7, b = e & 127;
        const int row = min(m0 + ri, m - 1);
        const uint32_t off = b < len && ri < 32 ? ((uint32_t)row * nb + b0 + b) * 2 : 0x80000000u;
        xv[i] = __builtin_amdgcn_raw_buffer_load_b16(rx, off, 0, 0);
    }
    }
    __builtin_amdgcn_sched_barrier(0);
    // P blocks of weights in flight; each stage's loads stay together and
    // in stage order (scheduling barriers), and every load is issued (a
    // valid block past the end): the wait before a block then counts the
    // same later loads on every path into it
    BdStage<TN> st[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        load(st[i]);
        __builtin_amdgcn_sched_barrier(0);
    }
    // everything but the weight stages complete (lgkmcnt and expcnt free)
    if constexpr (!DA) {
    {
        constexpr int VM = P * 2 * TN;  // weight loads issued after the fill
        static_assert(VM <= 63, "vmcnt holds 6 bits");
        __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (15 << 8));
    }
#pragma unroll
    for (int i = 0; i < BD_FILL; ++i) {
        const int p4 = (tid >> 8) + (BD_T >> 8) * i;  // the wavefront's group of 4 blocks
        if (4 * p4 < len) {
            const int p = tid + BD_T * i, t8 = p & 7, ri = (p >> 3) & 31;
            const int b = 4 * p4 + (t8 >> 1);
            // 16 bytes = elements 16*part .. +15: bytes 0..7 go to half 0,
            // bytes 8..15 to half 1, at offset 8*part of the row's slot
            uint8_t *d = a_l + ((size_t)b * 64 + (ri ^ ((b & 3) << 1))) * 16 + (t8 & 1) * 8;
            *(v2i *)d = (v2i){fv[i][0], fv[i][1]};
            *(v2i *)(d + 512) = (v2i){fv[i][2], fv[i][3]};
        }
    }
#pragma unroll
    for (int i = 0; i < BD_XFILL; ++i) {
        const int e = tid + BD_T * i;
        if ((e & 127) < len && e < 32 * 128) x_l[(e >> 7) * xst + (e & 127)] = (uint16_t)xv[i];
    }
    lds_barrier();
    }

    float acc[TN][16];
#pragma unroll
    for (int u = 0; u < TN; ++u)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[u][v] = 0.0f;
    const uint32_t la = (uint32_t)(g * 32 + (j ^ ((wave & 3) << 1))) * 16;  // this wave's slots
    // the activation operands of a step, read one step ahead of their use
    v4i a_nx;
    uint16_t x_nx;
    auto fetch = [&](int ck) {
        if constexpr (!DA) {
            const int rel = min(BD_W * ck + wave, len - 1);
            a_nx = *(const v4i *)(a_l + (size_t)rel * 1024 + la);
            x_nx = x_l[j * xst + rel];
        }
    };
    auto compute = [&](const BdStage<TN> &st, const v4i &aop, uint16_t xs) {
        // scale product x.d * w.d in the output layout: A carries x.d at
        // k = 0 and k = 4, B carries w.d at k = 0 only.  Streamed
        // activations: every tile's products are issued before the first
        // epilogue, so one tile's conversions run while the next tile's
        // products are in flight (the staged kernel, with 4 stages of
        // weights in registers, would spill the extra products).
        const gh4 asc = __builtin_bit_cast(gh4, (v2u){(uint32_t)xs, 0u});
        // ((n ^ 8) << 4) per nibble: one shift and one three-input bitwise op
        // for the low nibbles, one op for the high ones
        auto bop_of = [&](int u) {
            const uint32_t w0 = st.w[u][0], w1 = st.w[u][1];
            return (v4i){(int)(((w0 << 4) ^ 0x80808080u) & 0xf0f0f0f0u),
                         (int)(((w1 << 4) ^ 0x80808080u) & 0xf0f0f0f0u),
                         (int)((w0 ^ 0x80808080u) & 0xf0f0f0f0u),
                         (int)((w1 ^ 0x80808080u) & 0xf0f0f0f0u)};
        };
        auto bsc_of = [&](int u) {
            return __builtin_bit_cast(gh4, (v2u){(uint32_t)st.ws[u], 0u});
        };
        if constexpr (DA) {
            v16i dot[TN];
            v16f sc[TN];
#pragma unroll
            for (int u = 0; u < TN; ++u) {
                v16i z = {};
                dot[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop_of(u), z, 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < TN; ++u) {
                v16f zf = {};
                sc[u] = __builtin_amdgcn_mfma_f32_32x32x8f16(asc, bsc_of(u), zf, 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < TN; ++u) {
                __builtin_amdgcn_sched_barrier(0);  // the epilogues in issue order
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    acc[u][v] = fmaf((float)dot[u][v], sc[u][v], acc[u][v]);
            }
        } else {
#pragma unroll
            for (int u = 0; u < TN; ++u) {
                v16i z = {};
                const v16i dot = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop_of(u), z, 0, 0, 0);
                v16f zf = {};
                const v16f sc = __builtin_amdgcn_mfma_f32_32x32x8f16(asc, bsc_of(u), zf, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[u][v] = fmaf((float)dot[v], sc[v], acc[u][v]);
            }
        }
    };
    // PIPE: the products of a block (issue), consumed one step later (epi).
    // A block past the range is issued with zero scales (its loads may hold
    // another panel's rows): its products add +0 to sums that are never -0
    // (they start at +0, and an exact zero sum rounds to +0), so they leave
    // them unchanged, and every step runs the same straight-line code.
    auto issue = [&](const BdStage<TN> &st, const v4i &aop, uint16_t xs, bool on, v16i &dot,
                     v16f &sc) {
        const gh4 asc = __builtin_bit_cast(gh4, (v2u){on ? (uint32_t)xs : 0u, 0u});
        const uint32_t w0 = st.w[0][0], w1 = st.w[0][1];
        const v4i bop = (v4i){(int)(((w0 << 4) ^ 0x80808080u) & 0xf0f0f0f0u),
                              (int)(((w1 << 4) ^ 0x80808080u) & 0xf0f0f0f0u),
                              (int)((w0 ^ 0x80808080u) & 0xf0f0f0f0u),
                              (int)((w1 ^ 0x80808080u) & 0xf0f0f0f0u)};
        const gh4 bsc = __builtin_bit_cast(gh4, (v2u){on ? (uint32_t)st.ws[0] : 0u, 0u});
        v16i z = {};
        dot = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop, z, 0, 0, 0);
        v16f zf = {};
        sc = __builtin_amdgcn_mfma_f32_32x32x8f16(asc, bsc, zf, 0, 0, 0);
    };
    auto epi = [&](const v16i &dot, const v16f &sc) {
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[0][v] = fmaf((float)dot[v], sc[v], acc[0][v]);
    };
    // (set 1 starts neutral: the first step's epilogue adds 0 * 0)
    v16i pdot[PIPE ? 2 : 1] = {};
    v16f psc[PIPE ? 2 : 1] = {};
    // a tile's partial sums added in a fixed order: wavefronts 8..W-1 hand
    // theirs to 0..W-9, then the 8 sums meet in LDS ([w][register][lane]
    // floats, so no register is repacked); wavefront w < 8 gets registers
    // 2w and 2w + 1 (rows 8(w/2) + 4g + 2(w%2) + {0, 1})
    float *redf = (float *)red;
    auto reduce = [&](float (&t)[16], float (&r)[2]) {  // t: this wavefront's sums (consumed)
        if (BD_W > 8) {
            if (wave >= 8)
#pragma unroll
                for (int v = 0; v < 16; ++v) redf[((wave - 8) * 16 + v) * 64 + lane] = t[v];
            lds_barrier();
            if (wave < BD_W - 8)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    t[v] = __fadd_rn(t[v], redf[(wave * 16 + v) * 64 + lane]);
            lds_barrier();
        }
        if (wave < 8)
#pragma unroll
            for (int v = 0; v < 16; ++v) redf[(wave * 16 + v) * 64 + lane] = t[v];
        lds_barrier();
        if (wave < 8) {
            float s0 = redf[(2 * wave) * 64 + lane], s1 = redf[(2 * wave + 1) * 64 + lane];
#pragma unroll
            for (int w = 1; w < 8; ++w) {
                s0 = __fadd_rn(s0, redf[(w * 16 + 2 * wave) * 64 + lane]);
                s1 = __fadd_rn(s1, redf[(w * 16 + 2 * wave + 1) * 64 + lane]);
            }
            r[0] = s0 * 0.0625f;  // the 16x of the operands, exactly
            r[1] = s1 * 0.0625f;
        }
        lds_barrier();  // the area is written again next
    };
    // MODE 1: SwiGLU + Q8_0 of the gate|up pair (row, feat); every lane of
    // the half-wavefront calls it (quant_block_lane reduces over the 32
    // features of the row's block)
    auto gateup_out = [&](int row, int feat, float gv, float uv) {
        const int f = go.f;
        const float silu = __fdiv_rn(gv, __fadd_rn(1.0f, expf(-gv)));
        const float av = __fmul_rn(silu, uv);
        uint16_t dbits;
        int bsum;
        const int qv = quant_block_lane(av, dbits, bsum);  // all 32 lanes of the half
        if (row < m && feat < f) {
            const size_t o = (size_t)row * f + feat;
            if (out) {
                out[(size_t)row * ldo + feat] = gv;
                out[(size_t)row * ldo + f + feat] = uv;
            }
            if (go.act) go.act[o] = av;
            go.qs[o] = (int8_t)qv;
            if (j == 0) {
                go.d[o / SI_QK] = dbits;
                if (go.s) go.s[o / SI_QK] = (int16_t)bsum;
            }
            if (go.tq) {
                const size_t pb = (size_t)(row >> 5) * (f / SI_QK) + feat / SI_QK;
                go.tq[q8_tiled_byte(pb, row & 31, j)] = (int8_t)qv;
                if (j == 0) go.td[pb * 32 + (row & 31)] = dbits;
            }
        }
    };
    // DEFER (gate|up with streamed activations, whose LDS is free): at a
    // tile's end every wavefront's partial sums go to LDS ([W][TN][16][64]
    // floats), one barrier, and all wavefronts sum the (tile, register)
    // pairs into the slot's sums ([units][TN][16][64]) in reduce()'s order
    // (w + 8 added to w < W - 8, then w = 0..7 in turn: the same bits);
    // SwiGLU + Q8_0 of all the slot's units run once after the last (every
    // wavefront takes (unit, register) items).  Two barriers per unit
    // instead of eight, and no epilogue between units.
    constexpr bool DEFER = MODE == 1 && DA;
    float *dpart = (float *)bd_sm;
    float *dsum = dpart + BD_W * TN * 16 * 64;
    auto finish_defer = [&](int iu) {
#pragma unroll
        for (int u = 0; u < TN; ++u)
#pragma unroll
            for (int v = 0; v < 16; ++v) dpart[((wave * TN + u) * 16 + v) * 64 + lane] = acc[u][v];
        lds_barrier();
        for (int q = wave; q < TN * 16; q += BD_W) {  // q = 16 u + v, wavefront-uniform
            auto part = [&](int w) {  // wavefront w's sum, with w + 8's added as reduce() does
                const float t = dpart[(w * TN * 16 + q) * 64 + lane];
                return w < BD_W - 8 ? __fadd_rn(t, dpart[((w + 8) * TN * 16 + q) * 64 + lane]) : t;
            };
            float sum = part(0);
#pragma unroll
            for (int w = 1; w < 8; ++w) sum = __fadd_rn(sum, part(w));
            dsum[(iu * TN * 16 + q) * 64 + lane] = sum * 0.0625f;  // the operands' 16x, exactly
        }
        lds_barrier();  // the partial area is written again next
#pragma unroll
        for (int u = 0; u < TN; ++u)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[u][v] = 0.0f;
    };
    auto finish = [&](int iu) {
        if constexpr (DEFER) {
            finish_defer(iu);
            return;
        }
        float r[TN][2];
#pragma unroll
        for (int u = 0; u < TN; ++u) reduce(acc[u], r[u]);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if (wave >= 8) break;  // the partial sums only
            const int row = m0 + 8 * (wave >> 1) + 4 * g + 2 * (wave & 1) + i;
            if (MODE == 1) {
                gateup_out(row, col0(iu, 0) + j, r[0][i], r[TN - 1][i]);
            } else if (MODE == 2) {
                // permuted column pc: head pc / hdim, element e = (pc % hdim)
                // / 2 of its first (even pc) or second half; the pair's other
                // value is the neighbouring lane's (j ^ 1, same rows)
                const int pc = col0(iu, 0) + j;
                const float y = r[0][i] + (bias ? bias[pc] : 0.0f);
                const float yo = dpp_f<DPP_XOR1>(y);
                const int half = ro.hdim >> 1, within = pc % ro.hdim, side = within & 1;
                const int e = within >> 1, col = pc - within + e + side * half;
                if (row < m) {
                    if (out) out[(size_t)row * ldo + col] = y;
                    const int pos = ro.pos0 + row;
                    if (pos < ro.max_pos) {
                        // qwen_one_layer.c:172-183 as k_rope_kv: (a, b) ->
                        // (a c - b s, b c + a s)
                        const float a = side ? yo : y, b = side ? y : yo;
                        const float cs = ro.rc[(size_t)pos * half + e];
                        const float sn = ro.rs[(size_t)pos * half + e];
                        const float x = side ? __fadd_rn(__fmul_rn(b, cs), __fmul_rn(a, sn))
                                             : __fsub_rn(__fmul_rn(a, cs), __fmul_rn(b, sn));
                        const size_t kvrow = (size_t)row * ro.kv_seq_stride + (size_t)pos * ro.kvd;
                        if (col < ro.qd)
                            ro.q_out[(size_t)row * ro.qd + col] = x;
                        else if (col < ro.qd + ro.kvd)
                            ro.kc[kvrow + (col - ro.qd)] = f2h(x);
                        else
                            ro.vc[kvrow + (col - ro.qd - ro.kvd)] = f2h(y);
                    }
                }
            } else {
                const int col = col0(iu, 0) + j;
                if (row < m && col < n) {
                    if (part) {
                        part[((size_t)c * m + row) * n + col] = r[0][i];
                    } else if (pre) {
                        float y = r[0][i] + (iu ? pb[1] : pb[0]);
                        if (residual) y = __fadd_rn(iu ? pr[1][i] : pr[0][i], y);
                        out[(size_t)row * ldo + col] = y;
                    } else {
                        float y = r[0][i] + (bias ? bias[col] : 0.0f);
                        if (residual) y = __fadd_rn(residual[(size_t)row * ldo + col], y);
                        out[(size_t)row * ldo + col] = y;
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < TN; ++u)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[u][v] = 0.0f;
    };

    {
        fetch(0);
        int cu = 0, ck = 0;  // the compute pointer
        int vrem = len - wave;  // len - (BD_W ck + wave): the block is in range while > 0
        for (int it0 = 0; it0 < total; it0 += P) {
#pragma unroll
            for (int i = 0; i < P; ++i) {
                if (it0 + i < total) {
                    const v4i aop = DA ? st[i].a : a_nx;
                    const uint16_t xs = DA ? st[i].xs : x_nx;
                    const bool valid = vrem > 0;  // BD_W ck + wave < len
                    const int ckn = ck + 1 == per ? 0 : ck + 1;
                    fetch(ckn);
                    if constexpr (PIPE) {
                        // this step's block goes to set i & 1, then the
                        // previous step's (set (i + 1) & 1, neutral at a
                        // tile's first step) is accumulated
                        issue(st[i], aop, xs, valid, pdot[i & 1], psc[i & 1]);
                        __builtin_amdgcn_sched_barrier(0);
                        epi(pdot[(i + 1) & 1], psc[(i + 1) & 1]);
                    } else {
                        if (valid) compute(st[i], aop, xs);
                    }
                    ck = ckn;
                    vrem = ck == 0 ? len - wave : vrem - BD_W;
                    if (ck == 0) {
                        if constexpr (PIPE) {
                            // the tile's last block, then its set made
                            // neutral for the next tile's first step
                            epi(pdot[i & 1], psc[i & 1]);
#pragma unroll
                            for (int v = 0; v < 16; ++v) psc[i & 1][v] = 0.0f;
                        }
                        finish(cu);
                        ++cu;
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                load(st[i]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    if constexpr (DEFER) {
        // the slot's sums are complete (the last tile ended on a barrier):
        // SwiGLU + Q8_0 of (unit, register) items; register v holds rows
        // 8 (v / 4) + 4 g + v % 4 of the tile, lane j feature j
        for (int it = wave; it < nu * 16; it += BD_W) {
            const int iu = it >> 4, v = it & 15;
            const float gv = dsum[((iu * TN) * 16 + v) * 64 + lane];
            const float uv = dsum[((iu * TN + TN - 1) * 16 + v) * 64 + lane];
            gateup_out(m0 + 8 * (v >> 2) + 4 * g + (v & 3), col0(iu, 0) + j, gv, uv);
        }
    }
}

// The gate|up split partials [splits][m][2f] summed in split order (as
// k_gemm_reduce4), gate|up written to gu (optional), then SwiGLU and Q8_0
// exactly as k_swiglu_q8: half a wavefront per 32-feature block of a row.
__global__ void __launch_bounds__(256) k_gemm_reduce_swiglu_q8(
    const float *__restrict__ part, int splits, int m, int f, float *__restrict__ gu,
    float *__restrict__ act, int8_t *__restrict__ qs, uint16_t *__restrict__ d,
    int16_t *__restrict__ bs, int8_t *__restrict__ tq, uint16_t *__restrict__ td) {
    const int nbr = f / SI_QK;
    const int blk = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int j = threadIdx.x & 31;
    if (blk >= m * nbr) return;  // whole half-wavefronts leave together
    const int r = blk / nbr, b = blk - r * nbr;
    const size_t mn = (size_t)m * 2 * f;
    const size_t og = (size_t)r * 2 * f + (size_t)b * SI_QK + j, ou = og + f;
    float g = part[og], u = part[ou];
#pragma unroll 4
    for (int sp = 1; sp < splits; ++sp) {
        g += part[sp * mn + og];
        u += part[sp * mn + ou];
    }
    if (gu) {
        gu[og] = g;
        gu[ou] = u;
    }
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
        if (bs) bs[blk] = (int16_t)bsum;
    }
    if (tq) {
        const size_t pb = (size_t)(r >> 5) * nbr + b;
        tq[q8_tiled_byte(pb, r & 31, j)] = (int8_t)q;
        if (j == 0) td[pb * 32 + (r & 31)] = dbits;
    }
}

// out = residual + (bias + sum_s part[s]), the split partial sums in order.
__global__ void __launch_bounds__(256) k_gemm_reduce(const float *__restrict__ part, int splits,
                                                     int m, int n, const float *__restrict__ bias,
                                                     const float *__restrict__ residual,
                                                     float *__restrict__ out, int ldo) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)m * n) return;
    const int row = (int)(i / n), col = (int)(i - (size_t)row * n);
    float y = part[i];
    for (int s = 1; s < splits; ++s) y += part[(size_t)s * m * n + i];
    if (bias) y += bias[col];
    if (residual) y = __fadd_rn(residual[(size_t)row * ldo + col], y);
    out[(size_t)row * ldo + col] = y;
}

// k_gemm_reduce over 4 consecutive outputs per thread (n % 4 == 0, ldo % 4
// == 0, 16-byte aligned buffers): the split sums stream as float4.
__global__ void __launch_bounds__(256) k_gemm_reduce4(const float *__restrict__ part, int splits,
                                                      int m, int n, const float *__restrict__ bias,
                                                      const float *__restrict__ residual,
                                                      float *__restrict__ out, int ldo) {
    const size_t i4 = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t tot4 = (size_t)m * n / 4;
    if (i4 >= tot4) return;
    const size_t i = 4 * i4;
    const int row = (int)(i / n), col = (int)(i - (size_t)row * n);
    float4 y = *(const float4 *)(part + i);
    for (int s = 1; s < splits; ++s) {
        const float4 p = *(const float4 *)(part + (size_t)s * m * n + i);
        y.x += p.x; y.y += p.y; y.z += p.z; y.w += p.w;
    }
    if (bias) {
        const float4 b = *(const float4 *)(bias + col);
        y.x += b.x; y.y += b.y; y.z += b.z; y.w += b.w;
    }
    float *o = out + (size_t)row * ldo + col;
    if (residual) {
        const float4 r = *(const float4 *)(residual + (size_t)row * ldo + col);
        y = make_float4(__fadd_rn(r.x, y.x), __fadd_rn(r.y, y.y), __fadd_rn(r.z, y.z),
                        __fadd_rn(r.w, y.w));
    }
    *(float4 *)o = y;
}

// k_gemm_h16 launch: its stage LDS exceeds the default 64 KB limit.
template <int WM, int WN, int TM, int TN, bool FUSE>
static void launch_h16(dim3 grid, const uint8_t *wqs, const uint16_t *wd, int tile, int n, int nb,
                       const int8_t *xqs, const uint16_t *xd, int m, const float *bias,
                       const float *residual, float *out, int ldo, float *part, int bps,
                       const GateUpOut &go, hipStream_t st) {
    using C = H16Cfg<WM, WN, TM, TN>;
    static bool big_lds = false;
    if (!big_lds) {
        // a failure here surfaces as the launch's error
        (void)hipFuncSetAttribute((const void *)k_gemm_h16<WM, WN, TM, TN, FUSE>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)C::lds_bytes());
        big_lds = true;
    }
    SI_LAUNCH((k_gemm_h16<WM, WN, TM, TN, FUSE>), grid, dim3(C::NT), C::lds_bytes(), st, wqs, wd,
              tile, n, nb, xqs, xd, m, bias, residual, out, ldo, part, bps, go);
}

// Tile choice and K splits of the fast path for an m x n x nb problem.
struct GemmPlan {
    int bm, bn, splits, bps;
};
static GemmPlan gemm_plan(int m, int n, int nb) {
    GemmPlan p;
    // 64-row tiles up to 512 rows: twice the workgroups of a grid that
    // would leave the SIMDs about one wavefront each (0.5B prefill, 512
    // rows: 143 -> 121 us per layer); at 2048 rows 128-row tiles win
    p.bm = m <= 512 ? 64 : 128;
    p.bn = 128;
    const int tiles = ((n + p.bn - 1) / p.bn) * ((m + p.bm - 1) / p.bm);
    // K splits: a grid of W ~ 4.5 sqrt(tiles * nb) workgroups balances the
    // CUs against the split partial-sum traffic (fitted on the 7B and 0.5B
    // projections at 64 and 2048 rows); a grid that already fills the chip
    // over a short K is not split (the partials would cost more than the
    // tail they remove).
    int s = 1;
    if (!(tiles >= 384 && nb < 256)) {
        const double w = 4.5 * sqrt((double)tiles * nb);
        s = (int)lround(w / tiles);
    }
    const int maxs = nb / (2 * G_KB);  // >= 2 stages per split
    if (s > maxs) s = maxs;
    if (s < 1) s = 1;
    p.bps = (nb + s - 1) / s;
    p.bps = (p.bps + G_KB - 1) / G_KB * G_KB;
    p.splits = (nb + p.bps - 1) / p.bps;
    return p;
}

// k_gemm_bd's layout: H 32-row halves, C K ranges of cb blocks, S
// workgroups (slots) per (half, range) sharing its tiles round robin, one
// workgroup per CU (its LDS is most of the CU's).  Workgroup i runs on XCD
// i % 8 and the H halves of a slot share one, so S is sized for at most 32
// (one XCD's CUs) per XCD: C * S <= 8 * floor(32 / H).
constexpr int BD_SMALL_M = 64;  // every projection and the gate|up pair
constexpr int BD_GU_W = 12;     // wavefronts of the gate|up instances
constexpr int BD_MAX_M = 512;   // one-tile projections, when bd_takes() says so
struct BdPlan {
    int H, C, S, cb, units, grid;
    bool da;  // streamed (operand-tiled) activations: one K range, no fill
    // streamed one-tile projection whose 32-row halves outnumber the CUs:
    // one unit per workgroup of 8 wavefronts, two workgroups per CU, so the
    // grid runs in one round (or fewer)
    bool wide = false;
    size_t lds;
};
static BdPlan bd_plan(int m, int n, int nb, int mode, bool da = false) {
    // (da: m <= 64; for mode 1 the caller keeps nb <= BD_MAX_CB as without)
    BdPlan p;
    p.H = (m + 31) / 32;
    p.da = da;
    p.C = da ? 1 : (nb + BD_MAX_CB - 1) / BD_MAX_CB;
    p.cb = (nb + p.C - 1) / p.C;
    p.units = mode == 1 ? n / 64 : (n + 31) / 32;
    const int per_xcd = std::max(1, 32 / p.H);
    p.S = std::max(1, std::min(8 * per_xcd / p.C, p.units));
    if (da && mode == 0 && p.units * p.H > 256) {
        p.S = p.units;
        p.wide = true;
    }
    p.grid = 8 * p.H * ((p.C * p.S + 7) / 8);
    p.lds = da ? (size_t)BD_RED : bd_lds(p.cb);
    if (da && mode == 1) {
        // k_gemm_bd's deferred gate|up epilogue: the wavefronts' partial
        // sums and the slot's unit sums, 8 KB each; too many units per slot
        // for the LDS: staged activations and the per-unit epilogue instead
        const size_t units_per_slot = (size_t)(p.units + p.S - 1) / p.S;
        p.lds = (BD_GU_W + units_per_slot) * 8192;
        if (p.lds > (size_t)BD_LDS_MAX) return bd_plan(m, n, nb, mode, false);
    }
    return p;
}

// Whether gemm_core takes k_gemm_bd for a one-tile projection: always up to
// BD_SMALL_M rows; up to BD_MAX_M while K fits two LDS ranges and a slot's
// serial work (tiles per slot x blocks per range) stays near 1000 blocks.
// Measured per GEMM against the tile kernel and its K-split reduce: 0.5B
// QKV, O and down at 96-512 rows 6-19 us against 10-22; 7B QKV and O 12-38
// against 19-41; 7B down (five ranges, 833-4522 blocks per slot) 48-159
// against 40-119, so it keeps the tile kernel.  The gate|up pair stays on
// the tile kernel past BD_SMALL_M (0.5B, 512 rows: each slot's ten units
// took 45 us against 28).
static bool bd_takes(int m, int n, int nb) {
    if (m <= BD_SMALL_M) return true;
    if (m > BD_MAX_M) return false;
    const BdPlan p = bd_plan(m, n, nb, 0);
    return p.C <= 2 && (p.units + p.S - 1) / p.S * p.cb <= 1024;
}

// K splits gemm_core plans for an m x n x nb problem (1: one pass, no
// partials); the workspace size and the gate|up launcher decide with it
static int gemm_splits(int m, int n, int nb) {
    return bd_takes(m, n, nb) ? bd_plan(m, n, nb, 0).C : gemm_plan(m, n, nb).splits;
}

size_t gemm_workspace_bytes(int m, int n, int k) {
    const int splits = gemm_splits(m, n, k / SI_QK);
    return splits > 1 ? (size_t)splits * m * n * sizeof(float) : 0;
}

size_t gemm_gateup_workspace_bytes(int m, int f, int k) {
    if (m <= BD_SMALL_M && k / SI_QK <= BD_MAX_CB) return 0;  // one fused pass
    return gemm_workspace_bytes(m, 2 * f, k);
}

// k_gemm_bd launch (mode 1: gate|up, f = n / 2 features, one K range).
static void launch_bd(const BdPlan &p, int mode, const uint8_t *wqs, const uint16_t *wd,
                      int tile, int n, int nb, const int8_t *xqs, const uint16_t *xd, int m,
                      const float *bias, const float *residual, float *out, int ldo, float *part,
                      const GateUpOut &go, hipStream_t st, const RopeOut &ro = RopeOut{}) {
#define BD(TN, P, MODE, W, DA, PIPE)                                                           \
    do {                                                                                       \
        static bool big_lds = false;                                                           \
        if (!big_lds) {                                                                        \
            /* a failure here surfaces as the launch's error */                                \
            (void)hipFuncSetAttribute((const void *)k_gemm_bd<TN, P, MODE, W, DA, PIPE>,       \
                                      hipFuncAttributeMaxDynamicSharedMemorySize, BD_LDS_MAX); \
            big_lds = true;                                                                    \
        }                                                                                      \
        SI_LAUNCH((k_gemm_bd<TN, P, MODE, W, DA, PIPE>), dim3(p.grid), dim3(64 * W), p.lds,   \
                  st, wqs, wd, tile, n, nb, xqs, xd, m, bias, residual, out, ldo, part, p.H,   \
                  p.C, p.S, p.cb, p.units, go, ro);                                            \
    } while (0)
    // gate|up: 12 wavefronts (3 per SIMD; 4 weight blocks in flight fit
    // their registers); one tile: 16 (4 per SIMD, 7 of 112 blocks each, 4
    // in flight; 8 wavefronts with 16 in flight took 56 us for QKV + O +
    // down at 7B x 64 rows, 16 with 2, 4, 6 or 8 in flight 50-54 us)
    // streamed one-tile projections: 12 wavefronts, 2 stages, pipelined (7B
    // x 64 rows, cold weights: down 24.4 -> 23.3 us, QKV 13.0 -> 12.0, O
    // 8.7 -> 7.8 against 16 wavefronts x 4 stages unpipelined; 8 or 16
    // wavefronts and 3-12 stages took as long or longer).  Streamed gate|up:
    // 12 wavefronts, 2 stages (7B x 64 rows, cold weights: 41.3 us; 3-6
    // stages 41.6-44.9, 16 wavefronts 42.9; staged 43.7)
    if (mode == 2) {
        // Q|K|V + RoPE: the staged one-tile kernel (same sums as mode 0)
        BD(1, 4, 2, 16, false, false);
    } else if (mode == 1) {
        if (p.da)
            BD(2, 2, 1, BD_GU_W, true, false);
        else
            BD(2, 4, 1, BD_GU_W, false, false);
    } else if (p.wide) {
        // 7B Q|K|V at 64 rows (288 halves on 256 CUs): 12-wavefront
        // workgroups left 32 CUs a second round (~12.2 us); 8 unpipelined
        // wavefronts (93 VGPRs) run two workgroups per CU in one (~10.8
        // us); 0.5B down at 512 rows (448 halves): 14.0 -> 12.6 us
        BD(1, 2, 0, 8, true, false);
    } else if (p.da) {
        BD(1, 2, 0, 12, true, true);
    } else {
        BD(1, 4, 0, 16, false, false);
    }
#undef BD
}

static int gemm_core(const uint8_t *wqs, const uint16_t *wd, int tile, int n, int k,
                     const int8_t *xqs, const uint16_t *xd, int m, const float *bias,
                     const float *residual, float *out, int ldo, bool exact, void *workspace,
                     size_t ws_bytes, bool want_part, hipStream_t st);

int launch_gemm_q4q8_parts(const uint8_t *wqs, const uint16_t *wd, int tile, int n, int k,
                           const int8_t *xqs, const uint16_t *xd, int m, float *out, bool exact,
                           void *workspace, size_t ws_bytes, hipStream_t st) {
    return gemm_core(wqs, wd, tile, n, k, xqs, xd, m, nullptr, nullptr, out, n, exact, workspace,
                     ws_bytes, true, st);
}

void launch_gemm_reduce(const float *part, int splits, int m, int n, float *out,
                        hipStream_t st) {
    const size_t tot = (size_t)m * n;
    if (!tot) return;
    SI_LAUNCH(k_gemm_reduce, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st,
              part, splits, m, n, nullptr, nullptr, out, n);
}

void launch_gemm_q4q8(const uint8_t *wqs, const uint16_t *wd, int tile, int n, int k,
                      const int8_t *xqs, const uint16_t *xd, int m, const float *bias,
                      const float *residual, float *out, int ldo, bool exact, void *workspace,
                      size_t ws_bytes, hipStream_t st) {
    gemm_core(wqs, wd, tile, n, k, xqs, xd, m, bias, residual, out, ldo, exact, workspace,
              ws_bytes, false, st);
}

void launch_gemm_q4q8_tiled(const uint8_t *wqs, const uint16_t *wd, int tile, int n, int k,
                            const int8_t *tq, const uint16_t *td, int m, const float *bias,
                            const float *residual, float *out, int ldo, hipStream_t st) {
    if (m <= 0 || n <= 0) return;
    const int nb = k / SI_QK;
    launch_bd(bd_plan(m, n, nb, 0, true), 0, wqs, wd, tile, n, nb, tq, td, m, bias, residual,
              out, ldo, nullptr, GateUpOut{}, st);
}

// gate|up's fused k_gemm_bd pass (default flags, no f16)
static bool gateup_bd(int m, int k) { return m <= BD_SMALL_M && k / SI_QK <= BD_MAX_CB; }

bool gemm_gateup_streams(int m, int f, int k) {
    return gateup_bd(m, k) && bd_plan(m, 2 * f, k / SI_QK, 1, true).da;
}

bool gemm_streams(int m, int n, int k) {
    const int nb = k / SI_QK;
    if (m <= BD_SMALL_M) return true;
    if (m > BD_MAX_M || !bd_takes(m, n, nb)) return false;
    // a slot's serial work with one K range, as bd_takes bounds it
    const BdPlan p = bd_plan(m, n, nb, 0, true);
    return (p.units + p.S - 1) / p.S * nb <= 1024;
}

bool launch_gemm_qkv_rope(const uint8_t *wqs, const uint16_t *wd, int tile, int n, int k,
                          const int8_t *xqs, const uint16_t *xd, int m, const float *bias_perm,
                          float *out, const RopeOut &ro, hipStream_t st) {
    const int nb = k / SI_QK;
    if (m <= BD_SMALL_M || m > BD_MAX_M || n % 32 || ro.hdim % 2 || !bd_takes(m, n, nb))
        return false;
    const BdPlan p = bd_plan(m, n, nb, 2);
    if (p.C != 1) return false;  // no K-split partials in this epilogue
    launch_bd(p, 2, wqs, wd, tile, n, nb, xqs, xd, m, bias_perm, nullptr, out, n, nullptr,
              GateUpOut{}, st, ro);
    return true;
}

static int gemm_core(const uint8_t *wqs, const uint16_t *wd, int tile, int n, int k,
                     const int8_t *xqs, const uint16_t *xd, int m, const float *bias,
                     const float *residual, float *out, int ldo, bool exact, void *workspace,
                     size_t ws_bytes, bool want_part, hipStream_t st) {
    if (m <= 0 || n <= 0) return 0;
    const int nb = k / SI_QK;
    if (exact) {
        const dim3 grid((n + BN - 1) / BN, (m + BM - 1) / BM);
        SI_LAUNCH(k_gemm_q4q8<true>, grid, dim3(256), 0, st, wqs, wd, tile, n, nb, xqs,
                  xd, m, bias, residual, out, ldo);
        return 0;
    }
    const auto fits = [&](int splits) {
        return workspace && ws_bytes >= (size_t)splits * m * n * sizeof(float);
    };
    float *part = nullptr;
    int splits;
    if (bd_takes(m, n, nb)) {
        const BdPlan p = bd_plan(m, n, nb, 0);
        if (p.C == 1 || fits(p.C)) {
            part = p.C > 1 ? (float *)workspace : nullptr;
            launch_bd(p, 0, wqs, wd, tile, n, nb, xqs, xd, m, bias, residual, out, ldo, part,
                      GateUpOut{}, st);
            splits = p.C;
        } else {
            // K longer than one LDS range and no workspace: the LDS-staged
            // kernel in one pass
            const dim3 grid((n + 127) / 128, (m + 63) / 64, 1);
            SI_LAUNCH((k_gemm_fast<1, 4, 2, 1, false>), grid, dim3(256),
                      (GemmCfg<1, 4, 2, 1>::lds_bytes()), st, wqs, wd, tile, n, nb, xqs, xd, m,
                      bias, residual, out, ldo, nullptr, nb, GateUpOut{});
            splits = 1;
        }
    } else {
        GemmPlan p = gemm_plan(m, n, nb);
        if (p.splits > 1 && !fits(p.splits)) {
            p.splits = 1;
            p.bps = nb;
        }
        part = p.splits > 1 ? (float *)workspace : nullptr;
        const dim3 grid((n + p.bn - 1) / p.bn, (m + p.bm - 1) / p.bm, p.splits);
#define CALL(WM, WN, TM, TN)                                                                   \
    SI_LAUNCH((k_gemm_fast<WM, WN, TM, TN, false>), grid, dim3(256),                           \
              (GemmCfg<WM, WN, TM, TN>::lds_bytes()), st, wqs, wd, tile, n, nb, xqs,           \
              xd, m, bias, residual, out, ldo, part, p.bps, GateUpOut{})
        if (p.bm == 64)
            CALL(1, 4, 2, 1);
        else
            CALL(2, 2, 2, 2);
#undef CALL
        splits = p.splits;
    }
    if (part && want_part) return splits;
    if (part) {
        const size_t tot = (size_t)m * n;
        const auto al = [](const void *q) { return ((uintptr_t)q & 15) == 0; };
        if (n % 4 == 0 && ldo % 4 == 0 && al(out) && al(bias) && al(residual))
            SI_LAUNCH(k_gemm_reduce4, dim3((unsigned)((tot / 4 + 255) / 256)), dim3(256),
                      0, st, part, splits, m, n, bias, residual, out, ldo);
        else
            SI_LAUNCH(k_gemm_reduce, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0,
                      st, part, splits, m, n, bias, residual, out, ldo);
    }
    return 0;
}

// ===========================================================================
// Operands of the fp6 formulation (k_gemm_fast with F6)

// 32 codes (8 dwords of 4) -> 24 bytes, code i at bit 6 i of six little-
// endian dwords (the operand packing of the fp6 matrix instructions); bytes
// 0..15 to p16, 16..23 to p8
__device__ __forceinline__ void f6_store(uint8_t *p16, uint8_t *p8, const uint32_t (&c)[8]) {
    uint32_t q[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) q[k] = f6_pack4(c[k]);
    // 8-byte stores: a region of an odd row count starts only 8-byte aligned
    *(uint2 *)p16 = make_uint2(q[0] | q[1] << 24, q[1] >> 8 | q[2] << 16);
    *(uint2 *)(p16 + 8) = make_uint2(q[2] >> 16 | q[3] << 8, q[4] | q[5] << 24);
    *(uint2 *)p8 = make_uint2(q[5] >> 8 | q[6] << 16, q[6] >> 16 | q[7] << 8);
}

// Q8 values, planar [m][nb * 32] -> x6: per block the region of the codes of
// hi = q >> 4 (-8..7), then that of lo = q & 15 (q = 16 hi + lo), each m rows
// as [m][16] then [m][8].  Grid (ceil(m / 64), nb), a thread per (row,
// block), consecutive threads consecutive rows (one-wavefront workgroups: a
// few hundred rows still spread over the CUs).
__global__ void __launch_bounds__(64) k_q8_to_x6(const int8_t *__restrict__ qs, int m, int nb,
                                                 uint8_t *__restrict__ x6) {
    const int row = blockIdx.x * 64 + threadIdx.x, blk = blockIdx.y;
    if (row >= m) return;
    const int8_t *src = qs + ((size_t)row * nb + blk) * SI_QK;
    const uint4 q0 = *(const uint4 *)src, q1 = *(const uint4 *)(src + 16);
    const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    uint32_t hi[8], lo[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        hi[k] = f6_codes4((w[k] >> 4) & 0x0f0f0f0fu, true);
        lo[k] = f6_codes4(w[k] & 0x0f0f0f0fu, false);
    }
    uint8_t *rh = x6 + (size_t)(2 * blk) * m * F6_BYTES, *rl = rh + (size_t)m * F6_BYTES;
    f6_store(rh + (size_t)row * 16, rh + (size_t)m * 16 + (size_t)row * 8, hi);
    f6_store(rl + (size_t)row * 16, rl + (size_t)m * 16 + (size_t)row * 8, lo);
}

// Repacked Q4 [nb][n][16] (byte i: element i low nibble, i + 16 high) and its
// tiled scales -> w6 (per block a region of n rows, [n][16] then [n][8], codes
// of nibble - 8: the two's-complement table at nibble ^ 8) and d6 [nb][n];
// logical row r is physical row gate_up_row(r, gu_f) when gu_f > 0.
__global__ void __launch_bounds__(256) k_q4_to_w6(const uint8_t *__restrict__ qs,
                                                  const uint16_t *__restrict__ d, int n, int nb,
                                                  int tile, int gu_f, uint8_t *__restrict__ w6,
                                                  uint16_t *__restrict__ d6) {
    const int r = blockIdx.x * 256 + threadIdx.x, blk = blockIdx.y;
    if (r >= n) return;
    const int pr = gu_f ? gate_up_row(r, gu_f) : r;
    const uint4 b = *(const uint4 *)(qs + ((size_t)blk * n + pr) * 16);
    const uint32_t w[4] = {b.x, b.y, b.z, b.w};
    uint32_t c[8];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        c[t] = f6_codes4((w[t] & 0x0f0f0f0fu) ^ 0x08080808u, true);             // elements 4t..
        c[4 + t] = f6_codes4(((w[t] >> 4) & 0x0f0f0f0fu) ^ 0x08080808u, true);  // 16 + 4t..
    }
    uint8_t *rg = w6 + (size_t)blk * n * F6_BYTES;
    f6_store(rg + (size_t)r * 16, rg + (size_t)n * 16 + (size_t)r * 8, c);
    d6[(size_t)blk * n + r] = d[q4_scale_index(pr, blk, nb, tile)];
}

void launch_q8_to_x6(const int8_t *qs, int m, int nb, uint8_t *x6, hipStream_t st) {
    if (m <= 0 || nb <= 0) return;
    SI_LAUNCH(k_q8_to_x6, dim3((unsigned)((m + 63) / 64), (unsigned)nb), dim3(64), 0, st, qs, m,
              nb, x6);
}

void launch_q4_to_w6(const uint8_t *qs, const uint16_t *d, int n, int nb, int tile, int gu_f,
                     uint8_t *w6, uint16_t *d6, hipStream_t st) {
    if (n <= 0 || nb <= 0) return;
    SI_LAUNCH(k_q4_to_w6, dim3((unsigned)((n + 255) / 256), (unsigned)nb), dim3(256), 0, st, qs, d,
              n, nb, tile, gu_f, w6, d6);
}

size_t gemm_f6_partial_bytes(int m, int n, int k) {
    const GemmPlan p = gemm_plan(m, n, k / SI_QK);
    return p.splits > 1 ? (size_t)p.splits * m * n * sizeof(float) : 0;
}

int launch_gemm_f6(const uint8_t *w6, const uint16_t *d6, int n, int k, const uint8_t *x6,
                   const uint16_t *xd, int m, const float *bias, const float *residual,
                   float *out, int ldo, void *workspace, size_t ws_bytes, bool want_part,
                   int gu_f, float *act, int8_t *aqs, uint16_t *ad, int16_t *as, hipStream_t st,
                   int8_t *atq, uint16_t *atd) {
    if (m <= 0 || n <= 0) return 0;
    const int nb = k / SI_QK;
    GemmPlan p = gemm_plan(m, n, nb);
    if (gu_f && p.splits > 1) return -1;
    if (p.splits > 1 && !(workspace && ws_bytes >= (size_t)p.splits * m * n * sizeof(float))) {
        p.splits = 1;
        p.bps = nb;
    }
    float *part = p.splits > 1 ? (float *)workspace : nullptr;
    const dim3 grid((m + p.bm - 1) / p.bm, (n + p.bn - 1) / p.bn, p.splits);
    const GateUpOut go{gu_f, act, aqs, ad, as, atq, atd};
#define CALL(WM, WN, TM, TN, FUSE)                                                             \
    SI_LAUNCH((k_gemm_f6<WM, WN, TM, TN, FUSE>), grid, dim3(256), 0, st, w6, d6, n, nb, x6, xd, \
              m, bias, residual, out, ldo, part, p.bps, go)
    if (gu_f) {
        if (p.bm == 64)
            CALL(2, 2, 1, 2, true);
        else
            CALL(2, 2, 2, 2, true);
    } else {
        if (p.bm == 64)
            CALL(1, 4, 2, 1, false);
        else
            CALL(2, 2, 2, 2, false);
    }
#undef CALL
    if (!part) return 0;
    if (want_part) return p.splits;
    const size_t tot = (size_t)m * n;
    const auto al = [](const void *q) { return ((uintptr_t)q & 15) == 0; };
    if (n % 4 == 0 && ldo % 4 == 0 && al(out) && al(bias) && al(residual))
        SI_LAUNCH(k_gemm_reduce4, dim3((unsigned)((tot / 4 + 255) / 256)), dim3(256), 0, st,
                  part, p.splits, m, n, bias, residual, out, ldo);
    else
        SI_LAUNCH(k_gemm_reduce, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st, part,
                  p.splits, m, n, bias, residual, out, ldo);
    return 0;
}

// gate|up GEMM with SwiGLU + Q8_0: f features, weights the physical
// [gate; up] rows.  One fused kernel when the plan needs no K split; with a
// split, the GEMM's partials then k_gemm_reduce_swiglu_q8 (split sums,
// gate|up, SwiGLU and Q8 in one pass); in exact mode the GEMM into gu, then
// k_swiglu_q8.
void launch_gemm_gateup_q8(const uint8_t *wqs, const uint16_t *wd, int tile, int f, int k,
                           const int8_t *xqs, const uint16_t *xd, int m, float *gu, float *act,
                           int8_t *qs, uint16_t *d, int16_t *s, bool exact, void *workspace,
                           size_t ws_bytes, hipStream_t st, bool f16, int8_t *tq, uint16_t *td,
                           const int8_t *txq, const uint16_t *txd) {
    if (m <= 0) return;
    const int n = 2 * f, nb = k / SI_QK;
    if (f16 && !exact) {
        // the f16 formulation: 128 x 256 tiles (the fastest of the tilings
        // measured), one pass over K
        launch_h16<2, 4, 2, 2, true>(dim3((n + 255) / 256, (m + 127) / 128, 1), wqs, wd, tile, n,
                                     nb, xqs, xd, m, nullptr, nullptr, gu, n, nullptr, nb,
                                     GateUpOut{f, act, qs, d, s, tq, td}, st);
        return;
    }
    if (!exact && gateup_bd(m, k)) {
        // the activations streamed when given operand-tiled (txq / txd)
        const BdPlan p = bd_plan(m, n, nb, 1, txq && txd);
        launch_bd(p, 1, wqs, wd, tile, n, nb, p.da ? txq : xqs, p.da ? txd : xd, m, nullptr,
                  nullptr, gu, n, nullptr, GateUpOut{f, act, qs, d, s, tq, td}, st);
        return;
    }
    // a K split (gemm_core's own plan: k_gemm_bd's K-range partials or the
    // tile kernel's), or, with too little workspace, one pass into gu; then
    // the split reduce.  Without a split gemm_core would write gu, which is
    // optional here: the fused pass below.
    const bool split = exact || gemm_splits(m, n, nb) > 1;
    if (split) {
        const int splits = gemm_core(wqs, wd, tile, n, k, xqs, xd, m, nullptr, nullptr, gu, n,
                                     exact, workspace, ws_bytes, true, st);
        if (splits > 1) {
            const int tot = m * (f / SI_QK);
            SI_LAUNCH(k_gemm_reduce_swiglu_q8, dim3((tot + 7) / 8), dim3(256), 0, st,
                      (const float *)workspace, splits, m, f, gu, act, qs, d, s, tq, td);
        } else {
            launch_swiglu_q8(gu, m, f, act, qs, d, s, st, tq, td);
        }
        return;
    }
    const GemmPlan p = gemm_plan(m, n, nb);
    const GateUpOut go{f, act, qs, d, s, tq, td};
    const dim3 grid((n + p.bn - 1) / p.bn, (m + p.bm - 1) / p.bm, 1);
#define CALL(WM, WN, TM, TN)                                                                   \
    SI_LAUNCH((k_gemm_fast<WM, WN, TM, TN, true>), grid, dim3(256),                            \
              (GemmCfg<WM, WN, TM, TN>::lds_bytes()), st, wqs, wd, tile, n, nb, xqs,           \
              xd, m, nullptr, nullptr, gu, n, nullptr, nb, go)
    if (p.bm == 64)
        CALL(2, 2, 1, 2);
    else
        CALL(2, 2, 2, 2);
#undef CALL
}

}  // namespace si
