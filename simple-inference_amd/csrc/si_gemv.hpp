// si_gemv.hpp -- Q4_0 x Q8_0 mat-vec core shared by the decode kernels.
//
// matvec_q4q8 (qwen_one_layer.c:148-162) for one activation row.  The RVV
// design put output neurons on vector lanes (fused_column_matvec,
// fused_layer.h:169-245); here a workgroup owns R output rows and the whole
// K: thread t takes row t % R and every KL-th block starting at t / R
// (KL = T / R).  Weights are block-major ([K/32][N][16] nibble bytes,
// [K/32][N] fp16 scales), so one wavefront load of a block touches R
// consecutive rows (R*16 contiguous bytes) for 64/R blocks.  Each thread
// loads U blocks at a time (U = 2: deeper batches measured slower).
// Per block: 8 AND/shift unpacks, 8 v_dot4 int8 dots and one -8*sum(a)
// correction give the exact int32 dot; the fp32 epilogue applies both fp16
// scales.  Partial sums meet
// through wavefront shuffles and LDS in a fixed order (deterministic).
// With R = T (one thread per row, KL = 1) a row's blocks are accumulated in
// order with the reference's roundings, y = bias; y = y + ((float)dot *
// w.d) * x.d: bit-exact (the EXACT instantiation).
#pragma once
#include "si_device.hpp"

namespace si {

// ---------------------------------------------------------------------------
// integer block dot: Q4_0 block (16 nibble bytes) x Q8_0 block (32 int8)
// ---------------------------------------------------------------------------
__device__ __forceinline__ int dot_q4_q8(const uint4 w, const int4 alo, const int4 ahi,
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
    return acc - 8 * asum;  // nibble - 8 applied as one correction per block
}

// A Q8_0 activation row: int8 values, fp16 scale bits and int block sums.
struct Q8Row {
    const int8_t *qs;
    const uint16_t *d;
    const int16_t *s;
};

// Logical row -> stored row.  Identity, or the gate|up pairing: logical rows
// 64b..64b+31 are gate rows 32b.. and 64b+32..64b+63 the up rows 32b.. (up
// rows stored after the F gate rows), so one wavefront ends with the gate
// and up values of the same 32 outputs: one Q8_0 block of the activation.
struct RowIdentity {
    __device__ int operator()(int r) const { return r; }
};
struct RowGateUp {
    int f;
    __device__ int operator()(int r) const {
        const int j = 32 * (r >> 6) + (r & 31);
        return (r & 32) ? f + j : j;
    }
};

// The mat-vec of the rows [tile0, tile0 + R) of a matrix with n logical
// rows and nb K blocks, in two phases so a kernel can put its first weight
// loads in flight before it builds the activation row:
//   GemvRows<R, T, EXACT, Map> g(wqs, wd, tile, nstore, n, nb, tile0, map);
//   g.start();                 // first U blocks per thread requested
//   ... prologue (activation row into LDS) ...
//   y = g.finish(x, init, red) // row sums in threads t < R (0 elsewhere)
// wd: scales in the tile-major layout of q4_scale_index with `tile` rows
// per tile (mat-vec workgroups use R = tile, so the scales of a wavefront's
// rows and blocks are one contiguous run that no other workgroup reads).
// red: LDS scratch of red_floats<R, T>() floats.
template <int R, int T, bool EXACT, typename Map, int U = 2>
struct GemvRows {
    static_assert(!EXACT || R == T, "exact mode keeps one thread per row");
    static constexpr int KL = T / R;  // K lanes per row
    __amdgpu_buffer_rsrc_t wrs, drs;  // the whole weight and scale arrays
    uint32_t woff, doff;              // this row's block-0 byte offsets
    uint32_t bstride, sstride;        // bytes per block step
    int nb, kl, r;
    uint4 w[U];
    uint16_t ws[U];

    __device__ __forceinline__ GemvRows(const uint8_t *__restrict__ wqs,
                                        const uint16_t *__restrict__ wd, int tile, int nstore,
                                        int n, int nb_, int tile0, Map map) {
        const int t = threadIdx.x;
        r = t % R;
        kl = t / R;
        nb = nb_;
        const int srow = map(min(tile0 + r, n - 1));
        bstride = (uint32_t)nstore * 16;  // bytes per block plane
        sstride = (uint32_t)tile * 2;     // scale bytes per block
        wrs = buf_rsrc(wqs, (uint32_t)nb * bstride);
        drs = buf_rsrc(wd, (uint32_t)(q4_scale_count(nstore, nb, tile) * 2));
        woff = (uint32_t)srow * 16;
        doff = (uint32_t)(q4_scale_index(srow, 0, nb, tile) * 2);
    }
    // Branch-free buffer loads: a block past the end lies past the weight
    // array and reads as zero with no memory access (skipped by finish()),
    // so the compiler can count the loads in flight exactly (a load under a
    // branch makes later waits drain all).  The caller keeps the weight and
    // scale arrays under 4 GiB.
    __device__ __forceinline__ void load(int b0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t b = (uint32_t)(b0 + u * KL);
            w[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 wrs, woff + b * bstride, 0, 0));
            ws[u] = __builtin_amdgcn_raw_buffer_load_b16(drs, doff + b * sstride, 0, 0);
        }
    }
    __device__ __forceinline__ void start() { load(kl); }

    __device__ __forceinline__ float finish(const Q8Row x, float init, float *red) {
        float acc = init;
        for (int b0 = kl; b0 < nb; b0 += U * KL) {
            if (b0 != kl) load(b0);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int b = b0 + u * KL;
                if (b < nb) {
                    const int4 alo = *(const int4 *)(x.qs + b * SI_QK);
                    const int4 ahi = *(const int4 *)(x.qs + b * SI_QK + 16);
                    const int dot = dot_q4_q8(w[u], alo, ahi, x.s[b]);
                    if (EXACT)
                        acc = __fadd_rn(acc, __fmul_rn(__fmul_rn((float)dot, h2f(ws[u])),
                                                       h2f(x.d[b])));
                    else
                        acc = fmaf((float)dot, h2f_fast(ws[u]) * h2f_fast(x.d[b]), acc);
                }
            }
        }
        if (EXACT) return acc;
        const int t = threadIdx.x;
        // rows r of one wavefront: lanes r + R*j; fold j with shuffles
        if (R < 64) acc = fold_rows<R>(acc);
        constexpr int P = R >= 64 ? KL : T / 64;  // partials per row
        const int p = R >= 64 ? kl : (t >> 6);
        if (R >= 64 || (t & 63) < R) red[p * R + r] = acc;
        __syncthreads();
        float y = 0.0f;
        if (t < R) {
            y = red[t];
#pragma unroll
            for (int q = 1; q < P; ++q) y += red[q * R + t];
        }
        return y;
    }
};

template <int R, int T>
constexpr int red_floats() {
    return (R >= 64 ? T / R : T / 64) * R;
}

// Rows per workgroup and scale tile of a matrix used by the mat-vec: the
// smallest R in {8, 16, 32, 64} that keeps the grid at <= 1200 workgroups.
inline int gemv_tile_for(int n) {
    int r = 8;
    while (r < 64 && (n + r - 1) / r > 1200) r *= 2;
    return r;
}

// Threads per workgroup for R rows and nb blocks: K lanes per row
// KL = T / R up to 64 (R = 8, 16), 8 (R = 32) or 4 (R = 64) and at most
// the largest power of two <= nb; at least one wavefront.
inline int gemv_threads(int r, int nb) {
    int kl = r <= 16 ? 512 / r : 256 / r;
    while (kl > 1 && kl > nb) kl >>= 1;
    int t = r * kl;
    return t < 64 ? 64 : t;
}

// Threads for the decode kernels that also build their activation row: 512
// (8 wavefronts: all four SIMDs busy, two wavefronts each) so the row's
// per-thread share stays small.
inline int dec_threads(int r, int nb) {
    const int t = gemv_threads(r, nb);
    return t > 512 ? t : 512;
}

// Instantiates CALL(R, T, false) for the (R, T) pairs gemv_threads and
// dec_threads return.
#define SI_GEMV_SWITCH(r, t, CALL)               \
    switch ((r) * 1000 + (t)) {                  \
        case 8064: CALL(8, 64, false); break;    \
        case 8128: CALL(8, 128, false); break;   \
        case 8256: CALL(8, 256, false); break;   \
        case 8512: CALL(8, 512, false); break;   \
        case 16064: CALL(16, 64, false); break;  \
        case 16128: CALL(16, 128, false); break; \
        case 16256: CALL(16, 256, false); break; \
        case 16512: CALL(16, 512, false); break; \
        case 32064: CALL(32, 64, false); break;  \
        case 32128: CALL(32, 128, false); break; \
        case 32256: CALL(32, 256, false); break; \
        case 32512: CALL(32, 512, false); break; \
        case 64064: CALL(64, 64, false); break;  \
        case 64128: CALL(64, 128, false); break; \
        case 64512: CALL(64, 512, false); break; \
        default: CALL(64, 256, false); break;    \
    }

}  // namespace si
