// si_device.hpp -- device helpers shared by the gfx950 kernels.
//
// Every helper that feeds a bit-exact result (Q8 scales, fp16 K/V) spells
// out its rounding with the correctly rounded __f*_rn operations, so the
// result does not depend on contraction or fast-math settings.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define SI_QK 32

namespace si {

// Correctly rounded binary32 square root (glibc sqrtf, as rmsnorm uses it,
// qwen_one_layer.c:167).  HIP's __fsqrt_rn is the hardware v_sqrt_f32 (about
// 1 ulp) unless OCML_BASIC_ROUNDED_OPERATIONS is defined; the builtin
// compiles to v_sqrt_f32 plus a two-neighbour correction by fma.
__device__ __forceinline__ float sqrt_rn(float x) { return __builtin_sqrtf(x); }

// Operand-tiled Q8_0: the activation operand of the batched-decode GEMM
// (k_gemm_bd's streamed mode) in the order its matrix-core lanes take it.
// Rows are grouped in panels of 32; block b of panel p (pb = p * nb + b) is
// one 1 KB run [half g][row j][16 bytes], half g of row j holding the
// block's bytes 8g..8g+7 then 16+8g..16+8g+7 (the elements lane (j, g) of a
// 32x32x32 i8 MFMA supplies).  Scales are [panel][block][row] fp16 bits
// (q8_tiled_d index pb * 32 + j).  Byte i (0..31) of row j of block pb:
__host__ __device__ constexpr size_t q8_tiled_byte(size_t pb, int j, int i) {
    return pb * 1024 + (size_t)((i >> 3) & 1) * 512 + (size_t)j * 16 +
           (size_t)((i & 7) | ((i >> 4) << 3));
}

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }

// IEEE binary16 -> binary32, exact for every input (qwen_one_layer.c:42-59).
__device__ __forceinline__ float h2f(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) {
        const float v = __fmul_rn((float)m, 0x1p-24f);
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

// Hardware widening for finite cache values (exact for all finite halves).
__device__ __forceinline__ float h2f_fast(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// IEEE binary32 -> binary16, round-to-nearest-even, gradual underflow,
// NaN -> sign|0x7e00, overflow -> sign|inf (qwen_one_layer.c:61-86).
// Integer-only, so it does not depend on the denormal mode.
__device__ __forceinline__ uint16_t f2h(float x) {
    const uint32_t b = f2u(x);
    const uint32_t sign = (b >> 16) & 0x8000u;
    const uint32_t a = b & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (a < 0x38800000u) {
        const uint32_t e = a >> 23;
        if (e < 102u) return (uint16_t)sign;
        const uint32_t m = (a & 0x7fffffu) | 0x800000u;  // e >= 102 > 0: normal
        const uint32_t shift = 126u - e;                 // 14..24
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        q += (rem > half) || (rem == half && (q & 1u));
        return (uint16_t)(sign | q);
    }
    uint32_t r = a - 0x38000000u;
    r += 0x0fffu + ((r >> 13) & 1u);
    return (uint16_t)(sign | (r >> 13));
}

// ---------------------------------------------------------------------
// Cross-lane data movement without the LDS crossbar.  A wavefront is four
// rows of 16 lanes.  DPP moves within a row (quad_perm, row_ror,
// row_half_mirror); gfx950's v_permlane16_swap / v_permlane32_swap exchange
// rows 0<->1, 2<->3 and halves 0<->1.  (__shfl_xor lowers to
// ds_bpermute_b32, a round trip through LDS, ten of which per Q8 block
// dominated the small decode kernels.)  Every lane of a group must be
// active.  The lane layouts are checked on the device by the test-only
// probe library (tests/probe).
// ---------------------------------------------------------------------
enum : int {
    DPP_XOR1 = 0xB1,      // quad_perm [1,0,3,2]
    DPP_XOR2 = 0x4E,      // quad_perm [2,3,0,1]
    DPP_ROR4 = 0x124,     // row_ror:4  (lane i <- lane (i-4) % 16 of its row)
    DPP_ROR8 = 0x128,     // row_ror:8
    DPP_HMIRROR = 0x141,  // row_half_mirror (lane i <- 7-i within 8)
    DPP_SHL1 = 0x101,     // row_shl:1 (lane i <- lane i+1 of its row; the row's last lane gets 0)
};

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}
// partner value of the lane 16 (swap16) or 32 (swap32) lanes away
__device__ __forceinline__ int swap16_i(int v) {
    const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
    return (int)((threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ int swap32_i(int v) {
    const auto r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
    return (int)((threadIdx.x & 32) ? r[0] : r[1]);
}
__device__ __forceinline__ float swap16_f(float v) { return __int_as_float(swap16_i(__float_as_int(v))); }
__device__ __forceinline__ float swap32_f(float v) { return __int_as_float(swap32_i(__float_as_int(v))); }

// gfx950 transposing LDS read (ds_read_b64_tr_b16).  Within each group of
// 16 lanes, lane i receives as element e (0..3) the 16-bit value i % 4 of
// the 8 bytes read at the address of lane 4*e + i/4 of its group (lane
// layout measured on the device).  So if lane s of a group points at
// row[r0 + s/4][c0 + 4*(s%4)] of a row-major fp16 matrix, lane i receives
// column c0 + i of rows r0..r0+3: the A/B operand of a 16x16x16 f16 MFMA
// whose reduction runs down the rows.  p must be 8-byte aligned.
typedef short tr_s4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ tr_s4 lds_read_tr16(const void *p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) tr_s4 *)(__attribute__((address_space(3))) void *)
            const_cast<void *>(p));
}

// Reductions over groups of 8 lanes (i & ~7), 32 lanes and the wavefront;
// every lane of the group gets the result.
__device__ __forceinline__ float oct_max(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    return fmaxf(v, dpp_f<DPP_HMIRROR>(v));
}
__device__ __forceinline__ int oct_sum(int v) {
    v += dpp_i<DPP_XOR1>(v);
    v += dpp_i<DPP_XOR2>(v);
    return v + dpp_i<DPP_HMIRROR>(v);
}
__device__ __forceinline__ float half_wave_max(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_ROR4>(v));
    v = fmaxf(v, dpp_f<DPP_ROR8>(v));
    return fmaxf(v, swap16_f(v));
}
__device__ __forceinline__ int half_wave_sum(int v) {
    v += dpp_i<DPP_XOR1>(v);
    v += dpp_i<DPP_XOR2>(v);
    v += dpp_i<DPP_ROR4>(v);
    v += dpp_i<DPP_ROR8>(v);
    return v + swap16_i(v);
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<DPP_XOR1>(v);
    v += dpp_f<DPP_XOR2>(v);
    v += dpp_f<DPP_ROR4>(v);
    v += dpp_f<DPP_ROR8>(v);
    v += swap16_f(v);
    return v + swap32_f(v);
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_ROR4>(v));
    v = fmaxf(v, dpp_f<DPP_ROR8>(v));
    v = fmaxf(v, swap16_f(v));
    return fmaxf(v, swap32_f(v));
}
__device__ __forceinline__ double dpp_d_add(double v, int which) {
    const long long b = __double_as_longlong(v);
    int lo = (int)b, hi = (int)(b >> 32);
    switch (which) {
        case 0: lo = dpp_i<DPP_XOR1>(lo); hi = dpp_i<DPP_XOR1>(hi); break;
        case 1: lo = dpp_i<DPP_XOR2>(lo); hi = dpp_i<DPP_XOR2>(hi); break;
        case 2: lo = dpp_i<DPP_ROR4>(lo); hi = dpp_i<DPP_ROR4>(hi); break;
        case 3: lo = dpp_i<DPP_ROR8>(lo); hi = dpp_i<DPP_ROR8>(hi); break;
        case 4: lo = swap16_i(lo); hi = swap16_i(hi); break;
        default: lo = swap32_i(lo); hi = swap32_i(hi); break;
    }
    return v + __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int w = 0; w < 6; ++w) v = dpp_d_add(v, w);
    return v;
}
// Sum over the lanes r, r+R, r+2R, ... of a wavefront (R = 4..32), for the
// mat-vec's K lanes of one row; lane r (and every partner) gets the total.
template <int R>
__device__ __forceinline__ float fold_rows(float v) {
    if (R <= 4) v += dpp_f<DPP_ROR4>(v);
    if (R <= 8) v += dpp_f<DPP_ROR8>(v);
    if (R <= 16) v += swap16_f(v);
    if (R <= 32) v += swap32_f(v);
    return v;
}

// ---------------------------------------------------------------------
// quantize_q8 of one 32-value block held one value per lane of a half
// wavefront (qwen_one_layer.c:98-116), bit-exact:
//   amax = max|x| (NaN ignored, as the reference's `a > amax` test does)
//   d    = amax / 127 (correctly rounded), stored as fp16(d)
//   inv  = d == 0 ? 0 : 1/d  from the unrounded d
//   q    = lrintf(x*inv) clamped to [-127, 127]; lrintf of a NaN or
//          infinite product yields LONG_MIN on x86-64, i.e. -127 here.
// Returns q; every lane gets the block's fp16 scale bits and int sum.
// ---------------------------------------------------------------------
__device__ __forceinline__ int quant_block_lane(float x, uint16_t &dbits, int &bsum) {
    const float a = fmaxf(0.0f, fabsf(x));  // NaN -> 0
    const float amax = half_wave_max(a);
    const float d = __fdiv_rn(amax, 127.0f);
    dbits = f2h(d);
    const float inv = (d == 0.0f) ? 0.0f : __fdiv_rn(1.0f, d);
    const float y = __fmul_rn(x, inv);
    int q;
    if (!(fabsf(y) <= 3.0e38f)) {
        q = -127;  // NaN or +-inf
    } else {
        q = (int)rintf(fminf(fmaxf(y, -200.0f), 200.0f));
        q = q > 127 ? 127 : (q < -127 ? -127 : q);
    }
    bsum = half_wave_sum(q);
    return q;
}

// quantize_q8 of one 32-value block spread over a group of 8 lanes, 4
// consecutive values per lane (lane i & 7 holds values 4*(i&7) .. +3), with
// exactly quant_block_lane's rules.  Returns the lane's 4 int8 values packed
// little-endian; every lane gets the fp16 scale bits and the block sum.
__device__ __forceinline__ uint32_t quant_block_oct(const float (&x)[4], uint16_t &dbits,
                                                    int &bsum) {
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) a = fmaxf(a, fabsf(x[k]));  // NaN ignored
    const float amax = oct_max(a);
    const float d = __fdiv_rn(amax, 127.0f);
    dbits = f2h(d);
    const float inv = (d == 0.0f) ? 0.0f : __fdiv_rn(1.0f, d);
    uint32_t packed = 0;
    int sum = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float y = __fmul_rn(x[k], inv);
        int q;
        if (!(fabsf(y) <= 3.0e38f)) {
            q = -127;
        } else {
            q = (int)rintf(fminf(fmaxf(y, -200.0f), 200.0f));
            q = q > 127 ? 127 : (q < -127 ? -127 : q);
        }
        sum += q;
        packed |= (uint32_t)(q & 0xff) << (8 * k);
    }
    bsum = oct_sum(sum);
    return packed;
}

// quantize_q8 of one 32-value block held as 16 values in lane l and 16 in
// lane l ^ 32 (the two halves of a 32x32 MFMA output column), with exactly
// quant_block_lane's rules.  q[k] receives the lane's int8 values; every
// lane of the pair gets the fp16 scale bits and the block sum.
__device__ __forceinline__ void quant_block_pair16(const float (&x)[16], int (&q)[16],
                                                   uint16_t &dbits, int &bsum) {
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) a = fmaxf(a, fabsf(x[k]));  // NaN ignored
    const float amax = fmaxf(a, swap32_f(a));
    const float d = __fdiv_rn(amax, 127.0f);
    dbits = f2h(d);
    const float inv = (d == 0.0f) ? 0.0f : __fdiv_rn(1.0f, d);
    int sum = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const float y = __fmul_rn(x[k], inv);
        int v;
        if (!(fabsf(y) <= 3.0e38f)) {
            v = -127;
        } else {
            v = (int)rintf(fminf(fmaxf(y, -200.0f), 200.0f));
            v = v > 127 ? 127 : (v < -127 ? -127 : v);
        }
        q[k] = v;
        sum += v;
    }
    bsum = sum + swap32_i(sum);
}

// Scale layout of a repacked Q4_0 matrix (n rows, nb blocks per row): tiles
// of `tile` rows (a power of two), tile-major, so the scales of the rows a
// mat-vec workgroup owns are one contiguous run per block:
//   index(row, b) = (row / tile) * nb * tile + b * tile + row % tile.
// The array holds round_up(n, tile) * nb entries.
__host__ __device__ __forceinline__ size_t q4_scale_index(int row, int b, int nb, int tile) {
    return (size_t)(row / tile) * nb * tile + (size_t)b * tile + (row % tile);
}
__host__ __device__ __forceinline__ size_t q4_scale_count(int n, int nb, int tile) {
    return (size_t)((n + tile - 1) / tile) * tile * nb;
}

// Buffer descriptor of `bytes` bytes at p (raw buffer: a load whose offset
// lies at or past the end returns zero without a memory access, instead of
// faulting).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes,
                                             0x00020000);
}

// Signed 8-bit 4-way dot product with int32 accumulate (v_dot4_i32_i8).
__device__ __forceinline__ int sdot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// e2m3 codes of v / 2 for four 4-bit values n, one per byte (each value's
// half is an e2m3 number: 0.5 subnormal, 1..7.5 normal): unsigned, v = n
// (0..15), or two's complement, v = n - 16 for n >= 8 (-8..7), sign in bit 5.
// Two byte lookups (v_perm) from 8-entry tables and a select on bit 3.
__device__ __forceinline__ uint32_t f6_codes4(uint32_t n, bool sgn) {
    const uint32_t t0 = 0x0c080400u, t1 = 0x16141210u;   // v = 0..3, 4..7
    const uint32_t u0 = sgn ? 0x32343638u : 0x1b1a1918u;  // n = 8..11
    const uint32_t u1 = sgn ? 0x24282c30u : 0x1f1e1d1cu;  // n = 12..15
    const uint32_t idx = n & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, idx), hi = __builtin_amdgcn_perm(u1, u0, idx);
    const uint32_t m = ((n >> 3) & 0x01010101u) * 0xffu;
    return (hi & m) | (lo & ~m);
}

// four codes (bytes of c, each < 64) -> 24 bits, code k at bit 6 k
__device__ __forceinline__ uint32_t f6_pack4(uint32_t c) {
    return (c & 0x3fu) | ((c >> 2) & 0xfc0u) | ((c >> 4) & 0x3f000u) | ((c >> 6) & 0xfc0000u);
}

// The fp6 GEMM's activation codes (launch_q8_to_x6's layout: per block blk
// the region of the hi codes then that of the lo codes, each of m rows as
// [m][16 B] then [m][8 B]) written by an 8-lane group holding one Q8 block of
// row row, lane t = lane & 7 with its values 4t..4t+3 as the bytes of q: the
// lane's four hi (lo) codes are 24 bits, and lanes 0-2 and 4-6 each complete
// one dword with the next lane's bits (every lane of the group active).
__device__ __forceinline__ void f6_store_oct(uint32_t q, uint8_t *x6, int m, int row, int blk) {
    const int t = threadIdx.x & 7, tq = t & 3;
    const uint32_t ph = f6_pack4(f6_codes4((q >> 4) & 0x0f0f0f0fu, true));
    const uint32_t pl = f6_pack4(f6_codes4(q & 0x0f0f0f0fu, false));
    const uint32_t nh = (uint32_t)dpp_i<DPP_SHL1>((int)ph), nl = (uint32_t)dpp_i<DPP_SHL1>((int)pl);
    if (tq == 3) return;  // lanes 3 and 7 start no dword
    uint8_t *rh = x6 + (size_t)(2 * blk) * m * 24, *rl = rh + (size_t)m * 24;
    const int k = t - (t >> 2);  // dword k of the row's 24 bytes
    const size_t o = k < 4 ? (size_t)row * 16 + 4 * k : (size_t)m * 16 + (size_t)row * 8 + 4 * (k - 4);
    *(uint32_t *)(rh + o) = (ph >> (8 * tq)) | (nh << (24 - 8 * tq));
    *(uint32_t *)(rl + o) = (pl >> (8 * tq)) | (nl << (24 - 8 * tq));
}

}  // namespace si
