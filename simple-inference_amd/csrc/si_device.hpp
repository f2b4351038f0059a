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
// Cross-lane reductions inside a 32-lane half wavefront (one Q8 block).
// ---------------------------------------------------------------------
__device__ __forceinline__ float half_wave_max(float v) {
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 32));
    return v;
}

__device__ __forceinline__ int half_wave_sum(int v) {
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) v += __shfl_xor(v, o, 32);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
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

// Signed 8-bit 4-way dot product with int32 accumulate (v_dot4_i32_i8).
__device__ __forceinline__ int sdot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

}  // namespace si
