// si_probe.hip -- TEST-ONLY device probes (lib: tests/probe/libsi_probe.so).
//
// Not part of the product ABI (include/si_abi.h): these entry points run the
// product's own device helpers (src: simple-inference_amd/csrc/si_device.hpp)
// on test inputs, so the tests can pin the lane layouts and the conversions
// the hot-path kernels rely on.  Only tests/ loads this library.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../simple-inference_amd/csrc/si_device.hpp"
#include "si_probe.h"

using namespace si;

typedef _Float16 ph8 __attribute__((ext_vector_type(8)));
typedef _Float16 ph4 __attribute__((ext_vector_type(4)));
typedef float pf4 __attribute__((ext_vector_type(4)));

// Every lane feeds its index; out[k*64 + lane] is what lane received from
// cross-lane operation k (the helpers of si_device.hpp).
__global__ void __launch_bounds__(64) k_probe_lane_ops(int *__restrict__ out) {
    const int l = threadIdx.x;
    const float f = (float)l;
    out[0 * 64 + l] = dpp_i<DPP_XOR1>(l);
    out[1 * 64 + l] = dpp_i<DPP_XOR2>(l);
    out[2 * 64 + l] = dpp_i<DPP_ROR4>(l);
    out[3 * 64 + l] = dpp_i<DPP_ROR8>(l);
    out[4 * 64 + l] = dpp_i<DPP_HMIRROR>(l);
    out[5 * 64 + l] = swap16_i(l);
    out[6 * 64 + l] = swap32_i(l);
    out[7 * 64 + l] = oct_sum(l);
    out[8 * 64 + l] = half_wave_sum(l);
    out[9 * 64 + l] = (int)wave_sum(f);
    out[10 * 64 + l] = (int)half_wave_max(f);
    out[11 * 64 + l] = (int)wave_max(f);
    out[12 * 64 + l] = (int)oct_max(f);
    out[13 * 64 + l] = (int)fold_rows<4>(f);
    out[14 * 64 + l] = (int)fold_rows<8>(f);
    out[15 * 64 + l] = (int)fold_rows<16>(f);
    out[16 * 64 + l] = (int)fold_rows<32>(f);
    out[17 * 64 + l] = (int)wave_sum_d((double)l);
    out[18 * 64 + l] = dpp_i<DPP_SHL1>(l + 1);
}

// One 16x16 tile with each of the two f16 matrix-core shapes the attention
// kernels use, operands placed with the lane layouts those kernels assume,
// the output scattered back to row-major with the assumed output layout.
__global__ void k_probe_mfma_f16(const _Float16 *A, const _Float16 *B, float *D32, float *D16) {
    const int lane = threadIdx.x, col = lane & 15, grp = lane >> 4;
    ph8 a8, b8;
    for (int e = 0; e < 8; ++e) {
        a8[e] = A[col * 32 + 8 * grp + e];
        b8[e] = B[(8 * grp + e) * 16 + col];
    }
    pf4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a8, b8, (pf4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    for (int r = 0; r < 4; ++r) D32[(4 * grp + r) * 16 + col] = d[r];
    ph4 a4, b4;
    for (int e = 0; e < 4; ++e) {
        a4[e] = A[col * 32 + 4 * grp + e];
        b4[e] = B[(4 * grp + e) * 16 + col];
    }
    pf4 d2 = __builtin_amdgcn_mfma_f32_16x16x16f16(a4, b4, (pf4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    for (int r = 0; r < 4; ++r) D16[(4 * grp + r) * 16 + col] = d2[r];
}

// h2f (exact software widening) and h2f_fast (hardware widening) of every
// input half.
__global__ void k_probe_h2f(const uint16_t *__restrict__ h, float *__restrict__ exact,
                            float *__restrict__ fast, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    exact[i] = h2f(h[i]);
    fast[i] = h2f_fast(h[i]);
}

// f2h of the fp32 bit patterns start + i*stride (mod 2^32), i < n.
__global__ void k_probe_f2h_sweep(uint32_t start, uint32_t stride, size_t n,
                                  uint16_t *__restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[i] = f2h(u2f(start + (uint32_t)i * stride));
}

static int done() { return hipGetLastError() == hipSuccess ? 0 : 2; }

extern "C" {

int si_probe_lane_ops(int *out, void *stream) {
    if (!out) return 1;
    hipLaunchKernelGGL(k_probe_lane_ops, dim3(1), dim3(64), 0, (hipStream_t)stream, out);
    return done();
}

int si_probe_mfma_f16(const void *a, const void *b, float *d32, float *d16, void *stream) {
    if (!a || !b || !d32 || !d16) return 1;
    hipLaunchKernelGGL(k_probe_mfma_f16, dim3(1), dim3(64), 0, (hipStream_t)stream,
                       (const _Float16 *)a, (const _Float16 *)b, d32, d16);
    return done();
}

int si_probe_h2f(const uint16_t *h, float *exact, float *fast, size_t n, void *stream) {
    if (!n) return 0;
    if (!h || !exact || !fast || n > ((size_t)1 << 32)) return 1;
    hipLaunchKernelGGL(k_probe_h2f, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, h, exact, fast, n);
    return done();
}

int si_probe_f2h_sweep(uint32_t start, uint32_t stride, size_t n, uint16_t *out, void *stream) {
    if (!n) return 0;
    if (!out || n > ((size_t)1 << 32)) return 1;
    hipLaunchKernelGGL(k_probe_f2h_sweep, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, start, stride, n, out);
    return done();
}

}  // extern "C"
