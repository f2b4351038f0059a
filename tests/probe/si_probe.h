/*
 * si_probe.h -- TEST-ONLY probes of the device helpers the hot-path kernels
 * share (tests/probe/libsi_probe.so).  Not part of the product ABI: no
 * product code calls these, and they have no counterpart in the reference.
 * Each returns 0, 1 for a bad argument, 2 for a failed launch.
 */
#ifndef SI_PROBE_H
#define SI_PROBE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* Cross-lane moves (DPP quad_perm / row_ror / row_half_mirror / row_shl,
 * v_permlane16/32_swap) and the reductions built on them: each lane of one
 * wavefront feeds its index (row_shl: index + 1); out[k*64 + lane] (19 x 64
 * ints) is what lane received from operation k. */
int si_probe_lane_ops(int *out, void *stream);

/* fp16 matrix-core lane layouts: a [16][32] and b [32][16] fp16 (row-major)
 * -> d32 = a.b with the 16x16x32 shape and d16 = a[:, :16].b[:16, :] with the
 * 16x16x16 shape (fp32 [16][16] row-major). */
int si_probe_mfma_f16(const void *a, const void *b, float *d32, float *d16, void *stream);

/* The kernels' fp16 widening: exact[i] = h2f(h[i]) (software, every input),
 * fast[i] = h2f_fast(h[i]) (hardware conversion, used for finite cache
 * values).  Device buffers of n elements. */
int si_probe_h2f(const uint16_t *h, float *exact, float *fast, size_t n, void *stream);

/* The kernels' fp16 narrowing f2h of the fp32 bit patterns
 * start + i*stride (mod 2^32), i < n, into out (device). */
int si_probe_f2h_sweep(uint32_t start, uint32_t stride, size_t n, uint16_t *out, void *stream);

#ifdef __cplusplus
}
#endif
#endif
