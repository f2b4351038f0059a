// si_stream.hip -- the streaming-read ceiling the kernels are measured
// against: one pass over a buffer with 16-byte loads, nothing else.
//
// Workgroup g reads the contiguous slice [g*len, (g+1)*len) of the buffer
// (len a multiple of 4 KB): each round, thread t issues DEPTH independent
// 16-byte loads at t*16 + j*4 KB (j < DEPTH), all in flight together, and
// folds them into one XOR; the workgroup writes one word, so no load can be
// dropped.  The achieved rate for a buffer of the size a kernel moves bounds
// what a single launch of that size reaches (launch ramp, tail and the HBM
// rate).
#include "si_device.hpp"
#include "si_kernels.hpp"

namespace si {

template <int DEPTH>
__global__ void __launch_bounds__(256) k_stream_read(const uint4 *__restrict__ src, size_t n16,
                                                     size_t per_wg16,
                                                     uint32_t *__restrict__ sink) {
    const size_t b0 = (size_t)blockIdx.x * per_wg16;
    const size_t b1 = b0 + per_wg16 < n16 ? b0 + per_wg16 : n16;
    uint32_t acc = 0;
    size_t i = b0 + threadIdx.x;
    for (; i + (DEPTH - 1) * 256 < b1; i += DEPTH * 256) {
        uint4 v[DEPTH];
#pragma unroll
        for (int j = 0; j < DEPTH; ++j) v[j] = src[i + j * 256];
#pragma unroll
        for (int j = 0; j < DEPTH; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    for (; i < b1; i += 256) {
        const uint4 a = src[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    __shared__ uint32_t red[4];
    for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

void launch_stream_read(const void *buf, size_t bytes, uint32_t *sink, int workgroups,
                        int depth, hipStream_t st) {
    const size_t n16 = bytes / 16;
    // whole 4 KB rounds per workgroup (the last slice takes the tail)
    size_t per = (n16 + workgroups - 1) / workgroups;
    per = (per + 255) / 256 * 256;
    const dim3 grid((unsigned)((n16 + per - 1) / per));
#define SR(D) \
    SI_LAUNCH(k_stream_read<D>, grid, dim3(256), 0, st, (const uint4 *)buf, n16, per, sink)
    if (depth <= 4) SR(4);
    else if (depth <= 8) SR(8);
    else SR(16);
#undef SR
}

}  // namespace si
