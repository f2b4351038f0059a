// si_handoff.hip -- TEST-ONLY measurement (executable tests/probe/si_handoff):
// what a hand-off of data between the workgroups of ONE launch costs on this
// GPU, against a kernel boundary in a HIP graph.  It is the evidence behind
// keeping the single-token decode layer as a chain of kernels instead of
// one launch whose phases wait for each other.
//
// A launch holds NPH phases of workgroups (512 threads), all co-resident;
// phase p waits until every workgroup of phase p-1 has written its output
// (`per` floats each), reads either one producer's output or all of them,
// then writes its own.  Protocols:
//   counters: a device-scope atomic counter per phase (release add by the
//     producer, acquire loads by the consumer), the last workgroup to finish
//     resets them;
//   flags: every workgroup owns a generation word; launch k raises each to
//     k + 1 exactly once; consumers poll their producers' words; data moves
//     with device-scope (sc1) stores and loads, no cache write-back.
// against the same phases as NPH kernels in one HIP graph.  Every wait is
// bounded (1 s of the 100 MHz constant clock); a timeout is counted and
// reported, and the kernel still ends.  Prints one JSON line per setup.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>

#define CK(x)                                                                          \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
            exit(1);                                                                   \
        }                                                                              \
    } while (0)

constexpr int T = 512, NPH = 4;
struct Cfg {
    int n[NPH], off[NPH + 1];
};
constexpr long LIMIT = 100000000;  // 1 s at 100 MHz

__device__ __forceinline__ int phase_of(const Cfg &c, int b) {
    int p = 0;
    while (p + 1 < NPH && b >= c.off[p + 1]) ++p;
    return p;
}

// the consumer's read: one producer's output (the first `per` floats of
// producer i % n) or all of them
template <bool SC1>
__device__ float consume(const Cfg &c, int p, int i, const float *buf, int per, int all) {
    const float *src = buf + (size_t)(p - 1) * 4096 * per;
    const int cnt = all ? c.n[p - 1] * per : per;
    if (!all) src += (size_t)(i % c.n[p - 1]) * per;
    float acc = 0.0f;
    for (int j = threadIdx.x; j < cnt; j += T)
        acc += SC1 ? __hip_atomic_load((float *)src + j, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT)
                   : src[j];
    return acc;
}

__global__ void __launch_bounds__(T) k_counters(Cfg c, int *ctr, float *buf, int per, int all,
                                                int *err) {
    const int b = blockIdx.x, p = phase_of(c, b), i = b - c.off[p];
    float acc = 0.0f;
    if (p > 0) {
        if (threadIdx.x == 0) {
            const long t0 = __builtin_amdgcn_s_memrealtime();
            while (__hip_atomic_load(&ctr[p - 1], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) <
                   c.n[p - 1]) {
                if (__builtin_amdgcn_s_memrealtime() - t0 > LIMIT) {
                    atomicAdd(err, 1);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        __syncthreads();
        acc = consume<false>(c, p, i, buf, per, all);
    }
    float *dst = buf + (size_t)p * 4096 * per + (size_t)i * per;
    for (int j = threadIdx.x; j < per; j += T) dst[j] = acc + j;
    __syncthreads();
    if (threadIdx.x == 0) {
        __hip_atomic_fetch_add(&ctr[p], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        if (__hip_atomic_fetch_add(&ctr[NPH], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            c.off[NPH] - 1)
            for (int q = 0; q <= NPH; ++q)
                __hip_atomic_store(&ctr[q], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

__global__ void __launch_bounds__(T) k_flags(Cfg c, unsigned *flag, float *buf, int per, int all,
                                             int *err) {
    const int b = blockIdx.x, p = phase_of(c, b), i = b - c.off[p];
    __shared__ unsigned gen_s;
    if (threadIdx.x == 0)
        gen_s = __hip_atomic_load(flag + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
    __syncthreads();
    const unsigned gen = gen_s;
    float acc = 0.0f;
    if (p > 0) {
        if (threadIdx.x < 64) {  // one wavefront polls the producers' words
            const unsigned *pf = flag + c.off[p - 1];
            const long t0 = __builtin_amdgcn_s_memrealtime();
            while (true) {
                bool ok = true;
                for (int j = threadIdx.x; j < c.n[p - 1]; j += 64)
                    ok = ok && (int)(__hip_atomic_load((unsigned *)pf + j, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT) - gen) >= 0;
                if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
                if (__builtin_amdgcn_s_memrealtime() - t0 > LIMIT) {
                    if (threadIdx.x == 0) atomicAdd(err, 1);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        __syncthreads();
        acc = consume<true>(c, p, i, buf, per, all);
    }
    float *dst = buf + (size_t)p * 4096 * per + (size_t)i * per;
    for (int j = threadIdx.x; j < per; j += T)
        __hip_atomic_store(dst + j, acc + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's stores are performed
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_store(flag + b, gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// one phase as its own kernel
__global__ void __launch_bounds__(T) k_phase(Cfg c, int p, float *buf, int per, int all) {
    const int i = blockIdx.x;
    const float acc = p > 0 ? consume<false>(c, p, i, buf, per, all) : 0.0f;
    float *dst = buf + (size_t)p * 4096 * per + (size_t)i * per;
    for (int j = threadIdx.x; j < per; j += T) dst[j] = acc + j;
}

int main(int argc, char **argv) {
    // setups: phases, floats per workgroup, read all producers
    const struct {
        int n[NPH], per, all;
    } setups[] = {{{224, 112, 152, 112}, 16, 0},  // the 0.5B decode layer's grids
                  {{16, 16, 16, 16}, 16, 0},
                  {{224, 112, 152, 112}, 64, 1}};
    const int reps = argc > 1 ? atoi(argv[1]) : 200;
    hipStream_t st;
    CK(hipStreamCreate(&st));
    int *ctr, *err;
    unsigned *flag;
    float *buf;
    CK(hipMalloc(&ctr, 64));
    CK(hipMalloc(&err, 4));
    CK(hipMalloc(&flag, 4096 * sizeof(unsigned)));
    CK(hipMalloc(&buf, (size_t)NPH * 4096 * 64 * sizeof(float)));
    for (const auto &su : setups) {
        Cfg c;
        c.off[0] = 0;
        for (int q = 0; q < NPH; ++q) {
            c.n[q] = su.n[q];
            c.off[q + 1] = c.off[q] + su.n[q];
        }
        const int tot = c.off[NPH];
        CK(hipMemset(ctr, 0, 64));
        CK(hipMemset(err, 0, 4));
        CK(hipMemset(flag, 0, 4096 * sizeof(unsigned)));
        int occ = 0, ncu = 0;
        CK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_flags, T, 0));
        CK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, 0));
        if (occ * ncu < tot) {
            fprintf(stderr, "%d workgroups do not fit %d x %d co-resident\n", tot, occ, ncu);
            return 1;
        }
        auto time_graph = [&](auto body) {
            hipGraph_t g;
            hipGraphExec_t ge;
            CK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
            for (int r = 0; r < reps; ++r) body();
            CK(hipStreamEndCapture(st, &g));
            CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
            hipEvent_t a, b;
            CK(hipEventCreate(&a));
            CK(hipEventCreate(&b));
            CK(hipGraphLaunch(ge, st));
            CK(hipStreamSynchronize(st));
            float best = 1e30f;
            for (int t = 0; t < 5; ++t) {
                CK(hipEventRecord(a, st));
                CK(hipGraphLaunch(ge, st));
                CK(hipEventRecord(b, st));
                CK(hipEventSynchronize(b));
                float ms;
                CK(hipEventElapsedTime(&ms, a, b));
                if (ms < best) best = ms;
            }
            CK(hipGraphExecDestroy(ge));
            CK(hipGraphDestroy(g));
            return best * 1000.0f / reps;  // us per step
        };
        const float us_kernels = time_graph([&] {
            for (int q = 0; q < NPH; ++q)
                hipLaunchKernelGGL(k_phase, dim3(su.n[q]), dim3(T), 0, st, c, q, buf, su.per,
                                   su.all);
        });
        const float us_counters = time_graph([&] {
            hipLaunchKernelGGL(k_counters, dim3(tot), dim3(T), 0, st, c, ctr, buf, su.per, su.all,
                               err);
        });
        const float us_flags = time_graph([&] {
            hipLaunchKernelGGL(k_flags, dim3(tot), dim3(T), 0, st, c, flag, buf, su.per, su.all,
                               err);
        });
        int e = 0, ctr_after[NPH + 1];
        unsigned f0 = 0, flast = 0;
        CK(hipMemcpy(&e, err, 4, hipMemcpyDeviceToHost));
        CK(hipMemcpy(ctr_after, ctr, sizeof ctr_after, hipMemcpyDeviceToHost));
        CK(hipMemcpy(&f0, flag, 4, hipMemcpyDeviceToHost));
        CK(hipMemcpy(&flast, flag + tot - 1, 4, hipMemcpyDeviceToHost));
        int ctr_sum = 0;
        for (int q = 0; q <= NPH; ++q) ctr_sum += ctr_after[q];
        printf("{\"phases\": [%d, %d, %d, %d], \"floats_per_workgroup\": %d, "
               "\"read_all_producers\": %d, \"us_four_kernels\": %.3f, "
               "\"us_one_launch_counters\": %.3f, \"us_one_launch_flags\": %.3f, "
               "\"timeouts\": %d, \"counters_left\": %d, \"flag_generations\": [%u, %u], "
               "\"launches_per_protocol\": %d}\n",
               su.n[0], su.n[1], su.n[2], su.n[3], su.per, su.all, us_kernels, us_counters,
               us_flags, e, ctr_sum, f0, flast, 6 * reps);
        fflush(stdout);
    }
    return 0;
}
