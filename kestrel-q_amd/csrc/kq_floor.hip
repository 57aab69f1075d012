/*
 * kq_floor.hip — reference kernels for bench.py's floors (libkq_floor.so,
 * not part of the kq_hip library): what a launch costs with no work, and how
 * long a plain streaming read of a given size takes on this part. The
 * matvec workloads are compared with these at the same sizes.
 *
 *   floor_empty: a kernel with nothing in it, one workgroup per launch;
 *   floor_read<L>: each thread issues L 16-byte loads (all before any is
 *     used), folds them with xor and stores nothing unless the fold hits a
 *     fixed word, so every load stays. Threads read consecutive 16-byte
 *     words, L strides of the whole grid apart.
 * and a timing helper:
 *   hold: one wave that waits a given number of microseconds on the
 *     100 MHz constant clock (at most 10 ms, and at most 2^24 polls), so
 *     the host can enqueue a timed region behind it before it starts.
 */
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__global__ void floor_empty() {}

template <int L>
__global__ __launch_bounds__(512) void floor_read(const uint4 *__restrict__ p, uint64_t n16,
                                                  uint32_t *__restrict__ sink) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint4 v[L];
#pragma unroll
    for (int i = 0; i < L; ++i) {
        const uint64_t k = t + (uint64_t)i * stride;
        v[i] = k < n16 ? p[k] : make_uint4(0u, 0u, 0u, 0u);
    }
    uint32_t acc = 0u;
#pragma unroll
    for (int i = 0; i < L; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (acc == 0x9e3779b9u) sink[0] = acc;
}

__global__ void hold(uint64_t ticks) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (uint32_t i = 0; i < (1u << 24); ++i) {
        if (__builtin_amdgcn_s_memrealtime() - t0 >= ticks) break;
        __builtin_amdgcn_s_sleep(8);
    }
}

}  // namespace

/* the stream waits about `us` microseconds (clamped to 10 ms) */
extern "C" hipError_t kq_floor_hold(uint32_t us, hipStream_t s) {
    const uint64_t ticks = (uint64_t)(us > 10000u ? 10000u : us) * 100u; /* 100 MHz */
    hipLaunchKernelGGL(hold, dim3(1), dim3(64), 0, s, ticks);
    return hipGetLastError();
}

extern "C" hipError_t kq_floor_empty(hipStream_t s) {
    hipLaunchKernelGGL(floor_empty, dim3(1), dim3(64), 0, s);
    return hipGetLastError();
}

/* bytes rounded down to 16; loads_per_thread 1, 2, 4 or 8 */
extern "C" hipError_t kq_floor_read(const void *p, uint64_t bytes, int loads_per_thread,
                                    uint32_t *sink, hipStream_t s) {
    const uint64_t n16 = bytes / 16u;
    const uint64_t threads = (n16 + (uint64_t)loads_per_thread - 1u) / (uint64_t)loads_per_thread;
    const uint64_t blocks = (threads + 511u) / 512u;
    if (n16 == 0u || blocks > 0x7fffffffu) return hipErrorInvalidValue;
    const uint4 *q = (const uint4 *)p;
    switch (loads_per_thread) {
    case 1: hipLaunchKernelGGL(floor_read<1>, dim3(blocks), dim3(512), 0, s, q, n16, sink); break;
    case 2: hipLaunchKernelGGL(floor_read<2>, dim3(blocks), dim3(512), 0, s, q, n16, sink); break;
    case 4: hipLaunchKernelGGL(floor_read<4>, dim3(blocks), dim3(512), 0, s, q, n16, sink); break;
    case 8: hipLaunchKernelGGL(floor_read<8>, dim3(blocks), dim3(512), 0, s, q, n16, sink); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
