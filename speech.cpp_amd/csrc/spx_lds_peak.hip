// spx_lds_peak.hip — a measurement kernel, not part of the sampler: the LDS read bandwidth of the device, against
// which the benchmark rates the rows small enough to be held in LDS. Every lane reads 16-byte words of a 64 KiB LDS
// array (consecutive lanes, consecutive words: no bank conflicts), four a step, and folds them into registers it
// stores at the end, so that no read can be dropped.

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kThreads = 1024;
constexpr int kWords = 4096;  // 64 KiB of 16-byte words

__global__ __launch_bounds__(kThreads) void lds_read_kernel(uint4 * out, int steps) {
    __shared__ uint4 buf[kWords];
    const int tid = threadIdx.x;
    for (int i = tid; i < kWords; i += kThreads) buf[i] = make_uint4(i, 3 * i, 5 * i, 7 * i);
    __syncthreads();
    uint4 acc = make_uint4(0u, 0u, 0u, 0u);
    for (int s = 0; s < steps; s++) {
        // the base moves every step (the reads cannot be hoisted); the four words are 16 KiB apart (one offset each)
        const int base = (tid + s) & (kThreads - 1);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint4 v = buf[base + j * kThreads];
            acc.x ^= v.x;
            acc.y ^= v.y;
            acc.z ^= v.z;
            acc.w ^= v.w;
        }
    }
    out[(size_t) blockIdx.x * kThreads + tid] = acc;
}

}  // namespace

// The LDS read bandwidth in GB/s: `groups` work-groups of 1024 lanes, each lane reading 4 x 16 bytes a step for
// `steps` steps, timed with HIP events on the null stream (the median of `reps` launches after one untimed launch).
// Returns 0 on success, -1 on a HIP error.
extern "C" int spx_lds_peak(int groups, int steps, int reps, double * gbs) {
    uint4 * out = nullptr;
    if (groups <= 0 || steps <= 0 || reps <= 0 || reps > 64 || !gbs) return -1;
    if (hipMalloc(&out, (size_t) groups * kThreads * sizeof(uint4)) != hipSuccess) return -1;
    hipEvent_t a = nullptr, b = nullptr;
    hipError_t e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&b);
    float ms[64];
    if (e == hipSuccess) {
        hipLaunchKernelGGL(lds_read_kernel, dim3(groups), dim3(kThreads), 0, 0, out, steps);
        e = hipGetLastError();
    }
    for (int r = 0; r < reps && e == hipSuccess; r++) {
        e = hipEventRecord(a, 0);
        hipLaunchKernelGGL(lds_read_kernel, dim3(groups), dim3(kThreads), 0, 0, out, steps);
        if (e == hipSuccess) e = hipGetLastError();
        if (e == hipSuccess) e = hipEventRecord(b, 0);
        if (e == hipSuccess) e = hipEventSynchronize(b);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms[r], a, b);
    }
    if (a) (void) hipEventDestroy(a);
    if (b) (void) hipEventDestroy(b);
    (void) hipFree(out);
    if (e != hipSuccess) return -1;
    for (int i = 1; i < reps; i++)  // insertion sort, then the median
        for (int j = i; j > 0 && ms[j] < ms[j - 1]; j--) {
            const float t = ms[j];
            ms[j] = ms[j - 1];
            ms[j - 1] = t;
        }
    const double bytes = (double) groups * kThreads * steps * 4 * 16;
    *gbs = bytes / (ms[reps / 2] * 1e-3) / 1e9;
    return 0;
}
