// spx_noalloc.hip — spx_sample_rows_noalloc: the sampling call over a workspace in static device memory, for callers
// that cannot allocate. The array `scratch` holds the workspace of kStaticRows rows; its device address is taken
// once per device (hipGetSymbolAddress, with the device current) and kept in that device's slot, and only that
// address reaches kernels. The kernels are spx_sample_rows's, through a handle of static storage bound to it.

#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/spx_sampler.h"
#include "spx_internal.h"
#include "spx_plan.h"

namespace {

constexpr size_t kScratchBytes = spx::workspace_bytes(spx::kStaticRows, false);

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

struct Slot {
    std::mutex lock;  // orders the host side of calls on the device (the handle's call parity)
    bool ready = false;
    void * ptr = nullptr;  // the device's copy of scratch
    spx_sampler * handle = nullptr;
};
Slot g_slots[spx::kMaxDevices];

// Zeroes the array at set-up: the rows' arrival counters and the resolving list's counts start at zero (each call
// leaves them at zero again), and a kernel rather than a memset, so that no memset node is ever queued.
__global__ void zero_kernel(uint4 * p, size_t n) {
    for (size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t) gridDim.x * blockDim.x)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

}  // namespace

extern "C" spx_status spx_sample_rows_noalloc(const void * d_logits, int dtype, int rows, int vocab, int64_t ld,
                                              const int32_t * d_hist, const int32_t * d_hist_off, int max_hist,
                                              const uint32_t * d_banned, int64_t banned_stride,
                                              const spx_row_params * d_params, const double * d_u, int32_t * d_out_ids,
                                              int32_t * d_out_status, int32_t * d_out_kept, int32_t * d_out_cand_ids,
                                              double * d_out_cand_weights, int max_out, void * stream) {
    if (rows < 0 || rows > spx::kStaticRows) return spx::report(SPX_ERR_INVALID_ARGUMENT, "rows outside [0, SPX_NOALLOC_MAX_ROWS]");
    if (vocab <= 0 || max_hist < 0 || max_out < 0 || max_out > spx::kKeep) return spx::report(SPX_ERR_INVALID_ARGUMENT, "vocab, max_hist or max_out out of range");
    if (d_out_cand_ids && max_out == 0) return spx::report(SPX_ERR_INVALID_ARGUMENT, "candidate outputs with max_out 0");
    if (spx::lds_bound(vocab, max_hist) > spx::kLdsMax) return spx::report(SPX_ERR_INVALID_ARGUMENT, "vocab and max_hist need more LDS than a CU holds");
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return spx::report_hip(e, "hipGetDevice");
    if (device < 0 || device >= spx::kMaxDevices) return spx::report(SPX_ERR_INVALID_ARGUMENT, "device index above the no-alloc entry's table");
    Slot & slot = g_slots[device];
    std::lock_guard<std::mutex> guard(slot.lock);
    if (!slot.ready) {
        void * ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return spx::report_hip(e, "hipGetSymbolAddress");
        hipLaunchKernelGGL(zero_kernel, dim3(1024), dim3(256), 0, (hipStream_t) stream, (uint4 *) ptr, kScratchBytes / 16);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t) stream);
        if (e != hipSuccess) return spx::report_hip(e, "zeroing the no-alloc workspace");
        spx_sampler * h = nullptr;
        const spx_status st = spx::bind_scratch(device, ptr, spx::kStaticRows, &h);
        if (st != SPX_OK) return st;
        slot.ptr = ptr;
        slot.handle = h;
        slot.ready = true;
    }
    spx::set_call_limits(slot.handle, vocab, max_hist, max_out);
    return spx_sample_rows(slot.handle, d_logits, dtype, rows, vocab, ld, d_hist, d_hist_off, d_banned, banned_stride,
                           d_params, d_u, d_out_ids, d_out_status, d_out_kept, d_out_cand_ids, d_out_cand_weights,
                           stream);
}
