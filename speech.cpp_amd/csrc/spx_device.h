// spx_device.h — device helpers of the gfx950 token sampler: ordered keys, the exact float quotient, wave-level
// reductions and scans. Wave64 only (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace spx {

constexpr int kWave = 64;

// A total order of non-NaN floats as unsigned ints: a < b  <=>  key(a) < key(b). -0 is taken as +0 first, so that the
// two zeros tie as they do under the reference's float comparisons. NaN gets no key (callers exclude it).
__device__ __forceinline__ uint32_t order_key(float f) {
    const uint32_t b = __float_as_uint(f + 0.0f);
    return b ^ ((uint32_t) ((int32_t) b >> 31) | 0x80000000u);
}

__device__ __forceinline__ float key_float(uint32_t k) {
    const uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(b);
}

// A candidate: its key in the high word and the complement of its id in the low word, so that a larger entry comes
// first in the order the reference's samplers sort by: falling logit, then rising id.
__device__ __forceinline__ uint64_t make_entry(uint32_t key, uint32_t id) {
    return ((uint64_t) key << 32) | (uint64_t) (~id);
}
__device__ __forceinline__ uint32_t entry_id(uint64_t e) { return ~(uint32_t) e; }
__device__ __forceinline__ uint32_t entry_key(uint64_t e) { return (uint32_t) (e >> 32); }
__device__ __forceinline__ float entry_value(uint64_t e) { return key_float(entry_key(e)); }

// x / t rounded to nearest, given r = 1/t rounded to nearest: Markstein's correction step, q = x*r, then
// q + (x - q*t)*r with the remainder exact by fma. It is correctly rounded wherever the quotient is a normal float
// clear of overflow; elsewhere (zero, subnormal, huge, non-finite) the IEEE division is taken.
__device__ __forceinline__ float div_rn(float x, float t, float r) {
    const float q0 = x * r;
    const float e = __builtin_fmaf(-q0, t, x);
    float q = __builtin_fmaf(e, r, q0);
    const float a = __builtin_fabsf(q0);
    if (__builtin_expect(!(a < 0x1p126f && a >= 0x1p-125f), 0)) q = x / t;
    return q;
}

__device__ __forceinline__ float bf16_to_float(uint16_t h) { return __uint_as_float((uint32_t) h << 16); }

__device__ __forceinline__ int lane_id() { return (int) __lane_id(); }

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

// Number of set bits of m below this lane.
__device__ __forceinline__ int lanes_below(uint64_t m) {
    return (int) __builtin_amdgcn_mbcnt_hi((uint32_t) (m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t) m, 0u));
}

template <typename T>
__device__ __forceinline__ T wave_shfl_xor(T v, int mask) {
    return __shfl_xor(v, mask, kWave);
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    for (int m = 32; m >= 1; m >>= 1) {
        const uint64_t o = __shfl_xor(v, m, kWave);
        v = o > v ? o : v;
    }
    return v;
}
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
    for (int m = 32; m >= 1; m >>= 1) {
        const uint64_t o = __shfl_xor(v, m, kWave);
        v = o < v ? o : v;
    }
    return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    for (int m = 32; m >= 1; m >>= 1) {
        const uint32_t o = __shfl_xor(v, m, kWave);
        v = o > v ? o : v;
    }
    return v;
}
__device__ __forceinline__ int wave_sum_i32(int v) {
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
    return v;
}
__device__ __forceinline__ uint32_t wave_or_u32(uint32_t v) {
    for (int m = 32; m >= 1; m >>= 1) v |= __shfl_xor(v, m, kWave);
    return v;
}
__device__ __forceinline__ double wave_sum_f64(double v) {
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
    return v;
}

// Inclusive prefix sum over the wave's lanes (Hillis-Steele with shuffles).
__device__ __forceinline__ double wave_incl_scan_f64(double v) {
    const int l = lane_id();
    for (int d = 1; d < kWave; d <<= 1) {
        const double o = __shfl_up(v, d, kWave);
        if (l >= d) v += o;
    }
    return v;
}
__device__ __forceinline__ int wave_incl_scan_i32(int v) {
    const int l = lane_id();
    for (int d = 1; d < kWave; d <<= 1) {
        const int o = __shfl_up(v, d, kWave);
        if (l >= d) v += o;
    }
    return v;
}

}  // namespace spx
