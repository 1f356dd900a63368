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

// Wave reductions through DPP: within each row of 16 lanes a quad swap, a pair swap and two rotations leave every
// lane with its row's result; the four rows are then combined from one lane each. Every lane must be active.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t) __builtin_amdgcn_update_dpp(0, (int) v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ uint32_t lane_u32(uint32_t v, int l) { return (uint32_t) __builtin_amdgcn_readlane((int) v, l); }

template <typename Op>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v, Op op) {
    v = op(v, dpp_u32<0xB1>(v));   // quad_perm [1,0,3,2]
    v = op(v, dpp_u32<0x4E>(v));   // quad_perm [2,3,0,1]
    v = op(v, dpp_u32<0x124>(v));  // row_ror:4
    v = op(v, dpp_u32<0x128>(v));  // row_ror:8
    return op(op(lane_u32(v, 0), lane_u32(v, 16)), op(lane_u32(v, 32), lane_u32(v, 48)));
}
template <typename Op>
__device__ __forceinline__ uint64_t wave_reduce_u64(uint64_t v, Op op) {
    auto step = [&](uint64_t a, uint32_t lo, uint32_t hi) { return op(a, ((uint64_t) hi << 32) | lo); };
    v = step(v, dpp_u32<0xB1>((uint32_t) v), dpp_u32<0xB1>((uint32_t) (v >> 32)));
    v = step(v, dpp_u32<0x4E>((uint32_t) v), dpp_u32<0x4E>((uint32_t) (v >> 32)));
    v = step(v, dpp_u32<0x124>((uint32_t) v), dpp_u32<0x124>((uint32_t) (v >> 32)));
    v = step(v, dpp_u32<0x128>((uint32_t) v), dpp_u32<0x128>((uint32_t) (v >> 32)));
    auto at = [&](int l) { return ((uint64_t) lane_u32((uint32_t) (v >> 32), l) << 32) | lane_u32((uint32_t) v, l); };
    return op(op(at(0), at(16)), op(at(32), at(48)));
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    return wave_reduce_u64(v, [](uint64_t a, uint64_t b) { return a > b ? a : b; });
}
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
    return wave_reduce_u64(v, [](uint64_t a, uint64_t b) { return a < b ? a : b; });
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    return wave_reduce_u32(v, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    return wave_reduce_u32(v, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}
__device__ __forceinline__ int wave_sum_i32(int v) {
    return (int) wave_reduce_u32((uint32_t) v, [](uint32_t a, uint32_t b) { return a + b; });
}
__device__ __forceinline__ uint32_t wave_or_u32(uint32_t v) {
    return wave_reduce_u32(v, [](uint32_t a, uint32_t b) { return a | b; });
}
// The largest of the lanes' floats (no NaN among them).
__device__ __forceinline__ float wave_max_f32(float v) {
    return __uint_as_float(wave_reduce_u32(__float_as_uint(v), [](uint32_t a, uint32_t b) {
        return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
    }));
}
__device__ __forceinline__ double wave_sum_f64(double v) {
    const uint64_t r = wave_reduce_u64((uint64_t) __double_as_longlong(v), [](uint64_t a, uint64_t b) {
        return (uint64_t) __double_as_longlong(__longlong_as_double((long long) a) + __longlong_as_double((long long) b));
    });
    return __longlong_as_double((long long) r);
}

// A double moved by one DPP control, each 32-bit half on its own (0.0 where no lane feeds it).
template <int CTRL, int ROWS, bool BOUND>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t u = (uint64_t) __double_as_longlong(v);
    const uint32_t lo = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) (uint32_t) u, CTRL, ROWS, 0xf, BOUND);
    const uint32_t hi = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) (uint32_t) (u >> 32), CTRL, ROWS, 0xf, BOUND);
    return __longlong_as_double((long long) (((uint64_t) hi << 32) | lo));
}
// Inclusive prefix sum of doubles over the wave's lanes through DPP, in the order of wave_incl_scan_i32 (every lane
// active).
__device__ __forceinline__ double wave_incl_scan_f64(double v) {
    v += dpp_f64<0x111, 0xf, true>(v);   // row_shr:1
    v += dpp_f64<0x112, 0xf, true>(v);   // row_shr:2
    v += dpp_f64<0x114, 0xf, true>(v);   // row_shr:4
    v += dpp_f64<0x118, 0xf, true>(v);   // row_shr:8
    v += dpp_f64<0x142, 0xa, false>(v);  // row_bcast:15
    v += dpp_f64<0x143, 0xc, false>(v);  // row_bcast:31
    return v;
}
// Inclusive prefix sum of ints over the wave's lanes through DPP (every lane active).
__device__ __forceinline__ int wave_incl_scan_i32(int v) {
    // within each row of 16 lanes by shifts, then rows 1 and 3 add lane 15 of the row before, rows 2 and 3 lane 31
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false); // row_bcast:15
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false); // row_bcast:31
    return v;
}

}  // namespace spx
