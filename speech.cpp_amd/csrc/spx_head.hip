// spx_head.hip — the LM head's pick fused with its product (src/common/qwen3-decoder.cpp:422-429, `outputs()` with
// Qwen3Readback::Pick, and :497-501, `verify()`): each row's hidden state RMS-normalized and scaled by the norm weight,
// multiplied by the head's bf16 weights on the matrix cores, and the first largest logit taken, without the logits
// ever reaching memory.
//
// Three launches: the rows' normalized hidden states as bf16 (the operand type of the head's bf16 product, as ggml's
// bf16 matrix product converts them), with each row's pick key cleared; the product, each wave a 32-token tile of the
// vocabulary against up to 64 rows (two 32 x 32 MFMA accumulators) over the hidden size in blocks of 16, keeping its
// best per row, one atomic max per row per work-group; the ids from the keys.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/spx_sampler.h"
#include "spx_internal.h"

namespace spx {

namespace {

typedef short bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kHeadThreads = 256;
constexpr int kHeadWaves = kHeadThreads / 64;
constexpr int kTileM = 32;  // vocabulary rows of a wave's tile (the MFMA's M)

// float to bf16, round to nearest even (NaN kept a NaN)
__device__ __forceinline__ uint16_t to_bf16(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t) ((u >> 16) | 0x40u);
    return (uint16_t) ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// The pick's order as one integer: NaN above everything (torch.argmax, which the reference's ggml argmax follows),
// then by value, equal values to the lower id.
__device__ __forceinline__ uint64_t pick_key(float v, uint32_t id) {
    uint32_t k;
    if (v != v) k = 0xffffffffu;
    else {
        const uint32_t u = __float_as_uint(v);
        k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    }
    return ((uint64_t) k << 32) | (uint64_t) (~id);
}

// ggml's rms_norm (a double sum of squares, the mean cast to float, scale = 1 / sqrtf(mean + eps)), times the norm
// weight, as bf16; one work-group per row.
__global__ __launch_bounds__(256) void head_prep_kernel(const float * hidden, int64_t ld, const float * w, float eps,
                                                        int d, uint16_t * hn, uint64_t * keys) {
    __shared__ double part[4];
    const int r = blockIdx.x, tid = threadIdx.x;
    const float * x = hidden + (int64_t) r * ld;
    double s = 0.0;
    for (int k = tid; k < d; k += 256) s += (double) x[k] * (double) x[k];
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if ((tid & 63) == 0) part[tid >> 6] = s;
    __syncthreads();
    const double sum = (part[0] + part[1]) + (part[2] + part[3]);
    const float mean = (float) (sum / (double) d);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int k = tid; k < d; k += 256) {
        const float y = x[k] * scale;
        hn[(int64_t) r * d + k] = to_bf16(w ? y * w[k] : y);
    }
    if (tid == 0) keys[r] = 0ull;
}

// The product and the pick. hn: rows x d bf16 (d a multiple of 64), head: vocab rows of ld bf16, 16-byte aligned.
// COLS: 32-row column tiles (1 for up to 32 rows, 2 for up to 64). Each wave takes a 32-token tile of the vocabulary;
// the work-group's four waves share the hidden rows' blocks of 64, which its threads bring into LDS a turn ahead, so
// that a wave's loads from memory are its tile's only.
template <int COLS>
__global__ __launch_bounds__(kHeadThreads) void head_pick_kernel(const uint16_t * head, int64_t ld, const uint16_t * hn,
                                                                 int rows, int d, int vocab, uint64_t * keys) {
    constexpr int kPitch = 9;  // 16-byte words per hidden row in LDS (8 used; the ninth spreads the rows over banks)
    __shared__ uint4 bs[2][64 * kPitch];
    __shared__ uint64_t wbest[kHeadWaves][64];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int m = lane & 31, half = lane >> 5;
    const int tiles = (vocab + kTileM - 1) / kTileM;
    const int t = blockIdx.x * kHeadWaves + wave;  // this wave's tile (past the last: it only helps with the loads)
    const int v0 = t * kTileM;
    // tokens past the vocabulary read its last row, hidden rows past the batch the batch's last (every load in
    // bounds); their products are never taken
    const uint4 * __restrict__ ap = (const uint4 *) (head + (int64_t) min(v0 + m, vocab - 1) * ld);
    // the work-group's share of a turn's hidden blocks: 64 rows x 8 words, two words a thread
    const int e0 = tid, e1 = tid + kHeadThreads;
    const uint4 * __restrict__ hp0 = (const uint4 *) (hn + (int64_t) min(e0 >> 3, rows - 1) * d) + (e0 & 7);
    const uint4 * __restrict__ hp1 = (const uint4 *) (hn + (int64_t) min(e1 >> 3, rows - 1) * d) + (e1 & 7);
    f32x16 acc0 = {}, acc1 = {};
    auto mac = [&](const uint4 & a, const uint4 & b, const uint4 & c) __attribute__((always_inline)) {
        const bf16x4 alo = __builtin_bit_cast(bf16x4, make_uint2(a.x, a.y));
        const bf16x4 ahi = __builtin_bit_cast(bf16x4, make_uint2(a.z, a.w));
        acc0 = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(alo, __builtin_bit_cast(bf16x4, make_uint2(b.x, b.y)), acc0, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(ahi, __builtin_bit_cast(bf16x4, make_uint2(b.z, b.w)), acc0, 0, 0, 0);
        if (COLS > 1) {
            acc1 = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(alo, __builtin_bit_cast(bf16x4, make_uint2(c.x, c.y)), acc1, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(ahi, __builtin_bit_cast(bf16x4, make_uint2(c.z, c.w)), acc1, 0, 0, 0);
        }
    };
    // Turns of 64: lane (m, half) holds elements 16*j + 8*half .. +7 of its rows for j < 4, the first four of each to
    // one MFMA and the last four to the next (the same split on both operands, so each product pairs the same k).
    // Turn k computes from its LDS buffer k % 2 with the tile's words loaded a turn ahead; the hidden blocks of turn
    // k + 1, loaded a turn ahead too, go to the other buffer meanwhile. Loads go only to the `n` registers, and the
    // first pass (k = -1) only issues them and fills buffer 0, so no register in use has a load pending on it.
    const int turns = d >> 6;
    uint4 na[4], nh0, nh1;
#pragma unroll
    for (int j = 0; j < 4; j++) na[j] = make_uint4(0u, 0u, 0u, 0u);
    nh0 = nh1 = make_uint4(0u, 0u, 0u, 0u);
    for (int k = -1; k < turns; k++) {
        uint4 a[4];
#pragma unroll
        for (int j = 0; j < 4; j++) a[j] = na[j];
        const uint4 h0 = nh0, h1 = nh1;  // turn k + 1's hidden blocks (k >= 0)
        if (k + 1 < turns) {
            const int q = (k + 1) * 8;  // turn k + 1's first 16-byte word of a row
#pragma unroll
            for (int j = 0; j < 4; j++) na[j] = ap[q + 2 * j + half];
        }
        if (k + 2 < turns) {
            nh0 = hp0[(k + 2) * 8];
            nh1 = hp1[(k + 2) * 8];
        }
        if (k >= 0) {
            const uint4 * b = bs[k & 1];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint4 b0 = b[m * kPitch + 2 * j + half];
                const uint4 b1 = COLS > 1 ? b[(32 + m) * kPitch + 2 * j + half] : b0;
                mac(a[j], b0, b1);
            }
        }
        if (k == -1) {
            bs[0][(e0 >> 3) * kPitch + (e0 & 7)] = hp0[0];
            bs[0][(e1 >> 3) * kPitch + (e1 & 7)] = hp1[0];
        } else if (k + 1 < turns) {
            uint4 * bn = bs[(k + 1) & 1];  // last read by turn k - 1, before the barrier that ended it
            bn[(e0 >> 3) * kPitch + (e0 & 7)] = h0;
            bn[(e1 >> 3) * kPitch + (e1 & 7)] = h1;
        }
        __syncthreads();
    }
    uint64_t best0 = 0ull, best1 = 0ull;  // this lane's best of hidden rows m and 32 + m
    if (t < tiles) {
        // output i of lane (m, half): vocabulary row 8*(i/4) + 4*half + i%4 of the tile, hidden row m (of the tile)
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int v = v0 + 8 * (i >> 2) + 4 * half + (i & 3);
            if (v < vocab) {
                const uint64_t k0 = pick_key(acc0[i], (uint32_t) v);
                best0 = k0 > best0 ? k0 : best0;
                if (COLS > 1) {
                    const uint64_t k1 = pick_key(acc1[i], (uint32_t) v);
                    best1 = k1 > best1 ? k1 : best1;
                }
            }
        }
    }
    // the two halves of the wave hold other vocabulary rows of the same hidden rows
    {
        const uint64_t o0 = __shfl_xor(best0, 32), o1 = __shfl_xor(best1, 32);
        best0 = o0 > best0 ? o0 : best0;
        best1 = o1 > best1 ? o1 : best1;
    }
    if (half == 0) {
        wbest[wave][m] = best0;
        wbest[wave][32 + m] = best1;
    }
    __syncthreads();
    if (tid < rows) {
        uint64_t b = 0ull;
        for (int w = 0; w < kHeadWaves; w++) b = wbest[w][tid] > b ? wbest[w][tid] : b;
        if (b) atomicMax((unsigned long long *) &keys[tid], (unsigned long long) b);
    }
}

__global__ void head_ids_kernel(const uint64_t * keys, int rows, int32_t * ids, float * maxv) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const uint64_t k = keys[r];
    ids[r] = k ? (int32_t) ~(uint32_t) (k & 0xffffffffu) : -1;
    if (maxv) {
        const uint32_t h = (uint32_t) (k >> 32);
        const uint32_t u = h == 0xffffffffu ? 0x7fc00000u : ((h & 0x80000000u) ? (h & 0x7fffffffu) : ~h);
        maxv[r] = __uint_as_float(u);
    }
}

}  // namespace

hipError_t launch_head_pick(const HeadArgs & h, hipStream_t s) {
    if (h.rows == 0) return hipSuccess;
    hipLaunchKernelGGL(head_prep_kernel, dim3(h.rows), dim3(256), 0, s, h.hidden, h.hidden_ld, h.norm_w, h.eps, h.d,
                       h.hn, h.keys);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int tiles = (h.vocab + kTileM - 1) / kTileM;
    const int groups = (tiles + kHeadWaves - 1) / kHeadWaves;
    const dim3 grid(groups);
    if (h.rows > 32)
        hipLaunchKernelGGL(head_pick_kernel<2>, grid, dim3(kHeadThreads), 0, s, h.head, h.head_ld, h.hn, h.rows, h.d,
                           h.vocab, h.keys);
    else
        hipLaunchKernelGGL(head_pick_kernel<1>, grid, dim3(kHeadThreads), 0, s, h.head, h.head_ld, h.hn, h.rows, h.d,
                           h.vocab, h.keys);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(head_ids_kernel, dim3((h.rows + 63) / 64), dim3(64), 0, s, h.keys, h.rows, h.out_ids, h.out_max);
    return hipGetLastError();
}

}  // namespace spx
