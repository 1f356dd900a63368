// spx_kernel.h — the gfx950 kernel of the batched token sampler, included by one source file per variant (logit
// type x work-group size), so that the variants compile in parallel.
//
// One launch samples a batch. Each work-group takes one chunk of one row (a row is cut into `splits` chunks when the
// batch alone would not fill the CUs) and reads the chunk's logits once, 16 bytes per lane per load with the next
// step's loads in flight. Per step every lane holds 16 logits in registers and keeps, for the whole chunk:
//   - the exact quotient q = l/t of each logit (Markstein's correction step, correctly rounded like the reference's
//     float division), and the sum of exp(q - m) as one fma, one exp2 and one add per logit against 2^hi, hi an
//     integer exponent at or above m*log2(e), so that sums move between references by powers of two;
//   - every token whose quotient reaches the chunk's threshold tau, appended to one candidate buffer in LDS. tau
//     starts at a bound taken from the first step's lane maxima (at least K tokens lie above it) and rises from a
//     256-bin count of the appended quotients (an exact search of the buffer where the bins cannot bound it), so
//     appends become rare after the first steps;
//   - the special tokens (a penalized row's history and the banned ids) as a bitmap in LDS: they are masked to -inf
//     with two bit operations per logit, and a history token's raw logit is captured for the penalty stage, which
//     runs on the few hundred history tokens after the stream.
// A logit whose term is not finite (NaN, infinities, a quotient out of range) sends its group of 16 to an exact path
// that sets the flags the reference's checks read. After the stream the chunk's candidates at or above the final
// threshold are sorted and the row is finished by the flavor's rule (softmax weights in double, top-k/top-p, pick()
// with the row's uniform) - by the chunk itself, or by the last chunk of the row to arrive, which merges the others'.
// A row whose draw runs past the candidates held, or whose flags need every token, is resolved by the multi-pass path
// (exact radix selects over the whole row) in that same work-group.
//
// Citations are relative to the reference checkout (nyosegawa/speech.cpp 0.11.1).

#pragma once

#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "../../include/spx_sampler.h"
#include "spx_device.h"
#include "spx_internal.h"

namespace spx {

constexpr float kL2e = 1.4426950408889634f;  // log2(e), rounded to float
constexpr uint32_t kNegInfBits = 0xff800000u;

// ------------------------------------------------------------------------------------------------------------------
// Row plans
// ------------------------------------------------------------------------------------------------------------------

enum Mode : int { kGreedy = 0, kTopK = 1, kFull = 2, kInvalid = 3 };

enum Flag : uint32_t {
    kNaN = 1u,        // a NaN among the final logits
    kPosInf = 2u,     // a final logit is +inf
    kFinite = 4u,     // a final logit is finite
    kTempOver = 8u,   // a finite final logit whose quotient is not finite (src/families/haru/sampler.cpp:33-35)
    kNaN0 = 16u,      // the final logit of token 0 is NaN (std::max_element then answers 0)
    kNegInf = 32u,    // a final logit of a token that is not banned is -inf
    kBadHist = 64u,   // the row's history is longer than the handle was created for
    kTempOverPos = 128u,  // a finite final logit whose quotient is +inf (the largest quotient is then not finite)
};

struct Plan {
    int mode;
    int flavor;
    int k;        // the flavor's top-k count: the candidates the reference sorts
    int K;        // entries held at least: k for a top-k row, kKeepFull for a row drawing over more
    float t;      // the divisor of the flavor
    float rt;     // 1/t rounded
    float top_p;
    bool need_s;  // sum of exp over the whole vocabulary
    bool pen;     // penalties read the history
    bool counts;  // the frequency penalty: the history's counts
    bool xmin;    // greedy FISH: track the smallest raw logit (its -inf check)
    bool nanchk;  // greedy: look for NaN among the final logits
};

__device__ __forceinline__ bool neutral(const spx_row_params & p) {
    return p.repetition_penalty == 1.0f && p.presence_penalty == 0.0f && p.frequency_penalty == 0.0f;
}

__device__ __forceinline__ Plan make_plan(const spx_row_params & p, int vocab, bool has_ban, bool has_hist, int max_out) {
    Plan pl;
    pl.flavor = p.flavor;
    pl.top_p = p.top_p;
    pl.pen = !neutral(p) && has_hist;
    pl.counts = pl.pen && p.frequency_penalty != 0.0f;
    pl.need_s = false;
    pl.k = 1;
    pl.K = 1;
    pl.t = 1.0f;
    pl.rt = 1.0f;
    pl.xmin = false;
    pl.nanchk = false;
    bool bad = p.flavor < SPX_FLAVOR_TRANSFORMERS || p.flavor > SPX_FLAVOR_FISH;
    bad = bad || __builtin_isnan(p.temperature) || __builtin_isnan(p.top_p) ||
          __builtin_isnan(p.repetition_penalty) || __builtin_isnan(p.presence_penalty) ||
          __builtin_isnan(p.frequency_penalty);
    bad = bad || (p.flavor == SPX_FLAVOR_FISH && has_ban);
    bad = bad || (p.flavor == SPX_FLAVOR_TRANSFORMERS && !p.greedy && !(p.temperature > 0.0f));
    // a temperature the float rounds to infinity, which the reference's engines refuse
    // (src/engines/qwen3-tts-engine.cpp:47-56)
    bad = bad || (!p.greedy && p.temperature == INFINITY);
    if (bad) {
        pl.mode = kInvalid;
        return pl;
    }
    if (p.greedy || (p.flavor == SPX_FLAVOR_HARU && p.temperature <= 0.0f)) {
        pl.mode = kGreedy;
        pl.nanchk = p.flavor != SPX_FLAVOR_TRANSFORMERS;
        pl.xmin = p.flavor == SPX_FLAVOR_FISH;
        return pl;
    }
    int k;
    if (p.flavor == SPX_FLAVOR_TRANSFORMERS) k = p.top_k > 0 ? min(p.top_k, vocab) : vocab;   // qwen3-tts/sampler.cpp:77
    else if (p.flavor == SPX_FLAVOR_HARU) k = (p.top_k > 0 && p.top_k < vocab) ? p.top_k : vocab;  // haru/sampler.cpp:36
    else k = min(max(p.top_k, 1), vocab);                                                  // drama3/sampler.cpp:44
    pl.k = k;
    pl.t = p.flavor == SPX_FLAVOR_FISH ? fmaxf(p.temperature, 1e-5f) : p.temperature;
    pl.rt = 1.0f / pl.t;
    pl.mode = k <= kKeep ? kTopK : kFull;
    // a row listing its candidates holds at least the max_out it lists
    pl.K = pl.mode == kTopK ? k : max(kKeepFull, min(max_out, kKeep));
    pl.need_s = pl.mode == kFull || p.flavor == SPX_FLAVOR_FISH;
    return pl;
}

// The penalty stage on one history token's raw logit: presence/frequency (no reference counterpart), then
// restricted()'s repetition penalty once (src/families/qwen3-tts/sampler.cpp:37).
__device__ __forceinline__ float penalize(float x, int count, const spx_row_params & p) {
    if (count > 0) {
        if (p.frequency_penalty != 0.0f) x = __fsub_rn(x, __fmul_rn(p.frequency_penalty, (float) count));
        if (p.presence_penalty != 0.0f) x = __fsub_rn(x, p.presence_penalty);
    }
    if (p.repetition_penalty != 1.0f) x = x < 0.0f ? __fmul_rn(x, p.repetition_penalty) : x / p.repetition_penalty;
    return x;
}

__device__ __forceinline__ float uniform_f(float v) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

// v, or -inf where bit k of `kill` is set: a sign-extended bit field and a bitfield insert.
__device__ __forceinline__ float kill_to(float v, uint32_t kill, int k) {
    const uint32_t mk = (uint32_t) __builtin_amdgcn_sbfe((int) kill, k, 1);
    return __uint_as_float((mk & kNegInfBits) | (~mk & __float_as_uint(v)));
}

// kill_to for every element of a group, as two bit operations each (a sign-extending bit field extract and a
// bit-field insert), written out so that they stay bit operations and take no scalar registers.
template <int K>
__device__ __forceinline__ float kill_bit(float v, uint32_t kill, uint32_t ninf) {
    uint32_t mk, r;
    asm("v_bfe_i32 %0, %1, %2, 1" : "=v"(mk) : "v"(kill), "n"(K));
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(mk), "v"(ninf), "v"(__float_as_uint(v)));
    return __uint_as_float(r);
}
template <int... K>
__device__ __forceinline__ void kill_group(float * q, uint32_t kill, std::integer_sequence<int, K...>) {
    const uint32_t ninf = kNegInfBits;
    ((q[K] = kill_bit<K>(q[K], kill, ninf)), ...);
}

// ------------------------------------------------------------------------------------------------------------------
// Work-group helpers
// ------------------------------------------------------------------------------------------------------------------

// LDS scratch of the reductions.
struct Red {
    int i[64];
    double d[32];
    uint64_t u[32];
    float f[64];
    uint32_t w[32];
};

template <int B>
__device__ __forceinline__ int block_excl_scan_i32(int v, int * red, int & total) {
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    const int inc = wave_incl_scan_i32(v);
    if (lane == kWave - 1) red[wave] = inc;
    __syncthreads();
    int base = 0, tot = 0;
    for (int w = 0; w < B / kWave; w++) {
        const int x = red[w];
        if (w < wave) base += x;
        tot += x;
    }
    __syncthreads();
    total = tot;
    return base + inc - v;
}

template <int B>
__device__ __forceinline__ uint32_t block_or_u32(uint32_t v, uint32_t * red) {
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    v = wave_or_u32(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    uint32_t t = 0;
    for (int w = 0; w < B / kWave; w++) t |= red[w];
    __syncthreads();
    return t;
}

template <int B>
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t * red) {
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    v = wave_max_u64(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    uint64_t t = 0;
    for (int w = 0; w < B / kWave; w++) t = red[w] > t ? red[w] : t;
    __syncthreads();
    return t;
}

template <int B>
__device__ __forceinline__ uint64_t block_min_u64(uint64_t v, uint64_t * red) {
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    v = wave_min_u64(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    uint64_t t = ~0ull;
    for (int w = 0; w < B / kWave; w++) t = red[w] < t ? red[w] : t;
    __syncthreads();
    return t;
}

// The control block of a chunk, in LDS.
constexpr int kBins = 256;

struct Ctl {
    uint32_t bins[kBins];  // candidate entries per bin of quotient (sampling rows, from the first step on)
    uint32_t n;         // candidate entries reserved
    uint32_t tau_key;   // order key of the threshold (0: none yet)
    uint32_t overflow;  // entries were dropped for want of room
    uint32_t last;      // this work-group merges its row
    uint32_t resolved;  // the finishing wave settled the row
    uint32_t ncomp;     // candidates at or above the final threshold
    uint32_t kkey;      // the chunk's K-th key
    uint32_t n_own;     // distinct history tokens listed
    // The bins of the candidates' quotients, set by the first step: bin (q - lo) * scale clamped to [0, kBins), a
    // bin `width` about 1 / scale wide; scale 0: no bins (the first step gave no finite bound), the threshold moves
    // by exact searches. Kept here rather than in registers: they are read where a candidate is appended.
    float bin_lo, bin_scale, bin_width;
    float wave_t[16];   // per wave: its bound on the K-th quotient, and its largest quotient, of the first step
    float wave_m[16];
};
static_assert(sizeof(Ctl) <= kCtlBytes, "the control block outgrows its LDS");

// ------------------------------------------------------------------------------------------------------------------
// Special tokens of a chunk, in LDS
// ------------------------------------------------------------------------------------------------------------------

// Per 32 tokens of the chunk one word of special bits: a banned token, or a history token of a penalized row; the
// stream masks them to -inf. The penalty stage takes the chunk's distinct history tokens (in range, not banned) from
// a list, each once: the thread whose atomicOr set a token's bit first appends it. A row with a frequency penalty
// lists every occurrence instead, sorted, so that each token's occurrences are one run of the list: the run's first
// entry stands for the token and the run's length is its count.
struct Specials {
    uint32_t * kill;
    int32_t * own;     // the distinct history tokens of the chunk, or (frequency rows) all its history ids, sorted
    int own_cap;       // entries the list has room for: a power of two
    int n_own;
    bool any;
};

__device__ __forceinline__ void specials_at(Specials & sp, const Launch & a, unsigned char * lds) {
    sp.kill = (uint32_t *) (lds + a.off_spec);
    sp.own = (int32_t *) (lds + a.off_own);
    sp.own_cap = a.own_cap;
    sp.n_own = 0;
}

template <typename T>
struct Elt;
template <>
struct Elt<float> {
    static constexpr int V = 4;  // tokens per 16-byte vector
    static constexpr int U = 4;  // vectors per lane per step
};
template <>
struct Elt<uint16_t> {
    static constexpr int V = 8;
    static constexpr int U = 2;
};

// The logits row a sampled row reads.
__device__ __forceinline__ int64_t logits_row(const Launch & a, int row) { return a.row_map ? a.row_map[row] : row; }

// Row r's history range [h0, h1) of the ids: from the offsets, or strided (see Launch).
__device__ __forceinline__ void hist_bounds(const Launch & a, int row, int & h0, int & h1) {
    if (a.hist_off) {
        h0 = a.hist_off[row];
        h1 = a.hist_off[row + 1];
    } else {
        h0 = (int) ((int64_t) row * a.hist_stride) + a.hist_first;
        h1 = h0 + a.hist_len;
    }
}

// The row's history range [h0, h1) of the concatenated ids; flags a history longer than the handle takes.
__device__ __forceinline__ void hist_range(const Launch & a, int row, const Plan & pl, int & h0, int & h1, uint32_t & bad) {
    h0 = h1 = 0;
    if (!pl.pen) return;
    hist_bounds(a, row, h0, h1);
    if (h1 - h0 > a.max_hist || h1 < h0) {
        bad |= kBadHist;
        h1 = h0;
    }
}

// Sorts v[0..n) ascending in place, n a power of two, by a bitonic network over the work-group.
template <int B>
__device__ __forceinline__ void block_bitonic_sort(int32_t * v, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (int i = threadIdx.x; i < (n >> 1); i += B) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool up = (lo & size) == 0;
                const int32_t x = v[lo], y = v[hi];
                if ((x > y) == up) {
                    v[lo] = y;
                    v[hi] = x;
                }
            }
        }
    }
    __syncthreads();
}

// The chunk's special bits and its list of history tokens (see Specials). c0 is a multiple of 64, so the chunk's
// words are whole words of the ban mask. The history ids are read from memory in slabs of B, h0..h1 of the row
// (first: this thread's id of the first slab where the caller read it already, else -1).
template <int B>
__device__ __forceinline__ void build_specials(Specials & sp, int c0, int c1, const Plan & pl, const uint32_t * banned_row,
                                      const int32_t * hist, int h0, int h1, int first, uint32_t * n_own) {
    const int nw = (c1 - c0 + 31) >> 5;
    const int tid = threadIdx.x;
    for (int w = tid; w < nw; w += B) {
        uint32_t bw = 0;
        if (banned_row) {
            bw = banned_row[(c0 >> 5) + w];
            const int base = c0 + (w << 5);
            if (base + 32 > c1) bw &= (1u << (c1 - base)) - 1u;  // 0 < c1 - base < 32 here
        }
        sp.kill[w] = bw;
    }
    if (tid == 0) *n_own = 0u;
    __syncthreads();
    if (!pl.pen) return;
    for (int j = h0 + tid; j < h1; j += B) {
        const int t = j == h0 + tid && first >= 0 ? first : hist[j];
        if (t >= c0 && t < c1) {
            const uint32_t bit = 1u << ((t - c0) & 31);
            const bool banned = banned_row && ((banned_row[t >> 5] >> (t & 31)) & 1u);
            const uint32_t old = atomicOr(&sp.kill[(t - c0) >> 5], bit);
            // a banned token stays -inf whatever its history (restricted() bans after the penalty)
            if (!banned && (pl.counts || !(old & bit))) {
                const uint32_t at = atomicAdd(n_own, 1u);
                if (at < (uint32_t) sp.own_cap) sp.own[at] = t;
            }
        }
    }
    __syncthreads();
    sp.n_own = min((int) *n_own, sp.own_cap);
    if (pl.counts) {
        // every occurrence listed: sort them, padded with a value above every token, so that equal ids form runs
        for (int i = sp.n_own + tid; i < sp.own_cap; i += B) sp.own[i] = 0x7fffffff;
        block_bitonic_sort<B>(sp.own, sp.own_cap);
    }
}

// Entry i of the history list: the token it stands for, or -1 where it repeats the entry before (a frequency row's
// run), with `count` the occurrences of its token.
__device__ __forceinline__ int own_token(const Specials & sp, const Plan & pl, int i, int & count) {
    const int t = sp.own[i];
    count = 1;
    if (!pl.counts) return t;
    if (i > 0 && sp.own[i - 1] == t) return -1;
    int j = i + 1;
    while (j < sp.n_own && sp.own[j] == t) j++;
    count = j - i;
    return t;
}

template <typename T>
__device__ __forceinline__ float load_one(const T * p);
template <>
__device__ __forceinline__ float load_one<float>(const float * p) {
    return *p;
}
template <>
__device__ __forceinline__ float load_one<uint16_t>(const uint16_t * p) {
    return bf16_to_float(*p);
}

// A history token's final logit: its raw logit, read again from memory, penalized (count: its occurrences).
template <typename T>
__device__ __forceinline__ float hist_value(int t, int count, const spx_row_params & p, const T * rowp) {
    return penalize(load_one<T>(rowp + t), count, p);
}

// ------------------------------------------------------------------------------------------------------------------
// The stream: sampling rows
// ------------------------------------------------------------------------------------------------------------------

struct SampleSt {
    double s;        // lane: sum of 2^(q*L - hi) over its groups, L = log2(e) in float
    float m, hi;     // wave: the reference quotient and ceil(m*L), an integer (-FLT_MAX while no finite quotient is known)
    float tau;       // wave: a quotient at or above it enters the buffer
    uint32_t flags;  // lane
};

// The largest float below a finite t (t itself when it is infinite).
__device__ __forceinline__ float next_down(float t) {
    const uint32_t u = __float_as_uint(t);
    if (!(__builtin_fabsf(t) < INFINITY)) return t;
    if (t == 0.0f) return -0x1p-149f;
    return __uint_as_float(t > 0.0f ? u - 1u : u + 1u);
}

// The bin of a candidate's quotient (monotone in q).
__device__ __forceinline__ int value_bin(float lo, float scale, float q) {
    return (int) fminf(fmaxf((q - lo) * scale, 0.0f), (float) (kBins - 1));
}

// A threshold from the bins: the highest bin b whose bins b.. hold at least K candidates, and the threshold one bin
// below it (every candidate of bins b.. is at or above it, whatever the rounding of the bin's computation); -inf
// when fewer than K candidates are binned or b is the lowest bin. `held`: the candidates of bins b-1.. (about those
// at or above the threshold). One wave; each lane reads four bins.
__device__ __forceinline__ float bin_bound(const Ctl * ctl, int K, uint32_t & held) {
    const int l = lane_id();
    const uint4 c = ((const uint4 *) ctl->bins)[l];
    const uint32_t s4 = c.x + c.y + c.z + c.w;
    const uint32_t incl = (uint32_t) wave_incl_scan_i32((int) s4);
    const uint32_t total = (uint32_t) __builtin_amdgcn_readlane((int) incl, kWave - 1);
    held = 0;
    // candidates in bins 4l+j and above
    const uint32_t s3 = total - incl + c.w, s2 = s3 + c.z, s1 = s2 + c.y, s0 = s1 + c.x;
    const uint64_t ok = ballot(s0 >= (uint32_t) K);
    if (!ok) return -INFINITY;
    const int top = kWave - 1 - (int) __builtin_clzll(ok);
    const uint32_t uk = (uint32_t) K;
    const int b = s3 >= uk ? 4 * l + 3 : s2 >= uk ? 4 * l + 2 : s1 >= uk ? 4 * l + 1 : 4 * l;
    const int bb = __builtin_amdgcn_readlane(b, top);
    if (bb < 1) return -INFINITY;
    const int hb = bb - 1, hj = hb & 3;
    held = (uint32_t) __builtin_amdgcn_readlane((int) (hj == 0 ? s0 : hj == 1 ? s1 : hj == 2 ? s2 : s3), hb >> 2);
    // lo + (b-1) * width in one rounding, then one float down: below the exact edge
    return next_down(__builtin_fmaf((float) (bb - 1), ctl->bin_width, ctl->bin_lo));
}

// The exponent the terms of a sum are taken against: an integer, so that moving a sum to a new one is exact.
__device__ __forceinline__ float ref_exponent(float m) { return __builtin_ceilf(m * kL2e); }

// A sum of 2^(q*L - hi) moved to the exponent nhi >= hi: a multiplication by a power of two.
__device__ __forceinline__ double rescale(double s, float hi, float nhi) {
    return __builtin_ldexp(s, (int) fmaxf(hi - nhi, -2000.0f));
}

// The first step: every wave bounds the K-th quotient by the kw-th largest of its lanes' maxima (each lane's maximum
// is a distinct token), the work-group takes the smallest bound (kw lanes of every wave lie at or above it: at least
// K tokens) and the largest quotient as the reference m.
template <int B>
__device__ __forceinline__ void bootstrap(const Plan & pl, SampleSt & st, Ctl * ctl, const float (&q)[kE]) {
    constexpr int W = B / kWave;
    float lm = -INFINITY;
#pragma unroll
    for (int k = 0; k < kE; k++) lm = fmaxf(lm, q[k] < INFINITY ? q[k] : -INFINITY);
    const float wmax = wave_max_f32(lm);
    const int kw = (pl.K + W - 1) / W;
    float v = lm, kth = -INFINITY;
    for (int r = 0; r < kw; r++) {
        const float mx = uniform_f(wave_max_f32(v));
        kth = mx;
        if (!(mx > -INFINITY)) break;
        const uint64_t eq = ballot(v == mx);
        if (lane_id() == (int) __builtin_ctzll(eq)) v = -INFINITY;
    }
    const int wave = threadIdx.x / kWave;
    if (lane_id() == 0) {
        ctl->wave_t[wave] = kth;
        ctl->wave_m[wave] = wmax;
    }
    __syncthreads();
    float tau0 = INFINITY, mref = -INFINITY;
    for (int w = 0; w < W; w++) {
        tau0 = fminf(tau0, ctl->wave_t[w]);
        mref = fmaxf(mref, ctl->wave_m[w]);
    }
    tau0 = uniform_f(tau0);
    mref = uniform_f(mref);
    st.tau = tau0;
    float scale = 0.0f, width = 0.0f;
    if (tau0 > -INFINITY && mref > tau0) {
        const float span = mref - tau0;
        const float sc = (float) kBins / span;
        if (sc > 0.0f && sc < INFINITY && span < INFINITY) {
            scale = sc;
            width = span / (float) kBins;
        }
    }
    // every wave writes the same values before it reads them
    if (lane_id() == 0) {
        __hip_atomic_store(&ctl->bin_lo, tau0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        __hip_atomic_store(&ctl->bin_scale, scale, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        __hip_atomic_store(&ctl->bin_width, width, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    __builtin_amdgcn_wave_barrier();
    st.m = mref;
    st.hi = mref > -INFINITY ? ref_exponent(mref) : -FLT_MAX;
    if (lane_id() == 0) atomicMax(&ctl->tau_key, order_key(tau0));
}

// A group with a term that is not a finite number below 2^100: exact quotients, the flags, a new reference m where a
// finite quotient passes the old one, and the group's sum again. The logits are read again (element k is token
// id_base + (k / VV) * B * VV + k % VV): the stream does not keep them past the quotients.
template <typename T, int B, int VV>
__device__ __forceinline__ void slow_group(const Plan & pl, SampleSt & st, float (&q)[kE], const T * rowp, int id_base,
                                  uint32_t kill, bool mask) {
    float gm = -INFINITY;
    uint32_t fl = 0;
#pragma unroll
    for (int k = 0; k < kE; k++) {
        float qe = -INFINITY;
        if (!(mask && ((kill >> k) & 1u))) {
            const float xv = load_one<T>(rowp + id_base + (k / VV) * (B * VV) + (k % VV));
            qe = div_rn(xv, pl.t, pl.rt);
            if (__builtin_isnan(qe)) fl |= kNaN;
            else if (qe == INFINITY) fl |= xv == INFINITY ? kPosInf : (kTempOver | kTempOverPos);
            else if (qe == -INFINITY) fl |= xv == -INFINITY ? kNegInf : kTempOver;
            else gm = fmaxf(gm, qe);
            if (__builtin_isfinite(xv)) fl |= kFinite;
        }
        q[k] = qe;
    }
    st.flags |= fl;
    const float wm = uniform_f(wave_max_f32(gm));
    if (wm > st.m) {
        const float nhi = ref_exponent(wm);
        if (st.m > -INFINITY) st.s = rescale(st.s, st.hi, nhi);
        st.m = wm;
        st.hi = nhi;
    }
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < kE; k++) {
        const float qv = q[k];
        if (qv > -INFINITY && qv < INFINITY) acc += __builtin_amdgcn_exp2f(__builtin_fmaf(qv, kL2e, -st.hi));
    }
    st.s += (double) acc;
}

// The K-th largest key among the first `lim` entries of the buffer, by one wave (entries other waves have reserved
// but not written yet read as 0 and are not counted); 0 when there are fewer than K. A bitwise search from the top
// key bit down, each candidate counted with one ballot per 64 keys: the first 1024 keys held in registers, those of a
// longer buffer read again from LDS.
__device__ __forceinline__ uint32_t buffer_bound(const uint64_t * cand, int lim, int K) {
    constexpr int kHeld = 16;
    // the lane's keys: words 2(l + 64j) + 1, one address and immediate offsets; lane l holds key j when l < lim - 64j
    int l = lane_id();
    asm volatile("" : "+v"(l));  // formed here, where the bound is taken, not kept live across the stream
    const uint32_t * kw = (const uint32_t *) cand + 2 * l + 1;
    const int nj = (lim + kWave - 1) / kWave;
    uint32_t keys[kHeld];
#pragma unroll
    for (int j = 0; j < kHeld; j++) keys[j] = (j < nj && l < lim - kWave * j) ? kw[2 * kWave * j] : 0u;
    uint32_t key = 0;
    for (int b = 31; b >= 0; b--) {
        const uint32_t c = key | (1u << b);
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < kHeld; j++)
            if (j < nj) cnt += (int) __popcll(ballot(keys[j] >= c));
        for (int j = kHeld; j < nj; j++) cnt += (int) __popcll(ballot(l < lim - kWave * j && kw[2 * kWave * j] >= c));
        if (cnt >= K) key = c;
    }
    return key;
}

// Appends the passing elements of a step to the buffer: each lane counts its own, a scan over the wave places them,
// one atomic per wave takes the room, and each lane writes its elements in order and counts each in its bin. `all`
// (no bound yet) takes every valid element, -inf ones included. The wave whose appends pass a multiple of 32 entries
// raises the work-group's threshold from the bins; with no bins, or when the top bin alone holds K (the quotients
// run so far above the first step's largest that the bins no longer tell them apart), an exact search of the buffer
// does so at every 128 entries. Every wave takes the threshold up at its next step. Called by the whole wave.
template <typename T, int B, int VV, bool MASK>
__device__ __forceinline__ void insert_entries(const Plan & pl, SampleSt & st, Ctl * ctl, uint64_t * cand, int cap,
                                               const float (&q)[kE], const T * rowp, uint32_t kill, int id_base,
                                               bool all) {
    float tau = uniform_f(st.tau);
    auto pass = [&](int k) {
        const bool live = !MASK || !((kill >> k) & 1u);
        return all ? (live && !__builtin_isnan(q[k])) : (q[k] >= tau);
    };
    int cnt = 0;
#pragma unroll
    for (int k = 0; k < kE; k++) cnt += pass(k) ? 1 : 0;
    const int incl = wave_incl_scan_i32(cnt);
    const int total = __builtin_amdgcn_readlane(incl, kWave - 1);
    if (total == 0) return;
    uint32_t base = 0;
    if (lane_id() == 0) base = atomicAdd(&ctl->n, (uint32_t) total);
    base = (uint32_t) __builtin_amdgcn_readfirstlane((int) base);
    if (base + (uint32_t) total > (uint32_t) cap && lane_id() == 0) ctl->overflow = 1u;
    const float blo = ctl->bin_lo, bscale = ctl->bin_scale;
    const bool binned = bscale > 0.0f;
    // the compares again, not their results of the count kept across it
    asm volatile("" : "+s"(tau));
    int pos = (int) base + incl - cnt;
#pragma unroll
    for (int k = 0; k < kE; k++) {
        if (pass(k)) {
            if (pos < cap) {
                // a quotient in the subnormal range: the division itself (the correction step assumes a normal one)
                const int id = id_base + (k / VV) * (B * VV) + (k % VV);
                float qq = q[k];
                if (qq != 0.0f && __builtin_fabsf(qq) < 0x1p-125f) qq = load_one<T>(rowp + id) / pl.t;
                cand[pos] = make_entry(order_key(qq), (uint32_t) id);
                if (binned) atomicAdd(&ctl->bins[value_bin(blo, bscale, qq)], 1u);
            }
            pos++;
        }
    }
    const uint32_t end = base + (uint32_t) total;
    if ((base >> 5) == (end >> 5)) return;
    uint32_t held;
    float tn = binned ? bin_bound(ctl, pl.K, held) : -INFINITY;
    if ((base >> 7) != (end >> 7) && (!binned || ctl->bins[kBins - 1] >= (uint32_t) pl.K)) {
        const uint32_t kk = buffer_bound(cand, min((int) (end & ~127u), cap), pl.K);
        if (kk) tn = fmaxf(tn, key_float(kk));
    }
    tn = uniform_f(tn);
    if (tn > st.tau) {
        st.tau = tn;
        if (lane_id() == 0) atomicMax(&ctl->tau_key, order_key(tn));
    }
}

// One group of kE final logits per lane. x: raw logits; kill: elements that are special tokens or out of range;
// rdead: those out of range. Element k's token is id_base + (k / VV) * B * VV + k % VV; rowp: the row's logits.
template <typename T, int B, int VV, bool MASK, bool BOOT>
__device__ __forceinline__ void sample_core(const Plan & pl, SampleSt & st, Ctl * ctl, uint64_t * cand, int cap,
                                            const float (&x)[kE], uint32_t kill, uint32_t rdead, int id_base,
                                            const T * rowp) {
    float q[kE];
#pragma unroll
    for (int k = 0; k < kE; k++) {
        // x / t correctly rounded for a quotient in the normal range (Markstein's correction step)
        const float q0 = x[k] * pl.rt;
        q[k] = __builtin_fmaf(__builtin_fmaf(-q0, pl.t, x[k]), pl.rt, q0);
    }
    if (MASK) kill_group(q, kill, std::make_integer_sequence<int, kE>{});
    // token 0's final logit, where it is not special, for std::max_element's NaN in front
    if (BOOT && id_base == 0 && !(kill & 1u) && __builtin_isnan(x[0])) st.flags |= kNaN0;
    if (BOOT) bootstrap<B>(pl, st, ctl, q);
    // the work-group's threshold, raised by whichever wave last refreshed it
    const uint32_t tk = BOOT ? 0u : __hip_atomic_load(&ctl->tau_key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    float t[kE];
#pragma unroll
    for (int k = 0; k < kE; k++) t[k] = __builtin_amdgcn_exp2f(__builtin_fmaf(q[k], kL2e, -st.hi));
#pragma unroll
    for (int w = kE / 2; w >= 1; w >>= 1) {
#pragma unroll
        for (int k = 0; k < w; k++) t[k] += t[k + w];
    }
    if (ballot(!(t[0] <= 0x1p100f))) slow_group<T, B, VV>(pl, st, q, rowp, id_base, kill, MASK);
    else st.s += (double) t[0];
    if (!BOOT && tk) st.tau = fmaxf(st.tau, uniform_f(key_float(tk)));
    // Candidates: the appends only where a lane's largest quotient reaches tau (a NaN is no lane's largest unless
    // all of its are NaN, and never passes).
    if (st.tau > -INFINITY) {
        float lm = q[0];
#pragma unroll
        for (int k = 1; k < kE; k++) lm = fmaxf(lm, q[k]);
        if (ballot(lm >= st.tau)) insert_entries<T, B, VV, MASK>(pl, st, ctl, cand, cap, q, rowp, kill, id_base, false);
    } else {
        // no bound yet: every valid token of the chunk enters
        insert_entries<T, B, VV, MASK>(pl, st, ctl, cand, cap, q, rowp, kill, id_base, true);
    }
}

// ------------------------------------------------------------------------------------------------------------------
// The stream: greedy rows
// ------------------------------------------------------------------------------------------------------------------

struct GreedySt {
    float bx;       // lane: its largest final logit and the first token holding it (tokens come in rising order)
    int bi;
    float xmin;     // lane: smallest raw logit in range
    uint64_t nanb;  // wave: lanes that met a NaN final logit
};

template <int B, int VV, bool MASK>
__device__ __forceinline__ void greedy_core(const Plan & pl, GreedySt & g, const float (&x)[kE], uint32_t kill,
                                            uint32_t rdead, int id_base) {
    float xm[kE];
#pragma unroll
    for (int k = 0; k < kE; k++) xm[k] = x[k];
    if (MASK) kill_group(xm, kill, std::make_integer_sequence<int, kE>{});
    if (pl.nanchk) {
#pragma unroll
        for (int k = 0; k < kE; k++) g.nanb |= ballot(xm[k] != xm[k]);
    }
    if (pl.xmin) {
#pragma unroll
        for (int k = 0; k < kE; k++) g.xmin = fminf(g.xmin, ((rdead >> k) & 1u) ? INFINITY : x[k]);
    }
    float t[kE];
#pragma unroll
    for (int k = 0; k < kE; k++) t[k] = xm[k];
#pragma unroll
    for (int w = kE / 2; w >= 1; w >>= 1) {
#pragma unroll
        for (int k = 0; k < w; k++) t[k] = fmaxf(t[k], t[k + w]);
    }
    const float gx = t[0];
    if (ballot(gx > g.bx)) {
        if (gx > g.bx) {
            int idx = 0;
#pragma unroll
            for (int k = kE - 1; k >= 0; k--) idx = xm[k] == gx ? k : idx;
            g.bx = gx;
            g.bi = id_base + (idx / VV) * (B * VV) + (idx % VV);
        }
    }
}

// ------------------------------------------------------------------------------------------------------------------
// The stream over a chunk
// ------------------------------------------------------------------------------------------------------------------

using U32x4 = uint32_t __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ void unpack(const U32x4 & r, float * x);
template <>
__device__ __forceinline__ void unpack<float>(const U32x4 & r, float * x) {
    x[0] = __uint_as_float(r.x);
    x[1] = __uint_as_float(r.y);
    x[2] = __uint_as_float(r.z);
    x[3] = __uint_as_float(r.w);
}
template <>
__device__ __forceinline__ void unpack<uint16_t>(const U32x4 & r, float * x) {
    x[0] = __uint_as_float(r.x << 16);
    x[1] = __uint_as_float(r.x & 0xffff0000u);
    x[2] = __uint_as_float(r.y << 16);
    x[3] = __uint_as_float(r.y & 0xffff0000u);
    x[4] = __uint_as_float(r.z << 16);
    x[5] = __uint_as_float(r.z & 0xffff0000u);
    x[6] = __uint_as_float(r.w << 16);
    x[7] = __uint_as_float(r.w & 0xffff0000u);
}

struct StreamCtx {
    const Plan * pl;
    const Specials * sp;
    SampleSt * st;
    GreedySt * g;
    Ctl * ctl;
    uint64_t * cand;
    int cap;
    const void * rowp;  // the row's logits
};

template <typename T, int B, int VV, bool MASK, bool BOOT, bool GREEDY>
__device__ __forceinline__ void run_core(StreamCtx & c, const float (&x)[kE], uint32_t kill, uint32_t rdead, int id_base) {
    if constexpr (GREEDY) greedy_core<B, VV, MASK>(*c.pl, *c.g, x, kill, rdead, id_base);
    else sample_core<T, B, VV, MASK, BOOT>(*c.pl, *c.st, c.ctl, c.cand, c.cap, x, kill, rdead, id_base, (const T *) c.rowp);
}

// A step's vectors of a chunk (lanes past the last whole vector load it again; none when the step has none).
template <typename T, int B>
__device__ __forceinline__ void load_step(const Launch & a, const T * rowp, int c0, int c1, int step,
                                          U32x4 (&v)[Elt<T>::U]) {
    constexpr int V = Elt<T>::V, U = Elt<T>::U;
    const int ng = a.vec_ok ? (c1 - c0) / V : 0;
    const U32x4 * vp = (const U32x4 *) (rowp + c0);
#pragma unroll
    for (int u = 0; u < U; u++) v[u] = U32x4{0u, 0u, 0u, 0u};
    if (ng > step * U * B) {
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = vp[min(step * U * B + (int) threadIdx.x + u * B, ng - 1)];
    }
}

// kE tokens per lane, one each at chunk offsets o0 + k*B: rows that are not 16-byte aligned, and a chunk's tail.
template <typename T, int B, bool SPEC, bool GREEDY, bool BOOT>
__device__ __forceinline__ void scalar_group(StreamCtx & c, const T * rowp, int c0, int n, int o0) {
    float x[kE];
    uint32_t kill = 0, rdead = 0;
#pragma unroll
    for (int k = 0; k < kE; k++) {
        const int o = o0 + k * B;
        x[k] = 0.0f;
        if (o < n) {
            const T raw = rowp[c0 + o];
            x[k] = load_one<T>(&raw);
            if (SPEC && ((c.sp->kill[o >> 5] >> (o & 31)) & 1u)) kill |= 1u << k;
        } else {
            rdead |= 1u << k;
        }
    }
    run_core<T, B, 1, true, BOOT, GREEDY>(c, x, kill | rdead, rdead, c0 + o0);
}

// One step of the vector stream: U vectors per lane, vector g0 + u*B for u < U, of which those past the last whole
// vector (ng) are out of range when RANGE; BOOT is the first step. A vector's special bits are V bits of one word.
template <typename T, int B, bool SPEC, bool GREEDY, bool RANGE, bool BOOT>
__device__ __forceinline__ void vec_step(StreamCtx & c, const U32x4 (&cur)[Elt<T>::U], int c0, int g0, int ng, int gl) {
    constexpr int V = Elt<T>::V, U = Elt<T>::U, VW = 32 / V;
    constexpr uint32_t VM = (1u << V) - 1u;
    uint32_t kill = 0;
    if (SPEC) {
        uint32_t kw[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int gg = RANGE ? min(g0 + u * B, gl) : g0 + u * B;
            kw[u] = c.sp->kill[gg / VW] >> ((gg & (VW - 1)) * V);
        }
#pragma unroll
        for (int u = 0; u < U; u++) kill |= (kw[u] & VM) << (u * V);
    }
    float x[kE];
#pragma unroll
    for (int u = 0; u < U; u++) unpack<T>(cur[u], x + u * V);
    uint32_t rdead = 0;
    if (RANGE) {
#pragma unroll
        for (int u = 0; u < U; u++) rdead |= (g0 + u * B < ng) ? 0u : (VM << (u * V));
    }
    run_core<T, B, V, SPEC || RANGE, BOOT, GREEDY>(c, x, kill | rdead, rdead, c0 + g0 * V);
}

// The chunk's stream; after_first() runs once the first step is done (its bound and bins are set).
template <typename T, int B, bool SPEC, bool GREEDY, typename F>
__device__ __forceinline__ void stream_chunk(StreamCtx & c, const Launch & a, const T * rowp, int c0, int c1,
                                    const U32x4 (&first)[Elt<T>::U], F && after_first) {
    constexpr int V = Elt<T>::V, U = Elt<T>::U;
    const int n = c1 - c0, tid = threadIdx.x;
    if (!a.vec_ok) {
        const int nit = max(1, (n + kE * B - 1) / (kE * B));
        scalar_group<T, B, SPEC, GREEDY, true>(c, rowp, c0, n, tid);
        after_first();
        for (int it = 1; it < nit; it++) scalar_group<T, B, SPEC, GREEDY, false>(c, rowp, c0, n, it * kE * B + tid);
        return;
    }
    const int ng = n / V;  // whole vectors
    constexpr int per = U * B;
    const int nit = ng > 0 ? (ng + per - 1) / per : 1;
    const int nfull = ng / per;  // steps without a lane past the last vector
    const int gl = max(ng - 1, 0);
    const U32x4 * vp = (const U32x4 *) (rowp + c0);
    // The first and last steps (lanes past the last vector load it again and take nothing from it) are peeled off
    // the steady loop, whose loads for the next step are in flight while a step is worked on. The steady loop takes
    // two steps a turn, its two buffers trading places, while both steps it requests are whole (a lane's vectors at
    // fixed offsets from the step's start); the rest go one step a turn.
    U32x4 b0[U], b1[U];
#pragma unroll
    for (int u = 0; u < U; u++) b0[u] = first[u];  // requested before the special tokens were built
    load_step<T, B>(a, rowp, c0, c1, 1, b1);
    vec_step<T, B, SPEC, GREEDY, true, true>(c, b0, c0, tid, ng, gl);
    after_first();
    int it = 1;
    for (; it + 2 < nfull; it += 2) {
        const U32x4 * s1 = vp + (it + 1) * per;
#pragma unroll
        for (int u = 0; u < U; u++) b0[u] = s1[tid + u * B];
        vec_step<T, B, SPEC, GREEDY, false, false>(c, b1, c0, it * per + tid, ng, gl);
        const U32x4 * s2 = vp + (it + 2) * per;
#pragma unroll
        for (int u = 0; u < U; u++) b1[u] = s2[tid + u * B];
        vec_step<T, B, SPEC, GREEDY, false, false>(c, b0, c0, (it + 1) * per + tid, ng, gl);
    }
    for (; it + 1 < nit; it++) {
        U32x4 cur[U];
#pragma unroll
        for (int u = 0; u < U; u++) cur[u] = b1[u];
        const int g0 = it * per + tid;
#pragma unroll
        for (int u = 0; u < U; u++) b1[u] = vp[min(g0 + per + u * B, gl)];
        vec_step<T, B, SPEC, GREEDY, false, false>(c, cur, c0, g0, ng, gl);
    }
    if (nit > 1) vec_step<T, B, SPEC, GREEDY, true, false>(c, b1, c0, (nit - 1) * per + tid, ng, gl);
    if (n - ng * V > 0) scalar_group<T, B, SPEC, GREEDY, false>(c, rowp, c0, n, ng * V + tid);
}

// ------------------------------------------------------------------------------------------------------------------
// Finishing a row: the flavor's rule on its sorted top entries
// ------------------------------------------------------------------------------------------------------------------

struct RowTotals {
    uint64_t best;   // greedy: the largest entry of the final logits (0: none above -inf)
    double s;        // sum of exp(q - m) over the row
    float m;
    uint32_t flags;
};

// The row status, as the reference's checks order them; -1 when the row goes on.
__device__ __forceinline__ int row_status(const Plan & pl, const spx_row_params & p, uint32_t f, bool top_finite) {
    if (pl.mode == kInvalid || (f & kBadHist)) return SPX_ROW_INVALID_PARAMS;
    const bool pen = !neutral(p);
    const bool posinf = (f & kPosInf) != 0;
    const bool anyf = (f & (kFinite | kPosInf)) != 0;  // the largest final logit is above -inf
    if (pl.flavor == SPX_FLAVOR_TRANSFORMERS) {
        // restricted(): std::max_element's largest, a NaN in front taken as it (src/families/qwen3-tts/sampler.cpp:43-49)
        if (f & kNaN0) return SPX_ROW_NO_FINITE_LOGIT;
        if (posinf) return pen ? SPX_ROW_REP_PENALTY_OVERFLOW : SPX_ROW_NO_FINITE_LOGIT;
        if (!anyf) return SPX_ROW_NO_FINITE_LOGIT;
        if (pl.mode == kGreedy) return -1;
        if (f & kNaN) return SPX_ROW_NONFINITE_INPUT;
        if (!top_finite) return SPX_ROW_TEMPERATURE_OVERFLOW;  // qwen3-tts/sampler.cpp:82-83
        return -1;
    }
    if (!(f & kNaN0) && posinf && pen) return SPX_ROW_REP_PENALTY_OVERFLOW;
    if (pl.flavor == SPX_FLAVOR_HARU) {
        if ((f & kNaN) || posinf) return SPX_ROW_NONFINITE_INPUT;  // haru/sampler.cpp:21-23
        if (pl.mode == kGreedy) return -1;
        if (f & kTempOver) return SPX_ROW_TEMPERATURE_OVERFLOW;  // haru/sampler.cpp:33-35
        return -1;
    }
    if ((f & kNaN) || posinf || (f & kNegInf)) return SPX_ROW_NONFINITE_INPUT;  // drama3/sampler.cpp:35-37
    if (pl.mode == kGreedy) return -1;
    if (!top_finite) return SPX_ROW_TEMPERATURE_OVERFLOW;  // drama3/sampler.cpp:46-47
    return -1;
}

__device__ __forceinline__ void write_row(const Launch & a, int row, int id, int status, int kept) {
    a.out_ids[(int64_t) row * a.out_stride] = status == SPX_ROW_OK ? id : -1;
    if (a.out_status) a.out_status[row] = status;
    if (a.out_kept) a.out_kept[row] = status == SPX_ROW_OK ? kept : 0;
}

// The flags a greedy row's largest entry settles.
__device__ __forceinline__ uint32_t best_flags(uint64_t best) {
    if (!best) return 0u;
    const float v = entry_value(best);
    return v == INFINITY ? kPosInf : (v > -INFINITY ? kFinite : 0u);
}

constexpr int kNone = 0x7fffffff;
// Entries the finishing wave takes: four per lane.
constexpr int kFinishMax = 4 * kWave;

// Helpers of the finishing wave: element i of a row's sorted entries sits in lane i/4, slot i%4.
struct Cum4 {
    double c[4];
};
// Inclusive running sums over the elements in their order.
__device__ __forceinline__ Cum4 wave_cum4(const double (&x)[4]) {
    Cum4 r;
    r.c[0] = x[0];
    r.c[1] = r.c[0] + x[1];
    r.c[2] = r.c[1] + x[2];
    r.c[3] = r.c[2] + x[3];
    const double incl = wave_incl_scan_f64(r.c[3]);
    const double excl = incl - r.c[3];
    for (int j = 0; j < 4; j++) r.c[j] += excl;
    return r;
}
// The first element whose predicate holds (kNone when none).
__device__ __forceinline__ int wave_first4(const bool (&pred)[4]) {
    int fj = 4;
    for (int j = 3; j >= 0; j--) fj = pred[j] ? j : fj;
    const uint64_t m = ballot(fj < 4);
    if (!m) return kNone;
    const int l = (int) __builtin_ctzll(m);
    return 4 * l + __builtin_amdgcn_readlane(fj, l);
}
__device__ __forceinline__ double wave_sum4(const double (&x)[4]) { return wave_sum_f64((x[0] + x[1]) + (x[2] + x[3])); }

// Finishes a row from its totals and its n sorted top entries e[0..n), n <= kFinishMax, in one wave (the caller's
// wave 0). Returns true when the row is done, false when it needs the multi-pass path (its top-p set or its draw
// runs beyond the entries held). pf: LDS scratch of kFinishMax floats.
__device__ __forceinline__ bool finish_wave(const Launch & a, int row, const spx_row_params & p, const Plan & pl,
                                   const RowTotals & tot, const uint64_t * e, int n, bool complete, float * pf) {
    const int lane = lane_id();
    const double u = a.u ? a.u[(int64_t) row * a.u_stride] : 0.0;
    const float top = n > 0 ? entry_value(e[0]) : -INFINITY;
    const int st = row_status(pl, p, tot.flags, n > 0 && __builtin_isfinite(top));
    if (st >= 0) {
        if (lane == 0) write_row(a, row, -1, st, 0);
        return true;
    }
    if (pl.mode == kGreedy) {
        // std::max_element: the first largest, or token 0 when its logit is NaN.
        const int id = ((tot.flags & kNaN0) || tot.best == 0) ? 0 : (int) entry_id(tot.best);
        if (lane == 0) write_row(a, row, id, SPX_ROW_OK, 1);
        if (a.out_cand_ids) {
            // the one candidate of a greedy pick, weight 1 (src/families/haru/sampler.cpp:27-31)
            for (int j = lane; j < a.max_out; j += kWave) {
                a.out_cand_ids[(int64_t) row * a.max_out + j] = j == 0 ? id : -1;
                a.out_cand_w[(int64_t) row * a.max_out + j] = j == 0 ? 1.0 : 0.0;
            }
        }
        return true;
    }
    const int nk = min(n, pl.k);  // entries that belong to the flavor's top k
    // Every candidate of the reference with a weight is held: its top k, or every token that has a key (the rest of
    // a short row are banned tokens, last in the order with weight 0).
    const bool full_known = nk >= pl.k || complete;
    const bool last_held = nk >= pl.k;  // the k-th candidate itself is held
    // Transformers and Haru normalize over their top k; beyond the entries held, only a top k of the whole
    // vocabulary has a known sum (the stream's). Other rows take the wide path. Haru's sum is a float32 sum in the
    // row's order, which only the wide path takes beyond the entries held.
    if (!full_known && pl.k < a.vocab && pl.flavor != SPX_FLAVOR_FISH) return false;
    if (!full_known && pl.flavor == SPX_FLAVOR_HARU) return false;
    // The sum of exp over the whole vocabulary, relative to the top value (m of the totals is that value or below).
    const double s_all = pl.need_s ? tot.s * exp((double) tot.m - (double) top) : 0.0;
    bool valid[4];
    float v[4];
    int idx[4];
    for (int j = 0; j < 4; j++) {
        idx[j] = 4 * lane + j;
        valid[j] = idx[j] < nk;
        v[j] = valid[j] ? entry_value(e[idx[j]]) : -INFINITY;
    }
    int kept = 0, pick = -1;
    bool resolved = true;
    // The candidates' weights as the reference's Candidates holds them: TRANSFORMERS normalized over the top k and not
    // again after top-p, HARU float32 probabilities with the zeroed ones kept, FISH the unnormalized exponentials.
    double outp[4] = {0.0, 0.0, 0.0, 0.0};
    int nout = 0;  // candidates listed

    if (pl.flavor == SPX_FLAVOR_TRANSFORMERS) {
        // candidates(): double softmax over the k kept, normalized by their sum (src/families/qwen3-tts/sampler.cpp:84-87)
        double w[4], q[4];
        for (int j = 0; j < 4; j++) w[j] = valid[j] ? exp((double) v[j] - (double) top) : 0.0;
        const double sum = full_known ? wave_sum4(w) : s_all;
        for (int j = 0; j < 4; j++) q[j] = w[j] / sum;
        int keep = -1;
        if (pl.top_p < 1.0f) {
            // the smallest prefix whose cumulative weight reaches top_p, at least one (:88-99)
            const Cum4 c = wave_cum4(q);
            bool pr[4];
            for (int j = 0; j < 4; j++) pr[j] = valid[j] && c.c[j] >= (double) pl.top_p;
            const int first = wave_first4(pr);
            if (first != kNone) keep = first + 1;
            else if (full_known) keep = nk;
            else resolved = false;
        } else if (full_known) {
            keep = nk;
        } else {
            // A draw over every token: pick()'s running share must pass u within the entries held. The shares are
            // the weights over the whole vocabulary's sum, which is what pick() divides by, to rounding.
            const Cum4 c = wave_cum4(q);
            bool pr[4];
            for (int j = 0; j < 4; j++) pr[j] = valid[j] && c.c[j] > u;
            const int first = wave_first4(pr);
            if (first != kNone && first < pl.k - 1) {
                pick = first;
                kept = pl.k;
                for (int j = 0; j < 4; j++) outp[j] = q[j];
                nout = nk;
            } else {
                resolved = false;
            }
        }
        if (keep > 0) {
            // pick() over the kept weights (src/common/sampling.cpp:9-19). Where every token is held but fewer than
            // k have a key (banned ones, weight 0, are the rest of the k), the last held is not pick()'s last.
            const bool short_k = pl.top_p >= 1.0f && !last_held;
            const int lim = short_k ? keep : keep - 1;
            double kq[4];
            for (int j = 0; j < 4; j++) kq[j] = idx[j] < keep ? q[j] : 0.0;
            const double ksum = wave_sum4(kq);
            for (int j = 0; j < 4; j++) kq[j] /= ksum;
            const Cum4 c = wave_cum4(kq);
            bool pr[4];
            for (int j = 0; j < 4; j++) pr[j] = idx[j] < lim && c.c[j] > u;
            const int first = wave_first4(pr);
            if (first != kNone) pick = first;
            else if (!short_k) pick = keep - 1;
            else resolved = false;
            kept = short_k ? pl.k : keep;
            for (int j = 0; j < 4; j++) outp[j] = q[j];
            nout = keep;
        }
    } else if (pl.flavor == SPX_FLAVOR_HARU) {
        // torch's float32 softmax over the k kept and its top-p zeroing (src/families/haru/sampler.cpp:44-59), the
        // float sums in the reference's order by one lane
        for (int j = 0; j < 4; j++)
            if (valid[j]) pf[idx[j]] = (float) exp((double) (v[j] - top));
        __builtin_amdgcn_wave_barrier();  // lane 0 reads what the wave wrote (LDS keeps one wave's order)
        float sumf = 0.0f;
        int zeros = 0;
        if (lane == 0) {
            if (full_known) {
                for (int i = 0; i < nk; i++) sumf += pf[i];
            } else {
                sumf = (float) s_all;
            }
            if (pl.top_p > 0.0f && pl.top_p < 1.0f) {
                // The zeroing, position by position as the reference's loop runs it, in float (:52-59); pf[i] keeps
                // p_i, or -p_i where it is zeroed.
                float run = 0.0f;
                for (int i = 0; i < nk; i++) {
                    const float pi = pf[i] / sumf;
                    run += pi;
                    const bool zero = !(run - pi < pl.top_p);
                    zeros += zero ? 1 : 0;
                    pf[i] = zero ? -pi : pi;
                }
            } else {
                for (int i = 0; i < nk; i++) pf[i] = pf[i] / sumf;
            }
        }
        zeros = __builtin_amdgcn_readfirstlane(zeros);
        // Beyond the entries held the weights must be 0: a zero among them, the cumulative share only rising.
        if (!full_known && zeros == 0) resolved = false;
        if (resolved) {
            double w[4], wd[4];
            for (int j = 0; j < 4; j++) {
                const float x = valid[j] ? pf[idx[j]] : 0.0f;
                wd[j] = x > 0.0f ? (double) x : 0.0;
                w[j] = wd[j];
            }
            const double ksum = wave_sum4(w);
            for (int j = 0; j < 4; j++) w[j] /= ksum;
            // pick() over all k weights, zeros included: the held k-th is its last; short of it, its last lies beyond
            const int lim = last_held ? nk - 1 : nk;
            const Cum4 c = wave_cum4(w);
            bool pr[4];
            for (int j = 0; j < 4; j++) pr[j] = valid[j] && idx[j] < lim && c.c[j] > u;
            const int first = wave_first4(pr);
            if (first != kNone) pick = first;
            else if (last_held) pick = nk - 1;
            else resolved = false;
            kept = pl.k;
            for (int j = 0; j < 4; j++) outp[j] = wd[j];
            nout = nk;
        }
    } else {
        // fish-speech: shares over the softmax of every logit, the token passing top_p dropped
        // (src/families/drama3/sampler.cpp:48-59)
        double w[4], sh[4];
        for (int j = 0; j < 4; j++) {
            w[j] = valid[j] ? exp((double) v[j] - (double) top) : 0.0;
            sh[j] = w[j] / s_all;
        }
        const Cum4 c = wave_cum4(sh);
        bool pr[4];
        for (int j = 0; j < 4; j++) pr[j] = valid[j] && idx[j] > 0 && c.c[j] > (double) pl.top_p;
        const int first = wave_first4(pr);
        int keep = -1;
        if (first != kNone) keep = first;
        else if (full_known) keep = nk;
        else resolved = false;
        if (resolved) {
            double kw[4];
            for (int j = 0; j < 4; j++) kw[j] = idx[j] < keep ? w[j] : 0.0;
            const double ksum = wave_sum4(kw);
            for (int j = 0; j < 4; j++) kw[j] /= ksum;
            const Cum4 cc = wave_cum4(kw);
            bool pr2[4];
            for (int j = 0; j < 4; j++) pr2[j] = idx[j] < keep - 1 && cc.c[j] > u;
            const int f2 = wave_first4(pr2);
            pick = f2 != kNone ? f2 : keep - 1;
            kept = keep;
            for (int j = 0; j < 4; j++) outp[j] = idx[j] < keep ? w[j] : 0.0;
            nout = keep;
        }
    }
    if (!resolved) return false;
    if (lane == 0) write_row(a, row, (int) entry_id(e[pick]), SPX_ROW_OK, kept);
    if (a.out_cand_ids) {
        for (int j = 0; j < 4; j++) {
            const int i = idx[j];
            if (i < nout && i < a.max_out) {
                a.out_cand_ids[(int64_t) row * a.max_out + i] = (int32_t) entry_id(e[i]);
                a.out_cand_w[(int64_t) row * a.max_out + i] = outp[j];
            }
        }
        // entries past those written above
        for (int j = min(kept, nk) + lane; j < a.max_out; j += kWave) {
            if (j >= nout) {
                a.out_cand_ids[(int64_t) row * a.max_out + j] = -1;
                a.out_cand_w[(int64_t) row * a.max_out + j] = 0.0;
            }
        }
    }
    return true;
}

// Wave 0 finishes the row; the work-group learns whether it must take the multi-pass path.
template <int B>
__device__ __forceinline__ bool finish_block(const Launch & a, int row, const spx_row_params & p, const Plan & pl,
                                    const RowTotals & tot, const uint64_t * e, int n, bool complete, float * pf,
                                    Ctl * ctl) {
    if (threadIdx.x < kWave) {
        // the entries past the finishing wave's share are not seen: the list then holds less than every token
        const bool ok = finish_wave(a, row, p, pl, tot, e, min(n, kFinishMax), complete && n <= kFinishMax, pf);
        if (threadIdx.x == 0) ctl->resolved = ok ? 1u : 0u;
    }
    __syncthreads();
    return ctl->resolved != 0;
}

// Appends the entries of src[0..n) at or above `floor` to dst (at most kSortCap), one wave at a time per 64: a ballot,
// one atomic per wave on the LDS count, no barrier. The order among the appended is free; the caller sorts.
template <int B>
__device__ __forceinline__ void gather_append(const uint64_t * src, int n, uint64_t floor, uint64_t * dst, uint32_t * count) {
    const int lane = lane_id();
    for (int i0 = (threadIdx.x / kWave) * kWave; i0 < n; i0 += B) {
        const int i = i0 + lane;
        const uint64_t e = i < n ? src[i] : 0ull;
        const bool keep = e != 0 && e >= floor;
        const uint64_t m = ballot(keep);
        if (!m) continue;
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd(count, (uint32_t) __popcll(m));
        base = (uint32_t) __builtin_amdgcn_readfirstlane((int) base);
        const uint32_t pos = base + (uint32_t) lanes_below(m);
        if (keep && pos < (uint32_t) kSortCap) dst[pos] = e;
    }
}

// Sorts src[0..n) into falling order in dst by rank: each entry counts the entries above it (entries are distinct,
// their ids differ). A short list takes T = 2, 4, 8 or 16 threads of one wave per entry, each counting over a 1/T
// share of the list, their counts added by lane shuffles; the list is read as LDS broadcasts, eight entries at a time.
template <int B>
__device__ __forceinline__ void rank_sort(const uint64_t * src, int n, uint64_t * dst) {
    int T = 1;
    while (T < 16 && n * T * 2 <= B) T *= 2;
    const int share = (n + T - 1) / T;
    const int part = (int) threadIdx.x & (T - 1);
    const int j0 = min(n, part * share), j1 = min(n, j0 + share);
    for (int i0 = 0; i0 < n; i0 += B / T) {
        const int i = i0 + (int) threadIdx.x / T;
        const uint64_t e = i < n ? src[i] : ~0ull;
        int r = 0;
        int j = j0;
        for (; j + 8 <= j1; j += 8) {
            uint64_t v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = src[j + u];
#pragma unroll
            for (int u = 0; u < 8; u++) r += v[u] > e ? 1 : 0;
        }
        for (; j < j1; j++) r += src[j] > e ? 1 : 0;
        for (int o = 1; o < T; o <<= 1) r += __shfl_xor(r, o, kWave);
        if (i < n && part == 0) dst[r] = e;
    }
    __syncthreads();
}

// The chunk's candidates at or above `floor`, gathered from buf[0..nb) and sorted into dst; returns how many there
// are (beyond kSortCap only the count is exact).
template <int B>
__device__ __forceinline__ int gather_sort(const uint64_t * buf, int nb, uint64_t floor, uint64_t * tmp, uint64_t * dst,
                                  uint32_t * count) {
    gather_append<B>(buf, nb, floor, tmp, count);
    __syncthreads();
    const int total = (int) *count;
    rank_sort<B>(tmp, min(total, kSortCap), dst);
    return total;
}

// The kernel's launch record where the kernel's arguments lie in memory (it is the kernel's one argument).
__device__ __forceinline__ const Launch * kernel_args() {
    return (const Launch *) __builtin_amdgcn_kernarg_segment_ptr();
}

// ------------------------------------------------------------------------------------------------------------------
// The multi-pass path: exact radix selects over the whole row
// ------------------------------------------------------------------------------------------------------------------

// Fixed-point scale of the masses the selects add up: exact, order-free sums of exp(q - top) rounded to 2^-40.
constexpr double kFix = 1099511627776.0;  // 2^40

__device__ __forceinline__ uint64_t mass_fixed(float q, float top) {
    // -inf weighs 0 (also against a top of -inf, where the reference's weights are NaN and pick() takes its last)
    if (!(q > -INFINITY) || !(top > -INFINITY)) return 0;
    return (uint64_t) (exp((double) q - (double) top) * kFix + 0.5);
}

struct Select {
    uint64_t prefix;   // the high `bits` bits of the entry fixed so far
    int bits;
    uint64_t above_n;  // entries above the prefix's range
    uint64_t above_m;  // their mass, fixed point
    uint64_t entry;    // the entry found
    uint64_t own_m;    // its own mass
};

// One row's whole-vocabulary state in the work-group that resolves it.
struct FbRow {
    const Launch * a;
    int row;
    spx_row_params p;
    Plan pl;
    Specials sp;
    const uint32_t * banned_row;
    float top;  // the largest final quotient
    Red * red;
    uint32_t * n_own;
    // A read that needs only quotients within a range: the raw logits that can reach it (a conservative window), so
    // that every other token other than the special ones is passed over before its division. win false: every token.
    bool win = false;
    float wlo = -INFINITY, whi = INFINITY;
};

// Visits every token of the row, chunk by chunk: f(entry, final logit, quotient, banned, id), the entry 0 for a NaN
// quotient; a banned token is visited as -inf, once; a history token with its penalized logit, once. The chunk's
// special tokens are those the kernel built in LDS when the launch has one chunk per row, else they are rebuilt per
// chunk. Whole 16-byte vectors are read a step ahead of the step being visited (kE tokens per lane per step), so that
// a pass runs at the rate of the loads rather than their latency.
template <typename T, int B, typename F>
__device__ __forceinline__ void fb_visit(FbRow & r, F && f) {
    constexpr int V = Elt<T>::V, U = Elt<T>::U;
    const Launch & a = *r.a;
    const T * rowp = (const T *) a.logits + logits_row(a, r.row) * a.ld;
    const bool spec = r.pl.pen || r.banned_row;
    const uint32_t ninf = order_key(-INFINITY);
    const int tid = threadIdx.x;
    // one token: its special bit, then its quotient. A special token is visited after the chunk's stream: a banned one
    // from the ban mask's words, a history token from the list. (No other memory is read per token, so that the wait
    // for the next step's vectors comes only at the step's end.)
    auto visit = [&](int c0, int i, float x) __attribute__((always_inline)) {
        if (spec) {
            const int o = i - c0;
            if ((r.sp.kill[o >> 5] >> (o & 31)) & 1u) return;
        }
        if (r.win && !(x >= r.wlo && x <= r.whi)) return;  // its quotient lies outside the read's range (or NaN)
        const float q = div_rn(x, r.pl.t, r.pl.rt);
        f(__builtin_isnan(q) ? 0ull : make_entry(order_key(q), (uint32_t) i), x, q, false, i);
    };
    // the same for a token of a vector whose special bits are known (one read of the word for the vector's V tokens)
    auto visit_known = [&](int i, float x, bool special) __attribute__((always_inline)) {
        if (special) return;
        if (r.win && !(x >= r.wlo && x <= r.whi)) return;
        const float q = div_rn(x, r.pl.t, r.pl.rt);
        f(__builtin_isnan(q) ? 0ull : make_entry(order_key(q), (uint32_t) i), x, q, false, i);
    };
    for (int c0 = 0; c0 < a.vocab; c0 += a.chunk) {
        const int c1 = min(a.vocab, c0 + a.chunk);
        if (spec && a.splits > 1) {
            __syncthreads();  // the previous chunk's special tokens are read no more
            uint32_t bad = 0;
            int h0, h1;
            hist_range(a, r.row, r.pl, h0, h1, bad);
            build_specials<B>(r.sp, c0, c1, r.pl, r.banned_row, a.hist, h0, h1, -1, r.n_own);
        } else if (spec) {
            r.sp.n_own = min((int) *r.n_own, r.sp.own_cap);  // built by the kernel for the whole row
        }
        const int ng = a.vec_ok ? (c1 - c0) / V : 0;  // whole vectors
        const U32x4 * vp = (const U32x4 *) (rowp + c0);
        constexpr int per = U * B;
        // Loads are issued only here, into nxt; a step's vectors are copied out of it at the step's start (its one
        // wait), then the next step's are requested. The first turn only requests step 0: with no load before the
        // loop, no register the steps work in has a load pending on it when the loop is entered, and the compiler
        // waits for memory once a step rather than at each reuse of a register.
        U32x4 nxt[U];
#pragma unroll
        for (int u = 0; u < U; u++) nxt[u] = U32x4{0u, 0u, 0u, 0u};
        for (int g0 = -per; g0 < ng; g0 += per) {
            U32x4 cur[U];
#pragma unroll
            for (int u = 0; u < U; u++) cur[u] = nxt[u];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int g = g0 + per + tid + u * B;
                nxt[u] = g < ng ? vp[g] : U32x4{0u, 0u, 0u, 0u};
            }
            if (g0 < 0) continue;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int g = g0 + tid + u * B;
                if (g < ng) {
                    float x[V];
                    unpack<T>(cur[u], x);
                    // the vector's V special bits: one word holds them (V divides 32, the vector starts at a
                    // multiple of V from c0)
                    const uint32_t kb = spec ? r.sp.kill[(g * V) >> 5] >> ((g * V) & 31) : 0u;
#pragma unroll
                    for (int j = 0; j < V; j++) visit_known(c0 + g * V + j, x[j], (kb >> j) & 1u);
                }
            }
        }
        for (int i = c0 + ng * V + tid; i < c1; i += B) visit(c0, i, load_one<T>(rowp + i));
        if (r.banned_row) {
            // the banned tokens as -inf, once each (history or not: restricted() bans after the penalty); c0 is a
            // multiple of 64, so the chunk's words are whole words of the mask
            for (int w = (c0 >> 5) + tid; w < (c1 + 31) >> 5; w += B) {
                uint32_t bw = r.banned_row[w];
                while (bw) {
                    const int i = (w << 5) + __builtin_ctz(bw);
                    bw &= bw - 1u;
                    if (i < c1) f(make_entry(ninf, (uint32_t) i), -INFINITY, -INFINITY, true, i);
                }
            }
        }
        if (r.pl.pen) {
            for (int k = tid; k < r.sp.n_own; k += B) {
                int cnt;
                const int id = own_token(r.sp, r.pl, k, cnt);
                if (id < 0) continue;
                const float v = hist_value<T>(id, cnt, r.p, rowp);
                const float q = div_rn(v, r.pl.t, r.pl.rt);
                f(__builtin_isnan(q) ? 0ull : make_entry(order_key(q), (uint32_t) id), v, q, false, id);
            }
        }
    }
    if (spec && a.splits > 1) __syncthreads();
}

// The first entry in falling order whose running count (by_mass false) or running mass reaches `target` (strict:
// passes it), by radix passes of 8 bits over the 64-bit entries. False when no entry does.
template <typename T, int B>
__device__ __forceinline__ bool fb_select(FbRow & r, bool by_mass, uint64_t target, bool strict, Select & out,
                                 uint32_t * hist_n, unsigned long long * hist_m) {
    int * ired = r.red->i;
    Select s;
    s.prefix = 0;
    s.bits = 0;
    s.above_n = 0;
    s.above_m = 0;
    s.own_m = 0;
    unsigned long long * shared = (unsigned long long *) r.red->u;
    while (s.bits < 64) {
        for (int i = threadIdx.x; i < 256; i += B) {
            hist_n[i] = 0;
            hist_m[i] = 0;
        }
        __syncthreads();
        const int shift = 56 - s.bits;
        const uint64_t pre = s.prefix;
        const int bits = s.bits;
        const float top = r.top;
        fb_visit<T, B>(r, [&](uint64_t e, float, float q, bool, int) {
            if (!e) return;
            if (bits == 0 || (e >> (64 - bits)) == pre) {
                const int d = (int) ((e >> shift) & 255u);
                atomicAdd(&hist_n[d], 1u);
                atomicAdd(&hist_m[d], (unsigned long long) mass_fixed(q, top));
            }
        });
        __syncthreads();
        if (threadIdx.x == 0) {
            uint64_t cn = s.above_n, cm = s.above_m;
            int found = -1;
            for (int d = 255; d >= 0; d--) {
                const uint64_t nn = cn + hist_n[d], nm = cm + hist_m[d];
                const uint64_t v = by_mass ? nm : nn;
                if (hist_n[d] && (strict ? v > target : v >= target)) {
                    found = d;
                    break;
                }
                cn = nn;
                cm = nm;
            }
            ired[0] = found;
            shared[0] = cn;
            shared[1] = cm;
            shared[2] = found >= 0 ? hist_m[found] : 0;
        }
        __syncthreads();
        const int d = ired[0];
        const uint64_t cn = shared[0], cm = shared[1], own = shared[2];
        __syncthreads();
        if (d < 0) return false;
        s.prefix = (s.prefix << 8) | (uint64_t) d;
        s.bits += 8;
        s.above_n = cn;
        s.above_m = cm;
        s.own_m = own;
    }
    s.entry = s.prefix;
    out = s;
    return true;
}

// Resolves one row the one-pass path could not finish, in a work-group of its own row, with exact passes over the
// whole row: the flags and the row status, then radix selects. `extra` carries the flags found before (a history
// longer than the handle allows).
template <typename T, int B>
__device__ __forceinline__ void fallback_row(const Launch & a, int row, const spx_row_params & p, const Plan & pl,
                                    uint32_t extra, unsigned char * lds) {
    const int tid = threadIdx.x;
    Red * red = (Red *) (lds + a.off_red);
    uint32_t * hist_n = (uint32_t *) (lds + a.off_sort);
    unsigned long long * hist_m = (unsigned long long *) (lds + a.off_sort + 1024);
    FbRow r;
    r.a = kernel_args();
    r.row = row;
    r.p = p;
    r.pl = pl;
    r.banned_row = a.banned ? a.banned + (int64_t) row * a.banned_stride : nullptr;
    specials_at(r.sp, a, lds);
    r.sp.any = pl.pen || r.banned_row;
    r.top = 0.0f;
    r.red = red;
    r.n_own = &((Ctl *) (lds + a.off_ctl))->n_own;
    // The flags, exactly, and the first and last entries of the order.
    uint32_t fl = 0;
    uint64_t hi_e = 0, lo_e = ~0ull;
    fb_visit<T, B>(r, [&](uint64_t e, float v, float q, bool banned, int id) {
        if (!banned) {
            if (__builtin_isnan(v)) fl |= kNaN;
            else if (v == INFINITY) fl |= kPosInf;
            else if (v == -INFINITY) fl |= kNegInf;
            else {
                fl |= kFinite;
                if (!__builtin_isfinite(q)) fl |= q > 0.0f ? (kTempOver | kTempOverPos) : kTempOver;
            }
            if (id == 0 && __builtin_isnan(v)) fl |= kNaN0;
        }
        if (e) {
            hi_e = e > hi_e ? e : hi_e;
            lo_e = e < lo_e ? e : lo_e;
        }
    });
    fl = block_or_u32<B>(fl, red->w) | (extra & kBadHist);
    hi_e = block_max_u64<B>(hi_e, red->u);
    lo_e = block_min_u64<B>(lo_e, red->u);
    const bool top_finite = hi_e != 0 && __builtin_isfinite(entry_value(hi_e));
    const int st = row_status(pl, p, fl, top_finite);
    if (st >= 0) {
        if (tid == 0) write_row(a, row, -1, st, 0);
        return;
    }
    r.top = entry_value(hi_e);
    // The total mass over the row, as the selects count it.
    unsigned long long * tot_m = (unsigned long long *) &red->u[16];
    if (tid == 0) *tot_m = 0;
    __syncthreads();
    {
        unsigned long long mine = 0;
        const float top = r.top;
        fb_visit<T, B>(r, [&](uint64_t e, float, float q, bool, int) {
            if (e) mine += mass_fixed(q, top);
        });
        atomicAdd(tot_m, mine);
    }
    __syncthreads();
    const uint64_t all_m = *tot_m;
    __syncthreads();
    const double u = a.u[(int64_t) row * a.u_stride];
    const int fl_ = pl.flavor;
    auto sel = [&](bool by_mass, uint64_t target, bool strict, Select & out) {
        return fb_select<T, B>(r, by_mass, target, strict, out, hist_n, hist_m);
    };
    // The flavor's k candidates: the k-th entry and their mass.
    uint64_t kmass = all_m, kcount = (uint64_t) a.vocab;
    Select sk;
    bool have_k_entry = false;
    if (pl.k < a.vocab && sel(false, (uint64_t) pl.k, false, sk)) {
        kmass = sk.above_m + sk.own_m;
        kcount = sk.above_n + 1;
        have_k_entry = true;
    }
    // The kept prefix: its last entry, count and mass.
    uint64_t kept_m = kmass, kept_n = kcount;
    Select scut;
    bool have_cut = false;
    if (fl_ == SPX_FLAVOR_TRANSFORMERS || fl_ == SPX_FLAVOR_HARU) {
        // transformers keeps the token reaching top_p (qwen3-tts/sampler.cpp:92-96); torch's zeroing in
        // sample_token keeps the same prefix, the tokens after it weighing 0 (haru/sampler.cpp:52-59)
        const bool applies = fl_ == SPX_FLAVOR_TRANSFORMERS ? pl.top_p < 1.0f : (pl.top_p > 0.0f && pl.top_p < 1.0f);
        if (applies) {
            const uint64_t target = (uint64_t) ((double) kmass * (double) pl.top_p + 0.5);
            if (sel(true, target, false, scut) && scut.above_n + 1 <= kcount) {
                kept_m = scut.above_m + scut.own_m;
                kept_n = scut.above_n + 1;
                have_cut = true;
            }
        }
    } else {
        // fish-speech drops the token passing top_p, the first always kept (drama3/sampler.cpp:53-58)
        const uint64_t target = (uint64_t) ((double) all_m * (double) pl.top_p + 0.5);
        if (sel(true, target, true, scut) && scut.above_n < kcount) {
            kept_m = scut.above_n >= 1 ? scut.above_m : scut.own_m;
            kept_n = scut.above_n >= 1 ? scut.above_n : 1;
            have_cut = true;
        }
    }
    // pick(): the first kept entry whose running share passes u, else the last kept.
    Select spk;
    int id = -1;
    const uint64_t utarget = (uint64_t) ((double) kept_m * u);
    // pick()'s last: the last kept entry for TRANSFORMERS and FISH, which draw over the kept set alone; Haru's pick()
    // runs over all k weights (those past the kept prefix weigh 0), so any entry of the kept prefix is a hit there
    const bool found = sel(true, utarget, true, spk);
    const bool hit = found && (fl_ == SPX_FLAVOR_HARU ? spk.above_n < kept_n : spk.above_n + 1 < kept_n);
    if (hit) {
        id = (int) entry_id(spk.entry);
    } else if (fl_ == SPX_FLAVOR_HARU) {
        // pick() over all k weights, zeros included: the k-th token
        id = have_k_entry ? (int) entry_id(sk.entry) : (int) entry_id(lo_e);
    } else if (have_cut && fl_ == SPX_FLAVOR_TRANSFORMERS) {
        id = (int) entry_id(scut.entry);
    } else if (have_cut) {
        Select sl;
        if (sel(false, kept_n, false, sl)) id = (int) entry_id(sl.entry);
    } else if (have_k_entry) {
        id = (int) entry_id(sk.entry);
    } else {
        id = (int) entry_id(lo_e);
    }
    const int kept_list = fl_ == SPX_FLAVOR_HARU ? pl.k : (int) kept_n;
    if (tid == 0) {
        write_row(a, row, id, SPX_ROW_OK, kept_list);
        atomicAdd(a.fb_count, 1);  // rows resolved past the one-pass path since the handle was made
    }
    if (!a.out_cand_ids) return;
    // The listed candidates: the entry at the list's length by a count select, then every entry at or above it
    // gathered and sorted (at most max_out <= 256 of them).
    const int nlist = min(kept_list, a.max_out);
    for (int j = nlist + tid; j < a.max_out; j += B) {
        a.out_cand_ids[(int64_t) row * a.max_out + j] = -1;
        a.out_cand_w[(int64_t) row * a.max_out + j] = 0.0;
    }
    Select sl;
    if (nlist == 0 || !sel(false, (uint64_t) nlist, false, sl)) return;
    uint64_t * lst = (uint64_t *) (lds + a.off_cand);  // 2 x kKeep entries, before the histograms at off_sort
    uint32_t * nl = &((Ctl *) (lds + a.off_ctl))->ncomp;
    if (tid == 0) *nl = 0u;
    __syncthreads();
    fb_visit<T, B>(r, [&](uint64_t e, float, float, bool, int) {
        if (e && e >= sl.entry) {
            const uint32_t at = atomicAdd(nl, 1u);
            if (at < (uint32_t) kKeep) lst[at] = e;
        }
    });
    __syncthreads();
    const int n = min((int) *nl, nlist);
    rank_sort<B>(lst, n, lst + kKeep);
    const double skd = (double) kmass / kFix;  // the top k's mass relative to the largest weight
    for (int i = tid; i < n; i += B) {
        const uint64_t e = lst[kKeep + i];
        const float q = entry_value(e);
        const double w = q > -INFINITY ? exp((double) q - (double) r.top) : 0.0;
        double out;
        if (fl_ == SPX_FLAVOR_TRANSFORMERS) out = w / skd;
        else if (fl_ == SPX_FLAVOR_HARU) out = (uint64_t) i < kept_n ? (double) (float) (w / skd) : 0.0;
        else out = w;
        a.out_cand_ids[(int64_t) row * a.max_out + i] = (int32_t) entry_id(e);
        a.out_cand_w[(int64_t) row * a.max_out + i] = out;
    }
}


// ------------------------------------------------------------------------------------------------------------------
// The wide path: rows whose draw runs past the candidates held
// ------------------------------------------------------------------------------------------------------------------
//
// A row whose top-k set or top-p set is larger than the buffer holds is resolved with further reads of the row in the
// same work-group. The first builds a histogram in LDS of the row's final quotients: bins 1/64 wide below the largest
// quotient (its last finite bin takes everything more than 32 below), plus one bin for the tokens at -inf, each with
// its token count and the exact sum of the tokens' masses exp(q - top) in fixed point, so that the sums do not depend
// on the order of the additions. The prefix sums of the bins then name the bin that holds each answer: the k-th token,
// the token where the top-p rule cuts, the pick, the last kept token, the candidates listed. A read gathers the tokens
// of those bins alone; each gathered token counts the tokens of its bin above it and their mass, which gives its rank
// and its cumulative mass in the row's order, and the one token whose place answers a question writes itself. A
// question whose answer depends on another's gets a range of bins from the bins of that one, so that usually one
// gathering read answers all; where the bins of the exact questions alone hold more tokens than LDS takes, the row
// goes to the radix path.

// Bins per unit of quotient (a power of two, so that the bin of a quotient is exact).
constexpr float kWideScale = 64.0f;

// exp(q - top) * 2^shift rounded to an integer, 0 for q = -inf: the exponent's integer part split off exactly in double,
// the fraction raised by one float exp2 (relative error about 1e-7).
__device__ __forceinline__ uint64_t fixed_mass(float q, float top, int shift) {
    if (!(q > -INFINITY)) return 0;
    const double a = ((double) q - (double) top) * 1.4426950408889634074;
    if (!(a > -(double) (shift + 2))) return 0;  // below 2^-2 of a unit: rounds to 0
    const double n = __builtin_floor(a);
    const float f = (float) (a - n);
    const double v = __builtin_ldexp((double) __builtin_amdgcn_exp2f(f), shift + (int) n);
    return (uint64_t) (v + 0.5);
}

// The bin of a finite quotient q <= top: the distance below the top in 1/64 units, the last finite bin beyond.
template <int NB>
__device__ __forceinline__ int wide_bin(float q, float top) {
    const float d = (top - q) * kWideScale;
    return d < (float) (NB - 1) ? (int) d : NB - 1;
}

// The raw-logit window of the bins b0..b1 (NB - 1 the last finite bin, NB the -inf one): quotients in
// (top - (b1 + 1) / 64, top - b0 / 64], widened by far more than the roundings of the bin's arithmetic and of the
// division (2^-16 relative), then the logits whose correctly rounded quotient can fall there (the division by t > 0
// is monotone), widened again. Tokens outside are in none of the bins.
template <int NB>
__device__ __forceinline__ void set_window(FbRow & r, float top, int b0, int b1) {
    constexpr float kRel = 1.0f / 65536.0f;
    const float slack = (__builtin_fabsf(top) + 1.0f) * kRel;
    const float qhi = top - (float) b0 / kWideScale + slack;
    const float qlo = b1 >= NB - 1 ? -INFINITY : top - (float) (b1 + 1) / kWideScale - slack;
    const float t = r.pl.t;
    r.win = true;
    r.whi = qhi * t + __builtin_fabsf(qhi * t) * kRel + 1e-30f;
    r.wlo = qlo == -INFINITY ? -INFINITY : qlo * t - __builtin_fabsf(qlo * t) * kRel - 1e-30f;
}

// Sorts v[0..n) in falling order (bitonic, over the next power of two, padded with 0, below every entry); v holds at
// least that many. Ends with a barrier.
template <int B, typename K>
__device__ __forceinline__ void block_sort_desc(K * v, int n) {
    int p = 1;
    while (p < n) p <<= 1;
    for (int i = n + (int) threadIdx.x; i < p; i += B) v[i] = 0ull;
    for (int size = 2; size <= p; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (int i = threadIdx.x; i < (p >> 1); i += B) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool down = (lo & size) == 0;
                const K x = v[lo], y = v[hi];
                if ((x < y) == down) {
                    v[lo] = y;
                    v[hi] = x;
                }
            }
        }
    }
    __syncthreads();
}
template <int B>
__device__ __forceinline__ void block_sort_desc_u64(uint64_t * v, int n) {
    block_sort_desc<B, uint64_t>(v, n);
}

// Exclusive prefix sum of one 64-bit value per thread over the work-group; `total` gets the sum. red: LDS of B/64.
template <int B>
__device__ __forceinline__ uint64_t block_excl_scan_u64(uint64_t v, uint64_t * red, uint64_t & total) {
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    uint64_t inc = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const uint64_t t = __shfl_up(inc, (unsigned) o, kWave);
        if (lane >= o) inc += t;
    }
    if (lane == kWave - 1) red[wave] = inc;
    __syncthreads();
    uint64_t base = 0, tot = 0;
    for (int w = 0; w < B / kWave; w++) {
        const uint64_t x = red[w];
        if (w < wave) base += x;
        tot += x;
    }
    __syncthreads();
    total = tot;
    return base + inc - v;
}

// A question the wide path answers: the token at a rank, or the first token whose cumulative mass reaches a target
// (GE: >=) or passes it (GT: >). lo..hi: the target or the range it lies in while it depends on another answer.
enum WideKind : int { kQNone = 0, kQRank = 1, kQGe = 2, kQGt = 3 };
struct WideQ {
    int kind;
    bool exact;       // the target is known
    bool done;
    uint64_t lo, hi;  // target (rank, or fixed-point mass), lo == hi when exact
    // the answer
    uint64_t entry;
    uint64_t before, through;  // cumulative mass of the tokens above it, and with it
    uint32_t rank;
};
enum WideQIdx : int { kQK = 0, kQCut = 1, kQPick = 2, kQLast = 3 };

// The first bin whose tokens bring the cumulative count past `rank` (pre_cnt[b] <= rank < pre_cnt[b + 1]).
// The fixed-point mass of an entry's quotient (0 for -inf).
__device__ __forceinline__ uint64_t entry_mass(uint64_t e, float top, int shift) {
    const float q = entry_value(e);
    return q > -INFINITY ? fixed_mass(q, top, shift) : 0ull;
}

// pre[i] = the masses of ent[0..i) (ent sorted, n <= CAP), each thread a run of CAP / B of them. Ends with a barrier.
template <int B, int CAP>
__device__ __forceinline__ void excl_mass_scan(const uint64_t * ent, uint64_t * pre, int n, float top, int shift,
                                               uint64_t * red) {
    constexpr int P = CAP / B;
    const int i0 = (int) threadIdx.x * P;
    uint64_t ms[P];
    uint64_t sum = 0;
#pragma unroll
    for (int j = 0; j < P; j++) {
        ms[j] = i0 + j < n ? entry_mass(ent[i0 + j], top, shift) : 0ull;
        sum += ms[j];
    }
    uint64_t total;
    uint64_t base = block_excl_scan_u64<B>(sum, red, total);
#pragma unroll
    for (int j = 0; j < P; j++) {
        if (i0 + j < n) pre[i0 + j] = base;
        base += ms[j];
    }
    __syncthreads();
}

template <int NB>
__device__ __forceinline__ int bin_of_rank(const uint32_t * pre_cnt, uint64_t rank) {
    int lo = 0, hi = NB;  // pre_cnt[0] = 0 <= rank < pre_cnt[NB + 1]
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if ((uint64_t) pre_cnt[mid] <= rank) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}
// The bin holding the first token whose cumulative mass reaches x (ge) or passes it (gt); NB + 1 when none does.
template <int NB>
__device__ __forceinline__ int bin_of_mass(const uint64_t * pre_mass, uint64_t x, bool gt) {
    // the first b with pre_mass[b + 1] >= x (ge) or > x (gt)
    int lo = 0, hi = NB + 1;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        const uint64_t c = pre_mass[mid + 1];
        if (gt ? c > x : c >= x) hi = mid;
        else lo = mid + 1;
    }
    return lo;
}

// The bins a question reads: its target's bin, or the bins its target range spans (lo..hi inclusive; hi < lo: none).
template <int NB>
__device__ __forceinline__ void question_bins(const WideQ & q, const uint32_t * pre_cnt, const uint64_t * pre_mass,
                                              int & b0, int & b1) {
    b0 = 1;
    b1 = 0;
    if (q.kind == kQNone || q.done) return;
    if (q.kind == kQRank) {
        b0 = bin_of_rank<NB>(pre_cnt, q.lo);
        b1 = bin_of_rank<NB>(pre_cnt, q.hi);
    } else {
        const bool gt = q.kind == kQGt;
        b0 = bin_of_mass<NB>(pre_mass, q.lo, gt);
        b1 = min(bin_of_mass<NB>(pre_mass, q.hi, gt), NB);
    }
}

// Haru's float32 exponential of a token: std::exp of the float difference from the largest quotient, in float
// (src/families/haru/sampler.cpp:47), correctly rounded.
__device__ __forceinline__ float haru_exp(float q, float top) {
    return q > -INFINITY ? (float) exp((double) (q - top)) : 0.0f;
}

// Half a unit in the last place of a positive float s: a term below it leaves s as it is when added.
__device__ __forceinline__ float half_ulp(float s) {
    if (!(s > 0.0f)) return 0.0f;
    const int e = (int) ((__float_as_uint(s) >> 23) & 0xffu);
    return e > 24 ? __uint_as_float((uint32_t) (e - 24) << 23) : 0x1p-149f * 0.5f;
}

// Gathers the tokens of the contiguous bins b0..b1 (at most CAP of them) and writes them to out[] in the row's order:
// out[i] is the token of rank pre_cnt[b0] + i.
template <typename T, int B, int NB, int CAP>
__device__ __forceinline__ void gather_in_order(FbRow & r, WideMem<NB, CAP> & m, float top, int b0, int b1,
                                                uint64_t * out) {
    const int tid = threadIdx.x;
    const uint32_t base = m.pre_cnt[b0];
    for (int b = b0 + tid; b <= b1; b += B) m.seg[b] = m.pre_cnt[b] - base;
    __syncthreads();
    set_window<NB>(r, top, b0, b1);
    fb_visit<T, B>(r, [&](uint64_t e, float, float qq, bool banned, int) {
        if (!e) return;
        const int b = (banned || !(qq > -INFINITY)) ? NB : wide_bin<NB>(qq, top);
        if (b < b0 || b > b1) return;
        m.ent[atomicAdd(&m.seg[b], 1u)] = e;
    });
    r.win = false;
    __syncthreads();
    // the batch's bins hold falling ranges of entries: sorted, the tokens are in the row's order
    const int n = (int) (m.pre_cnt[b1 + 1] - base);
    block_sort_desc_u64<B>(m.ent, n);
    for (int i = tid; i < n; i += B) out[i] = m.ent[i];
    __syncthreads();
}

// The tokens of bin b (a finite bin before the last) when they are a run of one value, at most 2 x CAP of them: their
// entries' low words (the ids complemented) sorted falling, so ids rising, which is the row's order, in the words at
// m.ent. Returns the run's key + 1, or 0 when the bin holds more than one value, or more than 2 x CAP tokens. With
// any_len a longer run is found too, its ids not kept.
template <typename T, int B, int NB, int CAP>
__device__ __forceinline__ uint64_t gather_run(FbRow & r, WideMem<NB, CAP> & m, float top, int b, bool any_len = false) {
    const int tid = threadIdx.x;
    const uint32_t n = m.pre_cnt[b + 1] - m.pre_cnt[b];
    if (b >= NB - 1 || (n > (uint32_t) (2 * CAP) && !any_len)) return 0;
    uint32_t * gid = (uint32_t *) m.ent;
    uint32_t * kr = (uint32_t *) m.wb;  // the bin's smallest and largest key
    if (tid == 0) {
        m.n_gath = 0u;
        kr[0] = ~0u;
        kr[1] = 0u;
    }
    __syncthreads();
    set_window<NB>(r, top, b, b);
    uint32_t klo = ~0u, khi = 0u;
    fb_visit<T, B>(r, [&](uint64_t e, float, float qq, bool banned, int) {
        if (!e || banned || !(qq > -INFINITY) || wide_bin<NB>(qq, top) != b) return;
        const uint32_t at = atomicAdd(&m.n_gath, 1u);
        if (at < (uint32_t) (2 * CAP)) gid[at] = (uint32_t) e;
        klo = min(klo, entry_key(e));
        khi = max(khi, entry_key(e));
    });
    r.win = false;
    if (klo != ~0u) {
        atomicMin(&kr[0], klo);
        atomicMax(&kr[1], khi);
    }
    __syncthreads();
    const bool run = m.n_gath == n && kr[0] == kr[1];
    const uint32_t key = kr[0];
    __syncthreads();
    if (!run) return 0;
    if (n <= (uint32_t) (2 * CAP)) block_sort_desc<B, uint32_t>(gid, (int) n);
    return (uint64_t) key + 1;
}

// The last bin of a batch starting at bin b0 whose tokens fit CAP; -1 when bin b0 alone holds more.
template <int NB, int CAP>
__device__ __forceinline__ int batch_end(const WideMem<NB, CAP> & m, int b0) {
    if (m.pre_cnt[b0 + 1] - m.pre_cnt[b0] > (uint32_t) CAP) return -1;
    int b1 = b0;
    while (b1 < NB && m.pre_cnt[b1 + 2] - m.pre_cnt[b0] <= (uint32_t) CAP) b1++;
    return b1;
}

// Haru's sums in float32, as src/families/haru/sampler.cpp:44-59 adds them, token after token in the row's order: the
// sum of the top k exponentials (sum_f), and, with 0 < top_p < 1, the running sum of the probabilities that zeroes every
// token whose sum before it reaches top_p. Both are taken by one lane over batches of bins gathered in order; the sum
// stops at the first term below half a unit of it (every later term is smaller and leaves it as it is), the zeroing
// once the running sum has passed top_p by two units (every later token is zeroed). Where top_p applies this also
// resolves the row: its pick and its listed candidates. A bin of more tokens than a batch takes is a batch of its own
// when it is a run of one value (gather_run). Returns 0: the row is not resolved here (the pick is left to the
// fixed-point questions), 1: resolved, -1: a bin holds more tokens than a batch takes and is no such run.
template <typename T, int B, int NB, int CAP>
__device__ __forceinline__ int haru_exact(const Launch & a, int row, const Plan & pl, FbRow & r, WideMem<NB, CAP> & m,
                                          float top, uint64_t lowest, float & sum_out) {
    const int tid = threadIdx.x;
    const uint64_t k = (uint64_t) pl.k;
    uint64_t * ord = m.mass;  // the batch in the row's order
    float * sh = (float *) m.red;
    // the sum of the top k exponentials
    float sumf = 0.0f;
    {
        int b0 = 0;
        bool stop = false;
        while (!stop && b0 <= NB && m.pre_cnt[b0] < k) {
            // The tokens from bin b0 on weigh at most what its upper edge does (widened past the roundings of the
            // bins): below half a unit of the sum, the sum is final (the far bin, too large for a batch, among them).
            if (b0 > 0) {
                const float qhi = b0 == NB ? -INFINITY
                                           : top - (float) b0 / kWideScale + (__builtin_fabsf(top) + 1.0f) * (1.0f / 65536.0f);
                if (haru_exp(qhi, top) < half_ulp(sumf)) break;
            }
            int b1 = batch_end(m, b0);
            const uint64_t runk = b1 < 0 ? gather_run<T, B>(r, m, top, b0, true) : 0;  // the sum needs no ids
            if (b1 < 0 && !runk) return -1;
            if (runk) b1 = b0;
            else gather_in_order<T, B>(r, m, top, b0, b1, ord);
            if (tid == 0) {
                const uint32_t base = m.pre_cnt[b0];
                const int n = (int) (m.pre_cnt[b1 + 1] - base);
                const float erun = runk ? haru_exp(key_float((uint32_t) (runk - 1)), top) : 0.0f;
                float s = sumf;
                bool st = false;
                for (int i = 0; i < n && !st; i++) {
                    if (base + (uint32_t) i >= k) {
                        st = true;
                        break;
                    }
                    const float e = runk ? erun : haru_exp(entry_value(ord[i]), top);
                    if (e < half_ulp(s)) st = true;
                    else s += e;
                }
                sh[0] = s;
                sh[1] = st ? 1.0f : 0.0f;
            }
            __syncthreads();
            sumf = sh[0];
            stop = sh[1] != 0.0f;
            __syncthreads();
            b0 = b1 + 1;
        }
    }
    sum_out = sumf;
    if (!(pl.top_p > 0.0f && pl.top_p < 1.0f)) return 0;

    // The zeroing, the weights' double sum, the listed candidates; then the pick. One lane keeps the state in LDS.
    const float tp = pl.top_p;
    const float stop_at = __uint_as_float(__float_as_uint(tp) + 2u);
    const double u = a.u[(int64_t) row * a.u_stride];
    const int nl = a.out_cand_ids ? (int) min((uint64_t) a.max_out, k) : 0;
    double * dsh = (double *) &m.red[4];
    uint64_t * ush = &m.red[8];
    // state: cum (float), done zeroing; total (double); pick found, cumulative share (double)
    if (tid == 0) {
        sh[0] = 0.0f;
        sh[1] = 0.0f;
        dsh[0] = 0.0;
        dsh[1] = 0.0;
        ush[0] = 0;
        ush[1] = 0;
        ush[2] = 0;  // a place the sweeps need lies in a run whose ids are not kept
    }
    __syncthreads();
    for (int sweep = 0; sweep < 2; sweep++) {
        // sweep 0: the zeroing and the total of the weights; sweep 1: pick() over them
        int b0 = 0;
        bool stop = false;
        while (!stop && b0 <= NB && m.pre_cnt[b0] < k) {
            int b1 = batch_end(m, b0);
            const uint64_t runk = b1 < 0 ? gather_run<T, B>(r, m, top, b0, true) : 0;
            if (b1 < 0 && !runk) return -1;
            if (runk) b1 = b0;
            else gather_in_order<T, B>(r, m, top, b0, b1, ord);
            const uint32_t base = m.pre_cnt[b0];
            const int n = (int) (m.pre_cnt[b1 + 1] - base);
            // a run longer than 2 x CAP keeps no ids: the weights run through it, but a listed candidate or the pick
            // inside it sends the row to the radix path
            const bool ids = !runk || n <= 2 * CAP;
            if (tid == 0) {
                // the batch's entry at place i: a run's from its sorted ids
                const uint32_t * gid = (const uint32_t *) m.ent;
                auto at = [&](int i) { return runk ? ((runk - 1) << 32) | (uint64_t) gid[i] : ord[i]; };
                const float erun = runk ? haru_exp(key_float((uint32_t) (runk - 1)), top) : 0.0f;
                float cum = sh[0];
                bool st = false;
                double total = dsh[0], share = dsh[1];
                for (int i = 0; i < n && !st; i++) {
                    const uint64_t rank = base + (uint64_t) i;
                    if (rank >= k) {
                        st = true;
                        break;
                    }
                    const float e = runk ? erun : haru_exp(entry_value(ord[i]), top);
                    const float pr = e / sumf;
                    const float c = cum + pr;
                    const bool zero = !(c - pr < tp);
                    cum = c;
                    const double w = zero ? 0.0 : (double) pr;
                    if (sweep == 0) {
                        total += w;
                        if (rank < (uint64_t) nl) {
                            if (!ids) {
                                ush[2] = 1;
                                st = true;
                                break;
                            }
                            a.out_cand_ids[(int64_t) row * a.max_out + (int64_t) rank] = (int32_t) entry_id(at(i));
                            a.out_cand_w[(int64_t) row * a.max_out + (int64_t) rank] = w;
                        }
                        if (zero && cum >= stop_at && rank + 1 >= (uint64_t) nl) st = true;
                    } else {
                        // src/common/sampling.cpp:9-19 over the k weights; its last is the k-th token
                        share += w / total;
                        if (rank + 1 < k && share > u) {
                            if (ids) {
                                ush[0] = 1;
                                ush[1] = at(i);
                            } else {
                                ush[2] = 1;
                            }
                            st = true;
                        } else if (zero && cum >= stop_at) {
                            st = true;  // every later weight is 0: the share rises no more
                        }
                    }
                }
                sh[0] = cum;
                sh[1] = st ? 1.0f : 0.0f;
                dsh[0] = total;
                dsh[1] = share;
            }
            __syncthreads();
            stop = sh[1] != 0.0f;
            if (ush[2]) return -1;  // every thread reads it before any writes it again
            __syncthreads();
            b0 = b1 + 1;
        }
        if (tid == 0) {
            sh[0] = 0.0f;
            sh[1] = 0.0f;
            dsh[1] = 0.0;
        }
        __syncthreads();
    }
    // no weight passed u before the last of the k: pick() answers the k-th token
    uint64_t pick = ush[0] ? ush[1] : 0;
    if (!pick && k == (uint64_t) a.vocab) {
        pick = lowest;
    } else if (!pick) {
        const int b = bin_of_rank<NB>(m.pre_cnt, k - 1);
        if (m.pre_cnt[b + 1] - m.pre_cnt[b] > (uint32_t) CAP) {
            const uint64_t runk = gather_run<T, B>(r, m, top, b);
            if (!runk) return -1;
            pick = ((runk - 1) << 32) | (uint64_t) ((const uint32_t *) m.ent)[k - 1 - m.pre_cnt[b]];
        } else {
            gather_in_order<T, B>(r, m, top, b, b, ord);
            pick = ord[k - 1 - m.pre_cnt[b]];
        }
    }
    if (tid == 0) {
        write_row(a, row, (int) entry_id(pick), SPX_ROW_OK, (int) k);
        atomicAdd(a.fb_count, 1);
    }
    for (int j = nl + tid; j < a.max_out && a.out_cand_ids; j += B) {
        a.out_cand_ids[(int64_t) row * a.max_out + j] = -1;
        a.out_cand_w[(int64_t) row * a.max_out + j] = 0.0;
    }
    return 1;
}

// The row's answers from its histogram and at most a few gathering reads. Returns false when a question's bins hold
// more tokens than LDS takes (the caller then takes the radix path).
template <typename T, int B>
__device__ __forceinline__ bool wide_row(const Launch & a, int row, const spx_row_params & p, const Plan & pl, float top,
                                         unsigned char * lds) {
    constexpr int NB = WideDims<B>::NB, CAP = WideDims<B>::CAP;
    using Mem = WideMem<NB, CAP>;
    Mem & m = *(Mem *) (lds + a.off_cand);
    const int tid = threadIdx.x;
    const int shift = 62 - (a.vocab > 1 ? 32 - __builtin_clz((uint32_t) (a.vocab - 1)) : 0);
    FbRow r;
    r.a = kernel_args();
    r.row = row;
    r.p = p;
    r.pl = pl;
    r.banned_row = a.banned ? a.banned + (int64_t) row * a.banned_stride : nullptr;
    specials_at(r.sp, a, lds);
    r.sp.any = pl.pen || r.banned_row;
    r.top = top;
    r.red = (Red *) (lds + a.off_red);
    r.n_own = &((Ctl *) (lds + a.off_ctl))->n_own;

    // The histogram: counts in pre_cnt, masses in pre_mass (made prefix sums below).
    for (int i = tid; i < NB + 2; i += B) {
        m.pre_cnt[i] = 0;
        m.pre_mass[i] = 0;
    }
    if (tid == 0) m.lo_e = ~0ull;
    __syncthreads();
    uint64_t lo_e = ~0ull;
    // the crowded bins, counted in registers: -inf tokens, and tokens of the last finite bin whose mass rounds to 0
    uint32_t n_ninf = 0, n_far = 0;
    fb_visit<T, B>(r, [&](uint64_t e, float, float q, bool banned, int) {
        if (!e) return;  // NaN: none in a row that reaches here
        lo_e = e < lo_e ? e : lo_e;
        if (banned || !(q > -INFINITY)) {
            n_ninf++;
            return;
        }
        const int b = wide_bin<NB>(q, top);
        const uint64_t fm = fixed_mass(q, top, shift);
        if (b == NB - 1 && !fm) {
            n_far++;
            return;
        }
        atomicAdd(&m.pre_cnt[b], 1u);
        if (fm) atomicAdd((unsigned long long *) &m.pre_mass[b], (unsigned long long) fm);
    });
    lo_e = wave_min_u64(lo_e);
    n_ninf = (uint32_t) wave_sum_i32((int) n_ninf);
    n_far = (uint32_t) wave_sum_i32((int) n_far);
    if (lane_id() == 0) {
        atomicMin((unsigned long long *) &m.lo_e, (unsigned long long) lo_e);
        if (n_ninf) atomicAdd(&m.pre_cnt[NB], n_ninf);
        if (n_far) atomicAdd(&m.pre_cnt[NB - 1], n_far);
    }
    __syncthreads();
    // prefix sums over the NB + 1 bins, each thread a contiguous run of them
    {
        constexpr int P = (NB + 1 + B - 1) / B;
        const int b0 = min(tid * P, NB + 1), b1 = min(b0 + P, NB + 1);
        uint32_t c = 0;
        uint64_t s = 0;
        for (int b = b0; b < b1; b++) {
            c += m.pre_cnt[b];
            s += m.pre_mass[b];
        }
        int ctot;
        uint64_t stot;
        const int cb = block_excl_scan_i32<B>((int) c, r.red->i, ctot);
        const uint64_t sb = block_excl_scan_u64<B>(s, m.red, stot);
        uint32_t cr = (uint32_t) cb;
        uint64_t sr = sb;
        uint32_t cnt[P];
        uint64_t ms[P];
        for (int j = 0; j < P; j++) {
            const int b = b0 + j;
            cnt[j] = b < b1 ? m.pre_cnt[b] : 0u;
            ms[j] = b < b1 ? m.pre_mass[b] : 0ull;
        }
        __syncthreads();
        for (int j = 0; j < P; j++) {
            const int b = b0 + j;
            if (b < b1) {
                m.pre_cnt[b] = cr;
                m.pre_mass[b] = sr;
                cr += cnt[j];
                sr += ms[j];
            }
        }
        if (tid == 0) {
            m.pre_cnt[NB + 1] = (uint32_t) ctot;
            m.pre_mass[NB + 1] = stot;
        }
        __syncthreads();
    }
    const uint64_t total = m.pre_mass[NB + 1];
    const uint64_t lowest = m.lo_e;
    // Haru's float32 sums, token after token: the zeroing rows are resolved there, the others keep its sum of the top k
    // for their listed weights and draw by the questions below
    float haru_sum = 1.0f;
    if (pl.flavor == SPX_FLAVOR_HARU) {
        const int h = haru_exact<T, B>(a, row, pl, r, m, top, lowest, haru_sum);
        if (h < 0) return false;
        if (h > 0) return true;
    }

    // The questions of the row's flavor (the rules of src/families/qwen3-tts/sampler.cpp:77-99,
    // src/families/haru/sampler.cpp:36-59, src/families/drama3/sampler.cpp:44-59 and src/common/sampling.cpp:9-19).
    const int fl = pl.flavor;
    const uint64_t k = (uint64_t) pl.k;
    const double u = a.u[(int64_t) row * a.u_stride];
    WideQ q[kWideQs];
    for (int i = 0; i < kWideQs; i++) {
        q[i].kind = kQNone;
        q[i].exact = true;
        q[i].done = false;
        q[i].lo = q[i].hi = 0;
    }
    const bool has_k = k < (uint64_t) a.vocab;
    if (has_k) {
        q[kQK].kind = kQRank;
        q[kQK].lo = q[kQK].hi = k - 1;
    }
    const bool cut_tf = (fl == SPX_FLAVOR_TRANSFORMERS && pl.top_p < 1.0f) ||
                        (fl == SPX_FLAVOR_HARU && pl.top_p > 0.0f && pl.top_p < 1.0f);
    const bool cut_fish = fl == SPX_FLAVOR_FISH;
    if (cut_tf || cut_fish) q[kQCut].kind = cut_tf ? kQGe : kQGt;
    q[kQPick].kind = kQGt;
    // What is known so far of the top-k mass, the kept count and the kept mass.
    uint64_t sk_lo = total, sk_hi = total;  // mass of the top k
    bool sk_known = !has_k;
    uint64_t kept_n = k, km_lo = total, km_hi = total;
    bool kept_known = false;
    bool pick_fell = false;  // the pick passed no kept token before the last: it is the last kept token

    auto ceil_mul = [](double f, uint64_t x) { return (uint64_t) __builtin_ceil(f * (double) x); };
    auto floor_mul = [](double f, uint64_t x) { return (uint64_t) __builtin_floor(f * (double) x); };

    // Refreshes the targets of the questions from what is known.
    auto targets = [&]() {
        if (has_k && q[kQK].done) {
            sk_lo = sk_hi = q[kQK].through;
            sk_known = true;
        } else if (has_k) {
            const int b = bin_of_rank<NB>(m.pre_cnt, k - 1);
            sk_lo = m.pre_mass[b];
            sk_hi = m.pre_mass[b + 1];
        }
        if (q[kQCut].kind != kQNone && !q[kQCut].done) {
            const double tp = (double) pl.top_p;
            if (cut_tf) {
                q[kQCut].lo = ceil_mul(tp, sk_lo);
                q[kQCut].hi = ceil_mul(tp, sk_hi);
            } else {
                q[kQCut].lo = q[kQCut].hi = floor_mul(tp, total);
            }
            q[kQCut].exact = q[kQCut].lo == q[kQCut].hi;
        }
        // the kept set
        if (q[kQCut].kind == kQNone) {
            kept_n = k;
            km_lo = sk_lo;
            km_hi = sk_hi;
            kept_known = sk_known;
        } else if (q[kQCut].done) {
            const WideQ & c = q[kQCut];
            if (cut_tf) {
                // transformers keeps the token reaching top_p; Haru zeroes every token after it
                kept_n = (uint64_t) c.rank + 1;
                km_lo = km_hi = c.through;
                kept_known = true;
            } else if (c.rank == ~0u || (uint64_t) c.rank >= k) {
                // fish-speech: no token of the top k passes top_p, all k are kept
                kept_n = k;
                km_lo = sk_lo;
                km_hi = sk_hi;
                kept_known = sk_known;
            } else {
                // fish-speech drops the token passing top_p; the first token always stays
                kept_n = c.rank >= 1 ? (uint64_t) c.rank : 1;
                km_lo = km_hi = c.rank >= 1 ? c.before : c.through;
                kept_known = true;
            }
        } else {
            // the cut's bins bound the kept mass
            int b0, b1;
            question_bins<NB>(q[kQCut], m.pre_cnt, m.pre_mass, b0, b1);
            km_lo = m.pre_mass[min(b0, NB + 1)];
            km_hi = m.pre_mass[min(b1 + 1, NB + 1)];
            if (cut_fish) km_hi = max(km_hi, sk_hi);
        }
        if (!q[kQPick].done) {
            q[kQPick].lo = floor_mul(u, km_lo);
            q[kQPick].hi = floor_mul(u, km_hi);
            q[kQPick].exact = kept_known;
        }
    };

    // Whether every bin question i reads is among those gathered.
    auto gathered = [&](int i) {
        int b0, b1;
        question_bins<NB>(q[i], m.pre_cnt, m.pre_mass, b0, b1);
        for (int b = b0; b <= b1 && b <= NB; b++)
            if (!((m.need[b >> 5] >> (b & 31)) & 1u)) return false;
        return true;
    };
    // After an answer: the pick either hit a kept token before pick()'s last, or its answer is that last token (the
    // k-th for Haru, whose pick() runs over all k weights; the last kept otherwise), often already known.
    auto settle_pick = [&]() {
        if (!q[kQPick].done || pick_fell || !kept_known) return;
        const WideQ & P = q[kQPick];
        const bool hit = P.rank != ~0u && (fl == SPX_FLAVOR_HARU ? (uint64_t) P.rank < kept_n
                                                                 : (uint64_t) P.rank + 1 < kept_n);
        if (hit) return;
        pick_fell = true;
        const uint64_t last = fl == SPX_FLAVOR_HARU ? k - 1 : kept_n - 1;
        q[kQLast].kind = kQRank;
        q[kQLast].lo = q[kQLast].hi = last;
        q[kQLast].exact = true;
        uint64_t known = 0;
        if (q[kQCut].done && q[kQCut].rank != ~0u && (uint64_t) q[kQCut].rank == last) known = q[kQCut].entry;
        else if (has_k && q[kQK].done && last == k - 1) known = q[kQK].entry;
        else if (last + 1 == (uint64_t) a.vocab) known = lowest;
        if (known) {
            q[kQLast].done = true;
            q[kQLast].entry = known;
        }
    };

    // A question whose target is known but whose one bin holds more tokens than a read gathers: a finer histogram of
    // that bin alone (SNB sub-bins: the bin's quotient range cut evenly; the last finite bin's over the 64 below it;
    // the -inf bin's by token id, its order), then a read that gathers the sub-bin holding the target.
    constexpr int SNB = NB / 2;
    auto refine = [&](int i) -> bool {
        WideQ & Q = q[i];
        int b, b1;
        question_bins<NB>(Q, m.pre_cnt, m.pre_mass, b, b1);
        if (b > NB) {  // no token reaches the target
            Q.done = true;
            Q.entry = 0;
            Q.before = Q.through = total;
            Q.rank = ~0u;
            return true;
        }
        if constexpr (sizeof(T) == 2) {
            // bfloat16 logits crowd a bin with one value: a read of the run's ids answers the question (each token
            // weighs the same, so the target's place is arithmetic, and the run's order is by id)
            const uint64_t runk = gather_run<T, B>(r, m, top, b);
            if (runk) {
                const uint32_t key = (uint32_t) (runk - 1);
                const float qk = key_float(key);
                const uint64_t m1 = qk > -INFINITY ? fixed_mass(qk, top, shift) : 0ull;
                const uint64_t base_c = m.pre_cnt[b], base_m = m.pre_mass[b];
                const uint64_t ng = m.pre_cnt[b + 1] - m.pre_cnt[b];
                uint64_t j;
                if (Q.kind == kQRank) j = Q.lo - base_c;
                else if (m1 == 0) j = 0;
                else if (Q.kind == kQGe) j = Q.lo == 0 ? 0 : (Q.lo - base_m + m1 - 1) / m1 - 1;
                else j = (Q.lo - base_m) / m1;
                if (j >= ng) return false;
                const uint64_t entry = ((uint64_t) key << 32) | (uint64_t) ((const uint32_t *) m.ent)[j];
                __syncthreads();
                Q.done = true;
                Q.entry = entry;
                Q.rank = (uint32_t) (base_c + j);
                Q.before = base_m + j * m1;
                Q.through = Q.before + m1;
                return true;
            }
        }
        auto sub_of = [&](float qq, int id) {
            if (b == NB) return (int) (((uint64_t) id * (uint64_t) SNB) / (uint64_t) a.vocab);
            const float x = (top - qq) * kWideScale - (float) b;
            const float y = b == NB - 1 ? x * ((float) SNB / 64.0f) : x * (float) SNB;
            return y < (float) (SNB - 1) ? max((int) y, 0) : SNB - 1;
        };
        auto in_bin = [&](uint64_t e, float qq, bool banned) {
            const bool ninf = banned || !(qq > -INFINITY);
            return e != 0 && (ninf ? NB : wide_bin<NB>(qq, top)) == b;
        };
        // per sub-bin: count, mass, and the smallest and largest key (a sub-bin of one key is a run of equal tokens)
        set_window<NB>(r, top, b, b);  // every read below takes tokens of bin b only
        uint32_t * scnt = (uint32_t *) m.ent;
        uint32_t * smin = scnt + (SNB + 1);
        uint32_t * smax = smin + SNB;
        uint64_t * smass = m.mass;
        for (int j = tid; j <= SNB; j += B) {
            scnt[j] = 0u;
            smass[j] = 0ull;
            if (j < SNB) {
                smin[j] = ~0u;
                smax[j] = 0u;
            }
        }
        __syncthreads();
        // Each thread sums the run of its tokens that fall in one sub-bin in registers and adds it when the sub-bin
        // changes: a bin of one value (a run of equal logits) takes one set of atomics per thread, not per token.
        int acc_sb = -1;
        uint32_t acc_n = 0, acc_lo = ~0u, acc_hi = 0u;
        uint64_t acc_m = 0;
        auto flush = [&]() {
            if (acc_sb < 0) return;
            atomicAdd(&scnt[acc_sb], acc_n);
            atomicMin(&smin[acc_sb], acc_lo);
            atomicMax(&smax[acc_sb], acc_hi);
            if (acc_m) atomicAdd((unsigned long long *) &smass[acc_sb], (unsigned long long) acc_m);
        };
        fb_visit<T, B>(r, [&](uint64_t e, float, float qq, bool banned, int id) {
            if (!in_bin(e, qq, banned)) return;
            const int sb = sub_of(qq, id);
            if (sb != acc_sb) {
                flush();
                acc_sb = sb;
                acc_n = 0;
                acc_lo = ~0u;
                acc_hi = 0u;
                acc_m = 0;
            }
            const uint32_t key = entry_key(e);
            acc_n++;
            acc_lo = min(acc_lo, key);
            acc_hi = max(acc_hi, key);
            acc_m += (banned || !(qq > -INFINITY)) ? 0ull : fixed_mass(qq, top, shift);
        });
        flush();
        __syncthreads();
        // the sub-bin of the target: the first non-empty one whose running count or mass reaches it, found by every
        // thread over its run of sub-bins from the exclusive sums before the run
        {
            constexpr int SP = (SNB + B - 1) / B;
            const int j0 = tid * SP;
            uint32_t cl = 0;
            uint64_t ml = 0;
            for (int k = 0; k < SP; k++)
                if (j0 + k < SNB) {
                    cl += scnt[j0 + k];
                    ml += smass[j0 + k];
                }
            int ctot;
            uint64_t mtot;
            uint32_t c = m.pre_cnt[b] + (uint32_t) block_excl_scan_i32<B>((int) cl, r.red->i, ctot);
            uint64_t ms = m.pre_mass[b] + block_excl_scan_u64<B>(ml, m.red, mtot);
            if (tid == 0) m.wb[0] = SNB;
            __syncthreads();
            int sbm = SNB;
            uint32_t cb = 0;
            uint64_t mb = 0;
            for (int k = 0; k < SP && sbm == SNB; k++) {
                const int j = j0 + k;
                if (j >= SNB) break;
                const uint32_t c1 = c + scnt[j];
                const uint64_t m1 = ms + smass[j];
                bool here;
                if (Q.kind == kQRank) here = Q.lo < (uint64_t) c1;
                else if (Q.kind == kQGe) here = Q.lo == 0 ? true : m1 >= Q.lo;
                else here = m1 > Q.lo;
                if (here && scnt[j] > 0) {
                    sbm = j;
                    cb = c;
                    mb = ms;
                } else {
                    c = c1;
                    ms = m1;
                }
            }
            if (sbm < SNB) atomicMin(&m.wb[0], sbm);
            __syncthreads();
            const int first = m.wb[0];
            if (tid == 0 && first == SNB) {
                m.ans[0].found = 0u;
                m.ans[0].rank = 0u;
                m.n_gath = 0u;
                m.ans[0].entry = 0ull;
            }
            if (sbm < SNB && sbm == first) {
                m.ans[0].found = 1u;
                m.ans[0].rank = (uint32_t) sbm;
                m.ans[0].before = mb;
                m.ans[0].through = cb;
                m.n_gath = scnt[sbm];
                m.ans[0].entry = smin[sbm] == smax[sbm] ? (uint64_t) smin[sbm] + 1 : 0ull;  // its one key + 1
            }
        }
        __syncthreads();
        const int sb = (int) m.ans[0].rank;
        const bool found = m.ans[0].found != 0u;
        const uint64_t base_m = m.ans[0].before, base_c = m.ans[0].through;
        const int ng = (int) m.n_gath;
        const uint64_t one_key = m.ans[0].entry;
        __syncthreads();
        if (!found) {
            Q.done = true;
            Q.entry = 0;
            Q.before = Q.through = total;
            Q.rank = ~0u;
            return true;
        }
        if (ng > CAP && one_key) {
            // A run of ng equal tokens (bfloat16 logits make long ones): each weighs the same, so the target's place
            // in the run is arithmetic, and the run's order is the tokens' order by id; the token at that place is
            // found by a read that gathers the run's ids (up to twice CAP, as 32-bit words), or by a count over id
            // ranges and a read that gathers one range.
            const uint32_t key = (uint32_t) (one_key - 1);
            const float qk = key_float(key);
            const uint64_t m1 = qk > -INFINITY ? fixed_mass(qk, top, shift) : 0ull;
            uint64_t j;
            if (Q.kind == kQRank) j = Q.lo - base_c;
            else if (m1 == 0) j = 0;
            else if (Q.kind == kQGe) j = Q.lo == 0 ? 0 : (Q.lo - base_m + m1 - 1) / m1 - 1;
            else j = (Q.lo - base_m) / m1;
            if (j >= (uint64_t) ng) return false;
            if (ng <= 2 * CAP) {
                // the entries' low words (the ids complemented) of the whole run, sorted falling: ids rising
                uint32_t * gid = (uint32_t *) m.ent;  // CAP entries hold 2 x CAP words
                if (tid == 0) m.n_gath = 0u;
                __syncthreads();
                fb_visit<T, B>(r, [&](uint64_t e, float, float qq, bool banned, int) {
                    if (!in_bin(e, qq, banned) || entry_key(e) != key) return;
                    const uint32_t at = atomicAdd(&m.n_gath, 1u);
                    if (at < (uint32_t) (2 * CAP)) gid[at] = (uint32_t) e;
                });
                __syncthreads();
                if ((int) m.n_gath != ng) return false;  // the run is the sub-bin's tokens: a count that differs is no run
                block_sort_desc<B, uint32_t>(gid, ng);
                const uint64_t entry = ((uint64_t) key << 32) | (uint64_t) gid[j];
                __syncthreads();
                Q.done = true;
                Q.entry = entry;
                Q.rank = (uint32_t) (base_c + j);
                Q.before = base_m + j * m1;
                Q.through = Q.before + m1;
                return true;
            }
            auto idbin = [&](int id) { return (int) (((uint64_t) id * (uint64_t) SNB) / (uint64_t) a.vocab); };
            for (int x = tid; x <= SNB; x += B) scnt[x] = 0u;
            __syncthreads();
            fb_visit<T, B>(r, [&](uint64_t e, float, float qq, bool banned, int id) {
                if (in_bin(e, qq, banned) && entry_key(e) == key) atomicAdd(&scnt[idbin(id)], 1u);
            });
            __syncthreads();
            {
                // the id range holding place j of the run: the first whose running count passes j (the last one where
                // none does), every thread over its run of ranges
                constexpr int SP = (SNB + B - 1) / B;
                const int i0 = tid * SP;
                uint32_t cl = 0;
                for (int k = 0; k < SP; k++)
                    if (i0 + k < SNB) cl += scnt[i0 + k];
                int ctot;
                uint32_t c = (uint32_t) block_excl_scan_i32<B>((int) cl, r.red->i, ctot);
                if (tid == 0) m.wb[0] = SNB - 1;
                __syncthreads();
                int ibm = SNB;
                for (int k = 0; k < SP && ibm == SNB; k++) {
                    const int ib = i0 + k;
                    if (ib >= SNB) break;
                    if (ib == SNB - 1 || (uint64_t) (c + scnt[ib]) > j) ibm = ib;
                    else c += scnt[ib];
                }
                if (ibm < SNB) atomicMin(&m.wb[0], ibm);
                __syncthreads();
                if (ibm < SNB && ibm == m.wb[0]) {
                    m.ans[0].rank = (uint32_t) ibm;
                    m.ans[0].through = c;
                    m.n_gath = 0u;
                }
            }
            __syncthreads();
            const int ib = (int) m.ans[0].rank;
            const uint64_t jb = j - m.ans[0].through;  // the place within the id range
            const uint32_t nib = scnt[ib];
            __syncthreads();
            if (nib > (uint32_t) CAP) return false;
            for (int t = tid; t < kWideQs; t += B) m.ans[t].found = 0u;
            fb_visit<T, B>(r, [&](uint64_t e, float, float qq, bool banned, int id) {
                if (!in_bin(e, qq, banned) || entry_key(e) != key || idbin(id) != ib) return;
                m.ent[atomicAdd(&m.n_gath, 1u)] = e;
            });
            __syncthreads();
            const int n2 = (int) m.n_gath;
            block_sort_desc_u64<B>(m.ent, n2);
            if (tid == 0 && jb < (uint64_t) n2) {
                m.ans[0].entry = m.ent[jb];
                m.ans[0].found = 1u;
            }
            __syncthreads();
            if (!m.ans[0].found) return false;
            Q.done = true;
            Q.entry = m.ans[0].entry;
            Q.rank = (uint32_t) (base_c + j);
            Q.before = base_m + j * m1;
            Q.through = Q.before + m1;
            __syncthreads();
            return true;
        }
        if (ng > CAP) return false;
        if (tid == 0) m.n_gath = 0u;
        __syncthreads();
        fb_visit<T, B>(r, [&](uint64_t e, float, float qq, bool banned, int id) {
            if (!in_bin(e, qq, banned) || sub_of(qq, id) != sb) return;
            m.ent[atomicAdd(&m.n_gath, 1u)] = e;
        });
        for (int t = tid; t < kWideQs; t += B) m.ans[t].found = 0u;
        __syncthreads();
        block_sort_desc_u64<B>(m.ent, ng);
        excl_mass_scan<B, CAP>(m.ent, m.mass, ng, top, shift, m.red);
        for (int x = tid; x < ng; x += B) {
            const uint64_t e = m.ent[x];
            const uint64_t rank = base_c + (uint64_t) x, before = base_m + m.mass[x];
            const uint64_t through = before + entry_mass(e, top, shift);
            bool hit;
            if (Q.kind == kQRank) hit = rank == Q.lo;
            else if (Q.kind == kQGe) hit = Q.lo == 0 ? rank == 0 : (before < Q.lo && Q.lo <= through);
            else hit = before <= Q.lo && Q.lo < through;
            if (hit) {
                m.ans[0].entry = e;
                m.ans[0].before = before;
                m.ans[0].through = through;
                m.ans[0].rank = (uint32_t) rank;
                m.ans[0].found = 1u;
            }
        }
        __syncthreads();
        Q.done = true;
        if (m.ans[0].found) {
            Q.entry = m.ans[0].entry;
            Q.before = m.ans[0].before;
            Q.through = m.ans[0].through;
            Q.rank = m.ans[0].rank;
        } else {
            Q.entry = 0;
            Q.before = Q.through = total;
            Q.rank = ~0u;
        }
        __syncthreads();
        return true;
    };

    // Gathering reads until every question is answered: each read takes the bins of the questions whose targets are
    // known, and while they fit those of the others' target ranges; the tokens it gathers then answer every question
    // whose target becomes known and whose bins they cover.
    constexpr int TPT = CAP / B;  // gathered tokens per thread
    for (int round = 0; round < 12; round++) {
        targets();
        bool open = false;
        for (int i = 0; i < kWideQs; i++) open = open || (q[i].kind != kQNone && !q[i].done);
        if (!open) break;
        // a known target whose bin alone is more than a read gathers: the finer histogram, then the next round
        {
            bool refined = false;
            for (int i = 0; i < kWideQs && !refined; i++) {
                if (q[i].kind == kQNone || q[i].done || !q[i].exact) continue;
                int b0, b1;
                question_bins<NB>(q[i], m.pre_cnt, m.pre_mass, b0, b1);
                if (b0 > NB || m.pre_cnt[min(b1, NB) + 1] - m.pre_cnt[b0] <= (uint32_t) CAP) continue;
                if (!refine(i)) return false;
                refined = true;
            }
            if (refined) {
                targets();
                settle_pick();
                continue;
            }
        }
        for (int i = tid; i < (NB + 1 + 31) / 32; i += B) m.need[i] = 0u;
        __syncthreads();
        uint32_t want = 0;
        for (int pass = 0; pass < 2; pass++) {
            for (int i = 0; i < kWideQs; i++) {
                if (q[i].kind == kQNone || q[i].done || q[i].exact != (pass == 0)) continue;
                int b0, b1;
                question_bins<NB>(q[i], m.pre_cnt, m.pre_mass, b0, b1);
                uint32_t add = 0;
                for (int b = b0; b <= b1 && b <= NB; b++)
                    if (!((m.need[b >> 5] >> (b & 31)) & 1u)) add += m.pre_cnt[b + 1] - m.pre_cnt[b];
                if (want + add > (uint32_t) CAP) continue;  // gathered in a later round
                want += add;
                __syncthreads();
                if (tid == 0)
                    for (int b = b0; b <= b1 && b <= NB; b++) m.need[b >> 5] |= 1u << (b & 31);
                __syncthreads();
            }
        }
        // the segments of the gathered bins, in bin order, and the first and last of them
        if (tid == 0) {
            m.wb[0] = NB + 1;
            m.wb[1] = -1;
        }
        __syncthreads();
        {
            constexpr int P = (NB + 1 + B - 1) / B;
            const int b0 = min(tid * P, NB + 1), b1 = min(b0 + P, NB + 1);
            int c = 0, first = NB + 1, lastb = -1;
            for (int b = b0; b < b1; b++)
                if ((m.need[b >> 5] >> (b & 31)) & 1u) {
                    c += (int) (m.pre_cnt[b + 1] - m.pre_cnt[b]);
                    first = min(first, b);
                    lastb = max(lastb, b);
                }
            if (lastb >= 0) {
                atomicMin(&m.wb[0], first);
                atomicMax(&m.wb[1], lastb);
            }
            int tot;
            int off = block_excl_scan_i32<B>(c, r.red->i, tot);
            for (int b = b0; b < b1; b++) {
                m.seg[b] = (uint32_t) off;
                if ((m.need[b >> 5] >> (b & 31)) & 1u) off += (int) (m.pre_cnt[b + 1] - m.pre_cnt[b]);
            }
            if (tid == 0) m.n_gath = (uint32_t) tot;
            __syncthreads();
        }
        // the gathering read: each token of a needed bin appended to its bin's segment
        if (m.wb[1] >= 0) set_window<NB>(r, top, m.wb[0], m.wb[1]);
        fb_visit<T, B>(r, [&](uint64_t e, float, float qq, bool banned, int) {
            if (!e) return;
            const bool ninf = banned || !(qq > -INFINITY);
            const int b = ninf ? NB : wide_bin<NB>(qq, top);
            if (!((m.need[b >> 5] >> (b & 31)) & 1u)) return;
            m.ent[atomicAdd(&m.seg[b], 1u)] = e;  // its mass follows from the entry once sorted
        });
        r.win = false;
        __syncthreads();
        // each gathered token's rank and cumulative masses, from the tokens of its bin above it, kept in registers
        const int ng = (int) m.n_gath;
        // sorted, the gathered bins keep their segments (a bin holds a falling range of entries), each in the row's
        // order; the masses' running sums give each token's mass above it
        block_sort_desc_u64<B>(m.ent, ng);
        excl_mass_scan<B, CAP>(m.ent, m.mass, ng, top, shift, m.red);
        uint64_t te[TPT], tbefore[TPT], tthrough[TPT], trank[TPT];
#pragma unroll
        for (int x = 0; x < TPT; x++) {
            const int i = tid + x * B;
            te[x] = 0;
            trank[x] = ~0ull;
            tbefore[x] = tthrough[x] = 0;
            if (i >= ng) continue;
            const uint64_t e = m.ent[i];
            const float qq = entry_value(e);
            const int b = !(qq > -INFINITY) ? NB : wide_bin<NB>(qq, top);
            const int s0 = (int) m.seg[b] - (int) (m.pre_cnt[b + 1] - m.pre_cnt[b]);
            te[x] = e;
            trank[x] = (uint64_t) m.pre_cnt[b] + (uint64_t) (i - s0);
            tbefore[x] = m.pre_mass[b] + (m.mass[i] - m.mass[s0]);
            tthrough[x] = tbefore[x] + entry_mass(e, top, shift);
        }
        // answer every question the gathered tokens can, as long as answers make more targets known
        for (int step = 0; step < kWideQs + 1; step++) {
            bool ask[kWideQs];
            bool any = false;
            for (int t = 0; t < kWideQs; t++) {
                ask[t] = q[t].kind != kQNone && !q[t].done && q[t].exact && gathered(t);
                any = any || ask[t];
            }
            if (!any) break;
            for (int t = tid; t < kWideQs; t += B) m.ans[t].found = 0u;
            __syncthreads();
#pragma unroll
            for (int x = 0; x < TPT; x++) {
                if (trank[x] == ~0ull) continue;
                for (int t = 0; t < kWideQs; t++) {
                    if (!ask[t]) continue;
                    const WideQ & Q = q[t];
                    bool hit;
                    if (Q.kind == kQRank) hit = trank[x] == Q.lo;
                    else if (Q.kind == kQGe) hit = Q.lo == 0 ? trank[x] == 0 : (tbefore[x] < Q.lo && Q.lo <= tthrough[x]);
                    else hit = tbefore[x] <= Q.lo && Q.lo < tthrough[x];
                    if (hit) {
                        m.ans[t].entry = te[x];
                        m.ans[t].before = tbefore[x];
                        m.ans[t].through = tthrough[x];
                        m.ans[t].rank = (uint32_t) trank[x];
                        m.ans[t].found = 1u;
                    }
                }
            }
            __syncthreads();
            for (int t = 0; t < kWideQs; t++) {
                if (!ask[t]) continue;
                WideQ & Q = q[t];
                Q.done = true;
                if (m.ans[t].found) {
                    Q.entry = m.ans[t].entry;
                    Q.before = m.ans[t].before;
                    Q.through = m.ans[t].through;
                    Q.rank = m.ans[t].rank;
                } else {
                    // no token reaches the target
                    Q.entry = 0;
                    Q.before = Q.through = total;
                    Q.rank = ~0u;
                }
            }
            __syncthreads();
            targets();
            settle_pick();
        }
        settle_pick();
    }
    for (int i = 0; i < kWideQs; i++)
        if (q[i].kind != kQNone && !q[i].done) return false;
    const uint64_t pick_e = pick_fell ? q[kQLast].entry : q[kQPick].entry;
    const int kept_out = fl == SPX_FLAVOR_HARU ? (int) k : (int) kept_n;
    if (tid == 0) {
        write_row(a, row, (int) entry_id(pick_e), SPX_ROW_OK, kept_out);
        atomicAdd(a.fb_count, 1);  // rows resolved past the one-pass path since the handle was made
    }
    if (!a.out_cand_ids) return true;

    // The listed candidates: the first min(list, max_out) tokens of the order, read in order by batches of bins (one
    // read each; a list of up to a whole vocabulary takes as many as its tokens need).
    const uint64_t nlist = min((uint64_t) kept_out, (uint64_t) a.max_out);
    const double sk = __builtin_ldexp((double) (has_k ? q[kQK].through : total), -shift);  // the top k's mass
    for (int j = (int) nlist + tid; j < a.max_out; j += B) {
        a.out_cand_ids[(int64_t) row * a.max_out + j] = -1;
        a.out_cand_w[(int64_t) row * a.max_out + j] = 0.0;
    }
    for (int b0 = 0; b0 <= NB && (uint64_t) m.pre_cnt[b0] < nlist;) {
        const int b1 = batch_end(m, b0);
        if (b1 < 0) return false;  // one bin holds more tokens than a batch takes
        uint64_t * ord = m.mass;
        gather_in_order<T, B>(r, m, top, b0, b1, ord);
        const uint64_t base = m.pre_cnt[b0];
        const int n = (int) min((uint64_t) m.pre_cnt[b1 + 1], nlist) - (int) base;
        for (int i = tid; i < n; i += B) {
            const uint64_t e = ord[i], rank = base + (uint64_t) i;
            const float qq = entry_value(e);
            const double w = qq > -INFINITY ? exp((double) qq - (double) top) : 0.0;
            double out;
            if (fl == SPX_FLAVOR_TRANSFORMERS) out = w / sk;
            else if (fl == SPX_FLAVOR_HARU) out = rank < kept_n ? (double) (haru_exp(qq, top) / haru_sum) : 0.0;
            else out = w;
            a.out_cand_ids[(int64_t) row * a.max_out + (int64_t) rank] = (int32_t) entry_id(e);
            a.out_cand_w[(int64_t) row * a.max_out + (int64_t) rank] = out;
        }
        __syncthreads();
        b0 = b1 + 1;
    }
    return true;
}

// A row the one-pass path could not finish: its status from the stream's flags and its largest quotient, then the
// wide path, or where the bins it needs hold more tokens than LDS takes, the radix path. `top`: the largest final
// quotient where the one-pass path knows it (its sorted candidates' first), else NaN, and a read finds it.
// The launch record is read where the kernel's arguments lie (ka), so that the kernel keeps no copy of it in scratch
// memory.
template <typename T, int B>
__device__ __forceinline__ void resolve_row(const Launch * ka, int row, const spx_row_params & p, const Plan & pl,
                                            uint32_t F, float top, unsigned char * lds) {
    const Launch & a = *ka;
    if (__builtin_isnan(top)) {
        FbRow r;
        r.a = kernel_args();
        r.row = row;
        r.p = p;
        r.pl = pl;
        r.banned_row = a.banned ? a.banned + (int64_t) row * a.banned_stride : nullptr;
        specials_at(r.sp, a, lds);
        r.sp.any = pl.pen || r.banned_row;
        r.top = 0.0f;
        r.red = (Red *) (lds + a.off_red);
        r.n_own = &((Ctl *) (lds + a.off_ctl))->n_own;
        uint64_t hi = 0;
        fb_visit<T, B>(r, [&](uint64_t e, float, float, bool banned, int) {
            if (e && !banned) hi = e > hi ? e : hi;
        });
        hi = block_max_u64<B>(hi, r.red->u);
        top = hi ? entry_value(hi) : -INFINITY;
    }
    const int st = row_status(pl, p, F, __builtin_isfinite(top) && !(F & kTempOverPos));
    if (st >= 0) {
        if (threadIdx.x == 0) write_row(a, row, -1, st, 0);
        return;
    }
    if (wide_row<T, B>(a, row, p, pl, top, lds)) return;
    __syncthreads();
    fallback_row<T, B>(a, row, p, pl, F, lds);
}

// Leaves a row to the resolving kernel, which runs after this kernel on the same stream.
__device__ __forceinline__ void defer_row(const Launch & a, int row, uint32_t flags, float top) {
    if (threadIdx.x == 0) {
        const uint32_t i = atomicAdd(&a.pend_ctr[a.parity], 1u);
        Pending pe;
        pe.row = row;
        pe.flags = flags;
        pe.top = top;
        pe.pad = 0;
        a.pending[i] = pe;
    }
}

// ------------------------------------------------------------------------------------------------------------------
// Chunks and rows
// ------------------------------------------------------------------------------------------------------------------

__device__ __forceinline__ void xcd_map(int bid, int nwg, int splits, int & row, int & split) {
    // Work-groups are dispatched round-robin over the 8 XCDs; give the chunks of one row consecutive slots of one
    // XCD, so that the partials the last chunk reads were written through the same L2.
    const int x = bid & 7, l = bid >> 3;
    const int per = nwg >> 3, extra = nwg & 7;
    const int g = x * per + min(x, extra) + l;
    row = g / splits;
    split = g - row * splits;
}

// Counts this chunk in after wave 0 has written its partial: a release at agent scope by that wave (the L2 of this
// XCD written back), one atomic per chunk; true in the row's last chunk, whose acquire (its caches invalidated) lets
// every thread then read the other chunks' partials. The other waves take no fence.
template <int B>
__device__ __forceinline__ bool arrive_last(const Launch & a, int row, Ctl * ctl) {
    if (threadIdx.x < kWave) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        if (threadIdx.x == 0) {
            const unsigned prev = __hip_atomic_fetch_add(&a.counters[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const bool last = prev == (unsigned) (a.splits - 1);
            if (last) {
                a.counters[row] = 0;  // ready for the next launch
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            }
            ctl->last = last ? 1u : 0u;
        }
    }
    __syncthreads();
    return ctl->last != 0;
}

// Token 0's final logit, where it is not a history token, for std::max_element's NaN in front.
template <typename T>
__device__ __forceinline__ uint32_t nan0_flag(const T * rowp, const Plan & pl, const Specials & sp, const uint32_t * banned_row) {
    const bool ban0 = banned_row && (banned_row[0] & 1u);
    const bool hist0 = pl.pen && sp.any && (sp.kill[0] & 1u) && !ban0;
    if (ban0 || hist0) return 0u;
    return __builtin_isnan(load_one<T>(rowp)) ? kNaN0 : 0u;
}

template <typename T, int B>
__device__ __forceinline__ void sample_row(const Launch & a, int row, int split, const spx_row_params & p, const Plan & pl,
                                  int c0, int c1, const T * rowp, const uint32_t * banned_row, Specials & sp,
                                  uint32_t bad, unsigned char * lds, const U32x4 (&first)[Elt<T>::U]) {
    constexpr int W = B / kWave;
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    Ctl * ctl = (Ctl *) (lds + a.off_ctl);
    Red * red = (Red *) (lds + a.off_red);
    uint64_t * cand = (uint64_t *) (lds + a.off_cand);
    uint64_t * sorted = (uint64_t *) (lds + a.off_sort);
    const int cap = a.cand_cap;

    SampleSt st;
    st.s = 0.0;
    st.m = -INFINITY;
    st.hi = -FLT_MAX;
    st.tau = -INFINITY;
    st.flags = 0;
    GreedySt g;
    StreamCtx c{&pl, &sp, &st, &g, ctl, cand, cap, rowp};

    // The history tokens (the penalties), one per thread, once the first step has set the bound and the bins: their
    // raw logits read again (the first of each thread's requested before the stream), a term against the wave's
    // reference (raised first where a quotient passes it), the flags, and an entry where the quotient reaches the
    // threshold of the moment (it only rises, so every token at or above the final one is kept).
    const bool hist_pass = pl.pen && sp.n_own > 0;
    float raw0 = 0.0f;
    if (hist_pass && tid < sp.n_own) raw0 = load_one<T>(rowp + sp.own[tid]);
    auto history = [&]() __attribute__((always_inline)) {
        if (!hist_pass) return;
        const uint32_t tk = __hip_atomic_load(&ctl->tau_key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        const float tau = tk ? key_float(tk) : -INFINITY;
        for (int i0 = 0; i0 < sp.n_own; i0 += B) {
            const int i = i0 + tid;
            bool live = i < sp.n_own;
            int hid = 0, cnt = 1;
            float hv = 0.0f;
            if (live) {
                hid = own_token(sp, pl, i, cnt);
                live = hid >= 0;
            }
            if (live) {
                const float raw = i0 == 0 ? raw0 : load_one<T>(rowp + hid);
                hv = penalize(raw, cnt, p);
            }
            float q = -INFINITY;
            if (live && hid == 0 && __builtin_isnan(hv)) st.flags |= kNaN0;
            if (live) {
                q = div_rn(hv, pl.t, pl.rt);
                if (__builtin_isnan(hv)) st.flags |= kNaN;
                else if (hv == INFINITY) st.flags |= kPosInf;
                else if (hv == -INFINITY) st.flags |= kNegInf;
                else {
                    st.flags |= kFinite;
                    if (!__builtin_isfinite(q)) st.flags |= q > 0.0f ? (kTempOver | kTempOverPos) : kTempOver;
                }
            }
            const bool fin = live && q > -INFINITY && q < INFINITY;
            const float wm = uniform_f(wave_max_f32(fin ? q : -INFINITY));
            if (wm > st.m) {
                const float nhi = ref_exponent(wm);
                if (st.m > -INFINITY) st.s = rescale(st.s, st.hi, nhi);
                st.m = wm;
                st.hi = nhi;
            }
            if (fin) st.s += (double) __builtin_amdgcn_exp2f(__builtin_fmaf(q, kL2e, -st.hi));
            if (live && !__builtin_isnan(q) && q >= tau) {
                const uint32_t pos = atomicAdd(&ctl->n, 1u);
                if (pos < (uint32_t) cap) {
                    cand[pos] = make_entry(order_key(q), (uint32_t) hid);
                    if (ctl->bin_scale > 0.0f) atomicAdd(&ctl->bins[value_bin(ctl->bin_lo, ctl->bin_scale, q)], 1u);
                } else {
                    ctl->overflow = 1u;
                }
            }
        }
    };
    if (sp.any) stream_chunk<T, B, true, false>(c, a, rowp, c0, c1, first, history);
    else stream_chunk<T, B, false, false>(c, a, rowp, c0, c1, first, history);

    // The chunk's totals: each wave's sum is relative to 2^hi, hi = ceil(m*L) an integer; moved to the largest
    // exponent H by powers of two, then to the largest quotient M by one factor 2^(H - M*L).
    {
        const double ws = wave_sum_f64(st.s);
        const uint32_t wf = wave_or_u32(st.flags);
        if (lane == 0) {
            red->d[wave] = st.m > -INFINITY ? ws : 0.0;
            red->f[wave] = st.m;
            red->f[32 + wave] = st.hi;
            red->w[wave] = wf;
        }
        if (tid == 0) ctl->ncomp = 0;
    }
    __syncthreads();
    // lane w < W takes wave w's values; every wave reduces them in the same order, so all agree on S, M and F
    const bool has = lane < W;
    const float mw = has ? red->f[lane] : -INFINITY;
    const float hw = has && mw > -INFINITY ? red->f[32 + lane] : -FLT_MAX;
    const float M = uniform_f(wave_max_f32(mw));
    const float H = uniform_f(wave_max_f32(hw));
    uint32_t F = bad | wave_or_u32(has ? red->w[lane] : 0u);
    double S = wave_sum_f64(mw > -INFINITY ? rescale(red->d[lane], hw, H) : 0.0);
    if (M > -INFINITY) S *= exp2(-(double) __builtin_fmaf(M, kL2e, -H));
    // A finite quotient has a term above 0 against the largest one: S > 0. Every logit that is not finite, and every
    // finite one whose quotient is not (the correction step gives NaN for both), went through the exact path, which
    // set the flags.
    if (S > 0.0) F |= kFinite;

    // The candidates at or above the final threshold, gathered, then sorted by rank.
    const uint32_t nres = ctl->n;
    const bool overflow = ctl->overflow != 0 || nres > (uint32_t) cap;
    const int nb = min((int) nres, cap);
    const uint32_t tkey = ctl->tau_key;
    const bool complete = tkey <= order_key(-INFINITY) && !overflow;  // the threshold never left -inf
    // The chunk's floor: at or above every threshold the stream had (every token at or above it is in the buffer),
    // with at least K entries at or above it: from the bins, by every wave alike (no barrier), or the exact K-th key
    // by wave 0 where the bins would leave more than the sort takes (the same choice in every wave).
    uint32_t kk = 0;
    if (!complete) {
        if (ctl->bin_scale > 0.0f) {
            uint32_t held;
            const float tb = bin_bound(ctl, pl.K, held);
            if (tb > -INFINITY && held + 64u <= (uint32_t) kSortCap) kk = order_key(tb);
        }
        kk = (uint32_t) __builtin_amdgcn_readfirstlane((int) kk);
        if (kk == 0) {
            if (tid < kWave) {
                const uint32_t kb = buffer_bound(cand, nb, pl.K);
                if (tid == 0) ctl->kkey = kb;
            }
            __syncthreads();
            kk = ctl->kkey;
        }
    }
    const uint32_t fkey = complete ? tkey : (kk > tkey ? kk : tkey);
    const uint64_t floor = (uint64_t) fkey << 32;
    const int total = gather_sort<B>(cand, nb, floor, sorted, cand, &ctl->ncomp);
    const bool too_many = total > kSortCap;
    const bool broken = overflow || too_many;
    const int ntot = min(total, kSortCap);
    float * pf = (float *) sorted;  // the gathered copy is read no more

    if (a.splits == 1) {
        RowTotals t{0ull, S, M, F};
        if (a.list_all || broken || !finish_block<B>(a, row, p, pl, t, cand, ntot, complete, pf, ctl)) {
            // the largest quotient: the sorted candidates' first, unless entries were dropped
            const float top = broken ? NAN : (ntot > 0 ? entry_value(cand[0]) : -INFINITY);
            defer_row(a, row, F, top);
        }
        return;
    }

    // Publish this chunk's partial; the last chunk of the row to arrive merges them.
    Partial * part = a.partials + (int64_t) row * a.splits + split;
    uint64_t * pc = a.part_cands + ((int64_t) row * a.splits + split) * kKeep;
    const int npub = min(ntot, kKeep);
    if (tid < kWave) {
        for (int i = tid; i < npub; i += kWave) pc[i] = cand[i];
    }
    if (tid == 0) {
        part->best = 0;
        part->floor = ntot > kKeep ? cand[kKeep - 1] : floor;
        part->s = S;
        part->m = M;
        part->flags = F;
        part->n = npub;
        part->complete = (complete && ntot <= kKeep) ? 1 : 0;
        part->broken = broken ? 1 : 0;
    }
    if (!arrive_last<B>(a, row, ctl)) return;
    RowTotals t{0ull, 0.0, -INFINITY, 0u};
    uint64_t fl = 0;
    bool all_complete = true, any_broken = false;
    const Partial * pr = a.partials + (int64_t) row * a.splits;
    for (int s2 = 0; s2 < a.splits; s2++) {
        const Partial q = pr[s2];
        t.flags |= q.flags;
        t.m = fmaxf(t.m, q.m);
        fl = q.floor > fl ? q.floor : fl;
        all_complete = all_complete && q.complete;
        any_broken = any_broken || q.broken;
    }
    for (int s2 = 0; s2 < a.splits; s2++) {
        const Partial q = pr[s2];
        if (q.m > -INFINITY) t.s += q.s * exp((double) q.m - (double) t.m);
    }
    if (t.s > 0.0) t.flags |= kFinite;
    int tot = 0;
    if (!any_broken) {
        // the chunks' entries at or above the highest floor, one chunk after the other, then sorted by rank
        if (tid == 0) ctl->ncomp = 0;
        __syncthreads();
        for (int s2 = 0; s2 < a.splits; s2++) {
            const int ns = pr[s2].n;
            const uint64_t * src = a.part_cands + ((int64_t) row * a.splits + s2) * kKeep;
            gather_append<B>(src, ns, fl, sorted, &ctl->ncomp);
        }
        __syncthreads();
        tot = min((int) ctl->ncomp, kSortCap);
        rank_sort<B>(sorted, tot, cand);
    }
    if (a.list_all || any_broken || !finish_block<B>(a, row, p, pl, t, cand, tot, all_complete, pf, ctl)) {
        const float top = any_broken ? NAN : (tot > 0 ? entry_value(cand[0]) : -INFINITY);
        defer_row(a, row, t.flags, top);
    }
}

template <typename T, int B>
__device__ __forceinline__ void greedy_row(const Launch & a, int row, int split, const spx_row_params & p, const Plan & pl,
                                  int c0, int c1, const T * rowp, const uint32_t * banned_row, Specials & sp,
                                  uint32_t bad, unsigned char * lds, const U32x4 (&first)[Elt<T>::U]) {
    constexpr int W = B / kWave;
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    Ctl * ctl = (Ctl *) (lds + a.off_ctl);
    Red * red = (Red *) (lds + a.off_red);

    GreedySt g;
    g.bx = -INFINITY;
    g.bi = -1;
    g.xmin = INFINITY;
    g.nanb = 0;
    SampleSt st;
    StreamCtx c{&pl, &sp, &st, &g, ctl, nullptr, 0, rowp};
    auto none = []() __attribute__((always_inline)) {};
    if (sp.any) stream_chunk<T, B, true, true>(c, a, rowp, c0, c1, first, none);
    else stream_chunk<T, B, false, true>(c, a, rowp, c0, c1, first, none);

    {
        const uint64_t be = g.bi >= 0 ? make_entry(order_key(g.bx), (uint32_t) g.bi) : 0ull;
        const uint64_t wb = wave_max_u64(be);
        const float wx = -wave_max_f32(-g.xmin);
        const uint32_t f0 = (c0 == 0 && tid == 0) ? nan0_flag<T>(rowp, pl, sp, banned_row) : 0u;
        if (lane == 0) {
            red->u[wave] = wb;
            red->f[wave] = wx;
            red->w[wave] = (g.nanb ? kNaN : 0u) | f0;
        }
    }
    __syncthreads();
    uint64_t best = 0;
    float xmin = INFINITY;
    uint32_t F = bad;
    for (int w = 0; w < W; w++) {
        best = red->u[w] > best ? red->u[w] : best;
        xmin = fminf(xmin, red->f[w]);
        F |= red->w[w];
    }
    __syncthreads();
    if (pl.pen && sp.n_own > 0) {
        uint64_t hb = 0;
        uint32_t hf = 0;
        for (int i = tid; i < sp.n_own; i += B) {
            int cnt;
            const int hid = own_token(sp, pl, i, cnt);
            if (hid < 0) continue;
            const float hv = hist_value<T>(hid, cnt, p, rowp);
            if (hid == 0 && __builtin_isnan(hv)) hf |= kNaN0;
            if (__builtin_isnan(hv)) hf |= kNaN;
            else if (hv == -INFINITY) hf |= kNegInf;
            else {
                const uint64_t e = make_entry(order_key(hv), (uint32_t) hid);
                hb = e > hb ? e : hb;
            }
        }
        const uint64_t b2 = block_max_u64<B>(hb, red->u);
        best = b2 > best ? b2 : best;
        F |= block_or_u32<B>(hf, red->w);
    }
    if (pl.xmin && xmin == -INFINITY) F |= kNegInf;

    if (a.splits == 1) {
        RowTotals t{best, 0.0, 0.0f, F | best_flags(best)};
        if (tid < kWave) finish_wave(a, row, p, pl, t, nullptr, 0, true, nullptr);
        return;
    }
    Partial * part = a.partials + (int64_t) row * a.splits + split;
    if (tid == 0) {
        part->best = best;
        part->flags = F;
        part->n = 0;
        part->broken = 0;
    }
    if (!arrive_last<B>(a, row, ctl)) return;
    RowTotals t{0ull, 0.0, 0.0f, 0u};
    const Partial * pr = a.partials + (int64_t) row * a.splits;
    for (int s2 = 0; s2 < a.splits; s2++) {
        const Partial q = pr[s2];
        t.best = q.best > t.best ? q.best : t.best;
        t.flags |= q.flags;
    }
    t.flags |= best_flags(t.best);
    if (tid < kWave) finish_wave(a, row, p, pl, t, nullptr, 0, true, nullptr);
}

template <typename T, int B>
__global__ __launch_bounds__(B, 4) void sampler_kernel(Launch a) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int tid = threadIdx.x;
    int row, split;
    xcd_map((int) blockIdx.x, a.nwg, a.splits, row, split);
    if (row >= a.rows) return;
    const int c0 = split * a.chunk, c1 = min(a.vocab, c0 + a.chunk);
    const T * rowp = (const T *) a.logits + logits_row(a, row) * a.ld;
    // The row's history offsets and parameters are requested first (they need only the row), then the first step's
    // logits, then the history ids once their offsets are in; the special tokens are built once those are in.
    int h0 = 0, h1 = 0;
    if (a.hist) hist_bounds(a, row, h0, h1);
    spx_row_params p;
    if (a.params) {
        p = a.params[row];
    } else {
        // spx_argmax_rows: std::max_element of the suppressed logits
        p.flavor = SPX_FLAVOR_TRANSFORMERS;
        p.greedy = 1;
        p.temperature = 1.0f;
        p.top_k = 0;
        p.top_p = 1.0f;
        p.repetition_penalty = 1.0f;
        p.presence_penalty = 0.0f;
        p.frequency_penalty = 0.0f;
    }
    U32x4 first[Elt<T>::U];
    load_step<T, B>(a, rowp, c0, c1, 0, first);
    const Plan pl = make_plan(p, a.vocab, a.banned != nullptr, a.hist != nullptr, a.max_out);
    if (pl.mode == kInvalid) {
        if (split == 0 && tid == 0) write_row(a, row, -1, SPX_ROW_INVALID_PARAMS, 0);
        return;
    }
    const uint32_t * banned_row = a.banned ? a.banned + (int64_t) row * a.banned_stride : nullptr;
    Ctl * ctl = (Ctl *) (lds + a.off_ctl);
    const bool sampling = pl.mode != kGreedy;

    if (tid == 0) {
        ctl->n = 0;
        ctl->tau_key = 0;
        ctl->overflow = 0;
        ctl->last = 0;
        ctl->bin_lo = -INFINITY;
        ctl->bin_scale = 0.0f;
        ctl->bin_width = 0.0f;
    }
    if (sampling) {
        uint64_t * cand = (uint64_t *) (lds + a.off_cand);
        for (int i = tid; i < a.cand_cap; i += B) cand[i] = 0;
        for (int i = tid; i < kBins; i += B) ctl->bins[i] = 0;
    }
    uint32_t bad = 0;
    if (!pl.pen) h1 = h0;
    if (h1 - h0 > a.max_hist || h1 < h0) {
        bad |= kBadHist;
        h1 = h0;
    }
    // the first slab of history ids, requested before the LDS set-up
    const int hfirst = h0 + tid < h1 ? a.hist[h0 + tid] : -1;
    Specials sp;
    specials_at(sp, a, lds);
    sp.any = pl.pen || banned_row != nullptr;
    if (sp.any) build_specials<B>(sp, c0, c1, pl, banned_row, a.hist, h0, h1, hfirst, &ctl->n_own);
    __syncthreads();
    if (sampling) sample_row<T, B>(a, row, split, p, pl, c0, c1, rowp, banned_row, sp, bad, lds, first);
    else greedy_row<T, B>(a, row, split, p, pl, c0, c1, rowp, banned_row, sp, bad, lds, first);
}

// The rows the one-pass kernel left: the work-groups take list entries one at a time, each row resolved with its
// special tokens built over the whole row, by the wide path (or the radix path). A launch that finds the list empty
// ends at once. The list's count and the count of entries taken are one of two slots that calls alternate between:
// this kernel clears the other slots, which the next call uses, so that no kernel clears a count it reads. The launch record is this kernel's
// own: one chunk per row, and the LDS layout of the wide path.
template <typename T, int B>
__global__ __launch_bounds__(B, 1) void resolve_kernel(Launch a) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int tid = threadIdx.x;
    if (blockIdx.x == 0 && tid == 0) {
        a.pend_ctr[a.parity ^ 1] = 0u;
        a.pend_ctr[2 + (a.parity ^ 1)] = 0u;
    }
    const uint32_t n = a.pend_ctr[a.parity];
    if (n == 0) return;
    Ctl * ctl = (Ctl *) (lds + a.off_ctl);
    for (;;) {
        // rows are taken one at a time, so that work-groups whose rows resolve fast take more of them
        if (tid == 0) ctl->last = atomicAdd(&a.pend_ctr[2 + a.parity], 1u);
        __syncthreads();
        const uint32_t idx = ctl->last;
        __syncthreads();
        if (idx >= n) break;
        const Pending pe = a.pending[idx];
        const int row = pe.row;
        const spx_row_params p = a.params[row];
        const Plan pl = make_plan(p, a.vocab, a.banned != nullptr, a.hist != nullptr, a.max_out);
        const uint32_t * banned_row = a.banned ? a.banned + (int64_t) row * a.banned_stride : nullptr;
        uint32_t bad = 0;
        int h0, h1;
        hist_range(a, row, pl, h0, h1, bad);
        Specials sp;
        specials_at(sp, a, lds);
        if (pl.pen || banned_row) build_specials<B>(sp, 0, a.vocab, pl, banned_row, a.hist, h0, h1, -1, &ctl->n_own);
        __syncthreads();
        resolve_row<T, B>(kernel_args(), row, p, pl, pe.flags, pe.top, lds);
        __syncthreads();
    }
}

}  // namespace spx

// A variant of the sampling kernel alone (its rows resolved by another variant's resolving kernel): the launcher
// spx::launch_<NAME> and its LDS limit spx::lds_limit_<NAME>.
#define SPX_SAMPLER_VARIANT(T, B, NAME)                                                                         \
    namespace spx {                                                                                             \
    hipError_t launch_##NAME(const Launch & a, hipStream_t s) {                                                 \
        hipLaunchKernelGGL((sampler_kernel<T, B>), dim3(a.nwg), dim3(B), a.lds_bytes, s, a);                    \
        return hipGetLastError();                                                                               \
    }                                                                                                           \
    hipError_t lds_limit_##NAME(int bytes) {                                                                    \
        return hipFuncSetAttribute((const void *) sampler_kernel<T, B>,                                         \
                                   hipFuncAttributeMaxDynamicSharedMemorySize, bytes);                          \
    }                                                                                                           \
    }

// One variant of the kernels: the launchers spx::launch_<NAME> and spx::resolve_<NAME>, and their LDS limit
// spx::lds_limit_<NAME>.
#define SPX_KERNEL_VARIANT(T, B, NAME)                                                                          \
    namespace spx {                                                                                             \
    hipError_t launch_##NAME(const Launch & a, hipStream_t s) {                                                 \
        hipLaunchKernelGGL((sampler_kernel<T, B>), dim3(a.nwg), dim3(B), a.lds_bytes, s, a);                    \
        return hipGetLastError();                                                                               \
    }                                                                                                           \
    hipError_t resolve_##NAME(const Launch & a, int grid, hipStream_t s) {                                       \
        if constexpr (B == kBlockBig) {                                                                         \
            if (a.block == kBlockResolveNarrow)                                                                 \
                hipLaunchKernelGGL((resolve_kernel<T, kBlockResolveNarrow>), dim3(grid), dim3(kBlockResolveNarrow), \
                                   a.lds_bytes, s, a);                                                          \
            else                                                                                                \
                hipLaunchKernelGGL((resolve_kernel<T, kBlockResolve>), dim3(grid), dim3(kBlockResolve),         \
                                   a.lds_bytes, s, a);                                                          \
        } else {                                                                                                \
            hipLaunchKernelGGL((resolve_kernel<T, B>), dim3(grid), dim3(B), a.lds_bytes, s, a);                 \
        }                                                                                                       \
        return hipGetLastError();                                                                               \
    }                                                                                                           \
    hipError_t lds_limit_##NAME(int bytes) {                                                                    \
        hipError_t e = hipFuncSetAttribute((const void *) sampler_kernel<T, B>,                                 \
                                           hipFuncAttributeMaxDynamicSharedMemorySize, bytes);                  \
        if (e != hipSuccess) return e;                                                                          \
        if constexpr (B == kBlockBig) {                                                                         \
            e = hipFuncSetAttribute((const void *) resolve_kernel<T, kBlockResolveNarrow>,                      \
                                    hipFuncAttributeMaxDynamicSharedMemorySize, bytes);                         \
            if (e != hipSuccess) return e;                                                                      \
            return hipFuncSetAttribute((const void *) resolve_kernel<T, kBlockResolve>,                         \
                                       hipFuncAttributeMaxDynamicSharedMemorySize, bytes);                      \
        } else {                                                                                                \
            return hipFuncSetAttribute((const void *) resolve_kernel<T, B>,                                     \
                                       hipFuncAttributeMaxDynamicSharedMemorySize, bytes);                      \
        }                                                                                                       \
    }                                                                                                           \
    }
