// spx_kernels.hip — the gfx950 kernel of the batched token sampler.
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

__device__ __forceinline__ Plan make_plan(const spx_row_params & p, int vocab, bool has_ban, bool has_hist) {
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
    pl.K = pl.mode == kTopK ? k : kKeepFull;
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
// a list, each once: the thread whose atomicOr set a token's bit first appends it. Rows with a frequency penalty also
// count each token's occurrences, in an open-addressing table keyed by token.
struct Specials {
    uint32_t * kill;
    int32_t * own;     // the distinct history tokens of the chunk
    uint32_t * tab;    // frequency counts: tab[2i] the key (token + 1; 0 empty), tab[2i + 1] the count
    int tab_mask;      // table entries - 1, a power of two - 1
    int n_own;
    bool any;
};

__device__ __forceinline__ void specials_at(Specials & sp, const Launch & a, unsigned char * lds) {
    sp.kill = (uint32_t *) (lds + a.off_spec);
    sp.own = (int32_t *) (lds + a.off_own);
    sp.tab = (uint32_t *) (lds + a.off_tab);
    sp.tab_mask = a.tab_mask;
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

// History ids each thread holds: thread t the row's ids t, t + B, ... (a history is at most kMaxHist ids).
template <int B>
struct HistIds {
    static constexpr int R = kMaxHist / B;
    int id[R];
};

// The row's history ids [h0, h1) of the history (-1 past the row's history).
template <int B>
__device__ __forceinline__ void load_hist_ids(const Launch & a, const Plan & pl, int h0, int h1, HistIds<B> & h,
                                              uint32_t & bad) {
#pragma unroll
    for (int r = 0; r < HistIds<B>::R; r++) h.id[r] = -1;
    if (!pl.pen) return;
    if (h1 - h0 > a.max_hist || h1 < h0) {
        bad |= kBadHist;
        h1 = h0;
    }
#pragma unroll
    for (int r = 0; r < HistIds<B>::R; r++) {
        const int j = h0 + (int) threadIdx.x + r * B;
        if (j < h1) h.id[r] = a.hist[j];
    }
}

// The same, the row's offsets read here.
template <int B>
__device__ __forceinline__ void load_hist(const Launch & a, int row, const Plan & pl, HistIds<B> & h, uint32_t & bad) {
    const int h0 = pl.pen ? a.hist_off[row] : 0, h1 = pl.pen ? a.hist_off[row + 1] : 0;
    load_hist_ids<B>(a, pl, h0, h1, h, bad);
}

__device__ __forceinline__ uint32_t token_hash(int t) { return (uint32_t) t * 2654435761u; }

// One occurrence of token t in the frequency table.
__device__ __forceinline__ void count_add(const Specials & sp, int t) {
    const uint32_t h = token_hash(t), key = (uint32_t) t + 1u;
    for (int probe = 0; probe <= sp.tab_mask; probe++) {
        const uint32_t i = (h + (uint32_t) probe) & (uint32_t) sp.tab_mask;
        const uint32_t prev = atomicCAS(&sp.tab[2 * i], 0u, key);
        if (prev == 0u || prev == key) {
            atomicAdd(&sp.tab[2 * i + 1], 1u);
            return;
        }
    }
}

// The occurrences of token t counted by count_add.
__device__ __forceinline__ int count_of(const Specials & sp, int t) {
    const uint32_t h = token_hash(t), key = (uint32_t) t + 1u;
    for (int probe = 0; probe <= sp.tab_mask; probe++) {
        const uint32_t i = (h + (uint32_t) probe) & (uint32_t) sp.tab_mask;
        const uint32_t k = sp.tab[2 * i];
        if (k == key) return (int) sp.tab[2 * i + 1];
        if (k == 0u) return 0;
    }
    return 0;
}

// The chunk's special bits, its list of distinct history tokens and (frequency rows) their counts. c0 is a multiple
// of 64, so the chunk's words are whole words of the ban mask.
template <int B>
__device__ __forceinline__ void build_specials(Specials & sp, int c0, int c1, const Plan & pl, const uint32_t * banned_row,
                                      const HistIds<B> & hist, uint32_t * n_own) {
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
    if (pl.counts) {
        for (int i = tid; i <= 2 * sp.tab_mask + 1; i += B) sp.tab[i] = 0u;
    }
    if (tid == 0) *n_own = 0u;
    __syncthreads();
    if (pl.pen) {
#pragma unroll
        for (int r = 0; r < HistIds<B>::R; r++) {
            const int t = hist.id[r];
            if (t >= c0 && t < c1) {
                const uint32_t bit = 1u << ((t - c0) & 31);
                const uint32_t old = atomicOr(&sp.kill[(t - c0) >> 5], bit);
                if (!(old & bit)) sp.own[atomicAdd(n_own, 1u)] = t;
                if (pl.counts) count_add(sp, t);
            }
        }
        __syncthreads();
        sp.n_own = (int) *n_own;
    }
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

// A distinct history token's final logit: its raw logit, read again from memory, penalized.
template <typename T>
__device__ __forceinline__ float hist_value(const Specials & sp, int t, const spx_row_params & p, const Plan & pl,
                                   const T * rowp) {
    const int c = pl.counts ? count_of(sp, t) : 1;
    return penalize(load_one<T>(rowp + t), c, p);
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
            else if (qe == INFINITY) fl |= xv == INFINITY ? kPosInf : kTempOver;
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
    a.out_ids[row] = status == SPX_ROW_OK ? id : -1;
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
    const double u = a.u ? a.u[row] : 0.0;
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
            for (int j = lane; j < a.max_out; j += kWave) {
                a.out_cand_ids[(int64_t) row * a.max_out + j] = j == 0 ? id : -1;
                a.out_cand_probs[(int64_t) row * a.max_out + j] = j == 0 ? 1.0f : 0.0f;
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
    // vocabulary has a known sum (the stream's). Other rows take the multi-pass path.
    if (!full_known && pl.k < a.vocab && pl.flavor != SPX_FLAVOR_FISH) return false;
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
    double outp[4] = {0.0, 0.0, 0.0, 0.0};  // the candidates' reported weights
    int nout = 0;                           // reported candidates

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
            for (int j = 0; j < 4; j++) outp[j] = kq[j];
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
            double w[4];
            for (int j = 0; j < 4; j++) {
                const float x = valid[j] ? pf[idx[j]] : 0.0f;
                w[j] = x > 0.0f ? (double) x : 0.0;
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
            for (int j = 0; j < 4; j++) outp[j] = w[j];
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
            for (int j = 0; j < 4; j++) outp[j] = kw[j];
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
                a.out_cand_probs[(int64_t) row * a.max_out + i] = (float) outp[j];
            }
        }
        // entries past those written above
        for (int j = min(kept, nk) + lane; j < a.max_out; j += kWave) {
            if (j >= nout) {
                a.out_cand_ids[(int64_t) row * a.max_out + j] = -1;
                a.out_cand_probs[(int64_t) row * a.max_out + j] = 0.0f;
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
        const bool ok = finish_wave(a, row, p, pl, tot, e, min(n, kFinishMax), complete, pf);
        if (threadIdx.x == 0) ctl->resolved = ok ? 1u : 0u;
    }
    __syncthreads();
    return ctl->resolved != 0;
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
};

// Visits every token of the row, chunk by chunk, each chunk's special tokens rebuilt in LDS: f(entry, final logit,
// quotient, banned, id), the entry 0 for a NaN quotient. A banned token is visited as -inf, once.
template <typename T, int B, typename F>
__device__ __forceinline__ void fb_visit(FbRow & r, F && f) {
    const Launch & a = *r.a;
    const T * rowp = (const T *) a.logits + (int64_t) r.row * a.ld;
    const bool spec = r.pl.pen || r.banned_row;
    const uint32_t ninf = order_key(-INFINITY);
    for (int c0 = 0; c0 < a.vocab; c0 += a.chunk) {
        const int c1 = min(a.vocab, c0 + a.chunk);
        if (spec) {
            __syncthreads();  // the previous chunk's special tokens are read no more
            uint32_t bad = 0;
            HistIds<B> hist;
            load_hist<B>(a, r.row, r.pl, hist, bad);
            build_specials<B>(r.sp, c0, c1, r.pl, r.banned_row, hist, r.n_own);
        }
        for (int i = c0 + threadIdx.x; i < c1; i += B) {
            if (spec) {
                const int o = i - c0;
                if ((r.sp.kill[o >> 5] >> (o & 31)) & 1u) {
                    // history tokens are visited below; a banned one (history or not) here
                    if (r.banned_row && ((r.banned_row[i >> 5] >> (i & 31)) & 1u))
                        f(make_entry(ninf, (uint32_t) i), -INFINITY, -INFINITY, true, i);
                    continue;
                }
            }
            const float x = load_one<T>(rowp + i);
            const float q = div_rn(x, r.pl.t, r.pl.rt);
            f(__builtin_isnan(q) ? 0ull : make_entry(order_key(q), (uint32_t) i), x, q, false, i);
        }
        if (r.pl.pen) {
            for (int k = threadIdx.x; k < r.sp.n_own; k += B) {
                const int id = r.sp.own[k];
                const float v = hist_value<T>(r.sp, id, r.p, r.pl, rowp);
                const float q = div_rn(v, r.pl.t, r.pl.rt);
                f(__builtin_isnan(q) ? 0ull : make_entry(order_key(q), (uint32_t) id), v, q, false, id);
            }
        }
    }
    if (spec) __syncthreads();
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
    r.a = &a;
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
                if (!__builtin_isfinite(q)) fl |= kTempOver;
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
    const double u = a.u[row];
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
    const bool hit = sel(true, utarget, true, spk) && spk.above_n + 1 < kept_n;
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
    if (tid == 0) {
        write_row(a, row, id, SPX_ROW_OK, fl_ == SPX_FLAVOR_HARU ? pl.k : (int) kept_n);
        if (a.out_cand_ids) {
            // This path reports the id and the count of the kept candidates alone.
            for (int j = 0; j < a.max_out; j++) {
                a.out_cand_ids[(int64_t) row * a.max_out + j] = -1;
                a.out_cand_probs[(int64_t) row * a.max_out + j] = 0.0f;
            }
        }
        atomicAdd(a.fb_count, 1);  // rows this path has resolved since the handle was made
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
            const bool live = i < sp.n_own;
            int hid = 0;
            float hv = 0.0f;
            if (live) {
                hid = sp.own[i];
                const float raw = i0 == 0 ? raw0 : load_one<T>(rowp + hid);
                hv = penalize(raw, pl.counts ? count_of(sp, hid) : 1, p);
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
                    if (!__builtin_isfinite(q)) st.flags |= kTempOver;
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
        if (broken || !finish_block<B>(a, row, p, pl, t, cand, ntot, complete, pf, ctl)) {
            __syncthreads();
            fallback_row<T, B>(a, row, p, pl, F, lds);
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
    if (any_broken || !finish_block<B>(a, row, p, pl, t, cand, tot, all_complete, pf, ctl)) {
        __syncthreads();
        fallback_row<T, B>(a, row, p, pl, t.flags, lds);
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
            const int hid = sp.own[i];
            const float hv = hist_value<T>(sp, hid, p, pl, rowp);
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
    const T * rowp = (const T *) a.logits + (int64_t) row * a.ld;
    // The row's history offsets and parameters are requested first (they need only the row), then the first step's
    // logits, then the history ids once their offsets are in; the special tokens are built once those are in.
    int h0 = 0, h1 = 0;
    if (a.hist) {
        h0 = a.hist_off[row];
        h1 = a.hist_off[row + 1];
    }
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
    const Plan pl = make_plan(p, a.vocab, a.banned != nullptr, a.hist != nullptr);
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
    HistIds<B> hist;
    load_hist_ids<B>(a, pl, h0, h1, hist, bad);
    Specials sp;
    specials_at(sp, a, lds);
    sp.any = pl.pen || banned_row != nullptr;
    if (sp.any) build_specials<B>(sp, c0, c1, pl, banned_row, hist, &ctl->n_own);
    __syncthreads();
    if (sampling) sample_row<T, B>(a, row, split, p, pl, c0, c1, rowp, banned_row, sp, bad, lds, first);
    else greedy_row<T, B>(a, row, split, p, pl, c0, c1, rowp, banned_row, sp, bad, lds, first);
}

// ------------------------------------------------------------------------------------------------------------------
// Launchers
// ------------------------------------------------------------------------------------------------------------------

hipError_t launch_sampler(const Launch & a, hipStream_t s) {
    if (a.nwg == 0) return hipSuccess;
    if (a.block == kBlockBig) {
        if (a.dtype == SPX_BF16)
            hipLaunchKernelGGL((sampler_kernel<uint16_t, kBlockBig>), dim3(a.nwg), dim3(kBlockBig), a.lds_bytes, s, a);
        else
            hipLaunchKernelGGL((sampler_kernel<float, kBlockBig>), dim3(a.nwg), dim3(kBlockBig), a.lds_bytes, s, a);
    } else {
        if (a.dtype == SPX_BF16)
            hipLaunchKernelGGL((sampler_kernel<uint16_t, kBlockSmall>), dim3(a.nwg), dim3(kBlockSmall), a.lds_bytes, s, a);
        else
            hipLaunchKernelGGL((sampler_kernel<float, kBlockSmall>), dim3(a.nwg), dim3(kBlockSmall), a.lds_bytes, s, a);
    }
    return hipGetLastError();
}

hipError_t set_lds_limits(int bytes) {
    if (bytes <= 65536) return hipSuccess;
    const void * fns[4] = {(const void *) sampler_kernel<float, kBlockBig>, (const void *) sampler_kernel<uint16_t, kBlockBig>,
                           (const void *) sampler_kernel<float, kBlockSmall>,
                           (const void *) sampler_kernel<uint16_t, kBlockSmall>};
    for (const void * f : fns) {
        const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace spx
