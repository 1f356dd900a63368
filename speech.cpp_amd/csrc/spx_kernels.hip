// spx_kernels.hip — the gfx950 kernels of the batched token sampler.
//
// One launch of stream_kernel samples a batch. Each work-group takes one chunk of one row (a row is cut into
// `splits` chunks so that small batches still fill the 256 CUs), reads its logits once from HBM with 16-byte loads,
// and keeps on chip only what the draw needs:
//   - the row's special tokens (history ids, banned ids) as an LDS bitmap over the chunk plus a sorted slot list, so
//     the penalty arithmetic runs once per special token instead of once per logit;
//   - the exact quotient l/T of every logit (Markstein's correction, correctly rounded like the reference's division);
//   - an online (max, sum of exp) pair per thread, summed in double, for the rows whose normalization spans the whole
//     vocabulary (top-k off, or the FISH flavor);
//   - per wave, a buffer of the best entries (key, id) seen so far with a rising threshold: each compaction keeps the
//     wave's exact top K, so the union over waves holds the row's top K without a sort of the row.
// The last work-group of a row (an atomic counter per row, reset by that work-group) merges the chunks' partial
// results, sorts the few hundred surviving entries in LDS and applies the flavor's rule: softmax weights in double,
// the top-p cut, and pick() with the row's uniform. A row whose top-p set runs beyond the entries kept is resolved
// by that same work-group with radix selects over (count, mass) histograms of the whole row.
//
// Citations are relative to the reference checkout (nyosegawa/speech.cpp 0.11.1).

#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/spx_sampler.h"
#include "spx_device.h"
#include "spx_internal.h"

namespace spx {

// ------------------------------------------------------------------------------------------------------------------
// Row plans
// ------------------------------------------------------------------------------------------------------------------

enum Mode : int { kGreedy = 0, kTopK = 1, kFull = 2, kInvalid = 3 };

enum Flag : uint32_t {
    kNaN = 1u,        // a NaN among the final logits
    kTempOver = 8u,   // HARU: a finite logit whose quotient is not finite (src/families/haru/sampler.cpp:34)
    kNaN0 = 16u,      // the final logit of token 0 is NaN (std::max_element then answers 0)
    kBadHist = 64u,   // the row's history is longer than the handle was created for
};

struct Plan {
    int mode;
    int flavor;
    int k;          // the flavor's top-k count: the candidates the reference sorts
    int kc;         // entries kept per wave: min(k, kKeep) for top-k rows, kKeep for full rows
    float t;        // the divisor of the flavor
    float rt;       // 1/t rounded
    float top_p;
    bool need_s;    // sum of exp over the whole vocabulary
    bool need_low;  // the last token in the order, for a draw over the whole vocabulary
    bool pen;       // penalties read the history
    bool counts;    // presence or frequency: the history's counts
};

__device__ inline bool neutral(const spx_row_params & p) {
    return p.repetition_penalty == 1.0f && p.presence_penalty == 0.0f && p.frequency_penalty == 0.0f;
}

__device__ inline Plan make_plan(const spx_row_params & p, int vocab, bool has_ban, bool has_hist) {
    Plan pl;
    pl.flavor = p.flavor;
    pl.top_p = p.top_p;
    pl.pen = !neutral(p) && has_hist;
    pl.counts = pl.pen && (p.presence_penalty != 0.0f || p.frequency_penalty != 0.0f);
    pl.need_s = false;
    pl.need_low = false;
    pl.k = 1;
    pl.kc = 1;
    pl.t = 1.0f;
    pl.rt = 1.0f;
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
        return pl;
    }
    int k;
    if (p.flavor == SPX_FLAVOR_TRANSFORMERS) k = p.top_k > 0 ? min(p.top_k, vocab) : vocab;   // qwen3-tts/sampler.cpp:77
    else if (p.flavor == SPX_FLAVOR_HARU) k = (p.top_k > 0 && p.top_k < vocab) ? p.top_k : vocab;  // haru/sampler.cpp:36
    else k = min(max(p.top_k, 1), vocab);                                                  // drama3/sampler.cpp:44
    pl.k = k;
    pl.t = p.flavor == SPX_FLAVOR_FISH ? fmaxf(p.temperature, 1e-5f) : p.temperature;
    pl.rt = 1.0f / pl.t;
    if (k <= kKeep) {
        pl.mode = kTopK;
        pl.kc = k;
    } else {
        pl.mode = kFull;
        pl.kc = kKeepFull;
    }
    pl.need_s = pl.mode == kFull || p.flavor == SPX_FLAVOR_FISH;
    // The last token of a draw over every token: pick() returns it where u passes every cumulative share.
    pl.need_low = pl.mode == kFull && k == vocab &&
                  (p.flavor == SPX_FLAVOR_HARU || !(p.top_p < 1.0f));
    return pl;
}

// The penalty stage on one history token's raw logit: presence/frequency (no reference counterpart), then
// restricted()'s repetition penalty once (src/families/qwen3-tts/sampler.cpp:37).
__device__ inline float penalize(float x, int count, const spx_row_params & p) {
    if (count > 0) {
        if (p.frequency_penalty != 0.0f) x = __fsub_rn(x, __fmul_rn(p.frequency_penalty, (float) count));
        if (p.presence_penalty != 0.0f) x = __fsub_rn(x, p.presence_penalty);
    }
    if (p.repetition_penalty != 1.0f) x = x < 0.0f ? __fmul_rn(x, p.repetition_penalty) : x / p.repetition_penalty;
    return x;
}

// ------------------------------------------------------------------------------------------------------------------
// Block-wide helpers (kBlock threads)
// ------------------------------------------------------------------------------------------------------------------

template <int B>
__device__ inline int block_excl_scan_i32(int v, int * red, int & total) {
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
__device__ inline double block_sum_f64(double v, double * red) {
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    v = wave_sum_f64(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    double t = 0;
    for (int w = 0; w < B / kWave; w++) t += red[w];
    __syncthreads();
    return t;
}

template <int B>
__device__ inline double block_incl_scan_f64(double v, double * red) {
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    const double inc = wave_incl_scan_f64(v);
    if (lane == kWave - 1) red[wave] = inc;
    __syncthreads();
    double base = 0;
    for (int w = 0; w < wave; w++) base += red[w];
    __syncthreads();
    return base + inc;
}

template <int B>
__device__ inline int block_min_i32(int v, int * red) {
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    for (int m = 32; m >= 1; m >>= 1) v = min(v, __shfl_xor(v, m, kWave));
    if (lane == 0) red[wave] = v;
    __syncthreads();
    int t = red[0];
    for (int w = 1; w < B / kWave; w++) t = min(t, red[w]);
    __syncthreads();
    return t;
}

// Sorts a[0..n) (n a power of two, n <= 2*B*8) into falling order, in LDS.
template <int B>
__device__ inline void block_sort_desc(uint64_t * a, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int t = threadIdx.x; t < (n >> 1); t += B) {
                const int lo = 2 * t - (t & (stride - 1));
                const int hi = lo + stride;
                const bool desc = (lo & size) == 0;
                const uint64_t x = a[lo], y = a[hi];
                if ((x < y) == desc) {
                    a[lo] = y;
                    a[hi] = x;
                }
            }
            __syncthreads();
        }
    }
}

// ------------------------------------------------------------------------------------------------------------------
// The wave's candidate buffer
// ------------------------------------------------------------------------------------------------------------------

// Number of set predicates over the wave.
__device__ __forceinline__ int wave_count(bool p) { return (int) __popcll(ballot(p)); }

// The K-th largest entry of the n entries the wave holds in v[] (kPerLane per lane, 0 for none), 1 <= K <= n. The
// counts of each step are ballots, so the search stays in scalar registers.
__device__ __forceinline__ uint64_t wave_kth_largest(const uint64_t (&v)[kPerLane], int K) {
    // First the K-th largest key (the high word), by a bitwise search from the highest bit where keys differ.
    uint32_t hi = 0, lo = 0xffffffffu;
#pragma unroll
    for (int j = 0; j < kPerLane; j++) {
        if (v[j]) {
            hi = max(hi, entry_key(v[j]));
            lo = min(lo, entry_key(v[j]));
        }
    }
    hi = wave_max_u32(hi);
    lo = wave_min_u32(lo);
    uint32_t key = hi;
    if (hi != lo) {
        const int top = 31 - __builtin_clz(hi ^ lo);
        key = hi & ~((top == 31) ? 0xffffffffu : ((2u << top) - 1u));
        for (int b = top; b >= 0; b--) {
            const uint32_t c = key | (1u << b);
            int cnt = 0;
#pragma unroll
            for (int j = 0; j < kPerLane; j++) cnt += wave_count(v[j] != 0 && entry_key(v[j]) >= c);
            if (cnt >= K) key = c;
        }
    }
    // Entries above that key, and the ties at it.
    int gt = 0, eq = 0;
#pragma unroll
    for (int j = 0; j < kPerLane; j++) {
        gt += wave_count(v[j] != 0 && entry_key(v[j]) > key);
        eq += wave_count(v[j] != 0 && entry_key(v[j]) == key);
    }
    const int need = K - gt;  // 1 <= need <= eq
    // Among the ties, the need-th largest low word (the lowest ids come first).
    uint32_t lw;
    if (need == eq) {
        uint32_t m = 0xffffffffu;
#pragma unroll
        for (int j = 0; j < kPerLane; j++) {
            if (v[j] != 0 && entry_key(v[j]) == key) m = min(m, (uint32_t) v[j]);
        }
        lw = wave_min_u32(m);
    } else {
        lw = 0;
        for (int b = 31; b >= 0; b--) {
            const uint32_t c = lw | (1u << b);
            int cnt = 0;
#pragma unroll
            for (int j = 0; j < kPerLane; j++) cnt += wave_count(v[j] != 0 && entry_key(v[j]) == key && (uint32_t) v[j] >= c);
            if (cnt >= need) lw = c;
        }
    }
    return ((uint64_t) key << 32) | lw;
}

// Keeps the wave's top K of its n entries (exactly K), in buf[0..K); returns the K-th, the new threshold. Out of
// line: it runs a few times per wave and row.
__device__ __attribute__((noinline)) uint64_t wave_compact(uint64_t * buf, int * n, int K) {
    uint64_t v[kPerLane];
    const int lane = lane_id();
    const int cnt = *n;
#pragma unroll
    for (int j = 0; j < kPerLane; j++) {
        const int i = lane + kWave * j;
        v[j] = i < cnt ? buf[i] : 0;
    }
    const uint64_t kth = wave_kth_largest(v, K);
    int pos = 0;
#pragma unroll
    for (int j = 0; j < kPerLane; j++) {
        const bool keep = v[j] != 0 && v[j] >= kth;
        const uint64_t m = ballot(keep);
        if (keep) buf[pos + lanes_below(m)] = v[j];
        pos += __popcll(m);
    }
    *n = pos;
    return kth;
}

struct WaveBuf {
    uint64_t * buf;
    int n;            // entries held (wave-uniform)
    uint64_t thr;     // entries must exceed this to enter
    uint32_t thr_key; // its key: the fast test
    int K;
};

// ------------------------------------------------------------------------------------------------------------------
// Per-lane state of the streaming pass
// ------------------------------------------------------------------------------------------------------------------

struct Lane {
    float bestx;    // greedy: this lane's largest final logit, and the first id holding it
    int besti;
    float lowq;     // the smallest quotient and the largest id holding it: the last token of the order
    int lowi;
    float mx, mn;   // largest and smallest final logits (NaN ignored)
    double s;       // sum of exp(q - m) ...
    float m;        // ... against m, the wave's running largest quotient (the same in every lane)
    uint32_t flags; // kNaN, kTempOver, kNaN0, kBadHist
};

__device__ inline void lane_init(Lane & ln) {
    ln.bestx = -INFINITY;
    ln.besti = -1;
    ln.lowq = INFINITY;
    ln.lowi = -1;
    ln.mx = -INFINITY;
    ln.mn = INFINITY;
    ln.s = 0.0;
    ln.m = -FLT_MAX;
    ln.flags = 0;
}

// ------------------------------------------------------------------------------------------------------------------
// Special tokens of one chunk in LDS: for each 32 tokens a pair of words, the history bits and the banned bits, and
// the number of history tokens before them, so a history token finds its slot in O(1)
// ------------------------------------------------------------------------------------------------------------------

struct Specials {
    uint2 * bits;      // .x history, .y banned
    int32_t * rank;    // history tokens before each word
    int32_t * slot_id; // history ids of the chunk, rising
    float * slot_raw;  // their raw logits, written by the stream
    int32_t * slot_cnt;
    int n_slots;
    bool any;
};

__device__ __forceinline__ int slot_of(const Specials & sp, int w, uint32_t hbits, int bit) {
    return sp.rank[w] + __popc(hbits & ((1u << bit) - 1u));
}

template <int B>
__device__ inline void build_specials(Specials & sp, const Launch & a, int row, int c0, int c1, const Plan & pl,
                                      const uint32_t * banned_row, int * red, uint32_t & bad) {
    const int nw = (c1 - c0 + 31) >> 5;
    const int tid = threadIdx.x;
    for (int w = tid; w < nw; w += B) sp.bits[w] = make_uint2(0u, 0u);
    __syncthreads();
    int h0 = 0, h1 = 0;
    if (pl.pen) {
        h0 = a.hist_off[row];
        h1 = a.hist_off[row + 1];
        if (h1 - h0 > a.max_hist || h1 < h0) {
            bad |= kBadHist;
            h1 = h0;
        }
        for (int j = h0 + tid; j < h1; j += B) {
            const int t = a.hist[j];
            if (t >= c0 && t < c1) atomicOr(&sp.bits[(t - c0) >> 5].x, 1u << ((t - c0) & 31));
        }
    }
    __syncthreads();
    // Ranks and the slot list, each thread taking a run of words.
    const int wpt = (nw + B - 1) / B;
    const int w0 = min(nw, tid * wpt), w1 = min(nw, w0 + wpt);
    int cnt = 0;
    for (int w = w0; w < w1; w++) cnt += __popc(sp.bits[w].x);
    int total;
    int pos = block_excl_scan_i32<B>(cnt, red, total);
    for (int w = w0; w < w1; w++) {
        sp.rank[w] = pos;
        uint32_t b = sp.bits[w].x;
        while (b) {
            const int bit = __builtin_ctz(b);
            b &= b - 1;
            sp.slot_id[pos++] = c0 + (w << 5) + bit;
        }
    }
    sp.n_slots = total;
    __syncthreads();
    if (pl.counts) {
        for (int s = tid; s < total; s += B) sp.slot_cnt[s] = 0;
        __syncthreads();
        for (int j = h0 + tid; j < h1; j += B) {
            const int t = a.hist[j];
            if (t >= c0 && t < c1) {
                const int o = t - c0;
                atomicAdd(&sp.slot_cnt[slot_of(sp, o >> 5, sp.bits[o >> 5].x, o & 31)], 1);
            }
        }
    }
    if (banned_row) {
        for (int w = tid; w < nw; w += B) {
            uint32_t bw = banned_row[(c0 >> 5) + w];
            const int base = c0 + (w << 5);
            if (base + 32 > c1) bw &= (1u << (c1 - base)) - 1u;  // 0 < c1 - base < 32 here
            sp.bits[w].y = bw;
        }
    }
    __syncthreads();
}

// ------------------------------------------------------------------------------------------------------------------
// Finishing a row: the flavor's rule on its sorted top entries
// ------------------------------------------------------------------------------------------------------------------

struct RowTotals {
    uint64_t best;  // greedy: make_entry(key, id) of the first largest final logit (0: none above -inf)
    uint64_t low;   // (key << 32 | ~id) of the last token of the order (all ones: none)
    double s;       // sum of exp(q - m) ...
    float m;        // ... relative to m
    float mx, mn;
    uint32_t flags;
};

// The row status, as the reference's checks order them; -1 when the row goes on.
__device__ inline int row_status(const Plan & pl, const spx_row_params & p, const RowTotals & t, bool top_finite) {
    const uint32_t f = t.flags;
    if (pl.mode == kInvalid || (f & kBadHist)) return SPX_ROW_INVALID_PARAMS;
    const bool pen = !neutral(p);
    const bool posinf = t.mx == INFINITY;
    if (pl.flavor == SPX_FLAVOR_TRANSFORMERS) {
        // restricted(): std::max_element's largest, a NaN in front taken as it (src/families/qwen3-tts/sampler.cpp:43-49)
        if (f & kNaN0) return SPX_ROW_NO_FINITE_LOGIT;
        if (posinf) return pen ? SPX_ROW_REP_PENALTY_OVERFLOW : SPX_ROW_NO_FINITE_LOGIT;
        if (!(t.mx > -INFINITY)) return SPX_ROW_NO_FINITE_LOGIT;
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
    if ((f & kNaN) || posinf || t.mn == -INFINITY) return SPX_ROW_NONFINITE_INPUT;  // drama3/sampler.cpp:35-37
    if (pl.mode == kGreedy) return -1;
    if (!top_finite) return SPX_ROW_TEMPERATURE_OVERFLOW;  // drama3/sampler.cpp:46-47
    return -1;
}

__device__ inline void write_row(const Launch & a, int row, int id, int status, int kept) {
    a.out_ids[row] = status == SPX_ROW_OK ? id : -1;
    if (a.out_status) a.out_status[row] = status;
    if (a.out_kept) a.out_kept[row] = status == SPX_ROW_OK ? kept : 0;
}

// Scratch of the finishing step, in LDS.
struct FinishLds {
    double * w;     // weights, kKeep
    double * red;   // reduction scratch
    int * ired;
    float * pf;     // float weights (HARU), kKeep
};

// Finishes a row from its totals and its n sorted top entries e[0..n). Returns true when the row is done, false when
// it needs the multi-pass path (its top-p set or its draw runs beyond the entries kept).
template <int B>
__device__ inline bool finish_row(const Launch & a, int row, const spx_row_params & p, const Plan & pl,
                                  const RowTotals & tot, const uint64_t * e, int n, bool complete, FinishLds & L) {
    const int tid = threadIdx.x;
    const double u = a.u ? a.u[row] : 0.0;
    const float top = n > 0 ? entry_value(e[0]) : -INFINITY;
    const int st = row_status(pl, p, tot, n > 0 && __builtin_isfinite(top));
    if (st >= 0) {
        if (tid == 0) write_row(a, row, -1, st, 0);
        return true;
    }
    if (pl.mode == kGreedy) {
        // std::max_element: the first largest, or token 0 when its logit is NaN.
        const int id = ((tot.flags & kNaN0) || tot.best == 0) ? 0 : (int) entry_id(tot.best);
        if (tid == 0) {
            write_row(a, row, id, SPX_ROW_OK, 1);
            if (a.out_cand_ids) {
                for (int j = 0; j < a.max_out; j++) {
                    a.out_cand_ids[(int64_t) row * a.max_out + j] = j == 0 ? id : -1;
                    a.out_cand_probs[(int64_t) row * a.max_out + j] = j == 0 ? 1.0f : 0.0f;
                }
            }
        }
        return true;
    }
    const int nk = min(n, pl.k);  // entries that belong to the flavor's top k
    // Every candidate of the reference with a weight is held: its top k, or every token that has a key (the rest of
    // a short row are banned tokens, last in the order with weight 0).
    const bool full_known = nk >= pl.k || complete;
    const bool valid = tid < nk;
    const float vi = valid ? entry_value(e[tid]) : -INFINITY;
    // The sum of exp over the whole vocabulary, relative to the top value (the m of the totals is that value).
    const double s_all = pl.need_s ? tot.s * exp((double) tot.m - (double) top) : 0.0;
    int kept = 0, pick = -1;
    bool resolved = true;
    // Transformers and Haru normalize over their top k; beyond the entries held, only a top k of the whole
    // vocabulary has a known sum (the stream's). Other rows take the multi-pass path.
    if (!full_known && pl.k < a.vocab && pl.flavor != SPX_FLAVOR_FISH) return false;

    if (pl.flavor == SPX_FLAVOR_TRANSFORMERS) {
        // candidates(): double softmax over the k kept, normalized by their sum (src/families/qwen3-tts/sampler.cpp:84-87)
        const double w = valid ? exp((double) vi - (double) top) : 0.0;
        const double sum = full_known ? block_sum_f64<B>(w, L.red) : s_all;
        const double q = w / sum;
        int keep = -1;
        if (pl.top_p < 1.0f) {
            // the smallest prefix whose cumulative weight reaches top_p, at least one (:88-99)
            const double c = block_incl_scan_f64<B>(q, L.red);
            const int first = block_min_i32<B>(valid && c >= (double) pl.top_p ? tid : 0x7fffffff, L.ired);
            if (first != 0x7fffffff) keep = first + 1;
            else if (full_known) keep = nk;
            else resolved = false;
        } else if (full_known) {
            keep = nk;
        } else {
            // A draw over every token: pick()'s running share must pass u within the entries held. The shares are
            // the weights over the whole vocabulary's sum, which is what pick() divides by, to rounding.
            const double c = block_incl_scan_f64<B>(q, L.red);
            const int first = block_min_i32<B>(valid && c > u ? tid : 0x7fffffff, L.ired);
            if (first != 0x7fffffff && first < pl.k - 1) {
                pick = first;
                kept = pl.k;
                if (a.out_cand_ids && valid && tid < a.max_out) {
                    a.out_cand_ids[(int64_t) row * a.max_out + tid] = (int32_t) entry_id(e[tid]);
                    a.out_cand_probs[(int64_t) row * a.max_out + tid] = (float) q;
                }
            } else {
                resolved = false;
            }
        }
        if (keep > 0) {
            // pick() over the kept weights (src/common/sampling.cpp:9-19)
            const bool in = tid < keep;
            const double kq = in ? q : 0.0;
            const double ksum = block_sum_f64<B>(kq, L.red);
            const double c = block_incl_scan_f64<B>(in ? kq / ksum : 0.0, L.red);
            const int first = block_min_i32<B>(in && tid < keep - 1 && c > u ? tid : 0x7fffffff, L.ired);
            pick = first != 0x7fffffff ? first : keep - 1;
            kept = keep;
            if (a.out_cand_ids && in && tid < a.max_out) {
                a.out_cand_ids[(int64_t) row * a.max_out + tid] = (int32_t) entry_id(e[tid]);
                a.out_cand_probs[(int64_t) row * a.max_out + tid] = (float) (kq / ksum);
            }
        }
    } else if (pl.flavor == SPX_FLAVOR_HARU) {
        // torch's float32 softmax over the k kept and its top-p zeroing (src/families/haru/sampler.cpp:44-59)
        if (valid) L.pf[tid] = (float) exp((double) (vi - top));
        __syncthreads();
        if (tid == 0) {
            float sum = 0.0f;
            if (full_known) {
                for (int i = 0; i < nk; i++) sum += L.pf[i];
            } else {
                sum = (float) s_all;
            }
            L.red[0] = (double) sum;
        }
        __syncthreads();
        const float sumf = (float) L.red[0];
        __syncthreads();
        if (valid) L.pf[tid] = L.pf[tid] / sumf;
        __syncthreads();
        // The zeroing, position by position as the reference's loop runs it, in float (:52-59).
        if (pl.top_p > 0.0f && pl.top_p < 1.0f) {
            if (tid == 0) {
                float run = 0.0f;
                int zeros = 0;
                for (int i = 0; i < nk; i++) {
                    const float pi = L.pf[i];
                    run += pi;
                    const bool zero = !(run - pi < pl.top_p);
                    L.w[i] = zero ? 0.0 : (double) pi;
                    zeros += zero ? 1 : 0;
                }
                L.ired[8] = zeros;
            }
        } else if (tid == 0) {
            for (int i = 0; i < nk; i++) L.w[i] = (double) L.pf[i];
            L.ired[8] = 0;
        }
        __syncthreads();
        // Beyond the entries held the weights must be 0: a zero among them, the cumulative share only rising.
        if (!full_known && L.ired[8] == 0) resolved = false;
        const double w = valid ? L.w[tid] : 0.0;
        __syncthreads();
        if (resolved) {
            const double ksum = block_sum_f64<B>(w, L.red);
            const double c = block_incl_scan_f64<B>(w / ksum, L.red);
            const int first = block_min_i32<B>(valid && tid < nk - 1 && c > u ? tid : 0x7fffffff, L.ired);
            if (first != 0x7fffffff) pick = first;
            else if (full_known) pick = nk - 1;  // pick()'s last, which may weigh 0
            else if (pl.need_low) pick = -2;     // the last token of the whole order
            else resolved = false;
            kept = pl.k;
            if (a.out_cand_ids && valid && tid < a.max_out) {
                a.out_cand_ids[(int64_t) row * a.max_out + tid] = (int32_t) entry_id(e[tid]);
                a.out_cand_probs[(int64_t) row * a.max_out + tid] = (float) (w / ksum);
            }
        }
    } else {
        // fish-speech: shares over the softmax of every logit, the token passing top_p dropped
        // (src/families/drama3/sampler.cpp:48-59)
        const double w = valid ? exp((double) vi - (double) top) : 0.0;
        const double c = block_incl_scan_f64<B>(w / s_all, L.red);
        const int first = block_min_i32<B>(valid && tid > 0 && c > (double) pl.top_p ? tid : 0x7fffffff, L.ired);
        int keep;
        if (first != 0x7fffffff) keep = first;
        else if (full_known) keep = nk;
        else {
            keep = -1;
            resolved = false;
        }
        if (resolved) {
            const bool in = tid < keep;
            const double kw = in ? w : 0.0;
            const double ksum = block_sum_f64<B>(kw, L.red);
            const double cc = block_incl_scan_f64<B>(kw / ksum, L.red);
            const int f2 = block_min_i32<B>(in && tid < keep - 1 && cc > u ? tid : 0x7fffffff, L.ired);
            pick = f2 != 0x7fffffff ? f2 : keep - 1;
            kept = keep;
            if (a.out_cand_ids && in && tid < a.max_out) {
                a.out_cand_ids[(int64_t) row * a.max_out + tid] = (int32_t) entry_id(e[tid]);
                a.out_cand_probs[(int64_t) row * a.max_out + tid] = (float) (kw / ksum);
            }
        }
    }
    if (!resolved) return false;
    if (tid == 0) {
        const int id = pick == -2 ? (int) ~(uint32_t) tot.low : (int) entry_id(e[pick]);
        write_row(a, row, id, SPX_ROW_OK, kept);
    }
    if (a.out_cand_ids) {
        // entries past those written above
        for (int j = min(kept, nk) + tid; j < a.max_out; j += B) {
            a.out_cand_ids[(int64_t) row * a.max_out + j] = -1;
            a.out_cand_probs[(int64_t) row * a.max_out + j] = 0.0f;
        }
    }
    return true;
}

// ------------------------------------------------------------------------------------------------------------------
// The streaming pass
// ------------------------------------------------------------------------------------------------------------------

template <typename T>
__device__ inline float load_one(const T * p);
template <>
__device__ inline float load_one<float>(const float * p) {
    return *p;
}
template <>
__device__ inline float load_one<uint16_t>(const uint16_t * p) {
    return bf16_to_float(*p);
}

using U32x4 = uint32_t __attribute__((ext_vector_type(4)));

template <typename T>
struct Vec;
template <>
struct Vec<float> {
    static constexpr int n = 4;
    __device__ static inline void unpack(const U32x4 & r, float (&x)[4]) {
        x[0] = __uint_as_float(r.x);
        x[1] = __uint_as_float(r.y);
        x[2] = __uint_as_float(r.z);
        x[3] = __uint_as_float(r.w);
    }
};
template <>
struct Vec<uint16_t> {
    static constexpr int n = 8;
    __device__ static inline void unpack(const U32x4 & r, float (&x)[8]) {
        x[0] = __uint_as_float(r.x << 16);
        x[1] = __uint_as_float(r.x & 0xffff0000u);
        x[2] = __uint_as_float(r.y << 16);
        x[3] = __uint_as_float(r.y & 0xffff0000u);
        x[4] = __uint_as_float(r.z << 16);
        x[5] = __uint_as_float(r.z & 0xffff0000u);
        x[6] = __uint_as_float(r.w << 16);
        x[7] = __uint_as_float(r.w & 0xffff0000u);
    }
};

// The wave's candidate offers of one vector: lanes of `ok` whose quotient reaches tf enter the buffer, after a
// compaction where the buffer would overflow (which raises tf to the wave's new K-th key).
template <int V>
__device__ __forceinline__ void offer_vec(WaveBuf & wb, uint32_t * wg_tau, const float (&q)[V], uint32_t ok, float & tf,
                                          int i0) {
    uint64_t m[V];
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < V; j++) {
        m[j] = ballot(((ok >> j) & 1u) && q[j] >= tf);
        cnt += (int) __popcll(m[j]);
    }
    if (cnt == 0) return;
    if (wb.n + cnt > kCap) {
        wb.thr = wave_compact(wb.buf, &wb.n, wb.K);
        wb.thr_key = entry_key(wb.thr);
        tf = key_float(wb.thr_key);
        if (lane_id() == 0) atomicMax(wg_tau, wb.thr_key);
#pragma unroll
        for (int j = 0; j < V; j++) m[j] = ballot(((ok >> j) & 1u) && q[j] >= tf);
    }
#pragma unroll
    for (int j = 0; j < V; j++) {
        if (m[j]) {
            if (((ok >> j) & 1u) && q[j] >= tf)
                wb.buf[wb.n + lanes_below(m[j])] = make_entry(order_key(q[j]), (uint32_t) (i0 + j));
            wb.n += (int) __popcll(m[j]);
        }
    }
}

// U vectors of V final logits per lane; vector u holds tokens i0[u] .. i0[u]+V-1. Bit j of live[u] is set where token
// i0[u]+j is this lane's to take, and of ban[u] where that token is banned (its x is -inf). x of a token not live is
// -inf or a copy of one taken elsewhere, so the group's largest x is a largest final logit. Every lane takes part.
template <int U, int V>
__device__ __forceinline__ void take_group(const Plan & pl, Lane & ln, WaveBuf & wb, uint32_t * wg_tau,
                                           const float (&x)[U][V], const uint32_t (&live)[U], const uint32_t (&ban)[U],
                                           const int (&i0)[U]) {
    float gx = -INFINITY;
#pragma unroll
    for (int u = 0; u < U; u++) {
#pragma unroll
        for (int j = 0; j < V; j++) gx = fmaxf(gx, x[u][j]);
    }
    ln.mx = fmaxf(ln.mx, gx);
    if (pl.flavor == SPX_FLAVOR_FISH) {
#pragma unroll
        for (int u = 0; u < U; u++) {
#pragma unroll
            for (int j = 0; j < V; j++) ln.mn = fminf(ln.mn, ((live[u] >> j) & 1u) ? x[u][j] : INFINITY);
        }
    }
    if (pl.mode == kGreedy) {
        // tokens come to a lane by rising id: the first largest is the first strictly above all before it
#pragma unroll
        for (int u = 0; u < U; u++) {
#pragma unroll
            for (int j = 0; j < V; j++) {
                if (((live[u] >> j) & 1u) && x[u][j] > ln.bestx) {
                    ln.bestx = x[u][j];
                    ln.besti = i0[u] + j;
                }
                if (((live[u] >> j) & 1u) && __builtin_isnan(x[u][j])) ln.flags |= kNaN;
            }
        }
        return;
    }
    if (pl.need_s) {
        // The wave's reference for the sum of exp: its largest quotient so far. Division by t > 0 rounded to nearest
        // keeps the order, so the group's largest quotient is its largest logit divided.
        const float wx = wave_max_f32(gx);
        if (wx > -INFINITY) {
            const float wm = div_rn(wx, pl.t, pl.rt);
            if (wm > ln.m) {
                ln.s *= exp((double) ln.m - (double) wm);
                ln.m = wm;
            }
        }
    }
    const uint32_t tk = max(wb.thr_key, *(volatile uint32_t *) wg_tau);
    float tf = tk ? key_float(tk) : -INFINITY;
#pragma unroll
    for (int u = 0; u < U; u++) {
        const uint32_t act = live[u] & ~ban[u];  // tokens whose quotient is computed
        float q[V];
        uint32_t nan = 0;
#pragma unroll
        for (int j = 0; j < V; j++) {
            // x / t by Markstein's correction, the IEEE division where the quotient leaves the normal range
            const float xv = x[u][j];
            const float q0 = xv * pl.rt;
            float qq = __builtin_fmaf(__builtin_fmaf(-q0, pl.t, xv), pl.rt, q0);
            const float aq = __builtin_fabsf(q0);
            if (__builtin_expect(((act >> j) & 1u) && !(aq >= 0x1p-125f && aq < INFINITY), 0)) qq = xv / pl.t;
            if (pl.flavor == SPX_FLAVOR_HARU && ((act >> j) & 1u) && __builtin_isfinite(xv) && !__builtin_isfinite(qq))
                ln.flags |= kTempOver;
            qq = ((act >> j) & 1u) ? qq : -INFINITY;
            nan |= __builtin_isnan(qq) ? (1u << j) : 0u;
            q[j] = qq;
        }
        if (nan) ln.flags |= kNaN;
        const uint32_t ok = act & ~nan;
        if (pl.need_low) {
#pragma unroll
            for (int j = 0; j < V; j++) {
                // banned tokens are the last of the order, -inf
                const float qv = ((ban[u] >> j) & 1u) ? -INFINITY : q[j];
                if ((((ok | ban[u]) & live[u]) >> j & 1u) && qv <= ln.lowq) {
                    ln.lowq = qv;
                    ln.lowi = i0[u] + j;
                }
            }
        }
        if (pl.need_s) {
#pragma unroll
            for (int j = 0; j < V; j++) ln.s += (double) __builtin_amdgcn_exp2f((q[j] - ln.m) * 1.4426950408889634f);
        }
        offer_vec<V>(wb, wg_tau, q, ok, tf, i0[u]);
    }
}

// The special tokens among V consecutive tokens at chunk offset `off`: a history token is set aside for the post-pass
// (its raw logit to its slot, -inf in x, out of `live`), a banned one becomes -inf and is marked in `ban`.
template <int V>
__device__ __forceinline__ void special_vec(const Specials & sp, float (&x)[V], uint32_t & live, uint32_t & ban, int off,
                                            bool in) {
    const uint2 pair = in ? sp.bits[off >> 5] : make_uint2(0u, 0u);
    const int sh = off & 31;
    const uint32_t mask = (1u << V) - 1u;
    const uint32_t nh = (pair.x >> sh) & mask, nb = (pair.y >> sh) & mask & ~nh;
    if (ballot(nh != 0)) {
        if (nh) {
            const int base = sp.rank[off >> 5];
#pragma unroll
            for (int j = 0; j < V; j++) {
                if ((nh >> j) & 1u) sp.slot_raw[base + __popc(pair.x & ((1u << (sh + j)) - 1u))] = x[j];
            }
        }
#pragma unroll
        for (int j = 0; j < V; j++) x[j] = ((nh >> j) & 1u) ? -INFINITY : x[j];
        live &= ~nh;
    }
    if (ballot(nb != 0)) {
#pragma unroll
        for (int j = 0; j < V; j++) x[j] = ((nb >> j) & 1u) ? -INFINITY : x[j];
        ban = nb;
    }
}

template <typename T, int B>
__device__ __forceinline__ void stream_chunk(const Launch & a, const T * rowp, int c0, int c1, const Plan & pl,
                                             const Specials & sp, Lane & ln, WaveBuf & wb, uint32_t * wg_tau) {
    constexpr int V = Vec<T>::n;
    const int n = c1 - c0;
    const int tid = threadIdx.x;
    int done = 0;
    if (a.vec_ok) {
        const int ng = n / V;  // whole vectors
        const U32x4 * vp = (const U32x4 *) (rowp + c0);
        // Four 16-byte loads in flight per lane before any is used; lanes past the end load the last vector again
        // and take nothing from it.
        for (int base = 0; base < ng; base += 4 * B) {
            const int g0 = base + tid, g1 = g0 + B, g2 = g1 + B, g3 = g2 + B;
            const U32x4 r0 = vp[min(g0, ng - 1)];
            const U32x4 r1 = vp[min(g1, ng - 1)];
            const U32x4 r2 = vp[min(g2, ng - 1)];
            const U32x4 r3 = vp[min(g3, ng - 1)];
            float x[4][V];
            Vec<T>::unpack(r0, x[0]);
            Vec<T>::unpack(r1, x[1]);
            Vec<T>::unpack(r2, x[2]);
            Vec<T>::unpack(r3, x[3]);
            const int g[4] = {g0, g1, g2, g3};
            uint32_t live[4], ban[4];
            int i0[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const bool in = g[u] < ng;
                live[u] = in ? (1u << V) - 1u : 0u;
                ban[u] = 0u;
                i0[u] = c0 + g[u] * V;
                if (sp.any) special_vec<V>(sp, x[u], live[u], ban[u], g[u] * V, in);
            }
            take_group<4, V>(pl, ln, wb, wg_tau, x, live, ban, i0);
        }
        done = ng * V;
    }
    // One token per lane: a row that is not 16-byte aligned, and the tail of one that is.
    for (int base = done; base < n; base += B) {
        const int i = base + tid;
        const bool in = i < n;
        float x[1][1] = {{in ? load_one<T>(rowp + c0 + i) : -INFINITY}};
        uint32_t live[1] = {in ? 1u : 0u}, ban[1] = {0u};
        const int i0[1] = {c0 + i};
        if (sp.any) special_vec<1>(sp, x[0], live[0], ban[0], i, in);
        take_group<1, 1>(pl, ln, wb, wg_tau, x, live, ban, i0);
    }
}

// The history tokens of the chunk, after the stream: penalties, the ban, then the same statistics.
template <int B>
__device__ __forceinline__ void take_specials(const spx_row_params & p, const Plan & pl, const Specials & sp,
                                              const uint32_t * banned_row, Lane & ln, WaveBuf & wb, uint32_t * wg_tau) {
    for (int base = 0; base < sp.n_slots; base += B) {
        const int s = base + threadIdx.x;
        const bool in = s < sp.n_slots;
        float x[1][1] = {{-INFINITY}};
        int i0[1] = {0};
        uint32_t live[1] = {in ? 1u : 0u}, ban[1] = {0u};
        if (in) {
            const int id = sp.slot_id[s];
            float v = penalize(sp.slot_raw[s], pl.counts ? sp.slot_cnt[s] : 0, p);
            if (banned_row && ((banned_row[id >> 5] >> (id & 31)) & 1u)) {
                v = -INFINITY;
                ban[0] = 1u;
            }
            if (id == 0 && __builtin_isnan(v)) ln.flags |= kNaN0;
            x[0][0] = v;
            i0[0] = id;
        }
        take_group<1, 1>(pl, ln, wb, wg_tau, x, live, ban, i0);
    }
}

// Reduces the lanes' states over the work-group, through LDS; every thread gets the totals.
template <int B>
__device__ inline RowTotals reduce_lanes(const Lane & ln, uint64_t * red64, double * redd, float * redf, uint32_t * redu) {
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    const uint64_t be = ln.besti >= 0 ? make_entry(order_key(ln.bestx), (uint32_t) ln.besti) : 0;
    const uint64_t lo = ln.lowi >= 0 ? (((uint64_t) order_key(ln.lowq) << 32) | (uint64_t) (~(uint32_t) ln.lowi)) : ~0ull;
    const uint64_t best = wave_max_u64(be);
    const uint64_t low = wave_min_u64(lo);
    const double s = wave_sum_f64(ln.s);  // m is the same in every lane of a wave
    const float mx = wave_max_f32(ln.mx);
    const float mn = -wave_max_f32(-ln.mn);
    const uint32_t flags = wave_or_u32(ln.flags);
    if (lane == 0) {
        red64[2 * wave] = best;
        red64[2 * wave + 1] = low;
        redd[wave] = s;
        redf[4 * wave] = ln.m;
        redf[4 * wave + 1] = mx;
        redf[4 * wave + 2] = mn;
        redu[wave] = flags;
    }
    __syncthreads();
    RowTotals t;
    t.best = 0;
    t.low = ~0ull;
    t.m = -FLT_MAX;
    t.mx = -INFINITY;
    t.mn = INFINITY;
    t.flags = 0;
    t.s = 0;
    for (int w = 0; w < B / kWave; w++) t.m = fmaxf(t.m, redf[4 * w]);
    for (int w = 0; w < B / kWave; w++) {
        t.best = red64[2 * w] > t.best ? red64[2 * w] : t.best;
        t.low = red64[2 * w + 1] < t.low ? red64[2 * w + 1] : t.low;
        t.flags |= redu[w];
        t.mx = fmaxf(t.mx, redf[4 * w + 1]);
        t.mn = fminf(t.mn, redf[4 * w + 2]);
        t.s += redd[w] * ((redf[4 * w] == t.m) ? 1.0 : exp((double) redf[4 * w] - (double) t.m));
    }
    __syncthreads();
    return t;
}

// Gathers the waves' entries at or above the largest of their K-th entries into dst (a power-of-two padded array),
// sorts it, and returns how many of its first entries are real.
template <int B>
__device__ inline int union_and_sort(uint64_t * wave_bufs, const int * wave_n, const uint64_t * wave_thr, uint64_t * dst,
                                     int cap, int * red) {
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    uint64_t floor = 0;
    for (int w = 0; w < B / kWave; w++) floor = wave_thr[w] > floor ? wave_thr[w] : floor;
    const int n = wave_n[wave];
    const uint64_t * src = wave_bufs + wave * kCap;
    int mine = 0;
    for (int i0 = 0; i0 < n; i0 += kWave) mine += (int) __popcll(ballot(i0 + lane < n && src[i0 + lane] >= floor));
    if (lane == 0) red[wave] = mine;
    __syncthreads();
    int base = 0, total = 0;
    for (int w = 0; w < B / kWave; w++) {
        if (w < wave) base += red[w];
        total += red[w];
    }
    __syncthreads();
    total = min(total, cap);
    int pos = base;
    for (int i0 = 0; i0 < n; i0 += kWave) {
        const int i = i0 + lane;
        const bool keep = i < n && src[i] >= floor;
        const uint64_t m = ballot(keep);
        if (keep && pos + lanes_below(m) < cap) dst[pos + lanes_below(m)] = src[i];
        pos += (int) __popcll(m);
    }
    int np2 = 1;
    while (np2 < total) np2 <<= 1;
    for (int i = total + threadIdx.x; i < np2; i += B) dst[i] = 0;
    __syncthreads();
    block_sort_desc<B>(dst, np2);
    return total;
}

__device__ inline void xcd_map(int bid, int nwg, int splits, int & row, int & split) {
    // Work-groups are dispatched round-robin over the 8 XCDs; give the chunks of one row consecutive slots of one
    // XCD, so that the partials the last chunk reads were written through the same L2.
    const int x = bid & 7, l = bid >> 3;
    const int per = nwg >> 3, extra = nwg & 7;
    const int g = x * per + min(x, extra) + l;
    row = g / splits;
    split = g - row * splits;
}


// ------------------------------------------------------------------------------------------------------------------
// The multi-pass path: exact radix selects over the whole row
// ------------------------------------------------------------------------------------------------------------------

// Fixed-point scale of the masses the selects add up: exact, order-free sums of exp(q - top) rounded to 2^-40.
constexpr double kFix = 1099511627776.0;  // 2^40

__device__ __forceinline__ uint64_t mass_fixed(float q, float top) {
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
    int * ired;
};

// Visits every token's entry and fixed-point mass (a NaN quotient carries neither), chunk by chunk, each chunk's
// special tokens rebuilt in LDS as the stream had them: a banned token as -inf, a history token by its final quotient.
template <typename T, int B, typename F>
__device__ inline void fb_visit(FbRow & r, F && f) {
    const Launch & a = *r.a;
    const T * rowp = (const T *) a.logits + (int64_t) r.row * a.ld;
    const bool spec = r.pl.pen || r.banned_row;
    for (int c0 = 0; c0 < a.vocab; c0 += a.chunk) {
        const int c1 = min(a.vocab, c0 + a.chunk);
        if (spec) {
            __syncthreads();  // the previous chunk's special tokens are read no more
            uint32_t bad = 0;
            build_specials<B>(r.sp, a, r.row, c0, c1, r.pl, r.banned_row, r.ired, bad);
            for (int s = threadIdx.x; s < r.sp.n_slots; s += B) {
                const int id = r.sp.slot_id[s];
                float v = penalize(load_one<T>(rowp + id), r.pl.counts ? r.sp.slot_cnt[s] : 0, r.p);
                if (r.banned_row && ((r.banned_row[id >> 5] >> (id & 31)) & 1u)) v = -INFINITY;
                r.sp.slot_raw[s] = div_rn(v, r.pl.t, r.pl.rt);  // from here on the final quotient
            }
            __syncthreads();
        }
        for (int i = c0 + threadIdx.x; i < c1; i += B) {
            float x;
            if (spec) {
                const uint2 pair = r.sp.bits[(i - c0) >> 5];
                const uint32_t bit = 1u << ((i - c0) & 31);
                if (pair.x & bit) continue;
                x = (pair.y & bit) ? -INFINITY : load_one<T>(rowp + i);
            } else {
                x = load_one<T>(rowp + i);
            }
            const float q = div_rn(x, r.pl.t, r.pl.rt);
            if (__builtin_isnan(q)) continue;
            f(make_entry(order_key(q), (uint32_t) i), mass_fixed(q, r.top));
        }
        if (spec) {
            for (int s = threadIdx.x; s < r.sp.n_slots; s += B) {
                const float q = r.sp.slot_raw[s];
                if (__builtin_isnan(q)) continue;
                f(make_entry(order_key(q), (uint32_t) r.sp.slot_id[s]), mass_fixed(q, r.top));
            }
        }
    }
    if (spec) __syncthreads();
}

// The first entry in falling order whose running count (by_mass false) or running mass reaches `target` (strict:
// passes it), by radix passes of 8 bits over the 64-bit entries. False when no entry does.
template <typename T, int B>
__device__ inline bool fb_select(FbRow & r, bool by_mass, uint64_t target, bool strict, Select & out,
                                 uint32_t * hist_n, unsigned long long * hist_m) {
    int * ired = r.ired;
    Select s;
    s.prefix = 0;
    s.bits = 0;
    s.above_n = 0;
    s.above_m = 0;
    s.own_m = 0;
    unsigned long long * shared = (unsigned long long *) (ired + 2);
    while (s.bits < 64) {
        for (int i = threadIdx.x; i < 256; i += B) {
            hist_n[i] = 0;
            hist_m[i] = 0;
        }
        __syncthreads();
        const int shift = 56 - s.bits;
        const uint64_t pre = s.prefix;
        const int bits = s.bits;
        fb_visit<T, B>(r, [&](uint64_t e, uint64_t w) {
            if (bits == 0 || (e >> (64 - bits)) == pre) {
                const int d = (int) ((e >> shift) & 255u);
                atomicAdd(&hist_n[d], 1u);
                atomicAdd(&hist_m[d], (unsigned long long) w);
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

// Resolves one row the one-pass path could not finish, in the row's last work-group, with radix selects over the
// whole row (the candidate and sort regions of LDS are free by now).
template <typename T, int B>
__device__ inline void fallback_row(const Launch & a, int row, const spx_row_params & p, const Plan & pl, uint64_t low,
                                    float top, unsigned char * lds) {
    const int tid = threadIdx.x;
    int * ired = (int *) (lds + a.off_red);
    uint32_t * hist_n = (uint32_t *) (lds + a.off_sort);
    unsigned long long * hist_m = (unsigned long long *) (lds + a.off_sort + 1024);
    FbRow r;
    r.a = &a;
    r.row = row;
    r.p = p;
    r.pl = pl;
    r.banned_row = a.banned ? a.banned + (int64_t) row * a.banned_stride : nullptr;
    r.sp.any = pl.pen || r.banned_row;
    r.sp.n_slots = 0;
    r.sp.bits = (uint2 *) (lds + a.off_bits);
    r.sp.rank = (int32_t *) (lds + a.off_rank);
    r.sp.slot_id = (int32_t *) (lds + a.off_slots);
    r.sp.slot_raw = (float *) (lds + a.off_slots + 4 * a.slot_cap);
    r.sp.slot_cnt = (int32_t *) (lds + a.off_slots + 8 * a.slot_cap);
    r.top = top;
    r.ired = ired;
    // The total mass over the row, as the selects count it.
    unsigned long long * tot_m = (unsigned long long *) (ired + 8);
    if (tid == 0) *tot_m = 0;
    __syncthreads();
    {
        unsigned long long mine = 0;
        fb_visit<T, B>(r, [&](uint64_t, uint64_t w) { mine += w; });
        atomicAdd(tot_m, mine);
    }
    __syncthreads();
    const uint64_t all_m = *tot_m;
    __syncthreads();
    const double u = a.u[row];
    const int fl = pl.flavor;
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
    if (fl == SPX_FLAVOR_TRANSFORMERS || fl == SPX_FLAVOR_HARU) {
        // transformers keeps the token reaching top_p (qwen3-tts/sampler.cpp:92-96); torch's zeroing in
        // sample_token keeps the same prefix, the tokens after it weighing 0 (haru/sampler.cpp:52-59)
        const bool applies = fl == SPX_FLAVOR_TRANSFORMERS ? pl.top_p < 1.0f : (pl.top_p > 0.0f && pl.top_p < 1.0f);
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
    } else if (fl == SPX_FLAVOR_HARU) {
        // pick() over all k weights, zeros included: the k-th token
        id = have_k_entry ? (int) entry_id(sk.entry) : (int) ~(uint32_t) low;
    } else if (have_cut && fl == SPX_FLAVOR_TRANSFORMERS) {
        id = (int) entry_id(scut.entry);
    } else if (have_cut) {
        Select sl;
        if (sel(false, kept_n, false, sl)) id = (int) entry_id(sl.entry);
    } else if (have_k_entry) {
        id = (int) entry_id(sk.entry);
    } else {
        id = (int) ~(uint32_t) low;
    }
    if (tid == 0) {
        write_row(a, row, id, SPX_ROW_OK, fl == SPX_FLAVOR_HARU ? pl.k : (int) kept_n);
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

template <typename T>
__global__ __launch_bounds__(kBlock) void stream_kernel(Launch a) {
    extern __shared__ __align__(16) unsigned char lds[];
    constexpr int B = kBlock;
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    int row, split;
    xcd_map((int) blockIdx.x, a.nwg, a.splits, row, split);
    if (row >= a.rows) return;

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
    const Plan pl = make_plan(p, a.vocab, a.banned != nullptr, a.hist != nullptr);
    const int c0 = split * a.chunk, c1 = min(a.vocab, c0 + a.chunk);
    const uint32_t * banned_row = a.banned ? a.banned + (int64_t) row * a.banned_stride : nullptr;
    const T * rowp = (const T *) a.logits + (int64_t) row * a.ld;

    int * ired = (int *) (lds + a.off_red);
    double * dred = (double *) (lds + a.off_red + 256);
    uint64_t * red64 = (uint64_t *) (lds + a.off_red + 512);
    float * fred = (float *) (lds + a.off_red + 768);
    uint32_t * ured = (uint32_t *) (lds + a.off_red + 1024);
    int * wave_n = (int *) (lds + a.off_red + 1088);
    uint64_t * wave_thr = (uint64_t *) (lds + a.off_red + 1152);
    uint32_t * wg_tau = (uint32_t *) (ired + 60);  // the largest K-th key any wave has published

    Lane ln;
    lane_init(ln);
    Specials sp;
    sp.any = false;
    sp.n_slots = 0;
    sp.bits = (uint2 *) (lds + a.off_bits);
    sp.rank = (int32_t *) (lds + a.off_rank);
    sp.slot_id = (int32_t *) (lds + a.off_slots);
    sp.slot_raw = (float *) (lds + a.off_slots + 4 * a.slot_cap);
    sp.slot_cnt = (int32_t *) (lds + a.off_slots + 8 * a.slot_cap);
    uint32_t bad = 0;
    if (tid == 0) *wg_tau = 0;
    if (pl.mode != kInvalid && (pl.pen || banned_row)) {
        sp.any = true;
        build_specials<B>(sp, a, row, c0, c1, pl, banned_row, ired, bad);
    }
    __syncthreads();
    ln.flags |= bad;

    const bool sampling = pl.mode == kTopK || pl.mode == kFull;
    WaveBuf wb;
    wb.buf = (uint64_t *) (lds + a.off_cand) + wave * kCap;
    wb.n = 0;
    wb.thr = 0;
    wb.thr_key = 0;
    wb.K = pl.kc;

    if (pl.mode != kInvalid) {
        stream_chunk<T, B>(a, rowp, c0, c1, pl, sp, ln, wb, wg_tau);
        // Token 0, where it is not a history token, for std::max_element's NaN in front.
        if (c0 == 0 && tid == 0) {
            const uint2 pair = sp.any ? sp.bits[0] : make_uint2(0u, 0u);
            if (!(pair.x & 1u)) {
                const float x0 = (pair.y & 1u) ? -INFINITY : load_one<T>(rowp);
                if (__builtin_isnan(x0)) ln.flags |= kNaN0;
            }
        }
        if (sp.any) {
            __syncthreads();
            take_specials<B>(p, pl, sp, banned_row, ln, wb, wg_tau);
        }
    }

    // Each wave keeps exactly its top K; its K-th entry bounds the row's K-th from below.
    uint64_t thr = 0;
    if (sampling) {
        if (wb.n > wb.K) {
            thr = wave_compact(wb.buf, &wb.n, wb.K);
        } else if (wb.n == wb.K) {
            uint64_t m = ~0ull;
            for (int i = lane; i < wb.n; i += kWave) m = wb.buf[i] < m ? wb.buf[i] : m;
            thr = wave_min_u64(m);
        }
    }
    if (lane == 0) {
        wave_n[wave] = sampling ? wb.n : 0;
        wave_thr[wave] = thr;
    }
    const RowTotals tot = reduce_lanes<B>(ln, red64, dred, fred, ured);  // its barriers publish wave_n

    uint64_t * sorted = (uint64_t *) (lds + a.off_sort);
    int n = 0;
    bool complete = true;
    if (sampling) {
        n = union_and_sort<B>((uint64_t *) (lds + a.off_cand), wave_n, wave_thr, sorted, a.sort_cap, ired);
        complete = n < pl.kc;  // fewer than K: no wave ever dropped an entry
        n = min(n, pl.kc);
    }

    FinishLds L;
    L.w = (double *) (lds + a.off_cand);
    L.red = dred;
    L.ired = ired;
    L.pf = (float *) (lds + a.off_cand + 8 * kKeep);

    if (a.splits > 1) {
        // Publish this chunk's partial; the last chunk of the row to arrive merges them.
        Partial * part = a.partials + (int64_t) row * a.splits + split;
        uint64_t * pc = a.part_cands + ((int64_t) row * a.splits + split) * kKeep;
        for (int i = tid; i < n; i += B) pc[i] = sorted[i];
        if (tid == 0) {
            part->best = tot.best;
            part->low = tot.low;
            part->s = tot.s;
            part->m = tot.m;
            part->mx = tot.mx;
            part->mn = tot.mn;
            part->flags = tot.flags;
            part->n = n;
            part->complete = complete ? 1 : 0;
            part->kth = (n >= pl.kc && n > 0) ? sorted[n - 1] : 0;
        }
        // One wave makes the partial visible device-wide and counts the chunk in; the last chunk's first wave makes
        // the others' visible to its work-group.
        __syncthreads();
        if (tid == 0) {
            __threadfence();
            const unsigned prev = atomicAdd(&a.counters[row], 1u);
            const int last = prev == (unsigned) (a.splits - 1);
            if (last) {
                __threadfence();
                a.counters[row] = 0;  // ready for the next launch
            }
            ired[0] = last;
        }
        __syncthreads();
        if (!ired[0]) return;
        RowTotals t;
        t.best = 0;
        t.low = ~0ull;
        t.flags = 0;
        t.m = -FLT_MAX;
        t.mx = -INFINITY;
        t.mn = INFINITY;
        t.s = 0;
        uint64_t floor = 0;
        bool all_complete = true;
        const Partial * pr = a.partials + (int64_t) row * a.splits;
        for (int s2 = 0; s2 < a.splits; s2++) {
            const Partial q = pr[s2];
            t.best = q.best > t.best ? q.best : t.best;
            t.low = q.low < t.low ? q.low : t.low;
            t.flags |= q.flags;
            t.m = fmaxf(t.m, q.m);
            t.mx = fmaxf(t.mx, q.mx);
            t.mn = fminf(t.mn, q.mn);
            floor = q.kth > floor ? q.kth : floor;
            all_complete = all_complete && q.complete;
        }
        for (int s2 = 0; s2 < a.splits; s2++) {
            const Partial q = pr[s2];
            t.s += q.s * ((q.m == t.m) ? 1.0 : exp((double) q.m - (double) t.m));
        }
        int total = 0;
        if (sampling) {
            for (int s2 = 0; s2 < a.splits; s2++) {
                const int ns = pr[s2].n;
                const uint64_t * src = a.part_cands + ((int64_t) row * a.splits + s2) * kKeep;
                for (int i0 = 0; i0 < ns; i0 += B) {
                    const int i = i0 + tid;
                    const bool keep = i < ns && src[i] >= floor;
                    int cnt_total;
                    const int pos = block_excl_scan_i32<B>(keep ? 1 : 0, ired + 32, cnt_total);
                    if (keep && total + pos < a.sort_cap) sorted[total + pos] = src[i];
                    total += cnt_total;
                }
            }
            total = min(total, a.sort_cap);
            int np2 = 1;
            while (np2 < total) np2 <<= 1;
            for (int i = total + tid; i < np2; i += B) sorted[i] = 0;
            __syncthreads();
            block_sort_desc<B>(sorted, np2);
        }
        n = min(total, pl.kc);
        if (!finish_row<B>(a, row, p, pl, t, sorted, n, all_complete, L)) {
            const float top = entry_value(sorted[0]);
            __syncthreads();
            fallback_row<T, B>(a, row, p, pl, t.low, top, lds);
        }
        return;
    }
    if (!finish_row<B>(a, row, p, pl, tot, sorted, n, complete, L)) {
        const float top = entry_value(sorted[0]);
        __syncthreads();
        fallback_row<T, B>(a, row, p, pl, tot.low, top, lds);
    }
}

// ------------------------------------------------------------------------------------------------------------------
// Launchers
// ------------------------------------------------------------------------------------------------------------------

hipError_t launch_stream(const Launch & a, hipStream_t s) {
    if (a.nwg == 0) return hipSuccess;
    if (a.dtype == SPX_BF16) {
        hipLaunchKernelGGL(stream_kernel<uint16_t>, dim3(a.nwg), dim3(kBlock), a.lds_bytes, s, a);
    } else {
        hipLaunchKernelGGL(stream_kernel<float>, dim3(a.nwg), dim3(kBlock), a.lds_bytes, s, a);
    }
    return hipGetLastError();
}

hipError_t set_lds_limits(int stream_bytes) {
    hipError_t e = hipSuccess;
    if (stream_bytes > 65536) {
        e = hipFuncSetAttribute((const void *) stream_kernel<float>, hipFuncAttributeMaxDynamicSharedMemorySize, stream_bytes);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void *) stream_kernel<uint16_t>, hipFuncAttributeMaxDynamicSharedMemorySize, stream_bytes);
    }
    return e;
}

}  // namespace spx
