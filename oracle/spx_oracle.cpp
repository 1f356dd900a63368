// spx_oracle.cpp — TEST INFRASTRUCTURE ONLY: the CPU restatement of speech.cpp's token samplers that checks the HIP
// sampler and serves as bench.py's CPU baseline. Nothing in the product links it. Paths in citations are relative to
// the reference checkout (nyosegawa/speech.cpp 0.11.1). Built with -ffp-contract=off so that every float and double
// operation rounds where the reference's does.

#include "spx_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <numeric>
#include <random>
#include <thread>
#include <map>
#include <vector>

namespace {

constexpr double kInf = std::numeric_limits<double>::infinity();

struct Drawn {
    std::vector<int32_t> tokens;
    std::vector<double> weights;
    int status = SPX_ROW_OK;
    double cut = kInf;  // nearest top-p decision to its threshold
};

// pick(): src/common/sampling.cpp:9-19. The sum of the weights first, then each weight's share accumulated in order;
// the first index below the last whose running share passes u, else the last.
int pick_index(const std::vector<double> & w, double u) {
    double total = 0;
    for (double x : w) total += x;
    const int last = (int) w.size() - 1;
    double running = 0;
    for (int i = 0; i < last; i++) {
        running += w[(size_t) i] / total;
        if (running > u) return i;
    }
    return last;
}

// The distance of u from the nearest boundary pick_index() compares it with (the running shares before the last),
// as checks/qwen3-tts/qwen3-tts-graph-sampler-check.cpp:98-106 measures it.
double boundary_distance(const std::vector<double> & w, double u) {
    double total = 0;
    for (double x : w) total += x;
    double running = 0, nearest = kInf;
    for (size_t i = 0; i + 1 < w.size(); i++) {
        running += w[i] / total;
        nearest = std::min(nearest, std::fabs(running - u));
    }
    return nearest;
}

bool neutral_penalties(const spx_row_params & p) {
    return p.repetition_penalty == 1.0f && p.presence_penalty == 0.0f && p.frequency_penalty == 0.0f;
}

// The first index of the largest value as std::max_element finds it: a NaN is never larger, and a NaN in the first
// position stays the answer (src/families/qwen3-tts/sampler.cpp:43, src/families/qwen3-asr/decoder.cpp:112).
int first_max(const std::vector<float> & l) {
    return (int) (std::max_element(l.begin(), l.end()) - l.begin());
}

// The penalty stage. Presence and frequency have no reference: l = (l - frequency*count) - presence, in float, on
// every in-range id the history holds, before the repetition penalty. The repetition penalty is restricted()'s:
// once per distinct in-range id, l*r below 0 and l/r otherwise (src/families/qwen3-tts/sampler.cpp:31-39).
void penalize(std::vector<float> & l, const spx_row_params & p, const int32_t * hist, int n_hist) {
    const int n = (int) l.size();
    if (p.presence_penalty != 0.0f || p.frequency_penalty != 0.0f) {
        std::vector<int32_t> count((size_t) n, 0);
        for (int j = 0; j < n_hist; j++) {
            const int32_t t = hist[j];
            if (t >= 0 && t < n) count[(size_t) t]++;
        }
        for (int t = 0; t < n; t++) {
            if (count[(size_t) t] == 0) continue;
            float v = l[(size_t) t];
            if (p.frequency_penalty != 0.0f) v = v - p.frequency_penalty * (float) count[(size_t) t];
            if (p.presence_penalty != 0.0f) v = v - p.presence_penalty;
            l[(size_t) t] = v;
        }
    }
    if (p.repetition_penalty != 1.0f) {
        std::vector<bool> seen((size_t) n, false);
        for (int j = 0; j < n_hist; j++) {
            const int32_t t = hist[j];
            if (t < 0 || t >= n || seen[(size_t) t]) continue;
            seen[(size_t) t] = true;
            const float v = l[(size_t) t];
            l[(size_t) t] = v < 0 ? v * p.repetition_penalty : v / p.repetition_penalty;
        }
    }
}

// The suppression stage: banned ids to -inf (src/families/qwen3-tts/sampler.cpp:40-42; Haru's session does the same
// before sampling, src/families/haru/sampler.cpp:116-124).
void suppress(std::vector<float> & l, const uint8_t * banned) {
    if (!banned) return;
    for (size_t i = 0; i < l.size(); i++) {
        if (banned[i]) l[i] = -INFINITY;
    }
}

bool valid_params(const spx_row_params & p, bool has_ban) {
    if (p.flavor < SPX_FLAVOR_TRANSFORMERS || p.flavor > SPX_FLAVOR_FISH) return false;
    if (std::isnan(p.temperature) || std::isnan(p.top_p) || std::isnan(p.repetition_penalty) ||
        std::isnan(p.presence_penalty) || std::isnan(p.frequency_penalty)) {
        return false;
    }
    if (p.flavor == SPX_FLAVOR_FISH && has_ban) return false;
    if (p.flavor == SPX_FLAVOR_TRANSFORMERS && !p.greedy && !(p.temperature > 0.0f)) return false;
    // A temperature that rounds to infinity, which the reference's engines refuse before sampling
    // (src/engines/qwen3-tts-engine.cpp:47-56).
    if (!p.greedy && p.temperature == INFINITY) return false;
    return true;
}

// After the penalties and the bans: restricted()'s refusals (src/families/qwen3-tts/sampler.cpp:43-49). A row whose
// largest logit is +inf under a penalty is refused naming the penalty; under TRANSFORMERS any row without a finite
// largest logit is refused. The other flavors make their own checks afterwards.
int restricted_checks(const std::vector<float> & l, const spx_row_params & p) {
    const float top = l[(size_t) first_max(l)];
    if (top == INFINITY && !neutral_penalties(p)) return SPX_ROW_REP_PENALTY_OVERFLOW;
    if (p.flavor == SPX_FLAVOR_TRANSFORMERS && !std::isfinite(top)) return SPX_ROW_NO_FINITE_LOGIT;
    return SPX_ROW_OK;
}

// candidates(): src/families/qwen3-tts/sampler.cpp:69-101, on logits that restricted() has made.
Drawn tf_draw(std::vector<float> l, const spx_row_params & p) {
    Drawn d;
    for (float v : l) {
        if (std::isnan(v)) {
            d.status = SPX_ROW_NONFINITE_INPUT;
            return d;
        }
    }
    const int n = (int) l.size();
    for (float & v : l) v /= p.temperature;
    d.tokens.resize((size_t) n);
    std::iota(d.tokens.begin(), d.tokens.end(), 0);
    const int k = p.top_k > 0 ? std::min(p.top_k, n) : n;
    std::partial_sort(d.tokens.begin(), d.tokens.begin() + k, d.tokens.end(),
                      [&](int32_t a, int32_t b) { return l[(size_t) a] > l[(size_t) b]; });
    d.tokens.resize((size_t) k);
    const float largest = l[(size_t) d.tokens[0]];
    if (!std::isfinite(largest)) {
        d.status = SPX_ROW_TEMPERATURE_OVERFLOW;
        return d;
    }
    d.weights.resize((size_t) k);
    double sum = 0;
    for (int i = 0; i < k; i++) {
        d.weights[(size_t) i] = std::exp((double) l[(size_t) d.tokens[(size_t) i]] - largest);
        sum += d.weights[(size_t) i];
    }
    for (double & w : d.weights) w /= sum;
    if (p.top_p < 1.0f) {
        double running = 0;
        int keep = 0;
        while (keep < k) {
            running += d.weights[(size_t) keep++];
            d.cut = std::min(d.cut, std::fabs(running - (double) p.top_p));
            if (running >= p.top_p) break;
        }
        d.tokens.resize((size_t) keep);
        d.weights.resize((size_t) keep);
    }
    return d;
}

// candidates(): src/families/haru/sampler.cpp:18-61, from the division by the temperature on (the greedy branch is
// handled by the caller).
Drawn haru_draw(const std::vector<float> & l, float temperature, int top_k, float top_p) {
    Drawn d;
    const int64_t v = (int64_t) l.size();
    std::vector<float> scaled(l.size());
    for (size_t i = 0; i < l.size(); i++) {
        scaled[i] = l[i] / temperature;
        if (std::isfinite(l[i]) && !std::isfinite(scaled[i])) {
            d.status = SPX_ROW_TEMPERATURE_OVERFLOW;
            return d;
        }
    }
    const int64_t k = top_k > 0 && top_k < v ? top_k : v;
    std::vector<int32_t> order((size_t) v);
    std::iota(order.begin(), order.end(), 0);
    std::partial_sort(order.begin(), order.begin() + k, order.end(), [&](int32_t a, int32_t b) {
        return scaled[(size_t) a] > scaled[(size_t) b] || (scaled[(size_t) a] == scaled[(size_t) b] && a < b);
    });
    order.resize((size_t) k);
    std::vector<float> prob((size_t) k);
    float sum = 0.0f;
    for (int64_t i = 0; i < k; i++) {
        prob[(size_t) i] = std::exp(scaled[(size_t) order[(size_t) i]] - scaled[(size_t) order[0]]);
        sum += prob[(size_t) i];
    }
    for (float & x : prob) x /= sum;
    d.tokens = order;
    d.weights.assign(prob.begin(), prob.end());
    if (top_p > 0.0f && top_p < 1.0f) {
        float running = 0.0f;
        for (int64_t i = 0; i < k; i++) {
            running += prob[(size_t) i];
            const float before = running - prob[(size_t) i];
            d.cut = std::min(d.cut, std::fabs((double) before - (double) top_p));
            if (!(before < top_p)) d.weights[(size_t) i] = 0.0;
        }
    }
    return d;
}

// candidates(): src/families/drama3/sampler.cpp:30-60, on logits already checked finite.
Drawn fish_draw(const std::vector<float> & l, float temperature, int top_k, float top_p) {
    Drawn d;
    const float t = std::max(temperature, 1e-5f);
    const int n = (int) l.size();
    std::vector<float> scaled((size_t) n);
    for (int i = 0; i < n; i++) scaled[(size_t) i] = l[(size_t) i] / t;
    const int k = std::min(std::max(top_k, 1), n);
    std::vector<int32_t> order((size_t) n);
    std::iota(order.begin(), order.end(), 0);
    std::partial_sort(order.begin(), order.begin() + k, order.end(), [&](int32_t a, int32_t b) {
        return scaled[(size_t) a] > scaled[(size_t) b] || (scaled[(size_t) a] == scaled[(size_t) b] && a < b);
    });
    const float top = scaled[(size_t) order[0]];
    if (!std::isfinite(top)) {
        d.status = SPX_ROW_TEMPERATURE_OVERFLOW;
        return d;
    }
    double sum = 0;
    for (float x : scaled) sum += std::exp((double) x - top);
    double running = 0;
    for (int r = 0; r < k; r++) {
        const double w = std::exp((double) scaled[(size_t) order[(size_t) r]] - top);
        running += w / sum;
        if (r > 0) d.cut = std::min(d.cut, std::fabs(running - (double) top_p));
        if (r > 0 && running > top_p) break;
        d.tokens.push_back(order[(size_t) r]);
        d.weights.push_back(w);
    }
    return d;
}

// The penalty and suppression stages and the flavor's refusals; on OK `l` holds the logits candidates() receives.
int prepare(std::vector<float> & l, const spx_row_params & p, const int32_t * hist, int n_hist, const uint8_t * banned) {
    if (!valid_params(p, banned != nullptr)) return SPX_ROW_INVALID_PARAMS;
    if (!neutral_penalties(p)) penalize(l, p, hist, n_hist);
    suppress(l, banned);
    const int s = restricted_checks(l, p);
    if (s != SPX_ROW_OK) return s;
    if (p.flavor == SPX_FLAVOR_HARU) {
        // src/families/haru/sampler.cpp:21-23
        for (float v : l) {
            if (std::isnan(v) || v == INFINITY) return SPX_ROW_NONFINITE_INPUT;
        }
    } else if (p.flavor == SPX_FLAVOR_FISH) {
        // src/families/drama3/sampler.cpp:35-37
        for (float v : l) {
            if (!std::isfinite(v)) return SPX_ROW_NONFINITE_INPUT;
        }
    }
    return SPX_ROW_OK;
}

bool is_greedy(const spx_row_params & p) {
    return p.greedy || (p.flavor == SPX_FLAVOR_HARU && p.temperature <= 0.0f);
}

struct RowOut {
    orc_row_report report{};
    Drawn drawn;
};

RowOut sample_one(const float * row, int vocab, const spx_row_params & p, const int32_t * hist, int n_hist,
                  const uint8_t * banned, double u) {
    RowOut out;
    out.report.id = -1;
    out.report.boundary = kInf;
    out.report.cut = kInf;
    std::vector<float> l(row, row + vocab);
    int s = prepare(l, p, hist, n_hist, banned);
    if (s == SPX_ROW_OK && is_greedy(p)) {
        out.report.id = first_max(l);
        out.report.kept = 1;
        out.drawn.tokens = {out.report.id};
        out.drawn.weights = {1.0};
    } else if (s == SPX_ROW_OK) {
        if (p.flavor == SPX_FLAVOR_TRANSFORMERS) out.drawn = tf_draw(l, p);
        else if (p.flavor == SPX_FLAVOR_HARU) out.drawn = haru_draw(l, p.temperature, p.top_k, p.top_p);
        else out.drawn = fish_draw(l, p.temperature, p.top_k, p.top_p);
        s = out.drawn.status;
        if (s == SPX_ROW_OK) {
            const int i = pick_index(out.drawn.weights, u);
            out.report.id = out.drawn.tokens[(size_t) i];
            out.report.kept = (int32_t) out.drawn.tokens.size();
            out.report.boundary = boundary_distance(out.drawn.weights, u);
            out.report.cut = out.drawn.cut;
        }
    }
    out.report.status = s;
    if (s != SPX_ROW_OK) {
        out.report.id = -1;
        out.report.kept = 0;
        out.drawn.tokens.clear();
        out.drawn.weights.clear();
    }
    return out;
}

float widen_bf16(uint16_t h) {
    const uint32_t b = (uint32_t) h << 16;
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

// The first `cap` candidates and their weights as the reference's Candidates holds them (src/common/sampling.h:10-13):
// TRANSFORMERS normalized over the top k and not again after top-p, HARU float32 probabilities with the zeroed ones
// kept, FISH the unnormalized exponentials; -1 and 0 past the candidates.
void fill_outputs(const Drawn & d, int32_t * ids, double * weights, int cap) {
    for (int i = 0; i < cap; i++) {
        if (i < (int) d.tokens.size()) {
            ids[i] = d.tokens[(size_t) i];
            weights[i] = d.weights[(size_t) i];
        } else {
            ids[i] = -1;
            weights[i] = 0;
        }
    }
}

int copy_out(const Drawn & d, int32_t * tokens, double * weights, int cap, int * n_out) {
    const int n = d.status == SPX_ROW_OK ? (int) d.tokens.size() : 0;
    for (int i = 0; i < n && i < cap; i++) {
        tokens[i] = d.tokens[(size_t) i];
        weights[i] = d.weights[(size_t) i];
    }
    *n_out = n;
    return d.status;
}

}  // namespace

extern "C" {

void orc_uniform_fill(uint64_t seed, int n, double * out) {
    std::mt19937_64 rng(seed);
    for (int i = 0; i < n; i++) out[i] = (double) rng() * 0x1.0p-64;  // src/common/sampling.cpp:5-7
}

int orc_pick(const double * weights, int n, double u) {
    return pick_index(std::vector<double>(weights, weights + n), u);
}

int orc_tf_candidates(const float * logits, int vocab, const spx_row_params * p, const int32_t * hist, int n_hist,
                      const uint8_t * banned, int32_t * tokens, double * weights, int cap, int * n_out) {
    spx_row_params q = *p;
    q.flavor = SPX_FLAVOR_TRANSFORMERS;
    q.greedy = 0;
    *n_out = 0;
    std::vector<float> l(logits, logits + vocab);
    const int s = prepare(l, q, hist, n_hist, banned);
    if (s != SPX_ROW_OK) return s;
    return copy_out(tf_draw(l, q), tokens, weights, cap, n_out);
}

int orc_haru_candidates(const float * logits, int vocab, float temperature, int top_k, float top_p, int32_t * tokens,
                        double * weights, int cap, int * n_out) {
    std::vector<float> l(logits, logits + vocab);
    *n_out = 0;
    for (float v : l) {
        if (std::isnan(v) || v == INFINITY) return SPX_ROW_NONFINITE_INPUT;
    }
    if (temperature <= 0.0f) {
        Drawn d;
        d.tokens = {first_max(l)};
        d.weights = {1.0};
        return copy_out(d, tokens, weights, cap, n_out);
    }
    return copy_out(haru_draw(l, temperature, top_k, top_p), tokens, weights, cap, n_out);
}

int orc_fish_candidates(const float * logits, int vocab, float temperature, int top_k, float top_p, int32_t * tokens,
                        double * weights, int cap, int * n_out) {
    std::vector<float> l(logits, logits + vocab);
    *n_out = 0;
    for (float v : l) {
        if (!std::isfinite(v)) return SPX_ROW_NONFINITE_INPUT;
    }
    return copy_out(fish_draw(l, temperature, top_k, top_p), tokens, weights, cap, n_out);
}

void orc_sample_rows(const void * logits, int dtype, int rows, int vocab, int64_t ld, const int32_t * hist,
                     const int32_t * hist_off, const uint32_t * banned, int64_t banned_stride,
                     const spx_row_params * params, const double * u, orc_row_report * reports, int32_t * cand_ids,
                     double * cand_weights, int cap, int threads) {
    auto work = [&](int begin, int end) {
        std::vector<float> row((size_t) vocab);
        std::vector<uint8_t> ban;
        for (int r = begin; r < end; r++) {
            if (dtype == SPX_BF16) {
                const uint16_t * src = (const uint16_t *) logits + (int64_t) r * ld;
                for (int i = 0; i < vocab; i++) row[(size_t) i] = widen_bf16(src[i]);
            } else {
                const float * src = (const float *) logits + (int64_t) r * ld;
                std::memcpy(row.data(), src, sizeof(float) * (size_t) vocab);
            }
            const uint8_t * ban_ptr = nullptr;
            if (banned) {
                const uint32_t * words = banned + (int64_t) r * banned_stride;
                ban.assign((size_t) vocab, 0);
                for (int i = 0; i < vocab; i++) ban[(size_t) i] = (uint8_t) ((words[i >> 5] >> (i & 31)) & 1u);
                ban_ptr = ban.data();
            }
            const int32_t * h = hist ? hist + hist_off[r] : nullptr;
            const int nh = hist ? hist_off[r + 1] - hist_off[r] : 0;
            const RowOut o = sample_one(row.data(), vocab, params[r], h, nh, ban_ptr, u ? u[r] : 0.0);
            reports[r] = o.report;
            if (cand_ids && cap > 0) {
                fill_outputs(o.drawn, cand_ids + (int64_t) r * cap, cand_weights + (int64_t) r * cap, cap);
            }
        }
    };
    if (threads <= 1 || rows <= 1) {
        work(0, rows);
        return;
    }
    const int t = std::min(threads, rows);
    std::vector<std::thread> pool;
    for (int i = 0; i < t; i++) {
        const int b = (int) ((int64_t) rows * i / t), e = (int) ((int64_t) rows * (i + 1) / t);
        pool.emplace_back(work, b, e);
    }
    for (auto & th : pool) th.join();
}

void orc_talker_bans(int vocab, int suppressed_tokens, int32_t end_of_speech, int frames, int min_frames,
                     uint8_t * out) {
    // Generation::banned: src/families/qwen3-tts/sampler.cpp:62-67
    std::vector<bool> b((size_t) vocab, false);
    for (int i = vocab - suppressed_tokens; i < vocab; i++) b[(size_t) i] = i != end_of_speech;
    if (frames < min_frames) b[(size_t) end_of_speech] = true;
    for (int i = 0; i < vocab; i++) out[i] = b[(size_t) i] ? 1 : 0;
}

int orc_drama3_main(const float * logits, int vocab, const spx_row_params * first, const spx_row_params * again,
                    double u_first, double u_again, const int32_t * token_ids, int32_t semantic_begin,
                    int32_t semantic_end, int window, const int32_t * history, int n_history, int32_t * out_id) {
    // FrameSampler::main: src/families/drama3/sampler.cpp:70-79, both candidates() first
    *out_id = -1;
    std::vector<float> l(logits, logits + vocab);
    for (float v : l) {
        if (!std::isfinite(v)) return SPX_ROW_NONFINITE_INPUT;  // drama3/sampler.cpp:35-37, in either call
    }
    const Drawn drawn = fish_draw(l, first->temperature, first->top_k, first->top_p);
    if (drawn.status != SPX_ROW_OK) return drawn.status;
    const Drawn redrawn = fish_draw(l, again->temperature, again->top_k, again->top_p);
    if (redrawn.status != SPX_ROW_OK) return redrawn.status;
    const int32_t id = token_ids[drawn.tokens[(size_t) pick_index(drawn.weights, u_first)]];
    const int32_t other = token_ids[redrawn.tokens[(size_t) pick_index(redrawn.weights, u_again)]];
    const int from = n_history - std::min(window, n_history);
    const bool recent = std::find(history + from, history + n_history, id) != history + n_history;
    const bool semantic = id >= semantic_begin && id <= semantic_end;
    *out_id = semantic && recent ? other : id;
    return SPX_ROW_OK;
}

int orc_final_logits(const float * logits, int vocab, const spx_row_params * p, const int32_t * hist, int n_hist,
                     const uint8_t * banned, float * out) {
    std::vector<float> l(logits, logits + vocab);
    const int s = prepare(l, *p, hist, n_hist, banned);
    if (s == SPX_ROW_OK && !is_greedy(*p)) {
        const float t = p->flavor == SPX_FLAVOR_FISH ? std::max(p->temperature, 1e-5f) : p->temperature;
        for (float & v : l) v /= t;
    }
    std::memcpy(out, l.data(), sizeof(float) * (size_t) vocab);
    return s;
}

}  // extern "C"

// ---- Haru's DRY and shape_logits ----

// Dry (src/families/haru/sampler.cpp:83-114) run over `tokens` from a fresh state: the history it keeps and the
// penalties of its last update, by rising token (std::map order), as doubles.
int orc_dry_run(const spx_dry_config * c, const int32_t * exempt, int n_exempt, const int32_t * tokens, int n_tokens,
                int32_t * hist_out, int * n_hist, int32_t * pen_tokens, double * pen, int cap) {
    auto is_exempt = [&](int32_t t) {
        for (int i = 0; i < n_exempt; i++)
            if (exempt[i] == t) return true;
        return false;
    };
    std::vector<int32_t> h;
    std::vector<std::pair<int32_t, double>> out;
    const size_t size = (size_t) c->lookback + (size_t) c->max_match_length + 1;
    for (int s = 0; s < n_tokens; s++) {
        const int32_t token = tokens[s];
        if (is_exempt(token)) continue;  // the state and its penalties stay
        h.push_back(token);
        if (h.size() > size) h.erase(h.begin(), h.begin() + (std::ptrdiff_t) (h.size() - size));
        out.clear();
        const int64_t n = (int64_t) h.size();
        if (n < std::max(1, c->allowed_length)) continue;
        std::map<int32_t, int> best;  // token -> its longest match
        const int32_t last = h[(size_t) (n - 1)];
        const int64_t stop = std::max<int64_t>(0, n - 1 - c->lookback);
        for (int64_t j = n - 2; j >= stop; j--) {
            if (h[(size_t) j] != last) continue;
            int len = 1;
            while (len < c->max_match_length && j - len >= 0 && h[(size_t) (j - len)] == h[(size_t) (n - 1 - len)]) len++;
            if (len < c->allowed_length) continue;
            const int32_t next = h[(size_t) (j + 1)];
            auto it = best.find(next);
            if (it == best.end()) best.emplace(next, len);
            else if (len > it->second) it->second = len;
        }
        for (const auto & kv : best) {
            if (is_exempt(kv.first)) continue;
            out.emplace_back(kv.first, std::min(c->max_penalty,
                                                c->multiplier * std::pow(c->base, kv.second - c->allowed_length)));
        }
    }
    if (hist_out) std::copy(h.begin(), h.end(), hist_out);
    if (n_hist) *n_hist = (int) h.size();
    for (size_t i = 0; i < out.size() && (int) i < cap; i++) {
        pen_tokens[i] = out[i].first;
        pen[i] = out[i].second;
    }
    return (int) out.size();
}

// shape_logits (src/families/haru/sampler.cpp:112-124) with the penalties of orc_dry_run.
void orc_haru_shape(float * logits, const int32_t * pen_tokens, const double * pen, int n_pen, const float * silent,
                    int32_t pad, int32_t eop, int32_t eos, float eop_bias, int must_speak) {
    for (int i = 0; i < n_pen; i++) logits[pen_tokens[i]] -= (float) pen[i];
    logits[pad] = silent[0];
    logits[eop] = silent[1];
    if (eop_bias != 0.0f) logits[eop] += eop_bias;
    if (must_speak) logits[pad] = logits[eop] = logits[eos] = -INFINITY;
}
