// spx_host.cpp — the reference's sampler entry points over the C ABI (include/spx_sampler.h), one row per call.
// Each function fills one spx_row_params record the way the reference's function reads its settings, samples the row
// on the device, and turns the row status back into the exception the reference throws.

#include "spx_host.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>

#include "../../include/spx_sampler.h"

namespace spx_host {
namespace {

std::string number(float v) {
    char b[32];
    std::snprintf(b, sizeof b, "%.9g", (double) v);
    return b;
}

void check_hip(hipError_t e, const char * what) {
    if (e == hipErrorOutOfMemory) throw Error(Fault::OutOfMemory, std::string(what) + ": " + hipGetErrorString(e));
    if (e != hipSuccess) throw Error(Fault::Device, std::string(what) + ": " + hipGetErrorString(e));
}

void check_spx(spx_status s) {
    switch (s) {
    case SPX_OK: return;
    case SPX_ERR_OUT_OF_MEMORY: throw Error(Fault::OutOfMemory, spx_last_error());
    case SPX_ERR_INVALID_ARGUMENT: throw Error(Fault::InvalidArgument, spx_last_error());
    default: throw Error(Fault::Device, spx_last_error());
    }
}

// The candidates the device lists per row (the C ABI's limit on max_out).
constexpr int kListed = 256;

// One device's handle, staging buffers and stream, for rows of at most `vocab` logits and `hist` history ids.
class Workspace {
public:
    Workspace(int device, int vocab, int hist)
        : device_(device), vocab_(vocab), hist_(hist), listed_(std::min(vocab, kListed)) {
        check_hip(hipSetDevice(device), "hipSetDevice");
        check_spx(spx_sampler_create(&handle_, 1, vocab, hist, listed_));
        const size_t words = (size_t) (vocab + 31) / 32;
        const size_t bytes = (size_t) vocab * 4 + sizeof(spx_row_params) + 8 + (size_t) std::max(hist, 1) * 4 + 8 +
                             words * 4 + 3 * 4 + (size_t) listed_ * 12 + 64;
        check_hip(hipMalloc(&base_, bytes), "hipMalloc");
        char * p = (char *) base_;
        auto take = [&](size_t n) { void * r = p; p += (n + 15) / 16 * 16; return r; };
        logits_ = (float *) take((size_t) vocab * 4);
        params_ = (spx_row_params *) take(sizeof(spx_row_params));
        u_ = (double *) take(8);
        hist_ids_ = (int32_t *) take((size_t) std::max(hist, 1) * 4);
        hist_off_ = (int32_t *) take(8);
        banned_ = (uint32_t *) take(words * 4);
        out_ = (int32_t *) take(3 * 4);
        cand_ids_ = (int32_t *) take((size_t) listed_ * 4);
        cand_w_ = (double *) take((size_t) listed_ * 8);
        check_hip(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
    }
    ~Workspace() {
        if (stream_) (void) hipStreamDestroy(stream_);
        if (base_) (void) hipFree(base_);
        spx_sampler_destroy(handle_);
    }
    Workspace(const Workspace &) = delete;
    Workspace & operator=(const Workspace &) = delete;

    bool fits(int vocab, int hist) const { return vocab <= vocab_ && hist <= hist_; }

    struct Row {
        int32_t id, status, kept;
        std::vector<int32_t> ids;
        std::vector<double> weights;
    };

    Row run(const std::vector<float> & logits, const spx_row_params & p, const std::vector<int32_t> * history,
            const std::vector<bool> * banned, double u, bool want_candidates) {
        const int vocab = (int) logits.size();
        check_hip(hipSetDevice(device_), "hipSetDevice");
        check_hip(hipMemcpyAsync(logits_, logits.data(), (size_t) vocab * 4, hipMemcpyHostToDevice, stream_), "copy logits");
        check_hip(hipMemcpyAsync(params_, &p, sizeof p, hipMemcpyHostToDevice, stream_), "copy params");
        check_hip(hipMemcpyAsync(u_, &u, 8, hipMemcpyHostToDevice, stream_), "copy u");
        const int32_t * d_hist = nullptr;
        const int32_t * d_hist_off = nullptr;
        if (history) {
            const int32_t off[2] = {0, (int32_t) history->size()};
            staged_off_.assign(off, off + 2);
            if (!history->empty())
                check_hip(hipMemcpyAsync(hist_ids_, history->data(), history->size() * 4, hipMemcpyHostToDevice, stream_),
                          "copy history");
            check_hip(hipMemcpyAsync(hist_off_, staged_off_.data(), 8, hipMemcpyHostToDevice, stream_), "copy offsets");
            d_hist = hist_ids_;
            d_hist_off = hist_off_;
        }
        const uint32_t * d_banned = nullptr;
        if (banned) {
            // bit i%32 of word i/32 for each banned id below the vocabulary (restricted() reads min(V, banned.size()))
            staged_bits_.assign((size_t) (vocab + 31) / 32, 0u);
            const size_t n = std::min(banned->size(), (size_t) vocab);
            for (size_t i = 0; i < n; i++)
                if ((*banned)[i]) staged_bits_[i >> 5] |= 1u << (i & 31);
            check_hip(hipMemcpyAsync(banned_, staged_bits_.data(), staged_bits_.size() * 4, hipMemcpyHostToDevice, stream_),
                      "copy banned");
            d_banned = banned_;
        }
        check_spx(spx_sample_rows(handle_, logits_, SPX_F32, 1, vocab, vocab, d_hist, d_hist_off, d_banned, 0, params_, u_,
                                  out_, out_ + 1, out_ + 2, want_candidates ? cand_ids_ : nullptr,
                                  want_candidates ? cand_w_ : nullptr, stream_));
        int32_t o[3];
        check_hip(hipMemcpyAsync(o, out_, sizeof o, hipMemcpyDeviceToHost, stream_), "copy result");
        Row r;
        if (want_candidates) {
            r.ids.resize((size_t) listed_);
            r.weights.resize((size_t) listed_);
            check_hip(hipMemcpyAsync(r.ids.data(), cand_ids_, (size_t) listed_ * 4, hipMemcpyDeviceToHost, stream_),
                      "copy ids");
            check_hip(hipMemcpyAsync(r.weights.data(), cand_w_, (size_t) listed_ * 8, hipMemcpyDeviceToHost, stream_),
                      "copy weights");
        }
        check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");
        r.id = o[0];
        r.status = o[1];
        r.kept = o[2];
        return r;
    }

private:
    int device_, vocab_, hist_, listed_;
    spx_sampler * handle_ = nullptr;
    void * base_ = nullptr;
    float * logits_ = nullptr;
    spx_row_params * params_ = nullptr;
    double * u_ = nullptr;
    int32_t * hist_ids_ = nullptr;
    int32_t * hist_off_ = nullptr;
    uint32_t * banned_ = nullptr;
    int32_t * out_ = nullptr;
    int32_t * cand_ids_ = nullptr;
    double * cand_w_ = nullptr;
    hipStream_t stream_ = nullptr;
    std::vector<int32_t> staged_off_;
    std::vector<uint32_t> staged_bits_;
};

Workspace & workspace(int vocab, int hist) {
    thread_local std::map<int, std::unique_ptr<Workspace>> by_device;
    int device = 0;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    std::unique_ptr<Workspace> & w = by_device[device];
    if (!w || !w->fits(vocab, hist)) {
        w.reset();
        w = std::make_unique<Workspace>(device, std::max(vocab, 1), std::max(hist, 0));
    }
    return *w;
}

// The exception the reference throws for a row status of `flavor` (the messages of the throw sites cited in
// include/spx_sampler.h).
void raise(int32_t status, int flavor, const spx_row_params & p) {
    switch (status) {
    case SPX_ROW_OK: return;
    case SPX_ROW_REP_PENALTY_OVERFLOW:
        throw Error(Fault::OutOfRange,
                    "the repetition penalty " + number(p.repetition_penalty) +
                        " pushes a logit beyond the range of a float; give a penalty nearer 1",
                    "repetition_penalty");
    case SPX_ROW_TEMPERATURE_OVERFLOW:
        throw Error(Fault::OutOfRange,
                    "the temperature " + number(p.temperature) +
                        " pushes the logits beyond the range of a float; give a temperature nearer 1",
                    "temperature");
    case SPX_ROW_NO_FINITE_LOGIT: throw std::runtime_error("no token has a finite logit to pick from");
    case SPX_ROW_NONFINITE_INPUT:
        if (flavor == SPX_FLAVOR_FISH)
            throw Error(Fault::Device, "the device computed logits that are not finite numbers; run the model on another "
                                       "device or with another weight type");
        throw Error(Fault::Device, "the model computed a logit that is not a number; run it on another device");
    default: throw Error(Fault::InvalidArgument, "the sampling settings are not ones the sampler takes");
    }
}

spx_row_params transformers_params(const SamplingParams & p, const ExtraPenalties & e) {
    spx_row_params r{};
    r.flavor = SPX_FLAVOR_TRANSFORMERS;
    r.greedy = p.greedy ? 1 : 0;
    r.temperature = p.temperature;
    r.top_k = p.top_k;
    r.top_p = p.top_p;
    r.repetition_penalty = p.repetition_penalty;
    r.presence_penalty = e.presence;
    r.frequency_penalty = e.frequency;
    return r;
}

template <typename S>
spx_row_params family_params(int flavor, const S & s) {
    spx_row_params r{};
    r.flavor = flavor;
    r.greedy = 0;
    r.temperature = s.temperature;
    r.top_k = s.top_k;
    r.top_p = s.top_p;
    r.repetition_penalty = 1.0f;
    return r;
}

// The kept candidates of a row the device listed in full (at most kListed; a longer list is refused).
Candidates to_candidates(const Workspace::Row & r) {
    Candidates c;
    for (int i = 0; i < r.kept; i++) {
        if (i >= (int) r.ids.size() || r.ids[(size_t) i] < 0)
            throw Error(Fault::InvalidArgument, "the draw keeps " + std::to_string(r.kept) +
                                                    " tokens, more than the device lists; sample() draws from them");
        c.tokens.push_back(r.ids[(size_t) i]);
        c.weights.push_back(r.weights[(size_t) i]);
    }
    return c;
}

}  // namespace

Candidates candidates(const std::vector<float> & logits, const SamplingParams & p, const std::vector<int32_t> & history,
                      const std::vector<bool> & banned) {
    SamplingParams q = p;
    q.greedy = false;
    const spx_row_params r = transformers_params(q, ExtraPenalties{});
    Workspace::Row row = workspace((int) logits.size(), (int) history.size()).run(logits, r, &history, &banned, 0.5, true);
    raise(row.status, SPX_FLAVOR_TRANSFORMERS, r);
    return to_candidates(row);
}

int32_t sample(const std::vector<float> & logits, const SamplingParams & p, const std::vector<int32_t> & history,
               const std::vector<bool> & banned, double u, const ExtraPenalties & extra) {
    const spx_row_params r = transformers_params(p, extra);
    Workspace::Row row = workspace((int) logits.size(), (int) history.size()).run(logits, r, &history, &banned, u, false);
    raise(row.status, SPX_FLAVOR_TRANSFORMERS, r);
    return row.id;
}

int32_t sample(const std::vector<float> & logits, const SamplingParams & p, const std::vector<int32_t> & history,
               const std::vector<bool> & banned, double u) {
    return sample(logits, p, history, banned, u, ExtraPenalties{});
}

int32_t argmax(const std::vector<float> & logits, const std::vector<bool> & banned) {
    SamplingParams p;
    p.greedy = true;
    const spx_row_params r = transformers_params(p, ExtraPenalties{});
    Workspace::Row row = workspace((int) logits.size(), 0).run(logits, r, nullptr, &banned, 0.0, false);
    raise(row.status, SPX_FLAVOR_TRANSFORMERS, r);
    return row.id;
}

namespace haru {
Candidates candidates(const std::vector<float> & logits, const Sampling & s) {
    const spx_row_params r = family_params(SPX_FLAVOR_HARU, s);
    Workspace::Row row = workspace((int) logits.size(), 0).run(logits, r, nullptr, nullptr, 0.5, true);
    raise(row.status, SPX_FLAVOR_HARU, r);
    return to_candidates(row);
}
int32_t draw(const std::vector<float> & logits, const Sampling & s, double u) {
    const spx_row_params r = family_params(SPX_FLAVOR_HARU, s);
    Workspace::Row row = workspace((int) logits.size(), 0).run(logits, r, nullptr, nullptr, u, false);
    raise(row.status, SPX_FLAVOR_HARU, r);
    return row.id;
}
}  // namespace haru

namespace drama3 {
Candidates candidates(const std::vector<float> & logits, const Sampling & s) {
    const spx_row_params r = family_params(SPX_FLAVOR_FISH, s);
    Workspace::Row row = workspace((int) logits.size(), 0).run(logits, r, nullptr, nullptr, 0.5, true);
    raise(row.status, SPX_FLAVOR_FISH, r);
    return to_candidates(row);
}
int32_t draw(const std::vector<float> & logits, const Sampling & s, double u) {
    const spx_row_params r = family_params(SPX_FLAVOR_FISH, s);
    Workspace::Row row = workspace((int) logits.size(), 0).run(logits, r, nullptr, nullptr, u, false);
    raise(row.status, SPX_FLAVOR_FISH, r);
    return row.id;
}
}  // namespace drama3

}  // namespace spx_host

// ------------------------------------------------------------------------------------------------------------------
// A C surface of the layer above, for foreign-function callers and the tests: one row, host pointers, the exception
// caught and reported as (fault + 1, message, input); 0 when the call returned. fault: the Fault's value, or -1 for a
// std::runtime_error that is not an Error.
// ------------------------------------------------------------------------------------------------------------------

extern "C" {

int spx_host_call(int which, const float * logits, int vocab, const spx_row_params * p, const int32_t * history,
                  int hist_len, const uint8_t * banned, int banned_len, double u, int32_t * out_id, int32_t * out_tokens,
                  double * out_weights, int out_cap, int32_t * out_n, char * message, int message_cap, char * input,
                  int input_cap) {
    using namespace spx_host;
    auto put = [](char * dst, int cap, const char * src) {
        if (!dst || cap <= 0) return;
        std::strncpy(dst, src, (size_t) cap - 1);
        dst[cap - 1] = 0;
    };
    put(message, message_cap, "");
    put(input, input_cap, "");
    try {
        const std::vector<float> l(logits, logits + vocab);
        const std::vector<int32_t> h(history, history + (history ? hist_len : 0));
        std::vector<bool> b;
        for (int i = 0; banned && i < banned_len; i++) b.push_back(banned[i] != 0);
        SamplingParams sp;
        sp.greedy = p->greedy != 0;
        sp.temperature = p->temperature;
        sp.top_k = p->top_k;
        sp.top_p = p->top_p;
        sp.repetition_penalty = p->repetition_penalty;
        Candidates c;
        bool listed = false;
        switch (which) {
        case 0: *out_id = sample(l, sp, h, b, u, ExtraPenalties{p->presence_penalty, p->frequency_penalty}); break;
        case 1: c = candidates(l, sp, h, b); listed = true; break;
        case 2: *out_id = haru::draw(l, haru::Sampling{p->temperature, p->top_k, p->top_p}, u); break;
        case 3: c = haru::candidates(l, haru::Sampling{p->temperature, p->top_k, p->top_p}); listed = true; break;
        case 4: *out_id = drama3::draw(l, drama3::Sampling{p->temperature, p->top_k, p->top_p}, u); break;
        case 5: c = drama3::candidates(l, drama3::Sampling{p->temperature, p->top_k, p->top_p}); listed = true; break;
        case 6: *out_id = argmax(l, b); break;
        default: throw Error(Fault::InvalidArgument, "unknown entry point");
        }
        if (listed) {
            *out_n = (int32_t) c.tokens.size();
            for (int i = 0; i < (int) c.tokens.size() && i < out_cap; i++) {
                out_tokens[i] = c.tokens[(size_t) i];
                out_weights[i] = c.weights[(size_t) i];
            }
        }
        return 0;
    } catch (const Error & e) {
        put(message, message_cap, e.what());
        put(input, input_cap, e.input().c_str());
        return (int) e.fault() + 1;
    } catch (const std::exception & e) {
        put(message, message_cap, e.what());
        return -1;
    }
}

}  // extern "C"
