// spx_host.cpp — the reference's sampler entry points over the C ABI (include/spx_sampler.h), one row per call.
// Each function fills one spx_row_params record the way the reference's function reads its settings, samples the row
// on the device, and turns the row status back into the exception the reference throws.

#include "spx_host.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>

#include "../../include/spx_sampler.h"

namespace spx_host {
namespace {

// A float in an error message as the reference writes it (src/common/json.h:39-63, json_number of a float): the
// shortest %g that reads back as the same float, in fixed notation where %g would take an exponent for a magnitude
// from 1e-4 to below 1e17; "null" for infinities and NaN.
std::string number(float v) {
    if (!std::isfinite(v)) return "null";
    char b[64];
    for (int precision = 1; precision <= 9; precision++) {
        std::snprintf(b, sizeof b, "%.*g", precision, (double) v);
        if (std::strtof(b, nullptr) == v) break;
    }
    const double magnitude = std::fabs((double) v);
    if (std::strchr(b, 'e') && magnitude >= 1e-4 && magnitude < 1e17) {
        for (int decimals = 0; decimals <= 20; decimals++) {
            std::snprintf(b, sizeof b, "%.*f", decimals, (double) v);
            if (std::strtof(b, nullptr) == v) break;
        }
    }
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

// One device's handle, staging buffers and stream, for rows of at most `vocab` logits and `hist` history ids.
class Workspace {
public:
    Workspace(int device, int vocab, int hist)
        : device_(device), vocab_(vocab), hist_(hist), listed_(vocab) {
        check_hip(hipSetDevice(device), "hipSetDevice");
        check_spx(spx_sampler_create(&handle_, 1, vocab, hist, 0));
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
        // candidates() lists every kept token (the row's whole list); a draw lists none
        if (want_candidates)
            check_spx(spx_candidates_rows(handle_, logits_, SPX_F32, 1, vocab, vocab, d_hist, d_hist_off, d_banned, 0,
                                          params_, vocab, cand_ids_, cand_w_, out_ + 2, out_ + 1, stream_));
        else
            check_spx(spx_sample_rows(handle_, logits_, SPX_F32, 1, vocab, vocab, d_hist, d_hist_off, d_banned, 0, params_,
                                      u_, out_, out_ + 1, out_ + 2, nullptr, nullptr, stream_));
        int32_t o[3];
        check_hip(hipMemcpyAsync(o, out_, sizeof o, hipMemcpyDeviceToHost, stream_), "copy result");
        Row r;
        check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");
        r.id = o[0];
        r.status = o[1];
        r.kept = o[2];
        if (want_candidates && r.status == SPX_ROW_OK) {
            // the list's own length
            const size_t n = (size_t) std::max(0, std::min(r.kept, listed_));
            r.ids.resize(n);
            r.weights.resize(n);
            check_hip(hipMemcpy(r.ids.data(), cand_ids_, n * 4, hipMemcpyDeviceToHost), "copy ids");
            check_hip(hipMemcpy(r.weights.data(), cand_w_, n * 8, hipMemcpyDeviceToHost), "copy weights");
        }
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

// A row's Candidates as the device listed them, every kept token.
Candidates to_candidates(const Workspace::Row & r) {
    Candidates c;
    c.tokens = r.ids;
    c.weights = r.weights;
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

std::vector<bool> Generation::banned(int vocab, int32_t end_of_speech, int frames) const {
    std::vector<bool> b((size_t) vocab, false);
    for (int i = std::max(0, vocab - suppressed_tokens); i < vocab; i++) b[(size_t) i] = i != end_of_speech;
    if (frames < min_frames) b[(size_t) end_of_speech] = true;
    return b;
}

// The chain's device buffers: the sampler, the codes (streams x (picks + 1)), the numbers, the settings, the statuses.
// ---- haru::Dry and shape_logits over the device entries ----

namespace haru {

struct Dry::Device {
    int32_t * hist = nullptr;  // size_ ids, then the length, then the update's token
    float * row = nullptr;     // a logits row (shape_logits, the penalties' read-back)
    int row_cap = 0;
    int32_t * pen_tokens = nullptr;
    double * pen = nullptr;
    int32_t * npen = nullptr;
    float * silent = nullptr;
    uint8_t * speak = nullptr;
};

namespace {
spx_dry_config dry_config(const DryConfig & c) {
    spx_dry_config k{};
    k.multiplier = c.multiplier;
    k.base = c.base;
    k.max_penalty = c.max_penalty;
    k.allowed_length = c.allowed_length;
    k.lookback = c.lookback;
    k.max_match_length = c.max_match_length;
    return k;
}
}  // namespace

Dry::Dry(const DryConfig & config, std::vector<int32_t> exempt)
    : config_(config), exempt_(std::move(exempt)), d_(new Device()) {
    if (config.lookback < 0 || config.max_match_length < 0) throw std::invalid_argument("negative DRY lookback or match length");
    size_ = config.lookback + config.max_match_length + 1;
    const size_t bytes = (size_t) (size_ + 2) * 4 + (size_t) size_ * 12 + 8 + 16;
    check_hip(hipMalloc((void **) &d_->hist, bytes), "hipMalloc");
    d_->pen_tokens = d_->hist + size_ + 2;
    d_->pen = (double *) (((uintptr_t) (d_->pen_tokens + size_) + 7) & ~(uintptr_t) 7);
    d_->npen = (int32_t *) (d_->pen + size_);
    d_->silent = (float *) (d_->npen + 1);
    d_->speak = (uint8_t *) (d_->silent + 2);
    check_hip(hipMemset(d_->hist, 0, (size_t) (size_ + 2) * 4), "hipMemset");
}

Dry::~Dry() {
    if (d_->hist) (void) hipFree(d_->hist);
    if (d_->row) (void) hipFree(d_->row);
    delete d_;
}

void Dry::update(int32_t token) {
    int32_t * tok = d_->hist + size_ + 1;
    check_hip(hipMemcpy(tok, &token, 4, hipMemcpyHostToDevice), "copy token");
    const spx_dry_config c = dry_config(config_);
    check_spx(spx_dry_update_rows(1, &c, exempt_.data(), (int) exempt_.size(), tok, d_->hist, d_->hist + size_,
                                  size_, nullptr));
    check_hip(hipDeviceSynchronize(), "dry update");
    if (std::find(exempt_.begin(), exempt_.end(), token) == exempt_.end()) top_id_ = std::max(top_id_, token);
    fresh_ = true;
}

const std::vector<std::pair<int32_t, double>> & Dry::penalties() const {
    if (!fresh_) return penalties_;
    // a row spanning every token the history holds; its logits are not read back
    const int vocab = std::max(top_id_ + 1, 1);
    if (d_->row_cap < vocab) {
        if (d_->row) (void) hipFree(d_->row);
        d_->row = nullptr;
        check_hip(hipMalloc((void **) &d_->row, (size_t) vocab * 4), "hipMalloc");
        d_->row_cap = vocab;
    }
    const float zero[2] = {0.0f, 0.0f};
    check_hip(hipMemcpy(d_->silent, zero, 8, hipMemcpyHostToDevice), "copy silent");
    const spx_dry_config c = dry_config(config_);
    check_spx(spx_haru_shape_rows(d_->row, 1, vocab, vocab, &c, exempt_.data(), (int) exempt_.size(), d_->hist,
                                  d_->hist + size_, size_, d_->silent, 0, 0, 0, 0.0f, nullptr, d_->pen_tokens, d_->pen,
                                  d_->npen, size_, nullptr));
    int32_t n = 0;
    check_hip(hipMemcpy(&n, d_->npen, 4, hipMemcpyDeviceToHost), "copy count");
    n = std::min(n, size_);
    std::vector<int32_t> t((size_t) n);
    std::vector<double> w((size_t) n);
    if (n) {
        check_hip(hipMemcpy(t.data(), d_->pen_tokens, (size_t) n * 4, hipMemcpyDeviceToHost), "copy penalties");
        check_hip(hipMemcpy(w.data(), d_->pen, (size_t) n * 8, hipMemcpyDeviceToHost), "copy penalties");
    }
    penalties_.clear();
    for (int i = 0; i < n; i++) penalties_.emplace_back(t[(size_t) i], w[(size_t) i]);
    fresh_ = false;
    return penalties_;
}

void Dry::apply(std::vector<float> & logits) const {
    for (const auto & [t, penalty] : penalties()) logits[(size_t) t] -= (float) penalty;
}

void shape_logits(std::vector<float> & logits, const Dry & dry, const float silent[2], const TextIds & ids,
                  float eop_bias, bool must_speak) {
    const int vocab = (int) logits.size();
    Dry::Device & d = *dry.d_;
    if (d.row_cap < vocab) {
        if (d.row) (void) hipFree(d.row);
        d.row = nullptr;
        check_hip(hipMalloc((void **) &d.row, (size_t) vocab * 4), "hipMalloc");
        d.row_cap = vocab;
    }
    const uint8_t speak = must_speak ? 1 : 0;
    check_hip(hipMemcpy(d.row, logits.data(), (size_t) vocab * 4, hipMemcpyHostToDevice), "copy logits");
    check_hip(hipMemcpy(d.silent, silent, 8, hipMemcpyHostToDevice), "copy silent");
    check_hip(hipMemcpy(d.speak, &speak, 1, hipMemcpyHostToDevice), "copy must_speak");
    const spx_dry_config c = dry_config(dry.config_);
    check_spx(spx_haru_shape_rows(d.row, 1, vocab, vocab, &c, dry.exempt_.data(), (int) dry.exempt_.size(), d.hist,
                                  d.hist + dry.size_, dry.size_, d.silent, ids.pad, ids.eop, ids.eos, eop_bias, d.speak,
                                  nullptr, nullptr, nullptr, 0, nullptr));
    check_hip(hipMemcpy(logits.data(), d.row, (size_t) vocab * 4, hipMemcpyDeviceToHost), "copy logits");
}

}  // namespace haru

struct GraphSampler::Device {
    spx_sampler * handle = nullptr;
    void * base = nullptr;
    int32_t * codes = nullptr;
    double * u = nullptr;
    spx_row_params * params = nullptr;
    int32_t * status = nullptr;
    void * last_stream = nullptr;
};

bool GraphSampler::follows(const SamplingParams & p) { return p.greedy || (p.temperature > 0.0f && std::isfinite(p.temperature)); }

GraphSampler::GraphSampler(const SamplingParams & p, int vocab, int picks, int streams)
    : p_(p), vocab_(vocab), picks_(picks), streams_(streams), d_(new Device()) {
    if (!follows(p)) throw std::logic_error("the chain cannot pick under a temperature that is not a positive number");
    check_spx(spx_sampler_create(&d_->handle, streams, vocab, picks, 0));
    const size_t bytes = (size_t) streams * ((picks + 1) * 4 + picks * 8 + sizeof(spx_row_params) + 4) + 256;
    check_hip(hipMalloc(&d_->base, bytes), "hipMalloc");
    char * q = (char *) d_->base;
    d_->u = (double *) q;
    q += (size_t) streams * picks * 8;
    d_->params = (spx_row_params *) q;
    q += (size_t) streams * sizeof(spx_row_params);
    d_->codes = (int32_t *) q;
    q += (size_t) streams * (picks + 1) * 4;
    d_->status = (int32_t *) q;
    std::vector<spx_row_params> rp((size_t) streams, transformers_params(p, ExtraPenalties{}));
    check_hip(hipMemcpy(d_->params, rp.data(), rp.size() * sizeof(spx_row_params), hipMemcpyHostToDevice), "copy params");
    std::vector<double> zero((size_t) streams * picks, 0.0);
    check_hip(hipMemcpy(d_->u, zero.data(), zero.size() * 8, hipMemcpyHostToDevice), "copy u");
}

GraphSampler::~GraphSampler() {
    if (d_->base) (void) hipFree(d_->base);
    spx_sampler_destroy(d_->handle);
    delete d_;
}

void GraphSampler::start(const std::vector<int32_t> & first_codes) {
    if ((int) first_codes.size() != streams_) throw std::logic_error("a frame was started with another count of streams");
    std::vector<int32_t> frame((size_t) streams_ * (picks_ + 1), -1);
    for (int r = 0; r < streams_; r++) frame[(size_t) r * (picks_ + 1)] = first_codes[(size_t) r];
    check_hip(hipMemcpy(d_->codes, frame.data(), frame.size() * 4, hipMemcpyHostToDevice), "copy codes");
}

void GraphSampler::draw(const std::vector<double> & u) {
    // src/families/qwen3-tts/graph-sampler.cpp:62-73
    if (p_.greedy) {
        if (!u.empty()) throw std::logic_error("greedy picks were given numbers to draw with");
        return;
    }
    if ((int) u.size() != picks_ * streams_) throw std::logic_error("picks in a chain were given another count of numbers to draw with");
    check_hip(hipMemcpy(d_->u, u.data(), u.size() * 8, hipMemcpyHostToDevice), "copy u");
}

void GraphSampler::pick(int i, const float * d_logits, void * stream) {
    if (i < 0 || i >= picks_) throw std::logic_error("a pick outside the chain's picks");
    check_spx(spx_sample_chain(d_->handle, d_logits, SPX_F32, streams_, vocab_, vocab_, d_->codes, picks_ + 1, i, picks_,
                               d_->params, d_->u, d_->status, stream));
    d_->last_stream = stream;
}

std::vector<int32_t> GraphSampler::read() {
    check_hip(hipStreamSynchronize((hipStream_t) d_->last_stream), "hipStreamSynchronize");
    std::vector<int32_t> frame((size_t) streams_ * (picks_ + 1)), status((size_t) streams_);
    check_hip(hipMemcpy(frame.data(), d_->codes, frame.size() * 4, hipMemcpyDeviceToHost), "copy codes");
    check_hip(hipMemcpy(status.data(), d_->status, status.size() * 4, hipMemcpyDeviceToHost), "copy status");
    const spx_row_params rp = transformers_params(p_, ExtraPenalties{});
    for (int32_t st : status) raise(st, SPX_FLAVOR_TRANSFORMERS, rp);
    std::vector<int32_t> ids((size_t) streams_ * picks_);
    for (int r = 0; r < streams_; r++)
        for (int i = 0; i < picks_; i++) ids[(size_t) r * picks_ + i] = frame[(size_t) r * (picks_ + 1) + 1 + i];
    return ids;
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

FrameSampler::FrameSampler(const Sampling & request, const Sampling & repeat, int window, int32_t semantic_begin,
                           int32_t semantic_end, std::vector<int32_t> token_ids)
    : request_(request), repeat_(repeat), window_(window), semantic_begin_(semantic_begin), semantic_end_(semantic_end),
      token_ids_(std::move(token_ids)) {}

int32_t FrameSampler::main(const std::vector<float> & logits, const std::vector<int32_t> & history, double first,
                           double again) const {
    const int vocab = (int) logits.size();
    if ((int) token_ids_.size() < vocab) throw Error(Fault::InvalidArgument, "fewer token ids than logits");
    int device = 0;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    thread_local std::map<int, std::unique_ptr<spx_sampler, void (*)(spx_sampler *)>> handles;
    auto it = handles.find(device);
    if (it == handles.end()) {
        spx_sampler * h = nullptr;
        check_spx(spx_sampler_create(&h, 2, std::max(vocab, 4097), 0, 0));
        it = handles.emplace(device, std::unique_ptr<spx_sampler, void (*)(spx_sampler *)>(h, spx_sampler_destroy)).first;
    }
    const spx_row_params r1 = family_params(SPX_FLAVOR_FISH, request_), r2 = family_params(SPX_FLAVOR_FISH, repeat_);
    const size_t nh = history.size();
    const size_t bytes = (size_t) vocab * 4 * 2 + 2 * sizeof(spx_row_params) + 16 + (nh + 2) * 4 + 8 + 64;
    void * base = nullptr;
    check_hip(hipMalloc(&base, bytes), "hipMalloc");
    std::unique_ptr<void, hipError_t (*)(void *)> guard(base, hipFree);
    char * q = (char *) base;
    auto take = [&](size_t n) { void * p = q; q += (n + 15) / 16 * 16; return p; };
    float * d_logits = (float *) take((size_t) vocab * 4);
    int32_t * d_ids = (int32_t *) take((size_t) vocab * 4);
    spx_row_params * d_p = (spx_row_params *) take(2 * sizeof(spx_row_params));
    double * d_u = (double *) take(16);
    int32_t * d_hist = (int32_t *) take((nh + 1) * 4);
    int32_t * d_off = (int32_t *) take(8);
    int32_t * d_out = (int32_t *) take(8);
    const spx_row_params ps[2] = {r1, r2};
    const double us[2] = {first, again};
    const int32_t off[2] = {0, (int32_t) nh};
    check_hip(hipMemcpy(d_logits, logits.data(), (size_t) vocab * 4, hipMemcpyHostToDevice), "copy logits");
    check_hip(hipMemcpy(d_ids, token_ids_.data(), (size_t) vocab * 4, hipMemcpyHostToDevice), "copy token ids");
    check_hip(hipMemcpy(d_p, ps, sizeof ps, hipMemcpyHostToDevice), "copy params");
    check_hip(hipMemcpy(d_u, us, sizeof us, hipMemcpyHostToDevice), "copy u");
    if (nh) check_hip(hipMemcpy(d_hist, history.data(), nh * 4, hipMemcpyHostToDevice), "copy history");
    check_hip(hipMemcpy(d_off, off, sizeof off, hipMemcpyHostToDevice), "copy offsets");
    check_spx(spx_drama3_main(it->second.get(), d_logits, SPX_F32, 1, vocab, vocab, d_p, d_p + 1, d_u, d_u + 1, d_ids,
                              semantic_begin_, semantic_end_, window_, d_hist, d_off, d_out, d_out + 1, nullptr));
    int32_t out[2];
    check_hip(hipMemcpy(out, d_out, sizeof out, hipMemcpyDeviceToHost), "copy result");
    raise(out[1], SPX_FLAVOR_FISH, r1);
    return out[0];
}

int32_t FrameSampler::code(const std::vector<float> & logits, double u) const { return draw(logits, request_, u); }
}  // namespace drama3

}  // namespace spx_host

// ------------------------------------------------------------------------------------------------------------------
// A C surface of the layer above, for foreign-function callers and the tests: one row, host pointers, the exception
// caught and reported as (fault + 1, message, input); 0 when the call returned. fault: the Fault's value, or -1 for a
// std::runtime_error that is not an Error.
// ------------------------------------------------------------------------------------------------------------------

extern "C" {

// The exception the host layer throws for a row status, as (fault + 1, message, input): 0 for SPX_ROW_OK, -1 for a
// std::runtime_error. It needs no device: the formatting of the reference's messages is checked on the host.
int spx_host_row_error(int status, const spx_row_params * p, char * message, int message_cap, char * input,
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
        raise(status, p->flavor, *p);
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

// ------------------------------------------------------------------------------------------------------------------
// C surfaces of the families' classes above, for foreign-function callers and the tests; an exception is reported as
// in spx_host_call.
// ------------------------------------------------------------------------------------------------------------------

namespace {

template <typename F>
int report(char * message, int message_cap, F && f) {
    auto put = [&](const char * src) {
        if (!message || message_cap <= 0) return;
        std::strncpy(message, src, (size_t) message_cap - 1);
        message[message_cap - 1] = 0;
    };
    put("");
    try {
        f();
        return 0;
    } catch (const spx_host::Error & e) {
        put(e.what());
        return (int) e.fault() + 1;
    } catch (const std::exception & e) {
        put(e.what());
        return -1;
    }
}

}  // namespace

extern "C" {

void spx_host_talker_banned(int vocab, int suppressed_tokens, int32_t end_of_speech, int frames, int min_frames,
                            uint8_t * out) {
    spx_host::Generation g;
    g.suppressed_tokens = suppressed_tokens;
    g.min_frames = min_frames;
    const std::vector<bool> b = g.banned(vocab, end_of_speech, frames);
    for (int i = 0; i < vocab; i++) out[i] = b[(size_t) i] ? 1 : 0;
}

int spx_host_frame_main(const float * logits, int vocab, const spx_row_params * request, const spx_row_params * repeat,
                        int window, int32_t semantic_begin, int32_t semantic_end, const int32_t * token_ids,
                        const int32_t * history, int n_history, double first, double again, int32_t * out_id,
                        char * message, int message_cap) {
    return report(message, message_cap, [&] {
        using spx_host::drama3::Sampling;
        const spx_host::drama3::FrameSampler f(Sampling{request->temperature, request->top_k, request->top_p},
                                               Sampling{repeat->temperature, repeat->top_k, repeat->top_p}, window,
                                               semantic_begin, semantic_end,
                                               std::vector<int32_t>(token_ids, token_ids + vocab));
        *out_id = f.main(std::vector<float>(logits, logits + vocab),
                         std::vector<int32_t>(history, history + (history ? n_history : 0)), first, again);
    });
}

// Haru's Dry over `n` tokens, then its penalties (by rising token, the first `cap`); returns their count in *n_out.
int spx_host_dry_penalties(const double * cfg3, const int32_t * cfg_ints, const int32_t * exempt, int n_exempt,
                           const int32_t * tokens, int n, int32_t * out_tokens, double * out_pen, int cap, int * n_out,
                           char * message, int message_cap) {
    return report(message, message_cap, [&] {
        spx_host::haru::DryConfig c;
        c.multiplier = cfg3[0];
        c.base = cfg3[1];
        c.max_penalty = cfg3[2];
        c.allowed_length = cfg_ints[0];
        c.lookback = cfg_ints[1];
        c.max_match_length = cfg_ints[2];
        spx_host::haru::Dry dry(c, std::vector<int32_t>(exempt, exempt + n_exempt));
        for (int i = 0; i < n; i++) dry.update(tokens[i]);
        const auto & p = dry.penalties();
        *n_out = (int) p.size();
        for (int i = 0; i < (int) p.size() && i < cap; i++) {
            out_tokens[i] = p[(size_t) i].first;
            out_pen[i] = p[(size_t) i].second;
        }
    });
}

// shape_logits of one row after Dry over `n` tokens, in place.
int spx_host_haru_shape(const double * cfg3, const int32_t * cfg_ints, const int32_t * exempt, int n_exempt,
                        const int32_t * tokens, int n, float * logits, int vocab, const float * silent, int32_t pad,
                        int32_t eop, int32_t eos, float eop_bias, int must_speak, char * message, int message_cap) {
    return report(message, message_cap, [&] {
        spx_host::haru::DryConfig c;
        c.multiplier = cfg3[0];
        c.base = cfg3[1];
        c.max_penalty = cfg3[2];
        c.allowed_length = cfg_ints[0];
        c.lookback = cfg_ints[1];
        c.max_match_length = cfg_ints[2];
        spx_host::haru::Dry dry(c, std::vector<int32_t>(exempt, exempt + n_exempt));
        for (int i = 0; i < n; i++) dry.update(tokens[i]);
        std::vector<float> l(logits, logits + vocab);
        spx_host::haru::shape_logits(l, dry, silent, spx_host::haru::TextIds{pad, eop, eos}, eop_bias, must_speak != 0);
        std::copy(l.begin(), l.end(), logits);
    });
}

// The chain over host logits (picks x streams x vocab), each step's copied to the device before its pick.
int spx_host_graph_chain(const float * logits, int streams, int vocab, int picks, const spx_row_params * p,
                         const int32_t * first_codes, const double * u, int32_t * out_codes, char * message,
                         int message_cap) {
    return report(message, message_cap, [&] {
        spx_host::SamplingParams sp;
        sp.greedy = p->greedy != 0;
        sp.temperature = p->temperature;
        sp.top_k = p->top_k;
        sp.top_p = p->top_p;
        sp.repetition_penalty = p->repetition_penalty;
        spx_host::GraphSampler g(sp, vocab, picks, streams);
        g.start(std::vector<int32_t>(first_codes, first_codes + streams));
        if (!sp.greedy) g.draw(std::vector<double>(u, u + (size_t) picks * streams));
        float * d = nullptr;
        spx_host::check_hip(hipMalloc((void **) &d, (size_t) streams * vocab * 4), "hipMalloc");
        std::unique_ptr<void, hipError_t (*)(void *)> guard(d, hipFree);
        for (int i = 0; i < picks; i++) {
            spx_host::check_hip(hipMemcpy(d, logits + (size_t) i * streams * vocab, (size_t) streams * vocab * 4,
                                hipMemcpyHostToDevice), "copy logits");
            g.pick(i, d, nullptr);
        }
        const std::vector<int32_t> ids = g.read();
        std::copy(ids.begin(), ids.end(), out_codes);
    });
}

}  // extern "C"
