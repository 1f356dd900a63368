// spx_host.hpp — the C++ host layer over the sampler's C ABI: the reference's sampler entry points with the same
// names, arguments and errors, computed on the GPU. A speech.cpp build links this and calls it where it called its
// host sampler; nothing else changes.
//
//   spx_host::sample()             src/families/qwen3-tts/sampler.h:59-60 (sample(logits, p, history, banned, u))
//   spx_host::candidates()         src/families/qwen3-tts/sampler.h:52-53
//   spx_host::haru::candidates()   src/families/haru/sampler.h:32
//   spx_host::drama3::candidates() src/families/drama3/sampler.h:32
//   spx_host::haru::draw(), drama3::draw()   the pick() the families make from candidates() with one uniform
//                                  (src/families/haru/dialogue.cpp:214, src/families/drama3/sampler.cpp:70-84),
//                                  in one device call
//   spx_host::argmax()             std::max_element of the suppressed logits (src/families/qwen3-asr/decoder.cpp:112)
//   spx_host::Generation::banned() src/families/qwen3-tts/sampler.h:42
//   spx_host::GraphSampler         src/families/qwen3-tts/graph-sampler.h:18-57, the chain of picks on the device
//   spx_host::drama3::FrameSampler src/families/drama3/sampler.h:35-61
//
// Errors are the reference's: Error(Fault::OutOfRange, ..., "repetition_penalty" | "temperature"),
// Error(Fault::Device, ...) for logits that are not finite where a family refuses them, std::runtime_error where
// no logit is finite (src/common/error.h:8-39, src/families/qwen3-tts/sampler.cpp:44-49). The types below mirror
// error.h and sampling.h field for field, so that a build of the reference maps them one to one.
//
// The functions take host vectors: each call copies the row to the device, samples it there and copies the answer
// back on a stream of its own. They serve a host loop one row at a time; batched callers with device buffers call
// spx_sample_rows() directly. A thread keeps one device workspace per device, sized by the largest row it has seen.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace spx_host {

/** src/common/error.h:8-21 */
enum class Fault { InvalidArgument, OutOfRange, File, Device, OutOfMemory, Io };

/** src/common/error.h:27-39 */
class Error : public std::runtime_error {
public:
    Error(Fault fault, const std::string & message, std::string input = "")
        : std::runtime_error(message), fault_(fault), input_(std::move(input)) {}
    Fault fault() const { return fault_; }
    const std::string & input() const { return input_; }

private:
    Fault fault_;
    std::string input_;
};

/** src/common/sampling.h:10-13. Weights are proportional to the probabilities (normalized over the kept tokens). */
struct Candidates {
    std::vector<int32_t> tokens;
    std::vector<double> weights;
};

/** src/families/qwen3-tts/sampler.h:12-24 */
struct SamplingParams {
    bool greedy = false;
    float temperature = 1.0f;
    int top_k = 0;
    float top_p = 1.0f;
    float repetition_penalty = 1.0f;
};

/** Penalties the reference does not have (0 = off), applied as l = (l - frequency*c) - presence before the
    repetition penalty, for each token occurring c > 0 times in the history. */
struct ExtraPenalties {
    float presence = 0.0f;
    float frequency = 0.0f;
};

/**
 * src/families/qwen3-tts/sampler.h:26-43 without the model file: the stacks' settings, the frame bounds and the count
 * of suppressed ids at the end of the talker's vocabulary, which the caller reads from its file.
 */
struct Generation {
    SamplingParams talker, code_predictor;
    int min_frames = 0, max_frames = 0;
    int suppressed_tokens = 0;
    /** src/families/qwen3-tts/sampler.cpp:62-67 */
    std::vector<bool> banned(int vocab, int32_t end_of_speech, int frames) const;
};

/**
 * The code predictor's picks kept on the device (src/families/qwen3-tts/graph-sampler.h:18-57): `picks` picks per
 * frame for `streams` streams, each from the logits of its step's head on the device, its history the frame's codes
 * picked before it, so that a repetition penalty other than 1 stays on the device too. A frame: start() with the
 * first codes, draw() with the frame's numbers, pick() once per step between the predictor's forwards (asynchronous on
 * the given stream), read() for the codes.
 */
class GraphSampler {
public:
    /** Every setting the sampler takes is followed on the device, penalties included. */
    static bool follows(const SamplingParams & p);
    GraphSampler(const SamplingParams & p, int vocab, int picks, int streams = 1);
    ~GraphSampler();
    GraphSampler(const GraphSampler &) = delete;
    GraphSampler & operator=(const GraphSampler &) = delete;
    const SamplingParams & params() const { return p_; }
    /** The frame's first codes (the talker's), one per stream. */
    void start(const std::vector<int32_t> & first_codes);
    /** The numbers of the frame's draws, picks per stream in order, stream after stream; none for greedy picks. */
    void draw(const std::vector<double> & u);
    /** Pick `i` from the step's logits on the device, streams x vocab float32, on `stream` (a hipStream_t). */
    void pick(int i, const float * d_logits, void * stream);
    /** The codes of the frame, picks per stream, stream after stream; throws as candidates() does. */
    std::vector<int32_t> read();

private:
    SamplingParams p_;
    int vocab_, picks_, streams_;
    struct Device;
    Device * d_;
};

Candidates candidates(const std::vector<float> & logits, const SamplingParams & p, const std::vector<int32_t> & history,
                      const std::vector<bool> & banned);
int32_t sample(const std::vector<float> & logits, const SamplingParams & p, const std::vector<int32_t> & history,
               const std::vector<bool> & banned, double u);
int32_t sample(const std::vector<float> & logits, const SamplingParams & p, const std::vector<int32_t> & history,
               const std::vector<bool> & banned, double u, const ExtraPenalties & extra);
int32_t argmax(const std::vector<float> & logits, const std::vector<bool> & banned);

namespace haru {
/** src/families/haru/sampler.h:13-19 */
struct Sampling {
    float temperature = 0.7f;
    int top_k = 25;
    float top_p = 1.0f;
};
Candidates candidates(const std::vector<float> & logits, const Sampling & s);
int32_t draw(const std::vector<float> & logits, const Sampling & s, double u);

/** src/families/haru/sampler.h:35-38 */
struct DryConfig {
    double multiplier = 0, base = 0, max_penalty = 0;
    int allowed_length = 0, lookback = 0, max_match_length = 0;
};

/** src/families/haru/sampler.h:43-46 */
struct TextIds {
    int32_t pad = 0, eop = 0, eos = 0;
};

/**
 * The DRY state of one text stream (src/families/haru/sampler.h:55-75), kept on the device: update() appends there,
 * penalties() reads back the list the device forms from it, apply() subtracts them as the reference does.
 */
class Dry {
public:
    Dry(const DryConfig & config, std::vector<int32_t> exempt);
    ~Dry();
    Dry(const Dry &) = delete;
    Dry & operator=(const Dry &) = delete;
    void update(int32_t token);
    const std::vector<std::pair<int32_t, double>> & penalties() const;
    void apply(std::vector<float> & logits) const;

private:
    friend void shape_logits(std::vector<float> & logits, const Dry & dry, const float silent[2], const TextIds & ids,
                             float eop_bias, bool must_speak);
    DryConfig config_;
    std::vector<int32_t> exempt_;
    int size_ = 0;
    int32_t top_id_ = 0;  // the largest token appended (the penalties' read-back row spans it)
    struct Device;
    Device * d_;
    mutable std::vector<std::pair<int32_t, double>> penalties_;
    mutable bool fresh_ = true;
};

/** src/families/haru/sampler.cpp:116-124, on the device with the stream's DRY state. */
void shape_logits(std::vector<float> & logits, const Dry & dry, const float silent[2], const TextIds & ids,
                  float eop_bias, bool must_speak);
}  // namespace haru

namespace drama3 {
/** src/families/drama3/sampler.h:12-17 */
struct Sampling {
    float temperature = 1.0f;
    int top_k = 1;
    float top_p = 1.0f;
};
Candidates candidates(const std::vector<float> & logits, const Sampling & s);
int32_t draw(const std::vector<float> & logits, const Sampling & s, double u);

/**
 * src/families/drama3/sampler.h:35-61 without the model file: the request's settings, the redraw's, its window, the
 * semantic id range and the map from the output's logits to text-model ids, which the caller reads from its file.
 */
class FrameSampler {
public:
    FrameSampler(const Sampling & request, const Sampling & repeat, int window, int32_t semantic_begin,
                 int32_t semantic_end, std::vector<int32_t> token_ids);
    /** src/families/drama3/sampler.cpp:70-79, both draws and the redraw rule in one device call */
    int32_t main(const std::vector<float> & logits, const std::vector<int32_t> & history, double first,
                 double again) const;
    /** src/families/drama3/sampler.cpp:81-84 */
    int32_t code(const std::vector<float> & logits, double u) const;
    bool semantic(int32_t id) const { return id >= semantic_begin_ && id <= semantic_end_; }

private:
    Sampling request_, repeat_;
    int window_;
    int32_t semantic_begin_, semantic_end_;
    std::vector<int32_t> token_ids_;
};
}  // namespace drama3

}  // namespace spx_host
