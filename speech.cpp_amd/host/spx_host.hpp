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
}  // namespace drama3

}  // namespace spx_host
