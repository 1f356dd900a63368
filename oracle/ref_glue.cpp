// ref_glue.cpp — TEST INFRASTRUCTURE ONLY. C entry points over the reference's own src/common/sampling.cpp, which the
// oracle Makefile compiles unchanged from the reference checkout into oracle/_ref/. Only tests load the result, to
// check the oracle's uniform() and pick() restatements bit for bit against the reference's compiled code.

#include <cstdint>
#include <cstring>
#include <random>
#include <vector>

#include "sampling.h"  // the reference's header, found through -I<reference>/src/common

extern "C" {

void ref_uniform_fill(uint64_t seed, int n, double * out) {
    std::mt19937_64 rng(seed);
    for (int i = 0; i < n; i++) out[i] = uniform(rng);
}

int ref_pick(const double * weights, int n, double u) {
    return pick(std::vector<double>(weights, weights + n), u);
}

// The Error temperature_overflow() makes: its fault as an int, its message and the input it names.
int ref_temperature_overflow(float temperature, char * message, int message_cap, char * input, int input_cap) {
    const Error e = temperature_overflow(temperature);
    std::strncpy(message, e.what(), (size_t) message_cap - 1);
    message[message_cap - 1] = 0;
    std::strncpy(input, e.input().c_str(), (size_t) input_cap - 1);
    input[input_cap - 1] = 0;
    return (int) e.fault();
}

}  // extern "C"
