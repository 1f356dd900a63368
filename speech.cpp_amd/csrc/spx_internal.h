// spx_internal.h — what the host side of the sampler and its kernel share: the launch record, the workspace records
// and the fixed sizes of the one-pass path.
#pragma once

#include <stdint.h>

#include "../../include/spx_sampler.h"

namespace spx {

// Threads per work-group: 1024 for rows of at least kBigVocab tokens (one work-group per CU streams a whole row),
// 256 below.
constexpr int kBlockBig = 1024;
constexpr int kBlockSmall = 256;
constexpr int kBigVocab = 16384;
// Final logits each lane holds per step of the stream (four 16-byte vectors of fp32, two of bf16).
constexpr int kE = 16;
// The top-k of a row with top_k <= kKeep is held exactly; a row drawing over more tokens holds at least its top
// kKeepFull (its top-p set must end within what is held, or the row takes the multi-pass path).
constexpr int kKeep = 256;
constexpr int kKeepFull = 128;
// Entries one chunk's sorted candidates can hold, and the merge of kMaxSplits chunks of kKeep each.
constexpr int kSortCap = 1024;
constexpr int kMaxSplits = 4;
constexpr int kMaxSplitsGreedy = 16;
// LDS bytes of a chunk's control block (its counters, bins and first-step bounds).
constexpr int kCtlBytes = 2048;
// The largest history a handle takes: slot ranks are kept in 24 bits and the LDS must hold the slots.
constexpr int kMaxHist = 4096;

// What a chunk of a row leaves for the last chunk of its row.
struct Partial {
    uint64_t best;     // greedy: the largest entry of the final logits (0: none above -inf)
    uint64_t floor;    // every entry of the chunk at or above it is among those published
    double s;          // sum of exp(q - m) over the chunk
    float m;
    uint32_t flags;
    int32_t n;         // sorted entries published
    int32_t complete;  // 1 when they are every valid token of the chunk
    int32_t broken;    // 1 when the chunk could not keep its candidates (the row takes the multi-pass path)
    int32_t pad;
};

struct Launch {
    const void * logits;
    int64_t ld;
    int rows, vocab, dtype, vec_ok;
    const int32_t * hist;
    const int32_t * hist_off;
    int max_hist;
    const uint32_t * banned;
    int64_t banned_stride;
    const spx_row_params * params;
    const double * u;
    int32_t * out_ids;
    int32_t * out_status;
    int32_t * out_kept;
    int32_t * out_cand_ids;
    float * out_cand_probs;
    int max_out;
    int block, splits, chunk, nwg;
    int cand_cap;  // entries of a chunk's candidate buffer
    int tab_mask;  // entries of the frequency-count table - 1 (a power of two - 1)
    // LDS layout (byte offsets)
    int off_ctl, off_red, off_spec, off_own, off_tab, off_cand, off_sort, lds_bytes;
    // workspace
    uint32_t * counters;   // [max_rows], each back to 0 after its row's last chunk
    Partial * partials;    // [max_rows * kMaxSplitsGreedy]
    uint64_t * part_cands; // [max_rows * kMaxSplits * kKeep]
    int32_t * fb_count;    // rows the multi-pass path has resolved since the handle was made
};

}  // namespace spx

#include <hip/hip_runtime.h>

namespace spx {
hipError_t launch_sampler(const Launch & a, hipStream_t s);
hipError_t set_lds_limits(int bytes);
}  // namespace spx
