// spx_internal.h — what the host side of the sampler and its kernels share: the launch record, the workspace records
// and the fixed sizes of the one-pass path.
#pragma once

#include <stdint.h>

#include "../../include/spx_sampler.h"

namespace spx {

// Threads per work-group.
constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;
// Entries a wave keeps: the top-k of a row with top_k <= kKeep, and the top kKeep of a row drawing over more
// (its top-p set must end within them, or the row takes the multi-pass path).
constexpr int kKeep = 256;
// Entries a wave keeps for a row drawing over more than kKeep tokens.
constexpr int kKeepFull = 128;
// A wave's buffer: its kKeep best plus one offer of 64 lanes x 4 elements before it must compact.
constexpr int kCap = 512;
constexpr int kPerLane = kCap / 64;
// Entries the last chunk of a row can merge: kKeep from each of at most kMaxSplits chunks.
constexpr int kMaxSplits = 4;
constexpr int kMaxSplitsGreedy = 16;
constexpr int kSortCap = 1024;  // >= kWaves * kKeep and >= kMaxSplits * kKeep, a power of two

// What a chunk of a row leaves for the last chunk of its row.
struct Partial {
    uint64_t best;     // greedy: the largest entry of the final logits (0: none)
    uint64_t low;      // the last token of the order
    double s;          // sum of exp(q - m)
    float m;
    float mx, mn;      // range of the final logits
    uint32_t flags;
    int32_t n;         // sorted entries published
    int32_t complete;  // 1 when the chunk's every valid token is among them
    uint64_t kth;      // its K-th entry (0 when it holds fewer than K)
};

struct Launch {
    const void * logits;
    int64_t ld;
    int rows, vocab, dtype, vec_ok;
    const int32_t * hist;
    const int32_t * hist_off;
    int max_hist;
    int slot_cap;
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
    int splits, chunk, nwg;
    int sort_cap;
    // LDS layout (byte offsets). The multi-pass path keeps its radix histograms in the sort region.
    int off_bits, off_rank, off_slots, off_cand, off_sort, off_red, lds_bytes;
    // workspace
    uint32_t * counters;   // [max_rows], each back to 0 after its row's last chunk
    Partial * partials;    // [max_rows * kMaxSplitsGreedy]
    uint64_t * part_cands; // [max_rows * kMaxSplits * kKeep]
    int32_t * fb_count;    // rows the multi-pass path has resolved since the handle was made
};

}  // namespace spx

#include <hip/hip_runtime.h>

namespace spx {
hipError_t launch_stream(const Launch & a, hipStream_t s);
hipError_t set_lds_limits(int stream_bytes);
}  // namespace spx
