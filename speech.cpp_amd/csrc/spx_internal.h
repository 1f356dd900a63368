// spx_internal.h — what the host side of the sampler and its kernel share: the launch record, the workspace records
// and the fixed sizes of the one-pass path.
#pragma once

#include <stdint.h>

#include "../../include/spx_sampler.h"

namespace spx {

// Threads per work-group: 1024 for rows of at least kBigVocab tokens (one work-group per CU streams a whole row), 512
// for such rows in batches of at least two rows per CU (two work-groups per CU, one row's fixed phases under the other's
// stream), 256 below.
constexpr int kBlockBig = 1024;
constexpr int kBlockMid = 512;
constexpr int kBlockSmall = 256;
// Threads per work-group of the resolving kernel for large vocabularies (256 below): 1024 (16 waves a CU to hide the
// latency of each token's work; 128 VGPRs a lane), or 512 with the smaller wide-path layout where the 1024-thread
// one's LDS does not fit beside a long history list.
constexpr int kBlockResolve = 1024;
constexpr int kBlockResolveNarrow = 512;
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
// The wide path's LDS (rows whose draw runs past the candidates held): NB bins of the row's quotients and room for CAP
// gathered tokens, per work-group size. A bin holding more than CAP tokens takes a finer histogram and more reads, so
// the 1024-thread layout, with most of a CU's LDS, gathers twice as many.
template <int B>
struct WideDims;
template <>
struct WideDims<1024> {
    static constexpr int NB = 2048;
    static constexpr int CAP = 4096;
};
template <>
struct WideDims<512> {
    static constexpr int NB = 2048;
    static constexpr int CAP = 2048;
};
template <>
struct WideDims<256> {
    static constexpr int NB = 1024;
    static constexpr int CAP = 1024;
};
constexpr int kWideQs = 4;  // questions: the k-th token, the top-p cut, the pick, the last kept token
struct WideAns {            // written by the gathered token that answers a question
    uint64_t entry, before, through;
    uint32_t rank, found;
};
template <int NB, int CAP>
struct WideMem {
    uint32_t pre_cnt[NB + 2];   // tokens in the bins before b; [NB + 1]: every token
    uint64_t pre_mass[NB + 2];  // their fixed-point mass
    uint32_t seg[NB + 1];       // where the gathered tokens of bin b go (the read appends there)
    uint32_t need[(NB + 1 + 31) / 32];
    uint64_t ent[CAP];
    uint64_t mass[CAP];
    WideAns ans[kWideQs];
    uint64_t red[16];
    uint64_t lo_e;              // the lowest entry of the row (its last token in the order)
    uint32_t n_gath;
    int32_t wb[2];              // the first and last bin a gathering read needs
};
template <int B>
constexpr size_t wide_lds_bytes() {
    return sizeof(WideMem<WideDims<B>::NB, WideDims<B>::CAP>);
}

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

// A row the one-pass kernel leaves to the resolving kernel: its status flags and its largest final quotient (NaN where
// the one-pass kernel does not know it).
struct Pending {
    int32_t row;
    uint32_t flags;
    float top;
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
    double * out_cand_w;   // the candidates' weights (rows x max_out)
    int max_out;
    int block, splits, chunk, nwg;
    int cand_cap;  // entries of a chunk's candidate buffer
    int own_cap;   // entries of the history list: a power of two at least max_hist
    // LDS layout (byte offsets); the wide path's region overlays the candidate buffer and the sort area at off_cand
    int off_ctl, off_red, off_spec, off_own, off_cand, off_sort, lds_bytes;
    // workspace
    uint32_t * counters;   // [max_rows], each back to 0 after its row's last chunk
    Partial * partials;    // [max_rows * kMaxSplitsGreedy]
    uint64_t * part_cands; // [max_rows * kMaxSplits * kKeep]
    int32_t * fb_count;    // rows resolved past the one-pass path since the handle was made
    // Row addressing beyond the dense layout (the device chain and the two-draw entries): the logits row each sampled
    // row reads (null: its own), a strided history (row r's ids at hist[r * hist_stride + hist_first], hist_len of
    // them, where hist_off is null), and strides of the uniforms and of the ids written.
    const int32_t * row_map;
    int64_t hist_stride;
    int hist_first, hist_len;
    int64_t u_stride, out_stride;
    int list_all;          // every drawing row goes to the resolving kernel, which lists its candidates (max_out: any)
    Pending * pending;     // [max_rows]: the rows left to the resolving kernel
    uint32_t * pend_ctr;   // [4]: the count of rows left and of rows taken, one of each per call parity
    int parity;            // this call's slot of pend_ctr: calls alternate, so that no kernel has to clear its own
};

constexpr size_t round256(size_t x) { return (x + 255) / 256 * 256; }

// The workspace of `max_rows` rows, in the order it is laid out: the rows' arrival counters, the chunks' partials and
// published candidates, the resolved-row count with the resolving list's counts, the resolving list, and (`pairs`)
// the records of the two-draw and listing entries.
constexpr size_t kWsFb = 256;
constexpr size_t ws_counters(int max_rows) { return round256((size_t) max_rows * 4); }
constexpr size_t ws_partials(int max_rows) { return round256((size_t) max_rows * kMaxSplitsGreedy * sizeof(Partial)); }
constexpr size_t ws_cands(int max_rows) { return round256((size_t) max_rows * kMaxSplits * kKeep * 8); }
constexpr size_t ws_pending(int max_rows) { return round256((size_t) max_rows * sizeof(Pending)); }
constexpr size_t ws_pairs(int max_rows) {
    return round256((size_t) max_rows * (sizeof(spx_row_params) + 8 + 3 * 4 + 8) + 8) + 256;
}
constexpr size_t workspace_bytes(int max_rows, bool pairs) {
    return ws_counters(max_rows) + ws_partials(max_rows) + ws_cands(max_rows) + kWsFb + ws_pending(max_rows) +
           (pairs ? ws_pairs(max_rows) : 0);
}

// The no-alloc entry's rows per call, and the devices it keeps a handle for.
constexpr int kStaticRows = SPX_NOALLOC_MAX_ROWS;
constexpr int kMaxDevices = 64;

}  // namespace spx

#include <hip/hip_runtime.h>

namespace spx {
// The kernels' variants (spx_k_*.hip): logits of fp32 or bf16, work-groups of 1024, 512 or 256 threads. Each
// variant has the one-pass sampling kernel (launch_*) and, but for the 512-thread ones, the kernel that resolves the
// rows it leaves (resolve_*); lds_limit_* lets them take `bytes` of dynamic LDS.
hipError_t launch_f32_1024(const Launch & a, hipStream_t s);
hipError_t launch_bf16_1024(const Launch & a, hipStream_t s);
hipError_t launch_f32_512(const Launch & a, hipStream_t s);
hipError_t launch_bf16_512(const Launch & a, hipStream_t s);
hipError_t launch_f32_256(const Launch & a, hipStream_t s);
hipError_t launch_bf16_256(const Launch & a, hipStream_t s);
hipError_t resolve_f32_1024(const Launch & a, int grid, hipStream_t s);
hipError_t resolve_bf16_1024(const Launch & a, int grid, hipStream_t s);
hipError_t resolve_f32_256(const Launch & a, int grid, hipStream_t s);
hipError_t resolve_bf16_256(const Launch & a, int grid, hipStream_t s);
// The kernels of spx_aux.hip.
hipError_t launch_talker_bans(uint32_t * words, int vocab, int suppressed, int32_t eos, int frames, int min_frames,
                              hipStream_t s);
hipError_t launch_pair_prep(int rows, const spx_row_params * first, const spx_row_params * again, const double * u_first,
                            const double * u_again, spx_row_params * params, double * u, int32_t * row_map,
                            hipStream_t s);
hipError_t launch_pair_pick(int rows, const int32_t * ids, const int32_t * status, const int32_t * token_ids,
                            int32_t sem_lo, int32_t sem_hi, int window, const int32_t * hist, const int32_t * hist_off,
                            int32_t * out_ids, int32_t * out_status, hipStream_t s);
// Haru's DRY: the penalty of a match `length - allowed_length` = e past the allowed length is table[e] for
// e < n_table and `sat` beyond (the table holds every e up to max_match_length - allowed_length, or ends where it has
// reached max_penalty with base >= 1, after which every penalty is max_penalty). The host computes the table with its
// std::pow, the function Dry::update calls, so the device's penalties are the reference's bit for bit.
constexpr int kDryTable = 128;
struct DryArgs {
    float * logits;
    int64_t ld;
    int rows, vocab;
    const int32_t * hist;
    const int32_t * len;
    int hist_stride, allowed, lookback, max_match, size, n_table, n_exempt;
    int32_t exempt[SPX_DRY_MAX_EXEMPT];
    const int32_t * tokens;  // the update's drawn tokens
    int32_t * hist_w;        // the update's histories and lengths
    int32_t * len_w;
    const float * silent;
    int32_t pad, eop, eos;
    float eop_bias;
    const uint8_t * must_speak;
    int32_t * out_pen_tokens;
    double * out_pen;
    int32_t * out_npen;
    int pen_cap;
    double sat;
    double table[kDryTable];
};

// The fused head pick (spx_head.hip): its operands, and the normalized hidden states and the pick keys in the
// handle's workspace.
constexpr int kHeadMaxRows = 64;
struct HeadArgs {
    const float * hidden;
    int64_t hidden_ld;
    const float * norm_w;
    float eps;
    const uint16_t * head;
    int64_t head_ld;
    int rows, d, vocab;
    uint16_t * hn;
    uint64_t * keys;
    int32_t * out_ids;
    float * out_max;
};

// spx_api.cpp's pieces of the no-alloc entry (spx_noalloc.hip): its error messages, a handle of static storage over
// a workspace the caller owns, and the per-call limits of such a handle.
spx_status report(spx_status s, const char * msg);  // sets spx_last_error()'s message
spx_status report_hip(hipError_t e, const char * what);
spx_status bind_scratch(int device, void * ws, int max_rows, spx_sampler ** out);
void set_call_limits(spx_sampler * s, int vocab, int max_hist, int max_out);
spx_status dry_args(DryArgs & d, const spx_dry_config * c, const int32_t * exempt, int n_exempt, int hist_stride);
hipError_t launch_dry_update(const DryArgs & d, hipStream_t s);
hipError_t launch_head_pick(const HeadArgs & h, hipStream_t s);
hipError_t launch_haru_shape(const DryArgs & d, hipStream_t s);
hipError_t lds_limit_f32_1024(int bytes);
hipError_t lds_limit_bf16_1024(int bytes);
hipError_t lds_limit_f32_512(int bytes);
hipError_t lds_limit_bf16_512(int bytes);
hipError_t lds_limit_f32_256(int bytes);
hipError_t lds_limit_bf16_256(int bytes);
}  // namespace spx
