// spx_api.cpp — the C ABI of the sampler (include/spx_sampler.h): the handle and its workspace, the checks of each
// call, the launch shape, and the kernels' LDS layout.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/spx_sampler.h"
#include "spx_internal.h"
#include "spx_plan.h"

struct spx_sampler {
    int device = 0;
    int max_rows = 0, max_vocab = 0, max_hist = 0, max_out = 0;
    int cus = 256;
    void * ws = nullptr;
    spx::Launch base{};
    int last_block = 0, last_splits = 0;
    int parity = 0;  // the slot of the resolving list's count this call uses
    // the two-draw entry's records: max_rows each (a call draws 2 rows per row)
    spx_row_params * pair_params = nullptr;
    double * pair_u = nullptr;
    int32_t * pair_map = nullptr;
    int32_t * pair_ids = nullptr;
    int32_t * pair_status = nullptr;
    double * zero_u = nullptr;  // max_rows zeros: the numbers of a listing call, which draws nothing
};

namespace {

thread_local std::string g_error;

spx_status fail(spx_status s, const std::string & msg) {
    g_error = msg;
    return s;
}

spx_status hip_fail(hipError_t e, const char * what) {
    return fail(SPX_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

void plan_launch(spx_sampler * s, spx::Launch & a, bool greedy_only, bool has_hist, bool has_ban) {
    spx::plan_rows(a, s->cus, s->max_hist, greedy_only, has_hist, has_ban);
    s->last_block = a.block;
    s->last_splits = a.splits;
}

spx_status check_common(spx_sampler * s, const void * logits, int dtype, int rows, int vocab, int64_t ld,
                        const uint32_t * banned, int64_t banned_stride, const int32_t * out_ids) {
    if (!s) return fail(SPX_ERR_INVALID_ARGUMENT, "null sampler handle");
    if (rows < 0 || rows > s->max_rows) return fail(SPX_ERR_INVALID_ARGUMENT, "rows outside [0, max_rows]");
    if (vocab <= 0 || vocab > s->max_vocab) return fail(SPX_ERR_INVALID_ARGUMENT, "vocab outside [1, max_vocab]");
    if (ld < vocab) return fail(SPX_ERR_INVALID_ARGUMENT, "ld is smaller than vocab");
    if (dtype != SPX_F32 && dtype != SPX_BF16) return fail(SPX_ERR_INVALID_ARGUMENT, "dtype is neither SPX_F32 nor SPX_BF16");
    if (rows > 0 && (!logits || !out_ids)) return fail(SPX_ERR_INVALID_ARGUMENT, "null logits or out_ids");
    if (banned && banned_stride < 0) return fail(SPX_ERR_INVALID_ARGUMENT, "negative banned_stride");
    if (banned && banned_stride != 0 && banned_stride < (vocab + 31) / 32)
        return fail(SPX_ERR_INVALID_ARGUMENT, "banned_stride shorter than a mask of vocab bits");
    return SPX_OK;
}

// The variant of the kernel for the call's logit type and work-group size.
hipError_t launch_sampler(const spx::Launch & a, hipStream_t s) {
    using namespace spx;
    if (a.nwg == 0) return hipSuccess;
    if (a.block == kBlockBig) return a.dtype == SPX_BF16 ? launch_bf16_1024(a, s) : launch_f32_1024(a, s);
    if (a.block == kBlockMid) return a.dtype == SPX_BF16 ? launch_bf16_512(a, s) : launch_f32_512(a, s);
    return a.dtype == SPX_BF16 ? launch_bf16_256(a, s) : launch_f32_256(a, s);
}

// The resolving kernel after a sampling launch: `grid` work-groups take the rows the sampling kernel left, if any.
hipError_t launch_resolver(const spx::Launch & r, int grid, hipStream_t s) {
    using namespace spx;
    if (r.block != kBlockSmall) return r.dtype == SPX_BF16 ? resolve_bf16_1024(r, grid, s) : resolve_f32_1024(r, grid, s);
    return r.dtype == SPX_BF16 ? resolve_bf16_256(r, grid, s) : resolve_f32_256(r, grid, s);
}

// Lets every variant take `bytes` of dynamic LDS (above the 64 KiB a launch gets without asking).
hipError_t set_lds_limits(int bytes) {
    using namespace spx;
    if (bytes <= 65536) return hipSuccess;
    for (auto f : {lds_limit_f32_1024, lds_limit_bf16_1024, lds_limit_f32_512, lds_limit_bf16_512, lds_limit_f32_256,
                   lds_limit_bf16_256}) {
        const hipError_t e = f(bytes);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// A sampling launch and the resolving launch after it, on the stream (the call parity alternates the list's count).
spx_status run_sampling(spx_sampler * s, spx::Launch & a, void * stream) {
    a.parity = s->parity;
    s->parity ^= 1;
    hipError_t e = launch_sampler(a, (hipStream_t) stream);
    if (e != hipSuccess) return hip_fail(e, "sampler_kernel launch");
    // the rows the sampling kernel left, resolved by a work-group each (a launch that finds none ends at once)
    spx::Launch r;
    plan_resolve(r, a, s->max_hist);
    e = launch_resolver(r, std::min(a.rows, s->cus), (hipStream_t) stream);
    if (e != hipSuccess) return hip_fail(e, "resolve_kernel launch");
    return SPX_OK;
}

// The common part of a sampling call's launch record.
void fill_launch(spx::Launch & a, const void * logits, int dtype, int rows, int vocab, int64_t ld) {
    a.logits = logits;
    a.ld = ld;
    a.rows = rows;
    a.vocab = vocab;
    a.dtype = dtype;
    const size_t esz = dtype == SPX_BF16 ? 2 : 4;
    a.vec_ok = ((uintptr_t) logits % 16 == 0) && (((size_t) ld * esz) % 16 == 0);
}

// The handle's workspace pointers over `ws` (workspace_bytes(max_rows, pairs) bytes), and its fixed launch fields.
void carve_workspace(spx_sampler * s, void * ws, int max_rows, bool pairs) {
    using namespace spx;
    char * p = (char *) ws;
    s->base.counters = (uint32_t *) p;
    p += ws_counters(max_rows);
    s->base.partials = (Partial *) p;
    p += ws_partials(max_rows);
    s->base.part_cands = (uint64_t *) p;
    p += ws_cands(max_rows);
    s->base.fb_count = (int32_t *) p;
    s->base.pend_ctr = (uint32_t *) (p + 64);
    p += kWsFb;
    s->base.pending = (Pending *) p;
    p += ws_pending(max_rows);
    if (pairs) {
        s->pair_params = (spx_row_params *) p;
        p += (size_t) max_rows * sizeof(spx_row_params);
        s->pair_u = (double *) p;
        p += (size_t) max_rows * 8;
        s->pair_map = (int32_t *) p;
        s->pair_ids = s->pair_map + max_rows;
        s->pair_status = s->pair_ids + max_rows;
        s->zero_u = (double *) spx::align_up((size_t) (s->pair_status + max_rows), 8);
    }
    s->base.row_map = nullptr;
    s->base.hist_stride = 0;
    s->base.hist_first = s->base.hist_len = 0;
    s->base.u_stride = 1;
    s->base.out_stride = 1;
    s->base.list_all = 0;
    s->base.max_hist = s->max_hist;
}

}  // namespace

namespace spx {

spx_status report(spx_status s, const char * msg) { return fail(s, msg); }
spx_status report_hip(hipError_t e, const char * what) { return hip_fail(e, what); }

// Handles over the no-alloc entry's workspace: host records of static storage, one per device.
spx_sampler g_bound[kMaxDevices];

spx_status bind_scratch(int device, void * ws, int max_rows, spx_sampler ** out) {
    if (device < 0 || device >= kMaxDevices) return fail(SPX_ERR_INVALID_ARGUMENT, "device index above the no-alloc entry's table");
    spx_sampler * s = &g_bound[device];
    s->device = device;
    s->max_rows = max_rows;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0) s->cus = cus;
    const hipError_t e = set_lds_limits((int) spx::kLdsMax);
    if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute");
    carve_workspace(s, ws, max_rows, false);
    s->ws = nullptr;  // not the handle's to free
    *out = s;
    return SPX_OK;
}

void set_call_limits(spx_sampler * s, int vocab, int max_hist, int max_out) {
    s->max_vocab = vocab;
    s->max_hist = max_hist;
    s->max_out = max_out;
    s->base.max_hist = max_hist;
}

// The DRY settings a call runs with: checked, and the penalty of every match length computed on the host (std::pow,
// as Dry::update computes it).
spx_status dry_args(DryArgs & d, const spx_dry_config * c, const int32_t * exempt, int n_exempt, int hist_stride) {
    if (!c) return fail(SPX_ERR_INVALID_ARGUMENT, "null DRY config");
    if (n_exempt < 0 || n_exempt > SPX_DRY_MAX_EXEMPT || (n_exempt > 0 && !exempt))
        return fail(SPX_ERR_INVALID_ARGUMENT, "exempt ids: null, or more than SPX_DRY_MAX_EXEMPT");
    if (c->lookback < 0 || c->max_match_length < 0) return fail(SPX_ERR_INVALID_ARGUMENT, "negative lookback or max_match_length");
    const int64_t size = (int64_t) c->lookback + c->max_match_length + 1;
    if (size > hist_stride || hist_stride > SPX_DRY_MAX_HISTORY)
        return fail(SPX_ERR_INVALID_ARGUMENT, "hist_stride below lookback + max_match_length + 1, or above SPX_DRY_MAX_HISTORY");
    d = DryArgs{};
    d.hist_stride = hist_stride;
    d.allowed = c->allowed_length;
    d.lookback = c->lookback;
    d.max_match = c->max_match_length;
    d.size = (int) size;
    d.n_exempt = n_exempt;
    for (int i = 0; i < n_exempt; i++) d.exempt[i] = exempt[i];
    // a match is 1 .. max(1, max_match_length) long; its penalty's exponent e = length - allowed_length
    const int64_t emax = (int64_t) std::max(1, c->max_match_length) - c->allowed_length;
    const int n = (int) std::max<int64_t>(0, std::min<int64_t>(emax + 1, kDryTable));
    for (int e = 0; e < n; e++) d.table[e] = std::min(c->max_penalty, c->multiplier * std::pow(c->base, (double) e));
    d.n_table = n;
    d.sat = c->max_penalty;
    if (emax >= kDryTable) {
        // every longer match takes max_penalty only where the penalties rise with the length and have reached it
        const bool rising = c->base >= 1.0 && c->multiplier >= 0.0;
        if (!rising || d.table[kDryTable - 1] != c->max_penalty)
            return fail(SPX_ERR_INVALID_ARGUMENT, "DRY penalties that do not reach max_penalty within 128 lengths");
    }
    return SPX_OK;
}

}  // namespace spx

extern "C" {

const char * spx_last_error(void) { return g_error.c_str(); }

spx_status spx_sampler_create(spx_sampler ** out, int max_rows, int max_vocab, int max_hist, int max_out) {
    using namespace spx;
    if (!out) return fail(SPX_ERR_INVALID_ARGUMENT, "null output pointer");
    *out = nullptr;
    if (max_rows <= 0 || max_vocab <= 0 || max_hist < 0 || max_out < 0)
        return fail(SPX_ERR_INVALID_ARGUMENT, "sizes must be positive");
    if (max_out > kKeep) return fail(SPX_ERR_INVALID_ARGUMENT, "max_out above 256");
    auto * s = new spx_sampler();
    s->max_rows = max_rows;
    s->max_vocab = max_vocab;
    s->max_hist = max_hist;
    s->max_out = max_out;
    hipError_t e = hipGetDevice(&s->device);
    if (e != hipSuccess) {
        delete s;
        return hip_fail(e, "hipGetDevice");
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, s->device) == hipSuccess && cus > 0)
        s->cus = cus;
    const size_t lds_max = spx::lds_bound(max_vocab, max_hist);
    if (lds_max > spx::kLdsMax) {
        delete s;
        return fail(SPX_ERR_INVALID_ARGUMENT, "max_vocab and max_hist need more LDS than a CU holds");
    }
    e = set_lds_limits((int) lds_max);
    if (e != hipSuccess) {
        delete s;
        return hip_fail(e, "hipFuncSetAttribute");
    }
    // One allocation for the workspace.
    const size_t bytes = workspace_bytes(max_rows, true);
    e = hipMalloc(&s->ws, bytes);
    if (e != hipSuccess) {
        delete s;
        return e == hipErrorOutOfMemory ? fail(SPX_ERR_OUT_OF_MEMORY, "workspace allocation") : hip_fail(e, "hipMalloc");
    }
    e = hipMemset(s->ws, 0, bytes);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void) hipFree(s->ws);
        delete s;
        return hip_fail(e, "hipMemset");
    }
    carve_workspace(s, s->ws, max_rows, true);
    *out = s;
    return SPX_OK;
}

void spx_sampler_destroy(spx_sampler * s) {
    if (!s) return;
    if (s->ws) (void) hipFree(s->ws);
    delete s;
}

spx_status spx_sample_rows(spx_sampler * s, const void * d_logits, int dtype, int rows, int vocab, int64_t ld,
                           const int32_t * d_hist, const int32_t * d_hist_off, const uint32_t * d_banned,
                           int64_t banned_stride, const spx_row_params * d_params, const double * d_u,
                           int32_t * d_out_ids, int32_t * d_out_status, int32_t * d_out_kept,
                           int32_t * d_out_cand_ids, double * d_out_cand_weights, void * stream) {
    spx_status st = check_common(s, d_logits, dtype, rows, vocab, ld, d_banned, banned_stride, d_out_ids);
    if (st != SPX_OK) return st;
    if (rows > 0 && (!d_params || !d_u)) return fail(SPX_ERR_INVALID_ARGUMENT, "null params or u");
    if ((d_hist == nullptr) != (d_hist_off == nullptr)) return fail(SPX_ERR_INVALID_ARGUMENT, "hist and hist_off go together");
    if ((d_out_cand_ids == nullptr) != (d_out_cand_weights == nullptr))
        return fail(SPX_ERR_INVALID_ARGUMENT, "cand_ids and cand_weights go together");
    if (d_out_cand_ids && s->max_out <= 0) return fail(SPX_ERR_INVALID_ARGUMENT, "the handle was created with max_out 0");
    if (rows == 0) return SPX_OK;
    spx::Launch a = s->base;
    fill_launch(a, d_logits, dtype, rows, vocab, ld);
    a.hist = d_hist;
    a.hist_off = d_hist_off;
    a.banned = d_banned;
    a.banned_stride = banned_stride;
    a.params = d_params;
    a.u = d_u;
    a.out_ids = d_out_ids;
    a.out_status = d_out_status;
    a.out_kept = d_out_kept;
    a.out_cand_ids = d_out_cand_ids;
    a.out_cand_w = d_out_cand_weights;
    a.max_out = d_out_cand_ids ? s->max_out : 0;
    plan_launch(s, a, false, d_hist != nullptr, d_banned != nullptr);
    return run_sampling(s, a, stream);
}

spx_status spx_argmax_rows(spx_sampler * s, const void * d_logits, int dtype, int rows, int vocab, int64_t ld,
                           const uint32_t * d_banned, int64_t banned_stride, int32_t * d_out_ids, void * stream) {
    spx_status st = check_common(s, d_logits, dtype, rows, vocab, ld, d_banned, banned_stride, d_out_ids);
    if (st != SPX_OK) return st;
    if (rows == 0) return SPX_OK;
    spx::Launch a = s->base;
    fill_launch(a, d_logits, dtype, rows, vocab, ld);
    a.hist = nullptr;
    a.hist_off = nullptr;
    a.banned = d_banned;
    a.banned_stride = banned_stride;
    a.params = nullptr;
    a.u = nullptr;
    a.out_ids = d_out_ids;
    a.out_status = nullptr;
    a.out_kept = nullptr;
    a.out_cand_ids = nullptr;
    a.out_cand_w = nullptr;
    a.max_out = 0;
    plan_launch(s, a, true, false, d_banned != nullptr);
    hipError_t e = launch_sampler(a, (hipStream_t) stream);
    if (e != hipSuccess) return hip_fail(e, "sampler_kernel launch");
    return SPX_OK;
}

spx_status spx_candidates_rows(spx_sampler * s, const void * d_logits, int dtype, int rows, int vocab, int64_t ld,
                               const int32_t * d_hist, const int32_t * d_hist_off, const uint32_t * d_banned,
                               int64_t banned_stride, const spx_row_params * d_params, int cap, int32_t * d_out_tokens,
                               double * d_out_weights, int32_t * d_out_n, int32_t * d_out_status, void * stream) {
    spx_status st = check_common(s, d_logits, dtype, rows, vocab, ld, d_banned, banned_stride, d_out_n);
    if (st != SPX_OK) return st;
    if (rows > 0 && (!d_params || !d_out_tokens || !d_out_weights))
        return fail(SPX_ERR_INVALID_ARGUMENT, "null params or candidate outputs");
    if ((d_hist == nullptr) != (d_hist_off == nullptr)) return fail(SPX_ERR_INVALID_ARGUMENT, "hist and hist_off go together");
    if (cap <= 0) return fail(SPX_ERR_INVALID_ARGUMENT, "cap must be positive");
    if (rows == 0) return SPX_OK;
    // the ids of the draws (with u = 0, unread) go to the pair area's id slots, which this call does not otherwise use
    spx::Launch a = s->base;
    fill_launch(a, d_logits, dtype, rows, vocab, ld);
    a.hist = d_hist;
    a.hist_off = d_hist_off;
    a.banned = d_banned;
    a.banned_stride = banned_stride;
    a.params = d_params;
    a.u = s->zero_u;
    a.out_ids = s->pair_ids;
    a.out_status = d_out_status;
    a.out_kept = d_out_n;
    a.out_cand_ids = d_out_tokens;
    a.out_cand_w = d_out_weights;
    a.max_out = cap;
    a.list_all = 1;
    plan_launch(s, a, false, d_hist != nullptr, d_banned != nullptr);
    return run_sampling(s, a, stream);
}

spx_status spx_talker_bans(uint32_t * d_words, int vocab, int suppressed_tokens, int32_t end_of_speech, int frames,
                           int min_frames, void * stream) {
    if (!d_words || vocab <= 0) return fail(SPX_ERR_INVALID_ARGUMENT, "null mask or empty vocabulary");
    if (suppressed_tokens < 0 || suppressed_tokens > vocab) return fail(SPX_ERR_INVALID_ARGUMENT, "suppressed_tokens outside [0, vocab]");
    if (end_of_speech < 0 || end_of_speech >= vocab) return fail(SPX_ERR_INVALID_ARGUMENT, "end_of_speech outside the vocabulary");
    const hipError_t e = spx::launch_talker_bans(d_words, vocab, suppressed_tokens, end_of_speech, frames, min_frames,
                                                 (hipStream_t) stream);
    return e == hipSuccess ? SPX_OK : hip_fail(e, "talker_bans launch");
}

spx_status spx_sample_chain(spx_sampler * s, const void * d_logits, int dtype, int rows, int vocab, int64_t ld,
                            int32_t * d_codes, int codes_stride, int step, int picks, const spx_row_params * d_params,
                            const double * d_u, int32_t * d_out_status, void * stream) {
    spx_status st = check_common(s, d_logits, dtype, rows, vocab, ld, nullptr, 0, d_codes);
    if (st != SPX_OK) return st;
    if (rows > 0 && (!d_params || !d_u)) return fail(SPX_ERR_INVALID_ARGUMENT, "null params or u");
    if (step < 0 || step >= picks || codes_stride < picks + 1)
        return fail(SPX_ERR_INVALID_ARGUMENT, "step outside [0, picks) or codes_stride below picks + 1");
    if (step > s->max_hist) return fail(SPX_ERR_INVALID_ARGUMENT, "the handle's max_hist is below the chain's picks");
    if (rows == 0) return SPX_OK;
    spx::Launch a = s->base;
    fill_launch(a, d_logits, dtype, rows, vocab, ld);
    // pick `step` reads codes 1..step of its stream as the history and writes code step + 1
    a.hist = d_codes;
    a.hist_off = nullptr;
    a.hist_stride = codes_stride;
    a.hist_first = 1;
    a.hist_len = step;
    a.banned = nullptr;
    a.banned_stride = 0;
    a.params = d_params;
    a.u = d_u + step;
    a.u_stride = picks;
    a.out_ids = d_codes + step + 1;
    a.out_stride = codes_stride;
    a.out_status = d_out_status;
    a.out_kept = nullptr;
    a.out_cand_ids = nullptr;
    a.out_cand_w = nullptr;
    a.max_out = 0;
    plan_launch(s, a, false, true, false);
    return run_sampling(s, a, stream);
}

spx_status spx_drama3_main(spx_sampler * s, const void * d_logits, int dtype, int rows, int vocab, int64_t ld,
                           const spx_row_params * d_first, const spx_row_params * d_again, const double * d_u_first,
                           const double * d_u_again, const int32_t * d_token_ids, int32_t semantic_begin,
                           int32_t semantic_end, int window, const int32_t * d_hist, const int32_t * d_hist_off,
                           int32_t * d_out_ids, int32_t * d_out_status, void * stream) {
    spx_status st = check_common(s, d_logits, dtype, 2 * rows, vocab, ld, nullptr, 0, d_out_ids);
    if (st != SPX_OK) return st;
    if (rows > 0 && (!d_first || !d_again || !d_u_first || !d_u_again || !d_token_ids))
        return fail(SPX_ERR_INVALID_ARGUMENT, "null params, u or token ids");
    if ((d_hist == nullptr) != (d_hist_off == nullptr)) return fail(SPX_ERR_INVALID_ARGUMENT, "hist and hist_off go together");
    if (rows == 0) return SPX_OK;
    hipError_t e = spx::launch_pair_prep(rows, d_first, d_again, d_u_first, d_u_again, s->pair_params, s->pair_u,
                                         s->pair_map, (hipStream_t) stream);
    if (e != hipSuccess) return hip_fail(e, "pair_prep launch");
    spx::Launch a = s->base;
    fill_launch(a, d_logits, dtype, 2 * rows, vocab, ld);
    a.row_map = s->pair_map;
    a.hist = nullptr;
    a.hist_off = nullptr;
    a.banned = nullptr;
    a.banned_stride = 0;
    a.params = s->pair_params;
    a.u = s->pair_u;
    a.out_ids = s->pair_ids;
    a.out_status = s->pair_status;
    a.out_kept = nullptr;
    a.out_cand_ids = nullptr;
    a.out_cand_w = nullptr;
    a.max_out = 0;
    plan_launch(s, a, false, false, false);
    st = run_sampling(s, a, stream);
    if (st != SPX_OK) return st;
    e = spx::launch_pair_pick(rows, s->pair_ids, s->pair_status, d_token_ids, semantic_begin, semantic_end, window,
                              d_hist, d_hist_off, d_out_ids, d_out_status, (hipStream_t) stream);
    return e == hipSuccess ? SPX_OK : hip_fail(e, "pair_pick launch");
}

spx_status spx_dry_update_rows(int rows, const spx_dry_config * config, const int32_t * exempt, int n_exempt,
                               const int32_t * d_tokens, int32_t * d_hist, int32_t * d_len, int hist_stride,
                               void * stream) {
    spx::DryArgs d;
    const spx_status st = spx::dry_args(d, config, exempt, n_exempt, hist_stride);
    if (st != SPX_OK) return st;
    if (rows < 0) return fail(SPX_ERR_INVALID_ARGUMENT, "negative rows");
    if (rows > 0 && (!d_tokens || !d_hist || !d_len)) return fail(SPX_ERR_INVALID_ARGUMENT, "null tokens, hist or len");
    d.rows = rows;
    d.tokens = d_tokens;
    d.hist_w = d_hist;
    d.len_w = d_len;
    const hipError_t e = spx::launch_dry_update(d, (hipStream_t) stream);
    return e == hipSuccess ? SPX_OK : hip_fail(e, "dry_update launch");
}

spx_status spx_haru_shape_rows(float * d_logits, int rows, int vocab, int64_t ld, const spx_dry_config * config,
                               const int32_t * exempt, int n_exempt, const int32_t * d_hist, const int32_t * d_len,
                               int hist_stride, const float * d_silent, int32_t pad, int32_t eop, int32_t eos,
                               float eop_bias, const uint8_t * d_must_speak, int32_t * d_out_pen_tokens,
                               double * d_out_pen, int32_t * d_out_npen, int pen_cap, void * stream) {
    spx::DryArgs d;
    const spx_status st = spx::dry_args(d, config, exempt, n_exempt, hist_stride);
    if (st != SPX_OK) return st;
    if (rows < 0 || vocab <= 0 || ld < vocab) return fail(SPX_ERR_INVALID_ARGUMENT, "rows, vocab or ld out of range");
    if (rows > 0 && (!d_logits || !d_hist || !d_len || !d_silent))
        return fail(SPX_ERR_INVALID_ARGUMENT, "null logits, hist, len or silent logits");
    if (pad < 0 || pad >= vocab || eop < 0 || eop >= vocab || eos < 0 || eos >= vocab)
        return fail(SPX_ERR_INVALID_ARGUMENT, "pad, eop or eos outside the vocabulary");
    if ((d_out_pen_tokens == nullptr) != (d_out_pen == nullptr) || (d_out_pen_tokens && pen_cap <= 0))
        return fail(SPX_ERR_INVALID_ARGUMENT, "penalty outputs: tokens and penalties go together, with pen_cap > 0");
    d.logits = d_logits;
    d.ld = ld;
    d.rows = rows;
    d.vocab = vocab;
    d.hist = d_hist;
    d.len = d_len;
    d.silent = d_silent;
    d.pad = pad;
    d.eop = eop;
    d.eos = eos;
    d.eop_bias = eop_bias;
    d.must_speak = d_must_speak;
    d.out_pen_tokens = d_out_pen_tokens;
    d.out_pen = d_out_pen;
    d.out_npen = d_out_npen;
    d.pen_cap = pen_cap;
    const hipError_t e = spx::launch_haru_shape(d, (hipStream_t) stream);
    return e == hipSuccess ? SPX_OK : hip_fail(e, "haru_shape launch");
}

spx_status spx_head_argmax_rows(spx_sampler * s, const float * d_hidden, int64_t hidden_ld, const float * d_norm_weight,
                                float eps, const uint16_t * d_head, int64_t head_ld, int rows, int d, int vocab,
                                int32_t * d_out_ids, float * d_out_max, void * stream) {
    using namespace spx;
    if (!s) return fail(SPX_ERR_INVALID_ARGUMENT, "null sampler handle");
    if (rows < 0 || rows > kHeadMaxRows || rows > s->max_rows) return fail(SPX_ERR_INVALID_ARGUMENT, "rows outside [0, min(64, max_rows)]");
    if (d <= 0 || d % 64 != 0 || vocab <= 0) return fail(SPX_ERR_INVALID_ARGUMENT, "d must be a positive multiple of 64, vocab positive");
    if (hidden_ld < d || head_ld < d || head_ld % 8 != 0) return fail(SPX_ERR_INVALID_ARGUMENT, "hidden_ld or head_ld below d, or head_ld not a multiple of 8");
    if ((size_t) rows * (size_t) d * 2 > ws_cands(s->max_rows))
        return fail(SPX_ERR_INVALID_ARGUMENT, "rows x d bf16 exceed the handle's workspace");
    if (rows == 0) return SPX_OK;
    if (!d_hidden || !d_head || !d_out_ids) return fail(SPX_ERR_INVALID_ARGUMENT, "null hidden, head or out_ids");
    if ((uintptr_t) d_head % 16 != 0) return fail(SPX_ERR_INVALID_ARGUMENT, "head not 16-byte aligned");
    HeadArgs h{};
    h.hidden = d_hidden;
    h.hidden_ld = hidden_ld;
    h.norm_w = d_norm_weight;
    h.eps = eps;
    h.head = d_head;
    h.head_ld = head_ld;
    h.rows = rows;
    h.d = d;
    h.vocab = vocab;
    h.hn = (uint16_t *) s->base.part_cands;   // rows x d bf16: within the published candidates' region
    h.keys = (uint64_t *) s->base.partials;   // rows picks: within the partials' region
    h.out_ids = d_out_ids;
    h.out_max = d_out_max;
    const hipError_t e = launch_head_pick(h, (hipStream_t) stream);
    return e == hipSuccess ? SPX_OK : hip_fail(e, "head pick launch");
}

spx_status spx_sampler_last_stats(spx_sampler * s, spx_stats * out) {
    if (!s || !out) return fail(SPX_ERR_INVALID_ARGUMENT, "null argument");
    int32_t c = 0;
    hipError_t e = hipMemcpy(&c, s->base.fb_count, sizeof(c), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpy");
    out->rows_fallback = c;
    out->splits = s->last_splits;
    out->block = s->last_block;
    out->reserved = 0;
    return SPX_OK;
}

}  // extern "C"
