// spx_aux.hip — the small kernels around the sampler's: the Qwen3-TTS talker's suppress mask, and the two draws of
// Drama 3's main token (their records laid out for one sampling launch, then the redraw rule applied to its picks).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/spx_sampler.h"
#include "spx_internal.h"

namespace spx {

// Generation::banned (src/families/qwen3-tts/sampler.cpp:62-67) as mask words, one thread per word: the last
// `suppressed` ids banned except end_of_speech, and end_of_speech banned before min_frames frames.
__global__ void talker_bans_kernel(uint32_t * words, int vocab, int suppressed, int32_t eos, int frames, int min_frames) {
    const int w = blockIdx.x * blockDim.x + threadIdx.x;
    const int nw = (vocab + 31) / 32;
    if (w >= nw) return;
    const int lo = vocab - suppressed;  // the first suppressed id (the loop's i = vocab - suppressed_tokens)
    uint32_t bits = 0;
    for (int j = 0; j < 32; j++) {
        const int i = w * 32 + j;
        if (i >= vocab) break;
        bool b = i >= lo && i != eos;
        if (i == eos && frames < min_frames) b = true;
        bits |= b ? (1u << j) : 0u;
    }
    words[w] = bits;
}

// Row 2r draws with the request's settings and u_first[r], row 2r + 1 with the redraw's and u_again[r], both from
// logits row r.
__global__ void pair_prep_kernel(int rows, const spx_row_params * first, const spx_row_params * again,
                                 const double * u_first, const double * u_again, spx_row_params * params, double * u,
                                 int32_t * row_map) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    params[2 * r] = first[r];
    params[2 * r + 1] = again[r];
    u[2 * r] = u_first[r];
    u[2 * r + 1] = u_again[r];
    row_map[2 * r] = r;
    row_map[2 * r + 1] = r;
}

// FrameSampler::main's choice (src/families/drama3/sampler.cpp:70-79): both candidates() run, so an error of either
// is the row's (the first's first); the first draw's text-model id stands unless it is a semantic id among the last
// `window` ids of the row's history, when the redraw's stands.
__global__ void pair_pick_kernel(int rows, const int32_t * ids, const int32_t * status, const int32_t * token_ids,
                                 int32_t sem_lo, int32_t sem_hi, int window, const int32_t * hist,
                                 const int32_t * hist_off, int32_t * out_ids, int32_t * out_status) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const int s1 = status[2 * r], s2 = status[2 * r + 1];
    const int st = s1 != SPX_ROW_OK ? s1 : s2;
    int32_t id = -1;
    if (st == SPX_ROW_OK) {
        id = token_ids[ids[2 * r]];
        if (id >= sem_lo && id <= sem_hi && hist) {
            const int h0 = hist_off[r], h1 = hist_off[r + 1];
            const int from = h1 - (window < h1 - h0 ? window : h1 - h0);
            bool recent = false;
            for (int j = from; j < h1 && !recent; j++) recent = hist[j] == id;
            if (recent) id = token_ids[ids[2 * r + 1]];
        }
    }
    out_ids[r] = id;
    if (out_status) out_status[r] = st;
}

hipError_t launch_talker_bans(uint32_t * words, int vocab, int suppressed, int32_t eos, int frames, int min_frames,
                              hipStream_t s) {
    const int nw = (vocab + 31) / 32;
    hipLaunchKernelGGL(talker_bans_kernel, dim3((nw + 255) / 256), dim3(256), 0, s, words, vocab, suppressed, eos,
                       frames, min_frames);
    return hipGetLastError();
}

hipError_t launch_pair_prep(int rows, const spx_row_params * first, const spx_row_params * again, const double * u_first,
                            const double * u_again, spx_row_params * params, double * u, int32_t * row_map,
                            hipStream_t s) {
    hipLaunchKernelGGL(pair_prep_kernel, dim3((rows + 255) / 256), dim3(256), 0, s, rows, first, again, u_first, u_again,
                       params, u, row_map);
    return hipGetLastError();
}

hipError_t launch_pair_pick(int rows, const int32_t * ids, const int32_t * status, const int32_t * token_ids,
                            int32_t sem_lo, int32_t sem_hi, int window, const int32_t * hist, const int32_t * hist_off,
                            int32_t * out_ids, int32_t * out_status, hipStream_t s) {
    hipLaunchKernelGGL(pair_pick_kernel, dim3((rows + 255) / 256), dim3(256), 0, s, rows, ids, status, token_ids, sem_lo,
                       sem_hi, window, hist, hist_off, out_ids, out_status);
    return hipGetLastError();
}

}  // namespace spx

namespace spx {

// Dry::update (src/families/haru/sampler.cpp:87-92) for one text stream a work-group: the drawn token appended unless
// exempt, the history cut to its last `size` tokens (staged in registers, then written shifted).
__global__ __launch_bounds__(256) void dry_update_kernel(DryArgs d) {
    constexpr int B = 256, PER = SPX_DRY_MAX_HISTORY / B;
    const int r = blockIdx.x, tid = threadIdx.x;
    const int32_t t = d.tokens[r];
    bool skip = t < 0;
    for (int i = 0; i < d.n_exempt; i++) skip = skip || d.exempt[i] == t;
    if (skip) return;  // the same in every thread
    int32_t * h = d.hist_w + (int64_t) r * d.hist_stride;
    const int n = min(max(d.len_w[r], 0), d.hist_stride);
    const int keep = min(n + 1, d.size);  // the new length
    const int drop = n + 1 - keep;        // tokens dropped from the front
    int32_t v[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int i = tid + k * B;  // the new position i holds the old token i + drop, or t at the end
        v[k] = i < keep - 1 ? h[i + drop] : t;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int i = tid + k * B;
        if (i < keep) h[i] = v[k];
    }
    if (tid == 0) d.len_w[r] = keep;
}

// shape_logits (src/families/haru/sampler.cpp:116-124) for one row a work-group. The penalties as Dry::update forms
// them (:93-109): the positions j of the last lookback tokens before the last that hold the last token, each match
// extended backwards up to max_match tokens; those of at least allowed_length name the token after j, and each token
// takes the longest. Applied, then the silent tokens' logits.
__global__ __launch_bounds__(256) void haru_shape_kernel(DryArgs d) {
    constexpr int B = 256, CAP = SPX_DRY_MAX_HISTORY;
    __shared__ int32_t ctok[CAP];
    __shared__ int32_t clen[CAP];
    __shared__ uint8_t cwin[CAP];
    __shared__ uint32_t nc;
    const int r = blockIdx.x, tid = threadIdx.x;
    const int32_t * h = d.hist + (int64_t) r * d.hist_stride;
    const int n = min(max(d.len[r], 0), d.hist_stride);
    float * lrow = d.logits + (int64_t) r * d.ld;
    if (tid == 0) nc = 0u;
    __syncthreads();
    if (n >= max(1, d.allowed)) {
        const int32_t last = h[n - 1];
        const int lo = max(0, n - 1 - d.lookback);
        for (int j = n - 2 - tid; j >= lo; j -= B) {
            if (h[j] != last) continue;
            int length = 1;
            while (length < d.max_match && j - length >= 0 && h[j - length] == h[n - 1 - length]) length++;
            if (length >= d.allowed) {
                const uint32_t at = atomicAdd(&nc, 1u);  // at most n - 1 < CAP positions
                ctok[at] = h[j + 1];
                clen[at] = length;
            }
        }
    }
    __syncthreads();
    const int m = (int) nc;
    // each token's longest match, once (the first listed among equals, the positions' order being the atomics'), not
    // an exempt token
    for (int i = tid; i < m; i += B) {
        const int32_t tk = ctok[i];
        const int L = clen[i];
        bool win = true;
        for (int k = 0; k < m && win; k++)
            if (ctok[k] == tk && (clen[k] > L || (clen[k] == L && k < i))) win = false;
        for (int x = 0; x < d.n_exempt; x++) win = win && d.exempt[x] != tk;
        cwin[i] = win ? 1 : 0;
    }
    __syncthreads();
    // applied, and listed at its place among the row's penalties by rising token
    int nwin = 0;
    for (int i = tid; i < m; i += B) {
        if (!cwin[i]) continue;
        const int32_t tk = ctok[i];
        const int e = clen[i] - d.allowed;
        const double pen = e < d.n_table ? d.table[e] : d.sat;
        if (tk >= 0 && tk < d.vocab) lrow[tk] = lrow[tk] - (float) pen;
        if (d.out_pen_tokens) {
            int pos = 0;
            for (int k = 0; k < m; k++) pos += cwin[k] && ctok[k] < tk ? 1 : 0;
            if (pos < d.pen_cap) {
                d.out_pen_tokens[(int64_t) r * d.pen_cap + pos] = tk;
                d.out_pen[(int64_t) r * d.pen_cap + pos] = pen;
            }
        }
        nwin++;
    }
    if (d.out_npen) {
        __shared__ uint32_t total;
        if (tid == 0) total = 0u;
        __syncthreads();
        if (nwin) atomicAdd(&total, (uint32_t) nwin);
        __syncthreads();
        if (tid == 0) d.out_npen[r] = (int32_t) total;
    }
    __syncthreads();
    if (tid == 0) {
        lrow[d.pad] = d.silent[2 * r];
        lrow[d.eop] = d.silent[2 * r + 1];
        if (d.eop_bias != 0.0f) lrow[d.eop] = lrow[d.eop] + d.eop_bias;
        if (d.must_speak && d.must_speak[r]) lrow[d.pad] = lrow[d.eop] = lrow[d.eos] = -INFINITY;
    }
}

hipError_t launch_dry_update(const DryArgs & d, hipStream_t s) {
    if (d.rows == 0) return hipSuccess;
    hipLaunchKernelGGL(dry_update_kernel, dim3(d.rows), dim3(256), 0, s, d);
    return hipGetLastError();
}

hipError_t launch_haru_shape(const DryArgs & d, hipStream_t s) {
    if (d.rows == 0) return hipSuccess;
    hipLaunchKernelGGL(haru_shape_kernel, dim3(d.rows), dim3(256), 0, s, d);
    return hipGetLastError();
}

}  // namespace spx
