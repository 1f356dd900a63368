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
