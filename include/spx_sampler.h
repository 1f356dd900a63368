/*
 * spx_sampler.h — the C ABI of the MI355X (gfx950) batched token sampler.
 *
 * One call samples many rows of logits that already live in device memory: suppress-token masking, presence /
 * frequency / repetition penalties over each row's token history, temperature, top-k, top-p, the softmax and the
 * categorical draw from a caller-supplied uniform, or greedy argmax. Every row carries its own parameters and its own
 * "flavor", the sampling semantics of one speech.cpp family:
 *
 *   SPX_FLAVOR_TRANSFORMERS  Qwen3-TTS talker / code predictor and Qwen3-ASR greedy decoding, as
 *                            src/families/qwen3-tts/sampler.cpp:29-116 restates transformers' logits processors.
 *   SPX_FLAVOR_HARU          Haru's sample_token(), src/families/haru/sampler.cpp:18-61.
 *   SPX_FLAVOR_FISH          Drama 3's fish-speech sample_top_k_top_p(), src/families/drama3/sampler.cpp:30-60.
 *
 * The draw itself is src/common/sampling.cpp:9-19 (pick): the first candidate whose cumulative share of the kept
 * weights passes u, the last where none does. u comes from the caller (src/common/sampling.cpp:5-7, uniform()),
 * one double per row, so results are deterministic and independent of the launch shape.
 *
 * Conventions: no exception or C++ type crosses this boundary. Pointers named d_* are device pointers; all work is
 * queued on the given stream and is asynchronous; the sampler handle owns a preallocated workspace and must not be
 * used from two streams at once (calls on one handle serialize on its stream). A handle is bound to the device that
 * was current when it was created.
 */
#ifndef SPX_SAMPLER_H
#define SPX_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Call-level status. */
typedef enum spx_status {
    SPX_OK = 0,
    SPX_ERR_INVALID_ARGUMENT = 1, /* a null pointer, a size beyond what the handle was created for, a bad dtype */
    SPX_ERR_DEVICE = 2,           /* a HIP call failed; spx_last_error() has its message */
    SPX_ERR_OUT_OF_MEMORY = 3,
} spx_status;

/*
 * Row-level status, written to d_out_status[row]. Each non-OK code stands for the exception the reference throws for
 * that row (the C++ host layer rethrows it as the same Error kind naming the same input):
 */
typedef enum spx_row_status {
    SPX_ROW_OK = 0,
    /* Error(Fault::OutOfRange, ..., "repetition_penalty"): src/families/qwen3-tts/sampler.cpp:44-48 */
    SPX_ROW_REP_PENALTY_OVERFLOW = 1,
    /* temperature_overflow(): src/common/sampling.cpp:21-25, raised at qwen3-tts/sampler.cpp:83,
       haru/sampler.cpp:34, drama3/sampler.cpp:47 */
    SPX_ROW_TEMPERATURE_OVERFLOW = 2,
    /* std::runtime_error("no token has a finite logit to pick from"): qwen3-tts/sampler.cpp:49 */
    SPX_ROW_NO_FINITE_LOGIT = 3,
    /* Error(Fault::Device, ...): haru/sampler.cpp:21-23 (NaN or +inf), drama3/sampler.cpp:35-37 (any non-finite);
       also a NaN logit drawn under SPX_FLAVOR_TRANSFORMERS, whose reference order is undefined there */
    SPX_ROW_NONFINITE_INPUT = 4,
    /* parameters the reference's engines refuse before sampling (a temperature <= 0 or NaN where a draw needs one,
       a ban list under SPX_FLAVOR_FISH, an unknown flavor) */
    SPX_ROW_INVALID_PARAMS = 5,
} spx_row_status;

typedef enum spx_dtype { SPX_F32 = 0, SPX_BF16 = 1 } spx_dtype;

typedef enum spx_flavor { SPX_FLAVOR_TRANSFORMERS = 0, SPX_FLAVOR_HARU = 1, SPX_FLAVOR_FISH = 2 } spx_flavor;

/*
 * Per-row parameters, 32 bytes. The first five fields are SamplingParams (src/families/qwen3-tts/sampler.h:12-24),
 * haru::Sampling (src/families/haru/sampler.h:13-19) and drama3::Sampling (src/families/drama3/sampler.h:12-17).
 * top_k <= 0 keeps every token (TRANSFORMERS, HARU); FISH clamps it to [1, vocab] as drama3/sampler.cpp:44 does.
 * presence_penalty and frequency_penalty have no counterpart in the reference: where non-zero they are applied to the
 * raw logit of every token that occurs c > 0 times in the history, as l = (l - frequency*c) - presence in float, before
 * the repetition penalty. Neutral values (rep 1, presence 0, frequency 0) leave the history unread.
 */
typedef struct spx_row_params {
    int32_t flavor;           /* spx_flavor */
    int32_t greedy;           /* nonzero: argmax of the penalized, suppressed logits; u unused */
    float temperature;
    int32_t top_k;
    float top_p;
    float repetition_penalty; /* 1 = off */
    float presence_penalty;   /* 0 = off */
    float frequency_penalty;  /* 0 = off */
} spx_row_params;

typedef struct spx_sampler spx_sampler;

/*
 * Creates a handle on the current HIP device with a workspace for calls of at most max_rows rows of at most
 * max_vocab logits and at most max_hist history ids per row, and room for max_out kept candidates per row in the
 * optional candidate outputs of spx_sample_rows.
 */
spx_status spx_sampler_create(spx_sampler ** out, int max_rows, int max_vocab, int max_hist, int max_out);
void spx_sampler_destroy(spx_sampler * s);

/*
 * Samples `rows` rows. Replaces, batched and on the device, the per-row host calls
 *   sample(logits, p, history, banned, u)         src/families/qwen3-tts/sampler.cpp:103-111 (and :113-116)
 *   tokens[pick(candidates(logits, s).weights, u)] src/families/haru/sampler.h:32, drama3/sampler.h:32, :49-52
 *   max_element(logits)                            src/families/qwen3-asr/decoder.cpp:112, greedy
 *
 *   d_logits       rows x vocab logits, row r at d_logits + r*ld elements of `dtype`
 *   d_hist         the history ids of all rows, concatenated; row r's are d_hist[d_hist_off[r] .. d_hist_off[r+1]);
 *                  ids outside [0, vocab) are skipped as restricted() skips them. May be null when every row has
 *                  neutral penalties.
 *   d_hist_off     rows+1 offsets into d_hist (null with d_hist)
 *   d_banned       suppress mask, bit i%32 of word i/32 set = token i removed (-inf); row r's mask starts at
 *                  d_banned + r*banned_stride words, so a stride of 0 shares one mask by every row. May be null.
 *   d_params       rows spx_row_params
 *   d_u            rows doubles in [0, 1], the uniform() of each drawing row (unread for greedy rows)
 *   d_out_ids      rows int32: the token picked (-1 where the row status is not OK)
 *   d_out_status   rows int32: spx_row_status
 *   d_out_kept     optional (may be null): rows int32, the size of the row's Candidates (src/common/sampling.h:10-13),
 *                  the list the draw pick()s from: the tokens kept by top-k and top-p (TRANSFORMERS, FISH), all k
 *                  tokens of the top-k (HARU, whose top-p gives weight 0 rather than dropping), 1 for greedy rows
 *   d_out_cand_ids, d_out_cand_weights   optional (both null or both set): rows x max_out, the first
 *                  min(kept, max_out) tokens of the Candidates by falling logit and their weights as the reference's
 *                  Candidates holds them: TRANSFORMERS the softmax over the top k, not normalized again after top-p
 *                  (src/families/qwen3-tts/sampler.cpp:84-99); HARU the float32 probabilities over the top k, 0 for
 *                  the tokens top-p zeroes (src/families/haru/sampler.cpp:44-59); FISH the exponentials relative to
 *                  the largest logit, not normalized (src/families/drama3/sampler.cpp:48-59); greedy rows their one
 *                  token with weight 1. Entries past the list are -1 and 0.
 */
spx_status spx_sample_rows(spx_sampler * s, const void * d_logits, int dtype, int rows, int vocab, int64_t ld,
                           const int32_t * d_hist, const int32_t * d_hist_off, const uint32_t * d_banned,
                           int64_t banned_stride, const spx_row_params * d_params, const double * d_u,
                           int32_t * d_out_ids, int32_t * d_out_status, int32_t * d_out_kept,
                           int32_t * d_out_cand_ids, double * d_out_cand_weights, void * stream);

/*
 * The candidates of `rows` rows, every one of them: the reference's Candidates (src/common/sampling.h:10-13) of
 *   candidates(logits, p, history, banned)   src/families/qwen3-tts/sampler.cpp:69-101 (TRANSFORMERS)
 *   haru::candidates(logits, s)              src/families/haru/sampler.cpp:18-61 (HARU)
 *   drama3::candidates(logits, s)            src/families/drama3/sampler.cpp:30-60 (FISH)
 * as the first min(n, cap) tokens by falling logit and their weights (as d_out_cand_weights of spx_sample_rows
 * describes them), -1 and 0 past them, rows x cap each; d_out_n gets n, the list's full length (up to vocab: a cap of
 * vocab lists them all). Same layout rules as spx_sample_rows; greedy rows list their one token. A long list is read
 * in order by batches of the row, so it costs reads of the row in proportion to its length.
 */
spx_status spx_candidates_rows(spx_sampler * s, const void * d_logits, int dtype, int rows, int vocab, int64_t ld,
                               const int32_t * d_hist, const int32_t * d_hist_off, const uint32_t * d_banned,
                               int64_t banned_stride, const spx_row_params * d_params, int cap, int32_t * d_out_tokens,
                               double * d_out_weights, int32_t * d_out_n, int32_t * d_out_status, void * stream);

/*
 * Greedy argmax of `rows` rows with a shared or per-row suppress mask: the first largest logit, NaN ignored except in
 * the first position, as std::max_element does (src/families/qwen3-asr/decoder.cpp:112,
 * src/common/qwen3-decoder.cpp:427-429 with the fork's first-of-equals argmax). Same layout rules as spx_sample_rows.
 */
spx_status spx_argmax_rows(spx_sampler * s, const void * d_logits, int dtype, int rows, int vocab, int64_t ld,
                           const uint32_t * d_banned, int64_t banned_stride, int32_t * d_out_ids, void * stream);

/*
 * One pick of Qwen3-TTS's code-predictor chain for `rows` streams at once, kept on the device between the predictor's
 * forwards: pick `step` (0-based: the frame's code step + 1) of every stream, drawn from d_logits (rows x vocab, the
 * step's head) with the stream's codes picked so far this frame as the history, and written into the codes array
 * where the next pick reads it. The penalties of d_params apply, repetition included, so that the picks stay on the
 * device where GraphSampler (src/families/qwen3-tts/graph-sampler.h:18-57) falls back to the host for a repetition
 * penalty other than 1 (src/families/qwen3-tts/talker.cpp:145-153). Replaces, per stream,
 *   sample(logits, cp_sampling, cp_history, none, cp_draws[code - 1])   src/families/qwen3-tts/synthesizer.cpp:92-93,
 *   with cp_history the frame's codes 1 .. code - 1                       :130-139
 *   d_codes        rows x codes_stride int32 (codes_stride >= picks + 1): stream r's frame at d_codes + r*codes_stride,
 *                  [0] the talker's first code, [1 .. step] the codes picked so far; pick `step` writes [step + 1]
 *   d_params       rows spx_row_params (the code predictor's settings, per stream)
 *   d_u            rows x picks doubles: stream r's uniform() numbers for its picks in order (r*picks + step is read;
 *                  unread for greedy rows)
 *   d_out_status   optional: rows int32 spx_row_status of this pick
 * The handle's max_hist must be at least picks.
 */
spx_status spx_sample_chain(spx_sampler * s, const void * d_logits, int dtype, int rows, int vocab, int64_t ld,
                            int32_t * d_codes, int codes_stride, int step, int picks, const spx_row_params * d_params,
                            const double * d_u, int32_t * d_out_status, void * stream);

/*
 * Drama 3's main token (FrameSampler::main, src/families/drama3/sampler.cpp:70-79) for `rows` rows at once: each row
 * drawn twice from its logits, with the request's settings d_first and u d_u_first, and with the file's redraw settings
 * d_again and u d_u_again (both SPX_FLAVOR_FISH); the first draw's id mapped through d_token_ids (the file's
 * output.token_ids, one per logit) stands, unless it is a semantic id (semantic_begin .. semantic_end) among the last
 * `window` ids of the row's history (CSR, d_hist / d_hist_off: the main tokens so far, may be null), where the redraw's
 * mapped id stands. An error of either draw is the row's status, the first draw's first, as both candidates() calls
 * run. The handle's max_rows must be at least 2 * rows.
 */
spx_status spx_drama3_main(spx_sampler * s, const void * d_logits, int dtype, int rows, int vocab, int64_t ld,
                           const spx_row_params * d_first, const spx_row_params * d_again, const double * d_u_first,
                           const double * d_u_again, const int32_t * d_token_ids, int32_t semantic_begin,
                           int32_t semantic_end, int window, const int32_t * d_hist, const int32_t * d_hist_off,
                           int32_t * d_out_ids, int32_t * d_out_status, void * stream);

/*
 * The Qwen3-TTS talker's suppress mask as mask words (the layout of d_banned): Generation::banned(vocab,
 * end_of_speech, frames) of src/families/qwen3-tts/sampler.cpp:62-67, the last suppressed_tokens ids banned except
 * end_of_speech, and end_of_speech banned while frames < min_frames. Writes (vocab + 31) / 32 words on the stream.
 */
spx_status spx_talker_bans(uint32_t * d_words, int vocab, int suppressed_tokens, int32_t end_of_speech, int frames,
                           int min_frames, void * stream);

/* Message of the last failed call on this thread ("" when none). */
const char * spx_last_error(void);

/* Diagnostics of a handle (a host-side copy; synchronizes with the device). */
typedef struct spx_stats {
    int32_t rows_fallback; /* rows resolved by the multi-pass path since the handle was created */
    int32_t splits;        /* reserved */
    int32_t block;         /* threads per work-group */
    int32_t reserved;
} spx_stats;
spx_status spx_sampler_last_stats(spx_sampler * s, spx_stats * out);

/*
 * Haru's DRY repetition penalty (src/families/haru/sampler.h:35-38, DryConfig): the settings the model file holds.
 */
typedef struct spx_dry_config {
    double multiplier, base, max_penalty;
    int32_t allowed_length, lookback, max_match_length, reserved;
} spx_dry_config;

/* Tokens a DRY state may hold (lookback + max_match_length + 1) and exempt ids a call takes. */
#define SPX_DRY_MAX_HISTORY 4096
#define SPX_DRY_MAX_EXEMPT 8

/*
 * Dry::update (src/families/haru/sampler.cpp:87-110) for many text streams at once, their states on the device: row r
 * appends d_tokens[r] to its history d_hist[r * hist_stride ...] of d_len[r] tokens unless the token is one of the
 * n_exempt ids (or negative: a row whose draw failed), keeping the last lookback + max_match_length + 1 tokens.
 * hist_stride must hold that many (at most SPX_DRY_MAX_HISTORY). The penalties follow from the history when
 * spx_haru_shape_rows reads it, as Dry::update computes them.
 */
spx_status spx_dry_update_rows(int rows, const spx_dry_config * config, const int32_t * exempt, int n_exempt,
                               const int32_t * d_tokens, int32_t * d_hist, int32_t * d_len, int hist_stride,
                               void * stream);

/*
 * haru::shape_logits (src/families/haru/sampler.cpp:116-124) for many rows of fp32 text logits, in place: each row's
 * DRY penalties (Dry::update's, from its history: for every token that would extend a sequence of at least
 * allowed_length that occurred within the last lookback tokens, min(max_penalty, multiplier *
 * base^(length - allowed_length)) of its longest one, in double) subtracted as floats (Dry::apply, :112-114); the
 * logits of pad and eop replaced by d_silent[2r] and d_silent[2r + 1]; eop_bias added to eop's where it is not 0;
 * and, where d_must_speak[r] is nonzero, pad, eop and eos set to -inf (d_must_speak may be null). History ids
 * outside [0, vocab) are never written. The optional outputs list each row's penalties as Dry::penalties() does, by
 * rising token: d_out_pen_tokens and d_out_pen of rows x pen_cap, d_out_npen their count (may exceed pen_cap).
 */
spx_status spx_haru_shape_rows(float * d_logits, int rows, int vocab, int64_t ld, const spx_dry_config * config,
                               const int32_t * exempt, int n_exempt, const int32_t * d_hist, const int32_t * d_len,
                               int hist_stride, const float * d_silent, int32_t pad, int32_t eop, int32_t eos,
                               float eop_bias, const uint8_t * d_must_speak, int32_t * d_out_pen_tokens,
                               double * d_out_pen, int32_t * d_out_npen, int pen_cap, void * stream);

/*
 * The LM head's pick fused with its product: Qwen3Decoder::outputs() with Qwen3Readback::Pick
 * (src/common/qwen3-decoder.cpp:422-429) and verify()'s picks (:497-501). For each of `rows` hidden states (fp32, rows
 * hidden_ld floats apart): ggml's rms_norm with eps, times d_norm_weight (null: 1), the product with the head (vocab
 * rows of d bf16 weights, head_ld elements apart, 16-byte aligned; d a multiple of 64) in bf16 on the matrix cores
 * with fp32 sums, and the first largest logit (a NaN before any number, as torch.argmax): d_out_ids[r], and that
 * logit in d_out_max[r] (may be null). The logits never reach memory. At most 64 rows, and rows * d * 2 bytes within
 * the handle's workspace (8 KiB per row of max_rows).
 */
spx_status spx_head_argmax_rows(spx_sampler * s, const float * d_hidden, int64_t hidden_ld, const float * d_norm_weight,
                                float eps, const uint16_t * d_head, int64_t head_ld, int rows, int d, int vocab,
                                int32_t * d_out_ids, float * d_out_max, void * stream);

/* Rows per call of spx_sample_rows_noalloc. */
#define SPX_NOALLOC_MAX_ROWS 2048

/*
 * spx_sample_rows without a handle and without allocating: no counterpart in the reference. It is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The arguments mean what spx_sample_rows's do; max_hist bounds every row's history (a longer one is the row's
 * SPX_ROW_INVALID_PARAMS) and max_out (0..256) is the row stride of the candidate outputs. The workspace is a static
 * device array of the library (about 18.4 MB per device, held until the process ends) for up to SPX_NOALLOC_MAX_ROWS
 * rows; larger calls, and a vocab and max_hist whose launch needs more than a CU's 160 KiB of LDS, are refused with
 * SPX_ERR_INVALID_ARGUMENT. Every call on one device shares that device's array: calls that overlap on one device
 * (on two streams, or from two threads without ordering) race, and must be ordered by the caller. The first call on
 * a device sets the array up and waits for its stream once.
 */
spx_status spx_sample_rows_noalloc(const void * d_logits, int dtype, int rows, int vocab, int64_t ld,
                                   const int32_t * d_hist, const int32_t * d_hist_off, int max_hist,
                                   const uint32_t * d_banned, int64_t banned_stride, const spx_row_params * d_params,
                                   const double * d_u, int32_t * d_out_ids, int32_t * d_out_status,
                                   int32_t * d_out_kept, int32_t * d_out_cand_ids, double * d_out_cand_weights,
                                   int max_out, void * stream);

#ifdef __cplusplus
}
#endif

#endif /* SPX_SAMPLER_H */
