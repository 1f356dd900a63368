/*
 * spx_oracle.h — TEST INFRASTRUCTURE ONLY. A CPU restatement of speech.cpp's token samplers, used as the checker of
 * the HIP sampler (tests/, __graft_entry__.smoke()) and as the timed CPU baseline of bench.py. No product code links,
 * loads or calls it.
 *
 * Each function follows one reference function step by step (same copies, same float/double arithmetic, the same
 * std::partial_sort with the same comparator, the same top-p rule) and cites it. Paths are relative to the reference
 * checkout (nyosegawa/speech.cpp 0.11.1).
 *
 * Parity pins (tests/test_oracle_ref.py, test_golden.py, test_oracle_semantics.py, test_oracle_families.py,
 * test_host_layer.py):
 *   orc_uniform_fill, orc_pick        bit-exact against the reference's own src/common/sampling.cpp, compiled
 *                                     unchanged into oracle/_ref (and the fixtures tests/golden/reference_sampling.npz
 *                                     it wrote), and the known answers of checks/qwen3-tts/qwen3-tts-sampler-check.cpp
 *                                     :98-115
 *   orc_tf_candidates / orc_tf_sample the refusals of qwen3-tts-sampler-check.cpp:70-91 and
 *                                     qwen3-tts-graph-sampler-check.cpp:162-186; closed forms: greedy = the first
 *                                     maximum, top-k 1 = argmax, top-k 0 and top-p 1 = the full softmax, top-p after
 *                                     top-k normalized over the k kept and not again after the cut, the crossing
 *                                     token kept (>=), the repetition penalty's sign rule over a deduplicated history;
 *                                     brute-force draw frequencies on tiny vocabularies
 *   orc_haru_candidates               ties to the lower id; every token listed with the zeroed ones; the float32
 *                                     running sum of the top-p rule (rows where a double sum decides otherwise);
 *                                     greedy at temperature <= 0; brute force
 *   orc_fish_candidates               the temperature floor of 1e-5; shares over the softmax of every logit; the token
 *                                     passing top_p dropped, the first always kept; ties to the lower id; brute force
 *   orc_talker_bans, orc_drama3_main  transformers' SuppressTokens / MinNewTokensLength definitions; the redraw rules
 *                                     of checks/drama3/drama3-sampler-check.cpp:121-142
 *   the refusal messages              the reference's temperature_overflow() from oracle/_ref, for several
 *                                     temperatures (shortest round-trip floats)
 *   orc_dry_run, orc_haru_shape       hand-derived known answers of Dry::update (matches, the longest per token, the
 *                                     lookback and max_match_length limits, exempt ids, the window's trimming) and
 *                                     shape_logits (the order of its edits); the reference's DRY fixtures
 *                                     (dry.jsonl of checks/haru/haru-sampling-check.cpp) are not in the checkout
 *   presence / frequency penalty      parity unpinned against any reference (the reference has none); pinned by its
 *                                     closed form l - frequency*count - presence
 */
#ifndef SPX_ORACLE_H
#define SPX_ORACLE_H

#include <stdint.h>

#include "../include/spx_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

/* n numbers of uniform() (src/common/sampling.cpp:5-7) from std::mt19937_64(seed). */
void orc_uniform_fill(uint64_t seed, int n, double * out);

/* pick() (src/common/sampling.cpp:9-19). */
int orc_pick(const double * weights, int n, double u);

/*
 * candidates() of one flavor on one row, after the row has been through the penalty and suppression stages.
 * Returns a spx_row_status; fills up to `cap` tokens and their unnormalized weights, and *n_out with the full count.
 */
int orc_tf_candidates(const float * logits, int vocab, const spx_row_params * p, const int32_t * hist, int n_hist,
                      const uint8_t * banned, int32_t * tokens, double * weights, int cap, int * n_out);
int orc_haru_candidates(const float * logits, int vocab, float temperature, int top_k, float top_p, int32_t * tokens,
                        double * weights, int cap, int * n_out);
int orc_fish_candidates(const float * logits, int vocab, float temperature, int top_k, float top_p, int32_t * tokens,
                        double * weights, int cap, int * n_out);

/* What the oracle reports about one row beyond its pick, to classify a differing pick of the device. */
typedef struct orc_row_report {
    int32_t id;
    int32_t status;
    int32_t kept;          /* candidates the draw picked from */
    int32_t pad;
    double boundary;       /* distance of u from the nearest boundary between two kept candidates' cumulative shares */
    double cut;            /* distance of the top-p rule's nearest decision from its threshold (inf without one) */
} orc_row_report;

/*
 * The batched semantics of spx_sample_rows on host memory, row by row as the reference's callers do. `threads` > 1
 * splits the rows over that many std::threads. cand_ids/cand_weights (rows x cap) may be null: the first cap
 * candidates of each row and their weights as the reference's Candidates holds them, -1 and 0 past them.
 */
void orc_sample_rows(const void * logits, int dtype, int rows, int vocab, int64_t ld, const int32_t * hist,
                     const int32_t * hist_off, const uint32_t * banned, int64_t banned_stride,
                     const spx_row_params * params, const double * u, orc_row_report * reports, int32_t * cand_ids,
                     double * cand_weights, int cap, int threads);

/*
 * The logits one row draws from after the penalty, suppression and temperature stages of its flavor (the values the
 * candidates are ordered by); greedy rows and HARU rows with temperature <= 0 get no temperature. Returns the status
 * of the stages.
 */
int orc_final_logits(const float * logits, int vocab, const spx_row_params * p, const int32_t * hist, int n_hist,
                     const uint8_t * banned, float * out);

/* Generation::banned (src/families/qwen3-tts/sampler.cpp:62-67): out[i] = 1 for each banned id of the talker's frame. */
void orc_talker_bans(int vocab, int suppressed_tokens, int32_t end_of_speech, int frames, int min_frames,
                     uint8_t * out);

/*
 * FrameSampler::main (src/families/drama3/sampler.cpp:70-79) with the request's and the redraw's settings as two
 * records (their temperature, top_k and top_p): the mapped id of the first draw, or of the redraw where the first is a
 * semantic id among the last `window` ids of the history. Returns a spx_row_status.
 */
int orc_drama3_main(const float * logits, int vocab, const spx_row_params * first, const spx_row_params * again,
                    double u_first, double u_again, const int32_t * token_ids, int32_t semantic_begin,
                    int32_t semantic_end, int window, const int32_t * history, int n_history, int32_t * out_id);

/*
 * Haru's Dry (src/families/haru/sampler.cpp:83-114) run over n_tokens tokens from a fresh state: writes the history it
 * keeps (hist_out, *n_hist) and the penalties of its last update by rising token (the first `cap`); returns their
 * count.
 */
int orc_dry_run(const spx_dry_config * c, const int32_t * exempt, int n_exempt, const int32_t * tokens, int n_tokens,
                int32_t * hist_out, int * n_hist, int32_t * pen_tokens, double * pen, int cap);

/* haru::shape_logits (src/families/haru/sampler.cpp:116-124) of one row in place, with orc_dry_run's penalties. */
void orc_haru_shape(float * logits, const int32_t * pen_tokens, const double * pen, int n_pen, const float * silent,
                    int32_t pad, int32_t eop, int32_t eos, float eop_bias, int must_speak);

#ifdef __cplusplus
}
#endif

#endif
