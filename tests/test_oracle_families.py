"""Pins of the oracle's restatements of the families' steps around the draw: the Qwen3-TTS talker's suppress mask
(Generation::banned, src/families/qwen3-tts/sampler.cpp:62-67) and Drama 3's main-token redraw (FrameSampler::main,
src/families/drama3/sampler.cpp:70-79)."""

import numpy as np

import oracle_lib
import workloads


def test_talker_mask_is_transformers_suppress_and_min_new_tokens():
    # The official generate() the mask restates: SuppressTokens over range(vocab - 1024, vocab) without the end of
    # speech (reference/qwen3-tts/sampling_cases.py:56), and MinNewTokensLength banning the end of speech before
    # min_new_tokens frames.
    vocab, eos = 3072, 2150
    for frames, min_frames in ((0, 2), (1, 2), (2, 2), (7, 2)):
        suppress = set(i for i in range(vocab - 1024, vocab) if i != eos)
        want = np.array([i in suppress or (i == eos and frames < min_frames) for i in range(vocab)], dtype=np.uint8)
        np.testing.assert_array_equal(oracle_lib.talker_bans(vocab, 1024, eos, frames, min_frames), want)


def test_talker_mask_with_the_end_outside_the_suppressed_ids():
    vocab, eos = 3072, 10
    got = oracle_lib.talker_bans(vocab, 1024, eos, 0, 5)
    assert got[vocab - 1024:].all() and got[eos] == 1 and got[:vocab - 1024].sum() == 1


def _fish(n, t=1.0, k=50, p=1.0):
    spx = workloads.spx_module()
    return spx.row_params(n, spx.FISH, temperature=t, top_k=k, top_p=p)


def test_drama3_redraw_rules():
    # checks/drama3/drama3-sampler-check.cpp:121-142 on synthetic logits: with a first draw of 0 (the most likely
    # token) and a redraw of almost 1 (the redraw's least likely kept token), the main token is the first draw unless
    # the history's last `window` ids hold it; an end id, made the most likely, is never drawn again.
    rng = np.random.default_rng(3)
    vocab, window = 4097, 16
    logits = rng.normal(0, 2, vocab).astype(np.float32)
    token_ids = rng.permutation(np.arange(100000, 100000 + vocab)).astype(np.int32)
    eos = int(token_ids[0])
    sem_lo, sem_hi = 100001, 100000 + vocab  # every id but some are semantic; the end id below is made not semantic
    token_ids[0] = 99999
    eos = 99999
    first, again = _fish(1, 1.0, 30, 0.9), _fish(1, 1.0, 30, 0.9)
    st, top = oracle_lib.drama3_main(logits, first[0], again[0], 0.0, 0.0, token_ids, sem_lo, sem_hi, window, None)
    assert st == 0 and sem_lo <= top <= sem_hi
    st, redrawn = oracle_lib.drama3_main(logits, first[0], again[0], 0.0, 1.0 - 1e-12, token_ids, sem_lo, sem_hi,
                                         window, np.array([top]))
    assert st == 0 and redrawn != top and sem_lo <= redrawn <= sem_hi
    other = int(token_ids[1]) if int(token_ids[1]) != top else int(token_ids[2])
    old = np.array([top] + [other] * window)
    st, kept = oracle_lib.drama3_main(logits, first[0], again[0], 0.0, 1.0 - 1e-12, token_ids, sem_lo, sem_hi,
                                      window, old)
    assert st == 0 and kept == top
    l2 = logits.copy()
    l2[0] = logits.max() + 50.0
    st, end = oracle_lib.drama3_main(l2, first[0], again[0], 0.0, 1.0 - 1e-12, token_ids, sem_lo, sem_hi, window,
                                     np.array([eos]))
    assert st == 0 and end == eos


def test_drama3_main_refuses_what_either_draw_refuses():
    # both candidates() calls run before the choice (drama3/sampler.cpp:71-74): a non-finite logit is refused
    logits = np.zeros(64, dtype=np.float32)
    logits[5] = np.inf
    st, _ = oracle_lib.drama3_main(logits, _fish(1)[0], _fish(1)[0], 0.5, 0.5, np.arange(64), 0, 63, 4, None)
    assert st == 4  # SPX_ROW_NONFINITE_INPUT
