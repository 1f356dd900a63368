"""Pins of the oracle's Haru DRY (Dry::update, src/families/haru/sampler.cpp:87-110) and shape_logits (:116-124) by
answers worked out by hand from the rule: the sequences that repeat, the token after each earlier occurrence, the
longest match per token, the lookback and max_match_length limits, the exempt ids and the order of shape_logits's
edits. The reference's own DRY cases (dry.jsonl, read by checks/haru/haru-sampling-check.cpp:104-128) are not in the
checkout, so these stand in for them."""

import numpy as np

import oracle_lib
import workloads

spx = workloads.spx_module()


def cfg(allowed=2, lookback=8, max_match=5, multiplier=0.8, base=1.75, max_penalty=3.0):
    return spx.DryConfig(multiplier, base, max_penalty, allowed, lookback, max_match, 0)


EXEMPT = [0, 1, 2]  # pad, eop, eos in these cases


def pens(config, tokens):
    _, t, p = oracle_lib.dry_run(config, EXEMPT, tokens)
    return dict(zip(t.tolist(), p.tolist()))


def test_a_repeated_pair_penalizes_what_followed_it():
    # 5 6 was followed by 7; after 5 6 again, 7 would extend a match of length 2 = allowed: multiplier * base^0
    assert pens(cfg(), [5, 6, 7, 5, 6]) == {7: 0.8}
    # one short of allowed_length: nothing
    assert pens(cfg(allowed=3), [5, 6, 7, 5, 6]) == {}


def test_the_longest_match_wins_and_is_capped():
    # 3 4 5 3 4 5 3 4: the last 4 matched at position 4 over 5 tokens (max_match_length), at position 1 over 2; both
    # name 5, which takes the longer: 0.8 * 1.75^3 = 4.29 above max_penalty 3
    assert pens(cfg(), [3, 4, 5, 3, 4, 5, 3, 4]) == {5: 3.0}
    assert pens(cfg(max_penalty=10.0), [3, 4, 5, 3, 4, 5, 3, 4]) == {5: 0.8 * 1.75 ** 3}
    # a match of three: 0.8 * 1.75
    assert pens(cfg(), [3, 4, 5, 9, 3, 4, 5]) == {9: 0.8 * 1.75}
    # the nearer occurrence of 6 matches 5 6 (then 7 against 4), the older one 4 5 6; both were followed by 9, which
    # takes the older, longer match
    assert pens(cfg(), [3, 4, 5, 6, 9, 7, 5, 6, 9, 4, 5, 6]) == {9: 0.8 * 1.75}


def test_every_token_that_followed_is_listed_by_rising_id():
    # with allowed_length 1 each earlier 4 names the token after it
    _, t, p = oracle_lib.dry_run(cfg(allowed=1), EXEMPT, [4, 9, 4, 8, 4])
    assert t.tolist() == [8, 9] and p.tolist() == [0.8, 0.8]


def test_lookback_limits_where_matches_are_found():
    # the positions searched run from n - 2 down to n - 1 - lookback: with lookback 2 positions 3 and 2, neither
    # holding 6; with 3 also position 1, which does
    assert pens(cfg(lookback=2), [5, 6, 7, 5, 6]) == {}
    assert pens(cfg(lookback=3), [5, 6, 7, 5, 6]) == {7: 0.8}


def test_exempt_tokens_leave_the_state():
    # an exempt token is not recorded and keeps the penalties of the update before it
    assert pens(cfg(), [5, 6, 0, 7, 5, 1, 6]) == {7: 0.8}
    assert pens(cfg(), [5, 6, 7, 5, 6, 2]) == {7: 0.8}
    # the history is 5 6 5 6 without the exempt 0: the 5 after the first 5 6 is penalized, never the 0
    assert pens(cfg(), [5, 6, 0, 5, 6]) == {5: 0.8}


def test_the_window_keeps_lookback_plus_max_match_plus_one():
    c = cfg(lookback=4, max_match=3)  # 8 tokens kept
    h, _, _ = oracle_lib.dry_run(c, EXEMPT, list(range(10, 30)))
    assert h.tolist() == list(range(22, 30))
    # 5 6 7 at the start has left the window by the time 5 6 comes back
    assert pens(c, [5, 6, 7, 10, 11, 12, 13, 14, 15, 5, 6]) == {}


def test_shape_logits_order_of_edits():
    logits = np.linspace(-1, 1, 16).astype(np.float32)
    out = oracle_lib.haru_shape(logits, [7, 9], [0.8, 3.0], [1.5, -2.0], 0, 1, 2, eop_bias=0.25)
    want = logits.copy()
    want[7] = np.float32(want[7] - np.float32(0.8))
    want[9] = np.float32(want[9] - np.float32(3.0))
    want[0] = 1.5
    want[1] = np.float32(np.float32(-2.0) + np.float32(0.25))
    assert np.array_equal(out, want)
    out = oracle_lib.haru_shape(logits, [7], [0.8], [1.5, -2.0], 0, 1, 2, eop_bias=0.25, must_speak=True)
    assert np.all(np.isneginf(out[[0, 1, 2]])) and out[7] == want[7] and np.array_equal(out[3:7], logits[3:7])
