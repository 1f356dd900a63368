"""Pins of the oracle's family samplers that need no reference binary: the refusals of the reference's checks,
closed forms, invariants and brute force on tiny vocabularies. A plausible slip (a dropped dedup of the history, the
wrong side of a top-p comparison, a tie broken the other way, a normalization over the wrong set) fails one of them."""

import numpy as np
import pytest

import oracle_lib
import workloads

spx = workloads.spx_module()


def tf(**kw):
    return spx.row_params(1, spx.TRANSFORMERS, **kw)[0]


def test_penalty_1e40_refused_greedy_and_drawing():
    # checks/qwen3-tts/qwen3-tts-sampler-check.cpp:70-91
    for greedy in (True, False):
        st, _, _ = oracle_lib.tf_candidates([1.0, 2.0], tf(greedy=greedy, repetition_penalty=1e-40), hist=[0, 1])
        assert st == spx.ROW_REP_PENALTY_OVERFLOW


def test_temperature_1e38_refused():
    # checks/qwen3-tts/qwen3-tts-graph-sampler-check.cpp:162-186
    st, _, _ = oracle_lib.tf_candidates(np.linspace(-3, 10, 300), tf(temperature=1e-38, top_k=50))
    assert st == spx.ROW_TEMPERATURE_OVERFLOW


def sample_one(logits, params, u, hist=None, banned=None):
    rows = 1
    h, off = (None, None)
    if hist is not None:
        h, off = workloads.csr([hist])
    w = workloads.Workload(name="one", logits=np.asarray([logits], dtype=np.float32), dtype="f32",
                           params=np.asarray([params]), u=np.array([u]), hist=h, hist_off=off,
                           banned=banned, banned_stride=0)
    rep, _, _ = oracle_lib.sample_rows(w)
    return rep[0]


@pytest.mark.parametrize("flavor", [0, 1, 2])
def test_greedy_is_the_first_largest(flavor):
    rng = np.random.default_rng(flavor)
    for _ in range(200):
        l = rng.integers(-3, 4, 17).astype(np.float32)  # many ties
        rep = sample_one(l, spx.row_params(1, flavor, greedy=True)[0], 0.5)
        assert rep["id"] == int(np.argmax(l))


@pytest.mark.parametrize("flavor", [0, 1, 2])
def test_top_k_1_is_the_argmax(flavor):
    rng = np.random.default_rng(10 + flavor)
    for _ in range(200):
        l = rng.normal(0, 2, 50).astype(np.float32)
        rep = sample_one(l, spx.row_params(1, flavor, temperature=0.8, top_k=1)[0], float(rng.random()))
        assert rep["id"] == int(np.argmax(l)) and rep["kept"] == 1


def full_softmax(l, t):
    s = (np.asarray(l, np.float32) / np.float32(t)).astype(np.float64)  # the float division, then double
    e = np.exp(s - s.max())
    return e / e.sum()


def test_transformers_full_vocab_is_the_softmax():
    rng = np.random.default_rng(3)
    l = rng.normal(0, 2, 300).astype(np.float32)
    st, tok, w = oracle_lib.tf_candidates(l, tf(temperature=0.7))
    assert st == 0 and len(tok) == 300
    p = full_softmax(l, 0.7)
    assert np.max(np.abs(w - p[tok])) < 1e-15
    assert np.all(np.diff(p[tok]) <= 0)  # by falling logit


def test_fish_normalizes_over_every_logit():
    # drama3/sampler.cpp:48-50: the shares of the kept tokens are over the softmax of the whole vocabulary, so a
    # top_p of 1 keeps every one of the top k.
    rng = np.random.default_rng(4)
    l = rng.normal(0, 2, 400).astype(np.float32)
    st, tok, w = oracle_lib.fish_candidates(l, 1.0, 30, 1.0)
    assert st == 0 and len(tok) == 30
    p = full_softmax(l, 1.0)
    assert np.allclose(w / w.sum(), p[tok] / p[tok].sum(), rtol=1e-13)
    # top_p below the largest share keeps only the first (the passing token is dropped, r=0 always kept)
    st, tok, _ = oracle_lib.fish_candidates(l, 1.0, 30, float(p.max()) * 0.5)
    assert list(tok) == [int(np.argmax(l))]


def test_top_p_rules_of_the_three_flavors():
    # Weights 0.5, 0.25, 0.125, 0.125 exactly: logits ln of them at temperature 1 are not exact in float, so use the
    # shares the oracle computes and place top_p between and on them.
    l = np.log(np.array([0.5, 0.25, 0.125, 0.125])).astype(np.float32)
    p = full_softmax(l, 1.0)
    c = np.cumsum(p)
    # transformers: the smallest prefix reaching top_p, the crossing token kept
    st, tok, _ = oracle_lib.tf_candidates(l, tf(top_p=float(np.float32(c[1] - 1e-4))))
    assert len(tok) == 2
    st, tok, _ = oracle_lib.tf_candidates(l, tf(top_p=float(np.float32(c[0] + 1e-4))))
    assert len(tok) == 2
    # fish: the token passing top_p dropped
    st, tok, _ = oracle_lib.fish_candidates(l, 1.0, 4, float(np.float32(c[1] - 1e-4)))
    assert len(tok) == 1
    st, tok, _ = oracle_lib.fish_candidates(l, 1.0, 4, float(np.float32(c[1] + 1e-4)))
    assert len(tok) == 2
    # haru: every candidate stays in the list; those whose share before them reaches top_p weigh 0
    st, tok, w = oracle_lib.haru_candidates(l, 1.0, 0, float(np.float32(c[1] - 1e-4)))
    assert len(tok) == 4 and np.count_nonzero(w) == 2


def test_ties_to_the_lower_id_in_haru_and_fish():
    l = np.array([1.0, 3.0, 3.0, 2.0, 3.0], dtype=np.float32)
    for fn in (lambda: oracle_lib.haru_candidates(l, 0.9, 3, 1.0), lambda: oracle_lib.fish_candidates(l, 0.9, 3, 1.0)):
        st, tok, _ = fn()
        assert list(tok) == [1, 2, 4]


def test_repetition_penalty_closed_form():
    rng = np.random.default_rng(5)
    l = rng.normal(0, 2, 64).astype(np.float32)
    hist = [3, 3, 3, 7, 11, 11, 63, -1, 64, 1000]  # duplicates and ids out of range
    r = np.float32(1.3)
    want = l.copy()
    for t in {3, 7, 11, 63}:
        want[t] = want[t] * r if want[t] < 0 else want[t] / r
    st, got = oracle_lib.final_logits(l, tf(greedy=True, repetition_penalty=1.3), hist=hist)
    assert st == 0 and np.array_equal(got, want)


def test_presence_frequency_closed_form():
    # No reference counterpart: l - frequency*count - presence on every id the history holds, in float, then the
    # repetition penalty.
    l = np.array([1.0, 2.0, -3.0, 0.5], dtype=np.float32)
    hist = [2, 2, 2, 1, 9]
    want = l.copy()
    want[2] = np.float32(np.float32(l[2] - np.float32(0.25) * np.float32(3)) - np.float32(0.5))
    want[1] = np.float32(np.float32(l[1] - np.float32(0.25)) - np.float32(0.5))
    want[1] = want[1] / np.float32(1.1)
    want[2] = want[2] * np.float32(1.1)
    st, got = oracle_lib.final_logits(l, tf(greedy=True, presence_penalty=0.5, frequency_penalty=0.25,
                                            repetition_penalty=1.1), hist=hist)
    assert st == 0 and np.array_equal(got, want)


def test_banned_tokens_get_no_chance():
    rng = np.random.default_rng(6)
    l = rng.normal(0, 2, 40).astype(np.float32)
    banned = np.zeros(40, np.uint8)
    banned[np.argsort(-l)[:5]] = 1
    st, tok, w = oracle_lib.tf_candidates(l, tf(top_k=10), banned=banned)
    assert st == 0 and not set(tok.tolist()) & set(np.nonzero(banned)[0].tolist())


@pytest.mark.parametrize("flavor,k,p", [(0, 0, 1.0), (0, 3, 1.0), (0, 0, 0.8), (1, 0, 1.0), (1, 4, 0.7), (2, 5, 0.9)])
def test_brute_force_draw_frequencies(flavor, k, p):
    # Over a fine grid of u the picks must reproduce the candidates' weights: pick() partitions [0, 1) into
    # intervals of the weights' shares.
    rng = np.random.default_rng(7)
    l = rng.normal(0, 1, 6).astype(np.float32)
    params = spx.row_params(1, flavor, temperature=0.9, top_k=k, top_p=p)[0]
    if flavor == 0:
        st, tok, w = oracle_lib.tf_candidates(l, params)
    elif flavor == 1:
        st, tok, w = oracle_lib.haru_candidates(l, 0.9, k, p)
    else:
        st, tok, w = oracle_lib.fish_candidates(l, 0.9, k, p)
    grid = (np.arange(20000) + 0.5) / 20000
    counts = {}
    for u in grid:
        t = int(tok[oracle_lib.pick(w, float(u))])
        counts[t] = counts.get(t, 0) + 1
    share = w / w.sum()
    for t, s in zip(tok.tolist(), share.tolist()):
        assert abs(counts.get(t, 0) / len(grid) - s) < 2.0 / len(grid) + 1e-12


def test_transformers_top_p_after_top_k_is_over_the_k_kept():
    # qwen3-tts/sampler.cpp:84-99: the weights are normalized over the top k before the top-p rule reads them, and
    # are not normalized again after it. Weights 0.4, 0.3, 0.2, 0.1 with k = 2 are 4/7 and 3/7 over the two kept, so
    # top_p 0.55 keeps one token (4/7 >= 0.55), where shares over the whole vocabulary (0.4 < 0.55) would keep two.
    l = np.log(np.array([0.4, 0.3, 0.2, 0.1])).astype(np.float32)
    st, tok, w = oracle_lib.tf_candidates(l, tf(top_k=2, top_p=0.55))
    assert st == 0 and list(tok) == [0] and abs(w[0] - 4 / 7) < 1e-6
    st, tok, w = oracle_lib.tf_candidates(l, tf(top_k=0, top_p=0.55))
    assert list(tok) == [0, 1] and np.allclose(w, [0.4, 0.3], rtol=1e-6)
    st, tok, w = oracle_lib.tf_candidates(l, tf(top_k=3, top_p=0.99))
    assert list(tok) == [0, 1, 2] and np.allclose(w, [4 / 9, 3 / 9, 2 / 9], rtol=1e-6)
    # top_p just above 4/7 + 3/7 - 1e-6: both kept, weights still over k
    st, tok, w = oracle_lib.tf_candidates(l, tf(top_k=2, top_p=0.6))
    assert list(tok) == [0, 1] and np.allclose(w, [4 / 7, 3 / 7], rtol=1e-6)


def test_fish_temperature_floor():
    # drama3/sampler.cpp:31: t = max(temperature, 1e-5). At or below the floor the logits are divided by 1e-5, so
    # logits 0, -1e-5, -3e-5 weigh exp(0), exp(-1), exp(-3) (the weights are the unnormalized exponentials).
    l = np.array([0.0, -1e-5, -3e-5], dtype=np.float32)
    want = np.exp(np.array([0.0, -1.0, -3.0]))
    for t in (1e-5, 1e-7, 0.0, -2.0):
        st, tok, w = oracle_lib.fish_candidates(l, t, 3, 2.0)
        assert st == 0 and list(tok) == [0, 1, 2]
        assert np.allclose(w, want, rtol=1e-6), (t, w)
    st, tok, w = oracle_lib.fish_candidates(l, 2e-5, 3, 2.0)  # above the floor: half the spread
    assert np.allclose(w, np.exp(np.array([0.0, -0.5, -1.5])), rtol=1e-6)


def test_haru_top_p_reads_a_float32_running_sum():
    # haru/sampler.cpp:54-58: the top-p rule compares a float32 running sum less the token's own float32 probability
    # with top_p. Rows whose float32 and double sums put a token on different sides of top_p must follow float32.
    rng = np.random.default_rng(8)
    found = 0
    for _ in range(50):
        l = rng.normal(0, 1.5, 512).astype(np.float32)
        t = oracle_lib.haru_float_flip(l, 1.0)
        if t is None:
            continue
        _, _, p = oracle_lib.haru_candidates(l, 1.0, 0, 1.0)
        st, tok, w = oracle_lib.haru_candidates(l, 1.0, 0, t)
        assert st == 0 and len(tok) == 512
        zeroed = w == 0
        assert np.array_equal(zeroed, oracle_lib.haru_zeroing(p, t))
        assert not np.array_equal(zeroed, oracle_lib.haru_zeroing(p, t, double_sum=True))
        found += 1
    assert found >= 5
