"""The C++ host layer (speech.cpp_amd/host/spx_host.cpp): the reference's sampler entry points with their names,
arguments and exceptions, computed on the GPU. Reached through its C surface spx_host_call(), which runs the C++
function and reports the exception it threw. Ids and candidates are checked against the oracle on inputs with no
ties and u away from every boundary; the exceptions against the reference's throw sites."""

import ctypes
import os

import numpy as np
import pytest

import oracle_lib
import workloads

HOST_SO = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "speech.cpp_amd", "lib",
                       "libspx_host.so")
SAMPLE, CANDIDATES, HARU_DRAW, HARU_CANDIDATES, FISH_DRAW, FISH_CANDIDATES, ARGMAX = range(7)
# Fault (src/common/error.h:8-21) + 1, as spx_host_call reports it; -1 for a std::runtime_error
OUT_OF_RANGE, DEVICE, RUNTIME_ERROR = 2, 4, -1


def host():
    if not os.path.exists(HOST_SO):
        pytest.fail(f"{HOST_SO} is not built (make -C speech.cpp_amd)")
    lib = ctypes.CDLL(HOST_SO)
    vp, i32 = ctypes.c_void_p, ctypes.c_int
    lib.spx_host_call.argtypes = [i32, vp, i32, vp, vp, i32, vp, i32, ctypes.c_double, vp, vp, vp, i32, vp,
                                  ctypes.c_char_p, i32, ctypes.c_char_p, i32]
    lib.spx_host_call.restype = i32
    return lib


def call(which, logits, params, hist=None, banned=None, u=0.5):
    lib = host()
    l = np.ascontiguousarray(logits, dtype=np.float32)
    p = np.ascontiguousarray(params)
    h = None if hist is None else np.ascontiguousarray(hist, dtype=np.int32)
    b = None if banned is None else np.ascontiguousarray(banned, dtype=np.uint8)
    oid = np.full(1, -7, dtype=np.int32)
    toks = np.zeros(len(l), dtype=np.int32)
    wts = np.zeros(len(l), dtype=np.float64)
    n = np.zeros(1, dtype=np.int32)
    msg = ctypes.create_string_buffer(512)
    inp = ctypes.create_string_buffer(64)
    ptr = lambda a: None if a is None else a.ctypes.data_as(ctypes.c_void_p)
    rc = lib.spx_host_call(which, ptr(l), len(l), ptr(p), ptr(h), 0 if h is None else len(h), ptr(b),
                           0 if b is None else len(b), u, ptr(oid), ptr(toks), ptr(wts), len(l), ptr(n), msg, 512, inp,
                           64)
    return rc, int(oid[0]), toks[:n[0]], wts[:n[0]], msg.value.decode(), inp.value.decode()


def test_host_library_exports_its_c_surface():
    lib = host()
    assert hasattr(lib, "spx_host_call")


def distinct_logits(rng, vocab, scale=2.0):
    # distinct values: no ties for any order to settle
    x = rng.permutation(vocab).astype(np.float64) / vocab * 8.0 * scale - 4.0 * scale
    return (x + rng.normal(0, 1e-3, vocab)).astype(np.float32)


def safe_u(weights, rng):
    """A uniform at least 1e-4 from every boundary of the cumulative shares."""
    cum = np.cumsum(np.asarray(weights, dtype=np.float64) / np.sum(weights))
    for _ in range(1000):
        u = rng.uniform(0.02, 0.98)
        if np.min(np.abs(cum - u)) > 1e-4:
            return u
    return 0.5


def same_list(got, want, logits):
    """The same candidates in the same order, where tokens of equal logits may trade places (the Qwen3-TTS sampler
    sorts with std::partial_sort and no tie-break)."""
    if len(got) != len(want):
        return False
    return np.array_equal(got, want) or (np.array_equal(logits[got], logits[want]) and
                                         np.array_equal(np.sort(got), np.sort(want)))


@pytest.mark.gpu
def test_sample_and_candidates_match_the_oracle():
    spx = workloads.spx_module()
    rng = np.random.default_rng(31)
    # top-k off with a top-p set of about 70 tokens (a steep ramp), and with one of about 100,000: candidates() lists
    # them all
    for vocab, k, p, scale in ((3072, 50, 1.0, 2.0), (2048, 50, 0.8, 2.0), (151936, 20, 1.0, 2.0), (40000, 0, 0.3, 12.0),
                               (151936, 0, 0.99, 2.0)):
        logits = distinct_logits(rng, vocab, scale)
        hist = rng.integers(0, vocab, 64).astype(np.int32)
        banned = np.zeros(vocab, dtype=np.uint8)
        banned[rng.choice(vocab, 10, replace=False)] = 1
        params = spx.row_params(1, spx.TRANSFORMERS, temperature=0.9, top_k=k, top_p=p, repetition_penalty=1.05)[0]
        st, toks, wts = oracle_lib.tf_candidates(logits, params, hist, banned)
        assert st == 0
        rc, _, ctoks, cwts, msg, _ = call(CANDIDATES, logits, params, hist, banned)
        assert rc == 0, msg
        final = oracle_lib.final_logits(logits, params, hist, banned)[1]
        assert same_list(ctoks, toks, final)
        np.testing.assert_allclose(cwts, wts, rtol=1e-5, atol=1e-12)
        u = safe_u(wts, rng)
        rc, tok, *_ = call(SAMPLE, logits, params, hist, banned, u=u)
        assert rc == 0
        cum = np.cumsum(wts / wts.sum())[:-1]
        if len(cum) == 0 or np.min(np.abs(cum - u)) > 1e-6:  # a long list leaves u near a boundary: excused there
            want = toks[oracle_lib.pick(wts, u)]
            assert tok == want or final[tok] == final[want]


@pytest.mark.gpu
@pytest.mark.parametrize("flavor", ["haru", "fish"])
def test_family_draws_and_candidates_match_the_oracle(flavor):
    spx = workloads.spx_module()
    rng = np.random.default_rng(37)
    for vocab, t, k, p in ((4097, 0.8, 30, 0.9), (151936, 0.7, 25, 1.0), (4096, 1.0, 1, 1.0)):
        logits = distinct_logits(rng, vocab)
        fn = oracle_lib.haru_candidates if flavor == "haru" else oracle_lib.fish_candidates
        st, toks, wts = fn(logits, t, k, p)
        assert st == 0
        params = spx.row_params(1, spx.HARU if flavor == "haru" else spx.FISH, temperature=t, top_k=k, top_p=p)[0]
        which_c, which_d = (HARU_CANDIDATES, HARU_DRAW) if flavor == "haru" else (FISH_CANDIDATES, FISH_DRAW)
        rc, _, ctoks, cwts, msg, _ = call(which_c, logits, params)
        assert rc == 0, msg
        np.testing.assert_array_equal(ctoks, toks)
        np.testing.assert_allclose(cwts, wts, rtol=1e-5, atol=1e-12)
        u = safe_u(wts, rng)
        rc, tok, *_ = call(which_d, logits, params, u=u)
        assert rc == 0
        assert tok == toks[oracle_lib.pick(wts, u)]


@pytest.mark.gpu
def test_argmax_with_bans():
    spx = workloads.spx_module()
    rng = np.random.default_rng(41)
    logits = distinct_logits(rng, 151936)
    top = int(np.argmax(logits))
    banned = np.zeros(151936, dtype=np.uint8)
    banned[top] = 1
    params = spx.row_params(1, spx.TRANSFORMERS, greedy=True)[0]
    rc, tok, *_ = call(ARGMAX, logits, params, banned=banned)
    assert rc == 0
    masked = logits.copy()
    masked[top] = -np.inf
    assert tok == int(np.argmax(masked))


@pytest.mark.gpu
def test_exceptions_are_the_references():
    spx = workloads.spx_module()
    rng = np.random.default_rng(43)
    logits = distinct_logits(rng, 3072)
    # qwen3-tts/sampler.cpp:44-48: a penalty that pushes the largest logit past a float, greedy and drawing
    for greedy in (True, False):
        params = spx.row_params(1, spx.TRANSFORMERS, greedy=greedy, temperature=0.9, top_k=50,
                                repetition_penalty=1e-40)[0]
        hist = np.array([int(np.argmax(logits))], dtype=np.int32)
        rc, _, _, _, msg, inp = call(SAMPLE, logits, params, hist)
        assert (rc, inp) == (OUT_OF_RANGE, "repetition_penalty"), msg
    # sampling.cpp:21-25 through qwen3-tts/sampler.cpp:83: a temperature of 1e-38
    params = spx.row_params(1, spx.TRANSFORMERS, temperature=1e-38, top_k=50)[0]
    rc, _, _, _, msg, inp = call(SAMPLE, logits, params)
    assert (rc, inp) == (OUT_OF_RANGE, "temperature"), msg
    # haru/sampler.cpp:21-23: NaN is an error of the device
    bad = logits.copy()
    bad[7] = np.nan
    params = spx.row_params(1, spx.HARU, temperature=0.7, top_k=25)[0]
    rc, _, _, _, msg, inp = call(HARU_DRAW, bad, params)
    assert (rc, inp) == (DEVICE, ""), msg
    # qwen3-tts/sampler.cpp:49: every token banned
    params = spx.row_params(1, spx.TRANSFORMERS, temperature=0.9, top_k=50)[0]
    rc, _, _, _, msg, _ = call(SAMPLE, logits, params, banned=np.ones(3072, dtype=np.uint8))
    assert rc == RUNTIME_ERROR and "finite" in msg


def row_error(status, params):
    lib = host()
    lib.spx_host_row_error.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int, ctypes.c_char_p,
                                       ctypes.c_int]
    lib.spx_host_row_error.restype = ctypes.c_int
    msg = ctypes.create_string_buffer(512)
    inp = ctypes.create_string_buffer(64)
    p = np.ascontiguousarray(params)
    rc = lib.spx_host_row_error(status, p.ctypes.data_as(ctypes.c_void_p), msg, 512, inp, 64)
    return rc, msg.value.decode(), inp.value.decode()


def test_error_messages_are_the_references():
    # temperature_overflow() (src/common/sampling.cpp:21-25) writes the temperature as json_number() does, the
    # shortest decimal that reads back as the float (src/common/json.h:39-63): the host layer's message must be the
    # reference's, word for word, as the reference's compiled sampling.cpp wrote it into the golden fixture.
    spx = workloads.spx_module()
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_sampling.npz"))
    for t, want in zip(g["temperatures"].tolist(), g["temperature_messages"].tolist()):
        p = spx.row_params(1, spx.TRANSFORMERS, temperature=t)[0]
        rc, msg, inp = row_error(spx.ROW_TEMPERATURE_OVERFLOW, p)
        assert (rc, inp) == (OUT_OF_RANGE, "temperature")
        assert msg == want
        if oracle_lib.ref() is not None:
            m2 = ctypes.create_string_buffer(512)
            i2 = ctypes.create_string_buffer(64)
            oracle_lib.ref().ref_temperature_overflow(np.float32(t), m2, 512, i2, 64)
            assert msg == m2.value.decode()
    # the repetition penalty's message (src/families/qwen3-tts/sampler.cpp:44-48) writes its penalty the same way
    p = spx.row_params(1, spx.TRANSFORMERS, repetition_penalty=1e-40)[0]
    rc, msg, inp = row_error(spx.ROW_REP_PENALTY_OVERFLOW, p)
    assert (rc, inp) == (OUT_OF_RANGE, "repetition_penalty")
    assert msg.startswith("the repetition penalty 1e-40 pushes a logit beyond the range of a float")
    rc, msg, _ = row_error(spx.ROW_NO_FINITE_LOGIT, p)
    assert rc == RUNTIME_ERROR and msg == "no token has a finite logit to pick from"


def test_generation_banned_is_the_oracles():
    lib = host()
    lib.spx_host_talker_banned.argtypes = [ctypes.c_int] * 5 + [ctypes.c_void_p]
    lib.spx_host_talker_banned.restype = None
    for vocab, sup, eos, frames, min_frames in ((3072, 1024, 2150, 0, 2), (3072, 1024, 2150, 9, 2), (3072, 1024, 5, 1, 3)):
        out = np.zeros(vocab, dtype=np.uint8)
        lib.spx_host_talker_banned(vocab, sup, eos, frames, min_frames, out.ctypes.data_as(ctypes.c_void_p))
        np.testing.assert_array_equal(out, oracle_lib.talker_bans(vocab, sup, eos, frames, min_frames))


@pytest.mark.gpu
def test_frame_sampler_main_is_the_oracles():
    spx = workloads.spx_module()
    lib = host()
    lib.spx_host_frame_main.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                        ctypes.c_double, ctypes.c_double, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int]
    lib.spx_host_frame_main.restype = ctypes.c_int
    rng = np.random.default_rng(53)
    vocab, window = 4097, 8
    token_ids = rng.permutation(np.arange(151000, 151000 + vocab)).astype(np.int32)
    request = spx.row_params(1, spx.FISH, temperature=0.8, top_k=30, top_p=0.9)[0]
    repeat = spx.row_params(1, spx.FISH, temperature=1.0, top_k=50, top_p=0.95)[0]
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    for trial in range(12):
        logits = distinct_logits(rng, vocab)
        top = token_ids[np.argsort(-logits)[:2]]
        history = np.concatenate([rng.integers(151000, 151000 + vocab, 10), top[: trial % 3]]).astype(np.int32)
        u1, u2 = float(rng.random()), float(rng.random())
        out = np.full(1, -7, dtype=np.int32)
        msg = ctypes.create_string_buffer(256)
        rc = lib.spx_host_frame_main(ptr(logits), vocab, ptr(np.ascontiguousarray(request)),
                                     ptr(np.ascontiguousarray(repeat)), window, 151005, 151000 + vocab - 1,
                                     ptr(token_ids), ptr(history), len(history), u1, u2, ptr(out), msg, 256)
        assert rc == 0, msg.value
        st, want = oracle_lib.drama3_main(logits, request, repeat, u1, u2, token_ids, 151005, 151000 + vocab - 1,
                                          window, history)
        assert st == 0 and out[0] == want, trial


@pytest.mark.gpu
def test_graph_sampler_chain_is_the_oracles():
    spx = workloads.spx_module()
    lib = host()
    lib.spx_host_graph_chain.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                         ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int]
    lib.spx_host_graph_chain.restype = ctypes.c_int
    rng = np.random.default_rng(55)
    streams, picks, vocab = 4, 15, 2048
    logits = np.stack([np.stack([distinct_logits(rng, vocab) for _ in range(streams)]) for _ in range(picks)])
    p = spx.row_params(1, spx.TRANSFORMERS, temperature=0.9, top_k=50, top_p=1.0, repetition_penalty=1.05)[0]
    first = rng.integers(0, 3072, streams).astype(np.int32)
    u = rng.uniform(0.02, 0.98, streams * picks)
    out = np.full(streams * picks, -7, dtype=np.int32)
    msg = ctypes.create_string_buffer(256)
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    rc = lib.spx_host_graph_chain(ptr(np.ascontiguousarray(logits)), streams, vocab, picks,
                                  ptr(np.ascontiguousarray(p)), ptr(first), ptr(u), ptr(out), msg, 256)
    assert rc == 0, msg.value
    got = out.reshape(streams, picks)
    for r in range(streams):
        for i in range(picks):
            st, toks, wts = oracle_lib.tf_candidates(logits[i, r], p, got[r, :i], None)
            assert st == 0
            assert got[r, i] == toks[oracle_lib.pick(wts, u[r * picks + i])], (r, i)


@pytest.mark.gpu
def test_haru_dry_and_shape_logits_are_the_oracles():
    # haru::Dry (src/families/haru/sampler.cpp:87-114) and shape_logits (:116-124) of the host layer, their state on the
    # device, against the oracle: the penalties after each prefix of a sequence, and the shaped logits, bit for bit.
    spx = workloads.spx_module()
    lib = host()
    vp, i32 = ctypes.c_void_p, ctypes.c_int
    lib.spx_host_dry_penalties.argtypes = [vp, vp, vp, i32, vp, i32, vp, vp, i32, vp, ctypes.c_char_p, i32]
    lib.spx_host_dry_penalties.restype = i32
    lib.spx_host_haru_shape.argtypes = [vp, vp, vp, i32, vp, i32, vp, i32, vp, i32, i32, i32, ctypes.c_float, i32,
                                        ctypes.c_char_p, i32]
    lib.spx_host_haru_shape.restype = i32
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    rng = np.random.default_rng(71)
    vocab, pad, eop, eos = 512, 509, 510, 511
    exempt = np.array([pad, eop, eos], dtype=np.int32)
    for allowed, lookback, max_match in ((2, 32, 6), (1, 8, 3)):
        config = spx.DryConfig(0.8, 1.75, 3.0, allowed, lookback, max_match, 0)
        cfg3 = np.array([0.8, 1.75, 3.0])
        cfgi = np.array([allowed, lookback, max_match], dtype=np.int32)
        seq = rng.choice(np.r_[np.arange(6), exempt], 60).astype(np.int32)
        for n in (0, 5, 17, 40, 60):
            cap = lookback + max_match + 1
            toks, pens, nout = np.zeros(cap, np.int32), np.zeros(cap), ctypes.c_int()
            msg = ctypes.create_string_buffer(256)
            assert lib.spx_host_dry_penalties(ptr(cfg3), ptr(cfgi), ptr(exempt), 3, ptr(seq), n, ptr(toks), ptr(pens),
                                              cap, ctypes.byref(nout), msg, 256) == 0, msg.value
            _, ot, op = oracle_lib.dry_run(config, exempt, seq[:n])
            assert nout.value == len(ot)
            np.testing.assert_array_equal(toks[:len(ot)], ot)
            np.testing.assert_array_equal(pens[:len(ot)].view(np.int64), op.view(np.int64))
            logits = rng.normal(0, 2, vocab).astype(np.float32)
            silent = rng.normal(0, 2, 2).astype(np.float32)
            got = logits.copy()
            assert lib.spx_host_haru_shape(ptr(cfg3), ptr(cfgi), ptr(exempt), 3, ptr(seq), n, ptr(got), vocab,
                                           ptr(silent), pad, eop, eos, 0.25, n % 2, msg, 256) == 0, msg.value
            want = oracle_lib.haru_shape(logits, ot, op, silent, pad, eop, eos, 0.25, bool(n % 2))
            np.testing.assert_array_equal(got.view(np.int32), want.view(np.int32))
