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


@pytest.mark.gpu
def test_sample_and_candidates_match_the_oracle():
    spx = workloads.spx_module()
    rng = np.random.default_rng(31)
    # the last case is top-k off with a top-p set of about 70 tokens (a steep ramp), within what the device lists
    for vocab, k, p, scale in ((3072, 50, 1.0, 2.0), (2048, 50, 0.8, 2.0), (151936, 20, 1.0, 2.0), (40000, 0, 0.3, 12.0)):
        logits = distinct_logits(rng, vocab, scale)
        hist = rng.integers(0, vocab, 64).astype(np.int32)
        banned = np.zeros(vocab, dtype=np.uint8)
        banned[rng.choice(vocab, 10, replace=False)] = 1
        params = spx.row_params(1, spx.TRANSFORMERS, temperature=0.9, top_k=k, top_p=p, repetition_penalty=1.05)[0]
        st, toks, wts = oracle_lib.tf_candidates(logits, params, hist, banned)
        assert st == 0
        rc, _, ctoks, cwts, msg, _ = call(CANDIDATES, logits, params, hist, banned)
        assert rc == 0, msg
        np.testing.assert_array_equal(ctoks, toks)
        np.testing.assert_allclose(cwts, wts, rtol=1e-5, atol=1e-12)
        u = safe_u(wts, rng)
        rc, tok, *_ = call(SAMPLE, logits, params, hist, banned, u=u)
        assert rc == 0
        assert tok == toks[oracle_lib.pick(wts, u)]


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
