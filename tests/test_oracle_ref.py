"""Pins of the oracle's uniform() and pick() restatements: bit for bit against the reference's own
src/common/sampling.cpp (compiled unchanged into oracle/_ref by oracle/Makefile), and the known answers of
checks/qwen3-tts/qwen3-tts-sampler-check.cpp:93-116."""

import os

import numpy as np
import pytest

import oracle_lib
import workloads

# Whether oracle/_ref was built; the library itself is loaded only by the tests that use it, so collecting this file
# maps nothing built from the reference's sources.
needs_ref = pytest.mark.skipif(not os.path.exists(oracle_lib.REF_SO),
                               reason="oracle/_ref was not built (reference checkout absent)")


@needs_ref
@pytest.mark.parametrize("seed", [0, 1, 5489, 2 ** 63 + 17])
def test_uniform_matches_reference(seed):
    assert np.array_equal(oracle_lib.uniform_fill(seed, 100000), oracle_lib.ref_uniform_fill(seed, 100000))


def test_mt64_restatement_matches_std_mt19937_64():
    # tests/workloads.py's MT19937-64, which makes the uniforms of the device's inputs, against std::mt19937_64.
    for seed in (1, 1234, 2 ** 40 + 3):
        assert np.array_equal(workloads.uniforms(seed, 1000), oracle_lib.uniform_fill(seed, 1000))


@needs_ref
def test_pick_matches_reference_bit_for_bit():
    rng = np.random.default_rng(0)
    ref = oracle_lib.ref()
    for trial in range(3000):
        n = int(rng.integers(1, 40))
        w = rng.exponential(1.0, n) * (rng.random(n) < 0.8)
        if trial % 7 == 0:
            w[rng.integers(0, n)] = 0.0
        w = np.ascontiguousarray(w)
        # u anywhere, at the cumulative shares themselves, and at the ends
        shares = np.cumsum(w / w.sum()) if w.sum() > 0 else np.zeros(n)
        for u in [0.0, 1.0, float(rng.random()), float(shares[min(n - 1, int(rng.integers(0, n)))])]:
            assert oracle_lib.pick(w, u) == ref.ref_pick(w.ctypes.data_as(oracle_lib.ctypes.c_void_p), n, u)


def test_pick_known_answers():
    # qwen3-tts-sampler-check.cpp:98-102: the edges of the cumulative shares of weights 1, 2, 3, 4.
    w = [1.0, 2.0, 3.0, 4.0]
    for u, want in [(0.0, 0), (0.0999, 0), (0.1, 1), (0.2999, 1), (0.3000001, 2), (0.65, 3), (1.0, 3)]:
        assert oracle_lib.pick(w, u) == want, u
    assert oracle_lib.pick([5.0], 1.0) == 0


def test_uniform_shares_of_400000_draws():
    # qwen3-tts-sampler-check.cpp:103-115: 400000 draws of uniform() from seed 1 pick weights 1..4 within 0.004.
    u = oracle_lib.uniform_fill(1, 400000)
    assert u.min() >= 0.0 and u.max() <= 1.0
    w = np.array([1.0, 2.0, 3.0, 4.0])
    edges = np.cumsum(w / w.sum())[:-1]
    picks = np.searchsorted(edges, u, side="right")
    worst = np.max(np.abs(np.bincount(picks, minlength=4) / len(u) - w / 10))
    assert worst <= 0.004


@needs_ref
def test_temperature_overflow_names_the_temperature():
    # The Error the host layer must raise for SPX_ROW_TEMPERATURE_OVERFLOW (src/common/sampling.cpp:21-25).
    msg = oracle_lib.ctypes.create_string_buffer(512)
    inp = oracle_lib.ctypes.create_string_buffer(64)
    fault = oracle_lib.ref().ref_temperature_overflow(1e-38, msg, 512, inp, 64)
    assert fault == 1  # Fault::OutOfRange
    assert inp.value == b"temperature"
    assert b"temperature 1e-38" in msg.value
