"""ctypes binding of the oracle (oracle/libspx_oracle.so, the CPU restatement of the reference's samplers) and of
oracle/_ref/libref_sampling.so (the reference's own src/common/sampling.cpp). Test infrastructure only."""

import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "libspx_oracle.so")
REF_SO = os.path.join(ORACLE_DIR, "_ref", "libref_sampling.so")


class RowReport(ctypes.Structure):
    _fields_ = [("id", ctypes.c_int32), ("status", ctypes.c_int32), ("kept", ctypes.c_int32), ("pad", ctypes.c_int32),
                ("boundary", ctypes.c_double), ("cut", ctypes.c_double)]


REPORT = np.dtype([("id", "<i4"), ("status", "<i4"), ("kept", "<i4"), ("pad", "<i4"), ("boundary", "<f8"),
                   ("cut", "<f8")])

_oracle = None
_ref = None


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def oracle():
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_SO):
            subprocess.run(["make", "-C", ORACLE_DIR, "libspx_oracle.so"], check=True, capture_output=True)
        lib = ctypes.CDLL(ORACLE_SO)
        vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
        lib.orc_uniform_fill.argtypes = [ctypes.c_uint64, i32, vp]
        lib.orc_pick.argtypes = [vp, i32, ctypes.c_double]
        lib.orc_pick.restype = i32
        lib.orc_tf_candidates.argtypes = [vp, i32, vp, vp, i32, vp, vp, vp, i32, vp]
        lib.orc_tf_candidates.restype = i32
        for f in (lib.orc_haru_candidates, lib.orc_fish_candidates):
            f.argtypes = [vp, i32, ctypes.c_float, i32, ctypes.c_float, vp, vp, i32, vp]
            f.restype = i32
        lib.orc_sample_rows.argtypes = [vp, i32, i32, i32, i64, vp, vp, vp, i64, vp, vp, vp, vp, vp, i32, i32]
        lib.orc_sample_rows.restype = None
        lib.orc_final_logits.argtypes = [vp, i32, vp, vp, i32, vp, vp]
        lib.orc_final_logits.restype = i32
        lib.orc_talker_bans.argtypes = [i32, i32, i32, i32, i32, vp]
        lib.orc_talker_bans.restype = None
        lib.orc_drama3_main.argtypes = [vp, i32, vp, vp, ctypes.c_double, ctypes.c_double, vp, i32, i32, i32, vp, i32,
                                        vp]
        lib.orc_drama3_main.restype = i32
        lib.orc_dry_run.argtypes = [vp, vp, i32, vp, i32, vp, vp, vp, vp, i32]
        lib.orc_dry_run.restype = i32
        lib.orc_haru_shape.argtypes = [vp, vp, vp, i32, vp, i32, i32, i32, ctypes.c_float, i32]
        lib.orc_haru_shape.restype = None
        _oracle = lib
    return _oracle


def ref():
    """The reference's own sampling.cpp, or None where the reference checkout was absent when oracle/ was built."""
    global _ref
    if _ref is None and os.path.exists(REF_SO):
        lib = ctypes.CDLL(REF_SO)
        vp, i32 = ctypes.c_void_p, ctypes.c_int
        lib.ref_uniform_fill.argtypes = [ctypes.c_uint64, i32, vp]
        lib.ref_pick.argtypes = [vp, i32, ctypes.c_double]
        lib.ref_pick.restype = i32
        lib.ref_temperature_overflow.argtypes = [ctypes.c_float, ctypes.c_char_p, i32, ctypes.c_char_p, i32]
        lib.ref_temperature_overflow.restype = i32
        _ref = lib
    return _ref


def uniform_fill(seed, n):
    out = np.zeros(n, dtype=np.float64)
    oracle().orc_uniform_fill(seed, n, _ptr(out))
    return out


def ref_uniform_fill(seed, n):
    out = np.zeros(n, dtype=np.float64)
    ref().ref_uniform_fill(seed, n, _ptr(out))
    return out


def pick(weights, u):
    w = np.ascontiguousarray(weights, dtype=np.float64)
    return oracle().orc_pick(_ptr(w), len(w), u)


def _cands(fn, *args, cap):
    tok = np.zeros(cap, dtype=np.int32)
    wts = np.zeros(cap, dtype=np.float64)
    n = ctypes.c_int(0)
    st = fn(*args, _ptr(tok), _ptr(wts), cap, ctypes.byref(n))
    return st, tok[:min(n.value, cap)], wts[:min(n.value, cap)]


def tf_candidates(logits, params, hist=None, banned=None):
    """Returns (status, tokens, weights) of the Qwen3-TTS candidates() with the penalty and suppression stages."""
    l = np.ascontiguousarray(logits, dtype=np.float32)
    p = np.ascontiguousarray(params)
    h = None if hist is None else np.ascontiguousarray(hist, dtype=np.int32)
    b = None if banned is None else np.ascontiguousarray(banned, dtype=np.uint8)
    return _cands(oracle().orc_tf_candidates, _ptr(l), len(l), _ptr(p), _ptr(h), 0 if h is None else len(h), _ptr(b),
                  cap=len(l))


def haru_candidates(logits, temperature, top_k, top_p):
    l = np.ascontiguousarray(logits, dtype=np.float32)
    return _cands(oracle().orc_haru_candidates, _ptr(l), len(l), temperature, top_k, top_p, cap=len(l))


def fish_candidates(logits, temperature, top_k, top_p):
    l = np.ascontiguousarray(logits, dtype=np.float32)
    return _cands(oracle().orc_fish_candidates, _ptr(l), len(l), temperature, top_k, top_p, cap=len(l))


def final_logits(logits, params, hist=None, banned=None):
    l = np.ascontiguousarray(logits, dtype=np.float32)
    out = np.zeros_like(l)
    h = None if hist is None else np.ascontiguousarray(hist, dtype=np.int32)
    b = None if banned is None else np.ascontiguousarray(banned, dtype=np.uint8)
    st = oracle().orc_final_logits(_ptr(l), len(l), _ptr(np.ascontiguousarray(params)), _ptr(h),
                                   0 if h is None else len(h), _ptr(b), _ptr(out))
    return st, out


def sample_rows(w, threads=8, cap=0):
    """The oracle over a tests.workloads.Workload: per-row reports, and the first `cap` candidates and their weights
    (the reference's Candidates.weights)."""
    rows, vocab = w["logits"].shape
    reports = np.zeros(rows, dtype=REPORT)
    cids = np.zeros((rows, cap), dtype=np.int32) if cap else None
    cweights = np.zeros((rows, cap), dtype=np.float64) if cap else None
    logits = np.ascontiguousarray(w["logits"])
    dtype = 1 if w["dtype"] == "bf16" else 0
    oracle().orc_sample_rows(_ptr(logits), dtype, rows, vocab, vocab, _ptr(w["hist"]), _ptr(w["hist_off"]),
                             _ptr(w["banned"]), w["banned_stride"], _ptr(np.ascontiguousarray(w["params"])),
                             _ptr(w["u"]), _ptr(reports), _ptr(cids), _ptr(cweights), cap, threads)
    return reports, cids, cweights


def talker_bans(vocab, suppressed_tokens, end_of_speech, frames, min_frames):
    """Generation::banned as a 0/1 array of vocab entries."""
    out = np.zeros(vocab, dtype=np.uint8)
    oracle().orc_talker_bans(vocab, suppressed_tokens, end_of_speech, frames, min_frames, _ptr(out))
    return out


def drama3_main(logits, first, again, u_first, u_again, token_ids, semantic_begin, semantic_end, window, history):
    """FrameSampler::main: (status, text-model id)."""
    l = np.ascontiguousarray(logits, dtype=np.float32)
    f = np.ascontiguousarray(first)
    g = np.ascontiguousarray(again)
    t = np.ascontiguousarray(token_ids, dtype=np.int32)
    h = np.ascontiguousarray(history if history is not None else np.zeros(0), dtype=np.int32)
    out = np.full(1, -7, dtype=np.int32)
    st = oracle().orc_drama3_main(_ptr(l), len(l), _ptr(f), _ptr(g), u_first, u_again, _ptr(t), semantic_begin,
                                  semantic_end, window, _ptr(h), len(h), _ptr(out))
    return st, int(out[0])


def haru_zeroing(p32, top_p, double_sum=False):
    """Which of Haru's probabilities (float32, in the row's order) the top-p rule zeroes: !(cumulative - p < top_p),
    with the running sum in float32 as src/families/haru/sampler.cpp:54-58 keeps it, or (double_sum) in double."""
    p32 = np.asarray(p32, dtype=np.float32)
    if double_sum:
        before = np.concatenate([[0.0], np.cumsum(p32.astype(np.float64))[:-1]])
        return ~(before < float(np.float32(top_p)))
    cum = np.add.accumulate(p32, dtype=np.float32)  # sequential, in order
    return ~((cum - p32) < np.float32(top_p))


def haru_float_flip(logits, temperature):
    """A top_p (float32, below 1) at which Haru's float32 running sum zeroes a different set of tokens than a double
    sum would, for a row drawing over every token, or None. Reads the probabilities from the oracle at top_p 1."""
    st, _, p = haru_candidates(logits, temperature, 0, 1.0)
    if st != 0:
        return None
    p32 = p.astype(np.float32)
    cum = np.add.accumulate(p32, dtype=np.float32)
    before_f = cum - p32
    before_d = np.concatenate([[0.0], np.cumsum(p32.astype(np.float64))[:-1]])
    # a token whose float32 share before it lies above the double one: top_p = that float32 value zeroes it in float32
    # (not below itself) and keeps it in double
    for i in np.nonzero(before_f.astype(np.float64) > before_d)[0]:
        t = np.float32(before_f[i])
        if 0 < t < 1 and not np.array_equal(haru_zeroing(p32, t), haru_zeroing(p32, t, True)):
            return float(t)
    return None


def dry_run(config, exempt, tokens):
    """Haru's Dry over `tokens` from a fresh state: (history kept, penalty tokens, penalties)."""
    ex = np.ascontiguousarray(exempt, dtype=np.int32)
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    size = config.lookback + config.max_match_length + 1
    hist = np.zeros(max(size, 1), dtype=np.int32)
    nh = ctypes.c_int()
    cap = max(size, 1)
    pt = np.zeros(cap, dtype=np.int32)
    pv = np.zeros(cap, dtype=np.float64)
    n = oracle().orc_dry_run(ctypes.byref(config), _ptr(ex), len(ex), _ptr(t), len(t), _ptr(hist), ctypes.byref(nh),
                             _ptr(pt), _ptr(pv), cap)
    return hist[:nh.value].copy(), pt[:n].copy(), pv[:n].copy()


def haru_shape(logits, pen_tokens, pens, silent, pad, eop, eos, eop_bias=0.0, must_speak=False):
    out = np.ascontiguousarray(logits, dtype=np.float32).copy()
    pt = np.ascontiguousarray(pen_tokens, dtype=np.int32)
    pv = np.ascontiguousarray(pens, dtype=np.float64)
    sl = np.ascontiguousarray(silent, dtype=np.float32)
    oracle().orc_haru_shape(_ptr(out), _ptr(pt), _ptr(pv), len(pt), _ptr(sl), pad, eop, eos, eop_bias, int(must_speak))
    return out


def bf16_round(x):
    """float32 -> the float32 values of their bfloat16 rounding (to nearest even; NaN kept)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), np.float32(np.nan), out)


def head_pick(hidden, norm_w, eps, head_bits):
    """The pick of Qwen3Decoder::outputs() (src/common/qwen3-decoder.cpp:422-429) on the CPU: ggml's rms_norm (a double
    sum of squares, the mean as float, scale = 1 / sqrtf(mean + eps), x * scale in float) times the norm weight in
    float, rounded to bf16 as ggml's product with bf16 weights converts its operand; the products with the bf16 head
    summed in double; the first largest (np.argmax: a NaN first). Returns (ids, logits rows x vocab, abs sums)."""
    x = np.ascontiguousarray(hidden, dtype=np.float32)
    d = x.shape[1]
    mean = ((x.astype(np.float64) ** 2).sum(1) / d).astype(np.float32)
    scale = (np.float32(1.0) / np.sqrt(mean + np.float32(eps))).astype(np.float32)
    y = (x * scale[:, None]).astype(np.float32)
    if norm_w is not None:
        y = (y * np.asarray(norm_w, dtype=np.float32)[None, :]).astype(np.float32)
    hb = bf16_round(y).astype(np.float64)
    h = (np.ascontiguousarray(head_bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    logits = hb @ h.T
    absum = np.abs(hb) @ np.abs(h).T
    return np.argmax(logits, axis=1).astype(np.int32), logits, absum
