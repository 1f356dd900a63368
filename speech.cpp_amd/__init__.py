"""Python binding of the gfx950 token sampler's C ABI (include/spx_sampler.h), for tests and bench.py.

The sampler itself is lib/libspx_sampler.so, built from csrc/ by the Makefile beside this file (``make -C
speech.cpp_amd``). There is no other implementation: when the library is missing this module raises, it never falls
back to a CPU path.

The row parameters mirror SamplingParams (src/families/qwen3-tts/sampler.h:12-24), haru::Sampling
(src/families/haru/sampler.h:13-19) and drama3::Sampling (src/families/drama3/sampler.h:12-17), one record per row.
"""

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libspx_sampler.so")

F32, BF16 = 0, 1
TRANSFORMERS, HARU, FISH = 0, 1, 2
ROW_OK, ROW_REP_PENALTY_OVERFLOW, ROW_TEMPERATURE_OVERFLOW, ROW_NO_FINITE_LOGIT, ROW_NONFINITE_INPUT, \
    ROW_INVALID_PARAMS = range(6)
ROW_STATUS_NAMES = ["OK", "REP_PENALTY_OVERFLOW", "TEMPERATURE_OVERFLOW", "NO_FINITE_LOGIT", "NONFINITE_INPUT",
                    "INVALID_PARAMS"]

# spx_row_params, 32 bytes
ROW_PARAMS = np.dtype([("flavor", "<i4"), ("greedy", "<i4"), ("temperature", "<f4"), ("top_k", "<i4"),
                       ("top_p", "<f4"), ("repetition_penalty", "<f4"), ("presence_penalty", "<f4"),
                       ("frequency_penalty", "<f4")])
assert ROW_PARAMS.itemsize == 32

# Every symbol include/spx_sampler.h declares.
EXPORTS = ["spx_sampler_create", "spx_sampler_destroy", "spx_sample_rows", "spx_argmax_rows", "spx_candidates_rows",
           "spx_sample_chain",
           "spx_drama3_main", "spx_talker_bans", "spx_last_error", "spx_sampler_last_stats", "spx_sample_rows_noalloc",
           "spx_dry_update_rows", "spx_haru_shape_rows", "spx_head_argmax_rows"]


class DryConfig(ctypes.Structure):
    """spx_dry_config: Haru's DRY settings (src/families/haru/sampler.h:35-38)."""
    _fields_ = [("multiplier", ctypes.c_double), ("base", ctypes.c_double), ("max_penalty", ctypes.c_double),
                ("allowed_length", ctypes.c_int32), ("lookback", ctypes.c_int32), ("max_match_length", ctypes.c_int32),
                ("reserved", ctypes.c_int32)]


class SpxStats(ctypes.Structure):
    _fields_ = [("rows_fallback", ctypes.c_int32), ("splits", ctypes.c_int32), ("block", ctypes.c_int32),
                ("reserved", ctypes.c_int32)]


_lib = None


def load_library(path=LIB_PATH):
    """The sampler's shared library with its C signatures declared. Raises when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"the HIP sampler library is not built: {path} is missing (run make -C {HERE})")
    # The binding hands the library torch's device buffers and streams, so both must use one HIP runtime: torch is
    # loaded first, and the library then binds to the runtime torch brought (the same soname), not to a second copy.
    import torch  # noqa: F401
    lib = ctypes.CDLL(path)
    p, i32, i64, vp = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_void_p
    lib.spx_sampler_create.argtypes = [ctypes.POINTER(p), i32, i32, i32, i32]
    lib.spx_sampler_create.restype = i32
    lib.spx_sampler_destroy.argtypes = [p]
    lib.spx_sampler_destroy.restype = None
    lib.spx_sample_rows.argtypes = [p, vp, i32, i32, i32, i64, vp, vp, vp, i64, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.spx_sample_rows.restype = i32
    lib.spx_argmax_rows.argtypes = [p, vp, i32, i32, i32, i64, vp, i64, vp, vp]
    lib.spx_argmax_rows.restype = i32
    lib.spx_candidates_rows.argtypes = [p, vp, i32, i32, i32, i64, vp, vp, vp, i64, vp, i32, vp, vp, vp, vp, vp]
    lib.spx_candidates_rows.restype = i32
    lib.spx_sample_chain.argtypes = [p, vp, i32, i32, i32, i64, vp, i32, i32, i32, vp, vp, vp, vp]
    lib.spx_sample_chain.restype = i32
    lib.spx_drama3_main.argtypes = [p, vp, i32, i32, i32, i64, vp, vp, vp, vp, vp, i32, i32, i32, vp, vp, vp, vp, vp]
    lib.spx_drama3_main.restype = i32
    lib.spx_talker_bans.argtypes = [vp, i32, i32, i32, i32, i32, vp]
    lib.spx_talker_bans.restype = i32
    lib.spx_last_error.argtypes = []
    lib.spx_last_error.restype = ctypes.c_char_p
    lib.spx_sampler_last_stats.argtypes = [p, ctypes.POINTER(SpxStats)]
    lib.spx_sampler_last_stats.restype = i32
    lib.spx_sample_rows_noalloc.argtypes = [vp, i32, i32, i32, i64, vp, vp, i32, vp, i64, vp, vp, vp, vp, vp, vp, vp,
                                            i32, vp]
    lib.spx_sample_rows_noalloc.restype = i32
    lib.spx_dry_update_rows.argtypes = [i32, ctypes.POINTER(DryConfig), vp, i32, vp, vp, vp, i32, vp]
    lib.spx_dry_update_rows.restype = i32
    lib.spx_haru_shape_rows.argtypes = [vp, i32, i32, i64, ctypes.POINTER(DryConfig), vp, i32, vp, vp, i32, vp, i32,
                                        i32, i32, ctypes.c_float, vp, vp, vp, vp, i32, vp]
    lib.spx_haru_shape_rows.restype = i32
    lib.spx_head_argmax_rows.argtypes = [p, vp, i64, vp, ctypes.c_float, vp, i64, i32, i32, i32, vp, vp, vp]
    lib.spx_head_argmax_rows.restype = i32
    _lib = lib
    return lib


def row_params(n, flavor=TRANSFORMERS, greedy=False, temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0,
               presence_penalty=0.0, frequency_penalty=0.0):
    """n rows of spx_row_params; each field a scalar or an array of n."""
    p = np.zeros(n, dtype=ROW_PARAMS)
    p["flavor"] = flavor
    p["greedy"] = np.asarray(greedy).astype(np.int32)
    p["temperature"] = temperature
    p["top_k"] = top_k
    p["top_p"] = top_p
    p["repetition_penalty"] = repetition_penalty
    p["presence_penalty"] = presence_penalty
    p["frequency_penalty"] = frequency_penalty
    return p


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


class SamplerError(RuntimeError):
    pass


class Sampler:
    """A handle of the sampler on the current device, with its workspace for calls up to the given sizes."""

    def __init__(self, max_rows, max_vocab, max_hist=0, max_out=0):
        self.lib = load_library()
        h = ctypes.c_void_p()
        self._check(self.lib.spx_sampler_create(ctypes.byref(h), max_rows, max_vocab, max_hist, max_out))
        self.handle = h
        self.max_out = max_out

    def _check(self, status):
        if status != 0:
            raise SamplerError(f"spx status {status}: {self.lib.spx_last_error().decode()}")

    def close(self):
        if getattr(self, "handle", None):
            self.lib.spx_sampler_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def sample_rows(self, logits, params, u, hist=None, hist_off=None, banned=None, banned_stride=0, out_ids=None,
                    out_status=None, out_kept=None, out_cand_ids=None, out_cand_weights=None, stream=None):
        """Samples every row of `logits` (a 2-D float32 or bfloat16 device tensor, rows may be strided). `params` is a
        device tensor holding spx_row_params records (see device_params), `u` a float64 device tensor. The optional
        candidate outputs are int32 and float64 tensors of rows x max_out."""
        import torch
        rows, vocab = logits.shape
        dtype = BF16 if logits.dtype == torch.bfloat16 else F32
        if logits.stride(1) != 1:
            raise ValueError("logits rows must be contiguous")
        ld = logits.stride(0) if rows > 1 else vocab
        dev = logits.device
        if out_ids is None:
            out_ids = torch.empty(rows, dtype=torch.int32, device=dev)
        if out_status is None:
            out_status = torch.empty(rows, dtype=torch.int32, device=dev)
        for t, dt in ((out_ids, torch.int32), (out_status, torch.int32), (out_kept, torch.int32)):
            if t is not None and (t.dtype != dt or t.numel() < rows or not t.is_contiguous()):
                raise ValueError("per-row outputs are contiguous int32 tensors of at least rows entries")
        for t, dt in ((out_cand_ids, torch.int32), (out_cand_weights, torch.float64)):
            if t is not None and (t.dtype != dt or t.numel() < rows * self.max_out or not t.is_contiguous()):
                raise ValueError("candidate outputs are contiguous tensors of rows x max_out (the handle's)")
        s = stream if stream is not None else torch.cuda.current_stream(dev).cuda_stream
        self._check(self.lib.spx_sample_rows(
            self.handle, _ptr(logits), dtype, rows, vocab, ld, _ptr(hist), _ptr(hist_off), _ptr(banned),
            banned_stride, _ptr(params), _ptr(u), _ptr(out_ids), _ptr(out_status), _ptr(out_kept), _ptr(out_cand_ids),
            _ptr(out_cand_weights), ctypes.c_void_p(s)))
        return out_ids, out_status

    def argmax_rows(self, logits, banned=None, banned_stride=0, out_ids=None, stream=None):
        import torch
        rows, vocab = logits.shape
        dtype = BF16 if logits.dtype == torch.bfloat16 else F32
        if out_ids is None:
            out_ids = torch.empty(rows, dtype=torch.int32, device=logits.device)
        if logits.stride(1) != 1:
            raise ValueError("logits rows must be contiguous")
        ld = logits.stride(0) if rows > 1 else vocab
        s = stream if stream is not None else torch.cuda.current_stream(logits.device).cuda_stream
        self._check(self.lib.spx_argmax_rows(self.handle, _ptr(logits), dtype, rows, vocab, ld,
                                             _ptr(banned), banned_stride, _ptr(out_ids), ctypes.c_void_p(s)))
        return out_ids

    def candidates_rows(self, logits, params, cap, hist=None, hist_off=None, banned=None, banned_stride=0,
                        stream=None):
        """Every row's candidates, the first `cap`: (tokens rows x cap int32, weights rows x cap float64, n, status)."""
        import torch
        rows, vocab = logits.shape
        dev = logits.device
        dtype = BF16 if logits.dtype == torch.bfloat16 else F32
        ld = logits.stride(0) if rows > 1 else vocab
        toks = torch.empty((rows, cap), dtype=torch.int32, device=dev)
        wts = torch.empty((rows, cap), dtype=torch.float64, device=dev)
        n = torch.empty(rows, dtype=torch.int32, device=dev)
        status = torch.empty(rows, dtype=torch.int32, device=dev)
        s = stream if stream is not None else torch.cuda.current_stream(dev).cuda_stream
        self._check(self.lib.spx_candidates_rows(self.handle, _ptr(logits), dtype, rows, vocab, ld, _ptr(hist),
                                                 _ptr(hist_off), _ptr(banned), banned_stride, _ptr(params), cap,
                                                 _ptr(toks), _ptr(wts), _ptr(n), _ptr(status), ctypes.c_void_p(s)))
        return toks, wts, n, status

    def sample_chain(self, logits, codes, step, params, u, out_status=None, stream=None):
        """Pick `step` of the code-predictor chain: logits (streams x vocab), codes (streams x >= picks + 1 int32, row
        r: [first code, picked codes...]), u (streams x picks float64). Writes codes[:, step + 1]."""
        import torch
        rows, vocab = logits.shape
        picks = u.shape[1]
        if codes.dtype != torch.int32 or not codes.is_contiguous() or codes.shape[0] < rows:
            raise ValueError("codes are a contiguous int32 tensor of streams x (picks + 1) or more")
        if u.dtype != torch.float64 or not u.is_contiguous():
            raise ValueError("u is a contiguous float64 tensor of streams x picks")
        dtype = BF16 if logits.dtype == torch.bfloat16 else F32
        ld = logits.stride(0) if rows > 1 else vocab
        s = stream if stream is not None else torch.cuda.current_stream(logits.device).cuda_stream
        self._check(self.lib.spx_sample_chain(self.handle, _ptr(logits), dtype, rows, vocab, ld, _ptr(codes),
                                              codes.shape[1], step, picks, _ptr(params), _ptr(u), _ptr(out_status),
                                              ctypes.c_void_p(s)))

    def drama3_main(self, logits, first, again, u_first, u_again, token_ids, semantic_begin, semantic_end, window,
                    hist=None, hist_off=None, out_ids=None, out_status=None, stream=None):
        import torch
        rows, vocab = logits.shape
        dtype = BF16 if logits.dtype == torch.bfloat16 else F32
        ld = logits.stride(0) if rows > 1 else vocab
        if out_ids is None:
            out_ids = torch.empty(rows, dtype=torch.int32, device=logits.device)
        if out_status is None:
            out_status = torch.empty(rows, dtype=torch.int32, device=logits.device)
        s = stream if stream is not None else torch.cuda.current_stream(logits.device).cuda_stream
        self._check(self.lib.spx_drama3_main(self.handle, _ptr(logits), dtype, rows, vocab, ld, _ptr(first),
                                             _ptr(again), _ptr(u_first), _ptr(u_again), _ptr(token_ids),
                                             semantic_begin, semantic_end, window, _ptr(hist), _ptr(hist_off),
                                             _ptr(out_ids), _ptr(out_status), ctypes.c_void_p(s)))
        return out_ids, out_status

    def head_argmax(self, hidden, norm_weight, eps, head, out_ids=None, out_max=None, stream=None):
        """The fused LM-head pick: hidden (rows x d float32), norm_weight (d float32 or None), head (vocab x d
        bfloat16, device tensors). Returns (ids, max logits)."""
        import torch
        rows, d = hidden.shape
        vocab = head.shape[0]
        dev = hidden.device
        if out_ids is None:
            out_ids = torch.empty(rows, dtype=torch.int32, device=dev)
        if out_max is None:
            out_max = torch.empty(rows, dtype=torch.float32, device=dev)
        s = stream if stream is not None else torch.cuda.current_stream(dev).cuda_stream
        self._check(self.lib.spx_head_argmax_rows(self.handle, _ptr(hidden), hidden.stride(0), _ptr(norm_weight), eps,
                                                  _ptr(head), head.stride(0), rows, d, vocab, _ptr(out_ids),
                                                  _ptr(out_max), ctypes.c_void_p(s)))
        return out_ids, out_max

    def last_stats(self):
        st = SpxStats()
        self._check(self.lib.spx_sampler_last_stats(self.handle, ctypes.byref(st)))
        return st


def talker_bans(vocab, suppressed_tokens, end_of_speech, frames, min_frames, device="cuda", stream=None):
    """The talker's suppress mask (Generation::banned) built on the device, as int32 words."""
    import torch
    lib = load_library()
    words = torch.empty((vocab + 31) // 32, dtype=torch.int32, device=device)
    s = stream if stream is not None else torch.cuda.current_stream(words.device).cuda_stream
    st = lib.spx_talker_bans(_ptr(words), vocab, suppressed_tokens, end_of_speech, frames, min_frames,
                             ctypes.c_void_p(s))
    if st != 0:
        raise SamplerError(f"spx status {st}: {lib.spx_last_error().decode()}")
    return words


def device_params(params, device="cuda"):
    """spx_row_params records (a numpy array of ROW_PARAMS) as a device tensor."""
    import torch
    return torch.from_numpy(np.ascontiguousarray(params).view(np.int32)).to(device)


def pack_bans(banned_ids_per_row, vocab):
    """Suppress masks (uint32 words, bit i%32 of word i/32) from lists of banned ids; one row per list."""
    words = (vocab + 31) // 32
    out = np.zeros((len(banned_ids_per_row), words), dtype=np.uint32)
    for r, ids in enumerate(banned_ids_per_row):
        ids = np.asarray(ids, dtype=np.int64)
        ids = ids[(ids >= 0) & (ids < vocab)]
        np.bitwise_or.at(out[r], ids >> 5, (np.uint32(1) << (ids & 31).astype(np.uint32)))
    return out


class DryStates:
    """The DRY states of `rows` text streams on the device (Haru's Dry per stream): histories of `hist_stride` ids and
    their lengths, the config and the exempt ids (pad, eop, eos in the reference)."""

    def __init__(self, rows, config, exempt, hist_stride=None, device="cuda"):
        import torch
        self.lib = load_library()
        self.config = config
        self.exempt = np.ascontiguousarray(exempt, dtype=np.int32)
        self.stride = hist_stride or (config.lookback + config.max_match_length + 1)
        self.rows = rows
        self.hist = torch.zeros((rows, self.stride), dtype=torch.int32, device=device)
        self.len = torch.zeros(rows, dtype=torch.int32, device=device)

    def _check(self, status):
        if status != 0:
            raise SamplerError(f"spx status {status}: {self.lib.spx_last_error().decode()}")

    def update(self, tokens, stream=None):
        """Dry::update of every stream with its drawn token (an int32 device tensor of rows)."""
        import torch
        s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
        self._check(self.lib.spx_dry_update_rows(self.rows, ctypes.byref(self.config),
                                                 self.exempt.ctypes.data_as(ctypes.c_void_p), len(self.exempt),
                                                 _ptr(tokens), _ptr(self.hist), _ptr(self.len), self.stride,
                                                 ctypes.c_void_p(s)))

    def shape(self, logits, silent, pad, eop, eos, eop_bias=0.0, must_speak=None, pen_cap=0, stream=None):
        """shape_logits of every row of `logits` (rows x vocab float32, in place) with its stream's penalties; returns
        (penalty tokens, penalties, counts) when pen_cap > 0."""
        import torch
        rows, vocab = logits.shape
        s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
        toks = pens = n = None
        if pen_cap:
            toks = torch.full((rows, pen_cap), -1, dtype=torch.int32, device=logits.device)
            pens = torch.zeros((rows, pen_cap), dtype=torch.float64, device=logits.device)
            n = torch.zeros(rows, dtype=torch.int32, device=logits.device)
        self._check(self.lib.spx_haru_shape_rows(
            _ptr(logits), rows, vocab, logits.stride(0), ctypes.byref(self.config),
            self.exempt.ctypes.data_as(ctypes.c_void_p), len(self.exempt), _ptr(self.hist), _ptr(self.len),
            self.stride, _ptr(silent), pad, eop, eos, eop_bias, _ptr(must_speak), _ptr(toks), _ptr(pens), _ptr(n),
            pen_cap, ctypes.c_void_p(s)))
        return toks, pens, n
