"""Seeded synthetic inputs of the sampler's five workloads, shared by the tests and bench.py.

Every array is made on the host with numpy from a seed, so the device and the oracle see the same values. The
uniforms are uniform() of src/common/sampling.cpp:5-7 over std::mt19937_64(seed), computed by MT64 below (the published
MT19937-64 of Matsumoto and Nishimura, 2004), one per drawing row in row order.

The workloads (sizes at rows=None):
  talker     Qwen3-TTS talker step: 1 x 3072 fp32 ~N(0, 2^2) with 8 logits at exactly +8; repetition 1.05 over 128 ids
             uniform in [0, 3072); temperature 0.9, top-k 50, top-p 1
  predictor  Qwen3-TTS code-predictor batch: 480 x 2048 fp32 ~N(0, 2.5^2); 64 history ids per row; repetition 1.05,
             temperature 0.9, top-k 50
  asr        Qwen3-ASR greedy: 64 x 151936 fp32, logit of rank r = -1.1 ln r + N(0, 0.3^2), ids permuted per row; 300
             banned ids shared by every row; argmax
  haru       Haru-4B text sampling: 256 x 151936 fp32, the same profile; 1024 history ids per row (half drawn from the
             row's 2000 likeliest ids, half uniform); repetition 1.1, presence 0.5; temperature 0.7, top-k off, top-p 0.9
  mixed      2048 x 151936 bf16, the same profile; per row temperature U[0.5, 1.2], top-k in {0, 20, 50, 200}, top-p
             U[0.8, 1.0], history length U[0, 2048], 1% greedy; repetition 1.05, presence 0
"""

import numpy as np

import importlib.util
import os

_spec = importlib.util.spec_from_file_location(
    "speech_cpp_amd", os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "speech.cpp_amd",
                                   "__init__.py"))


def spx_module():
    """The sampler's Python binding (the package directory speech.cpp_amd/ is not an importable name)."""
    import sys
    if "speech_cpp_amd" in sys.modules:
        return sys.modules["speech_cpp_amd"]
    mod = importlib.util.module_from_spec(_spec)
    sys.modules["speech_cpp_amd"] = mod
    _spec.loader.exec_module(mod)
    return mod


class MT64:
    """MT19937-64 (Matsumoto and Nishimura), the generator behind std::mt19937_64."""
    N, M = 312, 156
    MATRIX_A = 0xB5026F5AA96619E9
    UPPER, LOWER = 0xFFFFFFFF80000000, 0x7FFFFFFF
    MASK = (1 << 64) - 1

    def __init__(self, seed=5489):
        self.mt = [0] * self.N
        self.mt[0] = seed & self.MASK
        for i in range(1, self.N):
            self.mt[i] = (6364136223846793005 * (self.mt[i - 1] ^ (self.mt[i - 1] >> 62)) + i) & self.MASK
        self.i = self.N

    def _twist(self):
        mt = self.mt
        for k in range(self.N):
            x = (mt[k] & self.UPPER) | (mt[(k + 1) % self.N] & self.LOWER)
            y = x >> 1
            if x & 1:
                y ^= self.MATRIX_A
            mt[k] = mt[(k + self.M) % self.N] ^ y
        self.i = 0

    def next(self):
        if self.i >= self.N:
            self._twist()
        x = self.mt[self.i]
        self.i += 1
        x ^= (x >> 29) & 0x5555555555555555
        x ^= (x << 17) & 0x71D67FFFEDA60000
        x ^= (x << 37) & 0xFFF7EEE000000000
        x ^= x >> 43
        return x & self.MASK

    def uniform(self):
        """(double) rng() * 2^-64, as src/common/sampling.cpp:5-7: the conversion of the 64-bit integer to double
        rounds to nearest, so the largest draws give exactly 1."""
        return float(self.next()) * 2.0 ** -64


def uniforms(seed, n):
    rng = MT64(seed)
    return np.array([rng.uniform() for _ in range(n)], dtype=np.float64)


def to_bf16_bits(x):
    """float32 -> bfloat16 bits, round to nearest even."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_bits_to_f32(h):
    return (h.astype(np.uint32) << 16).view(np.float32)


def zipf_logits(rng, rows, vocab, noise=0.3, slope=1.1):
    base = (-slope * np.log(np.arange(1, vocab + 1, dtype=np.float64))).astype(np.float32)
    out = np.empty((rows, vocab), dtype=np.float32)
    for r in range(rows):
        perm = rng.permutation(vocab)
        out[r, perm] = base + rng.normal(0.0, noise, vocab).astype(np.float32)
    return out


def csr(hists):
    off = np.zeros(len(hists) + 1, dtype=np.int32)
    off[1:] = np.cumsum([len(h) for h in hists])
    flat = np.concatenate([np.asarray(h, dtype=np.int32) for h in hists]) if hists else np.zeros(0, np.int32)
    return flat.astype(np.int32), off


class Workload(dict):
    """A batch: logits (float32, or uint16 bfloat16 bits with dtype 'bf16'), params, u, hist, hist_off, banned."""

    @property
    def rows(self):
        return self["logits"].shape[0]

    @property
    def vocab(self):
        return self["logits"].shape[1]

    def logits_f32(self):
        return bf16_bits_to_f32(self["logits"]) if self["dtype"] == "bf16" else self["logits"]

    def row_f32(self, r):
        """Row r's logits as float32 (bfloat16 rows widened alone, not the whole batch)."""
        return bf16_bits_to_f32(self["logits"][r]) if self["dtype"] == "bf16" else self["logits"][r]


def make(name, rows=None, seed=1234):
    spx = spx_module()
    rng = np.random.default_rng(seed)
    banned, hist, hist_off = None, None, None
    if name == "talker":
        rows = rows or 1
        vocab = 3072
        logits = rng.normal(0.0, 2.0, (rows, vocab)).astype(np.float32)
        for r in range(rows):
            logits[r, rng.choice(vocab, 8, replace=False)] = 8.0
        hist, hist_off = csr([rng.integers(0, vocab, 128) for _ in range(rows)])
        params = spx.row_params(rows, spx.TRANSFORMERS, temperature=0.9, top_k=50, top_p=1.0, repetition_penalty=1.05)
        dtype = "f32"
    elif name == "predictor":
        rows = rows or 480
        vocab = 2048
        logits = rng.normal(0.0, 2.5, (rows, vocab)).astype(np.float32)
        hist, hist_off = csr([rng.integers(0, vocab, 64) for _ in range(rows)])
        params = spx.row_params(rows, spx.TRANSFORMERS, temperature=0.9, top_k=50, top_p=1.0, repetition_penalty=1.05)
        dtype = "f32"
    elif name == "asr":
        rows = rows or 64
        vocab = 151936
        logits = zipf_logits(rng, rows, vocab)
        banned = spx.pack_bans([rng.choice(vocab, 300, replace=False)], vocab)
        params = spx.row_params(rows, spx.TRANSFORMERS, greedy=True)
        dtype = "f32"
    elif name == "haru":
        rows = rows or 256
        vocab = 151936
        logits = zipf_logits(rng, rows, vocab)
        hists = []
        for r in range(rows):
            likely = np.argsort(-logits[r])[:2000]
            hists.append(np.concatenate([rng.choice(likely, 512), rng.integers(0, vocab, 512)]))
        hist, hist_off = csr(hists)
        params = spx.row_params(rows, spx.TRANSFORMERS, temperature=0.7, top_k=0, top_p=0.9, repetition_penalty=1.1,
                                presence_penalty=0.5)
        dtype = "f32"
    elif name == "haru-flavor":
        # Haru's own rules at its file's defaults (haru::Sampling: T 0.7, top-k 25, top-p 1), no penalties (its DRY
        # shapes the logits before the draw)
        rows = rows or 256
        vocab = 151936
        logits = zipf_logits(rng, rows, vocab)
        params = spx.row_params(rows, spx.HARU, temperature=0.7, top_k=25, top_p=1.0)
        dtype = "f32"
    elif name == "mixed":
        rows = rows or 2048
        vocab = 151936
        logits = to_bf16_bits(zipf_logits(rng, rows, vocab))
        hists = []
        for r in range(rows):
            n = int(rng.integers(0, 2049))
            hists.append(rng.integers(0, vocab, n))
        hist, hist_off = csr(hists)
        greedy = rng.random(rows) < 0.01
        params = spx.row_params(rows, spx.TRANSFORMERS, greedy=greedy,
                                temperature=rng.uniform(0.5, 1.2, rows).astype(np.float32),
                                top_k=rng.choice([0, 20, 50, 200], rows), top_p=rng.uniform(0.8, 1.0, rows).astype(np.float32),
                                repetition_penalty=1.05)
        dtype = "bf16"
    else:
        raise ValueError(name)
    u = np.zeros(rows, dtype=np.float64)
    drawing = np.nonzero(params["greedy"] == 0)[0]
    u[drawing] = uniforms(seed, len(drawing))
    return Workload(name=name, logits=logits, dtype=dtype, params=params, u=u, hist=hist, hist_off=hist_off,
                    banned=banned, banned_stride=0)


NAMES = ["talker", "predictor", "asr", "haru", "mixed"]

# Bytes the sampler must move per row, the algorithmic traffic of the roofline: the logits once, the history ids,
# the uniform, the parameters and the id written.
def algorithmic_bytes(w):
    esz = 2 if w["dtype"] == "bf16" else 4
    hist = int(w["hist_off"][-1]) * 4 if w["hist"] is not None else 0
    banned = w["banned"].nbytes if w["banned"] is not None else 0
    return w.rows * w.vocab * esz + hist + banned + w.rows * (8 + 32 + 4)
