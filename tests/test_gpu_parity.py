"""Parity of the HIP sampler with the oracle, through the C ABI, on the five workloads and on the edge cases the
reference's checks exercise (checks/qwen3-tts/qwen3-tts-sampler-check.cpp, qwen3-tts-graph-sampler-check.cpp,
checks/haru/haru-sampling-check.cpp, checks/drama3/drama3-sampler-check.cpp)."""

import numpy as np
import pytest

import gpu_harness
import oracle_lib
import workloads

pytestmark = pytest.mark.gpu

MAX_OUT = 64


@pytest.fixture(scope="module")
def sampler():
    spx = workloads.spx_module()
    return spx.Sampler(max_rows=2048, max_vocab=151936, max_hist=2048, max_out=MAX_OUT)


# Rows a test may excuse for lying within 1e-6 of a boundary or of the top-p decision: such rows are rare (about 2e-6
# of the draws), so more than one in a test means an error of the device larger than the excuse.
NEAR_BUDGET = 1


def check(sampler, w, allow_explained=True):
    cap = sampler.max_out  # the candidate outputs are rows x the handle's max_out
    reports, cids, cweights = oracle_lib.sample_rows(w, cap=cap)
    print(w["name"], w.rows, "x", w.vocab, "oracle done", flush=True)
    gpu = gpu_harness.run_gpu(sampler, w, max_out=cap)
    counts, bad = gpu_harness.compare(w, gpu, reports, cids, cweights)
    print(w["name"], counts, bad[:5], flush=True)
    assert not bad, f"{len(bad)} unexplained rows, first: {bad[:5]}"
    assert counts["boundary"] + counts["cut"] <= NEAR_BUDGET, counts
    if not allow_explained:
        assert counts["tie"] + counts["boundary"] + counts["cut"] == 0
    return counts, gpu, reports


@pytest.mark.parametrize("name,rows", [("talker", 64), ("predictor", 480), ("asr", 64), ("haru", 32), ("mixed", 96)])
def test_workload_parity(sampler, name, rows):
    w = workloads.make(name, rows=rows, seed=7)
    counts, gpu, _ = check(sampler, w)
    # Explained differences are counted, not hidden: ties dominate the talker rows, whose 8 largest logits are equal.
    assert counts["same"] + counts["tie"] >= 0.95 * w.rows


def test_mixed_full_batch(sampler):
    # The heterogeneous batch at its own launch shape: 2048 x 151936 bf16, one row per work-group, the rows whose
    # top-p set runs past the buffer resolved by the wide path; every row against the oracle.
    w = workloads.make("mixed", seed=1234)
    print("mixed batch made", flush=True)
    counts, _, _ = check(sampler, w)
    assert counts["same"] + counts["tie"] == w.rows - counts["boundary"] - counts["cut"]


def test_talker_spikes_are_ties(sampler):
    # Eight logits at exactly +8: the reference's order among them is libstdc++'s heap order, a pick between them is
    # an explained tie (checks/qwen3-tts/qwen3-tts-graph-sampler-check.cpp:124-125).
    w = workloads.make("talker", rows=256, seed=11)
    check(sampler, w)


def test_haru_full_rows(sampler):
    w = workloads.make("haru", rows=256, seed=3)
    counts, gpu, reports = check(sampler, w)
    assert counts["same"] >= 250


def test_argmax_rows_banned(sampler):
    import torch
    spx = workloads.spx_module()
    w = workloads.make("asr", rows=64, seed=5)
    d = gpu_harness.to_device(w)
    ids = sampler.argmax_rows(d["logits"], banned=d["banned"], banned_stride=0)
    torch.cuda.synchronize()
    logits = w["logits"].copy()
    words = w["banned"][0]
    i = np.arange(w.vocab)
    mask = ((words[i >> 5] >> (i & 31).astype(np.uint32)) & 1).astype(bool)
    logits[:, mask] = -np.inf
    assert np.array_equal(ids.cpu().numpy(), np.argmax(logits, axis=1))


def _one(params_kw, logits, hist=None, banned_ids=None, u=0.5, dtype="f32"):
    spx = workloads.spx_module()
    logits = np.atleast_2d(np.asarray(logits, dtype=np.float32))
    rows, vocab = logits.shape
    p = spx.row_params(rows, **params_kw)
    h, off = (None, None)
    if hist is not None:
        h, off = workloads.csr([hist] * rows)
    banned = spx.pack_bans([banned_ids] * 1, vocab) if banned_ids is not None else None
    if dtype == "bf16":
        logits = workloads.to_bf16_bits(logits)
    return workloads.Workload(name="edge", logits=logits, dtype=dtype, params=p, u=np.full(rows, u), hist=h,
                              hist_off=off, banned=banned, banned_stride=0)


EDGE = [
    ("penalty 1e-40 greedy", dict(greedy=True, repetition_penalty=1e-40), [1.0, 2.0], [0, 1]),
    ("penalty 1e-40 draw", dict(repetition_penalty=1e-40), [1.0, 2.0], [0, 1]),
    ("temperature 1e-38", dict(temperature=1e-38, top_k=50), np.linspace(-3, 10, 300), None),
    ("all equal", dict(temperature=0.8, top_k=0, top_p=0.9), np.zeros(1000), None),
    ("all equal top-k", dict(temperature=0.8, top_k=7), np.zeros(1000), None),
    ("single token", dict(temperature=0.8), [0.3], None),
    ("two tokens", dict(temperature=0.8, top_p=0.5), [0.3, 0.1], None),
    ("vocab 5", dict(temperature=1.0, top_k=3), [0.1, 0.5, -1.0, 2.0, 0.7], None),
    ("nan first", dict(greedy=True), [np.nan, 1.0, 2.0], None),
    ("nan later greedy", dict(greedy=True), [1.0, np.nan, 2.0, 2.0], None),
    ("nan later draw", dict(temperature=1.0), [1.0, np.nan, 2.0], None),
    ("+inf", dict(temperature=1.0), [1.0, np.inf, 2.0], None),
    ("+inf penalty", dict(temperature=1.0, repetition_penalty=1.1), [1.0, np.inf, 2.0], [2]),
    ("-inf all", dict(temperature=1.0), [-np.inf] * 10, None),
    ("haru all -inf", dict(flavor=1, temperature=0.7, top_k=3), [-np.inf] * 10, None),
    ("haru nan", dict(flavor=1, temperature=0.7), [1.0, np.nan], None),
    ("haru -inf ok", dict(flavor=1, temperature=0.7, top_k=0), [1.0, -np.inf, 0.5], None),
    ("haru greedy T0", dict(flavor=1, temperature=0.0), [1.0, 3.0, 3.0], None),
    ("haru tiny T", dict(flavor=1, temperature=1e-38, top_k=5), [1.0, 2.0, -3.0], None),
    ("fish -inf", dict(flavor=2, temperature=1.0, top_k=3), [1.0, -np.inf, 0.5], None),
    ("fish T0", dict(flavor=2, temperature=0.0, top_k=3, top_p=0.9), [1.0, 1.0 + 1e-6, 0.5], None),
    ("fish top-k 0", dict(flavor=2, temperature=1.0, top_k=0, top_p=0.9), np.linspace(0, 1, 64), None),
    ("negative logits penalty", dict(temperature=1.0, repetition_penalty=1.3), [-1.0, -2.0, 0.5, 3.0], [0, 0, 1, 3, 9, -4]),
    ("presence frequency", dict(temperature=1.0, presence_penalty=0.5, frequency_penalty=0.25), [1.0, 2.0, 3.0, 0.0],
     [2, 2, 2, 1]),
    ("top-p 0", dict(temperature=0.9, top_p=0.0), np.linspace(-1, 1, 50), None),
    ("top-k beyond vocab", dict(temperature=1.1, top_k=5000), np.random.default_rng(0).normal(0, 2, 2048), None),
    ("top-k 300 fallback", dict(temperature=1.0, top_k=300), np.random.default_rng(1).normal(0, 1, 4096), None),
    ("haru top-k 1000", dict(flavor=1, temperature=1.2, top_k=1000, top_p=0.9), np.random.default_rng(2).normal(0, 2, 8192), None),
    ("wide top-p fallback", dict(temperature=2.5, top_k=0, top_p=0.99), np.random.default_rng(3).normal(0, 2, 3072), None),
    ("full draw fallback", dict(temperature=3.0, top_k=0, top_p=1.0), np.random.default_rng(4).normal(0, 1, 20000), None),
    ("haru ties", dict(flavor=1, temperature=1.0, top_k=0, top_p=1.0), [1.0, 3.0, 3.0, 2.0, 3.0], None),
    ("haru ties top-p", dict(flavor=1, temperature=1.0, top_k=4, top_p=0.5), [1.0, 3.0, 3.0, 2.0, 3.0], None),
    ("fish ties", dict(flavor=2, temperature=1.0, top_k=5, top_p=1.0), [1.0, 3.0, 3.0, 2.0, 3.0], None),
    ("greedy ties", dict(greedy=True), [2.0, 2.0], None),
    ("haru greedy ties", dict(flavor=1, temperature=0.0), [2.0, 2.0, 1.0], None),
    ("fish greedy ties", dict(flavor=2, greedy=True), [1.0, 2.0, 2.0], None),
    # one token reaches top_p under a top-k the buffer does not hold: Haru's pick() still runs over all k weights
    ("haru one token past top-p, top-k 1000", dict(flavor=1, temperature=1.0, top_k=1000, top_p=0.5),
     np.concatenate([[12.0], np.random.default_rng(5).normal(0, 1, 4095)]), None),
    ("transformers one token past top-p, top-k 1000", dict(temperature=1.0, top_k=1000, top_p=0.5),
     np.concatenate([[12.0], np.random.default_rng(5).normal(0, 1, 4095)]), None),
    ("fish top-k 1000", dict(flavor=2, temperature=1.3, top_k=1000, top_p=0.95),
     np.random.default_rng(6).normal(0, 1, 4097), None),
    ("invalid flavor", dict(flavor=7), [1.0, 2.0], None),
    ("invalid temperature", dict(temperature=0.0), [1.0, 2.0], None),
]


@pytest.mark.parametrize("name,kw,logits,hist", EDGE, ids=[e[0] for e in EDGE])
@pytest.mark.parametrize("u", [0.0, 0.37, 0.999, 1.0])
def test_edge(sampler, name, kw, logits, hist, u):
    w = _one(kw, logits, hist=hist, u=u)
    check(sampler, w)


def test_banned_per_row_bf16(sampler):
    spx = workloads.spx_module()
    rng = np.random.default_rng(9)
    rows, vocab = 16, 5003  # a vocabulary that leaves the rows unaligned
    logits = rng.normal(0, 2, (rows, vocab)).astype(np.float32)
    banned = spx.pack_bans([rng.choice(vocab, 40 + r, replace=False) for r in range(rows)], vocab)
    p = spx.row_params(rows, temperature=0.8, top_k=np.array([0, 5, 50, 0] * 4), top_p=0.95)
    w = workloads.Workload(name="bans", logits=workloads.to_bf16_bits(logits), dtype="bf16", params=p,
                           u=workloads.uniforms(5, rows), hist=None, hist_off=None, banned=banned,
                           banned_stride=banned.shape[1])
    check(sampler, w)


def test_flavors_mixed_batch(sampler):
    spx = workloads.spx_module()
    rng = np.random.default_rng(12)
    rows, vocab = 60, 4097  # Drama 3's main-token vocabulary
    logits = rng.normal(0, 3, (rows, vocab)).astype(np.float32)
    flavor = np.array([0, 1, 2] * 20)
    p = spx.row_params(rows, flavor=flavor, temperature=rng.uniform(0.3, 1.5, rows).astype(np.float32),
                       top_k=rng.choice([0, 1, 25, 30, 200], rows), top_p=rng.uniform(0.5, 1.0, rows).astype(np.float32))
    hist, off = workloads.csr([rng.integers(-5, vocab + 5, 40) for _ in range(rows)])
    p["repetition_penalty"][flavor == 0] = 1.2
    w = workloads.Workload(name="flavors", logits=logits, dtype="f32", params=p, u=workloads.uniforms(8, rows),
                           hist=hist, hist_off=off, banned=None, banned_stride=0)
    check(sampler, w)


def test_merge_of_three_chunks_with_wide_top_k(sampler):
    # 4 rows of 16000 tokens are cut into 3 chunks each; with top-k 256 (and 0) every chunk publishes up to 256
    # candidates, which the row's last chunk merges and sorts.
    spx = workloads.spx_module()
    rng = np.random.default_rng(14)
    rows, vocab = 4, 16000
    logits = rng.normal(0, 1, (rows, vocab)).astype(np.float32)
    p = spx.row_params(rows, temperature=1.0, top_k=np.array([256, 256, 0, 200]), top_p=np.array([1.0, 0.9, 0.5, 1.0]))
    w = workloads.Workload(name="merge3", logits=logits, dtype="f32", params=p, u=workloads.uniforms(15, rows),
                           hist=None, hist_off=None, banned=None, banned_stride=0)
    check(sampler, w)


def test_heavy_ban_leaves_few_tokens_across_the_vocabulary(sampler):
    # A mask that leaves about 400 tokens spread over 151936: the row is cut into chunks each holding every live
    # token, more of them together than the finishing wave takes.
    spx = workloads.spx_module()
    rng = np.random.default_rng(16)
    rows, vocab = 4, 151936
    logits = rng.normal(0, 1, (rows, vocab)).astype(np.float32)
    live = rng.choice(vocab, 400, replace=False)
    ban = np.setdiff1d(np.arange(vocab), live)
    banned = spx.pack_bans([ban], vocab)
    p = spx.row_params(rows, temperature=1.0, top_k=0, top_p=np.array([1.0, 0.99, 0.5, 1.0]))
    w = workloads.Workload(name="heavy ban", logits=logits, dtype="f32", params=p, u=workloads.uniforms(17, rows),
                           hist=None, hist_off=None, banned=banned, banned_stride=0)
    check(sampler, w)


def test_bf16_runs_of_equal_logits(sampler):
    # bfloat16 logits of a narrow spread take few distinct values, in runs of thousands of equal tokens: the top-p cut
    # and the pick land inside such runs, whose order is by id (the lower id first) for Haru and Drama 3.
    spx = workloads.spx_module()
    rng = np.random.default_rng(33)
    rows, vocab = 6, 151936
    logits = workloads.to_bf16_bits(rng.normal(0, 0.5, (rows, vocab)).astype(np.float32))
    flavor = np.array([0, 1, 2, 0, 1, 2])
    p = spx.row_params(rows, flavor=flavor, temperature=1.0, top_k=np.array([0, 0, 100000, 70000, 0, 5000]),
                       top_p=np.array([0.95, 0.5, 0.9, 1.0, 1.0, 0.8], dtype=np.float32))
    w = workloads.Workload(name="bf16 runs", logits=logits, dtype="bf16", params=p, u=workloads.uniforms(35, rows),
                           hist=None, hist_off=None, banned=None, banned_stride=0)
    check(sampler, w)


@pytest.mark.parametrize("run", [6000, 20000])
def test_runs_longer_than_a_read(sampler, run):
    # A run of equal bfloat16 logits longer than a gathering read takes, with the top-p cut and the pick inside it:
    # up to twice that length the run's ids are gathered in one read, beyond it an id range is counted first. FISH and
    # Haru order a run by id, so the token at each place is exact. Haru's float32 running sums step through a run of
    # any length, but keep its ids only up to twice a read's tokens: a Haru pick or listed candidate inside a longer
    # run takes the radix path, whose Haru weights use the exact sum, so the longer case has Haru rows whose pick and
    # listed candidates lie before the run (u below the top tokens' share).
    spx = workloads.spx_module()
    rng = np.random.default_rng(37 + run)
    rows, vocab = 6, 151936
    x = np.full((rows, vocab), -30.0, dtype=np.float32)
    for r in range(rows):
        pos = rng.permutation(vocab)
        x[r, pos[:1000]] = 2.0
        x[r, pos[1000:1000 + run]] = 0.0
    logits = workloads.to_bf16_bits(x)
    p = spx.row_params(rows, flavor=np.array([2, 2, 2, 1, 1, 0]), temperature=1.0, top_k=0,
                       top_p=np.array([0.9, 0.99, 0.75, 0.9, 1.0, 0.9], dtype=np.float32))
    # u past the 2.0 tokens' share, so that the picks land in the run too (but for the Haru rows of the longer run)
    u = np.array([0.7, 0.95, 0.8, 0.75, 0.9, 0.6])
    if run > 8192:
        u[3:5] = 0.1
    w = workloads.Workload(name=f"run {run}", logits=logits, dtype="bf16", params=p, u=u, hist=None, hist_off=None,
                           banned=None, banned_stride=0)
    check(sampler, w)


def test_repeated_calls_reuse_workspace(sampler):
    # The per-row counters and the fallback list reset themselves: calls in a row give the same answers.
    w = workloads.make("mixed", rows=64, seed=21)
    reports, _, _ = oracle_lib.sample_rows(w)
    d = gpu_harness.to_device(w)
    first = gpu_harness.run_gpu(sampler, w, d)
    for _ in range(3):
        again = gpu_harness.run_gpu(sampler, w, d)
        assert np.array_equal(first["ids"], again["ids"])
        assert np.array_equal(first["status"], again["status"])


def test_empty_batch(sampler):
    import torch
    spx = workloads.spx_module()
    logits = torch.zeros((0, 100), device="cuda")
    p = spx.device_params(spx.row_params(0))
    u = torch.zeros(0, dtype=torch.float64, device="cuda")
    ids, st = sampler.sample_rows(logits, p, u)
    torch.cuda.synchronize()
    assert ids.numel() == 0


def _share_rows(name):
    """One row of a workload shape and its settings, for the draw-share test."""
    spx = workloads.spx_module()
    rng = np.random.default_rng(23)
    if name == "talker":
        logits = rng.normal(0.0, 2.0, 3072).astype(np.float32)
        p = spx.row_params(1, spx.TRANSFORMERS, temperature=0.9, top_k=50, top_p=1.0)
    elif name == "haru-shape":
        logits = workloads.zipf_logits(rng, 1, 151936)[0]
        p = spx.row_params(1, spx.TRANSFORMERS, temperature=0.7, top_k=0, top_p=0.9)
    elif name == "haru-flavor":
        logits = workloads.zipf_logits(rng, 1, 151936)[0]
        p = spx.row_params(1, spx.HARU, temperature=0.7, top_k=25, top_p=0.9)
    else:
        logits = rng.normal(0.0, 2.0, 4097).astype(np.float32)
        p = spx.row_params(1, spx.FISH, temperature=0.8, top_k=30, top_p=0.9)
    return logits, p


@pytest.mark.parametrize("name", ["talker", "haru-shape", "haru-flavor", "fish"])
def test_draws_over_one_row(sampler, name):
    # checks/qwen3-tts/qwen3-tts-graph-sampler-check.cpp:97-160 on the device: one row drawn with 64 numbers, half
    # spread evenly over [0, 1] and half from uniform() of seed 1, each pick against the oracle's; then 25,600 draws
    # from uniform(), whose shares must lie within five standard deviations of the candidates' probabilities, a pick
    # of a token that is no candidate failing however rare.
    import torch
    logits, p = _share_rows(name)
    vocab = len(logits)
    rng = workloads.MT64(1)
    u = np.array([(i + 0.5) / 32 for i in range(32)] + [rng.uniform() for _ in range(32)])
    w = workloads.Workload(name="draws " + name, logits=np.tile(logits, (64, 1)), dtype="f32", params=np.repeat(p, 64),
                           u=u, hist=None, hist_off=None, banned=None, banned_stride=0)
    check(sampler, w)
    # the shares of 25,600 draws
    st, toks, wts = (oracle_lib.tf_candidates(logits, p[0]) if p["flavor"][0] == 0 else
                     oracle_lib.haru_candidates(logits, float(p["temperature"][0]), int(p["top_k"][0]),
                                                float(p["top_p"][0])) if p["flavor"][0] == 1 else
                     oracle_lib.fish_candidates(logits, float(p["temperature"][0]), int(p["top_k"][0]),
                                                float(p["top_p"][0])))
    assert st == 0
    prob = np.zeros(vocab)
    prob[toks] = wts / wts.sum()
    rows = 2048
    spx = workloads.spx_module()
    d_logits = torch.from_numpy(logits).cuda().expand(rows, vocab).contiguous()
    d_params = spx.device_params(np.repeat(p, rows))
    counts = np.zeros(vocab, dtype=np.int64)
    draws = 400 * 64
    done = 0
    while done < draws:
        n = min(rows, draws - done)
        du = torch.from_numpy(np.array([rng.uniform() for _ in range(n)])).cuda()
        ids, status = sampler.sample_rows(d_logits[:n], d_params[:n], du)
        torch.cuda.synchronize()
        assert (status.cpu().numpy() == 0).all()
        counts += np.bincount(ids.cpu().numpy(), minlength=vocab)
        done += n
    share = counts / draws
    assert not np.any((prob == 0) & (counts > 0)), "a token that is no candidate was picked"
    dev = np.abs(share - prob) / (np.sqrt(prob * (1 - prob) / draws) + 1 / draws)
    assert dev.max() <= 5.0, (int(np.argmax(dev)), dev.max())


@pytest.mark.parametrize("vocab", [512, 8192, 151936])
def test_haru_float32_running_sum_on_the_device(sampler, vocab):
    # Rows whose float32 running sum and a double sum put a token on different sides of top_p
    # (src/families/haru/sampler.cpp:54-58): the whole candidate list, zeros included, must be the oracle's, and u
    # aimed inside the flipped token's share must pick it or not as the float32 rule says.
    import torch
    spx = workloads.spx_module()
    rng = np.random.default_rng(vocab)
    rows, ts = [], []
    while len(rows) < 3:
        l = rng.normal(0, 1.5, vocab).astype(np.float32)
        t = oracle_lib.haru_float_flip(l, 1.0)
        if t is not None:
            rows.append(l)
            ts.append(t)
    logits = np.stack(rows)
    p = spx.row_params(3, spx.HARU, temperature=1.0, top_k=0, top_p=np.array(ts, dtype=np.float32))
    d_logits, d_params = torch.from_numpy(logits).cuda(), spx.device_params(p)
    toks, wts, n, status = sampler.candidates_rows(d_logits, d_params, vocab)
    torch.cuda.synchronize()
    toks, wts, n, status = toks.cpu().numpy(), wts.cpu().numpy(), n.cpu().numpy(), status.cpu().numpy()
    us = []
    for r in range(3):
        st, otok, ow = oracle_lib.haru_candidates(logits[r], 1.0, 0, ts[r])
        assert status[r] == st == 0 and n[r] == len(otok) == vocab
        np.testing.assert_array_equal(toks[r], otok)
        np.testing.assert_array_equal(wts[r] == 0, ow == 0)
        np.testing.assert_allclose(wts[r], ow, rtol=1e-6, atol=0)
        # u in the middle of the share the double sum would give the first token the two sums treat differently
        _, _, p1 = oracle_lib.haru_candidates(logits[r], 1.0, 0, 1.0)
        i = int(np.argmax(oracle_lib.haru_zeroing(p1, ts[r]) != oracle_lib.haru_zeroing(p1, ts[r], True)))
        wd = np.where(oracle_lib.haru_zeroing(p1, ts[r], True), 0.0, p1)
        c = np.cumsum(wd) / wd.sum()
        lo = c[i - 1] if i > 0 else 0.0
        us.append(lo + (c[i] - lo) / 2)
    w = workloads.Workload(name="haru float32 sum", logits=logits, dtype="f32", params=p, u=np.array(us), hist=None,
                           hist_off=None, banned=None, banned_stride=0)
    reports, _, _ = oracle_lib.sample_rows(w)
    gpu = gpu_harness.run_gpu(sampler, w)
    for r in range(3):  # no excuse: the decision at top_p is the point of the row
        assert reports[r]["boundary"] > 1e-12, r
        assert (gpu["status"][r], gpu["ids"][r], gpu["kept"][r]) == (0, reports[r]["id"], reports[r]["kept"]), r


def test_transformers_top_p_over_the_top_k_and_fish_floor_on_the_device(sampler):
    # The closed forms the oracle is pinned by, on the device: top-k 2 then top-p 0.55 over weights 0.4, 0.3, 0.2, 0.1
    # keeps one token (normalized over the two kept); Drama 3's temperature floor of 1e-5.
    spx = workloads.spx_module()
    tf_l = np.log(np.array([0.4, 0.3, 0.2, 0.1] * 1)).astype(np.float32)
    for u in (0.0, 0.5, 0.99):
        w = _one(dict(temperature=1.0, top_k=2, top_p=0.55), tf_l, u=u)
        _, gpu, reps = check(sampler, w, allow_explained=False)
        assert gpu["ids"][0] == 0 and gpu["kept"][0] == 1
    fish_l = np.array([0.0, -1e-5, -3e-5], dtype=np.float32)
    for t in (1e-7, 0.0):
        for u in (0.2, 0.8, 0.99):
            w = _one(dict(flavor=spx.FISH, temperature=t, top_k=3, top_p=1.0), fish_l, u=u)
            check(sampler, w, allow_explained=False)


@pytest.mark.parametrize("n_hist", [8192, 16384])
def test_long_histories(sampler, n_hist):
    # Histories of 8192 and 16384 ids (the talker's grows one id per frame without a bound), with repetition, presence
    # and frequency penalties, on both work-group sizes; at 16384 ids the resolving kernel takes its 512-thread layout.
    spx = workloads.spx_module()
    big = spx.Sampler(max_rows=8, max_vocab=151936, max_hist=n_hist, max_out=MAX_OUT)
    rng = np.random.default_rng(29)
    for vocab in (151936, 3072):
        rows = 4
        logits = workloads.zipf_logits(rng, rows, vocab)
        logits[2] = rng.normal(0, 1, vocab)  # a flat row: its top-p set is wider than the sampling kernel holds
        hists = [np.concatenate([np.argsort(-logits[r])[:100].repeat(8), rng.integers(0, vocab, n_hist - 800)])
                 for r in range(rows)]
        hist, off = workloads.csr(hists)
        p = spx.row_params(rows, temperature=0.8, top_k=np.array([0, 50, 0, 300]), top_p=0.9,
                           repetition_penalty=1.1, presence_penalty=0.3,
                           frequency_penalty=np.array([0.0, 0.05, 0.1, 0.0], dtype=np.float32))
        w = workloads.Workload(name=f"hist {n_hist} x {vocab}", logits=logits, dtype="f32", params=p,
                               u=workloads.uniforms(31, rows), hist=hist, hist_off=off, banned=None, banned_stride=0)
        check(big, w)
