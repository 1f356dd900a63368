"""The families' device entries against the oracle, through the C ABI: the code predictor's chain of picks kept on the
device (spx_sample_chain), the talker's suppress mask built on the device (spx_talker_bans) and used by a talker
step, and Drama 3's two draws of the main token with the redraw rule (spx_drama3_main)."""

import numpy as np
import pytest

import gpu_harness
import oracle_lib
import workloads

pytestmark = pytest.mark.gpu


def test_chain_of_picks_matches_sequential_samples():
    # 32 streams x 15 codes of 2048 (the code-predictor batch's shape) with repetition 1.05, T 0.9, top-k 50: each
    # pick reads the codes its stream picked before in the frame as the history (src/families/qwen3-tts/
    # synthesizer.cpp:130-139), against 15 sequential oracle samples per stream.
    import torch
    spx = workloads.spx_module()
    rng = np.random.default_rng(41)
    streams, picks, vocab = 32, 15, 2048
    logits = rng.normal(0, 2.5, (picks, streams, vocab)).astype(np.float32)
    for i in range(picks):  # repeated codes make the penalty matter
        logits[i, :, :8] += 6.0
    p = spx.row_params(streams, spx.TRANSFORMERS, temperature=0.9, top_k=50, top_p=1.0, repetition_penalty=1.05)
    p["greedy"][::7] = 1
    gen = workloads.MT64(43)
    u = np.array([[gen.uniform() for _ in range(picks)] for _ in range(streams)])
    s = spx.Sampler(max_rows=streams, max_vocab=vocab, max_hist=picks, max_out=0)
    codes = torch.full((streams, picks + 1), -1, dtype=torch.int32, device="cuda")
    codes[:, 0] = torch.from_numpy(rng.integers(0, 3072, streams).astype(np.int32))
    d_params = spx.device_params(p)
    d_u = torch.from_numpy(u).cuda()
    status = torch.full((streams,), -7, dtype=torch.int32, device="cuda")
    d_logits = torch.from_numpy(logits).cuda()
    for i in range(picks):
        s.sample_chain(d_logits[i], codes, i, d_params, d_u, out_status=status)
        torch.cuda.synchronize()
        assert (status.cpu().numpy() == 0).all()
    got = codes.cpu().numpy()
    want = np.full((streams, picks + 1), -1, dtype=np.int32)
    want[:, 0] = got[:, 0]
    for i in range(picks):
        hist, off = workloads.csr([want[r, 1:i + 1] for r in range(streams)])
        w = workloads.Workload(name="chain", logits=logits[i], dtype="f32", params=p, u=u[:, i].copy(), hist=hist,
                               hist_off=off, banned=None, banned_stride=0)
        reports, _, _ = oracle_lib.sample_rows(w)
        for r in range(streams):
            if reports[r]["id"] != got[r, i + 1]:
                fl = gpu_harness.final_logits_row(w, r)
                # equal final logits may trade places on drawing rows (std::partial_sort without a tie-break)
                assert not p["greedy"][r] and fl[reports[r]["id"]] == fl[got[r, i + 1]], (r, i)
        want[:, i + 1] = got[:, i + 1]  # the next pick's history is the device's picks


def test_talker_mask_on_the_device():
    import torch
    spx = workloads.spx_module()
    for vocab, eos, frames, min_frames in ((3072, 2150, 0, 2), (3072, 2150, 5, 2), (3072, 17, 1, 3), (100, 99, 0, 0)):
        words = spx.talker_bans(vocab, min(1024, vocab), eos, frames, min_frames)
        torch.cuda.synchronize()
        w = words.cpu().numpy().view(np.uint32)
        i = np.arange(vocab)
        bits = ((w[i >> 5] >> (i & 31).astype(np.uint32)) & 1).astype(np.uint8)
        np.testing.assert_array_equal(bits, oracle_lib.talker_bans(vocab, min(1024, vocab), eos, frames, min_frames))


def test_talker_step_with_its_suppress_mask():
    # The talker workload with the talker's real mask (the last 1024 ids banned but the end of speech, which is banned
    # too before min_frames), one mask per row at different frame counts.
    import torch
    spx = workloads.spx_module()
    w = workloads.make("talker", rows=48, seed=45)
    vocab, eos = w.vocab, 2150
    masks = []
    for r in range(w.rows):
        words = spx.talker_bans(vocab, 1024, eos, r % 4, 2)
        torch.cuda.synchronize()
        masks.append(words.cpu().numpy().view(np.uint32))
    w["banned"] = np.stack(masks)
    w["banned_stride"] = w["banned"].shape[1]
    w["logits"][:, eos] = 9.0  # the end of speech likely where it is allowed
    s = spx.Sampler(max_rows=w.rows, max_vocab=vocab, max_hist=2048, max_out=16)
    reports, cids, cw = oracle_lib.sample_rows(w, cap=16)
    gpu = gpu_harness.run_gpu(s, w, max_out=16)
    counts, bad = gpu_harness.compare(w, gpu, reports, cids, cw)
    print(counts, flush=True)
    assert not bad, bad[:5]
    assert counts["boundary"] + counts["cut"] <= 1


def test_drama3_main_tokens():
    # FrameSampler::main over 64 rows of 4097 (Drama 3's main vocabulary): the request's settings, the redraw's, the
    # token map, the semantic range and a window of 16 over each row's history, against the oracle.
    import torch
    spx = workloads.spx_module()
    rng = np.random.default_rng(47)
    rows, vocab, window = 64, 4097, 16
    logits = rng.normal(0, 2, (rows, vocab)).astype(np.float32)
    token_ids = rng.permutation(np.arange(150000, 150000 + vocab)).astype(np.int32)
    sem_lo, sem_hi = 150010, 150000 + vocab - 1
    first = spx.row_params(rows, spx.FISH, temperature=rng.uniform(0.5, 1.2, rows).astype(np.float32), top_k=30,
                           top_p=0.9)
    again = spx.row_params(rows, spx.FISH, temperature=1.0, top_k=50, top_p=0.95)
    u1, u2 = workloads.uniforms(49, rows), workloads.uniforms(51, rows)
    # histories that often hold the first draw: the row's likeliest ids mapped, plus others
    hists = []
    for r in range(rows):
        top = token_ids[np.argsort(-logits[r])[:3]]
        hists.append(np.concatenate([rng.integers(150000, 150000 + vocab, 20), top[: r % 4]]).astype(np.int32))
    hist, off = workloads.csr(hists)
    s = spx.Sampler(max_rows=2 * rows, max_vocab=vocab, max_hist=64, max_out=0)
    ids, status = s.drama3_main(torch.from_numpy(logits).cuda(), spx.device_params(first), spx.device_params(again),
                                torch.from_numpy(u1).cuda(), torch.from_numpy(u2).cuda(),
                                torch.from_numpy(token_ids).cuda(), sem_lo, sem_hi, window,
                                hist=torch.from_numpy(hist).cuda(), hist_off=torch.from_numpy(off).cuda())
    torch.cuda.synchronize()
    ids, status = ids.cpu().numpy(), status.cpu().numpy()
    redrawn = 0
    for r in range(rows):
        st, want = oracle_lib.drama3_main(logits[r], first[r], again[r], u1[r], u2[r], token_ids, sem_lo, sem_hi,
                                          window, hists[r])
        assert (status[r], ids[r]) == (st, want), r
        _, plain = oracle_lib.drama3_main(logits[r], first[r], again[r], u1[r], u2[r], token_ids, sem_lo, sem_hi,
                                          window, None)
        redrawn += int(plain != want)
    assert redrawn > 0  # the rule was exercised


@pytest.mark.parametrize("cap", [100, 4096])
def test_candidate_lists_of_a_mixed_batch(cap):
    # spx_candidates_rows over rows of the three flavors, top-k on and off, wide and narrow top-p: the first `cap`
    # candidates of each row in the reference's order with its weights, and the kept count, against the oracle.
    import torch
    spx = workloads.spx_module()
    rng = np.random.default_rng(cap)
    rows, vocab = 24, 4096
    logits = rng.normal(0, 2, (rows, vocab)).astype(np.float32)
    flavor = np.array([0, 1, 2] * (rows // 3), dtype=np.int32)
    p = spx.row_params(rows, 0, temperature=rng.uniform(0.6, 1.4, rows).astype(np.float32),
                       top_k=rng.choice([0, 40, 300, 5000], rows), top_p=rng.choice([0.5, 0.9, 1.0], rows).astype(np.float32))
    p["flavor"] = flavor
    w = workloads.Workload(name="lists", logits=logits, dtype="f32", params=p, u=np.zeros(rows), hist=None,
                           hist_off=None, banned=None, banned_stride=0)
    reports, cids, cw = oracle_lib.sample_rows(w, cap=cap)
    s = spx.Sampler(max_rows=rows, max_vocab=vocab, max_hist=0, max_out=0)
    toks, wts, n, status = s.candidates_rows(torch.from_numpy(logits).cuda(), spx.device_params(p), cap)
    torch.cuda.synchronize()
    toks, wts, n, status = toks.cpu().numpy(), wts.cpu().numpy(), n.cpu().numpy(), status.cpu().numpy()
    for r in range(rows):
        assert status[r] == reports[r]["status"] == 0, r
        assert n[r] == reports[r]["kept"], (r, n[r], reports[r]["kept"])
        m = min(cap, int(n[r]))
        why = gpu_harness._check_candidates(w, r, toks[r, :m], wts[r, :m], cids[r, :m], cw[r, :m], flavor[r] == 0, None)
        assert why is None, (r, why)
