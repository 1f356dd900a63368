"""The LM head's pick fused with its product (spx_head_argmax_rows) against the oracle's restatement of
Qwen3Decoder::outputs() with Qwen3Readback::Pick (src/common/qwen3-decoder.cpp:422-429) and verify() (:497-501).

The device sums each logit's d products in float32 on the matrix cores, in an order of its own, as ggml's backends do;
the oracle sums them in double. The bar: the id is the oracle's, or the two ids' logits lie within the float32
summation bound d * 2^-24 * sum |products| of each other (a near tie, counted: at most one row in a hundred); the
returned logit within the same bound of the oracle's logit of the returned id; equal rows of the head pick the lower id
and a NaN hidden state picks id 0, exactly."""

import numpy as np
import pytest

import oracle_lib
import workloads

pytestmark = pytest.mark.gpu


def _run(rows, vocab, d, seed, weight=True, nan_row=None, dup=None):
    import torch
    spx = workloads.spx_module()
    rng = np.random.default_rng(seed)
    hidden = rng.normal(0, 1, (rows, d)).astype(np.float32)
    if nan_row is not None:
        hidden[nan_row, d // 3] = np.nan
    w = rng.uniform(0.5, 1.5, d).astype(np.float32) if weight else None
    head = workloads.to_bf16_bits(rng.normal(0, 0.05, (vocab, d)).astype(np.float32))
    if dup is not None:
        src, dst = dup  # row dst repeats row src, made the largest for every hidden row
        head[src] = workloads.to_bf16_bits((np.sign(hidden.sum(0)) * 0.2).astype(np.float32))[None, :]
        head[dst] = head[src]
    s = spx.Sampler(max_rows=max(rows, 64), max_vocab=16, max_hist=0, max_out=0)
    d_head = torch.from_numpy(head.view(np.int16)).cuda().view(torch.bfloat16)
    ids, mx = s.head_argmax(torch.from_numpy(hidden).cuda(), torch.from_numpy(w).cuda() if weight else None, 1e-6,
                            d_head)
    torch.cuda.synchronize()
    return hidden, w, head, ids.cpu().numpy(), mx.cpu().numpy()


@pytest.mark.parametrize("rows,vocab,d", [(1, 151936, 1024), (7, 1000, 64), (32, 4096, 2048), (33, 5003, 576),
                                          (64, 151936, 1024)])
def test_head_pick_matches_the_oracle(rows, vocab, d):
    print("head", rows, vocab, d, flush=True)
    hidden, w, head, ids, mx = _run(rows, vocab, d, seed=rows * 7 + d)
    want, logits, absum = oracle_lib.head_pick(hidden, w, 1e-6, head)
    near = 0
    for r in range(rows):
        tol = d * 2.0 ** -24 * absum[r]
        g, o = int(ids[r]), int(want[r])
        assert 0 <= g < vocab
        assert abs(float(mx[r]) - logits[r, g]) <= tol[g], (r, mx[r], logits[r, g])
        if g != o:
            assert logits[r, o] - logits[r, g] <= tol[o] + tol[g], (r, g, o)
            near += 1
    assert near <= max(1, rows // 100), near


def test_head_pick_ties_and_nan():
    rows, vocab, d = 8, 3000, 256
    hidden, w, head, ids, _ = _run(rows, vocab, d, seed=5, dup=(1707, 1234))
    assert (ids == 1234).all(), ids  # two equal rows of the head, the largest: the lower id
    hidden, w, head, ids, _ = _run(rows, vocab, d, seed=6, nan_row=3)
    assert ids[3] == 0
    want, _, _ = oracle_lib.head_pick(hidden, w, 1e-6, head)
    assert want[3] == 0
