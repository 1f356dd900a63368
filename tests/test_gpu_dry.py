"""Haru's DRY and shape_logits on the device (spx_dry_update_rows, spx_haru_shape_rows) against the oracle: 64 text
streams whose states stay on the device, updated with each frame's drawn token, and their logits shaped at several
frames; the shaped logits and the penalty lists must be the oracle's bit for bit (the penalty of each match length is
the host's std::pow, as the reference computes it)."""

import numpy as np
import pytest

import oracle_lib
import workloads

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("allowed,lookback,max_match", [(2, 64, 8), (1, 16, 3), (3, 256, 200)])
def test_dry_states_and_shaped_logits(allowed, lookback, max_match):
    import torch
    spx = workloads.spx_module()
    rows, vocab, frames = 64, 4096, 160
    pad, eop, eos = 4093, 4094, 4095
    config = spx.DryConfig(0.8, 1.75, 3.0, allowed, lookback, max_match, 0)
    states = spx.DryStates(rows, config, [pad, eop, eos])
    rng = np.random.default_rng(allowed * 1000 + lookback)
    # small alphabets per stream make repeats; the silent ids and the ends of the vocabulary now and then
    alphabet = [rng.choice(np.r_[np.arange(8 + r % 5), [pad, eop, eos, vocab - 4]], 12) for r in range(rows)]
    seqs = np.stack([rng.choice(alphabet[r], frames) for r in range(rows)]).astype(np.int32)
    print("config", allowed, lookback, max_match, flush=True)
    penalized = 0
    for f in range(frames):
        if f % 23 == 5 or f == frames - 1:
            logits = rng.normal(0, 2, (rows, vocab)).astype(np.float32)
            silent = rng.normal(0, 2, (rows, 2)).astype(np.float32)
            speak = (rng.random(rows) < 0.2).astype(np.uint8)
            d_logits = torch.from_numpy(logits).cuda()
            cap = lookback + max_match + 1
            toks, pens, n = states.shape(d_logits, torch.from_numpy(silent).cuda(), pad, eop, eos, eop_bias=0.5,
                                         must_speak=torch.from_numpy(speak).cuda(), pen_cap=cap)
            torch.cuda.synchronize()
            got = d_logits.cpu().numpy()
            toks, pens, n = toks.cpu().numpy(), pens.cpu().numpy(), n.cpu().numpy()
            penalized += int((n > 0).sum())
            for r in range(rows):
                _, ot, op = oracle_lib.dry_run(config, [pad, eop, eos], seqs[r, :f])
                assert n[r] == len(ot), (f, r)
                np.testing.assert_array_equal(toks[r, :len(ot)], ot)
                np.testing.assert_array_equal(pens[r, :len(ot)].view(np.int64), op.view(np.int64))
                want = oracle_lib.haru_shape(logits[r], ot, op, silent[r], pad, eop, eos, 0.5, bool(speak[r]))
                np.testing.assert_array_equal(got[r].view(np.int32), want.view(np.int32))
        states.update(torch.from_numpy(seqs[:, f].copy()).cuda())
    torch.cuda.synchronize()
    assert penalized > rows  # the rule was exercised
    # the device's histories are the oracle's windows
    h, ln = states.hist.cpu().numpy(), states.len.cpu().numpy()
    for r in range(rows):
        oh, _, _ = oracle_lib.dry_run(config, [pad, eop, eos], seqs[r])
        assert ln[r] == len(oh)
        np.testing.assert_array_equal(h[r, :ln[r]], oh)
