"""Running the HIP sampler on a tests.workloads.Workload and comparing it with the oracle. Used by the GPU tests,
__graft_entry__.smoke() and bench.py."""

import numpy as np

import workloads

# The north star's bars: a token id may differ only where u lies within 1e-6 of a boundary between two kept
# candidates' cumulative shares, where the top-p rule's decision lies within 1e-6 of top_p, or between candidates of
# equal final logits (whose order the Qwen3-TTS reference leaves to std::partial_sort). Probabilities agree within 1e-5
# relative.
BOUNDARY = 1e-6
PROB_RTOL = 1e-5


def to_device(w, device="cuda"):
    import torch
    spx = workloads.spx_module()
    if w["dtype"] == "bf16":
        logits = torch.from_numpy(w["logits"].view(np.int16)).to(device).view(torch.bfloat16)
    else:
        logits = torch.from_numpy(w["logits"]).to(device)
    d = dict(logits=logits, params=spx.device_params(w["params"], device), u=torch.from_numpy(w["u"]).to(device))
    d["hist"] = torch.from_numpy(w["hist"]).to(device) if w["hist"] is not None else None
    d["hist_off"] = torch.from_numpy(w["hist_off"]).to(device) if w["hist"] is not None else None
    d["banned"] = torch.from_numpy(w["banned"].view(np.int32)).to(device) if w["banned"] is not None else None
    return d


def run_gpu(sampler, w, d=None, max_out=0):
    """The device's ids, statuses, kept counts and candidate outputs for a workload."""
    import torch
    d = d or to_device(w)
    rows = w.rows
    dev = d["logits"].device
    ids = torch.full((rows,), -7, dtype=torch.int32, device=dev)
    status = torch.full((rows,), -7, dtype=torch.int32, device=dev)
    kept = torch.full((rows,), -7, dtype=torch.int32, device=dev)
    cids = torch.full((rows, max_out), -7, dtype=torch.int32, device=dev) if max_out else None
    cprobs = torch.full((rows, max_out), -7.0, dtype=torch.float32, device=dev) if max_out else None
    sampler.sample_rows(d["logits"], d["params"], d["u"], hist=d["hist"], hist_off=d["hist_off"], banned=d["banned"],
                        banned_stride=w["banned_stride"], out_ids=ids, out_status=status, out_kept=kept,
                        out_cand_ids=cids, out_cand_probs=cprobs)
    torch.cuda.synchronize()
    out = dict(ids=ids.cpu().numpy(), status=status.cpu().numpy(), kept=kept.cpu().numpy())
    if max_out:
        out["cand_ids"] = cids.cpu().numpy()
        out["cand_probs"] = cprobs.cpu().numpy()
    return out


def final_logits_row(w, r):
    """The oracle's final logits of row r (after penalties, bans and temperature), for classifying ties."""
    import oracle_lib
    h = None
    if w["hist"] is not None:
        h = w["hist"][w["hist_off"][r]:w["hist_off"][r + 1]]
    b = None
    if w["banned"] is not None:
        words = w["banned"][0 if w["banned_stride"] == 0 else r]
        i = np.arange(w.vocab)
        b = ((words[i >> 5] >> (i & 31).astype(np.uint32)) & 1).astype(np.uint8)
    return oracle_lib.final_logits(w.logits_f32()[r], w["params"][r], h, b)[1]


def compare(w, gpu, reports, cand_ids=None, cand_probs=None):
    """Classifies every row: 'same', or an explained difference ('tie', 'boundary', 'cut'), or 'unexplained'.
    Returns (counts, list of unexplained (row, reason))."""
    counts = dict(same=0, tie=0, boundary=0, cut=0, unexplained=0, prob_checked=0)
    bad = []
    for r in range(w.rows):
        rep = reports[r]
        if gpu["status"][r] != rep["status"]:
            counts["unexplained"] += 1
            bad.append((r, f"status {gpu['status'][r]} vs oracle {rep['status']}"))
            continue
        same_id = gpu["ids"][r] == rep["id"]
        excused = None
        if rep["cut"] < BOUNDARY:
            excused = "cut"
        elif rep["boundary"] < BOUNDARY:
            excused = "boundary"
        if not same_id:
            if excused:
                counts[excused] += 1
                continue
            fl = final_logits_row(w, r)
            if 0 <= gpu["ids"][r] < w.vocab and fl[gpu["ids"][r]] == fl[rep["id"]]:
                counts["tie"] += 1
                continue
            counts["unexplained"] += 1
            bad.append((r, f"id {gpu['ids'][r]} vs oracle {rep['id']} (boundary {rep['boundary']:.3g}, cut {rep['cut']:.3g})"))
            continue
        if rep["status"] == 0 and gpu["kept"][r] != rep["kept"] and not excused:
            counts["unexplained"] += 1
            bad.append((r, f"kept {gpu['kept'][r]} vs oracle {rep['kept']}"))
            continue
        counts["same"] += 1
        if cand_ids is not None and "cand_ids" in gpu and rep["status"] == 0 and not excused:
            g_ids, g_p = gpu["cand_ids"][r], gpu["cand_probs"][r]
            written = g_ids >= 0
            if not written.any():
                continue  # rows the multi-pass path finished report no candidates
            n = min(int(written.sum()), cand_ids.shape[1])
            o_ids, o_p = cand_ids[r, :n], cand_probs[r, :n]
            gi, gp = g_ids[:n], g_p[:n].astype(np.float64)
            if not np.array_equal(np.sort(gi), np.sort(o_ids)):
                # Ties reorder tokens of equal final logits; the lists must then hold the same values, and the
                # probabilities are compared value by value.
                fl = final_logits_row(w, r)
                if not np.array_equal(np.sort(fl[gi]), np.sort(fl[o_ids])):
                    counts["unexplained"] += 1
                    counts["same"] -= 1
                    bad.append((r, "candidate sets differ"))
                    continue
                pairs = zip(np.sort(o_p).tolist(), np.sort(gp).tolist())
            else:
                go = dict(zip(gi.tolist(), gp.tolist()))
                pairs = [(p, go[t]) for t, p in zip(o_ids.tolist(), o_p.tolist())]
            worst = 0.0
            for p, q in pairs:
                worst = max(worst, abs(q - p) / p if p > 1e-12 else abs(q - p))
            counts["prob_checked"] += 1
            if worst > PROB_RTOL:
                counts["unexplained"] += 1
                counts["same"] -= 1
                bad.append((r, f"probability off by {worst:.3g} relative"))
    return counts, bad
