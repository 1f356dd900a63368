"""Running the HIP sampler on a tests.workloads.Workload and comparing it with the oracle. Used by the GPU tests,
__graft_entry__.smoke() and bench.py."""

import numpy as np

import workloads

# The parity bars: a token id may differ only where u lies within 1e-6 of a boundary between two kept candidates'
# cumulative shares, where the top-p rule's decision lies within 1e-6 of top_p, or between candidates of equal final
# logits on the rows whose reference leaves their order to std::partial_sort. Weights agree within 1e-5 relative.
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
    """The device's ids, statuses, kept counts and candidate outputs for a workload (max_out: the handle's)."""
    import torch
    assert not max_out or max_out == sampler.max_out, "candidate outputs are rows x the handle's max_out"
    d = d or to_device(w)
    rows = w.rows
    dev = d["logits"].device
    ids = torch.full((rows,), -7, dtype=torch.int32, device=dev)
    status = torch.full((rows,), -7, dtype=torch.int32, device=dev)
    kept = torch.full((rows,), -7, dtype=torch.int32, device=dev)
    cids = torch.full((rows, max_out), -7, dtype=torch.int32, device=dev) if max_out else None
    cweights = torch.full((rows, max_out), -7.0, dtype=torch.float64, device=dev) if max_out else None
    sampler.sample_rows(d["logits"], d["params"], d["u"], hist=d["hist"], hist_off=d["hist_off"], banned=d["banned"],
                        banned_stride=w["banned_stride"], out_ids=ids, out_status=status, out_kept=kept,
                        out_cand_ids=cids, out_cand_weights=cweights)
    torch.cuda.synchronize()
    out = dict(ids=ids.cpu().numpy(), status=status.cpu().numpy(), kept=kept.cpu().numpy())
    if max_out:
        out["cand_ids"] = cids.cpu().numpy()
        out["cand_weights"] = cweights.cpu().numpy()
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
    return oracle_lib.final_logits(w.row_f32(r), w["params"][r], h, b)[1]


def compare(w, gpu, reports, cand_ids=None, cand_weights=None):
    """Classifies every row: 'same', an excused difference ('boundary', 'cut', 'tie'), or 'unexplained'. Returns
    (counts, list of unexplained (row, reason)).

    A pick may differ where u lies within 1e-6 of a boundary between two kept candidates' cumulative shares
    ('boundary') or where the top-p rule's decision lies within 1e-6 of top_p ('cut'). It may also differ between
    candidates of equal final logits ('tie'), but only on drawing rows of the Qwen3-TTS flavor, whose reference sorts
    with std::partial_sort and no tie-break (src/families/qwen3-tts/sampler.cpp:78-79). Haru and Drama 3 break ties to
    the lower id (src/families/haru/sampler.cpp:39, src/families/drama3/sampler.cpp:43-45) and greedy rows take the
    first maximum (std::max_element): those must match bit for bit. The candidate lists must hold the oracle's ids in
    its order (equal final logits may trade places on the same drawing rows) and weights within 1e-5 relative."""
    counts = dict(same=0, tie=0, boundary=0, cut=0, unexplained=0, cand_checked=0)
    bad = []
    flavor = w["params"]["flavor"]
    greedy = w["params"]["greedy"] != 0
    for r in range(w.rows):
        rep = reports[r]
        if gpu["status"][r] != rep["status"]:
            counts["unexplained"] += 1
            bad.append((r, f"status {gpu['status'][r]} vs oracle {rep['status']}"))
            continue
        tie_order_free = flavor[r] == 0 and not greedy[r]
        # the top-p decision near top_p may change the kept set and so the pick; u near a boundary the pick alone
        cut = rep["cut"] < BOUNDARY
        near = rep["boundary"] < BOUNDARY
        fl = None
        same_id = gpu["ids"][r] == rep["id"]
        if not same_id:
            fl = final_logits_row(w, r) if tie_order_free else None
            if tie_order_free and 0 <= gpu["ids"][r] < w.vocab and fl[gpu["ids"][r]] == fl[rep["id"]]:
                counts["tie"] += 1
            elif cut or near:
                counts["cut" if cut else "boundary"] += 1
            else:
                counts["unexplained"] += 1
                bad.append((r, f"id {gpu['ids'][r]} vs oracle {rep['id']} (boundary {rep['boundary']:.3g}, "
                               f"cut {rep['cut']:.3g})"))
                continue
        if rep["status"] == 0 and gpu["kept"][r] != rep["kept"] and not cut:
            counts["unexplained"] += 1
            bad.append((r, f"kept {gpu['kept'][r]} vs oracle {rep['kept']}"))
            continue
        if same_id:
            counts["same"] += 1
        if cand_ids is None or "cand_ids" not in gpu or rep["status"] != 0 or cut:
            continue
        why = _check_candidates(w, r, gpu["cand_ids"][r], gpu["cand_weights"][r], cand_ids[r], cand_weights[r],
                                tie_order_free, fl)
        counts["cand_checked"] += 1
        if why:
            counts["unexplained"] += 1
            bad.append((r, why))
    return counts, bad


def _check_candidates(w, r, g_ids, g_w, o_ids, o_w, tie_order_free, fl):
    """None when the device's listed candidates are the oracle's (see compare), else the reason they are not."""
    if not np.array_equal(g_ids, o_ids):
        if not tie_order_free:
            return f"candidate ids differ at {int(np.argmax(g_ids != o_ids))}"
        fl = final_logits_row(w, r) if fl is None else fl
        listed = o_ids >= 0
        if not np.array_equal(g_ids >= 0, listed) and not np.all(fl[o_ids[listed & (g_ids < 0)]] == -np.inf):
            return "candidate lists differ in length"
        both = listed & (g_ids >= 0)
        if not np.array_equal(fl[g_ids[both]], fl[o_ids[both]]):
            return f"candidate ids differ beyond equal final logits at {int(np.argmax(fl[g_ids[both]] != fl[o_ids[both]]))}"
    o = np.asarray(o_w, dtype=np.float64)
    g = np.asarray(g_w, dtype=np.float64)
    err = np.abs(g - o) / np.where(o > 1e-300, o, 1.0)
    if np.any(err > PROB_RTOL):
        i = int(np.argmax(err))
        return f"candidate weight {i} off by {err[i]:.3g} relative ({g[i]!r} vs {o[i]!r})"
    return None
