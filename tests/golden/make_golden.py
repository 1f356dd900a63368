"""Writes the golden fixtures of tests/golden/ (run from the repository root: python tests/golden/make_golden.py).

reference_sampling.npz: the outputs of the reference's own src/common/sampling.cpp, compiled unchanged into
    oracle/_ref/ (this container only: the reference checkout is not on the GPU machine): uniform() of four seeds and
    pick() on weight vectors with zeros, ties and the edges of u. Tests compare the oracle's restatement with them
    wherever the reference is absent.
workloads.npz: per workload of tests/workloads.py at a reduced row count, the digest of the seeded inputs and the
    oracle's answer per row (id, status, kept, distance of u to the nearest boundary and of the top-p decision to
    top_p) plus its first 8 candidates and their weights (the reference's Candidates). The GPU tests hold the HIP path
    to them.
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib  # noqa: E402
import workloads  # noqa: E402

SEEDS = [1, 5489, 42, 2 ** 63 + 3]
PICK_CASES = [
    ([5.0], [0.0, 0.5, 1.0]),
    ([1.0, 1.0], [0.0, 0.25, 0.5, 0.5000000001, 0.75, 1.0]),
    ([0.0, 3.0, 0.0, 1.0], [0.0, 0.1, 0.74, 0.75, 0.76, 1.0]),
    ([0.25, 0.25, 0.25, 0.25], [0.25, 0.5, 0.75, 0.9999999999, 1.0]),
    ([1e-300, 1.0, 1e300], [0.0, 0.5, 1.0]),
    ([0.1] * 10, [0.1, 0.2, 0.3, 0.30000000000000004, 0.7, 0.99]),
]
# temperature_overflow()'s message (src/common/sampling.cpp:21-25) is kept for these temperatures
TEMPERATURES = [1e-38, 0.7, 1e-5, 3e-45, 123456.0, 1e20, 0.1, 2.5e-4, float("inf")]
# (workload, rows, seed)
WORKLOADS = [("talker", 1, 1234), ("predictor", 32, 1234), ("asr", 4, 1234), ("haru", 4, 1234), ("mixed", 16, 1234)]
NCAND = 8


def digest(w):
    h = hashlib.sha256()
    for key in ("logits", "params", "u", "hist", "hist_off", "banned"):
        a = w[key]
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def reference_fixture():
    if oracle_lib.ref() is None:
        print("oracle/_ref/libref_sampling.so is absent (build oracle/ with the reference checkout): skipped")
        return
    uni = np.stack([oracle_lib.ref_uniform_fill(s, 64) for s in SEEDS])
    w_flat, w_off, u_flat, u_off, picks = [], [0], [], [0], []
    for weights, us in PICK_CASES:
        w_flat += weights
        w_off.append(len(w_flat))
        for u in us:
            u_flat.append(u)
            picks.append(oracle_lib.ref().ref_pick(np.asarray(weights, dtype=np.float64).ctypes.data_as(
                oracle_lib.ctypes.c_void_p), len(weights), u))
        u_off.append(len(u_flat))
    messages = []
    for t in TEMPERATURES:
        msg = oracle_lib.ctypes.create_string_buffer(512)
        inp = oracle_lib.ctypes.create_string_buffer(64)
        oracle_lib.ref().ref_temperature_overflow(t, msg, 512, inp, 64)
        messages.append(msg.value.decode())
    np.savez(os.path.join(HERE, "reference_sampling.npz"), seeds=np.array(SEEDS, dtype=np.uint64), uniform=uni,
             weights=np.array(w_flat), weight_off=np.array(w_off), u=np.array(u_flat), u_off=np.array(u_off),
             pick=np.array(picks, dtype=np.int32), temperatures=np.array(TEMPERATURES, dtype=np.float32),
             temperature_messages=np.array(messages))
    print("wrote reference_sampling.npz")


def workload_fixture():
    out = {}
    for name, rows, seed in WORKLOADS:
        w = workloads.make(name, rows=rows, seed=seed)
        reports, cids, cweights = oracle_lib.sample_rows(w, cap=NCAND)
        out[name + "/digest"] = np.array(digest(w))
        out[name + "/rows"] = np.array(rows)
        out[name + "/seed"] = np.array(seed)
        out[name + "/id"] = reports["id"].copy()
        out[name + "/status"] = reports["status"].copy()
        out[name + "/kept"] = reports["kept"].copy()
        out[name + "/boundary"] = reports["boundary"].copy()
        out[name + "/cut"] = reports["cut"].copy()
        out[name + "/cand_ids"] = cids
        out[name + "/cand_weights"] = cweights
    np.savez(os.path.join(HERE, "workloads.npz"), **out)
    print("wrote workloads.npz")


if __name__ == "__main__":
    reference_fixture()
    workload_fixture()
