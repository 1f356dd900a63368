"""The committed golden fixtures (tests/golden/, written by tests/golden/make_golden.py).

reference_sampling.npz holds what the reference's own src/common/sampling.cpp (compiled unchanged) returned for
uniform() and pick(): the oracle's restatement must reproduce it bit for bit, also where the reference checkout is
absent. workloads.npz holds the oracle's answers on the five seeded workloads at reduced row counts: the inputs must
regenerate to the same digest, the oracle must reproduce the answers, and the HIP path must match them (to the bar
of the parity tests: ids bit-exact except within 1e-6 of a boundary or of the top-p decision, or between equal final
logits)."""

import os

import numpy as np
import pytest

import gpu_harness
import oracle_lib
import workloads
from golden.make_golden import NCAND, WORKLOADS, digest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(HERE, name), allow_pickle=False)


def test_uniform_and_pick_reproduce_the_reference_outputs():
    g = load("reference_sampling.npz")
    for i, seed in enumerate(g["seeds"].tolist()):
        np.testing.assert_array_equal(oracle_lib.uniform_fill(int(seed), g["uniform"].shape[1]), g["uniform"][i])
    w, wo, u, uo, picks = g["weights"], g["weight_off"], g["u"], g["u_off"], g["pick"]
    for c in range(len(wo) - 1):
        weights = w[wo[c]:wo[c + 1]]
        for j in range(uo[c], uo[c + 1]):
            assert oracle_lib.pick(weights, float(u[j])) == picks[j], (c, u[j])


@pytest.mark.parametrize("name,rows,seed", WORKLOADS)
def test_workload_inputs_regenerate(name, rows, seed):
    g = load("workloads.npz")
    assert digest(workloads.make(name, rows=rows, seed=seed)) == str(g[name + "/digest"])


@pytest.mark.parametrize("name,rows,seed", WORKLOADS)
def test_oracle_reproduces_the_workload_answers(name, rows, seed):
    g = load("workloads.npz")
    w = workloads.make(name, rows=rows, seed=seed)
    reports, cids, cweights = oracle_lib.sample_rows(w, cap=NCAND)
    for key in ("id", "status", "kept", "boundary", "cut"):
        np.testing.assert_array_equal(reports[key], g[name + "/" + key], err_msg=key)
    np.testing.assert_array_equal(cids, g[name + "/cand_ids"])
    np.testing.assert_array_equal(cweights, g[name + "/cand_weights"])


@pytest.mark.gpu
@pytest.mark.parametrize("name,rows,seed", WORKLOADS)
def test_hip_path_matches_the_workload_answers(name, rows, seed):
    g = load("workloads.npz")
    w = workloads.make(name, rows=rows, seed=seed)
    reports = np.zeros(rows, dtype=oracle_lib.REPORT)
    for key in ("id", "status", "kept", "boundary", "cut"):
        reports[key] = g[name + "/" + key]
    spx = workloads.spx_module()
    sampler = spx.Sampler(max_rows=rows, max_vocab=w.vocab, max_hist=2048, max_out=NCAND)
    gpu = gpu_harness.run_gpu(sampler, w, max_out=NCAND)
    counts, bad = gpu_harness.compare(w, gpu, reports, g[name + "/cand_ids"], g[name + "/cand_weights"])
    print(name, counts)
    assert not bad, bad[:5]
