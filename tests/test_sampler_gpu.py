"""Device top-k / top-p sampling (toyinfer_sample_topk_topp_f32) against the
oracle's restatement of src/sampler.cpp:18-67 on the same logits and draw.

The pick is an index, so the bar is exact: for a draw u placed in the middle
of kept interval j (intervals wider than MIN_P, so that the device's
parallel sums, which differ from the sequential ones by a few float ulps,
cannot cross a boundary), the device returns the oracle's order[j].  A draw
just below 1 checks the top-p cut (the last kept token) where no running sum
lies within CUT_MARGIN of top_p.  Greedy settings must return the first
maximum; ties at the k-th value keep the lowest indices on both sides.
"""
import numpy as np
import pytest
import torch

import oracle
from tests import helpers as H
from toyinfer_amd import attn

pytestmark = pytest.mark.gpu

MIN_P = 1e-4
CUT_MARGIN = 1e-4


class Sampler:
    def __init__(self, dev):
        self.dev = dev
        self.ws = torch.zeros(attn.sample_workspace_bytes(), dtype=torch.uint8, device=dev)
        self.coin = torch.zeros(1, dtype=torch.float32, device=dev)
        self.out = torch.zeros(1, dtype=torch.int32, device=dev)

    def __call__(self, logits_dev, T, k, p, u):
        self.coin.fill_(float(u))
        self.out.fill_(-7)
        attn.sample_topk_topp_f32(logits_dev, logits_dev.numel(), T, k, p, self.coin, self.out,
                                  self.ws)
        H.sync()
        return int(self.out.cpu().numpy().view(np.uint32)[0])


def draws(probs, kept):
    """(u, expected position in order) at the middle of every kept interval
    wider than MIN_P (at most 24 of them, spread), plus u = 0."""
    cum = np.cumsum(probs.astype(np.float64))[:kept]
    lo = np.concatenate([[0.0], cum[:-1]])
    js = [j for j in range(kept) if probs[j] > MIN_P]
    if len(js) > 24:
        js = [js[i] for i in np.linspace(0, len(js) - 1, 24).astype(int)]
    return [(0.0, 0)] + [((lo[j] + cum[j]) / 2 / cum[-1], j) for j in js]


def check_case(smp, lg, T, k, p, label):
    dev_lg = torch.from_numpy(lg).to(smp.dev)
    _, order, probs, kept = oracle.sample_topk_topp(lg, T, k, p, 0.0)
    for u, j in draws(probs, kept):
        got = smp(dev_lg, T, k, p, u)
        assert got == order[j], f"{label}: u={u:.6f} expected order[{j}]={order[j]}, got {got}"
    cum = np.cumsum(probs.astype(np.float64))
    if (len(cum) == 1 or np.min(np.abs(cum[:-1] - p)) > CUT_MARGIN) and probs[kept - 1] > MIN_P:
        got = smp(dev_lg, T, k, p, 1 - 2 ** -24)
        assert got == order[kept - 1], f"{label}: last kept {order[kept - 1]}, got {got}"


@pytest.mark.parametrize("V", [151936, 262144, 1000, 37])
@pytest.mark.parametrize("k", [2, 20, 50, 256])
def test_sample_vs_oracle(dev, V, k):
    print(f"[step] sample V={V} k={k}", flush=True)
    smp = Sampler(dev)
    rng = np.random.default_rng(V + k)
    lg = (rng.standard_normal(V) * 3).astype(np.float32)
    for T, p in ((0.6, 0.95), (1.0, 0.5), (1.7, 1.0)):
        check_case(smp, lg, T, k, p, f"V={V} k={k} T={T} p={p}")


def test_sample_ties_and_duplicates(dev):
    """Integer-valued logits: many exact ties, also at the k-th value."""
    smp = Sampler(dev)
    rng = np.random.default_rng(3)
    for V, k in ((151936, 20), (5000, 256), (300, 64)):
        lg = np.round(rng.standard_normal(V) * 2).astype(np.float32)
        check_case(smp, lg, 1.0, k, 0.9, f"ties V={V} k={k}")
        _, order, _, _ = oracle.sample_topk_topp(lg, 1.0, k, 0.9, 0.0)
        assert np.all(np.diff(lg[order]) <= 0)


def test_sample_greedy_settings(dev):
    smp = Sampler(dev)
    rng = np.random.default_rng(4)
    lg = rng.standard_normal(151936).astype(np.float32)
    lg[[500, 90000]] = lg.max() + 1.0                      # tie for the maximum: first wins
    d = torch.from_numpy(lg).to(dev)
    for T, k in ((0.0, 20), (5e-4, 50), (0.8, 1), (2.0, 1)):
        assert smp(d, T, k, 0.95, 0.99) == 500 == oracle.argmax(lg)


def test_workspace_reuse_across_shapes(dev):
    """One workspace, calls of different vocabularies and k in a row: the
    ticket re-arms itself."""
    smp = Sampler(dev)
    rng = np.random.default_rng(5)
    for V, k in ((151936, 256), (1000, 5), (262144, 20), (37, 37), (151936, 20)):
        lg = (rng.standard_normal(V) * 2).astype(np.float32)
        check_case(smp, lg, 0.8, k, 0.95, f"reuse V={V} k={k}")


def test_sample_frequencies(dev):
    """4000 uniform draws: token frequencies match the kept probabilities
    (chi-square over the kept tokens below the 0.999 quantile)."""
    smp = Sampler(dev)
    rng = np.random.default_rng(6)
    lg = (rng.standard_normal(1000) * 1.5).astype(np.float32)
    T, k, p = 1.0, 12, 0.9
    _, order, probs, kept = oracle.sample_topk_topp(lg, T, k, p, 0.0)
    d = torch.from_numpy(lg).to(dev)
    n = 4000
    picks = [smp(d, T, k, p, u) for u in rng.random(n).astype(np.float32)]
    pos = {int(t): i for i, t in enumerate(order[:kept])}
    assert all(t in pos for t in picks)
    obs = np.bincount([pos[t] for t in picks], minlength=kept)
    exp = probs[:kept].astype(np.float64) / probs[:kept].sum() * n
    chi2 = float(((obs - exp) ** 2 / exp).sum())
    from scipy.stats import chi2 as chi2_dist
    assert chi2 < chi2_dist.ppf(0.999, kept - 1), (obs, exp)


@pytest.mark.parametrize("V,k", [(7, 100), (256, 256), (1000, 64), (1000, 65), (151936, 128),
                                 (151936, 129), (262144, 256), (4097, 3), (1, 5)])
def test_sample_boundaries(dev, V, k):
    """k clamped to the vocabulary, every candidate kept, the one-wave sort
    (k <= 64) against the workgroup sort, the 64/32 workgroup switch at
    k = 128, odd vocabulary sizes, a one-entry vocabulary."""
    print(f"[step] sample boundary V={V} k={k}", flush=True)
    smp = Sampler(dev)
    rng = np.random.default_rng(V * 7 + k)
    lg = (rng.standard_normal(V) * 2).astype(np.float32)
    check_case(smp, lg, 1.3, k, 0.97, f"boundary V={V} k={k}")
