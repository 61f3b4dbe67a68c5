"""Shared cases and distribution checks for rejection-sampling acceptance (R16): a k = 3
case on a small vocab and the chi-square / binomial p-values of every distribution that
speculative sampling fixes (Leviathan et al. 2023; Chen et al. 2023)."""
from __future__ import annotations

import numpy as np
from scipy import stats


def softmax_T(l, T):
    z = (np.asarray(l, np.float64) - np.max(l, axis=-1, keepdims=True)) / T
    e = np.exp(z)
    return e / e.sum(-1, keepdims=True)


def k3_case():
    """Four target rows and three draft rows on a vocab of 8 whose rows differ clearly from
    one another, with drafts near enough to their targets that about 3 rounds in 10 accept
    all three drafts."""
    rng = np.random.default_rng(7)
    V, k, T = 8, 3, 0.7
    tl = rng.normal(0, 0.9, (k + 1, V)).astype(np.float32)
    dl = (tl[:k] + rng.normal(0, 0.7, (k, V))).astype(np.float32)
    return tl, dl, T


def chi2_p(counts, probs):
    """Chi-square p-value of counts against probs; categories with expected count < 5 are
    pooled; counts outside the support (probs == 0) give p = 0."""
    counts = np.asarray(counts, np.float64)
    probs = np.asarray(probs, np.float64)
    if counts[probs == 0].sum() > 0:
        return 0.0
    n = counts.sum()
    exp = probs * n
    small = (exp < 5) & (probs > 0)
    keep = (exp >= 5)
    c = list(counts[keep]) + ([counts[small].sum()] if small.any() else [])
    e = list(exp[keep]) + ([exp[small].sum()] if small.any() else [])
    if len(c) < 2:
        return 1.0
    return stats.chisquare(c, e).pvalue


def k3_pvalues(tl, dl, T, drafts, acc, nxt):
    """p-values of every distribution the speculative-sampling theorem fixes at k = 3, from
    rounds with drafts [n, k] drawn from q, accepted counts acc [n] and emitted tokens nxt [n]:
    the token emitted at position j (j = 0..3, over rounds that reach j) against p_j; the
    draw after a first rejection at i against norm(max(0, p_i - q_i)); the all-accepted
    bonus against p_k; and the acceptance at i against sum_x min(p_i, q_i) (binomial).
    Also returns the histogram of accepted counts."""
    k, V = dl.shape
    p, q = softmax_T(tl, T), softmax_T(dl, T)
    out = {}
    for j in range(k + 1):
        reach = acc >= j
        tok = np.where(acc[reach] > j, drafts[reach, min(j, k - 1)], nxt[reach])
        out[f"pos{j}"] = chi2_p(np.bincount(tok, minlength=V), p[j])
    for i in range(k):
        r = np.maximum(p[i] - q[i], 0.0)
        out[f"res{i}"] = chi2_p(np.bincount(nxt[acc == i], minlength=V), r / r.sum())
        reach = int((acc >= i).sum())
        out[f"acc{i}"] = stats.binomtest(int((acc > i).sum()), reach, float(np.minimum(p[i], q[i]).sum())).pvalue
    out["bonus"] = chi2_p(np.bincount(nxt[acc == k], minlength=V), p[k])
    return out, np.bincount(acc, minlength=k + 1)
