"""Synthetic workload inputs for the prefill-width MoE benchmark and its parity tests.

The prefill workload sends 512 token rows through one MoE layer with the expert popularity
skewed like Zipf(s = 1.1): expert e gets popularity rank rank[e] (a seeded permutation of
1..E), and its router logits are shifted by

    bias[e] = tau * ln(rank[e] ** -s) = -s * tau * ln(rank[e])

before the softmax (q38_moe_layer_set_router_bias). With the layer's N(0, 0.9) logits,
tau = 0.28 puts the hottest experts at 60-200 of 512 rows (188 at most for the benchmark
seed) and leaves more than a third of the experts with 0-4 rows.
"""
from __future__ import annotations

import numpy as np

ZIPF_S = 1.1
ZIPF_TAU = 0.28


def zipf_router_bias(experts: int, seed: int, s: float = ZIPF_S, tau: float = ZIPF_TAU) -> np.ndarray:
    """[experts] float32 additive router-logit bias of the Zipf(s) popularity workload."""
    rng = np.random.default_rng(seed)
    rank = np.empty(experts, np.int64)
    rank[rng.permutation(experts)] = np.arange(1, experts + 1)
    return (-s * tau * np.log(rank.astype(np.float64))).astype(np.float32)
