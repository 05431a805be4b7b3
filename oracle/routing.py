"""numpy routing front-ends for the synthetic MoE workloads.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`).

The reference leaves routing to the caller (`build_moe_ffn_latent`, described
in README.md:111 and implemented in the empty patch 004).  These functions
define the routing of the benchmark configurations in closed form:

* `softmax_topk`: softmax over experts in float64, top-k by descending
  probability (ties -> lower expert id), weights renormalised over the k kept
  experts, stored fp32.
* `zipf_logits`: N(0,1) logits plus `gamma * (-alpha * ln rank(e))` for a fixed
  random expert->popularity-rank permutation.
* `adaptive_drop`: slots whose renormalised weight is below a threshold become
  id -1 / weight 0 without re-renormalising.  This is a simpler rule than the
  cumulative-mass rule of loader/adaptive_topk.py:29-55; `adaptive_topk_inclusive`
  restates that rule too.
"""

from __future__ import annotations

import numpy as np


def softmax_topk(logits: np.ndarray, k: int):
    lg = np.asarray(logits, dtype=np.float64)
    p = np.exp(lg - lg.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    order = np.argsort(-p, axis=1, kind="stable")[:, :k]
    top = np.take_along_axis(p, order, axis=1)
    w = top / top.sum(axis=1, keepdims=True)
    return order.astype(np.int32), w.astype(np.float32)


def zipf_logits(rng: np.random.Generator, n_tokens: int, n_expert: int, gamma: float, alpha: float = 1.1):
    perm = rng.permutation(n_expert)
    rank = perm.astype(np.float64) + 1.0
    bias = gamma * (-alpha * np.log(rank))
    return (rng.standard_normal((n_tokens, n_expert)) + bias[np.newaxis, :]).astype(np.float32)


def adaptive_drop(ids: np.ndarray, w: np.ndarray, threshold: float):
    ids = np.array(ids, dtype=np.int32, copy=True)
    w = np.array(w, dtype=np.float32, copy=True)
    drop = w < np.float32(threshold)
    ids[drop] = -1
    w[drop] = 0.0
    return ids, w


def adaptive_topk_inclusive(sorted_scores: np.ndarray, threshold: float = 0.95) -> int:
    """Number of experts kept under the cumulative-mass rule.  loader/adaptive_topk.py:29-55."""
    scores = np.asarray(sorted_scores)
    if scores.size == 0:
        return 0
    if not 0.0 < threshold <= 1.0:
        raise ValueError(f"threshold must be in (0, 1], got {threshold}")
    total = float(np.sum(scores))
    if total <= 0:
        return 0
    target = threshold * total
    cumulative = 0.0
    for i, score in enumerate(scores):
        if cumulative + score > target:
            return i
        cumulative += score
    return int(scores.size)


def router_logits(x: np.ndarray, router: np.ndarray) -> np.ndarray:
    """x [T, d] . W_r [d, E] in float64 (the GPU sums fp32 products)."""
    return np.asarray(x, np.float64) @ np.asarray(router, np.float64)


def inclusive_drop(ids: np.ndarray, w: np.ndarray, threshold: float):
    """Per token, keep the leading slots chosen by adaptive_topk_inclusive on the
    descending top-k weights (adaptive_topk_batch, loader/adaptive_topk.py:58-90);
    the rest become id -1 / weight 0."""
    ids = np.array(ids, dtype=np.int32, copy=True)
    w = np.array(w, dtype=np.float32, copy=True)
    for t in range(ids.shape[0]):
        n = adaptive_topk_inclusive(w[t], threshold)
        ids[t, n:] = -1
        w[t, n:] = 0.0
    return ids, w


def route(logits: np.ndarray, k: int, drop: str = "none", drop_param: float = 0.0):
    """softmax_topk followed by the drop rule ('none', 'below', 'inclusive')."""
    ids, w = softmax_topk(logits, k)
    if drop == "below":
        return adaptive_drop(ids, w, drop_param)
    if drop == "inclusive":
        return inclusive_drop(ids, w, drop_param)
    if drop != "none":
        raise ValueError(drop)
    return ids, w
