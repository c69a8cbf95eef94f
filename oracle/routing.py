"""Routing oracle (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

Restates the top-k routing that vLLM's select_experts performs for the
supported models, as called by the router-split entry
(src/sluice/offloader.py:2583-2585):

  softmax_topk   softmax over E, top-k, optional renormalisation and scale
                 (DeepSeek-V2-Lite: greedy, no renorm, scale 1.0; Qwen3-MoE:
                 renorm).  Optional group limit on the group max (DeepSeek-V2
                 group_limited_greedy).
  sigmoid_topk   sigmoid scores + e_score_correction_bias, groups ranked by
                 the sum of their two best biased scores, top topk_group
                 groups eligible, top-k among them, weights from the unbiased
                 sigmoid, renormalised (+1e-20) and scaled (DeepSeek-V3).

Tie rule (the reference leaves it to torch.topk, whose order on ties is
unspecified): candidates are ranked by (key descending, expert id ascending);
softmax ranks on the logit (softmax is monotone), sigmoid on
fp32(fp32(1/(1+exp(-x))) + bias) with the sigmoid evaluated in fp64 and
rounded to fp32 once.
"""

from __future__ import annotations

import numpy as np


def _rank_select(keys: np.ndarray, eligible: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k best eligible keys, best first, ties -> lower index."""
    E = keys.shape[0]
    ids = np.arange(E)
    cand = ids[eligible]
    # lexsort: last key is primary.  Primary: -key (descending key); then id.
    order = np.lexsort((cand, -keys[cand].astype(np.float64)))
    return cand[order[:k]]


def sigmoid_fp32(logits: np.ndarray) -> np.ndarray:
    x = np.asarray(logits, dtype=np.float32).astype(np.float64)
    return (1.0 / (1.0 + np.exp(-x))).astype(np.float32)


def group_eligible(group_scores: np.ndarray, topk_group: int) -> np.ndarray:
    order = np.lexsort((np.arange(group_scores.shape[0]), -group_scores.astype(np.float64)))
    ok = np.zeros(group_scores.shape[0], dtype=bool)
    ok[order[:topk_group]] = True
    return ok


def softmax_topk(logits: np.ndarray, k: int, renorm: bool = False, scale: float = 1.0,
                 n_group: int = 1, topk_group: int = 1):
    """logits [T,E] (fp32 values) -> (ids [T,k] int32, weights [T,k] fp32)."""
    logits = np.asarray(logits, dtype=np.float32)
    T, E = logits.shape
    ids = np.zeros((T, k), dtype=np.int32)
    w = np.zeros((T, k), dtype=np.float32)
    for t in range(T):
        l = logits[t]
        elig = np.ones(E, dtype=bool)
        if n_group > 1:
            gs = l.reshape(n_group, E // n_group).max(axis=1)
            gok = group_eligible(gs, topk_group)
            elig = np.repeat(gok, E // n_group)
        sel = _rank_select(l, elig, k)
        l64 = l.astype(np.float64)
        p = np.exp(l64 - l64.max())
        p = p / p.sum()
        ws = p[sel]
        if renorm:
            ws = ws / ws.sum()
        ids[t] = sel
        w[t] = (ws * scale).astype(np.float32)
    return ids, w


def sigmoid_topk(logits: np.ndarray, bias, k: int, n_group: int = 1, topk_group: int = 1,
                 renorm: bool = True, scale: float = 1.0):
    """DeepSeek-V3 routing; logits [T,E], bias [E] or None."""
    logits = np.asarray(logits, dtype=np.float32)
    T, E = logits.shape
    s = sigmoid_fp32(logits)
    b = np.zeros(E, dtype=np.float32) if bias is None else np.asarray(bias, dtype=np.float32)
    key = (s + b[None, :]).astype(np.float32)  # fp32 add
    ids = np.zeros((T, k), dtype=np.int32)
    w = np.zeros((T, k), dtype=np.float32)
    for t in range(T):
        elig = np.ones(E, dtype=bool)
        if n_group > 1:
            g = key[t].reshape(n_group, E // n_group)
            top2 = -np.sort(-g, axis=1)[:, :2]
            gs = (top2[:, 0] + top2[:, 1]).astype(np.float32) if g.shape[1] >= 2 else top2[:, 0]
            gok = group_eligible(gs, topk_group)
            elig = np.repeat(gok, E // n_group)
        sel = _rank_select(key[t], elig, k)
        ws = s[t, sel].astype(np.float64)
        if renorm:
            ws = ws / (ws.sum() + 1e-20)
        ids[t] = sel
        w[t] = (ws * scale).astype(np.float32)
    return ids, w


def route(logits, *, k, scoring="softmax", renorm=False, scale=1.0, bias=None, n_group=1,
          topk_group=1):
    if scoring == "softmax":
        return softmax_topk(logits, k, renorm=renorm, scale=scale, n_group=n_group,
                            topk_group=topk_group)
    return sigmoid_topk(logits, bias, k, n_group=n_group, topk_group=topk_group, renorm=renorm,
                        scale=scale)
