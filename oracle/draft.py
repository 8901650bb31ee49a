"""Drafter top-k and best-first tree build, restated.  TEST INFRASTRUCTURE ONLY.

  topk_log_softmax  log-softmax over the vocabulary and the top k per row,
                    ranked by descending log-probability with equal values
                    in increasing index order (cast_trees/tree.py:20-26,
                    the stable sort; cast_trees/verify.py:8-12 for the
                    log-softmax + top-k the serving path runs)
  build_tree        the best-first heap of cast_trees/tree.py:29-49: entries
                    (-score, depth, parent, rank, counter), scores summed in
                    Python floats
"""
import heapq

import numpy as np


def topk_log_softmax(logits, k):
    """logits [rows, V] (any float dtype) -> (idx int64 [rows, k], lp float64 [rows, k])."""
    x = np.asarray(logits, dtype=np.float64)
    lp = x - x.max(axis=-1, keepdims=True)
    lp = lp - np.log(np.exp(lp).sum(axis=-1, keepdims=True))
    idx = np.argsort(-x, axis=-1, kind="stable")[:, :k]
    return idx, np.take_along_axis(lp, idx, axis=-1)


def build_tree(top_idx, top_lp, budget, k=8):
    """[(token, depth, parent, score)] in pop order."""
    L = top_idx.shape[0]
    k = min(k, top_idx.shape[1])
    heap, out, cnt = [], [], 0
    for r in range(k):
        heapq.heappush(heap, (-float(top_lp[0, r]), 1, -1, r, cnt))
        cnt += 1
    while heap and len(out) < budget:
        neg, d, parent, r, _ = heapq.heappop(heap)
        me = len(out)
        out.append((int(top_idx[d - 1, r]), d, parent, -neg))
        if d < L:
            for r2 in range(k):
                heapq.heappush(heap, (neg - float(top_lp[d, r2]), d + 1, me, r2, cnt))
                cnt += 1
    return out
