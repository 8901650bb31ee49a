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
import itertools

import numpy as np


def topk_log_softmax(logits, k):
    """logits [rows, V] (any float dtype) -> (idx int64 [rows, k], lp float64 [rows, k]).

    Log-probabilities in float64 with the row max taken out first.  The rank
    is a lexicographic sort on (-logit, index): the log-softmax keeps the
    logits' order, so this is the stable descending order of
    cast_trees/tree.py:20-26 (pinned by that module's fixtures).  A NaN logit
    sorts last and never ranks, as in the device kernel; the reference sorts
    the log-probabilities instead, which a NaN anywhere in the row turns all
    to NaN, leaving such a row in index order."""
    x = np.asarray(logits, dtype=np.float64)
    shifted = x - x.max(axis=-1, keepdims=True)
    logp = shifted - np.log(np.exp(shifted).sum(axis=-1, keepdims=True))
    index = np.broadcast_to(np.arange(x.shape[-1]), x.shape)
    order = np.lexsort((index, -x), axis=-1)[:, :k]
    return order, np.take_along_axis(logp, order, axis=-1)


def build_tree(top_idx, top_lp, budget, k=8):
    """[(token, depth, parent, score)] in the order cast_trees/tree.py:29-49
    pops them.

    Best-first expansion: the frontier holds (-score, depth, parent, rank,
    arrival) entries, the smallest is taken next, and taking a node offers
    its `width` children one position deeper, each scored as the parent's
    score plus its log-probability (Python floats, as the reference sums
    them).  (depth, parent, rank) is unique, so the arrival number never
    decides an order."""
    max_depth = top_idx.shape[0]
    width = min(k, top_idx.shape[1])
    arrival = itertools.count()
    frontier = []

    def offer(neg_score, depth, parent):
        row = top_lp[depth - 1]
        for rank in range(width):
            heapq.heappush(frontier, (neg_score - float(row[rank]), depth, parent, rank, next(arrival)))

    offer(0.0, 1, -1)
    taken = []
    while frontier and len(taken) < budget:
        neg_score, depth, parent, rank, _ = heapq.heappop(frontier)
        taken.append((int(top_idx[depth - 1, rank]), depth, parent, -neg_score))
        if depth < max_depth:
            offer(neg_score, depth + 1, len(taken) - 1)
    return taken
