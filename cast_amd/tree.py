"""Candidate trees and their packed verify layout (host side, numpy only).

A verify pass packs every request's tree as ``[root] + nodes``: pack index 0
is the pending root token and pack index ``i + 1`` is ``nodes[i]``.  Nodes are
listed parent-before-child, so each node's parent has a smaller pack index.
This module produces that layout from drafter block scores and flattens a
batch of trees into the int32 arrays the device kernels read.

Mirrors the public tree API of cast_trees/tree.py:
  TreeNode                  cast_trees/tree.py:12-17
  block_topk                cast_trees/tree.py:20-26
  build_tree                cast_trees/tree.py:29-49
  build_chain               cast_trees/tree.py:52-55
  expected_accepted_length  cast_trees/tree.py:58-60
  select_global_topk        cast_trees/tree.py:63-82
  ancestor_matrix           cast_trees/tree.py:85-93
and the host-side packing of cast_trees/serving.py:211-231.
"""
from __future__ import annotations

import heapq
from dataclasses import dataclass

import numpy as np

MAX_PACK = 128          # two 64-bit ancestor words per packed token


@dataclass
class TreeNode:
    """One drafted token of a candidate tree.

    token   vocabulary id
    depth   how many tokens after the pending root it sits (1 = a root child,
            at most L, the drafter's block length)
    parent  position of its parent in the same node list; -1 when the parent
            is the root itself
    score   summed drafter log-probabilities from the root down to this node
    """
    token: int
    depth: int
    parent: int
    score: float


def _log_softmax64(x):
    x = np.asarray(x, dtype=np.float64)
    z = x - x.max(axis=-1, keepdims=True)
    return z - np.log(np.exp(z).sum(axis=-1, keepdims=True))


def block_topk(logits, k=8):
    """Per future position (row of ``logits``, shape (L, V)): the k most
    likely token ids and their log-softmax values, best first.

    Ties are broken towards the smaller token id (a stable descending sort).
    Only the k best columns are fully sorted: an ``argpartition`` picks every
    column whose log-prob reaches the k-th largest value, and those few are
    ordered by (-log-prob, id), which is exactly the head of a stable sort.
    """
    lp = _log_softmax64(logits)
    L, V = lp.shape
    k = min(k, V)
    idx = np.empty((L, k), dtype=np.int64)
    for r in range(L):
        row = lp[r]
        if V > 4 * k:
            kth = -np.partition(-row, k - 1)[k - 1]
            cand = np.nonzero(row >= kth)[0]
        else:
            cand = np.arange(V)
        order = np.lexsort((cand, -row[cand]))[:k]
        idx[r] = cand[order]
    return idx, np.take_along_axis(lp, idx, axis=-1)


def build_tree(top_idx, top_lp, budget, k=8):
    """Grow a tree of ``budget`` nodes (root excluded) by always adding the
    candidate with the highest path log-prob; a node joins only after its
    parent, so every prefix of a path is in the tree.

    Candidates are expanded in order of path log-prob; equal scores fall back
    to (depth, parent, rank, insertion order), so the node order is fully
    determined.  The returned list is in expansion order, parents first.
    """
    top_idx = np.asarray(top_idx)
    top_lp = np.asarray(top_lp, dtype=np.float64)
    L = top_idx.shape[0]
    k = min(k, top_idx.shape[1])
    frontier = []
    serial = 0

    def offer(neg_score, depth, parent):
        nonlocal serial
        for rank in range(k):
            key = (neg_score - float(top_lp[depth - 1, rank]), depth, parent, rank, serial)
            heapq.heappush(frontier, key)
            serial += 1

    offer(0.0, 1, -1)
    nodes: list[TreeNode] = []
    while frontier and len(nodes) < budget:
        neg, depth, parent, rank, _ = heapq.heappop(frontier)
        nodes.append(TreeNode(int(top_idx[depth - 1, rank]), depth, parent, -neg))
        if depth < L:
            offer(neg, depth + 1, len(nodes) - 1)
    return nodes


def build_chain(top_idx, top_lp, length):
    """Rank-0 path of the given length (the plain block draft)."""
    top_lp = np.asarray(top_lp, dtype=np.float64)
    out, acc = [], 0.0
    for d in range(1, length + 1):
        acc = float(top_lp[:d, 0].sum())
        out.append(TreeNode(int(top_idx[d - 1][0]), d, d - 2, acc))
    return out


def expected_accepted_length(nodes):
    """Sum of path masses: expected accepted draft tokens under the drafter."""
    return float(sum(np.exp(n.score) for n in nodes))


def select_global_topk(trees, total):
    """Share a budget of ``total`` nodes across requests by global score.

    Scores never increase from parent to child, so the pooled top set is
    prefix-closed per tree; parents are re-indexed into each kept list.
    """
    pool = sorted(((-n.score, b, j) for b, t in enumerate(trees) for j, n in enumerate(t)))
    kept = [[] for _ in trees]
    for _, b, j in pool[:total]:
        kept[b].append(j)
    out = []
    for b, t in enumerate(trees):
        keep = sorted(kept[b])
        new_of = {old: new for new, old in enumerate(keep)}
        out.append([TreeNode(t[i].token, t[i].depth, new_of.get(t[i].parent, -1), t[i].score)
                    for i in keep])
    return out


def pack_parents(nodes):
    """Pack-local parent array of one tree: ``[-1] + [n.parent + 1 ...]``."""
    return np.array([-1] + [n.parent + 1 for n in nodes], dtype=np.int32)


def ancestor_matrix(nodes):
    """(1+N, 1+N) bool; row i marks packed token i and its ancestors."""
    par = pack_parents(nodes)
    n = par.shape[0]
    vis = np.zeros((n, n), dtype=bool)
    for i in range(n):
        if par[i] >= 0:
            vis[i] = vis[par[i]]
        vis[i, i] = True
    return vis


@dataclass
class PackedTrees:
    """A batch of trees flattened in the verify layout (all numpy, host)."""
    cu_q: np.ndarray        # int32 [B+1], pack offsets
    pack_len: np.ndarray    # int32 [B], 1 + nodes per tree
    parent: np.ndarray      # int32 [total_q], pack-local parent, -1 at each root
    token: np.ndarray       # int64 [total_q], root token then node tokens
    depth: np.ndarray       # int32 [total_q], 0 at the root

    @property
    def total_q(self):
        return int(self.cu_q[-1])

    @property
    def batch(self):
        return int(self.pack_len.shape[0])


def pack_trees(trees, roots=None):
    """Flatten a batch of trees (lists of TreeNode) into the packed layout.

    Follows the packing order of cast_trees/serving.py:213-226: per request
    the root first, then its nodes in list order.  Raises ValueError when a
    tree is not parent-before-child or a pack exceeds MAX_PACK tokens.
    """
    B = len(trees)
    if roots is None:
        roots = [0] * B
    pack_len = np.array([1 + len(t) for t in trees], dtype=np.int32)
    if B and int(pack_len.max()) > MAX_PACK:
        raise ValueError(f"a pack holds at most {MAX_PACK} tokens, got {int(pack_len.max())}")
    cu_q = np.zeros(B + 1, dtype=np.int32)
    np.cumsum(pack_len, out=cu_q[1:])
    parent = np.empty(int(cu_q[-1]), dtype=np.int32)
    token = np.empty(int(cu_q[-1]), dtype=np.int64)
    depth = np.empty(int(cu_q[-1]), dtype=np.int32)
    for b, nodes in enumerate(trees):
        base = int(cu_q[b])
        parent[base] = -1
        token[base] = int(roots[b])
        depth[base] = 0
        for i, nd in enumerate(nodes):
            if not -1 <= nd.parent < i:
                raise ValueError(f"tree {b}: node {i} has parent {nd.parent}; parents must come first")
            parent[base + i + 1] = nd.parent + 1
            token[base + i + 1] = nd.token
            depth[base + i + 1] = nd.depth
    return PackedTrees(cu_q, pack_len, parent, token, depth)
