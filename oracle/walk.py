"""Greedy accepted-path oracle (CPU).  Test infrastructure only.

Restates the temperature-0 branch of cast_trees/decode.py:85-103 with the
pick rule of decode.py:13-15.  From the root (logits row 0), the target's
choice is the first index of the row maximum (``torch.argmax``: a NaN counts
as the maximum, the earliest one wins).  The walk moves to the first child,
in node order, whose token equals that choice, and stops when no child
matches.  Node c's logits row is c + 1.  Returns (path, bonus): the accepted
node indices root-to-leaf and the target's token after the last one.
"""
import numpy as np
import torch


def row_argmax(row):
    """First index of the maximum, NaN treated as the maximum (torch rule)."""
    r = row.detach().float().cpu() if torch.is_tensor(row) else torch.as_tensor(row).float()
    nan = torch.isnan(r)
    if bool(nan.any()):
        return int(torch.nonzero(nan)[0, 0])
    return int(torch.argmax(r))


def greedy_walk(nodes, logits):
    """nodes: list of objects with .token/.parent; logits: [1+N, V]."""
    kids = {i: [] for i in range(-1, len(nodes))}
    for i, nd in enumerate(nodes):
        kids[nd.parent].append(i)
    path, cur = [], -1
    while True:
        tok = row_argmax(logits[cur + 1])
        hit = None
        for c in kids[cur]:
            if nodes[c].token == tok:
                hit = c
                break
        if hit is None:
            return path, tok
        path.append(hit)
        cur = hit


def greedy_walk_batch(trees, logits, cu_q):
    """Per request (path, bonus) over packed logits [total_q, V]."""
    cu = [int(x) for x in (cu_q.tolist() if hasattr(cu_q, "tolist") else cu_q)]
    return [greedy_walk(t, logits[cu[b]:cu[b + 1]]) for b, t in enumerate(trees)]


def row_argmax_all(logits):
    """First-max indices of every row (NaN-as-max), int64 numpy."""
    x = logits.detach().float().cpu()
    am = torch.argmax(x, dim=-1).numpy().astype(np.int64)
    nan = torch.isnan(x)
    if bool(nan.any()):
        for r in torch.nonzero(nan.any(dim=-1)).flatten().tolist():
            am[r] = int(torch.nonzero(nan[r])[0, 0])
    return am
