"""Drafter top-k marginals and best-first candidate trees on the device.

  topk_marginals     drop-in for cast_trees/verify.py:8-12 (log-softmax over
                     the vocabulary, top-k per future position); the result
                     stays on the device with ``on_device=True``
  build_trees        cast_trees/tree.py:29-49 for a whole batch on the device:
                     one tree per request, nodes in heap pop order
  build_tree_device  drop-in for cast_trees/tree.py:29 build_tree returning
                     TreeNode lists (one copy back)

Ranking: descending log-probability, equal values in increasing token order
(the stable sort of cast_trees/tree.py:20-26).  Tree scores are summed in
double precision in the reference's order, so the trees match the
reference's heap exactly for the same (top_idx, top_lp).
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib
from .tree import MAX_PACK, TreeNode


def topk_marginals(d_logits, k, *, on_device=False, splits=0):
    """Top-k token ids and log-probs at each future position.

    d_logits: [L, V] (or [rows, V]) bf16/fp16/fp32 on the device (other float
    dtypes are widened to fp32 first).  Returns (indices
    int64 [L, k], values float32 [L, k]), moved to the host like the reference
    unless ``on_device``.  ``splits`` sets the workgroups per row (0: chosen
    from the shape); the results do not depend on it beyond float rounding
    of the log-sum-exp.
    """
    lib = _lib.load()
    x = d_logits
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        x = x.float()
    if x.dim() != 2 or not x.is_cuda:
        raise ValueError("d_logits must be a [rows, V] device tensor")
    if x.stride(1) != 1:
        x = x.contiguous()
    rows, V = x.shape
    dt = {torch.bfloat16: _lib.BF16, torch.float16: _lib.FP16}.get(x.dtype, _lib.FP32)
    idx = torch.empty((rows, k), dtype=torch.int64, device=x.device)
    lp = torch.empty((rows, k), dtype=torch.float32, device=x.device)
    ws_bytes = lib.cast_draft_topk_workspace_size(rows, V, dt, k, int(splits)) if 1 <= k <= 16 else 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
    with _lib.on_device(x.device):
        st = lib.cast_draft_topk(_lib.ptr(x), x.stride(0), rows, V, dt, k, _lib.ptr(idx), _lib.ptr(lp),
                                 int(splits), _lib.ptr(ws), ws_bytes, _lib.stream_of(x))
    _lib.check(st, "cast_draft_topk")
    return (idx, lp) if on_device else (idx.cpu(), lp.cpu())


def build_trees(top_idx, top_lp, budget, k=None, *, check=False):
    """Best-first trees of a batch on the device.

    top_idx int64 / top_lp float32 or float64: [B, L, k] device tensors (the
    reference sums Python floats: float64 top_lp reproduces its trees from
    float64 block scores bit for bit); budget: int or
    int32 [B] non-root nodes per request (<= 127).  Returns device tensors
    (token int64 [B, 127], depth int32, parent int32, score float64 [B, 127],
    n_nodes int32 [B]), nodes in pop order.
    """
    lib = _lib.load()
    if top_idx.dim() == 2:
        top_idx, top_lp = top_idx[None], top_lp[None]
    if top_idx.dim() != 3 or top_lp.shape != top_idx.shape:
        raise ValueError("top_idx and top_lp must both be [B, L, k] (or [L, k])")
    if isinstance(budget, int) or not (isinstance(budget, torch.Tensor) and budget.is_cuda):
        # budgets known on the host are checked here; a device tensor above 127
        # is clamped by the kernel and flagged in the status word
        b_host = np.asarray(budget.cpu() if isinstance(budget, torch.Tensor) else budget).reshape(-1)
        if b_host.size and (b_host.min() < 0 or b_host.max() > MAX_PACK - 1):
            raise ValueError(f"budget must be in [0, {MAX_PACK - 1}] nodes per tree (packs of up to {MAX_PACK} tokens)")
    if not (top_idx.is_cuda and top_lp.is_cuda) or top_lp.device != top_idx.device:
        raise ValueError("top_idx and top_lp must be on one GPU")
    B, L, kk = top_idx.shape
    k = kk if k is None else min(int(k), kk)
    if L < 1 or L > 255 or k < 1 or k > 16:
        raise ValueError("build_trees needs 1 <= L <= 255 future positions and 1 <= k <= 16 candidates")
    dev = top_idx.device
    ti = top_idx[..., :k].to(torch.int64).contiguous()
    tl = top_lp[..., :k]
    if tl.dtype != torch.float64:
        tl = tl.to(torch.float32)
    tl = tl.contiguous()
    if isinstance(budget, int):
        budget = torch.full((B,), budget, dtype=torch.int32, device=dev)
    budget = torch.as_tensor(budget, device=dev).to(torch.int32).contiguous()
    if budget.shape != (B,):
        raise ValueError(f"budget must be an int or [{B}] per-request node counts")
    n = MAX_PACK - 1
    token = torch.empty((B, n), dtype=torch.int64, device=dev)
    depth = torch.empty((B, n), dtype=torch.int32, device=dev)
    parent = torch.empty((B, n), dtype=torch.int32, device=dev)
    score = torch.empty((B, n), dtype=torch.float64, device=dev)
    n_nodes = torch.empty(B, dtype=torch.int32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev) if check else None
    with _lib.on_device(dev):
        st = lib.cast_build_trees(_lib.ptr(ti), _lib.ptr(tl), _lib.FP64 if tl.dtype == torch.float64 else _lib.FP32,
                                  B, L, k, _lib.ptr(budget), _lib.ptr(token),
                                  _lib.ptr(depth), _lib.ptr(parent), _lib.ptr(score), _lib.ptr(n_nodes),
                                  _lib.ptr(status), _lib.stream_of(ti))
    _lib.check(st, "cast_build_trees")
    if check:
        _lib.raise_device_flags(status.item(), "build_trees")
    return token, depth, parent, score, n_nodes


def build_tree_device(top_idx, top_lp, budget, k=8):
    """build_tree (cast_trees/tree.py:29) on the device: [L, >=k] candidates
    (device or host tensors) -> TreeNode list in pop order."""
    dev = torch.device("cuda", torch.cuda.current_device())
    ti = torch.as_tensor(top_idx).to(dev)
    tl = torch.as_tensor(top_lp)
    tl = tl.to(dev, torch.float64 if tl.dtype == torch.float64 else torch.float32)
    k = min(k, ti.shape[-1])
    token, depth, parent, score, n_nodes = build_trees(ti, tl, int(budget), k)
    m = int(n_nodes[0].item())
    rows = zip(token[0, :m].tolist(), depth[0, :m].tolist(), parent[0, :m].tolist(), score[0, :m].tolist())
    return [TreeNode(int(t), int(d), int(p), float(s)) for t, d, p, s in rows]
