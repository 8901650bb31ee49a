"""Device-side verification glue: ancestor bitmask and greedy accepted path.

  tree_bitmask        K1, replaces the host bitmask loop of
                      cast_trees/serving.py:213-222
  greedy_accept       K3, the temperature-0 walk of cast_trees/decode.py:85-103
                      for a whole packed batch, results left on the device
  walk_tree           drop-in for cast_trees/decode.py:85 at temperature 0:
                      (nodes, logits) -> (accepted node indices, bonus token)
  walk_trees          the per-request loop of cast_trees/serving.py:326-335 in
                      one device pass and one copy back
  tree_attention_mask the dense additive mask of cast_trees/verify.py:15-25
                      (host side; the batch-one decoder's mask semantics)
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib
from .tree import MAX_PACK, ancestor_matrix, pack_trees


def tree_bitmask(parent, cu_q, words=2, *, check=False):
    """Ancestor words of every packed row, computed on the device.

    parent: int32 [total_q] pack-local parents (-1 at each root); cu_q: int32
    [B+1].  Returns int64 [total_q, 2] (``words=2``, packs <= 128 tokens) or
    the reference's int64 [total_q] (``words=1``, packs <= 64 tokens).
    """
    lib = _lib.load()
    if words not in (1, 2):
        raise ValueError("words must be 1 or 2")
    parent = torch.as_tensor(parent)
    dev = parent.device if parent.is_cuda else torch.device("cuda", torch.cuda.current_device())
    parent = parent.to(dev, torch.int32).contiguous()
    cu_q = torch.as_tensor(cu_q, device=dev).to(torch.int32).contiguous()
    total_q = int(parent.shape[0])
    B = int(cu_q.shape[0]) - 1
    out = torch.empty((total_q, words), dtype=torch.int64, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev) if check else None
    with torch.cuda.device(dev):
        st = lib.cast_tree_bitmask(_lib.ptr(parent), _lib.ptr(cu_q), B, total_q, words, _lib.ptr(out),
                                   _lib.ptr(status), _lib.stream_of(parent))
    _lib.check(st, "cast_tree_bitmask")
    if check:
        _lib.raise_device_flags(status.item(), "tree_bitmask")
    return out[:, 0] if words == 1 else out


def greedy_accept(logits, cu_q, parent, token, *, check=False):
    """Greedy accepted paths of a packed batch, without host synchronisation.

    logits: [total_q, V] bf16/fp32 on the device (row r = packed row r);
    cu_q int32 [B+1]; parent int32 [total_q] pack-local; token int64
    [total_q] draft tokens (the root's entry is ignored).  Returns device
    tensors (path int32 [B,128] of node indices, -1 padded; path_len int32
    [B]; bonus int64 [B]; argmax int32 [total_q]).
    """
    lib = _lib.load()
    dev = logits.device
    if logits.dtype not in (torch.bfloat16, torch.float32):
        logits = logits.float()
    if logits.dim() != 2:
        raise ValueError("logits must be [total_q, V]")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    total_q, V = logits.shape
    cu_q = torch.as_tensor(cu_q, device=dev).to(torch.int32).contiguous()
    parent = torch.as_tensor(parent, device=dev).to(torch.int32).contiguous()
    token = torch.as_tensor(token, device=dev).to(torch.int64).contiguous()
    if parent.shape[0] != total_q or token.shape[0] != total_q:
        raise ValueError("parent and token need one entry per logits row")
    B = int(cu_q.shape[0]) - 1
    path = torch.empty((B, MAX_PACK), dtype=torch.int32, device=dev)
    path_len = torch.empty(B, dtype=torch.int32, device=dev)
    bonus = torch.empty(B, dtype=torch.int64, device=dev)
    argmax = torch.empty(total_q, dtype=torch.int32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev) if check else None
    dt = _lib.BF16 if logits.dtype == torch.bfloat16 else _lib.FP32
    with torch.cuda.device(dev):
        st = lib.cast_greedy_accept(_lib.ptr(logits), logits.stride(0), V, dt, _lib.ptr(cu_q), _lib.ptr(parent),
                                    _lib.ptr(token), B, total_q, _lib.ptr(argmax), _lib.ptr(path),
                                    _lib.ptr(path_len), _lib.ptr(bonus), _lib.ptr(status), _lib.stream_of(logits))
    _lib.check(st, "cast_greedy_accept")
    if check:
        _lib.raise_device_flags(status.item(), "greedy_accept")
    return path, path_len, bonus, argmax


def walk_trees(trees, logits, cu_q=None, roots=None):
    """Greedy (path, bonus) for every request of a packed verify pass.

    ``logits`` is either packed [total_q, V] (rows in pack order) or padded
    [B, P_max, V] as cast_trees/serving.py:256-261 lays it out.
    """
    pk = pack_trees(trees, roots)
    dev = logits.device
    if logits.dim() == 3:
        rows = torch.from_numpy(np.concatenate(
            [b * logits.shape[1] + np.arange(int(p)) for b, p in enumerate(pk.pack_len)])).to(dev)
        flat = logits.reshape(-1, logits.shape[-1]).index_select(0, rows)
    else:
        flat = logits[:pk.total_q]
    meta = torch.from_numpy(np.concatenate([pk.cu_q, pk.parent]).astype(np.int32)).to(dev)
    tok = torch.from_numpy(pk.token).to(dev)
    path, plen, bonus, _ = greedy_accept(flat, meta[:pk.batch + 1], meta[pk.batch + 1:], tok)
    host = torch.cat([plen.to(torch.int64), bonus, path.to(torch.int64).flatten()]).cpu().tolist()
    B = pk.batch
    lens, bon, paths = host[:B], host[B:2 * B], host[2 * B:]
    return [(paths[b * MAX_PACK:b * MAX_PACK + lens[b]], bon[b]) for b in range(B)]


def walk_tree(nodes, logits, temperature=0.0, d_logits=None, draft_temp=1.0, generator=None):
    """Walk the verified tree and return (accepted path, next root token).

    Same signature as cast_trees/decode.py:85.  Greedy (temperature 0) runs
    on the device with a single copy back; sampling (temperature > 0) is not
    part of this library.
    """
    if temperature >= 1e-5:
        raise NotImplementedError("walk_tree: only the greedy (temperature 0) walk runs on the device")
    if logits.dim() != 2:
        raise ValueError("logits must be [1 + len(nodes), V]")
    return walk_trees([nodes], logits[:1 + len(nodes)])[0]


def tree_attention_mask(n_prefix, nodes, device, dtype):
    """Additive mask (1, 1, 1+N, n_prefix+1+N): 0 where visible (the prefix
    and each row's ancestor chain), ``finfo(dtype).min`` elsewhere."""
    vis = torch.from_numpy(ancestor_matrix(nodes))
    n = vis.shape[0]
    mask = torch.zeros((1, 1, n, n_prefix + n), dtype=dtype)
    mask[0, 0, :, n_prefix:].masked_fill_(~vis, torch.finfo(dtype).min)
    return mask.to(device)
