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
  cache_layers        (n_layers, get, put) over a transformers DynamicCache
                      (cast_trees/verify.py:28-45)
  gather_cache        drop-in for cast_trees/verify.py:48-60: the accepted
                      rows move in place on the device, all layers in one
                      launch (K4), and the layers are cut to the kept length
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from .tree import MAX_PACK, ancestor_matrix, pack_trees


def _i32_on(x, dev):
    """x as a contiguous int32 tensor on dev (no copy when it already is one)."""
    if isinstance(x, torch.Tensor) and x.dtype is torch.int32 and x.device == dev and x.is_contiguous():
        return x
    return torch.as_tensor(x, device=dev).to(torch.int32).contiguous()


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
    parent = _i32_on(parent, dev)
    cu_q = _i32_on(cu_q, dev)
    total_q = int(parent.shape[0])
    B = int(cu_q.shape[0]) - 1
    out = torch.empty((total_q, words), dtype=torch.int64, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev) if check else None
    with _lib.on_device(dev):
        st = lib.cast_tree_bitmask(_lib.ptr(parent), _lib.ptr(cu_q), B, total_q, words, _lib.ptr(out),
                                   _lib.ptr(status), _lib.stream_of(parent))
    _lib.check(st, "cast_tree_bitmask")
    if check:
        _lib.raise_device_flags(status.item(), "tree_bitmask")
    return out[:, 0] if words == 1 else out


def greedy_accept(logits, cu_q, parent, token, *, check=False):
    """Greedy accepted paths of a packed batch, without host synchronisation.

    logits: [total_q, V] bf16/fp16/fp32 on the device (row r = packed row r;
    other float dtypes are widened to fp32 first);
    cu_q int32 [B+1]; parent int32 [total_q] pack-local; token int64
    [total_q] draft tokens (the root's entry is ignored).  Returns device
    tensors (path int32 [B,128] of node indices, -1 padded; path_len int32
    [B]; bonus int64 [B]; argmax int32 [total_q]).
    """
    lib = _lib.load()
    if not logits.is_cuda:
        raise ValueError("greedy_accept runs on the GPU: logits must be a device tensor")
    dev = logits.device
    if logits.dtype not in (torch.bfloat16, torch.float16, torch.float32):
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
    dt = {torch.bfloat16: _lib.BF16, torch.float16: _lib.FP16}.get(logits.dtype, _lib.FP32)
    with _lib.on_device(dev):
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


def ancestor_words(vis):
    """Two 64-bit words per row of a boolean visibility matrix (n <= 128):
    bit j of word j // 64 is vis[i, j] (the layout of the reference's int64
    mask, cast_trees/serving.py:218-222, extended to a second word)."""
    vis = np.asarray(vis, dtype=bool)
    n = vis.shape[0]
    if vis.shape != (n, n) or n > MAX_PACK:
        raise ValueError(f"a square visibility matrix of at most {MAX_PACK} rows")
    bits = np.zeros((n, 2 * 64), dtype=np.uint8)
    bits[:, :n] = vis
    return np.packbits(bits, axis=1, bitorder="little").view(np.int64)


def tree_attention_mask(n_prefix, nodes, device, dtype):
    """Additive mask (1, 1, 1+N, n_prefix+1+N): 0 where visible (the prefix
    and each row's ancestor chain), ``finfo(dtype).min`` elsewhere.

    On a GPU the mask is uploaded from pinned memory without a host wait,
    and the kernel metadata of the "cast_tree" attention (cu_q, cu_kv,
    prefix_len, pack_len and the ancestor words, from the same host
    ancestor matrix) rides along as an attribute of the returned tensor, so
    the verify forward reads nothing back from the device.
    """
    vis_np = ancestor_matrix(nodes)
    vis = torch.from_numpy(vis_np)
    n = vis.shape[0]
    device = torch.device(device)
    pinned = device.type == "cuda"
    mask = torch.zeros((1, 1, n, n_prefix + n), dtype=dtype, pin_memory=pinned)
    mask[0, 0, :, n_prefix:].masked_fill_(~vis, torch.finfo(dtype).min)
    if not pinned:
        return mask.to(device)
    dev_mask = mask.to(device, non_blocking=True)
    if n <= MAX_PACK:
        # int32 [4n + 6]: the words (n x 2 int64) first, then
        # cu_q [0, n], cu_kv [0, S + n], prefix_len [S], pack_len [n]
        host = torch.zeros(4 * n + 6, dtype=torch.int32, pin_memory=True)
        host[:4 * n].view(torch.int64).view(n, 2).copy_(torch.from_numpy(ancestor_words(vis_np)))
        host[4 * n:] = torch.tensor([0, n, 0, n_prefix + n, n_prefix, n], dtype=torch.int32)
        d = host.to(device, non_blocking=True)
        meta = (d[4 * n:4 * n + 2], d[4 * n + 2:4 * n + 4], d[4 * n + 4:4 * n + 5], d[4 * n + 5:],
                d[:4 * n].view(torch.int64).view(n, 2))
        dev_mask._cast_tree_meta = (None if dev_mask.is_inference() else dev_mask._version, n_prefix + n, meta)
    return dev_mask


def cache_layers(cache):
    """(n_layers, get, put) over a transformers DynamicCache.

    Recent transformers keep one object per layer with ``.keys`` /
    ``.values``; older releases keep two lists, ``key_cache`` and
    ``value_cache``.  ``get(i)`` returns layer i's (K, V) and ``put(i, k, v)``
    replaces them, whichever layout the cache has (cast_trees/verify.py:28-45
    serves the same two layouts).
    """
    per_layer = getattr(cache, "layers", None)
    if per_layer and hasattr(per_layer[0], "keys"):
        def get(i):
            entry = per_layer[i]
            return entry.keys, entry.values

        def put(i, k, v):
            entry = per_layer[i]
            entry.keys = k
            entry.values = v
        return len(per_layer), get, put
    k_list, v_list = cache.key_cache, cache.value_cache

    def get(i):
        return k_list[i], v_list[i]

    def put(i, k, v):
        k_list[i] = k
        v_list[i] = v
    return len(k_list), get, put


def gather_cache(cache, n_prefix, keep):
    """Keep the first ``n_prefix`` cached positions and then the packed
    entries ``keep`` (``[0] + [i + 1 for i in path]``, as the decoder builds
    it), in order, in every layer of a batch-one cache.

    The kept rows n_prefix + keep[j] move to n_prefix + j in place, K and V
    of all layers in one cast_store_append launch (each workgroup reads its
    rows before it writes any, so the overlap is safe), and every layer
    becomes a view of length n_prefix + len(keep).  The reference's
    index_select copies every layer whole.
    """
    from .tree_attn import _DTYPES
    n_layers, get, put = cache_layers(cache)
    keep = [int(x) for x in keep]
    if n_layers == 0:
        return cache
    layers = [get(i) for i in range(n_layers)]
    k0 = layers[0][0]
    if k0.dim() != 4 or k0.shape[0] != 1:
        raise ValueError("gather_cache: a batch-one cache of [1, heads, seq, head_dim] layers")
    if not k0.is_cuda:
        raise ValueError("gather_cache runs on the GPU: the cache must hold device tensors")
    _, Hkv, T, D = k0.shape
    n = len(keep)
    n_pack = T - n_prefix
    if n and (keep[0] != 0 or n > min(MAX_PACK, n_pack) or min(keep[1:], default=1) < 1 or max(keep) >= n_pack):
        raise ValueError(f"keep must be [0] + pack indices in [1, {n_pack}) with at most {MAX_PACK} entries")
    if n_prefix < 0 or n_pack < 0:
        raise ValueError("n_prefix beyond the cached length")
    if n > 1:
        shape, stride = k0.shape, k0.stride()
        for k, v in layers:
            if k.shape != shape or v.shape != shape or k.stride() != stride or v.stride() != stride \
                    or k.dtype != k0.dtype or v.dtype != k0.dtype or k.device != k0.device or v.device != k0.device:
                raise ValueError("gather_cache: every layer's K and V must share shape, strides, dtype and device")
        if stride[3] != 1 or (stride[2] * k0.element_size()) % 16:
            raise ValueError("gather_cache: contiguous head_dim rows, 16-byte aligned")
        lib = _lib.load()
        step = n_prefix * stride[2] * k0.element_size()   # the pack starts at row n_prefix
        addrs = [k.data_ptr() for k, _ in layers] + [v.data_ptr() for _, v in layers]
        if any(a % 16 for a in addrs):
            raise ValueError("gather_cache: 16-byte aligned layers")
        L = n_layers
        ptrs = lambda xs: (ctypes.c_void_p * L)(*xs)
        # one host-to-device copy of the int32 metadata: src_row, path_len,
        # store_len, new_len, then the [1, MAX_PACK] path
        meta = np.full(4 + MAX_PACK, -1, dtype=np.int32)
        meta[:4] = (0, n - 1, n_prefix, 0)
        meta[4:4 + n - 1] = [x - 1 for x in keep[1:]]
        d32 = torch.from_numpy(meta).to(k0.device)
        with _lib.on_device(k0.device):
            st = lib.cast_store_append(
                ptrs([a + step for a in addrs[:L]]), ptrs([a + step for a in addrs[L:]]), ptrs(addrs[:L]),
                ptrs(addrs[L:]), L, _lib.ptr(d32[0:1]), _lib.ptr(d32[4:]), MAX_PACK,
                _lib.ptr(d32[1:2]), _lib.ptr(d32[2:3]), _lib.ptr(d32[3:4]), 1, n_pack, T, Hkv, D,
                stride[2], stride[1], stride[2], stride[1], stride[0], stride[1], stride[2],
                stride[0], stride[1], stride[2], _DTYPES[k0.dtype], None, _lib.stream_of(k0))
        _lib.check(st, "cast_store_append")
    for i, (k, v) in enumerate(layers):
        put(i, k[:, :, :n_prefix + n], v[:, :, :n_prefix + n])
    if hasattr(cache, "_seen_tokens"):
        cache._seen_tokens = n_prefix + n
    return cache
