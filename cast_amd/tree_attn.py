"""Ragged tree-verification attention on MI355X (HIP, gfx950), forward only.

Drop-in for cast_trees/tree_attn.py:116-139 ``varlen_tree_attention``: same
positional signature, argument meaning and result, with these additions
(keyword-only, all optional):

  return_lse  also return the natural-log log-sum-exp [total_q, Hq] (fp32)
  kv_split    keys per split-K chunk (0: library heuristic, SPLIT_STREAM:
              the stream-K schedule, other values < 0: no split)
  check       synchronise once and raise ValueError if the kernels flagged
              inconsistent metadata (off by default: the call never syncs)
  out         preallocated output [total_q, Hq, D]
  workspace   preallocated split-K scratch (uint8 device tensor of at least
              plan(...).workspace_bytes); one is allocated when missing
              or too small.  Calls that share a workspace must not overlap.

Each request b owns query rows [cu_q[b], cu_q[b+1]) (its pack of
P_b = pack_len[b] tokens) and key/value rows [cu_kv[b], cu_kv[b+1]) =
concat(prefix of S_b = prefix_len[b] tokens, pack).  A query sees the whole
prefix and, inside the pack, the keys whose bit is set in its ancestor words.
``ancestor_mask`` may be the reference's int64 [total_q] (one word, packs up
to 64 tokens) or an int64/uint64 [total_q, 2] (packs up to 128 tokens), as
built by ``cast_amd.tree_bitmask``.

Unlike the reference, the call needs no device-to-host copy of cu_q
(tree_attn.py:128): the kernels derive their schedule on the device.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib

_DTYPES = {torch.bfloat16: _lib.BF16, torch.float16: _lib.FP16, torch.float32: _lib.FP32}
# kv_split value asking for the stream-K schedule (CAST_SPLIT_STREAM in the C header)
SPLIT_STREAM = -2


def _as_i32(x, device):
    t = torch.as_tensor(x, device=device)
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return t.contiguous()


def _mask_words(mask, total_q, device):
    m = torch.as_tensor(mask, device=device)
    if m.dtype == torch.uint64:
        m = m.view(torch.int64)
    if m.dtype != torch.int64:
        m = m.to(torch.int64)
    if m.dim() == 1:
        words = 1
    elif m.dim() == 2 and m.shape[1] in (1, 2):
        words = int(m.shape[1])
    else:
        raise ValueError(f"ancestor_mask must be [total_q] or [total_q, 2], got {tuple(m.shape)}")
    if m.shape[0] != total_q:
        raise ValueError(f"ancestor_mask has {m.shape[0]} rows for {total_q} packed queries")
    return m.contiguous(), words


def _host_side(x):
    """Metadata the caller holds on the host (list, tuple, numpy, CPU tensor)."""
    return not (isinstance(x, torch.Tensor) and x.is_cuda)


def check_host_metadata(cu_q, prefix_len, pack_len, total_q, total_kv, words, cu_kv=None, cap=None):
    """Validate host-side packing metadata before any launch (ValueError).

    The rules are the ones the kernels apply to device-side metadata, where a
    failure only skips the request (its rows come back as zeros with
    lse = -inf): cu_q / cu_kv start at >= 0 and grow by each pack / by each
    prefix + pack, stay within total_q / total_kv, and no pack is longer than
    the ancestor words cover (64 tokens per word).  ``cap`` bounds the prefix
    in the store layout.
    """
    cq = np.asarray(cu_q.cpu() if isinstance(cu_q, torch.Tensor) else cu_q, dtype=np.int64).reshape(-1)
    S = np.asarray(prefix_len.cpu() if isinstance(prefix_len, torch.Tensor) else prefix_len,
                   dtype=np.int64).reshape(-1)
    P = np.asarray(pack_len.cpu() if isinstance(pack_len, torch.Tensor) else pack_len, dtype=np.int64).reshape(-1)
    B = P.shape[0]
    if cq.shape[0] != B + 1 or S.shape[0] != B:
        raise ValueError("cu_q needs B+1 entries and prefix_len / pack_len B entries")
    if B == 0:
        return
    if (P < 0).any() or (S < 0).any():
        raise ValueError("negative prefix_len or pack_len")
    if int(P.max()) > 64 * words:
        raise ValueError(f"a pack of {int(P.max())} tokens exceeds the {64 * words} bits of the ancestor mask "
                         f"({words} word{'s' if words > 1 else ''} per row)")
    if cq[0] < 0 or not np.array_equal(np.diff(cq), P) or cq[-1] > total_q:
        raise ValueError("cu_q must start at >= 0, grow by pack_len and end within total_q")
    if cap is not None and int(S.max()) > cap:
        raise ValueError(f"prefix_len exceeds the store capacity {cap}")
    if cu_kv is not None:
        ck = np.asarray(cu_kv.cpu() if isinstance(cu_kv, torch.Tensor) else cu_kv, dtype=np.int64).reshape(-1)
        if ck.shape[0] != B + 1 or ck[0] < 0 or not np.array_equal(np.diff(ck), S + P) or ck[-1] > total_kv:
            raise ValueError("cu_kv must start at >= 0, grow by prefix_len + pack_len and end within total_kv")
    elif int((S + P).sum()) > total_kv:
        raise ValueError("sum(prefix_len + pack_len) exceeds total_kv")


def _require_on(dev, **tensors):
    """Every given tensor (None skipped) on q's device: the kernels take raw
    device pointers, so a host or other-GPU tensor is refused here."""
    for name, t in tensors.items():
        if t is not None and t.device != dev:
            raise ValueError(f"{name} is on {t.device}, q on {dev}: all tensors must be on one GPU")


def _ready(x, esz):
    """Last dim contiguous, 16-byte aligned base and strides."""
    if x.stride(-1) != 1 or x.data_ptr() % 16 or any((s * esz) % 16 for s in x.stride()[:-1]):
        return x.contiguous()
    return x


@dataclass
class TreeAttnPlan:
    """Host-side launch geometry of one call (for benchmarks and tests)."""
    kv_split: int
    workspace_bytes: int


def plan(batch, total_q, total_kv, Hq, Hkv, D, dtype=torch.bfloat16, kv_split=0):
    lib = _lib.load()
    dt = _DTYPES[dtype]
    ws = lib.cast_tree_attn_workspace_size(batch, total_q, total_kv, Hq, Hkv, D, dt, kv_split)
    chunk = kv_split if kv_split != 0 else lib.cast_tree_attn_default_split(batch, total_q, total_kv, Hq, Hkv, D, dt)
    return TreeAttnPlan(kv_split=int(chunk), workspace_bytes=int(ws))


def varlen_tree_attention(q, k, v, cu_q, cu_kv, prefix_len, pack_len, ancestor_mask, sm_scale=None, *,
                          return_lse=False, kv_split=0, check=False, out=None, workspace=None, _stage_hook=None):
    """q: [total_q, H_q, D], k/v: [total_kv, H_kv, D] -> [total_q, H_q, D].

    cu_q / cu_kv: int32 [B+1] offsets of packs and of concat(prefix, pack).
    prefix_len / pack_len: int32 [B].  ancestor_mask: int64 [total_q] or
    [total_q, 2].  Returns ``out`` (and ``lse`` with ``return_lse``).
    """
    lib = _lib.load()
    total_q, H_q, D = q.shape
    total_kv, H_kv = k.shape[0], k.shape[1]
    assert H_q % H_kv == 0
    if not q.is_cuda:
        raise ValueError("varlen_tree_attention runs on the GPU: q/k/v must be device tensors")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    if q.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {q.dtype}: use bfloat16, float16 or float32")
    if k.dtype != q.dtype:
        k = k.to(q.dtype)
    if v.dtype != q.dtype:
        v = v.to(q.dtype)
    if tuple(v.shape) != tuple(k.shape) or k.shape[2] != D:
        raise ValueError("k and v must both be [total_kv, H_kv, D] with the head dim of q")
    esz = q.element_size()
    dev = q.device
    _require_on(dev, k=k, v=v, out=out, workspace=workspace)
    q, k, v = _ready(q, esz), _ready(k, esz), _ready(v, esz)
    mask, words = _mask_words(ancestor_mask, total_q, dev)
    if any(_host_side(x) for x in (cu_q, cu_kv, prefix_len, pack_len)):
        check_host_metadata(cu_q, prefix_len, pack_len, total_q, total_kv, words, cu_kv=cu_kv)
    cu_q = _as_i32(cu_q, dev)
    cu_kv = _as_i32(cu_kv, dev)
    prefix_len = _as_i32(prefix_len, dev)
    pack_len = _as_i32(pack_len, dev)
    B = int(pack_len.shape[0])
    if cu_q.shape[0] != B + 1 or cu_kv.shape[0] != B + 1 or prefix_len.shape[0] != B:
        raise ValueError("cu_q / cu_kv need B+1 entries and prefix_len / pack_len B entries")
    if out is None:
        out = torch.empty((total_q, H_q, D), dtype=q.dtype, device=dev)
    elif out.shape != q.shape or out.dtype != q.dtype or out.stride(-1) != 1:
        raise ValueError("out must match q's shape and dtype with a contiguous head dim")
    lse = torch.empty((total_q, H_q), dtype=torch.float32, device=dev) if return_lse else None
    dt = _DTYPES[q.dtype]
    ws_bytes = lib.cast_tree_attn_workspace_size(B, total_q, total_kv, H_q, H_kv, D, dt, kv_split)
    if ws_bytes and (workspace is None or workspace.numel() * workspace.element_size() < ws_bytes):
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev) if check else None
    args = (_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out), _lib.ptr(lse),
            _lib.ptr(cu_q), _lib.ptr(cu_kv), _lib.ptr(prefix_len), _lib.ptr(pack_len), _lib.ptr(mask), words,
            B, total_q, total_kv, H_q, H_kv, D,
            q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
            out.stride(0), out.stride(1), dt, float(sm_scale), int(kv_split),
            _lib.ptr(workspace) if ws_bytes else None, ws_bytes, _lib.ptr(status), _lib.stream_of(q))
    with _lib.on_device(dev):
        if _stage_hook is None:
            _lib.check(lib.cast_tree_attn_fwd(*args), "cast_tree_attn_fwd")
        else:
            # same two launches, with a caller callback between them (event timing)
            _stage_hook(0)
            _lib.check(lib.cast_tree_attn_partial(*args), "cast_tree_attn_partial")
            _stage_hook(1)
            _lib.check(lib.cast_tree_attn_combine(*args), "cast_tree_attn_combine")
            _stage_hook(2)
    if check:
        _lib.raise_device_flags(status.item(), "varlen_tree_attention")
    return (out, lse) if return_lse else out


def store_tree_attention(q, k_store, v_store, k_pack, v_pack, cu_q, prefix_len, pack_len, ancestor_mask,
                         sm_scale=None, *, total_kv=None, return_lse=False, kv_split=0, check=False, out=None,
                         workspace=None):
    """Tree-verification attention reading the prefix K/V where it is stored.

    The same attention as ``varlen_tree_attention``, but request b's keys are
    its first S_b = prefix_len[b] store slots followed by its pack, with no
    ragged K/V assembled (cast_trees/serving.py:61-68 copies both into one
    tensor per layer):

      q                [total_q, H_q, D]  (any token/head strides)
      k_store/v_store  [B, H_kv, cap, D]  per-request store (serving.py:191-205)
      k_pack/v_pack    [H_kv, total_q, D] the pass's own K/V, pack token j of
                       request b at index cu_q[b] + j (HF's key[0] / value[0])
      total_kv         host bound on sum(S_b + P_b) used to size the launch and
                       workspace (default B*cap + total_q, always valid)

    Returns ``out`` [total_q, H_q, D] (and ``lse`` with ``return_lse``).
    """
    lib = _lib.load()
    total_q, H_q, D = q.shape
    if k_store.dim() != 4 or k_pack.dim() != 3:
        raise ValueError("k_store must be [B, H_kv, cap, D] and k_pack [H_kv, total_q, D]")
    B, H_kv, cap = int(k_store.shape[0]), int(k_store.shape[1]), int(k_store.shape[2])
    assert H_q % H_kv == 0
    if not q.is_cuda:
        raise ValueError("store_tree_attention runs on the GPU: tensors must be on the device")
    if tuple(v_store.shape) != tuple(k_store.shape) or k_store.shape[3] != D:
        raise ValueError("k_store and v_store must both be [B, H_kv, cap, D] with the head dim of q")
    if tuple(k_pack.shape) != (H_kv, total_q, D) or tuple(v_pack.shape) != (H_kv, total_q, D):
        raise ValueError(f"k_pack/v_pack must be [{H_kv}, {total_q}, {D}]")
    if q.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {q.dtype}: use bfloat16, float16 or float32")
    if any(t.dtype != q.dtype for t in (k_store, v_store, k_pack, v_pack)):
        raise ValueError("q, the store and the pack K/V must share one dtype (the store is read in place)")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    esz = q.element_size()
    dev = q.device
    _require_on(dev, k_store=k_store, v_store=v_store, k_pack=k_pack, v_pack=v_pack, out=out, workspace=workspace)
    q, k_pack, v_pack = _ready(q, esz), _ready(k_pack, esz), _ready(v_pack, esz)
    if _ready(k_store, esz) is not k_store or _ready(v_store, esz) is not v_store:
        raise ValueError("the store needs a contiguous head dim and 16-byte aligned strides")
    if total_kv is None:
        total_kv = B * cap + total_q
    total_kv = int(total_kv)
    mask, words = _mask_words(ancestor_mask, total_q, dev)
    if any(_host_side(x) for x in (cu_q, prefix_len, pack_len)):
        check_host_metadata(cu_q, prefix_len, pack_len, total_q, total_kv, words, cap=cap)
    cu_q = _as_i32(cu_q, dev)
    prefix_len = _as_i32(prefix_len, dev)
    pack_len = _as_i32(pack_len, dev)
    if cu_q.shape[0] != B + 1 or prefix_len.shape[0] != B or pack_len.shape[0] != B:
        raise ValueError("cu_q needs B+1 entries and prefix_len / pack_len B entries (B = store batch)")
    if out is None:
        out = torch.empty((total_q, H_q, D), dtype=q.dtype, device=dev)
    elif tuple(out.shape) != tuple(q.shape) or out.dtype != q.dtype or out.stride(-1) != 1:
        raise ValueError("out must match q's shape and dtype with a contiguous head dim")
    lse = torch.empty((total_q, H_q), dtype=torch.float32, device=dev) if return_lse else None
    dt = _DTYPES[q.dtype]
    ws_bytes = lib.cast_tree_attn_workspace_size(B, total_q, total_kv, H_q, H_kv, D, dt, kv_split)
    if ws_bytes and (workspace is None or workspace.numel() * workspace.element_size() < ws_bytes):
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev) if check else None
    with _lib.on_device(dev):
        st = lib.cast_tree_attn_store_fwd(
            _lib.ptr(q), _lib.ptr(k_store), _lib.ptr(v_store), _lib.ptr(k_pack), _lib.ptr(v_pack), _lib.ptr(out),
            _lib.ptr(lse), _lib.ptr(cu_q), _lib.ptr(prefix_len), _lib.ptr(pack_len), _lib.ptr(mask), words,
            B, total_q, total_kv, cap, H_q, H_kv, D, q.stride(0), q.stride(1),
            k_store.stride(0), k_store.stride(1), k_store.stride(2), v_store.stride(0), v_store.stride(1),
            v_store.stride(2), k_pack.stride(1), k_pack.stride(0), v_pack.stride(1), v_pack.stride(0),
            out.stride(0), out.stride(1), dt, float(sm_scale), int(kv_split),
            _lib.ptr(workspace) if ws_bytes else None, ws_bytes, _lib.ptr(status), _lib.stream_of(q))
    _lib.check(st, "cast_tree_attn_store_fwd")
    if check:
        _lib.raise_device_flags(status.item(), "store_tree_attention")
    return (out, lse) if return_lse else out
