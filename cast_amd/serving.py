"""The verify pass's attention hook, reading the per-request KV store in place.

Mirrors the attention side of cast_trees/serving.py:

  VarlenPlan / PLAN   state of one ragged verify pass (serving.py:30-44),
                      read by the hook once per layer
  PACK_KV             the pass's post-RoPE pack K/V of every layer
                      (serving.py:45), for the caller's accepted-path append
  _varlen_attention   the HF AttentionInterface callee (serving.py:48-72),
                      registered as "cast_varlen" (serving.py:75) when
                      transformers is importable
  begin_verify        the packing half of BatchedServer._verify_varlen
                      (serving.py:208-253): packed tokens, positions,
                      offsets and ancestor words, then PLAN.set
  append_store        BatchedServer._append_store (serving.py:264-289): the
                      accepted rows of every layer into the store in one
                      launch; append_accepted does it from greedy_accept's
                      device outputs without a host sync
  _tree_attention     the batch-one verify of cast_trees/decode.py:166-171
                      (target forward with the additive tree mask of
                      cast_trees/verify.py:15-25) through the same kernel,
                      registered as "cast_tree"

The reference hook assembles a ragged [total_kv, Hkv, D] K/V per layer by
gathering every request's prefix out of the store and scattering the pack
behind it, up-casts all of it to fp32, and only then calls the attention
(serving.py:61-71).  Here the kernel reads the prefix where it lies in
buf_k/buf_v [B, Hkv, cap, D] and the pack from the forward's own K/V, in the
store's dtype (bf16 products are exact in the fp32 MFMA accumulators, so the
up-cast adds no precision to the score dot products; the probabilities are
rounded to bf16 before the value product, as the reference kernel does for
bf16 inputs, tree_attn.py:66,87).
"""
from __future__ import annotations

import ctypes
import weakref

import numpy as np
import torch
import torch.nn.functional as F

from .tree import MAX_PACK
from .tree_attn import store_tree_attention
from .verify import _i32_on, tree_bitmask


class VerifyPassState:
    """Everything the attention hook reads while one batched verify forward
    runs: the per-layer stores, the packed metadata and the index of the
    next layer.  ``set`` arms the hook with those fields; ``clear`` disarms
    it and drops the store references.  (The method names are the ones the
    reference's server calls, cast_trees/serving.py:244, 253.)"""

    def __init__(self):
        self.active = False
        self.layer = 0
        self.workspace = None

    def set(self, **fields):
        for name, value in fields.items():
            setattr(self, name, value)
        self.layer = 0
        self.active = True

    def clear(self):
        self.active = False
        self.buf_k = None
        self.buf_v = None
        self.workspace = None


PLAN = VerifyPassState()
# Per-layer K and V of the packed tree tokens (rotary already applied), as the
# current verify forward hands them to the hook: PACK_KV["k"][layer] is
# [Hkv, total_q, D].  The accepted-path append reads them after the forward.
PACK_KV = {"k": [], "v": []}


class _PackRecord:
    """The pack K/V addresses of the current verify pass, recorded by the
    hook as each layer's key[0] / value[0] arrives and checked then (shape,
    strides, dtype, device and alignment alike in every layer), so that the
    append after the forward needs no per-layer Python checks."""

    def __init__(self):
        self.begin(0)

    def begin(self, layers):
        self.k = (ctypes.c_void_p * layers)()
        self.v = (ctypes.c_void_p * layers)()
        self.objs = [None] * layers
        self.sig = None
        self.ok = True

    def note(self, li, k, v):
        if li >= len(self.objs):
            self.ok = False
            return
        sig = (k.shape, k.stride(), v.shape, v.stride(), k.dtype, v.dtype, k.get_device(), v.get_device())
        if self.sig is None:
            self.sig = sig
        elif sig != self.sig:
            self.ok = False
        kp, vp = k.data_ptr(), v.data_ptr()
        if (kp | vp) & 15:
            self.ok = False
        self.k[li], self.v[li] = kp, vp
        self.objs[li] = (k, v)

    def arrays_for(self, lay, pack_k, pack_v):
        """(k_ptrs, v_ptrs, k_strides, v_strides, total_q) when the record
        covers exactly these per-layer tensors, else None."""
        if not self.ok or self.sig is None or len(self.objs) != lay["L"] or len(pack_k) != lay["L"]:
            return None
        for (k, v), pk, pv in zip(self.objs, pack_k, pack_v):
            if k is not pk or v is not pv:
                return None
        kshape, kstride, vshape, vstride, kdt, vdt, kdev, vdev = self.sig
        Hkv, D = lay["Hkv"], lay["D"]
        if (len(kshape) != 3 or tuple(kshape) != tuple(vshape) or kshape[0] != Hkv or kshape[2] != D
                or kstride[2] != 1 or vstride[2] != 1 or kdt is not lay["dtype"] or vdt is not lay["dtype"]
                or kdev != lay["dev_index"] or vdev != lay["dev_index"]):
            return None
        return self.k, self.v, (kstride[1], kstride[0]), (vstride[1], vstride[0]), int(kshape[1])


_PACK_REC = _PackRecord()


def _plain_attention(query, key, value, attention_mask, scaling):
    """A forward that is not a tree verify (prefill, ordinary decode): torch
    SDPA on HF's [1, H, n, D] layout, causal when there is no mask and more
    than one query, handed back token-major as HF's attention callees do."""
    mask = None if isinstance(attention_mask, bool) else attention_mask
    causal = mask is None and query.shape[2] > 1
    o = F.scaled_dot_product_attention(query, key, value, attn_mask=mask, scale=scaling, is_causal=causal,
                                       enable_gqa=True)
    return o.transpose(1, 2).contiguous(), None


def _varlen_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kw):
    """HF attention callee: query [1, Hq, total_q, D], key/value [1, Hkv, total_q, D]
    -> ([1, total_q, Hq, D], None).  Outside a verify pass (cast_trees/
    serving.py:49-55) it is plain SDPA."""
    if not PLAN.active:
        return _plain_attention(query, key, value, attention_mask, scaling)

    li = PLAN.layer
    PLAN.layer += 1
    while len(PACK_KV["k"]) <= li:
        PACK_KV["k"].append(None)
        PACK_KV["v"].append(None)
    PACK_KV["k"][li], PACK_KV["v"][li] = key[0], value[0]
    _PACK_REC.note(li, key[0], value[0])
    buf_k, buf_v = PLAN.buf_k[li], PLAN.buf_v[li]
    q = query[0].transpose(0, 1)                          # [total_q, Hq, D] view
    dt = buf_k.dtype
    k_pack, v_pack = key[0], value[0]
    if q.dtype != dt:
        q = q.to(dt)
    if k_pack.dtype != dt:
        k_pack, v_pack = k_pack.to(dt), v_pack.to(dt)
    if getattr(PLAN, "workspace", None) is None:
        # split-K scratch, sized once per pass and shared by every layer
        PLAN.workspace = torch.empty(max(workspace_bytes(q, buf_k, PLAN.total_kv), 256), dtype=torch.uint8,
                                     device=q.device)
    out = store_tree_attention(q, buf_k, buf_v, k_pack, v_pack, PLAN.cu_q, PLAN.prefix_len, PLAN.pack_len,
                               PLAN.ancestor_mask, sm_scale=scaling, total_kv=PLAN.total_kv,
                               workspace=PLAN.workspace)
    return out.to(query.dtype).unsqueeze(0), None


def workspace_bytes(q, buf_k, total_kv):
    """Split-K workspace of one layer call with these shapes."""
    from . import _lib
    from .tree_attn import _DTYPES
    B, H_kv = int(buf_k.shape[0]), int(buf_k.shape[1])
    total_q, H_q, D = q.shape
    return int(_lib.load().cast_tree_attn_workspace_size(B, total_q, int(total_kv), H_q, H_kv, D,
                                                         _DTYPES[buf_k.dtype], 0))


def begin_verify(buf_k, buf_v, store_len, roots, trees, seq_lens, device=None):
    """Pack B trees for one verify forward and activate the hook.

    buf_k / buf_v: per-layer stores [B, Hkv, cap, D]; store_len[b]: tokens of
    request b in the store; roots[b]: the root token (last committed token);
    trees[b]: its TreeNode list; seq_lens[b]: the root's position.  Returns
    (input_ids [1, total_q], position_ids [1, total_q], cu_q list), the inputs
    of the target forward, which runs with ``_attn_implementation =
    "cast_varlen"``; call ``PLAN.clear()`` afterwards (serving.py:244-253).
    """
    dev = torch.device(device) if device is not None else buf_k[0].device
    B = len(trees)
    pack_len = [1 + len(t) for t in trees]
    if max(pack_len) > MAX_PACK:
        raise ValueError(f"a pack holds at most {MAX_PACK} tokens (root + {MAX_PACK - 1} nodes)")
    cap = int(buf_k[0].shape[2])
    if max(store_len) > cap:
        raise ValueError("store_len exceeds the store capacity")
    tok, pos, parent = [], [], []
    for b, nodes in enumerate(trees):
        tok.append(int(roots[b]))
        pos.append(int(seq_lens[b]))
        parent.append(-1)
        for nd in nodes:
            tok.append(int(nd.token))
            pos.append(int(seq_lens[b]) + int(nd.depth))
            parent.append(int(nd.parent) + 1)
    cu_q = [0]
    for p in pack_len:
        cu_q.append(cu_q[-1] + p)
    total_q = cu_q[-1]
    # one host-to-device copy for all int32 metadata
    meta = torch.from_numpy(np.asarray(cu_q + list(store_len) + pack_len + parent, dtype=np.int32)).to(dev)
    cu_q_t = meta[:B + 1]
    prefix_t = meta[B + 1:2 * B + 1]
    pack_t = meta[2 * B + 1:3 * B + 1]
    parent_t = meta[3 * B + 1:]
    words = tree_bitmask(parent_t, cu_q_t, 2)
    n_layers = len(buf_k)
    PACK_KV["k"], PACK_KV["v"] = [None] * n_layers, [None] * n_layers
    _PACK_REC.begin(n_layers)
    PLAN.set(buf_k=buf_k, buf_v=buf_v, prefix_len=prefix_t, pack_len=pack_t, cu_q=cu_q_t,
             total_kv=int(sum(store_len)) + total_q, ancestor_mask=words, parent=parent_t, workspace=None)
    ids = torch.tensor([tok], dtype=torch.long, device=dev)
    pos_ids = torch.tensor([pos], dtype=torch.long, device=dev)
    return ids, pos_ids, cu_q


# ---- accepted-path KV append (cast_trees/serving.py:264-289)

_STORE_LAYOUTS = {}   # (id and address of layer 0's K store, layers) -> (weakrefs, addresses, checked layout)


def _ptr_array(tensors):
    """Host array of the tensors' device addresses (the C ABI copies it into
    the kernel arguments)."""
    return (ctypes.c_void_p * len(tensors))(*[t.data_ptr() for t in tensors])


def _store_layout(buf_k, buf_v):
    """Check the per-layer stores once and keep their address arrays.  The
    stores of a decode loop persist across rounds, so the result is reused
    while the same tensor objects sit at the same addresses (weak references
    tell a live object from a new one that got a freed object's id)."""
    L = len(buf_k)
    if len(buf_v) != L or L == 0:
        raise ValueError("one K and one V store per layer")
    tensors = (*buf_k, *buf_v)
    addrs = [t.data_ptr() for t in tensors]
    key = (id(buf_k[0]), addrs[0], L)
    hit = _STORE_LAYOUTS.get(key)
    if hit is not None and hit[1] == addrs and all(r() is t for r, t in zip(hit[0], tensors)):
        return hit[2]
    k0 = buf_k[0]
    B, Hkv, cap, D = (int(x) for x in k0.shape)
    for t in tensors:
        if tuple(t.shape) != (B, Hkv, cap, D) or t.stride() != k0.stride() or t.dtype != k0.dtype:
            raise ValueError("every layer's store must share shape, strides and dtype")
        if t.device != k0.device:
            raise ValueError("every layer's store must be on one device")
    if k0.stride(-1) != 1 or any(t.data_ptr() % 16 for t in tensors):
        raise ValueError("the store needs a contiguous, 16-byte aligned head dim")
    layout = dict(k=_ptr_array(buf_k), v=_ptr_array(buf_v), L=L, B=B, Hkv=Hkv, cap=cap, D=D, dtype=k0.dtype,
                  device=k0.device, dev_index=k0.get_device(), store_k=tuple(k0.stride()[:3]),
                  store_v=tuple(buf_v[0].stride()[:3]))
    if len(_STORE_LAYOUTS) >= 8:
        _STORE_LAYOUTS.clear()
    _STORE_LAYOUTS[key] = (tuple(weakref.ref(t) for t in tensors), addrs, layout)
    return layout


def _pack_arrays(lay, pack_k, pack_v):
    """Check one round's pack K/V (new tensors every verify pass) against the
    stores and return their address arrays, strides and total_q.  One tight
    pass over the 2L tensors: the common shape, strides, dtype and device,
    and 16-byte aligned bases."""
    L = lay["L"]
    if len(pack_k) != L or len(pack_v) != L:
        raise ValueError("one pack K and one pack V tensor per layer")
    Hkv, D, dt, dev = lay["Hkv"], lay["D"], lay["dtype"], lay["dev_index"]
    out = []
    for ps in (pack_k, pack_v):
        ref = ps[0]
        shape, stride = ref.shape, ref.stride()
        if len(shape) != 3 or shape[0] != Hkv or shape[2] != D or stride[2] != 1:
            raise ValueError(f"pack K/V must be [{Hkv}, total_q, {D}] with a contiguous head dim")
        ptrs = []
        for t in ps:
            if t.shape != shape or t.stride() != stride or t.dtype is not dt or t.get_device() != dev:
                raise ValueError("pack K/V must share shape, strides, the store's dtype and device in every layer")
            ptrs.append(t.data_ptr())
        if any(a & 15 for a in ptrs):
            raise ValueError("pack K/V need 16-byte aligned rows")
        out.append(((ctypes.c_void_p * L)(*ptrs), (stride[1], stride[0]), int(shape[1])))
    (kp, kst, tq), (vp, vst, tq_v) = out
    if tq_v != tq:
        raise ValueError("pack K and V must hold the same packed tokens")
    return kp, vp, kst, vst, tq


def _append_launch(buf_k, buf_v, pack_k, pack_v, src_row, path, path_len, store_len, new_len, status=None):
    """The KV append over every layer (all arguments device tensors; buf_* /
    pack_* lists of per-layer tensors).  Stream-ordered, no host sync."""
    from . import _lib
    from .tree_attn import _DTYPES
    lib = _lib.load()
    lay = _store_layout(buf_k, buf_v)
    dev = lay["device"]
    if dev.type != "cuda":
        raise ValueError("the KV append runs on the GPU: stores and packs must be device tensors")
    rec = _PACK_REC.arrays_for(lay, pack_k, pack_v)
    kp, vp, kp_st, vp_st, total_q = rec if rec is not None else _pack_arrays(lay, pack_k, pack_v)
    di = lay["dev_index"]
    for name, t in (("src_row", src_row), ("path", path), ("path_len", path_len), ("store_len", store_len),
                    ("new_len", new_len), ("status", status)):
        if t is not None and t.get_device() != di:
            raise ValueError(f"{name} must be on the stores' device {dev}")
    n = int(src_row.shape[0])
    if n > lay["B"] or path.dim() != 2 or path.shape[0] < n or path.shape[1] < MAX_PACK:
        raise ValueError("path must be [B, >=128] (as written by greedy_accept) for B <= the store batch")
    with _lib.on_device(dev):
        st = lib.cast_store_append(
            kp, vp, lay["k"], lay["v"], lay["L"], _lib.ptr(src_row), _lib.ptr(path), path.stride(0),
            _lib.ptr(path_len), _lib.ptr(store_len), _lib.ptr(new_len), n, total_q, lay["cap"], lay["Hkv"],
            lay["D"], *kp_st, *vp_st, *lay["store_k"], *lay["store_v"], _DTYPES[lay["dtype"]], _lib.ptr(status),
            _lib.stream_of(buf_k[0]))
    _lib.check(st, "cast_store_append")


def append_accepted(buf_k, buf_v, store_len, cu_q, path, path_len, pack_k=None, pack_v=None, *, check=False):
    """Append every request's root and accepted nodes to its store slot, all
    layers in one launch, straight from greedy_accept's device outputs.

    store_len, cu_q: int32 device tensors [B] / [B+1]; path int32 [B, 128],
    path_len int32 [B] (greedy_accept).  pack_k / pack_v default to PACK_KV.
    Returns the new lengths (int32 [B], on the device).  No host sync.
    """
    pack_k = PACK_KV["k"] if pack_k is None else pack_k
    pack_v = PACK_KV["v"] if pack_v is None else pack_v
    dev = buf_k[0].device
    store_len = _i32_on(store_len, dev)
    cu_q = _i32_on(cu_q, dev)
    new_len = torch.empty_like(store_len)
    status = torch.zeros(1, dtype=torch.int32, device=dev) if check else None
    _append_launch(buf_k, buf_v, pack_k, pack_v, cu_q[:-1], _i32_on(path, dev), _i32_on(path_len, dev), store_len,
                   new_len, status)
    if check:
        from . import _lib
        _lib.raise_device_flags(status.item(), "append_accepted")
    return new_len


def append_store(buf_k, buf_v, store_len, cu_q, keep, accepted, rows):
    """Drop-in for BatchedServer._append_store (cast_trees/serving.py:264-289).

    Keeps the surviving requests ``rows`` (compacting the stores when some
    finished, growing them when a slot would overflow, as the reference does)
    and appends request b's packed rows cu_q[b] + keep[b][j] (keep[b] = [0] +
    [i + 1 for i in path]) at slots store_len[b] + j.  The scatter over every
    layer is one kernel launch.  Returns (buf_k, buf_v, new_len).
    """
    dev = buf_k[0].device
    if len(rows) != len(store_len):
        # requests that finished leave the batch: keep only the store rows of `rows`
        survivors = torch.as_tensor(list(rows), dtype=torch.long, device=dev)
        buf_k = [x.index_select(0, survivors) for x in buf_k]
        buf_v = [x.index_select(0, survivors) for x in buf_v]
    new_len = [int(store_len[b]) + int(accepted[b]) for b in rows]
    cap = int(buf_k[0].shape[2])
    need = max(new_len, default=0)
    if need > cap:
        # a slot would overflow: every store is widened to max(need, 2 * cap)
        # slots, the new ones zero (the reference's growth rule)
        wide = max(need, 2 * cap)

        def widen(x):
            y = x.new_zeros((x.shape[0], x.shape[1], wide, x.shape[3]))
            y[:, :, :cap].copy_(x)
            return y
        buf_k = [widen(x) for x in buf_k]
        buf_v = [widen(x) for x in buf_v]
    if not rows:
        return buf_k, buf_v, new_len
    path = np.full((len(rows), MAX_PACK), -1, dtype=np.int32)
    meta = np.zeros((3, len(rows)), dtype=np.int32)
    for nb, b in enumerate(rows):
        kb = list(keep[b])
        if not kb or kb[0] != 0 or len(kb) != int(accepted[b]) or len(kb) > MAX_PACK:
            raise ValueError("keep[b] must be [0] + [i + 1 for i in path] with accepted[b] entries")
        path[nb, :len(kb) - 1] = [k - 1 for k in kb[1:]]
        meta[:, nb] = (int(cu_q[b]), len(kb) - 1, int(store_len[b]))
    host = torch.from_numpy(np.concatenate([meta.ravel(), path.ravel()])).to(dev)
    n = len(rows)
    _append_launch(buf_k, buf_v, PACK_KV["k"], PACK_KV["v"], host[:n], host[3 * n:].view(n, MAX_PACK),
                   host[n:2 * n], host[2 * n:3 * n], None)
    return buf_k, buf_v, new_len


# ---- batch-one verify (cast_trees/decode.py:166-171): the target forward over
# [root] + nodes with the additive tree mask of cast_trees/verify.py:15-25,
# routed through the same kernel

# the last mask seen (weak reference, so a new tensor never matches) with its
# version and key length, and the kernel metadata derived from it
_TREE_META = {"ref": None, "key": None, "meta": None}


def _tree_meta(mask, n_kv):
    """Kernel metadata for a (1, 1, n, S + n) additive tree mask, or None when
    the mask is not one (a masked prefix key, or a pack longer than 128).  The
    same mask object is handed to every layer of one forward: derived once.
    A mask made by ``cast_amd.verify.tree_attention_mask`` carries its
    metadata (built on the host from the same ancestor matrix) and is never
    read back; any other mask is checked on the device, with one host wait."""
    key = (None if mask.is_inference() else mask._version, n_kv)
    tag = getattr(mask, "_cast_tree_meta", None)
    if tag is not None and (tag[0], tag[1]) == key:
        return tag[2]
    ref = _TREE_META["ref"]
    if ref is not None and ref() is mask and _TREE_META["key"] == key:
        return _TREE_META["meta"]
    n, width = int(mask.shape[-2]), int(mask.shape[-1])
    S = width - n
    if mask.dim() != 4 or mask.shape[0] != 1 or mask.shape[1] != 1 or S < 0 or width != n_kv or n > MAX_PACK:
        return None
    vis = mask[0, 0] == 0
    if S and not bool(vis[:, :S].all()):
        return None
    tree = vis[:, S:].to(torch.int64)
    j = torch.arange(n, device=mask.device)
    bits = tree << (j % 64)
    words = torch.zeros((n, 2), dtype=torch.int64, device=mask.device)
    words[:, 0] = bits[:, :64].sum(dim=1)          # distinct bits: the sum is the OR
    if n > 64:
        words[:, 1] = bits[:, 64:].sum(dim=1)
    meta = torch.tensor([0, n, 0, n_kv, S, n], dtype=torch.int32, device=mask.device)
    out = (meta[0:2], meta[2:4], meta[4:5], meta[5:6], words)
    _TREE_META.update(ref=weakref.ref(mask), key=key, meta=out)
    return out


def _tree_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kw):
    """HF attention callee for the batch-one tree verify pass: query [1, Hq, n, D],
    key/value [1, Hkv, S + n, D] (the cache after its update), attention_mask the
    (1, 1, n, S + n) additive tree mask -> ([1, n, Hq, D], None).  Anything else
    (prefill, no mask, a non-tree mask) runs plain SDPA."""
    meta = None
    if (isinstance(attention_mask, torch.Tensor) and query.shape[0] == 1 and query.is_cuda
            and query.dtype in (torch.bfloat16, torch.float16, torch.float32)):
        meta = _tree_meta(attention_mask, int(key.shape[2]))
    if meta is None:
        return _plain_attention(query, key, value, attention_mask, scaling)
    from .tree_attn import varlen_tree_attention
    cu_q, cu_kv, prefix_len, pack_len, words = meta
    out = varlen_tree_attention(query[0].transpose(0, 1), key[0].transpose(0, 1), value[0].transpose(0, 1),
                                cu_q, cu_kv, prefix_len, pack_len, words, sm_scale=scaling)
    return out.unsqueeze(0), None


def register():
    """Register the HF attention implementations (cast_trees/serving.py:75):
    "cast_varlen" (the batched verify over the KV store) and "cast_tree" (the
    batch-one verify over a DynamicCache with the additive tree mask).
    Returns False when transformers is absent."""
    try:
        from transformers import AttentionInterface
    except ImportError:
        return False
    AttentionInterface.register("cast_varlen", _varlen_attention)
    AttentionInterface.register("cast_tree", _tree_attention)
    return True


register()
