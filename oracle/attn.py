"""Dense masked-softmax oracle for ragged tree attention (CPU, torch).
Test infrastructure only.

Restates the dense check of cast_trees' kernel test
(tests/test_tree_attn.py:40-59): per request, q [P,Hq,D] against
concat(prefix, pack) keys with GQA by ``repeat_interleave`` (query head h
reads KV head h // (Hq/Hkv), cast_trees/tree_attn.py:30), scale 1/sqrt(D)
by default (tree_attn.py:125-126), every prefix key visible and pack key j
visible iff bit j of the row's ancestor words is set and j < P
(tree_attn.py:73-75).  A row with no visible key returns zeros
(tree_attn.py:62,89).  Adds the natural-log log-sum-exp of the scaled scores
over visible keys, ``lse = ln sum exp(sm_scale * q.k)``, -inf for an empty
row.
"""
import math

import numpy as np
import torch


def _mask_words(mask, total_q):
    m = mask.detach().cpu().numpy() if torch.is_tensor(mask) else np.asarray(mask)
    if m.ndim == 1:
        m = np.stack([m.view(np.uint64) if m.dtype == np.int64 else m.astype(np.uint64),
                      np.zeros_like(m, dtype=np.uint64)], axis=1)
    m = m.view(np.uint64) if m.dtype == np.int64 else m.astype(np.uint64)
    assert m.shape[0] == total_q
    return m


def visible(words_row, S, P):
    """Bool [S+P]: the keys one packed row may attend to."""
    j = np.arange(P)
    bits = (words_row[j >> 6] >> (j & 63).astype(np.uint64)) & np.uint64(1)
    return np.concatenate([np.ones(S, dtype=bool), bits.astype(bool)])


def dense_tree_attention(q, k, v, cu_q, cu_kv, prefix_len, pack_len, mask, sm_scale=None,
                         compute_dtype=torch.float32, requests=None, kv_heads=None):
    """Returns (out [total_q,Hq,D], lse [total_q,Hq]) in ``compute_dtype``.

    ``requests`` / ``kv_heads`` restrict the work to a subset (other rows stay
    NaN), so very large workloads can be checked on a sample.
    """
    total_q, Hq, D = q.shape
    Hkv = k.shape[1]
    assert Hq % Hkv == 0, "query heads must be a multiple of KV heads"
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    words = _mask_words(mask, total_q)
    cq = [int(x) for x in torch.as_tensor(cu_q).tolist()]
    ckv = [int(x) for x in torch.as_tensor(cu_kv).tolist()]
    S_all = [int(x) for x in torch.as_tensor(prefix_len).tolist()]
    P_all = [int(x) for x in torch.as_tensor(pack_len).tolist()]
    out = torch.full((total_q, Hq, D), float("nan"), dtype=compute_dtype)
    lse = torch.full((total_q, Hq), float("nan"), dtype=compute_dtype)
    reqs = range(len(P_all)) if requests is None else requests
    heads = range(Hkv) if kv_heads is None else kv_heads
    qh = torch.tensor([h * G + g for h in heads for g in range(G)], dtype=torch.long)
    kh = torch.tensor(list(heads), dtype=torch.long)
    for b in reqs:
        S, P = S_all[b], P_all[b]
        if P == 0:
            continue
        allowed = torch.from_numpy(np.stack([visible(words[cq[b] + i], S, P) for i in range(P)]))
        qb = q[cq[b]:cq[b] + P].index_select(1, qh).to(compute_dtype).transpose(0, 1)
        kb = k[ckv[b]:ckv[b] + S + P].index_select(1, kh).to(compute_dtype).transpose(0, 1)
        vb = v[ckv[b]:ckv[b] + S + P].index_select(1, kh).to(compute_dtype).transpose(0, 1)
        kb = kb.repeat_interleave(G, 0).contiguous()
        vb = vb.repeat_interleave(G, 0).contiguous()
        s = torch.matmul(qb, kb.transpose(1, 2).contiguous()) * scale
        s = s.masked_fill(~allowed, float("-inf"))
        l = torch.logsumexp(s, dim=-1)                       # [H, P], -inf if empty
        safe = torch.where(torch.isinf(l), torch.zeros_like(l), l)
        p = torch.exp(s - safe[..., None])
        o = torch.matmul(p, vb)
        out[cq[b]:cq[b] + P, qh] = o.transpose(0, 1)
        lse[cq[b]:cq[b] + P, qh] = l.transpose(0, 1)
    return out, lse
