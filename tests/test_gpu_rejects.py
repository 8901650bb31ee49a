"""Defined results for requests the kernels reject, with check=False.

A request whose device-side metadata is inconsistent (pack longer than the
mask words, offsets that disagree with prefix/pack lengths) is skipped by the
kernels; a batch whose accepted packs would overlap or exceed total_q /
total_kv is rejected whole.  Every row no accepted request owns comes back as
zeros with lse = -inf (never uninitialised memory); accepted requests match
the oracle as usual.  The reference fails loudly at the same points
(cast_trees/serving.py:212 asserts P <= 64; tree_attn.py:124 the head ratio).
"""
import math

import numpy as np
import pytest
import torch

from cast_amd import scenarios as SC
from oracle import attn as OA
from oracle import bitmask as OB

pytestmark = pytest.mark.gpu


def _setup(gpu, packs, prefix, seed=0, D=128):
    from cast_amd.tree import TreeNode
    rng = np.random.default_rng(seed)
    trees = []
    for P in packs:
        par = [-1] + [int(rng.integers(0, i)) for i in range(1, P)]
        depth = [0] * P
        nodes = []
        for i in range(1, P):
            depth[i] = depth[par[i]] + 1
            nodes.append(TreeNode(int(rng.integers(0, 1000)), depth[i], par[i] - 1, 0.0))
        trees.append(nodes)
    wl = SC._make("rejects", trees, prefix, dict(Hq=16, Hkv=4, D=D, vocab=1000), "bf16", seed, 1 / math.sqrt(D))
    q, k, v = wl.qkv(device=gpu)
    words = OB.chain_walk_words(wl.packed.parent, wl.cu_q)
    return wl, q, k, v, words


def _poison(t):
    return t.fill_(float("nan"))


def _check(wl, q, k, v, words, out, lse, accepted):
    torch.cuda.synchronize()
    ref_o, ref_l = OA.dense_tree_attention(q.float().cpu(), k.float().cpu(), v.float().cpu(), wl.cu_q, wl.cu_kv,
                                           wl.prefix_len, wl.pack_len, words, requests=accepted)
    o, l = out.float().cpu(), lse.cpu()
    cq = wl.cu_q
    for b in range(wl.B):
        rows = slice(int(cq[b]), int(cq[b + 1]))
        if b in accepted:
            assert (o[rows] - ref_o[rows]).abs().max() <= 2e-2, f"request {b}"
            assert (l[rows] - ref_l[rows]).abs().max() <= 1e-3, f"request {b}"
        else:
            assert torch.all(o[rows] == 0), f"rejected request {b} not zero"
            assert torch.all(torch.isneginf(l[rows])), f"rejected request {b} lse not -inf"


@pytest.mark.parametrize("kv_split", [0, -1, 128, -2])
def test_pack_longer_than_one_mask_word(gpu, kv_split):
    from cast_amd import varlen_tree_attention
    wl, q, k, v, words = _setup(gpu, [10, 100, 20], [300, 50, 700])
    print(f"case reject-long-pack split={kv_split}: packs {list(wl.pack_len)}", flush=True)
    meta = wl.meta_tensors(gpu)
    one_word = torch.from_numpy(words[:, 0].view(np.int64).copy()).to(gpu)
    out, lse = _poison(torch.empty_like(q)), _poison(torch.empty(q.shape[:2], device=gpu))
    out, lse = varlen_tree_attention(q, k, v, meta["cu_q"], meta["cu_kv"], meta["prefix_len"], meta["pack_len"],
                                     one_word, return_lse=True, kv_split=kv_split, out=out)
    _check(wl, q, k, v, words, out, lse, accepted=[0, 2])


@pytest.mark.parametrize("kv_split", [0, 160])
def test_rejects_past_the_first_64_requests(gpu, kv_split):
    # a 70-request batch (batch-order schedule) whose request 66 is too long
    # for one mask word: only that request's rows are zeros / -inf
    from cast_amd import varlen_tree_attention
    rng = np.random.default_rng(70)
    packs = [int(x) for x in rng.integers(1, 60, size=70)]
    packs[66] = 90
    prefix = [int(x) for x in rng.integers(10, 400, size=70)]
    wl, q, k, v, words = _setup(gpu, packs, prefix, seed=5)
    print(f"case reject-past-64 split={kv_split}: B={wl.B} total_q={wl.total_q}", flush=True)
    meta = wl.meta_tensors(gpu)
    one_word = torch.from_numpy(words[:, 0].view(np.int64).copy()).to(gpu)
    out, lse = _poison(torch.empty_like(q)), _poison(torch.empty(q.shape[:2], device=gpu))
    out, lse = varlen_tree_attention(q, k, v, meta["cu_q"], meta["cu_kv"], meta["prefix_len"], meta["pack_len"],
                                     one_word, return_lse=True, kv_split=kv_split, out=out)
    _check(wl, q, k, v, words, out, lse, accepted=[b for b in range(70) if b != 66])


def test_offsets_that_disagree(gpu):
    from cast_amd import varlen_tree_attention
    wl, q, k, v, words = _setup(gpu, [10, 40, 20], [300, 50, 700], seed=1)
    print("case reject-offsets", flush=True)
    meta = wl.meta_tensors(gpu)
    bad_prefix = meta["prefix_len"].clone()
    bad_prefix[1] += 3                     # cu_kv no longer grows by S + P for request 1
    out = _poison(torch.empty_like(q))
    out, lse = varlen_tree_attention(q, k, v, meta["cu_q"], meta["cu_kv"], bad_prefix, meta["pack_len"],
                                     torch.from_numpy(words.view(np.int64).copy()).to(gpu), return_lse=True,
                                     out=out)
    _check(wl, q, k, v, words, out, lse, accepted=[0, 2])
    with pytest.raises(ValueError, match="inconsistent"):
        varlen_tree_attention(q, k, v, meta["cu_q"], meta["cu_kv"], bad_prefix, meta["pack_len"],
                              torch.from_numpy(words.view(np.int64).copy()).to(gpu), check=True)


def test_overlapping_packs_reject_the_batch(gpu):
    from cast_amd import varlen_tree_attention
    wl, q, k, v, words = _setup(gpu, [10, 10, 20], [30, 50, 70], seed=2)
    print("case reject-decreasing-cu_q", flush=True)
    meta = wl.meta_tensors(gpu)
    cu_q = meta["cu_q"].clone()
    cu_q[2] = 5                            # request 1 would start inside request 0
    out = _poison(torch.empty_like(q))
    out, lse = varlen_tree_attention(q, k, v, cu_q, meta["cu_kv"], meta["prefix_len"], meta["pack_len"],
                                     torch.from_numpy(words.view(np.int64).copy()).to(gpu), return_lse=True,
                                     out=out)
    _check(wl, q, k, v, words, out, lse, accepted=[])


@pytest.mark.parametrize("kv_split", [0, -1, -2])
def test_store_batch_above_total_kv(gpu, kv_split):
    from cast_amd.tree_attn import store_tree_attention
    wl, q, k, v, words = _setup(gpu, [10, 40, 20], [300, 50, 700], seed=3)
    print(f"case reject-store-total-kv split={kv_split}", flush=True)
    meta = wl.meta_tensors(gpu)
    B, Hkv, D, cap = wl.B, wl.Hkv, wl.D, 800
    k_store = torch.zeros((B, Hkv, cap, D), dtype=q.dtype, device=gpu)
    v_store = torch.zeros_like(k_store)
    k_pack = torch.zeros((Hkv, wl.total_q, D), dtype=q.dtype, device=gpu)
    v_pack = torch.zeros_like(k_pack)
    mask = torch.from_numpy(words.view(np.int64).copy()).to(gpu)
    out = _poison(torch.empty_like(q))
    out, lse = store_tree_attention(q, k_store, v_store, k_pack, v_pack, meta["cu_q"], meta["prefix_len"],
                                    meta["pack_len"], mask, total_kv=wl.total_kv - 1, return_lse=True,
                                    kv_split=kv_split, out=out)
    torch.cuda.synchronize()
    assert torch.all(out == 0) and torch.all(torch.isneginf(lse))


def test_fp32_mfma_kernel_rejects_too(gpu):
    # fp32 at head dim 128: tree_attn_f32_kernel
    from cast_amd import varlen_tree_attention
    wl, q, k, v, words = _setup(gpu, [10, 100, 20], [300, 50, 700], seed=4)
    q, k, v = q.float(), k.float(), v.float()
    print("case reject-long-pack-fp32-mfma", flush=True)
    meta = wl.meta_tensors(gpu)
    one_word = torch.from_numpy(words[:, 0].view(np.int64).copy()).to(gpu)
    out = _poison(torch.empty_like(q))
    out, lse = varlen_tree_attention(q, k, v, meta["cu_q"], meta["cu_kv"], meta["prefix_len"], meta["pack_len"],
                                     one_word, return_lse=True, out=out)
    _check(wl, q, k, v, words, out, lse, accepted=[0, 2])


@pytest.mark.parametrize("dtype,D", [("bf16", 96), ("fp32", 96), ("bf16", 192)])
def test_scalar_kernel_rejects_too(gpu, dtype, D):
    # head dims off the MFMA kernels take tree_attn_generic_kernel: its
    # batch prologue zero-fills the rejected request's rows the same way
    from cast_amd import varlen_tree_attention
    wl, q, k, v, words = _setup(gpu, [10, 100, 20], [300, 50, 700], seed=6, D=D)
    if dtype == "fp32":
        q, k, v = q.float(), k.float(), v.float()
    print(f"case reject-long-pack-scalar-{dtype}-D{D}", flush=True)
    meta = wl.meta_tensors(gpu)
    one_word = torch.from_numpy(words[:, 0].view(np.int64).copy()).to(gpu)
    out, lse = _poison(torch.empty_like(q)), _poison(torch.empty(q.shape[:2], device=gpu))
    out, lse = varlen_tree_attention(q, k, v, meta["cu_q"], meta["cu_kv"], meta["prefix_len"], meta["pack_len"],
                                     one_word, return_lse=True, out=out)
    _check(wl, q, k, v, words, out, lse, accepted=[0, 2])
