"""Pins the CPU oracle against checks that do not restate its own formulas.

Bitmask: the reference's int64 recurrence (a different algorithm), the
ancestor-matrix invariant, chain/star closed forms.  Attention: reductions
to torch SDPA (decode and causal), poisoned masked keys, logsumexp.  Walk:
replay-style accepted length, brute force over root paths, planted paths.
Each family also plants a mistake in the oracle and checks that the same
comparison catches it.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from cast_amd import scenarios as SC
from cast_amd import tree as T
from oracle import attn as OA
from oracle import bitmask as OB
from oracle import walk as OW


# ---------------------------------------------------------------- bitmask
def _quick_trees():
    idx, lp = T.block_topk(np.random.default_rng(0).normal(size=(15, 100)) * 3, 8)
    return [T.build_tree(idx, lp, n) for n in (0, 1, 15, 31, 63)]


def test_bitmask_word0_equals_reference_int64_recurrence():
    trees = _quick_trees()
    pk = T.pack_trees(trees)
    words = OB.chain_walk_words(pk.parent, pk.cu_q)
    ref = OB.reference_int64_words(trees)
    assert np.array_equal(words[:, 0].view(np.int64), ref)
    assert not words[:, 1].any()


def test_bitmask_is_the_ancestor_matrix_up_to_128():
    idx, lp = T.block_topk(np.random.default_rng(5).normal(size=(15, 100)) * 3, 8)
    trees = [T.build_tree(idx, lp, n) for n in (64, 100, 127)]
    pk = T.pack_trees(trees)
    words = OB.chain_walk_words(pk.parent, pk.cu_q)
    for b, nodes in enumerate(trees):
        vis = T.ancestor_matrix(nodes)
        P = len(nodes) + 1
        for i in range(P):
            assert np.array_equal(OB.words_to_bool(words[pk.cu_q[b] + i], P), vis[i])


def test_bitmask_closed_forms():
    P = 128
    chain = np.array([-1] + list(range(P - 1)), dtype=np.int32)       # row i: bits 0..i
    star = np.array([-1] + [0] * (P - 1), dtype=np.int32)             # row i: bits {0, i}
    cu = np.array([0, P], dtype=np.int32)
    wc = OB.chain_walk_words(chain, cu)
    ws = OB.chain_walk_words(star, cu)
    for i in range(P):
        want = np.zeros(2, dtype=np.uint64)
        for j in range(i + 1):
            want[j >> 6] |= np.uint64(1) << np.uint64(j & 63)
        assert np.array_equal(wc[i], want)
        want = np.zeros(2, dtype=np.uint64)
        for j in {0, i}:
            want[j >> 6] |= np.uint64(1) << np.uint64(j & 63)
        assert np.array_equal(ws[i], want)
    assert wc[127, 1] == np.uint64(0xFFFFFFFFFFFFFFFF) and wc[63, 1] == 0


def test_bitmask_rejects_a_cycle():
    with pytest.raises(ValueError):
        OB.chain_walk_words(np.array([-1, 2, 1], dtype=np.int32), np.array([0, 3]))


# ---------------------------------------------------------------- attention
def _single(S, parent, Hq=4, Hkv=2, D=32, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    P = len(parent)
    q = torch.randn(P, Hq, D, generator=g, dtype=dtype)
    k = torch.randn(S + P, Hkv, D, generator=g, dtype=dtype)
    v = torch.randn(S + P, Hkv, D, generator=g, dtype=dtype)
    words = OB.chain_walk_words(np.asarray(parent, dtype=np.int32), np.array([0, P]))
    meta = dict(cu_q=[0, P], cu_kv=[0, S + P], prefix_len=[S], pack_len=[P], mask=words)
    return q, k, v, meta


def _sdpa(q, k, v, allowed, scale=None):
    Hq, Hkv = q.shape[1], k.shape[1]
    qq, kk, vv = (x.transpose(0, 1)[None] for x in (q, k, v))
    o = F.scaled_dot_product_attention(qq, kk, vv, attn_mask=allowed, scale=scale, enable_gqa=Hq != Hkv)
    return o[0].transpose(0, 1)


def _run(q, k, v, meta, **kw):
    return OA.dense_tree_attention(q, k, v, meta["cu_q"], meta["cu_kv"], meta["prefix_len"],
                                   meta["pack_len"], meta["mask"], compute_dtype=torch.float64, **kw)


def test_attention_root_only_is_decode_sdpa():
    q, k, v, meta = _single(77, [-1])
    out, lse = _run(q, k, v, meta)
    assert torch.allclose(out, _sdpa(q, k, v, None), atol=1e-12)
    G = q.shape[1] // k.shape[1]
    s = torch.einsum("hd,shd->hs", q[0], k.repeat_interleave(G, 1)) / math.sqrt(q.shape[-1])
    assert torch.allclose(lse[0], torch.logsumexp(s, -1), atol=1e-12)


def test_attention_chain_is_causal_sdpa_with_offset():
    for S in (0, 5, 64):
        P = 20
        q, k, v, meta = _single(S, [-1] + list(range(P - 1)), seed=S)
        out, _ = _run(q, k, v, meta)
        causal = torch.ones(P, S + P, dtype=torch.bool).tril(diagonal=S)
        assert torch.allclose(out, _sdpa(q, k, v, causal), atol=1e-12)


def test_attention_random_tree_against_sdpa_with_ancestor_matrix():
    idx, lp = T.block_topk(np.random.default_rng(2).normal(size=(15, 100)) * 3, 8)
    nodes = T.build_tree(idx, lp, 90)
    parent = T.pack_parents(nodes)
    S = 33
    q, k, v, meta = _single(S, parent, Hq=8, Hkv=2, D=16, seed=3)
    vis = torch.from_numpy(T.ancestor_matrix(nodes))
    allowed = torch.cat([torch.ones(len(parent), S, dtype=torch.bool), vis], 1)
    out, lse = _run(q, k, v, meta, sm_scale=0.3)
    assert torch.allclose(out, _sdpa(q, k, v, allowed, scale=0.3), atol=1e-12)
    # lse: the normaliser of exactly those keys, from raw scores
    G = 4
    s = torch.einsum("phd,shd->phs", q, k.repeat_interleave(G, 1)) * 0.3
    s = s.masked_fill(~allowed[:, None, :], float("-inf"))
    assert torch.allclose(lse, torch.logsumexp(s, -1), atol=1e-12)


def test_attention_masked_keys_do_not_leak():
    idx, lp = T.block_topk(np.random.default_rng(4).normal(size=(15, 100)) * 3, 8)
    nodes = T.build_tree(idx, lp, 40)
    parent = T.pack_parents(nodes)
    S = 10
    q, k, v, meta = _single(S, parent)
    out, _ = _run(q, k, v, meta)
    vis = T.ancestor_matrix(nodes)
    # poison every pack key/value that row 5 may not see; row 5 must not move
    hidden = [S + j for j in range(len(parent)) if not vis[5, j]]
    k2, v2 = k.clone(), v.clone()
    k2[hidden] = 50.0
    v2[hidden] = 1e6
    out2, _ = _run(q, k2, v2, meta)
    assert torch.allclose(out[5], out2[5], atol=1e-12)


def test_attention_empty_row_is_zero_with_minus_inf_lse():
    q, k, v, meta = _single(0, [-1, 0, 1])
    meta["mask"] = meta["mask"].copy()
    meta["mask"][1] = 0
    out, lse = _run(q, k, v, meta)
    assert torch.all(out[1] == 0) and torch.all(torch.isneginf(lse[1]))


def test_attention_subset_matches_full():
    wl = SC.random_parent_batch(seed=1, B=3, Hq=8, Hkv=2, D=16, s_lo=5, s_hi=40, p_lo=2, p_hi=30)
    q, k, v = wl.qkv()
    words = OB.chain_walk_words(wl.packed.parent, wl.cu_q)
    full, lse = OA.dense_tree_attention(q, k, v, wl.cu_q, wl.cu_kv, wl.prefix_len, wl.pack_len, words)
    part, lse2 = OA.dense_tree_attention(q, k, v, wl.cu_q, wl.cu_kv, wl.prefix_len, wl.pack_len, words,
                                         requests=[1], kv_heads=[1])
    r = slice(int(wl.cu_q[1]), int(wl.cu_q[2]))
    assert torch.equal(part[r, 4:8], full[r, 4:8]) and torch.equal(lse2[r, 4:8], lse[r, 4:8])
    assert torch.isnan(part[r, :4]).all()


def test_planted_gqa_mistake_is_caught(monkeypatch):
    # plant a wrong head map (h % Hkv instead of h // G) in the oracle: SDPA disagrees
    q, k, v, meta = _single(12, [-1, 0, 0, 1], Hq=4, Hkv=2)
    good, _ = _run(q, k, v, meta)
    real = torch.Tensor.repeat_interleave
    monkeypatch.setattr(torch.Tensor, "repeat_interleave", lambda self, G, dim: self.repeat(G, 1, 1))
    bad, _ = _run(q, k, v, meta)
    monkeypatch.setattr(torch.Tensor, "repeat_interleave", real)
    vis = T.ancestor_matrix([T.TreeNode(0, 1, -1, 0), T.TreeNode(0, 1, -1, 0), T.TreeNode(0, 2, 0, 0)])
    allowed = torch.cat([torch.ones(4, 12, dtype=torch.bool), torch.from_numpy(vis)], 1)
    ref = _sdpa(q, k, v, allowed)
    assert torch.allclose(good, ref, atol=1e-12)
    assert not torch.allclose(bad, ref, atol=1e-3)


# ---------------------------------------------------------------- walk
def _accepted_len_by_rank_paths(nodes, top_idx, realized):
    """Replay formulation (cast_trees/replay.py:20-32): trees as sets of rank
    tuples; accepted = longest realized prefix that is a tree path."""
    ranks = []
    for nd in nodes:
        r = int(np.nonzero(top_idx[nd.depth - 1] == nd.token)[0][0])
        ranks.append((ranks[nd.parent] if nd.parent >= 0 else ()) + (r,))
    tree = set(ranks)
    tau, path = 0, ()
    for d in range(min(top_idx.shape[0], len(realized))):
        hit = np.nonzero(top_idx[d] == realized[d])[0]
        if len(hit) == 0 or path + (int(hit[0]),) not in tree:
            break
        tau, path = tau + 1, path + (int(hit[0]),)
    return tau


@pytest.mark.parametrize("seed", range(6))
def test_walk_matches_replay_accepted_length(seed):
    rng = np.random.default_rng(seed)
    V = 64
    idx, lp = T.block_topk(rng.normal(scale=3, size=(15, V)), 8)
    nodes = T.build_tree(idx, lp, 63)
    # realized continuation: mostly top-ranked tokens so that acceptance is long
    realized = [int(idx[d, rng.integers(0, 3)]) if d < 15 and rng.random() < 0.9
                else int(rng.integers(0, V)) for d in range(16)]
    depth = [0] + [n.depth for n in nodes]
    logits = torch.randn(len(nodes) + 1, V, generator=torch.Generator().manual_seed(seed))
    for r, d in enumerate(depth):
        logits[r, realized[d]] = 10.0
    path, bonus = OW.greedy_walk(nodes, logits)
    tau = _accepted_len_by_rank_paths(nodes, idx, realized)
    assert len(path) == tau
    assert bonus == realized[tau]
    assert [nodes[c].token for c in path] == realized[:tau]


def test_walk_brute_force_over_root_paths():
    rng = np.random.default_rng(11)
    for trial in range(30):
        V = 6
        P = int(rng.integers(1, 12))
        nodes = []
        for i in range(P - 1):
            par = int(rng.integers(-1, i)) if i else -1
            nodes.append(T.TreeNode(int(rng.integers(0, V)), 0, par, 0.0))
        logits = torch.from_numpy(rng.integers(0, 3, size=(P, V)).astype(np.float32))
        am = [int(torch.argmax(logits[r])) for r in range(P)]
        # brute force: a node is accepted iff every step root->node matches the
        # argmax and each step is the earliest sibling carrying that token
        def accepted(c):
            chain = []
            while c != -1:
                chain.append(c)
                c = nodes[c].parent
            chain = chain[::-1]
            prev = -1
            for c in chain:
                first = min(i for i, n in enumerate(nodes) if n.parent == prev and n.token == nodes[c].token)
                if nodes[c].token != am[prev + 1] or first != c:
                    return False
                prev = c
            return True
        acc = [c for c in range(len(nodes)) if accepted(c)]
        path, bonus = OW.greedy_walk(nodes, logits)
        assert sorted(path) == sorted(acc)
        last = path[-1] if path else -1
        assert bonus == am[last + 1]


def test_walk_planted_paths_and_ties_and_nan():
    wl = SC.qwen3_ragged(seed=0, B=3, lo=10, hi=20, packs=(16, 32), vocab=4096)
    logits, planted = SC.planted_logits(wl, seed=0)
    res = OW.greedy_walk_batch(wl.trees, logits, wl.cu_q)
    assert [p for p, _ in res] == planted
    row = torch.tensor([0.0, 2.0, 2.0, float("nan"), 2.0, float("nan")])
    assert OW.row_argmax(row) == 3 == int(torch.argmax(row))
    assert OW.row_argmax(torch.tensor([1.0, 3.0, 3.0])) == 1
    am = OW.row_argmax_all(torch.stack([row, torch.tensor([5.0, 5.0, 1.0, 0.0, 0.0, 0.0])]))
    assert am.tolist() == [3, 0]


def test_planted_walk_mistake_is_caught(monkeypatch):
    # plant "last matching sibling" in the oracle: the expected first-match
    # answer (node 0, then stop) no longer comes out
    nodes = [T.TreeNode(3, 1, -1, 0.0), T.TreeNode(3, 1, -1, 0.0), T.TreeNode(4, 2, 1, 0.0)]
    logits = torch.zeros(4, 6)
    logits[0, 3] = 1.0      # root -> token 3 (nodes 0 and 1 both carry it)
    logits[1, 5] = 1.0      # after node 0 -> token 5, no child: stop
    logits[2, 4] = 1.0      # after node 1 -> token 4 = node 2
    assert OW.greedy_walk(nodes, logits) == ([0], 5)
    kids_rev = [T.TreeNode(n.token, n.depth, n.parent, n.score) for n in nodes]
    # the mistake: siblings scanned in reverse, emulated by swapping nodes 0/1
    swapped = [kids_rev[1], kids_rev[0], T.TreeNode(4, 2, 0, 0.0)]
    lg = logits[[0, 2, 1, 3]]
    assert OW.greedy_walk(swapped, lg) != ([0], 5)


# ---------------------------------------------------------------- draft

def _fixture_scores(case):
    name = case["name"]
    if name == "quickstart-seed0":
        return np.random.default_rng(0).normal(scale=5, size=(15, 64))
    if name.startswith("scaled3-seed"):
        return np.random.default_rng(int(name[-1])).normal(size=(15, 100)) * 3
    seed = int(name.split("seed")[1].split("-")[0])
    scale = float(name.split("scale")[1])
    return np.random.default_rng(seed).normal(scale=scale, size=(15, 151936))


def test_draft_oracle_matches_reference_fixtures():
    # top-k ids and log-probs, and every tree, as the reference module wrote them
    import json
    from pathlib import Path
    from oracle import draft as OD
    fix = json.loads((Path(__file__).parent / "golden" / "tree_fixtures.json").read_text())
    for case in fix["cases"]:
        idx, lp = OD.topk_log_softmax(_fixture_scores(case), case["k"])
        assert idx.tolist() == case["top_idx"]
        assert np.array_equal(lp, np.asarray(case["top_lp"]))
        for n, want in case["trees"].items():
            got = OD.build_tree(idx, lp, int(n), case["k"])
            assert [list(g[:3]) for g in got] == [w[:3] for w in want]
            assert [g[3] for g in got] == [w[3] for w in want]


def test_draft_oracle_tree_invariants_and_ties():
    from oracle import draft as OD
    rng = np.random.default_rng(5)
    x = rng.normal(size=(15, 300)).astype(np.float32)
    x[:, 7] = x[:, 11] = x[:, 200] = x.max(axis=1) + 1.0           # a three-way tie at the top
    idx, lp = OD.topk_log_softmax(x, 8)
    assert (idx[:, :3] == [7, 11, 200]).all()                       # equal values: increasing index
    assert (np.diff(lp, axis=1) <= 0).all()
    nodes = OD.build_tree(idx, lp, 127)
    assert len(nodes) == 127
    for i, (_, d, p, s) in enumerate(nodes):
        assert p < i and (p == -1) == (d == 1)                       # parents first, prefix-closed
        if p >= 0:
            assert nodes[p][1] == d - 1 and nodes[p][3] >= s         # a child never outscores its parent
    assert [n[3] for n in nodes] == sorted([n[3] for n in nodes], reverse=True)   # best-first pop order


# ---- oracle/store.py: plain indexing, pinned on hand-built stores

def test_store_append_oracle_known_answers():
    import torch
    from oracle import store as OS
    B, Hkv, cap, D, total_q = 3, 2, 6, 4, 9
    buf_k = [torch.arange(B * Hkv * cap * D, dtype=torch.float32).view(B, Hkv, cap, D)]
    buf_v = [-buf_k[0]]
    pack_k = [1000 + torch.arange(Hkv * total_q * D, dtype=torch.float32).view(Hkv, total_q, D)]
    pack_v = [-pack_k[0]]
    cu_q = [0, 3, 5, 9]
    store_len = [2, 1, 3]
    keep = [[0, 2], [0], [0, 1, 3]]
    accepted = [2, 1, 3]
    # requests 0 and 2 survive, no growth (3 + 3 = 6 = cap)
    k, v, n = OS.append_store(buf_k, buf_v, pack_k, pack_v, store_len, cu_q, keep, accepted, [0, 2])
    assert n == [4, 6] and k[0].shape == (2, Hkv, cap, D)
    assert torch.equal(k[0][0, :, :2], buf_k[0][0, :, :2])          # old slots untouched
    assert torch.equal(k[0][1, :, :3], buf_k[0][2, :, :3])          # request 2 moved to batch row 1
    assert torch.equal(k[0][0, :, 2], pack_k[0][:, 0]) and torch.equal(k[0][0, :, 3], pack_k[0][:, 2])
    assert torch.equal(k[0][1, :, 3], pack_k[0][:, 5]) and torch.equal(k[0][1, :, 5], pack_k[0][:, 8])
    assert torch.equal(v[0], -k[0])
    assert torch.equal(k[0][0, :, 4:], buf_k[0][0, :, 4:])          # slots past the new length untouched
    # one more accepted row for request 2 overflows: stores double to 12 slots, zero-filled
    k, v, n = OS.append_store(buf_k, buf_v, pack_k, pack_v, store_len, cu_q, [[0, 2], [0], [0, 1, 2, 3]],
                              [2, 1, 4], [0, 1, 2])
    assert n == [4, 2, 7] and k[0].shape == (3, Hkv, 12, D)
    assert torch.equal(k[0][1, :, :1], buf_k[0][1, :, :1]) and torch.equal(k[0][1, :, 1], pack_k[0][:, 3])
    assert torch.equal(k[0][1, :, 2:cap], buf_k[0][1, :, 2:cap])
    assert torch.all(k[0][0, :, cap:] == 0) and torch.all(k[0][2, :, 7:] == 0)
    assert torch.equal(k[0][2, :, 6], pack_k[0][:, 8])


def test_gather_cache_oracle_matches_index_select():
    import torch
    from oracle import store as OS
    g = torch.Generator().manual_seed(0)
    layers = [(torch.randn(1, 2, 30, 8, generator=g), torch.randn(1, 2, 30, 8, generator=g)) for _ in range(3)]
    keep = [0, 4, 5, 9, 17]
    sel = torch.tensor(list(range(10)) + [10 + i for i in keep])
    for (k, v), (kk, vv) in zip(layers, OS.gather_cache(layers, 10, keep)):
        assert torch.equal(kk, k.index_select(2, sel)) and torch.equal(vv, v.index_select(2, sel))
