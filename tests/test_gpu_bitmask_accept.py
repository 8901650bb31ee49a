"""K1 ancestor bitmask and K3 greedy accept on the GPU: bit-exact vs the oracle."""
import numpy as np
import pytest
import torch

from cast_amd import scenarios as SC
from cast_amd import tree as T
from oracle import bitmask as OB
from oracle import walk as OW

pytestmark = pytest.mark.gpu


def _trees_mixed():
    chain = [T.TreeNode(i, i + 1, i - 1, 0.0) for i in range(127)]
    star = [T.TreeNode(i, 1, -1, 0.0) for i in range(127)]
    trees = [chain, star, [], chain[:63], star[:64]]
    trees += SC.random_parent_batch(seed=4, B=6, p_lo=1, p_hi=129).trees
    trees += SC.qwen3_ragged(seed=1, B=4, vocab=2048).trees
    trees += SC.cpu_plumbing().trees
    return trees


def test_bitmask_bit_exact_two_words(gpu):
    from cast_amd import tree_bitmask
    pk = T.pack_trees(_trees_mixed())
    print(f"case bitmask-2w: B={pk.batch} total_q={pk.total_q}", flush=True)
    got = tree_bitmask(torch.from_numpy(pk.parent).to(gpu), torch.from_numpy(pk.cu_q).to(gpu), 2, check=True)
    want = OB.chain_walk_words(pk.parent, pk.cu_q).view(np.int64)
    assert np.array_equal(got.cpu().numpy(), want)


def test_bitmask_one_word_is_the_reference_int64(gpu):
    from cast_amd import tree_bitmask
    trees = [t for t in _trees_mixed() if len(t) < 64]
    pk = T.pack_trees(trees)
    print(f"case bitmask-1w: B={pk.batch} total_q={pk.total_q}", flush=True)
    got = tree_bitmask(torch.from_numpy(pk.parent).to(gpu), torch.from_numpy(pk.cu_q).to(gpu), 1, check=True)
    assert np.array_equal(got.cpu().numpy(), OB.reference_int64_words(trees))


def test_bitmask_flags_bad_input(gpu):
    from cast_amd import tree_bitmask
    print("case bitmask-bad-input", flush=True)
    parent = torch.tensor([-1, 0, 5, 1], dtype=torch.int32, device=gpu)      # node 2 points forward
    with pytest.raises(ValueError):
        tree_bitmask(parent, torch.tensor([0, 4], dtype=torch.int32, device=gpu), 2, check=True)
    chain = np.array([-1] + list(range(99)), dtype=np.int32)                  # 100 tokens, one word
    with pytest.raises(ValueError):
        tree_bitmask(torch.from_numpy(chain).to(gpu), torch.tensor([0, 100], dtype=torch.int32, device=gpu), 1,
                     check=True)


def _accept_case(wl, logits, gpu, label, device_logits=None):
    from cast_amd import greedy_accept
    print(f"case accept {label}: B={wl.B} total_q={wl.total_q} V={logits.shape[1]} {logits.dtype}", flush=True)
    pk = wl.packed
    dl = logits.to(gpu) if device_logits is None else device_logits
    path, plen, bonus, am = greedy_accept(dl, torch.from_numpy(pk.cu_q).to(gpu),
                                          torch.from_numpy(pk.parent).to(gpu), torch.from_numpy(pk.token).to(gpu),
                                          check=True)
    am_ref = OW.row_argmax_all(logits)
    assert np.array_equal(am.cpu().numpy(), am_ref)
    ref = OW.greedy_walk_batch(wl.trees, logits, pk.cu_q)
    plen, bonus, path = plen.cpu().tolist(), bonus.cpu().tolist(), path.cpu().numpy()
    for b, (p, bo) in enumerate(ref):
        assert plen[b] == len(p) and path[b, :len(p)].tolist() == p and bonus[b] == bo
        assert (path[b, len(p):] == -1).all()
    return ref


def test_accept_planted_paths_small_vocab(gpu):
    wl = SC.qwen3_ragged(seed=2, B=8, lo=1, hi=2, vocab=3000)
    logits, planted = SC.planted_logits(wl, seed=1)
    ref = _accept_case(wl, logits, gpu, "planted-bf16")
    assert [p for p, _ in ref] == planted
    _accept_case(wl, logits.float(), gpu, "planted-fp32")


def test_accept_full_vocab_with_ties_and_nan(gpu):
    wl = SC.qwen3_ragged(seed=5, B=3, lo=1, hi=2, packs=(16, 32))
    logits, _ = SC.planted_logits(wl, seed=5, accept_p=0.9)
    # a NaN and exact ties on some off-path rows
    logits[3, 1000] = float("nan")
    logits[3, 77] = float("nan")
    logits[4, 5] = 50.0
    logits[4, 151935] = 50.0
    logits[5, :] = 0.0
    _accept_case(wl, logits, gpu, "vocab151936")


def test_accept_odd_vocab_and_strided_rows(gpu):
    wl = SC.random_parent_batch(seed=7, B=5, p_lo=1, p_hi=40)
    V = 1001
    g = torch.Generator().manual_seed(0)
    big = torch.randint(-3, 3, (wl.total_q, V + 7), generator=g).float()    # many ties
    dev = big.to(gpu)[:, :V]                                                  # row stride V + 7
    assert dev.stride(0) == V + 7
    _accept_case(wl, big[:, :V].contiguous(), gpu, "odd-vocab-strided", device_logits=dev)


def test_walk_tree_drop_in(gpu):
    from cast_amd import walk_tree, walk_trees
    wl = SC.qwen3_ragged(seed=8, B=4, lo=1, hi=2, packs=(16, 32, 64), vocab=5000)
    logits, planted = SC.planted_logits(wl, seed=3)
    P = int(wl.pack_len.max())
    padded = torch.zeros(wl.B, P, logits.shape[1], dtype=logits.dtype)
    for b in range(wl.B):
        padded[b, :wl.pack_len[b]] = logits[wl.cu_q[b]:wl.cu_q[b + 1]]
    print("case walk-tree-drop-in", flush=True)
    got = walk_trees(wl.trees, padded.to(gpu))
    want = OW.greedy_walk_batch(wl.trees, logits, wl.cu_q)
    assert got == [(p, b) for p, b in want]
    for b in range(wl.B):
        assert walk_tree(wl.trees[b], padded[b].to(gpu)) == want[b]
    with pytest.raises(NotImplementedError):
        walk_tree(wl.trees[0], padded[0].to(gpu), temperature=1.0)
