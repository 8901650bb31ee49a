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


@pytest.mark.parametrize("seed,accept_p", [(0, 0.8), (1, 0.8), (8, 1.0), (34, 1.0)])
def test_accept_cpu_plumbing_config(gpu, seed, accept_p):
    # the CPU-plumbing configuration's own leg: its N=15 tree (15 x 64 block
    # of N(0,5) scores, seed 0, cast_trees examples/quickstart.py:12) and
    # planted [16, 64] fp32 verify logits (walk of cast_trees/decode.py:96-103)
    wl = SC.cpu_plumbing()
    logits, planted = SC.planted_logits(wl, vocab=64, seed=seed, accept_p=accept_p)
    assert logits.shape == (16, 64) and logits.dtype == torch.float32
    ref = _accept_case(wl, logits, gpu, f"cpu-plumbing-seed{seed}")
    assert [p for p, _ in ref] == planted
    _accept_case(wl, logits.to(torch.bfloat16), gpu, f"cpu-plumbing-seed{seed}-bf16")


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


def _argmax_rows(gpu, logits_dev):
    """greedy_accept's per-row argmax over a one-request chain batch."""
    from cast_amd import greedy_accept
    R = logits_dev.shape[0]
    cu_q = torch.tensor([0, R], dtype=torch.int32, device=gpu)
    parent = torch.arange(-1, R - 1, dtype=torch.int32, device=gpu)
    token = torch.zeros(R, dtype=torch.int64, device=gpu)
    _, _, _, am = greedy_accept(logits_dev, cu_q, parent, token, check=True)
    return am.cpu().numpy()


def _bf16_bits(bits):
    return torch.tensor([bits - 65536 if bits >= 32768 else bits], dtype=torch.int16).view(torch.bfloat16)[0]


@pytest.mark.parametrize("V", [151936, 1001, 64])
def test_bf16_argmax_edge_rows(gpu, V):
    # the bf16 row scan compares 16-bit order keys: signed zeros, infinities,
    # denormals, NaNs of either sign, ties inside a 16-byte chunk and across
    # threads, the last element, rows whose start is not 16-byte aligned
    g = torch.Generator().manual_seed(V)
    rows = []
    def row(fill):
        return torch.full((V,), fill, dtype=torch.bfloat16)
    r = row(-0.0); r[V // 2] = 0.0; rows.append(r)                         # +0 ties -0: index 0
    rows.append(-(torch.rand(V, generator=g) + 0.5).bfloat16())            # negative only
    r = torch.randn(V, generator=g).bfloat16(); r[V // 3] = float("inf"); r[V // 5] = float("inf"); rows.append(r)
    r = row(float("-inf")); r[V - 7] = -1e30; rows.append(r)
    rows.append(row(float("-inf")))                                        # all -inf: index 0
    r = torch.zeros(V, dtype=torch.int16)
    r[:] = torch.randint(1, 120, (V,), generator=g, dtype=torch.int16)     # positive denormals
    r[V - 3] = 127
    rows.append(r.view(torch.bfloat16))
    r = torch.randn(V, generator=g).bfloat16(); r[V // 2] = float("nan"); r[3] = 1e30; rows.append(r)
    r = torch.randn(V, generator=g).bfloat16(); r[V // 4] = _bf16_bits(0xFFC0); rows.append(r)   # negative NaN
    r = torch.randn(V, generator=g).bfloat16(); r[2 * V // 3] = _bf16_bits(0xFF81); r[V // 3] = float("nan")
    rows.append(r)
    r = torch.randn(V, generator=g).bfloat16(); r[min(17, V - 1)] = 7.0; r[min(16, V - 1)] = 7.0
    r[V - 1] = 7.0; rows.append(r)                                         # ties: first index
    r = torch.randn(V, generator=g).bfloat16(); r[V - 1] = 9.0; rows.append(r)   # the last element
    r = torch.randint(-2, 3, (V,), generator=g).bfloat16(); rows.append(r)       # many ties everywhere
    r = torch.randn(V, generator=g).bfloat16(); r[::2] = -r[::2]; rows.append(r)
    logits = torch.stack(rows)
    print(f"case bf16-argmax-edges V={V}: {logits.shape[0]} rows", flush=True)
    want = OW.row_argmax_all(logits)
    assert np.array_equal(_argmax_rows(gpu, logits.to(gpu)), want)
    # rows at a 2-byte (not 16-byte) aligned stride
    wide = torch.cat([logits, logits[:, :3]], dim=1)
    dev = wide.to(gpu)[:, :V]
    assert dev.stride(0) == V + 3
    assert np.array_equal(_argmax_rows(gpu, dev), want)


def _f16_bits(bits):
    return torch.tensor([bits - 65536 if bits >= 32768 else bits], dtype=torch.int16).view(torch.float16)[0]


@pytest.mark.parametrize("V", [151936, 1001])
def test_fp16_argmax_edge_rows(gpu, V):
    # fp16 logits take the same 16-bit order keys with fp16's infinity
    # (0x7c00) as the NaN bound: signed zeros, infinities, denormals, NaNs of
    # either sign (quiet and signalling patterns), ties, the last element
    g = torch.Generator().manual_seed(V + 1)
    rows = []
    def row(fill):
        return torch.full((V,), fill, dtype=torch.float16)
    r = row(-0.0); r[V // 2] = 0.0; rows.append(r)
    rows.append(-(torch.rand(V, generator=g) + 0.5).half())
    r = torch.randn(V, generator=g).half(); r[V // 3] = float("inf"); r[V // 5] = float("inf"); rows.append(r)
    r = row(float("-inf")); r[V - 7] = -6e4; rows.append(r)
    rows.append(row(float("-inf")))
    r = torch.randint(1, 1023, (V,), generator=g, dtype=torch.int16); r[V - 3] = 1023
    rows.append(r.view(torch.float16))                                     # positive denormals
    r = torch.randn(V, generator=g).half(); r[V // 2] = float("nan"); r[3] = 6e4; rows.append(r)
    r = torch.randn(V, generator=g).half(); r[V // 4] = _f16_bits(0xFE00); rows.append(r)     # negative NaN
    r = torch.randn(V, generator=g).half(); r[2 * V // 3] = _f16_bits(0x7C01); rows.append(r)  # signalling NaN
    r = torch.randn(V, generator=g).half(); r[17] = 7.0; r[16] = 7.0; r[V - 1] = 7.0; rows.append(r)
    r = torch.randn(V, generator=g).half(); r[V - 1] = 9.0; rows.append(r)
    r = torch.randint(-2, 3, (V,), generator=g).half(); rows.append(r)
    logits = torch.stack(rows)
    print(f"case fp16-argmax-edges V={V}: {logits.shape[0]} rows", flush=True)
    want = OW.row_argmax_all(logits)
    assert np.array_equal(_argmax_rows(gpu, logits.to(gpu)), want)
    wide = torch.cat([logits, logits[:, :3]], dim=1)
    dev = wide.to(gpu)[:, :V]
    assert np.array_equal(_argmax_rows(gpu, dev), want)
