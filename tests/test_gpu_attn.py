"""Tree attention on the GPU (through the C ABI) vs the dense CPU oracle.

Bar: fp32-accumulated bf16 outputs within max-abs 2e-2 of the fp32 oracle on
the same (bf16-rounded) inputs, natural-log LSE within 1e-3; fp32 inputs
within 1e-4 / 1e-4.  The reference's own kernel test uses
max < 5e-2, mean < 5e-3 (tests/test_tree_attn.py:74); these bounds are tighter.
"""
import math

import numpy as np
import pytest
import torch

from cast_amd import scenarios as SC
from oracle import attn as OA
from oracle import bitmask as OB

pytestmark = pytest.mark.gpu

TOL = {"bf16": dict(out=2e-2, lse=1e-3, mean=2e-3), "fp16": dict(out=5e-3, lse=1e-3, mean=5e-4),
       "fp32": dict(out=1e-4, lse=1e-4, mean=1e-5)}


def _words(wl):
    return OB.chain_walk_words(wl.packed.parent, wl.cu_q)


def _run_and_check(wl, dev, requests=None, kv_heads=None, kv_split=0, one_word=False, q_noncontig=False,
                   label="", qkv=None, reference_bar=False, words=None):
    from cast_amd import varlen_tree_attention
    print(f"case {label or wl.name}: B={wl.B} total_q={wl.total_q} total_kv={wl.total_kv} "
          f"Hq={wl.Hq} Hkv={wl.Hkv} D={wl.D} {wl.dtype} split={kv_split}", flush=True)
    q, k, v = wl.qkv(device=dev) if qkv is None else (x.to(dev) for x in qkv)
    words = _words(wl) if words is None else words
    if one_word:
        assert not words[:, 1].any()
        mask_dev = torch.from_numpy(words[:, 0].view(np.int64).copy()).to(dev)
    else:
        mask_dev = torch.from_numpy(words.view(np.int64).copy()).to(dev)
    meta = wl.meta_tensors(dev)
    if q_noncontig:
        # the serving hook hands over query[0].transpose(0, 1): head-major storage
        q = q.transpose(0, 1).contiguous().transpose(0, 1)
    out, lse = varlen_tree_attention(q, k, v, meta["cu_q"], meta["cu_kv"], meta["prefix_len"], meta["pack_len"],
                                     mask_dev, return_lse=True, kv_split=kv_split, check=True)
    torch.cuda.synchronize()
    ref_o, ref_l = OA.dense_tree_attention(q.float().cpu(), k.float().cpu(), v.float().cpu(), wl.cu_q, wl.cu_kv,
                                           wl.prefix_len, wl.pack_len, words, requests=requests,
                                           kv_heads=kv_heads)
    sel = ~torch.isnan(ref_l)
    got_o, got_l = out.float().cpu(), lse.cpu()
    err_o = (got_o - ref_o).abs()[sel]
    err_l = (got_l - ref_l).abs()[sel & torch.isfinite(ref_l)]
    tol = TOL[wl.dtype]
    print(f"  out max {err_o.max():.3e} mean {err_o.mean():.3e}  lse max {err_l.max():.3e}", flush=True)
    if reference_bar:
        # the reference kernel test's own assertion (tests/test_tree_attn.py:73-74)
        assert err_o.max().item() < 5e-2 and err_o.mean().item() < 5e-3
    assert torch.isfinite(got_o[sel]).all()
    assert err_o.max() <= tol["out"] and err_o.mean() <= tol["mean"]
    assert err_l.max() <= tol["lse"]
    assert torch.equal(torch.isneginf(got_l[sel]), torch.isneginf(ref_l[sel]))
    return out, lse


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_reference_scenario(gpu, dtype):
    # the reference kernel test's batch: B=8, S~U[200,400), P~U[2,64), random parents
    wl = SC.random_parent_batch(seed=0, dtype=dtype)
    _run_and_check(wl, gpu, label=f"reference-scenario-{dtype}")
    _run_and_check(wl, gpu, one_word=True, label=f"reference-scenario-{dtype}-int64-mask")


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_reference_kernel_test_tensors(gpu, dtype):
    # the reference kernel test's exact tensors (same generator, same draw
    # order), cast to the dtype as it does (tests/test_tree_attn.py:64-72),
    # with its one-word int64 mask; the oracle runs on the rounded inputs in
    # fp32 as its dense reference does.  Both its bar and the tighter one.
    import dataclasses
    wl, q, k, v = SC.reference_test_batch(seed=0)
    wl = dataclasses.replace(wl, dtype=dtype)
    dt = SC.torch_dtype(dtype)
    _run_and_check(wl, gpu, one_word=True, qkv=(q.to(dt), k.to(dt), v.to(dt)), reference_bar=True,
                   label=f"reference-kernel-test-{dtype}")


def test_cpu_plumbing_config(gpu):
    _run_and_check(SC.cpu_plumbing(), gpu)


def test_qwen3_single(gpu):
    _run_and_check(SC.qwen3_single(), gpu)
    _run_and_check(SC.qwen3_single(), gpu, kv_split=-1, label="qwen3-single-nosplit")
    _run_and_check(SC.qwen3_single(), gpu, q_noncontig=True, label="qwen3-single-headmajor-q")


def test_qwen3_ragged_full_oracle(gpu):
    _run_and_check(SC.qwen3_ragged(seed=0), gpu)


@pytest.mark.parametrize("split", [64, 256, 1000, -1])
def test_split_k_variants_agree(gpu, split):
    wl = SC.qwen3_ragged(seed=3, B=4, lo=100, hi=3000)
    _run_and_check(wl, gpu, kv_split=split, label=f"ragged-split{split}")


def test_edge_packs(gpu):
    # S=0 pure tree, P=1 root only, P=128 chain, P=128 star, S not a multiple of 32
    from cast_amd.tree import TreeNode
    chain = [TreeNode(i, i + 1, i - 1, 0.0) for i in range(127)]
    star = [TreeNode(i, 1, -1, 0.0) for i in range(127)]
    wl = SC._make("edges", [chain, [], star, chain[:5], star[:63]], [0, 77, 1, 4099, 33],
                  SC.QWEN3_8B, "bf16", 5, 1 / math.sqrt(128))
    _run_and_check(wl, gpu)
    _run_and_check(wl, gpu, kv_split=64, label="edges-split64")


def test_gqa_ratios_and_head_dim_64(gpu):
    # includes one KV head for all query heads (MQA): a pack of 128 tokens is
    # then 4096 query rows, 16 row blocks of one (request, KV head)
    for Hq, Hkv, D, dt in [(8, 8, 64, "bf16"), (16, 2, 64, "bf16"), (64, 8, 128, "bf16"), (12, 4, 96, "bf16"),
                           (8, 2, 128, "fp32"), (32, 1, 128, "bf16"), (16, 1, 64, "fp32")]:
        wl = SC.random_parent_batch(seed=Hq + D, B=3, Hq=Hq, Hkv=Hkv, D=D, s_lo=50, s_hi=700, p_lo=1, p_hi=129,
                                    dtype=dt, qkv_scale=0.5)
        _run_and_check(wl, gpu, label=f"gqa{Hq}/{Hkv}-D{D}-{dt}")


def test_fp16_inputs(gpu):
    # the reference kernel runs on fp16 tensors as well (its tl.dot and
    # empty_like follow q's dtype): the MFMA kernels (f16 products, P rounded
    # to fp16), the split-K combine writing fp16, and the scalar kernel
    wl = SC.random_parent_batch(seed=0, dtype="fp16")
    _run_and_check(wl, gpu, label="reference-scenario-fp16")
    _run_and_check(wl, gpu, one_word=True, label="reference-scenario-fp16-int64-mask")
    wl = SC.random_parent_batch(seed=4, B=4, Hq=16, Hkv=4, D=64, s_lo=200, s_hi=3000, p_lo=1, p_hi=129,
                                dtype="fp16", qkv_scale=0.5)
    for split in (0, 128, -1):
        _run_and_check(wl, gpu, kv_split=split, label=f"fp16-d64-split{split}")
    for D in (96, 256):
        wl = SC.random_parent_batch(seed=D, B=3, Hq=8, Hkv=2, D=D, s_lo=20, s_hi=300, p_lo=1, p_hi=129,
                                    dtype="fp16", qkv_scale=0.5)
        _run_and_check(wl, gpu, label=f"fp16-scalar-d{D}")


def test_head_dims_above_128(gpu):
    # the reference kernel takes any power-of-two head_dim (tl.arange(0, D),
    # tree_attn.py:36): 256 runs the MFMA kernels at one wave per SIMD (bf16,
    # fp16 and fp32); the other multiples of 8 take the scalar kernel
    for Hq, Hkv, D, dt in [(8, 2, 256, "bf16"), (4, 4, 256, "fp32"), (8, 4, 192, "bf16"), (4, 1, 136, "fp32")]:
        wl = SC.random_parent_batch(seed=D + Hq, B=3, Hq=Hq, Hkv=Hkv, D=D, s_lo=20, s_hi=300, p_lo=1, p_hi=129,
                                    dtype=dt, qkv_scale=0.5)
        _run_and_check(wl, gpu, label=f"head-dim-{D}-{Hq}/{Hkv}-{dt}")
    # head_dim 256 on MFMA: long prefixes, split-K and the combine, every format
    for dt in ("bf16", "fp16", "fp32"):
        wl = SC.random_parent_batch(seed=7, B=4, Hq=16, Hkv=8, D=256, s_lo=500, s_hi=4000, p_lo=1, p_hi=129,
                                    dtype=dt, qkv_scale=0.5)
        for split in (0, 256, -1):
            _run_and_check(wl, gpu, kv_split=split, label=f"head-dim-256-mfma-{dt}-split{split}")


@pytest.mark.parametrize("B,dtype,kv_split", [(64, "bf16", 0), (65, "bf16", 0), (65, "bf16", 192),
                                               (130, "bf16", 0), (130, "fp32", 256)])
def test_batches_across_the_64_request_boundary(gpu, B, dtype, kv_split):
    # up to 64 requests: the longest-first schedule (one wave lane per
    # request); more: items in batch order, the metadata walked 64 at a time
    wl = SC.random_parent_batch(seed=B, B=B, Hq=8, Hkv=2, D=128, s_lo=20, s_hi=700, p_lo=1, p_hi=100,
                                dtype=dtype, qkv_scale=0.5)
    _run_and_check(wl, gpu, kv_split=kv_split, label=f"batch{B}-{dtype}-split{kv_split}")


@pytest.mark.parametrize("kv_split", [192, 128])
def test_many_splits_both_combine_paths(gpu, kv_split):
    # 8320 keys per request: 44 splits (per-head weights staged in LDS) and
    # 65 splits (the per-chunk loop for more than 64 splits)
    _run_and_check(SC.qwen3_headline(), gpu, requests=[3], kv_heads=[0, 5], kv_split=kv_split,
                   label=f"headline-split{kv_split}")


@pytest.mark.parametrize("make", [SC.qwen3_headline, SC.stress_mixed], ids=["headline", "stress-b32"])
def test_full_size_exact_properties(gpu, make):
    # size-independent checks at the benchmark shapes, bit for bit:
    #  - V -> 2V (exact in bf16) doubles the output and keeps the LSE;
    #  - permuting the KV heads, with their query-head groups, permutes the
    #    output: each (request, head) sums the same keys in the same order,
    #    whichever workgroup the schedule gives it
    from cast_amd import varlen_tree_attention
    wl = make()
    print(f"case full-size-properties {wl.name}: B={wl.B} total_q={wl.total_q} total_kv={wl.total_kv}", flush=True)
    q, k, v = wl.qkv(device=gpu)
    meta = wl.meta_tensors(gpu)
    mask = torch.from_numpy(_words(wl).view(np.int64).copy()).to(gpu)

    def run(q_, k_, v_):
        o, l = varlen_tree_attention(q_, k_, v_, meta["cu_q"], meta["cu_kv"], meta["prefix_len"], meta["pack_len"],
                                     mask, return_lse=True)
        torch.cuda.synchronize()
        return o, l

    out, lse = run(q, k, v)
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    out2, lse2 = run(q, k, v * 2)
    assert torch.equal(out2, out * 2) and torch.equal(lse2, lse)
    G = wl.Hq // wl.Hkv
    perm = torch.randperm(wl.Hkv, generator=torch.Generator().manual_seed(3)).to(gpu)
    qperm = (perm[:, None] * G + torch.arange(G, device=gpu)[None, :]).reshape(-1)
    out3, lse3 = run(q[:, qperm].contiguous(), k[:, perm].contiguous(), v[:, perm].contiguous())
    assert torch.equal(out3, out[:, qperm]) and torch.equal(lse3, lse[:, qperm])


def test_empty_rows_give_zero_and_minus_inf(gpu):
    from cast_amd import varlen_tree_attention
    wl = SC.random_parent_batch(seed=9, B=2, Hq=8, Hkv=2, D=128, s_lo=0, s_hi=1, p_lo=5, p_hi=6, dtype="bf16")
    q, k, v = wl.qkv(device=gpu)
    words = _words(wl)
    words[1] = 0                          # row 1 sees nothing (S = 0)
    meta = wl.meta_tensors(gpu)
    out, lse = varlen_tree_attention(q, k, v, meta["cu_q"], meta["cu_kv"], meta["prefix_len"], meta["pack_len"],
                                     torch.from_numpy(words.view(np.int64).copy()).to(gpu), return_lse=True)
    assert torch.all(out[1] == 0) and torch.all(torch.isneginf(lse[1]))
    assert torch.isfinite(lse[0]).all()


def test_large_configs_sampled(gpu):
    # full-size inputs, oracle on a sample of (request, KV head) pairs
    for wl, reqs in [(SC.qwen3_headline(), [0, 5]), (SC.llama_long(), [0]), (SC.stress_mixed(), [0, 1, 30])]:
        _run_and_check(wl, gpu, requests=reqs, kv_heads=[0, 7], label=wl.name)


def test_metadata_errors_are_flagged_not_faulted(gpu):
    from cast_amd import varlen_tree_attention
    wl = SC.random_parent_batch(seed=2, B=2, Hq=8, Hkv=2, D=128, s_lo=10, s_hi=20, p_lo=4, p_hi=8, dtype="bf16")
    q, k, v = wl.qkv(device=gpu)
    meta = wl.meta_tensors(gpu)
    mask = torch.from_numpy(_words(wl).view(np.int64).copy()).to(gpu)
    bad = meta["pack_len"].clone()
    bad[0] += 1                           # disagrees with cu_q
    with pytest.raises(ValueError):
        varlen_tree_attention(q, k, v, meta["cu_q"], meta["cu_kv"], meta["prefix_len"], bad, mask, check=True)
    with pytest.raises(AssertionError):
        varlen_tree_attention(q, k[:, :1].expand(-1, 3, -1), v[:, :1].expand(-1, 3, -1), meta["cu_q"],
                              meta["cu_kv"], meta["prefix_len"], meta["pack_len"], mask)


def test_request_order_is_irrelevant(gpu):
    # a full-size property of the static split schedule: each request is
    # computed on its own, and the split plan depends only on batch totals,
    # so reordering the requests of a packed batch reorders the outputs and
    # LSE bit for bit.  (The stream-K schedule cuts its lanes along the batch
    # order, so there the bits of a request depend on its neighbours.)
    from cast_amd import varlen_tree_attention
    wl = SC.qwen3_ragged(seed=5)
    print(f"case request-order: B={wl.B} total_q={wl.total_q} total_kv={wl.total_kv}", flush=True)
    q, k, v = wl.qkv(device=gpu)
    words = torch.from_numpy(_words(wl).view(np.int64).copy()).to(gpu)
    cu_q, cu_kv = list(wl.cu_q), list(wl.cu_kv)
    perm = [3, 0, 7, 5, 1, 6, 2, 4][:wl.B]
    assert sorted(perm) == list(range(wl.B))

    def run(order):
        qs = [q[cu_q[b]:cu_q[b + 1]] for b in order]
        ks = [k[cu_kv[b]:cu_kv[b + 1]] for b in order]
        vs = [v[cu_kv[b]:cu_kv[b + 1]] for b in order]
        ws = [words[cu_q[b]:cu_q[b + 1]] for b in order]
        lq = [int(cu_q[b + 1] - cu_q[b]) for b in order]
        lk = [int(cu_kv[b + 1] - cu_kv[b]) for b in order]
        cq = torch.tensor(np.concatenate([[0], np.cumsum(lq)]), dtype=torch.int32, device=gpu)
        ck = torch.tensor(np.concatenate([[0], np.cumsum(lk)]), dtype=torch.int32, device=gpu)
        pre = torch.tensor([int(wl.prefix_len[b]) for b in order], dtype=torch.int32, device=gpu)
        pk = torch.tensor([int(wl.pack_len[b]) for b in order], dtype=torch.int32, device=gpu)
        out, lse = varlen_tree_attention(torch.cat(qs), torch.cat(ks), torch.cat(vs), cq, ck, pre, pk,
                                         torch.cat(ws), return_lse=True, check=True, kv_split=1024)
        torch.cuda.synchronize()
        return out, lse, lq

    out0, lse0, lq0 = run(list(range(wl.B)))
    out1, lse1, lq1 = run(perm)
    start0 = np.concatenate([[0], np.cumsum(lq0)])
    start1 = np.concatenate([[0], np.cumsum(lq1)])
    for j, b in enumerate(perm):
        a0, a1 = slice(start0[b], start0[b] + lq0[b]), slice(start1[j], start1[j] + lq1[j])
        assert torch.equal(out0[a0], out1[a1]), f"request {b}"
        assert torch.equal(lse0[a0], lse1[a1]), f"request {b}"


def _fp32(wl):
    # the same workload with fp32 q/k/v (the reference hook's arithmetic,
    # cast_trees/serving.py:68-71)
    import dataclasses
    return dataclasses.replace(wl, dtype="fp32", name=wl.name + "-fp32")


def test_fp32_ragged_full_oracle(gpu):
    _run_and_check(_fp32(SC.qwen3_ragged(seed=1)), gpu)


@pytest.mark.parametrize("split", [0, 64, 448, -1])
def test_fp32_split_variants(gpu, split):
    wl = _fp32(SC.qwen3_ragged(seed=4, B=3, lo=100, hi=2500))
    _run_and_check(wl, gpu, kv_split=split, label=f"fp32-ragged-split{split}")


def test_fp32_edges_and_head_dim_64(gpu):
    from cast_amd.tree import TreeNode
    chain = [TreeNode(i, i + 1, i - 1, 0.0) for i in range(127)]
    star = [TreeNode(i, 1, -1, 0.0) for i in range(127)]
    wl = SC._make("edges-fp32", [chain, [], star, chain[:5], star[:63]], [0, 77, 1, 1999, 33],
                  SC.QWEN3_8B, "fp32", 5, 1 / math.sqrt(128))
    _run_and_check(wl, gpu)
    for Hq, Hkv in [(8, 8), (16, 2)]:
        wl = SC.random_parent_batch(seed=Hq, B=3, Hq=Hq, Hkv=Hkv, D=64, s_lo=50, s_hi=900, p_lo=1, p_hi=129,
                                    dtype="fp32")
        _run_and_check(wl, gpu, label=f"fp32-gqa{Hq}/{Hkv}-D64")


def test_fp32_large_configs_sampled(gpu):
    for wl, reqs in [(_fp32(SC.qwen3_headline()), [0, 7]), (_fp32(SC.stress_mixed()), [3, 30])]:
        _run_and_check(wl, gpu, requests=reqs, kv_heads=[0, 5], label=wl.name)


# ---- the stream-K schedule (kv_split=-2 asks for it; the library's own
# choice, kv_split=0, is always the static schedule)

def _edges(dtype="bf16"):
    from cast_amd.tree import TreeNode
    chain = [TreeNode(i, i + 1, i - 1, 0.0) for i in range(127)]
    star = [TreeNode(i, 1, -1, 0.0) for i in range(127)]
    return SC._make("edges", [chain, [], star, chain[:5], star[:63]], [0, 77, 1, 4099, 33], SC.QWEN3_8B, dtype, 5,
                    1 / math.sqrt(128))


STREAM_K_CASES = {
    # B=8, P < 64: one row block per head, two heads per super-group
    "reference-bf16": lambda: SC.random_parent_batch(seed=0, dtype="bf16"),
    "reference-fp32": lambda: SC.random_parent_batch(seed=0, dtype="fp32"),
    "reference-fp16": lambda: SC.random_parent_batch(seed=1, dtype="fp16"),
    # P up to 128 (two row blocks of one head per super-group), long prefixes
    "ragged-small": lambda: SC.qwen3_ragged(seed=3, B=4, lo=100, hi=3000),
    # one KV head (16 row blocks per request), head dim 64
    "mqa-d64": lambda: SC.random_parent_batch(seed=12, B=3, Hq=32, Hkv=1, D=64, s_lo=50, s_hi=1500, p_lo=1,
                                               p_hi=129, dtype="bf16", qkv_scale=0.5),
    # three KV heads with one row block each: the second super-group has one
    # unit, so one member of its lanes idles there
    "odd-heads": lambda: SC.random_parent_batch(seed=13, B=5, Hq=12, Hkv=3, D=128, s_lo=50, s_hi=2000, p_lo=1,
                                                 p_hi=30, dtype="bf16", qkv_scale=0.5),
    # S = 0, P = 1, 128-token chain and star, S not a multiple of 64
    "edges": _edges,
    "head-dim-256": lambda: SC.random_parent_batch(seed=7, B=4, Hq=16, Hkv=8, D=256, s_lo=500, s_hi=4000, p_lo=1,
                                                    p_hi=129, dtype="bf16", qkv_scale=0.5),
    "single-p16": lambda: SC.qwen3_single(),
    "fp32-ragged": lambda: _fp32(SC.qwen3_ragged(seed=4, B=3, lo=100, hi=2500)),
}


@pytest.mark.parametrize("case", list(STREAM_K_CASES))
def test_stream_k_schedule_matches_oracle(gpu, case):
    wl = STREAM_K_CASES[case]()
    _run_and_check(wl, gpu, kv_split=-2, label=f"stream-k-{case}")
    if case.startswith("reference"):
        _run_and_check(wl, gpu, kv_split=-2, one_word=True, label=f"stream-k-{case}-int64-mask")


def _call(wl, dev, kv_split, qkv=None):
    from cast_amd import varlen_tree_attention
    q, k, v = qkv if qkv is not None else wl.qkv(device=dev)
    meta = wl.meta_tensors(dev)
    mask = torch.from_numpy(_words(wl).view(np.int64).copy()).to(dev)
    out, lse = varlen_tree_attention(q, k, v, meta["cu_q"], meta["cu_kv"], meta["prefix_len"], meta["pack_len"],
                                     mask, return_lse=True, kv_split=kv_split, check=True)
    torch.cuda.synchronize()
    return out, lse


def test_schedule_choice_ragged_and_uniform(gpu):
    # The library's own choice (kv_split=0) keeps the static splits on the
    # benchmark's ragged batch (bit for bit the forced chunk); the forced
    # stream-K schedule cuts other pieces (other bits, within the bar).  The
    # uniform headline batch keeps its static splits too.
    from cast_amd.tree_attn import plan
    wl = SC.qwen3_ragged(seed=0)
    print(f"case schedule-choice ragged: B={wl.B} total_q={wl.total_q} total_kv={wl.total_kv}", flush=True)
    qkv = wl.qkv(device=gpu)
    chunk = plan(wl.B, wl.total_q, wl.total_kv, wl.Hq, wl.Hkv, wl.D).kv_split
    auto, sk, static = (_call(wl, gpu, s, qkv) for s in (0, -2, chunk))
    assert torch.equal(auto[0], static[0]) and torch.equal(auto[1], static[1])
    assert not torch.equal(sk[0], static[0])
    assert (sk[0].float() - static[0].float()).abs().max() <= 2e-2
    wl = SC.qwen3_headline()
    print("case schedule-choice headline", flush=True)
    qkv = wl.qkv(device=gpu, generator_device=gpu)
    chunk = plan(wl.B, wl.total_q, wl.total_kv, wl.Hq, wl.Hkv, wl.D).kv_split
    auto, static = (_call(wl, gpu, s, qkv) for s in (0, chunk))
    assert torch.equal(auto[0], static[0]) and torch.equal(auto[1], static[1])


def test_stream_k_exact_scaling_property(gpu):
    # V -> 2V (exact in bf16) doubles the output and keeps the LSE, bit for
    # bit, through the stream-K partials and their merge
    wl = SC.qwen3_ragged(seed=0)
    print("case stream-k-scaling", flush=True)
    q, k, v = wl.qkv(device=gpu)
    out, lse = _call(wl, gpu, -2, (q, k, v))
    out2, lse2 = _call(wl, gpu, -2, (q, k, v * 2))
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    assert torch.equal(out2, out * 2) and torch.equal(lse2, lse)


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("kind", ["far-below", "far-above", "mixed"])
def test_extreme_score_ranges(gpu, dtype, kind):
    # The kernel's online softmax only rescales once a tile's max exceeds
    # the running max by a slack of 2^8, and packs probabilities into the
    # 16-bit format before the PV product.  Scores far below zero, far above
    # it and rows of both kinds in one wave, against the oracle: the
    # probabilities must neither overflow the format nor flush to zero.
    # Keys share a direction u with weight 6; queries lie along +u or -u
    # with weight w, so scaled scores sit near +-6 w / sqrt(D).
    wl = SC.random_parent_batch(seed=21, B=3, Hq=8, Hkv=2, D=128, s_lo=300, s_hi=1500, p_lo=20, p_hi=129,
                                dtype=dtype, qkv_scale=0.3)
    q, k, v = wl.qkv(device="cpu")
    g = torch.Generator().manual_seed(5)
    u = torch.randn(wl.D, generator=g)
    u /= u.norm()
    w = {"bf16": 100.0, "fp16": 24.0}[dtype]   # scaled scores about 76 and 18 in log2 units
    k = (k.float() + 6.0 * u).to(k.dtype)
    sign = {"far-below": -1.0, "far-above": 1.0}.get(kind)
    if sign is None:
        sign = torch.where(torch.arange(wl.total_q) % 3 == 0, 1.0, -1.0)[:, None, None]
    q = (q.float() + sign * w * u).to(q.dtype)
    print(f"case extreme-scores {kind} {dtype}: scaled score ~ {float(6 * w / math.sqrt(wl.D)):.1f}", flush=True)
    _run_and_check(wl, gpu, qkv=(q, k, v), label=f"extreme-scores-{kind}-{dtype}")


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_tree_block_alone(gpu, dtype):
    # the stress batch's 32 trees with no prefix: every tile is a pack tile,
    # and the pack tiles past the last key a workgroup's rows see are skipped
    import dataclasses
    wl = SC.stress_trees_only()
    if dtype == "fp32":
        wl = dataclasses.replace(wl, dtype="fp32", qkv_scale=1.0)
    _run_and_check(wl, gpu, label=f"tree-block-alone-{dtype}")


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
@pytest.mark.parametrize("kv_split", [0, 64])
def test_arbitrary_visibility_words(gpu, dtype, kv_split):
    # Visibility words that no tree produces: random bits anywhere in the
    # pack (above a row's own index too), rows that see no pack key, rows
    # that see only the last pack key, and one-sided 64-key halves.  Skipped
    # pack tiles and blocks are decided from the words themselves, so every
    # case matches the oracle on the same words.
    wl = SC.random_parent_batch(seed=17, B=6, Hq=8, Hkv=2, D=128, s_lo=0, s_hi=300, p_lo=1, p_hi=129,
                                dtype=dtype)
    rng = np.random.default_rng(4)
    words = np.zeros((wl.total_q, 2), dtype=np.uint64)
    for b in range(wl.B):
        P, q0 = int(wl.pack_len[b]), int(wl.cu_q[b])
        for i in range(P):
            kind = (b + i) % 5
            if kind == 0:
                bits = rng.random(P) < 0.3                       # random, any position
            elif kind == 1:
                bits = np.zeros(P, dtype=bool)                   # no pack key
            elif kind == 2:
                bits = np.zeros(P, dtype=bool)
                bits[P - 1] = True                               # only the last pack key
            elif kind == 3:
                bits = np.zeros(P, dtype=bool)
                bits[: min(P, 64)] = rng.random(min(P, 64)) < 0.5    # first half only
            else:
                bits = np.zeros(P, dtype=bool)
                bits[64:] = rng.random(max(0, P - 64)) < 0.5         # second half only
            for j in np.flatnonzero(bits):
                words[q0 + i, j >> 6] |= np.uint64(1) << np.uint64(j & 63)
    print(f"case arbitrary-words {dtype} split={kv_split}: B={wl.B} total_q={wl.total_q}", flush=True)
    _run_and_check(wl, gpu, kv_split=kv_split, words=words, label=f"arbitrary-words-{dtype}-{kv_split}")


def test_fp32_head_dim_256_edges(gpu):
    # fp32 at head dim 256: 32-key tiles (one MFMA block a tile), the tree
    # block alone, a single root, chains and stars, the one-word mask, and
    # packs whose pack tiles no row of a workgroup sees past some key
    import dataclasses
    wl = dataclasses.replace(_edges("fp32"), Hq=8, Hkv=4, D=256, qkv_scale=0.5)
    for split in (0, 128):
        _run_and_check(wl, gpu, kv_split=split, label=f"fp32-d256-edges-split{split}")
    wl = SC.random_parent_batch(seed=31, B=4, Hq=8, Hkv=2, D=256, s_lo=0, s_hi=200, p_lo=1, p_hi=65,
                                dtype="fp32", qkv_scale=0.5)
    for split in (0, 64):
        _run_and_check(wl, gpu, kv_split=split, one_word=True, label=f"fp32-d256-one-word-split{split}")
