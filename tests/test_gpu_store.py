"""Tree attention over the per-request KV store, read in place, and the HF
attention hook built on it (cast_trees/serving.py:48-75, 191-253).

Bars:
  * store layout vs ragged concat layout: bit-identical outputs and LSE (the
    same keys in the same order through the same kernel; only the addressing
    differs), with the store slots past each prefix filled with NaN so a read
    beyond S_b cannot go unnoticed;
  * both vs the dense fp32 oracle: the tolerances of test_gpu_attn.py;
  * the hook inside a random-init Qwen3 (transformers), batched ragged verify
    vs the reference's batch-one dense path per request (SDPA with the additive
    tree mask of cast_trees/verify.py:15-25, cast_trees/decode.py:166-171):
    logits within 2e-2 of the logit scale and identical greedy walks.
"""
import numpy as np
import pytest
import torch

from cast_amd import scenarios as SC
from oracle import attn as OA
from oracle import bitmask as OB

pytestmark = pytest.mark.gpu

TOL = {"bf16": dict(out=2e-2, lse=1e-3, mean=2e-3), "fp16": dict(out=5e-3, lse=1e-3, mean=5e-4),
       "fp32": dict(out=1e-4, lse=1e-4, mean=1e-5)}


def _to_store(wl, q, k, v, dev, extra=37):
    """The reference server's layout: buf [B, Hkv, cap, D] holding request b's
    prefix in slots [0, S_b) (NaN after), and the pass's pack K/V as HF hands
    it over, [Hkv, total_q, D] viewed from token-major storage."""
    cap = int(max(wl.prefix_len)) + extra
    kst = torch.full((wl.B, wl.Hkv, cap, wl.D), float("nan"), dtype=q.dtype, device=dev)
    vst = torch.full_like(kst, float("nan"))
    kpk = torch.empty((wl.total_q, wl.Hkv, wl.D), dtype=q.dtype, device=dev)
    vpk = torch.empty_like(kpk)
    for b in range(wl.B):
        kv0, S, P, q0 = int(wl.cu_kv[b]), int(wl.prefix_len[b]), int(wl.pack_len[b]), int(wl.cu_q[b])
        kst[b, :, :S] = k[kv0:kv0 + S].transpose(0, 1)
        vst[b, :, :S] = v[kv0:kv0 + S].transpose(0, 1)
        kpk[q0:q0 + P] = k[kv0 + S:kv0 + S + P]
        vpk[q0:q0 + P] = v[kv0 + S:kv0 + S + P]
    return kst, vst, kpk.transpose(0, 1), vpk.transpose(0, 1)


def _check_store(wl, dev, kv_split=0, requests=None, label=""):
    from cast_amd import varlen_tree_attention
    from cast_amd.tree_attn import store_tree_attention
    print(f"case {label or wl.name}: B={wl.B} total_q={wl.total_q} total_kv={wl.total_kv} {wl.dtype} "
          f"split={kv_split}", flush=True)
    q, k, v = wl.qkv(device=dev)
    words = OB.chain_walk_words(wl.packed.parent, wl.cu_q)
    mask = torch.from_numpy(words.view(np.int64).copy()).to(dev)
    meta = wl.meta_tensors(dev)
    kst, vst, kpk, vpk = _to_store(wl, q, k, v, dev)
    # the hook's query: query[0].transpose(0, 1), head-major storage
    qh = q.transpose(0, 1).contiguous().transpose(0, 1)
    o_s, l_s = store_tree_attention(qh, kst, vst, kpk, vpk, meta["cu_q"], meta["prefix_len"], meta["pack_len"],
                                    mask, total_kv=wl.total_kv, return_lse=True, kv_split=kv_split, check=True)
    o_c, l_c = varlen_tree_attention(q, k, v, meta["cu_q"], meta["cu_kv"], meta["prefix_len"], meta["pack_len"],
                                     mask, return_lse=True, kv_split=kv_split, check=True)
    torch.cuda.synchronize()
    assert torch.equal(o_s, o_c), "store layout differs from the concat layout"
    assert torch.equal(l_s, l_c)
    ref_o, ref_l = OA.dense_tree_attention(q.float().cpu(), k.float().cpu(), v.float().cpu(), wl.cu_q, wl.cu_kv,
                                           wl.prefix_len, wl.pack_len, words, requests=requests)
    sel = ~torch.isnan(ref_l)
    err_o = (o_s.float().cpu() - ref_o).abs()[sel]
    fin = sel & torch.isfinite(ref_l)
    err_l = (l_s.cpu() - ref_l).abs()[fin]
    tol = TOL[wl.dtype]
    print(f"  out max {err_o.max():.3e} mean {err_o.mean():.3e}  lse max {err_l.max():.3e}", flush=True)
    assert torch.isfinite(o_s.float().cpu()[sel]).all()
    assert err_o.max() <= tol["out"] and err_o.mean() <= tol["mean"] and err_l.max() <= tol["lse"]


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32"])
def test_store_reference_scenario(gpu, dtype):
    _check_store(SC.random_parent_batch(seed=1, dtype=dtype), gpu, label=f"store-reference-scenario-{dtype}")


@pytest.mark.parametrize("dtype,B,kv_split", [("bf16", 4, 0), ("fp32", 4, 128), ("bf16", 70, 0), ("fp32", 70, -1),
                                              ("fp16", 4, 128), ("fp16", 70, 0)])
def test_store_head_dim_64_and_large_batches(gpu, dtype, B, kv_split):
    # D = 64 instances and batches past 64 requests (batch-order schedule) in the store layout
    wl = SC.random_parent_batch(seed=B + 3, B=B, Hq=16, Hkv=4, D=64, s_lo=30, s_hi=600, p_lo=1, p_hi=90,
                                dtype=dtype, qkv_scale=0.5)
    _check_store(wl, gpu, kv_split=kv_split, label=f"store-d64-b{B}-{dtype}-split{kv_split}")


def test_store_head_dim_256(gpu):
    # head_dim 256 (the MFMA kernels at one wave per SIMD) reading the store in place
    for dt, split in (("bf16", 0), ("fp16", 192), ("fp32", 0), ("fp32", 96)):
        wl = SC.random_parent_batch(seed=11, B=3, Hq=8, Hkv=4, D=256, s_lo=100, s_hi=2000, p_lo=1, p_hi=129,
                                    dtype=dt, qkv_scale=0.5)
        _check_store(wl, gpu, kv_split=split, label=f"store-d256-{dt}-split{split}")


@pytest.mark.parametrize("seed", range(64))
def test_random_configurations(gpu, seed):
    # seeded random shapes across features the other tests take one at a time:
    # batches past 64 requests, GQA ratios down to one KV head, head dims on
    # the MFMA and scalar kernels, the three element types, split-K settings
    # (stream-K included), short and long packs (trimmed pack tiles); both
    # K/V layouts, bit-identical to each other, and sampled requests against
    # the oracle
    rng = np.random.default_rng(1000 + seed)
    Hkv, G = int(rng.choice([1, 2, 4, 8])), int(rng.choice([1, 2, 4, 8]))
    D = int(rng.choice([64, 96, 128, 256]))
    dt = str(rng.choice(["bf16", "fp16", "fp32"]))
    B = int(rng.choice([1, 3, 8, 17, 40, 70]))
    s_hi = int(rng.choice([2, 300, 2500, 5000]))
    p_hi = int(rng.choice([17, 65, 129]))
    split = int(rng.choice([0, 64, 128, 320, -1, -2]))
    wl = SC.random_parent_batch(seed=seed, B=B, Hq=Hkv * G, Hkv=Hkv, D=D, s_lo=0, s_hi=s_hi, p_lo=1, p_hi=p_hi,
                                dtype=dt, qkv_scale=0.5)
    requests = sorted(rng.choice(B, size=min(B, 3), replace=False).tolist())
    _check_store(wl, gpu, kv_split=split, requests=requests,
                 label=f"random-{seed}: Hq={Hkv * G} Hkv={Hkv} D={D} {dt} B={B} S<{s_hi} P<{p_hi} split={split}")


def test_store_empty_and_tiny_prefixes(gpu):
    # S_b in {0, 1, 2}: tiles that start inside the pack, single-key prefixes
    wl = SC.random_parent_batch(seed=2, s_lo=0, s_hi=3, p_lo=1, p_hi=80, dtype="bf16")
    assert (wl.prefix_len == 0).any()
    _check_store(wl, gpu, label="store-empty-prefix")


def test_store_ragged_split_k(gpu):
    wl = SC.qwen3_ragged(seed=4, B=4, lo=300, hi=5000)
    for split in (0, 64, 1000, -1, -2):
        _check_store(wl, gpu, kv_split=split, requests=[0, 3], label=f"store-ragged-split{split}")


def test_store_rejects_prefix_beyond_capacity_and_low_total(gpu):
    from cast_amd.tree_attn import store_tree_attention
    wl = SC.random_parent_batch(seed=5, B=3, dtype="bf16")
    q, k, v = wl.qkv(device=gpu)
    mask = torch.from_numpy(OB.chain_walk_words(wl.packed.parent, wl.cu_q).view(np.int64).copy()).to(gpu)
    meta = wl.meta_tensors(gpu)
    kst, vst, kpk, vpk = _to_store(wl, q, k, v, gpu, extra=0)
    print("case store-errors: prefix beyond capacity", flush=True)
    bad = meta["prefix_len"].clone()
    bad[1] = kst.shape[2] + 1
    with pytest.raises(ValueError, match="inconsistent"):
        store_tree_attention(q, kst, vst, kpk, vpk, meta["cu_q"], bad, meta["pack_len"], mask, check=True)
    print("case store-errors: total_kv bound below the batch", flush=True)
    with pytest.raises(ValueError, match="inconsistent"):
        store_tree_attention(q, kst, vst, kpk, vpk, meta["cu_q"], meta["prefix_len"], meta["pack_len"], mask,
                             total_kv=wl.total_kv - 1, check=True)
    # host-side shape errors
    with pytest.raises(ValueError):
        store_tree_attention(q, kst, vst, kpk[:, :-1], vpk, meta["cu_q"], meta["prefix_len"], meta["pack_len"], mask)
    with pytest.raises(ValueError):
        store_tree_attention(q, kst.float(), vst, kpk, vpk, meta["cu_q"], meta["prefix_len"], meta["pack_len"], mask)


# ---------------------------------------------------------------- HF hook

def _tiny_qwen3(dev):
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen3Config(vocab_size=2048, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                                   num_attention_heads=8, num_key_value_heads=2, head_dim=128,
                                   max_position_embeddings=4096)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    model = transformers.Qwen3ForCausalLM(cfg)
    with torch.no_grad():
        for p in model.parameters():       # larger weights than the default init: non-trivial attention
            if p.dim() == 2:
                p.normal_(0.0, 0.06)
    return model.to(dev, torch.bfloat16).eval()


def _layer_kv(cache, li):
    layer = cache.layers[li]
    return layer.keys, layer.values


@torch.inference_mode()
def test_hf_hook_matches_dense_batch_one_path(gpu):
    transformers = pytest.importorskip("transformers")
    from cast_amd import serving, tree as T
    from cast_amd.verify import tree_attention_mask
    from oracle import walk as OW
    assert serving.register()
    model = _tiny_qwen3(gpu)
    V, L = model.config.vocab_size, model.config.num_hidden_layers
    rng = np.random.default_rng(7)
    prefix = [200, 333, 64]
    budgets = [15, 40, 127]
    B = len(prefix)
    prompts = [torch.from_numpy(rng.integers(0, V, size=S)).to(gpu) for S in prefix]
    caches = []
    for ids in prompts:
        c = transformers.DynamicCache()
        model(ids[None], past_key_values=c, use_cache=True)
        caches.append(c)
    cap = max(prefix) + 320
    Hkv, D = model.config.num_key_value_heads, model.config.head_dim
    buf_k = [torch.zeros((B, Hkv, cap, D), dtype=torch.bfloat16, device=gpu) for _ in range(L)]
    buf_v = [torch.zeros_like(x) for x in buf_k]
    for li in range(L):
        for b in range(B):
            kk, vv = _layer_kv(caches[b], li)
            buf_k[li][b, :, :prefix[b]] = kk[0]
            buf_v[li][b, :, :prefix[b]] = vv[0]
    trees = []
    for b in range(B):
        top_idx, top_lp = T.block_topk(rng.normal(scale=3.0, size=(15, V)), 8)
        trees.append(T.build_tree(top_idx, top_lp, budgets[b]))
    roots = [int(rng.integers(0, V)) for _ in range(B)]
    print(f"case hf-hook: prefixes {prefix}, packs {[1 + len(t) for t in trees]}", flush=True)

    ids, pos, cu_q = serving.begin_verify(buf_k, buf_v, prefix, roots, trees, prefix)
    prev = model.config._attn_implementation
    model.config._attn_implementation = "cast_varlen"
    try:
        got = model(ids, position_ids=pos, past_key_values=transformers.DynamicCache(), use_cache=True).logits[0]
    finally:
        model.config._attn_implementation = prev
        serving.PLAN.clear()
    assert all(serving.PACK_KV["k"][li] is not None for li in range(L))

    for b in range(B):
        nodes = trees[b]
        toks = torch.tensor([[roots[b]] + [nd.token for nd in nodes]], device=gpu)
        p = torch.tensor([[prefix[b]] + [prefix[b] + nd.depth for nd in nodes]], device=gpu)
        mask = tree_attention_mask(prefix[b], nodes, gpu, torch.bfloat16)
        want = model(toks, position_ids=p, past_key_values=caches[b], use_cache=True, attention_mask=mask).logits[0]
        g = got[cu_q[b]:cu_q[b + 1]].float()
        w = want.float()
        scale = w.abs().max().item()
        err = (g - w).abs().max().item()
        print(f"  request {b}: logits max |diff| {err:.3e} (scale {scale:.2f})", flush=True)
        assert err <= 2e-2 * scale
        assert OW.greedy_walk(nodes, g.cpu()) == OW.greedy_walk(nodes, w.cpu())


@torch.inference_mode()
def test_hf_batch_one_tree_hook_matches_sdpa(gpu):
    # cast_trees/decode.py:166-171: the target forward over [root] + nodes with
    # past_key_values = the prefix cache and the additive tree mask, here with
    # attn "cast_tree" (the tree kernel, K/V read from the cache in place) vs
    # "sdpa" on an identical cache
    import copy
    transformers = pytest.importorskip("transformers")
    from cast_amd import serving, tree as T
    from cast_amd.verify import tree_attention_mask
    from oracle import walk as OW
    assert serving.register()
    model = _tiny_qwen3(gpu)
    V = model.config.vocab_size
    rng = np.random.default_rng(11)
    for S, budget in ((77, 15), (300, 63), (1030, 127)):
        print(f"case hf-tree-hook: prefix {S}, nodes {budget}", flush=True)
        prompt = torch.from_numpy(rng.integers(0, V, size=S)).to(gpu)
        cache = transformers.DynamicCache()
        model(prompt[None], past_key_values=cache, use_cache=True)
        top_idx, top_lp = T.block_topk(rng.normal(scale=3.0, size=(15, V)), 8)
        nodes = T.build_tree(top_idx, top_lp, budget)
        toks = torch.tensor([[int(rng.integers(0, V))] + [nd.token for nd in nodes]], device=gpu)
        pos = torch.tensor([[S] + [S + nd.depth for nd in nodes]], device=gpu)
        mask = tree_attention_mask(S, nodes, gpu, torch.bfloat16)
        logits = {}
        for impl in ("sdpa", "cast_tree"):
            model.config._attn_implementation = impl
            c = copy.deepcopy(cache)
            logits[impl] = model(toks, position_ids=pos, past_key_values=c, use_cache=True,
                                 attention_mask=mask).logits[0].float()
        model.config._attn_implementation = "sdpa"
        w, g = logits["sdpa"], logits["cast_tree"]
        scale = w.abs().max().item()
        err = (g - w).abs().max().item()
        print(f"  logits max |diff| {err:.3e} (scale {scale:.2f})", flush=True)
        assert err <= 2e-2 * scale
        assert OW.greedy_walk(nodes, g.cpu()) == OW.greedy_walk(nodes, w.cpu())
    # a forward without a tree mask (prefill) goes through plain SDPA
    model.config._attn_implementation = "cast_tree"
    ids = torch.from_numpy(rng.integers(0, V, size=40)).to(gpu)[None]
    a = model(ids).logits
    model.config._attn_implementation = "sdpa"
    b = model(ids).logits
    assert torch.equal(a, b)


def test_bf16_hook_with_outlier_key_channels(gpu):
    # The reference hook up-casts to fp32 because "large outlier channels in
    # K make a bf16 dot lossy" (cast_trees/serving.py:68).  Plant such
    # channels at the headline shapes: four of the 128 head-dim channels of
    # K carry +-30 with a per-channel sign, Q carries 10 with the same signs,
    # so every score gets a large common offset plus a wide spread (a peaky
    # softmax).  The bf16 store path (fp32 accumulation, P rounded to bf16
    # before the value product) must stay within the bf16 bar of the fp32
    # oracle on the same bf16 inputs.
    from cast_amd.tree_attn import store_tree_attention
    wl = SC.qwen3_headline()
    print(f"case outlier-k: B={wl.B} total_q={wl.total_q} total_kv={wl.total_kv}", flush=True)
    q, k, v = wl.qkv(device=gpu)
    g = torch.Generator(device=gpu).manual_seed(17)
    chans = torch.tensor([3, 17, 64, 99], device=gpu)
    sign = torch.tensor([1.0, -1.0, 1.0, -1.0], device=gpu)
    kf, qf = k.float(), q.float()
    kf[:, :, chans] = sign * 30.0 + 5.0 * torch.randn((k.shape[0], k.shape[1], 4), generator=g, device=gpu)
    qf[:, :, chans] = sign * 10.0
    k, q = kf.to(torch.bfloat16), qf.to(torch.bfloat16)
    words = OB.chain_walk_words(wl.packed.parent, wl.cu_q)
    mask = torch.from_numpy(words.view(np.int64).copy()).to(gpu)
    meta = wl.meta_tensors(gpu)
    kst, vst, kpk, vpk = _to_store(wl, q, k, v, gpu)
    qh = q.transpose(0, 1).contiguous().transpose(0, 1)
    out, lse = store_tree_attention(qh, kst, vst, kpk, vpk, meta["cu_q"], meta["prefix_len"], meta["pack_len"],
                                    mask, total_kv=wl.total_kv, return_lse=True, check=True)
    torch.cuda.synchronize()
    reqs = [0, 3, 6]
    ref_o, ref_l = OA.dense_tree_attention(q.float().cpu(), k.float().cpu(), v.float().cpu(), wl.cu_q, wl.cu_kv,
                                           wl.prefix_len, wl.pack_len, words, requests=reqs, kv_heads=[0, 4, 7])
    sel = ~torch.isnan(ref_l)
    err_o = (out.float().cpu() - ref_o).abs()[sel]
    err_l = (lse.cpu() - ref_l).abs()[sel]
    # the planted channels add a common offset of ~106 to every score (LSE > 40)
    top = ref_l[sel]
    print(f"  lse range {top.min():.1f}..{top.max():.1f}; out max {err_o.max():.3e} mean {err_o.mean():.3e} "
          f"lse max {err_l.max():.3e}", flush=True)
    assert float(top.min()) > 40.0
    assert err_o.max() <= 2e-2 and err_o.mean() <= 2e-3 and err_l.max() <= 1e-3
