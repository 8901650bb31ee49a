"""A verify round's device steps make no host synchronisation: the bitmask,
the attention call (check=False, as the serving hook makes it), the greedy
accept and the accepted-path KV append (explicit pack lists, fresh views
every round, and the hook-recorded path), all with device-resident inputs.
torch's sync debug mode turns any synchronising torch operation inside them
into an error."""
import pytest
import torch

from cast_amd import scenarios as SC

pytestmark = pytest.mark.gpu


def test_round_steps_do_not_sync(gpu):
    from cast_amd import greedy_accept, serving, tree_bitmask, varlen_tree_attention
    wl = SC.qwen3_ragged(seed=2, B=4, lo=200, hi=1500, vocab=4096)
    print(f"case no-sync: B={wl.B} total_q={wl.total_q} total_kv={wl.total_kv}", flush=True)
    meta = wl.meta_tensors(gpu)
    q, k, v = wl.qkv(device=gpu)
    logits, _ = SC.planted_logits(wl, seed=1)
    logits = logits.to(gpu)
    token = torch.from_numpy(wl.packed.token).to(gpu)
    L, B, Hkv, D = 3, wl.B, wl.Hkv, wl.D
    cap = int(wl.prefix_len.max()) + 160
    g = torch.Generator(device=gpu).manual_seed(4)
    buf_k = [torch.zeros((B, Hkv, cap, D), dtype=torch.bfloat16, device=gpu) for _ in range(L)]
    buf_v = [torch.zeros_like(x) for x in buf_k]
    pack = [torch.randn((wl.total_q, Hkv, D), generator=g, device=gpu).to(torch.bfloat16) for _ in range(2 * L)]
    store_len = torch.from_numpy(wl.prefix_len.astype("int32")).to(gpu)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        for _ in range(2):
            mask = tree_bitmask(meta["parent"], meta["cu_q"], 2)
            varlen_tree_attention(q, k, v, meta["cu_q"], meta["cu_kv"], meta["prefix_len"], meta["pack_len"], mask)
            path, plen, _, _ = greedy_accept(logits, meta["cu_q"], meta["parent"], token)
            # the packs as HF hands them over: new [Hkv, total_q, D] views every round
            pk = [x.transpose(0, 1) for x in pack[:L]]
            pv = [x.transpose(0, 1) for x in pack[L:]]
            serving.append_accepted(buf_k, buf_v, store_len, meta["cu_q"], path, plen, pk, pv)
            # the serving flow: the hook recorded each layer's pack as the forward ran
            serving.PACK_KV["k"], serving.PACK_KV["v"] = pk, pv
            serving._PACK_REC.begin(L)
            for li in range(L):
                serving._PACK_REC.note(li, pk[li], pv[li])
            serving.append_accepted(buf_k, buf_v, store_len, meta["cu_q"], path, plen)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()


def test_batch_one_tree_hook_does_not_sync(gpu):
    # the "cast_tree" attention of the batch-one verify (cast_trees/decode.py:
    # 166-171): the mask from tree_attention_mask carries its kernel metadata,
    # so building it and running the hook for several layers never waits on
    # the device.  The result is then checked against SDPA with the same mask.
    from cast_amd import serving
    from cast_amd.verify import tree_attention_mask
    wl = SC.qwen3_single(seed=3, prefix=300, pack=40)
    nodes, S, n = wl.trees[0], 300, 40
    Hq, Hkv, D = wl.Hq, wl.Hkv, wl.D
    g = torch.Generator(device=gpu).manual_seed(5)
    q = torch.randn((1, Hq, n, D), generator=g, device=gpu).to(torch.bfloat16)
    key = torch.randn((1, Hkv, S + n, D), generator=g, device=gpu).to(torch.bfloat16)
    value = torch.randn((1, Hkv, S + n, D), generator=g, device=gpu).to(torch.bfloat16)
    print(f"case no-sync batch-one hook: S={S} n={n}", flush=True)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        mask = tree_attention_mask(S, nodes, gpu, torch.bfloat16)
        outs = [serving._tree_attention(None, q, key, value, mask, scaling=D ** -0.5)[0] for _ in range(3)]
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    assert all(torch.equal(o, outs[0]) for o in outs)
    G = Hq // Hkv
    kf = key.float().cpu().repeat_interleave(G, 1)
    vf = value.float().cpu().repeat_interleave(G, 1)
    want = torch.nn.functional.scaled_dot_product_attention(q.float().cpu(), kf, vf,
                                                            attn_mask=mask.float().cpu(), scale=D ** -0.5)
    err = (outs[0].float().cpu() - want.transpose(1, 2)).abs().max().item()
    print(f"  out max err {err:.3e}", flush=True)
    assert err <= 2e-2
