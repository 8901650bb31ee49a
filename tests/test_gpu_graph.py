"""The verify step's launches under HIP graph capture: the attention call
(split-K partials and combine), the ancestor bitmask and the greedy accept
record only kernel launches (no memsets, no allocation inside the library,
no host sync), so a captured round replays them.  Each replay runs on new
input values copied into the captured tensors, with eager calls and
synchronisations between replays, and must equal the eager result bit for
bit."""
import numpy as np
import pytest
import torch

from cast_amd import scenarios as SC

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,make,kv_split", [
    ("single-split128", lambda: SC.qwen3_single(), 0),
    ("ragged-b4-split256", lambda: SC.qwen3_ragged(seed=6, B=4, lo=150, hi=2000, vocab=4096), 256),
], ids=["single", "ragged"])
def test_captured_round_replays_match_eager(gpu, name, make, kv_split):
    from cast_amd import greedy_accept, tree_bitmask, varlen_tree_attention
    wl = make()
    print(f"case graph {name}: B={wl.B} total_q={wl.total_q} total_kv={wl.total_kv} split={kv_split}", flush=True)
    meta = wl.meta_tensors(gpu)
    q, k, v = (x.clone() for x in wl.qkv(device=gpu))
    V = 4096
    g = torch.Generator(device=gpu).manual_seed(9)
    logits = torch.randn((wl.total_q, V), generator=g, device=gpu).to(torch.bfloat16)
    token = torch.randint(0, V, (wl.total_q,), generator=g, device=gpu)
    out = torch.empty_like(q)
    ws = torch.empty(1 << 24, dtype=torch.uint8, device=gpu)

    def step():
        mask = tree_bitmask(meta["parent"], meta["cu_q"], 2)
        varlen_tree_attention(q, k, v, meta["cu_q"], meta["cu_kv"], meta["prefix_len"], meta["pack_len"], mask,
                              kv_split=kv_split, out=out, workspace=ws)
        return greedy_accept(logits, meta["cu_q"], meta["parent"], token)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()                                   # warm up outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gpath, glen, gbonus, garg = step()
    for rep in range(4):
        # new values in the captured inputs
        q.copy_(torch.randn(q.shape, generator=g, device=gpu).to(q.dtype))
        logits.copy_(torch.randn(logits.shape, generator=g, device=gpu).to(logits.dtype))
        graph.replay()
        torch.cuda.synchronize()
        got = [out.clone(), gpath.clone(), glen.clone(), gbonus.clone(), garg.clone()]
        # eager work between replays, then the eager reference on the same values
        ref_path, ref_len, ref_bonus, ref_arg = step()
        torch.cuda.synchronize()
        assert torch.equal(got[0], out), f"replay {rep}: attention"
        assert torch.equal(got[4], ref_arg) and torch.equal(got[2], ref_len) and torch.equal(got[3], ref_bonus)
        n = int(ref_len.max().item())
        assert torch.equal(got[1][:, :n], ref_path[:, :n]), f"replay {rep}: path"
        assert np.isfinite(got[0].float().cpu().numpy()).all()
