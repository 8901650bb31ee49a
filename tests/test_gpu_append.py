"""Accepted-path KV append (cast_trees/serving.py:264-289) on the GPU.

Bar: bit-identical stores and lengths against the oracle's row-by-row
restatement of the reference's _append_store (batch compaction, capacity
growth, then every kept pack row into its store slot) and of gather_cache
(cast_trees/verify.py:48-60).
"""
import numpy as np
import pytest
import torch

from cast_amd import scenarios as SC
from oracle import store as OS

pytestmark = pytest.mark.gpu


def _setup(dev, seed, B=5, L=3, Hkv=4, D=128, cap=96, dtype=torch.bfloat16):
    rng = np.random.default_rng(seed)
    g = torch.Generator(device=dev).manual_seed(seed)
    pack_len = [int(x) for x in rng.integers(1, 40, size=B)]
    cu_q = [0] + list(np.cumsum(pack_len))
    total_q = cu_q[-1]
    store_len = [int(x) for x in rng.integers(0, cap - 20, size=B)]
    buf_k = [torch.randn((B, Hkv, cap, D), generator=g, device=dev).to(dtype) for _ in range(L)]
    buf_v = [torch.randn((B, Hkv, cap, D), generator=g, device=dev).to(dtype) for _ in range(L)]
    # HF hands the pack over as key[0]: [Hkv, total_q, D] viewed from token-major storage
    pack_k = [torch.randn((total_q, Hkv, D), generator=g, device=dev).to(dtype).transpose(0, 1) for _ in range(L)]
    pack_v = [torch.randn((total_q, Hkv, D), generator=g, device=dev).to(dtype).transpose(0, 1) for _ in range(L)]
    keep, accepted = [], []
    for b in range(B):
        n = int(rng.integers(0, min(pack_len[b], 12)))
        path = sorted(rng.choice(np.arange(pack_len[b] - 1), size=min(n, pack_len[b] - 1), replace=False).tolist())
        keep.append([0] + [i + 1 for i in path])
        accepted.append(len(path) + 1)
    return buf_k, buf_v, pack_k, pack_v, store_len, cu_q, keep, accepted


@pytest.mark.parametrize("case", ["all-rows", "compact", "grow", "fp32-d64", "fp16", "fp32-d256", "bf16-d256"])
def test_append_store_matches_reference(gpu, case):
    # fp32 at head dim 256 has 1024-byte rows: two 512-byte column slices
    # per (request, layer, head), one workgroup each
    from cast_amd import serving
    kw = {"fp32-d64": dict(D=64, dtype=torch.float32), "fp16": dict(dtype=torch.float16),
          "fp32-d256": dict(D=256, dtype=torch.float32, Hkv=2),
          "bf16-d256": dict(D=256, Hkv=2)}.get(case, {})
    buf_k, buf_v, pack_k, pack_v, store_len, cu_q, keep, accepted = _setup(gpu, seed=len(case), **kw)
    B = len(store_len)
    rows = [0, 2, 3] if case == "compact" else list(range(B))
    if case == "grow":
        store_len[1] = buf_k[0].shape[2] - 1          # one slot left: the append must grow the stores
        keep[1], accepted[1] = [0, 1, 2], 3
    print(f"case append-{case}: B={B} rows={rows} store_len={store_len} accepted={accepted}", flush=True)
    ref = OS.append_store([x.clone() for x in buf_k], [x.clone() for x in buf_v], pack_k, pack_v, store_len,
                            cu_q, keep, accepted, rows)
    serving.PACK_KV["k"], serving.PACK_KV["v"] = pack_k, pack_v
    got = serving.append_store([x.clone() for x in buf_k], [x.clone() for x in buf_v], store_len, cu_q, keep,
                               accepted, rows)
    torch.cuda.synchronize()
    assert got[2] == ref[2]
    for a, b in zip(got[0] + got[1], ref[0] + ref[1]):
        assert a.shape == b.shape and torch.equal(a, b)


def test_append_accepted_from_greedy_accept(gpu):
    # the device path: greedy_accept's path / path_len drive the append, no host sync
    from cast_amd import greedy_accept, serving
    wl = SC.qwen3_ragged(seed=3, B=4, lo=64, hi=200, packs=(16, 64, 128), vocab=4096)
    logits, _ = SC.planted_logits(wl, seed=1)
    meta = wl.meta_tensors(gpu)
    path, plen, bonus, _ = greedy_accept(logits.to(gpu), meta["cu_q"], meta["parent"],
                                         torch.from_numpy(wl.packed.token).to(gpu))
    L, Hkv, D, cap = 2, wl.Hkv, wl.D, 400
    g = torch.Generator(device=gpu).manual_seed(0)
    store_len = [int(x) for x in wl.prefix_len]
    buf_k = [torch.randn((wl.B, Hkv, cap, D), generator=g, device=gpu).to(torch.bfloat16) for _ in range(L)]
    buf_v = [torch.randn((wl.B, Hkv, cap, D), generator=g, device=gpu).to(torch.bfloat16) for _ in range(L)]
    pack_k = [torch.randn((Hkv, wl.total_q, D), generator=g, device=gpu).to(torch.bfloat16) for _ in range(L)]
    pack_v = [torch.randn((Hkv, wl.total_q, D), generator=g, device=gpu).to(torch.bfloat16) for _ in range(L)]
    print(f"case append-accepted: B={wl.B} store_len={store_len}", flush=True)
    got_k, got_v = [x.clone() for x in buf_k], [x.clone() for x in buf_v]
    new_len = serving.append_accepted(got_k, got_v, store_len, meta["cu_q"], path, plen, pack_k, pack_v, check=True)
    plen_h, path_h = plen.cpu().tolist(), path.cpu().tolist()
    keep = [[0] + [i + 1 for i in path_h[b][:plen_h[b]]] for b in range(wl.B)]
    accepted = [len(k) for k in keep]
    ref = OS.append_store([x.clone() for x in buf_k], [x.clone() for x in buf_v], pack_k, pack_v, store_len,
                            [int(x) for x in wl.cu_q], keep, accepted, list(range(wl.B)))
    assert new_len.cpu().tolist() == ref[2]
    assert max(accepted) > 1
    for a, b in zip(got_k + got_v, ref[0] + ref[1]):
        assert torch.equal(a, b)


def _path_tensors(keep, dev):
    B = len(keep)
    path = torch.full((B, 128), -1, dtype=torch.int32, device=dev)
    for b in range(B):
        if len(keep[b]) > 1:
            path[b, :len(keep[b]) - 1] = torch.tensor([k - 1 for k in keep[b][1:]], dtype=torch.int32)
    plen = torch.tensor([len(k) - 1 for k in keep], dtype=torch.int32, device=dev)
    return path, plen


def test_append_more_layers_than_one_launch(gpu):
    # 130 layers: three launches of at most 64 layers.  Every launch reads
    # store_len as the caller passed it; new_len and the overflow flag come
    # from the first launch only.
    from cast_amd import serving
    L, B = 130, 4
    buf_k, buf_v, pack_k, pack_v, store_len, cu_q, keep, accepted = _setup(gpu, seed=33, B=B, L=L, Hkv=2, D=64)
    keep[1] = keep[1] if len(keep[1]) > 1 else [0, 1]
    accepted[1] = len(keep[1])
    path, plen = _path_tensors(keep, gpu)
    cq = torch.tensor(cu_q, dtype=torch.int32, device=gpu)
    print(f"case append-{L}-layers: B={B} store_len={store_len} accepted={accepted}", flush=True)
    got_k, got_v = [x.clone() for x in buf_k], [x.clone() for x in buf_v]
    new_len = serving.append_accepted(got_k, got_v, torch.tensor(store_len, dtype=torch.int32, device=gpu), cq,
                                      path, plen, pack_k, pack_v, check=True)
    ref = OS.append_store([x.clone() for x in buf_k], [x.clone() for x in buf_v], pack_k, pack_v, store_len,
                          cu_q, keep, accepted, list(range(B)))
    assert new_len.cpu().tolist() == ref[2]
    for i, (a, b) in enumerate(zip(got_k + got_v, ref[0] + ref[1])):
        assert torch.equal(a, b), f"layer {i % L} ({'KV'[i // L]})"
    # request 1 past its capacity: flagged and skipped in every layer, the
    # other requests appended as before
    cap = buf_k[0].shape[2]
    sl = list(store_len)
    sl[1] = cap - 1
    print(f"case append-{L}-layers-overflow: store_len={sl}", flush=True)
    flag_k, flag_v = [x.clone() for x in buf_k], [x.clone() for x in buf_v]
    with pytest.raises(ValueError, match="inconsistent"):
        serving.append_accepted(flag_k, flag_v, torch.tensor(sl, dtype=torch.int32, device=gpu), cq, path, plen,
                                pack_k, pack_v, check=True)
    for i in range(2 * L):
        got, old, want = (flag_k + flag_v)[i], (buf_k + buf_v)[i], (got_k + got_v)[i]
        assert torch.equal(got[1], old[1]), f"layer {i % L}: the flagged request was written"
        for b in (0, 2, 3):
            assert torch.equal(got[b], want[b]), f"layer {i % L} request {b}"


def test_append_overflow_is_flagged(gpu):
    from cast_amd import serving
    buf_k, buf_v, pack_k, pack_v, store_len, cu_q, keep, accepted = _setup(gpu, seed=9, B=2)
    cap = buf_k[0].shape[2]
    path = torch.full((2, 128), -1, dtype=torch.int32, device=gpu)
    path[:, 0] = 0
    plen = torch.tensor([1, 1], dtype=torch.int32, device=gpu)
    print("case append-overflow", flush=True)
    with pytest.raises(ValueError, match="inconsistent"):
        serving.append_accepted(buf_k, buf_v, [cap - 1, 0], cu_q, path, plen, pack_k, pack_v, check=True)


@pytest.mark.parametrize("case", ["path", "shift-by-one", "identity", "permuted", "root-only", "empty-prefix",
                                  "fp32-d64", "old-layout"])
def test_gather_cache_matches_reference(gpu, case):
    # the batch-one compaction in place (rows overlap their sources) against index_select
    from transformers import DynamicCache
    from cast_amd.verify import cache_layers, gather_cache
    rng = np.random.default_rng(sum(map(ord, case)))
    dtype, D = (torch.float32, 64) if case == "fp32-d64" else (torch.bfloat16, 128)
    L, Hkv, n_pack = 5, 4, 40
    n_prefix = 0 if case == "empty-prefix" else 77
    g = torch.Generator(device=gpu).manual_seed(7)
    layers = [(torch.randn((1, Hkv, n_prefix + n_pack, D), generator=g, device=gpu).to(dtype),
               torch.randn((1, Hkv, n_prefix + n_pack, D), generator=g, device=gpu).to(dtype)) for _ in range(L)]
    if case == "shift-by-one":
        keep = [0] + list(range(2, 30))
    elif case == "identity":
        keep = list(range(0, 25))
    elif case == "permuted":
        keep = [0] + rng.permutation(np.arange(1, n_pack))[:20].tolist()
    elif case == "root-only":
        keep = [0]
    else:
        keep = [0] + sorted(rng.choice(np.arange(1, n_pack), size=12, replace=False).tolist())
    want = OS.gather_cache(layers, n_prefix, keep)
    if case == "old-layout":
        class _OldCache:
            pass
        cache = _OldCache()
        cache.key_cache = [k.clone() for k, _ in layers]
        cache.value_cache = [v.clone() for _, v in layers]
    else:
        cache = DynamicCache()
        for i, (k, v) in enumerate(layers):
            cache.update(k.clone(), v.clone(), i)
    print(f"case gather_cache {case} keep={len(keep)}", flush=True)
    gather_cache(cache, n_prefix, keep)
    n_layers, get, _ = cache_layers(cache)
    assert n_layers == L
    for i in range(L):
        k, v = get(i)
        assert k.shape[2] == n_prefix + len(keep)
        assert torch.equal(k, want[i][0]) and torch.equal(v, want[i][1]), f"layer {i}"
    if case not in ("old-layout",):
        assert cache.get_seq_length() == n_prefix + len(keep)


def test_gather_cache_rejects_bad_keep(gpu):
    from transformers import DynamicCache
    from cast_amd.verify import gather_cache
    cache = DynamicCache()
    cache.update(torch.zeros((1, 2, 20, 64), device=gpu), torch.zeros((1, 2, 20, 64), device=gpu), 0)
    for keep in ([1, 2], [0, 0], [0, 15]):
        with pytest.raises(ValueError):
            gather_cache(cache, 10, keep)


def test_append_from_hook_record_matches_explicit_packs(gpu):
    # the serving flow: the attention hook records each layer's pack K/V as
    # the forward runs, and append_accepted (pack lists from PACK_KV) uses
    # those checked addresses; the result is the explicit-list result bit for bit
    from cast_amd import serving
    buf_k, buf_v, pack_k, pack_v, store_len, cu_q, keep, accepted = _setup(gpu, seed=21)
    B, L = len(store_len), len(buf_k)
    path, plen = _path_tensors(keep, gpu)
    sl = torch.tensor(store_len, dtype=torch.int32, device=gpu)
    cq = torch.tensor(cu_q, dtype=torch.int32, device=gpu)
    print(f"case append-hook-record: B={B} L={L}", flush=True)
    want_k, want_v = [x.clone() for x in buf_k], [x.clone() for x in buf_v]
    n_want = serving.append_accepted(want_k, want_v, sl, cq, path, plen, pack_k, pack_v, check=True)
    got_k, got_v = [x.clone() for x in buf_k], [x.clone() for x in buf_v]
    serving.PACK_KV["k"], serving.PACK_KV["v"] = list(pack_k), list(pack_v)
    serving._PACK_REC.begin(L)
    for li in range(L):
        serving._PACK_REC.note(li, pack_k[li], pack_v[li])
    assert serving._PACK_REC.arrays_for(serving._store_layout(got_k, got_v), pack_k, pack_v) is not None
    n_got = serving.append_accepted(got_k, got_v, sl, cq, path, plen, check=True)
    torch.cuda.synchronize()
    assert torch.equal(n_got, n_want)
    for a, b in zip(got_k + got_v, want_k + want_v):
        assert torch.equal(a, b)
    # a record of other tensors is not used: the lists are checked in full
    serving._PACK_REC.begin(L)
    for li in range(L):
        serving._PACK_REC.note(li, pack_k[li][:], pack_v[li][:])
    assert serving._PACK_REC.arrays_for(serving._store_layout(got_k, got_v), pack_k, pack_v) is None
    bad = list(pack_k)
    bad[1] = pack_k[1].contiguous()           # other strides than layer 0
    serving.PACK_KV["k"] = bad
    with pytest.raises(ValueError, match="strides"):
        serving.append_accepted(got_k, got_v, sl, cq, path, plen)
