"""Drafter top-k and best-first tree build on the GPU.

Bars: top-k token ids identical to the oracle (descending log-probability,
equal values by increasing index), log-probs within 2e-5; trees identical
node for node (token, depth, parent, and the double-precision score) to the
reference module's own trees (tests/golden/tree_fixtures.json) from the same
float64 log-probs, and to the oracle's heap from float32 log-probs.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import draft as OD

pytestmark = pytest.mark.gpu

FIX = json.loads((Path(__file__).parent / "golden" / "tree_fixtures.json").read_text())


@pytest.mark.parametrize("dtype,k", [(torch.float32, 8), (torch.bfloat16, 8), (torch.float32, 16), (torch.float16, 8),
                                     (torch.float16, 16)])
def test_topk_marginals_match_oracle(gpu, dtype, k):
    from cast_amd.draft import topk_marginals
    rng = np.random.default_rng(k)
    x = rng.normal(scale=5.0, size=(15, 151936)).astype(np.float32)
    x[3, [10, 99, 151935]] = x[3].max() + 2.0          # ties at the top of one row
    xd = torch.from_numpy(x).to(gpu).to(dtype)
    want_i, want_lp = OD.topk_log_softmax(xd.float().cpu().numpy(), k)
    for splits in (0, 1, 3, 4):   # one workgroup per row, and rows split across workgroups
        print(f"case topk {dtype} k={k} splits={splits}", flush=True)
        idx, lp = topk_marginals(xd, k, on_device=True, splits=splits)
        torch.cuda.synchronize()
        assert idx.cpu().numpy().tolist() == want_i.tolist(), f"splits={splits}"
        assert np.abs(lp.cpu().numpy() - want_lp).max() <= 2e-5, f"splits={splits}"
        if dtype == torch.float32:
            assert idx[3, :3].cpu().tolist() == [10, 99, 151935]
    # the drop-in returns host tensors like the reference
    hi, hl = topk_marginals(xd, k)
    assert hi.device.type == "cpu" and torch.equal(hi, idx.cpu())


@pytest.mark.parametrize("dtype,V,pad", [(torch.float32, 151936, 0), (torch.bfloat16, 151936, 0),
                                         (torch.bfloat16, 1000, 3), (torch.float32, 50000, 1),
                                         (torch.float16, 151936, 0), (torch.float16, 1000, 3)])
def test_topk_marginals_edge_rows(gpu, dtype, V, pad):
    # all-equal, increasing, decreasing, mostly -inf, integer-tied, NaN and +inf rows;
    # small vocabularies and unaligned row strides take the scalar path
    from cast_amd.draft import topk_marginals
    rng = np.random.default_rng(V + pad)
    x = np.empty((8, V + pad), dtype=np.float32)
    x[0] = 0.0
    x[1] = np.arange(V + pad) / 7.0
    x[2] = -np.arange(V + pad) / 7.0
    x[3] = -np.inf
    x[3, rng.integers(0, V, size=5)] = rng.normal(size=5)
    x[4] = np.round(rng.normal(scale=3.0, size=V + pad))
    x[5] = rng.normal(size=V + pad)
    x[6] = rng.normal(size=V + pad)     # a NaN never ranks and makes the row's log-probs NaN
    x[6, V // 3] = np.nan
    x[7] = rng.normal(size=V + pad)     # +inf ranks first; log-probs NaN as in log_softmax
    x[7, V // 2] = np.inf
    xd = torch.from_numpy(x).to(gpu).to(dtype)[:, :V]
    print(f"case topk-edge {dtype} V={V} ld={xd.stride(0)}", flush=True)
    for k in (1, 8, 16):
        want_i, want_lp = OD.topk_log_softmax(xd.float().cpu().numpy(), k)
        for splits in (0, 1, 4):
            idx, lp = topk_marginals(xd, k, on_device=True, splits=splits)
            assert idx.cpu().numpy().tolist() == want_i.tolist(), f"k={k} splits={splits}"
            got = lp.cpu().numpy()
            assert np.array_equal(np.isinf(got), np.isinf(want_lp))
            assert np.array_equal(np.isnan(got), np.isnan(want_lp))
            fin = np.isfinite(want_lp)
            assert np.abs(got[fin] - want_lp[fin]).max() <= 2e-5, f"k={k} splits={splits}"


def test_build_trees_match_reference_fixtures(gpu):
    from cast_amd.draft import build_trees
    cases = [c for c in FIX["cases"] if "127" in c["trees"]]
    budgets = [int(n) for n in ("15", "31", "63", "127")]
    print(f"case build-trees: {len(cases)} fixture blocks x budgets {budgets}", flush=True)
    ti = torch.tensor([c["top_idx"] for c in cases for _ in budgets], dtype=torch.int64, device=gpu)
    tl = torch.tensor([c["top_lp"] for c in cases for _ in budgets], dtype=torch.float64, device=gpu)
    bud = torch.tensor([n for _ in cases for n in budgets], dtype=torch.int32, device=gpu)
    token, depth, parent, score, n_nodes = build_trees(ti, tl, bud, check=True)
    token, depth, parent, score, n_nodes = (t.cpu() for t in (token, depth, parent, score, n_nodes))
    row = 0
    checked = 0
    for c in cases:
        for n in budgets:
            want = c["trees"].get(str(n))
            m = int(n_nodes[row])
            if want is not None:
                got = [[int(token[row, i]), int(depth[row, i]), int(parent[row, i]), float(score[row, i])]
                       for i in range(m)]
                assert got == want, f"{c['name']} budget {n}"
                checked += 1
            row += 1
    assert checked >= 20


def test_device_draft_pipeline_matches_oracle_heap(gpu):
    # topk on the device, then the tree on the device, vs the oracle's heap on
    # the same float32 log-probs; and the TreeNode drop-in
    from cast_amd.draft import build_tree_device, build_trees, topk_marginals
    rng = np.random.default_rng(3)
    B, L, V = 6, 15, 151936
    x = torch.from_numpy(rng.normal(scale=4.0, size=(B * L, V)).astype(np.float32)).to(gpu).to(torch.bfloat16)
    print(f"case draft-pipeline B={B}", flush=True)
    idx, lp = topk_marginals(x, 8, on_device=True)
    budgets = [15, 48, 127, 1, 63, 100]
    token, depth, parent, score, n_nodes = build_trees(idx.view(B, L, 8), lp.view(B, L, 8),
                                                       torch.tensor(budgets, device=gpu))
    idx_h, lp_h = idx.cpu().numpy().reshape(B, L, 8), lp.cpu().numpy().reshape(B, L, 8)
    for b in range(B):
        want = OD.build_tree(idx_h[b], lp_h[b], budgets[b])
        m = int(n_nodes[b])
        got = list(zip(token[b, :m].tolist(), depth[b, :m].tolist(), parent[b, :m].tolist(),
                       score[b, :m].tolist()))
        assert got == [(t, d, p, s) for t, d, p, s in want]
    nodes = build_tree_device(idx_h[2], lp_h[2], 127)
    assert [(n.token, n.depth, n.parent, n.score) for n in nodes] == OD.build_tree(idx_h[2], lp_h[2], 127)


@pytest.mark.parametrize("case", ["unsorted", "ties-sorted", "ties-unsorted", "one-position", "neg-inf-tails",
                                  "deep-k2", "k16-long"])
def test_build_trees_paths_match_oracle_heap(gpu, case):
    # sorted positions take the frontier search, others the full pool scan;
    # both must pop exactly the oracle heap's order, ties and -inf included
    from cast_amd.draft import build_trees
    rng = np.random.default_rng(sum(map(ord, case)))
    L, k, B = {"one-position": (1, 4, 3), "deep-k2": (255, 2, 3), "k16-long": (40, 16, 3)}.get(case, (15, 8, 4))
    lp = -np.abs(rng.normal(scale=2.0, size=(B, L, k)))
    if case.startswith("ties"):
        lp = np.round(lp * 2) / 2                          # many equal scores and sums
    lp = -np.sort(-lp, axis=-1)                            # non-increasing per position
    if case == "neg-inf-tails":
        lp[:, :, 5:] = -np.inf
    if case.endswith("unsorted"):
        lp = np.take_along_axis(lp, rng.permuted(np.tile(np.arange(k), (B, L, 1)), axis=-1), axis=-1)
    lp = lp.astype(np.float32)
    idx = rng.integers(0, 151936, size=(B, L, k))
    budgets = [127, 40, 1, 0][:B]
    print(f"case build-trees {case} L={L} k={k}", flush=True)
    token, depth, parent, score, n_nodes = build_trees(torch.from_numpy(idx).to(gpu), torch.from_numpy(lp).to(gpu),
                                                       torch.tensor(budgets, device=gpu), check=True)
    for b in range(B):
        want = OD.build_tree(idx[b], lp[b], budgets[b], k)
        m = int(n_nodes[b])
        got = list(zip(token[b, :m].tolist(), depth[b, :m].tolist(), parent[b, :m].tolist(),
                       score[b, :m].tolist()))
        assert got == [(int(t), d, p, s) for t, d, p, s in want], f"{case} request {b}"
