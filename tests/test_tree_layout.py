"""Host-side tree producers and packed layout vs the reference's own outputs.

Golden vectors in tests/golden/tree_fixtures.json were written by the
reference's cast_trees/tree.py (tests/golden/make_tree_fixtures.py); known
answers come from the reference README/quickstart (README.md:82-85,
tests/test_smoke.py:26).
"""
import itertools
import json
from pathlib import Path

import numpy as np
import pytest

from cast_amd import tree as T

FIX = json.loads((Path(__file__).parent / "golden" / "tree_fixtures.json").read_text())


def _scores(case):
    name = case["name"]
    if name == "quickstart-seed0":
        return np.random.default_rng(0).normal(scale=5, size=(15, 64))
    if name.startswith("scaled3-seed"):
        return np.random.default_rng(int(name[-1])).normal(size=(15, 100)) * 3
    seed = int(name.split("seed")[1].split("-")[0])
    scale = float(name.split("scale")[1])
    return np.random.default_rng(seed).normal(scale=scale, size=(15, 151936))


def _triples(nodes):
    return [[n.token, n.depth, n.parent] for n in nodes]


@pytest.mark.parametrize("case", FIX["cases"], ids=lambda c: c["name"])
def test_block_topk_and_build_tree_match_reference(case):
    idx, lp = T.block_topk(_scores(case), case["k"])
    assert idx.tolist() == case["top_idx"]
    assert np.array_equal(lp, np.asarray(case["top_lp"]))
    for n, want in case["trees"].items():
        got = T.build_tree(idx, lp, int(n))
        assert _triples(got) == [w[:3] for w in want]
        assert [g.score for g in got] == [w[3] for w in want]
    if "chain15" in case:
        got = T.build_chain(idx, lp, 15)
        assert _triples(got) == [w[:3] for w in case["chain15"]]
        assert np.allclose([g.score for g in got], [w[3] for w in case["chain15"]], rtol=0, atol=1e-12)


def test_quickstart_known_answers():
    # README.md:82-85: chain 1.01, N=15 1.78, N=127 3.54 on the seed-0 15x64 block
    idx, lp = T.block_topk(np.random.default_rng(0).normal(scale=5, size=(15, 64)))
    assert f"{T.expected_accepted_length(T.build_chain(idx, lp, 15)):.2f}" == "1.01"
    assert f"{T.expected_accepted_length(T.build_tree(idx, lp, 15)):.2f}" == "1.78"
    assert f"{T.expected_accepted_length(T.build_tree(idx, lp, 127)):.2f}" == "3.54"


def test_best_first_is_top_n_by_brute_force():
    # tests/test_tree.py:23-30: the 3-level universe with rank cap 4
    idx, lp = T.block_topk(np.random.default_rng(0).normal(size=(15, 100)) * 3, 8)
    small = T.build_tree(idx[:3], lp[:3], budget=20, k=4)
    scores = [sum(float(lp[j, r]) for j, r in enumerate(ranks))
              for d in range(1, 4) for ranks in itertools.product(range(4), repeat=d)]
    assert np.allclose(sorted(n.score for n in small), sorted(scores, reverse=True)[:20][::-1], atol=1e-9)


def test_tree_is_prefix_closed():
    idx, lp = T.block_topk(np.random.default_rng(3).normal(size=(15, 100)) * 3, 8)
    nodes = T.build_tree(idx, lp, 127)
    assert len(nodes) == 127
    par = np.array([n.parent for n in nodes])
    depth = np.array([n.depth for n in nodes])
    score = np.array([n.score for n in nodes])
    assert (par < np.arange(len(nodes))).all()                 # every parent listed first
    top, kid = par < 0, np.nonzero(par >= 0)[0]
    assert (depth[top] == 1).all()
    assert (depth[kid] == depth[par[kid]] + 1).all()           # one level below its parent
    assert (score[kid] <= score[par[kid]]).all()               # log-probs never add score


def test_select_global_topk_matches_reference():
    forest = []
    for s in range(8):
        idx, lp = T.block_topk(np.random.default_rng(s).normal(size=(15, 100)) * 3, 8)
        forest.append(T.build_tree(idx, lp, 48))
    split = T.select_global_topk(forest, 64)
    want = FIX["global_topk"]["split"]
    assert [_triples(t) for t in split] == [[w[:3] for w in t] for t in want]
    assert sum(map(len, split)) == 64


def test_ancestor_matrix_is_the_chain_walk():
    # the property of tests/test_tree.py:58-67, checked by walking every
    # packed row's parent chain at once (one step up per pass), independent
    # of the row-inheriting recurrence the product uses
    idx, lp = T.block_topk(np.random.default_rng(0).normal(size=(15, 100)) * 3, 8)
    nodes = T.build_tree(idx, lp, budget=31)
    vis = T.ancestor_matrix(nodes)
    up = np.array([-1] + [n.parent + 1 for n in nodes])        # packed parent, -1 above the root
    want = np.eye(len(up), dtype=bool)
    at = np.arange(len(up))
    while (at >= 0).any():
        at = np.where(at >= 0, up[np.maximum(at, 0)], -1)
        rows = np.nonzero(at >= 0)[0]
        want[rows, at[rows]] = True
    assert want[1:, 0].all() and not want[0, 1:].any()          # the root is everyone's ancestor, alone on row 0
    assert np.array_equal(vis, want)


def test_pack_trees_layout_and_errors():
    idx, lp = T.block_topk(np.random.default_rng(0).normal(scale=5, size=(15, 64)))
    trees = [T.build_tree(idx, lp, n) for n in (15, 3, 0)]
    pk = T.pack_trees(trees, roots=[7, 8, 9])
    assert pk.pack_len.tolist() == [16, 4, 1]
    assert pk.cu_q.tolist() == [0, 16, 20, 21]
    assert pk.parent[[0, 16, 20]].tolist() == [-1, -1, -1]
    assert pk.token[[0, 16, 20]].tolist() == [7, 8, 9]
    for i, nd in enumerate(trees[0]):
        assert pk.parent[i + 1] == nd.parent + 1 and pk.token[i + 1] == nd.token
    with pytest.raises(ValueError):
        T.pack_trees([T.build_tree(idx, lp, 128)])
    bad = [T.TreeNode(1, 1, -1, 0.0), T.TreeNode(2, 2, 1, 0.0)]
    with pytest.raises(ValueError):
        T.pack_trees([bad])


@pytest.mark.parametrize("budget", [0, 15, 63, 64, 127])
def test_host_ancestor_words_are_the_chain_walk_words(budget):
    # the words the batch-one mask carries for the "cast_tree" kernel equal
    # the oracle's chain walk (word 0 is the reference's int64 recurrence)
    from cast_amd.verify import ancestor_words
    from oracle import bitmask as OB
    idx, lp = T.block_topk(np.random.default_rng(budget).normal(scale=2, size=(15, 200)), 8)
    nodes = T.build_tree(idx, lp, budget=budget)
    pk = T.pack_trees([nodes])
    got = ancestor_words(T.ancestor_matrix(nodes))
    assert got.dtype == np.int64 and got.shape == (budget + 1, 2)
    assert np.array_equal(got, OB.chain_walk_words(pk.parent, pk.cu_q).view(np.int64))
    with pytest.raises(ValueError):
        ancestor_words(np.ones((129, 129), dtype=bool))
