"""Write tree_fixtures.json from the reference tree producers.

The reference's tests pin its tree builder only through score multisets and
expected accepted lengths (tests/test_tree.py:23-30, tests/test_smoke.py:26),
not the node order and parent indices that the packed verify layout depends
on.  This script imports cast_trees/tree.py (numpy only) from the reference
checkout, runs it on seeded block scores, and stores the resulting
(token, depth, parent, score) lists as data.  Run it in a checkout that has
the reference at /root/reference; the JSON it writes is committed and the
tests read only that.
"""
import json
import sys
from pathlib import Path

import numpy as np

sys.path.insert(0, "/root/reference")
from cast_trees import tree as ref  # noqa: E402

OUT = Path(__file__).with_name("tree_fixtures.json")


def nodes_of(nodes):
    return [[int(n.token), int(n.depth), int(n.parent), float(n.score)] for n in nodes]


def main():
    cases = []
    # the 15x64 N(0,5) seed-0 block of the quickstart (examples/quickstart.py:12)
    scores = np.random.default_rng(0).normal(scale=5, size=(15, 64))
    idx, lp = ref.block_topk(scores)
    cases.append(dict(name="quickstart-seed0", recipe="default_rng(0).normal(scale=5,size=(15,64))",
                      k=8, top_idx=idx.tolist(), top_lp=lp.tolist(),
                      trees={str(n): nodes_of(ref.build_tree(idx, lp, n)) for n in (15, 31, 63, 127)},
                      chain15=nodes_of(ref.build_chain(idx, lp, 15))))
    # tests/test_tree.py:12-13 recipe: normal(size=(15,100)) * 3
    for seed in range(4):
        scores = np.random.default_rng(seed).normal(size=(15, 100)) * 3
        idx, lp = ref.block_topk(scores, 8)
        cases.append(dict(name=f"scaled3-seed{seed}", recipe=f"default_rng({seed}).normal(size=(15,100))*3",
                          k=8, top_idx=idx.tolist(), top_lp=lp.tolist(),
                          trees={str(n): nodes_of(ref.build_tree(idx, lp, n)) for n in (31, 63, 127)}))
    # full Qwen3 vocabulary, N(0,5) and N(0,10)/N(0,2) blocks (top-k only stored)
    for seed, scale in ((0, 5.0), (1, 10.0), (2, 2.0)):
        scores = np.random.default_rng(seed).normal(scale=scale, size=(15, 151936))
        idx, lp = ref.block_topk(scores, 8)
        cases.append(dict(name=f"vocab151936-seed{seed}-scale{scale:g}",
                          recipe=f"default_rng({seed}).normal(scale={scale:g},size=(15,151936))",
                          k=8, top_idx=idx.tolist(), top_lp=lp.tolist(),
                          trees={str(n): nodes_of(ref.build_tree(idx, lp, n)) for n in (15, 31, 63, 127)}))
    # shared-budget allocation (tests/test_tree.py:47-55 recipe)
    forest = []
    for s in range(8):
        idx, lp = ref.block_topk(np.random.default_rng(s).normal(size=(15, 100)) * 3, 8)
        forest.append(ref.build_tree(idx, lp, 48))
    split = ref.select_global_topk(forest, 64)
    alloc = dict(recipe="8 trees, default_rng(s).normal(size=(15,100))*3, budget 48, total 64",
                 split=[nodes_of(t) for t in split])
    OUT.write_text(json.dumps(dict(cases=cases, global_topk=alloc), indent=None))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
