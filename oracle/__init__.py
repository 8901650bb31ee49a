"""CPU oracle for the tree-verification path.  TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this package, and only to check results against (or, for the
baseline, as the thing timed on host cores).  The product path in ``cast_amd`` never
imports it and fails loudly when its HIP library is missing.

Contents, each restating the reference algorithm it cites:
  bitmask.py   ancestor words by explicit chain walk
               (cast_trees/serving.py:213-222, tests/test_tree_attn.py:22-27,
               cast_trees/tree.py:85-93)
  attn.py      dense fp32 masked softmax attention + natural-log LSE
               (tests/test_tree_attn.py:40-59, cast_trees/tree_attn.py:30,45,
               62,73-75,89, cast_trees/verify.py:15-25)
  walk.py      greedy accepted-path walk
               (cast_trees/decode.py:13-17, 85-103)
  draft.py     drafter top-k over the log-softmax and the best-first tree
               build (cast_trees/tree.py:20-49, cast_trees/verify.py:8-12)
  store.py     accepted-path KV append and batch-one cache compaction, row
               by row (cast_trees/serving.py:264-289, cast_trees/verify.py:
               48-60)

Pinning (what fixes each function independently of its own formula):
  bitmask  - reference int64 recurrence of serving.py:218-222 (a different
             algorithm), the ancestor_matrix invariant of tests/test_tree.py:
             58-67, closed forms for chains (bit j set for j <= i) and stars.
  attn     - P=1 and chain trees reduce to torch SDPA (decode / causal);
             S=0 star trees reduce to per-row closed forms; masked keys with
             poisoned values must not leak; LSE matches torch.logsumexp.
  draft    - the reference module's own outputs on seeded inputs
             (tests/golden/tree_fixtures.json: top-k ids and log-probs,
             trees of 15..127 nodes), exact; prefix-closure and descending
             scores along every root path.
  store    - plain indexing checked bit for bit; tests/test_oracle.py pins
             it on hand-built stores (untouched slots, growth zero-filled,
             compaction order) and against index_select for gather_cache.
  walk     - replay-style accepted length (cast_trees/replay.py:20-32, a
             rank-tuple path-set formulation), planted-path workloads, and
             brute force over every root path on tiny trees.
No function of this oracle is left unpinned.
"""
