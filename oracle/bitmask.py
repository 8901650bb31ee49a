"""Ancestor bitmask oracle (CPU, numpy).  Test infrastructure only.

Bit j of row r's mask is set iff pack-local index j lies on the chain from
row r up to its pack's root, inclusive (cast_trees/tree_attn.py:73-75 reads
bit j as "key j visible").  Word w holds bits 64w..64w+63, so word 0 equals
the reference's single int64 word (cast_trees/serving.py:213-222, built by
the recurrence ``bits[i+1] = bits[parent+1] | 1 << (i+1)``) whenever P <= 64.
"""
import numpy as np

WORDS = 2


def chain_walk_words(parent, cu_q, words=WORDS):
    """uint64 [total_q, words] by walking every row's parent chain.

    Same walk as tests/test_tree_attn.py:22-27, on pack-local parents.
    """
    parent = np.asarray(parent, dtype=np.int64)
    cu_q = np.asarray(cu_q, dtype=np.int64)
    out = np.zeros((parent.shape[0], words), dtype=np.uint64)
    for b in range(cu_q.shape[0] - 1):
        base, end = int(cu_q[b]), int(cu_q[b + 1])
        for i in range(end - base):
            j, steps = i, 0
            while j != -1:
                out[base + i, j >> 6] |= np.uint64(1) << np.uint64(j & 63)
                j = int(parent[base + j])
                steps += 1
                if steps > end - base:
                    raise ValueError(f"pack {b}: parent chain of row {i} does not reach the root")
    return out


def reference_int64_words(trees):
    """The reference's int64 per-row word for P <= 64 (serving.py:213-222):
    root = 1, node i = bits of its parent's row | 1 << (i + 1)."""
    bits = []
    for nodes in trees:
        base = len(bits)
        bits.append(1)
        for i, nd in enumerate(nodes):
            bits.append(bits[base + nd.parent + 1] | (1 << (i + 1)))
    if any(b >= 1 << 64 for b in bits):
        raise ValueError("more than 64 pack tokens do not fit one word")
    return np.array(bits, dtype=np.uint64).view(np.int64)


def words_to_bool(words, P):
    """Expand one row's words into a bool vector over pack indices 0..P-1."""
    j = np.arange(P)
    return ((words[j >> 6] >> (j & 63).astype(np.uint64)) & np.uint64(1)).astype(bool)
