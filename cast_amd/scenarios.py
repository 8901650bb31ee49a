"""Seeded synthetic verify workloads at the shapes the benchmarks quote.

Every workload is one ragged verify pass: B requests, each with a cached
prefix of S_b tokens and a packed tree of P_b = 1 + nodes tokens.  Trees come
from drafter-like block scores (L=15 future positions) through ``block_topk``
and ``build_tree``; attention inputs are Gaussian.  Seeds are fixed: tree
scores use ``numpy.random.default_rng(seed)``, tensors use a CPU
``torch.Generator`` seeded the same way (or a device generator for the large
timing-only inputs).

K/V follow the ragged layout of cast_trees/serving.py:223-238: request b owns
rows ``[cu_kv[b], cu_kv[b+1])`` holding concat(prefix, pack).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from .tree import PackedTrees, block_topk, build_chain, build_tree, pack_trees

QWEN3_8B = dict(Hq=32, Hkv=8, D=128, vocab=151936)
LLAMA31_8B = dict(Hq=32, Hkv=8, D=128, vocab=128256)
HEADS_D256 = dict(Hq=16, Hkv=8, D=256, vocab=151936)   # 16 query / 8 KV heads of head_dim 256
DRAFT_LEN = 15          # future positions scored by one drafter pass


def torch_dtype(name):
    """The torch dtype of a workload dtype name ("bf16", "fp16" or "fp32")."""
    import torch
    return {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[name]


@dataclass
class Workload:
    name: str
    trees: list                 # per request: list of TreeNode
    packed: PackedTrees
    prefix_len: np.ndarray      # int32 [B]
    Hq: int
    Hkv: int
    D: int
    dtype: str                  # "bf16" | "fp16" | "fp32"
    vocab: int
    qkv_scale: float = 1.0
    seed: int = 0
    meta: dict = field(default_factory=dict)

    @property
    def B(self):
        return self.packed.batch

    @property
    def pack_len(self):
        return self.packed.pack_len

    @property
    def cu_q(self):
        return self.packed.cu_q

    @property
    def cu_kv(self):
        cu = np.zeros(self.B + 1, dtype=np.int32)
        np.cumsum(self.prefix_len.astype(np.int64) + self.pack_len, out=cu[1:])
        return cu

    @property
    def total_q(self):
        return self.packed.total_q

    @property
    def total_kv(self):
        return int(self.cu_kv[-1])

    def algorithmic_bytes(self, elem=None, mask_bytes=16, lse=True):
        """HBM bytes one attention call must move at minimum.

        K and V once per KV head, Q read and O written once, LSE written,
        the ancestor words read once.
        """
        e = elem or (4 if self.dtype == "fp32" else 2)
        S = self.prefix_len.astype(np.int64)
        P = self.pack_len.astype(np.int64)
        kv = int(((S + P) * self.Hkv * self.D * e * 2).sum())
        qo = int((P * self.Hq * self.D * e * 2).sum())
        extra = int((P * self.Hq * 4).sum()) if lse else 0
        return kv + qo + extra + int(P.sum()) * mask_bytes

    def algorithmic_flops(self):
        """QK^T and PV over every (query row, visible-or-not key) pair.

        The tree block is counted dense (P_b x P_b), as a kernel computes it.
        """
        S = self.prefix_len.astype(np.int64)
        P = self.pack_len.astype(np.int64)
        return int((4 * P * (S + P) * self.Hq * self.D).sum())

    # ---- tensors -----------------------------------------------------
    def qkv(self, device="cpu", generator_device="cpu"):
        """Seeded q [total_q,Hq,D], k/v [total_kv,Hkv,D] in the workload dtype."""
        import torch
        dt = torch_dtype(self.dtype)
        g = torch.Generator(device=generator_device).manual_seed(self.seed)

        def draw(*shape):
            x = torch.randn(*shape, generator=g, device=generator_device, dtype=torch.float32)
            if self.qkv_scale != 1.0:
                x.mul_(self.qkv_scale)
            return x.to(dt).to(device)

        q = draw(self.total_q, self.Hq, self.D)
        k = draw(self.total_kv, self.Hkv, self.D)
        v = draw(self.total_kv, self.Hkv, self.D)
        return q, k, v

    def meta_tensors(self, device="cpu"):
        import torch
        i32 = lambda a: torch.as_tensor(np.ascontiguousarray(a, dtype=np.int32), device=device)
        return dict(cu_q=i32(self.cu_q), cu_kv=i32(self.cu_kv), prefix_len=i32(self.prefix_len),
                    pack_len=i32(self.pack_len), parent=i32(self.packed.parent))


def _tree_from_scores(rng, P, scale, chain=False, vocab=151936):
    scores = rng.normal(scale=scale, size=(DRAFT_LEN, vocab))
    idx, lp = block_topk(scores, 8)
    if chain:
        return build_chain(idx, lp, min(P - 1, DRAFT_LEN))
    return build_tree(idx, lp, P - 1)


def _make(name, trees, prefix, shape, dtype, seed, qkv_scale, **meta):
    packed = pack_trees(trees, roots=[int(n[0].token) if n else 0 for n in trees])
    return Workload(name=name, trees=trees, packed=packed,
                    prefix_len=np.asarray(prefix, dtype=np.int32), Hq=shape["Hq"], Hkv=shape["Hkv"],
                    D=shape["D"], dtype=dtype, vocab=shape["vocab"], qkv_scale=qkv_scale, seed=seed,
                    meta=meta)


def cpu_plumbing(seed=0):
    """15x64 block of N(0,5) scores (seed 0), N=15 tree; 1 request, 128-token
    prefix, 4/4 heads, head_dim 64, fp32."""
    idx, lp = block_topk(np.random.default_rng(seed).normal(scale=5, size=(DRAFT_LEN, 64)))
    trees = [build_tree(idx, lp, 15)]
    return _make("cpu-plumbing", trees, [128], dict(Hq=4, Hkv=4, D=64, vocab=64), "fp32", seed, 1.0)


def qwen3_single(seed=0, prefix=2048, pack=16):
    """Qwen3-8B heads, 1 request, prefix 2048, P=16 from a 15x151936 N(0,5) block."""
    rng = np.random.default_rng(seed)
    trees = [_tree_from_scores(rng, pack, 5.0)]
    return _make("qwen3-8b-single", trees, [prefix], QWEN3_8B, "bf16", seed, 1 / math.sqrt(128))


def qwen3_ragged(seed=0, B=8, lo=1024, hi=8192, packs=(32, 64, 128), vocab=None):
    """Qwen3-8B heads, ragged batch: prefixes U[lo,hi], P uniform over ``packs``.

    ``vocab`` shrinks the drafter vocabulary (for small walk tests only).
    """
    rng = np.random.default_rng(seed)
    prefix = rng.integers(lo, hi + 1, size=B)
    P = rng.choice(np.asarray(packs), size=B)
    V = vocab or QWEN3_8B["vocab"]
    trees = [_tree_from_scores(rng, int(p), 5.0, vocab=V) for p in P]
    return _make("qwen3-8b-ragged", trees, prefix, dict(QWEN3_8B, vocab=V), "bf16", seed,
                 1 / math.sqrt(128))


def qwen3_headline(seed=0, B=8, prefix=8192, pack=128):
    """Qwen3-8B heads, B=8 requests, each prefix 8192 and a P=128 tree."""
    rng = np.random.default_rng(seed)
    trees = [_tree_from_scores(rng, pack, 5.0) for _ in range(B)]
    return _make("qwen3-8b-b8-ctx8k-p128", trees, [prefix] * B, QWEN3_8B, "bf16", seed,
                 1 / math.sqrt(128))


def llama_long(seed=0, prefix=32768, pack=128):
    """Llama-3.1-8B heads, batch 1, prefix 32k, P=128 (split-K path)."""
    rng = np.random.default_rng(seed)
    trees = [_tree_from_scores(rng, pack, 5.0, vocab=LLAMA31_8B["vocab"])]
    return _make("llama31-8b-ctx32k-p128", trees, [prefix], LLAMA31_8B, "bf16", seed,
                 1 / math.sqrt(128))


def head_dim_256(seed=0, B=8, prefix=8192, pack=128):
    """The headline batch with 16 query / 8 KV heads of head_dim 256 (the same
    FLOPs per call), bf16: the one-wave-per-SIMD MFMA instance."""
    rng = np.random.default_rng(seed)
    trees = [_tree_from_scores(rng, pack, 5.0) for _ in range(B)]
    return _make("d256-b8-ctx8k-p128", trees, [prefix] * B, HEADS_D256, "bf16", seed, 1 / math.sqrt(256))


def stress_mixed(seed=0, B=32, lo=256, hi=4096, pack=128):
    """B=32, prefixes U[256,4k], P=128 each; even requests use deep/narrow
    trees (scores N(0,10)), odd ones wide trees (scores N(0,2))."""
    rng = np.random.default_rng(seed)
    prefix = rng.integers(lo, hi + 1, size=B)
    trees = [_tree_from_scores(rng, pack, 10.0 if b % 2 == 0 else 2.0) for b in range(B)]
    return _make("qwen3-8b-stress-b32", trees, prefix, QWEN3_8B, "bf16", seed, 1 / math.sqrt(128))


def stress_trees_only(seed=0):
    """The stress batch's 32 trees (4096 packed tree tokens) with no prefix:
    every key tile is a tree-tree tile, so the masked block runs alone."""
    wl = stress_mixed(seed)
    return _make("qwen3-8b-stress-b32-trees", wl.trees, [0] * wl.B, QWEN3_8B, "bf16", seed, 1 / math.sqrt(128))


def random_parent_batch(seed=0, B=8, Hq=32, Hkv=8, D=128, s_lo=200, s_hi=400, p_lo=2, p_hi=64,
                        dtype="fp32", qkv_scale=1.0):
    """Random-parent packs, ``parent[i] ~ U[0, i)``, like the kernel test of
    cast_trees (tests/test_tree_attn.py:11-37); P_b ~ U[p_lo, p_hi)."""
    from .tree import TreeNode
    rng = np.random.default_rng(seed)
    trees, prefix = [], []
    for _ in range(B):
        S = int(rng.integers(s_lo, s_hi)) if s_hi > s_lo else s_lo
        P = int(rng.integers(p_lo, p_hi)) if p_hi > p_lo else p_lo
        par = [-1] + [int(rng.integers(0, i)) for i in range(1, P)]
        nodes = []
        depth = [0] * P
        for i in range(1, P):
            depth[i] = depth[par[i]] + 1
            nodes.append(TreeNode(int(rng.integers(0, 1000)), depth[i], par[i] - 1, 0.0))
        trees.append(nodes)
        prefix.append(S)
    return _make("random-parent", trees, prefix, dict(Hq=Hq, Hkv=Hkv, D=D, vocab=1000), dtype, seed,
                 qkv_scale)


def reference_test_batch(seed=0, B=8, Hq=32, Hkv=8, D=128):
    """The exact inputs of the reference's own kernel test
    (cast_trees tests/test_tree_attn.py:11-37): one CPU ``torch.Generator``
    seeded with ``seed`` draws, request by request, S ~ U[200, 400),
    P ~ U[2, 64), the parents ``parent[i] ~ U[0, i)`` one at a time, then
    q [P, Hq, D], k [S+P, Hkv, D] and v [S+P, Hkv, D] from N(0, 1), in that
    order.  Returns (workload, q, k, v) with fp32 tensors on the CPU; the
    workload holds the same trees and prefixes (its own ``qkv`` draws other
    tensors).
    """
    import torch
    from .tree import TreeNode
    g = torch.Generator().manual_seed(seed)
    draw_int = lambda lo, hi: int(torch.randint(lo, hi, (1,), generator=g))
    trees, prefix, qs, ks, vs = [], [], [], [], []
    for _ in range(B):
        S = draw_int(200, 400)
        P = draw_int(2, 64)
        par = [-1] + [draw_int(0, i) for i in range(1, P)]
        qs.append(torch.randn(P, Hq, D, generator=g))
        ks.append(torch.randn(S + P, Hkv, D, generator=g))
        vs.append(torch.randn(S + P, Hkv, D, generator=g))
        depth = [0] * P
        nodes = []
        for i in range(1, P):
            depth[i] = depth[par[i]] + 1
            nodes.append(TreeNode(0, depth[i], par[i] - 1, 0.0))
        trees.append(nodes)
        prefix.append(S)
    wl = _make("reference-kernel-test", trees, prefix, dict(Hq=Hq, Hkv=Hkv, D=D, vocab=1), "fp32", seed, 1.0)
    return wl, torch.cat(qs), torch.cat(ks), torch.cat(vs)


CONFIGS = {
    "cpu-plumbing": cpu_plumbing,
    "qwen3-8b-single": qwen3_single,
    "qwen3-8b-ragged": qwen3_ragged,
    "qwen3-8b-b8-ctx8k-p128": qwen3_headline,
    "llama31-8b-ctx32k-p128": llama_long,
    "qwen3-8b-stress-b32": stress_mixed,
    "qwen3-8b-stress-b32-trees": stress_trees_only,
    "d256-b8-ctx8k-p128": head_dim_256,
}


def planted_logits(workload, vocab=None, seed=0, accept_p=0.8, device="cpu", dtype=None,
                   generator_device="cpu"):
    """Verify logits [total_q, V] whose greedy walk accepts a planted path.

    Every row is Gaussian noise.  Per request a path is drawn from the root:
    at each visited node, with probability ``accept_p`` one child is chosen
    and its token is made the row's unique maximum (value 16); otherwise a
    token that no child carries is planted as the bonus.  Rows off the path
    keep their noise, so their argmax comes from ties among bf16 noise values
    (first index wins).  Returns (logits, planted_paths) with planted paths as
    lists of node indices.
    """
    import torch
    V = vocab or workload.vocab
    if int(workload.packed.token.max(initial=0)) >= V:
        raise ValueError("tree tokens must be smaller than the logits vocabulary")
    dt = dtype or torch_dtype(workload.dtype)
    rng = np.random.default_rng(seed + 7919)
    g = torch.Generator(device=generator_device).manual_seed(seed + 104729)
    logits = torch.randn(workload.total_q, V, generator=g, device=generator_device,
                         dtype=torch.float32).to(dt)
    paths = []
    pk = workload.packed
    for b, nodes in enumerate(workload.trees):
        base = int(pk.cu_q[b])
        kids = {i: [] for i in range(-1, len(nodes))}
        for i, nd in enumerate(nodes):
            kids[nd.parent].append(i)
        cur, path = -1, []
        while True:
            row = base + cur + 1
            ch = kids[cur]
            if ch and rng.random() < accept_p:
                pick = ch[int(rng.integers(0, len(ch)))]
                logits[row, nodes[pick].token] = 16.0
                path.append(pick)
                cur = pick
                continue
            taken = {nodes[c].token for c in ch}
            tok = int(rng.integers(0, V))
            while tok in taken:
                tok = (tok + 1) % V
            logits[row, tok] = 16.0
            break
        paths.append(path)
    return logits.to(device), paths
