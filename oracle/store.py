"""KV-store bookkeeping after a verify round, restated row by row.
TEST INFRASTRUCTURE ONLY (checker for the K4 append kernel).

append_store  follows cast_trees/serving.py:264-289 (_append_store):
    1. the surviving requests ``rows`` keep their store rows, in that order
       (requests that finished drop out of the batch, serving.py:272-275);
    2. if some request's new length store_len[b] + accepted[b] exceeds the
       capacity, every store grows to max(longest, 2 * capacity) slots, the
       new slots zero (serving.py:276-280);
    3. for surviving request b at new batch index nb, kept row j (pack index
       keep[b][j]) of every layer's pack K/V [Hkv, total_q, D] is written to
       slot store_len[b] + j of that layer's store [B, Hkv, cap, D]
       (serving.py:281-288).
gather_cache  follows cast_trees/verify.py:48-60: a batch-one cache keeps its
    first n_prefix positions followed by positions n_prefix + keep[j].

Both are written as explicit per-row copies (no index tensors), so they
share no code path with either the reference or the kernel they check.
"""
import torch


def append_store(buf_k, buf_v, pack_k, pack_v, store_len, cu_q, keep, accepted, rows):
    """Returns (new K stores, new V stores, new lengths) as fresh tensors."""
    new_len = [int(store_len[b]) + int(accepted[b]) for b in rows]
    cap = int(buf_k[0].shape[2])
    longest = max(new_len, default=0)
    cap2 = max(longest, 2 * cap) if longest > cap else cap

    def survivors(x):
        y = torch.zeros((len(rows), x.shape[1], cap2, x.shape[3]), dtype=x.dtype, device=x.device)
        for nb, b in enumerate(rows):
            y[nb, :, :cap] = x[b]
        return y

    out_k = [survivors(x) for x in buf_k]
    out_v = [survivors(x) for x in buf_v]
    for layer in range(len(buf_k)):
        for nb, b in enumerate(rows):
            for j, pk in enumerate(keep[b]):
                src = int(cu_q[b]) + int(pk)
                dst = int(store_len[b]) + j
                out_k[layer][nb, :, dst] = pack_k[layer][:, src]
                out_v[layer][nb, :, dst] = pack_v[layer][:, src]
    return out_k, out_v, new_len


def gather_cache(layers, n_prefix, keep):
    """layers: list of (K, V) [1, Hkv, T, D] -> list of compacted (K, V)."""
    positions = list(range(n_prefix)) + [n_prefix + int(i) for i in keep]
    out = []
    for k, v in layers:
        kk = torch.empty((1, k.shape[1], len(positions), k.shape[3]), dtype=k.dtype, device=k.device)
        vv = torch.empty_like(kk)
        for j, p in enumerate(positions):
            kk[:, :, j] = k[:, :, p]
            vv[:, :, j] = v[:, :, p]
        out.append((kk, vv))
    return out
