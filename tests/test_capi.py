"""The C ABI: the library loads, exports every declared symbol, and rejects
bad host-side arguments before touching the GPU (no GPU needed)."""
import re
from pathlib import Path

import pytest

from cast_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "cast_amd.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]*?\b(cast_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail("libcast_amd.so is not built (run `python -m cast_amd.build` or __graft_entry__.build())")
    return _lib.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = declared()
    assert names == sorted(_lib.SIGNATURES), "ctypes bindings and header disagree"
    for n in names:
        assert hasattr(lib, n), n
    # the measurement aids live in bench.py's own library only
    for n in ("cast_clock_sample", "cast_mfma_ceiling"):
        assert not hasattr(lib, n), n
    assert lib.cast_abi_version() == 4


def test_status_strings(lib):
    for code in range(14):
        assert lib.cast_status_string(code) != b"unknown status", code
    assert b"multiple of KV heads" in lib.cast_status_string(2)


def _attn(lib, **over):
    args = dict(q=None, k=None, v=None, out=None, lse=None, cu_q=None, cu_kv=None, prefix=None, pack=None,
                mask=None, words=2, B=1, tq=16, tkv=32, Hq=32, Hkv=8, D=128, strides=[0] * 8, dtype=0,
                scale=0.1, split=0, ws=None, wsb=0, status=None, stream=None)
    args.update(over)
    a = args
    return lib.cast_tree_attn_fwd(a["q"], a["k"], a["v"], a["out"], a["lse"], a["cu_q"], a["cu_kv"], a["prefix"],
                                  a["pack"], a["mask"], a["words"], a["B"], a["tq"], a["tkv"], a["Hq"], a["Hkv"],
                                  a["D"], *a["strides"], a["dtype"], a["scale"], a["split"], a["ws"], a["wsb"],
                                  a["status"], a["stream"])


def test_attention_host_validation(lib):
    assert _attn(lib, Hq=32, Hkv=7) == 2                 # head ratio
    assert _attn(lib, Hkv=0) == 2
    assert _attn(lib, dtype=5) == 4                      # dtype
    assert _attn(lib, words=3) == 7                      # mask words
    assert _attn(lib, scale=0.0) == 9                    # scale
    assert _attn(lib, scale=float("nan")) == 9
    assert _attn(lib, B=-1) == 7
    assert _attn(lib) == 1                               # null pointers
    assert _attn(lib, B=0) == 0 and _attn(lib, tq=0) == 0  # nothing to do


def test_workspace_and_split_are_host_only(lib):
    # the headline shape: 8 requests x (8192 prefix + 128 pack), Qwen3 heads
    split = lib.cast_tree_attn_default_split(8, 1024, 66560, 32, 8, 128, 0)
    assert split > 0 and split % 64 == 0
    ws = lib.cast_tree_attn_workspace_size(8, 1024, 66560, 32, 8, 128, 0, 0)
    assert ws > 0 and ws % 256 == 0
    assert lib.cast_tree_attn_workspace_size(8, 1024, 66560, 32, 8, 128, 0, -1) == 0     # no split
    assert lib.cast_tree_attn_workspace_size(1, 16, 144, 4, 4, 64, 1, 0) > 0             # fp32 MFMA path splits too
    assert lib.cast_tree_attn_workspace_size(1, 16, 144, 4, 4, 96, 1, 0) == 0            # generic path: no split
    assert lib.cast_tree_attn_workspace_size(8, 1024, 66560, 32, 7, 128, 0, 0) == 0      # bad ratio


def test_bitmask_and_accept_validation(lib):
    assert lib.cast_tree_bitmask(None, None, 1, 1, 3, None, None, None) == 7
    assert lib.cast_tree_bitmask(None, None, 1, 4, 2, None, None, None) == 1
    assert lib.cast_tree_bitmask(None, None, 0, 0, 2, None, None, None) == 0
    assert lib.cast_greedy_accept(None, 10, 10, 0, None, None, None, 1, 1, None, None, None, None, None, None) == 1
    assert lib.cast_greedy_accept(None, 5, 10, 0, None, None, None, 1, 1, None, None, None, None, None, None) == 7
    assert lib.cast_greedy_accept(None, 10, 10, 9, None, None, None, 1, 1, None, None, None, None, None, None) == 4


def test_python_layer_maps_errors():
    with pytest.raises(AssertionError):
        _lib.check(2, "x")
    with pytest.raises(_lib.CastError):
        _lib.check(10, "x")
    with pytest.raises(ValueError):
        _lib.raise_device_flags(_lib.FLAG_BAD_PARENT, "x")
    _lib.raise_device_flags(0, "x")


def _store(lib, **over):
    a = dict(ptrs=[None] * 11, words=2, B=1, tq=16, tkv=32, cap=64, Hq=32, Hkv=8, D=128, strides=[8] * 14,
             dtype=0, scale=0.1, split=0, ws=None, wsb=0, status=None, stream=None)
    a.update(over)
    return lib.cast_tree_attn_store_fwd(*a["ptrs"], a["words"], a["B"], a["tq"], a["tkv"], a["cap"], a["Hq"],
                                        a["Hkv"], a["D"], *a["strides"], a["dtype"], a["scale"], a["split"],
                                        a["ws"], a["wsb"], a["status"], a["stream"])


def test_store_attention_host_validation(lib):
    assert _store(lib) == 1                              # null pointers
    assert _store(lib, Hkv=3) == 2                       # head ratio
    assert _store(lib, cap=-1) == 7                      # negative capacity
    assert _store(lib, dtype=2) == 4
    assert _store(lib, scale=-1.0) == 9
    assert _store(lib, B=0) == 0                         # nothing to do


def test_store_append_host_validation(lib):
    f = lib.cast_store_append
    args = lambda **o: [o.get("ptr", None)] * 4 + [o.get("layers", 2)] + [None] * 2 + [o.get("stride", 128)] + \
        [None] * 3 + [o.get("B", 2), 16, 64, 4, 128] + [8] * 10 + [o.get("dtype", 0), None, None]
    assert f(*args()) == 1                       # null pointers
    assert f(*args(stride=64)) == 7              # path rows narrower than 128
    assert f(*args(dtype=2)) == 4                # dtype (fp64 has no row copy)
    assert f(*args(dtype=9)) == 4
    assert f(*args(B=0)) == 0 and f(*args(layers=0)) == 0


def test_store_append_refuses_lengths_written_over_its_inputs(lib):
    # new_len is written while other workgroups still read store_len,
    # path_len, src_row and path: any overlap is refused before a launch
    import ctypes
    fake = 1 << 20
    arr = (ctypes.c_void_p * 2)(fake, fake)
    B = 4
    src, path, plen, slen = fake + 0x1000, fake + 0x2000, fake + 0x4000, fake + 0x5000

    def call(new_len):
        return lib.cast_store_append(arr, arr, arr, arr, 2, src, path, 128, plen, slen, new_len, B, 16, 64, 4,
                                     128, *([8] * 10), 0, None, None)
    for alias in (slen, plen, src, path, path + 4 * 128 * B - 4, slen - 4 * B + 4, slen + 12):
        assert call(alias) == 13, hex(alias)


def test_store_layout_checked_once_and_rechecked_on_change():
    # the per-layer checks of the stores run once per set of stores; a
    # replaced layer tensor (new object, other shape) is checked again.  The
    # pack K/V are new tensors every verify pass and are checked per call.
    import torch
    from cast_amd import serving
    L = 4
    buf_k = [torch.empty((2, 2, 16, 64), dtype=torch.bfloat16) for _ in range(L)]
    buf_v = [torch.empty_like(x) for x in buf_k]
    first = serving._store_layout(buf_k, buf_v)
    assert serving._store_layout(buf_k, buf_v) is first
    assert list(first["k"]) == [t.data_ptr() for t in buf_k]
    assert list(first["v"]) == [t.data_ptr() for t in buf_v]
    buf_k[2] = torch.empty((2, 2, 8, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="share shape"):
        serving._store_layout(buf_k, buf_v)
    buf_k[2] = torch.empty((2, 2, 16, 64), dtype=torch.bfloat16)
    again = serving._store_layout(buf_k, buf_v)
    assert again is not first and again["k"][2] == buf_k[2].data_ptr()
    pack_k = [torch.empty((5, 2, 64), dtype=torch.bfloat16).transpose(0, 1) for _ in range(L)]
    pack_v = [torch.empty_like(x) for x in pack_k]
    kp, vp, kst, vst, total_q = serving._pack_arrays(again, pack_k, pack_v)
    assert list(kp) == [t.data_ptr() for t in pack_k] and total_q == 5 and kst == (128, 64)
    pack_v[1] = torch.empty((2, 5, 64), dtype=torch.float32)
    with pytest.raises(ValueError, match="dtype"):
        serving._pack_arrays(again, pack_k, pack_v)


def test_build_trees_checks_inputs_before_launch():
    # shape mismatches and host tensors are refused before any device work
    import torch
    from cast_amd.draft import build_trees
    ti = torch.zeros((2, 15, 8), dtype=torch.int64)
    with pytest.raises(ValueError, match="both be"):
        build_trees(ti, torch.zeros((2, 15, 4)), 15)
    with pytest.raises(ValueError, match="one GPU"):
        build_trees(ti, torch.zeros((2, 15, 8)), 15)


def test_greedy_accept_refuses_host_logits():
    import torch
    from cast_amd.verify import greedy_accept
    with pytest.raises(ValueError, match="device tensor"):
        greedy_accept(torch.zeros((3, 10)), [0, 3], [-1, 0, 0], [0, 1, 2])


def test_attention_wrappers_refuse_tensors_on_other_devices():
    # q on the "device" check passes only for CUDA tensors; a host K next to a
    # device q would hand host pointers to the kernel, so it is refused first
    import torch
    from cast_amd import tree_attn
    q = torch.zeros((4, 8, 64))
    with pytest.raises(ValueError, match="on the GPU|device"):
        tree_attn.varlen_tree_attention(q, torch.zeros((9, 2, 64)), torch.zeros((9, 2, 64)), [0, 4], [0, 9],
                                        [5], [4], torch.zeros(4, dtype=torch.int64))
    with pytest.raises(ValueError, match="one GPU"):
        tree_attn._require_on(torch.device("cuda", 0), k=torch.zeros(1))


def test_draft_topk_split_sizing_and_validation(lib):
    # automatic splits: about one workgroup per CU, at least one first batch
    # (8 x 512 chunks) per split and splits * k <= 64 for the combine wave
    part = 144                              # bytes per (row, split) record
    V, BF16, FP32 = 151936, 0, 1
    assert lib.cast_draft_topk_workspace_size(120, V, BF16, 8, 0) == 120 * 2 * part
    assert lib.cast_draft_topk_workspace_size(15, V, BF16, 8, 0) == 15 * 4 * part   # capped by the vocabulary
    assert lib.cast_draft_topk_workspace_size(300, V, BF16, 8, 0) == 0             # one workgroup per row
    assert lib.cast_draft_topk_workspace_size(8, V, FP32, 16, 0) == 8 * 4 * part    # 16 x 4 = 64 keys
    assert lib.cast_draft_topk_workspace_size(8, V, BF16, 8, 1) == 0
    assert lib.cast_draft_topk_workspace_size(8, 1000, BF16, 8, 4) == 0             # short rows never split
    assert lib.cast_draft_topk_workspace_size(0, V, BF16, 8, 0) == 0
    fake = 0x10000                          # never dereferenced: every case fails before a launch
    call = lambda rows=120, k=8, splits=0, ws=fake, wsb=120 * 2 * part: lib.cast_draft_topk(
        fake, V, rows, V, BF16, k, fake, fake, splits, ws, wsb, None)
    assert call(k=0) == 7 and call(k=17) == 7 and call(splits=-1) == 7
    assert lib.cast_draft_topk(fake, V - 1, 120, V, BF16, 8, fake, fake, 0, fake, 1 << 20, None) == 7   # ld < vocab
    assert lib.cast_draft_topk(fake, V, 120, V, 5, 8, fake, fake, 0, fake, 1 << 20, None) == 4          # dtype
    assert call(rows=0) == 0
    assert call(ws=None) == 1                               # two splits need the workspace
    assert call(wsb=120 * 2 * part - 1) == 8                # one byte short
    assert call(ws=fake + 8) == 6                           # 16-byte alignment


def test_host_metadata_is_checked_before_launch():
    # metadata already on the host (lists / numpy) is validated in Python:
    # the call raises before any device work
    import numpy as np
    from cast_amd.tree_attn import check_host_metadata
    ok = dict(cu_q=[0, 10, 30], prefix_len=[5, 7], pack_len=[10, 20], total_q=30, total_kv=42, words=2,
              cu_kv=[0, 15, 42])
    check_host_metadata(**ok)
    with pytest.raises(ValueError, match="exceeds the 64 bits"):
        check_host_metadata(**dict(ok, pack_len=[10, 70], cu_q=[0, 10, 80], total_q=80, cu_kv=[0, 15, 92],
                                   total_kv=92, words=1))
    with pytest.raises(ValueError, match="cu_q"):
        check_host_metadata(**dict(ok, cu_q=[0, 11, 31]))
    with pytest.raises(ValueError, match="cu_kv"):
        check_host_metadata(**dict(ok, cu_kv=[0, 16, 43]))
    with pytest.raises(ValueError, match="cu_q"):
        check_host_metadata(**dict(ok, total_q=29))
    with pytest.raises(ValueError, match="store capacity"):
        check_host_metadata(**dict(ok, cu_kv=None, cap=6))
    with pytest.raises(ValueError, match="total_kv"):
        check_host_metadata(**dict(ok, cu_kv=None, total_kv=41))
    check_host_metadata(**dict(ok, cu_q=np.array([0, 10, 30]), cu_kv=None))


def test_noalloc_entry_refuses_oversized_scratch_before_device_work(lib):
    # the headline shapes with 64-key splits need ~2 GiB of partials: far
    # above the static scratch, refused on the host (no GPU touched)
    assert lib.cast_tree_attn_noalloc_limit() == 72 << 20
    need = lib.cast_tree_attn_workspace_size(8, 1024, 66560, 32, 8, 128, 0, 64)
    assert need > lib.cast_tree_attn_noalloc_limit()
    st = lib.cast_tree_attn_fwd_noalloc(*([None] * 10), 2, 8, 1024, 66560, 32, 8, 128, *([128] * 8), 0, 0.1, 64,
                                        None, None)
    assert st == _lib.ERR_SCRATCH_LIMIT
    assert b"no-allocation" in lib.cast_status_string(st)


def test_build_trees_refuses_host_budgets_above_127():
    import torch
    from cast_amd.draft import build_trees
    ti = torch.zeros((2, 15, 8), dtype=torch.int64)
    tl = torch.zeros((2, 15, 8))
    for bad in (128, -1, [10, 200]):
        with pytest.raises(ValueError, match="budget must be in"):
            build_trees(ti, tl, bad)


def test_mfma_ceiling_host_validation():
    # bench.py's measurement aid (libcast_bench.so, not the product library)
    # rejects bad arguments before any launch
    from bench import bench_lib
    lib = bench_lib()
    fake = 1 << 20
    assert lib.cast_mfma_ceiling(None, 8, fake, fake, 1, 1, 0, None) == 1
    assert lib.cast_mfma_ceiling(fake, 0, fake, fake, 1, 1, 0, None) == 7
    assert lib.cast_mfma_ceiling(fake, 1 << 31, fake, fake, 1, 1, 0, None) == 7
    assert lib.cast_mfma_ceiling(fake, 8, fake, fake, 0, 1, 0, None) == 7
    assert lib.cast_mfma_ceiling(fake, 8, fake, fake, 1, -1, 0, None) == 7
    for mode in (2, 4, -1):
        assert lib.cast_mfma_ceiling(fake, 8, fake, fake, 1, 1, mode, None) == 7


def test_head_dim_bounds(lib):
    # MFMA kernels take 64 and 128; the scalar kernel any other multiple of 8
    # up to 256.  Out-of-range head dims are refused before any launch.
    fake = 1 << 20
    ptrs = dict(q=fake, k=fake, v=fake, out=fake, cu_q=fake, cu_kv=fake, prefix=fake, pack=fake, mask=fake)
    for D in (264, 100, 4, 512):
        assert _attn(lib, D=D, **ptrs) == 5, D


def test_build_fails_on_occupancy_and_pass_failed_warnings():
    # cast_amd.build stops on a kernel that misses its waves-per-SIMD target or
    # on any other -Wpass-failed warning, and drops only hipcc's note that the
    # host pass does not know the device-only packed-fp32 feature
    from cast_amd import build as B
    host_note = "warning: '-packed-fp32-ops' is not a recognized feature for this target (ignoring feature)"
    assert B._warnings(host_note) == ""
    occ = ("tree_attn.hip:700:1: warning: void cast::k(): failed to meet occupancy target given by "
           "'amdgpu-waves-per-eu' in 'k': desired occupancy was 2, final occupancy is 1 [-Wpass-failed]")
    unroll = "draft.hip:10:5: warning: loop not unrolled: the optimizer was unable to perform the " \
             "requested transformation [-Wpass-failed=transform-warning]"
    other = "store.hip:3:1: warning: unused variable 'x' [-Wunused-variable]"
    for text, fatal in ((occ, True), (unroll, True), (other, False)):
        kept = B._warnings(host_note + "\n" + text)
        assert kept == text
        assert any(f in kept for f in B._FATAL) == fatal
