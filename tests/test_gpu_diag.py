"""The measurement aids behind bench.py --clock-trace and --mfma-ceiling.

The MFMA ceiling loop must do the work it is timed for: over one wave, the
sum of every accumulator element of a v_mfma_f32_32x32x16_bf16 product is
sum_k (sum_i A[i][k]) * (sum_j B[k][j]), whatever the output layout, so the
wave's summed outputs pin which operands met in how many products (each mode's
operand addressing, the LDS tile alternation included)."""
import numpy as np
import pytest
import torch

from bench import bench_lib
from cast_amd import _lib

pytestmark = pytest.mark.gpu

KPAD, VPAD = 136, 72
TILE = 64 * KPAD + 128 * VPAD     # elements of one K + V^T tile buffer


def _pair(x, y):
    """Sum of all outputs of one 32x32x16 MFMA over a wave: lane l holds
    A[l % 32][8 (l // 32) + e] in x[l, e] and B[8 (l // 32) + e][l % 32] in y[l, e]."""
    return float((x.reshape(2, 32, 8).sum(1) * y.reshape(2, 32, 8).sum(1)).sum())


def _expected_wave(src, wave, tiles, mode):
    n = src.shape[0]                                     # 16-byte chunks of 8 values
    tid = wave * 64 + np.arange(64)
    a = [src[(tid * 16 + i) % n] for i in range(8)]      # [64, 8] each
    b = [src[(tid * 16 + 8 + i) % n] for i in range(8)]
    l32, g = np.arange(64) % 32, np.arange(64) // 32
    total = 0.0
    for t in range(tiles):
        base = (t & 1) * TILE

        def lds(elem):                                   # element offsets -> [64, 8] operand
            return src[((base + elem) // 8) % n]

        for kb in range(2):
            for ds in range(8):
                x = lds((kb * 32 + l32) * KPAD + ds * 16 + g * 8) if mode & 1 else a[ds]
                total += _pair(x, b[ds])
        for kb in range(2):
            for hf in range(2):
                for db in range(4):
                    if mode & 1:
                        x = lds(64 * KPAD + (db * 32 + l32) * VPAD + kb * 32 + hf * 16 + g * 8)
                    else:
                        x = a[(kb * 2 + hf + db) & 7]
                    total += _pair(x, b[kb * 2 + hf])
    return total


@pytest.mark.parametrize("mode", [0, 1, 3])
def test_mfma_ceiling_does_the_products_it_claims(gpu, mode):
    lib = bench_lib()
    grid, tiles = 2, 3                                   # odd: both LDS tile buffers are read
    g = torch.Generator(device=gpu).manual_seed(11)
    src = torch.randn(40000 * 8, generator=g, device=gpu).to(torch.bfloat16)   # 40000 chunks, read modulo
    out = torch.empty(grid * 512, dtype=torch.float32, device=gpu)
    clk = torch.zeros(2 * grid, dtype=torch.int64, device=gpu)
    print(f"case mfma ceiling mode {mode} grid {grid} tiles {tiles}", flush=True)
    _lib.check(lib.cast_mfma_ceiling(_lib.ptr(src), src.numel() // 8, _lib.ptr(out), _lib.ptr(clk), grid, tiles,
                                     mode, _lib.stream_of(src)), "cast_mfma_ceiling")
    torch.cuda.synchronize()
    s = src.float().cpu().numpy().astype(np.float64).reshape(-1, 8)
    got = out.cpu().numpy().astype(np.float64).reshape(grid, 8, 64).sum(-1)
    for w in range(8):
        want = _expected_wave(s, w, tiles, mode)
        # bf16 products are exact in fp32; what is left is fp32 accumulation over
        # 6144 outputs of magnitude ~20 (error ~1e-2), against ~1e3 for a wrong pairing
        bound = 1e-4 * abs(want) + 5e-2
        for blk in range(grid):
            assert abs(got[blk, w] - want) <= bound, (mode, blk, w, got[blk, w], want)
    c = clk.view(grid, 2).cpu().numpy()
    assert (c[:, 0] > 0).all() and (c[:, 1] > 0).all()


def test_clock_sample_reads_a_plausible_clock(gpu):
    lib = bench_lib()
    buf = torch.zeros(8, dtype=torch.int64, device=gpu)
    for slot in range(4):
        _lib.check(lib.cast_clock_sample(_lib.ptr(buf), slot, 20000, _lib.stream_of(buf)), "cast_clock_sample")
    torch.cuda.synchronize()
    c = buf.view(4, 2).cpu().numpy()
    assert (c > 0).all()
    ghz = c[:, 0] / (c[:, 1] / 100.0) / 1e3               # cycles per ns
    assert ((ghz > 0.3) & (ghz < 4.0)).all(), ghz
