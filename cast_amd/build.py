"""Build the HIP libraries for gfx950 with hipcc.

    python -m cast_amd.build            # cast_amd/libcast_amd.so and libcast_bench.so

libcast_amd.so (the product, the C ABI of include/cast_amd.h) comes from
cast_amd/csrc/*.hip; libcast_bench.so (bench.py's measurement aids,
cast_amd/csrc/bench/cast_bench.h) from cast_amd/csrc/bench/*.hip.  Compiler
warnings are printed; a register-budget miss in an attention kernel
(``-Wpass-failed``: an amdgpu_waves_per_eu target not met) fails the build.

The library links against the HIP runtime with an rpath to torch's bundled
``torch/lib`` so that, with or without torch imported first, the process
maps a single libamdhip64 (both carry the soname libamdhip64.so.7).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "libcast_amd.so"
BENCH_OUT = PKG / "libcast_bench.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # no packed-fp32 VALU forms (v_pk_add/mul/fma_f32) anywhere in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def _torch_lib():
    try:
        import importlib.util
        spec = importlib.util.find_spec("torch")
        if spec and spec.origin:
            lib = Path(spec.origin).parent / "lib"
            if (lib / "libamdhip64.so").exists():
                return lib
    except Exception:
        pass
    return None


def sources():
    return sorted(CSRC.glob("*.hip"))


def bench_sources():
    return sorted((CSRC / "bench").glob("*.hip"))


# warnings that fail the build: a kernel that misses its occupancy target
# runs with fewer waves than its tiling assumes
# a kernel that misses its amdgpu_waves_per_eu target, or any other pass the
# compiler was asked to apply and could not (an unroll pragma, for one)
_FATAL = ("failed to meet occupancy target", "-Wpass-failed")


def _compile(hipcc, src, objdir, inc):
    obj = objdir / (src.stem + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, *inc, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")
    return obj, res.stderr


def _link(hipcc, objs, out):
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(out) + ".tmp"]
    tl = _torch_lib()
    if tl is not None:
        link += [f"-Wl,-rpath,{tl}"]
    res = subprocess.run(link, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(str(out) + ".tmp", out)


def _warnings(stderr):
    """hipcc's warnings, without its note that the host pass does not know
    the device-only -packed-fp32-ops feature."""
    keep = []
    for line in stderr.splitlines():
        if "packed-fp32-ops" in line and "not a recognized feature" in line:
            continue
        if line.strip():
            keep.append(line)
    return "\n".join(keep)


def build(verbose: bool = True) -> Path:
    hipcc = _hipcc()
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    (objdir / "bench").mkdir(exist_ok=True)
    inc = ["-I", str(ROOT / "include"), "-I", str(CSRC), "-I", str(CSRC / "bench")]
    jobs = [(s, objdir) for s in sources()] + [(s, objdir / "bench") for s in bench_sources()]
    with ThreadPoolExecutor(max_workers=4) as ex:
        done = list(ex.map(lambda j: (j[0], *_compile(hipcc, j[0], j[1], inc)), jobs))
    fatal = []
    for src, _, err in done:
        text = _warnings(err)
        if text and verbose:
            print(f"hipcc warnings in {src.name}:\n{text}", file=sys.stderr)
        if any(f in text for f in _FATAL):
            fatal.append(src.name)
    if fatal:
        raise RuntimeError("a kernel misses its occupancy target (amdgpu_waves_per_eu) or a requested "
                           f"optimisation (-Wpass-failed) in {', '.join(fatal)}")
    n = len(sources())
    _link(hipcc, [o for _, o, _ in done[:n]], OUT)
    _link(hipcc, [o for _, o, _ in done[n:]], BENCH_OUT)
    return OUT


if __name__ == "__main__":
    print(build())
