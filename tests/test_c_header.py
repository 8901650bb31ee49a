"""The C ABI from plain C: include/cast_amd.h compiles as strict C99 (what a
cgo, JNI or other C binding compiles against), and a C program linked to the
built library gets answers from the host-only entry points without a GPU."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "cast_amd" / "libcast_amd.so"


@pytest.mark.skipif(shutil.which("gcc") is None, reason="no C compiler")
def test_header_is_c99_and_host_calls_answer(tmp_path):
    if not LIB.exists():
        pytest.skip("libcast_amd.so is not built")
    exe = tmp_path / "host_calls"
    cmd = ["gcc", "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", f"-I{ROOT / 'include'}",
           str(ROOT / "tests" / "c_abi" / "host_calls.c"), "-o", str(exe), f"-L{LIB.parent}", "-lcast_amd",
           f"-Wl,-rpath,{LIB.parent}"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.strip().endswith("ok")
