"""The host-side plan builders, router and diagnostics under AddressSanitizer,
UndefinedBehaviorSanitizer and LeakSanitizer (no GPU): tests/host_sanitize_driver.cpp
drives the host tile builder (every kind, fp16 and bf16, every exported array),
the production features, the router (both tables and portfolios), the
diagnostic extractor, and the invalid-input paths."""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "ra-spmm_amd" / "csrc"
SOURCES = ["tile_build.cpp", "router.cpp", "diagnostics.cpp", "common.cpp"]


def test_host_builders_clean_under_sanitizers(tmp_path):
    gxx = shutil.which("g++")
    hip = Path("/opt/rocm/lib/libamdhip64.so")
    if gxx is None or not hip.exists():
        pytest.skip("needs g++ and the ROCm runtime library")
    exe = tmp_path / "host_sanitize"
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-omit-frame-pointer",
           "-fno-sanitize-recover=undefined", "-D__HIP_PLATFORM_AMD__=1", "-I/opt/rocm/include",
           f"-I{ROOT / 'include'}", f"-I{CSRC}", str(Path(__file__).with_name("host_sanitize_driver.cpp"))]
    cmd += [str(CSRC / s) for s in SOURCES] + ["-L/opt/rocm/lib", "-lamdhip64", "-lpthread", "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True)
    assert build.returncode == 0, build.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    run = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=600)
    assert run.returncode == 0, (run.stdout + run.stderr)[-4000:]
    assert "0 failures" in run.stdout
