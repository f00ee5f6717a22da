"""The host library under AddressSanitizer, on the CPU.

tests/asan/host_sequence.c makes the bench's host-side calls (config 3's pack / dump / load / run / free for
uniform and NF4 with an importance vector, config 1's pack, runs and chain with device and host operands, fp16,
W4A4 and grouped W4A4) against tests/asan/orkh_host_stubs.c, which stands in for the HIP layer with host memory:
every transfer the library requests is a memcpy of exactly the requested size, so ASan checks the library's
buffer sizes on both sides. It runs with ORK_PROFILE set, so the per-call timing table is exercised as well. The
library's host sources are compiled with the ROCm clang (host code only; no GPU
code is built or run). No kernel runs, so nothing about results is checked here.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLANG = "/opt/rocm/llvm/bin/clang"
HOST = ["context.c", "quant.c", "panel.c", "plan.c", "weights.c", "persist.c", "run.c", "chain.c", "cpu_gemm.c", "prof.c"]


@pytest.mark.skipif(not os.path.exists(CLANG), reason="ROCm clang not installed")
def test_host_library_under_asan(tmp_path):
    hs = os.path.join(ROOT, "ork-driver_amd", "csrc", "host")
    exe = str(tmp_path / "host_sequence")
    cmd = [CLANG, "-O1", "-g", "-fsanitize=address", "-fno-omit-frame-pointer", "-std=gnu11", "-pthread",
           "-ffp-contract=off", "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(ROOT, "ork-driver_amd", "csrc", "hip"),
           "-I" + hs] + [os.path.join(hs, f) for f in HOST] + \
          [os.path.join(ROOT, "tests", "asan", "orkh_host_stubs.c"), os.path.join(ROOT, "tests", "asan", "host_sequence.c"),
           "-o", exe, "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    # ORK_PROFILE on: the per-call timing rows (events stand in as host memory) run under ASan too
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0", ORK_PROFILE="1")
    env.pop("ORK_NF4", None)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0 and r.stdout.strip().endswith("done"), (r.stdout[-2000:], r.stderr[-4000:])
    assert "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
    assert "[ork PROFILE] ork_i8_mm_run " in r.stderr, r.stderr[-4000:]
