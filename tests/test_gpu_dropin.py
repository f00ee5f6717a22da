"""Drop-in check: the reference's own C test program runs on this engine.

oracle/_ref/quant_on_mi355x is examples/quant.c from the reference, compiled unmodified against
include/ork_npu.h and linked to libork_npu.so (oracle/ref.mk). It packs with ork_i8_mm_pack, runs
ork_i8_mm_run at 7 shapes (M=1..512) and compares an FNV-64 of C with its embedded goldens
(examples/quant.c:72-81); with ORK_TEST_DMA set, A and C live in ork_dma_alloc buffers (:39-44).
The binary is built where the reference tree exists and travels with the repository.
"""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref", "quant_on_mi355x")


@pytest.mark.skipif(not os.path.exists(BIN), reason="oracle/_ref/quant_on_mi355x not built (needs the reference tree)")
@pytest.mark.parametrize("dma", [0, 1])
def test_reference_quant_example_runs_unmodified(dma):
    env = dict(os.environ)
    if dma:
        env["ORK_TEST_DMA"] = "1"
    print("[case] reference examples/quant.c, ORK_TEST_DMA=%d" % dma, flush=True)
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120, env=env)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ALL OK" in r.stdout
    assert r.stdout.count("golden") == 7  # every case took the golden (bit-exact) branch
