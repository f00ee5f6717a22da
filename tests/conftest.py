import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# The planner honours its test overrides (ORK_PLAN, ORK_TILE, ORK_KSPLIT, ORK_ALINE, ORK_STREAM_NP, ORK_WPG) only on
# a context made while ORK_PLAN_DEBUG is set; the forced-plan parity tests rely on it.
os.environ.setdefault("ORK_PLAN_DEBUG", "1")
for p in (os.path.join(ROOT, "ork-driver_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (run with -m gpu on the GPU box)")
    config.addinivalue_line("markers", "slow: CPU test that takes more than a few seconds")


@pytest.fixture(scope="session")
def npu():
    """One device context for the whole GPU session (the reference's one-context-per-process model)."""
    import ork

    ctx = ork.Npu()
    print(f"[gpu] {ork.lib().ork_npu_soc(ctx.h).decode()} cores={ork.lib().ork_npu_cores(ctx.h)}", flush=True)
    yield ctx
    ctx.close()
