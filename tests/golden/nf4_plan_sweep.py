"""Graph-timed NF4 (W4A8 codebook) launches of every kernel, tile and K split the planner offers, over the shapes the
planner's NF4 fits were made on; writes nf4_plan_sweep.json beside this file (read by tests/test_planner.py).

On one MI355X, from the repository root, with the library built:
    python3 tests/golden/nf4_plan_sweep.py                 # sweep (about 10 minutes), then write the fixture
    python3 tests/golden/nf4_plan_sweep.py --reduce LOG    # write the fixture from the JSON lines of an earlier sweep
Every launch's result is checked against the oracle's exact GEMM before it is timed; inexact ones are dropped.
"""
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "nf4_plan_sweep.json")
SHAPES = {(2048, 6144): (32, 48, 64, 96, 128, 192, 256, 384, 512, 1024),
          (6144, 2048): (32, 48, 64, 96, 128, 192, 256, 384, 512, 1024),
          (4096, 4096): (32, 48, 64, 96, 128, 192, 256, 384, 512, 1024),
          (2048, 2048): (32, 64, 96, 128, 192, 256, 512, 1024),
          (2048, 12288): (32, 64, 96, 128, 192, 256, 512)}
PLANS = [{}] + [{"ORK_PLAN": "stream", "ORK_KSPLIT": k} for k in (1, 2, 4)] \
    + [{"ORK_PLAN": "tiled", "ORK_TILE": t, "ORK_KSPLIT": k} for t in ("64x64", "128x96", "128x128") for k in (1, 2, 4, 8)] \
    + [{"ORK_TILE": t, "ORK_KSPLIT": k} for t in ("32x64", "64x64", "128x96", "128x128") for k in (1, 2, 4)]


def sweep():
    sys.path[:0] = [os.path.join(ROOT, "ork-driver_amd"), ROOT, os.path.join(ROOT, "oracle")]
    os.environ["ORK_PLAN_DEBUG"] = "1"
    import numpy as np
    import bench
    import ork
    import oracle as O
    rng = np.random.default_rng(3)
    hip, L = bench.Hip(), ork.lib()
    lines = []
    with ork.Npu() as npu:
        for (K, N), Ms in SHAPES.items():
            Mx = max(Ms)
            dA, dC = L.ork_dev_alloc(npu.h, Mx * K), L.ork_dev_alloc(npu.h, Mx * N * 4)
            A = rng.integers(-127, 128, size=(Mx, K), dtype=np.int8)
            assert L.ork_dev_upload(npu.h, dA, ork.ptr(A), A.nbytes) == 0
            W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
            os.environ["ORK_NF4"] = "1"
            ws = [npu.pack_i4a8(W)[0] for _ in range(48)]   # rotated: every launch reads its weight from HBM
            os.environ.pop("ORK_NF4", None)
            codes = O.pack_i4a8(W, nf4=True)[2]
            for M in Ms:
                want = O.gemm_i32(A[:M], codes)
                for env in PLANS:
                    if "ORK_TILE" in env and int(env["ORK_TILE"].split("x")[0]) > 2 * M:
                        continue
                    if env.get("ORK_PLAN") == "stream" and M > 64:
                        continue
                    os.environ.update({k: str(v) for k, v in env.items()})
                    try:
                        name = npu.plan_name(ws[0], M)
                        L.ork_npu_set_async(npu.h, 0)
                        C = np.empty((M, N), np.int32)
                        ok = L.ork_i8_mm_run(npu.h, ws[0], M, dA, dC) == 0 and \
                            L.ork_dev_download(npu.h, ork.ptr(C), dC, C.nbytes) == 0 and np.array_equal(C, want)
                        L.ork_npu_set_async(npu.h, 1)
                        t = [round(bench.measure(npu, hip, ws, M, dA, dC, 160, 16)[0] * 1e3, 2) for _ in range(2)] \
                            if ok else None
                    finally:
                        for k in env:
                            os.environ.pop(k, None)
                    r = {"K": K, "N": N, "M": M, "env": env, "plan": name, "exact": bool(ok), "us": t}
                    print(json.dumps(r), flush=True)
                    lines.append(r)
            for w in ws:
                L.ork_mm_free(npu.h, w)
            L.ork_dev_free(npu.h, dA)
            L.ork_dev_free(npu.h, dC)
    return lines


def reduce(lines):
    """per shape, the fastest exact time of each plan name (the same plan can be reached by several overrides)"""
    shapes = {}
    for r in lines:
        if not r["exact"] or not r["us"]:
            continue
        s = shapes.setdefault((r["K"], r["N"], r["M"]), {})
        s[r["plan"]] = min(s.get(r["plan"], 1e9), min(r["us"]))
    return {"units": "us per launch, graph-timed on one MI355X, weights rotated over 48 copies",
            "made_by": "tests/golden/nf4_plan_sweep.py",
            "shapes": [{"K": K, "N": N, "M": M, "us": dict(sorted(v.items()))} for (K, N, M), v in sorted(shapes.items())]}


if __name__ == "__main__":
    if len(sys.argv) == 3 and sys.argv[1] == "--reduce":
        lines = [json.loads(x) for x in open(sys.argv[2]) if x.startswith("{")]
    else:
        lines = sweep()
    with open(OUT, "w") as f:
        json.dump(reduce(lines), f, indent=0)
    print("wrote", OUT)
