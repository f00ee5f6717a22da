"""Graph-timed launches of the LDS-ring kernel (k_tiled2) for int8, fp16 and uniform-int4 weights: every tile and K
split the planner offers above 64 rows, over the shapes its per-tile fits for those kinds were made on; writes
mma_plan_sweep.json beside this file (read by tests/test_planner.py), and prints the fits.

On one MI355X, from the repository root, with the library built:
    python3 tests/golden/mma_plan_sweep.py KIND [KIND ...] > LOG   # sweep (int8, fp16, i4u: a few minutes each)
    python3 tests/golden/mma_plan_sweep.py --reduce LOG [LOG ...]  # write the fixture from the JSON lines, fit
Every launch's result is checked before it is timed (integer kinds exactly against the oracle's GEMM, fp16 within
2e-3 of an fp64-accumulated GEMM); inexact ones are dropped. uniform int4 runs as W4A4 (ork_i4_mm_run): the same
kernels as W4A8.

The fit of each candidate (kind, tile, split or not) is the form plan.c evaluates,
    t = a + rounds * (b + c * KiB) + [ks > 1] (d + e * ks * M * N * 4 / 1e6)   us,
KiB being the A and B bytes one workgroup loads, by least squares on the relative error with non-negative terms,
over the candidate's launches that ran within twice the fastest candidate at their shape (where the planner's choice
is made; the far slower ones, e.g. 4-way splits of many rounds, would otherwise pull the fit away from it).
"""
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "mma_plan_sweep.json")
SHAPES = {(2048, 6144): (96, 128, 192, 256, 384, 512, 768, 1024),
          (2048, 2048): (96, 128, 192, 256, 384, 512, 1024, 2048),
          (4096, 4096): (96, 128, 192, 256, 384, 512, 768, 1024),
          (6144, 2048): (96, 128, 192, 256, 384, 512, 1024),
          (2048, 12288): (96, 128, 256, 512, 1024)}
BIG = ("256x256", "128x128", "128x96", "64x192", "64x64")
SMALL = ("32x64", "32x32", "16x64", "16x32")   # offered for one round of the CUs only
KINDS = {"int8": 0, "i4u": 1, "fp16": 3}       # the planner's rkind numbers
CU = 256


def abpk(kind):
    return 128 if kind == "i4u" else 64


def cands(kind, M, K, N):
    """(tile, ks) pairs the planner may pick for this shape"""
    KB = K // (128 if kind == "i4u" else 64 if kind == "int8" else 32)
    out = []
    for t in BIG + SMALL:
        bm, bn = map(int, t.split("x"))
        if kind == "i4u" and t == "256x256":
            continue                        # not offered for uniform int4 (its registers spill)
        if bm > 2 * M:
            continue
        for ks in (1, 2, 4):
            kbs = -(-KB // ks)
            if -(-KB // kbs) != ks or (ks > 1 and kbs < 4):
                continue
            wgs = -(-M // bm) * -(-(N // 16) // (bn // 16)) * ks
            if t in SMALL and wgs > CU:
                continue
            out.append((t, ks))
    return out


def sweep(kinds):
    sys.path[:0] = [os.path.join(ROOT, "ork-driver_amd"), ROOT, os.path.join(ROOT, "oracle")]
    os.environ["ORK_PLAN_DEBUG"] = "1"
    import numpy as np
    import bench
    import ork
    import oracle as O
    rng = np.random.default_rng(5)
    hip, L = bench.Hip(), ork.lib()
    with ork.Npu() as npu:
        for kind in kinds:
            for (K, N), Ms in SHAPES.items():
                Mx = max(Ms)
                if kind == "fp16":
                    A = rng.standard_normal((Mx, K)).astype(np.float16)
                    B = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
                    ws = [npu.pack_f16(B) for _ in range(48)]
                    entry, cdt = "ork_f16_mm_run", np.float32
                elif kind == "int8":
                    A = rng.integers(-127, 128, size=(Mx, K), dtype=np.int8)
                    B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
                    ws = [npu.pack_i8(B) for _ in range(48)]
                    entry, cdt = "ork_i8_mm_run", np.int32
                else:
                    A = rng.integers(-8, 8, size=(Mx, K), dtype=np.int8)
                    B = rng.integers(-8, 8, size=(K, N), dtype=np.int8)
                    ws = [npu.pack_i4(B) for _ in range(48)]
                    entry, cdt = "ork_i4_mm_run", np.int32
                assert all(ws)
                run = getattr(L, entry)
                dA, dC = L.ork_dev_alloc(npu.h, A.nbytes), L.ork_dev_alloc(npu.h, Mx * N * 4)
                assert dA and dC and L.ork_dev_upload(npu.h, dA, ork.ptr(A), A.nbytes) == 0
                full = O.gemm_f16_f64acc(A, B) if kind == "fp16" else O.gemm_i32(A, B)
                for M in Ms:
                    want = full[:M]
                    for tile, ks in cands(kind, M, K, N):
                        env = {"ORK_TILE": tile, "ORK_KSPLIT": str(ks)}
                        os.environ.update(env)
                        try:
                            name = npu.plan_name(ws[0], M)
                            L.ork_npu_set_async(npu.h, 0)
                            C = np.empty((M, N), cdt)
                            ok = run(npu.h, ws[0], M, dA, dC) == 0 and \
                                L.ork_dev_download(npu.h, ork.ptr(C), dC, C.nbytes) == 0 and \
                                (O.fp16_err(C, want) <= 2e-3 if kind == "fp16" else np.array_equal(C, want))
                            L.ork_npu_set_async(npu.h, 1)
                            t = [round(bench.measure(npu, hip, ws, M, dA, dC, 160, 16, entry)[0] * 1e3, 2)
                                 for _ in range(2)] if ok else None
                        finally:
                            for k in env:
                                os.environ.pop(k, None)
                        print(json.dumps({"kind": kind, "K": K, "N": N, "M": M, "tile": tile, "ks": ks,
                                          "plan": name, "exact": bool(ok), "us": t}), flush=True)
                for w in ws:
                    L.ork_mm_free(npu.h, w)
                L.ork_dev_free(npu.h, dA)
                L.ork_dev_free(npu.h, dC)


def features(kind, tile, ks, M, K, N):
    bm, bn = map(int, tile.split("x"))
    KB = K // (128 if kind == "i4u" else 64 if kind == "int8" else 32)
    kbs = -(-KB // ks)
    wgs = -(-M // bm) * -(-(N // 16) // (bn // 16)) * ks
    rounds = -(-wgs // CU)
    kib = (bm * abpk(kind) + bn * 64) * kbs / 1024
    part = M * N * 4 / 1e6
    return [1.0, rounds, rounds * kib, 1.0 if ks > 1 else 0.0, ks * part if ks > 1 else 0.0]


def fit(rows):
    """non-negative least squares on the relative error"""
    import numpy as np
    from scipy.optimize import nnls
    X = np.array([r[0] for r in rows]) / np.array([[r[1]] for r in rows])
    y = np.ones(len(rows))
    coef, _ = nnls(X, y)
    pred = np.array([r[0] for r in rows]) @ coef
    t = np.array([r[1] for r in rows])
    return coef, float(np.sqrt(np.mean(((pred - t) / t) ** 2)))


def reduce(lines):
    """per shape, the fastest exact time of each plan name; per candidate, its fit"""
    shapes, groups = {}, {}
    lines = [r for r in lines if r["exact"] and r["us"]]
    fastest = {}
    for r in lines:
        k = (r["kind"], r["K"], r["N"], r["M"])
        fastest[k] = min(fastest.get(k, 1e9), min(r["us"]))
    for r in lines:
        s = shapes.setdefault((r["kind"], r["K"], r["N"], r["M"]), {})
        s[r["plan"]] = min(s.get(r["plan"], 1e9), min(r["us"]))
        if min(r["us"]) > 2 * fastest[(r["kind"], r["K"], r["N"], r["M"])]:
            continue
        groups.setdefault((r["kind"], r["tile"]), []).append(
            (features(r["kind"], r["tile"], r["ks"], r["M"], r["K"], r["N"]), min(r["us"]), r["ks"]))
    fits = {}
    for (kind, tile), rows in sorted(groups.items()):
        if len(rows) < 3:
            continue
        coef, rms = fit(rows)
        fits.setdefault(kind, {})[tile] = {"coef": [round(float(x), 4) for x in coef], "rms": round(rms, 4),
                                            "n": len(rows), "ksmax": max(r[2] for r in rows)}
    return {"units": "us per launch, graph-timed on one MI355X, weights rotated over 48 copies",
            "made_by": "tests/golden/mma_plan_sweep.py",
            "fits": fits,
            "shapes": [{"kind": k, "K": K, "N": N, "M": M, "us": dict(sorted(v.items()))}
                       for (k, K, N, M), v in sorted(shapes.items())]}


if __name__ == "__main__":
    if len(sys.argv) >= 3 and sys.argv[1] == "--reduce":
        lines = [json.loads(x) for f in sys.argv[2:] for x in open(f) if x.startswith("{")]
        data = reduce(lines)
        with open(OUT, "w") as f:
            json.dump(data, f, indent=0)
        for kind, fs in data["fits"].items():
            for tile, v in fs.items():
                print(kind, tile, v)
        print("wrote", OUT)
    else:
        sweep([k for k in sys.argv[1:] if k in KINDS] or list(KINDS))
