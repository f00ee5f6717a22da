"""GPU parity at BASELINE configs 3 and 5 as stated, and boundary guards of the run path.

C3 (w4a8): W f32[6144][2048] ~ N(0, 0.02) and an importance vector imatrix[2048] ~ U[0.5, 2], both seeded, packed
with ork_i4a8_mm_pack_im in the uniform-grid and the NF4-codebook mode (src/npu/i4/pack.c:30-87); A int8[M][2048]
~ U[-127, 127] at M = 1 and M = 64. Bit-exact against the oracle: bscale (the caller's array and the weight's
own), the O4N1 bytes (header, bscale, the whole nibble store), the same bytes from the device context's
ork_i4a8_pack_cpu_blob, and every row of C against the exact int32 product of the oracle's codes.

C5 (Qwen3-1.7B shape, examples/bench.c:19-28, :147-188): 28 layers, hidden 2048, 16 Q / 8 KV heads of 128, SwiGLU
6144, vocab 151936, seeded N(0, 0.02) weights packed w8a8, and the second run with NF4 w4a8 FFN weights; prefill 128
seeded tokens, then 256 greedy decode steps as replayed HIP graphs (context 384 <= 512). Checked for both runs:
logits finite and tokens in range at the end; graph replay and eager launches agree bit for bit (tokens and logits)
over the first 16 steps; and every layer pinned on its own at the reference's bar, max |got - ref| < 0.05 * max |ref|
+ 1e-2 (examples/layer.c:84, examples/model.c:96), by teacher forcing: the harness keeps the residual rows entering
each layer (q3_set_trace), the numpy restatement (oracle/qwen3_ref.py) runs that one layer on the GPU's own input
rows (its KV cache filled from the GPU's inputs of the earlier positions), and its output is compared with the rows
the GPU passed to the next layer; the final norm and LM head likewise. For the prefill (128 rows) and two decode
steps. Comparing layer by layer keeps the bar independent of depth: end to end, the int8 re-quantisation of every
matmul input flips codes at rounding boundaries, and such flips compound over 28 layers.
"""
import os

import numpy as np
import pytest

import oracle as O
import ork

pytestmark = pytest.mark.gpu

SEED = 0x6F726B00  # 'ork\0' + (config << 8) + tensor id


def _say(*a):
    print("[case]", *a, flush=True)


# ------------------------------------------------------------------------------------------------- C3
@pytest.mark.parametrize("nf4", [0, 1])
def test_c3_full_size_bit_exact(npu, nf4):
    K, N = 2048, 6144
    _say("C3 w4a8 K=2048 N=6144 imatrix", "nf4" if nf4 else "uniform")
    W = (np.random.default_rng(SEED + (3 << 8) + 0).standard_normal((N, K)) * 0.02).astype(np.float32)
    im = np.random.default_rng(SEED + (3 << 8) + 1).uniform(0.5, 2.0, K).astype(np.float32)
    if nf4:
        os.environ["ORK_NF4"] = "1"
    try:
        w, bs = npu.pack_i4a8(W, im)
    finally:
        os.environ.pop("ORK_NF4", None)
    assert w
    bs_ref, nib_ref, codes = O.pack_i4a8(W, im, nf4=bool(nf4))
    blob_ref = O.i4a8_blob(W, im, nf4=bool(nf4))
    assert np.array_equal(bs, bs_ref)
    assert np.array_equal(ork.bscale(w, N), bs_ref)
    assert ork.lib().ork_w_quant_kind(w) == nf4
    blob = ork.dump_i4a8(w)
    assert blob.nbytes == 6316052 and np.array_equal(blob, blob_ref)   # examples/test_matmul.c:528
    assert np.array_equal(blob[20 + 4 * N:].reshape(N, K // 2), nib_ref)
    assert np.array_equal(ork.cpu_blob(K, N, W, im, nf4=nf4, ctx=npu.h), blob_ref)
    rng = np.random.default_rng(SEED + (3 << 8) + 2)
    for M in (1, 64):
        A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
        rc, C = npu.run_i8(w, A)
        assert rc == 0, npu.plan_name(w, M)
        assert np.array_equal(C, O.gemm_i32(A, codes)), (M, npu.plan_name(w, M))
    # the blob loads back into a weight that runs bit-identically
    w2 = npu.load_i4a8(K, N, blob)
    A = rng.integers(-127, 128, size=(64, K), dtype=np.int8)
    rc, C = npu.run_i8(w2, A)
    assert rc == 0 and np.array_equal(C, O.gemm_i32(A, codes))
    ork.free(w)
    ork.free(w2)


# ------------------------------------------------------------------------------------------------- C5
class _ExactLinear:
    """qwen3_ref.Linear with its int32 product computed by float64 BLAS: every operand is an integer and every
    partial sum is below 127 * 128 * 6144 < 2^53, so the float64 result is the exact integer sum (any order,
    fused or not). Only the speed differs from oracle.gemm_i32."""

    def __init__(self, w_nk, nf4=False):
        if nf4:   # ork_i4a8_mm_pack with ORK_NF4 (src/npu/i4/pack.c:26-87), as the harness packs NF4 FFN weights
            self.ws, _, self.codes = O.pack_i4a8(w_nk, nf4=True)
        else:
            self.codes, self.ws = O.pack_i8_f32(w_nk)

    def __call__(self, x):
        import qwen3_ref as R

        a_s, q = R.quant_rows(x)
        P = np.rint(q.astype(np.float64) @ self.codes.astype(np.float64)).astype(np.int32)
        return R.dequant(P, a_s, self.ws)


def _c5_model(npu, layers, P, ffn_nf4=0):
    """The harness model at the Qwen3-1.7B widths with `layers` layers, its weights set explicitly (linears from
    the harness's own seeded generator, norms seeded here), and the restatement holding the same weights as
    int8 codes (NF4 codes for the FFN weights when ffn_nf4); the f32 weights pass through one linear at a time
    (all of them are ~7 GB at 28 layers)."""
    import qwen3 as Q
    import qwen3_ref as R

    cfg = Q.make_cfg(max_ctx=512, max_rows=P, ffn_nf4=ffn_nf4, **dict(Q.QWEN3_1P7B, layers=layers))
    m = Q.Model(npu, cfg)
    rng = np.random.default_rng(SEED + (5 << 8) + 1)
    ref = R.Qwen3Ref.__new__(R.Qwen3Ref)
    ref.c, ref.lin, ref.norms = cfg, {}, {}
    for l in range(-1, cfg.layers):
        if l % 7 == 6:
            _say(f"C5 model: layer {l} of {cfg.layers} set")
        for i in ((0,) if l == -1 else Q.LINEARS):
            w = Q.gen_linear(cfg, SEED + (5 << 8), 0.02, l, i)
            assert m.set_linear(l, i, w) == 0, (l, i)
            ref.lin[(l, i)] = _ExactLinear(w, nf4=bool(ffn_nf4) and l >= 0 and i in (Q.WG, Q.WU, Q.WD))
            if l == -1:
                ref.emb = w.astype(np.float16).astype(np.float32)
            del w
        for i in ((0,) if l == -1 else range(4)):
            n = cfg.head_dim if i in (Q.N_Q, Q.N_K) else cfg.hidden
            nw = (1 + 0.02 * rng.standard_normal(n)).astype(np.float32)
            assert m.set_norm(l, i, nw) == 0
            ref.norms[(l, i)] = nw
    ref.cos, ref.sin = R.rope_tables(cfg.max_ctx, cfg.head_dim, cfg.rope_theta)
    kvd = cfg.kv_heads * cfg.head_dim
    ref.kc = np.zeros((cfg.layers, cfg.max_ctx, kvd), np.float32)
    ref.vc = np.zeros((cfg.layers, cfg.max_ctx, kvd), np.float32)
    prompt = np.random.default_rng(SEED + (5 << 8) + 2).integers(0, cfg.vocab, P).astype(np.int32)
    return cfg, m, ref, prompt


def _errs(got, want):
    return (float(np.abs(got - want).max() / np.abs(want).max()), float(np.linalg.norm(got - want) / np.linalg.norm(want)))


def _teacher_forced(m, ref, prompt, steps=2):
    """Prefill, then `steps` decode steps, each compared with the restatement fed the GPU's own tokens:
    returns ([(max-norm error, L2 error, GPU token, ref logit of that token below ref max, relative)], the
    restatement's logits at each step)."""
    P = prompt.size
    assert m.prefill(prompt) == 0
    lg, lr = m.last_logits(), ref.forward(prompt, 0)
    out, refs = [], []
    for s in range(steps + 1):
        assert np.all(np.isfinite(lg))
        tok = int(m.tokens()[-1])
        assert tok == int(np.argmax(lg)), s
        out.append(_errs(lg, lr) + (tok, float((lr.max() - lr[tok]) / np.abs(lr).max())))
        refs.append(lr)
        if s == steps:
            break
        assert m.decode(1, graph=True) == 0
        lg, lr = m.last_logits(), ref.forward([tok], P + s)
    return out, refs


@pytest.mark.timeout(300)
def test_c5_depth_control(npu):
    """Four layers at the Qwen3-1.7B widths, the stated 128-token prefill and two decode steps: the reference's
    own bar, max |got - ref| < 5% of max |ref| (examples/layer.c:79)."""
    _say("C5 depth control: 4 layers, prefill 128")
    cfg, m, ref, prompt = _c5_model(npu, 4, 128)
    try:
        res, _ = _teacher_forced(m, ref, prompt)
        _say("C5 4 layers (max, L2, tok, ref gap):", res)
        for mx, l2, tok, gap in res:
            assert mx < 5e-2 and gap <= 5e-2, res
    finally:
        m.close()


def _bar(got, want):
    """The reference's layer / model bar (examples/layer.c:84, examples/model.c:96): (max |got - want|, the bound
    0.05 * max |want| + 1e-2, pass)."""
    mx, ref = float(np.abs(got - want).max()), float(np.abs(want).max())
    bound = 0.05 * ref + 1e-2
    return mx, bound, bool(np.all(np.isfinite(got)) and ref > 1e-3 and mx < bound)


def _per_layer_pin(m, ref, prompt, steps=2):
    """Prefill, then `steps` graph-replayed decode steps; in each pass every layer's output rows against the
    restatement's layer run on the GPU's own input rows, and the logits against its head on the GPU's last rows.
    Returns the worst (layer, max error / bound) per pass; asserts the bar everywhere."""
    c = ref.c
    P = prompt.size
    ref.kc[:] = 0
    ref.vc[:] = 0
    assert m.set_trace(True) == 0
    try:
        assert m.prefill(prompt) == 0
        worst = []
        for s in range(steps + 1):
            M, pos0 = (P, 0) if s == 0 else (1, P + s - 1)
            X = [m.layer_rows(l, M) for l in range(c.layers + 1)]
            w = (None, 0.0)
            for l in range(c.layers):
                y = ref.layer(l, X[l], pos0)
                mx, bound, ok = _bar(X[l + 1], y)
                assert ok, ("pass", s, "layer", l, mx, bound)
                if mx / bound > w[1]:
                    w = (l, mx / bound)
            lg = m.last_logits()
            mx, bound, ok = _bar(lg, ref.head(X[c.layers]))
            assert ok, ("pass", s, "logits", mx, bound)
            tok = int(m.tokens()[-1])
            assert tok == int(np.argmax(lg)), s
            worst.append((s, w[0], round(w[1], 3), round(mx / bound, 3)))
            if s < steps:
                assert m.decode(1, graph=True) == 0
        return worst
    finally:
        m.set_trace(False)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("ffn_nf4", [0, 1], ids=["w8a8", "nf4_ffn"])
def test_c5_full_config(npu, ffn_nf4):
    P, S = 128, 256
    run = "w8a8 with NF4 w4a8 FFNs" if ffn_nf4 else "w8a8"
    _say(f"C5 qwen3-1.7b {run}: 28 layers, prefill 128, 256 graph-replayed decode steps")
    cfg, m, ref, prompt = _c5_model(npu, 28, P, ffn_nf4=ffn_nf4)
    try:
        assert m.decode_fused()
        # eager decode of 16 steps, then the stated run: prefill + 256 graph-replayed steps
        assert m.prefill(prompt) == 0 and m.decode(16, graph=False) == 0
        eager_toks, eager_logits = m.tokens(), m.last_logits()
        assert m.prefill(prompt) == 0
        assert m.decode(16, graph=True) == 0
        assert np.array_equal(m.tokens(), eager_toks)
        assert np.array_equal(m.last_logits(), eager_logits)          # bit-identical
        assert m.decode(S - 16, graph=True) == 0
        toks, logits = m.tokens(), m.last_logits()
        assert m.positions() == P + S and toks.size == P + S + 1
        assert np.all(np.isfinite(logits)) and toks.min() >= 0 and toks.max() < cfg.vocab
        assert np.array_equal(toks[:P], prompt) and np.array_equal(toks[:P + 17], eager_toks)
        _say(f"C5 {run}: 256 steps done; tokens", toks[P:P + 8], "...")
        # every layer on its own, teacher-forced, at the reference's bar: prefill and two decode steps
        worst = _per_layer_pin(m, ref, prompt)
        _say(f"C5 {run} per-layer pin (pass, worst layer, its error / bound, logits error / bound):", worst)
    finally:
        m.close()


# ------------------------------------------------------------------------------------------- guards
def test_int4_k_bound(npu):
    """A uniform-int4 weight widens each nibble to 16 * v in an int8 lane, so its int32 sum is 16x the true one:
    at K = 131040 the worst case (A = -128, B = -8 everywhere: 16384 per product) stays below 2^31 and is exact;
    at K = 131072 it would reach 2^31 and wrap, so such a run is refused (-1)."""
    _say("int4 K bound")
    N = 64
    for K, ok in ((131040, True), (131072, False)):
        B = np.full((K, N), -8, np.int8)
        w = npu.pack_i4(B)
        assert w
        A = np.full((1, K), -128, np.int8)
        rc, C = npu.run_i4(w, A)
        if ok:
            assert rc == 0 and np.all(C == 1024 * K), (K, C[0, :4])
        else:
            assert rc == -1
        ork.free(w)


def test_plan_overrides_need_the_debug_switch(npu):
    """The planner's test overrides act only on a context made with ORK_PLAN_DEBUG set (the session's context
    has it); on a context made without it, ORK_PLAN is ignored."""
    _say("plan override gating")
    rng = np.random.default_rng(5)
    K, N, M = 1024, 512, 128
    B = rng.integers(-127, 128, size=(K, N), dtype=np.int8)
    w = npu.pack_i8(B)
    default = npu.plan_name(w, M)
    os.environ["ORK_PLAN"] = "tiled"
    saved = os.environ.pop("ORK_PLAN_DEBUG", None)
    try:
        forced = npu.plan_name(w, M)
        with ork.Npu() as plain:
            w2 = plain.pack_i8(B)
            assert plain.plan_name(w2, M) == default
            A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
            rc, C = plain.run_i8(w2, A)
            assert rc == 0 and np.array_equal(C, O.gemm_i32(A, B))
            ork.free(w2)
    finally:
        os.environ.pop("ORK_PLAN", None)
        if saved is not None:
            os.environ["ORK_PLAN_DEBUG"] = saved
    assert forced.startswith("tiled_") and forced != default, (forced, default)
    ork.free(w)


def test_wallclock_marks(npu):
    """ork_npu_mark: stamps written in stream order (also inside a captured graph, as bench.py uses them) increase,
    and the clock runs at the rate ork_npu_wallclock_khz reports (checked against host time over a sleep)."""
    import time

    _say("wall-clock marks")
    L = ork.lib()
    khz = L.ork_npu_wallclock_khz(npu.h)
    assert khz > 0
    ts = L.ork_dev_alloc(npu.h, 24)
    assert ts
    assert L.ork_npu_mark(npu.h, ts) == 0 and L.ork_npu_sync(npu.h) == 0
    t0 = time.perf_counter()
    time.sleep(0.2)
    assert L.ork_npu_mark(npu.h, ts + 8) == 0 and L.ork_npu_sync(npu.h) == 0
    dt_host = time.perf_counter() - t0
    assert L.ork_npu_mark(npu.h, ts + 3) == -1            # misaligned
    t = np.zeros(2, np.uint64)
    assert L.ork_dev_download(npu.h, ork.ptr(t), ts, 16) == 0
    dt_dev = float(t[1] - t[0]) / (khz * 1e3)
    assert abs(dt_dev - dt_host) < 0.05 * dt_host + 0.01, (dt_dev, dt_host)
    L.ork_dev_free(npu.h, ts)


def test_ork_profile_device_rows(capfd, monkeypatch):
    """ORK_PROFILE on a device context: each (entry point, kernel plan) row carries the device time of its launches
    (HIP events around them), also for async runs read back after the sync, and a chain is one row."""
    _say("ORK_PROFILE device rows")
    L = ork.lib()
    rng = np.random.default_rng(21)
    K, N = 2048, 1024
    B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    monkeypatch.setenv("ORK_PROFILE", "1")
    c = ork.Npu()
    monkeypatch.delenv("ORK_PROFILE")
    w = c.pack_i8(B)
    A = rng.integers(-128, 128, size=(64, K), dtype=np.int8)
    for _ in range(3):
        rc, Cm = c.run_i8(w, A[:1])
        assert rc == 0 and np.array_equal(Cm, O.gemm_i32(A[:1], B))
    rc, Cm = c.run_i8(w, A)
    assert rc == 0 and np.array_equal(Cm, O.gemm_i32(A, B))
    dA = L.ork_dev_alloc(c.h, A.nbytes)
    dC = L.ork_dev_alloc(c.h, 64 * N * 4)
    assert L.ork_dev_upload(c.h, dA, ork.ptr(A), A.nbytes) == 0
    L.ork_npu_set_async(c.h, 1)
    for _ in range(5):
        assert L.ork_i8_mm_run(c.h, w, 64, dA, dC) == 0
    assert L.ork_npu_sync(c.h) == 0
    L.ork_npu_set_async(c.h, 0)
    C2 = np.zeros((2, N), np.int32)     # kept alive: the task table holds only raw pointers
    t = ork.tasks(ork.TaskI8, [(w, 1, A[:1], C2[:1]), (w, 1, A[1:2], C2[1:])])
    assert L.ork_i8_mm_run_chain(c.h, 2, t) == 0
    assert np.array_equal(C2, O.gemm_i32(A[:2], B))
    names = (c.plan_name(w, 1), c.plan_name(w, 64))
    L.ork_dev_free(c.h, dA)
    L.ork_dev_free(c.h, dC)
    ork.free(w)
    capfd.readouterr()
    c.close()
    err = capfd.readouterr().err
    rows = [l for l in err.splitlines() if l.startswith("[ork PROFILE]")]
    _say("profile rows:", rows)
    assert any(l.startswith(f"[ork PROFILE] ork_i8_mm_run {names[0]}: 3 calls,") and "device" in l for l in rows), err
    assert any(l.startswith(f"[ork PROFILE] ork_i8_mm_run {names[1]}: 6 calls,") and "over 6" in l for l in rows), err
    assert any(l.startswith("[ork PROFILE] ork_i8_mm_run_chain 2 tasks: 1 calls,") for l in rows), err
    for l in rows:
        if "device" in l:
            us = float(l.split("device ")[1].split(" us")[0])
            assert 0.5 < us < 5000, l
