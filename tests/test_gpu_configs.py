"""GPU parity at BASELINE configs 3 and 5 as stated, and boundary guards of the run path.

C3 (w4a8): W f32[6144][2048] ~ N(0, 0.02) and an importance vector imatrix[2048] ~ U[0.5, 2], both seeded, packed
with ork_i4a8_mm_pack_im in the uniform-grid and the NF4-codebook mode (src/npu/i4/pack.c:30-87); A int8[M][2048]
~ U[-127, 127] at M = 1 and M = 64. Bit-exact against the oracle: bscale (the caller's array and the weight's
own), the O4N1 bytes (header, bscale, the whole nibble store), the same bytes from the device context's
ork_i4a8_pack_cpu_blob, and every row of C against the exact int32 product of the oracle's codes.

C5 (Qwen3-1.7B shape, examples/bench.c:19-28, :147-188): 28 layers, hidden 2048, 16 Q / 8 KV heads of 128, SwiGLU
6144, vocab 151936, seeded N(0, 0.02) weights packed w8a8; prefill 128 seeded tokens, then 256 greedy decode steps
as replayed HIP graphs (context 384 <= 512). Checked: logits finite and tokens in range at the end; graph replay
and eager launches agree bit for bit (tokens and logits) over the first 16 steps; and, teacher-forced, the
prefill's and two decode steps' logits against the numpy restatement (oracle/qwen3_ref.py).

The restatement computes the same formulas in float32 in other orders, and every matmul input is re-quantised to
int8 per row, so a value that lands within an ulp of a rounding boundary takes the neighbouring code on one side;
such flips compound with depth. How much is measured on the restatement itself: moving every embedding value by
one ulp moves its logits by ~4.7% (4 layers) and ~10% (28 layers) of their norm at these seeds. So the reference's
own bar (examples/layer.c:79, and examples/model.c for its stacks: max |got - ref| < 5% of max |ref|) is applied
at the real widths and prompt length over 4 layers (the depth control), and at 28 layers the logit error is bounded
by three times the restatement's own one-ulp response, computed in the test, with the GPU's sampled token among
the reference's near-maxima (within 5% of max |ref|) at every step.
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

    def __init__(self, w_nk):
        self.codes, self.ws = O.pack_i8_f32(w_nk)

    def __call__(self, x):
        import qwen3_ref as R

        a_s, q = R.quant_rows(x)
        P = np.rint(q.astype(np.float64) @ self.codes.astype(np.float64)).astype(np.int32)
        return R.dequant(P, a_s, self.ws)


def _c5_model(npu, layers, P):
    """The harness model at the Qwen3-1.7B widths with `layers` layers, its weights set explicitly (linears from
    the harness's own seeded generator, norms seeded here), and the restatement holding the same weights as
    int8 codes; the f32 weights pass through one linear at a time (all of them are ~7 GB at 28 layers)."""
    import qwen3 as Q
    import qwen3_ref as R

    cfg = Q.make_cfg(max_ctx=512, max_rows=P, ffn_nf4=0, **dict(Q.QWEN3_1P7B, layers=layers))
    m = Q.Model(npu, cfg)
    rng = np.random.default_rng(SEED + (5 << 8) + 1)
    ref = R.Qwen3Ref.__new__(R.Qwen3Ref)
    ref.c, ref.lin, ref.norms = cfg, {}, {}
    for l in range(-1, cfg.layers):
        for i in ((0,) if l == -1 else Q.LINEARS):
            w = Q.gen_linear(cfg, SEED + (5 << 8), 0.02, l, i)
            assert m.set_linear(l, i, w) == 0, (l, i)
            ref.lin[(l, i)] = _ExactLinear(w)
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


def _one_ulp_response(ref, prompt, toks, refs):
    """The restatement's own sensitivity: the same weights with every embedding value moved up by one ulp, fed the
    same tokens; the L2 distance of its logits from the unperturbed ones at each step."""
    import qwen3_ref as R

    c = ref.c
    r2 = R.Qwen3Ref.__new__(R.Qwen3Ref)
    r2.c, r2.lin, r2.norms, r2.cos, r2.sin = c, ref.lin, ref.norms, ref.cos, ref.sin
    r2.emb = np.nextafter(ref.emb, np.float32(np.inf)).astype(np.float32)
    r2.kc = np.zeros_like(ref.kc)
    r2.vc = np.zeros_like(ref.vc)
    out = [_errs(r2.forward(prompt, 0), refs[0])[1]]
    for s, tok in enumerate(toks[:-1]):
        out.append(_errs(r2.forward([tok], prompt.size + s), refs[s + 1])[1])
    return out


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


@pytest.mark.timeout(600)
def test_c5_full_config(npu):
    _say("C5 qwen3-1.7b w8a8: 28 layers, prefill 128, 256 graph-replayed decode steps")
    P, S = 128, 256
    cfg, m, ref, prompt = _c5_model(npu, 28, P)
    try:
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
        _say("C5 256 steps done; tokens", toks[P:P + 8], "...")

        # teacher-forced against the restatement: prefill and the first two decode steps
        res, refs = _teacher_forced(m, ref, prompt)
        sens = _one_ulp_response(ref, prompt, [r[2] for r in res], refs)
        _say("C5 28 layers (max, L2, tok, ref gap):", res, "restatement's one-ulp response (L2):", sens)
        for (mx, l2, tok, gap), se in zip(res, sens):
            assert 0 < se < 0.5 and l2 < 3 * se and gap <= 5e-2, (res, sens)
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
