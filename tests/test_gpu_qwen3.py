"""GPU parity of the Qwen3-shaped decoder harness (libork_qwen3.so) against its numpy restatement.

Each case packs the same f32 weights into the harness (through the public pack API) and into
oracle/qwen3_ref.py, prefills seeded tokens, then decodes greedily with the reference teacher-forced on
the GPU's tokens. Checked at every step:
  - the last row's logits agree to the reference's own layer bar (examples/layer.c:79: 5% of the largest
    output; int8 activation codes may flip at rounding boundaries between two float32 evaluation orders);
  - the GPU's sampled token is the first maximum of its own logits and a near-maximum of the reference's;
  - the token log holds the prompt and every sampled token.
Graph-replayed and eagerly launched decode steps must give identical tokens and bit-identical logits, and so
must the fused decode kernels (k_fgemv, k_attn_combine: 6 launches per layer) and the unfused operator sequence
(9), which do the same float operations in the same order; likewise prefill attention by blocks of rows
(k_attn_rows) and row by row.
"""
import numpy as np
import pytest

import qwen3 as Q
import qwen3_ref as R

pytestmark = pytest.mark.gpu
TOL = 5e-2


def _say(*a):
    print("[case]", *a, flush=True)


def _cfg(max_ctx=160, max_rows=80, nf4=False, **over):
    shape = dict(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=128, ffn=512, vocab=1024, rope_theta=1e6,
                 eps=1e-6)
    shape.update(over)
    return Q.make_cfg(max_ctx=max_ctx, max_rows=max_rows, ffn_nf4=nf4, **shape)


def _weights(cfg, seed, std=0.05):
    rng = np.random.default_rng(seed)
    W, Nm = {}, {}
    for l in range(cfg.layers):
        for i in Q.LINEARS:
            N, K = Q.lin_shape(cfg, l, i)
            W[(l, i)] = (rng.standard_normal((N, K)) * std).astype(np.float32)
        for i, n in ((0, cfg.hidden), (1, cfg.hidden), (2, cfg.head_dim), (3, cfg.head_dim)):
            Nm[(l, i)] = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    W[(-1, 0)] = (rng.standard_normal((cfg.vocab, cfg.hidden)) * std).astype(np.float32)
    Nm[(-1, 0)] = (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    return W, Nm


def _model(npu, cfg, W, Nm):
    m = Q.Model(npu, cfg)
    for (l, i), w in W.items():
        assert m.set_linear(l, i, w) == 0, (l, i)
    for (l, i), w in Nm.items():
        assert m.set_norm(l, i, w) == 0, (l, i)
    return m


def _check_logits(got, want, what):
    assert np.all(np.isfinite(got)), what
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err < TOL, (what, err)
    return err


def _check_sample(m, logits, ref_logits, what):
    tok = int(m.tokens()[-1])
    assert tok == int(np.argmax(logits)), what  # first maximum of the GPU's own logits
    assert ref_logits[tok] >= ref_logits.max() - TOL * np.abs(ref_logits).max(), what
    return tok


@pytest.mark.parametrize("case", [
    dict(name="gqa2-hd128", over={}, nf4=False, n=70, steps=12),
    dict(name="gqa4-hd64-nf4", over=dict(heads=8, kv_heads=2, head_dim=64), nf4=True, n=33, steps=10),
    dict(name="mha-hd128", over=dict(heads=2, kv_heads=2), nf4=False, n=1, steps=70),
    dict(name="gqa2-uniform-int4", over={}, nf4=2, n=24, steps=12),
])
def test_decoder_parity(npu, case):
    _say(case["name"])
    cfg = _cfg(nf4=case["nf4"], **case["over"])
    W, Nm = _weights(cfg, 17)
    ref = R.Qwen3Ref(cfg, W, Nm, ffn_nf4=case["nf4"])
    m = _model(npu, cfg, W, Nm)
    try:
        assert m.decode_fused()  # the decode steps below take the fused kernels
        n = case["n"]
        prompt = np.random.default_rng(23).integers(0, cfg.vocab, n).astype(np.int32)
        assert m.prefill(prompt) == 0
        lg, lr = m.last_logits(), ref.forward(prompt, 0)
        errs = [_check_logits(lg, lr, "prefill")]
        tok = _check_sample(m, lg, lr, "prefill")
        toks = [int(t) for t in prompt] + [tok]
        for s in range(case["steps"]):
            assert m.decode(1, graph=(s % 2 == 1)) == 0
            lg, lr = m.last_logits(), ref.forward([tok], n + s)
            errs.append(_check_logits(lg, lr, f"step {s}"))
            tok = _check_sample(m, lg, lr, f"step {s}")
            toks.append(tok)
        assert m.positions() == n + case["steps"]
        assert np.array_equal(m.tokens(), np.array(toks, np.int32))
        _say(case["name"], "max rel err", f"{max(errs):.2e}")
    finally:
        m.close()


def test_graph_replay_equals_eager(npu):
    _say("graph vs eager")
    cfg = _cfg(max_ctx=200)
    W, Nm = _weights(cfg, 29)
    prompt = np.random.default_rng(31).integers(0, cfg.vocab, 40).astype(np.int32)
    out = []
    for graph in (False, True):
        m = _model(npu, cfg, W, Nm)
        try:
            assert m.prefill(prompt) == 0
            assert m.decode(90, graph=graph) == 0  # crosses two 64-key chunk boundaries
            out.append((m.tokens(), m.last_logits()))
        finally:
            m.close()
    assert np.array_equal(out[0][0], out[1][0])
    assert np.array_equal(out[0][1], out[1][1])


@pytest.mark.parametrize("case", [
    dict(name="int8", over={}, nf4=0, n=20, steps=40),
    dict(name="nf4-gqa4-hd64", over=dict(heads=8, kv_heads=2, head_dim=64), nf4=1, n=9, steps=30),
    dict(name="uniform-int4-mha", over=dict(heads=2, kv_heads=2), nf4=2, n=1, steps=36),
    dict(name="qwen3-widths-2-layers", over=dict(Q.QWEN3_1P7B, layers=2, vocab=4096), nf4=1, n=12, steps=20),
])
def test_fused_decode_equals_unfused(npu, case):
    _say("fused vs unfused", case["name"])
    cfg = _cfg(nf4=case["nf4"], **case["over"])
    W, Nm = _weights(cfg, 53, std=0.05 if cfg.hidden < 1024 else 0.02)
    prompt = np.random.default_rng(59).integers(0, cfg.vocab, case["n"]).astype(np.int32)
    out = []
    for fused in (False, True):
        m = _model(npu, cfg, W, Nm)
        try:
            assert m.set_fused(fused) == 0
            assert m.decode_fused() == fused
            assert m.prefill(prompt) == 0
            lg = [m.last_logits()]  # prefill: attention by blocks of rows (fused) or row by row
            for s in range(case["steps"]):
                assert m.decode(1, graph=(s % 2 == 1)) == 0
                lg.append(m.last_logits())
            out.append((m.tokens(), np.stack(lg)))
        finally:
            m.close()
    assert np.array_equal(out[0][0], out[1][0])
    assert np.array_equal(out[0][1], out[1][1])


def test_second_prefill_restarts(npu):
    _say("second prefill")
    cfg = _cfg()
    W, Nm = _weights(cfg, 37)
    m = _model(npu, cfg, W, Nm)
    try:
        p1 = np.arange(20, dtype=np.int32)
        assert m.prefill(p1) == 0 and m.decode(5) == 0
        first = m.tokens()
        assert m.prefill(np.arange(100, 110, dtype=np.int32)) == 0 and m.decode(3) == 0
        assert m.prefill(p1) == 0 and m.decode(5) == 0
        assert np.array_equal(m.tokens(), first)
    finally:
        m.close()


def test_argument_errors(npu):
    _say("errors")
    cfg = _cfg(max_ctx=64, max_rows=32)
    W, Nm = _weights(cfg, 41)
    m = Q.Model(npu, cfg)
    try:
        assert m.prefill(np.zeros(4, np.int32)) == -2  # weights not set
        for (l, i), w in W.items():
            assert m.set_linear(l, i, w) == 0
        for (l, i), w in Nm.items():
            assert m.set_norm(l, i, w) == 0
        assert m.decode(1) == -2                                     # nothing sampled yet
        assert m.prefill(np.array([0, cfg.vocab], np.int32)) == -2   # token out of range
        assert m.prefill(np.zeros(33, np.int32)) == -2               # more rows than max_rows
        assert m.prefill(np.zeros(30, np.int32)) == 0
        assert m.decode(35) == -2                                    # 30 + 35 > max_ctx
        assert m.decode(34) == 0 and m.positions() == 64
        assert m.decode(1) == -2
    finally:
        m.close()


def test_qwen3_width_two_layers(npu):
    """Qwen3-1.7B widths (hidden 2048, 16/8 heads, head_dim 128, FFN 6144, vocab 151936), two layers."""
    _say("qwen3 widths, 2 layers")
    cfg = Q.make_cfg(max_ctx=64, max_rows=16, **dict(Q.QWEN3_1P7B, layers=2))
    W, Nm = _weights(cfg, 43, std=0.02)
    ref = R.Qwen3Ref(cfg, W, Nm)
    m = _model(npu, cfg, W, Nm)
    try:
        prompt = np.random.default_rng(47).integers(0, cfg.vocab, 16).astype(np.int32)
        assert m.prefill(prompt) == 0
        lg, lr = m.last_logits(), ref.forward(prompt, 0)
        _check_logits(lg, lr, "prefill")
        tok = _check_sample(m, lg, lr, "prefill")
        for s in range(3):
            assert m.decode(1, graph=True) == 0
            lg, lr = m.last_logits(), ref.forward([tok], 16 + s)
            _check_logits(lg, lr, f"step {s}")
            tok = _check_sample(m, lg, lr, f"step {s}")
    finally:
        m.close()
