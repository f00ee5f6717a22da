"""CPU tests of the decoder harness: the numpy restatement's pins and the harness library's host side.

The restatement (oracle/qwen3_ref.py) is pinned operator by operator against closed forms and
independent formulations (complex rotation for RoPE, expit for SiLU, a float64 softmax), and the whole
layer stack against a float64 brute-force evaluation written with different primitives (repeat-expanded
GQA heads, int64 matmuls). The harness library is checked for its exports, its weight generator and
its argument checks without a GPU.
"""
import ctypes as C

import numpy as np
import pytest
from scipy.special import expit

import oracle as O
import qwen3 as Q
import qwen3_ref as R


def test_rmsnorm_closed_form():
    for c in (3.0, -0.25, 1e-3):
        x = np.full((2, 64), c, np.float32)
        w = np.linspace(0.5, 1.5, 64).astype(np.float32)
        got = R.rmsnorm(x, w, 1e-6)
        want = c / np.sqrt(c * c + 1e-6) * w.astype(np.float64)
        np.testing.assert_allclose(got, np.broadcast_to(want, got.shape), rtol=1e-6)


def test_rope_properties():
    HD = 128
    cos, sin = R.rope_tables(64, HD, 1e6)
    rng = np.random.default_rng(1)
    q = rng.standard_normal(HD).astype(np.float32)
    k = rng.standard_normal(HD).astype(np.float32)
    np.testing.assert_array_equal(R.rope(q, cos[0], sin[0]), q)  # position 0: identity
    # independent formulation: halves as the real and imaginary parts of HD/2 complex numbers
    for p in (1, 7, 63):
        z = (q[:HD // 2] + 1j * q[HD // 2:]).astype(np.complex128)
        ang = p * np.power(1e6, -2.0 * np.arange(HD // 2) / HD)
        zr = z * np.exp(1j * ang)
        got = R.rope(q, cos[p], sin[p])
        np.testing.assert_allclose(got, np.concatenate([zr.real, zr.imag]), atol=2e-6)
    # relative position: <rope(q, a), rope(k, b)> depends on a - b only
    d1 = R.rope(q, cos[10], sin[10]) @ R.rope(k, cos[3], sin[3])
    d2 = R.rope(q, cos[40], sin[40]) @ R.rope(k, cos[33], sin[33])
    assert abs(d1 - d2) < 1e-4 * (1 + abs(d1))


def test_attend_closed_forms():
    rng = np.random.default_rng(2)
    K = rng.standard_normal((1, 64)).astype(np.float32)
    V = rng.standard_normal((1, 64)).astype(np.float32)
    np.testing.assert_allclose(R.attend(rng.standard_normal(64).astype(np.float32), K, V, 0.125), V[0], rtol=1e-6)
    K = rng.standard_normal((9, 64)).astype(np.float32)
    V = rng.standard_normal((9, 64)).astype(np.float32)
    np.testing.assert_allclose(R.attend(np.zeros(64, np.float32), K, V, 0.125), V.mean(0), rtol=1e-5, atol=1e-6)
    q = rng.standard_normal(64).astype(np.float32)
    s = (K.astype(np.float64) @ q) * 0.125
    p = np.exp(s - s.max())
    np.testing.assert_allclose(R.attend(q, K, V, 0.125), (p / p.sum()) @ V, rtol=1e-5, atol=1e-6)


def test_silu_mul():
    g = np.array([0.0, -30.0, 30.0, 1.5, -0.7], np.float32)
    u = np.array([2.0, 1.0, 3.0, -1.0, 0.5], np.float32)
    got = R.silu_mul(g, u)
    np.testing.assert_allclose(got, g * expit(g.astype(np.float64)) * u, rtol=1e-6, atol=1e-12)
    assert got[0] == 0.0


def test_greedy_first_maximum():
    assert R.greedy(np.array([1.0, 3.0, 3.0, 2.0], np.float32)) == 1


def _small_cfg(**over):
    shape = dict(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=384, vocab=512, rope_theta=1e4,
                 eps=1e-6)
    shape.update(over)
    return Q.make_cfg(max_ctx=96, max_rows=32, **shape)


def _weights(cfg, seed):
    rng = np.random.default_rng(seed)
    W, Nm = {}, {}
    for l in range(cfg.layers):
        for i in Q.LINEARS:
            N, K = Q.lin_shape(cfg, l, i)
            W[(l, i)] = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
        Nm[(l, 0)] = (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
        Nm[(l, 1)] = (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
        Nm[(l, 2)] = (1 + 0.1 * rng.standard_normal(cfg.head_dim)).astype(np.float32)
        Nm[(l, 3)] = (1 + 0.1 * rng.standard_normal(cfg.head_dim)).astype(np.float32)
    W[(-1, 0)] = (rng.standard_normal((cfg.vocab, cfg.hidden)) * 0.05).astype(np.float32)
    Nm[(-1, 0)] = (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    return W, Nm


def _brute(cfg, W, Nm, tokens):
    """float64 evaluation with its own primitives: kv heads expanded by np.repeat, int64 matmuls,
    complex RoPE, full softmax; int8 codes from the same per-channel / per-row rules."""
    NH, NKV, HD, eps = cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.eps
    G = NH // NKV

    def lin(x, w_nk):
        ws = np.maximum(np.abs(w_nk).max(1), 1e-9) / 127.0
        codes = np.clip(np.rint(w_nk / ws[:, None]), -127, 127).astype(np.int64)
        mx = np.abs(x).max(1)
        a_s = np.where(mx > 0, mx / 127.0, 1.0)
        a = np.clip(np.rint(x / a_s[:, None]), -127, 127).astype(np.int64)
        return (a @ codes.T) * a_s[:, None] * ws[None, :]

    def norm(x, w):
        return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w

    def rot(v, pos):
        z = v[..., :HD // 2] + 1j * v[..., HD // 2:]
        z = z * np.exp(1j * pos * np.power(cfg.rope_theta, -2.0 * np.arange(HD // 2) / HD))
        return np.concatenate([z.real, z.imag], -1)

    T = len(tokens)
    x = W[(-1, 0)].astype(np.float16).astype(np.float64)[tokens]
    pos = np.arange(T)[:, None, None]
    for l in range(cfg.layers):
        h = norm(x, Nm[(l, 0)])
        q = rot(norm(lin(h, W[(l, 0)]).reshape(T, NH, HD), Nm[(l, 2)]), pos)
        k = rot(norm(lin(h, W[(l, 1)]).reshape(T, NKV, HD), Nm[(l, 3)]), pos)
        v = lin(h, W[(l, 2)]).reshape(T, NKV, HD)
        k, v = np.repeat(k, G, axis=1), np.repeat(v, G, axis=1)
        s = np.einsum("thd,jhd->htj", q, k) / np.sqrt(HD)
        s = np.where(np.tril(np.ones((T, T), bool))[None], s, -np.inf)
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        att = np.einsum("htj,jhd->thd", p, v).reshape(T, NH * HD)
        x = x + lin(att, W[(l, 3)])
        h2 = norm(x, Nm[(l, 1)])
        g, u = lin(h2, W[(l, 4)]), lin(h2, W[(l, 5)])
        x = x + lin(g * expit(g) * u, W[(l, 6)])
    return lin(norm(x, Nm[(-1, 0)])[-1:], W[(-1, 0)])[0]


@pytest.mark.parametrize("kv_heads", [2, 1])
def test_reference_matches_float64_brute_force(kv_heads):
    cfg = _small_cfg(kv_heads=kv_heads)
    W, Nm = _weights(cfg, 5 + kv_heads)
    tokens = np.random.default_rng(3).integers(0, cfg.vocab, 20)
    ref = R.Qwen3Ref(cfg, W, Nm)
    got = ref.forward(tokens[:13], 0)
    got = ref.forward(tokens[13:], 13)  # prefill then a second batch over the cache
    want = _brute(cfg, W, Nm, tokens)
    # int8 activation codes can flip at rounding boundaries between float32 and float64: the bar is the
    # reference's own layer check (examples/layer.c:79, 5% of the largest output)
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err < 5e-2, err
    # a planted mistake (keys shifted by one position against their values) must fail it by far
    if kv_heads == 2:
        bad = R.Qwen3Ref(cfg, W, Nm)
        orig = R.attend
        try:
            def shuffled(q, K, V, scale, _o=orig):
                return _o(q, np.roll(K, 1, axis=0), V, scale)
            R.attend = shuffled
            wrong = bad.forward(tokens, 0)
        finally:
            R.attend = orig
        assert np.abs(wrong - want).max() / np.abs(want).max() > 0.3


def test_harness_library_exports():
    L = Q.lib()
    for name in Q.API:
        assert hasattr(L, name), name


def test_generator_is_seeded_normal():
    cfg = Q.make_cfg(max_ctx=64, max_rows=8, **Q.QWEN3_1P7B)
    a = Q.gen_linear(cfg, 11, 0.02, 3, Q.WG)
    b = Q.gen_linear(cfg, 11, 0.02, 3, Q.WG)
    c = Q.gen_linear(cfg, 11, 0.02, 3, Q.WU)
    d = Q.gen_linear(cfg, 12, 0.02, 3, Q.WG)
    assert a.shape == (6144, 2048)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, c) and not np.array_equal(a, d)
    assert abs(a.mean()) < 1e-4 and abs(a.std() - 0.02) < 1e-4
    # Gaussian tails: P(|z| > 3 sigma) = 0.27%
    assert 0.002 < np.mean(np.abs(a) > 0.06) < 0.0034
    assert abs(np.corrcoef(a.ravel()[:-1:2], a.ravel()[1::2])[0, 1]) < 2e-3


def test_create_needs_a_device_context():
    import ork

    ctx = ork.Npu(offline="gfx950")
    try:
        cfg = _small_cfg()
        assert not Q.lib().q3_create(ctx.h, C.byref(cfg))
        bad = _small_cfg(head_dim=96)  # not a multiple of 64
        assert not Q.lib().q3_create(ctx.h, C.byref(bad))
    finally:
        ctx.close()
