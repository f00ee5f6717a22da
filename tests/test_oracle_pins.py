"""Pins the oracle's quantisers and codec where no golden vector of the reference covers them (CPU only).

Each check is something the mathematics or the reference's own tests fix independently of the
oracle's code, chosen so that a plausible slip fails it:
- int8 per-channel quant (src/npu.c:854-865, src/npu/i8/pack.c:442-453): exact round-half-even ties,
  the dequantisation error bound, the 1e-9 floor, max|q| = 127, and the reference's own RMS gate
  (examples/test_matmul.c:280-306)
- NF4 (src/npu/i4/quant.c:70-90, src/npu/i4/pack.c:57): the int8 codebook, nearest-level by brute
  force, the exact float32 ties t == 0.5f (the upper level, :84 and :138) with the neighbours either
  side, the reference's accuracy gate (examples/test_matmul.c:402-427), and for stochastic rounding the
  bracket, the hit frequency P(hi) = t and the draw stream (which elements draw, channel order)
- imatrix clip search (src/npu/i4/quant.c:26, :130-161): the chosen scale is on the clip grid and is
  the grid's minimum of the weighted error (brute force in float64), each candidate's error equals an
  independent numpy float32 sequential sum bit for bit, exact ties keep the first candidate, the
  NULL path is absmax/7 exactly (examples/test_matmul.c:467-471), and the reference's importance gate
  (examples/test_matmul.c:430-500)
- O4N1 (src/npu/i4/pack.c:91-103, :115-122; src/npu/internal.h:584, :597): header bytes, section
  offsets, the C3 size the reference's test expects (examples/test_matmul.c:528), decode round trip,
  and qerr = sqrt(sum imp (w - q)^2 / sum imp w^2) recomputed from the decoded blob
"""
import numpy as np
import pytest

import oracle as O

# int8 codebook of the NF4 levels, rint(level * 127) (src/npu.c:888-892 with src/npu/i4/pack.c:57)
NF4_LUT = [-127, -88, -67, -50, -36, -23, -12, 0, 10, 20, 31, 43, 56, 71, 92, 127]
# the 16 normalised NF4 levels, transcribed from src/npu.c:888-892 (checked against the codebook below)
NF4_LEVELS = np.array([-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
                       -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
                       0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
                       0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0])
CLIP_GRID = [1.0, 0.92, 0.85, 0.78, 0.70, 0.62, 0.55]  # src/npu/i4/quant.c:26


# ------------------------------------------------------------------------------------------- int8
def test_i8_quant_exact_ties_and_floor():
    K, N = 64, 32
    W = np.zeros((N, K), np.float32)
    # channel 1: absmax 127 -> inv = 1.0 exactly, so w itself is rounded: half-even at every tie
    W[1, :8] = [127.0, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5]
    # channel 2: absmax 254 -> inv = 0.5 exactly
    W[2, :3] = [254.0, 5.0, 7.0]
    # channel 3: a value that rounds past 127 cannot occur; the clamp still bounds -127
    W[3, :2] = [-127.0, 126.5]
    codes, bs = O.pack_i8_f32(W)
    assert list(codes[:8, 1]) == [127, 2, 4, -2, -4, 0, 0, 2]
    assert list(codes[:3, 2]) == [127, 2, 4]
    assert list(codes[:2, 3]) == [-127, 126]
    # the all-zero channel: absmax floored at 1e-9, codes 0, bscale = 1e-9/127 in float32
    assert np.all(codes[:, 0] == 0) and bs[0] == np.float32(np.float32(1e-9) / np.float32(127.0))
    assert bs[1] == np.float32(1.0) and bs[2] == np.float32(2.0)


def test_i8_quant_bounds_and_gate():
    rng = np.random.default_rng(5)
    N, K = 96, 512
    W = (rng.standard_normal((N, K)) * rng.uniform(0.001, 3.0, (N, 1))).astype(np.float32)
    codes, bs = O.pack_i8_f32(W)
    q = codes.T.astype(np.float64)                      # [N][K]
    mx = np.max(np.abs(W), axis=1).astype(np.float64)
    assert np.all(np.max(np.abs(codes), axis=0) == 127)  # every channel reaches the grid end
    assert np.allclose(bs.astype(np.float64), mx / 127.0, rtol=1e-6)
    err = np.abs(q * bs[:, None].astype(np.float64) - W)
    assert np.all(err <= 0.5 * bs[:, None] * (1 + 1e-5) + 1e-12)  # nearest grid point, per channel

    # examples/test_matmul.c:280-306: weights and activations (rnd()-128)/64 from the test's LCG,
    # per-row int8 activations, dequantised int32 GEMM within 3% RMS of the fp64 product
    st = O.LCGState(12345)
    M, K, N = 8, 2048, 512
    Bf = ((O.gen_tm_rnd(st, N * K).astype(np.int32) - 128) / 64.0).astype(np.float32).reshape(N, K)
    Af = ((O.gen_tm_rnd(st, M * K).astype(np.int32) - 128) / 64.0).astype(np.float32).reshape(M, K)
    codes, bs = O.pack_i8_f32(Bf)
    amx = np.maximum(np.max(np.abs(Af), axis=1), np.float32(1e-9)).astype(np.float32)
    Ai = np.clip(np.rint(Af * (np.float32(127.0) / amx)[:, None]), -127, 127).astype(np.int8)
    C = O.gemm_i32(Ai, codes)
    got = (amx / np.float32(127.0))[:, None].astype(np.float64) * bs[None, :] * C
    ref = Af.astype(np.float64) @ Bf.astype(np.float64).T
    rms = np.sqrt(np.mean((got - ref) ** 2)) / (np.sqrt(np.mean(ref ** 2)) + 1e-9)
    assert rms < 0.03


# -------------------------------------------------------------------------------------------- NF4
def test_nf4_codebook():
    assert list(O.nf4_lut()) == NF4_LUT


def test_nf4_nearest_level_brute_force():
    rng = np.random.default_rng(21)
    K, N = 1024, 32
    W = rng.uniform(-1.0, 1.0, (N, K)).astype(np.float32)
    W[:, 0] = 1.0  # absmax 1 -> normalised weight == w, scale == 1/127
    bs, nib, codes = O.pack_i4a8(W, nf4=True)
    assert np.all(bs == np.float32(np.float32(1.0) / np.float32(127.0)))
    # idx recovered from the nibble store (low nibble = even k)
    idx = np.empty((N, K), np.int64)
    idx[:, 0::2] = nib & 0xF
    idx[:, 1::2] = nib >> 4
    lut = np.array(NF4_LUT)
    assert np.array_equal(lut[idx], codes.T.astype(np.int64))
    # brute force over the 16 levels in float64: the stored index is a nearest level (float32
    # near-ties excepted)
    L = NF4_LEVELS
    assert np.array_equal(np.rint(L * 127).astype(int), lut)
    d = np.abs(W.astype(np.float64)[:, :, None] - L[None, None, :])
    chosen = d[np.arange(N)[:, None], np.arange(K)[None, :], idx]
    assert np.all(chosen <= d.min(axis=2) + 1e-6)
    # a weight exactly on a level selects that level (the exact float32 midpoints: the next test)
    Wl = np.zeros((32, 64), np.float32)  # N % 32 == 0 (pack gate); rows 1.. are all-zero channels
    Wl[0, 0:16] = L.astype(np.float32)
    _, nibl, _ = O.pack_i4a8(Wl, nf4=True)
    il = np.empty(64, np.int64)
    il[0::2] = nibl[0] & 0xF
    il[1::2] = nibl[0] >> 4
    assert list(il[0:16]) == list(range(16))


def _nf4_tie_points():
    """For every adjacent NF4 level pair (lo, hi = lo + 1): float32 normalised weights wn strictly inside the
    bracket at which the reference's float32 position t = (wn - L[lo]) / (L[hi] - L[lo])
    (src/npu/i4/quant.c:80-81, one float32 subtraction then one float32 division) is exactly 0.5f, and the
    nearest weights on either side where t < 0.5f and t > 0.5f. Found by walking float32 neighbours of the
    real midpoint; every step below is one IEEE binary32 operation (numpy float32 scalars)."""
    L32 = NF4_LEVELS.astype(np.float32)
    pts = []
    for lo in range(15):
        hi = lo + 1
        d = np.float32(L32[hi] - L32[lo])
        mid = np.float32((NF4_LEVELS[lo] + NF4_LEVELS[hi]) / 2)
        ties, below, above = [], None, None
        x = mid
        for _ in range(64):                     # walk down to the last t < 0.5
            x = np.nextafter(x, np.float32(-2), dtype=np.float32)
        for _ in range(128):
            t = np.float32(np.float32(x - L32[lo]) / d)
            if t == np.float32(0.5):
                ties.append(x)
            elif t < np.float32(0.5):
                below = x
            elif above is None:
                above = x
            x = np.nextafter(x, np.float32(2), dtype=np.float32)
        pts.append((lo, hi, ties, below, above))
    return pts


def test_nf4_exact_tie_takes_the_upper_level():
    """src/npu/i4/quant.c:84 (and :138 in the clip search's error): idx = (t >= 0.5f) ? hi : lo. Where t is
    exactly 0.5f the upper level wins; a flipped rule (t > 0.5f) or a nearest-level choice in real
    arithmetic picks lo at some of these points. Checked on the oracle's packer, on its clip-search error
    (the dequantised values it returns), and on the product's own quantiser (offline cpu_blob)."""
    import ork

    pts = _nf4_tie_points()
    assert sum(len(t) for _, _, t, _, _ in pts) >= 5    # exact float32 ties exist for 6 of the 15 level pairs
    vals, want = [1.0], [15]                           # absmax 1 -> inv = 1.0f, so wn == w exactly
    for lo, hi, ties, below, above in pts:
        for x in ties:
            vals.append(float(x)); want.append(hi)
        vals.append(float(below)); want.append(lo)
        vals.append(float(above)); want.append(hi)
    K = (len(vals) + 31) // 32 * 32
    W = np.zeros((32, K), np.float32)
    W[0, :len(vals)] = vals
    W[0, len(vals):] = 0.0                             # exactly on level 7
    want += [7] * (K - len(vals))
    _, nib, _ = O.pack_i4a8(W, nf4=True)
    idx = np.empty(K, np.int64)
    idx[0::2] = nib[0] & 0xF
    idx[1::2] = nib[0] >> 4
    assert list(idx) == want
    # the clip search's error path: dq[k] = (float)lut[idx] * (absmax / 127.0f), absmax 1
    dq = np.zeros(K, np.float32)
    O.lib().oracle_wq_err_chan(O._ptr(W[0]), K, 1.0, 1, None, O._ptr(dq))
    lut32 = np.array(NF4_LUT, np.float32) * np.float32(np.float32(1.0) / np.float32(127.0))
    assert np.array_equal(dq, lut32[want])
    # the product's quantiser (its own quant.c, on an offline context) makes the same choice
    with ork.Npu(offline="gfx950") as off:
        blob = ork.cpu_blob(K, 32, W, None, nf4=1, ctx=off.h)
    assert np.array_equal(blob[20 + 4 * 32:20 + 4 * 32 + K // 2], nib[0])


def _wq_err32(fr, absmax, nf4, im):
    """The clip search's weighted error (src/npu/i4/quant.c:130-149) restated in numpy float32, op by op:
    the per-element dequantisation, d = w - dq, the term (im * d) * d, and a SEQUENTIAL float32 sum from
    0.0f (np.add.accumulate on float32 is sequential), no fused multiply-add."""
    f = np.float32
    fr = fr.astype(np.float32)
    if nf4:
        sc = f(f(absmax) / f(127.0))
        inv = f(f(1.0) / f(absmax)) if absmax > 0 else f(0.0)
        wn = np.clip((fr * inv).astype(np.float32), f(-1.0), f(1.0))
        L32 = NF4_LEVELS.astype(np.float32)
        hi = np.minimum(np.searchsorted(L32, wn, side="left"), 15)   # first level >= wn
        lo = np.maximum(hi - 1, 0)
        with np.errstate(invalid="ignore", divide="ignore"):
            t = ((wn - L32[lo]).astype(np.float32) / (L32[hi] - L32[lo]).astype(np.float32)).astype(np.float32)
        idx = np.where(lo == hi, hi, np.where(t >= f(0.5), hi, lo))
        dq = (np.array(NF4_LUT, np.float32)[idx] * sc).astype(np.float32)
    else:
        scale = f(f(absmax) / f(7.0))
        inv = f(f(1.0) / scale) if scale > 0 else f(0.0)
        q = np.clip(np.rint((fr * inv).astype(np.float32)), -7, 7).astype(np.float32)
        dq = (q * scale).astype(np.float32)
    d = (fr - dq).astype(np.float32)
    w = im.astype(np.float32) if im is not None else np.ones_like(fr)
    terms = ((w * d).astype(np.float32) * d).astype(np.float32)
    return np.add.accumulate(np.concatenate([[f(0.0)], terms]).astype(np.float32), dtype=np.float32)[-1]


@pytest.mark.parametrize("nf4", [0, 1])
def test_imatrix_error_is_float32_sequential(nf4):
    """The clip search's error value is the float32 sequential sum, bit for bit, for every grid candidate of
    random channels (a float64 or pairwise accumulation, or a fused multiply-add, changes the low bits of
    most of these sums), and the chosen scale is the FIRST strict minimum of those float32 values
    (src/npu/i4/quant.c:155-158) -- also where every candidate's error is exactly equal (a channel that
    is zero wherever the importance is non-zero), where `<=` would pick the last candidate."""
    rng = np.random.default_rng(60 + nf4)
    N, K = 48, 2048
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    W[:, ::53] *= 6
    im = rng.uniform(0.5, 2.0, K).astype(np.float32)
    im_sparse = np.zeros(K, np.float32)
    im_sparse[7] = 1.0
    Wt = W.copy()
    Wt[:8, 7] = 0.0        # channels 0..7: zero wherever im_sparse is non-zero -> every candidate's error is 0
    dq = np.zeros(K, np.float32)
    L = O.lib()
    for n in range(N):
        fr = np.ascontiguousarray(W[n])
        mx = np.float32(max(np.float32(1e-9), np.max(np.abs(fr))))
        errs = []
        for g in CLIP_GRID:
            cand = np.float32(mx * np.float32(g))
            e = L.oracle_wq_err_chan(O._ptr(fr), K, float(cand), nf4, O._ptr(im), O._ptr(dq))
            assert np.float32(e) == _wq_err32(fr, cand, nf4, im), (n, g)
            errs.append(np.float32(e))
        best = 0
        for g in range(1, 7):
            if errs[g] < errs[best]:
                best = g
        got = L.oracle_wq_best_absmax(O._ptr(fr), K, float(mx), nf4, O._ptr(im), O._ptr(dq))
        assert np.float32(got) == np.float32(mx * np.float32(CLIP_GRID[best])), n
    for n in range(8):
        fr = np.ascontiguousarray(Wt[n])
        mx = np.float32(np.max(np.abs(fr)))
        assert _wq_err32(fr, mx, nf4, im_sparse) == 0.0
        got = L.oracle_wq_best_absmax(O._ptr(fr), K, float(mx), nf4, O._ptr(im_sparse), O._ptr(dq))
        assert np.float32(got) == mx, n    # the first candidate (raw absmax) survives an exact tie
    # the same pack through the product's quantiser (offline cpu_blob) and the oracle: byte-identical
    import ork
    with ork.Npu(offline="gfx950") as off:
        for wv, iv in ((W, im), (Wt, im_sparse)):
            blob = ork.cpu_blob(K, N, wv, iv, nf4=nf4, ctx=off.h)
            assert np.array_equal(blob, O.i4a8_blob(wv, iv, nf4=bool(nf4)))


def _xs32_stream(seed, n):
    """xorshift32 (src/npu/internal.h:589): x ^= x << 13; x ^= x >> 17; x ^= x << 5, on uint32."""
    out = np.empty(n, np.uint32)
    x = np.uint32(seed)
    for i in range(n):
        x ^= np.uint32((int(x) << 13) & 0xFFFFFFFF)
        x ^= np.uint32(int(x) >> 17)
        x ^= np.uint32((int(x) << 5) & 0xFFFFFFFF)
        out[i] = x
    return out


def test_nf4_stochastic_rounding_draw_stream():
    """NF4 stochastic rounding (src/npu/i4/quant.c:78-84, seed src/npu/i4/pack.c:32): one xorshift32 draw
    u = (x >> 8) / 2^24 per element INSIDE a bracket (wn == -1 has lo == hi and draws nothing), idx = hi iff
    t > u, one stream running across the channels in order. The generator itself is pinned where the
    reference builds (its uniform-int4 SR through oracle/_ref draws the same stream); the draw-skip and
    cross-channel order are the reference's source read as text: a channel that starts with absmax-scaled
    -1 weights must shift no draws (while wn == +1 sits in the bracket (L[14], L[15]] and draws one), and
    channel 1 must continue channel 0's stream."""
    N, K = 32, 64
    L32 = NF4_LEVELS.astype(np.float32)
    W = np.zeros((N, K), np.float32)
    rng = np.random.default_rng(8)
    for n in range(2):
        W[n] = L32[7] + np.float32(0.5) * rng.uniform(0.05, 0.95, K).astype(np.float32) * (L32[8] - L32[7])
        W[n, 0] = 1.0                       # absmax 1: wn = +1, bracket (14, 15], t = 1 > u: one draw, idx 15
        W[n, 1:5] = -1.0                    # wn == -1: lo == hi == 0, no draw
    _, nib, _ = O.pack_i4a8(W, nf4=True, sr=True)
    u = (_xs32_stream(0x2545F491, 2 * K) >> np.uint32(8)).astype(np.float32) * np.float32(1.0 / 16777216.0)
    j = 0
    for n in range(2):
        idx = np.empty(K, np.int64)
        idx[0::2] = nib[n] & 0xF
        idx[1::2] = nib[n] >> 4
        assert idx[0] == 15 and list(idx[1:5]) == [0] * 4
        j += 1                              # the draw of element 0; elements 1..4 draw nothing
        for k in range(5, K):
            t = np.float32(np.float32(W[n, k] - L32[7]) / np.float32(L32[8] - L32[7]))
            assert idx[k] == (8 if t > u[j] else 7), (n, k)
            j += 1
    if O.ref_available():
        # the generator: the reference's own uniform SR consumes the same stream, one draw per element
        fr = np.full(K, 0.3, np.float32)
        seed = np.array([0x2545F491], np.uint32)
        nibr = np.zeros(K // 2, np.uint8)
        qf = np.zeros(K, np.float32)
        O.ref().ref_i4_quant_chan(O._ptr(fr), K, 1.0, 1, O._ptr(seed), O._ptr(nibr), O._ptr(qf))
        assert int(seed[0]) == int(_xs32_stream(0x2545F491, K)[-1])
        assert np.array_equal(qf, np.floor(fr * np.float32(1.0) + u[:K]).astype(np.float32))


def test_nf4_accuracy_gate():
    """examples/test_matmul.c:402-427: on N(0,1) weights NF4 reconstructs better than uniform int4."""
    rng = np.random.default_rng(3)
    K, N = 4096, 256
    W = rng.standard_normal((N, K)).astype(np.float32)
    bsu, _, cu = O.pack_i4a8(W, nf4=False)
    bsn, _, cn = O.pack_i4a8(W, nf4=True)
    eu = np.sqrt(np.mean((cu.T * bsu[:, None].astype(np.float64) - W) ** 2))
    en = np.sqrt(np.mean((cn.T * bsn[:, None].astype(np.float64) - W) ** 2))
    assert en < eu


def test_nf4_stochastic_rounding_frequency():
    """SR picks hi with probability t = (wn - L[lo]) / (L[hi] - L[lo]) and never leaves the bracket."""
    K = 8192
    L7, L8 = 0.0, 0.07958029955625534
    for t in (0.25, 0.7):
        W = np.full((32, K), np.float32(L7 + t * (L8 - L7)), np.float32)
        W[:, 0] = 1.0
        _, nib, _ = O.pack_i4a8(W, nf4=True, sr=True)
        idx = np.concatenate([(nib & 0xF)[:, 1:], (nib >> 4)], axis=1)
        assert set(np.unique(idx)) <= {7, 8}
        frac = float(np.mean(idx == 8))
        assert abs(frac - t) < 0.01, (t, frac)


# ---------------------------------------------------------------------------------- imatrix search
def _werr64(w, s, im, nf4):
    if nf4:
        wn = np.clip(w / (s * 127.0), -1, 1)
        # the level is chosen on the normalised levels, the value comes from the int8 codebook
        idx = np.argmin(np.abs(wn[:, None] - NF4_LEVELS[None, :]), axis=1)
        dq = np.array(NF4_LUT, np.float64)[idx] * s
    else:
        dq = np.clip(np.rint(w / s), -7, 7) * s
    return float(np.sum(im * (w - dq) ** 2))


@pytest.mark.parametrize("nf4", [False, True])
def test_imatrix_clip_is_grid_argmin(nf4):
    rng = np.random.default_rng(40 + nf4)
    N, K = 64, 256
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    W[:, ::37] *= 8  # outliers make clipping pay on some channels
    im = rng.uniform(0.5, 2.0, K).astype(np.float32)
    bs, _, _ = O.pack_i4a8(W, im, nf4=nf4)
    div = 127.0 if nf4 else 7.0
    mx = np.max(np.abs(W), axis=1).astype(np.float64)
    picked = []
    for n in range(N):
        r = bs[n] * div / mx[n]
        g = int(np.argmin([abs(r - x) for x in CLIP_GRID]))
        assert abs(r - CLIP_GRID[g]) < 1e-5, (n, r)
        picked.append(g)
        errs = [_werr64(W[n].astype(np.float64), mx[n] * x / div, im.astype(np.float64), nf4) for x in CLIP_GRID]
        assert errs[g] <= min(errs) * (1 + 1e-4), (n, g, errs)
    assert len(set(picked)) > 1  # the search is exercised, not stuck at absmax


def test_imatrix_null_path_and_importance_gate():
    """examples/test_matmul.c:430-500: with imatrix NULL, bscale == absmax/7 exactly; with important
    mid-range columns and unimportant outliers the imatrix pack has the lower weighted error."""
    rng = np.random.default_rng(9)
    N, K = 128, 2048
    im = np.where(np.arange(K) < 64, 50.0, 0.01).astype(np.float32)
    W = (rng.integers(0, 256, (N, K)) - 128).astype(np.float32) / 4096.0
    W[:, :64] = (rng.integers(0, 256, (N, 64)) - 128).astype(np.float32) / 256.0
    out = np.arange(K) % 401 == 0
    out[:64] = False
    W[:, out] = (rng.choice([-1.0, 1.0], (N, int(out.sum()))) * (6.0 + rng.integers(0, 8, (N, int(out.sum())))))
    W = W.astype(np.float32)
    bs0, _, _ = O.pack_i4a8(W, None)
    mx = np.maximum(np.max(np.abs(W), axis=1), np.float32(1e-9)).astype(np.float32)
    assert np.array_equal(bs0, (mx / np.float32(7.0)).astype(np.float32))
    bs1, _, _ = O.pack_i4a8(W, im)
    e0 = sum(_werr64(W[n].astype(np.float64), float(bs0[n]), im.astype(np.float64), False) for n in range(N))
    e1 = sum(_werr64(W[n].astype(np.float64), float(bs1[n]), im.astype(np.float64), False) for n in range(N))
    assert e1 < e0


# ------------------------------------------------------------------------------------------- O4N1
@pytest.mark.parametrize("nf4", [False, True])
def test_o4n1_layout_and_qerr(nf4):
    rng = np.random.default_rng(77 + nf4)
    N, K = 64, 96
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    im = rng.uniform(0.5, 2.0, K).astype(np.float32)
    blob, qerr = O.i4a8_blob(W, im, nf4=nf4, want_qerr=True)
    assert blob.nbytes == 20 + 4 * N + K * N // 2
    hdr = np.frombuffer(blob[:20].tobytes(), "<u4")
    assert list(hdr) == [0x4F344E31, 1, K, N, int(nf4)]
    assert blob[:4].tobytes() == b"1N4O"  # magic 'O4N1' as a little-endian u32
    bs, nib, codes = O.pack_i4a8(W, im, nf4=nf4)
    assert blob[20:20 + 4 * N].tobytes() == bs.astype("<f4").tobytes()
    assert np.array_equal(blob[20 + 4 * N:].reshape(N, K // 2), nib)
    dec = O.o4n1_decode(K, N, blob)
    assert dec is not None and np.array_equal(dec[0], bs) and np.array_equal(dec[1], codes)
    q = codes.T.astype(np.float64) * bs[:, None].astype(np.float64)
    w = W.astype(np.float64)
    ref = np.sqrt(np.sum(im * (w - q) ** 2) / np.sum(im * w * w))
    assert abs(qerr - ref) <= 1e-6 * ref
    # rejections: magic, version, K, N, kind, size
    for off, val in ((0, 0x4F344E30), (4, 2), (8, K + 32), (12, N + 32), (16, 2)):
        bad = blob.copy()
        bad[off:off + 4] = np.frombuffer(np.array([val], "<u4").tobytes(), np.uint8)
        assert O.o4n1_decode(K, N, bad) is None, off
    assert O.o4n1_decode(K, N, blob[:-1]) is None


def test_o4n1_c3_size():
    """examples/test_matmul.c:528: the K=2048, N=6144 blob is 20 + 4N + K*N/2 = 6,316,052 bytes."""
    assert O.lib().oracle_i4a8_blob(2048, 6144, O._ptr(np.zeros(1, np.float32)), None, 0, 0, None, 0, None) == 6316052


def _grouped_case(seed, M, K, N, G, w4=True):
    rng = np.random.default_rng(seed)
    lo, hi = (-8, 8) if w4 else (-128, 128)
    A = rng.integers(lo, hi, size=(M, K), dtype=np.int8)
    B = rng.integers(-8, 8, size=(K, N), dtype=np.int8)
    aS = rng.uniform(1e-3, 2e-2, size=(M, K // G)).astype(np.float32)
    bS = rng.uniform(1e-3, 2e-2, size=(K // G, N)).astype(np.float32)
    return A, B, aS, bS


@pytest.mark.parametrize("M,K,N,G", [(1, 2048, 256, 128), (4, 2048, 128, 64), (3, 512, 96, 32), (2, 256, 64, 256)])
def test_grouped_oracle_pins(M, K, N, G):
    """oracle_gemm_grouped against the reference's own compiled orki_cpu_gemm_grouped (bit for bit, where
    oracle/_ref builds), a numpy float32 restatement of the per-group order, and G = K closed form."""
    A, B, aS, bS = _grouped_case(M + K + N + G, M, K, N, G)
    C = O.gemm_grouped(A, B, aS, bS, G)
    if O.ref_available():
        assert np.array_equal(C, O.ref_gemm_grouped(A, B, aS, bS, G))
    Sk = K // G
    want = np.zeros((M, N), np.float32)
    for g in range(Sk):
        P = (A[:, g * G:(g + 1) * G].astype(np.int64) @ B[g * G:(g + 1) * G].astype(np.int64)).astype(np.int32)
        want = want + (P.astype(np.float32) * aS[:, g:g + 1]) * bS[g][None, :]
    assert np.array_equal(C, want)
    # a planted mistake (one group's scales transposed onto the next group) must not agree
    if Sk > 1:
        bad = bS.copy()
        bad[[0, 1]] = bad[[1, 0]]
        assert not np.array_equal(O.gemm_grouped(A, B, aS, bad, G), C)


def test_grouped_oracle_single_group_closed_form():
    A, B, aS, bS = _grouped_case(5, 3, 512, 64, 512, w4=False)
    C = O.gemm_grouped(A, B, aS, bS, 512)
    P = O.gemm_i32(A, B).astype(np.float32)
    assert np.array_equal(C, np.float32(0) + (P * aS) * bS)


# ---- rowops_ref: the one-row run's row operations (ork_i8_mm_run_row) -------------------------------------------
def test_rowops_quant_equals_the_division_quantiser():
    """The restatement's per-row quantisation (y * (1/s), the exact quotient within 1e-4 of a half-way point) gives
    exactly the codes and scale of the oracle's examples/quant.c:34-37 quantiser, which divides every element by s,
    over rows with dozens of elements near half-way points, as well as exact ties and a zero row."""
    import rowops_ref as R

    rng = np.random.default_rng(41)
    rows = [rng.standard_normal(2048).astype(np.float32) * np.float32(rng.uniform(0.01, 10)) for _ in range(96)]
    rows.append(np.array([127.0, 63.5, -0.5, 1.5, -2.5, 0.0] * 8, np.float32))     # s = 1: exact ties, half-even
    rows.append(np.zeros(64, np.float32))                                          # zero row: s = 1, codes 0
    near = 0
    for y in rows:
        q, s = R.quant_row(y)
        sref, qref = O.quant_test_acts(y[None, :])
        assert s == sref[0] and np.array_equal(q, qref[0])
        r = y * (np.float32(1) / s)
        near += int(np.sum(np.abs(r - np.floor(r) - np.float32(0.5)) < np.float32(1e-4)))
    assert near > 30   # the exact-quotient branch was exercised (72 elements at this seed)


def test_rowops_rmsnorm_closed_forms_and_bound():
    """RMSNorm in the documented summation order: exact where every partial sum is representable (dyadic rows), a
    constant row normalises to 1 / sqrt(1 + eps / c^2) of itself, and random rows stay within K ulp-relative of the
    float64 evaluation; a row that is not a multiple of 512 long pads with exact zeros."""
    import rowops_ref as R

    for K in (64, 512, 2048, 3000):
        x = np.full(K, 0.5, np.float32)
        assert R.sum_squares(x) == np.float32(0.25 * K)
        x = (np.arange(K) % 8 - 4).astype(np.float32) / 4        # squares are multiples of 1/16: exact sums
        assert R.sum_squares(x) == np.float32(np.sum(x.astype(np.float64) ** 2))
        y = R.rmsnorm(np.full(K, 3.0, np.float32), np.ones(K, np.float32), 0.0)
        assert np.all(y == np.float32(1.0))
    rng = np.random.default_rng(43)
    for K in (100, 2048, 6144, 8192):
        x = rng.standard_normal(K).astype(np.float32)
        ss, ss64 = R.sum_squares(x), np.sum(x.astype(np.float64) ** 2)
        assert abs(float(ss) - ss64) <= K * 2.0 ** -24 * ss64
        w = (1 + 0.02 * rng.standard_normal(K)).astype(np.float32)
        y, y64 = R.rmsnorm(x, w, 1e-6), x.astype(np.float64) / np.sqrt(ss64 / K + 1e-6) * w
        assert np.max(np.abs(y - y64)) <= 1e-5 * np.max(np.abs(y64))


def test_rowops_epilogues_closed_forms():
    """Residual add and SwiGLU: zero columns leave x as it is, unit scales add the integers exactly, silu(0) = 0 and
    silu agrees with a float64 logistic to float32 precision."""
    import rowops_ref as R
    from scipy.special import expit

    rng = np.random.default_rng(47)
    x = rng.standard_normal(256).astype(np.float32)
    c = rng.integers(-1000, 1000, 256).astype(np.int32)
    assert np.array_equal(R.resid(x, np.zeros(256, np.int32), 0.37, np.ones(256, np.float32)), x)
    assert np.array_equal(R.resid(np.zeros(256, np.float32), c, 1.0, np.ones(256, np.float32)), c.astype(np.float32))
    assert np.all(R.swiglu(np.zeros(4, np.int32), c[:4], 0.5, np.ones(4, np.float32), np.ones(4, np.float32)) == 0)
    cg, cu = rng.integers(-5000, 5000, 256).astype(np.int32), rng.integers(-5000, 5000, 256).astype(np.int32)
    wg, wu = rng.uniform(1e-4, 1e-3, 256).astype(np.float32), rng.uniform(1e-4, 1e-3, 256).astype(np.float32)
    y = R.swiglu(cg, cu, 0.9, wg, wu)
    g, u = cg * 0.9 * wg.astype(np.float64), cu * 0.9 * wu.astype(np.float64)
    assert np.max(np.abs(y - g * expit(g) * u)) <= 1e-6 * np.max(np.abs(g * expit(g) * u))
