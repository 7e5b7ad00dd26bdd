"""Pins the CPU oracle (oracle/pa_oracle.c) against things it did not write itself: numpy's float16, independent numpy
restatements of the block formats, brute-force fp64 attention, closed forms and invariants. Each check is chosen so a
plausible slip (a wrong rounding rule, a dropped rescale factor, a swapped nibble, an off-by-one block) fails it."""
import numpy as np
import pytest

import oracle as orc

RNG = np.random.default_rng(1234)


# ---------------------------------------------------------------- fp16
def test_f16_to_f32_exhaustive_vs_numpy():
    h = np.arange(65536, dtype=np.uint16)
    ours = orc.f16_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_vs_numpy():
    x = np.concatenate([
        RNG.standard_normal(200000).astype(np.float32) * 10.0 ** RNG.integers(-9, 6, 200000),
        np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65520.0, 65519.996, 6.1035156e-05, 5.9604645e-08, 2.9802322e-08,
                  2.9802326e-08, 1e-30, -1e-30, 1e30], np.float32),
        (np.arange(-2048, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -14),   # ties in the subnormal range
        np.arange(2048, 4096, dtype=np.float32) + 0.5,                                  # ties at |x| in [2048, 4096)
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(orc.f32_to_f16(x), ref)


# ---------------------------------------------------------------- block formats: independent numpy restatements
def np_q8_0(x):
    """ggml quantize_row_q8_0_ref, in numpy float32: d = amax/127, id = 1/d, q = roundf(x*id) (half away from zero)."""
    x = x.reshape(-1, 32).astype(np.float32)
    amax = np.abs(x).max(axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    idv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, 1), 0).astype(np.float32)
    v = (x * idv[:, None]).astype(np.float32).astype(np.float64)
    q = (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int8)
    out = np.zeros((x.shape[0], 34), np.uint8)
    out[:, :2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.ravel()


def np_q4_0(x):
    """ggml quantize_row_q4_0_ref: max = the value of largest magnitude (first), d = max/-8, q = min(15, trunc(x*id + 8.5))."""
    x = x.reshape(-1, 32).astype(np.float32)
    mx = x[np.arange(len(x)), np.abs(x).argmax(axis=1)]
    d = (mx / np.float32(-8.0)).astype(np.float32)
    idv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, 1), 0).astype(np.float32)
    v = ((x * idv[:, None]).astype(np.float32) + np.float32(8.5)).astype(np.float32)
    q = np.minimum(15, np.trunc(v).astype(np.int32)).astype(np.uint8)
    out = np.zeros((x.shape[0], 18), np.uint8)
    out[:, :2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q[:, :16] | (q[:, 16:] << 4)
    return out.ravel()


def np_deq(fmt, y, n):
    if fmt == orc.Q8_0:
        b = y.reshape(-1, 34)
        d = b[:, :2].copy().view(np.float16).astype(np.float32)
        return (b[:, 2:].view(np.int8).astype(np.float32) * d).ravel()[:n]
    if fmt == orc.Q4_0:
        b = y.reshape(-1, 18)
        d = b[:, :2].copy().view(np.float16).astype(np.float32)
        lo = (b[:, 2:] & 15).astype(np.int32) - 8
        hi = (b[:, 2:] >> 4).astype(np.int32) - 8
        return (np.concatenate([lo, hi], axis=1).astype(np.float32) * d).ravel()[:n]
    return y.view(np.float16).astype(np.float32)[:n]


def _blocks(n_blocks):
    x = RNG.standard_normal(n_blocks * 32).astype(np.float32) * np.repeat(10.0 ** RNG.uniform(-3, 3, n_blocks), 32).astype(np.float32)
    x[:32] = 0.0                                          # an all-zero block: d = 0, id = 0
    x[32:64] = np.arange(32, dtype=np.float32) - 16.0     # exact values, a -16 maximum magnitude
    x[64:96] = 0.5                                        # x*id lands exactly on .5 boundaries
    return x


def test_q8_0_vs_numpy():
    x = _blocks(4000)
    assert np.array_equal(orc.quantize(orc.Q8_0, x), np_q8_0(x))


def test_q4_0_vs_numpy():
    x = _blocks(4000)
    assert np.array_equal(orc.quantize(orc.Q4_0, x), np_q4_0(x))


def test_q8_0_known_answer():
    x = np.arange(32, dtype=np.float32) - 16.0           # amax 16: d = 16/127, q = round(x*127/16)
    y = orc.quantize(orc.Q8_0, x)
    d = np.float32(16.0) / np.float32(127.0)
    assert y[:2].view(np.float16)[0] == np.float16(d)
    assert y[2] == np.uint8(np.int8(-127).view(np.uint8))   # -16 -> -127
    assert y[2 + 16] == 0                                    # 0 -> 0
    assert y[2 + 31].view(np.int8) == np.int8(119)          # 15*127/16 = 119.06 -> 119


def test_q4_0_known_answer():
    x = np.zeros(32, np.float32)
    x[0] = -8.0; x[1] = 4.0; x[16] = 7.0                 # max = -8: d = 1, id = 1
    y = orc.quantize(orc.Q4_0, x)
    assert y[:2].view(np.float16)[0] == np.float16(1.0)
    assert y[2] == (0 | (15 << 4))                        # x0 = -8 -> 0 ; x16 = 7 -> 15.5 -> 15
    assert y[3] == (12 | (8 << 4))                        # x1 = 4 -> 12.5 -> 12 ; x17 = 0 -> 8


@pytest.mark.parametrize("fmt", [orc.F16, orc.Q8_0, orc.Q4_0])
def test_dequant_vs_numpy(fmt):
    x = _blocks(500)
    y = orc.quantize(fmt, x)
    assert np.array_equal(orc.dequantize(fmt, y, x.size), np_deq(fmt, y, x.size))
    if fmt != orc.F16:   # half a step (a whole one where q4_0 clamps at 15), plus |q| times the fp16 error of d
        qmax = 127.0 if fmt == orc.Q8_0 else 8.0
        step = np.abs(x.reshape(-1, 32)).max(axis=1).astype(np.float64) / qmax
        d16 = step.astype(np.float16).astype(np.float64)
        err = np.abs(orc.dequantize(fmt, y, x.size) - x).reshape(-1, 32).max(axis=1)
        bound = step * (0.5 if fmt == orc.Q8_0 else 1.0) + qmax * np.abs(d16 - step)
        assert np.all(err <= bound * 1.001 + 1e-30)


def test_patool_quantizers_differ_only_by_rounding_rule():
    x = _blocks(2000)
    a, b = orc.quantize(orc.Q8_0, x), orc.quantize(orc.Q8_0, x, variant="patool")
    da, db = np_deq(orc.Q8_0, a, x.size), np_deq(orc.Q8_0, b, x.size)
    step = np.repeat(np.abs(x.reshape(-1, 32)).max(axis=1) / 127.0, 32)
    assert np.all(np.abs(da - db) <= step * 1.01 + 1e-30)      # at most one step apart
    assert (a != b).mean() < 0.05


# ---------------------------------------------------------------- synthetic data
def test_normal_stream_stats_and_splitting():
    x = orc.normal(7, 0, 1 << 20).astype(np.float64)
    assert abs(x.mean()) < 5e-3 and abs(x.std() - 1) < 5e-3
    assert abs(((x - x.mean()) ** 4).mean() / x.var() ** 2 - 3) < 0.05
    assert np.array_equal(orc.normal(7, 1000, 77), orc.normal(7, 0, 2000)[1000:1077])
    assert not np.array_equal(orc.normal(7, 0, 64), orc.normal(8, 0, 64))


def test_fill_rows_layout_and_outliers():
    nkv, hd, n = 3, 128, 10
    for fmt in (orc.F16, orc.Q8_0, orc.Q4_0):
        rows = orc.fill_rows(11, fmt, nkv, hd, n, amp=1.0)
        hb = orc.head_bytes(fmt, hd)
        for j in (0, 7):
            for h in range(nkv):
                x = orc.normal(11, (j * nkv + h) * hd, hd)
                assert np.array_equal(rows[j * nkv * hb + h * hb:j * nkv * hb + (h + 1) * hb], orc.quantize(fmt, x))
        part = orc.fill_rows(11, fmt, nkv, hd, 4, j0=6)
        assert np.array_equal(part, rows[6 * nkv * hb:10 * nkv * hb])
    ch = orc.outlier_channels(5, 8, 128, 4)
    assert ch.shape == (8, 4) and all(len(set(r)) == 4 for r in ch) and ch.min() >= 0 and ch.max() < 128
    base = orc.fill_rows(5, orc.F16, 8, 128, 2)
    out = orc.fill_rows(5, orc.F16, 8, 128, 2, n_outliers=4, outlier_mul=8.0)
    xb = base.view(np.float16).astype(np.float32).reshape(2, 8, 128)
    xo = out.view(np.float16).astype(np.float32).reshape(2, 8, 128)
    for h in range(8):
        mask = np.zeros(128, bool); mask[ch[h]] = True
        assert np.allclose(xo[:, h, mask], xb[:, h, mask] * 8, rtol=2e-3)
        assert np.array_equal(xo[:, h, ~mask], xb[:, h, ~mask])


# ---------------------------------------------------------------- attention: fp64 closed form vs brute force
def brute(shape, Q, K, V, nk):
    """Dense numpy fp64 restatement: dequantize every row, S = scale*Q K^T, softmax pieces."""
    nkv, rows, hd, fmt, rs, hb = shape.nkv, shape.rows, shape.hd, shape.fmt, shape.rs, shape.hb
    Kr = K.reshape(-1, rs)[:nk]; Vr = V.reshape(-1, rs)[:nk]
    O = np.zeros((nkv * rows, hd)); m = np.full(nkv * rows, -np.inf); l = np.zeros(nkv * rows)
    for h in range(nkv):
        kf = np.stack([np_deq(fmt, Kr[j, h * hb:(h + 1) * hb], hd) for j in range(nk)]).astype(np.float64) if nk else np.zeros((0, hd))
        vf = np.stack([np_deq(fmt, Vr[j, h * hb:(h + 1) * hb], hd) for j in range(nk)]).astype(np.float64) if nk else np.zeros((0, hd))
        q = Q.reshape(nkv, rows, hd)[h].astype(np.float64)
        if shape.qmode == orc.QMODE_GGML and fmt != orc.F16:
            q = np.stack([np_deq(orc.Q8_0, np_q8_0(Q.reshape(nkv, rows, hd)[h][r]), hd) for r in range(rows)]).astype(np.float64)
            post = shape.scale
        elif shape.qmode == orc.QMODE_GGML:
            q = Q.reshape(nkv, rows, hd)[h].astype(np.float16).astype(np.float64); post = shape.scale
        elif shape.qmode == orc.QMODE_F16:
            q = (Q.reshape(nkv, rows, hd)[h] * np.float32(shape.scale)).astype(np.float32).astype(np.float16).astype(np.float64); post = 1.0
        else:
            post = shape.scale
        if nk == 0:
            continue
        S = (q @ kf.T) * post
        mm = S.max(axis=1)
        P = np.exp(S - mm[:, None])
        O[h * rows:(h + 1) * rows] = P @ vf
        m[h * rows:(h + 1) * rows] = mm
        l[h * rows:(h + 1) * rows] = P.sum(axis=1)
    return O, m, l


def _case(fmt, nkv=2, rows=5, hd=128, nk=70, seed=3, amp=1.0, rs_pad=0):
    hb = orc.head_bytes(fmt, hd)
    rs = nkv * hb + rs_pad
    K = orc.fill_rows(seed, fmt, nkv, hd, nk, rs=rs, amp=amp)
    V = orc.fill_rows(seed + 1, fmt, nkv, hd, nk, rs=rs)
    Q = orc.normal(seed + 2, 0, nkv * rows * hd).reshape(nkv * rows, hd)
    return K, V, Q, rs


@pytest.mark.parametrize("fmt", [orc.F16, orc.Q8_0, orc.Q4_0])
@pytest.mark.parametrize("qmode", [orc.QMODE_EXACT, orc.QMODE_F16, orc.QMODE_GGML])
def test_exact_vs_brute(fmt, qmode):
    K, V, Q, rs = _case(fmt, rs_pad=6)
    s = orc.make_shape(2, 5, 128, fmt, qmode, rs=rs)
    O, m, l = orc.attn_exact(s, Q, K, V, 70)
    Ob, mb, lb = brute(s, Q, K, V, 70)
    assert np.allclose(O, Ob, rtol=1e-12, atol=1e-12) and np.allclose(m, mb, rtol=1e-12) and np.allclose(l, lb, rtol=1e-12)


@pytest.mark.parametrize("fmt", [orc.F16, orc.Q8_0, orc.Q4_0])
def test_ggml_restatement_vs_exact(fmt):
    """The ggml online recurrence (fp32, key order, expf) equals the fp64 closed form with the same Q rounding to ~1e-6:
    a dropped rescale (ms) or a wrong vs/ms branch would be off by orders of magnitude."""
    K, V, Q, rs = _case(fmt, nkv=3, rows=9, nk=300, amp=3.0)
    s = orc.make_shape(3, 9, 128, fmt, orc.QMODE_GGML, rs=rs)
    O, m, l = orc.attn_ggml(s, Q, K, V, 300)
    Oe, me, le = orc.attn_exact(s, Q, K, V, 300)
    eo, em, el = orc.rel_err(O, m, l, Oe, me, le)
    assert eo < 2e-5 and em < 1e-5 and el < 2e-5, (eo, em, el)


def test_ggml_q_rounding_is_visible():
    """Quantizing Q to q8_0 moves the result by about 1e-3 relative at this shape: the oracle really applies it."""
    K, V, Q, rs = _case(orc.Q8_0, nkv=1, rows=8, nk=512, amp=2.0)
    s = orc.make_shape(1, 8, 128, orc.Q8_0, orc.QMODE_GGML, rs=rs)
    sx = orc.make_shape(1, 8, 128, orc.Q8_0, orc.QMODE_EXACT, rs=rs)
    eo, _, _ = orc.rel_err(*orc.attn_ggml(s, Q, K, V, 512), *orc.attn_exact(sx, Q, K, V, 512))
    assert 1e-5 < eo < 5e-2


# ---------------------------------------------------------------- invariants and special cases
def test_split_merge_invariance():
    K, V, Q, rs = _case(orc.Q8_0, nkv=2, rows=4, nk=200)
    s = orc.make_shape(2, 4, 128, orc.Q8_0, orc.QMODE_GGML, rs=rs)
    Of, mf, lf = orc.attn_ggml(s, Q, K, V, 200)
    a = 77
    O1, m1, l1 = orc.attn_ggml(s, Q, K[:a * rs], V[:a * rs], a)
    O2, m2, l2 = orc.attn_ggml(s, Q, K[a * rs:], V[a * rs:], 200 - a)
    orc.merge_partial(O2, m2, l2, O1, m1, l1)          # merge order must not matter either
    eo, em, el = orc.rel_err(O2, m2, l2, Of, mf, lf)
    assert eo < 1e-5 and em == 0 and el < 1e-5


def test_key_permutation_invariance():
    K, V, Q, rs = _case(orc.Q4_0, nkv=1, rows=3, nk=90)
    s = orc.make_shape(1, 3, 128, orc.Q4_0, orc.QMODE_GGML, rs=rs)
    perm = RNG.permutation(90)
    Kp = K.reshape(90, rs)[perm].ravel(); Vp = V.reshape(90, rs)[perm].ravel()
    eo, em, el = orc.rel_err(*orc.attn_exact(s, Q, Kp, Vp, 90), *orc.attn_exact(s, Q, K, V, 90))
    assert eo < 1e-12 and em < 1e-12 and el < 1e-12


def test_equal_keys_zero_query_and_empty():
    hd, nk = 128, 64
    x = orc.normal(9, 0, hd)
    row = orc.quantize(orc.Q8_0, x)
    K = np.tile(row, nk); V = np.tile(row, nk)
    Q = orc.normal(10, 0, 2 * hd).reshape(2, hd)
    s = orc.make_shape(1, 2, hd, orc.Q8_0, orc.QMODE_GGML)
    O, m, l = orc.attn_exact(s, Q, K, V, nk)
    v = np_deq(orc.Q8_0, row, hd)
    assert np.allclose(l, nk) and np.allclose(O / l[:, None], v[None, :], rtol=1e-12)
    Kr = orc.fill_rows(4, orc.Q8_0, 1, hd, nk); Vr = orc.fill_rows(5, orc.Q8_0, 1, hd, nk)
    O, m, l = orc.attn_exact(s, np.zeros((2, hd), np.float32), Kr, Vr, nk)
    vm = np.stack([np_deq(orc.Q8_0, Vr[j * 136:(j + 1) * 136], hd) for j in range(nk)]).mean(axis=0)
    assert np.all(m == 0) and np.allclose(l, nk) and np.allclose(O / l[:, None], vm[None, :], rtol=1e-10)
    for f in (orc.attn_exact, orc.attn_ggml):
        O, m, l = f(s, Q, Kr, Vr, 0)
        assert np.all(O == 0) and np.all(np.isneginf(m)) and np.all(l == 0)


def test_dominant_key():
    hd, nk = 128, 50
    K = orc.fill_rows(4, orc.F16, 1, hd, nk, amp=0.01)
    V = orc.fill_rows(5, orc.F16, 1, hd, nk)
    q = orc.normal(6, 0, hd)
    Kf = K.view(np.float16).reshape(nk, hd).copy()
    Kf[17] = (q * 4).astype(np.float16)
    K = Kf.view(np.uint8).ravel()
    s = orc.make_shape(1, 1, hd, orc.F16, orc.QMODE_EXACT)
    O, m, l = orc.attn_exact(s, q.reshape(1, hd), K, V, nk)
    v17 = V.view(np.float16).reshape(nk, hd)[17].astype(np.float64)
    assert np.allclose(O[0] / l[0], v17, atol=1e-6) and abs(l[0] - 1) < 1e-6


def test_merge_closed_form_and_skips():
    O = np.array([[1.0, 2.0]], np.float32); m = np.array([0.5], np.float32); l = np.array([2.0], np.float32)
    O2 = np.array([[3.0, -1.0]], np.float32); m2 = np.array([1.5], np.float32); l2 = np.array([4.0], np.float32)
    orc.merge_partial(O, m, l, O2, m2, l2)
    a = np.exp(np.float32(-1.0))
    assert np.allclose(O, [[1 * a + 3, 2 * a - 1]]) and m[0] == 1.5 and np.isclose(l[0], 2 * a + 4)
    Oz = np.zeros((1, 2), np.float32); mz = np.array([-np.inf], np.float32); lz = np.zeros(1, np.float32)
    O3 = O.copy(); m3 = m.copy(); l3 = l.copy()
    orc.merge_partial(O3, m3, l3, Oz, mz, lz)            # an empty partial changes nothing
    assert np.array_equal(O3, O) and m3[0] == m[0] and l3[0] == l[0]
    orc.merge_partial(Oz, mz, lz, O, m, l)               # into an empty one: copies
    assert np.array_equal(Oz, O) and mz[0] == m[0] and lz[0] == l[0]


def test_normalise_closed_form():
    O = RNG.standard_normal((5, 128)).astype(np.float32)
    m = RNG.standard_normal(5).astype(np.float32)
    l = np.array([1.5, 0.0, 3.0, 2.0, 0.25], np.float32)
    Oh, lse = orc.normalise(O, m, l)
    inv = np.where(l > 0, np.float32(1) / np.where(l > 0, l, 1), 0).astype(np.float32)
    assert np.array_equal(Oh, (O * inv[:, None]).astype(np.float32).astype(np.float16).view(np.uint16))
    assert np.isneginf(lse[1]) and np.allclose(lse[[0, 2, 3, 4]], (m + np.log(l))[[0, 2, 3, 4]], rtol=1e-6)


# ---------------------------------------------------------------- greedy acceptance
def brute_accept(logits, draft):
    am = np.array([int(np.argmax(r)) for r in logits])     # numpy: first maximum, first NaN
    k = 0
    while k < len(draft) and am[k] == draft[k]:
        k += 1
    return k, int(am[k]), am


def test_accept_vs_numpy_planted():
    vocab = 5000
    for k_true in range(17):
        logits = RNG.standard_normal((17, vocab)).astype(np.float32)
        draft = RNG.integers(0, vocab, 16).astype(np.int32)
        for i in range(k_true):
            logits[i, draft[i]] = logits[i].max() + 1.0
        if k_true < 16 and np.argmax(logits[k_true]) == draft[k_true]:
            logits[k_true, draft[k_true]] = logits[k_true].min() - 1.0
        k, b, am = orc.accept(logits, draft)
        kb, bb, amb = brute_accept(logits, draft)
        assert (k, b) == (kb, bb) == (k_true, int(np.argmax(logits[k_true])))
        assert np.array_equal(am, amb)


def test_accept_ties_zeros_nan():
    vocab = 1000
    logits = np.zeros((3, vocab), np.float32)
    logits[0, [5, 700, 3]] = 2.0                          # tie: lowest index 3 wins
    logits[1, 10] = -0.0; logits[1, :] = -1.0; logits[1, 400] = 0.0; logits[1, 20] = -0.0   # -0 == +0: 20 wins
    logits[2, 50] = np.nan; logits[2, 40] = np.inf; logits[2, 60] = np.nan   # first NaN wins
    draft = np.array([3, 20], np.int32)
    k, b, am = orc.accept(logits, draft)
    kb, bb, amb = brute_accept(logits, draft)
    assert list(am) == list(amb) == [3, 20, 50] and (k, b) == (kb, bb) == (2, 50)


@pytest.mark.parametrize("fmt", [orc.Q8_0, orc.Q4_0])
@pytest.mark.parametrize("nkv,rows,nk,pad", [(8, 8, 3000, 0), (2, 48, 1000, 16), (1, 5, 777, 0), (3, 130, 500, 8)])
def test_simd_cpu_baseline_equals_oracle(fmt, nkv, rows, nk, pad):
    """The vectorized CPU baseline (pa_cpu_simd.c) keeps orc_attn_ggml's operation order: equal bit for bit on every
    SIMD path this CPU has (outlier keys, padded rows, row counts that are not multiples of the task size)."""
    hb = orc.head_bytes(fmt, 128)
    rs = nkv * hb + pad
    K = orc.fill_rows(61, fmt, nkv, 128, nk, rs=rs, n_outliers=4, outlier_mul=8.0)
    V = orc.fill_rows(62, fmt, nkv, 128, nk, rs=rs)
    Q = orc.normal(63, 0, nkv * rows * 128).reshape(-1, 128)
    s = orc.make_shape(nkv, rows, 128, fmt, rs=rs)
    ref = orc.attn_ggml(s, Q, K, V, nk)
    best = orc.simd_path()
    levels = [1] + ([2] if best == "avx512-vnni" else [])
    for lv in levels:
        O, m, l, path = orc.attn_ggml_simd(s, Q, K, V, nk, 0, lv)
        assert path == ("avx512-vnni" if lv == 2 else "avx2")
        assert np.array_equal(O, ref[0]) and np.array_equal(m, ref[1]) and np.array_equal(l, ref[2]), path
