"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from the oracle) against the
oracle as it is now, and against independent numpy restatements: the ggml-semantics quantizers (tests/test_oracle.py's
np_q8_0 / np_q4_0), an fp64 brute-force attention over numpy-dequantized rows, and numpy.argmax for acceptance. A change
to the oracle that moves any stored answer fails here."""
from pathlib import Path

import numpy as np
import pytest

import oracle as orc
from test_oracle import np_deq, np_q4_0, np_q8_0

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    return np.load(GOLD / name, allow_pickle=False)


def test_quant_fixture():
    z = load("quant_cases.npz")
    x = z["x"].reshape(-1)
    assert np.array_equal(z["q8_0"], orc.quantize(orc.Q8_0, x))
    assert np.array_equal(z["q4_0"], orc.quantize(orc.Q4_0, x))
    assert np.array_equal(z["q8_0"], np_q8_0(x))
    assert np.array_equal(z["q4_0"], np_q4_0(x))


def attn_names():
    return [str(n) for n in load("attn_cases.npz")["names"]]


def case(z, name):
    fmt, nkv, rows, hd, nk, rs = (int(v) for v in z[f"{name}__meta"])
    return fmt, nkv, rows, hd, nk, rs, z[f"{name}__K"], z[f"{name}__V"], z[f"{name}__Q"]


@pytest.mark.parametrize("name", attn_names())
def test_attn_fixture_oracle(name):
    z = load("attn_cases.npz")
    fmt, nkv, rows, hd, nk, rs, K, V, Q = case(z, name)
    Og, mg, lg = orc.attn_ggml(orc.make_shape(nkv, rows, hd, fmt, orc.QMODE_GGML, rs=rs), Q, K, V, nk, 1)
    np.testing.assert_allclose(Og, z[f"{name}__O_ggml"], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(mg, z[f"{name}__m_ggml"], rtol=1e-6)
    np.testing.assert_allclose(lg, z[f"{name}__l_ggml"], rtol=1e-6)
    Oe, me, le = orc.attn_exact(orc.make_shape(nkv, rows, hd, fmt, orc.QMODE_F16, rs=rs), Q, K, V, nk, 1)
    np.testing.assert_allclose(Oe, z[f"{name}__O_exact_f16q"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(me, z[f"{name}__m_exact_f16q"], rtol=1e-12)
    np.testing.assert_allclose(le, z[f"{name}__l_exact_f16q"], rtol=1e-12)


@pytest.mark.parametrize("name", attn_names())
def test_attn_fixture_numpy_brute_force(name):
    """fp64 softmax over numpy-dequantized rows, Q rounded to f16(q*scale): the stored closed form, independently."""
    z = load("attn_cases.npz")
    fmt, nkv, rows, hd, nk, rs, K, V, Q = case(z, name)
    hb = orc.head_bytes(fmt, hd)
    scale = np.float32(1.0 / np.sqrt(hd))
    Oref, mref, lref = z[f"{name}__O_exact_f16q"], z[f"{name}__m_exact_f16q"], z[f"{name}__l_exact_f16q"]
    for h in range(nkv):
        qs = (Q[h * rows:(h + 1) * rows] * scale).astype(np.float16).astype(np.float64)
        if nk == 0:
            assert np.all(Oref[h * rows:(h + 1) * rows] == 0) and np.all(np.isneginf(mref[h * rows:(h + 1) * rows]))
            assert np.all(lref[h * rows:(h + 1) * rows] == 0)
            continue
        kr = K.reshape(nk, rs)[:, h * hb:(h + 1) * hb].reshape(-1)
        vr = V.reshape(nk, rs)[:, h * hb:(h + 1) * hb].reshape(-1)
        kd = np_deq(fmt, kr.copy(), nk * hd).reshape(nk, hd).astype(np.float64)
        vd = np_deq(fmt, vr.copy(), nk * hd).reshape(nk, hd).astype(np.float64)
        s = qs @ kd.T
        m = s.max(axis=1)
        p = np.exp(s - m[:, None])
        np.testing.assert_allclose(Oref[h * rows:(h + 1) * rows], p @ vd, rtol=1e-9, atol=1e-9)
        np.testing.assert_allclose(mref[h * rows:(h + 1) * rows], m, rtol=1e-12)
        np.testing.assert_allclose(lref[h * rows:(h + 1) * rows], p.sum(axis=1), rtol=1e-12)


def test_accept_fixture():
    z = load("accept_cases.npz")
    for c in range(3):
        logits, draft, expect = z[f"c{c}_logits"], z[f"c{c}_draft"], z[f"c{c}_expect"]
        k, bonus, am = orc.accept(logits, draft)
        assert [k, bonus] == list(expect[:2]) and np.array_equal(am, expect[2:])
        am_np = logits.argmax(axis=1)
        assert np.array_equal(am_np, expect[2:])
        k_np = 0
        while k_np < len(draft) and am_np[k_np] == draft[k_np]:
            k_np += 1
        assert k_np == expect[0] and am_np[k_np] == expect[1]
