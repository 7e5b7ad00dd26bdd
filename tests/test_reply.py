"""The reply side on the CPU: the oracle's co-attention merge (orc_coattn_merge) pinned by what the mathematics fixes.

Attention over a key set A u B equals the receiver's merge of the normalised reply over A (f16 O, lse: the ATTN reply,
phone-attn.h:651-655) with its own partial over B (phone-attn.h:21, 231-239). The fp64 closed form over A u B is the
check, so a dropped weight, a wrong sign in an exponent or a swapped operand fails it; the f16 rounding of the reply
bounds the error (2^-11 relative on A's share). Empty sides reduce to the other side exactly."""
import numpy as np
import pytest

import oracle as orc


def problem(seed, nk, nkv=2, rows=8, hd=128, fmt=orc.Q8_0):
    K = orc.fill_rows(seed, fmt, nkv, hd, nk)
    V = orc.fill_rows(seed + 1, fmt, nkv, hd, nk)
    Q = orc.normal(seed + 2, 0, nkv * rows * hd).reshape(nkv * rows, hd)
    shape = orc.make_shape(nkv, rows, hd, fmt, orc.QMODE_F16)
    return shape, K, V, Q


def partial(shape, K, V, Q, k0, k1):
    """fp64 closed form over keys [k0, k1), as the fp32 (O, m, l) an engine returns."""
    rs = shape.rs
    O, m, l = orc.attn_exact(shape, Q, K[k0 * rs:k1 * rs], V[k0 * rs:k1 * rs], k1 - k0)
    return O.astype(np.float32), m.astype(np.float32), l.astype(np.float32)


@pytest.mark.parametrize("nk,na", [(300, 100), (300, 1), (300, 299), (64, 32)])
def test_coattn_equals_attention_over_both_key_sets(nk, na):
    shape, K, V, Q = problem(40 + na, nk)
    Of, mf, lf = partial(shape, K, V, Q, 0, nk)
    full = Of / lf[:, None]
    lse_full = mf + np.log(lf)
    Oa, ma, la = partial(shape, K, V, Q, 0, na)
    Ob, mb, lb = partial(shape, K, V, Q, na, nk)
    Oh, lse = orc.normalise(Oa, ma, la)
    out, lse_out = orc.coattn_merge(Oh, lse, Ob, mb, lb)
    err = np.abs(out - full).max() / np.abs(full).max()
    assert err < 1e-3, err
    assert np.abs(lse_out - lse_full).max() < 1e-5 * max(1.0, np.abs(lse_full).max())
    # the other way round (the reply over B, the receiver's keys A) gives the same attention
    Oh2, lse2 = orc.normalise(Ob, mb, lb)
    out2, _ = orc.coattn_merge(Oh2, lse2, Oa, ma, la)
    assert np.abs(out2 - full).max() / np.abs(full).max() < 1e-3


def test_coattn_empty_sides():
    shape, K, V, Q = problem(7, 200)
    O, m, l = partial(shape, K, V, Q, 0, 200)
    Oh, lse = orc.normalise(O, m, l)
    rows = O.shape[0]
    zero_O = np.zeros_like(O); ninf = np.full(rows, -np.inf, np.float32); zero = np.zeros(rows, np.float32)
    # the receiver has no keys: the reply itself, exactly
    out, lse_out = orc.coattn_merge(Oh, lse, zero_O, ninf, zero)
    assert np.array_equal(out, orc.f16_to_f32(Oh).reshape(O.shape)) and np.array_equal(lse_out, lse)
    # the reply has no keys (lse = -inf, O = 0): the receiver's own normalised partial
    Oh0 = np.zeros(O.shape, np.uint16)
    out, lse_out = orc.coattn_merge(Oh0, ninf, O, m, l)
    assert np.allclose(out, O / l[:, None], rtol=1e-6, atol=0) and np.allclose(lse_out, m + np.log(l), rtol=1e-6)
    # neither: zeros and -inf
    out, lse_out = orc.coattn_merge(Oh0, ninf, zero_O, ninf, zero)
    assert np.all(out == 0) and np.all(np.isneginf(lse_out))


def test_normalise_then_merge_is_associative_over_three_engines():
    """The server's merge of several engines' partials (merge_partial) before the reply, then the receiver's merge, is
    attention over the union of all three key ranges."""
    shape, K, V, Q = problem(11, 400)
    Of, mf, lf = partial(shape, K, V, Q, 0, 400)
    full = Of / lf[:, None]
    P = [partial(shape, K, V, Q, a, b) for a, b in ((0, 120), (120, 250), (250, 400))]
    O, m, l = (np.array(x, np.float32, copy=True) for x in P[0])
    orc.merge_partial(O, m, l, *P[1])
    Oh, lse = orc.normalise(O, m, l)
    out, _ = orc.coattn_merge(Oh, lse, *P[2])
    assert np.abs(out - full).max() / np.abs(full).max() < 1e-3
