"""GPU parity of the reply side (through the C ABI): pa_hip_merge_partial, pa_hip_normalise, pa_hip_coattn_merge and
pa_hip_attn_reply, against the CPU oracle on the same inputs.

Bars: the fp16 reply O is bit-exact (the same IEEE division, product and round-to-nearest-even conversion on both
sides); values that pass through expf / logf match to 4 ulp-scale relative error (1e-6; the device's and the host
C library's transcendental functions may differ in the last bit); whole attention pipelines to the 2e-3 bar."""
import numpy as np
import pytest

import backburner_amd as bb
import oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ws():
    w = bb.Workspace()
    yield w
    w.close()


def dev(a):
    return bb.DeviceBuffer.from_array(np.ascontiguousarray(a))


def random_partials(seed, rows, hd):
    """(O, m, l) in natural-log units with special rows: empty (l = 0, m = -inf) on either side, equal maxima."""
    rng = np.random.default_rng(seed)
    O = rng.standard_normal((rows, hd)).astype(np.float32) * 10
    m = (rng.standard_normal(rows) * 4).astype(np.float32)
    l = rng.uniform(0.5, 100, rows).astype(np.float32)
    return O, m, l


def special_rows(O, m, l, idx):
    for i in idx:
        O[i] = 0; m[i] = -np.inf; l[i] = 0


@pytest.mark.parametrize("hd", [128, 256])
def test_merge_partial(hd):
    rows = 1000
    print(f"merge_partial rows={rows} hd={hd}", flush=True)
    O, m, l = random_partials(1, rows, hd)
    O2, m2, l2 = random_partials(2, rows, hd)
    special_rows(O, m, l, range(0, rows, 7))
    special_rows(O2, m2, l2, range(0, rows, 5))
    m2[3] = m[3]                                                     # equal maxima
    d = [dev(x) for x in (O, m, l, O2, m2, l2)]
    bb.merge_partial_device(*(b.ptr for b in d), rows, hd)
    bb.device_sync()
    gO = d[0].download(np.float32).reshape(rows, hd); gm = d[1].download(np.float32); gl = d[2].download(np.float32)
    orc.merge_partial(O, m, l, O2, m2, l2)
    assert np.array_equal(np.isneginf(gm), np.isneginf(m))
    fin = np.isfinite(m)
    np.testing.assert_allclose(gm[fin], m[fin], rtol=1e-6, atol=0)
    np.testing.assert_allclose(gl, l, rtol=1e-6, atol=0)
    np.testing.assert_allclose(gO, O, rtol=1e-5, atol=1e-5 * np.abs(O).max())


@pytest.mark.parametrize("hd", [128, 256])
def test_normalise(hd):
    rows = 777
    print(f"normalise rows={rows} hd={hd}", flush=True)
    O, m, l = random_partials(3, rows, hd)
    special_rows(O, m, l, range(0, rows, 11))
    d = [dev(x) for x in (O, m, l)]
    dOh = bb.DeviceBuffer(rows * hd * 2); dlse = bb.DeviceBuffer(rows * 4)
    bb.normalise_device(d[0].ptr, d[1].ptr, d[2].ptr, rows, hd, dOh.ptr, dlse.ptr)
    bb.device_sync()
    Oh_ref, lse_ref = orc.normalise(O, m, l)
    assert np.array_equal(dOh.download(np.uint16).reshape(rows, hd), Oh_ref)
    glse = dlse.download(np.float32)
    assert np.array_equal(np.isneginf(glse), np.isneginf(lse_ref))
    fin = np.isfinite(lse_ref)
    np.testing.assert_allclose(glse[fin], lse_ref[fin], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("hd", [128, 256])
def test_coattn_merge(hd):
    rows = 640
    print(f"coattn rows={rows} hd={hd}", flush=True)
    O, m, l = random_partials(4, rows, hd)
    Oh, lse = orc.normalise(*random_partials(5, rows, hd))
    special_rows(O, m, l, range(0, rows, 9))
    lse[::13] = -np.inf; Oh[::13] = 0
    d = [dev(x) for x in (Oh, lse, O, m, l)]
    dout = bb.DeviceBuffer(rows * hd * 4); dlse = bb.DeviceBuffer(rows * 4)
    bb.coattn_merge_device(*(b.ptr for b in d), rows, hd, dout.ptr, dlse.ptr)
    bb.device_sync()
    out_ref, lse_ref = orc.coattn_merge(Oh, lse, O, m, l)
    gout = dout.download(np.float32).reshape(rows, hd); glse = dlse.download(np.float32)
    np.testing.assert_allclose(gout, out_ref, rtol=1e-5, atol=1e-6 * np.abs(out_ref).max())
    assert np.array_equal(np.isneginf(glse), np.isneginf(lse_ref))
    fin = np.isfinite(lse_ref)
    np.testing.assert_allclose(glse[fin], lse_ref[fin], rtol=1e-6, atol=1e-6)


# decode (split-K merge over many slots), verify / prefill (MMA kernel + merge), a single-chunk call (direct write,
# normalised by its own kernel), hd 256 (the general kernel), an empty call
REPLY_CASES = [
    (bb.FMT_Q8_0, 8, 8, 128, 4096, bb.QMODE_GGML),
    (bb.FMT_Q4_0, 8, 8, 128, 2000, bb.QMODE_GGML),
    (bb.FMT_Q8_0, 2, 128, 128, 3000, bb.QMODE_GGML),
    (bb.FMT_Q8_0, 1, 512, 128, 1500, bb.QMODE_F16),
    (bb.FMT_Q8_0, 2, 8, 128, 20, bb.QMODE_GGML),
    (bb.FMT_Q8_0, 2, 48, 256, 900, bb.QMODE_F16),
    (bb.FMT_Q8_0, 2, 8, 128, 0, bb.QMODE_GGML),
]


@pytest.mark.parametrize("fmt,nkv,rows,hd,nk,qmode", REPLY_CASES)
def test_attn_reply(ws, fmt, nkv, rows, hd, nk, qmode):
    """pa_hip_attn_reply == normalise(pa_hip_attn) on the device bit for bit, and == the oracle's normalise of the
    device's (O, m, l) (Oh exact, lse to 1e-6)."""
    print(f"attn_reply fmt={fmt} nkv={nkv} rows={rows} hd={hd} nk={nk} qmode={qmode}", flush=True)
    hb = orc.head_bytes(fmt, hd); rs = nkv * hb
    K = orc.fill_rows(60 + nk, fmt, nkv, hd, nk, rs=rs)
    V = orc.fill_rows(61 + nk, fmt, nkv, hd, nk, rs=rs)
    Q = orc.normal(62 + nk, 0, nkv * rows * hd).reshape(nkv * rows, hd)
    shape = bb.make_shape(nkv, rows, hd, fmt, qmode, rs=rs)
    pages = bb.pages_from_rows(K, V, rs, 1024)
    n = nkv * rows
    dq = dev(Q)
    dOh = bb.DeviceBuffer(n * hd * 2); dlse = bb.DeviceBuffer(n * 4)
    dO = bb.DeviceBuffer(n * hd * 4); dml = bb.DeviceBuffer(n * 8)
    dOh2 = bb.DeviceBuffer(n * hd * 2); dlse2 = bb.DeviceBuffer(n * 4)
    try:
        ws.attn_reply(shape, pages, dq.ptr, dOh.ptr, dlse.ptr)
        ws.attn(shape, pages, dq.ptr, dO.ptr, dml.ptr, dml.ptr + n * 4)
        bb.normalise_device(dO.ptr, dml.ptr, dml.ptr + n * 4, n, hd, dOh2.ptr, dlse2.ptr)
        bb.device_sync()
        Oh = dOh.download(np.uint16).reshape(n, hd); lse = dlse.download(np.float32)
        assert np.array_equal(Oh, dOh2.download(np.uint16).reshape(n, hd))
        assert np.array_equal(lse, dlse2.download(np.float32))
        O = dO.download(np.float32).reshape(n, hd); ml = dml.download(np.float32)
        Oh_ref, lse_ref = orc.normalise(O, ml[:n], ml[n:])
        assert np.array_equal(Oh, Oh_ref)
        assert np.array_equal(np.isneginf(lse), np.isneginf(lse_ref))
        fin = np.isfinite(lse_ref)
        np.testing.assert_allclose(lse[fin], lse_ref[fin], rtol=1e-6, atol=1e-6)
        if nk == 0:
            assert np.all(Oh == 0) and np.all(np.isneginf(lse))
    finally:
        pages.close()


def test_reply_pipeline_equals_attention_over_all_keys(ws):
    """Old keys A on the engine (pa_hip_attn_reply), recent keys B on the receiver (pa_hip_attn), merged on the device
    by pa_hip_coattn_merge: equal to attention over A u B in one call, to the 2e-3 bar."""
    fmt, nkv, rows, hd, na, nb = bb.FMT_Q8_0, 8, 8, 128, 6000, 700
    print(f"reply pipeline na={na} nb={nb}", flush=True)
    hb = orc.head_bytes(fmt, hd); rs = nkv * hb
    nk = na + nb
    K = orc.fill_rows(70, fmt, nkv, hd, nk, rs=rs, n_outliers=4, outlier_mul=8.0)
    V = orc.fill_rows(71, fmt, nkv, hd, nk, rs=rs)
    Q = orc.normal(72, 0, nkv * rows * hd).reshape(nkv * rows, hd)
    shape = bb.make_shape(nkv, rows, hd, fmt, bb.QMODE_GGML, rs=rs)
    n = nkv * rows
    pa = bb.pages_from_rows(K[:na * rs], V[:na * rs], rs, 4096)
    pb = bb.pages_from_rows(K[na * rs:], V[na * rs:], rs, 4096)
    pall = bb.pages_from_rows(K, V, rs, 4096)
    dq = dev(Q)
    dOh = bb.DeviceBuffer(n * hd * 2); dlse = bb.DeviceBuffer(n * 4)
    dOb = bb.DeviceBuffer(n * hd * 4); dmlb = bb.DeviceBuffer(n * 8)
    dout = bb.DeviceBuffer(n * hd * 4)
    dO = bb.DeviceBuffer(n * hd * 4); dml = bb.DeviceBuffer(n * 8)
    try:
        ws.attn_reply(shape, pa, dq.ptr, dOh.ptr, dlse.ptr)
        ws.attn(shape, pb, dq.ptr, dOb.ptr, dmlb.ptr, dmlb.ptr + n * 4)
        bb.coattn_merge_device(dOh.ptr, dlse.ptr, dOb.ptr, dmlb.ptr, dmlb.ptr + n * 4, n, hd, dout.ptr)
        ws.attn(shape, pall, dq.ptr, dO.ptr, dml.ptr, dml.ptr + n * 4)
        bb.device_sync()
        out = dout.download(np.float32).reshape(n, hd)
        O = dO.download(np.float32).reshape(n, hd); l = dml.download(np.float32)[n:]
        full = O / l[:, None]
        err = np.abs(out - full).max(axis=1) / np.abs(full).max(axis=1)
        assert err.max() < 2e-3, err.max()
    finally:
        for p in (pa, pb, pall):
            p.close()


def server_row_map(ng, nkv, nr, ntok):
    """The reference Metal engine's row placement (pa-metal.mm:630-634, 661-672; merge: 501-505), restated with plain
    loops: for each call row (head h, row r) the server row (group g, head h, row i) it comes from, and the call rows
    per KV head."""
    nt = ntok if ng == 1 and 1 <= ntok < 8 else 0
    rows = (nr // 8) * nt if nt else ng * nr
    src = {}
    for h in range(nkv):
        if nt:
            for k in range(nr // 8):
                for t in range(nt):
                    src[(h, k * nt + t)] = (0, h, k * 8 + t)
        else:
            for g in range(ng):
                for i in range(nr):
                    src[(h, g * nr + i)] = (g, h, i)
    return rows, src


@pytest.mark.parametrize("ng,ntok", [(1, 1), (1, 3), (1, 7), (1, 8), (1, 0), (3, 8)])
def test_pack_q_and_unpack_rows(ng, ntok):
    """pa_hip_pack_q / pa_hip_unpack_rows at the reference shape (4 KV heads, 48 rows, hd 256) against the row map
    above: Q values convert exactly (f16 -> fp32), every call row lands where the map says, and the rows of tokens
    the call did not have come back as (0, -inf, 0)."""
    nkv, nr, hd = 4, 48, 256
    rows, src = server_row_map(ng, nkv, nr, ntok)
    rng = np.random.default_rng(ng * 10 + ntok)
    qs = orc.f32_to_f16(rng.standard_normal((ng, nkv, nr, hd)).astype(np.float32))
    dqs, dq = dev(qs), bb.DeviceBuffer(nkv * rows * hd * 4)
    bb.pack_q_device(dqs.ptr, ng, nkv, nr, hd, ntok, dq.ptr)
    bb.device_sync()
    q = dq.download(np.float32).reshape(nkv, rows, hd)
    qf = orc.f16_to_f32(qs)
    for (h, r), (g, hh, i) in src.items():
        assert np.array_equal(q[h, r], qf[g, hh, i]), (h, r)
    O = rng.standard_normal((nkv * rows, hd)).astype(np.float32)
    m = rng.standard_normal(nkv * rows).astype(np.float32)
    l = rng.uniform(1, 2, nkv * rows).astype(np.float32)
    dO, dm, dl = dev(O), dev(m), dev(l)
    sO, sm, sl = bb.DeviceBuffer(ng * nkv * nr * hd * 4), bb.DeviceBuffer(ng * nkv * nr * 4), bb.DeviceBuffer(ng * nkv * nr * 4)
    bb.unpack_rows_device(dO.ptr, dm.ptr, dl.ptr, ng, nkv, nr, hd, ntok, sO.ptr, sm.ptr, sl.ptr)
    bb.device_sync()
    Os = sO.download(np.float32).reshape(ng, nkv, nr, hd)
    ms, ls = sm.download(np.float32).reshape(ng, nkv, nr), sl.download(np.float32).reshape(ng, nkv, nr)
    seen = np.zeros((ng, nkv, nr), bool)
    for (h, r), (g, hh, i) in src.items():
        assert np.array_equal(Os[g, hh, i], O[h * rows + r]) and ms[g, hh, i] == m[h * rows + r] and ls[g, hh, i] == l[h * rows + r]
        seen[g, hh, i] = True
    assert np.all(Os[~seen] == 0) and np.all(np.isneginf(ms[~seen])) and np.all(ls[~seen] == 0)
    assert seen.sum() == nkv * rows
    for b in (dqs, dq, dO, dm, dl, sO, sm, sl):
        b.close()


def test_pack_rejects_bad_geometry():
    with pytest.raises(bb.PaHipError, match="bad geometry"):
        bb.pack_q_device(0, 2, 4, 48, 256, 3, 0)                 # fewer than 8 tokens needs one group
    with pytest.raises(bb.PaHipError, match="bad geometry"):
        bb.unpack_rows_device(0, 0, 0, 1, 4, 44, 256, 8, 0, 0, 0)  # rows per head not a multiple of 8
