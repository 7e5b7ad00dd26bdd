"""GPU parity of KV ingest into HBM pages (through the C ABI): pa_hip_append_rows (APPEND, phone-attn.h:403-421, with
the store_f16 conversion of store_rows, 305-319) and pa_hip_append_f32 (quantization on the device straight into page
rows). The stored bytes must equal the oracle's bit for bit; attention over ingested pages then meets the 2e-3 bar."""
import numpy as np
import pytest

import backburner_amd as bb
import oracle as orc

pytestmark = pytest.mark.gpu

PAGE_KEYS = 100
CHUNKS = [37, 150, 1, 12, 63]          # crosses page boundaries, single rows, a chunk spanning two boundaries


def page_bytes(pages, n_pages, page_bytes_each):
    return [np.concatenate([pages.bufs[2 * i + t].download(np.uint8, page_bytes_each) for i in range(n_pages)])
            for t in (0, 1)]


@pytest.mark.parametrize("fmt", [bb.FMT_Q8_0, bb.FMT_Q4_0, bb.FMT_F16])
@pytest.mark.parametrize("from_host", [False, True])
def test_append_rows_copy(fmt, from_host):
    nkv, hd = 8, 128
    hb = orc.head_bytes(fmt, hd); rs = nkv * hb
    n = sum(CHUNKS)
    print(f"append_rows fmt={fmt} host={from_host} n={n}", flush=True)
    K = orc.fill_rows(21, fmt, nkv, hd, n, rs=rs); V = orc.fill_rows(22, fmt, nkv, hd, n, rs=rs)
    shape = bb.make_shape(nkv, 8, hd, fmt, rs=rs)
    n_pages = (n + PAGE_KEYS - 1) // PAGE_KEYS
    pages = bb.alloc_pages(n_pages, PAGE_KEYS * rs)
    dK, dV = bb.DeviceBuffer.from_array(K), bb.DeviceBuffer.from_array(V)
    try:
        pos = 0
        for c in CHUNKS:
            if from_host:
                kh, vh = K[pos * rs:(pos + c) * rs], V[pos * rs:(pos + c) * rs]
                bb.append_rows(shape, pages, PAGE_KEYS, pos, kh.ctypes.data, vh.ctypes.data, c)
                bb.device_sync()                                         # the host rows stay alive until copied
            else:
                bb.append_rows(shape, pages, PAGE_KEYS, pos, dK.ptr + pos * rs, dV.ptr + pos * rs, c)
            pos += c
        bb.device_sync()
        gk, gv = page_bytes(pages, n_pages, PAGE_KEYS * rs)
        assert np.array_equal(gk[:n * rs], K) and np.array_equal(gv[:n * rs], V)
    finally:
        pages.close()


def test_append_rows_store_f16():
    """q8_0 rows stored as f16 rows (store_f16), then attention over the f16 pages meets the bar against the oracle."""
    nkv, hd, rows = 8, 128, 8
    hb = orc.head_bytes(bb.FMT_Q8_0, hd); rs = nkv * hb
    srs = nkv * hd * 2
    n = sum(CHUNKS)
    print(f"append_rows store_f16 n={n}", flush=True)
    K = orc.fill_rows(23, bb.FMT_Q8_0, nkv, hd, n, rs=rs, n_outliers=4, outlier_mul=8.0)
    V = orc.fill_rows(24, bb.FMT_Q8_0, nkv, hd, n, rs=rs)
    shape = bb.make_shape(nkv, rows, hd, bb.FMT_Q8_0, rs=rs)
    n_pages = (n + PAGE_KEYS - 1) // PAGE_KEYS
    pages = bb.alloc_pages(n_pages, PAGE_KEYS * srs)
    dK, dV = bb.DeviceBuffer.from_array(K), bb.DeviceBuffer.from_array(V)
    dq = do = dml = None
    try:
        pos = 0
        for c in CHUNKS:
            bb.append_rows(shape, pages, PAGE_KEYS, pos, dK.ptr + pos * rs, dV.ptr + pos * rs, c, store_f16=True)
            pos += c
        bb.device_sync()
        gk, gv = page_bytes(pages, n_pages, PAGE_KEYS * srs)
        ek = orc.store_rows_f16(K, n, nkv, hd, rs, hb).view(np.uint8).reshape(-1)
        ev = orc.store_rows_f16(V, n, nkv, hd, rs, hb).view(np.uint8).reshape(-1)
        assert np.array_equal(gk[:n * srs], ek) and np.array_equal(gv[:n * srs], ev)
        # attention over the stored f16 rows (the reference engines' rounding) against the oracle on the same bytes
        pages.nkeys = [min(PAGE_KEYS, n - i * PAGE_KEYS) for i in range(n_pages)]
        s16 = bb.make_shape(nkv, rows, hd, bb.FMT_F16, bb.QMODE_F16, rs=srs)
        Q = orc.normal(25, 0, nkv * rows * hd).reshape(nkv * rows, hd)
        dq = bb.DeviceBuffer.from_array(Q); do = bb.DeviceBuffer(nkv * rows * hd * 4); dml = bb.DeviceBuffer(nkv * rows * 8)
        ws = bb.Workspace()
        ws.attn(s16, pages, dq.ptr, do.ptr, dml.ptr, dml.ptr + nkv * rows * 4)
        bb.device_sync()
        ws.close()
        O = do.download(np.float32).reshape(nkv * rows, hd); ml = dml.download(np.float32)
        ref = orc.attn_exact(orc.make_shape(nkv, rows, hd, orc.F16, orc.QMODE_F16, rs=srs), Q, ek, ev, n)
        eo, em, el = orc.rel_err(O, ml[:nkv * rows], ml[nkv * rows:], *ref)
        assert eo < 2e-3 and em < 2e-3 and el < 2e-3, (eo, em, el)
    finally:
        pages.close()


@pytest.mark.parametrize("fmt", [bb.FMT_Q8_0, bb.FMT_Q4_0, bb.FMT_F16])
@pytest.mark.parametrize("hd", [128, 256])
def test_append_f32(fmt, hd):
    """fp32 keys quantized on the device into page rows: the oracle's quantizer bytes in the row layout, bit for bit
    (padding bytes past nkv*hb left as they were)."""
    nkv = 4
    hb = orc.head_bytes(fmt, hd); rs = nkv * hb + 16
    n = sum(CHUNKS)
    print(f"append_f32 fmt={fmt} hd={hd} n={n}", flush=True)
    X = (orc.normal(26, 0, n * nkv * hd) * 3).reshape(n, nkv, hd).astype(np.float32)
    Y = orc.normal(27, 0, n * nkv * hd).reshape(n, nkv, hd).astype(np.float32)
    X[5, 1, :32] = 0.0                                                   # an all-zero block (d = 0, q4_0's -0 scale)
    X[6, 0, 3] = 100.0                                                   # an outlier
    shape = bb.make_shape(nkv, 8, hd, fmt, rs=rs)
    n_pages = (n + PAGE_KEYS - 1) // PAGE_KEYS
    pages = bb.alloc_pages(n_pages, PAGE_KEYS * rs)
    for b in pages.bufs:                                                 # padding bytes must stay zero
        b.upload(np.zeros(b.nbytes, np.uint8))
    dX, dY = bb.DeviceBuffer.from_array(X), bb.DeviceBuffer.from_array(Y)
    try:
        pos = 0
        for c in CHUNKS:
            bb.append_f32(shape, pages, PAGE_KEYS, pos, dX.ptr + pos * nkv * hd * 4, dY.ptr + pos * nkv * hd * 4, c)
            pos += c
        bb.device_sync()
        gk, gv = page_bytes(pages, n_pages, PAGE_KEYS * rs)
        assert np.array_equal(gk[:n * rs], orc.rows_from_f32(fmt, X, rs, hb))
        assert np.array_equal(gv[:n * rs], orc.rows_from_f32(fmt, Y, rs, hb))
    finally:
        pages.close()


def test_append_rejects_positions_past_the_pages():
    shape = bb.make_shape(8, 8, 128, bb.FMT_Q8_0)
    pages = bb.alloc_pages(1, PAGE_KEYS * shape.rs)
    try:
        with pytest.raises(bb.PaHipError, match="past the last page"):
            bb.append_rows(shape, pages, PAGE_KEYS, 90, 1, 1, 11)        # never dereferenced: rejected on the host
    finally:
        pages.close()
