"""KV ingest on the CPU: the oracle's store_rows f16 conversion (phone-attn.h:305-319) and the row layout of quantized
fp32 keys, pinned by the already-pinned dequantizer and fp16 conversion, and by the quantizers' error bounds."""
import numpy as np

import oracle as orc


def test_store_rows_f16_is_f16_of_dequantized_rows():
    nkv, hd, n = 3, 128, 50
    hb = orc.head_bytes(orc.Q8_0, hd); rs = nkv * hb + 16                   # padded rows
    rows = orc.fill_rows(3, orc.Q8_0, nkv, hd, n, rs=rs, n_outliers=2, outlier_mul=8.0)
    got = orc.store_rows_f16(rows, n, nkv, hd, rs, hb)
    R = rows.reshape(n, rs)
    for h in range(nkv):
        deq = orc.dequantize(orc.Q8_0, np.ascontiguousarray(R[:, h * hb:(h + 1) * hb]).reshape(-1), n * hd)
        assert np.array_equal(got[:, h * hd:(h + 1) * hd], orc.f32_to_f16(deq).reshape(n, hd))


def test_rows_from_f32_layout_and_error_bound():
    nkv, hd, n = 2, 256, 20
    X = orc.normal(8, 0, n * nkv * hd).reshape(n, nkv, hd).astype(np.float32)
    # steps: q8_0 d/2 with d = amax/127, q4_0 d (the clamp at 15) with d = amax/8, plus |q| times the fp16 rounding of
    # d; f16 half an ulp
    for fmt, bound in ((orc.Q8_0, (0.5 + 127 * 2.0 ** -11) / 127), (orc.Q4_0, (1.0 + 8 * 2.0 ** -11) / 8),
                       (orc.F16, 2.0 ** -11)):
        hb = orc.head_bytes(fmt, hd); rs = nkv * hb + 8
        rows = orc.rows_from_f32(fmt, X, rs, hb).reshape(n, rs)
        assert np.all(rows[:, nkv * hb:] == 0)                               # row padding untouched
        for h in range(nkv):
            b = np.ascontiguousarray(rows[:, h * hb:(h + 1) * hb]).reshape(-1)
            deq = orc.dequantize(fmt, b, n * hd) if fmt != orc.F16 else orc.f16_to_f32(b.view(np.uint16))
            x = X[:, h, :].reshape(-1)
            amax = np.abs(x.reshape(-1, 32)).max(axis=1).repeat(32)
            assert np.all(np.abs(deq - x) <= bound * (amax if fmt != orc.F16 else np.abs(x)) * 1.0001 + 1e-30)


def test_ingest_rejects_misaligned_rows_pages_and_buffers():
    """The ingest kernels store 16-bit (q8_0, q4_0) or 32-bit (f16) words: odd strides, misaligned pages and a misaligned
    quantizer output are rejected on the host with a message, before any device call (the pointers here are never
    dereferenced)."""
    import pytest
    import backburner_amd as bb
    good = bb.Pages([0x10000], [0x20000], [0], [])
    odd = bb.make_shape(2, 8, 128, bb.FMT_Q8_0, rs=2 * 136 + 1)
    with pytest.raises(bb.PaHipError, match="multiples of 2"):
        bb.append_f32(odd, good, 100, 0, 0x30000, 0x40000, 3)
    f16 = bb.make_shape(2, 8, 128, bb.FMT_F16, rs=2 * 256 + 2)
    with pytest.raises(bb.PaHipError, match="multiples of 4"):
        bb.append_f32(f16, good, 100, 0, 0x30000, 0x40000, 3)
    shape = bb.make_shape(2, 8, 128, bb.FMT_Q8_0)
    with pytest.raises(bb.PaHipError, match="not 2-byte aligned"):
        bb.append_f32(shape, bb.Pages([0x10001], [0x20000], [0], []), 100, 0, 0x30000, 0x40000, 3)
    with pytest.raises(bb.PaHipError, match="not 4-byte aligned"):
        bb.append_rows(shape, bb.Pages([0x10002], [0x20000], [0], []), 100, 0, 0x30000, 0x40000, 3, store_f16=True)
    with pytest.raises(bb.PaHipError, match="2-byte aligned"):
        bb.quantize_device(bb.FMT_Q8_0, 0x30000, 0x40001, 64)
