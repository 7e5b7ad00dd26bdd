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
