"""Python view of the CPU oracle (liboracle.so, pa_oracle.c). TEST INFRASTRUCTURE ONLY: imported by tests/, by
__graft_entry__.smoke() and by bench.py's cpu_baseline leg, as the reference for parity checks or the timed CPU
baseline - never by the product package.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

F16, Q8_0, Q4_0 = 0, 1, 2
QMODE_GGML, QMODE_F16, QMODE_EXACT = 0, 1, 2


class Shape(C.Structure):
    _fields_ = [("nkv", C.c_uint32), ("rows", C.c_uint32), ("hd", C.c_uint32), ("fmt", C.c_uint32),
                ("rs", C.c_uint32), ("hb", C.c_uint32), ("qmode", C.c_uint32), ("scale", C.c_float)]


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB.exists():
        raise RuntimeError("oracle/liboracle.so is not built (make -C oracle)")
    L = C.CDLL(str(LIB))
    vp, i64 = C.c_void_p, C.c_int64
    L.orc_f32_to_f16.restype = C.c_uint16
    L.orc_f32_to_f16.argtypes = [C.c_float]
    L.orc_f16_to_f32.restype = C.c_float
    L.orc_f16_to_f32.argtypes = [C.c_uint16]
    for f in ("orc_f32_to_f16_n", "orc_f16_to_f32_n"):
        getattr(L, f).argtypes = [vp, vp, i64]
    L.orc_head_bytes.restype = C.c_uint32
    L.orc_head_bytes.argtypes = [C.c_int, C.c_int]
    for f in ("orc_quantize_q8_0", "orc_quantize_q4_0", "orc_quantize_q8_0_patool", "orc_quantize_q4_0_patool"):
        getattr(L, f).argtypes = [vp, vp, i64]
    L.orc_dequantize.argtypes = [C.c_int, vp, vp, i64]
    L.orc_quantize.argtypes = [C.c_int, vp, vp, i64]
    L.orc_normal.argtypes = [C.c_uint64, i64, i64, vp]
    L.orc_fill_rows.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_int, C.c_uint32, i64, i64, C.c_float, C.c_int, C.c_float, vp]
    L.orc_outlier_channels.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_int, vp]
    L.orc_attn_exact.argtypes = [C.POINTER(Shape), vp, vp, vp, i64, vp, vp, vp, C.c_int]
    L.orc_attn_ggml.argtypes = [C.POINTER(Shape), vp, vp, vp, i64, vp, vp, vp, C.c_int]
    L.orc_attn_ggml_simd.restype = C.c_char_p
    L.orc_attn_ggml_simd.argtypes = [C.POINTER(Shape), vp, vp, vp, i64, vp, vp, vp, C.c_int, C.c_int]
    L.orc_simd_path.restype = C.c_char_p
    L.orc_simd_path.argtypes = []
    L.orc_merge_partial.argtypes = [vp, vp, vp, vp, vp, vp, i64, C.c_int]
    L.orc_normalise.argtypes = [vp, vp, vp, i64, C.c_int, vp, vp]
    L.orc_coattn_merge.argtypes = [vp, vp, vp, vp, vp, i64, C.c_int, vp, vp]
    L.orc_store_rows_f16.argtypes = [vp, i64, C.c_int, C.c_int, C.c_uint32, C.c_uint32, vp]
    L.orc_accept.argtypes = [vp, C.c_int, i64, vp, vp, vp, vp]
    L.orc_quantize_q_row.argtypes = [vp, C.c_int, vp]
    _lib = L
    return L


def _p(a: np.ndarray):
    assert a.flags.c_contiguous
    return a.ctypes.data


def head_bytes(fmt: int, hd: int) -> int:
    return int(lib().orc_head_bytes(fmt, hd))


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_n(_p(x), _p(y), x.size)
    return y


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, np.uint16)
    y = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_n(_p(h), _p(y), h.size)
    return y


def quantize(fmt: int, x: np.ndarray, variant: str = "ggml") -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    n = x.size
    nb = head_bytes(fmt, 32) * (n // 32) if fmt != F16 else 2 * n
    y = np.empty(nb, np.uint8)
    if variant == "ggml":
        lib().orc_quantize(fmt, _p(x), _p(y), n)
    elif fmt == Q8_0:
        lib().orc_quantize_q8_0_patool(_p(x), _p(y), n)
    else:
        lib().orc_quantize_q4_0_patool(_p(x), _p(y), n)
    return y


def dequantize(fmt: int, y: np.ndarray, n: int) -> np.ndarray:
    y = np.ascontiguousarray(y, np.uint8)
    x = np.empty(n, np.float32)
    lib().orc_dequantize(fmt, _p(y), _p(x), n)
    return x


def normal(seed: int, i0: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_normal(seed, i0, n, _p(out))
    return out


def fill_rows(seed: int, fmt: int, nkv: int, hd: int, n_keys: int, rs: int | None = None, j0: int = 0, amp: float = 1.0,
              n_outliers: int = 0, outlier_mul: float = 8.0) -> np.ndarray:
    hb = head_bytes(fmt, hd)
    rs = rs if rs is not None else nkv * hb
    rows = np.zeros(n_keys * rs, np.uint8)
    lib().orc_fill_rows(seed, fmt, nkv, hd, rs, j0, n_keys, amp, n_outliers, outlier_mul, _p(rows))
    return rows


def outlier_channels(seed: int, nkv: int, hd: int, n_outliers: int) -> np.ndarray:
    ch = np.zeros((nkv, n_outliers), np.int32)
    lib().orc_outlier_channels(seed, nkv, hd, n_outliers, _p(ch))
    return ch


def make_shape(nkv, rows, hd, fmt, qmode=QMODE_GGML, scale=None, rs=None) -> Shape:
    hb = head_bytes(fmt, hd)
    return Shape(nkv, rows, hd, fmt, rs if rs is not None else nkv * hb, hb, qmode,
                 float(scale) if scale is not None else float(1.0 / np.sqrt(hd)))


def attn_exact(s: Shape, Q: np.ndarray, K: np.ndarray, V: np.ndarray, nk: int, threads: int = 0):
    rows = s.nkv * s.rows
    Q = np.ascontiguousarray(Q, np.float32)
    O = np.empty((rows, s.hd), np.float64)
    m = np.empty(rows, np.float64)
    l = np.empty(rows, np.float64)
    lib().orc_attn_exact(C.byref(s), _p(Q), _p(np.ascontiguousarray(K)), _p(np.ascontiguousarray(V)), nk, _p(O), _p(m), _p(l), threads)
    return O, m, l


def attn_ggml(s: Shape, Q: np.ndarray, K: np.ndarray, V: np.ndarray, nk: int, threads: int = 0):
    rows = s.nkv * s.rows
    Q = np.ascontiguousarray(Q, np.float32)
    O = np.empty((rows, s.hd), np.float32)
    m = np.empty(rows, np.float32)
    l = np.empty(rows, np.float32)
    lib().orc_attn_ggml(C.byref(s), _p(Q), _p(np.ascontiguousarray(K)), _p(np.ascontiguousarray(V)), nk, _p(O), _p(m), _p(l), threads)
    return O, m, l


def attn_ggml_simd(s: Shape, Q: np.ndarray, K: np.ndarray, V: np.ndarray, nk: int, threads: int = 0, level: int = -1):
    """The CPU baseline: attn_ggml's arithmetic, vectorized (AVX-512 VNNI / AVX2); equal to attn_ggml bit for bit.
    Returns (O, m, l, simd path)."""
    rows = s.nkv * s.rows
    Q = np.ascontiguousarray(Q, np.float32)
    O = np.empty((rows, s.hd), np.float32)
    m = np.empty(rows, np.float32)
    l = np.empty(rows, np.float32)
    path = lib().orc_attn_ggml_simd(C.byref(s), _p(Q), _p(np.ascontiguousarray(K)), _p(np.ascontiguousarray(V)), nk, _p(O), _p(m),
                                    _p(l), threads, level)
    return O, m, l, path.decode()


def simd_path() -> str:
    return lib().orc_simd_path().decode()


def merge_partial(O, m, l, O2, m2, l2):
    """In place on (O, m, l) float32 arrays (phone-attn.h:231-239)."""
    rows, hd = O.shape
    lib().orc_merge_partial(_p(O), _p(m), _p(l), _p(O2), _p(m2), _p(l2), rows, hd)


def normalise(O, m, l):
    O = np.ascontiguousarray(O, np.float32)
    m = np.ascontiguousarray(m, np.float32); l = np.ascontiguousarray(l, np.float32)
    rows, hd = O.shape
    Oh = np.empty((rows, hd), np.uint16)
    lse = np.empty(rows, np.float32)
    lib().orc_normalise(_p(O), _p(m), _p(l), rows, hd, _p(Oh), _p(lse))
    return Oh, lse


def store_rows_f16(rows: np.ndarray, n: int, nkv: int, hd: int, rs: int, hb: int) -> np.ndarray:
    """store_rows' q8_0 -> f16 conversion (phone-attn.h:305-319): the stored rows as fp16 bits [n][nkv*hd]."""
    rows = np.ascontiguousarray(rows, np.uint8)
    out = np.empty((n, nkv * hd), np.uint16)
    lib().orc_store_rows_f16(_p(rows), n, nkv, hd, rs, hb, _p(out))
    return out


def rows_from_f32(fmt: int, X: np.ndarray, rs: int, hb: int) -> np.ndarray:
    """fp32 [n][nkv][hd] -> the row bytes [n*rs] of that format (each head's hd values quantized as one row, padding 0)."""
    n, nkv, hd = X.shape
    out = np.zeros((n, rs), np.uint8)
    for h in range(nkv):
        q = quantize(fmt, np.ascontiguousarray(X[:, h, :]).reshape(-1)) if fmt != F16 else \
            f32_to_f16(X[:, h, :].reshape(-1)).view(np.uint8)
        out[:, h * hb:h * hb + head_bytes(fmt, hd)] = q.reshape(n, -1)
    return out.reshape(-1)


def coattn_merge(Oh, lse, O_loc, m_loc, l_loc):
    """The receiver's merge of a reply (Oh fp16 bits, lse) with its partial (O_loc, m_loc, l_loc): (out, lse_out)."""
    rows, hd = O_loc.shape
    Oh = np.ascontiguousarray(Oh, np.uint16); lse = np.ascontiguousarray(lse, np.float32)
    O_loc = np.ascontiguousarray(O_loc, np.float32)
    m_loc = np.ascontiguousarray(m_loc, np.float32); l_loc = np.ascontiguousarray(l_loc, np.float32)
    out = np.empty((rows, hd), np.float32)
    lse_out = np.empty(rows, np.float32)
    lib().orc_coattn_merge(_p(Oh), _p(lse), _p(O_loc), _p(m_loc), _p(l_loc), rows, hd, _p(out), _p(lse_out))
    return out, lse_out


def accept(logits: np.ndarray, draft: np.ndarray):
    logits = np.ascontiguousarray(logits, np.float32)
    n_rows, vocab = logits.shape
    draft = np.ascontiguousarray(draft, np.int32)
    am = np.empty(n_rows, np.int32)
    k = np.zeros(1, np.int32)
    b = np.zeros(1, np.int32)
    lib().orc_accept(_p(logits), n_rows, vocab, _p(draft), _p(am), _p(k), _p(b))
    return int(k[0]), int(b[0]), am


def rel_err(O, m, l, O_ref, m_ref, l_ref):
    """Per-row comparison of unnormalised partials: rebase (O, l) to the reference max, then
    (max_row max|O - O_ref| / max|O_ref|, max |m - m_ref| / max(1, |m_ref|), max |l - l_ref| / l_ref)."""
    O = np.asarray(O, np.float64); O_ref = np.asarray(O_ref, np.float64)
    m = np.asarray(m, np.float64); m_ref = np.asarray(m_ref, np.float64)
    l = np.asarray(l, np.float64); l_ref = np.asarray(l_ref, np.float64)
    live = np.isfinite(m_ref) & (l_ref > 0)
    eo = em = el = 0.0
    if live.any():
        f = np.exp(m[live] - m_ref[live])
        Ob = O[live] * f[:, None]
        den = np.maximum(np.abs(O_ref[live]).max(axis=1), 1e-30)
        eo = float((np.abs(Ob - O_ref[live]).max(axis=1) / den).max())
        em = float((np.abs(m[live] - m_ref[live]) / np.maximum(1.0, np.abs(m_ref[live]))).max())
        el = float((np.abs(l[live] * f - l_ref[live]) / l_ref[live]).max())
    dead = ~live
    if dead.any():   # empty rows must be exactly (0, -inf, 0)
        if not (np.all(O[dead] == 0) and np.all(l[dead] == 0) and np.all(np.isneginf(m[dead]))):
            eo = em = el = float("inf")
    return eo, em, el
