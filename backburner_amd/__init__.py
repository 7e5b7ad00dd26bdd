"""backburner_amd - phone-attn's old-KV partial attention on MI355X (gfx950).

Python side of the C ABI in include/phone_attn_hip.h (libpa_hip.so). It mirrors the reference's plug-in interface for
this path: the C-ABI engine (phone-attn/phone-attn.h:63-71: sme_ws_new, sme_attn_partial, sme2_available, sme_pipe_new,
sme_attn_pipe) with host numpy buffers, and the device-resident engine call (the role of pa::engine::begin/end,
phone-attn.h:166-183) over HBM pages.

All compute runs in the HIP kernels of libpa_hip.so. If the library is missing or no gfx950 device is present, every
call raises; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_HIP = PKG / "libpa_hip.so"
LIB_SYNTH = PKG / "libpa_synth.so"

FMT_F16, FMT_Q8_0, FMT_Q4_0 = 0, 1, 2          # config_req.is_q8 (phone-attn.h:15, 88)
QMODE_GGML, QMODE_F16 = 0, 1
PAGE = 4096                                      # keys per page (phone-attn.h:160)


def head_bytes(fmt: int, hd: int) -> int:
    """Bytes of one head's slice of a key row: q8_0 hd/32*34, q4_0 hd/32*18, f16 hd*2 (pa-tool.cpp:41-51)."""
    return hd // 32 * 34 if fmt == FMT_Q8_0 else hd // 32 * 18 if fmt == FMT_Q4_0 else hd * 2


class PaHipError(RuntimeError):
    pass


class Shape(C.Structure):
    """pa_hip_shape: nkv, rows per KV head, hd, fmt, rs, hb, qmode, scale."""
    _fields_ = [("nkv", C.c_uint32), ("rows", C.c_uint32), ("hd", C.c_uint32), ("fmt", C.c_uint32),
                ("rs", C.c_uint32), ("hb", C.c_uint32), ("qmode", C.c_uint32), ("scale", C.c_float)]


_hip = None
_synth = None


def _load(path: Path) -> C.CDLL:
    if not path.exists():
        raise PaHipError(f"{path.name} is not built: run `python -m backburner_amd.build` (or __graft_entry__.build())")
    return C.CDLL(str(path))


def lib() -> C.CDLL:
    """libpa_hip.so with argument types set."""
    global _hip
    if _hip is not None:
        return _hip
    L = _load(LIB_HIP)
    vp, f32p, u8p = C.c_void_p, C.POINTER(C.c_float), C.c_void_p
    L.sme_ws_new.restype = vp
    L.sme_ws_new.argtypes = []
    L.sme_attn_partial.restype = None
    L.sme_attn_partial.argtypes = [vp, f32p, C.c_int, u8p, u8p, C.c_size_t, C.c_int, C.c_int, C.c_float, C.c_int, f32p, f32p, f32p]
    L.sme2_available.restype = C.c_int
    L.sme2_available.argtypes = []
    L.sme_pipe_new.restype = vp
    L.sme_pipe_new.argtypes = [C.c_int]
    L.sme_attn_pipe.restype = None
    L.sme_attn_pipe.argtypes = [C.POINTER(vp), C.c_int, C.c_int, f32p, u8p, u8p, C.c_size_t, C.c_size_t, C.c_int, C.c_int,
                                C.c_int, C.c_float, f32p, f32p, f32p]
    L.pa_hip_last_error.restype = C.c_char_p
    L.pa_hip_last_error.argtypes = []
    L.pa_hip_set_compat_shape.restype = C.c_int
    L.pa_hip_set_compat_shape.argtypes = [C.c_int, C.c_int]
    L.pa_hip_ws_free.restype = None
    L.pa_hip_ws_free.argtypes = [vp]
    L.pa_hip_stream_wait.restype = C.c_int
    L.pa_hip_stream_wait.argtypes = [vp, C.c_int]
    L.pa_hip_shutdown.restype = C.c_int
    L.pa_hip_shutdown.argtypes = [C.c_int]
    L.pa_hip_ws_new.restype = vp
    L.pa_hip_ws_new.argtypes = [C.c_int]
    L.pa_hip_ws_destroy.restype = None
    L.pa_hip_ws_destroy.argtypes = [vp]
    L.pa_hip_alloc_page.restype = C.c_int
    L.pa_hip_alloc_page.argtypes = [C.c_size_t, C.POINTER(vp), C.POINTER(vp)]
    L.pa_hip_free_page.restype = None
    L.pa_hip_free_page.argtypes = [vp, vp]
    L.pa_hip_attn.restype = C.c_int
    L.pa_hip_attn.argtypes = [vp, C.POINTER(Shape), C.POINTER(vp), C.POINTER(vp), C.POINTER(C.c_uint32), C.c_int, vp, vp, vp, vp, vp]
    L.pa_hip_attn_noalloc.restype = C.c_int
    L.pa_hip_attn_noalloc.argtypes = [C.POINTER(Shape), C.POINTER(vp), C.POINTER(vp), C.POINTER(C.c_uint32), C.c_int, vp, vp, vp, vp, vp]
    L.pa_hip_accept.restype = C.c_int
    L.pa_hip_accept.argtypes = [vp, vp, C.c_int, C.c_int64, vp, vp, vp]
    L.pa_hip_ws_set_split.restype = C.c_int
    L.pa_hip_ws_set_split.argtypes = [vp, C.c_int, C.c_int]
    L.pa_hip_ws_set_chunk_keys.restype = C.c_int
    L.pa_hip_ws_set_chunk_keys.argtypes = [vp, C.c_uint32]
    L.pa_hip_warm.restype = C.c_int
    L.pa_hip_warm.argtypes = [vp]
    L.pa_hip_ws_time_next.restype = C.c_int
    L.pa_hip_ws_time_next.argtypes = [vp, vp, vp]
    L.pa_hip_quantize.restype = C.c_int
    L.pa_hip_quantize.argtypes = [C.c_int, vp, vp, C.c_int64, vp]
    L.pa_hip_attn_reply.restype = C.c_int
    L.pa_hip_attn_reply.argtypes = [vp, C.POINTER(Shape), C.POINTER(vp), C.POINTER(vp), C.POINTER(C.c_uint32), C.c_int, vp, vp,
                                    vp, vp]
    L.pa_hip_merge_partial.restype = C.c_int
    L.pa_hip_merge_partial.argtypes = [vp, vp, vp, vp, vp, vp, C.c_uint64, C.c_uint32, vp]
    L.pa_hip_normalise.restype = C.c_int
    L.pa_hip_normalise.argtypes = [vp, vp, vp, C.c_uint64, C.c_uint32, vp, vp, vp]
    L.pa_hip_pack_q.restype = C.c_int
    L.pa_hip_pack_q.argtypes = [vp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp]
    L.pa_hip_unpack_rows.restype = C.c_int
    L.pa_hip_unpack_rows.argtypes = [vp, vp, vp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp, vp, vp]
    L.pa_hip_append_rows.restype = C.c_int
    L.pa_hip_append_rows.argtypes = [C.POINTER(Shape), C.POINTER(vp), C.POINTER(vp), C.c_int, C.c_uint32, C.c_uint32, vp, vp,
                                     C.c_uint32, C.c_int, vp]
    L.pa_hip_append_f32.restype = C.c_int
    L.pa_hip_append_f32.argtypes = [C.POINTER(Shape), C.POINTER(vp), C.POINTER(vp), C.c_int, C.c_uint32, C.c_uint32, vp, vp,
                                    C.c_uint32, vp]
    L.pa_hip_coattn_merge.restype = C.c_int
    L.pa_hip_coattn_merge.argtypes = [vp, vp, vp, vp, vp, C.c_uint64, C.c_uint32, vp, vp, vp]
    _hip = L
    return L


def synth() -> C.CDLL:
    """libpa_synth.so (bench/test support: synthetic HBM pages, device memory, events)."""
    global _synth
    if _synth is not None:
        return _synth
    L = _load(LIB_SYNTH)
    vp = C.c_void_p
    L.pa_synth_normal.restype = C.c_int
    L.pa_synth_normal.argtypes = [vp, C.c_int64, C.c_uint64, C.c_int64, C.c_float, vp]
    L.pa_synth_fill_rows.restype = C.c_int
    L.pa_synth_fill_rows.argtypes = [vp, C.c_int, C.c_int, C.c_int, C.c_uint32, C.c_int64, C.c_int64, C.c_uint64, C.c_float,
                                     C.c_int, vp, C.c_float, vp]
    L.pa_synth_copy.restype = C.c_int
    L.pa_synth_copy.argtypes = [vp, vp, C.c_int64, C.c_int, vp]
    L.pa_synth_read.restype = C.c_int
    L.pa_synth_read.argtypes = [vp, C.c_int64, C.c_int, vp, vp]
    L.pa_synth_malloc.restype = vp
    L.pa_synth_malloc.argtypes = [C.c_size_t]
    L.pa_synth_free.restype = C.c_int
    L.pa_synth_free.argtypes = [vp]
    L.pa_synth_host_alloc.restype = vp
    L.pa_synth_host_alloc.argtypes = [C.c_size_t]
    L.pa_synth_host_free.restype = C.c_int
    L.pa_synth_host_free.argtypes = [vp]
    L.pa_synth_memset.restype = C.c_int
    L.pa_synth_memset.argtypes = [vp, C.c_int, C.c_size_t]
    L.pa_synth_h2d.restype = C.c_int
    L.pa_synth_h2d.argtypes = [vp, vp, C.c_size_t]
    L.pa_synth_d2h.restype = C.c_int
    L.pa_synth_d2h.argtypes = [vp, vp, C.c_size_t]
    L.pa_synth_sync.restype = C.c_int
    L.pa_synth_error.restype = C.c_char_p
    L.pa_synth_device_name.restype = C.c_int
    L.pa_synth_device_name.argtypes = [C.c_char_p, C.c_int]
    L.pa_synth_stream_new.restype = vp
    L.pa_synth_stream_sync.restype = C.c_int
    L.pa_synth_stream_sync.argtypes = [vp]
    L.pa_synth_event_new.restype = vp
    L.pa_synth_event_record.restype = C.c_int
    L.pa_synth_event_record.argtypes = [vp, vp]
    L.pa_synth_event_ms.restype = C.c_float
    L.pa_synth_event_ms.argtypes = [vp, vp]
    L.pa_synth_event_free.restype = C.c_int
    L.pa_synth_event_free.argtypes = [vp]
    L.pa_synth_capture_begin.restype = C.c_int
    L.pa_synth_capture_begin.argtypes = [vp]
    L.pa_synth_capture_end.restype = vp
    L.pa_synth_capture_end.argtypes = [vp]
    L.pa_synth_graph_launch.restype = C.c_int
    L.pa_synth_graph_launch.argtypes = [vp, vp]
    L.pa_synth_graph_free.restype = C.c_int
    L.pa_synth_graph_free.argtypes = [vp]
    _synth = L
    return L


def last_error() -> str:
    return lib().pa_hip_last_error().decode()


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise PaHipError(f"{what}: {last_error()}")


def _fp(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_float))


# ---------------------------------------------------------------- device memory (through libpa_synth)
class DeviceBuffer:
    """A hipMalloc'd buffer of `nbytes`; freed on close()/del."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = synth().pa_synth_malloc(max(self.nbytes, 1))
        if not self.ptr:
            raise PaHipError(f"hipMalloc({nbytes}) failed: {synth().pa_synth_error().decode()}")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        if a.nbytes and synth().pa_synth_h2d(self.ptr + offset, a.ctypes.data, a.nbytes) != 0:
            raise PaHipError("hipMemcpy H2D failed")

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        n = (self.nbytes - offset) // dtype.itemsize if count is None else int(count)
        out = np.empty(n, dtype)
        if out.nbytes and synth().pa_synth_d2h(out.ctypes.data, self.ptr + offset, out.nbytes) != 0:
            raise PaHipError("hipMemcpy D2H failed")
        return out

    def close(self) -> None:
        if getattr(self, "ptr", None):
            synth().pa_synth_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class PinnedArray:
    """A numpy array over pinned host memory (hipHostMalloc), as the HIP server engine's pages are; freed on close()."""

    def __init__(self, a: np.ndarray):
        a = np.ascontiguousarray(a)
        self.ptr = synth().pa_synth_host_alloc(max(a.nbytes, 1))
        if not self.ptr:
            raise PaHipError(f"hipHostMalloc({a.nbytes}) failed")
        self.array = np.ctypeslib.as_array((C.c_uint8 * a.nbytes).from_address(self.ptr)).view(a.dtype).reshape(a.shape)
        self.array[...] = a

    def close(self) -> None:
        if getattr(self, "ptr", None):
            self.array = None
            synth().pa_synth_host_free(self.ptr)
            self.ptr = None


def device_sync() -> None:
    if synth().pa_synth_sync() != 0:
        raise PaHipError(f"hipDeviceSynchronize failed: {synth().pa_synth_error().decode()}")


# ---------------------------------------------------------------- reference C ABI (host buffers)
def sme2_available() -> int:
    return int(lib().sme2_available())


def sme_ws_new() -> int:
    w = lib().sme_ws_new()
    if not w:
        raise PaHipError(f"sme_ws_new: {last_error()}")
    return w


def sme_pipe_new(nh: int = 1) -> int:
    w = lib().sme_pipe_new(nh)
    if not w:
        raise PaHipError(f"sme_pipe_new: {last_error()}")
    return w


def set_compat_shape(nr: int, hd: int) -> None:
    _check(lib().pa_hip_set_compat_shape(nr, hd), "pa_hip_set_compat_shape")


def sme_attn_partial(w, Q: np.ndarray, qrs: int, K: np.ndarray, V: np.ndarray, rs: int, is_q8: int, nk: int, scale: float,
                     bk: int, O: np.ndarray, m: np.ndarray, l: np.ndarray, k_off: int = 0) -> None:
    """sme_attn.c:271-306: one KV head; K/V are the page byte arrays and k_off the head's byte offset (h*hb)."""
    assert Q.dtype == np.float32 and O.dtype == np.float32 and m.dtype == np.float32 and l.dtype == np.float32
    lib().sme_attn_partial(w, _fp(Q), qrs, K.ctypes.data + k_off, V.ctypes.data + k_off, rs, is_q8, nk, scale, bk,
                           _fp(O), _fp(m), _fp(l))


def sme_attn_pipe(pp: list, Q: np.ndarray, K: np.ndarray, V: np.ndarray, rs: int, hb: int, is_q8: int, nkv: int, nk: int,
                  scale: float, O: np.ndarray, m: np.ndarray, l: np.ndarray, nw: int = 1, nh: int = 1) -> None:
    """sme_attn.c:437-463: all nkv heads in one call."""
    arr = (C.c_void_p * len(pp))(*pp)
    lib().sme_attn_pipe(arr, nw, nh, _fp(Q), K.ctypes.data, V.ctypes.data, rs, hb, is_q8, nkv, nk, scale, _fp(O), _fp(m), _fp(l))


# ---------------------------------------------------------------- device-resident engine path
@dataclass
class Pages:
    """HBM pages of one layer: K and V device pointers and the keys each holds (engine::alloc_page, phone-attn.h:168)."""
    k: list
    v: list
    nkeys: list
    bufs: list

    def close(self) -> None:
        for b in self.bufs:
            b.close()


class Workspace:
    """pa_hip_ws: split-K partials and prepared Q of one stream."""

    def __init__(self, device: int = 0):
        self.ptr = lib().pa_hip_ws_new(device)
        if not self.ptr:
            raise PaHipError(f"pa_hip_ws_new: {last_error()}")

    def attn(self, shape: Shape, pages: Pages, Q: int, O: int, m: int, l: int, stream=None) -> None:
        """Enqueue pa_hip_attn over the pages (Q, O, m, l are device pointers)."""
        n = len(pages.k)
        kp = (C.c_void_p * max(n, 1))(*pages.k)
        vp = (C.c_void_p * max(n, 1))(*pages.v)
        nk = (C.c_uint32 * max(n, 1))(*pages.nkeys)
        _check(lib().pa_hip_attn(self.ptr, C.byref(shape), kp, vp, nk, n, Q, O, m, l, stream), "pa_hip_attn")

    def attn_reply(self, shape: Shape, pages: Pages, Q: int, Oh: int, lse: int, stream=None) -> None:
        """Enqueue pa_hip_attn_reply: the call's reply format (f16 O / l, lse) at the device pointers Oh, lse."""
        n = len(pages.k)
        kp = (C.c_void_p * max(n, 1))(*pages.k)
        vp = (C.c_void_p * max(n, 1))(*pages.v)
        nk = (C.c_uint32 * max(n, 1))(*pages.nkeys)
        _check(lib().pa_hip_attn_reply(self.ptr, C.byref(shape), kp, vp, nk, n, Q, Oh, lse, stream), "pa_hip_attn_reply")

    def set_split(self, decode_groups: int = 0, mma_workgroups: int = 0) -> None:
        """pa_hip_ws_set_split: force the split-K geometry of this workspace's calls (0 = default)."""
        _check(lib().pa_hip_ws_set_split(self.ptr, decode_groups, mma_workgroups), "pa_hip_ws_set_split")

    def set_chunk_keys(self, keys: int = 0) -> None:
        """pa_hip_ws_set_chunk_keys: about `keys` keys per workgroup's split-K chunk (config_req.gpu_chunk; 0 = default)."""
        _check(lib().pa_hip_ws_set_chunk_keys(self.ptr, keys), "pa_hip_ws_set_chunk_keys")

    def time_next(self, ev_start, ev_end) -> None:
        """Record ev_start / ev_end around the attention kernel of the next attn() call."""
        _check(lib().pa_hip_ws_time_next(self.ptr, ev_start, ev_end), "pa_hip_ws_time_next")

    def accept(self, logits: int, n_rows: int, vocab: int, draft: int, out: int, stream=None) -> None:
        _check(lib().pa_hip_accept(self.ptr, logits, n_rows, vocab, draft, out, stream), "pa_hip_accept")

    def close(self) -> None:
        if self.ptr:
            lib().pa_hip_ws_destroy(self.ptr)
            self.ptr = None


def attn_noalloc(shape: Shape, pages: Pages, Q: int, O: int, m: int, l: int, stream=None) -> None:
    """Enqueue pa_hip_attn_noalloc (no workspace, nothing allocated; the split-K partials use the library's fixed
    per-GPU scratch)."""
    n = len(pages.k)
    kp = (C.c_void_p * max(n, 1))(*pages.k)
    vp = (C.c_void_p * max(n, 1))(*pages.v)
    nk = (C.c_uint32 * max(n, 1))(*pages.nkeys)
    _check(lib().pa_hip_attn_noalloc(C.byref(shape), kp, vp, nk, n, Q, O, m, l, stream), "pa_hip_attn_noalloc")


def quantize_device(fmt: int, x: int, y: int, n: int, stream=None) -> None:
    _check(lib().pa_hip_quantize(fmt, x, y, n, stream), "pa_hip_quantize")


def merge_partial_device(O: int, m: int, l: int, O2: int, m2: int, l2: int, rows: int, hd: int, stream=None) -> None:
    _check(lib().pa_hip_merge_partial(O, m, l, O2, m2, l2, rows, hd, stream), "pa_hip_merge_partial")


def normalise_device(O: int, m: int, l: int, rows: int, hd: int, Oh: int, lse: int, stream=None) -> None:
    _check(lib().pa_hip_normalise(O, m, l, rows, hd, Oh, lse, stream), "pa_hip_normalise")


def pack_q_device(qs: int, ng: int, nkv: int, nr: int, hd: int, ntok: int, q: int, stream=None) -> None:
    _check(lib().pa_hip_pack_q(qs, ng, nkv, nr, hd, ntok, q, stream), "pa_hip_pack_q")


def unpack_rows_device(O: int, m: int, l: int, ng: int, nkv: int, nr: int, hd: int, ntok: int, Os: int, ms: int, ls: int,
                       stream=None) -> None:
    _check(lib().pa_hip_unpack_rows(O, m, l, ng, nkv, nr, hd, ntok, Os, ms, ls, stream), "pa_hip_unpack_rows")


def coattn_merge_device(Oh: int, lse: int, O_loc: int, m_loc: int, l_loc: int, rows: int, hd: int, out: int, lse_out=None,
                        stream=None) -> None:
    _check(lib().pa_hip_coattn_merge(Oh, lse, O_loc, m_loc, l_loc, rows, hd, out, lse_out, stream), "pa_hip_coattn_merge")


def append_rows(shape: Shape, pages: Pages, page_keys: int, pos0: int, K: int, V: int, n: int, store_f16: bool = False,
                stream=None) -> None:
    """pa_hip_append_rows: n received rows (device or host pointers K, V) into the layer's pages at pos0."""
    m = max(len(pages.k), 1)
    kp = (C.c_void_p * m)(*pages.k); vp = (C.c_void_p * m)(*pages.v)
    _check(lib().pa_hip_append_rows(C.byref(shape), kp, vp, len(pages.k), page_keys, pos0, K, V, n, int(store_f16), stream),
           "pa_hip_append_rows")


def append_f32(shape: Shape, pages: Pages, page_keys: int, pos0: int, K: int, V: int, n: int, stream=None) -> None:
    """pa_hip_append_f32: fp32 K/V [n][nkv][hd] (device pointers) quantized into the pages at pos0."""
    m = max(len(pages.k), 1)
    kp = (C.c_void_p * m)(*pages.k); vp = (C.c_void_p * m)(*pages.v)
    _check(lib().pa_hip_append_f32(C.byref(shape), kp, vp, len(pages.k), page_keys, pos0, K, V, n, stream), "pa_hip_append_f32")


def alloc_pages(n_pages: int, page_bytes: int) -> Pages:
    """n_pages device pages of page_bytes each for K and for V (contents undefined), as engine::alloc_page does."""
    ks, vs, bufs = [], [], []
    for _ in range(n_pages):
        kb = DeviceBuffer(page_bytes); vb = DeviceBuffer(page_bytes)
        ks.append(kb.ptr); vs.append(vb.ptr); bufs += [kb, vb]
    return Pages(ks, vs, [0] * n_pages, bufs)


def make_shape(nkv: int, rows: int, hd: int, fmt: int, qmode: int = QMODE_GGML, scale: float | None = None,
               rs: int | None = None) -> Shape:
    hb = head_bytes(fmt, hd)
    return Shape(nkv, rows, hd, fmt, rs if rs is not None else nkv * hb, hb, qmode,
                 float(scale) if scale is not None else float(1.0 / np.sqrt(hd)))


def pages_from_rows(K: np.ndarray, V: np.ndarray, rs: int, page_keys=PAGE) -> Pages:
    """Upload host rows (bytes [n][rs]) into device pages of `page_keys` keys (a list gives each page's count)."""
    n = len(K) // rs
    counts = list(page_keys) if not isinstance(page_keys, int) else \
        [min(page_keys, n - i) for i in range(0, n, page_keys)] if n else []
    assert sum(counts) == n
    ks, vs, bufs, start = [], [], [], 0
    for c in counts:
        kb = DeviceBuffer(max(c, 1) * rs)
        vb = DeviceBuffer(max(c, 1) * rs)
        kb.upload(K[start * rs:(start + c) * rs])
        vb.upload(V[start * rs:(start + c) * rs])
        ks.append(kb.ptr); vs.append(vb.ptr); bufs += [kb, vb]
        start += c
    return Pages(ks, vs, counts, bufs)


def attn_host(shape: Shape, K: np.ndarray, V: np.ndarray, Q: np.ndarray, page_keys=PAGE, ws: Workspace | None = None):
    """Convenience for tests: upload rows and Q, run pa_hip_attn, return (O, m, l) as numpy arrays."""
    own = ws is None
    ws = ws or Workspace()
    pages = pages_from_rows(K, V, shape.rs, page_keys)
    rows = shape.nkv * shape.rows
    dq = DeviceBuffer.from_array(np.ascontiguousarray(Q, np.float32))
    do = DeviceBuffer(rows * shape.hd * 4)
    dml = DeviceBuffer(rows * 2 * 4)
    try:
        ws.attn(shape, pages, dq.ptr, do.ptr, dml.ptr, dml.ptr + rows * 4)
        device_sync()
        O = do.download(np.float32).reshape(rows, shape.hd)
        ml = dml.download(np.float32)
        return O, ml[:rows].copy(), ml[rows:].copy()
    finally:
        for b in (dq, do, dml):
            b.close()
        pages.close()
        if own:
            ws.close()
