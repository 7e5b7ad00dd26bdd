"""GPU parity at the exact workload shapes, on GPU-made pages, against the CPU oracle on the same bytes (2e-3 relative on
O, m and l; orc_attn_ggml in PA_QMODE_GGML):

- the one-layer decode shape of the ggml-parity workload (8 KV heads x 8 rows, 4,096 q8_0 keys in one page): 64 tile
  groups of two tiles per head pair, then the wide merge;
- the prefill chunk at full size (8 KV heads x 4,096 rows x 65,536 q8_0 keys, 16 pages), the geometry the benchmark
  times (8 heads x 16 row blocks x 2 key chunks, then the few-slot merge), checked on every 16th row of every head and
  row block at all keys, with plain and with x8 outlier-channel keys, and in the reference engines' rounding
  (f16 queries, fp16-dequantized K/V) against the fp64 form;
- the 16-token verify at 98,304 keys with x8 outlier-channel keys;
- more than 256 split-K slots (a decode over 129 pages: two launches, 272 slots, the batched merge);
- pages whose byte size exceeds 2^32 (rows of 4,352 bytes, 2^20 + 100 keys), through the decode and the matrix-core
  kernels;
- head dim 256 calls small enough for a single chunk (the kernel writes the result itself), and the
  reference's own shape (4 KV heads x 48 rows, head dim 256) at 65,536 keys on the head-dim-256 matrix-core kernel.

Every test prints its errors; the margins are recorded in the design notes."""
import numpy as np
import pytest

import backburner_amd as bb
import oracle as orc

pytestmark = pytest.mark.gpu
TOL = 2e-3
PAGE = 4096


@pytest.fixture(scope="module")
def ws():
    w = bb.Workspace()
    yield w
    w.close()


class DevCase:
    """Seeded K/V pages made on the device (the oracle's fill_rows bytes), Q, and the call's outputs."""

    def __init__(self, fmt, nkv, rows, nk, seed, hd=128, rs=None, outliers=0, page_keys=PAGE):
        self.fmt, self.nkv, self.rows, self.nk, self.hd = fmt, nkv, rows, nk, hd
        self.rs = rs if rs is not None else nkv * bb.head_bytes(fmt, hd)
        syn = bb.synth()
        self.kbuf, self.vbuf = bb.DeviceBuffer(nk * self.rs), bb.DeviceBuffer(nk * self.rs)
        self.bufs = [self.kbuf, self.vbuf]
        ch = None
        if outliers:
            ch = bb.DeviceBuffer.from_array(orc.outlier_channels(seed, nkv, hd, outliers))
            self.bufs.append(ch)
        assert syn.pa_synth_fill_rows(self.kbuf.ptr, fmt, nkv, hd, self.rs, 0, nk, seed, 1.0, outliers,
                                      ch.ptr if ch else None, 8.0, None) == 0
        assert syn.pa_synth_fill_rows(self.vbuf.ptr, fmt, nkv, hd, self.rs, 0, nk, seed + 1, 1.0, 0, None, 1.0, None) == 0
        self.Q = orc.normal(seed + 2, 0, nkv * rows * hd).reshape(nkv * rows, hd)
        self.dq = bb.DeviceBuffer.from_array(self.Q)
        n = nkv * rows
        self.do, self.dml = bb.DeviceBuffer(n * hd * 4), bb.DeviceBuffer(n * 8)
        self.bufs += [self.dq, self.do, self.dml]
        sizes = [min(page_keys, nk - i) for i in range(0, nk, page_keys)]
        offs = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
        self.pages = bb.Pages([self.kbuf.ptr + int(o) * self.rs for o in offs], [self.vbuf.ptr + int(o) * self.rs for o in offs],
                              sizes, [])
        bb.device_sync()

    def run(self, ws, qmode=bb.QMODE_GGML):
        ws.attn(bb.make_shape(self.nkv, self.rows, self.hd, self.fmt, qmode, rs=self.rs), self.pages, self.dq.ptr, self.do.ptr,
                self.dml.ptr, self.dml.ptr + self.nkv * self.rows * 4)
        bb.device_sync()
        n = self.nkv * self.rows
        ml = self.dml.download(np.float32)
        return self.do.download(np.float32).reshape(n, self.hd), ml[:n], ml[n:]

    def oracle(self, row_sel=None):
        """orc_attn_ggml over all keys, for the rows row_sel (indices within a KV head; all rows if None)."""
        rows = self.rows if row_sel is None else len(row_sel)
        Q = self.Q if row_sel is None else self.Q.reshape(self.nkv, self.rows, self.hd)[:, row_sel, :].reshape(-1, self.hd)
        K, V = self.kbuf.download(np.uint8), self.vbuf.download(np.uint8)
        return orc.attn_ggml(orc.make_shape(self.nkv, rows, self.hd, self.fmt, orc.QMODE_GGML, rs=self.rs), Q, K, V, self.nk)

    def close(self):
        for b in self.bufs:
            b.close()


def pick(out, nkv, rows, row_sel):
    O, m, l = out
    idx = (np.arange(nkv)[:, None] * rows + np.asarray(row_sel)[None, :]).reshape(-1)
    return O[idx], m[idx], l[idx]


def check(label, got, ref, tol=TOL):
    eo, em, el = orc.rel_err(*got, *ref)
    print(f"{label}: max rel err O {eo:.3e} m {em:.3e} l {el:.3e} (tolerance {tol:g})", flush=True)
    assert eo < tol and em < tol and el < tol, (label, eo, em, el)
    return eo


def test_decode_4096_one_page(ws):
    """8 KV heads x 8 rows (one token, GQA 8) over 4,096 q8_0 keys in one page: 64 two-tile groups per head pair."""
    print("decode 8x8 rows, 4096 q8_0 keys, one page", flush=True)
    c = DevCase(bb.FMT_Q8_0, 8, 8, 4096, 4101)
    try:
        check("decode 4096", c.run(ws), c.oracle())
    finally:
        c.close()


@pytest.mark.parametrize("outliers", [0, 4])
def test_prefill_full_size_sampled_rows(ws, outliers):
    """The prefill chunk as the benchmark runs it: 8 KV heads x 4,096 rows (512 tokens x GQA 8) x 65,536 q8_0 keys in 16
    pages; every 16th row of each head (offset 5, so every row block and every wave's row range is sampled) against the
    oracle at all keys, plain N(0,1) keys and x8 outlier-channel keys, both at the 2e-3 bar (exact integer block dots
    for QK, as ggml computes them)."""
    print(f"prefill full size, outliers={outliers}", flush=True)
    c = DevCase(bb.FMT_Q8_0, 8, 4096, 65536, 4201 + outliers, outliers=outliers)
    try:
        out = c.run(ws)
        sel = np.arange(5, 4096, 16)
        check(f"prefill 65536 outliers={outliers} (rows {len(sel)} of 4096 per head)", pick(out, 8, 4096, sel), c.oracle(sel))
    finally:
        c.close()


def test_prefill_full_size_reference_rounding(ws):
    """The same chunk in the reference engines' rounding (PA_QMODE_F16: queries f16(q*scale), K/V dequantized to fp16
    in LDS, fp16 MFMA with fp32 accumulation - the Metal engine's arithmetic, pa-metal.mm:379-487) on N(0,1) keys:
    every 64th row of each head (offset 9) against the fp64 closed form with the same query rounding, at 2e-3."""
    print("prefill full size, reference rounding", flush=True)
    c = DevCase(bb.FMT_Q8_0, 8, 4096, 65536, 4301)
    try:
        out = c.run(ws, qmode=bb.QMODE_F16)
        sel = np.arange(9, 4096, 64)
        Q = c.Q.reshape(8, 4096, 128)[:, sel, :].reshape(-1, 128)
        ref = orc.attn_exact(orc.make_shape(8, len(sel), 128, orc.Q8_0, orc.QMODE_F16, rs=c.rs), Q,
                             c.kbuf.download(np.uint8), c.vbuf.download(np.uint8), c.nk)
        check(f"prefill 65536 reference rounding (rows {len(sel)} of 4096 per head)", pick(out, 8, 4096, sel), ref)
    finally:
        c.close()


@pytest.mark.parametrize("fmt,nk", [(bb.FMT_Q8_0, 98304), (bb.FMT_Q4_0, 143360)])
def test_verify_full_size_outlier_keys(ws, fmt, nk):
    """16-token verify (8 KV heads x 128 rows) at full size with 4 x8 outlier channels per head in K: larger |q.k|.
    The verify kernel's block dots are exact (integer quants, exact fp16 scale products), so the only roundings left
    are P and V in fp16, as on plain keys (fp16 K and Q operands gave 4.7e-3 / 2.9e-3 here)."""
    print(f"verify full size with outlier keys fmt={fmt} nk={nk}", flush=True)
    c = DevCase(fmt, 8, 128, nk, 4301 + fmt, outliers=4)
    try:
        out = c.run(ws)
        sel = np.arange(128) if fmt == bb.FMT_Q8_0 else np.arange(3, 128, 4)
        check(f"verify {nk} fmt={fmt} outliers", pick(out, 8, 128, sel), c.oracle(sel))
    finally:
        c.close()


@pytest.mark.parametrize("rows", [8, 128])
def test_more_than_256_slots(ws, rows):
    """129 pages of 512 keys: two launches (128 pages, then 1). Decode with 256 tile groups per head pair (the q4_0
    default; set here for q8_0): 256 + 16 = 272 split-K slots per row (the batched merge); verify: 64 + 16 chunks (the
    wide merge over 80 slots)."""
    print(f"129 pages, rows={rows}", flush=True)
    c = DevCase(bb.FMT_Q8_0, 8, rows, 129 * 512, 4401 + rows, page_keys=512)
    try:
        if rows == 8:
            ws.set_split(decode_groups=256)
        try:
            out = c.run(ws)
        finally:
            ws.set_split()
        sel = np.arange(rows) if rows == 8 else np.arange(1, rows, 8)
        check(f"129 pages rows={rows}", pick(out, 8, rows, sel), c.oracle(sel))
    finally:
        c.close()


@pytest.mark.parametrize("rows", [8, 40])
def test_page_above_4_gib(ws, rows):
    """One page of 2^20 + 100 keys with rows of 4,352 bytes (2 KV heads, q8_0, rows padded): 4.56 GB per tensor, more
    than a 32-bit byte count spans. Every tile's buffer range covers its own 32 rows only, so the page needs no
    split. Decode (8 rows) and the matrix-core kernel (40 rows)."""
    nk, rs = (1 << 20) + 100, 4352
    print(f"page of {nk} keys x {rs} bytes, rows={rows}", flush=True)
    c = DevCase(bb.FMT_Q8_0, 2, rows, nk, 4501 + rows, rs=rs, page_keys=nk)
    try:
        assert len(c.pages.k) == 1 and nk * rs > 1 << 32
        check(f"page above 4 GiB rows={rows}", c.run(ws), c.oracle())
    finally:
        c.close()


@pytest.mark.parametrize("rows,qmode", [(8, bb.QMODE_GGML), (48, bb.QMODE_GGML), (48, bb.QMODE_F16)])
def test_hd256_single_chunk(ws, rows, qmode):
    """Head dim 256 over 40 keys (one chunk): the head-dim-256 kernel writes (O, m, l) itself, no merge."""
    print(f"hd 256 single chunk rows={rows} qmode={qmode}", flush=True)
    c = DevCase(bb.FMT_Q8_0, 2, rows, 40, 4601 + rows + qmode, hd=256)
    try:
        out = c.run(ws, qmode)
        if qmode == bb.QMODE_GGML:
            ref = c.oracle()
        else:
            K, V = c.kbuf.download(np.uint8), c.vbuf.download(np.uint8)
            ref = orc.attn_exact(orc.make_shape(2, rows, 256, orc.Q8_0, orc.QMODE_F16, rs=c.rs), c.Q, K, V, 40)
        check(f"hd256 40 keys rows={rows} qmode={qmode}", out, ref)
    finally:
        c.close()


@pytest.mark.parametrize("fmt,nk", [(bb.FMT_Q8_0, 65536), (bb.FMT_Q4_0, 65536)])
def test_reference_shape_full_size(ws, fmt, nk):
    """The reference's own shape at 65,536 keys: 4 KV heads x 48 rows (8 tokens x GQA 6), head dim 256, queries
    f16(q*scale) with scale 1/16 (pa-tool's), on the head-dim-256 matrix-core kernel, against the fp64 form."""
    print(f"reference shape 4 x 48 rows, hd 256, {nk} keys fmt={fmt}", flush=True)
    c = DevCase(fmt, 4, 48, nk, 4801 + fmt, hd=256)
    try:
        shape = bb.make_shape(4, 48, 256, fmt, bb.QMODE_F16, scale=1.0 / 16, rs=c.rs)
        ws.attn(shape, c.pages, c.dq.ptr, c.do.ptr, c.dml.ptr, c.dml.ptr + 4 * 48 * 4)
        bb.device_sync()
        ml = c.dml.download(np.float32)
        out = c.do.download(np.float32).reshape(4 * 48, 256), ml[:192], ml[192:]
        K, V = c.kbuf.download(np.uint8), c.vbuf.download(np.uint8)
        ref = orc.attn_exact(orc.make_shape(4, 48, 256, fmt, orc.QMODE_F16, scale=1.0 / 16, rs=c.rs), c.Q, K, V, nk)
        check(f"reference shape {nk} fmt={fmt}", out, ref)
    finally:
        c.close()


def test_growth_inside_capture_is_refused():
    """A workspace that would have to grow inside a stream capture returns an error instead of allocating (the capture
    then ends normally, and an eager call afterwards works)."""
    syn = bb.synth()
    ws = bb.Workspace()
    c = DevCase(bb.FMT_Q8_0, 8, 8, 8192, 4701)
    stream = syn.pa_synth_stream_new()
    gx = None
    try:
        assert syn.pa_synth_capture_begin(stream) == 0
        with pytest.raises(bb.PaHipError, match="inside a stream capture"):
            ws.attn(bb.make_shape(8, 8, 128, bb.FMT_Q8_0), c.pages, c.dq.ptr, c.do.ptr, c.dml.ptr, c.dml.ptr + 256, stream)
        gx = syn.pa_synth_capture_end(stream)
        check("decode after a refused capture", c.run(ws), c.oracle())
    finally:
        if gx:
            syn.pa_synth_graph_free(gx)
        syn.pa_synth_stream_sync(stream)
        c.close()
        ws.close()
