"""GPU parity of the device engine path (pa_hip_attn, through the C ABI) against the CPU oracle on the same bytes.

Tolerance: 2e-3 relative on O (per row, after rebasing to the oracle's max), on m
(relative to max(1, |m|)) and on l, against the ggml-faithful restatement (orc_attn_ggml) in PA_QMODE_GGML, and against
the fp64 closed form with the reference engines' rounding (f16(q*scale)) in PA_QMODE_F16."""
import numpy as np
import pytest

import backburner_amd as bb
import oracle as orc

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.fixture(scope="module")
def ws():
    w = bb.Workspace()
    yield w
    w.close()


def case(fmt, nkv, rows, hd, nk, seed, rs_pad=0, k_amp=1.0, outliers=0):
    hb = orc.head_bytes(fmt, hd)
    rs = nkv * hb + rs_pad
    K = orc.fill_rows(seed, fmt, nkv, hd, nk, rs=rs, amp=k_amp, n_outliers=outliers, outlier_mul=8.0)
    V = orc.fill_rows(seed + 1, fmt, nkv, hd, nk, rs=rs)
    Q = orc.normal(seed + 2, 0, nkv * rows * hd).reshape(nkv * rows, hd)
    return K, V, Q, rs


def run_and_check(ws, fmt, nkv, rows, hd, nk, seed, qmode=bb.QMODE_GGML, page_keys=bb.PAGE, rs_pad=0, k_amp=1.0, outliers=0,
                  tol=TOL):
    print(f"case fmt={fmt} nkv={nkv} rows={rows} hd={hd} nk={nk} qmode={qmode} pages={page_keys}", flush=True)
    K, V, Q, rs = case(fmt, nkv, rows, hd, nk, seed, rs_pad, k_amp, outliers)
    shape = bb.make_shape(nkv, rows, hd, fmt, qmode, rs=rs)
    O, m, l = bb.attn_host(shape, K, V, Q, page_keys=page_keys, ws=ws)
    if qmode == bb.QMODE_GGML:
        ref = orc.attn_ggml(orc.make_shape(nkv, rows, hd, fmt, orc.QMODE_GGML, rs=rs), Q, K, V, nk)
    else:
        ref = orc.attn_exact(orc.make_shape(nkv, rows, hd, fmt, orc.QMODE_F16, rs=rs), Q, K, V, nk)
    eo, em, el = orc.rel_err(O, m, l, *ref)
    assert eo < tol and em < tol and el < tol, (eo, em, el)
    return eo, em, el


@pytest.mark.parametrize("fmt", [bb.FMT_Q8_0, bb.FMT_Q4_0, bb.FMT_F16])
@pytest.mark.parametrize("rows", [8, 48, 128, 300])
@pytest.mark.parametrize("hd", [128, 256])
def test_parity_ggml(ws, fmt, rows, hd):
    run_and_check(ws, fmt, 2, rows, hd, 1000, seed=100 + rows + hd + fmt, page_keys=512)


@pytest.mark.parametrize("fmt", [bb.FMT_Q8_0, bb.FMT_Q4_0, bb.FMT_F16])
@pytest.mark.parametrize("rows", [9, 32, 33, 64, 100, 160, 224])
def test_mma_row_blocks(ws, fmt, rows):
    """One row block narrower than the workgroup's waves: 4 waves up to 128 rows (9-64 rows leave one to three waves
    that only stage; 100 rows leave none), 8 waves above (160 and 224 rows leave three and one)."""
    run_and_check(ws, fmt, 2, rows, 128, 1500, seed=300 + rows + fmt, page_keys=512)


@pytest.mark.parametrize("fmt", [bb.FMT_Q8_0, bb.FMT_Q4_0])
@pytest.mark.parametrize("nkv,rows", [(1, 8), (3, 8), (3, 128)])
def test_odd_kv_heads(ws, fmt, nkv, rows):
    """An odd KV-head count has no head pairs for the decode kernel: decode goes to the matrix-core kernel (one live
    wave per row block) and verify keeps its full row blocks; both over ragged pages."""
    run_and_check(ws, fmt, nkv, rows, 128, 2100, seed=500 + 10 * nkv + rows + fmt, page_keys=1000)


@pytest.mark.parametrize("fmt", [bb.FMT_Q8_0, bb.FMT_Q4_0, bb.FMT_F16])
@pytest.mark.parametrize("rows", [8, 48])
def test_parity_reference_rounding(ws, fmt, rows):
    run_and_check(ws, fmt, 4, rows, 256, 700, seed=7 + rows + fmt, qmode=bb.QMODE_F16, page_keys=256)


@pytest.mark.parametrize("fmt", [bb.FMT_Q8_0, bb.FMT_Q4_0, bb.FMT_F16])
@pytest.mark.parametrize("rows", [6, 16, 18, 48, 64, 96, 150])
def test_mma256_row_blocks(ws, fmt, rows):
    """Head dim 256 with fp16 queries (the reference engines' f16(q*scale)) on the matrix-core kernel: 16 rows per wave,
    64-row blocks. 6 to 48 rows leave one to three waves that only stage, 64 rows none; 96 and 150 rows take several
    row blocks, the last one partly past the rows."""
    run_and_check(ws, fmt, 2, rows, 256, 1500, seed=700 + rows + fmt, qmode=bb.QMODE_F16, page_keys=512)


@pytest.mark.parametrize("fmt", [bb.FMT_Q8_0, bb.FMT_F16])
def test_mma256_split_invariance(ws, fmt):
    """The head-dim-256 kernel at the reference's 48 rows x 4 KV heads over chunks of 1, 2, 3, 5 and 40 tiles and one
    chunk holding all 157 tiles (written directly): each split within the bar of the fp64 form, splits agreeing to the
    fp16 rounding of P."""
    nkv, rows, hd, nk = 4, 48, 256, 5000
    K, V, Q, rs = case(fmt, nkv, rows, hd, nk, 811 + fmt)
    shape = bb.make_shape(nkv, rows, hd, fmt, bb.QMODE_F16, rs=rs)
    ref = orc.attn_exact(orc.make_shape(nkv, rows, hd, fmt, orc.QMODE_F16, rs=rs), Q, K, V, nk)
    outs = []
    for want in (200, 100, 60, 35, 4, 1):
        print("mma256 split: workgroups", want * nkv, flush=True)
        ws.set_split(mma_workgroups=want * nkv)
        try:
            outs.append(bb.attn_host(shape, K, V, Q, page_keys=1500, ws=ws))
        finally:
            ws.set_split()
        eo, em, el = orc.rel_err(*outs[-1], *ref)
        assert eo < TOL and em < TOL and el < TOL, (want, eo, em, el)
    for O, m, l in outs[1:]:
        eo, em, el = orc.rel_err(O, m, l, *outs[0])
        assert eo < 1e-3 and em < 1e-6 and el < 1e-3, (eo, em, el)


def test_outlier_channels_and_padding(ws):
    """K with 4 x8 outlier channels per head (the long-context decode configuration) and rows padded past nkv*hb."""
    run_and_check(ws, bb.FMT_Q8_0, 8, 8, 128, 2048, seed=31, rs_pad=16, outliers=4)


@pytest.mark.parametrize("pages", [[3, 0, 64, 1, 130], [1], [4096, 4096, 17], [10] * 140, [1024, 1024, 1024, 5000], [64] * 140,
                                   [96, 96, 96], [512, 1024, 512]])
def test_ragged_pages(ws, pages):
    """Uneven page sizes, empty pages, single keys and more pages than one launch holds (140 > 128); equal power-of-two
    pages (found by shift in the decode kernel) with a shorter or a longer last page, in one launch and over two, and
    equal pages that are not a power of two of tiles or a longer page in the middle (found by the page-table walk)."""
    run_and_check(ws, bb.FMT_Q8_0, 2, 8, 128, sum(pages), seed=5 + len(pages), page_keys=pages)


@pytest.mark.parametrize("rows", [8, 128, 512])
def test_empty(ws, rows):
    shape = bb.make_shape(2, rows, 128, bb.FMT_Q8_0)
    Q = orc.normal(1, 0, 2 * rows * 128).reshape(2 * rows, 128)
    O, m, l = bb.attn_host(shape, np.zeros(0, np.uint8), np.zeros(0, np.uint8), Q, page_keys=[], ws=ws)
    assert np.all(O == 0) and np.all(np.isneginf(m)) and np.all(l == 0)


@pytest.mark.parametrize("fmt", [bb.FMT_Q8_0, bb.FMT_Q4_0])
def test_split_invariance(ws, fmt):
    """Splitting the keys over tile groups (split-K slots folded by the merge kernel, or one group writing the result
    itself) changes the result only by where P is rounded to fp16 (relative to a different running max): l and m agree
    to fp32 reordering, O within the P rounding (~2^-11 per weight); every split is also within the parity bar of the
    oracle."""
    K, V, Q, rs = case(fmt, 2, 8, 128, 5000, 77)            # pages of 1500 keys: 157 tiles
    shape = bb.make_shape(2, 8, 128, fmt, rs=rs)
    ref = orc.attn_ggml(orc.make_shape(2, 8, 128, fmt, orc.QMODE_GGML, rs=rs), Q, K, V, 5000)
    outs = []
    for groups in (1, 3, 17, 40, 64, 157):
        print("split: decode groups", groups, flush=True)
        ws.set_split(decode_groups=groups)
        try:
            outs.append(bb.attn_host(shape, K, V, Q, page_keys=1500, ws=ws))
        finally:
            ws.set_split()
        eo, em, el = orc.rel_err(*outs[-1], *ref)
        assert eo < TOL and em < TOL and el < TOL, (groups, eo, em, el)
    for O, m, l in outs[1:]:
        eo, em, el = orc.rel_err(O, m, l, *outs[0])
        assert eo < 1e-3 and em < 1e-6 and el < 1e-5, (eo, em, el)


@pytest.mark.parametrize("fmt", [bb.FMT_Q8_0, bb.FMT_Q4_0])
@pytest.mark.parametrize("rows", [128, 512])
def test_mma_split_invariance(ws, fmt, rows):
    """The verify / prefill kernel over chunks of 1, 2, 3, 5 and 40 tiles (the two-tile register prefetch with its
    empty-range loads past a chunk's end, uneven last chunks) and one chunk holding every tile (the result written
    directly): each split is within the parity bar of the oracle, and splits agree with each other to the fp16
    rounding of P, which the split moves (P is rounded relative to a different running max), in O and in l (the sum
    of the same fp16 P that the PV product uses, 2^-11 per term at most), and on m to fp32 rounding."""
    nkv, hd, nk = 2, 128, 5000                                # pages of 1500 keys: 157 tiles
    K, V, Q, rs = case(fmt, nkv, rows, hd, nk, 91 + rows)
    shape = bb.make_shape(nkv, rows, hd, fmt, rs=rs)
    ref = orc.attn_ggml(orc.make_shape(nkv, rows, hd, fmt, orc.QMODE_GGML, rs=rs), Q, K, V, nk)
    units = nkv * (2 if rows == 512 else 1)                   # KV heads x row blocks (256 rows per block at 512 rows)
    outs = []
    for want in (200, 100, 60, 35, 4, 1):                     # chunks of 1, 2, 3, 5, 40 and 157 tiles
        print("mma split: workgroups", want * units, flush=True)
        ws.set_split(mma_workgroups=want * units)
        try:
            outs.append(bb.attn_host(shape, K, V, Q, page_keys=1500, ws=ws))
        finally:
            ws.set_split()
        eo, em, el = orc.rel_err(*outs[-1], *ref)
        assert eo < TOL and em < TOL and el < TOL, (want, eo, em, el)
    for O, m, l in outs[1:]:
        eo, em, el = orc.rel_err(O, m, l, *outs[0])
        assert eo < 1e-3 and em < 1e-6 and el < 2.0 ** -11, (eo, em, el)


@pytest.mark.parametrize("fmt,rows,hd,qmode", [(bb.FMT_Q8_0, 8, 128, bb.QMODE_GGML), (bb.FMT_Q4_0, 128, 128, bb.QMODE_GGML),
                                               (bb.FMT_Q8_0, 48, 256, bb.QMODE_F16), (bb.FMT_Q8_0, 48, 256, bb.QMODE_GGML)])
@pytest.mark.parametrize("chunk", [64, 1000, 4096])
def test_chunk_keys(ws, fmt, rows, hd, qmode, chunk):
    """config_req.gpu_chunk (keys per workgroup, pa_hip_ws_set_chunk_keys) on the decode, verify and head-dim-256 kernels
    (fp16 queries, and ggml's rounding with exact block dots): every chunking within the parity bar of the oracle."""
    nkv, nk = 2, 5000
    print(f"chunk keys {chunk}: fmt={fmt} rows={rows} hd={hd} qmode={qmode}", flush=True)
    K, V, Q, rs = case(fmt, nkv, rows, hd, nk, 1200 + chunk + rows)
    shape = bb.make_shape(nkv, rows, hd, fmt, qmode, rs=rs)
    if qmode == bb.QMODE_GGML:
        ref = orc.attn_ggml(orc.make_shape(nkv, rows, hd, fmt, orc.QMODE_GGML, rs=rs), Q, K, V, nk)
    else:
        ref = orc.attn_exact(orc.make_shape(nkv, rows, hd, fmt, orc.QMODE_F16, rs=rs), Q, K, V, nk)
    ws.set_chunk_keys(chunk)
    try:
        out = bb.attn_host(shape, K, V, Q, page_keys=1500, ws=ws)
    finally:
        ws.set_chunk_keys(0)
    eo, em, el = orc.rel_err(*out, *ref)
    assert eo < TOL and em < TOL and el < TOL, (eo, em, el)


def test_bad_arguments(ws):
    with pytest.raises(bb.PaHipError, match="hd must be"):
        bb.attn_host(bb.make_shape(1, 8, 64, bb.FMT_Q8_0), np.zeros(68, np.uint8), np.zeros(68, np.uint8),
                     np.zeros((8, 64), np.float32), page_keys=[1], ws=ws)
    s = bb.make_shape(2, 8, 128, bb.FMT_Q8_0)
    s.rs = 100
    with pytest.raises(bb.PaHipError, match="too small"):
        bb.attn_host(s, np.zeros(100, np.uint8), np.zeros(100, np.uint8), np.zeros((16, 128), np.float32), page_keys=[1], ws=ws)


def test_decode_128k_full_size(ws):
    """The long-context decode layer at full size (131,072 q8_0 keys, 8 KV heads, GQA 8, outlier channels): GPU-made
    pages downloaded and checked against the oracle on the same bytes."""
    nkv, rows, hd, nk = 8, 8, 128, 131072
    hb = bb.head_bytes(bb.FMT_Q8_0, hd)
    rs = nkv * hb
    syn = bb.synth()
    kbuf, vbuf = bb.DeviceBuffer(nk * rs), bb.DeviceBuffer(nk * rs)
    ch = orc.outlier_channels(1001, nkv, hd, 4)
    dch = bb.DeviceBuffer.from_array(ch)
    assert syn.pa_synth_fill_rows(kbuf.ptr, 1, nkv, hd, rs, 0, nk, 1001, 1.0, 4, dch.ptr, 8.0, None) == 0
    assert syn.pa_synth_fill_rows(vbuf.ptr, 1, nkv, hd, rs, 0, nk, 1002, 1.0, 0, None, 1.0, None) == 0
    bb.device_sync()
    Q = orc.normal(1003, 0, nkv * rows * hd).reshape(nkv * rows, hd)
    pages = bb.Pages([kbuf.ptr + i * 4096 * rs for i in range(32)], [vbuf.ptr + i * 4096 * rs for i in range(32)], [4096] * 32, [])
    dq = bb.DeviceBuffer.from_array(Q)
    do, dml = bb.DeviceBuffer(nkv * rows * hd * 4), bb.DeviceBuffer(nkv * rows * 8)
    shape = bb.make_shape(nkv, rows, hd, bb.FMT_Q8_0)
    ws.attn(shape, pages, dq.ptr, do.ptr, dml.ptr, dml.ptr + nkv * rows * 4)
    bb.device_sync()
    O = do.download(np.float32).reshape(-1, hd)
    ml = dml.download(np.float32)
    K = kbuf.download(np.uint8)
    V = vbuf.download(np.uint8)
    ref = orc.attn_ggml(orc.make_shape(nkv, rows, hd, orc.Q8_0), Q, K, V, nk)
    eo, em, el = orc.rel_err(O, ml[:nkv * rows], ml[nkv * rows:], *ref)
    print("decode 128k parity", eo, em, el)
    assert eo < TOL and em < TOL and el < TOL, (eo, em, el)


@pytest.mark.parametrize("rows", [8, 128])
def test_page_above_2p20_keys(ws, rows):
    """One page of 2^20 + 100 keys, walked in place by the decode path (8 rows) and the matrix-core path (128 rows):
    each tile's buffer range covers its own 32 rows, so a page of any length needs no split. Both against the oracle
    on the same bytes."""
    nkv, hd, nk = 2, 128, (1 << 20) + 100
    print(f"page above 2^20 keys rows={rows}", flush=True)
    rs = nkv * bb.head_bytes(bb.FMT_Q8_0, hd)
    syn = bb.synth()
    kbuf, vbuf = bb.DeviceBuffer(nk * rs), bb.DeviceBuffer(nk * rs)
    assert syn.pa_synth_fill_rows(kbuf.ptr, 1, nkv, hd, rs, 0, nk, 2001, 1.0, 0, None, 1.0, None) == 0
    assert syn.pa_synth_fill_rows(vbuf.ptr, 1, nkv, hd, rs, 0, nk, 2002, 1.0, 0, None, 1.0, None) == 0
    bb.device_sync()
    Q = orc.normal(2003 + rows, 0, nkv * rows * hd).reshape(nkv * rows, hd)
    pages = bb.Pages([kbuf.ptr], [vbuf.ptr], [nk], [])
    dq = bb.DeviceBuffer.from_array(Q)
    do, dml = bb.DeviceBuffer(nkv * rows * hd * 4), bb.DeviceBuffer(nkv * rows * 8)
    ws.attn(bb.make_shape(nkv, rows, hd, bb.FMT_Q8_0), pages, dq.ptr, do.ptr, dml.ptr, dml.ptr + nkv * rows * 4)
    bb.device_sync()
    O = do.download(np.float32).reshape(-1, hd)
    ml = dml.download(np.float32)
    ref = orc.attn_ggml(orc.make_shape(nkv, rows, hd, orc.Q8_0), Q, kbuf.download(np.uint8), vbuf.download(np.uint8), nk)
    eo, em, el = orc.rel_err(O, ml[:nkv * rows], ml[nkv * rows:], *ref)
    print("page above 2^20 parity", eo, em, el)
    assert eo < TOL and em < TOL and el < TOL, (eo, em, el)


@pytest.mark.parametrize("fmt,rows,nk,nkv", [(bb.FMT_Q8_0, 128, 98304, 8), (bb.FMT_Q4_0, 8, 143360, 8),
                                             (bb.FMT_Q4_0, 128, 143360, 8), (bb.FMT_Q8_0, 4096, 4096, 8),
                                             (bb.FMT_Q8_0, 4096, 65536, 1)])
def test_full_size_verify_and_q4(ws, fmt, rows, nk, nkv):
    """The other full-size workloads: 16-token verify over 98,304 q8_0 keys, and 1-token decode / 16-token verify over
    143,360 q4_0 keys (8 KV heads, GQA 8, pages of 4096); the prefill chunk's 4096 rows per KV head over one page of 8
    heads, and over the full 65,536 keys for one head. GPU-made pages checked against the oracle on the same bytes."""
    hd = 128
    print(f"full size fmt={fmt} rows={rows} nk={nk}", flush=True)
    rs = nkv * bb.head_bytes(fmt, hd)
    syn = bb.synth()
    kbuf, vbuf = bb.DeviceBuffer(nk * rs), bb.DeviceBuffer(nk * rs)
    assert syn.pa_synth_fill_rows(kbuf.ptr, fmt, nkv, hd, rs, 0, nk, 3001 + fmt, 1.0, 0, None, 1.0, None) == 0
    assert syn.pa_synth_fill_rows(vbuf.ptr, fmt, nkv, hd, rs, 0, nk, 3002 + fmt, 1.0, 0, None, 1.0, None) == 0
    bb.device_sync()
    Q = orc.normal(3003 + rows, 0, nkv * rows * hd).reshape(nkv * rows, hd)
    npg = nk // 4096
    pages = bb.Pages([kbuf.ptr + i * 4096 * rs for i in range(npg)], [vbuf.ptr + i * 4096 * rs for i in range(npg)],
                     [4096] * npg, [])
    dq = bb.DeviceBuffer.from_array(Q)
    do, dml = bb.DeviceBuffer(nkv * rows * hd * 4), bb.DeviceBuffer(nkv * rows * 8)
    ws.attn(bb.make_shape(nkv, rows, hd, fmt), pages, dq.ptr, do.ptr, dml.ptr, dml.ptr + nkv * rows * 4)
    bb.device_sync()
    O = do.download(np.float32).reshape(-1, hd)
    ml = dml.download(np.float32)
    ref = orc.attn_ggml(orc.make_shape(nkv, rows, hd, fmt), Q, kbuf.download(np.uint8), vbuf.download(np.uint8), nk)
    eo, em, el = orc.rel_err(O, ml[:nkv * rows], ml[nkv * rows:], *ref)
    print("full size parity", fmt, rows, nk, eo, em, el)
    assert eo < TOL and em < TOL and el < TOL, (eo, em, el)
