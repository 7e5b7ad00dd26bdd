"""pa_hip_attn_noalloc (the engine call that allocates nothing: split-K partials in the library's fixed per-GPU scratch)
against pa_hip_attn on the same inputs, through the C ABI: two calls in a row, the second smaller (a 16-token verify
over 98,304 q8_0 keys, then a one-token decode over 4,096 keys), each equal to pa_hip_attn's output bit for bit (the
same split) and within the 2e-3 parity bar of the oracle; a call over 258 pages (three launches) whose default split
would overflow the scratch, with the split adapted to fit (within the bar of pa_hip_attn's output and of the oracle);
a call whose launches cannot each hold one split, refused with an error before anything is enqueued; and the call
captured in a HIP graph, every replay equal to the eager call."""
import numpy as np
import pytest

import backburner_amd as bb
import oracle as orc

pytestmark = pytest.mark.gpu
TOL = 2e-3


def make(fmt, nkv, rows, nk, seed, page_keys=4096):
    hb = bb.head_bytes(fmt, 128)
    rs = nkv * hb
    syn = bb.synth()
    kbuf, vbuf = bb.DeviceBuffer(nk * rs), bb.DeviceBuffer(nk * rs)
    assert syn.pa_synth_fill_rows(kbuf.ptr, fmt, nkv, 128, rs, 0, nk, seed, 1.0, 0, None, 1.0, None) == 0
    assert syn.pa_synth_fill_rows(vbuf.ptr, fmt, nkv, 128, rs, 0, nk, seed + 1, 1.0, 0, None, 1.0, None) == 0
    Q = orc.normal(seed + 2, 0, nkv * rows * 128).reshape(-1, 128)
    sizes = [min(page_keys, nk - i) for i in range(0, nk, page_keys)]
    pages = bb.Pages([kbuf.ptr + i * rs for i in range(0, nk, page_keys)], [vbuf.ptr + i * rs for i in range(0, nk, page_keys)],
                     sizes, [])
    bb.device_sync()
    return kbuf, vbuf, Q, pages, bb.make_shape(nkv, rows, 128, fmt)


def outputs(n, hd=128):
    return bb.DeviceBuffer(n * hd * 4), bb.DeviceBuffer(n * 8)


def read(do, dml, n):
    ml = dml.download(np.float32)
    return do.download(np.float32).reshape(n, 128), ml[:n], ml[n:]


def both(shape, pages, Q, ws):
    """(pa_hip_attn_noalloc's (O, m, l), pa_hip_attn's (O, m, l)) on the same inputs"""
    n = shape.nkv * shape.rows
    dq = bb.DeviceBuffer.from_array(Q)
    a, b = outputs(n), outputs(n)
    try:
        bb.attn_noalloc(shape, pages, dq.ptr, a[0].ptr, a[1].ptr, a[1].ptr + n * 4)
        ws.attn(shape, pages, dq.ptr, b[0].ptr, b[1].ptr, b[1].ptr + n * 4)
        bb.device_sync()
        return read(*a, n), read(*b, n)
    finally:
        for x in (dq, *a, *b):
            x.close()


def test_noalloc_matches_attn_two_calls():
    ws = bb.Workspace()
    try:
        for fmt, nkv, rows, nk, seed in ((bb.FMT_Q8_0, 8, 128, 98304, 7101), (bb.FMT_Q8_0, 8, 8, 4096, 7201)):
            print(f"noalloc: fmt={fmt} nkv={nkv} rows={rows} nk={nk}", flush=True)
            kbuf, vbuf, Q, pages, shape = make(fmt, nkv, rows, nk, seed)
            try:
                got, want = both(shape, pages, Q, ws)
                for x, y in zip(got, want):
                    assert np.array_equal(x, y)                      # the same split: bit for bit
                sel = np.arange(0, rows, 4 if rows > 8 else 1)
                idx = (np.arange(nkv)[:, None] * rows + sel[None, :]).reshape(-1)
                qs = Q.reshape(nkv, rows, 128)[:, sel, :].reshape(-1, 128)
                ref = orc.attn_ggml(orc.make_shape(nkv, len(sel), 128, fmt), qs, kbuf.download(np.uint8), vbuf.download(np.uint8), nk)
                eo, em, el = orc.rel_err(got[0][idx], got[1][idx], got[2][idx], *ref)
                print(f"  vs oracle: O {eo:.2e} m {em:.2e} l {el:.2e}", flush=True)
                assert eo < TOL and em < TOL and el < TOL
            finally:
                kbuf.close(); vbuf.close()
    finally:
        ws.close()


def test_noalloc_adapts_split_to_scratch():
    """258 pages of 512 keys (three launches of the verify kernel: 128, 128 and 2 pages): the default 64 chunks per
    launch of 128 rows x 8 heads would need 102 MB of partials, more than the 64 MiB scratch; the call takes 42 chunks
    per launch instead."""
    print("noalloc: 258 pages, verify rows", flush=True)
    ws = bb.Workspace()
    kbuf, vbuf, Q, pages, shape = make(bb.FMT_Q8_0, 8, 128, 258 * 512, 7301, page_keys=512)
    try:
        got, want = both(shape, pages, Q, ws)
        eo, em, el = orc.rel_err(*got, *want)
        print(f"  vs pa_hip_attn: O {eo:.2e} m {em:.2e} l {el:.2e}", flush=True)
        assert eo < TOL and em < TOL and el < TOL
        sel = np.arange(3, 128, 16)
        idx = (np.arange(8)[:, None] * 128 + sel[None, :]).reshape(-1)
        qs = Q.reshape(8, 128, 128)[:, sel, :].reshape(-1, 128)
        ref = orc.attn_ggml(orc.make_shape(8, len(sel), 128, bb.FMT_Q8_0), qs, kbuf.download(np.uint8), vbuf.download(np.uint8),
                            258 * 512)
        eo, em, el = orc.rel_err(got[0][idx], got[1][idx], got[2][idx], *ref)
        print(f"  vs oracle: O {eo:.2e} m {em:.2e} l {el:.2e}", flush=True)
        assert eo < TOL and em < TOL and el < TOL
    finally:
        kbuf.close(); vbuf.close(); ws.close()


@pytest.mark.parametrize("fmt,nkv,rows,nk", [(bb.FMT_Q8_0, 8, 8, 8192), (bb.FMT_Q4_0, 8, 128, 3000)])
def test_noalloc_graph_replays(fmt, nkv, rows, nk):
    """The callers the entry point is for include code under HIP graph capture: a captured pa_hip_attn_noalloc call
    (split-K partials in the fixed scratch, no allocation, no memset), replayed four times over a poisoned output with an
    eager call of another problem in between (which reuses the same scratch), equals the eager call bit for bit."""
    print(f"noalloc graph: fmt={fmt} nkv={nkv} rows={rows} nk={nk}", flush=True)
    syn = bb.synth()
    kbuf, vbuf, Q, pages, shape = make(fmt, nkv, rows, nk, 7401 + rows)
    Q2 = orc.normal(7501 + rows, 0, nkv * rows * 128).reshape(-1, 128)
    n = nkv * rows
    stream = syn.pa_synth_stream_new()
    dq, dq2 = bb.DeviceBuffer.from_array(Q), bb.DeviceBuffer.from_array(Q2)
    out, out2 = bb.DeviceBuffer(n * 128 * 4 + n * 8), bb.DeviceBuffer(n * 128 * 4 + n * 8)

    def call(q, o):
        bb.attn_noalloc(shape, pages, q.ptr, o.ptr, o.ptr + n * 128 * 4, o.ptr + n * 128 * 4 + n * 4, stream)

    gx = None
    try:
        call(dq, out)                                                # eager (the first call also looks up the scratch)
        assert syn.pa_synth_stream_sync(stream) == 0
        want = out.download(np.uint8)
        call(dq2, out2)
        assert syn.pa_synth_stream_sync(stream) == 0
        other = out2.download(np.uint8)
        assert not np.array_equal(want, other)
        assert syn.pa_synth_capture_begin(stream) == 0
        call(dq, out)
        gx = syn.pa_synth_capture_end(stream)
        assert gx, "capture failed"
        for rep in range(4):
            out.upload(np.full(n * 128 * 4 + n * 8, 0x7f, np.uint8))  # poison: every replay must write everything
            assert syn.pa_synth_graph_launch(gx, stream) == 0
            assert syn.pa_synth_stream_sync(stream) == 0
            assert np.array_equal(out.download(np.uint8), want), f"replay {rep} differs from the eager call"
            call(dq2, out2)                                          # eager work on the same scratch between replays
            assert syn.pa_synth_stream_sync(stream) == 0
            assert np.array_equal(out2.download(np.uint8), other)
    finally:
        if gx:
            syn.pa_synth_graph_free(gx)
        for x in (dq, dq2, out, out2, kbuf, vbuf):
            x.close()


def test_noalloc_refuses_what_cannot_fit():
    """385 pages (four launches) of 4,096 rows x 8 heads: one split per launch already needs 4 x 17 MB of partials; the
    host refuses the call before enqueueing anything (the pages are real memory: one 32-key buffer shared by all)."""
    nkv, rows = 8, 4096
    rs = nkv * bb.head_bytes(bb.FMT_Q8_0, 128)
    kv = bb.DeviceBuffer(32 * rs)
    n = nkv * rows
    dq, do, dml = bb.DeviceBuffer(n * 128 * 4), bb.DeviceBuffer(n * 128 * 4), bb.DeviceBuffer(n * 8)
    try:
        pages = bb.Pages([kv.ptr] * 385, [kv.ptr] * 385, [32] * 385, [])
        with pytest.raises(bb.PaHipError, match="more slots than the scratch holds"):
            bb.attn_noalloc(bb.make_shape(nkv, rows, 128, bb.FMT_Q8_0), pages, dq.ptr, do.ptr, dml.ptr, dml.ptr + n * 4)
    finally:
        for x in (kv, dq, do, dml):
            x.close()
