"""HIP-graph capture of the device engine path: a captured pa_hip_attn / pa_hip_attn_reply call, replayed several times
with eager work and synchronisations between the replays, must give the eager result bit for bit on every replay
(the kernels are deterministic; the call enqueues no memset, so nothing in the graph depends on a memset node).

The workspace is sized by one eager call before the capture (a capture may not allocate)."""
import numpy as np
import pytest

import backburner_amd as bb
import oracle as orc

pytestmark = pytest.mark.gpu

# decode (split-K + the wide merge), verify (MMA kernel + merge), prefill-like (MMA kernel, few slots), hd 256
CASES = [
    (bb.FMT_Q8_0, 8, 8, 128, 8192, bb.QMODE_GGML),
    (bb.FMT_Q4_0, 8, 128, 128, 3000, bb.QMODE_GGML),
    (bb.FMT_Q8_0, 2, 1024, 128, 2048, bb.QMODE_GGML),
    (bb.FMT_Q8_0, 2, 48, 256, 1500, bb.QMODE_F16),
]


@pytest.mark.parametrize("fmt,nkv,rows,hd,nk,qmode", CASES)
@pytest.mark.parametrize("reply", [False, True])
def test_graph_replays_match_eager(fmt, nkv, rows, hd, nk, qmode, reply):
    print(f"graph fmt={fmt} nkv={nkv} rows={rows} hd={hd} nk={nk} reply={reply}", flush=True)
    syn = bb.synth()
    hb = orc.head_bytes(fmt, hd); rs = nkv * hb
    K = orc.fill_rows(80 + rows, fmt, nkv, hd, nk, rs=rs); V = orc.fill_rows(81 + rows, fmt, nkv, hd, nk, rs=rs)
    Q = orc.normal(82 + rows, 0, nkv * rows * hd).reshape(nkv * rows, hd)
    Q2 = orc.normal(83 + rows, 0, nkv * rows * hd).reshape(nkv * rows, hd)
    shape = bb.make_shape(nkv, rows, hd, fmt, qmode, rs=rs)
    pages = bb.pages_from_rows(K, V, rs, 4096)
    n = nkv * rows
    ws = bb.Workspace()
    stream = syn.pa_synth_stream_new()
    dq = bb.DeviceBuffer.from_array(Q); dq2 = bb.DeviceBuffer.from_array(Q2)
    out_bytes = n * hd * (2 if reply else 4) + n * (4 if reply else 8)
    dout = bb.DeviceBuffer(out_bytes); dout2 = bb.DeviceBuffer(out_bytes)

    def call(q, out, st):
        if reply:
            ws.attn_reply(shape, pages, q.ptr, out.ptr, out.ptr + n * hd * 2, st)
        else:
            ws.attn(shape, pages, q.ptr, out.ptr, out.ptr + n * hd * 4, out.ptr + n * hd * 4 + n * 4, st)

    gx = None
    try:
        call(dq, dout, stream)                                       # eager: sizes the workspace, gives the answer
        assert syn.pa_synth_stream_sync(stream) == 0
        want = dout.download(np.uint8)
        call(dq2, dout2, stream)                                     # another problem's answer, to tell them apart
        assert syn.pa_synth_stream_sync(stream) == 0
        other = dout2.download(np.uint8)
        assert not np.array_equal(want, other)
        assert syn.pa_synth_capture_begin(stream) == 0
        call(dq, dout, stream)
        gx = syn.pa_synth_capture_end(stream)
        assert gx, "capture failed"
        for rep in range(4):
            dout.upload(np.full(out_bytes, 0x7f, np.uint8))          # poison: every replay must write everything
            assert syn.pa_synth_graph_launch(gx, stream) == 0
            assert syn.pa_synth_stream_sync(stream) == 0
            got = dout.download(np.uint8)
            assert np.array_equal(got, want), f"replay {rep} differs from the eager call"
            call(dq2, dout2, stream)                                 # eager work on the same workspace between replays
            assert syn.pa_synth_stream_sync(stream) == 0
            assert np.array_equal(dout2.download(np.uint8), other)
    finally:
        if gx:
            syn.pa_synth_graph_free(gx)
        ws.close()
        pages.close()


def test_graph_replays_accept():
    """pa_hip_accept captured in a graph (its completion counter is reset by the kernel itself, no memset): every replay
    over poisoned output equals the eager call, and the counter stays usable for the eager calls in between."""
    print("graph accept", flush=True)
    syn = bb.synth()
    rng = np.random.default_rng(44)
    logits = rng.standard_normal((17, 151936)).astype(np.float32)
    draft = rng.integers(0, 151936, 16).astype(np.int32)
    for i in range(6):
        logits[i, draft[i]] = logits[i].max() + 1.0
    dl, dd, do = bb.DeviceBuffer.from_array(logits), bb.DeviceBuffer.from_array(draft), bb.DeviceBuffer(19 * 4)
    ws = bb.Workspace()
    stream = syn.pa_synth_stream_new()
    gx = None
    try:
        ws.accept(dl.ptr, 17, 151936, dd.ptr, do.ptr, stream)
        assert syn.pa_synth_stream_sync(stream) == 0
        want = do.download(np.int32)
        k, bonus, am = orc.accept(logits, draft)
        assert want[0] == k == 6 and want[1] == bonus and np.array_equal(want[2:], am)
        assert syn.pa_synth_capture_begin(stream) == 0
        ws.accept(dl.ptr, 17, 151936, dd.ptr, do.ptr, stream)
        gx = syn.pa_synth_capture_end(stream)
        assert gx, "capture failed"
        for rep in range(4):
            do.upload(np.full(19, -7, np.int32))
            assert syn.pa_synth_graph_launch(gx, stream) == 0
            assert syn.pa_synth_stream_sync(stream) == 0
            assert np.array_equal(do.download(np.int32), want), f"replay {rep}"
            ws.accept(dl.ptr, 17, 151936, dd.ptr, do.ptr, stream)
            assert syn.pa_synth_stream_sync(stream) == 0
            assert np.array_equal(do.download(np.int32), want)
    finally:
        if gx:
            syn.pa_synth_graph_free(gx)
        ws.close()
