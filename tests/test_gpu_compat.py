"""GPU: the reference's C ABI exported by libpa_hip.so (sme_attn_partial / sme_attn_pipe, phone-attn.h:63-71) with host
buffers at the reference shape (48 rows per KV head, head dim 256); the reference's own pa-tool, compiled unchanged
and linked against libpa_hip.so, running its loopback fp64 check on the GPU engine; and the reference's unchanged
pa::server with the product's HIP pa::engine (backburner_amd/bin/pa-hip-serve), driven over the PATN wire by the unchanged
pa-tool client with every page on the GPU."""
import re
from pathlib import Path

import numpy as np
import pytest

import backburner_amd as bb
import oracle as orc
from tests.test_ref_patool import check_line, run_patool

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parents[1]
TOOL_HIP = ROOT / "oracle" / "_ref" / "pa-tool-hip"
TOOL_CPU = ROOT / "oracle" / "_ref" / "pa-tool-cpu"
SERVE_HIP = ROOT / "backburner_amd" / "bin" / "pa-hip-serve"
NR, HD = 48, 256


@pytest.fixture(scope="module", autouse=True)
def shape():
    bb.set_compat_shape(NR, HD)


def ref_case(fmt, nkv, nk, seed):
    hb = orc.head_bytes(fmt, HD)
    rs = nkv * hb
    K = orc.fill_rows(seed, fmt, nkv, HD, nk, rs=rs, amp=1.5)
    V = orc.fill_rows(seed + 1, fmt, nkv, HD, nk, rs=rs)
    Q = (orc.normal(seed + 2, 0, nkv * NR * HD) * 1.7).astype(np.float32).reshape(nkv * NR, HD)
    return K, V, Q, rs, hb


@pytest.mark.parametrize("fmt", [bb.FMT_Q8_0, bb.FMT_Q4_0, bb.FMT_F16])
def test_sme_attn_partial_per_head(fmt):
    assert bb.sme2_available() == 1
    nkv, nk = 4, 4096
    K, V, Q, rs, hb = ref_case(fmt, nkv, nk, 11 + fmt)
    w = bb.sme_ws_new()
    O = np.zeros((nkv * NR, HD), np.float32); m = np.zeros(nkv * NR, np.float32); l = np.zeros(nkv * NR, np.float32)
    for h in range(nkv):
        bb.sme_attn_partial(w, Q[h * NR:], HD, K, V, rs, fmt, nk, 1.0 / 16, 512, O[h * NR:], m[h * NR:], l[h * NR:], k_off=h * hb)
    ref = orc.attn_exact(orc.make_shape(nkv, NR, HD, fmt, orc.QMODE_F16, scale=1.0 / 16, rs=rs), Q, K, V, nk)
    eo, em, el = orc.rel_err(O, m, l, *ref)
    assert eo < 2e-3 and em < 2e-3 and el < 2e-3, (eo, em, el)


def test_sme_attn_partial_concurrent_threads():
    """The reference server's sme_page (phone-attn.h:509-520) calls sme_attn_partial from one thread per KV head at
    once, each thread with its own workspace (sme_ws_new): every call made concurrently returns, bit for bit, what
    the same call returns alone, and that matches the fp64 oracle. ctypes releases the GIL for the foreign call, so
    the eight calls overlap in the library (each workspace has its own stream, device buffers and pinned staging; the
    threads' K/V spans overlap in host memory, as the server's heads of one page do)."""
    import threading
    nkv, nk = 8, 4096
    K, V, Q, rs, hb = ref_case(bb.FMT_Q8_0, nkv, nk, 31)
    ws = [bb.sme_ws_new() for _ in range(nkv)]
    try:
        def call(h, O, m, l):
            bb.sme_attn_partial(ws[h], Q[h * NR:], HD, K, V, rs, 1, nk, 1.0 / 16, 512, O[h * NR:], m[h * NR:], l[h * NR:],
                                k_off=h * hb)

        def outs():
            return np.zeros((nkv * NR, HD), np.float32), np.zeros(nkv * NR, np.float32), np.zeros(nkv * NR, np.float32)

        Oa, ma, la = outs()
        for h in range(nkv):
            call(h, Oa, ma, la)
        for rep in range(4):
            print(f"concurrent round {rep}", flush=True)
            Ob, mb, lb = outs()
            threads = [threading.Thread(target=call, args=(h, Ob, mb, lb)) for h in range(nkv)]
            for t in threads:
                t.start()
            for t in threads:
                t.join()
            assert np.array_equal(Ob, Oa) and np.array_equal(mb, ma) and np.array_equal(lb, la), f"round {rep}"
    finally:
        for w in ws:
            bb.lib().pa_hip_ws_free(w)
    ref = orc.attn_exact(orc.make_shape(nkv, NR, HD, orc.Q8_0, orc.QMODE_F16, scale=1.0 / 16, rs=rs), Q, K, V, nk)
    eo, em, el = orc.rel_err(Oa, ma, la, *ref)
    print(f"sme_attn_partial from {nkv} threads: max rel err O {eo:.3e} m {em:.3e} l {el:.3e}", flush=True)
    assert eo < 2e-3 and em < 2e-3 and el < 2e-3, (eo, em, el)


def test_sme_attn_partial_pinned_pages():
    """K/V in pinned host memory (hipHostMalloc, as the HIP server engine allocates its pages for the reference server,
    whose CPU-engine path then hands them to sme_attn_partial): copied to the device directly, no staging copy. Eight
    threads at once over one page, results bit-identical to the same calls over pageable copies of the bytes."""
    import threading
    nkv, nk = 8, 4096
    K, V, Q, rs, hb = ref_case(bb.FMT_Q8_0, nkv, nk, 51)
    pk, pv = bb.PinnedArray(K), bb.PinnedArray(V)
    ws = [bb.sme_ws_new() for _ in range(nkv)]
    try:
        def run(Kx, Vx, threaded):
            O = np.zeros((nkv * NR, HD), np.float32); m = np.zeros(nkv * NR, np.float32); l = np.zeros(nkv * NR, np.float32)
            call = lambda h: bb.sme_attn_partial(ws[h], Q[h * NR:], HD, Kx, Vx, rs, 1, nk, 1.0 / 16, 512, O[h * NR:], m[h * NR:],
                                                  l[h * NR:], k_off=h * hb)
            if threaded:
                th = [threading.Thread(target=call, args=(h,)) for h in range(nkv)]
                for t in th:
                    t.start()
                for t in th:
                    t.join()
            else:
                for h in range(nkv):
                    call(h)
            return O, m, l
        ref = run(K, V, False)
        for rep in range(3):
            got = run(pk.array, pv.array, True)
            assert all(np.array_equal(a, b) for a, b in zip(got, ref)), f"round {rep}"
    finally:
        for w in ws:
            bb.lib().pa_hip_ws_free(w)
        pk.close(); pv.close()
    ex = orc.attn_exact(orc.make_shape(nkv, NR, HD, orc.Q8_0, orc.QMODE_F16, scale=1.0 / 16, rs=rs), Q, K, V, nk)
    eo, em, el = orc.rel_err(*ref, *ex)
    assert eo < 2e-3 and em < 2e-3 and el < 2e-3, (eo, em, el)


def test_stream_wait_is_bounded():
    """pa_hip_stream_wait, the wait every synchronous call uses: with a 0 ms limit on a stream that still has several
    milliseconds of attention work queued it returns -1 and says so; with a generous limit it returns 0 once the work
    is done, and the results equal a call made alone."""
    nkv, rows, hd, nk = 8, 4096, 128, 16384
    K, V, Q, rs = (lambda hb: (orc.fill_rows(41, orc.Q8_0, nkv, hd, nk, rs=nkv * hb), orc.fill_rows(42, orc.Q8_0, nkv, hd, nk, rs=nkv * hb),
                               orc.normal(43, 0, nkv * rows * hd).reshape(nkv * rows, hd), nkv * hb))(orc.head_bytes(orc.Q8_0, hd))
    shape = bb.make_shape(nkv, rows, hd, bb.FMT_Q8_0, rs=rs)
    ws = bb.Workspace()
    pages = bb.pages_from_rows(K, V, rs)
    dq = bb.DeviceBuffer.from_array(Q)
    outs = [bb.DeviceBuffer(nkv * rows * hd * 4), bb.DeviceBuffer(nkv * rows * 4), bb.DeviceBuffer(nkv * rows * 4)]
    try:
        ws.attn(shape, pages, dq.ptr, *(b.ptr for b in outs))
        bb.device_sync()
        first = [b.download(np.float32) for b in outs]
        for _ in range(20):                       # about 6 ms of queued work on the null stream
            ws.attn(shape, pages, dq.ptr, *(b.ptr for b in outs))
        rc0 = bb.lib().pa_hip_stream_wait(None, 0)
        msg = bb.last_error()
        rc1 = bb.lib().pa_hip_stream_wait(None, 60000)
        print(f"wait(0 ms) -> {rc0} ({msg}); wait(60 s) -> {rc1}", flush=True)
        assert rc0 == -1 and "did not finish" in msg
        assert rc1 == 0
        for a, b in zip(first, outs):
            assert np.array_equal(a, b.download(np.float32))
    finally:
        bb.device_sync()
        ws.close()


def test_sme_attn_pipe_all_heads_and_empty():
    nkv, nk = 4, 4160
    K, V, Q, rs, hb = ref_case(bb.FMT_Q8_0, nkv, nk, 21)
    pp = [bb.sme_pipe_new(1)]
    O = np.zeros((nkv * NR, HD), np.float32); m = np.zeros(nkv * NR, np.float32); l = np.zeros(nkv * NR, np.float32)
    bb.sme_attn_pipe(pp, Q, K, V, rs, hb, 1, nkv, nk, 1.0 / 16, O, m, l)
    ref = orc.attn_exact(orc.make_shape(nkv, NR, HD, orc.Q8_0, orc.QMODE_F16, scale=1.0 / 16, rs=rs), Q, K, V, nk)
    eo, em, el = orc.rel_err(O, m, l, *ref)
    assert eo < 2e-3 and em < 2e-3 and el < 2e-3, (eo, em, el)
    bb.sme_attn_pipe(pp, Q, K, V, rs, hb, 1, nkv, 0, 1.0 / 16, O, m, l)   # sme_attn.c:281: empty -> m = -1e30, l = 0
    assert np.all(O == 0) and np.all(m == np.float32(-1e30)) and np.all(l == 0)


def test_sme_attn_pipe_device_pages():
    """Pages already in HBM (pa_hip_alloc_page memory) are read in place."""
    nkv, nk = 2, 1000
    K, V, Q, rs, hb = ref_case(bb.FMT_Q8_0, nkv, nk, 31)
    dk, dv = bb.DeviceBuffer.from_array(K), bb.DeviceBuffer.from_array(V)
    import ctypes as C
    O = np.zeros((nkv * NR, HD), np.float32); m = np.zeros(nkv * NR, np.float32); l = np.zeros(nkv * NR, np.float32)
    arr = (C.c_void_p * 1)(bb.sme_pipe_new(1))
    bb.lib().sme_attn_pipe(arr, 1, 1, bb._fp(Q), dk.ptr, dv.ptr, rs, hb, 1, nkv, nk, 1.0 / 16, bb._fp(O), bb._fp(m), bb._fp(l))
    ref = orc.attn_exact(orc.make_shape(nkv, NR, HD, orc.Q8_0, orc.QMODE_F16, scale=1.0 / 16, rs=rs), Q, K, V, nk)
    eo, em, el = orc.rel_err(O, m, l, *ref)
    assert eo < 2e-3 and em < 2e-3 and el < 2e-3, (eo, em, el)


needs_tool = pytest.mark.skipif(not TOOL_HIP.exists(), reason="oracle/_ref/pa-tool-hip not built (reference checkout absent at build time)")


@needs_tool
@pytest.mark.parametrize("nkeys,ntok", [(8192, 8), (4096, 1)])
def test_reference_patool_on_gpu_engine(nkeys, ntok):
    """pa-tool serve (its C-ABI engine = libpa_hip.so) + pa-tool test: the reference's fp64 gate (5e-3)."""
    out = run_patool(TOOL_HIP, [nkeys, 3, 2], {"PA_NTOK": ntok})
    eo, el, verdict = check_line(out)
    print(out)
    assert verdict == "PASS" and eo < 2e-3 and el < 2e-3, out


@needs_tool
def test_reference_patool_big_on_gpu_engine():
    out = run_patool(TOOL_HIP, [4096, 2, 2], {"PA_BIG_TOK": 16})
    assert re.search(r"big vs one-group calls: .* -> PASS", out), out


needs_serve = pytest.mark.skipif(not (SERVE_HIP.exists() and TOOL_CPU.exists()),
                                 reason="backburner_amd/bin/pa-hip-serve not built (reference checkout absent at build time)")


@needs_serve
@pytest.mark.parametrize("q4,nkeys,ntok", [(0, 16384, 8), (1, 16384, 8), (0, 20480, 1)])
def test_wire_server_with_hip_engine(q4, nkeys, ntok):
    """pa-hip-serve (unchanged pa::server + the HIP pa::engine) answering the unchanged pa-tool client: gpu_permille 1000
    puts every page on the engine; pa-tool's fp64 gate (5e-3) on the normalised reply, held here to 2e-3."""
    print(f"wire server q4={q4} nkeys={nkeys} ntok={ntok}", flush=True)
    out = run_patool(TOOL_CPU, [nkeys, 3, 2, 1, 1, 1000, 1024], {"PA_Q4": q4, "PA_NTOK": ntok}, server=SERVE_HIP)
    print(out)
    eo, el, verdict = check_line(out)
    assert verdict == "PASS" and eo < 2e-3 and el < 2e-3, out
    m = re.search(r"check call: (\d+) of (\d+) pages on the GPU", out)
    assert m and m.group(1) == m.group(2) and int(m.group(1)) == (nkeys + 4095) // 4096, out


@needs_serve
def test_wire_server_big_calls():
    """ATTN_BIG (16 tokens = 2 groups in one engine call) against one-group calls, through the HIP engine."""
    out = run_patool(TOOL_CPU, [16384, 2, 2, 1, 1, 1000, 1024], {"PA_BIG_TOK": 16}, server=SERVE_HIP)
    assert re.search(r"big vs one-group calls: .* -> PASS", out), out


@needs_serve
@pytest.mark.parametrize("helpers", [0, 1])
def test_wire_server_mixed_engines(helpers):
    """gpu_permille 500: the reference server gives half of each call's pages to the HIP engine and the other half to its
    CPU-engine path, which calls the sme_* C ABI of libpa_hip.so while the engine's stream is busy - with sme_helpers 0
    from four threads at once, one workspace each (sme_page, phone-attn.h:509-520), with 1 through sme_attn_pipe. The
    two engines' partials are merged by the server (merge_partial, phone-attn.h:231-239); pa-tool's fp64 gate (5e-3) on
    the normalised reply, held here to 2e-3."""
    print(f"wire server, mixed engines, sme_helpers={helpers}", flush=True)
    out = run_patool(TOOL_CPU, [32768, 3, 2, 4, helpers, 500, 1024], {"PA_NTOK": 8}, server=SERVE_HIP)
    print(out)
    eo, el, verdict = check_line(out)
    assert verdict == "PASS" and eo < 2e-3 and el < 2e-3, out
    m = re.search(r"check call: (\d+) of (\d+) pages on the GPU", out)
    assert m and 0 < int(m.group(1)) < int(m.group(2)), out
