"""GPU: the HIP path (pa_hip_attn, pa_hip_accept, pa_hip_quantize through the C ABI) against the committed golden
fixtures - stored answers, no oracle call at run time. Tolerance 2e-3 relative (O per row after rebasing to the stored
max; m relative to max(1, |m|); l), against the ggml-faithful answers in PA_QMODE_GGML and the fp64 closed form with
f16(q*scale) queries in PA_QMODE_F16; acceptance and quantizers bit-exact."""
from pathlib import Path

import numpy as np
import pytest

import backburner_amd as bb
from oracle import rel_err   # numpy-only comparison helper

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
TOL = 2e-3


def load(name):
    return np.load(GOLD / name, allow_pickle=False)


@pytest.fixture(scope="module")
def ws():
    w = bb.Workspace()
    yield w
    w.close()


NAMES = [str(n) for n in np.load(GOLD / "attn_cases.npz", allow_pickle=False)["names"]]


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("qmode", [bb.QMODE_GGML, bb.QMODE_F16])
def test_attn_golden(ws, name, qmode):
    z = load("attn_cases.npz")
    fmt, nkv, rows, hd, nk, rs = (int(v) for v in z[f"{name}__meta"])
    print(f"golden {name} fmt={fmt} nkv={nkv} rows={rows} hd={hd} nk={nk} qmode={qmode}", flush=True)
    shape = bb.make_shape(nkv, rows, hd, fmt, qmode, rs=rs)
    O, m, l = bb.attn_host(shape, z[f"{name}__K"], z[f"{name}__V"], z[f"{name}__Q"], page_keys=[nk] if nk else [], ws=ws)
    tag = "ggml" if qmode == bb.QMODE_GGML else "exact_f16q"
    eo, em, el = rel_err(O, m, l, z[f"{name}__O_{tag}"], z[f"{name}__m_{tag}"], z[f"{name}__l_{tag}"])
    assert eo < TOL and em < TOL and el < TOL, (eo, em, el)


def test_accept_golden(ws):
    z = load("accept_cases.npz")
    for c in range(3):
        logits, draft, expect = z[f"c{c}_logits"], z[f"c{c}_draft"], z[f"c{c}_expect"]
        n_rows, vocab = logits.shape
        dl, dd, do = bb.DeviceBuffer.from_array(logits), bb.DeviceBuffer.from_array(draft), bb.DeviceBuffer((2 + n_rows) * 4)
        ws.accept(dl.ptr, n_rows, vocab, dd.ptr, do.ptr)
        bb.device_sync()
        assert np.array_equal(do.download(np.int32), expect)
        for b in (dl, dd, do):
            b.close()


@pytest.mark.parametrize("fmt,key", [(bb.FMT_Q8_0, "q8_0"), (bb.FMT_Q4_0, "q4_0")])
def test_quantizer_golden(fmt, key):
    z = load("quant_cases.npz")
    x = np.ascontiguousarray(z["x"].reshape(-1))
    dx = bb.DeviceBuffer.from_array(x)
    dy = bb.DeviceBuffer(z[key].size)
    bb.quantize_device(fmt, dx.ptr, dy.ptr, x.size)
    bb.device_sync()
    assert np.array_equal(dy.download(np.uint8), z[key])
