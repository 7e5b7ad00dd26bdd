"""GPU: fused greedy acceptance (bit-exact against the oracle and numpy.argmax) and the device quantizers (bit-exact
against the oracle's ggml-semantics quantizers, which tests/test_oracle.py pins against numpy)."""
import numpy as np
import pytest

import backburner_amd as bb
import oracle as orc

pytestmark = pytest.mark.gpu
VOCAB = 151936


@pytest.fixture(scope="module")
def ws():
    w = bb.Workspace()
    yield w
    w.close()


def gpu_accept(ws, logits, draft):
    n_rows, vocab = logits.shape
    dl = bb.DeviceBuffer.from_array(np.ascontiguousarray(logits, np.float32))
    dd = bb.DeviceBuffer.from_array(np.ascontiguousarray(draft, np.int32) if len(draft) else np.zeros(1, np.int32))
    do = bb.DeviceBuffer((2 + n_rows) * 4)
    ws.accept(dl.ptr, n_rows, vocab, dd.ptr, do.ptr)
    bb.device_sync()
    out = do.download(np.int32)
    return int(out[0]), int(out[1]), out[2:]


def planted(rng, k_true, n_rows=17, vocab=VOCAB, ties=True):
    logits = rng.standard_normal((n_rows, vocab)).astype(np.float32)
    draft = rng.integers(0, vocab, n_rows - 1).astype(np.int32)
    for i in range(min(k_true, n_rows - 1)):
        logits[i, draft[i]] = logits[i].max() + 0.5
        if ties:   # an exact tie above the draft token: the lower index must win
            j = int(rng.integers(0, vocab))
            logits[i, j] = logits[i, draft[i]]
            if j < draft[i]:
                draft[i] = j
    if k_true < n_rows - 1 and np.argmax(logits[k_true]) == draft[k_true]:
        logits[k_true, draft[k_true]] = logits[k_true].min() - 1.0
    return logits, draft


@pytest.mark.parametrize("k_true", list(range(17)))
def test_accept_planted_full_vocab(ws, k_true):
    rng = np.random.default_rng(500 + k_true)
    logits, draft = planted(rng, k_true)
    k, b, am = gpu_accept(ws, logits, draft)
    ko, bo, amo = orc.accept(logits, draft)
    assert np.array_equal(am, amo) and np.array_equal(am, np.argmax(logits, axis=1))
    assert (k, b) == (ko, bo) == (k_true, int(np.argmax(logits[k_true])))


def test_accept_edge_values(ws):
    vocab = 4099                                           # not a multiple of 4: the scalar path
    logits = np.full((5, vocab), -1.0, np.float32)
    logits[0, [5, 700, 3]] = 2.0                           # tie -> 3
    logits[1, 400] = 0.0; logits[1, 20] = -0.0             # -0 == +0 -> 20
    logits[2, 50] = np.nan; logits[2, 40] = np.inf         # first NaN -> 50
    logits[3, :] = -np.inf; logits[3, 4098] = -np.inf      # all equal -> 0
    logits[4, 4098] = 1e30                                 # last element
    draft = np.array([3, 20, 50, 1], np.int32)
    k, b, am = gpu_accept(ws, logits, draft)
    ko, bo, amo = orc.accept(logits, draft)
    assert list(am) == list(amo) == [3, 20, 50, 0, 4098] and (k, b) == (ko, bo) == (3, 0)
    for n_rows in (1, 2, 64):                              # n_rows limits
        rng = np.random.default_rng(n_rows)
        lg, dr = planted(rng, n_rows // 2, n_rows=n_rows, vocab=1000, ties=False)
        assert gpu_accept(ws, lg, dr)[:2] == orc.accept(lg, dr)[:2]


def test_accept_repeated_calls_reset_counter(ws):
    rng = np.random.default_rng(9)
    for it in range(5):
        logits, draft = planted(rng, it * 3, vocab=20000)
        assert gpu_accept(ws, logits, draft)[:2] == orc.accept(logits, draft)[:2]


@pytest.mark.parametrize("fmt", [bb.FMT_Q8_0, bb.FMT_Q4_0])
def test_device_quantizer_bitexact(fmt):
    rng = np.random.default_rng(3 + fmt)
    nb = 20000
    x = rng.standard_normal(nb * 32).astype(np.float32) * np.repeat(10.0 ** rng.uniform(-6, 4, nb), 32).astype(np.float32)
    x[:32] = 0.0
    x[32:64] = np.arange(32, dtype=np.float32) - 16.0
    x[64:96] = 0.5
    x[96:128] = -3.0
    x[128:160] = np.tile([2.0, -2.0], 16)                  # equal magnitudes, opposite signs: the first (+) sets q4_0's d
    x[160:192] = np.tile([-2.0, 2.0], 16)                  # ... the first (-)
    x[192:224] = -0.0                                      # an all -0 block: max stays +0, q4_0's d is -0
    x[224:256] = rng.uniform(-1, 1, 32)
    x[224 + 30], x[224 + 31] = -5.0, 5.0                   # the largest magnitude twice, at the block's end
    x[256:288] = rng.uniform(-1, 1, 32)
    x[256 + 17] = 7.0                                      # in the second half (the other 16 lanes' reduction)
    dx = bb.DeviceBuffer.from_array(x)
    hb = 34 if fmt == bb.FMT_Q8_0 else 18
    dy = bb.DeviceBuffer(nb * hb)
    bb.quantize_device(fmt, dx.ptr, dy.ptr, x.size)
    bb.device_sync()
    assert np.array_equal(dy.download(np.uint8), orc.quantize(fmt, x))


@pytest.mark.parametrize("fmt", [bb.FMT_Q8_0, bb.FMT_Q4_0, bb.FMT_F16])
def test_synth_pages_match_oracle_generator(fmt):
    """libpa_synth's device generator writes the oracle's rows (same stream, same quantizer)."""
    nkv, hd, nk = 8, 128, 777
    hb = bb.head_bytes(fmt, hd)
    rs = nkv * hb
    ch = orc.outlier_channels(42, nkv, hd, 4)
    dch = bb.DeviceBuffer.from_array(ch)
    buf = bb.DeviceBuffer(nk * rs)
    assert bb.synth().pa_synth_fill_rows(buf.ptr, fmt, nkv, hd, rs, 100, nk, 42, 1.0, 4, dch.ptr, 8.0, None) == 0
    bb.device_sync()
    got = buf.download(np.uint8)
    ref = orc.fill_rows(42, fmt, nkv, hd, nk, j0=100, n_outliers=4, outlier_mul=8.0)
    mism = int((got != ref).sum())
    print("synth byte mismatches:", mism, "of", ref.size)
    assert mism == 0
