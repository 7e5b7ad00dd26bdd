"""GPU: seeded random geometries through pa_hip_attn against the oracle, to catch dispatch and split-K geometry
mistakes that the fixed shapes miss. Each case draws KV heads (1-32: odd counts, where the decode kernel's head pairs
give way to the matrix-core kernel, and up to 16 head pairs), rows per KV head (1-300, across the decode, verify and
prefill row blocks), head dim, format, query rounding, row padding, ragged pages (empty pages, single keys, more than
one launch's worth of pages) and, for some, a forced split-K geometry (ws.set_split). Sizes keep the oracle within
about a second per case.

Tolerance 2e-3 as everywhere, on inputs inside the regimes the fixed tests pin at that bar: x8 outlier channels only
where the scores are exact block dots (q8_0 / q4_0 in ggml rounding: every kernel, every row count and head dim)."""
import numpy as np
import pytest

import backburner_amd as bb
import oracle as orc
from tests.test_gpu_attn import run_and_check

pytestmark = pytest.mark.gpu
N_CASES = 48


def draw(i: int):
    r = np.random.default_rng(1000 + i)
    fmt = int(r.choice([bb.FMT_Q8_0, bb.FMT_Q4_0, bb.FMT_F16]))
    hd = int(r.choice([128, 256]))
    qmode = int(r.choice([bb.QMODE_GGML, bb.QMODE_F16]))
    nkv = int(r.choice([1, 2, 3, 4, 5, 8, 9, 16, 32]))
    rows = int(r.choice([1, 3, 6, 8, 9, 16, 33, 48, 100, 128, 129, 200, 300]))
    if i % 6 == 0:                                                   # the decode kernel's shape (even heads, <= 8 rows)
        fmt, hd, qmode = int(r.choice([bb.FMT_Q8_0, bb.FMT_Q4_0])), 128, bb.QMODE_GGML
        nkv, rows = int(r.choice([2, 4, 8, 16, 32])), int(r.choice([1, 2, 5, 8]))
    kind = r.integers(0, 10)
    if kind == 0:                                                    # more pages than one launch holds
        pages = [int(x) for x in r.integers(0, 40, size=int(r.integers(129, 160)))]
    else:
        pages = [int(x) for x in r.integers(0, 3000, size=int(r.integers(1, 5)))]
        if r.random() < 0.3:
            pages[int(r.integers(0, len(pages)))] = 0
    budget = 1.5e9 / (rows * nkv * hd)                               # oracle work
    while sum(pages) > budget and max(pages) > 1:
        pages = [max(0, p // 2) for p in pages]
    rs_pad = int(r.choice([0, 16, 48]))
    exact = fmt != bb.FMT_F16 and qmode == bb.QMODE_GGML
    # outlier keys always on the prefill-sized and head-dim-256 exact calls, on half of the others
    outliers = 4 if exact and (hd == 256 or rows > 128 or r.random() < 0.5) else 0
    split = None
    if r.random() < 0.3:
        split = (int(r.choice([0, 1, 7, 64, 300])), int(r.choice([0, 1, 13, 200, 700])))
    return dict(fmt=fmt, hd=hd, qmode=qmode, nkv=nkv, rows=rows, pages=pages, rs_pad=rs_pad, outliers=outliers,
                split=split)


@pytest.fixture(scope="module")
def ws():
    w = bb.Workspace()
    yield w
    w.close()


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_geometry(ws, i):
    c = draw(i)
    print(f"fuzz case {i}: {c}", flush=True)
    if c["split"]:
        ws.set_split(decode_groups=c["split"][0], mma_workgroups=c["split"][1])
    try:
        eo, em, el = run_and_check(ws, c["fmt"], c["nkv"], c["rows"], c["hd"], sum(c["pages"]), seed=77 + i,
                                   qmode=c["qmode"], page_keys=c["pages"], rs_pad=c["rs_pad"], outliers=c["outliers"])
    finally:
        ws.set_split()
    print(f"fuzz case {i}: max rel err O {eo:.3e} m {em:.3e} l {el:.3e}", flush=True)


def test_draws_cover_the_kernels():
    """The draws reach every routing branch: the decode kernel (even heads, <= 8 rows, ggml rounding, hd 128), the
    4- and 8-wave matrix-core kernels, the head-dim-256 kernels in both roundings, more than 128 pages (two launches), forced splits."""
    cs = [draw(i) for i in range(N_CASES)]
    dec = [c for c in cs if c["hd"] == 128 and c["rows"] <= 8 and c["nkv"] % 2 == 0 and c["fmt"] != bb.FMT_F16
           and c["qmode"] == bb.QMODE_GGML]
    assert dec
    assert any(c["hd"] == 128 and c["rows"] > 128 for c in cs)
    assert any(c["hd"] == 128 and 8 < c["rows"] <= 128 for c in cs)
    assert any(c["hd"] == 256 and c["qmode"] == bb.QMODE_F16 for c in cs)
    assert any(c["hd"] == 256 and c["qmode"] == bb.QMODE_GGML and c["fmt"] != bb.FMT_F16 for c in cs)
    assert any(len(c["pages"]) > 128 for c in cs)
    assert any(c["nkv"] >= 16 for c in dec) and any(c["nkv"] >= 16 and c not in dec for c in cs)
    assert any(c["split"] for c in cs) and any(c["outliers"] for c in cs)
    assert any(c["outliers"] and c["rows"] > 128 for c in cs) and any(c["outliers"] and c["hd"] == 256 for c in cs)
