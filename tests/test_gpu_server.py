"""The reference's unchanged pa::server over the PATN wire, with the HIP engine (backburner_amd/bin/pa-hip-serve): pages stay in
HBM between calls, only appended rows are uploaded, TRUNCATE to the middle of a page followed by APPEND of different
rows to the same count is seen, and one-group calls with fewer than 8 tokens compute only the real rows.

The client is backburner_amd/patn_wire.py. Every reply is checked against the oracle's fp64 attention (orc_attn_exact,
PA_QMODE_F16: the server's f16(q*scale)) over the rows the layer holds at that moment, as pa-tool's gate does
(pa-tool.cpp:150-176: max|O - ref| / max|ref| per row and |lse - ref|, PASS below 5e-3; held here to 2e-3). The same
scenario runs on the CPU against the reference's own server with its C-ABI CPU engine (pa-tool serve linked with
oracle/sme_cpu.c), which pins the client and the expected values; the GPU run adds the upload counts and the packed
rows the engine reports in STATS."""
from __future__ import annotations

import os
import re
import socket
import subprocess
import time
from pathlib import Path

import numpy as np
import pytest

import oracle as orc
from backburner_amd.patn_wire import HD, NR, Client
from tests.test_ref_patool import free_port

ROOT = Path(__file__).resolve().parents[1]
SERVE_HIP = ROOT / "backburner_amd" / "bin" / "pa-hip-serve"
TOOL_CPU = ROOT / "oracle" / "_ref" / "pa-tool-cpu"
NKV, FMT = 4, orc.Q8_0
HB = orc.head_bytes(FMT, HD)
RS = NKV * HB
SCALE = 1.0 / 16
TOL = 2e-3


class Server:
    def __init__(self, cmd: list, arm: bool = False):
        self.port = free_port()
        # PA_GPU_MIN_KEYS=0: one-group calls go to the GPU engine below the server's default 16,384 keys too
        # (phone-attn.h:584-586), so these small layers exercise it; PA_GPU_ARM=1: the engine arms the call the server
        # names after each reply
        env = dict(os.environ, PA_GPU_MIN_KEYS="0", PA_GPU_ARM="1" if arm else "0")
        self.p = subprocess.Popen([str(c) for c in cmd] + [str(self.port), "2"], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                                  env=env)
        for _ in range(300):
            try:
                socket.create_connection(("127.0.0.1", self.port), timeout=0.2).close()
                return
            except OSError:
                time.sleep(0.1)
        raise RuntimeError("server did not start")

    def stop(self):
        self.p.kill()
        self.p.wait(timeout=30)


def rows(seed: int, n: int) -> np.ndarray:
    return orc.fill_rows(seed, FMT, NKV, HD, n, rs=RS, amp=1.5).reshape(n, RS)


def queries(seed: int, ng: int, ntok: int) -> np.ndarray:
    """f16 bits [ng][nkv][48][256]; rows of tokens >= ntok zero (pa-tool.cpp:126-129)."""
    q = (orc.normal(seed, 0, ng * NKV * NR * HD) * 1.7).astype(np.float32).reshape(ng, NKV, NR, HD)
    tok = np.arange(NR) % 8
    q[:, :, tok >= ntok, :] = 0
    return orc.f32_to_f16(q).reshape(ng, NKV, NR, HD)


def reply_err(O16: np.ndarray, lse: np.ndarray, Q16: np.ndarray, K: np.ndarray, V: np.ndarray, ntok: int, padded_empty: bool):
    """(max|O - ref|/max|ref|, max|lse - ref|) of every group's reply against the fp64 attention over K/V (the layer's
    rows); real rows only, as pa-tool."""
    ng = Q16.shape[0]
    nk = K.shape[0]
    eo = el = 0.0
    for g in range(ng):
        Qf = orc.f16_to_f32(Q16[g]).reshape(NKV * NR, HD)
        O, m, l = orc.attn_exact(orc.make_shape(NKV, NR, HD, FMT, orc.QMODE_F16, scale=SCALE, rs=RS), Qf, K, V, nk)
        ref_o, ref_lse = O / l[:, None], m + np.log(l)
        got_o = orc.f16_to_f32(O16[g]).reshape(NKV * NR, HD).astype(np.float64)
        got_lse = lse.reshape(ng, NKV * NR)[g].astype(np.float64)
        real = (np.arange(NKV * NR) % 8) < ntok
        den = np.maximum(np.abs(ref_o[real]).max(axis=1), 1e-30)
        eo = max(eo, float((np.abs(got_o[real] - ref_o[real]).max(axis=1) / den).max()))
        el = max(el, float(np.abs(got_lse[real] - ref_lse[real]).max()))
        if padded_empty and ntok < 8:        # tokens the call did not have: no keys -> O = 0, lse = -inf
            assert np.all(got_o[~real] == 0) and np.all(np.isneginf(got_lse[~real]))
    return eo, el


def check_reply(label, O16, lse, Q16, K, V, ntok, padded_empty):
    eo, el = reply_err(O16, lse, Q16, K, V, ntok, padded_empty)
    print(f"{label}: {K.shape[0]} keys, max|O - ref|/max|ref| {eo:.3e}, max|lse - ref| {el:.3e}", flush=True)
    assert eo < TOL and el < TOL, (label, eo, el)


def stat(c: Client, key: str) -> int:
    m = re.search(key + r"=(\d+)", c.stats())
    assert m, c.stats()
    return int(m.group(1))


def scenario(cmd: list, ntok: int, gpu: bool, arm: bool = False):
    """CONFIG 2 layers; APPEND 6144 keys per layer; ATTN twice; APPEND 64; ATTN; TRUNCATE to 5000 (inside page 1) and
    APPEND different rows back to 6208; ATTN; TRUNCATE to 3000 (page 1 dropped, inside page 0) and APPEND again;
    ATTN; then a 16-token ATTN_BIG over the same rows. With arm, the first call is followed by a call of layer 1 (the
    call the server arms after it, phone-attn.h:687-697), which runs as the engine's armed graph."""
    srv = Server(cmd, arm)
    c = Client(srv.port)
    try:
        c.hello()
        c.config(2, NKV, RS, HB, 1)
        held = rows(11, 6144)
        for L in range(2):
            src = held if L == 0 else rows(12, 6144)
            vs = rows(21 + L, 6144)
            for p0 in range(0, 6144, 4096):
                c.append(L, p0, src[p0:p0 + 4096], vs[p0:p0 + 4096])
            if L == 0:
                V0 = vs
            else:
                K1, V1 = src, vs
        K0 = held
        Q = queries(31, 1, ntok)

        def attn(label, stale=None):
            rep, O16, lse = c.attn(0, ntok, 0, SCALE, Q)
            assert rep["gpu_pages"] == rep["pages"] or not gpu, rep
            check_reply(f"{label} ntok={ntok}", O16, lse, Q, K0, V0, ntok, gpu)
            if stale is not None:        # the same reply is far from the rows the TRUNCATE replaced
                eo, el = reply_err(O16, lse, Q, stale[0], stale[1], ntok, False)
                assert eo > 50 * TOL, ("the scenario does not tell replaced rows apart", eo, el)
            return rep

        attn("first call")
        if gpu:
            up = stat(c, "rows_uploaded")
            assert up == 6144 and stat(c, "tracked") == 1
            assert stat(c, "call_rows_per_kv_head") == (6 * ntok if ntok < 8 else 48)
        if arm:                          # armed after the first call; the layer's 6144 rows are uploaded by it
            rep, O16, lse = c.attn(1, ntok, 0, SCALE, Q)
            check_reply(f"layer 1 after layer 0 (armed) ntok={ntok}", O16, lse, Q, K1, V1, ntok, gpu)
            assert stat(c, "armed_hits") == 1, c.stats()
            up += 6144
        attn("held rows again")          # armed after the layer-1 call when arm is set
        if arm:
            assert stat(c, "armed_hits") == 2, c.stats()
        if gpu:
            assert stat(c, "rows_uploaded") == up, "a call over held rows uploaded rows"
        extra_k, extra_v = rows(41, 64), rows(42, 64)
        assert c.append(0, 6144, extra_k, extra_v) == 6208
        K0, V0 = np.concatenate([K0, extra_k]), np.concatenate([V0, extra_v])
        attn("64 appended rows")
        if gpu:
            assert stat(c, "rows_uploaded") == up + 64
            up += 64
        for cut, seed in ((5000, 51), (3000, 61)):
            c.truncate(cut)
            nk_new = 6208 - cut
            nk_, nv_ = rows(seed, nk_new), rows(seed + 1, nk_new)
            for p0 in range(0, nk_new, 2048):
                assert c.append(0, cut + p0, nk_[p0:p0 + 2048], nv_[p0:p0 + 2048]) == cut + min(nk_new, p0 + 2048)
            stale = (K0, V0)
            K0 = np.concatenate([K0[:cut], nk_])
            V0 = np.concatenate([V0[:cut], nv_])
            attn(f"TRUNCATE {cut} + APPEND to 6208", stale)
            if gpu:
                assert stat(c, "rows_uploaded") == up + nk_new, "not exactly the rewritten rows were uploaded"
                up += nk_new
        Qb = queries(71, 2, 8)
        rep, O16, lse = c.attn(0, 16, 0, SCALE, Qb, big=True)
        check_reply("ATTN_BIG 16 tokens", O16, lse, Qb, K0, V0, 8, gpu)
        if gpu:
            assert stat(c, "rows_uploaded") == up and stat(c, "call_rows_per_kv_head") == 96
    finally:
        c.close()
        srv.stop()


needs_cpu_server = pytest.mark.skipif(not TOOL_CPU.exists(), reason="oracle/_ref/pa-tool-cpu not built (reference checkout absent at build time)")
needs_hip_server = pytest.mark.skipif(not SERVE_HIP.exists(), reason="backburner_amd/bin/pa-hip-serve not built (reference checkout absent at build time)")


@needs_cpu_server
def test_wire_scenario_on_reference_cpu_server():
    """The scenario against the reference's server with its CPU engine (no GPU): pins the client and the checks."""
    scenario([TOOL_CPU, "serve"], 8, gpu=False)


@pytest.mark.gpu
@needs_hip_server
@pytest.mark.parametrize("ntok", [1, 3, 8])
def test_wire_scenario_on_hip_engine(ntok):
    print(f"pa-hip-serve scenario ntok={ntok}", flush=True)
    scenario([SERVE_HIP], ntok, gpu=True)


@pytest.mark.gpu
@needs_hip_server
@pytest.mark.parametrize("ntok", [1, 8])
def test_wire_scenario_armed(ntok):
    print(f"pa-hip-serve scenario armed ntok={ntok}", flush=True)
    scenario([SERVE_HIP], ntok, gpu=True, arm=True)


def run_probe(server: Path, keys: int, calls: int, arm: bool = False) -> dict:
    import json
    import sys
    r = subprocess.run([sys.executable, str(ROOT / "tests" / "serve_probe.py"), "--server", str(server),
                        "--keys", str(keys), "--calls", str(calls)] + (["--arm"] if arm else []), capture_output=True, text=True, timeout=300,
                       env=dict(os.environ, PA_GPU_MIN_KEYS="0"))
    assert r.returncode == 0, r.stdout + r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1])


@needs_cpu_server
def test_serve_probe_on_reference_cpu_server():
    """The server probe's wire sequence against the reference's server with its CPU engine (no GPU): one JSON line
    with both timed phases; that server has no HIP engine, so no upload counts."""
    out = run_probe(TOOL_CPU, 4096, 2)
    assert out["held"]["calls"] == 2 and out["append64"]["calls"] == 2
    assert out["rows_uploaded_per_held_call"] is None


@pytest.mark.gpu
@needs_hip_server
def test_serve_probe_on_hip_engine():
    """The server probe through pa-hip-serve: calls over held rows upload nothing, a 64-row APPEND uploads 64 rows."""
    print("serve probe, 8192 keys", flush=True)
    out = run_probe(SERVE_HIP, 8192, 4)
    assert out["rows_uploaded"]["after_warmup"] == 8192
    assert out["rows_uploaded_per_held_call"] == 0 and out["rows_uploaded_per_append_call"] == 64
    assert out["held"]["gpu_ms_p50"] > 0
    assert out["armed_calls"] == {"held": 0, "append64": 0}, out["armed_calls"]


@pytest.mark.gpu
@needs_hip_server
def test_serve_probe_armed_calls():
    """PA_GPU_ARM=1: the server arms the next call after each reply (phone-attn.h:687-697), the engine captures it as a
    HIP graph. Every held-row call (same pages and key counts as the call before) runs as that graph; after an APPEND
    the last page's key count differs, so none does. (The probe checks no reply; test_wire_scenario_armed checks an
    armed call's reply against the fp64 form.)"""
    print("serve probe armed, 8192 keys", flush=True)
    out = run_probe(SERVE_HIP, 8192, 4, arm=True)
    assert out["armed_calls"] == {"held": 4, "append64": 0}, out["armed_calls"]
    assert out["rows_uploaded_per_held_call"] == 0 and out["rows_uploaded_per_append_call"] == 64
