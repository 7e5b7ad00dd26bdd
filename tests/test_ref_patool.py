"""The reference's own harness judges the oracle: pa-tool.cpp and phone-attn.h, compiled unchanged from the reference
checkout (oracle/Makefile), run as loopback server + test client. The server's C-ABI engine is oracle/sme_cpu.c (the
oracle's restatement of scripts/sme/sme_attn.c), so pa-tool's fp64 check (pa-tool.cpp:150-176, PASS below 5e-3) and
its ATTN_BIG vs one-group check (pa-tool.cpp:214-243) pin that restatement at the reference shape (4 KV heads, 48 rows,
head dim 256, q8_0 rows from pa-tool's own generator). The same binary linked against libpa_hip.so runs in
tests/test_gpu_compat.py."""
from __future__ import annotations

import os
import re
import socket
import subprocess
import time
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
TOOL_CPU = ROOT / "oracle" / "_ref" / "pa-tool-cpu"


def free_port() -> int:
    s = socket.socket()
    s.bind(("127.0.0.1", 0))
    p = s.getsockname()[1]
    s.close()
    return p


def run_patool(tool: Path, args: list, env_extra: dict, timeout: int = 600, server: Path | None = None) -> str:
    """Start `tool serve` (or `server PORT 2`) on a free loopback port, run `tool test 127.0.0.1 port ...args`, stop the
    server."""
    port = free_port()
    env = dict(os.environ, **{k: str(v) for k, v in env_extra.items()})
    cmd = [str(server), str(port), "2"] if server else [str(tool), "serve", str(port), "2"]
    srv = subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, env=env)
    try:
        for _ in range(100):
            try:
                socket.create_connection(("127.0.0.1", port), timeout=0.2).close()
                break
            except OSError:
                time.sleep(0.1)
        r = subprocess.run([str(tool), "test", "127.0.0.1", str(port)] + [str(a) for a in args], capture_output=True,
                           text=True, env=env, timeout=timeout)
        out = r.stdout + r.stderr
        assert r.returncode == 0, out
        return out
    finally:
        srv.kill()
        srv.wait(timeout=30)


def check_line(out: str) -> tuple:
    m = re.search(r"max\|O - ref\|/max\|ref\| = ([0-9.e+-]+)\s+max\|lse - ref\| = ([0-9.e+-]+)\s+-> (PASS|FAIL)", out)
    assert m, out
    return float(m.group(1)), float(m.group(2)), m.group(3)


needs_tool = pytest.mark.skipif(not TOOL_CPU.exists(), reason="oracle/_ref/pa-tool-cpu not built (reference checkout absent at build time)")


@needs_tool
@pytest.mark.parametrize("nkeys,ntok", [(4096, 8), (8192, 1), (4160, 3)])
def test_patool_fp64_check_passes_on_oracle(nkeys, ntok):
    out = run_patool(TOOL_CPU, [nkeys, 1, 2], {"PA_NTOK": ntok})
    eo, el, verdict = check_line(out)
    assert verdict == "PASS" and eo < 2e-3 and el < 1e-4, out


@needs_tool
def test_patool_big_vs_one_group_on_oracle():
    out = run_patool(TOOL_CPU, [4096, 1, 2], {"PA_BIG_TOK": 16})
    assert re.search(r"big vs one-group calls: .* -> PASS", out), out
