"""Drives pa-hip-serve (the reference's unchanged pa::server with the HIP engine) over the PATN wire at long context and
prints one JSON line: the client's wall time per ATTN, the engine's GPU time per call, how many K/V rows the engine
uploaded to HBM - once when the first call reads the held pages, then only rows appended since - and how many calls
ran as the engine's pre-armed graph (the server arms the next layer's call after each reply; with one layer that is
the same layer's next call; the engine arms only with --arm, PA_GPU_ARM=1).

    python3 tests/serve_probe.py [--keys 131072] [--calls 20] [--ntok 1] [--server PATH] [--arm]

Layout: the reference's shape (4 KV heads, 48 query rows, head dim 256), q8_0 rows of random quants, one layer. The
probe starts the server on a free loopback port, sends CONFIG, APPENDs the keys in messages of 4,096 rows, makes three
warm-up ATTN calls, then `calls` timed ATTN calls over the held rows, then `calls` decode steps that each APPEND 64 rows
(the server attends multiples of 64 keys) before the ATTN; it ends the session and stops the server with SIGTERM (a
normal exit, so a profiler wrapping this probe writes the server's results too)."""
from __future__ import annotations

import argparse
import json
import os
import signal
import socket
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
from backburner_amd.patn_wire import HD, NR, Client  # noqa: E402

NKV, HB = 4, 34 * (HD // 32)
RS = NKV * HB


def q8_rows(rng: np.random.Generator, n: int) -> np.ndarray:
    """n rows of NKV q8_0 heads: per 32-block an fp16 scale in [2^-7, 2^-5) and 32 random int8 quants."""
    rows = np.empty((n, NKV * HD // 32, 34), np.uint8)
    rows[:, :, :2] = rng.uniform(2.0 ** -7, 2.0 ** -5, (n, NKV * HD // 32)).astype(np.float16).view(np.uint8).reshape(n, -1, 2)
    rows[:, :, 2:] = rng.integers(-127, 128, (n, NKV * HD // 32, 32), dtype=np.int8).view(np.uint8)
    return rows.reshape(n, RS)


def free_port() -> int:
    s = socket.socket()
    s.bind(("127.0.0.1", 0))
    p = s.getsockname()[1]
    s.close()
    return p


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--server", default=str(ROOT / "backburner_amd" / "bin" / "pa-hip-serve"))
    ap.add_argument("--keys", type=int, default=131072)
    ap.add_argument("--calls", type=int, default=20)
    ap.add_argument("--ntok", type=int, default=1)
    ap.add_argument("--arm", action="store_true", help="run the server with PA_GPU_ARM=1 (pre-armed calls)")
    args = ap.parse_args()
    if args.keys % 4096:
        print(json.dumps({"error": "--keys must be a multiple of 4096"}))
        return 2
    port = free_port()
    cmd = [args.server] + (["serve"] if Path(args.server).name.startswith("pa-tool") else []) + [str(port), "2"]
    env = dict(os.environ, PA_GPU_ARM="1" if args.arm else "0")
    srv = subprocess.Popen(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.PIPE, env=env)
    try:
        for _ in range(600):
            try:
                socket.create_connection(("127.0.0.1", port), timeout=0.2).close()
                break
            except OSError:
                if srv.poll() is not None:
                    raise RuntimeError("server exited: " + srv.stderr.read().decode(errors="replace"))
                time.sleep(0.1)
        c = Client(port)
        device = c.hello()
        c.config(1, NKV, RS, HB, 1)
        rng = np.random.default_rng(7)
        t0 = time.perf_counter()
        for p0 in range(0, args.keys, 4096):
            c.append(0, p0, q8_rows(rng, 4096), q8_rows(rng, 4096))
        append_s = time.perf_counter() - t0
        q = (rng.standard_normal((1, NKV, NR, HD)) * 1.7).astype(np.float16)
        q[:, :, (np.arange(NR) % 8) >= args.ntok, :] = 0
        Q = q.view(np.uint16)
        def stat(key):                            # a count of the HIP engine's (None for a server without it)
            st = c.stats()
            return int(st.split(key + "=")[1].split()[0]) if key + "=" in st else None
        rows_stat = lambda: stat("rows_uploaded")
        for _ in range(3):
            c.attn(0, args.ntok, 0, 1.0 / 16, Q)
        up_warm = rows_stat()

        def timed(n, append_rows):
            wall, gpu = [], []
            for i in range(n):
                if append_rows:
                    held = args.keys + 64 * i
                    c.append(0, held, q8_rows(rng, 64), q8_rows(rng, 64))
                t = time.perf_counter()
                rep, _, _ = c.attn(0, args.ntok, 0, 1.0 / 16, Q)
                wall.append((time.perf_counter() - t) * 1e3)
                gpu.append(rep["gpu_ms"])
            return wall, gpu

        hits0 = stat("armed_hits")
        wall_h, gpu_h = timed(args.calls, False)
        up_held, hits_held = rows_stat(), stat("armed_hits")
        wall_a, gpu_a = timed(args.calls, True)
        up_end, hits_end = rows_stat(), stat("armed_hits")
        stats = c.stats()
        c.close()
        med = lambda v: round(float(np.median(v)), 4)
        print(json.dumps({
            "workload": f"pa-hip-serve ATTN, {args.keys} q8_0 keys x 4 KV heads, 48 rows (ntok {args.ntok}), head dim 256",
            "device": device, "append_mb_s": round(2 * args.keys * RS / append_s / 1e6, 1),
            "held": {"calls": args.calls, "wall_ms_p50": med(wall_h), "gpu_ms_p50": med(gpu_h)},
            "append64": {"calls": args.calls, "wall_ms_p50": med(wall_a), "gpu_ms_p50": med(gpu_a)},
            "rows_uploaded": {"after_warmup": up_warm, "after_held_calls": up_held, "after_append_calls": up_end},
            "rows_uploaded_per_held_call": None if up_warm is None else (up_held - up_warm) / args.calls,
            "rows_uploaded_per_append_call": None if up_warm is None else (up_end - up_held) / args.calls,
            "armed_calls": None if hits0 is None else {"held": hits_held - hits0, "append64": hits_end - hits_held},
            "server_stats": stats}), flush=True)
        return 0
    finally:
        if srv.poll() is None:
            srv.send_signal(signal.SIGTERM)
            try:
                srv.wait(timeout=60)
            except subprocess.TimeoutExpired:
                srv.kill()
                srv.wait(timeout=30)


if __name__ == "__main__":
    sys.exit(main())
