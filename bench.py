"""bench.py - phone-attn old-KV partial attention on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--secondary] [--no-cpu]

Headline workload: decode at long context, 64 layers in sequence, each layer = 1 query token x 64 query heads over 8 KV
heads (GQA 8), head dim 128, 131,072 old q8_0 positions in 32 pages of 4,096 keys, K with 4 x8 outlier channels per
head, 64 distinct seeded caches (18.25 GB in HBM, made on the device by libpa_synth). A step is one pass over the 64
layers: per layer one pa_hip_attn call (split-K attention kernel + merge kernel) on one stream.

Printed: ONE JSON line.
  value       microseconds per layer of the headline call sequence (lower is better): the 64 layers captured once as a
              HIP graph and replayed per step (the eager per-call figure is reported beside it);
  roofline    the decode kernel's algorithmic bytes per launch / its mean duration (start/end events recorded by the
              kernel launch itself, on its stream); traffic = HBM bytes per launch from the committed rocprofv3
              FETCH_SIZE / WRITE_SIZE summary (profiles/decode128k_pmc.json);
  cpu_baseline  the CPU path (oracle/pa_cpu_simd.c: ggml's CPU flash-attention arithmetic for q8_0 / q4_0, vectorized
              with AVX-512 VNNI or AVX2, equal to the oracle bit for bit) timed on this host's cores over a bounded sample
              of the workload, with the GPU's layer-0 output checked against it (parity_vs_cpu);
  prefill     the 512-token prefill chunk (4,096 rows per KV head, 65,536 q8_0 keys, 64 distinct caches) in ggml's
              rounding (exact integer block dots for QK): us/layer, TFLOP/s and the fraction of fp16 MFMA nameplate,
              counters from profiles/prefill_pmc.json, CPU leg over one layer at full size;
  prefill_f16 the same chunk in the reference engines' rounding (queries f16(q*scale), K/V dequantized to fp16 in LDS:
              the Metal engine's arithmetic), no CPU leg (the CPU path is ggml's);
  verify      the 16-token verify block (1,024 rows over 98,304 q8_0 keys, 64 layers): GB/s and the fraction of HBM
              nameplate, traffic from profiles/verify_pmc.json, CPU leg;
  decode_q4_0, verify_q4_0, decode_4096, accept   the 4-bit cache (143,360 positions), the 4,096-key decode layer of
              the ggml-parity workload, and the fused greedy acceptance over fp32 logits [17][151,936] (bit-exact);
  measured_bw_gbs  plain copy / read of 2 GiB, and read_layer: one launch reading exactly one headline layer's bytes,
              timed per launch (the practical floor of one decode launch).
--secondary adds the reply side, KV ingest and the reference's own shape (head dim 256).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E nameplate
FP16_PEAK_TFS = 2516.6         # MI355X dense fp16 MFMA nameplate
PAGE = 4096


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------- workload
def outlier_channels(seed: int, nkv: int, hd: int, n: int) -> np.ndarray:
    """n distinct channels per KV head (seeded) that the synthetic K scales up: the outlier channels of real keys."""
    rng = np.random.default_rng(seed)
    return np.stack([rng.choice(hd, n, replace=False) for _ in range(nkv)]).astype(np.int32)


class Layers:
    """n_layers distinct seeded caches: per layer one K slab and one V slab of n_keys rows, viewed as PAGE-key pages."""

    def __init__(self, bb, fmt, n_layers, n_keys, nkv=8, hd=128, rows=8, seed=0x5eed, outliers=4, qmode=None, scale=None):
        self.bb, self.fmt, self.n_layers, self.n_keys, self.nkv, self.hd, self.rows = bb, fmt, n_layers, n_keys, nkv, hd, rows
        self.hb = bb.head_bytes(fmt, hd)
        self.rs = nkv * self.hb
        syn = bb.synth()
        self.bufs = []
        self.kv = []
        self.pages = []
        self.q = []
        for L in range(n_layers):
            kb, vb = bb.DeviceBuffer(n_keys * self.rs), bb.DeviceBuffer(n_keys * self.rs)
            sk, sv, sq = seed + 1000 * L + 1, seed + 1000 * L + 2, seed + 1000 * L + 3
            ch = bb.DeviceBuffer.from_array(outlier_channels(sk, nkv, hd, outliers)) if outliers else None
            if syn.pa_synth_fill_rows(kb.ptr, fmt, nkv, hd, self.rs, 0, n_keys, sk, 1.0, outliers, ch.ptr if ch else None, 8.0, None) \
                    or syn.pa_synth_fill_rows(vb.ptr, fmt, nkv, hd, self.rs, 0, n_keys, sv, 1.0, 0, None, 1.0, None):
                raise RuntimeError("synthetic fill failed")
            qb = bb.DeviceBuffer(nkv * rows * hd * 4)
            syn.pa_synth_normal(qb.ptr, nkv * rows * hd, sq, 0, 1.0, None)
            np_ = (n_keys + PAGE - 1) // PAGE
            self.pages.append(bb.Pages([kb.ptr + i * PAGE * self.rs for i in range(np_)],
                                       [vb.ptr + i * PAGE * self.rs for i in range(np_)],
                                       [min(PAGE, n_keys - i * PAGE) for i in range(np_)], []))
            self.bufs += [kb, vb, qb] + ([ch] if ch else [])
            self.kv.append((kb, vb))
            self.q.append(qb)
        bb.device_sync()
        r = nkv * rows
        self.out = bb.DeviceBuffer(r * hd * 4 + 2 * r * 4)
        self.O, self.m, self.l = self.out.ptr, self.out.ptr + r * hd * 4, self.out.ptr + r * hd * 4 + r * 4
        self.shape = bb.make_shape(nkv, rows, hd, fmt, bb.QMODE_GGML if qmode is None else qmode, scale)

    def kv_bytes(self):
        return 2 * self.n_keys * self.rs

    def alg_bytes(self):
        """K/V + Q (fp32) + O, m, l (fp32): per layer."""
        r = self.nkv * self.rows
        return self.kv_bytes() + r * self.hd * 4 + r * self.hd * 4 + 2 * r * 4

    def flops(self):
        return 4.0 * self.nkv * self.rows * self.n_keys * self.hd

    def close(self):
        for b in self.bufs:
            b.close()
        self.out.close()


def time_layers(bb, ws, lay: Layers, steps: int, warmup: int):
    """W untimed steps, then K timed steps (each = every layer once); also the attention kernel alone per call."""
    syn = bb.synth()
    stream = syn.pa_synth_stream_new()
    for _ in range(warmup):
        for L in range(lay.n_layers):
            ws.attn(lay.shape, lay.pages[L], lay.q[L].ptr, lay.O, lay.m, lay.l, stream)
    syn.pa_synth_stream_sync(stream)
    ev = [(syn.pa_synth_event_new(), syn.pa_synth_event_new()) for _ in range(steps * lay.n_layers)]
    e0, e1 = syn.pa_synth_event_new(), syn.pa_synth_event_new()
    bb.device_sync()
    syn.pa_synth_event_record(e0, stream)
    i = 0
    t0 = time.perf_counter()
    for _ in range(steps):
        for L in range(lay.n_layers):
            ws.time_next(ev[i][0], ev[i][1])
            ws.attn(lay.shape, lay.pages[L], lay.q[L].ptr, lay.O, lay.m, lay.l, stream)
            i += 1
    syn.pa_synth_event_record(e1, stream)
    syn.pa_synth_stream_sync(stream)
    bb.device_sync()
    wall = time.perf_counter() - t0
    total_ms = syn.pa_synth_event_ms(e0, e1)
    kern = np.array([syn.pa_synth_event_ms(a, b) for a, b in ev])
    for a, b in ev:
        syn.pa_synth_event_free(a); syn.pa_synth_event_free(b)
    syn.pa_synth_event_free(e0); syn.pa_synth_event_free(e1)
    return total_ms, kern, wall


def time_layers_graph(bb, ws, lay: Layers, steps: int, reps: int = 1):
    """The layer sequence, repeated reps times, captured once as a HIP graph (one pa_hip_attn per layer, its kernels in
    stream order), then K timed replays: per-layer time without the host's per-launch overhead (a short sequence is
    repeated so that one graph launch does not dominate). Returns total ms per reps sequences, or None if the capture
    failed."""
    syn = bb.synth()
    stream = syn.pa_synth_stream_new()
    for L in range(lay.n_layers):                                   # sizes the workspace before the capture
        ws.attn(lay.shape, lay.pages[L], lay.q[L].ptr, lay.O, lay.m, lay.l, stream)
    syn.pa_synth_stream_sync(stream)
    if syn.pa_synth_capture_begin(stream) != 0:
        return None
    for _ in range(reps):
        for L in range(lay.n_layers):
            ws.attn(lay.shape, lay.pages[L], lay.q[L].ptr, lay.O, lay.m, lay.l, stream)
    gx = syn.pa_synth_capture_end(stream)
    if not gx:
        return None
    syn.pa_synth_graph_launch(gx, stream)
    syn.pa_synth_stream_sync(stream)
    e0, e1 = syn.pa_synth_event_new(), syn.pa_synth_event_new()
    syn.pa_synth_event_record(e0, stream)
    for _ in range(steps):
        if syn.pa_synth_graph_launch(gx, stream) != 0:
            raise RuntimeError("graph launch failed")
    syn.pa_synth_event_record(e1, stream)
    syn.pa_synth_stream_sync(stream)
    total_ms = syn.pa_synth_event_ms(e0, e1) / reps
    syn.pa_synth_event_free(e0); syn.pa_synth_event_free(e1)
    syn.pa_synth_graph_free(gx)
    return total_ms


def measured_bw(bb, layer_bytes: int, nbytes=2 << 30):
    """The achievable-bandwidth references: a plain device-to-device copy and a read-only stream of nbytes (10 launches
    back to back), and read_layer: one launch reading exactly layer_bytes (one headline layer's K and V), timed per
    launch by its own events, mean of 20 - the practical floor of one decode launch, ramp-up and tail included."""
    syn = bb.synth()
    a, b = bb.DeviceBuffer(nbytes), bb.DeviceBuffer(nbytes)
    sink = bb.DeviceBuffer(1 << 16)
    syn.pa_synth_memset(a.ptr, 1, nbytes)
    e0, e1 = syn.pa_synth_event_new(), syn.pa_synth_event_new()
    res = {}
    for name, fn, traffic in (("copy", lambda: syn.pa_synth_copy(a.ptr, b.ptr, nbytes, 4096, None), 2 * nbytes),
                              ("read", lambda: syn.pa_synth_read(a.ptr, nbytes, 4096, sink.ptr, None), nbytes)):
        fn(); fn()
        bb.device_sync()
        syn.pa_synth_event_record(e0, None)
        for _ in range(10):
            fn()
        syn.pa_synth_event_record(e1, None)
        ms = syn.pa_synth_event_ms(e0, e1) / 10
        res[name] = traffic / (ms * 1e-3) / 1e9
    # one layer per launch: 7 layer-sized windows of the 2 GiB buffer in turn, so no launch finds its bytes in the
    # 256 MB last-level cache from the launch before
    windows = [i * layer_bytes for i in range(nbytes // layer_bytes)]
    per = []
    for i in range(22):
        off = windows[i % len(windows)]
        syn.pa_synth_event_record(e0, None)
        syn.pa_synth_read(a.ptr + off, layer_bytes, 4096, sink.ptr, None)
        syn.pa_synth_event_record(e1, None)
        ms = syn.pa_synth_event_ms(e0, e1)
        if i >= 2:
            per.append(ms)
    us = float(np.mean(per)) * 1e3
    res["read_layer"] = layer_bytes / (us * 1e-6) / 1e9
    res["read_layer_us"] = us
    syn.pa_synth_event_free(e0); syn.pa_synth_event_free(e1)
    for x in (a, b, sink):
        x.close()
    return res


def cpu_info():
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count(), "threads": len(os.sched_getaffinity(0))}


def cpu_baseline(bb, lay: Layers, n_layers: int, row_step: int = 1):
    """Time the CPU path (orc_attn_ggml_simd: ggml's CPU flash-attention arithmetic, vectorized, equal to the oracle bit
    for bit) over the first n_layers layers of the workload at full size (every row_step-th row of each KV head),
    on every host core, and check the GPU's layer-0 output against the CPU's on the same bytes."""
    import oracle as orc
    info = cpu_info()
    threads = info["threads"]
    sel = np.arange(0, lay.rows, row_step)
    s = orc.make_shape(lay.nkv, len(sel), lay.hd, lay.fmt)
    r = lay.nkv * lay.rows
    nbytes = lay.n_keys * lay.rs
    total = 0.0
    parity = None
    path = "?"
    ws = bb.Workspace()
    for L in range(n_layers):
        kb = lay.kv[L][0].download(np.uint8, nbytes)
        vb = lay.kv[L][1].download(np.uint8, nbytes)
        q = lay.q[L].download(np.float32).reshape(lay.nkv, lay.rows, lay.hd)[:, sel, :].reshape(-1, lay.hd)
        t0 = time.perf_counter()
        O, m, l, path = orc.attn_ggml_simd(s, q, kb, vb, lay.n_keys, threads)
        total += time.perf_counter() - t0
        if L == 0:
            ws.attn(lay.shape, lay.pages[0], lay.q[0].ptr, lay.O, lay.m, lay.l)
            bb.device_sync()
            ml = lay.out.download(np.float32, 2 * r, offset=r * lay.hd * 4)
            Og = lay.out.download(np.float32, r * lay.hd).reshape(r, lay.hd)
            idx = (np.arange(lay.nkv)[:, None] * lay.rows + sel[None, :]).reshape(-1)
            eo, em, el = orc.rel_err(Og[idx], ml[:r][idx], ml[r:][idx], O, m, l)
            parity = {"max_rel_O": eo, "max_rel_m": em, "max_rel_l": el, "layer": 0, "keys": lay.n_keys,
                      "rows_checked": int(len(idx)), "tol": 2e-3}
        del kb, vb
    ws.close()
    frac = len(sel) / lay.rows
    per_layer_us = total * 1e6 / n_layers / frac          # a row sample is scaled to the whole layer
    sample = f"layers 0..{n_layers - 1} of {lay.n_layers} at full size ({lay.n_keys} keys"
    sample += f", all {r} rows)" if row_step == 1 else f", every {row_step}th row: {len(sel) * lay.nkv} of {r} rows, time scaled x{row_step})"
    return {"value": round(per_layer_us, 1), "unit": "us/layer", "cores": threads, "kind": "port", "simd": path,
            "cpu_model": info["cpu_model"], "nproc": info["nproc"],
            "sample": sample + f", oracle/pa_cpu_simd.c orc_attn_ggml_simd (ggml CPU flash-attention arithmetic: q8_0 "
                               f"query, integer block dots, expf online softmax, fp32 V accumulation; {path}, OpenMP over "
                               f"rows, {threads} threads), {total:.2f} s of CPU time",
            }, parity


def read_pmc(name: str):
    """The committed rocprofv3 counter summary of a kernel (profiles/<name>_pmc.json), or None."""
    p = ROOT / "profiles" / f"{name}_pmc.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text())
    except Exception:
        return None


def read_traffic(name: str):
    """HBM bytes per launch from the committed rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE, copy-kernel scaled)."""
    d = read_pmc(name)
    return None if d is None else d.get("traffic_bytes_per_launch")


def run_config(bb, ws, fmt, n_layers, n_keys, rows, steps, warmup, label, nkv=8, hd=128, outliers=4, qmode=None, scale=None):
    """Eager steps (per-kernel events), then the same layer sequence replayed as a HIP graph: the per-layer time is the
    graph's (no host launch cost), the eager one is kept beside it."""
    lay = Layers(bb, fmt, n_layers, n_keys, rows=rows, nkv=nkv, hd=hd, outliers=outliers, qmode=qmode, scale=scale)
    total_ms, kern, wall = time_layers(bb, ws, lay, steps, warmup)
    eager_us = total_ms * 1e3 / (steps * n_layers)
    g_ms = time_layers_graph(bb, ws, lay, steps, reps=max(1, 64 // n_layers))
    if g_ms is not None:
        total_ms = g_ms
    per_layer_us = total_ms * 1e3 / (steps * n_layers)
    kmean = float(kern.mean())
    res = {"workload": label, "layers": n_layers, "steps": steps, "us_per_layer": round(per_layer_us, 3),
           "us_per_layer_eager": round(eager_us, 3), "graph": g_ms is not None, "attn_kernel_us": round(kmean * 1e3, 3),
           "attn_kernel_us_p90": round(float(np.percentile(kern, 90)) * 1e3, 3),
           "alg_bytes_per_launch": lay.alg_bytes(), "flop_per_launch": lay.flops(),
           "gbs_kernel": round(lay.alg_bytes() / (kmean * 1e-3) / 1e9, 1),
           "gbs_call": round(lay.alg_bytes() / (per_layer_us * 1e-6) / 1e9, 1),
           "tflops_kernel": round(lay.flops() / (kmean * 1e-3) / 1e12, 2),
           "tflops_call": round(lay.flops() / (per_layer_us * 1e-6) / 1e12, 2)}
    res["hbm_frac_kernel"] = round(res["gbs_kernel"] / HBM_PEAK_GBS, 4)
    res["mfma_frac_kernel"] = round(res["tflops_kernel"] / FP16_PEAK_TFS, 4)
    return lay, res, total_ms, kern


def roofline(res, bound, kernel, pmc_name=None):
    """The roofline object of a workload's dominant kernel: algorithmic bytes (hbm) or flops (mfma) per launch / its
    mean duration, against MI355X nameplate; HBM traffic and counters from the committed PMC summary, if any."""
    if bound == "hbm":
        ach, peak, unit = res["gbs_kernel"], HBM_PEAK_GBS, "GB/s"
    else:
        ach, peak, unit = res["tflops_kernel"], FP16_PEAK_TFS, "TFLOP/s"
    pmc = read_pmc(pmc_name) if pmc_name else None
    out = {"bound": bound, "achieved": ach, "peak": peak, "unit": unit, "frac": round(ach / peak, 4),
           "traffic": pmc.get("traffic_bytes_per_launch") if pmc else None, "kernel": kernel,
           "kernel_us_mean": res["attn_kernel_us"]}
    if pmc and pmc.get("counters"):
        out["counters"] = pmc["counters"]
    return out


def workload(bb, ws, args, key, fmt, n_layers, n_keys, rows, label, bound, kernel, steps, cpu_layers, row_step=1,
             outliers=4, pmc=None, **shape):
    """One workload: timing, roofline, CPU leg (unless --no-cpu or cpu_layers is 0) and the GPU-vs-CPU parity of
    layer 0. shape: nkv, hd, qmode, scale (default 8 KV heads, head dim 128, ggml's query rounding)."""
    lay, res, _, _ = run_config(bb, ws, fmt, n_layers, n_keys, rows, steps, 1, label, outliers=outliers, **shape)
    res["roofline"] = roofline(res, bound, kernel, pmc)
    if not args.no_cpu and cpu_layers > 0:
        res["cpu_baseline"], res["parity_vs_cpu"] = cpu_baseline(bb, lay, min(cpu_layers, n_layers), row_step)
    lay.close()
    log(key, json.dumps(res))
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=64)
    ap.add_argument("--only", default="", help="comma list of the extra workloads to run (prefill, prefill_f16, verify, "
                                                "decode_q4_0, verify_q4_0, decode_4096, reference_shape, accept); default all")
    ap.add_argument("--secondary", action="store_true", help="also run the reply side, KV ingest and the head-dim-256 shape in ggml's rounding")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--cpu-layers", type=int, default=16, help="layers of the headline workload the CPU baseline runs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "one GPU only: sharding the old pages by position range over several GPUs is a design note, not built",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import backburner_amd as bb
    import ctypes as C
    nb = C.create_string_buffer(64)
    n_cu = bb.synth().pa_synth_device_name(nb, 64)
    log(f"device {nb.value.decode()} CUs {n_cu}")
    ws = bb.Workspace()
    alg = 2 * 131072 * 8 * 136 + 64 * 128 * 4 * 2 + 64 * 8
    bw = measured_bw(bb, 2 * 131072 * 8 * 136)
    log(f"copy {bw['copy']:.0f} GB/s, read {bw['read']:.0f} GB/s, one layer per launch {bw['read_layer']:.0f} GB/s "
        f"({bw['read_layer_us']:.2f} us)")

    lay, head, total_ms, kern = run_config(bb, ws, bb.FMT_Q8_0, args.layers, 131072, 8, args.steps, args.warmup,
                                           "decode 1 token x 64 q-heads / 8 kv-heads, hd 128, 131072 q8_0 keys, 64 layers")
    log("headline", json.dumps(head))
    cpu, parity = (None, None) if args.no_cpu else cpu_baseline(bb, lay, max(1, min(args.cpu_layers, args.layers)))
    lay.close()

    only = set(x for x in args.only.split(",") if x)
    want = lambda k: not only or k in only
    extra = {}
    nl = args.layers
    if want("prefill"):
        extra["prefill"] = workload(
            bb, ws, args, "prefill", bb.FMT_Q8_0, nl, 65536, 4096,
            f"prefill chunk: 512 tokens x 64 q-heads / 8 kv-heads (4096 rows per KV head), hd 128, 65536 q8_0 keys, "
            f"{nl} distinct caches", "mfma", "pa_hip::mma_kernel<1, 8, false, true> (q8_0 prefill, exact int8 block dots)",
            max(1, min(args.steps, 3)), 1, pmc="prefill", outliers=0)
    if want("prefill_f16"):
        extra["prefill_f16"] = workload(
            bb, ws, args, "prefill_f16", bb.FMT_Q8_0, nl, 65536, 4096,
            f"prefill chunk as above in the reference engines' rounding: queries f16(q*scale), K/V dequantized to fp16 in "
            f"LDS, fp16 MFMA with fp32 accumulation (the Metal engine's arithmetic), {nl} distinct caches", "mfma",
            "pa_hip::mma_kernel<1, 8, false, false> (q8_0 prefill, fp16 operands)",
            max(1, min(args.steps, 3)), 0, pmc="prefill_f16", outliers=0, qmode=bb.QMODE_F16)
    if want("verify"):
        extra["verify"] = workload(
            bb, ws, args, "verify", bb.FMT_Q8_0, nl, 98304, 128,
            f"draft-block verify: 16 tokens x 64 q-heads / 8 kv-heads (128 rows per KV head), hd 128, 98304 q8_0 keys, "
            f"{nl} layers", "hbm", "pa_hip::mma_kernel<1, 4, false, true> (q8_0 verify, exact int8 block dots)",
            max(2, min(args.steps, 10)), 4, pmc="verify", outliers=0)
    if want("decode_q4_0"):
        extra["decode_q4_0"] = workload(
            bb, ws, args, "decode_q4_0", bb.FMT_Q4_0, nl, 143360, 8,
            f"decode 1 token, 8 kv-heads x 8 rows, hd 128, 143360 q4_0 keys, {nl} layers", "hbm",
            "pa_hip::dec_kernel<2> (q4_0 decode)", args.steps, 16, outliers=0, pmc="decode_q4_0")
    if want("verify_q4_0"):
        extra["verify_q4_0"] = workload(
            bb, ws, args, "verify_q4_0", bb.FMT_Q4_0, nl, 143360, 128,
            f"verify 16 tokens, 8 kv-heads x 128 rows, hd 128, 143360 q4_0 keys, {nl} layers", "mfma",
            "pa_hip::mma_kernel<2, 4, false, true> (q4_0 verify, exact int8 block dots)", max(2, min(args.steps, 10)), 2, outliers=0,
            pmc="verify_q4_0")
    if want("decode_4096"):
        extra["decode_4096"] = workload(
            bb, ws, args, "decode_4096", bb.FMT_Q8_0, 1, 4096, 8,
            "decode 1 token, 8 kv-heads x 8 rows, hd 128, 4096 q8_0 keys, 1 layer (the ggml-parity workload)", "hbm",
            "pa_hip::dec_kernel<1> (q8_0 decode)", args.steps, 1, outliers=0)
    if want("reference_shape"):
        extra["reference_shape"] = workload(
            bb, ws, args, "reference_shape", bb.FMT_Q8_0, nl, 65536, 48,
            f"the reference's own shape: 8 tokens x GQA 6 = 48 rows x 4 KV heads, head dim 256, queries f16(q*scale) "
            f"(scale 1/16), 65536 q8_0 keys, {nl} layers", "hbm", "pa_hip::mma256_kernel<256, 1, true, false, 2> (q8_0, head dim 256)",
            max(2, min(args.steps, 10)), 0, outliers=0, pmc="reference_shape", nkv=4, hd=256, qmode=bb.QMODE_F16,
            scale=1.0 / 16)
    if want("accept"):
        extra["accept"] = bench_accept(bb, ws, args.steps)
        log("accept", json.dumps(extra["accept"]))

    secondary = []
    if args.secondary:
        l2, r2, _, _ = run_config(bb, ws, bb.FMT_Q8_0, 16, 65536, 48, max(2, min(args.steps, 10)), 1,
                                  "48 rows x 4 KV heads, head dim 256, 65536 q8_0 keys, 16 layers, ggml's q8_0 query "
                                  "rounding (the head-dim-256 kernel with exact block dots)", nkv=4, hd=256)
        l2.close()
        log("secondary", json.dumps(r2))
        secondary.append(r2)
        for fn in (bench_reply, bench_ingest):
            r = fn(bb, ws) if fn is bench_reply else fn(bb)
            log("secondary", json.dumps(r))
            secondary.append(r)

    kmean_s = float(kern.mean()) * 1e-3
    achieved = alg / kmean_s / 1e9
    out = {
        "metric": "old-KV attn us/layer + % HBM BW at 128k Q8_0 decode; prefill-chunk TFLOP/s",
        "value": head["us_per_layer"], "unit": "us/layer", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(total_ms / args.steps, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "q8_0 K/V; QK int8 MFMA (exact integer block dots), PV fp16 MFMA, fp32 softmax/accumulate",
        "data": "synthetic (seeded N(0,1), made on device)",
        "config": {"workload": "decode at long context: 1 token, 64 query heads / 8 KV heads (GQA 8), head dim 128, "
                               "131072 old q8_0 positions (32 pages of 4096), K with 4 x8 outlier channels per head",
                   "layers": args.layers, "global_batch": 1, "seq_len": 131072, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic("decode128k"),
                     "kernel": "pa_hip::dec_kernel<1> (q8_0 decode)", "alg_bytes_per_launch": alg,
                     "kernel_us_mean": round(kmean_s * 1e6, 3),
                     "frac_of_read_layer": round(bw["read_layer_us"] / (kmean_s * 1e6), 4)},
        "hbm_frac_call": round(alg / (head["us_per_layer"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "timing": {"value_from": "HIP graph of the 64-layer sequence, replayed per step" if head["graph"] else "eager launches",
                   "us_per_layer_eager": head["us_per_layer_eager"], "attn_kernel_us_p90": head["attn_kernel_us_p90"]},
        "measured_bw_gbs": {k: round(v, 1) if k != "read_layer_us" else round(v, 3) for k, v in bw.items()},
        "cpu_baseline": cpu, "parity_vs_cpu": parity,
    }
    out.update(extra)
    if secondary:
        out["secondary"] = secondary
    print(json.dumps(out), flush=True)


def graph_us(bb, fn, n_calls: int):
    """Mean device time per call of fn(stream), n_calls of them captured as one HIP graph and replayed once (3 eager
    calls first size any workspace); None if the capture failed."""
    syn = bb.synth()
    stream = syn.pa_synth_stream_new()
    for _ in range(3):
        fn(stream)
    syn.pa_synth_stream_sync(stream)
    if syn.pa_synth_capture_begin(stream) != 0:
        return None
    for _ in range(n_calls):
        fn(stream)
    gx = syn.pa_synth_capture_end(stream)
    if not gx:
        return None
    syn.pa_synth_graph_launch(gx, stream)                           # warm replay
    syn.pa_synth_stream_sync(stream)
    e0, e1 = syn.pa_synth_event_new(), syn.pa_synth_event_new()
    syn.pa_synth_event_record(e0, stream)
    syn.pa_synth_graph_launch(gx, stream)
    syn.pa_synth_event_record(e1, stream)
    syn.pa_synth_stream_sync(stream)
    us = syn.pa_synth_event_ms(e0, e1) * 1e3 / n_calls
    syn.pa_synth_event_free(e0); syn.pa_synth_event_free(e1)
    syn.pa_synth_graph_free(gx)
    return us


def bench_reply(bb, ws, n_layers=16):
    """Reply side at the headline shape: pa_hip_attn_reply (the split-K merge writes f16 O / l and lse itself) against
    pa_hip_attn on the same layers, per layer of a graph-replayed sequence; then the co-attention merge of the reply
    with a local partial (pa_hip_coattn_merge, 64 rows x 128) per call. The layer-0 reply is checked bit for bit
    against pa_hip_normalise of pa_hip_attn's output."""
    lay = Layers(bb, bb.FMT_Q8_0, n_layers, 131072, rows=8)
    r, hd = lay.nkv * lay.rows, lay.hd
    oh, lse = bb.DeviceBuffer(r * hd * 2), bb.DeviceBuffer(r * 4)
    oh2, lse2 = bb.DeviceBuffer(r * hd * 2), bb.DeviceBuffer(r * 4)
    rng = np.random.default_rng(91)                                  # a local partial (O, m, l) of the recent keys
    loc = bb.DeviceBuffer.from_array(np.concatenate([rng.standard_normal(r * hd), rng.standard_normal(r),
                                                     1.0 + rng.random(r)]).astype(np.float32))
    out = bb.DeviceBuffer(r * hd * 4 + r * 4)
    try:
        def seq_attn(st):
            for L in range(n_layers):
                ws.attn(lay.shape, lay.pages[L], lay.q[L].ptr, lay.O, lay.m, lay.l, st)

        def seq_reply(st):
            for L in range(n_layers):
                ws.attn_reply(lay.shape, lay.pages[L], lay.q[L].ptr, oh.ptr, lse.ptr, st)

        def coattn(st):
            bb.coattn_merge_device(oh.ptr, lse.ptr, loc.ptr, loc.ptr + r * hd * 4, loc.ptr + r * hd * 4 + r * 4, r, hd,
                                   out.ptr, out.ptr + r * hd * 4, st)
        t_attn = graph_us(bb, seq_attn, 4)
        t_reply = graph_us(bb, seq_reply, 4)
        t_co = graph_us(bb, coattn, 64)
        # layer 0: the fused reply against normalise(attn), bit for bit
        ws.attn_reply(lay.shape, lay.pages[0], lay.q[0].ptr, oh.ptr, lse.ptr)
        ws.attn(lay.shape, lay.pages[0], lay.q[0].ptr, lay.O, lay.m, lay.l)
        bb.normalise_device(lay.O, lay.m, lay.l, r, hd, oh2.ptr, lse2.ptr)
        bb.device_sync()
        exact = bool(np.array_equal(oh.download(np.uint16), oh2.download(np.uint16)) and
                     np.array_equal(lse.download(np.uint32), lse2.download(np.uint32)))
    finally:
        for b in (oh, lse, oh2, lse2, loc, out):
            b.close()
        lay.close()
    per = lambda t: None if t is None else round(t / n_layers, 3)
    return {"workload": "reply side: 128k q8_0 decode with the fp16 reply (O / l, lse) written by the merge, and the "
                        "co-attention merge with a local partial", "layers": n_layers,
            "us_per_layer_reply": per(t_reply), "us_per_layer_attn": per(t_attn),
            "coattn_merge_us_per_call": None if t_co is None else round(t_co, 3), "coattn_rows": r,
            "reply_bit_exact_vs_normalise": exact, "timing": "HIP graph replays"}


def bench_ingest(bb, n_calls=64):
    """On-device KV ingest into q8_0 pages (8 KV heads, hd 128, pages of 4096 keys): pa_hip_append_f32 of a 512-token
    chunk (fp32 K and V quantized in the kernel), of one decode token, and pa_hip_append_rows of 512 received q8_0 rows
    (device to device); mean device time per call over n_calls consecutive positions in one graph."""
    nkv, hd, pk = 8, 128, 4096
    shape = bb.make_shape(nkv, 8, hd, bb.FMT_Q8_0)
    rs = shape.rs
    n_pages = (n_calls * 512 + pk - 1) // pk
    pages = bb.alloc_pages(n_pages, pk * rs)
    syn = bb.synth()
    X, Y = bb.DeviceBuffer(512 * nkv * hd * 4), bb.DeviceBuffer(512 * nkv * hd * 4)
    syn.pa_synth_normal(X.ptr, 512 * nkv * hd, 71, 0, 1.0, None)
    syn.pa_synth_normal(Y.ptr, 512 * nkv * hd, 72, 0, 1.0, None)
    KR, VR = bb.DeviceBuffer(512 * rs), bb.DeviceBuffer(512 * rs)
    bb.device_sync()
    res = {"workload": "KV ingest into q8_0 pages, 8 KV heads x 128, pages of 4096 keys", "timing": "HIP graph replays"}
    try:
        pos = [0]

        def app_chunk(st):
            bb.append_f32(shape, pages, pk, pos[0] % (n_pages * pk - 511), X.ptr, Y.ptr, 512, st)
            pos[0] += 512

        def app_token(st):
            bb.append_f32(shape, pages, pk, pos[0] % (n_pages * pk), X.ptr, Y.ptr, 1, st)
            pos[0] += 1

        def app_rows(st):
            bb.append_rows(shape, pages, pk, pos[0] % (n_pages * pk - 511), KR.ptr, VR.ptr, 512, stream=st)
            pos[0] += 512
        t = graph_us(bb, app_chunk, n_calls)
        mb = (2 * 512 * nkv * hd * 4 + 2 * 512 * nkv * 136) / 1e6    # fp32 in, q8_0 out
        res["append_f32_512_us"] = None if t is None else round(t, 3)
        res["append_f32_512_gbs"] = None if t is None else round(mb * 1e3 / t, 1)
        pos[0] = 0
        t = graph_us(bb, app_token, n_calls)
        res["append_f32_1token_us"] = None if t is None else round(t, 3)
        pos[0] = 0
        t = graph_us(bb, app_rows, n_calls)
        mb = 2 * 2 * 512 * rs / 1e6                                  # read + write
        res["append_rows_512_us"] = None if t is None else round(t, 3)
        res["append_rows_512_gbs"] = None if t is None else round(mb * 1e3 / t, 1)
    finally:
        for b in (X, Y, KR, VR):
            b.close()
        pages.close()
    return res


def bench_accept(bb, ws, steps):
    """Fused greedy acceptance, logits fp32 [17][151936]: mean time per call of calls captured as one HIP graph (replayed
    once; the host's per-call launch cost is left out, as for the decode sequence), over one logits buffer (cache-resident)
    and over 32 distinct copies in turn (cold: 330 MB, more than the last-level cache holds); every output bit-exact."""
    syn = bb.synth()
    rng = np.random.default_rng(17)
    logits = rng.standard_normal((17, 151936)).astype(np.float32)
    draft = rng.integers(0, 151936, 16).astype(np.int32)
    k = int(rng.integers(0, 17))
    for i in range(k):
        logits[i, draft[i]] = logits[i].max() + 1
    dd = bb.DeviceBuffer.from_array(draft)
    stream = syn.pa_synth_stream_new()
    n_calls = max(steps, 10)

    def timed(bufs, outs, calls):
        """us per call over `calls` calls cycling through the logits buffers (one HIP graph, replayed once)"""
        for i in range(len(bufs)):
            ws.accept(bufs[i].ptr, 17, 151936, dd.ptr, outs[i].ptr, stream)
        syn.pa_synth_stream_sync(stream)
        gx = None
        if syn.pa_synth_capture_begin(stream) == 0:
            for c in range(calls):
                ws.accept(bufs[c % len(bufs)].ptr, 17, 151936, dd.ptr, outs[c % len(bufs)].ptr, stream)
            gx = syn.pa_synth_capture_end(stream)
        e0, e1 = syn.pa_synth_event_new(), syn.pa_synth_event_new()
        syn.pa_synth_event_record(e0, stream)
        if gx:
            syn.pa_synth_graph_launch(gx, stream)
        else:                                                        # eager fallback: includes host launch time
            for c in range(calls):
                ws.accept(bufs[c % len(bufs)].ptr, 17, 151936, dd.ptr, outs[c % len(bufs)].ptr, stream)
        syn.pa_synth_event_record(e1, stream)
        syn.pa_synth_stream_sync(stream)
        us = syn.pa_synth_event_ms(e0, e1) * 1e3 / calls
        if gx:
            syn.pa_synth_graph_free(gx)
        syn.pa_synth_event_free(e0); syn.pa_synth_event_free(e1)
        return us, gx is not None

    am = logits.argmax(axis=1)                                       # lowest index on ties
    ko = 0
    while ko < 16 and am[ko] == draft[ko]:
        ko += 1
    bo = am[ko]
    exact = lambda o: bool(o[0] == ko and o[1] == bo)
    # cache-resident: one 10.3 MB logits buffer replayed (after the first call it is served from the 256 MB last-level
    # cache); cold: 32 distinct copies (330 MB, more than that cache holds) taken in turn, so every call reads HBM
    hot_b, hot_o = [bb.DeviceBuffer.from_array(logits)], [bb.DeviceBuffer(19 * 4)]
    us_hot, g1 = timed(hot_b, hot_o, n_calls)
    hot_out = hot_o[0].download(np.int32)
    ok = exact(hot_out)
    n_cold = 32
    cold_b = [bb.DeviceBuffer.from_array(logits) for _ in range(n_cold)]
    cold_o = [bb.DeviceBuffer(19 * 4) for _ in range(n_cold)]
    us_cold, g2 = timed(cold_b, cold_o, 2 * n_cold)
    ok = ok and all(exact(o.download(np.int32)) for o in cold_o)
    for x in hot_b + hot_o + cold_b + cold_o + [dd]:
        x.close()
    return {"workload": "fused greedy acceptance, logits fp32 [17][151936]", "us_per_call": round(us_hot, 3),
            "timing": "HIP graph of %d calls" % n_calls if g1 else "eager calls",
            "cache": "resident: one 10.3 MB logits buffer replayed, read from the last-level cache after the first call",
            "gbs": round(logits.nbytes / (us_hot * 1e-6) / 1e9, 1),
            "cold": {"us_per_call": round(us_cold, 3), "gbs": round(logits.nbytes / (us_cold * 1e-6) / 1e9, 1),
                     "buffers": n_cold, "bytes": n_cold * logits.nbytes,
                     "timing": "HIP graph of %d calls over %d distinct logits buffers in turn (more than the last-level "
                               "cache holds, so each call reads HBM)" % (2 * n_cold, n_cold) if g2 else "eager calls"},
            "bit_exact": ok, "planted_k": k, "k": int(hot_out[0])}


if __name__ == "__main__":
    main()
