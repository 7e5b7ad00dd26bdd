"""bench.py's output contract: one JSON line with the metric, the roofline of the decode kernel (traffic from the
committed rocprofv3 counter summary) and the CPU baseline, and a refusal of more than one GPU. The CPU tests need no
device; the GPU test runs a short bench (2 layers, 1 CPU-baseline layer) in a child process."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
ALG_BYTES = 2 * 131072 * 8 * 136 + 64 * 128 * 4 * 2 + 64 * 8    # K + V + Q + O, m, l of one 128k q8_0 decode layer


def run_bench(*args, timeout=600):
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True, timeout=timeout)
    lines = [l for l in r.stdout.splitlines() if l.strip()]
    return r.returncode, lines, r.stderr


def test_more_than_one_gpu_is_refused():
    rc, lines, _ = run_bench("--gpus", "2", timeout=120)
    assert rc == 2 and len(lines) == 1
    out = json.loads(lines[0])
    assert out["n_gpus"] == 2 and "one GPU" in out["error"]


@pytest.mark.parametrize("name,kernel,alg", [("decode128k", "dec_kernel<1>", ALG_BYTES),
                                             ("decode_q4_0", "dec_kernel<2>", 2 * 143360 * 8 * 72 + 64 * 128 * 4 * 2 + 64 * 8)])
def test_committed_traffic_summary(name, kernel, alg):
    """The decode kernels' HBM bytes per launch from the two PMC passes: at least the algorithmic bytes (K/V are read
    once; FETCH_SIZE is scaled by the copy-kernel calibration), and not far above them."""
    d = json.loads((ROOT / "profiles" / f"{name}_pmc.json").read_text())
    assert kernel in d["kernel"] and d["alg_bytes_per_launch"] == alg
    t = d["traffic_bytes_per_launch"]
    assert alg <= t < 1.15 * alg
    assert d["fetch_scale"] == pytest.approx(2.0, rel=0.01) and d["write_scale"] == pytest.approx(1.0, rel=0.01)
    assert kernel in (ROOT / "profiles" / "bench_all_kernels.md").read_text()


@pytest.mark.parametrize("name,kernel,flop,extra", [("prefill", "mma_kernel<1, 8, false, true>", 4 * 4096 * 65536 * 128 * 8, 1.25),
                                                    ("prefill_f16", "mma_kernel<1, 8, false, false>", 4 * 4096 * 65536 * 128 * 8, 1.0),
                                                    ("verify", "mma_kernel<1, 4, false, true>", 4 * 128 * 98304 * 128 * 8, 1.25),
                                                    ("verify_q4_0", "mma_kernel<2, 4, false, true>", 4 * 128 * 143360 * 128 * 8, 1.3125),
                                                    ("reference_shape", "mma256_kernel<256, 1, true, false, 2>", 4 * 48 * 65536 * 256 * 4, 1.0)])
def test_committed_mma_counters(name, kernel, flop, extra):
    """The matrix-core kernels' counter summaries: the MFMA work the counters saw (fp16 MOPS_F16 x 512 plus int8
    MOPS_I8 x 512) is the algorithmic flops times what the form adds (the exact-dot forms one scale-product MFMA per
    32-dim block beside the 8 QK and PV MFMAs' worth of a 32 x 32 tile, 1.25x; q4_0 one more MFMA per tile for the
    nibble offset, 1.3125x; the exact forms take QK, half the flops, on the int8 matrix cores), K/V are fetched about
    once, and the MFMA busy fraction is derived from the raw cycle counters."""
    d = json.loads((ROOT / "profiles" / f"{name}_pmc.json").read_text())
    c = d["counters"]
    assert kernel in d["kernel"] and d["flop_per_launch"] == flop
    assert c["fp16_mfma_flops"] == c["SQ_INSTS_VALU_MFMA_MOPS_F16"] * 512
    assert c.get("int8_mfma_ops", 0) == c["SQ_INSTS_VALU_MFMA_MOPS_I8"] * 512
    work = c["fp16_mfma_flops"] + c.get("int8_mfma_ops", 0)
    assert work == pytest.approx(extra * flop, rel=1e-6)
    if kernel.endswith("false, true>"):                                # int8 QK: exactly half the algorithmic work
        assert c["int8_mfma_ops"] == flop // 2
    assert d["alg_bytes_per_launch"] <= d["traffic_bytes_per_launch"] < 1.6 * d["alg_bytes_per_launch"]
    assert 0 < c["mfma_busy_frac"] < 1 and 0 < c["MfmaUtil_pct"] < 100
    assert all("rocprofv3 --pmc" in x and "bench.py" in x for x in d["commands"])


@pytest.mark.gpu
def test_bench_json_contract():
    print("bench --steps 2 --warmup 1 --layers 2 --cpu-layers 1 --only prefill,verify", flush=True)
    rc, lines, err = run_bench("--steps", "2", "--warmup", "1", "--layers", "2", "--cpu-layers", "1", "--only", "prefill,verify")
    assert rc == 0, err[-2000:]
    assert len(lines) == 1, lines
    out = json.loads(lines[0])
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
              "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert k in out, k
    assert out["n_gpus"] == 1 and out["steps"] == 2 and out["warmup"] == 1 and out["unit"] == "us/layer"
    assert out["higher_is_better"] is False and out["vs_baseline"] is None and out["value"] > 0
    assert out["ms_per_step"] == pytest.approx(out["value"] * 2 / 1e3, rel=1e-3)   # 2 layers per step
    assert "workload" in out["config"] and out["config"]["seq_len"] == 131072
    rf = out["roofline"]
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert rf["alg_bytes_per_launch"] == ALG_BYTES
    assert rf["achieved"] == pytest.approx(ALG_BYTES / (rf["kernel_us_mean"] * 1e-6) / 1e9, rel=1e-3)
    assert rf["frac"] == pytest.approx(rf["achieved"] / rf["peak"], rel=1e-3) and 0 < rf["frac"] < 1
    assert rf["traffic"] >= ALG_BYTES
    cb = out["cpu_baseline"]
    assert cb["kind"] == "port" and cb["unit"] == "us/layer" and cb["cores"] >= 1 and cb["value"] > out["value"]
    assert "orc_attn_ggml" in cb["sample"]
    par = out["parity_vs_cpu"]
    assert par["max_rel_O"] < 2e-3 and par["max_rel_m"] < 2e-3 and par["max_rel_l"] < 2e-3
    assert cb["simd"] in ("avx512-vnni", "avx2", "scalar") and cb["cpu_model"] and cb["nproc"] >= 1
    assert out["measured_bw_gbs"]["read_layer"] > 0 and 0 < rf["frac_of_read_layer"] < 1.5
    assert out["parity_vs_cpu"]["max_rel_O"] < 2e-3
    # the prefill chunk (the metric's second half) and the verify block, each with its roofline and CPU leg
    pf, vf = out["prefill"], out["verify"]
    assert pf["roofline"]["bound"] == "mfma" and pf["roofline"]["unit"] == "TFLOP/s" and pf["roofline"]["peak"] == 2516.6
    assert pf["roofline"]["achieved"] == pytest.approx(pf["flop_per_launch"] / (pf["attn_kernel_us"] * 1e-6) / 1e12, rel=1e-2)
    assert 0 < pf["roofline"]["frac"] < 1 and pf["cpu_baseline"]["unit"] == "us/layer"
    assert "1 layer" in pf["cpu_baseline"]["sample"] or "layers 0..0" in pf["cpu_baseline"]["sample"]
    assert vf["roofline"]["bound"] == "hbm" and 0 < vf["roofline"]["frac"] < 1
    assert vf["roofline"]["achieved"] == pytest.approx(vf["alg_bytes_per_launch"] / (vf["attn_kernel_us"] * 1e-6) / 1e9, rel=1e-2)
    for w in (pf, vf):
        assert w["parity_vs_cpu"]["max_rel_O"] < 2e-3 and w["parity_vs_cpu"]["max_rel_l"] < 2e-3
