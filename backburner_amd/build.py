"""Builds the native libraries of backburner_amd in-tree (hipcc cross-compiles gfx950; no GPU needed).

    python -m backburner_amd.build          # libpa_hip.so, libpa_synth.so, oracle/liboracle.so (+ oracle/_ref)

libpa_hip.so   the product: HIP kernels + the C ABI of include/phone_attn_hip.h
libpa_synth.so bench/test support: synthetic HBM pages, device memory and event plumbing
bin/pa-hip-serve  the reference's phone-attn server (phone-attn.h, compiled unchanged from the reference checkout named
               by PA_REF_DIR, default /root/reference) with the HIP pa::engine of integration/; built only where that
               checkout is present (the built binary travels with the tree)
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = ROOT / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CLANGXX = "/opt/rocm/llvm/bin/clang++"
REF = Path(os.environ.get("PA_REF_DIR", "/root/reference"))

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    # packed fp32 VALU forms stay off (hipcc forms them by itself otherwise); fp16 packed math is unaffected
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # IEEE fp32 division: the device q8_0 quantizer must round exactly like the reference's (d = amax/127, id = 1/d)
    "-fhip-fp32-correctly-rounded-divide-sqrt",
]

# per-source extras:
#  - the decode kernel keeps its MFMA accumulators in ordinary VGPRs (the compiler's AGPR choice would copy them in and
#    out of the matrix-core registers on every tile);
#  - the two attention kernels' online softmax never forms a NaN from finite inputs (masked scores are -inf minus a
#    finite offset; every -inf reference max is tested before it is subtracted), so fmaxf chains need no NaN
#    canonicalisation: -fno-honor-nans drops those instructions (prefill 3 %, decode 1.5 % faster, measured).
SRC_FLAGS = {"pa_decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-fno-honor-nans"],
             "pa_mma.hip": ["-fno-honor-nans"], "pa_mma256.hip": ["-fno-honor-nans"]}

LIBS = {
    "libpa_hip.so": ["pa_merge.hip", "pa_decode.hip", "pa_mma.hip", "pa_mma256.hip", "pa_accept.hip", "pa_reply.hip", "pa_ingest.hip",
                     "pa_noalloc.hip", "pa_pack.hip", "pa_abi.cpp"],
    "libpa_synth.so": ["pa_synth.hip"],
}


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(x for x in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in x)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def build(verbose: bool = False) -> None:
    BUILD.mkdir(exist_ok=True)
    jobs = []
    for lib, srcs in LIBS.items():
        for s in srcs:
            obj = BUILD / (s + ".o")
            lang = ["-x", "hip"] if s.endswith(".hip") else []
            jobs.append([HIPCC, *HIP_FLAGS, *SRC_FLAGS.get(s, []), *lang, "-c", str(CSRC / s), "-o", str(obj)])
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        list(ex.map(lambda c: _run(c, verbose), jobs))
    for lib, srcs in LIBS.items():
        objs = [str(BUILD / (s + ".o")) for s in srcs]
        tmp = PKG / (lib + ".tmp")
        _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", f"-Wl,-soname,{lib}", *objs, "-o", str(tmp)], verbose)
        os.replace(tmp, PKG / lib)
    build_server(verbose)
    # the oracle (test infrastructure) and, where the reference checkout exists, its pa-tool builds
    _run(["make", "-s", "-C", str(ROOT / "oracle")], verbose)


def build_server(verbose: bool = False) -> None:
    """bin/pa-hip-serve: integration/pa_hip_serve.cpp (pa::server of phone-attn.h, unchanged, around the HIP engine)
    linked against libpa_hip.so. phone-attn.h compiles on Linux with clang++ given two macro definitions:
    TARGET_OS_IPHONE=0 (Apple's TargetConditionals value off the iPhone; phone-attn.h:413 uses it as an expression) and an
    empty __builtin_arm_yield() (an Arm spin hint, phone-attn.h:371). Nothing else is substituted."""
    hdr = REF / "phone-attn" / "phone-attn.h"
    if not hdr.exists():
        return
    out = PKG / "bin" / "pa-hip-serve"
    out.parent.mkdir(exist_ok=True)
    integ = PKG / "integration"
    _run([CLANGXX, "-std=c++17", "-O2", "-DTARGET_OS_IPHONE=0", "-D__builtin_arm_yield()=((void)0)", "-Wno-unused-result",
          "-pthread", "-D__HIP_PLATFORM_AMD__", f"-I{hdr.parent}", f"-I{ROOT / 'include'}", f"-I{integ}",
          "-I/opt/rocm/include", "-o", str(out) + ".tmp", str(integ / "pa_hip_serve.cpp"), f"-L{PKG}", "-lpa_hip",
          "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN/..", "-Wl,-rpath,/opt/rocm/lib"], verbose)
    os.replace(str(out) + ".tmp", out)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built:", ", ".join(sorted(p.name for p in PKG.glob("*.so"))))
