"""The drop-in boundary on the CPU: libpa_hip.so loads, exports every function include/phone_attn_hip.h declares (the
reference's five sme_* symbols among them), the header compiles as C and C++, and without a GPU the library refuses
work loudly instead of computing anything on the CPU."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "phone_attn_hip.h"
LIB = ROOT / "backburner_amd" / "libpa_hip.so"
REFERENCE_SYMBOLS = ["sme_ws_new", "sme_attn_partial", "sme2_available", "sme_pipe_new", "sme_attn_pipe"]   # phone-attn.h:63-71


def declared_functions(path: Path) -> list:
    src = path.read_text()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"//[^\n]*", "", src)
    src = "\n".join(ln for ln in src.splitlines() if not ln.lstrip().startswith("#"))
    names = []
    for stmt in src.split(";"):
        st = " ".join(stmt.split())
        if "(" not in st:
            continue
        head = st.split("(")[0].split("{")[-1].split("}")[-1].strip()
        if head.startswith("typedef") or not head:
            continue
        m = re.search(r"(\w+)$", head)
        if m:
            names.append(m.group(1))
    return names


def exported(lib: Path) -> set:
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True, check=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if " T " in ln}


def test_header_declares_reference_abi():
    names = declared_functions(HEADER)
    for s in REFERENCE_SYMBOLS:
        assert s in names
    assert "pa_hip_attn" in names and "pa_hip_accept" in names


def test_library_exports_every_declared_function():
    assert LIB.exists(), "build first (__graft_entry__.build())"
    missing = set(declared_functions(HEADER)) - exported(LIB)
    assert not missing, missing


@pytest.mark.parametrize("lang", ["c", "c++"])
def test_header_compiles(lang, tmp_path):
    src = tmp_path / ("t.c" if lang == "c" else "t.cpp")
    src.write_text('#include "phone_attn_hip.h"\nint main(void) { pa_hip_shape s; (void) s; return sme2_available(); }\n')
    cc = "gcc" if lang == "c" else "g++"
    subprocess.run([cc, "-fsyntax-only", "-Wall", "-Werror", f"-I{ROOT / 'include'}", str(src)], check=True)


def test_reference_signatures_match(tmp_path):
    """The reference's extern "C" block (phone-attn.h:63-71), restated, and this header declare the same functions:
    a C++ translation unit that includes both must compile (conflicting declarations would not)."""
    src = tmp_path / "t.cpp"
    src.write_text(
        '#include <cstddef>\n#include <cstdint>\n'
        'extern "C" {\n'
        'void * sme_ws_new(void);\n'
        'void   sme_attn_partial(void * w, const float * Q, int qrs, const uint8_t * K, const uint8_t * V, size_t rs,\n'
        '                        int is_q8, int nk, float scale, int bk, float * O, float * m, float * l);\n'
        'int    sme2_available(void);\n'
        'void * sme_pipe_new(int nh);\n'
        'void   sme_attn_pipe(void ** pp, int nw, int nh, const float * Q, const uint8_t * K, const uint8_t * V, size_t rs, size_t hb,\n'
        '                     int is_q8, int nkv, int nk, float scale, float * O, float * m, float * l);\n'
        '}\n#include "phone_attn_hip.h"\nint main() { return 0; }\n')
    subprocess.run(["g++", "-fsyntax-only", "-Wall", "-Werror", f"-I{ROOT / 'include'}", str(src)], check=True)


def test_no_gpu_fails_loudly():
    """In a process without a gfx950 device the library reports it and hands out no workspace (no CPU fallback)."""
    code = (
        "import ctypes as C, sys\n"
        f"L = C.CDLL({str(LIB)!r})\n"
        "L.pa_hip_ws_new.restype = C.c_void_p\n"
        "L.pa_hip_last_error.restype = C.c_char_p\n"
        "L.sme_ws_new.restype = C.c_void_p\n"
        "n = L.sme2_available()\n"
        "w = L.pa_hip_ws_new(0)\n"
        "s = L.sme_ws_new()\n"
        "print(n, w, s, L.pa_hip_last_error().decode())\n")
    out = subprocess.run(["python3", "-c", code], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    has_gpu = subprocess.run(["test", "-e", "/dev/kfd"]).returncode == 0
    if has_gpu:
        pytest.skip("a GPU is present: the no-GPU path is not observable here")
    n, w, s, *msg = out.stdout.split(maxsplit=3)
    assert n == "0" and w == "None" and s == "None" and msg and ("device" in msg[0])


def test_shutdown_gate_refuses_new_calls():
    """pa_hip_shutdown (the server's exit path): with no sme_* call running it returns 0 at once, and every sme_* call
    after it fails with that reason (run in a child process: the gate is process-wide)."""
    code = (
        "import ctypes as C\n"
        f"L = C.CDLL({str(LIB)!r})\n"
        "L.pa_hip_last_error.restype = C.c_char_p\n"
        "rc = L.pa_hip_shutdown(1000)\n"
        "f = (C.c_float * (48 * 256))()\n"
        "L.sme_attn_partial(None, f, 256, None, None, C.c_size_t(1088), 1, 64, C.c_float(0.0625), 512, f, f, f)\n"
        "print(rc, L.pa_hip_last_error().decode())\n")
    out = subprocess.run(["python3", "-c", code], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    rc, msg = out.stdout.split(maxsplit=1)
    assert rc == "0" and "shut down" in msg, out.stdout
