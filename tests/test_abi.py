"""The C-ABI boundary on the CPU: the library loads, exports every function include/*.h declares, the Python binding
declares every one of them, and include/sn.h is signature-compatible with the reference's own sn.h (both headers in one
C translation unit: a differing prototype is a compile error) and covers every name the reference's Rust `extern "C"`
block binds (engine/sllm-server/src/next_engine/ffi.rs:16-63). No compute call is made (no GPU here)."""
import ctypes as C
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")
REF = "/root/reference/engine"
REF_SN_H = os.path.join(REF, "sllm-next/proto/sn.h")
REF_FFI = os.path.join(REF, "sllm-server/src/next_engine/ffi.rs")
HEADERS = ["sn.h", "sn_kernels.h", "sn_synth.h", "sn_ext.h"]


def declared(header):
    """Function names declared in a header (text between `extern "C" {` and its close; comments stripped)."""
    src = open(os.path.join(INC, header)).read()
    src = re.sub(r"//[^\n]*", "", src)
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"\b([A-Za-z_]\w*)\s*\(", src)
    return sorted({n for n in names if re.match(r"^(sn|snk|snx)_", n)})


def lib_path():
    import sllm_next
    return sllm_next.LIB_PATH


@pytest.fixture(scope="module")
def lib():
    p = lib_path()
    if not os.path.exists(p):
        pytest.fail(f"{p} is not built (run __graft_entry__.build())")
    return C.CDLL(p)


@pytest.mark.parametrize("header", HEADERS)
def test_exports(lib, header):
    names = declared(header)
    assert names, header
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"{header}: not exported: {missing}"


def test_sn_h_has_49_functions():
    assert len(declared("sn.h")) == 49


def test_binding_declares_every_export():
    import sllm_next as S
    bound = {n for n, _, _ in S.SN_API + S.SNK_API + S.EXT_API + S.SYNTH_API}
    for h in HEADERS:
        missing = set(declared(h)) - bound
        assert not missing, f"{h}: no ctypes declaration for {sorted(missing)}"


def test_exports_are_c_symbols():
    """Every header function is an unmangled dynamic symbol (extern "C")."""
    out = subprocess.run(["nm", "-D", "--defined-only", lib_path()], capture_output=True, text=True, check=True).stdout
    syms = {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
    for h in HEADERS:
        for n in declared(h):
            assert n in syms, f"{n} is not an unmangled dynamic symbol"


def test_headers_compile_as_c_and_cxx(tmp_path):
    src = tmp_path / "h.c"
    src.write_text("".join(f'#include "{h}"\n' for h in HEADERS) + "int main(void) { return 0; }\n")
    for comp, extra in (("gcc", ["-std=c11"]), ("g++", ["-x", "c++", "-std=c++17"])):
        subprocess.run([comp, *extra, "-Wall", "-Werror", "-I", INC, "-c", str(src), "-o", str(tmp_path / "h.o")],
                       check=True)


@pytest.mark.skipif(not os.path.exists(REF_SN_H), reason="reference tree not present (only in the build container)")
def test_signatures_match_reference_header(tmp_path):
    """Both headers in one C file: C rejects two prototypes of one function that differ in any parameter type."""
    src = tmp_path / "both.c"
    # the reference header relies on its includer for size_t / int32_t
    src.write_text(f'#include <stddef.h>\n#include <stdint.h>\n#include "{REF_SN_H}"\n'
                   f'#include "{os.path.join(INC, "sn.h")}"\nint main(void) {{ return 0; }}\n')
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-c", str(src), "-o", str(tmp_path / "b.o")],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.skipif(not os.path.exists(REF_FFI), reason="reference tree not present (only in the build container)")
def test_rust_extern_block_links(lib):
    """Every `fn sn_*` the Rust binding declares is exported, so its extern block links unchanged."""
    txt = open(REF_FFI).read()
    names = sorted(set(re.findall(r"\bfn\s+(sn_\w+)\s*\(", txt)))
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
