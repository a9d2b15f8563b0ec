"""The C-ABI library loads and exports every symbol include/flashloop_amd.h declares
(CPU only: no compute call is made; only argument validation that fails before any
HIP call is exercised)."""

import ctypes as C
import re
from pathlib import Path

import pytest

from flashloop_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def _declared_functions():
    text = (ROOT / "include" / "flashloop_amd.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fl_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_signatures():
    assert _declared_functions() == sorted(_lib.SIGNATURES)


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
def test_library_exports_every_declared_symbol():
    lib = C.CDLL(str(_lib.LIB_PATH))
    for name in _declared_functions():
        assert hasattr(lib, name), name


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
def test_argument_errors_are_reported_without_launching():
    lib = _lib.load()
    assert lib.fl_abi_version() == 3
    rc = lib.fl_decode_topk(None, 1, 1, None, 1, 0.1, 64, None, None, None, None, None, None, None)
    assert rc == _lib.FL_E_INVALID
    assert b"null" in lib.fl_last_error()
    rc = lib.fl_decode_attn_dense(None, 0, None, None, None, 1.0, None, None, 0, None, 0, None)
    assert rc == _lib.FL_E_INVALID and b"view" in lib.fl_last_error()
    v = _lib.FlCacheView()
    rc = lib.fl_decode_attn_dense(C.byref(v), 7, None, None, None, 1.0, None, None, 0, None, 0, None)
    assert rc == _lib.FL_E_INVALID and b"loop" in lib.fl_last_error()
    rc = lib.fl_select_tokens(None, 1, 4, 0.5, None, 1, None, None, None, None, None)
    assert rc == _lib.FL_E_INVALID
    rc = lib.fl_gather_rows(None, 0, 0, 0, None, 0, 0, 0, 0, None, 0, None, None)
    assert rc == _lib.FL_E_INVALID
    # the fused chain + GEMV rejects its bad arguments before any launch
    ws = _lib.ptr_array([0x1000])
    outs = _lib.ptr_array([0x2000])
    chain = lambda m, k, x, r, wa, stride: lib.fl_gemv_bf16_chain(
        m, k, 1e-6, x, r, wa, None, None, None, stride, C.cast(ws, _lib._PP), 8, 0, C.cast(outs, _lib._PP), 8, None, 8,
        None, None, 128, None)
    assert chain(1, 2048, None, None, None, 2048) == _lib.FL_E_INVALID and b"null residual" in lib.fl_last_error()
    assert chain(1, 8192, None, 0x3000, None, 8192) == _lib.FL_E_INVALID and b"4096" in lib.fl_last_error()
    assert chain(1, 2048, 0x4000, 0x3000, None, 2048) == _lib.FL_E_INVALID and b"norm weight" in lib.fl_last_error()
    assert chain(1, 2048, None, 0x3008, None, 2048) == _lib.FL_E_INVALID and b"aligned" in lib.fl_last_error()


def test_struct_layout_matches_header(tmp_path):
    """The ctypes mirror of fl_cache_view has the C struct's size and field offsets
    (compiled from include/flashloop_amd.h with the host C compiler)."""
    import shutil
    import subprocess

    fields = [f[0] for f in _lib.FlCacheView._fields_]
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no host C compiler")
    inc = Path(__file__).resolve().parents[1] / "include"
    src = tmp_path / "layout.c"
    body = "".join(f'  printf("%zu\\n", offsetof(fl_cache_view, {f}));\n' for f in fields)
    src.write_text("#include <stddef.h>\n#include <stdio.h>\n#include \"flashloop_amd.h\"\n"
                   "int main(void) {\n" + body + '  printf("%zu\\n", sizeof(fl_cache_view));\n  return 0;\n}\n')
    exe = tmp_path / "layout"
    subprocess.run([cc, "-I", str(inc), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    want = [getattr(_lib.FlCacheView, f).offset for f in fields] + [C.sizeof(_lib.FlCacheView)]
    assert got == want
