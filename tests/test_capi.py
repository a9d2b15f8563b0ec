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


def test_header_parameter_counts_match_the_bindings():
    """Every declaration's parameter count equals its ctypes binding's: a parameter added
    on one side only (as the sparse readers' counts were) shifts every later argument."""
    text = (ROOT / "include" / "flashloop_amd.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    for name, params in re.findall(r"\b(fl_[a-z0-9_]+)\s*\(([^;]*?)\)\s*;", text):
        params = " ".join(params.split())
        n = 0 if params in ("", "void") else params.count(",") + 1
        assert n == len(_lib.SIGNATURES[name][1]), f"{name}: header {n} parameters, binding {len(_lib.SIGNATURES[name][1])}"


def test_sparse_reader_counts_only_for_ragged_batches():
    """The layer hands the selection's counts to the sparse readers only when its
    sequences differ in length (equal lengths leave no padding to skip)."""
    from flashloop_amd.cache import CrossLoopKVLayer, LayerGeometry

    layer = CrossLoopKVLayer(LayerGeometry(2, 1, 256, 128, (256, 256, 1, 1)), "cpu")
    counts = object()
    layer.packed_host, layer.tail_host = [192, 128], [70, 134]  # 262 keys each
    assert layer._reader_counts(counts) is None
    layer.tail_host = [70, 100]
    assert layer._reader_counts(counts) is counts
    assert layer._reader_counts(None) is None


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
def test_library_exports_every_declared_symbol():
    lib = C.CDLL(str(_lib.LIB_PATH))
    for name in _declared_functions():
        assert hasattr(lib, name), name


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
def test_argument_errors_are_reported_without_launching():
    lib = _lib.load()
    assert lib.fl_abi_version() == 4
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


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
def test_sparse_readers_require_value_codes_in_the_key_lines():
    """The sparse readers load a token's V codes from the second half of its K line, so a
    view whose value_codes[s] is not key_codes[s] + 64 is refused before any launch."""
    lib = _lib.load()
    v = _lib.FlCacheView()
    v.batch, v.heads, v.token_capacity, v.tail_capacity = 1, 1, 64, 64
    v.row_capacity[:] = [64, 64, 64, 64]
    v.max_packed_tokens = 64
    v.packed_tokens, v.tail_tokens, v.value_meta_token = 0x1000, 0x1100, 0x1200
    v.tail_key[0], v.tail_value[0] = 0x1300, 0x1400
    v.key_codes[0], v.key_meta[0], v.value_meta[0], v.key_meta_half[0] = 0x10000, 0x2000, 0x3000, 0x4000

    def call(value_codes):
        v.value_codes[0] = value_codes
        return lib.fl_decode_selected_pv(C.byref(v), 0, 0x5000, 0x6000, 0x7000, 16, None, 0x8000, 0x9000, 0x100000,
                                         0, None)

    assert call(0x20000) == _lib.FL_E_INVALID and b"second half" in lib.fl_last_error()
    # the laid-out view passes this check and stops at the next one (the workspace size)
    assert call(0x10000 + 64) == _lib.FL_E_INVALID and b"workspace" in lib.fl_last_error()
    # absent slots read row 0 of each stream and token 0's record, also with nothing packed
    # yet: a stream without rows or a missing pointer is refused, never dereferenced
    v.max_packed_tokens = 0
    v.row_capacity[0] = 0
    assert call(0x10000 + 64) == _lib.FL_E_INVALID and b"without rows" in lib.fl_last_error()
    v.row_capacity[0] = 64
    v.key_meta_half[0] = 0
    assert call(0x10000 + 64) == _lib.FL_E_INVALID and b"null stream" in lib.fl_last_error()
    v.key_meta_half[0] = 0x4000
    v.value_meta_token = 0
    assert call(0x10000 + 64) == _lib.FL_E_INVALID and b"token records" in lib.fl_last_error()
    # rows and tokens beyond what the readers' 32-bit line offsets address are refused
    v.value_meta_token = 0x1200
    v.token_capacity = (1 << 24) + 64
    assert call(0x10000 + 64) == _lib.FL_E_INVALID and b"token_capacity above" in lib.fl_last_error()
    v.token_capacity = 64
    v.row_capacity[0] = (1 << 24) + 1
    assert call(0x10000 + 64) == _lib.FL_E_INVALID and b"row_capacity above" in lib.fl_last_error()


@pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="library not built")
def test_dense_reader_refuses_streams_without_rows():
    lib = _lib.load()
    v = _lib.FlCacheView()
    v.batch, v.heads, v.token_capacity, v.tail_capacity = 1, 1, 64, 128
    v.row_capacity[:] = [64, 64, 0, 0]
    v.max_packed_tokens = 64
    v.packed_tokens, v.tail_tokens = 0x1000, 0x1100
    v.tail_key[2], v.tail_value[2] = 0x1300, 0x1400
    for s in range(4):
        v.key_codes[s], v.value_codes[s] = 0x10000 * (s + 1), 0x10000 * (s + 1) + 64
        v.key_meta_half[s], v.value_meta_half[s] = 0x2000 + 0x100 * s, 0x3000 + 0x100 * s
    v.rank[0], v.rank[1] = 0x5000, 0x6000
    rc = lib.fl_decode_attn_dense(C.byref(v), 2, 0x7000, 0x7100, 0x7200, 1.0, 0x8000, None, 0, 0x100000, 1 << 20,
                                  None)
    assert rc == _lib.FL_E_INVALID and b"without rows" in lib.fl_last_error()


def test_layer_geometry_needs_a_row_in_every_stream():
    from flashloop_amd.cache import CrossLoopKVLayer, LayerGeometry

    with pytest.raises(ValueError, match="row capacity"):
        CrossLoopKVLayer(LayerGeometry(1, 1, 64, 128, (64, 64, 0, 1)), "cpu")
