"""libpa.so loads and exports every entry point the headers declare.

CPU-only: nothing here launches a kernel.  The argument checks exercised
return before any HIP call, so they run without a GPU.
"""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("pa.h", "pa_kv_cache.h", "pa_dense.h")]


def declared_symbols():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names.update(re.findall(r"\b(pa_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


@pytest.fixture(scope="module")
def lib(pa):
    return pa._lib.load()


def test_headers_declare_the_path():
    names = declared_symbols()
    for required in ("pa_reshape_and_cache", "pa_decode", "pa_prefill", "pa_read_kv",
                     "pa_decode_workspace_size", "pa_last_error", "pa_kv_cache_write_kv"):
        assert required in names


def test_every_declared_symbol_is_exported(lib, pa):
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing
    # and the ctypes table covers exactly the declared set
    assert sorted(pa._lib.SIGNATURES) == declared_symbols()


def test_version_and_empty_error(lib):
    assert b"gfx950" in lib.pa_version()
    assert lib.pa_last_error() == b""


def test_workspace_size(lib):
    # one partition (<= 128 tokens) needs none; otherwise B*Hq*(P+2)*(D+2)
    # f32 with P = ceil(ctx / 128) (the f32 group kernel's shortest
    # partitions; a balanced launch writes up to ceil(ctx / 256) + 3 partial
    # results per row) and the shared-prefix group record (6 B + 2 ints)
    assert lib.pa_decode_workspace_size(64, 32, 128, 128) == 0
    assert lib.pa_decode_workspace_size(64, 32, 128, 4096) == 64 * 32 * 34 * 130 * 4 + 386 * 4
    assert lib.pa_decode_workspace_size(2, 4, 64, 257) == 2 * 4 * 5 * 66 * 4 + 14 * 4


def test_argument_errors_without_gpu(lib):
    null = None
    # unknown dtype
    rc = lib.pa_decode(null, null, null, null, null, 4, null, 64, 1, 8, 2, 64, 16, 1.0, null, 0,
                       7, null)
    assert rc == -1 and b"dtype" in lib.pa_last_error()
    # Hq not a multiple of Hkv
    rc = lib.pa_decode(null, null, null, null, null, 4, null, 64, 1, 7, 2, 64, 16, 1.0, null, 0,
                       1, null)
    assert rc == -1 and b"multiple" in lib.pa_last_error()
    # context longer than the block table
    rc = lib.pa_decode(null, null, null, null, null, 4, null, 65, 1, 8, 2, 64, 16, 1.0, null, 0,
                       1, null)
    assert rc == -2
    # missing workspace for a launch merged by the reduce kernel (more than 4
    # partitions; null pointers are checked first)
    rc = lib.pa_decode(C.c_void_p(8), C.c_void_p(8), C.c_void_p(8), C.c_void_p(8),
                       C.c_void_p(8), 256, C.c_void_p(8), 4096, 1, 8, 2, 64, 16, 1.0, null, 0, 1,
                       null)
    assert rc == -4 and b"workspace" in lib.pa_last_error()
    # pa_linear: f32, K not a multiple of 32, N not a multiple of 16, bias with SwiGLU
    p = C.c_void_p(16)
    assert lib.pa_linear(p, p, p, null, 4, 64, 96, 0, 0, 0, 0.0, null, 0, 0, null) == -3
    assert lib.pa_linear(p, p, p, null, 4, 64, 80, 0, 0, 0, 0.0, null, 0, 1, null) == -3
    assert b"multiple of 32" in lib.pa_last_error()
    assert lib.pa_linear(p, p, p, null, 4, 40, 96, 0, 0, 0, 0.0, null, 0, 1, null) == -3
    assert lib.pa_linear(p, p, p, p, 4, 48, 96, 1, 0, 0, 0.0, null, 0, 1, null) == -1
    assert lib.pa_linear(null, null, null, null, 0, 64, 96, 0, 0, 0, 0.0, null, 0, 1, null) == 0
    assert lib.pa_linear(p, p, p, null, 4, 64, 96, 1, 0, 2, 0.0, null, 0, 1, null) == -1  # add + SwiGLU
    assert lib.pa_linear(p, p, p, null, 4, 64, 96, 0, 0, 1, 0.0, null, 0, 1, null) == -1  # rms, eps 0
    # pa_linear_rope_cache / pa_linear_pack_qkv: f32, head_dim not a multiple of 32,
    # the residual-add flag
    assert lib.pa_linear_rope_cache(p, p, p, null, 4, 8, 2, 64, 128, 0, 0.0, p, p, p, p, p, 8,
                                    0, null) == -3
    assert lib.pa_linear_rope_cache(p, p, p, null, 4, 8, 2, 48, 128, 0, 0.0, p, p, p, p, p, 8,
                                    1, null) == -3
    assert lib.pa_linear_rope_cache(p, p, p, null, 4, 8, 2, 64, 128, 2, 0.0, p, p, p, p, p, 8,
                                    1, null) == -1
    assert lib.pa_linear_pack_qkv(p, C.c_void_p(32), null, 8, 2, 48, 128, 1, null) == -3
    # pa_linear's K split: long K over few tiles only; a workspace not 256-byte aligned
    assert lib.pa_linear_workspace_size(32, 896, 4864, 0) > 0
    assert lib.pa_linear_workspace_size(32, 896, 896, 0) == 0
    assert lib.pa_linear_workspace_size(32, 151936, 896, 0) == 0
    assert lib.pa_linear_workspace_size(0, 896, 4864, 0) == 0
    assert lib.pa_linear(p, p, p, null, 32, 896, 4864, 0, 0, 0, 0.0, C.c_void_p(16), 1 << 30, 1,
                         null) == -1
    assert lib.pa_linear_pack(p, C.c_void_p(32), null, 24, 64, 1, null) == -3  # rows not a multiple of 16
    # argmax: unknown dtype, row stride below cols, null pointer; no rows is a no-op
    assert lib.pa_argmax(p, p, 2, 8, 0, 9, null) == -1
    assert lib.pa_argmax(p, p, 2, 8, 4, 1, null) == -1
    assert lib.pa_argmax(null, p, 2, 8, 0, 1, null) == -1
    assert lib.pa_argmax(null, null, 0, 8, 0, 1, null) == 0
    # read_kv: table cannot hold seq_len
    rc = lib.pa_read_kv(null, null, null, 1, 17, 2, 4, 4, null, null, 0, null)
    assert rc == -2
    # prefill unsupported head_dim
    rc = lib.pa_prefill(null, null, null, null, null, 4, null, null, 1, 1, 1, 2, 2, 1024, 4,
                        1.0, 1, null)
    assert rc == -3
    # empty work is a no-op success
    assert lib.pa_reshape_and_cache(null, null, null, null, null, 0, 2, 4, 4, 0, 0, 0, null) == 0
    assert lib.pa_last_error() == b""


def test_kv_cache_create_rejects_bad_sizes(lib):
    h = C.c_void_p()
    assert lib.pa_kv_cache_create(0, 2, 4, 4, 0, C.byref(h)) == -1
    assert not h.value
