"""CPU tests of the C ABI: the library loads, exports every symbol that
include/memopt_hip.h declares, and its host-side logic (pool free list,
argument validation, error strings) behaves like the reference's
(src/csrc/kv_cache.cu:112-201, src/csrc/quantization.cu:294-311). No kernel
is launched here."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "memopt_hip.h")
LIB = os.path.join(ROOT, "memopt-transformer-runtime_amd", "memopt_C", "libmemopt_hip.so")

OK, ERR_INVALID, ERR_STATE = 0, 1, 2


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(memopt_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    import torch  # noqa: F401  (load torch's HIP runtime first, as the shim does)
    assert os.path.exists(LIB), "build the library first: python memopt-transformer-runtime_amd/build.py"
    lib = ctypes.CDLL(LIB)
    lib.memopt_last_error.restype = ctypes.c_char_p
    return lib


def test_header_declares_the_reference_surface():
    syms = declared_symbols()
    for name in ["memopt_init_pool", "memopt_allocate_block", "memopt_free_block", "memopt_free_blocks_count",
                 "memopt_write_cache", "memopt_evict_cache", "memopt_evict_tokens",
                 "memopt_dynamic_sparse_attention", "memopt_quantize_kv_cache_int4",
                 "memopt_dequantize_kv_cache_int4", "memopt_get_hello", "memopt_last_error"]:
        assert name in syms


def test_every_declared_symbol_is_exported(lib):
    nm = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (memopt_\w+)", nm))
    missing = [s for s in declared_symbols() if s not in exported]
    assert not missing, missing
    for s in declared_symbols():
        assert hasattr(lib, s)


def test_hello_string(lib):
    lib.memopt_get_hello.restype = ctypes.c_char_p
    # tests/test_import.py:9 of the reference accepts this substring
    assert "MemOpt C++ Backend Initialized" in lib.memopt_get_hello().decode()


def _init(lib, nb, bs=16, h=8, d=64, fmt=0):
    dummy = ctypes.c_void_p(16)  # registered, never dereferenced by host-only calls
    return lib.memopt_init_pool(ctypes.c_int64(nb), bs, h, d, fmt, dummy, dummy, dummy, dummy)


def test_pool_fifo_and_exhaustion(lib):
    assert _init(lib, 3) == OK
    out = ctypes.c_int64()
    got = []
    for _ in range(4):
        assert lib.memopt_allocate_block(ctypes.byref(out)) == OK
        got.append(out.value)
    assert got == [0, 1, 2, -1]  # FIFO, -1 when exhausted (not an error)
    assert lib.memopt_free_block(ctypes.c_int64(1)) == OK
    assert lib.memopt_free_block(ctypes.c_int64(0)) == OK
    cnt = ctypes.c_int64()
    lib.memopt_free_blocks_count(ctypes.byref(cnt))
    assert cnt.value == 2
    lib.memopt_allocate_block(ctypes.byref(out))
    assert out.value == 1  # returned blocks go to the back, FIFO order
    assert lib.memopt_free_block(ctypes.c_int64(3)) == ERR_INVALID
    assert b"out of range" in lib.memopt_last_error()
    lib.memopt_reset_pool()


def test_pool_info_and_reinit(lib):
    assert _init(lib, 5, 16, 4, 128, 1) == OK
    nb, bs, h, d, f = ctypes.c_int64(), *(ctypes.c_int32() for _ in range(4))
    assert lib.memopt_pool_info(ctypes.byref(nb), ctypes.byref(bs), ctypes.byref(h), ctypes.byref(d),
                                ctypes.byref(f)) == 1
    assert (nb.value, bs.value, h.value, d.value, f.value) == (5, 16, 4, 128, 1)
    assert _init(lib, 5, 16, 4, 96, 1) == ERR_INVALID  # INT4 needs head_dim % 64 == 0
    assert lib.memopt_pool_info(None, None, None, None, None) == 0  # failed init leaves no pool


def test_invalid_init_tears_down_and_write_reports_uninitialized(lib):
    assert _init(lib, 4) == OK
    assert _init(lib, 0) == ERR_INVALID
    assert b"num_blocks must be > 0" in lib.memopt_last_error()
    rc = lib.memopt_write_cache(None, None, ctypes.c_int64(1), 8, 64, None, None)
    assert rc == ERR_STATE
    # tests/test_attention.py:287 of the reference matches this message
    assert re.search(b"pool not initialized|out of bounds|exhausted", lib.memopt_last_error())
    out = ctypes.c_int64()
    assert lib.memopt_allocate_block(ctypes.byref(out)) == ERR_STATE


def test_quantize_argument_guards(lib):
    f = lib.memopt_quantize_kv_cache_int4
    f.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p,
                  ctypes.c_void_p, ctypes.c_void_p]
    assert f(None, 512, 128, 32, None, None, None) == ERR_INVALID      # group_size != 64
    assert b"group_size must equal 64" in lib.memopt_last_error()
    assert f(None, 100, 2, 64, None, None, None) == ERR_INVALID        # numel % 64 != 0
    assert f(None, 192, 3, 64, None, None, None) == ERR_INVALID        # odd last dim
    assert f(None, 0, 128, 64, None, None, None) == OK                 # empty is a no-op


def test_evict_workspace_size_and_guard(lib):
    """memopt_evict_workspace_size: a 256-byte header, 4 bytes of page mark per
    pool block (rounded to 256), plus long-row state only past 32768 tokens;
    memopt_evict_tokens refuses a smaller workspace before launching anything."""
    size = lib.memopt_evict_workspace_size
    size.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int64,
                     ctypes.POINTER(ctypes.c_int64)]
    out = ctypes.c_int64()
    assert size(2, 8, 4096, 256, 1000, ctypes.byref(out)) == OK
    assert out.value == 256 + 4096  # 4000 bytes of marks, rounded up to 256
    assert size(2, 8, 32768, 2048, 1000, ctypes.byref(out)) == OK and out.value == 256 + 4096
    assert size(2, 8, 32769, 2049, 1000, ctypes.byref(out)) == OK and out.value > 256 + 4096
    short = out.value
    assert size(2, 8, 200000, 12500, 1000, ctypes.byref(out)) == OK and out.value > short
    assert _init(lib, 64, 16, 8, 64, 1) == OK
    ev = lib.memopt_evict_tokens
    ev.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32,
                   ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int64,
                   ctypes.c_void_p]
    dummy = ctypes.c_void_p(256)
    assert size(1, 8, 64, 4, 64, ctypes.byref(out)) == OK
    rc = ev(dummy, 1, 8, 64, dummy, 4, dummy, 64, 0.5, 4, dummy, out.value - 1, None)
    assert rc == ERR_INVALID and b"workspace too small" in lib.memopt_last_error()
    rc = ev(dummy, 1, 8, 64, dummy, 4, dummy, 64, 0.5, 4, None, 0, None)
    assert rc == ERR_INVALID and b"workspace too small" in lib.memopt_last_error()
    lib.memopt_reset_pool()


def test_paged_attention_requires_its_workspace(lib):
    """A decode that splits needs the workspace memopt_attention_workspace_size
    reports: memopt_paged_attention refuses a call without it (no silent
    unsplit fallback) before launching anything."""
    import memopt_C
    d = memopt_C.AttnDesc()
    p = 256
    d.query = d.out = d.key_cache = d.block_tables = d.context_lens = p
    d.batch, d.q_len, d.num_heads, d.head_dim = 1, 1, 1, 128
    d.kv_format, d.block_size, d.num_kv_blocks = 1, 16, 4096
    d.max_blocks_per_seq, d.max_seq_len, d.window_size = 4096, 65536, 65536
    need = ctypes.c_int64()
    ws = lib.memopt_attention_workspace_size
    ws.argtypes = [ctypes.POINTER(memopt_C.AttnDesc), ctypes.POINTER(ctypes.c_int64)]
    assert ws(ctypes.byref(d), ctypes.byref(need)) == OK and need.value > 0
    attn = lib.memopt_paged_attention
    attn.argtypes = [ctypes.POINTER(memopt_C.AttnDesc), ctypes.c_void_p]
    assert attn(ctypes.byref(d), None) == ERR_INVALID
    assert b"workspace too small" in lib.memopt_last_error()
