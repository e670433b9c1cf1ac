"""memopt_C — drop-in for the reference's pybind11 extension, backed by gfx950 HIP.

Same module name, function names, argument order/keywords, return types and
error type (``RuntimeError``) as TheRadDani/memopt-transformer-runtime
``src/csrc/extension.cpp:10-124``, so ``memopt.DynamicAttention`` and the
reference tests run unchanged against it. Calls go through the C ABI of
``libmemopt_hip.so`` (declared in ``include/memopt_hip.h``); torch is used only
to allocate device tensors and to pass the current HIP stream.

Additions (new names or keyword-only arguments whose defaults keep the
reference behaviour):
  * ``get_key_pool()`` / ``get_value_pool()`` — called by the reference's
    ``DynamicAttention`` (src/memopt/attention.py:330-331) but missing from
    its extension;
  * ``init_pool(..., kv_format="int4")`` — INT4 page pool: one u8 buffer
    [nb, H, 17*D] of (page, head) blocks holding K codes, V codes, K scales
    and V scales (layout in csrc/page_format.hpp); ``write_cache`` then
    quantizes on the fly, ``get_int4_pages()`` returns the buffer and
    ``get_pool_scales()`` the fp16 scale regions;
  * ``dynamic_sparse_attention(..., *, num_sink_tokens=0, causal=False,
    key_scales=None, value_scales=None, kv_layout=None)`` — INT4 caches are
    dequantized just in time inside the kernel;
  * ``free_evicted_blocks(is_block_free)`` — the post-eviction sweep the
    reference documents but never implements (src/csrc/kv_cache.cu:1033-1036).

The library is loaded at import; a missing or unloadable library raises
``ImportError`` naming the path (there is no CPU fallback).
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import List, Optional, Tuple

import torch  # must precede the HIP library so both share one HIP runtime

__all__ = [
    "get_hello", "init_pool", "allocate_block", "free_block", "get_pool_tensors",
    "get_key_pool", "get_value_pool", "get_pool_scales", "get_int4_pages", "int4_layout", "free_blocks_count",
    "write_cache", "evict_cache", "evict_tokens", "free_evicted_blocks",
    "dynamic_sparse_attention", "PreparedAttention", "quantize_kv_cache_int4", "dequantize_kv_cache_int4",
    "library_path",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
library_path = os.environ.get("MEMOPT_HIP_LIB", os.path.join(_HERE, "libmemopt_hip.so"))

if not os.path.exists(library_path):
    raise ImportError(
        f"memopt_C: {library_path} is missing; build it with "
        "`python memopt-transformer-runtime_amd/build.py` (there is no CPU fallback)")
try:
    _lib = ctypes.CDLL(library_path)
except OSError as exc:  # pragma: no cover - environment specific
    raise ImportError(f"memopt_C: cannot load {library_path}: {exc}") from exc

_i32, _i64, _f32, _vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p


class AttnDesc(ctypes.Structure):
    """Mirror of ``memopt_attn_desc`` (include/memopt_hip.h)."""

    _fields_ = [
        ("query", _vp), ("out", _vp),
        ("batch", _i32), ("q_len", _i32), ("num_heads", _i32), ("head_dim", _i32),
        ("kv_format", _i32),
        ("key_cache", _vp), ("value_cache", _vp), ("key_scales", _vp), ("value_scales", _vp),
        ("scale_dtype", _i32), ("block_size", _i32), ("num_kv_blocks", _i64),
        ("kv_page_stride", _i64), ("kv_head_stride", _i64), ("kv_token_stride", _i64),
        ("sc_page_stride", _i64), ("sc_head_stride", _i64), ("sc_token_stride", _i64),
        ("block_tables", _vp), ("max_blocks_per_seq", _i32), ("context_lens", _vp),
        ("max_seq_len", _i32), ("window_size", _i32), ("num_sink_tokens", _i32), ("causal", _i32),
        ("workspace", _vp), ("workspace_bytes", _i64),
    ]


def _sig(name, args, res=_i32):
    f = getattr(_lib, name)
    f.argtypes = args
    f.restype = res
    return f


_lib.memopt_last_error.restype = ctypes.c_char_p
_lib.memopt_get_hello.restype = ctypes.c_char_p
_c_init_pool = _sig("memopt_init_pool", [_i64, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp])
_c_pool_info = _sig("memopt_pool_info", [ctypes.POINTER(_i64)] + [ctypes.POINTER(_i32)] * 4)
_c_reset_pool = _sig("memopt_reset_pool", [])
_c_set_storage = _sig("memopt_pool_set_storage", [_i32, _vp, _vp])
_c_pages_to_fp16 = _sig("memopt_int4_pages_to_fp16", [_vp, _i64, _i32, _i32, _vp, _vp, _vp])
_c_alloc = _sig("memopt_allocate_block", [ctypes.POINTER(_i64)])
_c_free = _sig("memopt_free_block", [_i64])
_c_free_count = _sig("memopt_free_blocks_count", [ctypes.POINTER(_i64)])
_c_write = _sig("memopt_write_cache", [_vp, _vp, _i64, _i32, _i32, _vp, _vp])
_c_evict_cache = _sig("memopt_evict_cache", [_vp, _i64, _f32, _i32, _vp])
_c_evict_tokens = _sig("memopt_evict_tokens",
                       [_vp, _i32, _i32, _i32, _vp, _i32, _vp, _i64, _f32, _i32, _vp, _i64, _vp])
_c_evict_ws = _sig("memopt_evict_workspace_size", [_i32, _i32, _i32, _i32, _i64, ctypes.POINTER(_i64)])
_c_quant = _sig("memopt_quantize_kv_cache_int4", [_vp, _i64, _i64, _i32, _vp, _vp, _vp])
_c_dequant = _sig("memopt_dequantize_kv_cache_int4", [_vp, _i64, _vp, _i64, _i32, _vp, _vp])
_c_dsa = _sig("memopt_dynamic_sparse_attention",
              [_vp, _i32, _i32, _i32, _i32, _vp, _vp, _i64, _i32, _vp, _i32, _vp, _i32, _i32, _vp, _vp])
_c_ws = _sig("memopt_attention_workspace_size", [ctypes.POINTER(AttnDesc), ctypes.POINTER(_i64)])
_c_attn = _sig("memopt_paged_attention", [ctypes.POINTER(AttnDesc), _vp])
_c_attn_noalloc = _sig("memopt_paged_attention_noalloc", [ctypes.POINTER(AttnDesc), _vp])

KV_FP16, KV_INT4, KV_INT4_ROWS = 0, 1, 2
_FORMATS = {"fp16": KV_FP16, "int4": KV_INT4}


def _check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(_lib.memopt_last_error().decode())


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _cuda(t: torch.Tensor, name: str, fn: str) -> None:
    _require(isinstance(t, torch.Tensor) and t.is_cuda, f"{fn}: {name} must be a CUDA tensor")


# ---------------------------------------------------------------------------
# Handshake
# ---------------------------------------------------------------------------

def get_hello() -> str:
    """src/csrc/extension.cpp:6-8 (string carries "MemOpt C++ Backend Initialized")."""
    return _lib.memopt_get_hello().decode()


# ---------------------------------------------------------------------------
# Pool — src/csrc/kv_cache.cu:83-201
# ---------------------------------------------------------------------------

_pool_lock = threading.Lock()
_pool: dict = {}


def init_pool(num_blocks: int, block_size: int, num_heads: int, head_dim: int,
              kv_format: str = "fp16") -> None:
    """Allocate zeroed pool storage on the current device and seed the FIFO free list.

    Idempotent for identical parameters (src/csrc/kv_cache.cu:115-122);
    different parameters reset the pool. Invalid parameters raise
    ``RuntimeError`` and leave no pool behind.
    """
    fmt = _FORMATS.get(kv_format)
    _require(fmt is not None, f"init_pool: kv_format must be one of {sorted(_FORMATS)}")
    with _pool_lock:
        nb, bs, h, d, f = _i64(), _i32(), _i32(), _i32(), _i32()
        if _c_pool_info(ctypes.byref(nb), ctypes.byref(bs), ctypes.byref(h), ctypes.byref(d), ctypes.byref(f)):
            if (nb.value, bs.value, h.value, d.value, f.value) == (num_blocks, block_size, num_heads, head_dim, fmt):
                return
        _pool.clear()
        _c_reset_pool()
        ok = num_blocks > 0 and block_size > 0 and num_heads > 0 and head_dim > 0 and head_dim % 2 == 0
        if not ok or (fmt == KV_INT4 and head_dim % 64):
            # Let the library produce the reference's message (and stay torn down).
            _check(_c_init_pool(num_blocks, block_size, num_heads, head_dim, fmt, 1, 1, 1, 1))
        if fmt == KV_INT4 and block_size != 16:
            _check(_c_init_pool(num_blocks, block_size, num_heads, head_dim, fmt, 1, None, None, None))
        dev = torch.device("cuda", torch.cuda.current_device())
        if fmt == KV_FP16:
            shape = (num_blocks, block_size, num_heads, head_dim)
            k = torch.zeros(shape, dtype=torch.float16, device=dev)
            v = torch.zeros(shape, dtype=torch.float16, device=dev)
            _check(_c_init_pool(num_blocks, block_size, num_heads, head_dim, fmt, k.data_ptr(), v.data_ptr(),
                                None, None))
            _pool.update(k=k, v=v, pages=None)
        else:
            lay = int4_layout(head_dim)
            pages = torch.empty((num_blocks, num_heads, lay["block"]), dtype=torch.uint8, device=dev)
            pages.copy_(_empty_int4_block(head_dim, dev).expand_as(pages))
            _check(_c_init_pool(num_blocks, block_size, num_heads, head_dim, fmt, pages.data_ptr(), None, None, None))
            _pool.update(pages=pages, k=pages[:, :, lay["kcodes"]:lay["vcodes"]],
                         v=pages[:, :, lay["vcodes"]:lay["kscales"]],
                         ks=pages[:, :, lay["kscales"]:lay["vscales"]].view(torch.float16),
                         vs=pages[:, :, lay["vscales"]:].view(torch.float16))
        _pool.update(fmt=fmt, nb=num_blocks, bs=block_size, h=num_heads, d=head_dim)


def reset_pool() -> None:
    """Drop the pool (storage and free list); the next ``init_pool`` starts fresh."""
    with _pool_lock:
        _pool.clear()
        _c_reset_pool()


def int4_layout(head_dim: int) -> dict:
    """Byte offsets of the regions of one (page, head) block of the INT4 page
    pool (include/memopt_hip.h MEMOPT_KV_INT4)."""
    D, G = head_dim, head_dim // 64
    return {"kcodes": 0, "vcodes": 8 * D, "kscales": 16 * D, "vscales": 16 * D + 32 * G, "block": 16 * D + 64 * G}


def _empty_int4_block(head_dim: int, dev) -> torch.Tensor:
    """One (page, head) block of an empty row set: codes 8 (0x88), scales 1.0."""
    lay = int4_layout(head_dim)
    blk = torch.full((lay["block"],), 0x88, dtype=torch.uint8)
    blk[lay["kscales"]:] = torch.ones((lay["block"] - lay["kscales"]) // 2, dtype=torch.float16).view(torch.uint8)
    return blk.to(dev)


def _pool_or_raise(fn: str) -> dict:
    _require(bool(_pool), f"{fn}: pool not initialized")
    return _pool


def allocate_block() -> int:
    """Pop one free block (FIFO); -1 when exhausted (src/csrc/kv_cache.cu:163-172)."""
    out = _i64()
    _check(_c_alloc(ctypes.byref(out)))
    return int(out.value)


def free_block(block_idx: int) -> None:
    """Return a block to the free list (src/csrc/kv_cache.cu:179-185)."""
    _check(_c_free(int(block_idx)))


def free_blocks_count() -> int:
    out = _i64()
    _check(_c_free_count(ctypes.byref(out)))
    return int(out.value)


def get_pool_tensors() -> Tuple[torch.Tensor, torch.Tensor]:
    """(key_pool, value_pool) aliases of the live storage (src/csrc/kv_cache.cu:190-193).

    fp16 pools: [nb, bs, H, D] fp16. INT4 pools: views of the K and V code
    regions of the page buffer, uint8 [nb, H, 8*D] (codes in the page
    layout); passing them to ``dynamic_sparse_attention`` attends over the pool.
    """
    p = _pool_or_raise("get_pool_tensors")
    return p["k"], p["v"]


def get_int4_pages() -> torch.Tensor:
    """The INT4 page buffer, uint8 [nb, H, 16*D + 64*(D/64)]."""
    p = _pool_or_raise("get_int4_pages")
    _require(p["fmt"] == KV_INT4, "get_int4_pages: pool is not an INT4 pool")
    return p["pages"]


def pool_kv_format() -> str:
    """Storage format of the live pool: ``"fp16"`` or ``"int4"``."""
    return "int4" if _pool_or_raise("pool_kv_format")["fmt"] == KV_INT4 else "fp16"


def get_key_pool() -> torch.Tensor:
    return _pool_or_raise("get_key_pool")["k"]


def get_value_pool() -> torch.Tensor:
    return _pool_or_raise("get_value_pool")["v"]


def get_pool_scales() -> Tuple[torch.Tensor, torch.Tensor]:
    """fp16 group-scale regions of an INT4 pool, views [nb, H, 16*D/64] (page layout order)."""
    p = _pool_or_raise("get_pool_scales")
    _require(p["fmt"] == KV_INT4, "get_pool_scales: pool is not an INT4 pool")
    return p["ks"], p["vs"]


def dequantize_int4_pages(pages: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Dequantize an INT4 page buffer ``[nb, H, block]`` (default: the live pool)
    into fresh fp16 ``(K, V)`` pools ``[nb, 16, H, D]``.

    Each value is ``fp16(float(code - 8) * page_scale)``, the arithmetic of
    the reference dequantize kernel (src/csrc/quantization.cu:232-270) on this
    build's page layout; the attention kernels read the same values.
    """
    p = _pool_or_raise("dequantize_int4_pages")
    if pages is None:
        _require(p["fmt"] == KV_INT4, "dequantize_int4_pages: pool is not an INT4 pool")
        pages, D = p["pages"], p["d"]
    else:
        _require(pages.dim() == 3 and pages.dtype == torch.uint8, "dequantize_int4_pages: pages must be u8 [nb, H, B]")
        D = next((d for d in (64, 128) if int4_layout(d)["block"] == pages.shape[2]), None)
        _require(D is not None, "dequantize_int4_pages: block size matches no supported head_dim (64, 128)")
        _cuda(pages, "pages", "dequantize_int4_pages")
    pages = pages.contiguous()
    nb, H = pages.shape[0], pages.shape[1]
    k = torch.empty((nb, 16, H, D), dtype=torch.float16, device=pages.device)
    v = torch.empty_like(k)
    with torch.cuda.device(pages.device):
        _check(_c_pages_to_fp16(pages.data_ptr(), nb, H, D, k.data_ptr(), v.data_ptr(), _stream(pages)))
    return k, v


def convert_pool(kv_format: str) -> None:
    """Switch the live pool between ``"fp16"`` and ``"int4"`` storage in place.

    The free list and every block table stay valid: fp16 pages are quantized
    into INT4 pages (what ``write_cache`` into an INT4 pool would store for
    the same rows), INT4 pages are dequantized into fp16 pools. This is the
    switch MemoryScheduler.use_int4 asks for (src/memopt/scheduler.py:15-18);
    the reference has no code that performs it.
    """
    fmt = _FORMATS.get(kv_format)
    _require(fmt is not None, f"convert_pool: kv_format must be one of {sorted(_FORMATS)}")
    with _pool_lock:
        p = _pool_or_raise("convert_pool")
        if p["fmt"] == fmt:
            return
        nb, bs, H, D = p["nb"], p["bs"], p["h"], p["d"]
        dev = p["k"].device
        if fmt == KV_INT4:
            _require(bs == 16 and D % 64 == 0, "convert_pool: INT4 pools need 16-token pages and head_dim % 64 == 0")
            lay = int4_layout(D)
            pages = torch.empty((nb, H, lay["block"]), dtype=torch.uint8, device=dev)
            old_k, old_v = p["k"], p["v"]
            _check(_c_set_storage(KV_INT4, pages.data_ptr(), None))
            slots = torch.arange(nb * bs, dtype=torch.int32, device=dev)
            with torch.cuda.device(dev):
                _check(_c_write(old_k.data_ptr(), old_v.data_ptr(), nb * bs, H, D, slots.data_ptr(),
                                _stream(old_k)))
            _pool.update(fmt=fmt, pages=pages, k=pages[:, :, lay["kcodes"]:lay["vcodes"]],
                         v=pages[:, :, lay["vcodes"]:lay["kscales"]],
                         ks=pages[:, :, lay["kscales"]:lay["vscales"]].view(torch.float16),
                         vs=pages[:, :, lay["vscales"]:].view(torch.float16))
        else:
            k, v = dequantize_int4_pages()
            _check(_c_set_storage(KV_FP16, k.data_ptr(), v.data_ptr()))
            _pool.update(fmt=fmt, pages=None, k=k, v=v, ks=None, vs=None)


# ---------------------------------------------------------------------------
# write_cache — src/csrc/kv_cache.cu:282-348
# ---------------------------------------------------------------------------

def write_cache(keys: torch.Tensor, values: torch.Tensor, block_tables: torch.Tensor,
                slot_mapping: torch.Tensor, *, validate_slots: bool = True) -> None:
    """Scatter [T, H, D] fp16 rows into pool slots (INT4 pools: quantize on the fly).

    ``block_tables`` is accepted and unused, as in the reference (:279-280).
    Slots outside the pool raise ``RuntimeError("... out of bounds")``; that
    check costs one device-to-host sync, so hot loops whose slots are known
    good may pass ``validate_slots=False`` (the kernel still skips, never
    writes, out-of-range slots).
    """
    p = _pool_or_raise("write_cache")
    _require(keys.dim() == 3, "write_cache: keys must be 3-D [num_tokens, num_heads, head_dim]")
    _require(values.dim() == 3, "write_cache: values must be 3-D [num_tokens, num_heads, head_dim]")
    _require(slot_mapping.dim() == 1, "write_cache: slot_mapping must be 1-D [num_tokens]")
    T, H, D = keys.shape
    _require(tuple(values.shape) == (T, H, D), "write_cache: keys/values shape mismatch")
    _require(slot_mapping.shape[0] == T, "write_cache: slot_mapping length != num_tokens")
    _require(H == p["h"], "write_cache: num_heads != pool.num_heads")
    _require(D == p["d"], "write_cache: head_dim != pool.head_dim")
    _require(keys.dtype == torch.float16 and values.dtype == torch.float16, "write_cache: keys/values must be fp16")
    _cuda(keys, "keys", "write_cache")
    _cuda(values, "values", "write_cache")
    _cuda(slot_mapping, "slot_mapping", "write_cache")
    _require(slot_mapping.dtype == torch.int32, "write_cache: slot_mapping must be int32")
    if T == 0:
        return
    keys, values, slot_mapping = keys.contiguous(), values.contiguous(), slot_mapping.contiguous()
    if validate_slots:
        lo, hi = (int(x) for x in torch.aminmax(slot_mapping))
        _require(lo >= 0 and hi < p["nb"] * p["bs"], "write_cache: slot_mapping out of bounds")
    with torch.cuda.device(keys.device):
        _check(_c_write(keys.data_ptr(), values.data_ptr(), T, H, D, slot_mapping.data_ptr(), _stream(keys)))


# ---------------------------------------------------------------------------
# Eviction — src/csrc/kv_cache.cu:503-559, :1053-1156
# ---------------------------------------------------------------------------

def evict_cache(block_tables: torch.Tensor, attention_scores: torch.Tensor, retain_ratio: float,
                num_sink_tokens: int = 4) -> None:
    """Pool-centric eviction over scores [num_blocks, block_size, H] (f32)."""
    p = _pool_or_raise("evict_cache")
    _require(0.0 < retain_ratio <= 1.0, "evict_cache: retain_ratio must be in (0, 1]")
    _require(attention_scores.dim() == 3,
             "evict_cache: attention_scores must be 3-D [num_blocks, block_size, num_heads]")
    _require(attention_scores.dtype == torch.float32, "evict_cache: attention_scores must be float32")
    nb, bs, h = attention_scores.shape
    _require(nb <= p["nb"], "evict_cache: attention_scores num_blocks > pool.num_blocks")
    _require(bs == p["bs"], "evict_cache: attention_scores block_size != pool.block_size")
    _require(h == p["h"], "evict_cache: attention_scores num_heads != pool.num_heads")
    _cuda(attention_scores, "attention_scores", "evict_cache")
    scores = attention_scores.contiguous()
    with torch.cuda.device(scores.device):
        _check(_c_evict_cache(scores.data_ptr(), nb, float(retain_ratio), int(num_sink_tokens), _stream(scores)))


def evict_workspace_bytes(num_seqs: int, num_heads: int, seq_len: int, max_blocks_per_seq: int,
                          total_pool_blocks: int) -> int:
    """Device workspace bytes an ``evict_tokens`` call of this shape needs
    (``memopt_evict_workspace_size``)."""
    need = _i64(0)
    _check(_c_evict_ws(num_seqs, num_heads, seq_len, max_blocks_per_seq, total_pool_blocks, ctypes.byref(need)))
    return need.value


def evict_tokens(attention_scores: torch.Tensor, block_tables: torch.Tensor, is_block_free: torch.Tensor,
                 retain_ratio: float, num_sink_tokens: int = 4, workspace: Optional[torch.Tensor] = None) -> None:
    """Sequence-centric Ada-KV eviction; mutates the pool, ``block_tables`` and ``is_block_free``.

    ``block_tables`` and ``is_block_free`` must be contiguous int32 CUDA
    tensors (the reference silently drops mutations of non-contiguous ones).
    ``workspace``: a contiguous uint8 tensor on the scores' device of at
    least ``evict_workspace_bytes`` bytes, any content (default: one from
    torch's caching allocator per call).
    """
    p = _pool_or_raise("evict_tokens")
    _require(0.0 < retain_ratio <= 1.0, "evict_tokens: retain_ratio must be in (0, 1]")
    _require(attention_scores.dim() == 3,
             "evict_tokens: attention_scores must be 3-D [num_seqs, num_heads, seq_len]")
    _require(attention_scores.dtype == torch.float32, "evict_tokens: attention_scores must be float32")
    _require(block_tables.dim() == 2, "evict_tokens: block_tables must be 2-D [num_seqs, max_blocks_per_seq]")
    _require(block_tables.dtype == torch.int32, "evict_tokens: block_tables must be int32")
    _require(is_block_free.dim() == 1, "evict_tokens: is_block_free must be 1-D [total_pool_blocks]")
    _require(is_block_free.dtype == torch.int32, "evict_tokens: is_block_free must be int32")
    N, H, L = attention_scores.shape
    _require(H == p["h"], "evict_tokens: attention_scores num_heads != pool.num_heads")
    _require(block_tables.shape[0] == N, "evict_tokens: block_tables batch size != num_seqs")
    _require(is_block_free.shape[0] <= p["nb"], "evict_tokens: is_block_free size > pool.num_blocks")
    for t, n in ((attention_scores, "attention_scores"), (block_tables, "block_tables"),
                 (is_block_free, "is_block_free")):
        _cuda(t, n, "evict_tokens")
        _require(t.device == attention_scores.device, f"evict_tokens: {n} on a different device")
    _require(block_tables.is_contiguous() and is_block_free.is_contiguous(),
             "evict_tokens: block_tables and is_block_free must be contiguous (they are mutated in place)")
    if N == 0 or L == 0:
        return
    scores = attention_scores.contiguous()
    M, nb = block_tables.shape[1], is_block_free.shape[0]
    need = evict_workspace_bytes(N, H, L, M, nb)
    with torch.cuda.device(scores.device):
        if workspace is None:
            # scratch from torch's caching allocator on the current stream (page
            # marks and long-row selection state; nothing is kept between calls)
            ws = torch.empty(need, dtype=torch.uint8, device=scores.device)
        else:
            _require(workspace.dtype == torch.uint8 and workspace.is_contiguous() and
                     workspace.device == scores.device and workspace.numel() >= need,
                     f"evict_tokens: workspace must be a contiguous uint8 tensor of >= {need} bytes on the "
                     "scores' device")
            ws = workspace
        _check(_c_evict_tokens(scores.data_ptr(), N, H, L, block_tables.data_ptr(), M,
                               is_block_free.data_ptr(), nb, float(retain_ratio),
                               int(num_sink_tokens), ws.data_ptr(), ws.numel(), _stream(scores)))


def free_evicted_blocks(is_block_free: torch.Tensor) -> List[int]:
    """Return every block with ``is_block_free == num_heads`` to the free list and reset its counter.

    The caller-side step documented at src/csrc/kv_cache.cu:1033-1036.
    Returns the freed block indices.
    """
    p = _pool_or_raise("free_evicted_blocks")
    idx = torch.nonzero(is_block_free == p["h"]).flatten()
    freed = [int(i) for i in idx.tolist()]
    for b in freed:
        free_block(b)
    if freed:
        is_block_free[idx] = 0
    return freed


# ---------------------------------------------------------------------------
# Quantization — src/csrc/quantization.cu:294-428
# ---------------------------------------------------------------------------

def quantize_kv_cache_int4(cache: torch.Tensor, group_size: int) -> List[torch.Tensor]:
    """[packed uint8 (last dim / 2), scales float32 [numel / 64]]."""
    _cuda(cache, "cache", "quantize_kv_cache_int4")
    _require(cache.is_contiguous(), "quantize_kv_cache_int4: cache must be contiguous")
    _require(cache.dtype == torch.float16, "quantize_kv_cache_int4: cache must be float16")
    _require(group_size == 64, f"quantize_kv_cache_int4: group_size must equal 64 (got {group_size})")
    _require(cache.dim() >= 1, "quantize_kv_cache_int4: cache must have at least one dimension")
    n = cache.numel()
    _require(n % group_size == 0,
             f"quantize_kv_cache_int4: total_elements ({n}) must be divisible by group_size ({group_size})")
    last = cache.shape[-1]
    _require(last % 2 == 0, f"quantize_kv_cache_int4: last dimension ({last}) must be even for INT4 packing")
    packed = torch.empty(cache.shape[:-1] + (last // 2,), dtype=torch.uint8, device=cache.device)
    scales = torch.empty((n // group_size,), dtype=torch.float32, device=cache.device)
    if n:
        with torch.cuda.device(cache.device):
            _check(_c_quant(cache.data_ptr(), n, last, group_size, packed.data_ptr(), scales.data_ptr(),
                            _stream(cache)))
    return [packed, scales]


def dequantize_kv_cache_int4(q_cache: torch.Tensor, scales: torch.Tensor, group_size: int) -> torch.Tensor:
    """fp16 tensor with the last dim doubled."""
    _cuda(q_cache, "q_cache", "dequantize_kv_cache_int4")
    _cuda(scales, "scales", "dequantize_kv_cache_int4")
    _require(q_cache.is_contiguous(), "dequantize_kv_cache_int4: q_cache must be contiguous")
    _require(scales.is_contiguous(), "dequantize_kv_cache_int4: scales must be contiguous")
    _require(q_cache.dtype == torch.uint8, "dequantize_kv_cache_int4: q_cache must be uint8")
    _require(scales.dtype == torch.float32, "dequantize_kv_cache_int4: scales must be float32")
    _require(group_size == 64, "dequantize_kv_cache_int4: group_size must equal 64")
    total = q_cache.numel() * 2
    _require(total % 64 == 0 and scales.numel() == total // 64,
             f"dequantize_kv_cache_int4: scales length ({scales.numel()}) != expected num_groups ({total // 64})")
    out = torch.empty(q_cache.shape[:-1] + (q_cache.shape[-1] * 2,), dtype=torch.float16, device=q_cache.device)
    if total:
        with torch.cuda.device(q_cache.device):
            _check(_c_dequant(q_cache.data_ptr(), q_cache.numel(), scales.data_ptr(), scales.numel(), group_size,
                              out.data_ptr(), _stream(q_cache)))
    return out


# ---------------------------------------------------------------------------
# Attention — src/csrc/attention.cu:371-521
# ---------------------------------------------------------------------------

def _int4_rows_layout(key_cache, key_scales, num_heads, head_dim):
    """Token-major INT4 codes [nb, bs, H, D/2] (quantize_kv_cache_int4 of an fp16
    pool) + f32/f16 scales [nb*bs*H*D/64]: (bs, nb, code strides, scale strides, scale dtype)."""
    G = head_dim // 64
    nb, bs, h, dh = key_cache.shape
    _require(h == num_heads and dh * 2 == head_dim, "dynamic_sparse_attention: INT4 cache shape mismatch")
    _require(key_cache.is_contiguous(), "key_cache must be contiguous")
    _require(key_scales.dtype in (torch.float16, torch.float32), "dynamic_sparse_attention: scales must be f16/f32")
    _require(key_scales.numel() == nb * bs * num_heads * G, "dynamic_sparse_attention: scales size mismatch")
    kv = (bs * h * dh, dh, h * dh)
    sc = (bs * h * G, G, h * G)
    return bs, nb, kv, sc, 1 if key_scales.dtype == torch.float16 else 0


def _int4_pages_base(key_cache, value_cache, num_heads, head_dim):
    """Base pointer and page count when the caches are the INT4 page buffer (or
    its K/V code views from get_pool_tensors), else None."""
    lay = int4_layout(head_dim)
    if _pool and _pool["fmt"] == KV_INT4 and _pool["d"] == head_dim and _pool["h"] == num_heads:
        base = _pool["pages"].data_ptr()
        if key_cache.data_ptr() in (base, base + lay["kcodes"]) and \
                value_cache.data_ptr() in (base, base + lay["vcodes"]):
            return base, _pool["nb"], _pool["pages"]
    if key_cache.dim() == 3 and key_cache.shape[1] == num_heads and key_cache.shape[2] == lay["block"]:
        _require(key_cache.is_contiguous(), "INT4 page buffer must be contiguous")
        _require(value_cache.data_ptr() == key_cache.data_ptr(),
                 "dynamic_sparse_attention: pass the INT4 page buffer as both key_cache and value_cache")
        return key_cache.data_ptr(), key_cache.shape[0], key_cache
    return None


def _attention_desc(query, key_cache, value_cache, block_tables, context_lens, max_seq_len, window_size,
                    num_sink_tokens, causal, key_scales, value_scales, kv_layout, out, alloc_workspace=True):
    """Validate like src/csrc/attention.cu:383-439 and fill an AttnDesc.

    Returns (desc, out, workspace, keepalive) or (None, out, None, ()) for empty shapes.
    """
    fn = "dynamic_sparse_attention"
    for t, n in ((query, "query"), (key_cache, "key_cache"), (value_cache, "value_cache"),
                 (block_tables, "block_tables"), (context_lens, "context_lens")):
        _require(isinstance(t, torch.Tensor) and t.is_cuda, f"{n} must be a CUDA tensor")
    for t, n in ((query, "query"), (block_tables, "block_tables"), (context_lens, "context_lens")):
        _require(t.is_contiguous(), f"{n} must be contiguous")
    _require(query.dim() == 4, "query must be 4-D [batch, q_len, num_heads, head_dim]")
    _require(block_tables.dim() == 2, "block_tables must be 2-D [batch, max_blocks_per_seq]")
    _require(context_lens.dim() == 1, "context_lens must be 1-D [batch]")
    _require(query.dtype == torch.float16, "query must be fp16")
    _require(block_tables.dtype == torch.int32, "block_tables must be int32")
    _require(context_lens.dtype == torch.int32, "context_lens must be int32")
    B, Lq, H, D = query.shape
    _require(block_tables.shape[0] == B, "block_tables batch dimension mismatch")
    _require(context_lens.shape[0] == B, "context_lens batch dimension mismatch")
    if out is None:
        out = torch.empty_like(query)
    _require(out.shape == query.shape and out.dtype == torch.float16 and out.is_contiguous() and out.is_cuda,
             f"{fn}: out must be a contiguous fp16 CUDA tensor shaped like query")
    keep = (query, key_cache, value_cache, block_tables, context_lens, key_scales, value_scales)
    fmt = KV_FP16
    sc = (0, 0, 0)
    sdt = 0
    kv = (0, 0, 0)
    base_k, base_v = key_cache.data_ptr(), value_cache.data_ptr()
    if key_cache.dtype == torch.uint8:
        _require(value_cache.dtype == torch.uint8, "value_cache must match key_cache (INT4 codes)")
        _require(D % 64 == 0, f"{fn}: INT4 caches need head_dim % 64 == 0")
        pages = _int4_pages_base(key_cache, value_cache, H, D) if kv_layout in (None, "pages") else None
        if pages is not None:
            fmt = KV_INT4
            base_k, nb, buf = pages
            base_v = base_k
            bs = 16
            keep = keep + (buf,)
        else:
            _require(kv_layout in (None, "token_major"), f"{fn}: not an INT4 page buffer")
            _require(key_cache.dim() == 4 and value_cache.shape == key_cache.shape and value_cache.is_contiguous(),
                     "key_cache must be 4-D [num_kv_blocks, block_size, num_heads, head_dim/2] (INT4 codes)")
            _require(key_scales is not None and value_scales is not None, f"{fn}: INT4 caches need key/value scales")
            for t, n in ((key_scales, "key_scales"), (value_scales, "value_scales")):
                _require(t.is_cuda and t.is_contiguous(), f"{n} must be a contiguous CUDA tensor")
            _require(key_scales.dtype == value_scales.dtype and key_scales.shape == value_scales.shape,
                     f"{fn}: key/value scales mismatch")
            fmt = KV_INT4_ROWS
            bs, nb, kv, sc, sdt = _int4_rows_layout(key_cache, key_scales, H, D)
    else:
        for t, n in ((key_cache, "key_cache"), (value_cache, "value_cache")):
            _require(t.is_contiguous(), f"{n} must be contiguous")
        _require(key_cache.dim() == 4, "key_cache must be 4-D [num_kv_blocks, block_size, num_heads, head_dim]")
        _require(value_cache.dim() == 4, "value_cache must be 4-D [num_kv_blocks, block_size, num_heads, head_dim]")
        _require(key_cache.dtype == torch.float16, "key_cache must be fp16")
        _require(value_cache.dtype == torch.float16, "value_cache must be fp16")
        nb, bs = key_cache.shape[0], key_cache.shape[1]
        _require(key_cache.shape[2] == H, f"key_cache num_heads {key_cache.shape[2]} != query num_heads {H}")
        _require(key_cache.shape[3] == D, f"key_cache head_dim {key_cache.shape[3]} != query head_dim {D}")
        _require(value_cache.shape[1] == bs, "value_cache block_size mismatch")
        _require(value_cache.shape[2] == H, "value_cache num_heads mismatch")
        _require(value_cache.shape[3] == D, "value_cache head_dim mismatch")
        kv = (bs * H * D, D, H * D)
    if B == 0 or Lq == 0 or H == 0 or D == 0:
        return None, out, None, ()
    d = AttnDesc()
    d.query, d.out = query.data_ptr(), out.data_ptr()
    d.batch, d.q_len, d.num_heads, d.head_dim = B, Lq, H, D
    d.kv_format = fmt
    d.key_cache, d.value_cache = base_k, base_v
    if fmt == KV_INT4_ROWS:
        d.key_scales, d.value_scales = key_scales.data_ptr(), value_scales.data_ptr()
    d.scale_dtype, d.block_size, d.num_kv_blocks = sdt, bs, nb
    d.kv_page_stride, d.kv_head_stride, d.kv_token_stride = kv
    d.sc_page_stride, d.sc_head_stride, d.sc_token_stride = sc
    d.block_tables, d.max_blocks_per_seq = block_tables.data_ptr(), block_tables.shape[1]
    d.context_lens = context_lens.data_ptr()
    d.max_seq_len, d.window_size = int(max_seq_len), int(window_size)
    d.num_sink_tokens, d.causal = int(num_sink_tokens), int(bool(causal))
    need = _i64()
    _check(_c_ws(ctypes.byref(d), ctypes.byref(need)))
    ws = None
    if need.value > 0 and alloc_workspace:
        # A decode workspace holds split-K arrival counters, which must start
        # from zero (later calls may reuse it without clearing); a
        # multi-query workspace may hold anything.
        alloc = torch.zeros if Lq == 1 else torch.empty
        ws = alloc(need.value, dtype=torch.uint8, device=query.device)
        d.workspace, d.workspace_bytes = ws.data_ptr(), need.value
    return d, out, ws, keep


def dynamic_sparse_attention(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                             block_tables: torch.Tensor, context_lens: torch.Tensor, max_seq_len: int,
                             window_size: int, *, num_sink_tokens: int = 0, causal: bool = False,
                             key_scales: Optional[torch.Tensor] = None, value_scales: Optional[torch.Tensor] = None,
                             kv_layout: Optional[str] = None) -> torch.Tensor:
    """Paged sparse attention; returns fp16 [batch, q_len, H, D].

    Reference semantics for fp16 caches with the default keywords:
    non-causal, keys [max(0, ctx-W), ctx), pages with block_tables < 0
    skipped, W <= 0 or W > max_seq_len -> max_seq_len, scale 1/sqrt(D),
    no visible key -> 0. uint8 caches are INT4: either the INT4 page pool
    (its code views from ``get_pool_tensors()``, or a page buffer
    [nb, H, 16*D + 64*D/64] passed as both caches; scales live in the
    pages), or token-major codes [nb, bs, H, D/2] from
    ``quantize_kv_cache_int4`` of an fp16 pool together with their
    ``key_scales`` / ``value_scales`` (``kv_layout="token_major"``).
    """
    _require(isinstance(query, torch.Tensor) and query.is_cuda, "query must be a CUDA tensor")
    with torch.cuda.device(query.device):
        d, out, ws, _keep = _attention_desc(query, key_cache, value_cache, block_tables, context_lens,
                                            max_seq_len, window_size, num_sink_tokens, causal, key_scales,
                                            value_scales, kv_layout, None)
        if d is not None:
            _check(_c_attn(ctypes.byref(d), _stream(query)))
    return out


class PreparedAttention:
    """A validated ``dynamic_sparse_attention`` call bound to fixed tensors.

    Construction does the argument checks and workspace allocation once;
    each call launches on the current stream with a single C-ABI call and
    returns ``out`` (overwritten in place). Intended for decode loops where
    only the tensor *contents* change between steps.

    ``no_alloc=True`` allocates no workspace and launches through
    ``memopt_paged_attention_noalloc``, whose split-K partials live in a
    static per-GPU scratch array; no call allocates device memory, which suits
    capture into a HIP graph. Calls sharing that array must not overlap on
    one GPU.
    """

    def __init__(self, query, key_cache, value_cache, block_tables, context_lens, max_seq_len, window_size, *,
                 num_sink_tokens=0, causal=False, key_scales=None, value_scales=None, kv_layout=None, out=None,
                 no_alloc=False):
        _require(isinstance(query, torch.Tensor) and query.is_cuda, "query must be a CUDA tensor")
        self.device = query.device
        with torch.cuda.device(self.device):
            self._d, self.out, self._ws, self._keep = _attention_desc(
                query, key_cache, value_cache, block_tables, context_lens, max_seq_len, window_size,
                num_sink_tokens, causal, key_scales, value_scales, kv_layout, out, alloc_workspace=not no_alloc)
        self._dp = ctypes.byref(self._d) if self._d is not None else None
        self._fn = _c_attn_noalloc if no_alloc else _c_attn

    @property
    def workspace_bytes(self) -> int:
        """Device workspace held for the call (split-K partials or staged K/V)."""
        return 0 if self._ws is None else self._ws.numel() * self._ws.element_size()

    def __call__(self, stream: Optional[int] = None) -> torch.Tensor:
        if self._dp is not None:
            s = stream if stream is not None else torch.cuda.current_stream(self.device).cuda_stream
            _check(self._fn(self._dp, s))
        return self.out
