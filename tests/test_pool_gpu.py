"""GPU tests of the paged pool and write_cache (src/csrc/kv_cache.cu:112-348),
fp16 and INT4 page pools."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import dev, memopt_C, same_bits, special_fp16, to_dev

pytestmark = pytest.mark.gpu


def test_init_idempotent_and_aliasing():
    memopt_C.init_pool(8, 16, 4, 64)
    k1, v1 = memopt_C.get_pool_tensors()
    a = memopt_C.allocate_block()
    memopt_C.init_pool(8, 16, 4, 64)  # same params: no-op, free list untouched
    assert memopt_C.free_blocks_count() == 7
    k2, _ = memopt_C.get_pool_tensors()
    assert k1.data_ptr() == k2.data_ptr() and memopt_C.get_key_pool().data_ptr() == k1.data_ptr()
    assert memopt_C.get_value_pool().data_ptr() == v1.data_ptr()
    assert k1.shape == (8, 16, 4, 64) and k1.dtype == torch.float16 and bool((k1 == 0).all())
    memopt_C.free_block(a)
    memopt_C.init_pool(9, 16, 4, 64)  # different params: reset
    assert memopt_C.free_blocks_count() == 9


def test_allocate_fifo_and_exhaustion():
    memopt_C.init_pool(3, 16, 2, 64)
    assert [memopt_C.allocate_block() for _ in range(4)] == [0, 1, 2, -1]
    memopt_C.free_block(2)
    assert memopt_C.allocate_block() == 2
    with pytest.raises(RuntimeError, match="out of range"):
        memopt_C.free_block(7)


def _setup_slots(nb, bs, T, rng):
    pages = rng.permutation(nb)[: (T + bs - 1) // bs]
    slots = np.array([pages[t // bs] * bs + t % bs for t in range(T)], np.int32)
    return pages, slots


def test_write_cache_fp16_scatter():
    rng = np.random.default_rng(0)
    nb, bs, H, D, T = 12, 16, 4, 64, 70
    memopt_C.init_pool(nb, bs, H, D)
    k = rng.standard_normal((T, H, D)).astype(np.float16)
    v = rng.standard_normal((T, H, D)).astype(np.float16)
    _, slots = _setup_slots(nb, bs, T, rng)
    memopt_C.write_cache(to_dev(k), to_dev(v), to_dev(np.zeros((1, 1), np.int32)), to_dev(slots))
    kp, vp = memopt_C.get_pool_tensors()
    wk, wv = np.zeros((nb, bs, H, D), np.float16), np.zeros((nb, bs, H, D), np.float16)
    O.write_cache(wk, k, slots)
    O.write_cache(wv, v, slots)
    same_bits(kp, wk)
    same_bits(vp, wv)


@pytest.mark.parametrize("D", [64, 128])
def test_write_cache_int4_pages_bit_exact(D):
    rng = np.random.default_rng(1)
    nb, bs, H, T = 10, 16, 3, 100
    memopt_C.init_pool(nb, bs, H, D, kv_format="int4")
    k = (rng.standard_normal((T, H, D)) * np.where(rng.random((T, H, D)) < 0.01, 8, 1)).astype(np.float16)
    v = rng.standard_normal((T, H, D)).astype(np.float16)
    _, slots = _setup_slots(nb, bs, T, rng)
    memopt_C.write_cache(to_dev(k), to_dev(v), to_dev(np.zeros((1, 1), np.int32)), to_dev(slots))
    # Oracle: scatter fp16 rows into an fp16 pool, then convert to INT4 pages;
    # untouched rows of a fresh INT4 pool hold codes 8 / scale 1.0 == zeros.
    wk, wv = np.zeros((nb, bs, H, D), np.float16), np.zeros((nb, bs, H, D), np.float16)
    O.write_cache(wk, k, slots)
    O.write_cache(wv, v, slots)
    same_bits(memopt_C.get_int4_pages(), O.to_int4_pages(wk, wv))
    gk, gv = memopt_C.get_pool_tensors()
    assert gk.shape == (nb, H, 8 * D) and gv.shape == (nb, H, 8 * D)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("order", ["scrambled", "shifted"])
def test_write_cache_int4_scatter_orders_bit_exact(D, order):
    """Slots that do not form aligned 16-token pages (scrambled across the pool,
    or pages filled from position 1) take the chunk-scatter path; groups that
    do form a page take the page path; both must give the oracle's bytes."""
    rng = np.random.default_rng(2)
    nb, bs, H, T = 12, 16, 3, 130
    memopt_C.init_pool(nb, bs, H, D, kv_format="int4")
    k = (rng.standard_normal((T, H, D)) * np.where(rng.random((T, H, D)) < 0.01, 8, 1)).astype(np.float16)
    v = rng.standard_normal((T, H, D)).astype(np.float16)
    if order == "scrambled":
        slots = rng.permutation(nb * bs)[:T].astype(np.int32)
    else:
        slots = (np.arange(T) + 1).astype(np.int32)  # every group straddles two pages
    memopt_C.write_cache(to_dev(k), to_dev(v), to_dev(np.zeros((1, 1), np.int32)), to_dev(slots))
    wk, wv = np.zeros((nb, bs, H, D), np.float16), np.zeros((nb, bs, H, D), np.float16)
    O.write_cache(wk, k, slots)
    O.write_cache(wv, v, slots)
    same_bits(memopt_C.get_int4_pages(), O.to_int4_pages(wk, wv))


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("order", ["pages", "shifted"])
def test_write_cache_int4_special_values_bit_exact(D, order):
    """write_cache into INT4 pages of K and V holding NaN of both signs,
    +-inf, -0, subnormals and +-65504 (aligned pages take the page path,
    slots shifted by one the chunk scatter): the pool's bytes equal the
    oracle's."""
    nb, bs, H, T = 12, 16, 3, 160
    memopt_C.init_pool(nb, bs, H, D, kv_format="int4")
    k, v = special_fp16((T, H, D), 6), special_fp16((T, H, D), 7)
    slots = (np.arange(T) + (order == "shifted")).astype(np.int32)
    memopt_C.write_cache(to_dev(k), to_dev(v), to_dev(np.zeros((1, 1), np.int32)), to_dev(slots))
    wk, wv = np.zeros((nb, bs, H, D), np.float16), np.zeros((nb, bs, H, D), np.float16)
    O.write_cache(wk, k, slots)
    O.write_cache(wv, v, slots)
    same_bits(memopt_C.get_int4_pages(), O.to_int4_pages(wk, wv))


def test_write_cache_out_of_bounds_raises():
    memopt_C.init_pool(2, 16, 2, 64)
    k = torch.zeros(1, 2, 64, dtype=torch.float16, device=dev())
    with pytest.raises(RuntimeError, match="out of bounds"):
        memopt_C.write_cache(k, k, torch.zeros(1, 1, dtype=torch.int32, device=dev()),
                             torch.tensor([32], dtype=torch.int32, device=dev()))


def test_pool_not_initialized_raises():
    """tests/test_attention.py:252-290, independent of earlier pool state."""
    memopt_C.init_pool(4, 16, 8, 64)
    keys = torch.zeros(1, 8, 64, dtype=torch.float16, device=dev())
    try:
        memopt_C.init_pool(0, 16, 8, 64)
    except Exception:
        pass
    with pytest.raises(RuntimeError, match="pool not initialized|out of bounds|exhausted"):
        memopt_C.write_cache(keys, keys, torch.zeros(1, 1, dtype=torch.int32, device=dev()),
                             torch.zeros(1, dtype=torch.int32, device=dev()))


def test_free_evicted_blocks_sweep():
    memopt_C.init_pool(6, 16, 2, 64)
    got = [memopt_C.allocate_block() for _ in range(6)]
    assert memopt_C.free_blocks_count() == 0
    ibf = torch.tensor([0, 2, 1, 2, 0, 0], dtype=torch.int32, device=dev())
    assert memopt_C.free_evicted_blocks(ibf) == [1, 3]
    assert ibf.tolist() == [0, 0, 1, 0, 0, 0] and memopt_C.free_blocks_count() == 2
    assert got == list(range(6))
