"""GPU parity of evict_tokens / evict_cache against the oracle (intended
semantics; the reference's literal defects are documented in the oracle)."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import dev, memopt_C, same_bits, to_dev

pytestmark = pytest.mark.gpu


def _pool_state(fmt):
    if fmt == "fp16":
        k, v = memopt_C.get_pool_tensors()
        return {"format": fmt, "k": k.cpu().numpy(), "v": v.cpu().numpy()}
    pages = memopt_C.get_int4_pages()
    return {"format": fmt, "pages": pages.cpu().numpy(), "D": pages.shape[2] // 17}


@pytest.mark.parametrize("fmt", ["fp16", "int4"])
@pytest.mark.parametrize("N,H,L,bs,r,sinks", [
    (2, 4, 100, 16, 0.5, 4), (3, 2, 64, 16, 0.75, 0), (1, 8, 4096, 16, 0.75, 4),
    (2, 2, 8192, 16, 0.3, 4), (2, 3, 50, 8, 0.1, 2), (1, 2, 40, 16, 1.0, 4),
    # 1024-thread kernels: keys in registers (L <= 32768), then streamed rows
    # read as float4 (L % 4 == 0) and token by token (L % 4 != 0)
    (1, 2, 20000, 16, 0.75, 4), (1, 2, 40000, 16, 0.6, 4), (1, 1, 40001, 16, 0.5, 3)])
def test_evict_tokens_vs_oracle(fmt, N, H, L, bs, r, sinks):
    if fmt == "int4" and bs != 16:
        pytest.skip("the INT4 page pool uses 16-token pages")
    rng = np.random.default_rng(L + N)
    D = 64
    M = (L + bs - 1) // bs
    nb = N * M + 3
    memopt_C.init_pool(nb, bs, H, D, kv_format=fmt)
    T = nb * bs
    k = rng.standard_normal((T, H, D)).astype(np.float16)
    v = rng.standard_normal((T, H, D)).astype(np.float16)
    memopt_C.write_cache(to_dev(k), to_dev(v), to_dev(np.zeros((1, 1), np.int32)),
                         to_dev(np.arange(T, dtype=np.int32)))
    scores = rng.lognormal(size=(N, H, L)).astype(np.float32)
    scores[0, :, 16:32] = 1e-6  # one logical block evicted in every head -> unlinked
    scores[:, 0, 1] = scores[:, 0, 2]  # ties
    bt = rng.permutation(nb)[:N * M].reshape(N, M).astype(np.int32)
    ibf = np.zeros(nb, np.int32)
    before = _pool_state(fmt)
    bt_d, ibf_d = to_dev(bt), to_dev(ibf)
    memopt_C.evict_tokens(to_dev(scores), bt_d, ibf_d, r, sinks)
    O.evict_tokens_intended(scores, bt, ibf, r, sinks, before, bs)
    after = _pool_state(fmt)
    for key in before:
        if isinstance(before[key], np.ndarray):
            same_bits(after[key], before[key])
    same_bits(bt_d, bt)
    same_bits(ibf_d, ibf)


@pytest.mark.parametrize("L", [40000, 40001])
def test_evict_tokens_streamed_rows_many_ties(L):
    """Streamed rows whose threshold bin holds far more keys than the LDS
    candidate buffer (scores take 4 values): the last radix pass streams the
    row again instead of reading the candidates."""
    rng = np.random.default_rng(L)
    N, H, bs, D, r, sinks = 1, 2, 16, 64, 0.6, 4
    M = (L + bs - 1) // bs
    nb = N * M + 1
    memopt_C.init_pool(nb, bs, H, D, kv_format="int4")
    T = nb * bs
    k = rng.standard_normal((T, H, D)).astype(np.float16)
    memopt_C.write_cache(to_dev(k), to_dev(k), to_dev(np.zeros((1, 1), np.int32)),
                         to_dev(np.arange(T, dtype=np.int32)))
    scores = rng.integers(1, 5, size=(N, H, L)).astype(np.float32)
    bt = rng.permutation(nb)[:N * M].reshape(N, M).astype(np.int32)
    ibf = np.zeros(nb, np.int32)
    before = _pool_state("int4")
    bt_d, ibf_d = to_dev(bt), to_dev(ibf)
    memopt_C.evict_tokens(to_dev(scores), bt_d, ibf_d, r, sinks)
    O.evict_tokens_intended(scores, bt, ibf, r, sinks, before, bs)
    after = _pool_state("int4")
    same_bits(after["pages"], before["pages"])
    same_bits(bt_d, bt)
    same_bits(ibf_d, ibf)


@pytest.mark.parametrize("D", [128, 192, 1088])
def test_evict_tokens_int4_head_dims(D):
    """INT4 zeroing over the scale-line path (G = D / 64 groups: 2 and 3
    give 8 and 5 blocks per wave step) and over the per-token fallback taken
    when G > 16 (D = 1088)."""
    rng = np.random.default_rng(D)
    N, H, L, bs, r, sinks = 2, 3, 300, 16, 0.6, 4
    M = (L + bs - 1) // bs
    nb = N * M + 2
    memopt_C.init_pool(nb, bs, H, D, kv_format="int4")
    T = nb * bs
    k = rng.standard_normal((T, H, D)).astype(np.float16)
    v = rng.standard_normal((T, H, D)).astype(np.float16)
    memopt_C.write_cache(to_dev(k), to_dev(v), to_dev(np.zeros((1, 1), np.int32)),
                         to_dev(np.arange(T, dtype=np.int32)))
    scores = rng.lognormal(size=(N, H, L)).astype(np.float32)
    scores[1, :, 32:48] = 1e-6  # one logical block evicted in every head -> unlinked
    bt = rng.permutation(nb)[:N * M].reshape(N, M).astype(np.int32)
    ibf = np.zeros(nb, np.int32)
    before = _pool_state("int4")
    bt_d, ibf_d = to_dev(bt), to_dev(ibf)
    memopt_C.evict_tokens(to_dev(scores), bt_d, ibf_d, r, sinks)
    O.evict_tokens_intended(scores, bt, ibf, r, sinks, before, bs)
    after = _pool_state("int4")
    for key in before:
        if isinstance(before[key], np.ndarray):
            same_bits(after[key], before[key])
    same_bits(bt_d, bt)
    same_bits(ibf_d, ibf)


def test_evict_then_free_sweep():
    memopt_C.init_pool(8, 16, 2, 64)
    bt = torch.tensor([[memopt_C.allocate_block() for _ in range(4)]], dtype=torch.int32, device=dev())
    scores = torch.ones(1, 2, 64, device=dev())
    scores[:, :, 16:32] = 0.0
    ibf = torch.zeros(8, dtype=torch.int32, device=dev())
    memopt_C.evict_tokens(scores, bt, ibf, 0.75, 4)
    assert bt.tolist() == [[0, -1, 2, 3]]
    assert memopt_C.free_evicted_blocks(ibf) == [1] and memopt_C.free_blocks_count() == 5


@pytest.mark.parametrize("fmt", ["fp16", "int4"])
def test_evict_cache_vs_oracle(fmt):
    rng = np.random.default_rng(5)
    nb, bs, H, D = 6, 16, 4, 64
    memopt_C.init_pool(nb, bs, H, D, kv_format=fmt)
    T = nb * bs
    k = rng.standard_normal((T, H, D)).astype(np.float16)
    memopt_C.write_cache(to_dev(k), to_dev(k), to_dev(np.zeros((1, 1), np.int32)),
                         to_dev(np.arange(T, dtype=np.int32)))
    scores = rng.standard_normal((nb, bs, H)).astype(np.float32)
    memopt_C.evict_cache(to_dev(np.zeros((1, 1), np.int32)), to_dev(scores), 0.4)
    if fmt == "fp16":
        kp = k.reshape(nb, bs, H, D).copy()
        vp = kp.copy()
        O.evict_cache(kp, vp, scores, 0.4)
        same_bits(memopt_C.get_key_pool(), kp)
    else:
        fp = k.reshape(nb, bs, H, D).copy()
        O.evict_cache(fp, fp.copy(), scores, 0.4)
        kd, vd = O.from_int4_pages(memopt_C.get_int4_pages().cpu().numpy(), D)
        zero = np.all(fp == 0, axis=-1)  # [nb, bs, H] evicted rows
        assert np.array_equal(np.all(kd == 0, axis=-1), zero) and np.array_equal(np.all(vd == 0, axis=-1), zero)


def test_evict_errors():
    memopt_C.init_pool(4, 16, 2, 64)
    s = torch.ones(1, 2, 64, device=dev())
    bt = torch.zeros(1, 4, dtype=torch.int32, device=dev())
    ibf = torch.zeros(4, dtype=torch.int32, device=dev())
    with pytest.raises(RuntimeError, match="retain_ratio"):
        memopt_C.evict_tokens(s, bt, ibf, 0.0)
    with pytest.raises(RuntimeError, match="num_heads"):
        memopt_C.evict_tokens(torch.ones(1, 3, 64, device=dev()), bt, ibf, 0.5)
    non_contig = torch.zeros(2, 8, dtype=torch.int32, device=dev())[:, ::2]
    assert not non_contig.is_contiguous()
    with pytest.raises(RuntimeError, match="contiguous"):
        memopt_C.evict_tokens(torch.ones(2, 2, 64, device=dev()), non_contig, ibf, 0.5)
