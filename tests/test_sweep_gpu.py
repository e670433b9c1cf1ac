"""Seeded sweeps of random shapes through the fused INT4 write, decode and
prefill paths against the CPU oracle. Each case draws its sizes from a fixed
seed (batch, heads, head_dim, ragged contexts, window, sinks, unlinked pages,
slot patterns), so the sweep is deterministic and covers combinations the
hand-written cases do not."""
import numpy as np
import pytest

import oracle as O
from gpu_helpers import assert_close, memopt_C, same_bits, to_dev

pytestmark = pytest.mark.gpu


def _kv(rng, shape):
    k = (rng.standard_normal(shape) * np.where(rng.random(shape) < 0.01, 8, 1)).astype(np.float16)
    v = rng.standard_normal(shape).astype(np.float16)
    return k, v


def _decode_case(seed):
    rng = np.random.default_rng(1000 + seed)
    B = int(rng.integers(1, 5))
    H = int(rng.integers(1, 5))
    D = int(rng.choice([64, 128]))
    ctx = rng.integers(1, 3000, size=B)
    W = int(rng.choice([int(rng.integers(1, 3000)), 1 << 20]))
    sinks = int(rng.integers(0, 24))
    return B, H, D, [int(c) for c in ctx], W, sinks, int(rng.integers(0, 4))


@pytest.mark.parametrize("seed", range(40))
def test_decode_sweep(seed):
    B, H, D, ctx, W, sinks, unlink = _decode_case(seed)
    rng = np.random.default_rng(seed)
    bs = 16
    M = (max(ctx) + bs - 1) // bs
    nb = B * M + 3
    kp, vp = _kv(rng, (nb, bs, H, D))
    q = rng.standard_normal((B, 1, H, D)).astype(np.float16)
    bt = rng.permutation(nb)[:B * M].reshape(B, M).astype(np.int32)
    for _ in range(unlink):
        bt[int(rng.integers(0, B)), int(rng.integers(0, M))] = -1
    cl = np.array(ctx, np.int32)
    pages = O.to_int4_pages(kp, vp)
    want = O.paged_attention_int4(q, pages, bt, cl, 1 << 20, W, num_sink_tokens=sinks)
    pg = to_dev(pages)
    got = memopt_C.dynamic_sparse_attention(to_dev(q), pg, pg, to_dev(bt), to_dev(cl), 1 << 20, W,
                                            num_sink_tokens=sinks)
    assert_close(got, want, what=f"decode seed {seed}: B{B} H{H} D{D} ctx{ctx} W{W} sinks{sinks}")


def _prefill_case(seed):
    rng = np.random.default_rng(2000 + seed)
    B = int(rng.integers(1, 3))
    H = int(rng.integers(1, 4))
    D = int(rng.choice([64, 128]))
    ctx = [int(c) for c in rng.integers(16, 1200, size=B)]
    Lq = int(rng.integers(16, min(ctx) + 1))
    causal = bool(rng.integers(0, 2))
    W = int(rng.choice([int(rng.integers(1, 1200)), 1 << 20]))
    sinks = int(rng.integers(0, 20))
    return B, H, D, ctx, Lq, causal, W, sinks, bool(rng.integers(0, 2))


@pytest.mark.parametrize("seed", range(32))
def test_prefill_sweep(seed):
    B, H, D, ctx, Lq, causal, W, sinks, unlink = _prefill_case(seed)
    rng = np.random.default_rng(seed + 50)
    bs = 16
    M = (max(ctx) + bs - 1) // bs
    nb = B * M + 3
    kp, vp = _kv(rng, (nb, bs, H, D))
    q = rng.standard_normal((B, Lq, H, D)).astype(np.float16)
    bt = rng.permutation(nb)[:B * M].reshape(B, M).astype(np.int32)
    if unlink:
        bt[0, int(rng.integers(0, M))] = -1
    cl = np.array(ctx, np.int32)
    pages = O.to_int4_pages(kp, vp)
    want = O.paged_attention_int4(q, pages, bt, cl, 1 << 20, W, num_sink_tokens=sinks, causal=causal)
    pg = to_dev(pages)
    got = memopt_C.dynamic_sparse_attention(to_dev(q), pg, pg, to_dev(bt), to_dev(cl), 1 << 20, W,
                                            num_sink_tokens=sinks, causal=causal)
    assert_close(got, want, what=f"prefill seed {seed}: B{B} H{H} D{D} ctx{ctx} Lq{Lq} causal{causal} W{W} "
                                 f"sinks{sinks}")


@pytest.mark.parametrize("seed", range(18))
def test_write_int4_sweep(seed):
    """Random token counts and slot patterns: whole aligned pages (the page
    path), shifted runs and scattered slots (the chunk path), mixed in one call."""
    rng = np.random.default_rng(3000 + seed)
    D = int(rng.choice([64, 128]))
    H = int(rng.integers(1, 5))
    nb, bs = int(rng.integers(4, 20)), 16
    T = int(rng.integers(1, nb * bs + 1))
    pattern = seed % 3
    if pattern == 0:  # contiguous from an aligned page
        start = 16 * int(rng.integers(0, max(1, nb - (T + 15) // 16 + 1)))
        slots = (start + np.arange(T)) % (nb * bs)
    elif pattern == 1:  # contiguous from an unaligned slot
        start = int(rng.integers(0, nb * bs))
        slots = (start + np.arange(T)) % (nb * bs)
    else:
        slots = rng.permutation(nb * bs)[:T]
    slots = slots.astype(np.int32)
    memopt_C.reset_pool()  # identical parameters would otherwise keep an earlier test's pages
    memopt_C.init_pool(nb, bs, H, D, kv_format="int4")
    k, v = _kv(rng, (T, H, D))
    memopt_C.write_cache(to_dev(k), to_dev(v), to_dev(np.zeros((1, 1), np.int32)), to_dev(slots))
    wk, wv = np.zeros((nb, bs, H, D), np.float16), np.zeros((nb, bs, H, D), np.float16)
    O.write_cache(wk, k, slots)
    O.write_cache(wv, v, slots)
    same_bits(memopt_C.get_int4_pages(), O.to_int4_pages(wk, wv))


@pytest.mark.parametrize("seed", range(16))
def test_decode_token_major_sweep(seed):
    """The same random decode shapes through the token-major INT4 layout (the
    reference's byte order and fp32 surface scales)."""
    B, H, D, ctx, W, sinks, unlink = _decode_case(100 + seed)
    rng = np.random.default_rng(seed + 7)
    bs = 16
    M = (max(ctx) + bs - 1) // bs
    nb = B * M + 3
    kp, vp = _kv(rng, (nb, bs, H, D))
    q = rng.standard_normal((B, 1, H, D)).astype(np.float16)
    bt = rng.permutation(nb)[:B * M].reshape(B, M).astype(np.int32)
    for _ in range(unlink):
        bt[int(rng.integers(0, B)), int(rng.integers(0, M))] = -1
    cl = np.array(ctx, np.int32)
    kc, ks = O.quantize_int4(kp)
    vc, vs = O.quantize_int4(vp)
    want = O.paged_attention(q, O.dequantize_int4(kc, ks), O.dequantize_int4(vc, vs), bt, cl, 1 << 20, W,
                             num_sink_tokens=sinks)
    got = memopt_C.dynamic_sparse_attention(to_dev(q), to_dev(kc), to_dev(vc), to_dev(bt), to_dev(cl), 1 << 20, W,
                                            num_sink_tokens=sinks, key_scales=to_dev(ks), value_scales=to_dev(vs),
                                            kv_layout="token_major")
    assert_close(got, want, what=f"token-major decode seed {seed}: B{B} H{H} D{D} ctx{ctx} W{W} sinks{sinks}")


@pytest.mark.parametrize("seed", range(16))
def test_prefill_fp16_pool_sweep(seed):
    """Random prefill shapes over fp16 pools (16- and 32-token pages)."""
    B, H, D, ctx, Lq, causal, W, sinks, unlink = _prefill_case(100 + seed)
    rng = np.random.default_rng(seed + 90)
    bs = 16 if seed % 2 == 0 else 32
    M = (max(ctx) + bs - 1) // bs
    nb = B * M + 3
    kp, vp = _kv(rng, (nb, bs, H, D))
    q = rng.standard_normal((B, Lq, H, D)).astype(np.float16)
    bt = rng.permutation(nb)[:B * M].reshape(B, M).astype(np.int32)
    if unlink:
        bt[0, int(rng.integers(0, M))] = -1
    cl = np.array(ctx, np.int32)
    want = O.paged_attention(q, kp, vp, bt, cl, 1 << 20, W, num_sink_tokens=sinks, causal=causal)
    got = memopt_C.dynamic_sparse_attention(to_dev(q), to_dev(kp), to_dev(vp), to_dev(bt), to_dev(cl), 1 << 20, W,
                                            num_sink_tokens=sinks, causal=causal)
    assert_close(got, want, what=f"fp16 prefill seed {seed}: B{B} H{H} D{D} bs{bs} ctx{ctx} Lq{Lq} causal{causal} "
                                 f"W{W} sinks{sinks}")


@pytest.mark.parametrize("seed", range(10))
def test_evict_tokens_sweep(seed):
    """Random (seq, head, length, retain ratio, sinks) through evict_tokens on
    both pool formats against the oracle's exact top-k eviction."""
    rng = np.random.default_rng(4000 + seed)
    fmt = "int4" if seed % 2 else "fp16"
    N, H = int(rng.integers(1, 4)), int(rng.integers(1, 5))
    L = int(rng.integers(1, 6000))
    r = float(rng.choice([0.1, 0.3, 0.5, 0.75, 0.9, 1.0]))
    sinks = int(rng.integers(0, 40))
    bs, D = 16, 64
    M = (L + bs - 1) // bs
    nb = N * M + 2
    memopt_C.reset_pool()
    memopt_C.init_pool(nb, bs, H, D, kv_format=fmt)
    k, v = _kv(rng, (nb * bs, H, D))
    memopt_C.write_cache(to_dev(k), to_dev(v), to_dev(np.zeros((1, 1), np.int32)),
                         to_dev(np.arange(nb * bs, dtype=np.int32)))
    scores = rng.lognormal(size=(N, H, L)).astype(np.float32)
    if L > 32:
        scores[0, :, 16:32] = 1e-6  # a logical block evicted in every head
    bt = rng.permutation(nb)[:N * M].reshape(N, M).astype(np.int32)
    ibf = np.zeros(nb, np.int32)
    if fmt == "fp16":
        kk, vv = memopt_C.get_pool_tensors()
        before = {"format": fmt, "k": kk.cpu().numpy(), "v": vv.cpu().numpy()}
    else:
        pages = memopt_C.get_int4_pages()
        before = {"format": fmt, "pages": pages.cpu().numpy(), "D": D}
    bt_d, ibf_d = to_dev(bt), to_dev(ibf)
    memopt_C.evict_tokens(to_dev(scores), bt_d, ibf_d, r, sinks)
    O.evict_tokens_intended(scores, bt, ibf, r, sinks, before, bs)
    if fmt == "fp16":
        kk, vv = memopt_C.get_pool_tensors()
        same_bits(kk, before["k"])
        same_bits(vv, before["v"])
    else:
        same_bits(memopt_C.get_int4_pages(), before["pages"])
    same_bits(bt_d, bt)
    same_bits(ibf_d, ibf)


@pytest.mark.parametrize("seed", range(6))
def test_evict_tokens_long_rows_sweep(seed):
    """Long rows (L > 32768: classify, resolve, apply) with a different score
    distribution per seed (lognormal, normal, few distinct integers, two
    tight modes, ascending, normal with many +-0 and some NaN of both signs)
    and block tables that share pages between sequences, hold unlinked
    entries and entries past the pool, against the oracle bit for bit."""
    rng = np.random.default_rng(9500 + seed)
    fmt = "fp16" if seed % 3 == 2 else "int4"
    N, H = 2, int(rng.integers(1, 3))
    L = int(rng.integers(32769, 90000))
    r = float(rng.choice([0.05, 0.25, 0.5, 0.75, 0.95]))
    sinks = int(rng.integers(0, 100))
    bs, D = 16, 64
    M = (L + bs - 1) // bs
    nb = N * M + 2
    memopt_C.reset_pool()
    memopt_C.init_pool(nb, bs, H, D, kv_format=fmt)
    k, v = _kv(rng, (nb * bs, H, D))
    memopt_C.write_cache(to_dev(k), to_dev(v), to_dev(np.zeros((1, 1), np.int32)),
                         to_dev(np.arange(nb * bs, dtype=np.int32)))
    shape = (N, H, L)
    dist = seed % 6
    if dist == 0:
        s = rng.lognormal(size=shape)
    elif dist == 1:
        s = rng.standard_normal(shape)
    elif dist == 2:
        s = rng.integers(0, 50, size=shape).astype(np.float64)
    elif dist == 3:
        s = np.where(rng.random(shape) < 0.5, rng.normal(-5, 0.01, shape), rng.normal(5, 0.01, shape))
    elif dist == 4:
        s = np.broadcast_to(np.arange(L, dtype=np.float64) * 1e-3, shape).copy()
    else:
        s = rng.standard_normal(shape)
        s[rng.random(shape) < 0.2] = 0.0
        s[rng.random(shape) < 0.1] = -0.0
        s[rng.random(shape) < 0.001] = np.nan
        s[rng.random(shape) < 0.001] = -np.nan
    scores = s.astype(np.float32)
    scores[0, :, 32:48] = -1e30  # a logical block evicted in every head
    bt = rng.permutation(nb)[:N * M].reshape(N, M).astype(np.int32)
    idx = rng.choice(M, M // 30, replace=False)
    bt[1, idx] = bt[0, rng.permutation(idx)]  # pages shared by the two sequences
    bt[rng.random(bt.shape) < 0.01] = -1
    bt[rng.random(bt.shape) < 0.005] = nb + 5
    ibf = np.zeros(nb, np.int32)
    if fmt == "fp16":
        kk, vv = memopt_C.get_pool_tensors()
        before = {"format": fmt, "k": kk.cpu().numpy(), "v": vv.cpu().numpy()}
    else:
        before = {"format": fmt, "pages": memopt_C.get_int4_pages().cpu().numpy(), "D": D}
    bt_d, ibf_d = to_dev(bt), to_dev(ibf)
    memopt_C.evict_tokens(to_dev(scores), bt_d, ibf_d, r, sinks)
    O.evict_tokens_intended(scores, bt, ibf, r, sinks, before, bs)
    if fmt == "fp16":
        kk, vv = memopt_C.get_pool_tensors()
        same_bits(kk, before["k"])
        same_bits(vv, before["v"])
    else:
        same_bits(memopt_C.get_int4_pages(), before["pages"])
    same_bits(bt_d, bt)
    same_bits(ibf_d, ibf)


@pytest.mark.parametrize("seed", range(24))
def test_decode_fp16_pool_sweep(seed):
    """Random decode shapes over fp16 page pools (16-, 32- and 64-token
    pages; the reference's default cache format)."""
    B, H, D, ctx, W, sinks, unlink = _decode_case(200 + seed)
    rng = np.random.default_rng(seed + 11)
    bs = (16, 32, 64)[seed % 3]
    M = (max(ctx) + bs - 1) // bs
    nb = B * M + 3
    kp, vp = _kv(rng, (nb, bs, H, D))
    q = rng.standard_normal((B, 1, H, D)).astype(np.float16)
    bt = rng.permutation(nb)[:B * M].reshape(B, M).astype(np.int32)
    for _ in range(unlink):
        bt[int(rng.integers(0, B)), int(rng.integers(0, M))] = -1
    cl = np.array(ctx, np.int32)
    want = O.paged_attention(q, kp, vp, bt, cl, 1 << 20, W, num_sink_tokens=sinks)
    got = memopt_C.dynamic_sparse_attention(to_dev(q), to_dev(kp), to_dev(vp), to_dev(bt), to_dev(cl), 1 << 20, W,
                                            num_sink_tokens=sinks)
    assert_close(got, want, what=f"fp16 decode seed {seed}: B{B} H{H} D{D} bs{bs} ctx{ctx} W{W} sinks{sinks}")


@pytest.mark.parametrize("seed", range(16))
def test_small_q_len_sweep(seed):
    """2..15 queries per sequence (speculative or short-chunk steps) on INT4
    pages and fp16 pools, causal and not."""
    rng = np.random.default_rng(5000 + seed)
    B, H = int(rng.integers(1, 3)), int(rng.integers(1, 4))
    D = int(rng.choice([64, 128]))
    ctx = [int(c) for c in rng.integers(16, 1500, size=B)]
    Lq = int(rng.integers(2, 16))
    causal = bool(seed % 2)
    W = int(rng.choice([int(rng.integers(1, 1500)), 1 << 20]))
    sinks = int(rng.integers(0, 20))
    int4 = seed % 4 >= 2
    bs = 16
    M = (max(ctx) + bs - 1) // bs
    nb = B * M + 3
    kp, vp = _kv(rng, (nb, bs, H, D))
    q = rng.standard_normal((B, Lq, H, D)).astype(np.float16)
    bt = rng.permutation(nb)[:B * M].reshape(B, M).astype(np.int32)
    cl = np.array(ctx, np.int32)
    if int4:
        pages = O.to_int4_pages(kp, vp)
        want = O.paged_attention_int4(q, pages, bt, cl, 1 << 20, W, num_sink_tokens=sinks, causal=causal)
        pg = to_dev(pages)
        got = memopt_C.dynamic_sparse_attention(to_dev(q), pg, pg, to_dev(bt), to_dev(cl), 1 << 20, W,
                                                num_sink_tokens=sinks, causal=causal)
    else:
        want = O.paged_attention(q, kp, vp, bt, cl, 1 << 20, W, num_sink_tokens=sinks, causal=causal)
        got = memopt_C.dynamic_sparse_attention(to_dev(q), to_dev(kp), to_dev(vp), to_dev(bt), to_dev(cl), 1 << 20,
                                                W, num_sink_tokens=sinks, causal=causal)
    assert_close(got, want, what=f"small q_len seed {seed}: B{B} H{H} D{D} ctx{ctx} Lq{Lq} causal{causal} W{W} "
                                 f"sinks{sinks} int4{int4}")
