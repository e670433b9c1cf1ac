"""GPU parity of the host runtime on top of memopt_C: INT4 page dequantize and
in-place pool format conversion (bit-exact against the oracle), the decode
append step (pool contents bit-exact, attention within tolerance), the
policy forward wrapper (MemoryScheduler policy -> format switch, eviction,
attention), and AutoChunk chunked prefill (same result as one-shot prefill
and the oracle)."""
import threading

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import assert_close, dev, memopt_C, same_bits, special_fp16, to_dev

pytestmark = pytest.mark.gpu


def _runtime():
    import memopt_runtime
    return memopt_runtime


def _rows(rng, T, H, D, outlier=0.01):
    x = rng.standard_normal((T, H, D)) * np.where(rng.random((T, H, D)) < outlier, 8, 1)
    return x.astype(np.float16)


@pytest.mark.parametrize("data", ["normal", "special"])
@pytest.mark.parametrize("D", [64, 128])
def test_dequantize_int4_pages_bit_exact(D, data):
    """special: NaN of both signs, +-inf, -0, subnormals and +-65504."""
    rng = np.random.default_rng(D)
    nb, H = 7, 3
    if data == "special":
        k = special_fp16((nb * 16, H, D), 1).reshape(nb, 16, H, D)
        v = special_fp16((nb * 16, H, D), 2).reshape(nb, 16, H, D)
    else:
        k = _rows(rng, nb * 16, H, D).reshape(nb, 16, H, D)
        v = _rows(rng, nb * 16, H, D).reshape(nb, 16, H, D)
    pages = O.to_int4_pages(k, v)
    memopt_C.init_pool(nb, 16, H, D, kv_format="int4")
    kd, vd = memopt_C.dequantize_int4_pages(to_dev(pages))
    wk, wv = O.from_int4_pages(pages, D)
    same_bits(kd, wk)
    same_bits(vd, wv)


@pytest.mark.parametrize("data", ["normal", "special"])
def test_convert_pool_round_trip_keeps_free_list(data):
    """special: rows holding NaN of both signs, +-inf, -0, subnormals and
    +-65504."""
    rng = np.random.default_rng(3)
    nb, H, D = 12, 2, 128
    memopt_C.init_pool(nb, 16, H, D, kv_format="fp16")
    taken = [memopt_C.allocate_block() for _ in range(5)]
    memopt_C.free_block(taken[1])
    before_free = memopt_C.free_blocks_count()
    if data == "special":
        k, v = special_fp16((nb * 16, H, D), 3), special_fp16((nb * 16, H, D), 4)
    else:
        k = _rows(rng, nb * 16, H, D)
        v = _rows(rng, nb * 16, H, D)
    slots = torch.arange(nb * 16, dtype=torch.int32, device=dev())
    memopt_C.write_cache(to_dev(k), to_dev(v), to_dev(np.zeros((1, 1), np.int32)), slots)
    kp, vp = (t.cpu().numpy() for t in memopt_C.get_pool_tensors())
    memopt_C.convert_pool("int4")
    assert memopt_C.pool_kv_format() == "int4"
    same_bits(memopt_C.get_int4_pages(), O.to_int4_pages(kp, vp))
    assert memopt_C.free_blocks_count() == before_free
    # the FIFO order survives: the next allocations continue where they were
    assert memopt_C.allocate_block() == 5
    memopt_C.convert_pool("fp16")
    wk, wv = O.from_int4_pages(O.to_int4_pages(kp, vp), D)
    same_bits(memopt_C.get_key_pool(), wk)
    same_bits(memopt_C.get_value_pool(), wv)
    assert memopt_C.allocate_block() == 6


@pytest.mark.parametrize("fmt", ["fp16", "int4"])
def test_decode_append_step(fmt):
    """Prefill three sequences of different lengths, then decode appends
    (one token per sequence per step); the pool holds every written row at
    its (page, position) and decode attention matches the oracle."""
    R = _runtime()
    rng = np.random.default_rng(11)
    H, D, nb = 4, 128, 64
    cache = R.PagedKVCache(nb, H, D, kv_format=fmt)
    seqs = [0, 1, 2]
    lens = [37, 16, 50]
    history = {s: ([], []) for s in seqs}
    for s, n in zip(seqs, lens):
        cache.add_sequence(s)
        k, v = _rows(rng, n, H, D), _rows(rng, n, H, D)
        cache.append([s], to_dev(k)[None], to_dev(v)[None])
        history[s][0].append(k)
        history[s][1].append(v)
    for _ in range(20):  # decode steps crossing page boundaries
        k, v = _rows(rng, 3, H, D), _rows(rng, 3, H, D)
        cache.append(seqs, to_dev(k), to_dev(v))
        for i, s in enumerate(seqs):
            history[s][0].append(k[i:i + 1])
            history[s][1].append(v[i:i + 1])
    assert [cache.length(s) for s in seqs] == [n + 20 for n in lens]
    # expected pool: every written row at its slot (INT4: the oracle's pages of that pool)
    kp = np.zeros((nb, 16, H, D), np.float16)
    vp = np.zeros((nb, 16, H, D), np.float16)
    for s in seqs:
        ks, vs = np.concatenate(history[s][0]), np.concatenate(history[s][1])
        slots = np.array(R.slots_for(cache.pages(s), 0, cache.length(s), 16))
        O.write_cache(kp, ks, slots)
        O.write_cache(vp, vs, slots)
    if fmt == "fp16":
        same_bits(memopt_C.get_key_pool(), kp)
        same_bits(memopt_C.get_value_pool(), vp)
        kd, vd = kp, vp
    else:
        pages = O.to_int4_pages(kp, vp)
        same_bits(memopt_C.get_int4_pages(), pages)
        kd, vd = O.from_int4_pages(pages, D)
    q = rng.standard_normal((3, 1, H, D)).astype(np.float16)
    bt, ctx, max_len = R.attention_inputs(cache, seqs)
    k_pool, v_pool = cache.key_value_pools()
    got = memopt_C.dynamic_sparse_attention(to_dev(q), k_pool, v_pool, bt, ctx, max_len, 40, num_sink_tokens=4)
    want = O.paged_attention(q, kd, vd, bt.cpu().numpy(), ctx.cpu().numpy(), max_len, 40, num_sink_tokens=4)
    assert_close(got, want, what=f"decode after appends ({fmt})")


class _Scheduler:
    """Stand-in with MemoryScheduler's policy fields and lock
    (src/memopt/scheduler.py:151-172)."""

    def __init__(self):
        self._lock = threading.Lock()
        self._retain_ratio = 1.0
        self._use_int4 = False

    @property
    def retain_ratio(self):
        with self._lock:
            return self._retain_ratio

    @property
    def use_int4(self):
        with self._lock:
            return self._use_int4

    def pressure(self, on):
        with self._lock:
            self._retain_ratio, self._use_int4 = (0.5, True) if on else (1.0, False)


def test_policy_forward_switches_format_and_evicts():
    R = _runtime()
    rng = np.random.default_rng(5)
    H, D, nb, W, sinks = 2, 128, 40, 64, 4
    cache = R.PagedKVCache(nb, H, D, kv_format="fp16")
    sched = _Scheduler()
    fwd = R.PolicyForward(cache, sched, window_size=W, num_sink_tokens=sinks)
    seqs = [0, 1]
    for s in seqs:
        cache.add_sequence(s)
    # 1. no pressure: prefill 96 tokens each into the fp16 pool, causal attention
    q, k, v = (rng.standard_normal((2, 96, H, D)).astype(np.float16) for _ in range(3))
    out = fwd.step(seqs, to_dev(q), to_dev(k), to_dev(v))
    assert cache.kv_format == "fp16" and fwd.conversions == 0
    kp, vp = (t.cpu().numpy() for t in cache.key_value_pools())
    bt, ctx, max_len = R.attention_inputs(cache, seqs)
    want = O.paged_attention(q, kp, vp, bt.cpu().numpy(), ctx.cpu().numpy(), max_len, W, sinks, causal=True)
    assert_close(out, want, what="prefill step")
    # 2. pressure: convert to INT4, append one decode token, attend, evict half
    sched.pressure(True)
    qd, kd, vd = (rng.standard_normal((2, 1, H, D)).astype(np.float16) for _ in range(3))
    scores = rng.lognormal(size=(2, H, 97)).astype(np.float32)
    scores[:, :, 16:32] = 1e-6  # logical block 1 evicted in every head of both sequences -> freed
    free0 = memopt_C.free_blocks_count()
    out = fwd.step(seqs, to_dev(qd), to_dev(kd), to_dev(vd), scores=to_dev(scores))
    assert cache.kv_format == "int4" and fwd.conversions == 1 and fwd.last_policy == R.Policy(0.5, True)
    # pool before eviction = quantized (converted pool + the appended rows)
    for i, s in enumerate(seqs):
        slot = R.slots_for(cache.pages(s), 96, 1, 16)
        O.write_cache(kp, kd[i], np.array(slot))
        O.write_cache(vp, vd[i], np.array(slot))
    pages = O.to_int4_pages(kp, vp)
    kq, vq = O.from_int4_pages(pages, D)
    bt_pre = bt.cpu().numpy()
    bt_pre = np.concatenate([bt_pre, np.array([[cache.pages(s)[6]] for s in seqs], np.int32)], axis=1)
    want = O.paged_attention(qd, kq, vq, bt_pre, np.array([97, 97], np.int32), 97, W, sinks)
    assert_close(out, want, what="decode step on the converted pool")
    ibf = np.zeros(nb, np.int32)
    bt_oracle = bt_pre.copy()
    state = {"format": "int4", "pages": pages, "D": D}
    O.evict_tokens_intended(scores, bt_oracle, ibf, 0.5, sinks, state, 16)
    same_bits(memopt_C.get_int4_pages(), state["pages"])
    same_bits(cache.block_tables(seqs), bt_oracle)
    freed = int((ibf == H).sum())
    assert freed == 2 and fwd.evicted_pages == freed and memopt_C.free_blocks_count() == free0 - 2 + freed
    # 3. relief: back to fp16 (pages dequantized in place), attention over the evicted cache
    sched.pressure(False)
    qe, ke, ve = (rng.standard_normal((2, 1, H, D)).astype(np.float16) for _ in range(3))
    out2 = fwd.step(seqs, to_dev(qe), to_dev(ke), to_dev(ve))
    assert cache.kv_format == "fp16" and fwd.conversions == 2
    kp2, vp2 = (t.cpu().numpy() for t in cache.key_value_pools())
    bt2, ctx2, max_len2 = R.attention_inputs(cache, seqs)
    want2 = O.paged_attention(qe, kp2, vp2, bt2.cpu().numpy(), ctx2.cpu().numpy(), max_len2, W, sinks)
    assert_close(out2, want2, what="step after relief")
    k_rest, v_rest = O.from_int4_pages(state["pages"], D)
    live = [p for s in seqs for p in cache.pages(s)[:6] if p >= 0]
    same_bits(kp2[live], k_rest[live])
    same_bits(vp2[live], v_rest[live])


@pytest.mark.parametrize("fmt,chunk,window,sinks", [("int4", 128, 256, 4), ("int4", 1000, -1, 0),
                                                     ("fp16", 300, 500, 4), ("int4", None, 512, 4)])
def test_autochunk_matches_one_shot_prefill(fmt, chunk, window, sinks):
    R = _runtime()
    rng = np.random.default_rng(21)
    S, H, D = 2304, 4, 128
    nb = 2 * (S // 16) + 8
    q, k, v = (torch.randn(S, H, D, device=dev(), dtype=torch.float16) * 0.5 for _ in range(3))
    cache = R.PagedKVCache(nb, H, D, kv_format=fmt)
    cache.add_sequence(0)
    budget = None if chunk is not None else (1 << 20) * 6
    out = R.autochunk_prefill(cache, 0, q, k, v, window_size=window, num_sink_tokens=sinks, chunk_tokens=chunk,
                              budget_bytes=budget)
    # one-shot prefill of the same prompt into a second sequence of the same pool
    cache.add_sequence(1)
    cache.append([1], k[None], v[None])
    bt, ctx, _ = R.attention_inputs(cache, [1])
    kp, vp = cache.key_value_pools()
    ref = memopt_C.dynamic_sparse_attention(q[None], kp, vp, bt, ctx, S, window, num_sink_tokens=sinks,
                                            causal=True)[0]
    assert_close(out, ref, what="chunked vs one-shot")
    # oracle on sampled rows (dequantized pool for INT4)
    if fmt == "int4":
        kd, vd = O.from_int4_pages(memopt_C.get_int4_pages().cpu().numpy(), D)
    else:
        kd, vd = kp.cpu().numpy(), vp.cpu().numpy()
    rows = [0, 1, 127, 128, 999, 1000, 1500, S - 1]
    bt0, ctx0, _ = R.attention_inputs(cache, [0])
    want = O.paged_attention(q[None].cpu().numpy(), kd, vd, bt0.cpu().numpy(), ctx0.cpu().numpy(), S, window,
                             sinks, causal=True)[0]
    assert_close(out[rows], want[rows], what="chunked vs oracle")


def test_cache_exhaustion_and_free():
    R = _runtime()
    rng = np.random.default_rng(1)
    cache = R.PagedKVCache(4, 1, 64, kv_format="int4")
    cache.add_sequence(7)
    cache.append([7], to_dev(_rows(rng, 60, 1, 64))[None], to_dev(_rows(rng, 60, 1, 64))[None])
    assert memopt_C.free_blocks_count() == 0
    with pytest.raises(RuntimeError, match="exhausted"):
        cache.append([7], to_dev(_rows(rng, 5, 1, 64))[None], to_dev(_rows(rng, 5, 1, 64))[None])
    assert cache.length(7) == 60 and memopt_C.free_blocks_count() == 0
    cache.free_sequence(7)
    assert memopt_C.free_blocks_count() == 4


def test_chunk_call_workspace_is_bounded_by_the_window():
    """A chunk call over the end of a long context stages only the sink tiles
    and the tiles its queries' windows reach, so its workspace does not grow
    with the context (the property AutoChunk's budget relies on)."""
    R = _runtime()
    H, D, S, Lq, W, sinks = 8, 128, 16384, 256, 1024, 4
    cache = R.PagedKVCache(S // 16 + 4, H, D, kv_format="int4")
    cache.add_sequence(0)
    k = torch.randn(S, H, D, device=dev(), dtype=torch.float16)
    cache.append([0], k[None], k[None])
    bt, ctx, _ = R.attention_inputs(cache, [0])
    kp, vp = cache.key_value_pools()
    q = torch.randn(1, Lq, H, D, device=dev(), dtype=torch.float16)
    win = memopt_C.PreparedAttention(q, kp, vp, bt, ctx, S, W, num_sink_tokens=sinks, causal=True)
    full = memopt_C.PreparedAttention(q, kp, vp, bt, ctx, S, -1, num_sink_tokens=sinks, causal=True)
    slots = 4 * ((Lq + W - 1 + 63) // 64 + 1) + 4  # window tiles + alignment + one sink tile
    assert win.workspace_bytes == (slots * H * 64 * D + slots * 4 + 7) // 8 * 8 + H * 256
    assert full.workspace_bytes == ((S // 16) * H * 64 * D + (S // 16) * 4 + 7) // 8 * 8 + H * 256
    chunk_bytes = R.chunk_call_bytes(Lq, S, H, D, W)
    assert win.workspace_bytes <= chunk_bytes
    # and the call is right: same rows as the whole-window reference on the dequantized pool
    out = win()
    kd, vd = O.from_int4_pages(memopt_C.get_int4_pages().cpu().numpy(), D)
    want = O.paged_attention(q.cpu().numpy(), kd, vd, bt.cpu().numpy(), ctx.cpu().numpy(), S, W, sinks,
                             causal=True)
    assert_close(out, want, what="chunk call at the end of a long context")


def test_config5_through_policy_forward():
    """BASELINE configs[4] at full size through the policy path: 4 x 131072
    tokens in an fp16 pool drawn from a fragmented FIFO free list; a
    ThresholdPolicy with MemoryScheduler's rule and a near-zero high mark
    flips to INT4 + retain 0.75; PolicyForward converts the pool, appends,
    decodes, and (second step) evicts. Checked: the policy and pool format,
    both steps' decode outputs against fp32 attention over the pool they
    read, exactly ceil(0.75 L) rows kept per (sequence, head) with the sinks
    kept, and a decode over the evicted pool."""
    from gpu_helpers import dequant_pages_dev, reference_decode_dev
    R = _runtime()
    B, H, D, L, sinks, spare = 4, 32, 128, 131072, 4, 4096
    nb = B * (L // 16) + spare
    cache = R.PagedKVCache(nb, H, D, 16, kv_format="fp16")
    got = [memopt_C.allocate_block() for _ in range(nb)]
    for i in torch.randperm(nb, generator=torch.Generator().manual_seed(5)).tolist():
        memopt_C.free_block(got[i])
    seqs = list(range(B))
    for s in seqs:
        cache.add_sequence(s)
    g = torch.Generator(device=dev()).manual_seed(5)

    def kv(T):
        out = []
        for _ in range(2):
            x = torch.randn(B, T, H, D, device=dev(), generator=g)
            m = torch.rand(B, T, H, D, device=dev(), generator=g) < 0.01
            out.append(torch.where(m, x * 8, x).half())
            del x, m
        return out

    for t0 in range(0, L - 2, 8192):
        k, v = kv(min(8192, L - 2 - t0))
        cache.append(seqs, k, v)
        del k, v
    assert cache.linked_pages(seqs) == B * (L // 16)
    policy = R.ThresholdPolicy(vram_high_threshold=1e-9, vram_low_threshold=0.0, drop_retain_ratio=0.75)
    assert policy.adjust_policy() and (policy.retain_ratio, policy.use_int4) == (0.75, True)
    pf = R.PolicyForward(cache, policy, window_size=-1, num_sink_tokens=sinks)

    def check_decode(out, b):
        pages = memopt_C.get_int4_pages()
        bt = cache.block_tables([b])
        used = torch.clamp(bt[0].long(), min=0)
        kp, vp = dequant_pages_dev(pages[used], D)
        local = torch.where(bt[0] >= 0, torch.arange(bt.shape[1], device=dev(), dtype=torch.int32), -1)[None]
        want = reference_decode_dev(q[b:b + 1], kp, vp, local, cache.context_lens([b]), cache.length(b), sinks)
        assert_close(out[b:b + 1], want, what=f"config5 policy b={b}")
        del kp, vp

    q = torch.randn(B, 1, H, D, device=dev(), generator=g).half()
    k1, v1 = kv(1)
    # 256 full pages sampled before the conversion (2.4e9 elements per pool,
    # converted in one page-writer launch): their INT4 pages must equal the
    # oracle's quantization of their fp16 rows, byte for byte
    pick = cache.block_tables(seqs)[:, :8000:125].reshape(-1).long()
    kf, vf = memopt_C.get_pool_tensors()
    k_s, v_s = kf[pick].cpu().numpy(), vf[pick].cpu().numpy()
    del kf, vf
    out1 = pf.step(seqs, q, k1, v1)                      # no scores: convert, append, decode
    assert pf.conversions == 1 and cache.kv_format == "int4" and pf.last_policy == R.Policy(0.75, True)
    assert np.array_equal(memopt_C.get_int4_pages()[pick].cpu().numpy(), O.to_int4_pages(k_s, v_s))
    del k_s, v_s
    check_decode(out1, 0)
    k2, v2 = kv(1)
    scores = torch.exp(torch.randn(B, H, L, device=dev(), generator=g))
    out2 = pf.step(seqs, q, k2, v2, scores)              # append, decode, evict
    assert all(cache.length(s) == L for s in seqs)
    # exactly ceil(0.75 L) rows per (sequence 0, head) survive; sinks survive
    bt0 = cache.block_tables([0])[0]
    kpool, _ = dequant_pages_dev(memopt_C.get_int4_pages()[torch.clamp(bt0.long(), min=0)], D)
    zero_rows = (kpool.reshape(-1, H, D)[:L] == 0).all(dim=-1)
    zero_rows |= (bt0 < 0).repeat_interleave(16)[:L, None]
    assert torch.equal(zero_rows.sum(dim=0).cpu(), torch.full((H,), L - int(np.ceil(np.float32(0.75) * L))))
    assert not zero_rows[:sinks].any()
    del kpool, zero_rows
    check_decode(pf.attend(seqs, q), 1)                  # decode over the evicted pool
    assert out2.shape == (B, 1, H, D) and torch.isfinite(out2).all()
