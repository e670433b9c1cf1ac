"""GPU parity of the fused INT4 paged decode kernel (q_len == 1, 16-token pages)
against the composition oracle dequantize -> attention
up to the full config 2 / 3 shapes."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import assert_close, dequant_pages_dev, dev, memopt_C, reference_decode_dev, to_dev

pytestmark = pytest.mark.gpu


def _decode_pages(q, pages, bt, cl, msl, W, sinks=0):
    pg = to_dev(pages)
    return memopt_C.dynamic_sparse_attention(to_dev(q), pg, pg, to_dev(bt), to_dev(cl), msl, W,
                                             num_sink_tokens=sinks)


def _decode_rows(q, kc, ks, vc, vs, bt, cl, msl, W, sinks=0):
    return memopt_C.dynamic_sparse_attention(to_dev(q), to_dev(kc), to_dev(vc), to_dev(bt), to_dev(cl), msl, W,
                                             num_sink_tokens=sinks, key_scales=to_dev(ks), value_scales=to_dev(vs),
                                             kv_layout="token_major")


def test_config1_decode():
    """[64, 16, 8, 64] K/V N(0,1) 1% x8 seed 0, batch 1,
    random page permutation, 1024 tokens, retain 1.0, 4 sinks."""
    g = torch.Generator().manual_seed(0)
    k = O.outlier_normal(g, (64, 16, 8, 64), 0.01, 8.0)
    v = O.outlier_normal(g, (64, 16, 8, 64), 0.01, 8.0)
    q = torch.randn((1, 1, 8, 64), generator=g).half().numpy()
    bt = torch.randperm(64, generator=g).to(torch.int32).numpy()[None]
    cl = np.array([1024], np.int32)
    # token-major surface INT4 (fp32 scales): exactly the reference's INT4 path
    kp, ks = O.quantize_int4(k)
    vp, vs = O.quantize_int4(v)
    want = O.paged_attention(q, O.dequantize_int4(kp, ks), O.dequantize_int4(vp, vs), bt, cl, 1024, 1024,
                             num_sink_tokens=4)
    got = _decode_rows(q, kp, ks, vp, vs, bt, cl, 1024, 1024, 4)
    assert_close(got, want, what="config1 token_major")
    # INT4 page pool (fp16 scales)
    pages = O.to_int4_pages(k, v)
    want_p = O.paged_attention_int4(q, pages, bt, cl, 1024, 1024, num_sink_tokens=4)
    assert_close(_decode_pages(q, pages, bt, cl, 1024, 1024, 4), want_p, what="config1 pages")


@pytest.mark.parametrize("B,H,D,ctx,W,sinks,unlink", [
    (1, 1, 128, [4096], 4096, 0, 0),      # long single sequence: many splits
    (2, 3, 64, [1000, 17], 200, 4, 2),    # ragged contexts, window, sinks, unlinked pages
    (4, 2, 128, [1, 15, 16, 33], 64, 0, 0),
    (2, 2, 128, [4100, 2050], 1024, 4, 5),
    (1, 4, 128, [300], 8, 20, 0),          # sinks larger than the window
])
def test_decode_vs_oracle(B, H, D, ctx, W, sinks, unlink):
    rng = np.random.default_rng(B * 7 + D)
    bs = 16
    M = (max(ctx) + bs - 1) // bs
    nb = B * M + 5
    kp = (rng.standard_normal((nb, bs, H, D)) * np.where(rng.random((nb, bs, H, D)) < 0.005, 10, 1)).astype(np.float16)
    vp = rng.standard_normal((nb, bs, H, D)).astype(np.float16)
    q = rng.standard_normal((B, 1, H, D)).astype(np.float16)
    bt = rng.permutation(nb)[:B * M].reshape(B, M).astype(np.int32)
    for i in range(unlink):
        bt[0, rng.integers(0, M)] = -1
    cl = np.array(ctx, np.int32)
    pages = O.to_int4_pages(kp, vp)
    want = O.paged_attention_int4(q, pages, bt, cl, 1 << 20, W, num_sink_tokens=sinks)
    got = _decode_pages(q, pages, bt, cl, 1 << 20, W, sinks)
    assert_close(got, want, what="pages")
    assert torch.equal(got, _decode_pages(q, pages, bt, cl, 1 << 20, W, sinks))  # deterministic
    # same inputs through the token-major (reference byte order, fp32 scales) kernel
    kc, ks = O.quantize_int4(kp)
    vc, vs = O.quantize_int4(vp)
    want_r = O.paged_attention(q, O.dequantize_int4(kc, ks), O.dequantize_int4(vc, vs), bt, cl, 1 << 20, W,
                               num_sink_tokens=sinks)
    assert_close(_decode_rows(q, kc, ks, vc, vs, bt, cl, 1 << 20, W, sinks), want_r, what="token_major")


# ---------------------------------------------------------------------------
# Full-size configs: reference computed on the GPU in fp32 from the INT4 pages
# dequantized by the (separately bit-exact) surface dequantize kernel.
# ---------------------------------------------------------------------------

def _fill_int4_pool(B, H, D, ctx, frac, mult, seed):
    nbps = ctx // 16
    nb = B * nbps
    memopt_C.init_pool(nb, 16, H, D, kv_format="int4")
    g = torch.Generator(device=dev()).manual_seed(seed)
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed)).to(torch.int32)
    bt = perm.reshape(B, nbps).to(dev())
    slots = (bt.long()[:, :, None] * 16 + torch.arange(16, device=dev())).reshape(-1).to(torch.int32)
    chunk = max(1, B // 4)  # write K/V a few sequences at a time to bound memory
    for b0 in range(0, B, chunk):
        n = chunk * ctx
        k = torch.randn(n, H, D, device=dev(), generator=g)
        k = torch.where(torch.rand(n, H, D, device=dev(), generator=g) < frac, k * mult, k).half()
        v = torch.randn(n, H, D, device=dev(), generator=g)
        v = torch.where(torch.rand(n, H, D, device=dev(), generator=g) < frac, v * mult, v).half()
        memopt_C.write_cache(k, v, bt, slots[b0 * ctx:(b0 + chunk) * ctx].contiguous())
        del k, v
    q = torch.randn(B, 1, H, D, device=dev(), generator=g).half()
    return q, bt


def test_config2_full_size():
    """Config 2: B16 H32 D128 ctx 4096, INT4 pages, random permutation, retain 1.0."""
    B, H, D, ctx = 16, 32, 128, 4096
    q, bt = _fill_int4_pool(B, H, D, ctx, 0.005, 10.0, 0)
    cl = torch.full((B,), ctx, dtype=torch.int32, device=dev())
    kc, vc = memopt_C.get_pool_tensors()
    got = memopt_C.dynamic_sparse_attention(q, kc, vc, bt, cl, ctx, ctx)
    pages = memopt_C.get_int4_pages()
    want = reference_decode_dev(q, *dequant_pages_dev(pages, D), bt, cl, ctx, 0)
    assert_close(got, want, what="config2")
    # CPU oracle on two sequences (composition through numpy)
    for b in (0, 11):
        sub = pages[bt[b].long()].cpu().numpy()
        w = O.paged_attention_int4(q[b:b + 1].cpu().numpy(), sub, np.arange(sub.shape[0], dtype=np.int32)[None],
                                   np.array([ctx], np.int32), ctx, ctx)
        assert_close(got[b:b + 1], w, what=f"config2 oracle b={b}")


def test_config3_evict_then_sparse_decode():
    """Config 3: ctx 8192, evict_tokens(r=0.75, 4 sinks) on LogNormal scores,
    then decode over 4 sinks + a 2048-token window; evicted rows read as zeros."""
    B, H, D, ctx, W, sinks = 16, 32, 128, 8192, 2048, 4
    q, bt = _fill_int4_pool(B, H, D, ctx, 0.005, 10.0, 1)
    scores = torch.exp(torch.randn(B, H, ctx, generator=torch.Generator().manual_seed(3))).to(dev())
    ibf = torch.zeros(bt.numel(), dtype=torch.int32, device=dev())
    bt0 = bt.clone()
    memopt_C.evict_tokens(scores, bt, ibf, 0.75, sinks)
    # unlinked pages are exactly those with H votes
    assert torch.equal(bt == -1, (ibf[bt0.long()] == H))
    cl = torch.full((B,), ctx, dtype=torch.int32, device=dev())
    kc, vc = memopt_C.get_pool_tensors()
    got = memopt_C.dynamic_sparse_attention(q, kc, vc, bt, cl, ctx, W, num_sink_tokens=sinks)
    want = reference_decode_dev(q, *dequant_pages_dev(memopt_C.get_int4_pages(), D), bt, cl, W, sinks)
    assert_close(got, want, what="config3")


def test_config5_long_context_fragmented_pool():
    """Config 5: B4, ctx 131072 (8192 pages per sequence, 32768 in use) in a
    pool with spare pages, block tables from a seeded FIFO alloc/free trace;
    evict_tokens(r=0.75, 4 sinks) on LogNormal scores (no length cap), then
    decode over the full context with 4 sinks."""
    B, H, D, ctx, sinks = 4, 32, 128, 131072, 4
    nbps, spare = ctx // 16, 4096
    nb = B * nbps + spare
    memopt_C.init_pool(nb, 16, H, D, kv_format="int4")
    got = [memopt_C.allocate_block() for _ in range(nb)]
    assert got == list(range(nb)) and memopt_C.allocate_block() == -1
    for i in torch.randperm(nb, generator=torch.Generator().manual_seed(5)).tolist():
        memopt_C.free_block(got[i])
    pages = [memopt_C.allocate_block() for _ in range(B * nbps)]
    assert len(set(pages)) == B * nbps and memopt_C.free_blocks_count() == spare
    bt = torch.tensor(pages, dtype=torch.int32).reshape(B, nbps).to(dev())
    g = torch.Generator(device=dev()).manual_seed(5)
    for b in range(B):
        slots = (bt[b].long()[:, None] * 16 + torch.arange(16, device=dev())).reshape(-1).to(torch.int32)
        k = torch.randn(ctx, H, D, device=dev(), generator=g)
        k = torch.where(torch.rand(ctx, H, D, device=dev(), generator=g) < 0.01, k * 8, k).half()
        v = torch.randn(ctx, H, D, device=dev(), generator=g)
        v = torch.where(torch.rand(ctx, H, D, device=dev(), generator=g) < 0.01, v * 8, v).half()
        memopt_C.write_cache(k, v, bt, slots)
        del k, v
    q = torch.randn(B, 1, H, D, device=dev(), generator=g).half()
    scores = torch.exp(torch.randn(B, H, ctx, device=dev(), generator=g))
    ibf = torch.zeros(nb, dtype=torch.int32, device=dev())
    bt0 = bt.clone()
    memopt_C.evict_tokens(scores, bt, ibf, 0.75, sinks)
    assert torch.equal(bt == -1, ibf[bt0.long()] == H)
    # keep count per (seq, head): exactly ceil(0.75 * L) rows survive (LogNormal scores have no ties)
    kpool, vpool = dequant_pages_dev(memopt_C.get_int4_pages()[bt0[0].long()], D)
    zero_rows = (kpool.reshape(ctx, H, D) == 0).all(dim=-1)      # [ctx, H] of sequence 0
    assert torch.equal(zero_rows.sum(dim=0).cpu(), torch.full((H,), ctx - int(np.ceil(np.float32(0.75) * ctx))))
    assert not zero_rows[:sinks].any()
    del kpool, vpool, zero_rows
    cl = torch.full((B,), ctx, dtype=torch.int32, device=dev())
    kc, vc = memopt_C.get_pool_tensors()
    out = memopt_C.dynamic_sparse_attention(q, kc, vc, bt, cl, ctx, ctx, num_sink_tokens=sinks)
    for b in range(B):  # one sequence at a time to bound the reference's memory
        used = bt0[b].long()
        kp, vp = dequant_pages_dev(memopt_C.get_int4_pages()[used], D)
        local = torch.where(bt[b] >= 0, torch.arange(nbps, device=dev(), dtype=torch.int32), -1)[None]
        want = reference_decode_dev(q[b:b + 1], kp, vp, local, cl[b:b + 1], ctx, sinks)
        assert_close(out[b:b + 1], want, what=f"config5 b={b}")
        del kp, vp


def test_config1_slice_golden_fixture():
    """Committed fixture: INT4 pages written on device == frozen bytes, and the
    decode output over them matches the frozen oracle output."""
    import os
    f = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config1_slice.npz"))
    nb, bs, H, D = f["k"].shape
    memopt_C.init_pool(nb, bs, H, D, kv_format="int4")
    slots = np.arange(nb * bs, dtype=np.int32)
    rows = lambda a: to_dev(a.reshape(nb * bs, H, D))
    memopt_C.write_cache(rows(f["k"]), rows(f["v"]), to_dev(np.zeros((1, 1), np.int32)), to_dev(slots))
    got_pages = memopt_C.get_int4_pages().cpu().numpy()
    assert np.array_equal(got_pages, f["int4_pages"])
    kc, vc = memopt_C.get_pool_tensors()
    out = memopt_C.dynamic_sparse_attention(to_dev(f["q"]), kc, vc, to_dev(f["block_tables"]),
                                            to_dev(f["context_lens"]), 64, 24, num_sink_tokens=4)
    assert_close(out, f["out_pages_window24_sinks4"], what="config1 slice fixture")


def _split_case(seed):
    """4 (b, h) units over 2048 tokens: the decode splits each into 4."""
    rng = np.random.default_rng(seed)
    nb, H, D = 130, 4, 128
    k = rng.standard_normal((nb, 16, H, D)).astype(np.float16)
    v = rng.standard_normal((nb, 16, H, D)).astype(np.float16)
    q = rng.standard_normal((1, 1, H, D)).astype(np.float16)
    bt = rng.permutation(nb)[:128][None].astype(np.int32)
    return q, O.to_int4_pages(k, v), bt, np.array([2048], np.int32)


def test_split_decode_workspace_counters():
    """The split-K arrival counters live in the workspace as (call id << 8 |
    count). A call reusing a workspace finds only earlier calls' counters
    there and needs no clearing; a fresh workspace is zeroed by the shim, so
    memory that held a word equal to (next call's id << 8 | count) cannot
    stop the merge. That memory is planted here: every freed block of the
    workspace's size holds the next call's id with count 1 in every word,
    and the call after it must still match the oracle (before the shim
    zeroed decode workspaces, the merge never ran and the output kept
    whatever its memory held)."""
    q, pages, bt, cl = _split_case(21)
    want = O.paged_attention_int4(q, pages, bt, cl, 2048, 2048)
    pg, dq, dbt, dcl = to_dev(pages), to_dev(q), to_dev(bt), to_dev(cl)
    call = memopt_C.PreparedAttention(dq, pg, pg, dbt, dcl, 2048, 2048)
    nbytes = call.workspace_bytes
    assert nbytes > 0                                   # split-K: partials and counters
    for _ in range(3):                                  # one workspace, no clearing between calls
        assert_close(call().clone(), want, what="reused workspace")
    torch.cuda.synchronize()
    cnt = call._ws[nbytes - 8 * 4:].view(torch.int64).cpu()
    assert (cnt & 0xFF).tolist() == [4] * 4             # each (b, h): 4 splits arrived
    nxt = int(cnt[0]) >> 8
    assert (cnt >> 8).tolist() == [nxt] * 4
    nxt += 1                                            # the next decode launch's id
    poison = [torch.full((nbytes // 8,), (nxt << 8) | 1, dtype=torch.int64, device=dev()) for _ in range(32)]
    torch.cuda.synchronize()
    del poison
    got = memopt_C.dynamic_sparse_attention(dq, pg, pg, dbt, dcl, 2048, 2048)
    assert torch.isfinite(got).all()
    assert_close(got, want, what="fresh workspace over stale memory")
