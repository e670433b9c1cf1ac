"""GPU parity of the multi-query (prefill / chunked-prefill) MFMA attention
path: q_len >= 2 over fp16 pools and INT4 page pools, causal StreamingLLM
masks (window + sinks), non-causal multi-query windows, unlinked pages,
contexts shorter than the query block, against the CPU oracle; and the
BASELINE config-4 shape at full size against an fp32 reference: sampled
query rows of every head, and every row of four heads."""
import math

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import ATOL, RTOL, assert_close, dev, memopt_C, to_dev

pytestmark = pytest.mark.gpu


def _case_inputs(seed, B, H, D, bs, nb, ctx, Lq):
    rng = np.random.default_rng(seed)
    kp = (rng.standard_normal((nb, bs, H, D)) * np.where(rng.random((nb, bs, H, D)) < 0.01, 8, 1)).astype(np.float16)
    vp = rng.standard_normal((nb, bs, H, D)).astype(np.float16)
    q = rng.standard_normal((B, Lq, H, D)).astype(np.float16)
    M = max(1, (max(ctx) + bs - 1) // bs)
    bt = rng.permutation(nb)[:B * M].reshape(B, M).astype(np.int32)
    return q, kp, vp, bt, np.array(ctx, np.int32)


PREFILL_CASES = [
    # B, H, D, bs, ctx, Lq, max_seq_len, W, sinks, causal, unlink
    (1, 2, 64, 16, [300], 300, 512, 512, 0, True, False),      # full causal prefill
    (2, 3, 128, 16, [700, 260], 200, 1024, 128, 4, True, True),  # chunked prefill, window + sinks
    (2, 2, 64, 16, [500, 333], 64, 512, 100, 4, False, False),  # non-causal multi-query window + sinks
    (1, 2, 128, 32, [260], 260, 300, 70, 2, True, False),      # 32-token fp16 pages
    (2, 2, 64, 16, [100, 40], 130, 256, 256, 0, True, False),   # ctx < q_len: leading queries see nothing
    (1, 1, 128, 16, [1100], 1100, 2048, 1024, 4, True, False),  # window just under the sequence
    (1, 2, 64, 16, [257], 17, 512, 33, 5, True, True),          # ragged sizes, sinks not tile-aligned
    (1, 2, 128, 16, [640], 16, 640, 640, 0, False, False),      # smallest q_len on this path
    (1, 2, 128, 16, [1500], 700, 2048, 256, 150, True, False),  # 150 sinks: three sink tiles before the window
    (2, 2, 64, 16, [900, 650], 128, 1024, 200, 100, False, True),  # non-causal, two sink tiles
]


@pytest.mark.parametrize("case", PREFILL_CASES)
def test_prefill_fp16_vs_oracle(case):
    B, H, D, bs, ctx, Lq, msl, W, sinks, causal, unlink = case
    nb = B * ((max(ctx) + bs - 1) // bs) + 3
    q, kp, vp, bt, cl = _case_inputs(21, B, H, D, bs, nb, ctx, Lq)
    if unlink:
        bt[0, 1] = -1
    want = O.paged_attention(q, kp, vp, bt, cl, msl, W, num_sink_tokens=sinks, causal=causal)
    got = memopt_C.dynamic_sparse_attention(to_dev(q), to_dev(kp), to_dev(vp), to_dev(bt), to_dev(cl), msl, W,
                                            num_sink_tokens=sinks, causal=causal)
    assert_close(got, want, what=str(case))


@pytest.mark.parametrize("case", [c for c in PREFILL_CASES if c[3] == 16])
def test_prefill_int4_pages_vs_composition_oracle(case):
    B, H, D, bs, ctx, Lq, msl, W, sinks, causal, unlink = case
    nb = B * ((max(ctx) + bs - 1) // bs) + 3
    q, kp, vp, bt, cl = _case_inputs(22, B, H, D, bs, nb, ctx, Lq)
    if unlink:
        bt[0, 1] = -1
    pages = O.to_int4_pages(kp, vp)
    want = O.paged_attention_int4(q, pages, bt, cl, msl, W, num_sink_tokens=sinks, causal=causal)
    pg = to_dev(pages)
    got = memopt_C.dynamic_sparse_attention(to_dev(q), pg, pg, to_dev(bt), to_dev(cl), msl, W,
                                            num_sink_tokens=sinks, causal=causal)
    assert_close(got, want, what=str(case))


@pytest.mark.parametrize("D,int4", [(64, False), (128, False), (128, True)])
def test_prefill_running_max_raised_every_tile(D, int4):
    """Keys that grow along a common direction make every query's scores
    climb about 9.6 log2 units per 64 keys, so the lazy running max (raised
    only when a score passes it by more than 8 log2 units) rises in every
    tile and the rescale of the held output and row sums runs tile after
    tile; the first keys' weights fall to zero in fp16 along the way."""
    B, H, bs, ctx = 1, 2, 16, 640
    rng = np.random.default_rng(31)
    u = np.ones(D) / np.sqrt(D)
    t = np.arange(ctx)
    # q . k_t = 30 * 25 * t / ctx raw; 0.1275 log2 units per raw unit at D = 128
    k_rows = (25.0 * t / ctx)[:, None] * u[None, :] + 0.05 * rng.standard_normal((ctx, D))
    nb = ctx // bs + 2
    kp = np.zeros((nb, bs, H, D), np.float16)
    vp = rng.standard_normal((nb, bs, H, D)).astype(np.float16)
    bt = rng.permutation(nb)[:ctx // bs].reshape(1, -1).astype(np.int32)
    for j in range(ctx // bs):
        kp[bt[0, j]] = k_rows[j * bs:(j + 1) * bs, None, :].astype(np.float16)
    q = (30.0 * u[None, None, None, :] + 0.05 * rng.standard_normal((B, ctx, H, D))).astype(np.float16)
    cl = np.array([ctx], np.int32)
    if int4:
        pages = O.to_int4_pages(kp, vp)
        want = O.paged_attention_int4(q, pages, bt, cl, ctx, ctx, num_sink_tokens=4, causal=True)
        kc = vc = to_dev(pages)
    else:
        want = O.paged_attention(q, kp, vp, bt, cl, ctx, ctx, num_sink_tokens=4, causal=True)
        kc, vc = to_dev(kp), to_dev(vp)
    got = memopt_C.dynamic_sparse_attention(to_dev(q), kc, vc, to_dev(bt), to_dev(cl), ctx, ctx,
                                            num_sink_tokens=4, causal=True)
    assert_close(got, want, what=f"climbing scores D={D} int4={int4}")


def test_prefill_out_of_pool_pages_are_skipped():
    """Block-table entries >= num_blocks contribute no keys, like entries < 0."""
    B, H, D, bs, ctx, Lq = 1, 2, 64, 16, [96], 96
    nb = 9
    q, kp, vp, bt, cl = _case_inputs(23, B, H, D, bs, nb, ctx, Lq)
    bad = bt.copy()
    bad[0, 2] = nb + 5
    skip = bt.copy()
    skip[0, 2] = -1
    want = O.paged_attention(q, kp, vp, skip, cl, 128, 128, causal=True)
    got = memopt_C.dynamic_sparse_attention(to_dev(q), to_dev(kp), to_dev(vp), to_dev(bad), to_dev(cl), 128, 128,
                                            causal=True)
    assert_close(got, want)


@pytest.mark.parametrize("int4", [False, True], ids=["fp16", "int4"])
@pytest.mark.parametrize("Lq", [1, 40])
def test_nan_past_context_is_ignored(int4, Lq):
    """Tokens of a linked page at or past the context length never reach the
    output, whatever their bits: the last page's tail holds NaN keys and
    values (fp16 pool) or NaN scales (INT4 pages). Decode (q_len 1) and
    prefill both follow the reference, which reads keys < context_len only
    (src/csrc/attention.cu:173)."""
    B, H, D, bs, ctx = 1, 2, 64, 16, 37
    nb = 6
    q, kp, vp, bt, cl = _case_inputs(24, B, H, D, bs, nb, [ctx], Lq)
    want = O.paged_attention(q, kp, vp, bt, cl, 64, 64, causal=True)
    tail = int(bt[0, 2])
    if int4:
        pages = O.to_int4_pages(kp, vp)
        want = O.paged_attention_int4(q, pages, bt, cl, 64, 64, causal=True)
        G = D // 64
        sc = pages[tail].reshape(H, -1)[:, 16 * D:].copy().view(np.float16).reshape(H, 2, G, 16)
        for t in range(ctx - 32, 16):
            sc[:, :, :, 2 * (t % 8) + t // 8] = np.float16(np.nan)
        pages[tail].reshape(H, -1)[:, 16 * D:] = sc.reshape(H, -1).view(np.uint8)
        pg = to_dev(pages)
        got = memopt_C.dynamic_sparse_attention(to_dev(q), pg, pg, to_dev(bt), to_dev(cl), 64, 64, causal=True)
    else:
        kp[tail, ctx - 32:] = np.float16(np.nan)
        vp[tail, ctx - 32:] = np.float16(np.nan)
        got = memopt_C.dynamic_sparse_attention(to_dev(q), to_dev(kp), to_dev(vp), to_dev(bt), to_dev(cl), 64, 64,
                                                causal=True)
    assert not torch.isnan(got).any()
    assert_close(got, want)


def test_non_finite_key_outside_window_is_ignored():
    """A NaN key inside the context reaches only the queries whose window
    holds it; the reference never reads keys outside a query's window
    (src/csrc/attention.cu:173-190), so every other row stays finite and
    matches the oracle."""
    B, H, D, bs, ctx, Lq, W, sinks = 1, 2, 64, 16, 300, 300, 64, 4
    nb = 22
    q, kp, vp, bt, cl = _case_inputs(25, B, H, D, bs, nb, [ctx], Lq)
    bad_tok = 100
    # expected rows from the finite cache: rows that cannot see the key do not
    # depend on its value (the oracle's additive mask cannot hide a NaN)
    want = O.paged_attention(q, kp, vp, bt, cl, 512, W, num_sink_tokens=sinks, causal=True)
    kp[bt[0, bad_tok // bs], bad_tok % bs, 1] = np.float16(np.nan)   # head 1 only
    got = memopt_C.dynamic_sparse_attention(to_dev(q), to_dev(kp), to_dev(vp), to_dev(bt), to_dev(cl), 512, W,
                                            num_sink_tokens=sinks, causal=True).cpu().numpy()
    sees = (np.arange(Lq) >= bad_tok) & (np.arange(Lq) < bad_tok + W)
    keep = ~sees
    assert not np.isnan(got[0, keep]).any()
    assert_close(torch.from_numpy(got[0, keep]), want[0, keep])
    assert_close(torch.from_numpy(got[0, :, 0]), want[0, :, 0])   # head 0 holds no NaN


def test_reference_math_equivalence_multi_query():
    """tests/test_attention.py:112-192 restated on this path: full window,
    non-causal, torch.rand inputs, == SDPA within atol = rtol = 1e-3, and
    deterministic across calls."""
    Bq, H, D, S = 2, 8, 64, 512
    g = torch.Generator().manual_seed(42)
    Q, K, V = (torch.rand(Bq, H, S, D, generator=g).half() for _ in range(3))
    base = torch.nn.functional.scaled_dot_product_attention(Q.float(), K.float(), V.float())
    nbps = S // 16
    kp = K.permute(0, 2, 1, 3).reshape(Bq * nbps, 16, H, D).contiguous()
    vp = V.permute(0, 2, 1, 3).reshape(Bq * nbps, 16, H, D).contiguous()
    bt = torch.arange(Bq * nbps, dtype=torch.int32).reshape(Bq, nbps)
    ctx = torch.full((Bq,), S, dtype=torch.int32)
    q = Q.permute(0, 2, 1, 3).contiguous()
    args = (q.to(dev()), kp.to(dev()), vp.to(dev()), bt.to(dev()), ctx.to(dev()), S, S)
    out = memopt_C.dynamic_sparse_attention(*args)
    assert torch.allclose(base.half().float(), out.permute(0, 2, 1, 3).float().cpu(), atol=1e-3, rtol=1e-3)
    assert torch.equal(out, memopt_C.dynamic_sparse_attention(*args))


def _fp32_rows_reference(q, k, v, rows, ctx, W, sinks):
    """fp32 causal StreamingLLM attention of the selected query rows (GPU).
    q [S, H, D] fp16, k/v [ctx, H, D] fp16 (dequantized values)."""
    D = q.shape[-1]
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    qs = q[rows].float().permute(1, 0, 2)              # [H, n, D]
    kk = k.float().permute(1, 2, 0).contiguous()       # [H, D, ctx]
    s = torch.matmul(qs, kk) * scale                   # [H, n, ctx]
    pos = (ctx - q.shape[0] + rows.to(torch.int64))[:, None]
    j = torch.arange(ctx, device=q.device)[None, :]
    vis = (j <= pos) & ((j < sinks) | (j >= pos - W + 1))
    s = s.masked_fill(~vis[None], float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, v.float().permute(1, 0, 2).contiguous()).permute(1, 0, 2)  # [n, H, D]


@pytest.mark.parametrize("S,H", [(2048, 4), (16384, 32)])
def test_config4_shape_int4_pages(S, H):
    """BASELINE config 4 (B 1, S 16384, H 32, D 128, causal, W 4096, sinks 4)
    and a reduced copy: K/V written through write_cache into an INT4 page pool
    (pages in a shuffled order), prefill over all S queries, checked on sampled
    rows (first, tile edges, window edge, last) against fp32 attention over
    the dequantized pool."""
    D, W, sinks = 128, min(4096, S // 4), 4
    torch.manual_seed(7)
    nb = S // 16 + 8
    memopt_C.init_pool(nb, 16, H, D, kv_format="int4")
    order = torch.randperm(nb)[: S // 16].to(torch.int32)
    bt = order[None].to(dev())
    slots = (order.to(dev()).long()[:, None] * 16 + torch.arange(16, device=dev())).reshape(-1).to(torch.int32)
    k = torch.randn(S, H, D, device=dev(), dtype=torch.float16)
    v = torch.randn(S, H, D, device=dev(), dtype=torch.float16)
    memopt_C.write_cache(k, v, bt, slots)
    del k, v
    q = torch.randn(1, S, H, D, device=dev(), dtype=torch.float16)
    ctx = torch.tensor([S], dtype=torch.int32, device=dev())
    out = memopt_C.dynamic_sparse_attention(q, memopt_C.get_key_pool(), memopt_C.get_value_pool(), bt, ctx, S, W,
                                            num_sink_tokens=sinks, causal=True)
    pages = memopt_C.get_int4_pages()
    kd, vd = O.dequant_pages_torch(pages[order.to(dev()).long()], D)   # [S/16, 16, H, D] in sequence order
    kd, vd = kd.reshape(S, H, D), vd.reshape(S, H, D)
    rows = torch.tensor(sorted({0, 1, 15, 63, 64, 127, 128, 255, W - 1, W, W + 1, S // 2 + 3, S - 129, S - 2, S - 1}),
                        device=dev())
    ref = _fp32_rows_reference(q[0], kd, vd, rows, S, W, sinks)
    assert_close(out[0, rows.long()], ref, what=f"S={S} H={H}")
    torch.cuda.synchronize()


def _fp32_head_reference(qh, kh, vh, r0, r1, ctx, W, sinks):
    """fp32 StreamingLLM causal attention of query rows [r0, r1) of one head
    (qh [Lq, D], kh / vh [ctx, D] dequantized), with 2-D matmuls only."""
    D = qh.shape[-1]
    s = torch.matmul(qh[r0:r1].float(), kh.float().t().contiguous()) * (1.0 / math.sqrt(D))  # [n, ctx]
    pos = (ctx - qh.shape[0] + torch.arange(r0, r1, device=qh.device))[:, None]
    j = torch.arange(ctx, device=qh.device)[None, :]
    vis = (j <= pos) & ((j < sinks) | (j >= pos - W + 1))
    p = torch.softmax(s.masked_fill(~vis, float("-inf")), dim=-1)
    return torch.matmul(p, vh.float())


def test_config4_full_rows_int4_pages():
    """BASELINE configs[3] at full size with its own inputs (Q/K/V ~ N(0, 0.5),
    B 1, S 16384, H 32, D 128, causal W 4096, 4 sinks, K/V written through
    write_cache into shuffled INT4 pages): every one of the 16384 output
    rows of heads 0, 11, 22 and 31 against fp32 attention over the
    dequantized pool, computed head by head on the GPU in 2048-row chunks."""
    S, H, D, W, sinks, std = 16384, 32, 128, 4096, 4, 0.5
    torch.manual_seed(11)
    nb = S // 16 + 8
    memopt_C.init_pool(nb, 16, H, D, kv_format="int4")
    order = torch.randperm(nb)[: S // 16].to(torch.int32)
    bt = order[None].to(dev())
    slots = (order.to(dev()).long()[:, None] * 16 + torch.arange(16, device=dev())).reshape(-1).to(torch.int32)
    k = (torch.randn(S, H, D, device=dev()) * std).half()
    v = (torch.randn(S, H, D, device=dev()) * std).half()
    memopt_C.write_cache(k, v, bt, slots)
    del k, v
    q = (torch.randn(1, S, H, D, device=dev()) * std).half()
    ctx = torch.tensor([S], dtype=torch.int32, device=dev())
    out = memopt_C.dynamic_sparse_attention(q, memopt_C.get_key_pool(), memopt_C.get_value_pool(), bt, ctx, S, W,
                                            num_sink_tokens=sinks, causal=True)
    pages = memopt_C.get_int4_pages()
    kd, vd = O.dequant_pages_torch(pages[order.to(dev()).long()], D)
    kd, vd = kd.reshape(S, H, D), vd.reshape(S, H, D)
    for h in (0, 11, 22, 31):
        for r0 in range(0, S, 2048):
            ref = _fp32_head_reference(q[0, :, h], kd[:, h], vd[:, h], r0, r0 + 2048, S, W, sinks)
            assert_close(out[0, r0:r0 + 2048, h], ref, what=f"config 4 head {h} rows {r0}..{r0 + 2047}")
    torch.cuda.synchronize()


def _prefill_with_env(env, *args, **kw):
    """One attention call with the given environment overrides in place."""
    import os
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        out = memopt_C.dynamic_sparse_attention(*args, **kw)
        torch.cuda.synchronize()
        return out
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


@pytest.mark.parametrize("D,fmt", [(128, "int4"), (64, "int4"), (128, "fp16")])
def test_in_kernel_staging_paths_agree(D, fmt):
    """Long causal prefill (q_len 4096, so the attention kernel stages the
    workspace itself: each XCD's first (sequence, head) unit by a staging
    launch, every later unit by the first workgroups of the unit before it)
    over three sequences whose first units on the XCDs include no head 0 of
    sequences 1 and 2, with unlinked pages in both: the in-kernel path, the
    staging-launch path (MEMOPT_PREFILL_STAGE_LAUNCH) and the path where every
    waiting workgroup stages its unit itself (MEMOPT_PREFILL_STAGE_SPIN=-1)
    agree, and sequence 0 matches fp32 attention over the dequantized pool
    on every row of two heads."""
    B, S, H, W, sinks = 3, 4096, 8, 1024, 4
    torch.manual_seed(13)
    nbps = S // 16
    nb = B * nbps + 8
    memopt_C.init_pool(nb, 16, H, D, kv_format=fmt)
    order = torch.randperm(nb)[:B * nbps].to(torch.int32).reshape(B, nbps)
    bt = order.to(dev())
    for b in range(B):
        slots = (bt[b].long()[:, None] * 16 + torch.arange(16, device=dev())).reshape(-1).to(torch.int32)
        k = torch.randn(S, H, D, device=dev(), dtype=torch.float16)
        v = torch.randn(S, H, D, device=dev(), dtype=torch.float16)
        memopt_C.write_cache(k, v, bt, slots)
    bt[1, 5] = -1
    bt[2, 100] = -1
    q = torch.randn(B, S, H, D, device=dev(), dtype=torch.float16)
    ctx = torch.full((B,), S, dtype=torch.int32, device=dev())
    args = (q, memopt_C.get_key_pool(), memopt_C.get_value_pool(), bt, ctx, S, W)
    kw = dict(num_sink_tokens=sinks, causal=True)
    ink = _prefill_with_env({}, *args, **kw)
    launch = _prefill_with_env({"MEMOPT_PREFILL_STAGE_LAUNCH": "1"}, *args, **kw)
    self_staged = _prefill_with_env({"MEMOPT_PREFILL_STAGE_SPIN": "-1"}, *args, **kw)
    assert torch.isfinite(ink).all()
    assert_close(ink, launch.float().cpu().numpy(), what="in-kernel vs staging launch")
    assert_close(self_staged, launch.float().cpu().numpy(), what="self-staged vs staging launch")
    if fmt == "int4":
        kd, vd = O.dequant_pages_torch(memopt_C.get_int4_pages()[order[0].to(dev()).long()], D)
    else:
        kc, vc = memopt_C.get_pool_tensors()
        kd, vd = kc[order[0].to(dev()).long()].float(), vc[order[0].to(dev()).long()].float()
    kd, vd = kd.reshape(S, H, D), vd.reshape(S, H, D)
    for h in (0, 5):
        ref = _fp32_head_reference(q[0, :, h], kd[:, h], vd[:, h], 0, S, S, W, sinks)
        assert_close(ink[0, :, h], ref, what=f"sequence 0 head {h}")
