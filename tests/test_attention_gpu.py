"""GPU parity of dynamic_sparse_attention (restates the reference's
tests/test_attention.py and extends it to windows, sinks, causal masks,
unlinked pages and INT4 caches, all against the CPU oracle)."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from gpu_helpers import assert_close, dev, memopt_C, to_dev

pytestmark = pytest.mark.gpu

BLOCK_SIZE, NUM_HEADS, HEAD_DIM, BATCH = 16, 8, 64, 2


def setup_pool(num_tokens, block_size, num_heads, head_dim, kv_format="fp16"):
    """tests/test_attention.py:38-105: allocate blocks per sequence, build slots."""
    seq_len = num_tokens // BATCH
    nbps = math.ceil(seq_len / block_size)
    memopt_C.init_pool(BATCH * nbps + 2, block_size, num_heads, head_dim, kv_format=kv_format)
    rows = [[memopt_C.allocate_block() for _ in range(nbps)] for _ in range(BATCH)]
    assert all(p != -1 for r in rows for p in r)
    slots = [rows[b][t // block_size] * block_size + t % block_size for b in range(BATCH) for t in range(seq_len)]
    return (torch.tensor(slots, dtype=torch.int32, device=dev()),
            torch.tensor(rows, dtype=torch.int32, device=dev()), nbps)


def _reference_inputs(seq_len, seed=42):
    g = torch.Generator().manual_seed(seed)
    mk = lambda: torch.rand(BATCH, NUM_HEADS, seq_len, HEAD_DIM, generator=g).half()
    return mk(), mk(), mk()


@pytest.mark.parametrize("seq_len", [512, 1024, 2048])
def test_math_equivalence(seq_len):
    """tests/test_attention.py:112-192: full window == non-causal SDPA, atol=rtol=1e-3."""
    Q, K, V = _reference_inputs(seq_len)
    baseline = F.scaled_dot_product_attention(Q.float().to(dev()), K.float().to(dev()), V.float().to(dev()))
    slot, bt, _ = setup_pool(BATCH * seq_len, BLOCK_SIZE, NUM_HEADS, HEAD_DIM)
    kf = K.permute(0, 2, 1, 3).contiguous().reshape(-1, NUM_HEADS, HEAD_DIM).to(dev())
    vf = V.permute(0, 2, 1, 3).contiguous().reshape(-1, NUM_HEADS, HEAD_DIM).to(dev())
    memopt_C.write_cache(kf, vf, bt, slot)
    kc, vc = memopt_C.get_pool_tensors()
    q = Q.permute(0, 2, 1, 3).contiguous().to(dev())
    ctx = torch.full((BATCH,), seq_len, dtype=torch.int32, device=dev())
    out = memopt_C.dynamic_sparse_attention(q, kc, vc, bt, ctx, seq_len, seq_len)
    assert out.shape == (BATCH, seq_len, NUM_HEADS, HEAD_DIM)
    assert torch.allclose(baseline.half().float(), out.permute(0, 2, 1, 3).float(), atol=1e-3, rtol=1e-3)
    out2 = memopt_C.dynamic_sparse_attention(q, kc, vc, bt, ctx, seq_len, seq_len)
    assert torch.equal(out, out2)  # determinism, tests/test_attention.py:293-349


def _random_case(seed, B, H, D, bs, nb, ctx, Lq, int4_scale_pages=False):
    rng = np.random.default_rng(seed)
    kp = (rng.standard_normal((nb, bs, H, D)) * np.where(rng.random((nb, bs, H, D)) < 0.01, 8, 1)).astype(np.float16)
    vp = rng.standard_normal((nb, bs, H, D)).astype(np.float16)
    q = rng.standard_normal((B, Lq, H, D)).astype(np.float16)
    M = max(1, (max(ctx) + bs - 1) // bs)
    bt = rng.permutation(nb)[:B * M].reshape(B, M).astype(np.int32)
    return q, kp, vp, bt, np.array(ctx, np.int32)


CASES = [
    # B, H, D, bs, ctx, Lq, max_seq_len, W, sinks, causal, unlink
    (2, 4, 64, 16, [200, 77], 1, 256, 256, 0, False, False),
    (2, 4, 128, 16, [200, 77], 1, 256, 48, 4, False, True),
    (3, 2, 64, 32, [100, 1, 64], 1, 128, 40, 0, False, False),
    (2, 4, 64, 16, [90, 120], 7, 128, 30, 4, False, False),
    (2, 2, 128, 16, [96, 50], 50, 128, 128, 0, True, False),
    (1, 2, 64, 16, [130], 40, 256, 24, 4, True, True),
    (2, 2, 96, 8, [33, 70], 3, 80, 16, 2, False, True),   # odd head_dim, 8-token pages
    (1, 2, 64, 16, [0], 1, 64, 64, 4, False, False),        # empty context -> zeros
]


@pytest.mark.parametrize("case", CASES)
def test_fp16_paged_vs_oracle(case):
    B, H, D, bs, ctx, Lq, msl, W, sinks, causal, unlink = case
    nb = B * ((max(ctx) + bs - 1) // bs) + 3
    q, kp, vp, bt, cl = _random_case(11, B, H, D, bs, nb, ctx, Lq)
    if unlink:
        bt[0, 1] = -1
    want = O.paged_attention(q, kp, vp, bt, cl, msl, W, num_sink_tokens=sinks, causal=causal)
    got = memopt_C.dynamic_sparse_attention(to_dev(q), to_dev(kp), to_dev(vp), to_dev(bt), to_dev(cl), msl, W,
                                            num_sink_tokens=sinks, causal=causal)
    assert_close(got, want, atol=1e-3, rtol=1e-3, what=str(case))


@pytest.mark.parametrize("case", [c for c in CASES if c[2] % 64 == 0])
@pytest.mark.parametrize("layout", ["token_major", "pages"])
def test_int4_paged_vs_composition_oracle(case, layout):
    """Fused INT4 attention == dequantize_kv_cache_int4 -> attention (the reference's INT4 path)."""
    B, H, D, bs, ctx, Lq, msl, W, sinks, causal, unlink = case
    if layout == "pages" and bs != 16:
        pytest.skip("the INT4 page pool uses 16-token pages")
    nb = B * ((max(ctx) + bs - 1) // bs) + 3
    q, kp, vp, bt, cl = _random_case(12, B, H, D, bs, nb, ctx, Lq)
    if unlink:
        bt[0, 1] = -1
    if layout == "token_major":
        kc, ks = O.quantize_int4(kp)
        vc, vs = O.quantize_int4(vp)
        want = O.paged_attention(q, O.dequantize_int4(kc, ks), O.dequantize_int4(vc, vs), bt, cl, msl, W,
                                 num_sink_tokens=sinks, causal=causal)
        got = memopt_C.dynamic_sparse_attention(to_dev(q), to_dev(kc), to_dev(vc), to_dev(bt), to_dev(cl), msl, W,
                                                num_sink_tokens=sinks, causal=causal, key_scales=to_dev(ks),
                                                value_scales=to_dev(vs), kv_layout=layout)
    else:
        pages = O.to_int4_pages(kp, vp)
        want = O.paged_attention_int4(q, pages, bt, cl, msl, W, num_sink_tokens=sinks, causal=causal)
        pg = to_dev(pages)
        got = memopt_C.dynamic_sparse_attention(to_dev(q), pg, pg, to_dev(bt), to_dev(cl), msl, W,
                                                num_sink_tokens=sinks, causal=causal)
    assert_close(got, want, what=f"{layout} {case}")


def test_reference_window_clamp_and_max_seq_len():
    """W > max_seq_len -> max_seq_len, and max_seq_len < ctx restricts the window
    (src/csrc/attention.cu:453-455; DynamicAttention passes max_seq_len = q_len)."""
    q, kp, vp, bt, cl = _random_case(13, 1, 2, 64, 16, 8, [100], 1)
    for msl, W in ((40, 1000), (40, 0), (40, -5), (1, 1)):
        want = O.paged_attention(q, kp, vp, bt, cl, msl, W)
        got = memopt_C.dynamic_sparse_attention(to_dev(q), to_dev(kp), to_dev(vp), to_dev(bt), to_dev(cl), msl, W)
        assert_close(got, want, atol=1e-3, rtol=1e-3, what=f"msl={msl} W={W}")


def test_int4_pool_via_pool_getters():
    """DynamicAttention's calling sequence on an INT4 pool: write_cache ->
    get_key_pool/get_value_pool -> dynamic_sparse_attention (scales implied)."""
    rng = np.random.default_rng(14)
    H, D, T = 4, 128, 64
    slot, bt, _ = setup_pool(BATCH * T, 16, H, D, kv_format="int4")
    k = rng.standard_normal((BATCH * T, H, D)).astype(np.float16)
    v = rng.standard_normal((BATCH * T, H, D)).astype(np.float16)
    memopt_C.write_cache(to_dev(k), to_dev(v), bt, slot)
    q = rng.standard_normal((BATCH, 1, H, D)).astype(np.float16)
    ctx = torch.full((BATCH,), T, dtype=torch.int32, device=dev())
    got = memopt_C.dynamic_sparse_attention(to_dev(q), memopt_C.get_key_pool(), memopt_C.get_value_pool(), bt, ctx,
                                            T, T)
    want = O.paged_attention_int4(q, memopt_C.get_int4_pages().cpu().numpy(), bt.cpu().numpy(),
                                  ctx.cpu().numpy(), T, T)
    assert_close(got, want)


def test_argument_errors():
    q = torch.zeros(1, 1, 2, 64, dtype=torch.float16, device=dev())
    kc = torch.zeros(2, 16, 2, 64, dtype=torch.float16, device=dev())
    bt = torch.zeros(1, 2, dtype=torch.int32, device=dev())
    cl = torch.ones(1, dtype=torch.int32, device=dev())
    with pytest.raises(RuntimeError):
        memopt_C.dynamic_sparse_attention(q.cpu(), kc, kc, bt, cl, 32, 32)
    with pytest.raises(RuntimeError):
        memopt_C.dynamic_sparse_attention(q.float(), kc, kc, bt, cl, 32, 32)
    with pytest.raises(RuntimeError):
        memopt_C.dynamic_sparse_attention(q, kc, kc, bt.long(), cl, 32, 32)
    with pytest.raises(RuntimeError):
        memopt_C.dynamic_sparse_attention(q, kc[:, :, :1].contiguous(), kc, bt, cl, 32, 32)
    with pytest.raises(RuntimeError):
        memopt_C.dynamic_sparse_attention(q, kc.to(torch.uint8), kc.to(torch.uint8), bt, cl, 32, 32)  # no scales
