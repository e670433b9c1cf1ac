"""memopt_paged_attention_noalloc (split-K partials and small prefill staging
in a static per-GPU scratch array, no allocation) against
memopt_paged_attention on the same descriptors, called through the C ABI:
two calls in a row with the second one smaller, for a split-K decode and for
a staged multi-query call; a decode whose partials exceed the scratch is
refused with a clear error."""
import ctypes
import os

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import assert_close, memopt_C, to_dev

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 4 << 20


def _entry_points():
    import memopt_C as M
    f = M._lib.memopt_paged_attention_noalloc
    f.argtypes = [ctypes.POINTER(M.AttnDesc), ctypes.c_void_p]
    f.restype = ctypes.c_int32
    g = M._lib.memopt_paged_attention
    g.argtypes = [ctypes.POINTER(M.AttnDesc), ctypes.c_void_p]
    g.restype = ctypes.c_int32
    return M, f, g


def _pages_case(seed, B, H, D, ctx, Lq):
    rng = np.random.default_rng(seed)
    M = (max(ctx) + 15) // 16
    nb = B * M + 2
    k = (rng.standard_normal((nb, 16, H, D)) * np.where(rng.random((nb, 16, H, D)) < 0.005, 10, 1)).astype(np.float16)
    v = rng.standard_normal((nb, 16, H, D)).astype(np.float16)
    q = rng.standard_normal((B, Lq, H, D)).astype(np.float16)
    bt = rng.permutation(nb)[:B * M].reshape(B, M).astype(np.int32)
    return q, O.to_int4_pages(k, v), bt, np.array(ctx, np.int32)


def _run_both(case, msl, W, sinks, causal):
    """(noalloc output, memopt_paged_attention output, workspace bytes the
    regular entry point was given) for one descriptor."""
    M, noalloc, regular = _entry_points()
    q, pages, bt, cl = case
    pg = to_dev(pages)
    args = (to_dev(q), pg, pg, to_dev(bt), to_dev(cl), msl, W, sinks, causal, None, None, None)
    stream = torch.cuda.current_stream().cuda_stream
    d, out, ws, keep = M._attention_desc(*args, None)
    out.fill_(float("nan"))
    assert regular(ctypes.byref(d), stream) == 0, M._lib.memopt_last_error().decode()
    want = out.clone()
    d2, out2, ws2, keep2 = M._attention_desc(*args, None, alloc_workspace=False)
    assert ws2 is None and d2.workspace is None
    out2.fill_(float("nan"))
    assert noalloc(ctypes.byref(d2), stream) == 0, M._lib.memopt_last_error().decode()
    torch.cuda.synchronize()
    return out2, want, 0 if ws is None else ws.numel()


def test_noalloc_split_k_decode_two_calls():
    first = _pages_case(1, 1, 4, 128, [8192], 1)        # 4 (b, h) units: many splits
    second = _pages_case(2, 2, 2, 64, [3000, 700], 1)   # smaller, other head_dim
    for case, W, sinks in ((first, 8192, 4), (second, 1024, 0)):
        got, want, ws_bytes = _run_both(case, 1 << 20, W, sinks, False)
        assert 0 < ws_bytes <= SCRATCH_BYTES          # the shape does use split-K partials
        assert torch.equal(got, want)                  # same kernels, same splits: same bits
        q, pages, bt, cl = case
        assert_close(got, O.paged_attention_int4(q, pages, bt, cl, 1 << 20, W, num_sink_tokens=sinks),
                     what="noalloc decode")


def test_noalloc_staged_prefill_two_calls():
    first = _pages_case(3, 1, 2, 128, [512], 128)
    second = _pages_case(4, 1, 2, 128, [256], 64)
    for case, W in ((first, 256), (second, 100)):
        got, want, ws_bytes = _run_both(case, 1 << 20, W, 4, True)
        assert 0 < ws_bytes <= SCRATCH_BYTES          # staged path, workspace in the scratch
        assert torch.equal(got, want)
        q, pages, bt, cl = case
        assert_close(got, O.paged_attention_int4(q, pages, bt, cl, 1 << 20, W, num_sink_tokens=4, causal=True),
                     what="noalloc prefill")


def test_noalloc_decode_after_staged_prefill():
    """A staged multi-query call writes its K/V over the scratch the split-K
    partials use; the decode after it must still merge its splits (its
    arrival counters live in the scratch's last 64 KiB, which nothing else
    writes)."""
    pre = _pages_case(7, 1, 2, 128, [512], 128)
    dec = _pages_case(8, 1, 4, 128, [8192], 1)
    for _ in range(2):
        got, want, _ = _run_both(pre, 1 << 20, 256, 4, True)
        assert torch.equal(got, want)
        got, want, ws_bytes = _run_both(dec, 1 << 20, 8192, 4, False)
        assert ws_bytes > 0 and torch.equal(got, want)
        q, pages, bt, cl = dec
        assert_close(got, O.paged_attention_int4(q, pages, bt, cl, 1 << 20, 8192, num_sink_tokens=4),
                     what="noalloc decode after a staged prefill")


@pytest.mark.parametrize("B,H,D,ctx,Lq,causal", [(2, 4, 128, [3835, 696], 2, False),
                                                 (3, 2, 64, [5243, 266, 2961], 120, True)])
def test_noalloc_large_prefill_runs_unstaged(B, H, D, ctx, Lq, causal):
    """A multi-query call whose staged K/V would not fit the static scratch
    runs the kernel that dequantizes into LDS itself (no scratch): its output
    and the regular entry point's (staged) are both within the tests'
    tolerance of the oracle; they need not be bit-identical."""
    case = _pages_case(11 + B, B, H, D, ctx, Lq)
    got, want, ws_bytes = _run_both(case, 1 << 20, 1 << 20, 16, causal)
    assert ws_bytes > (4 << 20)  # the staged workspace exceeds the scratch
    q, pages, bt, cl = case
    ref = O.paged_attention_int4(q, pages, bt, cl, 1 << 20, 1 << 20, num_sink_tokens=16, causal=causal)
    assert_close(got, ref, what="noalloc (unstaged) prefill")
    assert_close(want, ref, what="regular (staged) prefill")


def test_noalloc_prepared_attention_and_limit():
    """PreparedAttention(no_alloc=True) holds no workspace and matches the
    regular call; partials past the scratch (forced splits) are refused."""
    q, pages, bt, cl = _pages_case(5, 2, 4, 128, [4096, 2000], 1)
    pg = to_dev(pages)
    args = (to_dev(q), pg, pg, to_dev(bt), to_dev(cl), 4096, 4096)
    reg = memopt_C.PreparedAttention(*args)
    na = memopt_C.PreparedAttention(*args, no_alloc=True)
    assert reg.workspace_bytes > 0 and na.workspace_bytes == 0
    assert torch.equal(na().clone(), reg())
    old = os.environ.get("MEMOPT_DECODE_SPLITS")
    os.environ["MEMOPT_DECODE_SPLITS"] = "64"
    try:
        q2, pages2, bt2, cl2 = _pages_case(6, 4, 32, 128, [512] * 4, 1)
        pg2 = to_dev(pages2)
        big = memopt_C.PreparedAttention(to_dev(q2), pg2, pg2, to_dev(bt2), to_dev(cl2), 512, 512, no_alloc=True)
        with pytest.raises(RuntimeError, match="static scratch"):
            big()   # 4 * 32 * 64 * 130 * 4 bytes of partials > 4 MiB
    finally:
        if old is None:
            del os.environ["MEMOPT_DECODE_SPLITS"]
        else:
            os.environ["MEMOPT_DECODE_SPLITS"] = old
