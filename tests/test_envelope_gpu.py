"""GPU parity at the edges of the fp16 input range.

* Fused INT4 decode (page and token-major kernels) against the composition
  oracle (dequantize -> fp32 attention, the reference's INT4 path:
  src/csrc/quantization.cu:254-268 then src/csrc/attention.cu:301-324) for
  V groups with absmax up to 6e4 meeting a late key that outscores the
  running max, queries with |q| up to 1e3, and tiny K/V scales.
* Quantization of groups holding NaN or inf (the reference drops NaNs from
  the absmax with fmaxf, quantization.cu:151, :166), bit for bit.
* +-65504 rows written into INT4 pages: page scales, dequantized pools and
  attention stay finite and match the oracle.
"""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import assert_close, dev, memopt_C, same_bits, to_dev

pytestmark = pytest.mark.gpu


def _log2_scores(q, k):
    """Scores in log2 units, q [H, D], k [n, H, D] (fp32)."""
    D = q.shape[-1]
    return np.einsum("hd,nhd->nh", q.astype(np.float32), k.astype(np.float32)) / np.sqrt(D) * np.log2(np.e)


def _envelope_case(seed, H, D, ctx, qscale, kscale, vscale, late_v, late_gap):
    """K/V pools [nb, 16, H, D] and one query per head. When late_v is set, the
    token at ctx - 20 gets a key scoring late_gap log2 units above every other
    key of its head and a V row of absmax late_v; every earlier page has
    already set the running max of the wave that reads it."""
    rng = np.random.default_rng(seed)
    nbps = (ctx + 15) // 16
    nb = nbps + 2
    k = rng.standard_normal((nb, 16, H, D)) * kscale
    v = rng.standard_normal((nb, 16, H, D)) * vscale
    q = rng.standard_normal((1, 1, H, D)) * qscale
    bt = rng.permutation(nb)[:nbps].astype(np.int32)[None]
    q16 = q.astype(np.float16).astype(np.float64)
    if late_v:
        t = ctx - 20
        page, pos = bt[0, t // 16], t % 16
        flat = k[bt[0]].reshape(-1, H, D)[:ctx]
        smax = _log2_scores(q16[0, 0], flat).max(axis=0)                    # [H]
        qq = (q16[0, 0] ** 2).sum(-1)                                        # [H]
        c = (smax + late_gap) * np.sqrt(D) / np.log2(np.e) / qq
        k[page, pos] = q16[0, 0] * c[:, None]
        row = rng.standard_normal((H, D))
        v[page, pos] = row / np.abs(row).max(axis=-1, keepdims=True) * late_v
    q, k, v = q.astype(np.float16), k.astype(np.float16), v.astype(np.float16)
    assert all(np.isfinite(a.astype(np.float32)).all() for a in (q, k, v)), "inputs must be finite fp16"
    return q, k, v, bt


ENVELOPE = [
    # seed, H, D, ctx, |q|, K scale, V scale, late V absmax, late gap (log2 units)
    (0, 4, 128, 2048, 1.0, 1.0, 1.0, 1e3, 7.0),
    (1, 4, 128, 2048, 1.0, 1.0, 1.0, 7e3, 7.0),
    (2, 4, 128, 2048, 1.0, 1.0, 1.0, 6e4, 7.0),
    (3, 4, 64, 1500, 1.0, 1.0, 1.0, 6e4, 7.9),
    (4, 4, 128, 2048, 1.0, 1.0, 1.0, 6e4, 3.0),
    (5, 4, 128, 2048, 1.0, 1.0, 1e3, 6e4, 6.0),      # every V group large
    (6, 4, 128, 4096, 1.0, 1.0, 8e3, 0, 0),          # large V everywhere, no planted key
    (7, 4, 128, 2048, 100.0, 0.01, 1.0, 0, 0),       # |q| 100, scores of order 1
    (8, 4, 128, 2048, 1000.0, 1e-3, 1.0, 0, 0),      # |q| 1000, K scale 1e-3
    (9, 4, 64, 2048, 1000.0, 1e-3, 1.0, 7e3, 5.0),
    (10, 4, 128, 2048, 1000.0, 1.0, 1.0, 0, 0),      # |q| 1000 against N(0,1) K: one-hot
    (11, 4, 128, 2048, 1.0, 1e-3, 1e-3, 0, 0),       # tiny K and V
    (12, 4, 128, 2048, 1.0, 1e-3, 1e-3, 1.0, 7.0),
]


def _assert_close_scaled(got, want, vscale, what):
    """The north_star tolerance (2e-3 / 1e-2) applied to outputs divided by
    the V scale. The reference rounds each dequantized V element to fp16
    (relative error 2^-12), so when every V row is of size c its own output
    moves by amounts proportional to c; the absolute part of the tolerance
    scales with it. For vscale <= 1 this is the plain tolerance."""
    sc = max(1.0, float(vscale))
    g = got.float().cpu().numpy() / sc if isinstance(got, torch.Tensor) else np.asarray(got, np.float32) / sc
    assert_close(g, np.asarray(want, np.float32) / sc, what=what)


@pytest.mark.parametrize("case", ENVELOPE)
def test_decode_int4_pages_envelope(case):
    seed, H, D, ctx, qs, ks, vs, late_v, gap = case
    q, k, v, bt = _envelope_case(seed, H, D, ctx, qs, ks, vs, late_v, gap)
    cl = np.array([ctx], np.int32)
    pages = O.to_int4_pages(k, v)
    want = O.paged_attention_int4(q, pages, bt, cl, ctx, ctx)
    assert np.isfinite(want.astype(np.float32)).all()
    pg = to_dev(pages)
    got = memopt_C.dynamic_sparse_attention(to_dev(q), pg, pg, to_dev(bt), to_dev(cl), ctx, ctx)
    assert torch.isfinite(got).all(), f"{case}: non-finite output"
    _assert_close_scaled(got, want, vs, str(case))


@pytest.mark.parametrize("case", ENVELOPE)
def test_decode_int4_token_major_envelope(case):
    seed, H, D, ctx, qs, ks, vs, late_v, gap = case
    q, k, v, bt = _envelope_case(seed, H, D, ctx, qs, ks, vs, late_v, gap)
    cl = np.array([ctx], np.int32)
    kc, ksc = O.quantize_int4(k)
    vc, vsc = O.quantize_int4(v)
    want = O.paged_attention(q, O.dequantize_int4(kc, ksc), O.dequantize_int4(vc, vsc), bt, cl, ctx, ctx)
    got = memopt_C.dynamic_sparse_attention(to_dev(q), to_dev(kc), to_dev(vc), to_dev(bt), to_dev(cl), ctx, ctx,
                                            key_scales=to_dev(ksc), value_scales=to_dev(vsc), kv_layout="token_major")
    assert torch.isfinite(got).all(), f"{case}: non-finite output"
    _assert_close_scaled(got, want, vs, str(case))


def test_decode_envelope_split_k():
    """The same large-V case with one sequence long enough for split-K: the
    per-split reference points differ, and the in-kernel merge of the
    split partials must still agree."""
    q, k, v, bt = _envelope_case(20, 2, 128, 16384, 1.0, 1.0, 2e3, 6e4, 7.5)
    cl = np.array([16384], np.int32)
    pages = O.to_int4_pages(k, v)
    want = O.paged_attention_int4(q, pages, bt, cl, 16384, 16384)
    pg = to_dev(pages)
    got = memopt_C.dynamic_sparse_attention(to_dev(q), pg, pg, to_dev(bt), to_dev(cl), 16384, 16384)
    assert torch.isfinite(got).all()
    _assert_close_scaled(got, want, 2e3, "split-K large V")


def test_prefill_int4_pages_large_v():
    """Multi-query MFMA path over INT4 pages with V groups near the fp16 limit."""
    q, k, v, bt = _envelope_case(30, 2, 128, 640, 1.0, 1.0, 8e3, 6e4, 7.0)
    q = np.random.default_rng(31).standard_normal((1, 96, 2, 128)).astype(np.float16)
    cl = np.array([640], np.int32)
    pages = O.to_int4_pages(k, v)
    want = O.paged_attention_int4(q, pages, bt, cl, 640, 256, num_sink_tokens=4, causal=True)
    pg = to_dev(pages)
    got = memopt_C.dynamic_sparse_attention(to_dev(q), pg, pg, to_dev(bt), to_dev(cl), 640, 256,
                                            num_sink_tokens=4, causal=True)
    assert torch.isfinite(got).all()
    _assert_close_scaled(got, want, 8e3, "prefill large V")


# ---------------------------------------------------------------------------
# Non-finite groups and the fp16 extremes
# ---------------------------------------------------------------------------

def _nonfinite_rows():
    rng = np.random.default_rng(40)
    x = (rng.standard_normal((32, 4, 128)) * 2).astype(np.float16)   # [T, H, D]
    x[0, 0, 5] = np.nan
    x[1, 1, :64] = np.nan
    x[2, 2, :] = 0
    x[2, 2, 70] = np.nan
    x[3, 3, 9] = np.inf
    x[4, 0, 64], x[4, 0, 65] = -np.inf, np.nan
    x[5, 1, :] = 65504
    x[5, 1, ::2] = -65504
    x[6, 2, 3], x[6, 2, 4] = np.nan, 65504
    return x


def test_quantize_nonfinite_groups_bit_exact():
    x = _nonfinite_rows()
    packed, scales = memopt_C.quantize_kv_cache_int4(to_dev(x), 64)
    wp, ws = O.quantize_int4(x)
    cp, cs = O.quantize_int4_c(x)
    assert np.array_equal(wp, cp) and np.array_equal(ws.view(np.uint32), cs.view(np.uint32))
    same_bits(packed, wp)
    same_bits(scales, ws)


@pytest.mark.parametrize("aligned", [True, False])
def test_write_int4_pages_nonfinite_and_extremes(aligned):
    """write_cache into INT4 pages (whole-page and scattered slots) of rows with
    NaN, inf and +-65504: pages bit-exact against the oracle, the 65504 group
    stored with page scale 9352, and its dequantized rows finite."""
    k = _nonfinite_rows()
    v = k[::-1].copy()
    T, H, D = k.shape
    nb = 4
    memopt_C.init_pool(nb, 16, H, D, kv_format="int4")
    slots = np.arange(T, dtype=np.int32) if aligned else np.random.default_rng(41).permutation(nb * 16)[:T].astype(np.int32)
    memopt_C.write_cache(to_dev(k), to_dev(v), to_dev(np.zeros((1, 1), np.int32)), to_dev(slots))
    kp = np.zeros((nb, 16, H, D), np.float16)
    vp = np.zeros((nb, 16, H, D), np.float16)
    O.write_cache(kp, k, slots)
    O.write_cache(vp, v, slots)
    want = O.to_int4_pages(kp, vp)
    written = np.zeros((nb, 16), bool)
    written.reshape(-1)[slots] = True
    # rows never written keep the empty pattern (codes 8, scale 1.0); compare written pages only
    got = memopt_C.get_int4_pages().cpu().numpy()
    pages_with_rows = np.nonzero(written.any(axis=1))[0]
    kc_g, ks_g, vc_g, vs_g = O.int4_pages_split(got, D)
    kc_w, ks_w, vc_w, vs_w = O.int4_pages_split(want, D)
    for a, b in ((kc_g, kc_w), (ks_g, ks_w), (vc_g, vc_w), (vs_g, vs_w)):
        sel = written[pages_with_rows]
        same_bits(a[pages_with_rows][sel], b[pages_with_rows][sel])
    s5 = slots[5]
    assert ks_g[s5 // 16, s5 % 16, 1, 0] == np.float16(9352) and ks_g[s5 // 16, s5 % 16, 1, 1] == np.float16(9352)
    kd, vd = memopt_C.dequantize_int4_pages()
    row = kd[s5 // 16, s5 % 16, 1].float().cpu().numpy()
    assert np.isfinite(row).all() and np.abs(row).max() == float(np.float16(7 * 9352))   # 65464 -> fp16 65472


def test_attention_over_pm65504_rows():
    """Decode and prefill over INT4 pages whose rows hold +-65504: finite,
    and within tolerance of the oracle."""
    rng = np.random.default_rng(42)
    H, D, ctx = 2, 128, 256
    nb = ctx // 16
    k = (rng.standard_normal((nb, 16, H, D)) * 0.05).astype(np.float16)
    v = rng.standard_normal((nb, 16, H, D)).astype(np.float16)
    v[3, 4, 0, :] = 65504
    v[3, 4, 0, 1::2] = -65504
    v[7, 9, 1, :64] = 65504
    bt = rng.permutation(nb).astype(np.int32)[None]
    cl = np.array([ctx], np.int32)
    pages = O.to_int4_pages(k, v)
    pg = to_dev(pages)
    for lq, causal in ((1, False), (64, True)):
        q = (rng.standard_normal((1, lq, H, D)) * 0.05).astype(np.float16)
        want = O.paged_attention_int4(q, pages, bt, cl, ctx, ctx, causal=causal)
        got = memopt_C.dynamic_sparse_attention(to_dev(q), pg, pg, to_dev(bt), to_dev(cl), ctx, ctx, causal=causal)
        assert torch.isfinite(got).all(), f"q_len {lq}: non-finite output"
        assert_close(got, want, what=f"q_len {lq}")
