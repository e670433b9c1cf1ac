"""CPU checks that pin the oracle (oracle/oracle.py) independently of itself.

Each check is chosen so that a plausible slip in the restatement (round
half-to-even instead of half-away, swapped nibbles, a dropped sink, an
off-by-one window edge, a transposed page layout) fails it:
  * known answers from the reference's own tests (tests/test_quant.py:439-566);
  * exact rational (fractions.Fraction) evaluation of IEEE fp32 division and
    rounding, and C ``roundf``, on random and adversarial groups;
  * agreement with the independent C restatement (oracle/quant_ref.c, libm);
  * attention against torch's scaled_dot_product_attention on unpaged K/V
    and against a float64 brute-force loop on tiny inputs;
  * eviction against brute-force ``sorted()`` selection.
"""
from fractions import Fraction
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O


# ---------------------------------------------------------------------------
# Exact rational model of IEEE rounding
# ---------------------------------------------------------------------------

def round_ieee(x: Fraction, prec: int, emin: int) -> Fraction:
    """Round-to-nearest-even of an exact rational to a binary float with
    `prec` significand bits and minimum normal exponent `emin` (subnormals
    included, no overflow)."""
    if x == 0:
        return Fraction(0)
    s = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    quantum = Fraction(2) ** (e - prec + 1)
    m = a / quantum
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return s * n * quantum


def rn32(x):
    return round_ieee(x, 24, -126)


def rn16(x):
    return round_ieee(x, 11, -14)


def exact_quant_group(vals16: np.ndarray):
    """Reference quantizer evaluated in exact arithmetic (src/csrc/quantization.cu:129-202)."""
    v = [Fraction(float(x)) for x in vals16.astype(np.float64)]
    absmax = max(abs(x) for x in v)
    scale = rn32(absmax / 7) if absmax > 0 else Fraction(1)
    codes = []
    for x in v:
        q = rn32(x / scale)
        r = math.floor(abs(q) + Fraction(1, 2)) * (1 if q >= 0 else -1)  # roundf: half away from zero
        codes.append(min(max(r + 8, 0), 15))
    return codes, scale


# ---------------------------------------------------------------------------
# Quantize: known answers
# ---------------------------------------------------------------------------

def test_kat_zeros():
    packed, scales = O.quantize_int4(np.zeros((4, 128), np.float16))
    assert (packed == 0x88).all() and (scales == 1.0).all()
    assert (O.dequantize_int4(packed, scales) == 0).all()


def test_kat_alternating_pm7():
    x = np.empty(64, np.float16)
    x[0::2], x[1::2] = 7.0, -7.0
    packed, scales = O.quantize_int4(x)
    assert scales.tolist() == [1.0] and (packed == 0x1F).all()  # lo = 15 (+7), hi = 1 (-7)
    assert (O.dequantize_int4(packed, scales) == x).all()


def test_kat_constant_half():
    packed, scales = O.quantize_int4(np.full((4, 128), 0.5, np.float16))
    assert (packed == 0xFF).all()
    assert np.allclose(scales, np.float32(0.5) / np.float32(7))
    d = O.dequantize_int4(packed, scales).astype(np.float32)
    assert ((d - 0.5) ** 2).mean() < 1e-6


def test_kat_single_group_shapes():
    packed, scales = O.quantize_int4(np.random.default_rng(0).uniform(-1, 1, 64).astype(np.float16))
    assert packed.shape == (32,) and scales.shape == (1,)


def test_kat_round_half_away_and_nibble_order():
    # absmax 7 -> scale exactly 1.0: v/scale == v, so the rounding mode is visible.
    x = np.zeros(64, np.float16)
    x[:10] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 3.5, -3.5, 6.5, 7.0]
    packed, scales = O.quantize_int4(x)
    assert scales[0] == 1.0
    codes = O.unpack_codes(packed)[:10].tolist()
    # roundf: 0.5->1, -0.5->-1, 1.5->2, -1.5->-2, 2.5->3, -2.5->-3, 3.5->4, -3.5->-4, 6.5->7
    assert codes == [9, 7, 10, 6, 11, 5, 12, 4, 15, 15]
    # byte 0 = code[0] | code[1] << 4 (low nibble = even element)
    assert packed[0] == (9 | (7 << 4))


def test_quantize_exact_rational_random():
    rng = np.random.default_rng(1)
    groups = [
        rng.standard_normal(64),
        rng.standard_normal(64) * 1e-3,
        rng.uniform(-100, 100, 64),
        np.where(rng.random(64) < 0.05, 8.0, 1.0) * rng.standard_normal(64),
        rng.standard_normal(64) * 6e-6,             # fp16 subnormals
        np.linspace(-1, 1, 64),                     # many exact ties after scaling
        np.array([7.0 * k / 8 for k in range(-32, 32)]),
    ]
    for g in groups:
        x = g.astype(np.float16)
        packed, scales = O.quantize_int4(x)
        codes, scale = exact_quant_group(x)
        assert Fraction(float(scales[0])) == scale
        assert O.unpack_codes(packed).tolist() == codes


def test_quantize_c_restatement_agrees():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4096, 64)) * rng.choice([1.0, 8.0], size=(4096, 64), p=[0.99, 0.01])
    x[0] = 0.0
    x[1] = 1e-7
    x[2, :] = np.linspace(-7, 7, 64)
    x = x.astype(np.float16)
    p1, s1 = O.quantize_int4(x)
    p2, s2 = O.quantize_int4_c(x)
    assert np.array_equal(p1, p2)
    assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32))
    d1, d2 = O.dequantize_int4(p1, s1), O.dequantize_int4_c(p2, s2)
    assert np.array_equal(d1.view(np.uint16), d2.view(np.uint16))


def test_dequantize_exact_rational():
    rng = np.random.default_rng(3)
    scales = np.concatenate([rng.uniform(1e-6, 20, 30), [1.0, 0.5 / 7, 1e-7]]).astype(np.float32)
    codes = rng.integers(0, 16, size=(scales.size, 64)).astype(np.uint8)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    out = O.dequantize_int4(packed, scales)
    for g in range(scales.size):
        s = Fraction(float(scales[g]))
        for e in (0, 1, 31, 63):
            want = rn16(rn32((int(codes[g, e]) - 8) * s))
            assert Fraction(float(out[g, e])) == want


@pytest.mark.parametrize("dist,bound", [("uniform", 5e-3), ("normal", 5e-2), ("small", 5e-5)])
def test_mse_bounds(dist, bound):
    """Reference accuracy bounds (tests/test_quant.py:309-375) hold for the oracle."""
    rng = np.random.default_rng(4)
    x = {"uniform": rng.uniform(-1, 1, 8192), "normal": rng.standard_normal(8192),
         "small": rng.uniform(-0.1, 0.1, 8192)}[dist].astype(np.float16)
    p, s = O.quantize_int4(x)
    d = O.dequantize_int4(p, s).astype(np.float32)
    assert ((d - x.astype(np.float32)) ** 2).mean() < bound


def test_error_bound_half_step():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((256, 64)) * 3).astype(np.float16)
    p, s = O.quantize_int4(x)
    d = O.dequantize_int4(p, s).astype(np.float32)
    err = np.abs(d - x.astype(np.float32)).reshape(-1, 64)
    # |deq - v| <= scale/2 plus the final fp16 rounding of the dequantized value
    assert (err <= s[:, None] / 2 * (1 + 1e-6) + np.abs(d).reshape(-1, 64) * 2.0 ** -11).all()
    codes = O.unpack_codes(p)
    assert codes.min() >= 1 and codes.max() <= 15  # finite inputs never reach code 0


def test_int4_page_maps_are_bijections():
    for D in (64, 128, 192):
        k_off, v_off, s_idx = O.int4_page_maps(D)
        assert np.array_equal(np.sort(k_off.reshape(-1)), np.arange(8 * D))
        assert np.array_equal(np.sort(v_off.reshape(-1)), np.arange(8 * D))
        assert np.array_equal(np.sort(s_idx.reshape(-1)), np.arange(16 * (D // 64)))


def test_int4_page_layout_examples():
    """Hand-derived placements: lane 8p+c holds tokens (p, p+8) and dims [c*D/8, (c+1)*D/8)."""
    k_off, v_off, s_idx = O.int4_page_maps(128)
    # token 9 (p=1, second of the pair), dims 18/19 (c=1, r=2): K lane 9, byte 16*9 + 8 + 1
    assert k_off[9, 9] == 16 * 9 + 8 + 1
    # V: same dims -> unit 0 of lane 9, token-pair half 1, byte 1 of the unit
    assert v_off[9, 9] == 16 * 9 + 0 + 2 + 1
    # token 3, dims 126/127 (c=7, r=14): V unit 3 of lane 31, first token, second byte
    assert v_off[3, 63] == 16 * 31 + 12 + 0 + 1
    assert s_idx[9, 1] == 16 + 2 * 1 + 1 and s_idx[3, 0] == 6


def test_int4_pages_round_trip():
    rng = np.random.default_rng(6)
    kp = rng.standard_normal((3, 16, 4, 128)).astype(np.float16)
    vp = (rng.standard_normal((3, 16, 4, 128)) * 5).astype(np.float16)
    pages = O.to_int4_pages(kp, vp)
    assert pages.shape == (3, 4, 2176)
    kc, ks, vc, vs = O.int4_pages_split(pages, 128)
    pk, sk = O.quantize_int4(kp)
    pv, sv = O.quantize_int4(vp)
    assert np.array_equal(kc, pk) and np.array_equal(vc, pv)
    assert np.array_equal(ks.reshape(-1), sk.astype(np.float16)) and np.array_equal(vs.reshape(-1), sv.astype(np.float16))
    kd, vd = O.from_int4_pages(pages, 128)
    ref = O.dequantize_int4(pk, sk.astype(np.float16).astype(np.float32))
    assert np.array_equal(kd.view(np.uint16), ref.view(np.uint16))
    kt, vt = O.dequant_pages_torch(torch.as_tensor(pages), 128)
    assert np.array_equal(kt.numpy().view(np.uint16), kd.view(np.uint16))
    assert np.array_equal(vt.numpy().view(np.uint16), vd.view(np.uint16))


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------

def brute_attention(q, kpool, vpool, bt, ctx_lens, W, sinks, causal):
    """float64 loops straight from the visibility definitions."""
    B, Lq, H, D = q.shape
    bs = kpool.shape[1]
    out = np.zeros((B, Lq, H, D))
    for b in range(B):
        ctx = int(ctx_lens[b])
        for i in range(Lq):
            pos = ctx - Lq + i
            keys = []
            for j in range(ctx):
                page = int(bt[b, j // bs])
                if page < 0:
                    continue
                if causal:
                    vis = j <= pos and (j < sinks or j >= pos - W + 1)
                else:
                    vis = j >= ctx - W or j < sinks
                if vis:
                    keys.append((page, j % bs))
            if not keys:
                continue
            for h in range(H):
                qv = q[b, i, h].astype(np.float64)
                sc = np.array([qv @ kpool[p, s, h].astype(np.float64) for p, s in keys]) / math.sqrt(D)
                w = np.exp(sc - sc.max())
                w /= w.sum()
                out[b, i, h] = sum(wk * vpool[p, s, h].astype(np.float64) for wk, (p, s) in zip(w, keys))
    return out


def _paged_case(seed, B, H, D, bs, nb, ctx, Lq):
    rng = np.random.default_rng(seed)
    kp = rng.standard_normal((nb, bs, H, D)).astype(np.float16)
    vp = rng.standard_normal((nb, bs, H, D)).astype(np.float16)
    q = rng.standard_normal((B, Lq, H, D)).astype(np.float16)
    M = (max(ctx) + bs - 1) // bs
    bt = rng.permutation(nb)[:B * M].reshape(B, M).astype(np.int32)
    return q, kp, vp, bt, np.array(ctx, np.int32)


def test_attention_paged_equals_dense_sdpa():
    """Permuted pages + full window == torch SDPA on the unpaged K/V (tests/test_attention.py:112-192)."""
    q, kp, vp, bt, cl = _paged_case(0, 2, 4, 64, 16, 20, [128, 128], 128)
    out = O.paged_attention(q, kp, vp, bt, cl, 128, 128).astype(np.float32)
    for b in range(2):
        kd = torch.as_tensor(kp[bt[b]].reshape(-1, 4, 64)).float().permute(1, 0, 2)[None]
        vd = torch.as_tensor(vp[bt[b]].reshape(-1, 4, 64)).float().permute(1, 0, 2)[None]
        qb = torch.as_tensor(q[b:b + 1]).float().permute(0, 2, 1, 3)
        ref = F.scaled_dot_product_attention(qb, kd, vd)[0].permute(1, 0, 2).half().float().numpy()
        assert np.abs(out[b] - ref).max() <= 1e-3


@pytest.mark.parametrize("W,sinks,causal,ctx,Lq", [
    (24, 0, False, [50, 37], 1),
    (24, 4, False, [50, 37], 1),
    (10, 3, False, [64, 20], 3),
    (1000, 0, True, [40, 33], 40),   # plain causal
    (12, 4, True, [48, 30], 16),     # StreamingLLM sink + window
    (1, 1, True, [20, 17], 5),
])
def test_attention_brute_force(W, sinks, causal, ctx, Lq):
    Lq = min(Lq, min(ctx))
    q, kp, vp, bt, cl = _paged_case(1, 2, 2, 64, 8, 20, ctx, Lq)
    bt[1, 1] = -1  # an unlinked page
    out = O.paged_attention(q, kp, vp, bt, cl, max_seq_len=1000, window_size=W, num_sink_tokens=sinks,
                            causal=causal).astype(np.float64)
    ref = brute_attention(q, kp, vp, bt, cl, O.effective_window(W, 1000), sinks, causal)
    assert np.abs(out - ref).max() <= 2e-3


def test_attention_causal_equals_sdpa_is_causal():
    q, kp, vp, bt, cl = _paged_case(2, 1, 2, 64, 16, 4, [64], 64)
    out = O.paged_attention(q, kp, vp, bt, cl, 64, 64, causal=True).astype(np.float32)
    kd = torch.as_tensor(kp[bt[0]].reshape(-1, 2, 64)).float().permute(1, 0, 2)[None]
    vd = torch.as_tensor(vp[bt[0]].reshape(-1, 2, 64)).float().permute(1, 0, 2)[None]
    qb = torch.as_tensor(q).float().permute(0, 2, 1, 3)
    ref = F.scaled_dot_product_attention(qb, kd, vd, is_causal=True)[0].permute(1, 0, 2).half().float().numpy()
    assert np.abs(out[0] - ref).max() <= 1e-3


def test_attention_special_cases():
    q, kp, vp, bt, cl = _paged_case(3, 1, 2, 64, 16, 4, [1], 1)
    out = O.paged_attention(q, kp, vp, bt, np.array([1], np.int32), 16, 16)
    assert np.array_equal(out[0, 0], vp[bt[0, 0], 0])            # ctx = 1 -> the V row
    bt2 = np.full_like(bt, -1)
    out2 = O.paged_attention(q, kp, vp, bt2, np.array([16], np.int32), 16, 16)
    assert (out2 == 0).all()                                       # nothing visible -> 0
    assert O.effective_window(0, 77) == 77 and O.effective_window(100, 77) == 77 and O.effective_window(5, 77) == 5


def test_sdpa_fallback_matches_sink_window_rule():
    q, kp, vp, bt, cl = _paged_case(4, 1, 2, 64, 16, 8, [100], 1)
    a = O.sdpa_fallback(q, kp, vp, bt, cl, 1 << 20, 30, 4)
    b = O.paged_attention(q, kp, vp, bt, cl, 1 << 20, 30, num_sink_tokens=4)
    assert np.array_equal(a, b)


# ---------------------------------------------------------------------------
# Eviction
# ---------------------------------------------------------------------------

def _pools(fmt, nb, bs, H, D, rng):
    kp = rng.standard_normal((nb, bs, H, D)).astype(np.float16)
    vp = rng.standard_normal((nb, bs, H, D)).astype(np.float16)
    if fmt == "fp16":
        return {"format": "fp16", "k": kp, "v": vp}
    return {"format": "int4", "pages": O.to_int4_pages(kp, vp), "D": D}


def _row(pools, p, s, h):
    """K and V rows (token s of page p, head h) as fp16 values, any pool format."""
    if pools["format"] == "fp16":
        return np.stack([pools["k"][p, s, h], pools["v"][p, s, h]])
    k, v = O.from_int4_pages(pools["pages"][p:p + 1], pools["D"])
    return np.stack([k[0, s, h], v[0, s, h]])


@pytest.mark.parametrize("fmt", ["fp16", "int4"])
@pytest.mark.parametrize("r,sinks", [(0.5, 4), (0.75, 0), (0.1, 2), (1.0, 4)])
def test_evict_intended_brute_force(fmt, r, sinks):
    rng = np.random.default_rng(7)
    N, H, L, D = 2, 3, 40, 64
    bs = 4 if fmt == "fp16" else 16
    scores = rng.lognormal(size=(N, H, L)).astype(np.float32)
    scores[0, 1, 8:12] = 1e-9  # a block fully low in one head
    pools = _pools(fmt, 24, bs, H, D, rng)
    pools0 = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in pools.items()}
    bt = rng.permutation(24)[:N * 10].reshape(N, 10).astype(np.int32)
    bt0 = bt.copy()
    free = np.zeros(24, np.int32)
    ev = O.evict_tokens_intended(scores, bt, free, r, sinks, pools, bs)
    keep = max(1, min(L, math.ceil(np.float32(r) * np.float32(L))))
    for n in range(N):
        for h in range(H):
            boosted = [1e38 if t < sinks else float(scores[n, h, t]) for t in range(L)]
            tau = sorted(boosted, reverse=True)[keep - 1]
            want = [t >= sinks and boosted[t] < tau for t in range(L)]
            assert ev[n, h].tolist() == want
            for t in range(L):
                p, s = bt0[n, t // bs], t % bs
                row = _row(pools, p, s, h)
                assert (row == 0).all() if want[t] else np.array_equal(row, _row(pools0, p, s, h))
    # votes: block (seq 0, logical block 2) is fully evicted only in head 1 -> 1 vote, still linked
    assert ((bt == -1) == (free[np.clip(bt0, 0, None)] == H)).all()


@pytest.mark.parametrize("nan_frac,r", [(0.1, 0.5), (0.6, 0.75)])
def test_evict_intended_nan_scores(nan_frac, r):
    """NaN scores (both signs) next to +-0 and +-inf. The reference selects
    and evicts by float compares (src/csrc/kv_cache.cu:757-803, :814-868),
    which a NaN never passes, so a NaN is never evicted and takes no place in
    the ranking: tau = the keep-th largest non-NaN boosted score, and nothing
    is evicted when fewer than keep scores are non-NaN (nan_frac 0.6,
    keep 75 %). Brute force over Python floats, NaN filtered by math.isnan."""
    rng = np.random.default_rng(11)
    N, H, L, D, bs, sinks = 1, 2, 64, 64, 16, 3
    scores = rng.standard_normal((N, H, L)).astype(np.float32)
    neg_nan = np.frombuffer(np.uint32(0xFFC00000).tobytes(), np.float32)[0]
    nan = rng.random((N, H, L)) < nan_frac
    scores[nan] = np.where(rng.random(int(nan.sum())) < 0.5, np.float32(np.nan), neg_nan)
    scores[0, 0, 40:44] = [np.inf, -np.inf, 0.0, -0.0]
    pools = _pools("int4", 6, bs, H, D, rng)
    bt = rng.permutation(6)[:4].reshape(1, 4).astype(np.int32)
    ev = O.evict_tokens_intended(scores, bt, np.zeros(6, np.int32), r, sinks, pools, bs)
    keep = max(1, min(L, math.ceil(np.float32(r) * np.float32(L))))
    for h in range(H):
        boosted = [1e38 if t < sinks else float(scores[0, h, t]) for t in range(L)]
        ranked = sorted((x for x in boosted if not math.isnan(x)), reverse=True)
        want = [False] * L
        if len(ranked) >= keep:
            tau = ranked[keep - 1]
            want = [t >= sinks and not math.isnan(boosted[t]) and boosted[t] < tau for t in range(L)]
        assert ev[0, h].tolist() == want
        assert not any(ev[0, h, t] for t in range(L) if math.isnan(boosted[t]))
    if nan_frac > 0.5:
        assert not ev.any()


def test_evict_intended_unlinks_fully_evicted_blocks():
    N, H, L, bs = 1, 2, 16, 4
    scores = np.ones((N, H, L), np.float32)
    scores[:, :, 4:8] = 0.0  # lowest in every head
    pools = _pools("fp16", 8, bs, H, 64, np.random.default_rng(8))
    bt = np.arange(4, dtype=np.int32)[None]
    free = np.zeros(8, np.int32)
    O.evict_tokens_intended(scores, bt, free, 0.75, 0, pools, bs)
    assert bt.tolist() == [[0, -1, 2, 3]] and free.tolist() == [0, 2, 0, 0, 0, 0, 0, 0]


@pytest.mark.parametrize("heads_b", [(0, 1), (2, 3), (0, 1, 2, 3)])
def test_evict_intended_shared_page_gets_no_votes(heads_b):
    """A page named by both sequences (prefix sharing, page 0): sequence 0
    fully evicts it in heads 0 and 1, sequence 1 in `heads_b` (overlapping,
    disjoint, all). Per-(sequence, head) votes would reach H = 4 in the
    first two cases while heads still hold live rows; a shared page gets no
    votes and stays linked in both tables. Pages of one sequence vote as
    usual: page 1 (every head) is unlinked, the others collect partial
    votes. keep = ceil(0.33 * 48) = 16, so each head keeps its 16 highest
    scores and evicts the rest."""
    N, H, L, bs = 2, 4, 48, 16
    scores = np.ones((N, H, L), np.float32)
    scores[0, :, 16:32] = 0.01                 # seq 0, page 1: lowest in every head
    scores[0, [0, 1], 0:16] = 0.1              # heads 0, 1 keep block 2, evict blocks 0, 1
    scores[0, [2, 3], 0:16] = 2.0              # heads 2, 3 keep block 0, evict blocks 1, 2
    for h in range(H):                         # seq 1: evict block 0 in heads_b, blocks 1, 2 elsewhere
        scores[1, h, 0:16] = 0.1 if h in heads_b else 2.0
    pools = _pools("fp16", 5, bs, H, 64, np.random.default_rng(3))
    bt = np.array([[0, 1, 3], [0, 2, 4]], np.int32)
    free = np.zeros(5, np.int32)
    ev = O.evict_tokens_intended(scores, bt, free, 0.33, 0, pools, bs)
    other = H - len(heads_b)
    assert bt.tolist() == [[0, -1, 3], [0, 2, 4]]
    assert free.tolist() == [0, 4, other, 2, other]
    for h in range(H):
        assert ev[0, h, :16].all() == (h in (0, 1)) and ev[1, h, :16].all() == (h in heads_b)
        # the union of both sequences' evictions is zeroed on the shared page
        assert (pools["k"][0, :, h] == 0).all() == (h in (0, 1) or h in heads_b)


def test_evict_literal_defects():
    rng = np.random.default_rng(9)
    scores = rng.lognormal(size=(2, 2, 256)).astype(np.float32)
    thr, ev = O.evict_tokens_literal(scores, num_sink_tokens=4, retain_ratio=0.5)
    assert ev.sum() == 0  # G10: 1e38 sinks pin the bisection -> nothing evicted
    thr0, ev0 = O.evict_tokens_literal(scores, num_sink_tokens=0, retain_ratio=0.5)
    kept = (~ev0).sum(axis=2)
    assert (kept >= 128).all() and (kept <= 130).all()
    assert O.literal_block_counts(np.ones(256, bool), 16).max() == 1  # G12: never reaches 16
    assert O.literal_zeroed_dims([5], 128) == {5: [5, 37, 69, 101]}  # G11: 4 of 128 dims


def test_evict_cache_brute_force():
    rng = np.random.default_rng(10)
    nb, bs, H, D = 3, 8, 2, 64
    scores = rng.standard_normal((nb, bs, H)).astype(np.float32)
    kp = rng.standard_normal((nb, bs, H, D)).astype(np.float16)
    vp = kp.copy()
    O.evict_cache(kp, vp, scores, 0.4)
    keep = int(np.float32(0.4) * np.float32(bs))
    for b in range(nb):
        for h in range(H):
            tau = sorted(scores[b, :, h].tolist(), reverse=True)[keep - 1]
            for p in range(bs):
                assert (kp[b, p, h] == 0).all() == (scores[b, p, h] < tau)


def _evict_cache_literal(row, keep):
    """The reference's selection loop, src/csrc/kv_cache.cu:436-447, step by
    step in fp32: keep times take the largest remaining score above the
    running best (starting at the -1e38 sentinel), mark it taken; the last
    best is the threshold."""
    s = [np.float32(x) for x in row]
    thr = np.float32(-1e38)
    for _ in range(keep):
        best, best_pos = np.float32(-1e38), -1
        for pos, x in enumerate(s):
            if x > best:
                best, best_pos = x, pos
        thr = best
        if best_pos >= 0:
            s[best_pos] = np.float32(-1e38)
    return [bool(np.float32(x) < thr) for x in row]


@pytest.mark.parametrize("bs,r", [(8, 0.4), (16, 0.75), (128, 0.3), (256, 0.9)])
def test_evict_cache_matches_reference_selection_loop(bs, r):
    """oracle.evict_cache against the reference's own selection loop,
    including ties, -inf and scores at or below the -1e38 sentinel."""
    rng = np.random.default_rng(bs)
    nb, H, D = 3, 2, 16
    scores = rng.standard_normal((nb, bs, H)).astype(np.float32)
    scores[0, : bs // 2, 0] = 0.5                          # ties
    scores[1, :, 0] = -np.inf                              # nothing above the sentinel
    scores[1, :3, 1] = np.float32(-1e38)                   # at the sentinel
    scores[2, : bs - 1, 1] = np.float32(-2e38)             # fewer than keep above it
    kp = rng.standard_normal((nb, bs, H, D)).astype(np.float16)
    vp = kp.copy()
    O.evict_cache(kp, vp, scores, r)
    keep = max(1, min(bs, int(np.float32(r) * np.float32(bs))))
    for b in range(nb):
        for h in range(H):
            want = _evict_cache_literal(scores[b, :, h], keep)
            got = [bool((kp[b, p, h] == 0).all()) for p in range(bs)]
            assert got == want, (b, h)


def test_division_shortcut_matches_ieee_on_fp16_domain():
    """The device quantizer replaces the per-element IEEE division v / scale by
    y = RN(1/scale), q0 = RN(v*y), r = fma(-q0, scale, v), q = fma(r, y, q0)
    (Markstein). Over every finite fp16 value and every 8th possible group
    scale (scale = RN(a / 7) for a positive fp16 absmax a), q equals the IEEE
    quotient in value, so codes are unchanged. (The full sweep over all
    31743 scales also gives 0; it takes ~8 s.)"""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    v = h[np.isfinite(h)].astype(np.float32)
    a = v[v > 0][::8]
    s = (a / np.float32(7.0)).astype(np.float32)
    assert O.markstein_mismatches(v, s) == 0


def test_group_scale_shortcut_matches_ieee_on_fp16_domain():
    """The device computes scale = RN(absmax / 7) as q0 = RN(a * RN(1/7)),
    r = fma(-q0, 7, a), q = fma(r, RN(1/7), q0). For every positive finite
    fp16 absmax this equals the IEEE quotient; a perturbed constant does not."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    a = h[np.isfinite(h)].astype(np.float32)
    a = a[a > 0]
    assert a.size == 31743
    assert O.div7_mismatches(a) == 0


def test_rounding_shortcut_matches_roundf():
    """The device rounds half away from zero as (int)(q + copysign(h, q)) with
    h = 0.5 - 2^-25. Checked for every float with 2^-3 <= |q| < 16 (both
    signs; the sweep over all |q| < 16 also gives 0, ~8 s) and a sparse sweep
    below; h = 0.5 itself fails (0.49999997 + 0.5 rounds to 1)."""
    lo, hi = int(np.float32(0.125).view(np.uint32)), int(np.float32(16.0).view(np.uint32))
    assert O.round_shortcut_mismatches(lo, hi) == 0
    for b in range(0, lo, 4099):  # sparse sweep of |q| < 1/8 (every code 8)
        assert O.round_shortcut_mismatches(b, b + 1) == 0
    assert O.round_shortcut_mismatches(lo, hi, h=0.5) > 0
    assert O.round_shortcut_mismatches(lo, hi, h=0.4999999) > 0


# ---------------------------------------------------------------------------
# Non-finite groups: the reference reduces the absmax with fmaxf, which drops
# a NaN operand (src/csrc/quantization.cu:151, :166)
# ---------------------------------------------------------------------------

def _nonfinite_groups():
    rng = np.random.default_rng(11)
    g = (rng.standard_normal((8, 64)) * 2).astype(np.float16)
    g[0, 5] = np.nan                        # one NaN among finite values
    g[1, :] = np.nan                        # all NaN
    g[2, :] = 0
    g[2, 7] = np.nan                        # NaN among zeros
    g[3, 9] = np.inf                        # +inf
    g[4, 0], g[4, 1] = -np.inf, np.nan      # -inf next to a NaN
    g[5, :] = 65504
    g[5, ::2] = -65504                      # the fp16 extremes
    g[6, 3], g[6, 4] = np.nan, 65504        # NaN next to the largest finite value
    return g


def test_quantize_nonfinite_groups_match_c_restatement():
    g = _nonfinite_groups()
    p1, s1 = O.quantize_int4(g)
    p2, s2 = O.quantize_int4_c(g)
    assert np.array_equal(p1, p2)
    assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32))


def test_quantize_nan_left_out_of_absmax():
    g = _nonfinite_groups()
    p, s = O.quantize_int4(g)
    codes = O.unpack_codes(p).reshape(-1, 64)
    finite = np.where(np.isnan(g[0]), np.float16(0), np.abs(g[0])).astype(np.float32)
    assert s[0] == np.float32(finite.max()) / np.float32(7)      # the NaN never reaches the absmax
    assert codes[0, 5] == 8                                      # (int)NaN = 0 -> code 8
    assert s[1] == 1.0 and (codes[1] == 8).all()                 # all NaN: like an all-zero group
    assert s[2] == 1.0 and (codes[2] == 8).all()
    assert np.isinf(s[3]) and (codes[3] == 8).all()              # inf scale: every quotient is 0 or NaN
    assert np.isinf(s[4]) and (codes[4] == 8).all()
    assert s[6] == np.float32(65504) / np.float32(7) and codes[6, 4] == 15 and codes[6, 3] == 8


def test_page_scale_keeps_extremes_finite():
    """Every positive finite fp16 absmax: the page scale is the RNE fp16 of
    the fp32 scale except for 65504, and 7 * page scale stays <= 65504."""
    a = np.arange(1, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    s = a / np.float32(7)
    ps = O.page_scales(s)
    assert np.array_equal(ps == s.astype(np.float16), a != 65504)
    assert ps[a == 65504] == np.float16(9352)
    assert (ps.astype(np.float32) * 7 <= 65504).all()
    k = np.zeros((1, 16, 1, 64), np.float16)
    k[0, :, 0, 0] = 65504
    k[0, 3, 0, 1] = -65504
    pages = O.to_int4_pages(k, k)
    kd, vd = O.from_int4_pages(pages, 64)
    assert np.isfinite(kd.astype(np.float32)).all() and np.isfinite(vd.astype(np.float32)).all()
    assert kd[0, 0, 0, 0] == np.float16(65464) and kd[0, 3, 0, 1] == np.float16(-65464)


def _page_k_byte(t, d, D):
    """Int4Page::k_byte (memopt-transformer-runtime_amd/csrc/page_format.hpp)."""
    dpl = D // 8
    c, r = d // dpl, d % dpl
    return (8 * (t & 7) + c) * dpl + (t >> 3) * (dpl // 2) + r // 2


def _page_v_byte(t, d, D):
    """Int4Page::v_byte."""
    dpl = D // 8
    c, r = d // dpl, d % dpl
    return (8 * (t & 7) + c) * dpl + (r // 4) * 4 + (t >> 3) * 2 + (r % 4) // 2


def _page_scale_idx(t, g):
    """Int4Page::scale_idx."""
    return g * 16 + 2 * (t & 7) + (t >> 3)


@pytest.mark.parametrize("D", [64, 128])
def test_int4_pages_per_element_loop(D):
    """to_int4_pages equals a page buffer built one element at a time from
    the page-format formulas and the exact-rational quantizer."""
    rng = np.random.default_rng(12 + D)
    nb, H, G = 2, 3, D // 64
    kp = (rng.standard_normal((nb, 16, H, D)) * np.where(rng.random((nb, 16, H, D)) < 0.01, 8, 1)).astype(np.float16)
    vp = (rng.standard_normal((nb, 16, H, D)) * 3).astype(np.float16)
    vp[1, 5, 2, :64] = 65504                      # the clamped page scale
    got = O.to_int4_pages(kp, vp)
    want = np.zeros_like(got)
    for pool, code_base, scale_base, byte in ((kp, 0, 16 * D, _page_k_byte), (vp, 8 * D, 16 * D + 32 * G, _page_v_byte)):
        for b in range(nb):
            for t in range(16):
                for h in range(H):
                    for g in range(G):
                        codes, scale = exact_quant_group(pool[b, t, h, 64 * g:64 * g + 64])
                        for i, code in enumerate(codes):
                            d = 64 * g + i
                            want[b, h, code_base + byte(t, d, D)] |= code << (4 * (d & 1))
                        sc = np.float16(float(scale))
                        if sc == np.float16(9360):
                            sc = np.float16(9352)
                        j = scale_base + 2 * _page_scale_idx(t, g)
                        want[b, h, j:j + 2] = np.frombuffer(sc.tobytes(), np.uint8)
    assert np.array_equal(got, want)


def test_write_cache_loop():
    """oracle.write_cache against a token-by-token loop of pool[slot // bs, slot % bs] = row."""
    rng = np.random.default_rng(13)
    nb, bs, H, D, T = 9, 16, 2, 64, 70
    pool = rng.standard_normal((nb, bs, H, D)).astype(np.float16)
    rows = rng.standard_normal((T, H, D)).astype(np.float16)
    slots = rng.permutation(nb * bs)[:T].astype(np.int32)
    want = pool.copy()
    for t in range(T):
        s = int(slots[t])
        for h in range(H):
            for d in range(D):
                want[s // bs, s % bs, h, d] = rows[t, h, d]
    got = pool.copy()
    O.write_cache(got, rows, slots)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("seed,B,H,D,ctx,W,sinks,unlink", [
    (0, 2, 4, 128, [300, 77], 1 << 20, 0, 0),
    (1, 3, 2, 64, [1000, 17, 256], 200, 4, 2),
    (2, 2, 2, 128, [513, 1], 64, 20, 1),
    (3, 1, 3, 64, [160], 16, 4, 10),      # every page unlinked: zeros
])
def test_decode_int4_torch_matches_composition_oracle(seed, B, H, D, ctx, W, sinks, unlink):
    """The CPU baseline's vectorized decode (bench.py times it) computes the
    composition oracle's function: windows, sinks, unlinked pages, empty sets."""
    rng = np.random.default_rng(seed)
    M = (max(ctx) + 15) // 16
    nb = B * M + 3
    kp = (rng.standard_normal((nb, 16, H, D)) * np.where(rng.random((nb, 16, H, D)) < 0.005, 10, 1)).astype(np.float16)
    vp = rng.standard_normal((nb, 16, H, D)).astype(np.float16)
    q = rng.standard_normal((B, 1, H, D)).astype(np.float16)
    bt = rng.permutation(nb)[:B * M].reshape(B, M).astype(np.int32)
    for i in range(unlink):
        bt[0, i % M] = -1
    cl = np.array(ctx, np.int32)
    pages = O.to_int4_pages(kp, vp)
    want = O.paged_attention_int4(q, pages, bt, cl, 1 << 30, W, num_sink_tokens=sinks).astype(np.float32)
    got = O.decode_int4_torch(torch.as_tensor(q), torch.as_tensor(pages), torch.as_tensor(bt), torch.as_tensor(cl),
                              min(W, 1 << 30), sinks).float().numpy()
    assert np.abs(got - want).max() <= 1e-3
