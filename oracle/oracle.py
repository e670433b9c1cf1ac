"""CPU oracle for the INT4 KV-cache data plane — TEST INFRASTRUCTURE ONLY.

This module restates, on the CPU, what TheRadDani/memopt-transformer-runtime
computes on its hot path. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import it, and only as the checker or
as the timed CPU baseline; the product path (``memopt_C``) never calls it.

Every function cites the reference file:line it follows (paths relative to
the reference repository root). Pinning status (what, besides this
restatement, fixes each function's result) is recorded per function under
"Pinned by"; the checks live in ``tests/test_oracle.py``.

Functions
---------
quantize_int4 / dequantize_int4
    src/csrc/quantization.cu:104-203 / :232-270. Pinned by: the reference's
    known answers (tests/test_quant.py:439-566), an exact rational
    (``fractions.Fraction``) evaluation of IEEE division and roundf on random
    groups, and the independent C restatement ``oracle/quant_ref.c``
    (libm ``roundf``).
to_int4_pages / from_int4_pages
    Placement of the same group-64 codes in this build's INT4 page buffer
    ([nb, H, block], block = K codes | V codes | K scales | V scales, token
    pairs interleaved for the wave64 decode kernel); scales are RNE fp16 of
    the fp32 scale (9360 stored as 9352, ``page_scales``). This format has no
    reference counterpart; pinned by the writer/reader round trip, by direct
    comparison with ``quantize_int4`` of the token-major pool, and by a
    per-element loop over ``Int4Page``'s byte formulas.
write_cache
    src/csrc/kv_cache.cu:228-260. Pinned by the invariant pool[slot] == row.
paged_attention
    src/csrc/attention.cu:158-186, :333-338, :453-460 (window, skip -1, clamp,
    empty -> 0), extended with sinks (src/memopt/triton_attention.py:523-532)
    and causal StreamingLLM masking (scripts/bench_accuracy.py:253-280).
    Pinned by: torch ``scaled_dot_product_attention`` on dense unpaged K/V
    (library routine), a float64 brute-force loop on tiny inputs, and the
    special cases ctx=1 -> V row, all pages unlinked -> 0.
evict_tokens_intended
    Exact top-k form of src/csrc/kv_cache.cu:640-1015 (sinks boosted, keep
    = clamp(ceilf(r*L), 1, L), evict score < k-th largest, full-row zeroing,
    block votes). Pinned by a brute-force ``sorted()`` selection on tiny
    inputs.
evict_tokens_literal
    Line-level fp32 restatement of src/csrc/kv_cache.cu:714-1014 including
    its defects (bisection bounds with 1e38 sinks, 1/32 zeroing, lane-0-only
    counting). Pinned by the consequences those defects force (nothing
    evicted when sinks > 0 and keep > sinks; no block ever voted).
evict_cache
    src/csrc/kv_cache.cu:379-483. Pinned by brute-force selection.
"""
from __future__ import annotations

import ctypes
import math
import os
from typing import Optional, Tuple

import numpy as np

GROUP = 64
_HERE = os.path.dirname(os.path.abspath(__file__))


# ---------------------------------------------------------------------------
# Quantization — src/csrc/quantization.cu:104-270
# ---------------------------------------------------------------------------

def _roundf(x: np.ndarray) -> np.ndarray:
    """C ``roundf`` (half away from zero) on float32, exact.

    ``x + 0.5`` would round in fp32; ``x - trunc(x)`` is exact for |x| < 2^23.
    """
    x = np.asarray(x, dtype=np.float32)
    t = np.trunc(x)
    frac = np.abs(x - t)
    return (t + np.sign(x) * (frac >= np.float32(0.5))).astype(np.float32)


def quantize_int4(cache: np.ndarray, group_size: int = GROUP) -> Tuple[np.ndarray, np.ndarray]:
    """Group-wise symmetric INT4 quantization, bit-exact with the reference kernel.

    Follows src/csrc/quantization.cu:129-202: per 64 consecutive elements of
    the flattened tensor, ``scale = absmax > 0 ? absmax / 7 : 1`` in IEEE fp32
    (:166-168), ``code = clamp((int)roundf(v / scale) + 8, 0, 15)`` (:183-186),
    ``byte = code[2i] | code[2i+1] << 4`` (:198-200). NaN elements are left
    out of the absmax (fmaxf) and get code 8 ((int)NaN = 0 on the device).

    Returns (packed uint8 with last dim halved, scales float32 [numel/64]).
    """
    assert group_size == GROUP
    c = np.ascontiguousarray(cache)
    assert c.dtype == np.float16 and c.size % GROUP == 0 and c.shape[-1] % 2 == 0
    g = c.reshape(-1, GROUP).astype(np.float32)
    # fmaxf drops a NaN operand (quantization.cu:151, :166), so NaN elements
    # never reach the absmax; an all-NaN group reduces to NaN, and NaN > 0 is
    # false, which gives scale 1.0 like an all-zero group.
    absmax = np.fmax.reduce(np.abs(g), axis=1)
    with np.errstate(invalid="ignore"):
        scale = np.where(absmax > 0, absmax / np.float32(7.0), np.float32(1.0)).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        q = g / scale[:, None]
    r = _roundf(q)
    r = np.where(np.isnan(r), 0, r)  # (int)NaN -> 0 on both ISAs
    codes = np.clip(r.astype(np.int64) + 8, 0, 15).astype(np.uint8)
    codes = codes.reshape(-1, 2)
    packed = (codes[:, 0] | (codes[:, 1] << 4)).astype(np.uint8)
    return packed.reshape(c.shape[:-1] + (c.shape[-1] // 2,)), scale


def unpack_codes(packed: np.ndarray) -> np.ndarray:
    """Nibble codes in element order: element 2i = low nibble, 2i+1 = high."""
    p = np.asarray(packed, dtype=np.uint8).reshape(-1)
    out = np.empty(p.size * 2, dtype=np.uint8)
    out[0::2] = p & 0xF
    out[1::2] = p >> 4
    return out


def dequantize_int4(packed: np.ndarray, scales: np.ndarray, group_size: int = GROUP) -> np.ndarray:
    """fp16(RNE(float(code - 8) * scale)) — src/csrc/quantization.cu:254-268.

    ``scales`` may be float32 (surface) or float16 (INT4 pages); either way
    the product is formed in fp32 and rounded once to fp32, then to fp16.
    """
    assert group_size == GROUP
    codes = unpack_codes(packed).astype(np.float32) - np.float32(8.0)
    s = np.asarray(scales).astype(np.float32).reshape(-1)
    with np.errstate(invalid="ignore"):  # code 8 under an inf scale: 0 * inf = NaN, as on the device
        vals = (codes.reshape(-1, GROUP) * s[:, None]).astype(np.float32)
    shape = tuple(packed.shape[:-1]) + (packed.shape[-1] * 2,)
    return vals.astype(np.float16).reshape(shape)


# ---------------------------------------------------------------------------
# C restatement (oracle/quant_ref.c) — independent check of the rounding
# ---------------------------------------------------------------------------

_CLIB = None


def _clib():
    global _CLIB
    if _CLIB is None:
        path = os.path.join(_HERE, "_build", "liboracle_quant.so")
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        lib = ctypes.CDLL(path)
        lib.oracle_quantize_int4.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
        lib.oracle_quantize_int4.restype = None
        lib.oracle_dequantize_int4.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
        lib.oracle_dequantize_int4.restype = None
        lib.oracle_markstein_mismatches.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64]
        lib.oracle_markstein_mismatches.restype = ctypes.c_int64
        lib.oracle_div7_mismatches.argtypes = [ctypes.c_void_p, ctypes.c_int64]
        lib.oracle_div7_mismatches.restype = ctypes.c_int64
        lib.oracle_round_shortcut_mismatches.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float]
        lib.oracle_round_shortcut_mismatches.restype = ctypes.c_int64
        _CLIB = lib
    return _CLIB


def quantize_int4_c(cache: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Same contract as :func:`quantize_int4`, computed by oracle/quant_ref.c."""
    c = np.ascontiguousarray(cache, dtype=np.float16)
    f = np.ascontiguousarray(c.astype(np.float32).reshape(-1))
    packed = np.empty(f.size // 2, dtype=np.uint8)
    scales = np.empty(f.size // GROUP, dtype=np.float32)
    _clib().oracle_quantize_int4(f.ctypes.data, f.size // GROUP, packed.ctypes.data, scales.ctypes.data)
    return packed.reshape(c.shape[:-1] + (c.shape[-1] // 2,)), scales


def dequantize_int4_c(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Same contract as :func:`dequantize_int4` (fp32 scales), computed in C."""
    p = np.ascontiguousarray(packed, dtype=np.uint8).reshape(-1)
    s = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
    out = np.empty(p.size * 2, dtype=np.float32)
    _clib().oracle_dequantize_int4(p.ctypes.data, s.ctypes.data, s.size, out.ctypes.data)
    shape = tuple(packed.shape[:-1]) + (packed.shape[-1] * 2,)
    return out.astype(np.float16).reshape(shape)


def markstein_mismatches(values: np.ndarray, scales: np.ndarray) -> int:
    """Checker of the device quantizer's division shortcut (oracle/quant_ref.c):
    number of (v, s) pairs, |v| <= 7 s, whose fma-refined quotient differs
    from the IEEE quotient v / s in value."""
    v = np.ascontiguousarray(values, dtype=np.float32)
    sc = np.ascontiguousarray(scales, dtype=np.float32)
    return int(_clib().oracle_markstein_mismatches(v.ctypes.data, v.size, sc.ctypes.data, sc.size))


def div7_mismatches(absmax: np.ndarray) -> int:
    """Checker of the device's group-scale shortcut (oracle/quant_ref.c):
    number of positive a whose constant-reciprocal Markstein quotient differs
    from the IEEE quotient a / 7."""
    a = np.ascontiguousarray(absmax, dtype=np.float32)
    return int(_clib().oracle_div7_mismatches(a.ctypes.data, a.size))


def round_shortcut_mismatches(lo_bits: int, hi_bits: int, h: float = 0.49999997) -> int:
    """Checker of the device's rounding shortcut (oracle/quant_ref.c): number
    of floats +-q, bit patterns of |q| in [lo_bits, hi_bits), for which
    (int)(q + copysign(h, q)) differs from roundf(q)."""
    return int(_clib().oracle_round_shortcut_mismatches(lo_bits, hi_bits, h))


# ---------------------------------------------------------------------------
# INT4 page format of this build
# ---------------------------------------------------------------------------

PAGE_TOKENS = 16


def int4_block_bytes(D: int) -> int:
    """Bytes per (page, head) block: K codes 8D | V codes 8D | K scales 32G | V scales 32G."""
    return 16 * D + 64 * (D // GROUP)


def int4_page_maps(D: int):
    """Byte offsets inside a block for the code byte of (token t, dims 2j..2j+1)
    of K and of V, and fp16 indices of the (token, group) scales.

    Layout (one wave64 reads a block; lane 8p+c owns tokens p and p+8 and the
    D/8 dims starting at c*D/8, i.e. BPL = D/8 bytes of each code region):
      K byte = lane*BPL + (t // 8)*(BPL/2) + r/2           (r = dim offset in the lane chunk)
      V byte = lane*BPL + (r // 4)*4 + (t // 8)*2 + (r % 4)//2   (4-dim units, tokens interleaved)
      scale  = g*16 + 2*(t % 8) + t // 8
    Returns (k_off [16, D/2], v_off [16, D/2], s_idx [16, D/64]).
    """
    dpl = bpl = D // 8
    t = np.arange(PAGE_TOKENS)[:, None]
    d = np.arange(0, D, 2)[None, :]
    c, r = d // dpl, d % dpl
    lane = 8 * (t % 8) + c
    k_off = lane * bpl + (t // 8) * (bpl // 2) + r // 2
    v_off = lane * bpl + (r // 4) * 4 + (t // 8) * 2 + (r % 4) // 2
    g = np.arange(D // GROUP)[None, :]
    s_idx = g * 16 + 2 * (t % 8) + t // 8
    return k_off, v_off, s_idx


def page_scales(scales: np.ndarray) -> np.ndarray:
    """fp16 scales stored in INT4 pages: RNE fp16 of the fp32 scale, except
    9360 (= RNE(65504 / 7), the scale of a group whose absmax is 65504), which
    is stored as 9352 so that 7 * scale, the largest dequantized magnitude,
    stays finite in fp16 (7 * 9360 = 65520 rounds to inf)."""
    sc = np.asarray(scales, dtype=np.float32).astype(np.float16)
    return np.where(sc == np.float16(9360.0), np.float16(9352.0), sc)


def to_int4_pages(k_pool: np.ndarray, v_pool: np.ndarray) -> np.ndarray:
    """fp16 pools [nb, 16, H, D] (K, V) -> INT4 page buffer u8 [nb, H, block].

    Codes are the reference's group-64 codes of the token-major pools
    (src/csrc/quantization.cu:115-116 on a contiguous [nb, bs, H, D] tensor:
    groups = (page, token, head, 64-dim chunk)); scales are stored as
    :func:`page_scales` of the fp32 scale.
    """
    nb, bs, H, D = k_pool.shape
    assert bs == PAGE_TOKENS and D % GROUP == 0
    G = D // GROUP
    k_off, v_off, s_idx = int4_page_maps(D)
    out = np.zeros((nb, H, int4_block_bytes(D)), np.uint8)
    for pool, code_base, scale_base, off in ((k_pool, 0, 16 * D, k_off), (v_pool, 8 * D, 16 * D + 32 * G, v_off)):
        packed, scales = quantize_int4(pool)
        codes = packed.reshape(nb, bs, H, D // 2).transpose(0, 2, 1, 3)          # [nb, H, t, j]
        out[:, :, code_base + off.reshape(-1)] = codes.reshape(nb, H, -1)
        sc = page_scales(scales.reshape(nb, bs, H, G).transpose(0, 2, 1, 3))  # [nb, H, t, g]
        sb = sc.view(np.uint8).reshape(nb, H, bs, G, 2)
        idx = scale_base + 2 * s_idx
        out[:, :, idx.reshape(-1)] = sb[..., 0].reshape(nb, H, -1)
        out[:, :, idx.reshape(-1) + 1] = sb[..., 1].reshape(nb, H, -1)
    return out


def int4_pages_split(pages: np.ndarray, D: int):
    """Page buffer -> (K codes, K fp16 scales, V codes, V fp16 scales) in the
    reference's token-major order: codes [nb, 16, H, D/2], scales [nb, 16, H, D/64]."""
    nb, H, blk = pages.shape
    G = D // GROUP
    k_off, v_off, s_idx = int4_page_maps(D)
    res = []
    for code_base, scale_base, off in ((0, 16 * D, k_off), (8 * D, 16 * D + 32 * G, v_off)):
        codes = pages[:, :, code_base + off.reshape(-1)].reshape(nb, H, PAGE_TOKENS, D // 2)
        idx = (scale_base + 2 * s_idx).reshape(-1)
        sb = np.stack((pages[:, :, idx], pages[:, :, idx + 1]), axis=-1).reshape(nb, H, PAGE_TOKENS, G, 2)
        sc = np.ascontiguousarray(sb).view(np.float16).reshape(nb, H, PAGE_TOKENS, G)
        res += [codes.transpose(0, 2, 1, 3).copy(), sc.transpose(0, 2, 1, 3).copy()]
    return tuple(res)


def from_int4_pages(pages: np.ndarray, D: int):
    """Dequantize an INT4 page buffer back to fp16 pools (K, V) [nb, 16, H, D]."""
    kc, ks, vc, vs = int4_pages_split(pages, D)
    return dequantize_int4(kc, ks), dequantize_int4(vc, vs)


# ---------------------------------------------------------------------------
# write_cache — src/csrc/kv_cache.cu:228-260
# ---------------------------------------------------------------------------

def write_cache(pool: np.ndarray, rows: np.ndarray, slot_mapping: np.ndarray) -> None:
    """pool[slot // bs, slot % bs] = rows[t] (in place)."""
    nb, bs = pool.shape[:2]
    s = np.asarray(slot_mapping, dtype=np.int64)
    pool[s // bs, s % bs] = rows


# ---------------------------------------------------------------------------
# Paged attention — src/csrc/attention.cu:98-339 (+ sinks, causal)
# ---------------------------------------------------------------------------

def effective_window(window_size: int, max_seq_len: int) -> int:
    """src/csrc/attention.cu:453-455."""
    if window_size <= 0 or window_size > max_seq_len:
        return max_seq_len
    return window_size


def visible_mask(ctx: int, q_len: int, window: int, sinks: int, causal: bool) -> np.ndarray:
    """Boolean [q_len, ctx]: which keys each query sees.

    Non-causal (src/csrc/attention.cu:158-186): j in [max(0, ctx-W), ctx)
    for every query, plus sinks j < min(sinks, ctx)
    (src/memopt/triton_attention.py:523-532).
    Causal (scripts/bench_accuracy.py:271-275): query i sits at absolute
    position p = ctx - q_len + i; j <= p and (j < sinks or j >= p - W + 1).
    """
    j = np.arange(ctx)[None, :]
    if causal:
        p = (ctx - q_len + np.arange(q_len))[:, None]
        return (j <= p) & ((j < sinks) | (j >= p - window + 1))
    m = (j >= max(0, ctx - window)) | (j < sinks)
    return np.broadcast_to(m, (q_len, ctx)).copy()


def paged_attention(query, key_cache, value_cache, block_tables, context_lens,
                    max_seq_len: int, window_size: int, num_sink_tokens: int = 0,
                    causal: bool = False):
    """fp32 SDPA over gathered pages, cast to fp16 (torch CPU).

    query fp16 [B, Lq, H, D]; key/value_cache fp16 [nb, bs, H, D];
    block_tables int32 [B, M]; context_lens int32 [B]. Pages with a negative
    entry contribute no keys (src/csrc/attention.cu:173); a query with no
    visible key outputs 0 (:333-334). Scale 1/sqrtf(D) (:460).
    """
    import torch
    import torch.nn.functional as F

    q = torch.as_tensor(np.asarray(query)).float()
    kc = torch.as_tensor(np.asarray(key_cache))
    vc = torch.as_tensor(np.asarray(value_cache))
    bt = np.asarray(block_tables)
    cl = np.asarray(context_lens)
    B, Lq, H, D = q.shape
    bs = kc.shape[1]
    W = effective_window(window_size, max_seq_len)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    out = torch.zeros(B, Lq, H, D, dtype=torch.float32)
    for b in range(B):
        ctx = int(cl[b])
        if ctx <= 0:
            continue
        nblk = (ctx + bs - 1) // bs
        phys = bt[b, :nblk].astype(np.int64)
        tok_ok = np.repeat(phys >= 0, bs)[:ctx]
        idx = np.clip(phys, 0, None)
        kd = kc[torch.as_tensor(idx)].reshape(nblk * bs, H, D)[:ctx].float()
        vd = vc[torch.as_tensor(idx)].reshape(nblk * bs, H, D)[:ctx].float()
        vis = visible_mask(ctx, Lq, W, num_sink_tokens, causal) & tok_ok[None, :]
        keep_cols = np.nonzero(vis.any(axis=0))[0]
        if keep_cols.size == 0:
            continue
        kd = kd[torch.as_tensor(keep_cols)].permute(1, 0, 2)[None]
        vd = vd[torch.as_tensor(keep_cols)].permute(1, 0, 2)[None]
        m = torch.as_tensor(vis[:, keep_cols])
        qb = q[b:b + 1].permute(0, 2, 1, 3)
        o = F.scaled_dot_product_attention(qb, kd, vd, attn_mask=m[None, None], scale=scale)
        o = torch.nan_to_num(o, nan=0.0)
        o[:, :, ~m.any(dim=1)] = 0.0
        out[b] = o[0].permute(1, 0, 2)
    return out.to(torch.float16).numpy()


def paged_attention_int4(query, pages, block_tables, context_lens, max_seq_len, window_size,
                         num_sink_tokens=0, causal=False):
    """Composition oracle of the fused INT4 path on an INT4 page buffer (the
    reference has no fused INT4 attention; its INT4 path is
    dequantize_kv_cache_int4 followed by dynamic_sparse_attention,
    src/csrc/quantization.cu:371-428 and src/csrc/attention.cu:371)."""
    kp, vp = from_int4_pages(pages, query.shape[-1])
    return paged_attention(query, kp, vp, block_tables, context_lens, max_seq_len,
                           window_size, num_sink_tokens, causal)


def sdpa_fallback(query, key_cache, value_cache, block_tables, context_lens,
                  max_seq_len, window_size, num_sink_tokens=4):
    """Restatement of the reference's CPU path, src/memopt/triton_attention.py:473-550.

    Differences kept explicit: a -1 page is skipped here (the reference
    indexes the last page through Python's negative index, :514-516), and
    windowing applies only when ``window_size < max_seq_len and ctx > W``
    (:523). For bt >= 0 and W < max_seq_len this equals
    ``paged_attention(..., num_sink_tokens=s)``.
    """
    W = window_size if (window_size < max_seq_len) else 1 << 30
    return paged_attention(query, key_cache, value_cache, block_tables, context_lens,
                           1 << 30, W, num_sink_tokens if W < (1 << 30) else 0, False)


# ---------------------------------------------------------------------------
# Eviction — src/csrc/kv_cache.cu:379-483 and :640-1015
# ---------------------------------------------------------------------------

def keep_count(retain_ratio: float, L: int) -> int:
    """src/csrc/kv_cache.cu:754-755: clamp((int)ceilf(r * (float)L), 1, L) in fp32."""
    v = np.float32(retain_ratio) * np.float32(L)
    return max(1, min(L, int(np.ceil(v))))


def _zero_row(pools, phys: int, pos: int, head: int) -> None:
    """Zero one (token, head) row of K and V in every pool format. fp16: zeros.
    INT4 pages: the row's K and V group scales set to 0 with its codes kept,
    so every element dequantizes to (code - 8) * 0 = 0 (-0 for codes below 8)
    and attention sees a zeroed row (this build's representation; the
    reference zeroes fp16 rows only, src/csrc/kv_cache.cu:937-973)."""
    if pools["format"] == "fp16":
        pools["k"][phys, pos, head, :] = 0
        pools["v"][phys, pos, head, :] = 0
    else:
        D = pools["D"]
        G = D // GROUP
        _, _, s_idx = int4_page_maps(D)
        blk = pools["pages"][phys, head]
        for base in (16 * D, 16 * D + 32 * G):
            for g in range(G):
                i = base + 2 * s_idx[pos, g]
                blk[i], blk[i + 1] = 0, 0


def evict_tokens_intended(scores, block_tables, is_block_free, retain_ratio,
                          num_sink_tokens, pools, block_size):
    """Exact-top-k eviction (the reference's documented intent, src/csrc/kv_cache.cu:565-607).

    Per (seq, head): sink scores := 1e38 (:722-726); keep = keep_count;
    tau = keep-th largest boosted score; tokens with boosted score < tau are
    evicted (ties at tau kept; a NaN score, of either sign, is sorted after
    every number and fails s < tau: it takes no rank and is never evicted,
    as under the reference's float compares, :757-803, :814-868); every evicted (token, head) row is zeroed
    (fp16: zeros; INT4 pages: its scales set to 0, see _zero_row); pools = {"format": "fp16", "k", "v"} or
    {"format": "int4", "pages", "D"}. A logical block whose block_size positions are all
    evicted in this head votes is_block_free[phys] += 1; the vote that
    reaches H sets block_tables[seq, lb] = -1 (:993-1014).
    A physical page named by two or more live entries (lb < ceil(L / bs),
    page inside the pool) is shared between sequences, a case the reference
    never meets: it gets the union of the rows' evictions and no votes, so
    it is never unlinked or counted free (per-(seq, head) votes from two
    sequences could otherwise reach H while heads still hold live rows).
    Mutates block_tables, is_block_free and pools in place; returns the
    evicted mask [N, H, L].
    """
    s = np.array(scores, dtype=np.float32)
    N, H, L = s.shape
    ns = min(max(num_sink_tokens, 0), L)
    s[:, :, :ns] = np.float32(1e38)
    k = keep_count(retain_ratio, L)
    tau = -np.sort(-s, axis=2)[:, :, k - 1]
    evicted = s < tau[:, :, None]
    evicted[:, :, :ns] = False  # sinks are structurally protected
    M = block_tables.shape[1]
    nlb = (L + block_size - 1) // block_size
    bt0 = block_tables.copy()
    live = bt0[:, :min(nlb, M)].ravel()
    live = live[(live >= 0) & (live < is_block_free.shape[0])]
    pages, counts = np.unique(live, return_counts=True)
    shared = set(int(x) for x in pages[counts > 1])
    votes = []
    for n in range(N):
        for h in range(H):
            for t in np.nonzero(evicted[n, h])[0]:
                lb, pos = divmod(int(t), block_size)
                if lb >= M:
                    continue
                p = int(bt0[n, lb])
                if 0 <= p < is_block_free.shape[0]:
                    _zero_row(pools, p, pos, h)
            for lb in range(min(nlb, M)):
                t0, t1 = lb * block_size, min(L, (lb + 1) * block_size)
                if t1 - t0 == block_size and evicted[n, h, t0:t1].all():
                    p = int(bt0[n, lb])
                    if 0 <= p < is_block_free.shape[0] and p not in shared:
                        votes.append((n, lb, p))
    for n, lb, p in votes:
        is_block_free[p] += 1
        if is_block_free[p] == H:
            block_tables[n, lb] = -1
    return evicted


def evict_tokens_literal(scores, num_sink_tokens, retain_ratio, L_cap=4096):
    """Line-level restatement of the reference threshold search, src/csrc/kv_cache.cu:714-870.

    Returns (threshold [N, H] fp32, evicted [N, H, L]) exactly as the kernel
    computes them: sinks := 1e38, min/max bounds, 32 fp32 bisection steps on
    count(score >= mid) >= keep, evict score < lo. The zeroing/vote stages
    of the kernel (:937-1014) touch only dims d == lane (mod 32) of each
    evicted token and count at most one token per 32-token run; see
    :func:`literal_zeroed_dims` / :func:`literal_block_counts`.
    """
    s = np.array(scores, dtype=np.float32)
    N, H, L = s.shape
    assert L <= L_cap, "the reference rejects seq_len > 4096 (src/csrc/kv_cache.cu:1085)"
    s[:, :, :min(num_sink_tokens, L)] = np.float32(1e38)
    keep = keep_count(retain_ratio, L)
    thr = np.empty((N, H), dtype=np.float32)
    for n in range(N):
        for h in range(H):
            row = s[n, h]
            gmin, gmax = np.float32(row.min()), np.float32(row.max())
            if gmin >= gmax:
                thr[n, h] = np.float32(gmin - np.float32(1.0))
                continue
            lo, hi = gmin, gmax
            for _ in range(32):
                mid = np.float32(lo + np.float32(np.float32(hi - lo) * np.float32(0.5)))
                if int((row >= mid).sum()) >= keep:
                    lo = mid
                else:
                    hi = mid
            thr[n, h] = lo
    return thr, s < thr[:, :, None]


def literal_zeroed_dims(evicted_tokens: np.ndarray, head_dim: int):
    """Dims the reference zeroes for each evicted token t: d == t % 32 (mod 32)
    (src/csrc/kv_cache.cu:937-973: lane l handles token base+l and zeroes
    d = l, l+32, ...)."""
    return {int(t): list(range(int(t) % 32, head_dim, 32)) for t in evicted_tokens}


def literal_block_counts(evicted_row: np.ndarray, block_size: int) -> np.ndarray:
    """Per-logical-block count as the reference accumulates it: only lane 0 of
    each 32-token run counts (src/csrc/kv_cache.cu:978-980)."""
    L = evicted_row.size
    cnt = np.zeros((L + block_size - 1) // block_size, dtype=np.int64)
    for t in range(0, L, 32):
        if evicted_row[t]:
            cnt[t // block_size] += 1
    return cnt


def evict_cache(key_pool, value_pool, scores, retain_ratio):
    """src/csrc/kv_cache.cu:379-483: per (block, head) keep = max(1,
    (int)(r * bs)) (truncation, :426). The reference selects keep times the
    largest remaining score strictly above -1e38 (:436-447, its sentinel), so
    the threshold is the keep-th largest of the scores above -1e38, or -1e38
    itself when fewer than keep scores exceed it; positions with score <
    threshold are zeroed (:466-480). In place."""
    nb, bs, H = scores.shape
    keep = max(1, min(bs, int(np.float32(retain_ratio) * np.float32(bs))))
    floor = np.float32(-1e38)
    for b in range(nb):
        for h in range(H):
            row = scores[b, :, h].astype(np.float32)
            above = row[row > floor]
            thr = np.sort(above)[::-1][keep - 1] if above.size >= keep else floor
            for pos in np.nonzero(row < thr)[0]:
                key_pool[b, pos, h, :] = 0
                value_pool[b, pos, h, :] = 0


# ---------------------------------------------------------------------------
# Seeded inputs (CPU generator, fixed draw order)
# ---------------------------------------------------------------------------

def outlier_normal(gen, shape, frac: float, mult: float, std: float = 1.0):
    """x ~ N(0, std); a `frac` fraction scaled by `mult`; cast to fp16."""
    import torch
    x = torch.randn(shape, generator=gen) * std
    m = torch.rand(shape, generator=gen) < frac
    x[m] *= mult
    return x.half().numpy()


# ---------------------------------------------------------------------------
# Vectorized torch-CPU form of the INT4 decode path (CPU baseline timing)
# ---------------------------------------------------------------------------

def dequant_pages_torch(pages, D):
    """torch: INT4 page blocks [n, H, block] u8 -> fp16 (K, V) [n, 16, H, D];
    same values as :func:`from_int4_pages` (works on CPU or GPU tensors)."""
    import torch
    n, H, _ = pages.shape
    G = D // GROUP
    k_off, v_off, s_idx = (torch.as_tensor(a, device=pages.device) for a in int4_page_maps(D))
    outs = []
    for code_base, scale_base, off in ((0, 16 * D, k_off), (8 * D, 16 * D + 32 * G, v_off)):
        b = pages[:, :, code_base + off.reshape(-1)].reshape(n, H, PAGE_TOKENS, D // 2).to(torch.int16)
        vals = torch.stack(((b & 0xF) - 8, (b >> 4) - 8), dim=-1).reshape(n, H, PAGE_TOKENS, D).float()
        idx = (scale_base + 2 * s_idx).reshape(-1)
        sb = torch.stack((pages[:, :, idx], pages[:, :, idx + 1]), dim=-1).contiguous()
        sc = sb.view(torch.float16).reshape(n, H, PAGE_TOKENS, G).float().repeat_interleave(GROUP, dim=-1)
        outs.append((vals * sc).half().permute(0, 2, 1, 3).contiguous())
    return outs[0], outs[1]


def decode_int4_torch(q, pages, block_tables, context_lens, window, sinks):
    """The reference's CPU path for one decode step over INT4 pages (dequantize,
    gather, sinks U window selection, fp32 SDPA, fp16 cast — the torch-only
    route of src/memopt/triton_attention.py:473-550 after
    src/csrc/quantization.cu:232-270), vectorized per sequence. torch CPU
    tensors in, fp16 [B, 1, H, D] out. Pages with a block-table entry < 0
    contribute no keys, and a sequence with no visible key outputs 0, as in
    :func:`paged_attention`."""
    import torch
    import torch.nn.functional as F
    B, _, H, D = q.shape
    out = torch.zeros(B, 1, H, D, dtype=torch.float16)
    for b in range(B):
        ctx = int(context_lens[b])
        pg = block_tables[b, : (ctx + PAGE_TOKENS - 1) // PAGE_TOKENS].long()
        k, v = dequant_pages_torch(pages[pg.clamp(min=0)], D)
        k, v = k.reshape(-1, H, D)[:ctx], v.reshape(-1, H, D)[:ctx]
        j = torch.arange(ctx)
        keep = ((j >= ctx - window) | (j < sinks)) & (pg >= 0).repeat_interleave(PAGE_TOKENS)[:ctx]
        if not bool(keep.any()):
            continue
        k, v = k[keep].float().permute(1, 0, 2)[None], v[keep].float().permute(1, 0, 2)[None]
        o = F.scaled_dot_product_attention(q[b:b + 1].float().permute(0, 2, 1, 3), k, v,
                                           scale=float(np.float32(1.0) / np.sqrt(np.float32(D))))
        out[b] = o[0].permute(1, 0, 2).half()
    return out
