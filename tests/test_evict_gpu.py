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
    # 1024-thread kernel with keys in registers (L <= 32768), then the long-row
    # kernels (one workgroup per 65536-token span: sample bracket, classify,
    # resolve by the row's last span; then the apply): one span, two spans
    # with a 1-token second span, an unaligned row (L % 4 == 3) over two spans
    (1, 2, 20000, 16, 0.75, 4), (1, 2, 40000, 16, 0.6, 4), (1, 1, 40001, 16, 0.5, 3),
    (2, 3, 65536, 16, 0.75, 4), (1, 2, 33000, 32, 0.9, 0), (1, 2, 65537, 16, 0.75, 4),
    (1, 1, 131071, 16, 0.6, 5)])
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


@pytest.mark.parametrize("L", [40000, 40001, 131072])
def test_evict_tokens_long_rows_many_ties(L):
    """Long rows whose sample bracket holds far more tokens than the
    candidate lists (scores take 4 values): the row's resolving workgroup
    falls back to an exact select over the whole row and rewrites the
    bitmask (one span, and two spans)."""
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


def _evict_case(fmt, N, H, L, D, r, sinks, scores, bt=None, seed=0, extra_pages=2):
    """Fill a pool, evict on the GPU and with the oracle from the same state;
    pages, block tables and votes must agree bit for bit."""
    rng = np.random.default_rng(seed)
    bs = 16
    M = (L + bs - 1) // bs
    nb = N * M + extra_pages
    memopt_C.init_pool(nb, bs, H, D, kv_format=fmt)
    T = nb * bs
    k = rng.standard_normal((T, H, D)).astype(np.float16)
    v = rng.standard_normal((T, H, D)).astype(np.float16)
    memopt_C.write_cache(to_dev(k), to_dev(v), to_dev(np.zeros((1, 1), np.int32)),
                         to_dev(np.arange(T, dtype=np.int32)))
    if bt is None:
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


@pytest.mark.parametrize("order", ["ascending", "descending", "blocks"])
def test_evict_tokens_long_rows_ordered_scores(order):
    """Scores that depend on the position (sorted either way, or constant per
    64-token run): the sample bracket is stratified over the row and the
    result must not depend on how representative it is."""
    rng = np.random.default_rng(7)
    N, H, L = 1, 2, 50000
    s = np.sort(rng.lognormal(size=(N, H, L)).astype(np.float32), axis=-1)
    if order == "descending":
        s = s[:, :, ::-1].copy()
    elif order == "blocks":
        s = np.repeat(rng.lognormal(size=(N, H, (L + 63) // 64)).astype(np.float32), 64, axis=-1)[:, :, :L].copy()
    _evict_case("int4", N, H, L, 64, 0.7, 4, s)


def test_evict_tokens_longest_row():
    """One row of 2^19 tokens: 8 spans, and more bracket candidates (about
    21K) than the resolving workgroup holds in LDS, so the select reads the
    spans' candidate lists from memory. INT4 pool."""
    rng = np.random.default_rng(19)
    L = 1 << 19
    s = rng.lognormal(size=(1, 1, L)).astype(np.float32)
    _evict_case("int4", 1, 1, L, 64, 0.75, 4, s, extra_pages=1)


def test_evict_tokens_long_rows_clustered_candidates():
    """Candidates concentrated in the tokens one wave of the classify
    kernel reads (positions p with p % 4096 < 256 hold scores within 1e-3
    of 1, tau falls among them): that wave's candidate list overflows, and
    the resolve selects over the whole row instead of the spans' lists."""
    rng = np.random.default_rng(31)
    N, H, L = 1, 2, 70000
    s = np.empty((N, H, L), np.float32)
    pos = np.arange(L)
    cl = (pos % 4096) < 256
    for h in range(H):
        hi_mask = rng.random(L) < 0.5
        s[0, h] = np.where(hi_mask, rng.uniform(2, 10, L), rng.uniform(0.01, 0.5, L))
        s[0, h, cl] = 1.0 + rng.uniform(-1e-3, 1e-3, cl.sum())
    n_hi = int(((s[0, 0] > 1.5) & ~cl).sum())
    r = (n_hi + cl.sum() / 2 + 4) / L
    _evict_case("int4", N, H, L, 64, float(r), 4, s)


@pytest.mark.parametrize("L", [8192, 70000])
def test_evict_tokens_signed_zero_ties(L):
    """Scores of +0 and -0 (6 % of each row, random signs) between
    negative and positive scores, keep = half the row: tau is a zero, and
    +0 and -0 tie as in float compares (neither is evicted, the negative
    scores are). Short rows (one workgroup) and long rows (the bracket
    lands on the zeros: candidate lists and the resolve)."""
    rng = np.random.default_rng(L + 3)
    N, H = 1, 2
    s = rng.lognormal(size=(N, H, L)).astype(np.float32)
    neg = rng.random((N, H, L)) < 0.48
    s[neg] = -s[neg]
    zero = rng.random((N, H, L)) < 0.06
    s[zero] = np.where(rng.random(int(zero.sum())) < 0.5, np.float32(0.0), np.float32(-0.0))
    _evict_case("int4", N, H, L, 64, 0.5, 4, s)


@pytest.mark.parametrize("kind", ["scattered", "mostly_nan"])
@pytest.mark.parametrize("fmt,L", [("int4", 5000), ("fp16", 5000), ("int4", 70000), ("fp16", 40000)])
def test_evict_tokens_nan_scores(fmt, L, kind):
    """NaN scores of both signs, with +-0 and +-inf beside them: a NaN is
    never evicted and takes no place in the ranking, as under the
    reference's float compares (scattered: 1 % NaN, keep 75 %). mostly_nan:
    40 % NaN and keep 70 %, fewer non-NaN scores than keep, so nothing is
    evicted. Short rows (one workgroup) and long rows (a NaN becomes a
    candidate; the resolve and its whole-row select leave it in place)."""
    rng = np.random.default_rng(L + (7 if kind == "scattered" else 9))
    N, H = 1, 2
    s = rng.standard_normal((N, H, L)).astype(np.float32)
    nan = rng.random((N, H, L)) < (0.01 if kind == "scattered" else 0.4)
    neg_nan = np.frombuffer(np.uint32(0xFFC00000).tobytes(), np.float32)[0]
    s[nan] = np.where(rng.random(int(nan.sum())) < 0.5, np.float32(np.nan), neg_nan)
    s[0, 0, 100:104] = [np.inf, -np.inf, 0.0, -0.0]
    _evict_case(fmt, N, H, L, 64, 0.75 if kind == "scattered" else 0.7, 4, s)


@pytest.mark.parametrize("kind", ["wide", "cluster", "wide_cluster"])
def test_evict_tokens_long_rows_select_passes(kind):
    """The resolve's exact select over the candidates in [lo, hi], a 12-bit
    radix pass over key - lo, then either a pass over the picked bin or,
    when that bin holds at most 64 keys, a ranking by one wave. wide: scores
    spread log-uniformly over 200 octaves, so the bracket spans about 2^26
    keys (bins of 2^15 keys, then the ranking). cluster: 300 tokens share
    the score at the keep-th rank, so the picked bin holds more than 64 keys
    and takes a second radix pass (a tie at tau: all 300 are kept).
    wide_cluster: the wide row with 300 distinct scores within 1e-3 of the
    keep-th one (a crowded first bin, a second pass, then the ranking)."""
    rng = np.random.default_rng({"wide": 41, "cluster": 43, "wide_cluster": 47}[kind])
    N, H, L, r = 1, 2, 70000, 0.75
    if kind.startswith("wide"):
        s = np.exp2(rng.uniform(-100, 100, size=(N, H, L))).astype(np.float32)
    else:
        s = rng.lognormal(size=(N, H, L)).astype(np.float32)
    if kind != "wide":
        keep = int(np.ceil(np.float32(r) * np.float32(L)))
        for h in range(H):
            tau = np.sort(s[0, h])[::-1][keep - 1]
            pos = rng.choice(np.arange(8, L), 300, replace=False)
            if kind == "cluster":
                s[0, h, pos] = tau
            else:
                s[0, h, pos] = (tau * (1 + rng.uniform(-1e-3, 1e-3, 300))).astype(np.float32)
    _evict_case("int4", N, H, L, 64, r, 4, s)


def test_evict_tokens_long_rows_span_counts():
    """Back-to-back long-row calls with 4, 1 and 2 spans per row and several
    rows, each with a workspace sized for its own span count: a call must
    not depend on what an earlier call left in the span slots, candidate
    lists or bitmasks."""
    for i, (N, H, L) in enumerate([(1, 2, 200003), (2, 3, 50000), (3, 2, 131072), (1, 1, 65540)]):
        rng = np.random.default_rng(100 + i)
        s = rng.lognormal(size=(N, H, L)).astype(np.float32)
        _evict_case("int4", N, H, L, 64, 0.75, 4, s, seed=i)


@pytest.mark.parametrize("L", [300, 40000])
def test_evict_tokens_aliased_pages(L):
    """Two sequences whose block tables share every third physical page
    (prefix-sharing style): the INT4 scale rewrite switches to atomics, and
    both sequences' evictions land on the shared pages (their union, as
    applying the oracle sequence by sequence gives)."""
    rng = np.random.default_rng(L + 1)
    N, H, D, bs = 2, 2, 64, 16
    M = (L + bs - 1) // bs
    bt = rng.permutation(N * M + 2)[:N * M].reshape(N, M).astype(np.int32)
    bt[1, ::3] = bt[0, ::3]
    s = rng.lognormal(size=(N, H, L)).astype(np.float32)
    _evict_case("int4", N, H, L, D, 0.6, 4, s, bt=bt, seed=L + 1)
    # the fp16 pool's zero stores need no atomics and give the same union
    _evict_case("fp16", N, H, L, D, 0.6, 4, s, bt=bt, seed=L + 1)


@pytest.mark.parametrize("fmt", ["fp16", "int4"])
@pytest.mark.parametrize("L", [64, 40000])
@pytest.mark.parametrize("heads_b", [(0, 1), (2, 3), (0, 1, 2, 3)])
def test_evict_tokens_shared_page_votes(fmt, L, heads_b):
    """Two sequences name one page (prefix sharing) and both fully evict it:
    sequence 0 in heads 0 and 1, sequence 1 in `heads_b` (overlapping,
    disjoint, all). A shared page gets the union of the evictions and no
    votes, so it stays linked in both tables (votes per (sequence, head)
    would reach H = 4 while heads still hold live rows); every other page
    fully evicted in all heads is unlinked. Short rows and long rows."""
    rng = np.random.default_rng(L + len(heads_b))
    N, H, D, bs = 2, 4, 64, 16
    M = (L + bs - 1) // bs
    bt = rng.permutation(N * M + 2)[:N * M].reshape(N, M).astype(np.int32)
    bt[1, 2] = bt[0, 2]  # logical block 2 of both sequences: one page
    s = rng.lognormal(size=(N, H, L)).astype(np.float32)
    low = lambda n: (1e-6 * (1 + rng.random(n))).astype(np.float32)  # distinct, below every lognormal draw
    for h in (0, 1):
        s[0, h, 32:48] = low(16)
    for h in heads_b:
        s[1, h, 32:48] = low(16)
    for h in range(H):
        s[0, h, 16:32] = low(16)  # a block of sequence 0 alone, every head: unlinked
    # keep = ceil(0.4 L): at least 32 evictions per head, so the low blocks go
    _evict_case(fmt, N, H, L, D, 0.4, 4, s, bt=bt, seed=L + 7)
    shared = int(bt[0, 2])
    bt_d = to_dev(bt)
    ibf_d = to_dev(np.zeros(N * M + 2, np.int32))
    memopt_C.evict_tokens(to_dev(s), bt_d, ibf_d, 0.4, 4)
    got_bt, got_ibf = bt_d.cpu().numpy(), ibf_d.cpu().numpy()
    assert got_bt[0, 2] == shared and got_bt[1, 2] == shared and got_ibf[shared] == 0
    assert got_bt[0, 1] == -1


@pytest.mark.parametrize("D,N,H,L", [(128, 2, 3, 300), (192, 2, 3, 300), (1088, 2, 3, 300),
                                     (128, 1, 3, 40000), (192, 1, 5, 40000), (64, 1, 40, 33000),
                                     (1088, 1, 1, 33000)])
def test_evict_tokens_int4_head_dims(D, N, H, L):
    """INT4 zeroing over the scale-line path (G = D / 64 groups: 2 and 3
    give 8 and 5 blocks per wave step) and over the per-token fallback taken
    when G > 16 (D = 1088), for short rows (one workgroup per row) and long
    rows (the page-major apply over all heads of a page; 40 heads give 6
    logical blocks per workgroup, 240 items)."""
    rng = np.random.default_rng(D + L)
    bs, r, sinks = 16, 0.6, 4
    M = (L + bs - 1) // bs
    nb = N * M + 2
    memopt_C.init_pool(nb, bs, H, D, kv_format="int4")
    T = nb * bs
    k = rng.standard_normal((T, H, D)).astype(np.float16)
    v = rng.standard_normal((T, H, D)).astype(np.float16)
    memopt_C.write_cache(to_dev(k), to_dev(v), to_dev(np.zeros((1, 1), np.int32)),
                         to_dev(np.arange(T, dtype=np.int32)))
    scores = rng.lognormal(size=(N, H, L)).astype(np.float32)
    scores[N - 1, :, 32:48] = 1e-6  # one logical block evicted in every head -> unlinked
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


@pytest.mark.parametrize("fmt,bs", [("fp16", 16), ("int4", 16), ("fp16", 128), ("fp16", 256), ("fp16", 8),
                                    ("fp16", 512), ("fp16", 2048), ("fp16", 8192)])
def test_evict_cache_vs_oracle(fmt, bs):
    """evict_cache for pages of any size (the reference strides over
    block_size, src/csrc/kv_cache.cu:409, :454); pages over 256 tokens take
    the radix-select path, with the same ties and sentinel cases, and a NaN
    score (never exceeded, so never evicted) in one of them."""
    rng = np.random.default_rng(5 + bs)
    nb, H, D = 6, 4, 64
    memopt_C.init_pool(nb, bs, H, D, kv_format=fmt)
    T = nb * bs
    k = rng.standard_normal((T, H, D)).astype(np.float16)
    memopt_C.write_cache(to_dev(k), to_dev(k), to_dev(np.zeros((1, 1), np.int32)),
                         to_dev(np.arange(T, dtype=np.int32)))
    scores = rng.standard_normal((nb, bs, H)).astype(np.float32)
    scores[0, : bs // 2, 0] = 0.25                     # ties
    scores[1, :, 1] = -np.inf                          # nothing above the reference's -1e38 sentinel
    scores[2, 3, 2] = np.nan
    scores[2, 5, 2] = np.float32(-1e38)                # at the sentinel: exceeded by every valid score
    scores[3, :, 3] = np.where(np.arange(bs) % 2 == 0, 0.0, -0.0)  # -0 and +0 tie: none evicted
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


def test_evict_tokens_caller_workspace():
    """evict_tokens with a workspace the caller keeps, starting filled with
    0x5A bytes, over back-to-back calls (short and long rows): a call
    depends on nothing the workspace holds (page marks, span slots, lists,
    bitmasks and the alias flag are all overwritten or tag-checked)."""
    rng = np.random.default_rng(61)
    N, H, bs, D = 2, 4, 16, 64
    for L in (3000, 70000):
        M = (L + bs - 1) // bs
        nb = N * M + 2
        memopt_C.init_pool(nb, bs, H, D, kv_format="int4")
        T = nb * bs
        k = rng.standard_normal((T, H, D)).astype(np.float16)
        memopt_C.write_cache(to_dev(k), to_dev(k), to_dev(np.zeros((1, 1), np.int32)),
                             to_dev(np.arange(T, dtype=np.int32)))
        bt = rng.permutation(nb)[:N * M].reshape(N, M).astype(np.int32)
        bt[1, ::5] = bt[0, ::5]  # shared pages: the alias path
        ws = torch.full((memopt_C.evict_workspace_bytes(N, H, L, M, nb),), 0x5A, dtype=torch.uint8, device=dev())
        state = _pool_state("int4")
        bt_d, ibf = to_dev(bt), np.zeros(nb, np.int32)
        ibf_d = to_dev(ibf)
        for _ in range(3):
            s = rng.lognormal(size=(N, H, L)).astype(np.float32)
            memopt_C.evict_tokens(to_dev(s), bt_d, ibf_d, 0.9, 4, workspace=ws)
            O.evict_tokens_intended(s, bt, ibf, 0.9, 4, state, bs)
            same_bits(_pool_state("int4")["pages"], state["pages"])
            same_bits(bt_d, bt)
            same_bits(ibf_d, ibf)
    with pytest.raises(RuntimeError, match="workspace"):
        memopt_C.evict_tokens(to_dev(s), bt_d, ibf_d, 0.9, 4, workspace=ws[:16])


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
