"""Helpers shared by the GPU tests (inputs, oracle round trips, tolerances)."""
import numpy as np
import torch

# Floating-point tolerance of fused INT4 attention vs the composition oracle
# (max-abs 2e-3 / rtol 1e-2 in fp16).
ATOL, RTOL = 2e-3, 1e-2


def dev():
    return torch.device("cuda", 0)


def to_dev(a, dtype=None):
    t = torch.as_tensor(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(dev())


def assert_close(got, want, atol=ATOL, rtol=RTOL, what=""):
    g = got.detach().float().cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got, np.float32)
    w = want.detach().float().cpu().numpy() if isinstance(want, torch.Tensor) else np.asarray(want, np.float32)
    assert g.shape == w.shape, (g.shape, w.shape)
    err = np.abs(g - w)
    tol = atol + rtol * np.abs(w)
    bad = ~(err <= tol)
    if bad.any():
        i = np.unravel_index(np.argmax(np.where(bad, err / tol, -1.0)), g.shape)
        raise AssertionError(f"{what}: {bad.sum()} elements off, max abs err {np.nanmax(err):.3e}; "
                             f"worst at {tuple(int(x) for x in i)}: got {g[i]!r}, want {w[i]!r}")


def same_bits(got, want):
    g = got.detach().cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got)
    w = np.asarray(want)
    assert g.shape == w.shape, (g.shape, w.shape)
    assert g.dtype.itemsize == w.dtype.itemsize
    v = {1: np.uint8, 2: np.uint16, 4: np.uint32}[g.dtype.itemsize]
    diff = np.nonzero(g.view(v) != w.view(v))
    assert diff[0].size == 0, f"{diff[0].size} mismatches, first at {tuple(d[0] for d in diff)}"


class _LazyExtension:
    """Imports memopt_C on first use, so CPU-only collection never needs the
    built library while a GPU test without it fails loudly (ImportError)."""

    def __getattr__(self, name):
        import memopt_C
        return getattr(memopt_C, name)


memopt_C = _LazyExtension()


def dequant_pages_dev(pages, D):
    """INT4 page buffer -> fp16 pools (K, V) [nb, 16, H, D] on the GPU; equals
    oracle.from_int4_pages (checked in tests/test_oracle.py)."""
    import oracle as O
    return O.dequant_pages_torch(pages, D)


def reference_decode_dev(q, kpool, vpool, bt, ctx, W, sinks):
    """fp32 attention of one query per (b, h) over sinks U window on the GPU."""
    B, _, H, D = q.shape
    bs = kpool.shape[1]
    out = torch.zeros(B, H, D, device=q.device)
    for b in range(B):
        c = int(ctx[b])
        pages = bt[b, : (c + bs - 1) // bs].long()
        ok = (pages >= 0).repeat_interleave(bs)[:c]
        k = kpool[pages.clamp(min=0)].reshape(-1, H, D)[:c].float()
        v = vpool[pages.clamp(min=0)].reshape(-1, H, D)[:c].float()
        j = torch.arange(c, device=q.device)
        vis = ((j >= c - W) | (j < sinks)) & ok
        k, v = k[vis].permute(1, 0, 2), v[vis].permute(1, 0, 2)     # [H, n, D]
        s = (k @ q[b, 0].float()[:, :, None]).squeeze(-1) / D ** 0.5  # [H, n]
        p = torch.softmax(s, dim=-1)
        out[b] = (p[:, None, :] @ v).squeeze(1)
    return out.half()[:, None]


def special_fp16(shape, seed):
    """fp16 data with NaN of both signs, +-inf, -0, subnormals and +-65504
    scattered through normal values (3 %), and whole 64-element groups of
    them: all NaN, all -NaN, all inf, all subnormal, all -0, 65504 in every
    other element, one inf, one NaN (the first 8 groups of the flattened
    tensor, which must hold at least 8)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(shape).astype(np.float16)
    neg_nan = np.frombuffer(np.uint16(0xFE00).tobytes(), np.float16)[0]
    vals = np.array([np.nan, neg_nan, np.inf, -np.inf, -0.0, 6e-8, -6e-8, 1e-5, 65504, -65504], np.float16)
    flat = x.reshape(-1)
    m = rng.random(flat.size) < 0.03
    flat[m] = vals[rng.integers(0, vals.size, int(m.sum()))]
    g = flat.reshape(-1, 64)
    assert g.shape[0] >= 8
    g[0] = np.nan
    g[1] = neg_nan
    g[2] = np.inf
    g[3] = np.float16(6e-8)
    g[4] = np.float16(-0.0)
    g[5, ::2] = np.float16(65504)
    g[6, 0] = np.inf
    g[7, 0] = np.nan
    return x
