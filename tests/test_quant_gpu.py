"""GPU parity of quantize/dequantize (restates the reference's tests/test_quant.py,
with bit-exact comparison against the oracle where the reference used 1e-4 or +-1)."""
import os

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import dev, memopt_C, same_bits, special_fp16, to_dev

pytestmark = pytest.mark.gpu

G = 64
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def make(shape, dist, seed=42):
    g = torch.Generator().manual_seed(seed)
    t = {
        "uniform_unit": lambda: torch.rand(shape, generator=g) * 2 - 1,
        "uniform_pos": lambda: torch.rand(shape, generator=g),
        "uniform_neg": lambda: -torch.rand(shape, generator=g),
        "uniform_small": lambda: torch.rand(shape, generator=g) * 0.2 - 0.1,
        "normal_std": lambda: torch.randn(shape, generator=g),
        "normal_kv": lambda: torch.randn(shape, generator=g) * 0.02,
        "zeros": lambda: torch.zeros(shape),
        "constant": lambda: torch.full(shape, 0.5),
        "outliers": lambda: torch.randn(shape, generator=g) * torch.where(torch.rand(shape, generator=g) < 0.01, 8.0, 1.0),
        "large": lambda: torch.rand(shape, generator=g) * 200 - 100,
    }[dist]()
    return t.half()


def check_exact(cache_cpu):
    x = cache_cpu.numpy()
    packed, scales = memopt_C.quantize_kv_cache_int4(cache_cpu.to(dev()), G)
    wp, ws = O.quantize_int4(x)
    same_bits(packed, wp)
    same_bits(scales, ws)
    deq = memopt_C.dequantize_kv_cache_int4(packed, scales, G)
    same_bits(deq, O.dequantize_int4(wp, ws))
    return packed, scales, deq


SHAPES = [(128,), (4, 128), (2, 8, 64), (2, 4, 8, 64)]


@pytest.mark.parametrize("shape", SHAPES)
def test_shapes_and_dtypes(shape):
    packed, scales, deq = check_exact(make(shape, "uniform_unit"))
    assert packed.shape == shape[:-1] + (shape[-1] // 2,) and packed.dtype == torch.uint8
    assert scales.shape == (int(np.prod(shape)) // G,) and scales.dtype == torch.float32
    assert deq.shape == shape and deq.dtype == torch.float16


@pytest.mark.parametrize("dist", ["uniform_unit", "normal_std", "uniform_small", "uniform_pos", "uniform_neg",
                                  "normal_kv", "zeros", "constant", "outliers", "large"])
@pytest.mark.parametrize("shape", [(4, 128), (2, 8, 64), (129, 64), (64, 16, 8, 64)])
def test_bit_exact_vs_oracle(shape, dist):
    check_exact(make(shape, dist))


@pytest.mark.parametrize("shape", [(4, 128), (64, 16, 8, 64)])
def test_special_values_bit_exact(shape):
    """NaN of both signs, +-inf, -0, subnormals and +-65504, scattered and as
    whole groups: codes, scales and the dequantized values bit-exact with the
    oracle (the reference's fmaxf leaves a NaN out of the absmax; an inf
    absmax gives scale inf)."""
    check_exact(torch.from_numpy(special_fp16(shape, 5)))


@pytest.mark.parametrize("num_groups,dist,bound,relative", [
    (n, d, b, r) for n in (1, 4, 16, 128) for d, b, r in
    (("uniform_unit", 5e-3, False), ("normal_std", 5e-2, False), ("uniform_small", 5e-5, False),
     ("normal_kv", 0.02, True))])
def test_mse_bounds(num_groups, dist, bound, relative):
    """tests/test_quant.py:309-409 thresholds."""
    cache = make((num_groups * G,), dist).to(dev())
    p, s = memopt_C.quantize_kv_cache_int4(cache, G)
    d = memopt_C.dequantize_kv_cache_int4(p, s, G)
    err = ((d.float() - cache.float()) ** 2).mean().item()
    if relative:
        err /= cache.float().var().item()
    assert err < bound


def test_known_answers_fixture():
    f = np.load(os.path.join(GOLD, "kat_groups.npz"))
    p, s = memopt_C.quantize_kv_cache_int4(to_dev(f["x"]), G)
    same_bits(p, f["packed"])
    same_bits(s, f["scales"])
    same_bits(memopt_C.dequantize_kv_cache_int4(p, s, G), f["deq"])


def test_config1_slice_fixture():
    f = np.load(os.path.join(GOLD, "config1_slice.npz"))
    for n in ("k", "v"):
        p, s = memopt_C.quantize_kv_cache_int4(to_dev(f[n]), G)
        same_bits(p, f[f"{n}_packed"])
        same_bits(s, f[f"{n}_scales"])
        same_bits(memopt_C.dequantize_kv_cache_int4(p, s, G), f[f"{n}_deq"])


def test_config1_full_bit_exact():
    """K and V [64, 16, 8, 64] ~ N(0,1), 1% x8, seed 0."""
    g = torch.Generator().manual_seed(0)
    for _ in range(2):
        check_exact(torch.as_tensor(O.outlier_normal(g, (64, 16, 8, 64), 0.01, 8.0)))


def test_misaligned_storage_uses_scalar_path():
    base = make((64 * 33 + 1,), "normal_std")
    view = base[1:].view(33, 64)  # contiguous, 2-byte offset -> not 16-byte aligned on device
    big = base.to(dev())
    dview = big[1:].view(33, 64)
    assert dview.data_ptr() % 16 != 0
    p, s = memopt_C.quantize_kv_cache_int4(dview, G)
    wp, ws = O.quantize_int4(view.numpy())
    same_bits(p, wp)
    same_bits(s, ws)


def test_determinism():
    cache = make((4, 128), "normal_std").to(dev())
    a = memopt_C.quantize_kv_cache_int4(cache, G)
    b = memopt_C.quantize_kv_cache_int4(cache, G)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_large_tensor_properties():
    """268M elements (config 2's K cache size): round-trip bound on every group,
    codes in [1, 15], and exact agreement with the oracle on sampled groups."""
    n = 16 * 4096 * 32 * 128
    g = torch.Generator(device=dev()).manual_seed(0)
    x = torch.randn(n, device=dev(), generator=g)
    x = torch.where(torch.rand(n, device=dev(), generator=g) < 0.005, x * 10, x).half()
    p, s = memopt_C.quantize_kv_cache_int4(x, G)
    d = memopt_C.dequantize_kv_cache_int4(p, s, G)
    err = (d.float() - x.float()).abs().view(-1, G)
    bound = s[:, None] / 2 * (1 + 1e-6) + d.float().abs().view(-1, G) * 2.0 ** -11
    assert bool((err <= bound).all())
    lo, hi = (p & 0xF), (p >> 4)
    assert int(torch.minimum(lo.min(), hi.min())) >= 1 and int(torch.maximum(lo.max(), hi.max())) <= 15
    idx = torch.randint(0, n // G, (4096,), generator=torch.Generator().manual_seed(1))
    groups = x.view(-1, G)[idx.to(dev())].cpu().numpy()
    wp, ws = O.quantize_int4(groups)
    same_bits(p.view(-1, G // 2)[idx.to(dev())], wp)
    same_bits(s[idx.to(dev())], ws)


# --- error guards: tests/test_quant.py:702-771 --------------------------------

def test_error_wrong_group_size():
    with pytest.raises(RuntimeError):
        memopt_C.quantize_kv_cache_int4(make((4, 128), "uniform_unit").to(dev()), 32)


def test_error_fp32():
    with pytest.raises(RuntimeError):
        memopt_C.quantize_kv_cache_int4(torch.rand(4, 128, device=dev()), G)


def test_error_cpu_tensor():
    with pytest.raises(RuntimeError):
        memopt_C.quantize_kv_cache_int4(torch.rand(4, 128).half(), G)


def test_error_non_contiguous():
    with pytest.raises(RuntimeError):
        memopt_C.quantize_kv_cache_int4(torch.rand(128, 4, device=dev()).half().t(), G)


def test_error_odd_last_dim():
    with pytest.raises(RuntimeError):
        memopt_C.quantize_kv_cache_int4(torch.rand(4, 3, device=dev()).half(), G)


def test_error_not_divisible():
    with pytest.raises(RuntimeError):
        memopt_C.quantize_kv_cache_int4(torch.rand(50, 2, device=dev()).half(), G)


def test_dequant_error_scales_mismatch():
    p, s = memopt_C.quantize_kv_cache_int4(make((4, 128), "uniform_unit").to(dev()), G)
    with pytest.raises(RuntimeError):
        memopt_C.dequantize_kv_cache_int4(p, s[:-1].contiguous(), G)


def _boundary_groups(seed=31, n_scales=400):
    """Groups whose elements sit on, and 1-3 fp16 ulps around, every rounding
    boundary (k + 0.5) * scale of the group's own scale, for many absmax values:
    the inputs where an inexact quotient v / scale would flip a code."""
    rng = np.random.default_rng(seed)
    groups = []
    for _ in range(n_scales):
        a = np.float16(rng.uniform(1e-3, 200.0) * rng.choice([1, -1]))
        s = np.float32(abs(np.float32(a))) / np.float32(7.0)
        vals = []
        for k in range(-7, 7):
            mid = np.float16(np.float32(k + 0.5) * s)
            for d in (-3, -2, -1, 0, 1, 2, 3):
                v = np.nextafter(mid, np.float16(np.inf if d > 0 else -np.inf), dtype=np.float16) if d else mid
                for _ in range(abs(d) - 1 if d else 0):
                    v = np.nextafter(v, np.float16(np.inf if d > 0 else -np.inf), dtype=np.float16)
                if abs(np.float32(v)) <= abs(np.float32(a)):
                    vals.append(v)
        vals = np.array(vals, np.float16)
        for i in range(0, len(vals), 63):
            g = np.zeros(64, np.float16)
            g[0] = a
            chunk = vals[i:i + 63]
            g[1:1 + len(chunk)] = chunk
            groups.append(g)
    return np.stack(groups)


def test_quantize_rounding_boundaries_bit_exact():
    """Codes at (and next to) the .5 boundaries of v / scale equal the oracle's
    (IEEE division + roundf), through the surface quantize and write_cache."""
    x = _boundary_groups()
    want_p, want_s = O.quantize_int4(x)
    got_p, got_s = memopt_C.quantize_kv_cache_int4(to_dev(x), 64)
    same_bits(got_p, want_p)
    same_bits(got_s, want_s)
    # same groups through the fused page writer (rows of [tokens, 1 head, 64])
    T = x.shape[0] - x.shape[0] % 16
    rows = x[:T].reshape(T, 1, 64)
    nb = T // 16
    memopt_C.init_pool(nb, 16, 1, 64, kv_format="int4")
    slots = np.arange(T, dtype=np.int32)
    memopt_C.write_cache(to_dev(rows), to_dev(rows[::-1].copy()), to_dev(np.zeros((1, 1), np.int32)), to_dev(slots))
    wk = rows.reshape(nb, 16, 1, 64)
    wv = rows[::-1].reshape(nb, 16, 1, 64)
    same_bits(memopt_C.get_int4_pages(), O.to_int4_pages(wk, wv))
