"""Writes the committed golden fixtures under tests/golden/ from the CPU oracle.

The reference repository ships no vectors or fixtures for this path (its tests
draw inputs from the CUDA RNG), so the fixtures here are small, seeded slices
of BASELINE.json config 1 evaluated by the oracle, whose correctness is pinned
separately in tests/test_oracle.py. They freeze the expected bytes so a drift
in either the oracle or the device path is caught.

Run: ``python tests/golden/make_golden.py`` (rewrites the .npz files).
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as O  # noqa: E402


def config1_slice(pages=4):
    """Config 1, truncated to `pages` pages: K, V fp16 [pages, 16, 8, 64] ~ N(0,1)
    with 1% of elements x8, seed 0; draw order K, V, Q, permutation."""
    g = torch.Generator().manual_seed(0)
    k = O.outlier_normal(g, (pages, 16, 8, 64), 0.01, 8.0)
    v = O.outlier_normal(g, (pages, 16, 8, 64), 0.01, 8.0)
    q = torch.randn((1, 1, 8, 64), generator=g).half().numpy()
    bt = torch.randperm(pages, generator=g).to(torch.int32).numpy()[None]
    return k, v, q, bt


def main():
    k, v, q, bt = config1_slice()
    ctx = np.array([k.shape[0] * 16], np.int32)
    kp, ks = O.quantize_int4(k)
    vp, vs = O.quantize_int4(v)
    kd, vd = O.dequantize_int4(kp, ks), O.dequantize_int4(vp, vs)
    pages = O.to_int4_pages(k, v)
    out_full = O.paged_attention(q, kd, vd, bt, ctx, 64, 64, num_sink_tokens=4)
    out_win = O.paged_attention(q, kd, vd, bt, ctx, 64, 24, num_sink_tokens=4)
    out_pages = O.paged_attention_int4(q, pages, bt, ctx, 64, 24, num_sink_tokens=4)
    np.savez_compressed(
        os.path.join(HERE, "config1_slice.npz"),
        k=k, v=v, q=q, block_tables=bt, context_lens=ctx,
        k_packed=kp, k_scales=ks, v_packed=vp, v_scales=vs, k_deq=kd, v_deq=vd,
        int4_pages=pages,
        out_full_sinks4=out_full, out_window24_sinks4=out_win, out_pages_window24_sinks4=out_pages,
    )
    # Known-answer groups (reference tests/test_quant.py:439-566 plus rounding ties).
    kat = np.zeros((4, 64), np.float16)
    kat[1, 0::2], kat[1, 1::2] = 7.0, -7.0
    kat[2, :] = 0.5
    kat[3, :10] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 3.5, -3.5, 6.5, 7.0]
    p, s = O.quantize_int4(kat)
    np.savez_compressed(os.path.join(HERE, "kat_groups.npz"), x=kat, packed=p, scales=s,
                        deq=O.dequantize_int4(p, s))
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
