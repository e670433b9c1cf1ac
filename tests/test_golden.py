"""The oracle reproduces the committed golden fixtures bit-for-bit (CPU)."""
import os

import numpy as np

import oracle as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_kat_fixture():
    f = np.load(os.path.join(HERE, "kat_groups.npz"))
    p, s = O.quantize_int4(f["x"])
    assert np.array_equal(p, f["packed"]) and np.array_equal(s, f["scales"])
    assert (f["packed"][0] == 0x88).all() and (f["packed"][1] == 0x1F).all() and (f["packed"][2] == 0xFF).all()
    assert np.array_equal(O.dequantize_int4(p, s).view(np.uint16), f["deq"].view(np.uint16))


def test_config1_slice_fixture():
    f = np.load(os.path.join(HERE, "config1_slice.npz"))
    kp, ks = O.quantize_int4(f["k"])
    assert np.array_equal(kp, f["k_packed"]) and np.array_equal(ks.view(np.uint32), f["k_scales"].view(np.uint32))
    assert np.array_equal(O.to_int4_pages(f["k"], f["v"]), f["int4_pages"])
    out = O.paged_attention(f["q"], f["k_deq"], f["v_deq"], f["block_tables"], f["context_lens"], 64, 24,
                            num_sink_tokens=4)
    assert np.array_equal(out.view(np.uint16), f["out_window24_sinks4"].view(np.uint16))
