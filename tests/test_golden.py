"""The oracle still reproduces the committed golden fixtures (tests/golden/, written by tests/golden/make_golden.py).

These fixtures freeze the oracle's output on fixed inputs; the mathematical pins of the oracle itself are in
test_oracle.py. Quantized codes and scales must match bit for bit, the fp64 attention to 1e-12 relative.
"""
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
AHD, H, KV = 256, 16, 2
LD = H * 2 * AHD


@pytest.mark.parametrize("fmt,turbo", [("int8", 0), ("turbo", 1)])
def test_oracle_append_matches_golden(orc, fmt, turbo):
    g = np.load(os.path.join(GOLD, f"append_{fmt}.npz"))
    T, pos0 = g["k"].shape[0], int(g["pos0"])
    c = orc.HostCache(KV, int(g["max_t"]), turbo)
    orc.kv_append(c, g["k"], g["v"], KV * AHD, T, pos0)
    sl = slice(pos0, pos0 + T)
    assert np.array_equal(c.k[:, sl], g["kc"]) and np.array_equal(c.v[:, sl], g["vc"])
    assert np.array_equal(c.ks[:, sl].view(np.uint32), g["ks"].view(np.uint32))
    assert np.array_equal(c.vs[:, sl].view(np.uint32), g["vs"].view(np.uint32))


@pytest.mark.parametrize("fmt,turbo", [("int8", 0), ("turbo", 1)])
def test_oracle_attention_matches_golden(orc, fmt, turbo):
    g = np.load(os.path.join(GOLD, f"attn_{fmt}.npz"))
    c = orc.HostCache(KV, g["kc"].shape[1], turbo)
    c.k[:], c.v[:], c.ks[:], c.vs[:] = g["kc"], g["vc"], g["ks"], g["vs"]
    T = g["qo"].shape[0]
    rows = [(t, h) for t in range(T) for h in range(H)]
    out = orc.attn_rows_f64(g["qo"], None if turbo else g["qg"], LD, H, c, int(g["pos0"]), rows).reshape(T, H, AHD)
    assert np.max(np.abs(out - g["out"])) <= 1e-12 * np.max(np.abs(g["out"]))


def test_oracle_dense_matches_golden(orc):
    g = np.load(os.path.join(GOLD, "dense_i8.npz"))
    q, s = orc.quantize_rows_i8(g["w"])
    assert np.array_equal(q, g["q"]) and np.array_equal(s.view(np.uint32), g["s"].view(np.uint32))
    y = orc.dense_i8_f64(q, s, g["x"])
    assert np.abs(y - g["y"]).max() <= 1e-12 * np.abs(g["y"]).max()
