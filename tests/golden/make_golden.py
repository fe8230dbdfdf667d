"""Writes the small golden fixtures of tests/golden/ with the CPU oracle (oracle/moex_oracle.c).

The reference holds no vectors for this path (its tests draw seeded data at run time, tests/test_fa.cu:18,
tests/test_kernels.cu:787), so these fixtures freeze the oracle's outputs on fixed seeded inputs: the CPU suite checks
that the oracle still reproduces them, and the GPU suite checks the kernels against them. Run from the repository
root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle as orc  # noqa: E402

AHD, H, KV = 256, 16, 2
LD = H * 2 * AHD


def append_case(turbo, seed):
    """16 token rows appended at position 5 of a 24-row cache; includes a zero row and a tied-quotient row."""
    rng = np.random.default_rng(seed)
    T, pos0, max_t = 16, 5, 24
    k = (rng.standard_normal((T, KV * AHD)) * np.geomspace(0.01, 100, T)[:, None]).astype(np.float32)
    v = (rng.standard_normal((T, KV * AHD)) * np.geomspace(100, 0.01, T)[:, None]).astype(np.float32)
    k[2] = 0.0
    k[3, :AHD] = np.linspace(-127, 127, AHD, dtype=np.float32)
    c = orc.HostCache(KV, max_t, turbo)
    orc.kv_append(c, k, v, KV * AHD, T, pos0)
    sl = slice(pos0, pos0 + T)
    return dict(k=k, v=v, pos0=np.int32(pos0), max_t=np.int32(max_t), kc=c.k[:, sl].copy(), vc=c.v[:, sl].copy(),
                ks=c.ks[:, sl].copy(), vs=c.vs[:, sl].copy())


def attn_case(turbo, seed):
    """T = 3 query tokens at positions 60..62 over 63 keys (fp64 reference outputs, gated)."""
    rng = np.random.default_rng(seed)
    T, pos0, max_t = 3, 60, 64
    n = pos0 + T
    c = orc.HostCache(KV, max_t, turbo)
    kk = rng.standard_normal((n, KV * AHD)).astype(np.float32)
    vv = rng.standard_normal((n, KV * AHD)).astype(np.float32)
    orc.kv_append(c, kk, vv, KV * AHD, n, 0)
    qo = rng.standard_normal((T, H, AHD)).astype(np.float16).astype(np.float32)
    qg = rng.standard_normal((T, LD)).astype(np.float16).astype(np.float32)
    rows = [(t, h) for t in range(T) for h in range(H)]
    gate = None if turbo else qg
    out = orc.attn_rows_f64(qo, gate, LD, H, c, pos0, rows).reshape(T, H, AHD)
    return dict(kc=c.k, vc=c.v, ks=c.ks, vs=c.vs, qo=qo, qg=qg, pos0=np.int32(pos0), out=out.astype(np.float64))


def dense_case(seed):
    """A 24 x 512 fp16 weight block (incl. a zero row and a constant row), its int8 rows and scales, and the exact
    products with 3 input rows."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((24, 512)) * np.geomspace(1e-3, 1, 24)[:, None]).astype(np.float16)
    w[1] = 0
    w[2] = np.float16(0.125)
    q, s = orc.quantize_rows_i8(w)
    x = rng.standard_normal((3, 512)).astype(np.float32)
    return dict(w=w, q=q, s=s, x=x, y=orc.dense_i8_f64(q, s, x))


def main():
    for turbo in (0, 1):
        np.savez_compressed(os.path.join(HERE, f"append_{'turbo' if turbo else 'int8'}.npz"), **append_case(turbo, 100 + turbo))
        np.savez_compressed(os.path.join(HERE, f"attn_{'turbo' if turbo else 'int8'}.npz"), **attn_case(turbo, 200 + turbo))
    np.savez_compressed(os.path.join(HERE, "dense_i8.npz"), **dense_case(300))
    print("written:", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
