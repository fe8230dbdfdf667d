"""Kernels against the committed golden fixtures (tests/golden/): append codes and scales bit-exact; decode (split-K
GQA + combine, and the full dispatcher's turbo rotation) and FA prefill within the tolerances of test_gpu_decode.py
(1e-4 of max |ref|) and of tests/test_fa.cu:114 (here the fixed bound 2e-3 of max |ref| for T = 3)."""
import os

import numpy as np
import pytest

from tests.gpu_util import AHD, H, KV, LD, dev, download, pos_tensor, report

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("fmt,turbo", [("int8", 0), ("turbo", 1)])
def test_append_golden(fmt, turbo):
    import torch
    import moex_amd as M
    g = np.load(os.path.join(GOLD, f"append_{fmt}.npz"))
    T, pos0 = g["k"].shape[0], int(g["pos0"])
    cache = M.DeviceKVCache(KV, int(g["max_t"]), turbo)
    M.kv_append(dev(g["k"]), dev(g["v"]), cache, KV, pos_tensor(pos0), cache.max_t, KV * AHD, T)
    torch.cuda.synchronize()
    got = download(cache)
    sl = slice(pos0, pos0 + T)
    assert np.array_equal(got.k[:, sl], g["kc"]) and np.array_equal(got.v[:, sl], g["vc"])
    assert np.array_equal(got.ks[:, sl].view(np.uint32), g["ks"].view(np.uint32))
    assert np.array_equal(got.vs[:, sl].view(np.uint32), g["vs"].view(np.uint32))


def _cache(g, turbo):
    import torch
    import moex_amd as M
    c = M.DeviceKVCache(KV, g["kc"].shape[1], turbo)
    c.k.copy_(torch.from_numpy(g["kc"].view(np.uint8) if turbo else g["kc"]))
    c.v.copy_(torch.from_numpy(g["vc"].view(np.uint8) if turbo else g["vc"]))
    c.ks.copy_(torch.from_numpy(g["ks"]))
    c.vs.copy_(torch.from_numpy(g["vs"]))
    return c


@pytest.mark.parametrize("fmt,turbo", [("int8", 0), ("turbo", 1)])
@pytest.mark.parametrize("path", ["gqa", "fa"])
def test_attention_golden(fmt, turbo, path):
    import torch
    import moex_amd as M
    g = np.load(os.path.join(GOLD, f"attn_{fmt}.npz"))
    T, pos0 = g["qo"].shape[0], int(g["pos0"])
    c = _cache(g, turbo)
    qo, qg = dev(g["qo"]), dev(g["qg"])
    out = torch.zeros((T, H, AHD), dtype=torch.float32, device="cuda")
    gate = None if turbo else qg
    if path == "gqa":
        ns = 4
        part = torch.empty(T * H * ns * (AHD + 2), dtype=torch.float32, device="cuda")
        M.attn_gqa(qo, c, H, KV, pos_tensor(pos0), c.max_t, part, T, ns)
        M.attn_combine(part, gate, out, H, ns, LD, T)
        tol = 1e-4
    else:
        M.attn_fa(qo, gate, c, out, H, KV, pos_tensor(pos0), c.max_t, LD, T)
        tol = 2e-3
    torch.cuda.synchronize()
    ref = g["out"]
    err = float(np.abs(out.cpu().numpy() - ref).max())
    mag = float(np.abs(ref).max())
    report(f"golden {path} {fmt}", err=err, mag=mag, rel=err / mag)
    assert err <= tol * mag
