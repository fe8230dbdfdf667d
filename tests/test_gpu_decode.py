"""Split-K GQA decode / MTP verify (attn_gqa_k + attn_combine_k, kernels.cuh:1740-1844, 1317-1329) and the
per-head decode kernel (attn_decode_k, :1238-1315) against the fp64 oracle.

Tolerance: max |err| <= 1e-4 * max |ref| -- the reference's own bound between its two fp32 decode kernels
(tests/test_kernels.cu:849, K7G). Cases follow test_kernels.cu:838 ((pos, T, ns) = (0,1,16), (3,1,16), (1000,2,16),
(26000,1,64)) plus MTP verify windows and the 90k context of the benchmark.
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.gpu_util import AHD, H, KV, LD, dev, download, pos_tensor, random_int8_cache, report, upload

pytestmark = pytest.mark.gpu
TOL = 1e-4

# the MTP-verify windows also cover: a chunk boundary between the tokens' last keys (254, 4, 1), splits where the
# group's first tokens have no key (3, 4, 16), a partial token group (130, 3, 2) and groups of 4, 4, 1 (777, 9, 7)
CASES = [(0, 1, 16), (3, 1, 16), (1000, 2, 16), (26000, 1, 64), (5000, 4, 32), (777, 9, 7), (89999, 1, 256),
         (89996, 4, 256), (254, 4, 1), (3, 4, 16), (130, 3, 2), (2000, 2, 64), (89997, 3, 256), (255, 1, 2),
         (127, 1, 1), (40000, 1, 1)]


@pytest.fixture(scope="module")
def int8_setup():
    max_t = 90064
    hc = random_int8_cache(max_t, seed=11)
    dc = upload(hc)
    rng = np.random.default_rng(12)
    qo = (3 * rng.uniform(-1, 1, (9, H, AHD))).astype(np.float32)
    qg = rng.uniform(-1, 1, (9, LD)).astype(np.float32)
    return hc, dc, qo, qg


def _check(name, out, qo, qg, hc, pos0, T, tol=TOL):
    rows = [(t, h) for t in range(T) for h in range(H)]
    ref = orc.attn_rows_f64(qo, qg, LD, H, hc, pos0, rows)
    got = np.stack([out[t, h] for t, h in rows])
    err, mag = float(np.abs(got - ref).max()), float(np.abs(ref).max())
    report(name, pos0=pos0, T=T, err=err, mag=mag, rel=err / mag)
    assert np.all(np.isfinite(got))
    assert err <= tol * mag


@pytest.mark.parametrize("pos0,T,ns", CASES)
def test_gqa_int8(int8_setup, pos0, T, ns):
    import torch
    import moex_amd as M
    hc, dc, qo, qg = int8_setup
    part = torch.empty(T * H * ns * (AHD + 2), dtype=torch.float32, device="cuda")
    out = torch.zeros((T, H, AHD), dtype=torch.float32, device="cuda")
    qo_d, qg_d, p = dev(qo[:T]), dev(qg[:T]), pos_tensor(pos0)
    M.attn_gqa(qo_d, dc, H, KV, p, dc.max_t, part, T, ns)
    M.attn_combine(part, qg_d, out, H, ns, LD, T)
    torch.cuda.synchronize()
    _check(f"gqa int8 ns={ns}", out.cpu().numpy(), qo, qg, hc, pos0, T)


@pytest.mark.parametrize("pos0,T,ns", [(0, 1, 1), (3, 1, 16), (1000, 2, 1), (26000, 1, 64), (5000, 4, 3)])
def test_decode_heads_int8(int8_setup, pos0, T, ns):
    import torch
    import moex_amd as M
    hc, dc, qo, qg = int8_setup
    part = torch.empty(T * H * ns * (AHD + 2), dtype=torch.float32, device="cuda")
    out = torch.zeros((T, H, AHD), dtype=torch.float32, device="cuda")
    qo_d, qg_d, p = dev(qo[:T]), dev(qg[:T]), pos_tensor(pos0)
    M.attn_decode_heads(qo_d, qg_d, dc, out, H, KV, p, dc.max_t, LD, part, T, ns)
    if ns > 1:
        M.attn_combine(part, qg_d, out, H, ns, LD, T)
    torch.cuda.synchronize()
    _check(f"decode_heads int8 ns={ns}", out.cpu().numpy(), qo, qg, hc, pos0, T)


@pytest.fixture(scope="module")
def turbo_setup():
    """A turbo cache written by the GPU quantizer from N(0,1) rows (its codes are checked bit-exact elsewhere)."""
    import torch
    import moex_amd as M
    max_t, n = 40064, 40000
    dc = M.DeviceKVCache(KV, max_t, 1)
    g = torch.Generator(device="cuda").manual_seed(5)
    k = torch.randn((n, KV * AHD), generator=g, device="cuda")
    v = torch.randn((n, KV * AHD), generator=g, device="cuda")
    M.kv_append(k, v, dc, KV, pos_tensor(0), max_t, KV * AHD, n)
    torch.cuda.synchronize()
    hc = download(dc)
    rng = np.random.default_rng(13)
    qo = rng.standard_normal((9, H, AHD)).astype(np.float32)
    qg = rng.standard_normal((9, LD)).astype(np.float32)
    return hc, dc, qo, qg


@pytest.mark.parametrize("pos0,T,ns", [(0, 1, 16), (3, 1, 16), (1000, 2, 16), (39999, 1, 128), (39990, 4, 64)])
def test_gqa_turbo(turbo_setup, pos0, T, ns):
    """Attention in the rotated domain (no gate): the reference's combine output before turbo_out_k."""
    import torch
    import moex_amd as M
    hc, dc, qo, qg = turbo_setup
    part = torch.empty(T * H * ns * (AHD + 2), dtype=torch.float32, device="cuda")
    out = torch.zeros((T, H, AHD), dtype=torch.float32, device="cuda")
    M.attn_gqa(dev(qo[:T]), dc, H, KV, pos_tensor(pos0), dc.max_t, part, T, ns)
    M.attn_combine(part, None, out, H, ns, LD, T)
    torch.cuda.synchronize()
    _check(f"gqa turbo ns={ns}", out.cpu().numpy(), qo, None, hc, pos0, T)
    # + turbo_out (inverse WHT + gate) against the full turbo reference
    M.turbo_out(out, dev(qg[:T]), H, LD, T)
    torch.cuda.synchronize()
    _check(f"gqa turbo + turbo_out ns={ns}", out.cpu().numpy(), qo, qg, hc, pos0, T)


@pytest.mark.parametrize("pos0,T,ns", [(0, 1, 16), (1000, 2, 16), (39999, 1, 128), (39990, 4, 32)])
def test_gqa_out_turbo(turbo_setup, pos0, T, ns):
    """attn_gqa_out: the split kernel rotates its partials back, the gated combine then gives the full turbo output
    (what attn_decode runs); against the fp64 reference with the inverse WHT and the gate."""
    import torch
    import moex_amd as M
    hc, dc, qo, qg = turbo_setup
    part = torch.empty(T * H * ns * (AHD + 2), dtype=torch.float32, device="cuda")
    out = torch.zeros((T, H, AHD), dtype=torch.float32, device="cuda")
    M.attn_gqa_out(dev(qo[:T]), dc, H, KV, pos_tensor(pos0), dc.max_t, part, T, ns)
    M.attn_combine(part, dev(qg[:T]), out, H, ns, LD, T)
    torch.cuda.synchronize()
    _check(f"gqa_out turbo ns={ns}", out.cpu().numpy(), qo, qg, hc, pos0, T)


@pytest.mark.parametrize("pos0,T,ns", [(127, 1, 1), (128, 1, 1), (200, 1, 1), (2047, 3, 2), (39999, 1, 1),
                                       (16383, 1, 7)])
def test_gqa_turbo_steps(turbo_setup, pos0, T, ns):
    """The turbo split kernel's key assignment: chunks of 128 keys, chunk 0 the short one, wavefront w taking keys
    16w .. 16w + 15 of each chunk. 128 keys: one full chunk; 129: a one-key first chunk that seven wavefronts skip; 201:
    a first chunk that ends inside wavefront 4's keys; one split over 40000 keys (313 chunks through each wavefront's
    four-stage ring); a three-token window; splits of 2341 keys."""
    import torch
    import moex_amd as M
    hc, dc, qo, qg = turbo_setup
    part = torch.empty(T * H * ns * (AHD + 2), dtype=torch.float32, device="cuda")
    out = torch.zeros((T, H, AHD), dtype=torch.float32, device="cuda")
    M.attn_gqa_out(dev(qo[:T]), dc, H, KV, pos_tensor(pos0), dc.max_t, part, T, ns)
    M.attn_combine(part, dev(qg[:T]), out, H, ns, LD, T)
    torch.cuda.synchronize()
    _check(f"gqa_out turbo steps ns={ns}", out.cpu().numpy(), qo, qg, hc, pos0, T)


@pytest.mark.parametrize("pos0,T,ns", [(0, 1, 1), (1000, 2, 8)])
def test_decode_heads_turbo(turbo_setup, pos0, T, ns):
    import torch
    import moex_amd as M
    hc, dc, qo, qg = turbo_setup
    part = torch.empty(T * H * ns * (AHD + 2), dtype=torch.float32, device="cuda")
    out = torch.zeros((T, H, AHD), dtype=torch.float32, device="cuda")
    M.attn_decode_heads(dev(qo[:T]), None, dc, out, H, KV, pos_tensor(pos0), dc.max_t, LD, part, T, ns)
    if ns > 1:
        M.attn_combine(part, None, out, H, ns, LD, T)
    torch.cuda.synchronize()
    _check(f"decode_heads turbo ns={ns}", out.cpu().numpy(), qo, None, hc, pos0, T)
