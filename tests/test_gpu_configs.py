"""The benchmark configurations at their full sizes, with data drawn as the benchmark draws it (K/V ~ N(0,1) f32
quantized by the library's own append, Q and gate ~ N(0,1) rounded to fp16), checked against the fp64 oracle:

  configs[0]  int8 prefill, T = 2048 at pos0 = 0 (the tests/test_fa.cu shape), attn_fa and the attn_prefill fallback;
  configs[3]  turbo decode, one token at position 262143 over 262144 keys, through attn_decode (front + append +
              split-K GQA + combine + turbo_out) and through the raw launches;
  configs[4]  turbo prefill, T = 2048 at pos0 = 260096 over 262144 keys, attn_fa + turbo_out.

The quantized caches are compared bit for bit with the oracle's quantizer over every row. Prefill uses the rule of
tests/test_fa.cu:114 (e <= 2 e_ref + 1e-3 max|ref|, e_ref = the error of the oracle's precision model of attn_fa_k)
on the row sample of test_fa.cu:95; decode uses 1e-4 of max|ref| (test_kernels.cu:849, K7G), over all 16 heads.
The reference runs caches of this depth in tests/test_fa.cu:17,123,202-221.
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.gpu_util import (AHD, H, KV, LD, append_threaded, dev, download, pos_tensor, report, rows_threaded,
                            sample_rows)

pytestmark = pytest.mark.gpu
N_LONG = 262144


def _f16(a):
    return a.astype(np.float16).astype(np.float32)


def _filled_cache(n, max_t, turbo, seed):
    """K/V rows ~ N(0,1) quantized into a fresh cache by the library's append; the oracle's cache from the same rows
    must be identical to the bit."""
    import torch
    import moex_amd as M
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((n, KV * AHD), dtype=np.float32)
    v = rng.standard_normal((n, KV * AHD), dtype=np.float32)
    dc = M.DeviceKVCache(KV, max_t, turbo)
    for t in range(0, n, 65536):
        m = min(65536, n - t)
        M.kv_append(dev(k[t:t + m]), dev(v[t:t + m]), dc, KV, pos_tensor(t), max_t, KV * AHD, m)
    torch.cuda.synchronize()
    hc = download(dc)
    oc = orc.HostCache(KV, max_t, turbo)
    append_threaded(oc, k, v, KV * AHD, n, 0)
    for a, b, name in ((hc.k, oc.k, "k"), (hc.v, oc.v, "v"), (hc.ks, oc.ks, "ks"), (hc.vs, oc.vs, "vs")):
        assert np.array_equal(a[:, :n].view(np.uint8), b[:, :n].view(np.uint8)), f"cache {name} differs from the oracle"
    return dc, hc


def _prefill_gate(name, out, qo, qg, hc, pos0, T):
    rows = sample_rows(T)
    ref = rows_threaded(orc.attn_rows_f64, qo, qg, LD, H, hc, pos0, rows)
    emu = rows_threaded(orc.attn_rows_fa_emul, qo, qg, LD, H, hc, pos0, rows)
    got = np.stack([out[t, h] for t, h in rows])
    mag = float(np.abs(ref).max())
    e_new, e_ref = float(np.abs(got - ref).max()), float(np.abs(emu - ref).max())
    report(name, pos0=pos0, T=T, e_new=e_new, e_ref=e_ref, mag=mag)
    assert np.all(np.isfinite(out))
    assert e_new <= 2.0 * e_ref + 1e-3 * mag


def test_config0_int8_prefill():
    import torch
    import moex_amd as M
    T, pos0 = 2048, 0
    print("configs[0]: int8 prefill T=2048 pos0=0", flush=True)
    dc, hc = _filled_cache(T, T, 0, seed=100)
    rng = np.random.default_rng(101)
    qo = _f16(rng.standard_normal((T, H, AHD), dtype=np.float32))
    qg = _f16(rng.standard_normal((T, LD), dtype=np.float32))
    qo_d, qg_d = dev(qo), dev(qg)
    out = torch.full((T, H, AHD), float("nan"), device="cuda")
    M.attn_fa(qo_d, qg_d, dc, out, H, KV, pos_tensor(pos0), T, LD, T)
    torch.cuda.synchronize()
    o_fa = out.cpu().numpy()
    _prefill_gate("configs[0] attn_fa", o_fa, qo, qg, hc, pos0, T)
    out.fill_(float("nan"))
    M.attn_prefill(qo_d, qg_d, dc, out, H, KV, pos_tensor(pos0), T, LD, T)
    torch.cuda.synchronize()
    o_k7 = out.cpu().numpy()
    _prefill_gate("configs[0] attn_prefill", o_k7, qo, qg, hc, pos0, T)
    e_ab = float(np.abs(o_fa - o_k7).max())
    report("configs[0] fa vs fallback", e_ab=e_ab)
    assert e_ab <= 5e-3 * float(np.abs(o_k7).max())  # test_kernels.cu:809


@pytest.fixture(scope="module")
def turbo_long():
    print("turbo cache: 262144 keys", flush=True)
    return _filled_cache(N_LONG, N_LONG, 1, seed=300)


def test_config3_turbo_decode(turbo_long):
    import torch
    import moex_amd as M
    dc, hc = turbo_long
    pos = N_LONG - 1
    print("configs[3]: turbo decode, token at 262143", flush=True)
    rng = np.random.default_rng(301)
    qo = rng.standard_normal((1, H, AHD), dtype=np.float32)
    qg = rng.standard_normal((1, LD), dtype=np.float32)
    ns = M.decode_splits(N_LONG)
    nsg = M.gqa_splits(1, KV, ns, 1)
    part = torch.empty(H * ns * (AHD + 2), device="cuda")
    out = torch.full((1, H, AHD), float("nan"), device="cuda")
    M.attn_gqa(dev(qo), dc, H, KV, pos_tensor(pos), N_LONG, part, 1, nsg)
    M.attn_combine(part, None, out, H, nsg, LD, 1)
    M.turbo_out(out, dev(qg), H, LD, 1)
    torch.cuda.synchronize()
    rows = [(0, h) for h in range(H)]
    ref = rows_threaded(orc.attn_rows_f64, qo, qg, LD, H, hc, pos, rows)
    got = out.cpu().numpy()[0]
    err, mag = float(np.abs(got - ref).max()), float(np.abs(ref).max())
    report("configs[3] gqa+combine+turbo_out", splits=nsg, err=err, mag=mag, rel=err / mag)
    assert np.all(np.isfinite(got)) and err <= 1e-4 * mag
    # what attn_decode runs: the split kernel rotates its partials back, the combine gates them
    out.fill_(float("nan"))
    M.attn_gqa_out(dev(qo), dc, H, KV, pos_tensor(pos), N_LONG, part, 1, nsg)
    M.attn_combine(part, dev(qg), out, H, nsg, LD, 1)
    torch.cuda.synchronize()
    got = out.cpu().numpy()[0]
    err = float(np.abs(got - ref).max())
    report("configs[3] gqa_out+combine", splits=nsg, err=err, mag=mag, rel=err / mag)
    assert np.all(np.isfinite(got)) and err <= 1e-4 * mag


def test_config3_turbo_attn_decode(turbo_long):
    """The full step: raw q/k/v row of token 262143 -> front, append (row 262143 rewritten), split-K decode,
    combine, inverse rotation and gate. Checked against the oracle on the kernel's own qo and the cache it wrote."""
    import torch
    import moex_amd as M
    dc, _ = turbo_long
    pos = N_LONG - 1
    LQ = H * 2 * AHD + 2 * KV * AHD
    rng = np.random.default_rng(302)
    qkv = rng.standard_normal((1, LQ), dtype=np.float32)
    q_d = dev(qkv)
    qn = torch.zeros(AHD, dtype=torch.int16, device="cuda")
    ns = M.decode_splits(N_LONG)
    part = torch.empty(H * ns * (AHD + 2), device="cuda")
    qo = torch.empty((1, H, AHD), device="cuda")
    out = torch.full((1, H, AHD), float("nan"), device="cuda")
    M.attn_decode(q_d, q_d[:, H * 2 * AHD:], q_d[:, H * 2 * AHD + KV * AHD:], qn, qn, qo, dc, out, H, KV,
                  pos_tensor(pos), N_LONG, 64, 1e7, 1e-6, 1, LQ, None, part, ns)
    torch.cuda.synchronize()
    hc = download(dc)
    rows = [(0, h) for h in range(H)]
    ref = rows_threaded(orc.attn_rows_f64, qo.cpu().numpy(), qkv, LQ, H, hc, pos, rows)
    got = out.cpu().numpy()[0]
    err, mag = float(np.abs(got - ref).max()), float(np.abs(ref).max())
    report("configs[3] attn_decode", ns=ns, err=err, mag=mag, rel=err / mag)
    assert np.all(np.isfinite(got)) and err <= 1e-4 * mag


def test_config4_turbo_prefill(turbo_long):
    import torch
    import moex_amd as M
    dc, _ = turbo_long
    hc = download(dc)  # the attn_decode test above rewrote row 262143 with its own token
    T, pos0 = 2048, N_LONG - 2048
    print("configs[4]: turbo prefill T=2048 pos0=260096", flush=True)
    rng = np.random.default_rng(401)
    qo = _f16(rng.standard_normal((T, H, AHD), dtype=np.float32))
    qg = _f16(rng.standard_normal((T, LD), dtype=np.float32))
    out = torch.full((T, H, AHD), float("nan"), device="cuda")
    M.attn_fa(dev(qo), None, dc, out, H, KV, pos_tensor(pos0), N_LONG, LD, T)
    torch.cuda.synchronize()
    _prefill_gate("configs[4] attn_fa (rotated)", out.cpu().numpy(), qo, None, hc, pos0, T)
    M.turbo_out(out, dev(qg), H, LD, T)
    torch.cuda.synchronize()
    _prefill_gate("configs[4] attn_fa + turbo_out", out.cpu().numpy(), qo, qg, hc, pos0, T)


@pytest.mark.parametrize("Tq", [1, 4])
def test_config2_int8_decode_bench_data(Tq):
    """configs[2] on the benchmark's data: K/V ~ N(0,1) quantized by the library's append (bit-exact against the
    oracle over all 90000 rows), Q and gate ~ N(0,1) rounded to fp16, the last Tq positions of 90000 keys (causal
    among the Tq), through the split-K kernel + combine the benchmark times: 1e-4 of max|ref| over all heads."""
    import torch
    import moex_amd as M
    ctx = 90000
    print(f"configs[2]: int8 decode T={Tq} at {ctx} keys (N(0,1) data)", flush=True)
    dc, hc = _filled_cache(ctx, ctx + 64, 0, seed=200)
    rng = np.random.default_rng(201 + Tq)
    qo = _f16(rng.standard_normal((Tq, H, AHD), dtype=np.float32))
    qg = _f16(rng.standard_normal((Tq, LD), dtype=np.float32))
    ns = M.gqa_splits(Tq, KV, M.decode_splits(ctx))
    part = torch.empty(Tq * H * ns * (AHD + 2), device="cuda")
    out = torch.full((Tq, H, AHD), float("nan"), device="cuda")
    pos0 = ctx - Tq
    M.attn_gqa(dev(qo), dc, H, KV, pos_tensor(pos0), ctx + 64, part, Tq, ns)
    M.attn_combine(part, dev(qg), out, H, ns, LD, Tq)
    torch.cuda.synchronize()
    rows = [(t, h) for t in range(Tq) for h in range(H)]
    ref = rows_threaded(orc.attn_rows_f64, qo, qg, LD, H, hc, pos0, rows)
    got = np.stack([out.cpu().numpy()[t, h] for t, h in rows])
    err, mag = float(np.abs(got - ref).max()), float(np.abs(ref).max())
    report("configs[2] gqa+combine (N(0,1) data)", T=Tq, splits=ns, err=err, mag=mag, rel=err / mag)
    assert np.all(np.isfinite(got)) and err <= 1e-4 * mag
