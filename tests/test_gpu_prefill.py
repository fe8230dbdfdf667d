"""Chunked causal GQA prefill: attn_fa (kernels.cuh:1443-1728) and the int8 fallback attn_prefill (:1331-1441)
against the fp64 oracle, with the acceptance rule of tests/test_fa.cu:114:

    e_new <= 2 * e_ref + 1e-3 * mag

where e_ref is the error of the reference kernel's arithmetic (the oracle's precision model of attn_fa_k: fp16 Q,
fp16 P * vscale, fp32 softmax) on the same rows, mag = max |ref|. Cases and row sample follow test_fa.cu:82,95.
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.gpu_util import AHD, H, KV, LD, dev, download, pos_tensor, random_int8_cache, report, sample_rows, upload

pytestmark = pytest.mark.gpu

CASES = [(0, 37), (0, 1024), (5, 3), (1000, 100), (4093, 2048), (30000, 2048), (32768, 2048)]


@pytest.fixture(scope="module")
def setup():
    max_t = 34816 + 64
    hc = random_int8_cache(max_t, seed=1)
    dc = upload(hc)
    rng = np.random.default_rng(2)
    qo = rng.uniform(-2, 2, (2048, H, AHD)).astype(np.float32)
    qg = rng.uniform(-2, 2, (2048, LD)).astype(np.float32)
    return hc, dc, qo, qg, dev(qo), dev(qg)


def _gate(name, out, qo, qg, hc, pos0, T):
    rows = sample_rows(T)
    ref = orc.attn_rows_f64(qo, qg, LD, H, hc, pos0, rows)
    emu = orc.attn_rows_fa_emul(qo, qg, LD, H, hc, pos0, rows)
    got = np.stack([out[t, h] for t, h in rows])
    mag = float(np.abs(ref).max())
    e_new, e_ref = float(np.abs(got - ref).max()), float(np.abs(emu - ref).max())
    report(name, pos0=pos0, T=T, e_new=e_new, e_ref=e_ref, mag=mag)
    assert np.all(np.isfinite(got))
    assert e_new <= 2.0 * e_ref + 1e-3 * mag
    return e_new


@pytest.mark.parametrize("pos0,T", CASES)
def test_fa_int8(setup, pos0, T):
    import torch
    import moex_amd as M
    hc, dc, qo, qg, qo_d, qg_d = setup
    out = torch.zeros((T, H, AHD), dtype=torch.float32, device="cuda")
    M.attn_fa(qo_d, qg_d, dc, out, H, KV, pos_tensor(pos0), dc.max_t, LD, T)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    _gate("fa int8", o, qo, qg, hc, pos0, T)
    # every row of the chunk is finite and written
    assert np.all(np.isfinite(o)) and np.all(np.abs(o).max(axis=-1) > 0)


@pytest.mark.parametrize("pos0,T", [(32000, 64), (5000, 3), (34000, 17), (0, 37), (30000, 8)])
def test_fa_short_chunks_on_decode_kernels(setup, pos0, T, monkeypatch):
    """int8 chunks of at most 64 tokens run on the split-K decode kernels and the gated combine: the test_fa.cu gate,
    and agreement with the FA kernel on the same chunk (MOEX_FA_GQA_MAXT=0) to the FA split tolerance."""
    import torch
    import moex_amd as M
    hc, dc, qo, qg, qo_d, qg_d = setup
    outs = {}
    for maxt in ("64", "0"):
        monkeypatch.setenv("MOEX_FA_GQA_MAXT", maxt)
        out = torch.full((T, H, AHD), float("nan"), dtype=torch.float32, device="cuda")
        M.attn_fa(qo_d, qg_d, dc, out, H, KV, pos_tensor(pos0), dc.max_t, LD, T)
        torch.cuda.synchronize()
        outs[maxt] = out.cpu().numpy()
        assert np.all(np.isfinite(outs[maxt]))
        _gate(f"fa int8 short, gqa bound {maxt}", outs[maxt], qo, qg, hc, pos0, T)
    mag = float(np.abs(outs["0"]).max())
    d = float(np.abs(outs["64"] - outs["0"]).max())
    report("fa short: decode kernels vs FA kernel", pos0=pos0, T=T, maxdiff=d, mag=mag)
    assert d <= 2e-3 * mag


@pytest.mark.parametrize("pos0,T", [(32000, 64), (0, 1024), (5000, 3), (20000, 200), (34000, 17)])
def test_fa_key_split(setup, pos0, T, monkeypatch):
    """Chunks whose token tiles leave the chip underfilled (KV x tiles < CUs) split each token tile's keys over
    several workgroups, merged by a second kernel: both results meet the gate, and they agree with the unsplit kernel
    (MOEX_FA_SPLIT=1). The FA kernel also for the chunks of at most 64 tokens (MOEX_FA_GQA_MAXT=0), which by default
    run on the decode kernels."""
    import torch
    import moex_amd as M
    hc, dc, qo, qg, qo_d, qg_d = setup
    monkeypatch.setenv("MOEX_FA_GQA_MAXT", "0")
    outs = {}
    for cap in ("32", "1"):
        monkeypatch.setenv("MOEX_FA_SPLIT", cap)
        out = torch.full((T, H, AHD), float("nan"), dtype=torch.float32, device="cuda")
        M.attn_fa(qo_d, qg_d, dc, out, H, KV, pos_tensor(pos0), dc.max_t, LD, T)
        torch.cuda.synchronize()
        outs[cap] = out.cpu().numpy()
        e = _gate(f"fa int8 split cap {cap}", outs[cap], qo, qg, hc, pos0, T)
        assert np.all(np.isfinite(outs[cap]))
    mag = float(np.abs(outs["1"]).max())
    d = float(np.abs(outs["32"] - outs["1"]).max())
    report("fa split vs unsplit", pos0=pos0, T=T, maxdiff=d, mag=mag)
    assert d <= 2e-3 * mag


@pytest.mark.parametrize("pos0,T", CASES[:5])
def test_prefill_fallback_int8(setup, pos0, T):
    import torch
    import moex_amd as M
    hc, dc, qo, qg, qo_d, qg_d = setup
    out = torch.zeros((T, H, AHD), dtype=torch.float32, device="cuda")
    M.attn_prefill(qo_d, qg_d, dc, out, H, KV, pos_tensor(pos0), dc.max_t, LD, T)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    _gate("prefill(K7P) int8", o, qo, qg, hc, pos0, T)
    # FA vs the fallback over every row (test_fa.cu:107 prints it; K7P vs per-row decode is 5e-3, test_kernels.cu:809)
    o2 = torch.zeros_like(out)
    M.attn_fa(qo_d, qg_d, dc, o2, H, KV, pos_tensor(pos0), dc.max_t, LD, T)
    torch.cuda.synchronize()
    e_ab = float(np.abs(o2.cpu().numpy() - o).max())
    report("fa vs fallback", pos0=pos0, T=T, e_ab=e_ab)
    assert e_ab <= 5e-3 * float(np.abs(o).max())


@pytest.fixture(scope="module")
def turbo_setup():
    import torch
    import moex_amd as M
    max_t, n = 6208, 6144
    dc = M.DeviceKVCache(KV, max_t, 1)
    g = torch.Generator(device="cuda").manual_seed(9)
    k = torch.randn((n, KV * AHD), generator=g, device="cuda")
    v = torch.randn((n, KV * AHD), generator=g, device="cuda")
    M.kv_append(k, v, dc, KV, pos_tensor(0), max_t, KV * AHD, n)
    torch.cuda.synchronize()
    hc = download(dc)
    rng = np.random.default_rng(3)
    qo = rng.standard_normal((2048, H, AHD)).astype(np.float32)
    qg = rng.standard_normal((2048, LD)).astype(np.float32)
    return hc, dc, qo, qg, dev(qo), dev(qg)


@pytest.mark.parametrize("gqa_maxt", ["64", "0"])
@pytest.mark.parametrize("pos0,T", [(0, 37), (5, 3), (1000, 100), (4096, 2048), (6000, 16), (3000, 8)])
def test_fa_turbo(turbo_setup, pos0, T, gqa_maxt, monkeypatch):
    """No gate (turbo: attn_fa writes the rotated-domain output), then turbo_out -> the full turbo reference. Chunks
    of at most 16 tokens run on the turbo split-K decode kernel by default (bound 64 / 4), on the FA kernel with
    MOEX_FA_GQA_MAXT=0."""
    import torch
    import moex_amd as M
    monkeypatch.setenv("MOEX_FA_GQA_MAXT", gqa_maxt)
    hc, dc, qo, qg, qo_d, qg_d = turbo_setup
    out = torch.zeros((T, H, AHD), dtype=torch.float32, device="cuda")
    M.attn_fa(qo_d, None, dc, out, H, KV, pos_tensor(pos0), dc.max_t, LD, T)
    torch.cuda.synchronize()
    _gate("fa turbo (rotated)", out.cpu().numpy(), qo, None, hc, pos0, T)
    M.turbo_out(out, qg_d, H, LD, T)
    torch.cuda.synchronize()
    _gate("fa turbo + turbo_out", out.cpu().numpy(), qo, qg, hc, pos0, T)


@pytest.mark.parametrize("Hq,KVq,pos0,T", [(16, 4, 1000, 100), (16, 1, 300, 37), (32, 1, 0, 64), (2, 2, 500, 9),
                                           (16, 4, 0, 3)])
def test_prefill_fallback_other_groups(Hq, KVq, pos0, T):
    """attn_prefill takes any GQA group G = H / KV that divides 32 (kernels.cuh:1856; its kernel puts 32 / G tokens
    of G heads in a workgroup): G = 4, 16, 32 and 1 against the fp64 oracle with the test_fa.cu:114 rule."""
    import torch
    import moex_amd as M
    max_t = pos0 + T + 40
    hc = random_int8_cache(max_t, seed=31 + Hq + KVq, kv=KVq)
    dc = upload(hc)
    rng = np.random.default_rng(32)
    ld = Hq * 2 * AHD
    qo = rng.uniform(-2, 2, (T, Hq, AHD)).astype(np.float32)
    qg = rng.uniform(-2, 2, (T, ld)).astype(np.float32)
    out = torch.full((T, Hq, AHD), float("nan"), dtype=torch.float32, device="cuda")
    M.attn_prefill(dev(qo), dev(qg), dc, out, Hq, KVq, pos_tensor(pos0), max_t, ld, T)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    rows = sample_rows(T, range(Hq))
    ref = orc.attn_rows_f64(qo, qg, ld, Hq, hc, pos0, rows)
    emu = orc.attn_rows_fa_emul(qo, qg, ld, Hq, hc, pos0, rows)
    got = np.stack([o[t, h] for t, h in rows])
    mag = float(np.abs(ref).max())
    e_new, e_ref = float(np.abs(got - ref).max()), float(np.abs(emu - ref).max())
    report("prefill(K7P) G", G=Hq // KVq, pos0=pos0, T=T, e_new=e_new, e_ref=e_ref, mag=mag)
    assert np.all(np.isfinite(o)) and e_new <= 2.0 * e_ref + 1e-3 * mag
