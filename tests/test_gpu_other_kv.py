"""The GQA-8 kernels at kv head counts other than the bench's 2 (H = 8 KV): 1, 3, 4 and 8 kv heads.

attn_fa (kernels.cuh:1443-1728) and the split-K decode (attn_gqa_k + attn_combine_k, :1744-1844, :1317-1329) map
work to workgroups by kv head: the FA grid puts each kv head on 8 / KV of the eight XCDs when KV divides 8 (a plain
order otherwise), pairs heavy and light token tiles when KV x tiles fills the chip once, splits keys when it does not,
and the decode kernels take KV x splits workgroups. Each case below runs one of these layouts and is checked against
the fp64 oracle with the test_fa.cu:114 gate (prefill) or 1e-4 of max |ref| (decode, test_kernels.cu:849).
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.gpu_util import AHD, dev, pos_tensor, random_int8_cache, report, sample_rows

pytestmark = pytest.mark.gpu


def _setup(KV, max_t, T, seed):
    H = 8 * KV
    ld = H * 2 * AHD
    hc = random_int8_cache(max_t, seed=seed, kv=KV)
    from tests.gpu_util import upload
    dc = upload(hc)
    rng = np.random.default_rng(seed + 1)
    qo = rng.uniform(-2, 2, (T, H, AHD)).astype(np.float32)
    qg = rng.uniform(-2, 2, (T, ld)).astype(np.float32)
    return H, ld, hc, dc, qo, qg


# (KV, pos0, T): KV x token tiles <= 256 with >= 2 tiles -> heavy/light pairs; short -> key splits; long -> one
# workgroup per token tile (two waves of the chip)
FA_CASES = [(1, 0, 4096), (1, 3000, 1000), (4, 0, 1024), (4, 700, 130), (3, 0, 1360), (3, 2000, 64), (4, 0, 2048),
            (1, 5000, 17), (8, 0, 512), (8, 1000, 2048)]


@pytest.mark.parametrize("KV,pos0,T", FA_CASES)
def test_fa_other_kv(KV, pos0, T, monkeypatch):
    import torch
    import moex_amd as M
    monkeypatch.setenv("MOEX_FA_GQA_MAXT", "0")  # the FA kernel itself also for the 17-token chunk
    H, ld, hc, dc, qo, qg = _setup(KV, pos0 + T + 40, T, seed=60 + KV + T)
    out = torch.full((T, H, AHD), float("nan"), dtype=torch.float32, device="cuda")
    M.attn_fa(dev(qo), dev(qg), dc, out, H, KV, pos_tensor(pos0), dc.max_t, ld, T)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.all(np.isfinite(o))
    rows = sample_rows(T, range(H))
    ref = orc.attn_rows_f64(qo, qg, ld, H, hc, pos0, rows)
    emu = orc.attn_rows_fa_emul(qo, qg, ld, H, hc, pos0, rows)
    got = np.stack([o[t, h] for t, h in rows])
    mag = float(np.abs(ref).max())
    e_new, e_ref = float(np.abs(got - ref).max()), float(np.abs(emu - ref).max())
    report("fa other kv", KV=KV, pos0=pos0, T=T, e_new=e_new, e_ref=e_ref, mag=mag)
    assert e_new <= 2.0 * e_ref + 1e-3 * mag


@pytest.mark.parametrize("KV,pos,T", [(1, 20000, 1), (4, 20000, 1), (3, 9000, 1), (1, 20000, 4), (4, 5000, 2),
                                      (8, 20000, 1), (8, 3000, 4)])
def test_decode_other_kv(KV, pos, T):
    """Split-K decode over KV x splits workgroups, then the gated combine; T query tokens at positions pos .. pos+T-1
    (each sees its own prefix)."""
    import torch
    import moex_amd as M
    H, ld, hc, dc, qo, qg = _setup(KV, pos + T + 64, T, seed=70 + KV + T)
    ns = M.gqa_splits(T, KV, M.decode_splits(pos + T))
    part = torch.empty(T * H * ns * (AHD + 2), dtype=torch.float32, device="cuda")
    out = torch.full((T, H, AHD), float("nan"), dtype=torch.float32, device="cuda")
    M.attn_gqa(dev(qo), dc, H, KV, pos_tensor(pos), dc.max_t, part, T, ns)
    M.attn_combine(part, dev(qg), out, H, ns, ld, T)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    rows = [(t, h) for t in range(T) for h in range(H)]
    ref = orc.attn_rows_f64(qo, qg, ld, H, hc, pos, rows)
    got = np.stack([o[t, h] for t, h in rows])
    e = float(np.abs(got - ref).max())
    mag = float(np.abs(ref).max())
    report("decode other kv", KV=KV, pos=pos, T=T, ns=ns, err=e, mag=mag)
    assert np.all(np.isfinite(o)) and e <= 1e-4 * mag


@pytest.mark.parametrize("KV,pos0,T", [(1, 0, 2048), (4, 100, 1000)])
def test_turbo_other_kv(KV, pos0, T):
    """TurboQuant caches (appended by the product's kernel, read back for the oracle): attn_fa's rotated-domain output
    and one split-K decode token at the end of the chunk, at 1 and 4 kv heads."""
    import torch
    import moex_amd as M
    from tests.gpu_util import download
    H = 8 * KV
    n = pos0 + T + 1
    max_t = n + 63
    dc = M.DeviceKVCache(KV, max_t, 1)
    g = torch.Generator(device="cuda").manual_seed(80 + KV)
    k = torch.randn((n, KV * AHD), generator=g, device="cuda")
    v = torch.randn((n, KV * AHD), generator=g, device="cuda")
    M.kv_append(k, v, dc, KV, pos_tensor(0), max_t, KV * AHD, n)
    torch.cuda.synchronize()
    hc = download(dc)
    rng = np.random.default_rng(81 + KV)
    qo = rng.standard_normal((T + 1, H, AHD)).astype(np.float32)
    out = torch.full((T, H, AHD), float("nan"), dtype=torch.float32, device="cuda")
    M.attn_fa(dev(qo[:T]), None, dc, out, H, KV, pos_tensor(pos0), max_t, H * 2 * AHD, T)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    rows = sample_rows(T, range(H))
    ref = orc.attn_rows_f64(qo[:T], None, H * 2 * AHD, H, hc, pos0, rows)
    emu = orc.attn_rows_fa_emul(qo[:T], None, H * 2 * AHD, H, hc, pos0, rows)
    got = np.stack([o[t, h] for t, h in rows])
    mag = float(np.abs(ref).max())
    e_new, e_ref = float(np.abs(got - ref).max()), float(np.abs(emu - ref).max())
    report("fa turbo other kv", KV=KV, pos0=pos0, T=T, e_new=e_new, e_ref=e_ref, mag=mag)
    assert np.all(np.isfinite(o)) and e_new <= 2.0 * e_ref + 1e-3 * mag
    # one decode token at position pos0 + T over the same cache (partials in the rotated domain, as attn_gqa_k)
    pos = pos0 + T
    ns = M.gqa_splits(1, KV, M.decode_splits(pos + 1), 1)
    part = torch.empty(H * ns * (AHD + 2), dtype=torch.float32, device="cuda")
    od = torch.full((1, H, AHD), float("nan"), dtype=torch.float32, device="cuda")
    M.attn_gqa(dev(qo[T:]), dc, H, KV, pos_tensor(pos), max_t, part, 1, ns)
    M.attn_combine(part, None, od, H, ns, H * 2 * AHD, 1)
    torch.cuda.synchronize()
    refd = orc.attn_rows_f64(qo[T:], None, H * 2 * AHD, H, hc, pos, [(0, h) for h in range(H)])
    e = float(np.abs(od.cpu().numpy()[0] - refd).max())
    report("decode turbo other kv", KV=KV, pos=pos, ns=ns, err=e, mag=float(np.abs(refd).max()))
    assert e <= 1e-4 * float(np.abs(refd).max())


@pytest.mark.parametrize("KV,cus,T", [(3, 255, 1360), (3, 258, 1376), (1, 255, 4080)])
def test_pairs_other_kv(KV, cus, T, monkeypatch):
    """Pair grids at kv head counts whose layout the chip's CU count does not reach (planned as for `cus` CUs,
    MOEX_FA_CUS): 3 kv heads take the plain block order (3 does not divide the 8 XCDs), odd tile counts leave a middle
    tile alone. The test_fa.cu:114 gate against the oracle."""
    import torch
    import moex_amd as M
    monkeypatch.setenv("MOEX_FA_CUS", str(cus))
    pos0 = 100
    H, ld, hc, dc, qo, qg = _setup(KV, pos0 + T + 40, T, seed=90 + KV + T)
    out = torch.full((T, H, AHD), float("nan"), dtype=torch.float32, device="cuda")
    M.attn_fa(dev(qo), dev(qg), dc, out, H, KV, pos_tensor(pos0), dc.max_t, ld, T)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.all(np.isfinite(o))
    rows = sample_rows(T, range(H))
    ref = orc.attn_rows_f64(qo, qg, ld, H, hc, pos0, rows)
    emu = orc.attn_rows_fa_emul(qo, qg, ld, H, hc, pos0, rows)
    got = np.stack([o[t, h] for t, h in rows])
    mag = float(np.abs(ref).max())
    e_new, e_ref = float(np.abs(got - ref).max()), float(np.abs(emu - ref).max())
    report("fa pairs other kv", KV=KV, cus=cus, T=T, e_new=e_new, e_ref=e_ref, mag=mag)
    assert e_new <= 2.0 * e_ref + 1e-3 * mag
