"""The full attention step attn_decode (kernels.cuh:1846-1865): front + append + dispatch, int8 and turbo caches
written from the same N(0,1) q/k/v (tests/test_fa.cu:141-200):
  - turbo vs int8 outputs of the prefill chunk: cosine >= 0.97 (test_fa.cu:181);
  - the last token again through the split GQA decode and the per-head decode: within 2% of max |FA output|
    (test_fa.cu:198);
  - int8 chunk output against the fp64 oracle fed with the kernel's own qo and cache (test_fa.cu:114 rule).
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.gpu_util import AHD, H, KV, dev, download, pos_tensor, report, sample_rows

pytestmark = pytest.mark.gpu


def test_attn_decode_paths():
    import torch
    import moex_amd as M
    LQ = H * 2 * AHD + 2 * KV * AHD
    T, pos0 = 512, 1500
    ctx = pos0 + T + 8
    c8, ct = M.DeviceKVCache(KV, ctx, 0), M.DeviceKVCache(KV, ctx, 1)
    qn = torch.zeros(AHD, dtype=torch.int16, device="cuda")
    kn = torch.zeros(AHD, dtype=torch.int16, device="cuda")
    ns = 4
    qo = torch.empty((T, H, AHD), dtype=torch.float32, device="cuda")
    oa = torch.empty((T, H, AHD), dtype=torch.float32, device="cuda")
    ob = torch.empty_like(oa)
    part = torch.empty(T * H * ns * (AHD + 2), dtype=torch.float32, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(1)
    qkv = torch.empty((T, LQ), dtype=torch.float32, device="cuda")
    pos_d = torch.zeros(1, dtype=torch.int32, device="cuda")

    def run(c, out, p0, n, nsplit, pt, qov=qo):
        M.set_int(pos_d, p0)
        M.attn_decode(qkv, qkv[:, H * 2 * AHD:], qkv[:, H * 2 * AHD + KV * AHD:], qn, kn, qov, c, out, H, KV, pos_d,
                      ctx, 64, 1e7, 1e-6, n, LQ, None, pt, nsplit)
        torch.cuda.synchronize()

    for p in range(0, pos0, T):  # context before the chunk, the same rows in both caches
        n = min(T, pos0 - p)
        qkv.normal_(generator=g)
        run(c8, oa, p, n, 1, None)
        run(ct, ob, p, n, 1, None)
    qkv.normal_(generator=g)
    run(c8, oa, pos0, T, 1, None)
    qo8 = qo.clone()
    run(ct, ob, pos0, T, 1, None)
    a, b = oa.cpu().numpy().astype(np.float64), ob.cpu().numpy().astype(np.float64)
    cs = float((a * b).sum() / np.sqrt((a * a).sum() * (b * b).sum()))
    report("turbo vs int8 (FA path)", cosine=cs)
    assert np.all(np.isfinite(b)) and cs >= 0.97

    # int8 chunk vs the oracle on the kernel's own inputs
    hc = download(c8)
    q_host = qkv.cpu().numpy()
    rows = sample_rows(T)
    ref = orc.attn_rows_f64(qo8.cpu().numpy(), q_host, LQ, H, hc, pos0, rows)
    emu = orc.attn_rows_fa_emul(qo8.cpu().numpy(), q_host, LQ, H, hc, pos0, rows)
    got = np.stack([a[t, h] for t, h in rows])
    mag = float(np.abs(ref).max())
    e_new, e_ref = float(np.abs(got - ref).max()), float(np.abs(emu - ref).max())
    report("attn_decode int8 chunk vs fp64", e_new=e_new, e_ref=e_ref, mag=mag)
    assert e_new <= 2 * e_ref + 1e-3 * mag

    # the last token again through the decode paths (its K/V rows are rewritten with the same values)
    last = qkv[T - 1:T].clone()
    qkv[:1].copy_(last)
    d1 = torch.empty((1, H, AHD), dtype=torch.float32, device="cuda")
    d2 = torch.empty_like(d1)
    q1 = torch.empty((1, H, AHD), dtype=torch.float32, device="cuda")
    for cache, full in ((ct, b), (c8, a)):
        run(cache, d1, pos0 + T - 1, 1, ns, part, q1)   # GQA split + combine
        run(cache, d2, pos0 + T - 1, 1, 1, None, q1)    # ns = 1: split-K with the library's own partials
        f = full[T - 1]
        e1 = float(np.abs(d1.cpu().numpy()[0] - f).max())
        e2 = float(np.abs(d2.cpu().numpy()[0] - f).max())
        mg = float(np.abs(f).max())
        report("last token decode vs FA", turbo=cache.turbo, e_gqa=e1, e_heads=e2, mag=mg)
        assert e1 < 0.02 * mg and e2 < 0.02 * mg


def test_skip_flag_and_soft_errors():
    """g_skip makes the append/front and turbo_out return at once (kernels.cuh:1189,1732); argument errors go to the
    soft slot instead of exiting while it is installed (kernels.cuh:8-11)."""
    import ctypes
    import torch
    import moex_amd as M
    T, max_t = 4, 16
    cache = M.DeviceKVCache(KV, max_t, 0)
    cache.k.zero_(); cache.ks.zero_()
    LQ = H * 2 * AHD + 2 * KV * AHD
    k = torch.ones((T, LQ), dtype=torch.float32, device="cuda")
    M.set_skip(1)
    M.qk_norm_rope(k, k[:, H * 2 * AHD:], k[:, H * 2 * AHD + KV * AHD:], torch.zeros(AHD, dtype=torch.int16, device="cuda"),
                   torch.zeros(AHD, dtype=torch.int16, device="cuda"), torch.empty((T, H, AHD), device="cuda"),
                   cache, H, KV, pos_tensor(0), max_t, 64, 1e7, 1e-6, LQ, T)
    torch.cuda.synchronize()
    assert cache.ks.abs().sum().item() == 0
    M.set_skip(0)
    torch.cuda.synchronize()
    slot = ctypes.c_int(0)
    M.lib().moex_set_soft_error(ctypes.byref(slot))
    try:
        M.attn_fa(k, None, cache, k, 12, KV, pos_tensor(0), max_t, 0, T)  # H / KV == 6: unsupported
    finally:
        M.lib().moex_set_soft_error(None)
    assert slot.value == 1  # hipErrorInvalidValue


def _caches(M, torch, turbo, max_t, seed, n=2):
    """n caches with the same rows: int8 from the random int8 cache, turbo by appending the same random k / v rows"""
    from tests.gpu_util import random_int8_cache, upload
    if not turbo:
        hc = random_int8_cache(max_t, seed=seed)
        return hc, [upload(hc) for _ in range(n)]
    g = torch.Generator(device="cuda").manual_seed(seed)
    k = torch.randn((max_t, KV * AHD), generator=g, device="cuda")
    v = torch.randn((max_t, KV * AHD), generator=g, device="cuda")
    cs = []
    for _ in range(n):
        c = M.DeviceKVCache(KV, max_t, 1)
        M.kv_append(k, v, c, KV, pos_tensor(0), max_t, KV * AHD, max_t)
        cs.append(c)
    torch.cuda.synchronize()
    return download(cs[0]), cs


@pytest.mark.parametrize("turbo,T", [(0, 1), (1, 1), (0, 2), (0, 4), (1, 3)])
def test_skip_flag_fused_front(turbo, T):
    """With g_skip set, attn_decode's split-K step (whose split kernel runs the front and the appends in its prologue:
    T = 1, and int8 windows of up to 4) appends nothing, leaves qo as it was and attends with that qo, as the
    reference's attention after a skipped qk_norm_rope_k (kernels.cuh:1189) does: its output equals the split kernel
    + attn_combine on the same qo, bit for bit (turbo: the partials rotated back, as the step runs them)."""
    import torch
    import moex_amd as M
    pos, max_t = 3000, 3072
    hc, (dc,) = _caches(M, torch, turbo, max_t, 71, 1)
    rng = np.random.default_rng(72)
    LQ = H * 2 * AHD + 2 * KV * AHD
    qkv = dev(rng.standard_normal((T, LQ), dtype=np.float32))
    qo0 = rng.standard_normal((T, H, AHD), dtype=np.float32)
    qo = dev(qo0)
    qn = torch.zeros(AHD, dtype=torch.int16, device="cuda")
    ns = M.decode_splits(pos + T)
    assert ns > 1
    part = torch.empty(T * H * ns * (AHD + 2), device="cuda")
    out = torch.full((T, H, AHD), float("nan"), device="cuda")
    M.set_skip(1)
    try:
        M.attn_decode(qkv, qkv[:, H * 2 * AHD:], qkv[:, H * 2 * AHD + KV * AHD:], qn, qn, qo, dc, out, H, KV,
                      pos_tensor(pos), max_t, 64, 1e7, 1e-6, T, LQ, None, part, ns)
        torch.cuda.synchronize()
    finally:
        M.set_skip(0)
        torch.cuda.synchronize()
    after = download(dc)
    for a, b, name in ((after.k, hc.k, "k"), (after.v, hc.v, "v"), (after.ks, hc.ks, "ks"), (after.vs, hc.vs, "vs")):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"cache {name} changed under the skip flag"
    assert np.array_equal(qo.cpu().numpy(), qo0), "qo changed under the skip flag"
    nsg = M.gqa_splits(T, KV, ns, turbo)
    part2 = torch.empty(T * H * ns * (AHD + 2), device="cuda")
    out2 = torch.full((T, H, AHD), float("nan"), device="cuda")
    (M.attn_gqa_out if turbo else M.attn_gqa)(qo, dc, H, KV, pos_tensor(pos), max_t, part2, T, nsg)
    M.attn_combine(part2, qkv, out2, H, nsg, LQ, T)
    torch.cuda.synchronize()
    got, ref = out.cpu().numpy(), out2.cpu().numpy()
    report("skip flag, fused front", turbo=turbo, T=T, ns=nsg, same=bool(np.array_equal(got, ref)))
    assert np.all(np.isfinite(got)) and np.array_equal(got, ref)


@pytest.mark.parametrize("turbo", [0, 1])
@pytest.mark.parametrize("pos,ns", [(0, 4), (1, 2), (63, 2), (64, 2), (65, 7), (255, 3), (256, 128), (3000, 128),
                                    (5183, 5), (20480, 64), (89999, 128)])
def test_fused_front_matches_three_launches(pos, ns, turbo):
    """attn_decode's T = 1 split step runs the q/k front and the append inside the split kernel; the same step as
    three launches (qk_norm_rope, the split kernel, attn_combine) must give the same qo, cache rows and output, bit
    for bit. The positions put the new row alone in a split, alone in the short first chunk, at a chunk boundary and
    deep in the cache, and (pos 0) leave most splits empty."""
    import torch
    import moex_amd as M
    max_t = max(pos + 1, 1024)
    hc, (da, db) = _caches(M, torch, turbo, max_t, 81)
    rng = np.random.default_rng(82 + pos)
    LQ = H * 2 * AHD + 2 * KV * AHD
    qkv = dev(rng.standard_normal((1, LQ), dtype=np.float32))
    qn = dev((0.1 * rng.standard_normal(AHD)).astype(np.float16).view(np.int16))  # fp16 norm weights
    kn = dev((0.1 * rng.standard_normal(AHD)).astype(np.float16).view(np.int16))
    nsg = M.gqa_splits(1, KV, ns, turbo)
    part = torch.empty(H * ns * (AHD + 2), device="cuda")
    qa, qb = torch.full((1, H, AHD), float("nan"), device="cuda"), torch.full((1, H, AHD), float("nan"), device="cuda")
    oa, ob = torch.full((1, H, AHD), float("nan"), device="cuda"), torch.full((1, H, AHD), float("nan"), device="cuda")
    pd = pos_tensor(pos)
    M.attn_decode(qkv, qkv[:, H * 2 * AHD:], qkv[:, H * 2 * AHD + KV * AHD:], qn, kn, qa, da, oa, H, KV, pd, max_t,
                  64, 1e7, 1e-6, 1, LQ, None, part, ns)
    M.qk_norm_rope(qkv, qkv[:, H * 2 * AHD:], qkv[:, H * 2 * AHD + KV * AHD:], qn, kn, qb, db, H, KV, pd, max_t,
                   64, 1e7, 1e-6, LQ, 1)
    (M.attn_gqa_out if turbo else M.attn_gqa)(qb, db, H, KV, pd, max_t, part, 1, nsg)
    M.attn_combine(part, qkv, ob, H, nsg, LQ, 1)
    torch.cuda.synchronize()
    ca, cb = download(da), download(db)
    for x, y, name in ((ca.k, cb.k, "k"), (ca.v, cb.v, "v"), (ca.ks, cb.ks, "ks"), (ca.vs, cb.vs, "vs")):
        assert np.array_equal(x.view(np.uint8), y.view(np.uint8)), f"cache {name} differs"
    ga, gb = oa.cpu().numpy(), ob.cpu().numpy()
    report("fused front vs three launches", turbo=turbo, pos=pos, ns=nsg, maxdiff=float(np.abs(ga - gb).max()))
    assert np.array_equal(qa.cpu().numpy(), qb.cpu().numpy())
    assert np.all(np.isfinite(ga)) and np.array_equal(ga, gb)


def _crossing_pos(start, T, nsg):
    """the first position from start whose window [pos, pos + T) straddles a split boundary of nsg splits (windows
    only straddle one while the splits are shorter than about nsg + T keys; past that, the last one below start)"""
    def crosses(pos):
        L = -(-(pos + T) // nsg)
        return any(pos < b < pos + T for b in range(L, pos + T, L))
    for pos in range(start, start + 20000):
        if crosses(pos):
            return pos
    for pos in range(start, 0, -1):
        if crosses(pos):
            return pos
    raise AssertionError("no crossing window")


@pytest.mark.parametrize("turbo", [0, 1])
@pytest.mark.parametrize("T", [2, 3, 4])
@pytest.mark.parametrize("case", ["p0", "cross_small", "p100", "cross_3000", "p20480", "end", "cross_12000"])
def test_fused_front_window_matches_three_launches(T, case, turbo):
    """attn_decode's MTP step (T = 2..4, split-K; int8, and turbo with a workgroup per token) runs the q/k front and
    the appends inside the split kernel;
    the same step as three launches (qk_norm_rope, the split kernel, attn_combine) must give the same qo, cache rows
    and output, bit for bit. Cases: every row in a split's first chunks (pos 0), windows across a split boundary
    (some of the new rows at the start of the next split, whose first chunks must wait for them), short and deep
    caches."""
    import torch
    import moex_amd as M
    ns = {"p0": 4, "cross_small": 2, "p100": 3, "cross_3000": 128, "p20480": 64, "end": 128, "cross_12000": 128}[case]
    nsg = M.gqa_splits(T, KV, ns, turbo)
    pos = {"p0": 0, "cross_small": None, "p100": 100, "cross_3000": None, "p20480": 20480, "end": 89996 - T,
           "cross_12000": None}[case]
    if pos is None:
        pos = _crossing_pos({"cross_small": 1, "cross_3000": 3000, "cross_12000": 12000}[case], T, nsg)
    max_t = max(pos + T + 8, 1024)
    hc, (da, db) = _caches(M, torch, turbo, max_t, 91)
    rng = np.random.default_rng(92 + pos + T)
    LQ = H * 2 * AHD + 2 * KV * AHD
    qkv = dev(rng.standard_normal((T, LQ), dtype=np.float32))
    qn = dev((0.1 * rng.standard_normal(AHD)).astype(np.float16).view(np.int16))
    kn = dev((0.1 * rng.standard_normal(AHD)).astype(np.float16).view(np.int16))
    part = torch.empty(T * H * ns * (AHD + 2), device="cuda")
    qa, qb = torch.full((T, H, AHD), float("nan"), device="cuda"), torch.full((T, H, AHD), float("nan"), device="cuda")
    oa, ob = torch.full((T, H, AHD), float("nan"), device="cuda"), torch.full((T, H, AHD), float("nan"), device="cuda")
    pd = pos_tensor(pos)
    M.attn_decode(qkv, qkv[:, H * 2 * AHD:], qkv[:, H * 2 * AHD + KV * AHD:], qn, kn, qa, da, oa, H, KV, pd, max_t,
                  64, 1e7, 1e-6, T, LQ, None, part, ns)
    M.qk_norm_rope(qkv, qkv[:, H * 2 * AHD:], qkv[:, H * 2 * AHD + KV * AHD:], qn, kn, qb, db, H, KV, pd, max_t,
                   64, 1e7, 1e-6, LQ, T)
    (M.attn_gqa_out if turbo else M.attn_gqa)(qb, db, H, KV, pd, max_t, part, T, nsg)
    M.attn_combine(part, qkv, ob, H, nsg, LQ, T)
    torch.cuda.synchronize()
    ca, cb = download(da), download(db)
    for x, y, name in ((ca.k, cb.k, "k"), (ca.v, cb.v, "v"), (ca.ks, cb.ks, "ks"), (ca.vs, cb.vs, "vs")):
        assert np.array_equal(x.view(np.uint8), y.view(np.uint8)), f"cache {name} differs"
    ga, gb = oa.cpu().numpy(), ob.cpu().numpy()
    report("fused front window vs three launches", turbo=turbo, T=T, pos=pos, ns=nsg, maxdiff=float(np.abs(ga - gb).max()))
    assert np.array_equal(qa.cpu().numpy(), qb.cpu().numpy())
    assert np.all(np.isfinite(ga)) and np.array_equal(ga, gb)


@pytest.mark.parametrize("turbo", [0, 1])
@pytest.mark.parametrize("T", [1, 2])
def test_one_split_call_runs_split_k(turbo, T):
    """attn_decode with ns = 1 (the reference's one-split path, no partials) runs the split-K kernels with partials
    of the library's own, moex_gqa_splits(T, KV, moex_decode_splits(max_t)) splits: the same bits as a call that
    passes those splits and a partial buffer."""
    import torch
    import moex_amd as M
    LQ = H * 2 * AHD + 2 * KV * AHD
    n = 20000
    outs = []
    for ns in (1, M.decode_splits(n + 64)):
        c = M.DeviceKVCache(KV, n + 64, turbo)
        g = torch.Generator(device="cuda").manual_seed(40)
        k = torch.randn((n, KV * AHD), generator=g, device="cuda")
        v = torch.randn((n, KV * AHD), generator=g, device="cuda")
        M.kv_append(k, v, c, KV, pos_tensor(0), c.max_t, KV * AHD, n)
        qkv = torch.randn((T, LQ), generator=g, device="cuda")
        qn = torch.zeros(AHD, dtype=torch.int16, device="cuda")
        qo = torch.empty((T, H, AHD), device="cuda")
        out = torch.full((T, H, AHD), float("nan"), device="cuda")
        part = torch.empty(T * H * ns * (AHD + 2), device="cuda") if ns > 1 else None
        M.attn_decode(qkv, qkv[:, H * 2 * AHD:], qkv[:, H * 2 * AHD + KV * AHD:], qn, qn, qo, c, out, H, KV,
                      pos_tensor(n), c.max_t, 64, 1e7, 1e-6, T, LQ, None, part, ns)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    report("attn_decode ns=1 vs splits", turbo=turbo, T=T, maxdiff=float(np.abs(outs[0] - outs[1]).max()))
    assert np.all(np.isfinite(outs[0])) and np.array_equal(outs[0], outs[1])
