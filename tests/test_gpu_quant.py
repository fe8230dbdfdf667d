"""KV quantize-append parity (kernels.cuh:1185-1236): codes and scales/norms bit-exact against the oracle; the
query/key front (RMSNorm(1+w) + partial RoPE) within 1e-5 relative (tests/test_kernels.cu:773)."""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.gpu_util import AHD, H, KV, dev, download, pos_tensor, report

pytestmark = pytest.mark.gpu


def _rows(T, seed):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((T, KV * AHD)).astype(np.float32)
    v = rng.standard_normal((T, KV * AHD)).astype(np.float32)
    scales = np.geomspace(1e-4, 1e4, T).astype(np.float32)
    k *= scales[:, None]
    v *= scales[::-1, None]
    k[3] = 0.0                    # zero row: scale 1 / norm 0
    v[4, :AHD] = 0.0
    k[5, :AHD] = 1.0              # constant row
    k[6, :AHD] = np.linspace(-127, 127, AHD, dtype=np.float32)  # exact quotients: ties to even
    k[6, 7] = 2.5
    k[7, AHD:] = 1e-30            # tiny half norms (turbo: the 1e-20 guard)
    v[8, 128:AHD] = 0.0           # one zero half (turbo)
    return k, v


@pytest.mark.parametrize("turbo", [0, 1])
def test_append_bitexact(turbo):
    import torch
    import moex_amd as M
    T, pos0, max_t = 96, 7, 128
    k, v = _rows(T, 11 + turbo)
    cache = M.DeviceKVCache(KV, max_t, turbo)
    M.kv_append(dev(k), dev(v), cache, KV, pos_tensor(pos0), max_t, KV * AHD, T)
    torch.cuda.synchronize()
    got = download(cache)
    ref = orc.HostCache(KV, max_t, turbo)
    orc.kv_append(ref, k, v, KV * AHD, T, pos0)
    sl = slice(pos0, pos0 + T)
    for name in ("k", "v"):
        a, b = getattr(got, name)[:, sl], getattr(ref, name)[:, sl]
        bad = np.argwhere(a != b)
        assert bad.size == 0, f"{name} codes differ at {bad[:5].tolist()}"
    for name in ("ks", "vs"):
        a, b = getattr(got, name)[:, sl], getattr(ref, name)[:, sl]
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), name
    report("append", turbo=turbo, rows=T * KV)


@pytest.mark.parametrize("turbo,pos0", [(0, 0), (1, 0), (0, 1000), (1, 1000)])
def test_qk_norm_rope_front(turbo, pos0):
    """1e-5 relative at positions 0..23 (the golden positions of test_kernels.cu:742-785 are 0..11). At position
    ~1000 the fp32 angle pos * powf(theta, -2j/rot) itself (kernels.cuh:1203, the reference's own arithmetic) is
    off by up to ~pos * 2^-23 rad from the exact angle, so the bound there is 2e-4."""
    import torch
    import moex_amd as M
    T, max_t, rot, theta, eps = 24, 1100, 64, 1e7, 1e-6
    tol = 1e-5 if pos0 == 0 else 2e-4
    rng = np.random.default_rng(20 + turbo)
    LQ = H * 2 * AHD + 2 * KV * AHD
    qkv = (rng.standard_normal((T, LQ)) * 2).astype(np.float32)
    qn = (rng.standard_normal(AHD) * 0.1).astype(np.float16)
    kn = (rng.standard_normal(AHD) * 0.1).astype(np.float16)
    d = dev(qkv)
    qo = torch.zeros((T, H, AHD), dtype=torch.float32, device="cuda")
    cache = M.DeviceKVCache(KV, max_t, turbo)
    M.qk_norm_rope(d, d[:, H * 2 * AHD:], d[:, H * 2 * AHD + KV * AHD:], dev(qn.view(np.uint16)),
                   dev(kn.view(np.uint16)), qo, cache, H, KV, pos_tensor(pos0), max_t, rot, theta, eps, LQ, T)
    torch.cuda.synchronize()
    qg = qo.cpu().numpy()
    err = 0.0
    for t in range(T):
        for h in range(H):
            ref = orc.qk_norm_rope_row(qkv[t, h * 2 * AHD: h * 2 * AHD + AHD], qn.view(np.uint16), pos0 + t, rot,
                                       theta, eps, wht_fwd=bool(turbo))
            err = max(err, float(np.abs(qg[t, h] - ref).max() / np.abs(ref).max()))
    report("qk_norm_rope query", turbo=turbo, pos0=pos0, rel=err)
    assert err < tol
    # keys: the oracle quantizes its own (fp64-front) post-RoPE rows; codes agree except at rounding boundaries
    got = download(cache)
    kpost = np.stack([np.concatenate([orc.qk_norm_rope_row(qkv[t, H * 2 * AHD + h * AHD: H * 2 * AHD + (h + 1) * AHD],
                                                           kn.view(np.uint16), pos0 + t, rot, theta, eps)
                                      for h in range(KV)]) for t in range(T)])
    vraw = qkv[:, H * 2 * AHD + KV * AHD:]
    ref = orc.HostCache(KV, max_t, turbo)
    orc.kv_append(ref, kpost, vraw, KV * AHD, T, pos0)
    sl = slice(pos0, pos0 + T)
    # every code that differs must sit at a decision boundary within the front's own error (tol relative to the row's
    # largest value): a rounding tie of x / sk for int8, a centroid threshold of the rotated unit half-row for turbo
    tb = orc.tables()
    bad = 0
    ndiff = 0
    for t in range(T):
        for h in range(KV):
            x = kpost[t, h * AHD:(h + 1) * AHD].astype(np.float64)
            gk, rk = got.k[h, pos0 + t], ref.k[h, pos0 + t]
            if np.array_equal(gk, rk):
                continue
            eps_x = tol * np.abs(x).max()
            if not turbo:
                sk = np.abs(x).max() / 127.0
                q = x / sk
                diff = np.nonzero(gk != rk)[0]
                ndiff += diff.size
                near = np.abs(np.abs(q[diff] - np.floor(q[diff])) - 0.5) < 2 * eps_x / sk + 1e-6
                bad += int(np.sum(~near | (np.abs(gk[diff].astype(int) - rk[diff].astype(int)) != 1)))
            else:
                gi, _ = orc.turbo_unpack(gk.view(np.uint8), np.zeros(96, np.uint8))
                ri, _ = orc.turbo_unpack(rk.view(np.uint8), np.zeros(96, np.uint8))
                xn = np.concatenate([x[b * 128:(b + 1) * 128] / np.linalg.norm(x[b * 128:(b + 1) * 128])
                                     for b in range(2)]).astype(np.float32)
                r = orc.wht(xn).astype(np.float64)
                diff = np.nonzero(gi != ri)[0]
                ndiff += diff.size
                for d in diff:
                    lo_i, hi_i = sorted((int(gi[d]), int(ri[d])))
                    n = np.linalg.norm(x[(d // 128) * 128:(d // 128 + 1) * 128])
                    ok = hi_i == lo_i + 1 and abs(r[d] - tb["M4"][lo_i]) < 12 * eps_x / n + 1e-6
                    bad += int(not ok)
    report("qk_norm_rope keys", turbo=turbo, pos0=pos0, codes_differing=ndiff, unexplained=bad)
    assert bad == 0
    assert np.array_equal(got.v[:, sl], ref.v[:, sl])  # V is not normalized: bit-exact
    assert np.allclose(got.ks[:, sl], ref.ks[:, sl], rtol=1e-5)
    assert np.array_equal(got.vs[:, sl].view(np.uint32), ref.vs[:, sl].view(np.uint32))


@pytest.mark.parametrize("turbo", [0, 1])
def test_wavefront_kernels_match_block_kernels(turbo):
    """The one-wavefront-per-row kernels (front, append, turbo_out) against the 256-thread kernels that run when a row
    is not 16-byte aligned (a buffer one float past an aligned one, same values): the same bits in qo, the cache and
    the output."""
    import torch
    import moex_amd as M
    T, pos0, max_t = 37, 900, 1024
    LQ = H * 2 * AHD + 2 * KV * AHD
    rng = np.random.default_rng(91)
    qkv_h = rng.standard_normal((T, LQ), dtype=np.float32)
    qn = dev((0.1 * rng.standard_normal(AHD)).astype(np.float16).view(np.int16))
    kn = dev((0.1 * rng.standard_normal(AHD)).astype(np.float16).view(np.int16))
    res = []
    for off in (0, 1):  # 1: every row starts one float past a 16-byte boundary
        buf = torch.zeros(T * LQ + 4, device="cuda")
        qkv = buf[off:off + T * LQ].view(T, LQ)
        qkv.copy_(torch.from_numpy(qkv_h))
        qob = torch.zeros(T * H * AHD + 4, device="cuda")
        qo = qob[off:off + T * H * AHD].view(T, H, AHD)
        c = M.DeviceKVCache(KV, max_t, turbo)
        M.qk_norm_rope(qkv, qkv[:, H * 2 * AHD:], qkv[:, H * 2 * AHD + KV * AHD:], qn, kn, qo, c, H, KV,
                       pos_tensor(pos0), max_t, 64, 1e7, 1e-6, LQ, T)
        M.kv_append(qkv[:, :KV * AHD], qkv[:, KV * AHD:2 * KV * AHD], c, KV, pos_tensor(0), max_t, LQ, T)
        if turbo:
            M.turbo_out(qo, qkv, H, LQ, T)
        torch.cuda.synchronize()
        hc = download(c)
        res.append((qo.cpu().numpy().copy(), hc))
    (qa, ca), (qb, cb) = res
    assert np.array_equal(qa.view(np.uint32), qb.view(np.uint32))
    rows = np.r_[0:T, pos0:pos0 + T]  # the rows the two calls wrote (the rest of a new cache is not initialised)
    for x, y in ((ca.k, cb.k), (ca.v, cb.v), (ca.ks, cb.ks), (ca.vs, cb.vs)):
        a, b = np.ascontiguousarray(x[:, rows]), np.ascontiguousarray(y[:, rows])
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))


@pytest.mark.parametrize("turbo,KV", [(0, 2), (1, 2), (0, 3)])
def test_front_rows_per_wavefront(turbo, KV, monkeypatch):
    """front_rows_kernel puts RPW rows of one token on a wavefront, which computes the token's RoPE angles once for
    them (MOEX_FRONT_RPW): 1, 3, 6 and 9 rows per wavefront give the same qo and cache bytes (3 kv heads: 27 rows a
    token, so the last wavefront of a token is partial)."""
    import torch
    import moex_amd as M
    Hq = 8 * KV
    T, pos0, max_t = 29, 5000, 5120
    LQ = Hq * 2 * AHD + 2 * KV * AHD
    rng = np.random.default_rng(93 + KV)
    qkv = dev(rng.standard_normal((T, LQ), dtype=np.float32))
    qn = dev((0.1 * rng.standard_normal(AHD)).astype(np.float16).view(np.int16))
    kn = dev((0.1 * rng.standard_normal(AHD)).astype(np.float16).view(np.int16))
    res = []
    for rpw in ("1", "3", "6", "9"):
        monkeypatch.setenv("MOEX_FRONT_RPW", rpw)
        qo = torch.full((T, Hq, AHD), float("nan"), device="cuda")
        c = M.DeviceKVCache(KV, max_t, turbo)
        M.qk_norm_rope(qkv, qkv[:, Hq * 2 * AHD:], qkv[:, Hq * 2 * AHD + KV * AHD:], qn, kn, qo, c, Hq, KV,
                       pos_tensor(pos0), max_t, 64, 1e7, 1e-6, LQ, T)
        torch.cuda.synchronize()
        hc = download(c)
        res.append((qo.cpu().numpy(), [np.ascontiguousarray(x[:, pos0:pos0 + T]) for x in (hc.k, hc.v, hc.ks, hc.vs)]))
    q0, c0 = res[0]
    assert np.all(np.isfinite(q0))
    for qx, cx in res[1:]:
        assert np.array_equal(q0.view(np.uint32), qx.view(np.uint32))
        for a, b in zip(c0, cx):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
