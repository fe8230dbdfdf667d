"""Pins the CPU oracle (oracle/moex_oracle.c) against closed forms, invariants and independent formulations.

The reference holds no golden vectors for the attention path (its tests generate data at run time from seeded
std::mt19937: tests/test_fa.cu:18, tests/test_kernels.cu:787,820), so each oracle function is pinned here by
mathematics chosen so that a plausible mistake (wrong sign, dropped term, transposed index, wrong reduction order)
fails a check.
"""
import numpy as np
import pytest
from scipy.linalg import hadamard
from scipy.special import softmax
from scipy.stats import norm

AHD = 256


# ---------------- int8 quantizer (kernels.cuh:1227-1235) ----------------
def test_int8_closed_form(orc):
    rng = np.random.default_rng(0)
    for scale in (1.0, 1e-3, 37.0):
        x = (rng.standard_normal(AHD) * scale).astype(np.float32)
        q, s = orc.int8_quant_row(x)
        mk = np.max(np.abs(x))
        sk = np.float32(mk) / np.float32(127.0)
        assert np.float32(s) == sk
        expect = np.rint(x / sk).astype(np.int8)  # float32 divide, round half to even
        assert np.array_equal(q, expect)
        assert np.abs(q).max() == 127


def test_int8_ties_and_zero(orc):
    x = np.zeros(AHD, np.float32)
    x[:6] = [127.0, 2.5, 3.5, -2.5, 0.5, 1.5]  # sk = 1: quotients are the values themselves
    q, s = orc.int8_quant_row(x)
    assert s == 1.0
    assert list(q[:6]) == [127, 2, 4, -2, 0, 2]
    q, s = orc.int8_quant_row(np.zeros(AHD, np.float32))
    assert s == 1.0 and not q.any()


# ---------------- reductions (kernels.cuh:13-16, 1161-1169) ----------------
def test_half_sum_butterfly_tree(orc):
    # within a 32-lane group the xor tree adds lanes i and i^16 first: 2^24 + (-2^24) = 0, then + 1 -> 1.
    # A left-to-right sum would absorb the 1 into 2^24 and return 0.
    v = np.zeros(128, np.float32)
    v[0], v[1], v[16] = 2.0 ** 24, 1.0, -(2.0 ** 24)
    assert orc.half_sum(v) == 1.0
    # across groups the four partials are added in order: ((2^24 + 1) + 1) + (-2^24) = 0 (pairwise would give 1)
    v = np.zeros(128, np.float32)
    v[0], v[32], v[64], v[96] = 2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)
    assert orc.half_sum(v) == 0.0


def test_half_sum_value(orc):
    rng = np.random.default_rng(1)
    v = rng.standard_normal(128).astype(np.float32)
    assert abs(float(orc.half_sum(v)) - float(np.sum(v.astype(np.float64)))) < 1e-5


# ---------------- WHT (kernels.cuh:1143-1159) ----------------
def _wht_matrix(orc, inverse=False):
    W = np.zeros((AHD, AHD), np.float64)
    for i in range(AHD):
        e = np.zeros(AHD, np.float32)
        e[i] = 1.0
        W[:, i] = orc.wht(e, inverse)
    return W


def test_wht_is_signed_sylvester(orc):
    t = orc.tables()
    Hs = hadamard(128).astype(np.float64)  # natural (Sylvester) order
    assert set(np.unique(t["S1"])) == {-1.0, 1.0} and set(np.unique(t["S2"])) == {-1.0, 1.0}
    fwd = np.diag(t["S2"].astype(np.float64)) @ Hs @ np.diag(t["S1"].astype(np.float64)) / np.sqrt(128.0)
    inv = np.diag(t["S1"].astype(np.float64)) @ Hs @ np.diag(t["S2"].astype(np.float64)) / np.sqrt(128.0)
    W, Wi = _wht_matrix(orc), _wht_matrix(orc, True)
    for b in range(2):
        sl = slice(128 * b, 128 * (b + 1))
        assert np.abs(W[sl, sl] - fwd).max() < 1e-7
        assert np.abs(Wi[sl, sl] - inv).max() < 1e-7
    assert np.abs(W[:128, 128:]).max() == 0 and np.abs(W[128:, :128]).max() == 0
    assert np.abs(Hs @ Hs - 128 * np.eye(128)).max() == 0
    assert np.abs(W @ W.T - np.eye(AHD)).max() < 1e-6
    rng = np.random.default_rng(2)
    x = rng.standard_normal(AHD).astype(np.float32)
    assert np.abs(orc.wht(orc.wht(x), True) - x).max() < 1e-5


# ---------------- TurboQuant tables and quantizer (kernels.cuh:1112-1139, 1172-1183) ----------------
def _lloyd_max(levels, sigma, iters=2000):
    c = np.linspace(-2.5, 2.5, levels) * sigma
    for _ in range(iters):
        t = np.concatenate([[-np.inf], (c[:-1] + c[1:]) / 2, [np.inf]])
        a, b = t[:-1] / sigma, t[1:] / sigma
        c = sigma * (norm.pdf(a) - norm.pdf(b)) / (norm.cdf(b) - norm.cdf(a))
    return c, (c[:-1] + c[1:]) / 2


def test_tq_tables_are_lloyd_max(orc):
    t = orc.tables()
    sigma = 1.0 / np.sqrt(128.0)
    for levels, codes, k, m in ((16, t["I4"], t["K4"], t["M4"]), (8, t["I3"], t["K3"], t["M3"])):
        c, thr = _lloyd_max(levels, sigma)
        cmax = c[-1]
        assert abs(float(k) * 127 - cmax) < 2e-6
        assert np.array_equal(codes.astype(int), np.rint(127 * c / cmax).astype(int))
        assert np.abs(m.astype(np.float64) - thr).max() < 2e-6


def test_tq_quant_nearest_centroid_and_norm(orc):
    t = orc.tables()
    sigma = 1.0 / np.sqrt(128.0)
    W = _wht_matrix(orc)
    rng = np.random.default_rng(3)
    for bits, codes, k in ((4, t["I4"], t["K4"]), (3, t["I3"], t["K3"])):
        c, thr = _lloyd_max(2 ** bits, sigma)
        for trial in range(20):
            x = (rng.standard_normal(AHD) * (0.1 + trial)).astype(np.float32)
            idx, nrm = orc.tq_quant(x, bits)
            for b in range(2):
                sl = slice(128 * b, 128 * (b + 1))
                n = np.sqrt(np.sum(x[sl].astype(np.float64) ** 2))
                r = W[sl, sl] @ (x[sl] / n)
                near = np.argmin(np.abs(r[:, None] - c[None, :]), axis=1)
                clear = np.min(np.abs(r[:, None] - thr[None, :]), axis=1) > 1e-5
                assert np.array_equal(idx[sl][clear], near[clear])
                deq = codes[idx[sl]].astype(np.float64) * float(k) * float(nrm[b])
                assert abs(np.linalg.norm(deq) - n) < 1e-5 * n


def test_tq_quant_zero_row(orc):
    for bits, zidx in ((4, 8), (3, 4)):  # r = 0 >= every threshold up to and including the 0 one
        idx, nrm = orc.tq_quant(np.zeros(AHD, np.float32), bits)
        assert np.all(idx == zidx) and np.all(nrm == 0)


def test_turbo_packing(orc):
    ik = np.zeros(AHD, np.int32)
    iv = np.zeros(AHD, np.int32)
    ik[0], ik[1], ik[130], ik[131] = 1, 2, 15, 4
    iv[0], iv[5], iv[130], iv[255] = 5, 7, 2, 4
    kb, vb = orc.turbo_pack(ik, iv)
    assert kb[0] == 0x21 and kb[64 + 1] == 0x4F and kb.sum() == 0x21 + 0x4F
    assert vb[0] == 0x01 and vb[64] & 1 == 1          # dim 0: code 5 = low 01, high 1
    assert (vb[1] >> 2) & 3 == 3 and (vb[64] >> 5) & 1  # dim 5: code 7
    assert (vb[32] >> 4) & 3 == 2 and not (vb[80] >> 2) & 1  # dim 130 = half 1, j 2: code 2
    assert vb[32 + 31] == 0 and (vb[64 + 16 + 15] >> 7) & 1  # dim 255: code 4 = low 00, high 1
    rng = np.random.default_rng(4)
    for _ in range(10):
        ik = rng.integers(0, 16, AHD).astype(np.int32)
        iv = rng.integers(0, 8, AHD).astype(np.int32)
        a, b = orc.turbo_unpack(*orc.turbo_pack(ik, iv))
        assert np.array_equal(a, ik) and np.array_equal(b, iv)


# ---------------- fp64 attention (tests/test_fa.cu:59-80) ----------------
def _dense_reference(orc, qo, gate, ld, H, cache, pos0, t, h):
    """Independent formulation: dequantize the whole key range, scipy softmax, matrix products."""
    kvh = h // (H // cache.KV)
    n = pos0 + t + 1
    tb = orc.tables()
    if cache.turbo:
        K = np.zeros((n, AHD)); V = np.zeros((n, AHD))
        for j in range(n):
            ik, iv = orc.turbo_unpack(cache.k[kvh, j].view(np.uint8), cache.v[kvh, j].view(np.uint8))
            K[j] = tb["I4"][ik] * float(tb["K4"]) * np.repeat(cache.ks[kvh, j].astype(np.float64), 128)
            V[j] = tb["I3"][iv] * float(tb["K3"]) * np.repeat(cache.vs[kvh, j].astype(np.float64), 128)
    else:
        K = cache.k[kvh, :n].astype(np.float64) * cache.ks[kvh, :n, None]
        V = cache.v[kvh, :n].astype(np.float64) * cache.vs[kvh, :n, None]
    q = qo[t, h].astype(np.float64)
    o = softmax(K @ q / 16.0) @ V
    if gate is None:
        return o
    if cache.turbo:  # exact inverse rotation per half: S1 . H . S2 / sqrt(128)
        Wi = np.diag(tb["S1"].astype(np.float64)) @ hadamard(128) @ np.diag(tb["S2"].astype(np.float64)) / np.sqrt(128)
        o = np.concatenate([Wi @ o[:128], Wi @ o[128:]])
    g = gate.reshape(-1)[t * ld + h * 2 * AHD + AHD: t * ld + h * 2 * AHD + 2 * AHD].astype(np.float64)
    return o / (1 + np.exp(-g))


@pytest.mark.parametrize("turbo", [0, 1])
def test_attn_f64_against_dense(orc, turbo):
    rng = np.random.default_rng(5 + turbo)
    H, KV, max_t, T, pos0 = 16, 2, 48, 5, 30
    ld = H * 2 * AHD
    cache = orc.HostCache(KV, max_t, turbo)
    k = rng.standard_normal((T + pos0, KV * AHD)).astype(np.float32)
    v = rng.standard_normal((T + pos0, KV * AHD)).astype(np.float32)
    orc.kv_append(cache, k, v, KV * AHD, T + pos0, 0)
    qo = rng.standard_normal((T, H, AHD)).astype(np.float32)
    gate = rng.standard_normal((T, ld)).astype(np.float32)
    rows = [(t, h) for t in range(T) for h in (0, 7, 8, 15)]
    got = orc.attn_rows_f64(qo, gate, ld, H, cache, pos0, rows)
    for (t, h), g in zip(rows, got):
        ref = _dense_reference(orc, qo, gate, ld, H, cache, pos0, t, h)
        assert np.abs(g - ref).max() < 1e-12 * max(1.0, np.abs(ref).max())
    # no gate: the raw (for turbo: rotated-domain) attention output
    got = orc.attn_rows_f64(qo, None, ld, H, cache, pos0, rows[:3])
    for (t, h), g in zip(rows[:3], got):
        assert np.abs(g - _dense_reference(orc, qo, None, ld, H, cache, pos0, t, h)).max() < 1e-12


def test_attn_f64_closed_forms(orc):
    H, KV, max_t = 16, 2, 8
    ld = H * 2 * AHD
    rng = np.random.default_rng(7)
    cache = orc.HostCache(KV, max_t, 0)
    cache.k[:] = rng.integers(-127, 128, cache.k.shape)
    cache.v[:] = rng.integers(-127, 128, cache.v.shape)
    cache.ks[:] = 0.01
    cache.vs[:] = rng.uniform(0.005, 0.05, cache.vs.shape)
    qo = rng.standard_normal((1, H, AHD)).astype(np.float32)
    gate = rng.standard_normal((1, ld)).astype(np.float32)
    # a single visible key: out = v0 * vs0 * sigmoid(g)
    out = orc.attn_rows_f64(qo, gate, ld, H, cache, 0, [(0, 3)])[0]
    g = gate[0, 3 * 512 + 256: 3 * 512 + 512].astype(np.float64)
    assert np.allclose(out, cache.v[0, 0] * float(cache.vs[0, 0]) / (1 + np.exp(-g)), rtol=1e-13, atol=0)
    # identical keys: uniform weights, out = mean of v_j vs_j
    cache.k[1, :6] = cache.k[1, 0]
    out = orc.attn_rows_f64(qo, None, ld, H, cache, 5, [(0, 12)])[0]
    ref = np.mean(cache.v[1, :6].astype(np.float64) * cache.vs[1, :6, None], axis=0)
    assert np.allclose(out, ref, rtol=1e-12, atol=1e-15)


def test_fa_precision_model_close(orc):
    rng = np.random.default_rng(8)
    H, KV, max_t, T, pos0 = 16, 2, 300, 9, 200
    ld = H * 2 * AHD
    for turbo in (0, 1):
        cache = orc.HostCache(KV, max_t, turbo)
        k = rng.standard_normal((pos0 + T, KV * AHD)).astype(np.float32)
        v = rng.standard_normal((pos0 + T, KV * AHD)).astype(np.float32)
        orc.kv_append(cache, k, v, KV * AHD, pos0 + T, 0)
        qo = rng.standard_normal((T, H, AHD)).astype(np.float32)
        gate = rng.standard_normal((T, ld)).astype(np.float32)
        rows = [(0, 0), (4, 9), (8, 15)]
        a = orc.attn_rows_f64(qo, gate, ld, H, cache, pos0, rows)
        b = orc.attn_rows_fa_emul(qo, gate, ld, H, cache, pos0, rows)
        err = np.abs(a - b).max()
        assert 0 < err < 2e-3 * np.abs(a).max()


def test_round_f16(orc):
    x = np.array([1.0, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 65504.0, 65520.0, 2 ** -24, 2 ** -25, 3 * 2 ** -25,
                  -0.1, 1e-7], np.float32)
    assert np.array_equal(orc.round_f16(x), x.astype(np.float16).astype(np.float32))
    y = np.random.default_rng(9).standard_normal(10000).astype(np.float32) * 100
    assert np.array_equal(orc.round_f16(y), y.astype(np.float16).astype(np.float32))


# ---------------- query/key front (ref/qwen36_ref.py:62-76) ----------------
def test_qk_norm_rope_front(orc):
    rng = np.random.default_rng(10)
    x = rng.standard_normal(AHD).astype(np.float32) * 3
    w = (rng.standard_normal(AHD) * 0.1).astype(np.float16)
    wb = w.view(np.uint16)
    eps, rot, theta = 1e-6, 64, 1e7
    # pos 0: no rotation; weight 0: unit RMS
    y0 = orc.qk_norm_rope_row(x, np.zeros(AHD, np.uint16), 0, rot, theta, eps)
    assert abs(np.sqrt(np.mean(y0.astype(np.float64) ** 2)) - 1) < 1e-5
    # rotation of the first 64 dims preserves the pair norms and leaves the rest unchanged
    y = orc.qk_norm_rope_row(x, wb, 12345, rot, theta, eps)
    yn = orc.qk_norm_rope_row(x, wb, 0, rot, theta, eps)
    assert np.allclose(y[rot:], yn[rot:], rtol=0, atol=0)
    pn = lambda z: z[:32].astype(np.float64) ** 2 + z[32:64].astype(np.float64) ** 2
    assert np.allclose(pn(y), pn(yn), rtol=1e-5)
    # angle of pair j = pos * theta^(-2j/rot): the first pair rotates by exactly pos radians
    a0 = np.arctan2(yn[32], yn[0]); a1 = np.arctan2(y[32], y[0])
    assert abs(((a1 - a0 - 12345) + np.pi) % (2 * np.pi) - np.pi) < 1e-3


# ---- dense int8 projections (kernels.cuh:144-156 quantize_rows_i8_k, :98-141 gemv_i8) ----
def test_quantize_rows_closed_form(orc):
    """absmax / 127 per row (1 for a zero row), round-half-even of the binary32 quotient: numpy restates it."""
    rng = np.random.default_rng(31)
    w = (rng.standard_normal((40, 512)) * np.geomspace(1e-4, 10, 40)[:, None]).astype(np.float16)
    w[3] = 0
    w[4] = np.float16(0.25)                       # constant row: every quotient exactly 127
    w[5, :] = 0; w[5, 10] = np.float16(-2.5)      # one non-zero: +-127 and zeros
    w[6, :8] = np.float16(65504); w[6, 8:] = np.float16(-6e-8)  # the fp16 extremes
    q, s = orc.quantize_rows_i8(w)
    wf = w.astype(np.float32)
    m = np.abs(wf).max(1)
    sc = np.where(m > 0, m / np.float32(127), np.float32(1)).astype(np.float32)
    assert np.array_equal(s.view(np.uint32), sc.view(np.uint32))
    assert np.array_equal(q, np.rint(wf / sc[:, None]).astype(np.int8))
    assert np.all(q[4] == 127) and q[5, 10] == -127 and np.all(q[3] == 0) and s[3] == 1.0


def test_quantize_rows_ties(orc):
    """quotients landing exactly on .5 round to even (the scale makes q = w / s exact for these rows)."""
    w = np.zeros((1, 256), np.float16)
    w[0, 0] = np.float16(127.0)                    # scale 1
    w[0, 1:6] = np.array([0.5, 1.5, 2.5, -0.5, -3.5], np.float16)
    q, s = orc.quantize_rows_i8(w)
    assert s[0] == 1.0 and list(q[0, :6]) == [127, 0, 2, 2, 0, -4]


def test_dense_exact_product(orc):
    """fp64 sums of int8 x fp32 products are exact for I <= 2^20 terms of 24+8 bits: equal to numpy float64."""
    rng = np.random.default_rng(32)
    q = rng.integers(-127, 128, (37, 1024), dtype=np.int8)
    s = rng.uniform(1e-3, 1e-2, 37).astype(np.float32)
    x = rng.standard_normal((5, 1024)).astype(np.float32)
    y = orc.dense_i8_f64(q, s, x)
    ref = (x.astype(np.float64) @ q.T.astype(np.float64)) * s.astype(np.float64)
    assert np.abs(y - ref).max() <= 1e-12 * np.abs(ref).max()
    # the fp16-activation model differs from it exactly by rounding x
    y16 = orc.dense_i8_fp16x(q, s, x)
    ref16 = (x.astype(np.float16).astype(np.float64) @ q.T.astype(np.float64)) * s.astype(np.float64)
    assert np.abs(y16 - ref16).max() <= 1e-12 * np.abs(ref16).max()


def _fa_emul_2key(q, k, ks, v, vs, round_q=True, round_p=True):
    """numpy restatement of the precision model for one row over the keys given (one 64-key tile): fp32 score
    s = float32(q16 . k) * (ks * sl2), base-2 softmax against the tile max in fp32, P * vs rounded to fp16."""
    sl2 = np.float32(np.float32(1.0 / 16.0) * np.float32(1.4426950408889634))
    qq = q.astype(np.float16).astype(np.float64) if round_q else q.astype(np.float64)
    s = np.array([np.float32(np.float32(qq @ kj.astype(np.float64)) * np.float32(np.float32(ksj) * sl2))
                  for kj, ksj in zip(k, ks)], np.float32)
    e = np.exp2((s - s.max()).astype(np.float32)).astype(np.float32)
    pv = (e * vs.astype(np.float32)).astype(np.float32)
    if round_p:
        pv = pv.astype(np.float16).astype(np.float32)
    o = (pv.astype(np.float64)[:, None] * v.astype(np.float64)).sum(0)
    return o.astype(np.float32).astype(np.float64) / float(e.astype(np.float32).sum(dtype=np.float32))


def _one_head_cache(orc, k, ks, v, vs):
    c = orc.HostCache(1, len(k), 0)
    c.k[0], c.ks[0], c.v[0], c.vs[0] = k, ks, v, vs
    return c


def test_fa_precision_model_single_key(orc):
    """fp16-exact Q and V scale, one visible key: softmax weight 1, no rounding left, so the precision model equals
    the fp64 reference (and the closed form v * vs) to 1e-12."""
    rng = np.random.default_rng(12)
    q = rng.standard_normal(AHD).astype(np.float16).astype(np.float32)
    k = rng.integers(-127, 128, (1, AHD)).astype(np.int8)
    v = rng.integers(-127, 128, (1, AHD)).astype(np.int8)
    ks = np.array([0.0123], np.float32)
    vs = np.array([np.float16(0.0371)], np.float32)
    c = _one_head_cache(orc, k, ks, v, vs)
    qo = q.reshape(1, 1, AHD)
    a = orc.attn_rows_f64(qo, None, 2 * AHD, 1, c, 0, [(0, 0)])[0]
    b = orc.attn_rows_fa_emul(qo, None, 2 * AHD, 1, c, 0, [(0, 0)])[0]
    assert np.allclose(b, a, rtol=1e-12, atol=0)
    assert np.allclose(b, v[0].astype(np.float64) * float(vs[0]), rtol=1e-12, atol=0)


def test_fa_precision_model_rounding_points(orc):
    """Two keys whose rounding effects are known: the model equals the numpy restatement to 1e-6, and the same
    restatement with the P * vs rounding (or the Q rounding) dropped differs from it by far more, so a model that
    lost either rounding fails here."""
    # P * vs rounding: fp16-exact Q; key 1 scores about 1 below key 0 (weight ~1/2), P * vs1 not fp16-exact
    q = np.zeros(AHD, np.float32); q[0] = 1.0
    k = np.zeros((2, AHD), np.int8); k[0, 0] = 64; k[1, 0] = 0
    sl2 = np.float32(np.float32(1.0 / 16.0) * np.float32(1.4426950408889634))
    ks = np.array([1.0 / (64 * float(sl2)), 0.02], np.float32)   # s0 ~ 1, s1 = 0
    v = np.full((2, AHD), 100, np.int8); v[1] = -77
    vs = np.array([2.0 ** -16, 1.3e-5], np.float32)   # 0.5 * vs1 lands among the fp16 subnormals (spacing 2^-24)
    c = _one_head_cache(orc, k, ks, v, vs)
    qo = q.reshape(1, 1, AHD)
    got = orc.attn_rows_fa_emul(qo, None, 2 * AHD, 1, c, 1, [(0, 0)])[0]
    want = _fa_emul_2key(q, k, ks, v, vs)
    loose = _fa_emul_2key(q, k, ks, v, vs, round_p=False)
    tol = 1e-6 * np.abs(want).max()
    assert np.abs(got - want).max() <= tol
    assert np.abs(got - loose).max() > 50 * tol
    # Q rounding: every dim of q is 1 + 2^-12 (rounds to 1 in fp16) against a full key of 127s
    q = np.full(AHD, 1.0 + 2.0 ** -12, np.float32)
    k = np.zeros((2, AHD), np.int8); k[0] = 127
    ks = np.array([3.0 / (256 * 127 * float(sl2)), 0.02], np.float32)   # s0 ~ 3, s1 = 0
    v = np.full((2, AHD), 50, np.int8); v[1] = -120
    vs = np.array([np.float16(0.25), np.float16(0.125)], np.float32)
    c = _one_head_cache(orc, k, ks, v, vs)
    qo = q.reshape(1, 1, AHD)
    got = orc.attn_rows_fa_emul(qo, None, 2 * AHD, 1, c, 1, [(0, 0)])[0]
    want = _fa_emul_2key(q, k, ks, v, vs)
    loose = _fa_emul_2key(q, k, ks, v, vs, round_q=False)
    tol = 1e-6 * np.abs(want).max()
    assert np.abs(got - want).max() <= tol
    assert np.abs(got - loose).max() > 20 * tol


# ---- the other dense forms (kernels.cuh:186-196 Mat; :552-590 quantize_rows_q6_k / q4_k; :486-550 the GEMVs) ----
def _unpack_q4(q, I):
    """numpy: two's complement nibbles, weight 2j in the low nibble of byte j"""
    lo = (q & 15).astype(np.int16); hi = (q >> 4).astype(np.int16)
    v = np.stack([lo, hi], -1).reshape(q.shape[0], I)
    return np.where(v >= 8, v - 16, v)


def _unpack_q6(q, qh, I):
    lo = np.stack([q & 15, q >> 4], -1).reshape(q.shape[0], I).astype(np.int16)
    hi = np.stack([(qh >> (2 * k)) & 3 for k in range(4)], -1).reshape(q.shape[0], I).astype(np.int16)
    return (lo | (hi << 4)) - 32


def test_quantize_q4_known_bytes_and_ties(orc):
    """A group whose scale is exactly 1 (absmax 7): codes are the weights themselves, .5 quotients round to even,
    and the packed bytes are known by hand (low nibble first, two's complement)."""
    w = np.zeros((1, 128), np.float16)
    w[0, :8] = [7, -7, 1, 2, 0.5, 1.5, -2.5, -0.5]
    q, s = orc.quantize_rows_q4(w)
    assert s[0, 0] == 1.0 and s[0, 1] == 1.0                      # the second group is all zero: scale 1
    assert list(q[0, :4]) == [0x97, 0x21, 0x20, 0x0E]             # (7, -7), (1, 2), (0, 2), (-2, 0)
    assert np.all(q[0, 4:] == 0)


def test_quantize_q6_known_bytes_and_ties(orc):
    """Scale exactly 1 (absmax 31): u = round-half-even(w) + 32, so -30.5 -> u = 2; low nibbles as q4's, high 2-bit
    fields at bits 2 (i % 4) of byte i / 4; the zero weights of the group are u = 32 (high field 2)."""
    w = np.zeros((1, 64), np.float16)
    w[0, :6] = [31, -31, 1.5, -2.5, 16, -30.5]                     # u = 63, 1, 34, 30, 48, 2
    q, qh, s = orc.quantize_rows_q6(w)
    assert s[0, 0] == 1.0
    assert list(q[0, :4]) == [0x1F, 0xE2, 0x20, 0x00]
    assert list(qh[0, :3]) == [0x63, 0xA3, 0xAA]


@pytest.mark.parametrize("six", [False, True])
def test_quantize_gs64_random(orc, six):
    """Random rows over a range of magnitudes, a zero group and an fp16-extreme group: the scale is the group absmax
    / 7 (/ 31), every code is round-half-even of the binary32 quotient within the clamp, and dequantized weights lie
    within half a scale of the input."""
    rng = np.random.default_rng(33)
    w = (rng.standard_normal((24, 256)) * np.geomspace(1e-4, 30, 24)[:, None]).astype(np.float16)
    w[2, 64:128] = 0
    w[3, :64] = np.float16(65504); w[3, 1] = np.float16(-65504)
    qm = 31 if six else 7
    if six:
        q, qh, s = orc.quantize_rows_q6(w)
        v = _unpack_q6(q, qh, 256)
    else:
        q, s = orc.quantize_rows_q4(w)
        v = _unpack_q4(q, 256)
    wf = w.astype(np.float32).reshape(24, 4, 64)
    m = np.abs(wf).max(-1)
    sc = np.where(m > 0, m / np.float32(qm), np.float32(1)).astype(np.float32)
    assert np.array_equal(s.view(np.uint32), sc.view(np.uint32))
    ref = np.clip(np.rint(wf / sc[..., None]), -qm - 1, qm).astype(np.int16).reshape(24, 256)
    assert np.array_equal(v, ref)
    assert np.all(np.abs(v.reshape(24, 4, 64)).max(-1)[m > 0] == qm)  # the absmax weight takes the top code
    err = np.abs(v.reshape(24, 4, 64) * sc[..., None].astype(np.float64) - wf.astype(np.float64))
    assert np.all(err <= sc[..., None] * 0.5000001)


@pytest.mark.parametrize("fmt", ["q4", "q6", "f16"])
def test_dense_mat_exact_product(orc, fmt):
    """The exact product equals numpy's float64 matmul of independently unpacked weights; a matrix with a single
    non-zero weight gives that weight times x; the GEMM model equals the exact product when weights and inputs are
    fp16-exact and differs from it by rounding x alone otherwise."""
    rng = np.random.default_rng(34)
    O, I = 29, 256
    w16 = (rng.standard_normal((O, I)) * 0.1).astype(np.float16)
    x = rng.standard_normal((3, I)).astype(np.float32)
    if fmt == "q4":
        q, s = orc.quantize_rows_q4(w16); wh = None; F = orc.MAT_Q4
        wd = _unpack_q4(q, I) * np.repeat(s.astype(np.float64), 64, 1)
    elif fmt == "q6":
        q, wh, s = orc.quantize_rows_q6(w16); F = orc.MAT_Q6
        wd = _unpack_q6(q, wh, I) * np.repeat(s.astype(np.float64), 64, 1)
    else:
        q, wh, s, F = w16, None, None, orc.MAT_F16
        wd = w16.astype(np.float64)
    y = orc.dense_mat_f64(F, q, wh, s, x)
    ref = x.astype(np.float64) @ wd.T
    assert np.abs(y - ref).max() <= 1e-12 * np.abs(ref).max()
    # the GEMM precision model: fp16(fp32(code * scale)) and fp16(x)
    w32 = wd.astype(np.float32)
    w16m = w32 if fmt == "f16" else w32.astype(np.float16).astype(np.float64)
    ref16 = x.astype(np.float16).astype(np.float64) @ np.asarray(w16m, np.float64).T
    y16 = orc.dense_mat_fp16x(F, q, wh, s, x)
    assert np.abs(y16 - ref16).max() <= 1e-12 * np.abs(ref16).max()
    xh = x.astype(np.float16).astype(np.float32)
    if fmt == "f16":  # fp16 weights and fp16-exact inputs: the model is the exact product
        assert np.abs(orc.dense_mat_fp16x(F, q, wh, s, xh) - orc.dense_mat_f64(F, q, wh, s, xh)).max() == 0
    assert np.abs(y16 - y).max() > 0  # rounding x is not a no-op on these inputs


def test_dense_mat_single_weight(orc):
    """One non-zero int4 weight (code 3 at input 70 of row 5, group scale 0.25): y[5] = 0.75 x[70], all else 0."""
    O, I = 8, 128
    q = np.zeros((O, I // 2), np.uint8)
    q[5, 35] = 0x03                                   # input 70: the low nibble of byte 35
    s = np.full((O, I // 64), 0.25, np.float32)
    x = np.arange(1, I + 1, dtype=np.float32)[None]
    y = orc.dense_mat_f64(orc.MAT_Q4, q, None, s, x)
    assert y[0, 5] == 0.75 * 71 and np.count_nonzero(y) == 1
