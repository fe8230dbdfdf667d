"""The other weight forms of a dense matrix (struct Mat, kernels.cuh:186-196: int4 gs64, int6 gs64, fp16) through
moex_gemv / moex_gemm (include/moex_dense.h), with the reference's gates (tests/test_kernels.cu K11, K11b;
check() = max abs error / max |ref|):
  - quantize_rows_q4 / q6: codes, high planes and scales bit-exact against the oracle;
  - the GEMV vs the exact product of the dequantized weights: rel < 1e-5 (K11's gate, used here for all three
    forms, tighter than K11b's 1e-3 against an fp16 GEMV);
  - int6 with S <= 8 rows through gemm: every row bit-identical to the one-row GEMV (K11b asks 1e-7);
  - the fp16 MFMA GEMM (int4 / int6 / fp16 weights, S > 8, and int4 / fp16 from S = 3) vs the GEMV row by row:
    rel < 5e-3 (K11, K11b), and vs the precision model of its own rounding (weights fp16(fp32(code * scale)),
    activations fp16) at rel < 1e-5; ragged O and S included.
Shapes: the attention's qkv (2048 -> 9216) and o_proj (4096 -> 2048), and K11's 512-input shared-expert shape.
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.gpu_util import dev, report

pytestmark = pytest.mark.gpu

SHAPES = [(9216, 2048), (2048, 4096), (2048, 512)]


def _rel(got, ref):
    return float(np.abs(got - ref).max() / (np.abs(ref).max() + 1e-30))


def _make(fmt, w16):
    """quantize on the GPU into the form; returns (Mat, host arrays (w, wh, s), oracle format code)"""
    import torch
    import moex_amd as M
    O, I = w16.shape
    wd = dev(w16.view(np.int16))
    if fmt == "f16":
        return M.Mat(f16=wd), (w16, None, None), orc.MAT_F16, wd
    s = torch.empty((O, I // 64), dtype=torch.float32, device="cuda")
    q = torch.empty((O, I // 2), dtype=torch.uint8, device="cuda")
    if fmt == "q4":
        M.quantize_rows_q4(wd, q, s, O, I)
        torch.cuda.synchronize()
        return M.Mat(q4=q, s=s), (q.cpu().numpy(), None, s.cpu().numpy()), orc.MAT_Q4, (q, s)
    qh = torch.empty((O, I // 4), dtype=torch.uint8, device="cuda")
    M.quantize_rows_q6(wd, q, qh, s, O, I)
    torch.cuda.synchronize()
    return M.Mat(q6=q, q6h=qh, s=s), (q.cpu().numpy(), qh.cpu().numpy(), s.cpu().numpy()), orc.MAT_Q6, (q, qh, s)


@pytest.mark.parametrize("six", [False, True], ids=["q4", "q6"])
def test_quantize_bit_exact(six):
    rng = np.random.default_rng(51)
    w = (rng.standard_normal((300, 1024)) * np.geomspace(1e-4, 30, 300)[:, None]).astype(np.float16)
    w[0] = 0
    w[1, 64:128] = 0
    w[2, :64] = np.float16(65504); w[2, 5] = np.float16(-65504)
    w[3, :8] = [7, -7, 1, 2, 0.5, 1.5, -2.5, -0.5]; w[3, 8:64] = 0   # scale 1 (int4): ties
    w[4, :6] = [31, -31, 1.5, -2.5, 16, -30.5]; w[4, 6:64] = 0      # scale 1 (int6): ties
    m, host, _, _ = _make("q6" if six else "q4", w)
    if six:
        q, qh, s = orc.quantize_rows_q6(w)
        assert np.array_equal(host[1], qh)
    else:
        q, s = orc.quantize_rows_q4(w)
    assert np.array_equal(host[0], q) and np.array_equal(host[2].view(np.uint32), s.view(np.uint32))


@pytest.fixture(scope="module", params=SHAPES, ids=["qkv", "o_proj", "down512"])
def shape(request):
    return request.param


@pytest.mark.parametrize("fmt", ["q4", "q6", "f16"])
def test_gemv_vs_exact(shape, fmt):
    import torch
    import moex_amd as M
    O, I = shape
    rng = np.random.default_rng(O + 3 * I)
    w = (rng.standard_normal((O, I)) * 0.02).astype(np.float16)
    m, (hw, hh, hs), F, _keep = _make(fmt, w)
    x = rng.standard_normal(I).astype(np.float32)
    y = torch.full((O,), float("nan"), dtype=torch.float32, device="cuda")
    M.gemv(m, dev(x), y, I, O)
    torch.cuda.synchronize()
    R = min(O, 2048)  # K11 checks the first 2048 rows
    ref = orc.dense_mat_f64(F, hw[:R], None if hh is None else hh[:R], None if hs is None else hs[:R], x[None])[0]
    got = y.cpu().numpy()
    rel = _rel(got[:R].astype(np.float64), ref)
    report("gemv vs exact", fmt=fmt, O=O, I=I, rel=rel)
    assert np.all(np.isfinite(got)) and rel < 1e-5


@pytest.mark.parametrize("S", [2, 3, 5, 8])
def test_q6_rows_equal_gemv(shape, S):
    """int6 with S <= 8 rows: one GEMV pass, each row bit-identical to the one-row GEMV (K11b)."""
    import torch
    import moex_amd as M
    O, I = shape
    rng = np.random.default_rng(S + O)
    w = (rng.standard_normal((O, I)) * 0.02).astype(np.float16)
    m, _, _, _keep = _make("q6", w)
    x = rng.standard_normal((S, I)).astype(np.float32)
    xd = dev(x)
    Y = torch.empty((S, O), dtype=torch.float32, device="cuda")
    M.gemm(m, xd, Y, S, I, O)
    Yr = torch.empty_like(Y)
    for t in range(S):
        M.gemv(m, xd[t], Yr[t], I, O)
    torch.cuda.synchronize()
    assert np.array_equal(Y.cpu().numpy(), Yr.cpu().numpy())


@pytest.mark.parametrize("fmt,S", [("q4", 16), ("q4", 3), ("q6", 160), ("q6", 9), ("f16", 3), ("f16", 300)])
def test_gemm_vs_gemv_and_model(shape, fmt, S):
    import torch
    import moex_amd as M
    O, I = shape
    rng = np.random.default_rng(7 * S + O)
    w = (rng.standard_normal((O, I)) * 0.02).astype(np.float16)
    m, (hw, hh, hs), F, _keep = _make(fmt, w)
    x = rng.standard_normal((S, I)).astype(np.float32)
    xd = dev(x)
    Y = torch.full((S, O), float("nan"), dtype=torch.float32, device="cuda")
    M.gemm(m, xd, Y, S, I, O)
    Yr = torch.empty_like(Y)
    for t in range(S):
        M.gemv(m, xd[t], Yr[t], I, O)
    torch.cuda.synchronize()
    got, per_row = Y.cpu().numpy(), Yr.cpu().numpy()
    rel_gemv = _rel(got.astype(np.float64), per_row.astype(np.float64))
    rows = sorted({0, S // 2, S - 1})
    cols = np.arange(0, O, max(1, O // 256))
    model = orc.dense_mat_fp16x(F, hw[cols], None if hh is None else hh[cols], None if hs is None else hs[cols],
                                x[rows])
    rel_model = _rel(got[np.ix_(rows, cols)].astype(np.float64), model)
    report("gemm", fmt=fmt, O=O, I=I, S=S, rel_vs_gemv=rel_gemv, rel_vs_model=rel_model)
    assert np.all(np.isfinite(got)) and rel_gemv < 5e-3 and rel_model < 1e-5


@pytest.mark.parametrize("fmt", ["q4", "q6", "f16"])
def test_ragged(fmt):
    """O not a multiple of the GEMV row groups or the GEMM tile, S not a multiple of the GEMM tile; a wavefront
    with several row groups (O = 40000)."""
    import torch
    import moex_amd as M
    for O, I, S in ((1000, 512, 77), (40000, 256, 1)):
        rng = np.random.default_rng(O + S)
        w = (rng.standard_normal((O, I)) * 0.1).astype(np.float16)
        m, (hw, hh, hs), F, _keep = _make(fmt, w)
        x = rng.standard_normal((S, I)).astype(np.float32)
        Y = torch.full((S, O), float("nan"), dtype=torch.float32, device="cuda")
        M.gemm(m, dev(x), Y, S, I, O)
        y1 = torch.full((O,), float("nan"), dtype=torch.float32, device="cuda")
        M.gemv(m, dev(x[0]), y1, I, O)
        torch.cuda.synchronize()
        got = Y.cpu().numpy()
        if S > 2:
            ref = orc.dense_mat_fp16x(F, hw, hh, hs, x)
        else:
            ref = orc.dense_mat_f64(F, hw, hh, hs, x)
        rel = _rel(got.astype(np.float64), ref)
        rel1 = _rel(y1.cpu().numpy().astype(np.float64), orc.dense_mat_f64(F, hw, hh, hs, x[:1])[0])
        report("dense ragged", fmt=fmt, O=O, I=I, S=S, rel=rel, rel_gemv=rel1)
        assert np.all(np.isfinite(got)) and rel < 1e-5 and rel1 < 1e-5


def test_int8_mat_routes_to_gemm_i8():
    """A Mat holding int8 takes moex_gemm_i8's path: bit-identical results."""
    import torch
    import moex_amd as M
    O, I, S = 2048, 1024, 40
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((O, I)) * 0.05).astype(np.float16)
    q = torch.empty((O, I), dtype=torch.int8, device="cuda")
    s = torch.empty(O, dtype=torch.float32, device="cuda")
    M.quantize_rows_i8(dev(w.view(np.int16)), q, s, O, I)
    x = dev(rng.standard_normal((S, I)).astype(np.float32))
    for n in (1, 2, S):
        a = torch.empty((n, O), dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        M.gemm(M.Mat(q=q, s=s), x[:n], a, n, I, O)
        M.gemm_i8(q, s, x[:n], b, n, I, O)
        torch.cuda.synchronize()
        assert np.array_equal(a.cpu().numpy(), b.cpu().numpy())
