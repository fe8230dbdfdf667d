"""Dense int8 projections (include/moex_dense.h) against the oracle, with the reference's gates
(tests/test_kernels.cu K10, K12; check() = max abs error / max |ref|):
  - quantize_rows_i8: codes and scales bit-exact (the golden fixture and random rows with edge cases);
  - gemv_i8 vs the exact int8 product: rel < 1e-5 (K10), at the qkv (2048 -> 9216) and o_proj (4096 -> 2048) shapes;
  - gemm_i8 with S <= 8 rows: every row bit-identical to gemv_i8 of that row (K10 asks 1e-7);
  - gemm_i8 with S > 8 (the fp16 MFMA GEMM, K split over workgroups when the tile grid is short of one pass) vs the
    per-token GEMV: rel < 5e-3 (K12), and vs the precision model of its own rounding (fp16 activations, exact
    products) at rel < 1e-5; ragged S and O included.
"""
import os

import numpy as np
import pytest

from oracle import oracle as orc
from tests.gpu_util import dev, report

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _rel(got, ref):
    return float(np.abs(got - ref).max() / (np.abs(ref).max() + 1e-30))


def _quantize(w16):
    import torch
    import moex_amd as M
    O, I = w16.shape
    q = torch.empty((O, I), dtype=torch.int8, device="cuda")
    s = torch.empty(O, dtype=torch.float32, device="cuda")
    M.quantize_rows_i8(dev(w16.view(np.int16)), q, s, O, I)
    torch.cuda.synchronize()
    return q, s


def test_quantize_golden_and_edges():
    g = np.load(os.path.join(GOLD, "dense_i8.npz"))
    q, s = _quantize(g["w"])
    assert np.array_equal(q.cpu().numpy(), g["q"]) and np.array_equal(s.cpu().numpy().view(np.uint32), g["s"].view(np.uint32))
    rng = np.random.default_rng(41)
    w = (rng.standard_normal((300, 2048)) * np.geomspace(1e-4, 30, 300)[:, None]).astype(np.float16)
    w[0] = 0
    w[1] = np.float16(0.5)
    w[2, :] = 0; w[2, 100] = np.float16(-65504)
    w[3, 0] = np.float16(127); w[3, 1:] = np.array([0.5, 1.5, 2.5, -0.5, -3.5] * 409 + [0.5, 1.5], np.float16)
    q, s = _quantize(w)
    qr, sr = orc.quantize_rows_i8(w)
    assert np.array_equal(q.cpu().numpy(), qr) and np.array_equal(s.cpu().numpy().view(np.uint32), sr.view(np.uint32))


@pytest.fixture(scope="module", params=[(9216, 2048), (2048, 4096)], ids=["qkv", "o_proj"])
def weights(request):
    O, I = request.param
    rng = np.random.default_rng(O + I)
    w = (rng.standard_normal((O, I)) * 0.02).astype(np.float16)
    q, s = _quantize(w)
    return O, I, q, s, q.cpu().numpy(), s.cpu().numpy()


def test_gemv_vs_exact(weights):
    import torch
    import moex_amd as M
    O, I, q, s, qh, sh = weights
    rng = np.random.default_rng(7)
    x = rng.standard_normal(I).astype(np.float32)
    y = torch.empty(O, dtype=torch.float32, device="cuda")
    M.gemv_i8(q, s, dev(x), y, I, O)
    torch.cuda.synchronize()
    R = min(O, 4096)  # the reference's exact check covers the first 4096 rows
    ref = orc.dense_i8_f64(qh[:R], sh[:R], x[None])[0]
    rel = _rel(y.cpu().numpy()[:R].astype(np.float64), ref)
    report("gemv_i8 vs exact int8", O=O, I=I, rel=rel)
    assert rel < 1e-5


@pytest.mark.parametrize("S", [2, 3, 5, 8])
def test_gemm_small_rows_equal_gemv(weights, S):
    import torch
    import moex_amd as M
    O, I, q, s, _, _ = weights
    rng = np.random.default_rng(S)
    x = rng.standard_normal((S, I)).astype(np.float32)
    xd = dev(x)
    Y = torch.empty((S, O), dtype=torch.float32, device="cuda")
    M.gemm_i8(q, s, xd, Y, S, I, O)
    Yr = torch.empty_like(Y)
    for t in range(S):
        M.gemv_i8(q, s, xd[t], Yr[t], I, O)
    torch.cuda.synchronize()
    assert np.array_equal(Y.cpu().numpy(), Yr.cpu().numpy())


@pytest.mark.parametrize("S", [9, 64, 300, 1024])
def test_gemm_vs_gemv_and_model(weights, S):
    import torch
    import moex_amd as M
    O, I, q, s, qh, sh = weights
    rng = np.random.default_rng(100 + S)
    x = rng.standard_normal((S, I)).astype(np.float32)
    xd = dev(x)
    Y = torch.empty((S, O), dtype=torch.float32, device="cuda")
    M.gemm_i8(q, s, xd, Y, S, I, O)
    Yr = torch.empty_like(Y)
    for t in range(S):
        M.gemv_i8(q, s, xd[t], Yr[t], I, O)
    torch.cuda.synchronize()
    got, per_token = Y.cpu().numpy(), Yr.cpu().numpy()
    rel_k12 = _rel(got.astype(np.float64), per_token.astype(np.float64))
    rows = sorted({0, S // 2, S - 1})
    cols = np.arange(0, O, max(1, O // 512))
    model = orc.dense_i8_fp16x(qh[cols], sh[cols], x[rows])
    rel_model = _rel(got[np.ix_(rows, cols)].astype(np.float64), model)
    report("gemm_i8", O=O, I=I, S=S, rel_vs_gemv=rel_k12, rel_vs_model=rel_model)
    assert np.all(np.isfinite(got)) and rel_k12 < 5e-3 and rel_model < 1e-5


def test_ragged_rows():
    """O not a multiple of the GEMV row group (8) or the GEMM tile (128), S not a multiple of the GEMM tile."""
    import torch
    import moex_amd as M
    O, I, S = 1000, 512, 77
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((O, I)) * 0.1).astype(np.float16)
    q, s = _quantize(w)
    qh, sh = q.cpu().numpy(), s.cpu().numpy()
    x = rng.standard_normal((S, I)).astype(np.float32)
    Y = torch.full((S, O), float("nan"), dtype=torch.float32, device="cuda")
    M.gemm_i8(q, s, dev(x), Y, S, I, O)
    y1 = torch.full((O,), float("nan"), dtype=torch.float32, device="cuda")
    M.gemv_i8(q, s, dev(x[0]), y1, I, O)
    torch.cuda.synchronize()
    assert _rel(Y.cpu().numpy().astype(np.float64), orc.dense_i8_fp16x(qh, sh, x)) < 1e-5
    assert _rel(y1.cpu().numpy().astype(np.float64), orc.dense_i8_f64(qh, sh, x[:1])[0]) < 1e-5


def test_gemm_both_kernels_ragged():
    """A grid above one pass of the chip (the 4-wavefront kernel) and one within it (the warp-specialised kernel, here
    with K split in two and summed by a second kernel), both with O and S ragged against the 128 x 128 tile: each
    against the precision model, and a row shared by the two calls equal up to the fp32 order of the K sums."""
    import torch
    import moex_amd as M
    O, I = 9000, 1024
    rng = np.random.default_rng(8)
    w = (rng.standard_normal((O, I)) * 0.05).astype(np.float16)
    q, s = _quantize(w)
    qh, sh = q.cpu().numpy(), s.cpu().numpy()
    x = rng.standard_normal((1000, I)).astype(np.float32)
    xd = dev(x)
    outs = {}
    for S in (1000, 200):  # 71 x 8 = 568 blocks; 71 x 2 = 142 blocks
        Y = torch.full((S, O), float("nan"), dtype=torch.float32, device="cuda")
        M.gemm_i8(q, s, xd[:S], Y, S, I, O)
        torch.cuda.synchronize()
        got = Y.cpu().numpy()
        rows = [0, 129, S - 1]
        cols = np.r_[0:O:97, O - 1]
        rel = _rel(got[np.ix_(rows, cols)].astype(np.float64), orc.dense_i8_fp16x(qh[cols], sh[cols], x[rows]))
        report("gemm_i8 ragged", O=O, I=I, S=S, rel_vs_model=rel)
        assert np.all(np.isfinite(got)) and rel < 1e-5
        outs[S] = got
    assert _rel(outs[200].astype(np.float64), outs[1000][:200].astype(np.float64)) < 1e-6


def test_many_row_groups():
    """O large enough that a wavefront takes several row groups (the looped GEMV: lm_head-like shapes), 1 and 3 rows."""
    import torch
    import moex_amd as M
    O, I = 40000, 1024
    rng = np.random.default_rng(6)
    w = (rng.standard_normal((O, I)) * 0.05).astype(np.float16)
    q, s = _quantize(w)
    qh, sh = q.cpu().numpy(), s.cpu().numpy()
    x = rng.standard_normal((3, I)).astype(np.float32)
    Y = torch.full((3, O), float("nan"), dtype=torch.float32, device="cuda")
    M.gemm_i8(q, s, dev(x), Y, 3, I, O)
    y1 = torch.full((O,), float("nan"), dtype=torch.float32, device="cuda")
    M.gemv_i8(q, s, dev(x[1]), y1, I, O)
    torch.cuda.synchronize()
    got = Y.cpu().numpy()
    assert _rel(got.astype(np.float64), orc.dense_i8_f64(qh, sh, x)) < 1e-5
    assert np.array_equal(got[1], y1.cpu().numpy())
