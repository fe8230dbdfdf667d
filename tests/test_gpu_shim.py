"""The reference-side C++ shim of INTEGRATION.md (section 2), compiled verbatim by tests/shim/Makefile into
tests/shim/shim_driver, drives the library with the reference's own signatures (kernels.cuh:1713,1850,1867,1875):
kv_alloc + kv_bytes, attn_decode for a 64-token prefill chunk (the FA path), attn_fa again on the same queries,
then attn_decode for one token with split partials. Outputs are checked against the fp64 oracle on the driver's own
qo and cache: the test_fa.cu:114 rule for the chunk, 1e-4 of max|ref| for the token (test_kernels.cu:849)."""
import os
import subprocess

import numpy as np
import pytest

from oracle import oracle as orc
from tests.gpu_util import AHD, H, KV, report, sample_rows

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "tests", "shim", "shim_driver")
LQ = H * 2 * AHD + 2 * KV * AHD


def test_shim_builds_from_integration_md():
    """CPU: the shim block of INTEGRATION.md compiles with hipcc against include/moex_attn.h (make is a no-op when
    the driver is current)."""
    if not os.path.exists(os.path.join(ROOT, "moex_amd", "libmoex_attn.so")):
        pytest.skip("libmoex_attn.so not built")
    if not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("no hipcc")
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "tests", "shim")], check=True)
    assert os.path.exists(DRIVER)


@pytest.mark.gpu
@pytest.mark.parametrize("turbo", [0, 1])
def test_shim_drives_the_library(tmp_path, turbo):
    assert os.path.exists(DRIVER), "tests/shim/shim_driver is not built (run __graft_entry__.build())"
    T0, ns = 64, 16
    max_t = T0 + 8
    rng = np.random.default_rng(50 + turbo)
    qkv = rng.standard_normal((T0 + 1, LQ)).astype(np.float32)
    norm = (rng.standard_normal(2 * AHD) * 0.1).astype(np.float16)
    qkv.tofile(tmp_path / "qkv.bin")
    norm.tofile(tmp_path / "norm.bin")
    r = subprocess.run([DRIVER, str(tmp_path), str(turbo), str(T0), str(ns)], capture_output=True, text=True,
                       timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0
    hc = orc.HostCache(KV, max_t, turbo)
    hc.k[:] = np.fromfile(tmp_path / "cache_k.bin", np.int8).reshape(hc.k.shape)
    hc.v[:] = np.fromfile(tmp_path / "cache_v.bin", np.int8).reshape(hc.v.shape)
    hc.ks[:] = np.fromfile(tmp_path / "cache_ks.bin", np.float32).reshape(hc.ks.shape)
    hc.vs[:] = np.fromfile(tmp_path / "cache_vs.bin", np.float32).reshape(hc.vs.shape)
    f32 = lambda n, *s: np.fromfile(tmp_path / n, np.float32).reshape(s)
    qo, out, fa = f32("chunk_qo.bin", T0, H, AHD), f32("chunk_out.bin", T0, H, AHD), f32("chunk_fa.bin", T0, H, AHD)
    gate = qkv[:T0]
    rows = sample_rows(T0)
    if turbo:  # attn_fa alone writes the rotated-domain output (no gate); attn_decode adds turbo_out
        ref_fa = orc.attn_rows_f64(qo, None, LQ, H, hc, 0, rows)
        got_fa = np.stack([fa[t, h] for t, h in rows])
        e = float(np.abs(got_fa - ref_fa).max())
        assert e <= 2e-3 * float(np.abs(ref_fa).max())
    else:
        assert np.array_equal(out.view(np.uint32), fa.view(np.uint32))  # attn_decode's FA branch == attn_fa
    ref = orc.attn_rows_f64(qo, gate, LQ, H, hc, 0, rows)
    emu = orc.attn_rows_fa_emul(qo, gate, LQ, H, hc, 0, rows)
    got = np.stack([out[t, h] for t, h in rows])
    mag = float(np.abs(ref).max())
    e_new, e_ref = float(np.abs(got - ref).max()), float(np.abs(emu - ref).max())
    report("shim chunk", turbo=turbo, e_new=e_new, e_ref=e_ref, mag=mag)
    assert e_new <= 2 * e_ref + 1e-3 * mag
    dq, do = f32("dec_qo.bin", 1, H, AHD), f32("dec_out.bin", 1, H, AHD)
    ref = orc.attn_rows_f64(dq, qkv[T0:T0 + 1], LQ, H, hc, T0, [(0, h) for h in range(H)])
    err, mag = float(np.abs(do[0] - ref).max()), float(np.abs(ref).max())
    report("shim decode", turbo=turbo, err=err, mag=mag)
    assert err <= 1e-4 * mag


@pytest.mark.gpu
def test_shim_dense_forms(tmp_path):
    """The dense projections' shim block of INTEGRATION.md with the reference's struct Mat: int4 and int6 quantized
    through the library (bit-exact against the oracle), then gemv (1 row) and gemm (16 rows, the MFMA GEMM) for the
    int4, int6 and fp16 forms, against the exact product (K11: 1e-5) and the GEMM's precision model (1e-5)."""
    assert os.path.exists(DRIVER), "tests/shim/shim_driver is not built (run __graft_entry__.build())"
    O, I, S = 1000, 512, 16
    rng = np.random.default_rng(52)
    w = (rng.standard_normal((O, I)) * 0.05).astype(np.float16)
    x = rng.standard_normal((S, I)).astype(np.float32)
    w.tofile(tmp_path / "w16.bin")
    x.tofile(tmp_path / "x.bin")
    r = subprocess.run([DRIVER, str(tmp_path), "dense", str(O), str(I), str(S)], capture_output=True, text=True,
                       timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0
    rd = lambda n, t, *s: np.fromfile(tmp_path / n, t).reshape(s)
    q4, s4 = orc.quantize_rows_q4(w)
    q6, q6h, s6 = orc.quantize_rows_q6(w)
    assert np.array_equal(rd("q4.bin", np.uint8, O, I // 2), q4)
    assert np.array_equal(rd("s4.bin", np.float32, O, I // 64), s4)
    assert np.array_equal(rd("q6.bin", np.uint8, O, I // 2), q6) and np.array_equal(rd("q6h.bin", np.uint8, O, I // 4), q6h)
    assert np.array_equal(rd("s6.bin", np.float32, O, I // 64), s6)
    forms = {"q4": (orc.MAT_Q4, q4, None, s4), "q6": (orc.MAT_Q6, q6, q6h, s6), "f16": (orc.MAT_F16, w, None, None)}
    for nm, (F, a, b, c) in forms.items():
        y, Y = rd(f"y_{nm}.bin", np.float32, O), rd(f"Y_{nm}.bin", np.float32, S, O)
        ref = orc.dense_mat_f64(F, a, b, c, x[:1])[0]
        model = orc.dense_mat_fp16x(F, a, b, c, x)
        e1 = float(np.abs(y - ref).max() / np.abs(ref).max())
        e2 = float(np.abs(Y - model).max() / np.abs(model).max())
        report("dense shim", form=nm, rel_gemv=e1, rel_gemm=e2)
        assert e1 < 1e-5 and e2 < 1e-5
