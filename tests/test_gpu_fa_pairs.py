"""Full-grid attn_fa chunks (kernels.cuh:1443-1728): token tile t's keys grow with t, so the kernel pairs the heaviest
tile with the lightest on two workgroups, splits the heavy tile's keys between them so both do about half of the
pair, and merges the heavy tile's two halves in the kernel (the workgroup that finishes last merges). Checked here:

- the test_fa.cu:114 gate (e <= 2 e_ref + 1e-3 max|ref|) on rows of split heavy tiles and of light tiles;
- agreement over every row with one workgroup per token tile (MOEX_FA_PAIR=0) to the FA split tolerance;
- bit-identical results on repeated calls and on graph replays: the merge is symmetric in the two halves, so the
  bits do not depend on which workgroup arrives first, and the arrival counters stay consistent across launches.
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.gpu_util import AHD, H, KV, LD, dev, download, pos_tensor, random_int8_cache, report, upload

pytestmark = pytest.mark.gpu

# (pos0, T): pos0 = 0 is the most unbalanced; 4080 tokens give an odd tile count (255: a middle tile
# on one workgroup) and two workgroups per CU; 2047 a partial last tile
CASES = [(0, 2048), (0, 4080), (100, 2047), (4093, 2048)]


def _rows(T):
    toks = sorted({t for t in (0, T // 3, T // 2, (3 * T) // 4, T - 33, T - 16, T - 9, T - 1) if 0 <= t < T})
    return [(t, h) for t in toks for h in range(H)]


def _gate(name, out, qo, qg, hc, pos0, T):
    rows = _rows(T)
    ref = orc.attn_rows_f64(qo, qg, LD, H, hc, pos0, rows)
    emu = orc.attn_rows_fa_emul(qo, qg, LD, H, hc, pos0, rows)
    got = np.stack([out[t, h] for t, h in rows])
    mag = float(np.abs(ref).max())
    e_new, e_ref = float(np.abs(got - ref).max()), float(np.abs(emu - ref).max())
    report(name, pos0=pos0, T=T, e_new=e_new, e_ref=e_ref, mag=mag)
    assert np.all(np.isfinite(got))
    assert e_new <= 2.0 * e_ref + 1e-3 * mag


@pytest.fixture(scope="module")
def setup():
    max_t = 8192 + 64
    hc = random_int8_cache(max_t, seed=41)
    rng = np.random.default_rng(42)
    qo = rng.uniform(-2, 2, (4096, H, AHD)).astype(np.float32)
    qg = rng.uniform(-2, 2, (4096, LD)).astype(np.float32)
    return hc, upload(hc), qo, qg, dev(qo), dev(qg)


def _fa(dc, qo_d, qg_d, pos0, T, stream=None):
    import torch
    import moex_amd as M
    out = torch.full((T, H, AHD), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()  # the fill runs on torch's stream, the call on `stream`
    M.attn_fa(qo_d, qg_d, dc, out, H, KV, pos_tensor(pos0), dc.max_t, LD, T, stream)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("pos0,T", CASES)
def test_pairs_int8(setup, pos0, T, monkeypatch):
    hc, dc, qo, qg, qo_d, qg_d = setup
    monkeypatch.setenv("MOEX_FA_PAIR", "1")
    a = _fa(dc, qo_d[:T], qg_d[:T], pos0, T)
    b = _fa(dc, qo_d[:T], qg_d[:T], pos0, T)
    monkeypatch.setenv("MOEX_FA_PAIR", "0")
    one = _fa(dc, qo_d[:T], qg_d[:T], pos0, T)
    assert np.all(np.isfinite(a)) and np.all(np.isfinite(one))
    assert np.array_equal(a, b), "repeated pair calls differ"
    _gate("fa pairs int8", a, qo, qg, hc, pos0, T)
    _gate("fa one tile per workgroup int8", one, qo, qg, hc, pos0, T)
    mag = float(np.abs(one).max())
    d = float(np.abs(a - one).max())
    report("fa pairs vs one tile per workgroup", pos0=pos0, T=T, maxdiff=d, mag=mag)
    assert d <= 2e-3 * mag
    # the light tiles and unsplit pairs run the same arithmetic as one tile per workgroup: most rows are identical
    same = float(np.mean(np.all(a == one, axis=-1)))
    report("fa pairs: rows bit-identical to one tile per workgroup", frac=same)
    assert same > 0.4


def test_pairs_turbo():
    import torch
    import moex_amd as M
    max_t, n = 2112, 2048
    dc = M.DeviceKVCache(KV, max_t, 1)
    g = torch.Generator(device="cuda").manual_seed(43)
    k = torch.randn((n, KV * AHD), generator=g, device="cuda")
    v = torch.randn((n, KV * AHD), generator=g, device="cuda")
    M.kv_append(k, v, dc, KV, pos_tensor(0), max_t, KV * AHD, n)
    torch.cuda.synchronize()
    hc = download(dc)
    rng = np.random.default_rng(44)
    qo = rng.standard_normal((n, H, AHD)).astype(np.float32)
    out = _fa(dc, dev(qo), None, 0, n)
    assert np.array_equal(out, _fa(dc, dev(qo), None, 0, n))
    _gate("fa pairs turbo (rotated)", out, qo, None, hc, 0, n)


def test_pairs_graph_replays(setup):
    """A captured full-grid attn_fa replays bit-identically to the eager call, with eager calls between replays
    (each launch moves the arrival counters by two)."""
    import torch
    import moex_amd as M
    hc, dc, qo, qg, qo_d, qg_d = setup
    pos0, T = 0, 2048
    st = torch.cuda.Stream()
    pos = pos_tensor(pos0)
    out = torch.zeros((T, H, AHD), dtype=torch.float32, device="cuda")
    with torch.cuda.stream(st):
        M.attn_fa(qo_d[:T], qg_d[:T], dc, out, H, KV, pos, dc.max_t, LD, T, st)  # creates the stream's workspaces
    st.synchronize()
    ref = out.cpu().numpy().copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        M.attn_fa(qo_d[:T], qg_d[:T], dc, out, H, KV, pos, dc.max_t, LD, T, st)
    for i in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), ref), f"replay {i} differs"
        eager = _fa(dc, qo_d[:T], qg_d[:T], pos0, T, st)
        assert np.array_equal(eager, ref)


@pytest.mark.parametrize("cus,pos0,T", [(254, 500, 2030), (254, 0, 2024), (250, 3000, 2000)])
def test_pairs_odd_tile_count(setup, cus, pos0, T, monkeypatch):
    """A pair grid with an odd number of token tiles leaves the middle tile to one workgroup alone. At 2 kv heads
    and 256 CUs no chunk gets there (a pair grid needs 2 x tiles = the CU count), so the grids are planned as for a
    chip of `cus` CUs (MOEX_FA_CUS): 127 or 125 tiles a kv head. Gate and agreement with one tile per workgroup."""
    hc, dc, qo, qg, qo_d, qg_d = setup
    monkeypatch.setenv("MOEX_FA_CUS", str(cus))
    monkeypatch.setenv("MOEX_FA_PAIR", "1")
    a = _fa(dc, qo_d[:T], qg_d[:T], pos0, T)
    assert np.array_equal(a, _fa(dc, qo_d[:T], qg_d[:T], pos0, T)), "repeated pair calls differ"
    monkeypatch.setenv("MOEX_FA_PAIR", "0")
    one = _fa(dc, qo_d[:T], qg_d[:T], pos0, T)
    _gate("fa pairs, odd tile count", a, qo, qg, hc, pos0, T)
    mag = float(np.abs(one).max())
    d = float(np.abs(a - one).max())
    report("fa odd pairs vs one tile per workgroup", cus=cus, pos0=pos0, T=T, maxdiff=d, mag=mag)
    assert np.all(np.isfinite(a)) and d <= 2e-3 * mag
    # the middle tile's rows run alone, the same arithmetic as one tile per workgroup
    mid = ((T + 15) // 16) // 2
    assert np.array_equal(a[16 * mid:16 * mid + 16], one[16 * mid:16 * mid + 16])
