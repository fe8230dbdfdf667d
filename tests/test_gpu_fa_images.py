"""attn_fa's two staging paths and its tile-image workspace.

A chunk is widened once by the image pre-pass and copied into LDS by DMA; with MOEX_FA_IMAGES=0 the FA kernel widens
each tile itself. The two paths feed the same bytes to the same arithmetic, so the rows two chunks have in common
(same token tiles, same wavefronts, key splitting off) come out bit for bit the same. The workspace is per (device, stream) and grows with max_t; growing it, and a second stream, must not change a
result.
"""
import numpy as np
import pytest

from tests.gpu_util import AHD, H, KV, LD, dev, pos_tensor, random_int8_cache, report, upload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def data():
    rng = np.random.default_rng(21)
    qo = rng.uniform(-2, 2, (256, H, AHD)).astype(np.float32)
    qg = rng.uniform(-2, 2, (256, LD)).astype(np.float32)
    return dev(qo), dev(qg)


def _fa(dc, qo_d, qg_d, pos0, T, stream=None):
    import torch
    import moex_amd as M
    out = torch.zeros((T, H, AHD), dtype=torch.float32, device="cuda")
    M.attn_fa(qo_d, qg_d, dc, out, H, KV, pos_tensor(pos0), dc.max_t, LD, T, stream)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("turbo", [0, 1])
@pytest.mark.parametrize("pos0", [0, 777, 5000])
def test_image_path_matches_in_kernel_widening(data, turbo, pos0, monkeypatch):
    import torch
    import moex_amd as M
    # key splitting off: how a chunk's keys are split depends on T, so the two chunks would split differently
    monkeypatch.setenv("MOEX_FA_SPLIT", "1")
    qo_d, qg_d = data
    max_t = 5400
    if turbo:
        dc = M.DeviceKVCache(KV, max_t, 1)
        g = torch.Generator(device="cuda").manual_seed(5)
        k = torch.randn((max_t, KV * AHD), generator=g, device="cuda")
        v = torch.randn((max_t, KV * AHD), generator=g, device="cuda")
        M.kv_append(k, v, dc, KV, pos_tensor(0), max_t, KV * AHD, max_t)
        torch.cuda.synchronize()
    else:
        dc = upload(random_int8_cache(max_t, seed=4))
    gate = None if turbo else qg_d
    img = _fa(dc, qo_d, gate, pos0, 128)      # tile images + DMA
    img2 = _fa(dc, qo_d, gate, pos0, 128)     # the same call again: each path is deterministic
    monkeypatch.setenv("MOEX_FA_IMAGES", "0")
    ink = _fa(dc, qo_d, gate, pos0, 112)      # widened in the kernel
    ink2 = _fa(dc, qo_d, gate, pos0, 112)
    report("fa image vs in-kernel", turbo=turbo, pos0=pos0, maxdiff=float(np.abs(img[:112] - ink).max()),
           img_repeat=bool(np.array_equal(img, img2)), ink_repeat=bool(np.array_equal(ink, ink2)))
    assert np.all(np.isfinite(img))
    assert np.array_equal(img, img2) and np.array_equal(ink, ink2)
    assert np.array_equal(img[:112], ink)


def test_workspace_growth_and_streams(data):
    """Same prefix in a small and a larger cache: the larger max_t grows the stream's workspace (after the earlier
    call on the stream has finished with it); the small cache again, and the same call on a second stream, give the
    same bytes."""
    import torch
    qo_d, qg_d = data
    hs = random_int8_cache(3000, seed=8)
    hb = random_int8_cache(20000, seed=9)
    hb.k[:, :3000], hb.v[:, :3000] = hs.k, hs.v
    hb.ks[:, :3000], hb.vs[:, :3000] = hs.ks, hs.vs
    ds, db = upload(hs), upload(hb)
    pos0, T = 2700, 256
    a = _fa(ds, qo_d, qg_d, pos0, T)
    b = _fa(db, qo_d, qg_d, pos0, T)          # grows the workspace
    c = _fa(ds, qo_d, qg_d, pos0, T)
    s2 = torch.cuda.Stream()
    d = _fa(db, qo_d, qg_d, pos0, T, s2)      # a second stream: its own workspace
    report("fa workspace", maxdiff_ab=float(np.abs(a - b).max()), maxdiff_ad=float(np.abs(a - d).max()))
    assert np.all(np.isfinite(a))
    assert np.array_equal(a, b) and np.array_equal(a, c) and np.array_equal(a, d)


@pytest.mark.parametrize("wg", ["1", "3"])
def test_image_grid_loops(data, wg, monkeypatch):
    """The pre-pass grid is capped (MOEX_FA_IMG_WG workgroups per CU over the kv heads) and each workgroup loops over
    tiles: with 1 or 3 per CU the workgroups widen up to 5 of the chunk's 632 tiles per kv head each, which must give
    the bytes of the default grid (one tile per workgroup here)."""
    qo_d, qg_d = data
    dc = upload(random_int8_cache(20400, seed=12))
    pos0, T = 20000, 200
    ref = _fa(dc, qo_d, qg_d, pos0, T)
    monkeypatch.setenv("MOEX_FA_IMG_WG", wg)
    got = _fa(dc, qo_d, qg_d, pos0, T)
    report("fa image grid", wg=wg, maxdiff=float(np.abs(got - ref).max()))
    assert np.all(np.isfinite(got)) and np.array_equal(got, ref)
