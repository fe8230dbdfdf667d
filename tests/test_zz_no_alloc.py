"""moex_attn_decode_noalloc (no counterpart in the reference: attn_decode for callers that cannot allocate) against
moex_attn_decode on the same inputs, through the C ABI: the same bits wherever both run the same kernels with the
same split / piece counts (decode, per-head, short prefill chunks), two calls in a row with the second one smaller;
the FA tolerance where the scratch caps the key pieces; a clear argument error beyond the scratch's size."""
import ctypes

import numpy as np
import pytest

from tests.gpu_util import AHD, H, KV, random_int8_cache, report, upload

pytestmark = pytest.mark.gpu
LQ = H * 2 * AHD + 2 * KV * AHD


def _args(M, torch, T, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    qkv = torch.randn((T, LQ), generator=g, device="cuda")
    return qkv


def _both(M, torch, caches, qkv, pos, T, ns, max_t):
    """One step through each entry point, each on its own copy of the cache (the step appends the T rows)."""
    qn = torch.zeros(AHD, dtype=torch.int16, device="cuda")
    pos_d = torch.tensor([pos], dtype=torch.int32, device="cuda")
    L = M.lib()
    res = []
    for which, c in zip(("alloc", "noalloc"), caches):
        qo = torch.full((T, H, AHD), float("nan"), device="cuda")
        out = torch.full((T, H, AHD), float("nan"), device="cuda")
        q, k, v = qkv, qkv[:, H * 2 * AHD:], qkv[:, H * 2 * AHD + KV * AHD:]
        st = torch.cuda.current_stream().cuda_stream
        if which == "alloc":
            part = torch.empty(max(1, T * H * ns * (AHD + 2)), device="cuda")
            L.moex_attn_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), qn.data_ptr(), qn.data_ptr(), qo.data_ptr(),
                               c.c, out.data_ptr(), H, KV, pos_d.data_ptr(), max_t, 64, 1e7, 1e-6, T, LQ, st,
                               part.data_ptr(), ns)
        else:
            L.moex_attn_decode_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), qn.data_ptr(), qn.data_ptr(),
                                       qo.data_ptr(), c.c, out.data_ptr(), H, KV, pos_d.data_ptr(), max_t, 64, 1e7,
                                       1e-6, T, LQ, st, ns)
        torch.cuda.synchronize()
        res.append((qo.cpu().numpy(), out.cpu().numpy()))
    return res


@pytest.mark.parametrize("turbo", [0, 1])
def test_noalloc_matches_attn_decode(turbo):
    import torch
    import moex_amd as M
    max_t = 40064
    hc = random_int8_cache(max_t, seed=21) if not turbo else None
    if turbo:
        caches = [M.DeviceKVCache(KV, max_t, 1) for _ in range(2)]
        g = torch.Generator(device="cuda").manual_seed(22)
        kv = torch.randn((max_t, 2 * KV * AHD), generator=g, device="cuda")
        for c in caches:
            M.kv_append(kv[:, :KV * AHD], kv[:, KV * AHD:], c, KV, torch.zeros(1, dtype=torch.int32, device="cuda"),
                        max_t, 2 * KV * AHD, max_t)
    else:
        caches = [upload(hc), upload(hc)]
    torch.cuda.synchronize()
    held = M.lib().moex_workspace_held()
    # (pos, T, ns): split-K decode, then a smaller one; MTP window; a one-split call (ns == 1, T <= 2: the split-K
    # kernels with their partials in the scratch); short prefill chunks whose key pieces fit the scratch
    for i, (pos, T, ns) in enumerate([(39999, 1, 256), (5000, 1, 16), (30000, 4, 64), (1000, 2, 1),
                                      (34000, 17, 1), (5000, 3, 1)]):
        qkv = _args(M, torch, T, 100 + i)
        (qa, oa), (qb, ob) = _both(M, torch, caches, qkv, pos, T, ns, max_t)
        same = np.array_equal(oa.view(np.uint32), ob.view(np.uint32)) and np.array_equal(qa.view(np.uint32),
                                                                                      qb.view(np.uint32))
        report("noalloc vs attn_decode", turbo=turbo, pos=pos, T=T, ns=ns, identical=same)
        assert np.all(np.isfinite(ob)) and same
    # the no-allocation calls took no workspace (the attn_decode calls of these shapes had theirs before or take
    # them now; count only what the noalloc calls could have added by running one more of each)
    held = M.lib().moex_workspace_held()
    for i, (pos, T, ns) in enumerate([(39999, 1, 256), (1000, 2, 1), (5000, 3, 1)]):
        qkv = _args(M, torch, T, 200 + i)
        _noalloc_only(M, torch, caches[1], qkv, pos, T, ns, max_t)
    assert M.lib().moex_workspace_held() == held


def _noalloc_only(M, torch, c, qkv, pos, T, ns, max_t, st=None):
    qn = torch.zeros(AHD, dtype=torch.int16, device="cuda")
    pos_d = torch.tensor([pos], dtype=torch.int32, device="cuda")
    qo = torch.empty((T, H, AHD), device="cuda")
    out = torch.empty((T, H, AHD), device="cuda")
    s = st.cuda_stream if st is not None else torch.cuda.current_stream().cuda_stream
    M.lib().moex_attn_decode_noalloc(qkv.data_ptr(), qkv[:, H * 2 * AHD:].data_ptr(),
                                     qkv[:, H * 2 * AHD + KV * AHD:].data_ptr(), qn.data_ptr(), qn.data_ptr(),
                                     qo.data_ptr(), c.c, out.data_ptr(), H, KV, pos_d.data_ptr(), max_t, 64, 1e7, 1e-6,
                                     T, LQ, s, ns)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("turbo", [0, 1])
def test_noalloc_per_head_path(turbo):
    """A cache of 256 positions gives one split (moex_gqa_splits = 1): ns == 1, T <= 2 then runs the per-head kernel
    in both entry points, bit for bit, two calls in a row, the second smaller."""
    import torch
    import moex_amd as M
    max_t = 256
    assert M.lib().moex_gqa_splits(2, KV, M.lib().moex_decode_splits(max_t), turbo) == 1
    caches = [M.DeviceKVCache(KV, max_t, turbo) for _ in range(2)]
    g = torch.Generator(device="cuda").manual_seed(41)
    kv = torch.randn((max_t, 2 * KV * AHD), generator=g, device="cuda")
    for c in caches:
        M.kv_append(kv[:, :KV * AHD], kv[:, KV * AHD:], c, KV, torch.zeros(1, dtype=torch.int32, device="cuda"),
                    max_t, 2 * KV * AHD, max_t)
    torch.cuda.synchronize()
    for i, (pos, T) in enumerate([(200, 2), (100, 1)]):
        qkv = _args(M, torch, T, 300 + i)
        (qa, oa), (qb, ob) = _both(M, torch, caches, qkv, pos, T, 1, max_t)
        same = np.array_equal(oa.view(np.uint32), ob.view(np.uint32)) and np.array_equal(qa.view(np.uint32),
                                                                                      qb.view(np.uint32))
        report("noalloc per-head", turbo=turbo, pos=pos, T=T, identical=same)
        assert np.all(np.isfinite(ob)) and same


@pytest.mark.parametrize("turbo", [0, 1])
def test_noalloc_captured_first(turbo):
    """A no-allocation decode step captured into a HIP graph as the first library call on a new stream (the
    scratch's address is looked up before the capture by the library's first use on the device, or inside it):
    three replays, the position advanced eagerly between them, each equal bit for bit to an eager no-allocation call
    on a copy of the cache, and no workspace taken."""
    import torch
    import moex_amd as M
    max_t, base, ns = 8192, 6000, 64
    caches = [M.DeviceKVCache(KV, max_t, turbo) for _ in range(2)]
    g = torch.Generator(device="cuda").manual_seed(43)
    kv = torch.randn((base, 2 * KV * AHD), generator=g, device="cuda")
    for c in caches:
        M.kv_append(kv[:, :KV * AHD], kv[:, KV * AHD:], c, KV, torch.zeros(1, dtype=torch.int32, device="cuda"),
                    max_t, 2 * KV * AHD, base)
    torch.cuda.synchronize()
    held = M.lib().moex_workspace_held()
    L = M.lib()
    qn = torch.zeros(AHD, dtype=torch.int16, device="cuda")
    qkv_g = torch.zeros((1, LQ), device="cuda")
    qo_g, out_g = torch.empty((1, H, AHD), device="cuda"), torch.empty((1, H, AHD), device="cuda")
    pos_g = torch.zeros(1, dtype=torch.int32, device="cuda")
    st = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        L.moex_attn_decode_noalloc(qkv_g.data_ptr(), qkv_g[:, H * 2 * AHD:].data_ptr(),
                                   qkv_g[:, H * 2 * AHD + KV * AHD:].data_ptr(), qn.data_ptr(), qn.data_ptr(),
                                   qo_g.data_ptr(), caches[0].c, out_g.data_ptr(), H, KV, pos_g.data_ptr(), max_t, 64,
                                   1e7, 1e-6, 1, LQ, st.cuda_stream, ns)
    torch.cuda.synchronize()
    for i in range(3):
        pos = base + i
        row = torch.randn((1, LQ), generator=g, device="cuda")
        ref = _noalloc_only(M, torch, caches[1], row, pos, 1, ns, max_t)
        qkv_g.copy_(row)
        M.set_int(pos_g, pos)
        torch.cuda.synchronize()
        out_g.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        a, b = out_g.cpu().numpy(), ref.cpu().numpy()
        report("noalloc captured", turbo=turbo, replay=i, identical=bool(np.array_equal(a.view(np.uint32), b.view(np.uint32))))
        assert np.all(np.isfinite(a)) and np.array_equal(a.view(np.uint32), b.view(np.uint32)), i
    assert M.lib().moex_workspace_held() == held


def test_noalloc_capped_pieces_and_rejection(monkeypatch):
    """T = 64 at 32000 on the FA kernel (MOEX_FA_GQA_MAXT=0) would take 32 key pieces (34 MB of partials): the
    scratch (32 MiB) holds 31, so the result is within the FA split tolerance (2e-3 of max |out|, as split vs
    unsplit). T*H*ns*1032 beyond the scratch is an argument error that leaves out untouched."""
    import torch
    import moex_amd as M
    monkeypatch.setenv("MOEX_FA_GQA_MAXT", "0")
    max_t = 32064
    hc = random_int8_cache(max_t, seed=23)
    caches = [upload(hc), upload(hc)]
    T, pos = 64, 32000
    qkv = _args(M, torch, T, 7)
    (_, oa), (_, ob) = _both(M, torch, caches, qkv, pos, T, 1, max_t)
    d, mag = float(np.abs(oa - ob).max()), float(np.abs(oa).max())
    report("noalloc capped pieces", maxdiff=d, mag=mag)
    assert np.all(np.isfinite(ob)) and d <= 2e-3 * mag
    slot = ctypes.c_int(0)
    L = M.lib()
    L.moex_set_soft_error(ctypes.byref(slot))
    try:
        out = torch.zeros((4, H, AHD), device="cuda")
        qkv = _args(M, torch, 4, 8)
        qn = torch.zeros(AHD, dtype=torch.int16, device="cuda")
        pos_d = torch.tensor([100], dtype=torch.int32, device="cuda")
        L.moex_attn_decode_noalloc(qkv.data_ptr(), qkv[:, H * 2 * AHD:].data_ptr(),
                                   qkv[:, H * 2 * AHD + KV * AHD:].data_ptr(), qn.data_ptr(), qn.data_ptr(),
                                   out.data_ptr(), caches[1].c, out.data_ptr(), H, KV, pos_d.data_ptr(), max_t, 64,
                                   1e7, 1e-6, 4, LQ, torch.cuda.current_stream().cuda_stream, 1024)
        torch.cuda.synchronize()
    finally:
        L.moex_set_soft_error(None)
    assert slot.value == 1 and float(out.abs().max()) == 0.0
