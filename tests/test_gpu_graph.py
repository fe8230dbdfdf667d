"""attn_decode captured into a HIP graph, as the engine replays its decode step (moex.cu:1133): the whole step
(front + append, split GQA decode, combine, turbo_out for turbo) records with a device pos_d, and every replay -
with the position advanced and new q/k/v rows copied in eagerly between replays - matches an eager call on an
identical cache bit for bit (outputs and appended rows)."""
import numpy as np
import pytest

from tests.gpu_util import AHD, H, KV

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("turbo", [0, 1])
def test_attn_decode_graph_replays(turbo):
    import torch
    import moex_amd as M
    LQ = H * 2 * AHD + 2 * KV * AHD
    ctx, base, ns = 4096, 2999, 16
    ce, cg = M.DeviceKVCache(KV, ctx, turbo), M.DeviceKVCache(KV, ctx, turbo)
    qn = torch.zeros(AHD, dtype=torch.int16, device="cuda")
    kn = torch.zeros(AHD, dtype=torch.int16, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(5)
    # the same context rows in both caches (eager, chunked FA path)
    T0 = 1000
    qkv0 = torch.empty((T0, LQ), dtype=torch.float32, device="cuda")
    qo0 = torch.empty((T0, H, AHD), dtype=torch.float32, device="cuda")
    o0 = torch.empty((T0, H, AHD), dtype=torch.float32, device="cuda")
    p0 = torch.zeros(1, dtype=torch.int32, device="cuda")
    for p in range(0, base, T0):
        n = min(T0, base - p)
        qkv0.normal_(generator=g)
        for c in (ce, cg):
            M.set_int(p0, p)
            M.attn_decode(qkv0, qkv0[:, H * 2 * AHD:], qkv0[:, H * 2 * AHD + KV * AHD:], qn, kn, qo0, c, o0, H, KV, p0,
                          ctx, 64, 1e7, 1e-6, n, LQ, None, None, 1)
    torch.cuda.synchronize()

    def step_args(qkv, qo, out, pos_d, part, c):
        return (qkv, qkv[:, H * 2 * AHD:], qkv[:, H * 2 * AHD + KV * AHD:], qn, kn, qo, c, out, H, KV, pos_d, ctx, 64,
                1e7, 1e-6, 1, LQ)

    # graph-side static buffers
    qkv_g = torch.zeros((1, LQ), dtype=torch.float32, device="cuda")
    qo_g = torch.empty((1, H, AHD), dtype=torch.float32, device="cuda")
    out_g = torch.empty((1, H, AHD), dtype=torch.float32, device="cuda")
    part_g = torch.empty(H * ns * (AHD + 2), dtype=torch.float32, device="cuda")
    pos_g = torch.zeros(1, dtype=torch.int32, device="cuda")
    # eager-side buffers
    qkv_e = torch.empty((1, LQ), dtype=torch.float32, device="cuda")
    qo_e = torch.empty_like(qo_g)
    out_e = torch.empty_like(out_g)
    part_e = torch.empty_like(part_g)
    pos_e = torch.zeros(1, dtype=torch.int32, device="cuda")

    # one eager call on a scratch cache first: one-time set-up (function attributes) happens outside the capture
    scratch = M.DeviceKVCache(KV, ctx, turbo)
    M.attn_decode(*step_args(qkv_g, qo_g, out_g, pos_g, part_g, scratch), None, part_g, ns)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        M.attn_decode(*step_args(qkv_g, qo_g, out_g, pos_g, part_g, cg), None, part_g, ns)
    torch.cuda.synchronize()

    for i in range(4):
        pos = base + i
        row = torch.randn((1, LQ), generator=g, device="cuda")
        # eager reference on ce
        qkv_e.copy_(row)
        M.set_int(pos_e, pos)
        M.attn_decode(*step_args(qkv_e, qo_e, out_e, pos_e, part_e, ce), None, part_e, ns)
        torch.cuda.synchronize()
        # graph replay on cg (inputs updated eagerly)
        qkv_g.copy_(row)
        pos_g.fill_(pos)
        graph.replay()
        torch.cuda.synchronize()
        a, b = out_g.cpu().numpy(), out_e.cpu().numpy()
        assert np.all(np.isfinite(a)) and np.array_equal(a, b), f"replay {i}: max diff {np.abs(a - b).max()}"
    # every written row (context and the four appended ones) agrees byte for byte
    for name in ("k", "v", "ks", "vs"):
        te, tg = getattr(ce, name)[:, :base + 4], getattr(cg, name)[:, :base + 4]
        assert torch.equal(te, tg), name
