"""attn_decode captured into a HIP graph, as the engine replays its decode step (moex.cu:1133): the whole step
(front + append, split GQA decode, combine, turbo_out for turbo) records with a device pos_d, and every replay -
with the position advanced and new q/k/v rows copied in eagerly between replays - matches an eager call on an
identical cache bit for bit (outputs and appended rows)."""
import numpy as np
import pytest

from tests.gpu_util import AHD, H, KV

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("turbo,T", [(0, 1), (1, 1), (0, 4), (1, 4)])
def test_attn_decode_graph_replays(turbo, T):
    """attn_decode steps (T = 1, and an int8 MTP window of 4: the front inside the split kernel) captured once and
    replayed at four positions give the eager steps' outputs and cache rows, bit for bit."""
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
                1e7, 1e-6, T, LQ)

    # graph-side static buffers
    qkv_g = torch.zeros((T, LQ), dtype=torch.float32, device="cuda")
    qo_g = torch.empty((T, H, AHD), dtype=torch.float32, device="cuda")
    out_g = torch.empty((T, H, AHD), dtype=torch.float32, device="cuda")
    part_g = torch.empty(T * H * ns * (AHD + 2), dtype=torch.float32, device="cuda")
    pos_g = torch.zeros(1, dtype=torch.int32, device="cuda")
    # eager-side buffers
    qkv_e = torch.empty((T, LQ), dtype=torch.float32, device="cuda")
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
        pos = base + T * i
        row = torch.randn((T, LQ), generator=g, device="cuda")
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
        te, tg = getattr(ce, name)[:, :base + 4 * T], getattr(cg, name)[:, :base + 4 * T]
        assert torch.equal(te, tg), name


def test_fa_images_and_dense_graph_replays():
    """attn_fa of a long chunk (tile images: its workspace exists after one eager call on the stream) and the dense
    projections (GEMV pass, MFMA GEMM) captured on that stream: every replay, with other eager work on the device
    in between, matches the eager outputs bit for bit."""
    import torch
    import moex_amd as M
    from tests.gpu_util import LD, random_int8_cache, upload
    rng = np.random.default_rng(17)
    dc = upload(random_int8_cache(3000, seed=18))
    T, pos0 = 256, 2500
    qo = torch.from_numpy(rng.uniform(-2, 2, (T, H, AHD)).astype(np.float32)).cuda()
    qg = torch.from_numpy(rng.uniform(-2, 2, (T, LD)).astype(np.float32)).cuda()
    pos = torch.tensor([pos0], dtype=torch.int32, device="cuda")
    O, I = 1024, 2048
    w16 = torch.from_numpy((rng.standard_normal((O, I)) * 0.02).astype(np.float16)).cuda()
    qw = torch.empty((O, I), dtype=torch.int8, device="cuda")
    sw = torch.empty(O, dtype=torch.float32, device="cuda")
    M.quantize_rows_i8(w16, qw, sw, O, I)
    X2 = torch.randn((2, I), device="cuda")
    X64 = torch.randn((64, I), device="cuda")
    st = torch.cuda.Stream()

    def run(out, y2, y64):
        M.attn_fa(qo, qg, dc, out, H, KV, pos, dc.max_t, LD, T, st)
        M.gemm_i8(qw, sw, X2, y2, 2, I, O, st)
        M.gemm_i8(qw, sw, X64, y64, 64, I, O, st)

    out_e, y2_e, y64_e = (torch.empty((T, H, AHD), device="cuda"), torch.empty((2, O), device="cuda"),
                          torch.empty((64, O), device="cuda"))
    torch.cuda.synchronize()
    with torch.cuda.stream(st):
        run(out_e, y2_e, y64_e)  # eager: allocates the stream's workspace, sets the kernels' attributes
    st.synchronize()
    out_g, y2_g, y64_g = torch.zeros_like(out_e), torch.zeros_like(y2_e), torch.zeros_like(y64_e)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        run(out_g, y2_g, y64_g)
    torch.cuda.synchronize()
    for i in range(3):
        out_g.zero_(); y2_g.zero_(); y64_g.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e) and torch.equal(y2_g, y2_e) and torch.equal(y64_g, y64_e), i
        X2.mul_(1.0)  # unrelated eager work between replays
        torch.cuda.synchronize()


def test_dense_forms_graph_replays():
    """The int4 / int6 / fp16 matrix forms captured on a stream after one eager call (which allocates the GEMM's
    workspaces): int4 GEMV, int6 four-row GEMV pass, fp16 GEMM with a K split and int4 GEMM, every replay bit-identical
    to the eager outputs, with eager work in between."""
    import torch
    import moex_amd as M
    rng = np.random.default_rng(19)
    O, I = 2048, 1024
    w16 = torch.from_numpy((rng.standard_normal((O, I)) * 0.02).astype(np.float16)).cuda()
    q4 = torch.empty((O, I // 2), dtype=torch.uint8, device="cuda")
    s4 = torch.empty((O, I // 64), dtype=torch.float32, device="cuda")
    q6 = torch.empty_like(q4)
    q6h = torch.empty((O, I // 4), dtype=torch.uint8, device="cuda")
    s6 = torch.empty_like(s4)
    M.quantize_rows_q4(w16, q4, s4, O, I)
    M.quantize_rows_q6(w16, q6, q6h, s6, O, I)
    m4, m6, mf = M.Mat(q4=q4, s=s4), M.Mat(q6=q6, q6h=q6h, s=s6), M.Mat(f16=w16)
    x = torch.randn((64, I), device="cuda")
    st = torch.cuda.Stream()

    def run(ys):
        M.gemv(m4, x[0], ys[0], I, O, st)
        M.gemm(m6, x[:4], ys[1], 4, I, O, st)
        M.gemm(mf, x[:16], ys[2], 16, I, O, st)   # 16 tiles: K split over workgroups, summed by a second kernel
        M.gemm(m4, x, ys[3], 64, I, O, st)

    shapes = [(O,), (4, O), (16, O), (64, O)]
    ye = [torch.empty(sh, device="cuda") for sh in shapes]
    torch.cuda.synchronize()
    with torch.cuda.stream(st):
        run(ye)
    st.synchronize()
    yg = [torch.zeros_like(y) for y in ye]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        run(yg)
    torch.cuda.synchronize()
    for i in range(3):
        for y in yg:
            y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(yg, ye)), i
        x.mul_(1.0)
        torch.cuda.synchronize()


@pytest.mark.parametrize("gqa_maxt", ["0", "64"])
def test_fa_key_pieces_graph_new_position(gqa_maxt, monkeypatch):
    """A short chunk splits its token tiles' keys into pieces chosen on the device from pos_d: one captured attn_fa
    (image pre-pass, FA kernel + merge), replayed after the position changes, matches an eager call at each position
    bit for bit. The same for the decode kernels that run such a chunk by default (split kernel + combine)."""
    import torch
    import moex_amd as M
    monkeypatch.setenv("MOEX_FA_GQA_MAXT", gqa_maxt)
    from tests.gpu_util import LD, random_int8_cache, upload
    rng = np.random.default_rng(23)
    dc = upload(random_int8_cache(12000, seed=24))
    T = 64
    qo = torch.from_numpy(rng.uniform(-2, 2, (T, H, AHD)).astype(np.float32)).cuda()
    qg = torch.from_numpy(rng.uniform(-2, 2, (T, LD)).astype(np.float32)).cuda()
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    st = torch.cuda.Stream()
    eager = {}
    for p0 in (11000, 3000, 500):
        out = torch.empty((T, H, AHD), device="cuda")
        with torch.cuda.stream(st):
            M.set_int(pos, p0, st)
            M.attn_fa(qo, qg, dc, out, H, KV, pos, dc.max_t, LD, T, st)
        st.synchronize()
        eager[p0] = out
    out_g = torch.zeros((T, H, AHD), device="cuda")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        M.attn_fa(qo, qg, dc, out_g, H, KV, pos, dc.max_t, LD, T, st)
    torch.cuda.synchronize()
    for p0 in (3000, 11000, 500):
        M.set_int(pos, p0)
        torch.cuda.synchronize()
        out_g.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, eager[p0]), p0


@pytest.mark.parametrize("turbo", [0, 1])
@pytest.mark.parametrize("T", [1, 2])
def test_one_split_decode_captured_first(turbo, T):
    """attn_decode with ns = 1 and T <= 2 (the reference's one-split call, kernels.cuh:1861-1863, which allocates
    nothing) captured as the first call on a fresh stream with no soft-error slot: the capture takes the per-head
    kernel instead of a workspace it may not allocate, reports nothing, and every replay (position advanced, new rows
    copied in between) matches the fp64 oracle at 1e-4 of max |out|. An eager call on that stream afterwards runs the
    split-K kernels with a new workspace; the graph keeps replaying correctly."""
    import torch
    import moex_amd as M
    from oracle import oracle as orc
    from tests.gpu_util import download
    LQ = H * 2 * AHD + 2 * KV * AHD
    ctx, base = 2048, 1500
    c = M.DeviceKVCache(KV, ctx, turbo)
    g = torch.Generator(device="cuda").manual_seed(31 + T + 2 * turbo)
    kv = torch.randn((base, 2 * KV * AHD), generator=g, device="cuda")
    M.kv_append(kv[:, :KV * AHD], kv[:, KV * AHD:], c, KV, torch.zeros(1, dtype=torch.int32, device="cuda"), ctx,
                2 * KV * AHD, base)
    qn = torch.zeros(AHD, dtype=torch.int16, device="cuda")
    qkv = torch.zeros((T, LQ), device="cuda")
    qo = torch.empty((T, H, AHD), device="cuda")
    out = torch.empty((T, H, AHD), device="cuda")
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    held = M.lib().moex_workspace_held()
    st = torch.cuda.Stream()

    def step():
        M.attn_decode(qkv, qkv[:, H * 2 * AHD:], qkv[:, H * 2 * AHD + KV * AHD:], qn, qn, qo, c, out, H, KV, pos, ctx,
                      64, 1e7, 1e-6, T, LQ, st, None, 1)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        step()
    torch.cuda.synchronize()
    assert M.lib().moex_workspace_held() == held  # nothing allocated under capture
    for i in range(4):
        p = base + T * i
        qkv.copy_(torch.randn((T, LQ), generator=g, device="cuda"))
        M.set_int(pos, p)
        torch.cuda.synchronize()
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        if i == 2:  # an eager step on the capturing stream: split-K with its own workspace, then the graph again
            with torch.cuda.stream(st):
                step()
            st.synchronize()
        hc = download(c)
        rows = [(t, h) for t in range(T) for h in range(H)]
        ref = orc.attn_rows_f64(qo.cpu().numpy(), qkv.cpu().numpy(), LQ, H, hc, p, rows).reshape(T, H, AHD)
        got = out.cpu().numpy()
        err, mag = float(np.abs(got - ref).max()), float(np.abs(ref).max())
        print(f"one-split capture turbo={turbo} T={T} replay {i}: err={err:.3e} mag={mag:.3e}", flush=True)
        assert np.all(np.isfinite(got)) and err <= 1e-4 * mag, i
