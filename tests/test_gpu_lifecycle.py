"""KV-cache lifecycle inside a session: positions are overwritten, never invalidated.

The engine rolls back by position only (moex.cu:1943-1990, session.h:222-249): after an MTP verify window of T
draft tokens it continues at the first rejected position, and a checkpoint restore re-prefills from an earlier
position. The cache rows past pos_d + T are then stale drafts that every kernel must ignore (tests/test_fa.cu:23:
rows past the end are garbage). Checked here through attn_decode, int8 and turbo:
  - a verify window of 4 followed by a step at the first rejected position leaves rows [0, p + 1] bit-identical to a
    cache that only ever saw the accepted tokens, and that step's output is bit-identical too (the stale rows
    p + 2, p + 3 are not read);
  - re-prefilling a span of earlier positions with other tokens (a checkpoint restore) leaves the cache and the next
    chunk's output bit-identical to a cache built directly from the restored history.
"""
import numpy as np
import pytest

from tests.gpu_util import AHD, H, KV, report

pytestmark = pytest.mark.gpu

LQ = H * 2 * AHD + 2 * KV * AHD


class Session:
    def __init__(self, ctx, turbo):
        import torch
        import moex_amd as M
        self.M, self.torch, self.ctx = M, torch, ctx
        self.c = M.DeviceKVCache(KV, ctx, turbo)
        self.qn = torch.zeros(AHD, dtype=torch.int16, device="cuda")
        self.kn = torch.zeros(AHD, dtype=torch.int16, device="cuda")
        self.pos_d = torch.zeros(1, dtype=torch.int32, device="cuda")
        self.ns = 8
        self.part = torch.empty(8 * H * self.ns * (AHD + 2), dtype=torch.float32, device="cuda")

    def step(self, qkv, p0, splits):
        """attn_decode of len(qkv) tokens at position p0 (split decode when splits, else the FA / prefill path)."""
        torch, M = self.torch, self.M
        T = qkv.shape[0]
        qo = torch.empty((T, H, AHD), dtype=torch.float32, device="cuda")
        out = torch.empty((T, H, AHD), dtype=torch.float32, device="cuda")
        M.set_int(self.pos_d, p0)
        M.attn_decode(qkv, qkv[:, H * 2 * AHD:], qkv[:, H * 2 * AHD + KV * AHD:], self.qn, self.kn, qo, self.c, out,
                      H, KV, self.pos_d, self.ctx, 64, 1e7, 1e-6, T, LQ, None, self.part if splits else None,
                      self.ns if splits else 1)
        torch.cuda.synchronize()
        return out.cpu().numpy()

    def rows(self, n):
        return [a[:, :n].cpu().numpy() for a in (self.c.k, self.c.v, self.c.ks, self.c.vs)]


def _tokens(n, seed):
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn((n, LQ), generator=g, device="cuda")


@pytest.mark.parametrize("turbo", [0, 1])
def test_rejected_drafts_are_overwritten(turbo):
    ctx, p = 3000, 2000
    hist = _tokens(p, 1)
    draft = _tokens(4, 2)      # verify window: token p accepted, p + 1 .. p + 3 rejected
    nxt = _tokens(1, 3)        # the token the engine continues with at p + 1
    a, b = Session(ctx, turbo), Session(ctx, turbo)
    for s in (a, b):
        for q in range(0, p, 512):
            s.step(hist[q:q + 512], q, False)
    a.step(draft, p, True)             # writes rows p .. p + 3
    b.step(draft[:1], p, True)         # only the accepted token
    oa = a.step(nxt, p + 1, True)      # overwrites row p + 1; rows p + 2, p + 3 stay stale in a
    ob = b.step(nxt, p + 1, True)
    ra, rb = a.rows(p + 2), b.rows(p + 2)
    report("rejected drafts", turbo=turbo, maxdiff=float(np.abs(oa - ob).max()))
    assert all(np.array_equal(x, y) for x, y in zip(ra, rb))
    assert np.all(np.isfinite(oa)) and np.array_equal(oa, ob)


@pytest.mark.parametrize("turbo", [0, 1])
def test_checkpoint_restore_reprefill(turbo):
    ctx = 3000
    hist = _tokens(1600, 4)
    alt = _tokens(600, 5)      # the restored branch: positions 1000 .. 1599 get other tokens
    chunk = _tokens(256, 6)
    a, b = Session(ctx, turbo), Session(ctx, turbo)
    for q in range(0, 1600, 400):
        a.step(hist[q:q + 400], q, False)
    a.step(alt[:300], 1000, False)     # restore to 1000 and re-prefill in two chunks
    a.step(alt[300:], 1300, False)
    for q in range(0, 1000, 500):
        b.step(hist[q:q + 500], q, False)
    b.step(alt, 1000, False)
    oa = a.step(chunk, 1600, False)
    ob = b.step(chunk, 1600, False)
    ra, rb = a.rows(1856), b.rows(1856)
    report("checkpoint restore", turbo=turbo, maxdiff=float(np.abs(oa - ob).max()))
    assert all(np.array_equal(x, y) for x, y in zip(ra, rb))
    assert np.all(np.isfinite(oa)) and np.array_equal(oa, ob)


@pytest.mark.parametrize("turbo", [0, 1])
def test_kv_alloc_cache_serves_attention(turbo):
    """kv_alloc (kernels.cuh:1867) arrays hold the appended rows exactly as caller-owned ones do: the same rows
    appended into a kv_alloc cache and into torch-backed arrays give bit-identical attention, then kv_free."""
    import torch
    import moex_amd as M
    max_t, n = 2048, 1500
    assert M.kv_bytes(KV, max_t, turbo) == KV * max_t * (240 if turbo else 520)
    a = M.kv_alloc(KV, max_t, turbo)
    assert a.k and a.v and a.ks and a.vs and a.turbo == turbo
    b = M.DeviceKVCache(KV, max_t, turbo)
    g = torch.Generator(device="cuda").manual_seed(60 + turbo)
    k = torch.randn((n, KV * AHD), generator=g, device="cuda")
    v = torch.randn((n, KV * AHD), generator=g, device="cuda")
    qo = torch.randn((3, H, AHD), generator=g, device="cuda")
    pos = torch.tensor([0], dtype=torch.int32, device="cuda")
    outs = []
    for c in (a, b):
        M.kv_append(k, v, c, KV, pos, max_t, KV * AHD, n)
        o = torch.full((3, H, AHD), float("nan"), device="cuda")
        M.attn_decode_heads(qo, None, c, o, H, KV, torch.tensor([n - 3], dtype=torch.int32, device="cuda"), max_t,
                            H * 2 * AHD, None, 3, 1)
        torch.cuda.synchronize()
        outs.append(o.cpu().numpy())
    M.kv_free(a)
    torch.cuda.synchronize()
    report("kv_alloc cache", turbo=turbo, identical=bool(np.array_equal(outs[0], outs[1])))
    assert np.all(np.isfinite(outs[0])) and np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
