"""Shared helpers of the GPU parity tests: seeded inputs, device caches, oracle comparisons."""
import numpy as np

from oracle import oracle as orc

AHD = 256
H, KV = 16, 2
LD = H * 2 * AHD  # q rows as test_fa.cu: query ++ gate per head


def torch_dev():
    import torch
    return torch


def dev(a):
    torch = torch_dev()
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def pos_tensor(p):
    torch = torch_dev()
    return torch.tensor([p], dtype=torch.int32, device="cuda")


def random_int8_cache(max_t, seed, kv=KV):
    """tests/test_fa.cu:17-31: uniform int8 codes in [-127, 127], scales U(0.005, 0.05), the whole cache filled
    (rows past a case's end are garbage the kernels must ignore)."""
    rng = np.random.default_rng(seed)
    c = orc.HostCache(kv, max_t, 0)
    c.k[:] = rng.integers(-127, 128, c.k.shape, dtype=np.int8)
    c.v[:] = rng.integers(-127, 128, c.v.shape, dtype=np.int8)
    c.ks[:] = rng.uniform(0.005, 0.05, c.ks.shape).astype(np.float32)
    c.vs[:] = rng.uniform(0.005, 0.05, c.vs.shape).astype(np.float32)
    return c


def upload(hc):
    import moex_amd as M
    d = M.DeviceKVCache(hc.KV, hc.max_t, hc.turbo)
    torch = torch_dev()
    d.k.copy_(torch.from_numpy(hc.k.view(np.uint8) if hc.turbo else hc.k))
    d.v.copy_(torch.from_numpy(hc.v.view(np.uint8) if hc.turbo else hc.v))
    d.ks.copy_(torch.from_numpy(hc.ks))
    d.vs.copy_(torch.from_numpy(hc.vs))
    return d


def download(dc):
    hc = orc.HostCache(dc.KV, dc.max_t, dc.turbo)
    hc.k[:] = dc.k.cpu().numpy().view(np.int8)
    hc.v[:] = dc.v.cpu().numpy().view(np.int8)
    hc.ks[:] = dc.ks.cpu().numpy()
    hc.vs[:] = dc.vs.cpu().numpy()
    return hc


def sample_rows(T, heads=range(H)):
    """tests/test_fa.cu:95: tokens {0, T/3, T/2, T-2, T-1} x all heads."""
    toks = sorted({t for t in (0, T // 3, T // 2, T - 2, T - 1) if 0 <= t < T})
    return [(t, h) for t in toks for h in heads]


def max_err(got, ref):
    return float(np.abs(got.astype(np.float64) - ref).max())


def report(name, **kw):
    print(name, " ".join(f"{k}={v:.3e}" if isinstance(v, float) else f"{k}={v}" for k, v in kw.items()), flush=True)


def _threads():
    import os
    return max(1, min(16, os.cpu_count() or 1))  # the GPU box grants 16 host cores to a job


def rows_threaded(fn, qo, gate, ld, Hq, cache, pos0, rows):
    """fn (orc.attn_rows_f64 / orc.attn_rows_fa_emul) over the rows, spread over host threads (the C oracle releases
    the GIL): the long-context configs take ~0.5 s of fp64 work per row."""
    from concurrent.futures import ThreadPoolExecutor
    rows = list(rows)
    n = _threads()
    parts = [rows[i::n] for i in range(n) if rows[i::n]]
    with ThreadPoolExecutor(len(parts)) as ex:
        res = list(ex.map(lambda r: fn(qo, gate, ld, Hq, cache, pos0, r), parts))
    out = np.zeros((len(rows), AHD), np.float64)
    for i, r in enumerate(res):
        out[i::n][:len(r)] = r
    return out


def append_threaded(cache, k, v, ld, T, pos0, chunk=8192):
    """orc.kv_append in chunks of tokens over host threads (rows are independent)."""
    from concurrent.futures import ThreadPoolExecutor
    jobs = [(t, min(chunk, T - t)) for t in range(0, T, chunk)]
    with ThreadPoolExecutor(_threads()) as ex:
        list(ex.map(lambda j: orc.kv_append(cache, k[j[0]:j[0] + j[1]], v[j[0]:j[0] + j[1]], ld, j[1], pos0 + j[0]), jobs))
