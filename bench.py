"""Benchmark of the moex attention hot path on one MI355X.

Headline (BASELINE.json metric, configs[1]): one FA-2 prefill chunk of T=2048 query tokens at positions
32768..34815 over an int8 KV cache of 34816 keys (16 q heads, 2 KV heads, head_dim 256, gated), in TFLOPS with the
reference's flop count 4*H*D*T*(pos0 + T/2) (tests/test_fa.cu:137). A step = one attn_fa call; inputs (Q, gate,
cache) are resident in HBM before the timed region.

Also reported (other configs of BASELINE.json, same JSON line): decode / MTP verify at 90k context (T=1, T=4;
HBM GB/s over the 520 B/row KV, rotating over 4 caches that together exceed the MALL), TurboQuant decode at 262144 (rotating over 3 caches),
TurboQuant prefill at
260096..262143 and the int8 chunk at the same depth, and config 0 (pos0 = 0).

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--decode-only] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

H, KV, AHD = 16, 2, 256
LD = H * 2 * AHD
PEAK_F16 = 2500.0   # TFLOP/s, MI355X dense fp16 MFMA
PEAK_HBM = 8000.0   # GB/s
METRIC = "prefill attn TFLOPS @2048-chunk/32k ctx; decode attn HBM GB/s @90k ctx"


def flops_prefill(T, pos0):
    return 4.0 * H * AHD * T * (pos0 + T / 2.0)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--quick", action="store_true", help="headline only")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the configs[2] and configs[3] decode timings (for counter runs); prints their JSON")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--config4-only", action="store_true",
                    help="only the configs[4] prefill calls (for counter runs; prints no JSON line)")
    ap.add_argument("--config0-only", action="store_true",
                    help="only the configs[0] prefill calls (pos0 = 0; for counter runs; prints no JSON line)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="only run a plain 256 MiB device copy 5 times (calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--mfma-calib", action="store_true",
                    help="only time a library fp16 GEMM (torch.matmul, 8192^3) on random and on all-zero data: the "
                         "rate the chip sustains under dense MFMA load, for reading the FA kernel's roofline")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (the attention path of a batch-1 engine); "
              "--gpus must be 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import moex_amd as M
    torch.cuda.set_device(0)
    dev = "cuda"
    st = torch.cuda.current_stream()
    if a.copy_calib:
        src = torch.ones(64 << 20, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes_each_way": src.numel() * 4, "launches": 5}))
        return
    if a.mfma_calib:
        n = 8192
        g = torch.Generator(device=dev).manual_seed(3)
        res = {}
        for name, fill in (("random", True), ("zeros", False)):
            A = torch.randn((n, n), generator=g, device=dev).half() if fill else torch.zeros((n, n), device=dev).half()
            B = torch.randn((n, n), generator=g, device=dev).half() if fill else torch.zeros((n, n), device=dev).half()
            C = torch.empty((n, n), device=dev, dtype=torch.float16)
            for _ in range(10):
                torch.matmul(A, B, out=C)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(20):
                torch.matmul(A, B, out=C)
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / 20
            res[name] = {"ms": round(ms, 3), "TFLOPS": round(2 * n ** 3 / ms / 1e9, 1)}
        print(json.dumps({"mfma_calib_fp16_gemm_8192": res}))
        return

    def ev():
        return torch.cuda.Event(enable_timing=True)

    def fill_cache(cache, n, seed):
        """K, V ~ N(0,1) fp32 quantized by the product's own append kernel (int8 per row or TurboQuant)."""
        g = torch.Generator(device=dev).manual_seed(seed)
        zero = torch.zeros(1, dtype=torch.int32, device=dev)
        chunk = 32768
        for p in range(0, n, chunk):
            m = min(chunk, n - p)
            k = torch.randn((m, KV * AHD), generator=g, device=dev)
            v = torch.randn((m, KV * AHD), generator=g, device=dev)
            zero.fill_(p)
            M.kv_append(k, v, cache, KV, zero, cache.max_t, KV * AHD, m)
        torch.cuda.synchronize()

    def q_and_gate(T, seed):
        g = torch.Generator(device=dev).manual_seed(seed)
        qo = torch.randn((T, H, AHD), generator=g, device=dev).half().float()  # fp16-representable (BASELINE: fp16 Q)
        qg = torch.randn((T, LD), generator=g, device=dev).half().float()
        return qo, qg

    def settle(fn, ms=150.0):
        """Untimed: run fn for ~ms of wall time so the GPU clocks have ramped (measured on MI355X: after 5 launches
        of the configs[1] chunk it still runs 7 % slower than after 50)."""
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        while (time.perf_counter() - t0) * 1e3 < ms:
            fn()
            torch.cuda.synchronize()

    def time_steps(fn, steps, warmup):
        settle(fn)
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = ev(), ev()
        t0 = time.perf_counter()
        e0.record(st)
        for _ in range(steps):
            fn()
        e1.record(st)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3
        return e0.elapsed_time(e1) / steps, wall / steps

    def time_rotating(fns, steps):
        """Average time per call of fns[i % len(fns)] over `steps` back-to-back calls. Each fn reads its own KV
        cache and together they exceed the 256 MB MALL, so every call streams its cache from HBM; timing a loop
        avoids the event overhead that dominates a single ~20 us launch. The clocks are settled first: the
        configs[2] lines follow the CPU baseline, which leaves the GPU idle for seconds, and the compute-bound T = 4
        kernel measured 29.5 us instead of 24-25 us without this."""
        settle(lambda: [f() for f in fns], ms=100.0)
        e0, e1 = ev(), ev()
        e0.record(st)
        for i in range(steps):
            fns[i % len(fns)]()
        e1.record(st)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    def time_graph(fns, replays=10):
        """Average time per call of fns, captured in order into one HIP graph on a side stream and replayed (the way the
        engine runs its decode step): the launches' host overhead drops out, which dominates calls of a few µs made
        through Python."""
        gs = torch.cuda.Stream()
        with torch.cuda.stream(gs):
            for f in fns:
                f(gs)
        gs.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=gs):
            for f in fns:
                f(gs)
        with torch.cuda.stream(gs):
            settle(graph.replay, ms=50.0)
            e0, e1 = ev(), ev()
            e0.record(gs)
            for _ in range(replays):
                graph.replay()
            e1.record(gs)
        torch.cuda.synchronize()
        del graph
        return e0.elapsed_time(e1) / (replays * len(fns))

    res = {}
    # ---------------- headline: config 1, int8 prefill chunk at 32k ----------------
    T, pos0 = 2048, 32768
    n = pos0 + T
    c8 = M.DeviceKVCache(KV, 262144 + 64, 0)
    fill_cache(c8, 262144, seed=10)
    qo, qg = q_and_gate(T, seed=11)
    out = torch.empty((T, H, AHD), device=dev)
    pos_d = torch.tensor([pos0], dtype=torch.int32, device=dev)

    def prefill():
        M.attn_fa(qo, qg, c8, out, H, KV, pos_d, c8.max_t, LD, T, st)

    threads = cpu_threads()
    if a.config0_only:
        pz = torch.tensor([0], dtype=torch.int32, device=dev)
        ms0, _ = time_steps(lambda: M.attn_fa(qo, qg, c8, out, H, KV, pz, c8.max_t, LD, T, st), a.steps, a.warmup)
        print(f"[bench] config0 int8 prefill pos0=0: {ms0:.4f} ms, {flops_prefill(T, 0) / ms0 / 1e9:.1f} TFLOPS",
              flush=True)
        return
    want_cpu = not a.no_cpu and not a.decode_only and not a.config4_only
    hc8 = host_cache(c8, n) if want_cpu else None
    qh, gh = (qo.cpu().numpy(), qg.cpu().numpy()) if want_cpu else (None, None)
    if not a.decode_only and not a.config4_only:
        ms, wall_ms = time_steps(prefill, a.steps, a.warmup)
        tflops = flops_prefill(T, pos0) / (ms * 1e-3) / 1e12
        print(f"[bench] config1 int8 prefill T={T} pos0={pos0}: {ms:.3f} ms/step, {tflops:.1f} TFLOPS "
              f"({100 * tflops / PEAK_F16:.1f}% of {PEAK_F16:.0f})", flush=True)

    # HBM bytes per call from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes over this same call (counters
    # cannot be read inside this run); the file names the kernel source it was recorded on
    traffic, traffic_src = None, None
    tf = os.path.join(ROOT, "profiles", "fa_prefill_int8_c1_traffic.json")
    if os.path.exists(tf):
        tj = json.load(open(tf))
        traffic = tj.get("bytes_per_launch")
        traffic_src = ("profiles/fa_prefill_int8_c1_traffic.json (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; recorded on "
                       f"{tj.get('recorded_on', 'an earlier build')})")

    extra = {}
    if not a.quick:
        # ---------------- config 0: pos0 = 0 ----------------
        if not a.decode_only and not a.config4_only:
            pz = torch.tensor([0], dtype=torch.int32, device=dev)
            ms0, _ = time_steps(lambda: M.attn_fa(qo, qg, c8, out, H, KV, pz, c8.max_t, LD, T, st), 10, 3)
            extra["config0_prefill_int8"] = {"ms": round(ms0, 4),
                                             "tflops": round(flops_prefill(T, 0) / ms0 / 1e9, 1)}
            if want_cpu:
                extra["config0_prefill_int8"]["cpu"] = cpu_prefill(hc8, qh, gh, 0, T, threads, full=True)
            print(f"[bench] config0 int8 prefill pos0=0: {ms0:.3f} ms, "
                  f"{extra['config0_prefill_int8']['tflops']} TFLOPS", flush=True)
        # ---------------- config 2: decode + MTP verify at 90k (int8) ----------------
        dec = {}
        ctx = 90000
        NROT = 4  # 4 x 93.6 MB of KV > MALL
        rot = []
        for i in range(0 if a.config4_only else NROT):
            c = M.DeviceKVCache(KV, ctx + 64, 0)
            fill_cache(c, ctx, seed=20 + i)
            rot.append(c)
        for Tq in (() if a.config4_only else (1, 4)):
            ns = M.gqa_splits(Tq, KV, M.decode_splits(ctx))
            part = torch.empty(Tq * H * ns * (AHD + 2), device=dev)
            o1 = torch.empty((Tq, H, AHD), device=dev)
            pd = torch.tensor([ctx - Tq], dtype=torch.int32, device=dev)

            def gqa(c):
                return lambda: M.attn_gqa(qo[:Tq], c, H, KV, pd, c.max_t, part, Tq, ns, st)

            def full(c):
                def f():
                    M.attn_gqa(qo[:Tq], c, H, KV, pd, c.max_t, part, Tq, ns, st)
                    M.attn_combine(part, qg[:Tq], o1, H, ns, LD, Tq, st)
                return f

            t_k = time_rotating([gqa(c) for c in rot], 200)
            t_f = time_rotating([full(c) for c in rot], 200)
            # the engine replays its decode step as a graph (moex.cu:1133): 32 steps (split kernel + combine) over the
            # rotating caches captured once, replayed, timed per step
            NG = 32
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for i in range(NG):
                    c = rot[i % NROT]
                    M.attn_gqa(qo[:Tq], c, H, KV, pd, c.max_t, part, Tq, ns)
                    M.attn_combine(part, qg[:Tq], o1, H, ns, LD, Tq)
            for _ in range(3):
                graph.replay()
            torch.cuda.synchronize()
            e0, e1 = ev(), ev()
            e0.record(torch.cuda.current_stream())
            for _ in range(10):
                graph.replay()
            e1.record(torch.cuda.current_stream())
            torch.cuda.synchronize()
            t_g = e0.elapsed_time(e1) / (10 * NG)
            del graph
            kv_bytes = 2.0 * ctx * 520
            # the whole attn_decode step from the raw q/k/v rows (front, append, split kernel, combine; at T = 1
            # the split kernel runs the front and the append in its prologue). Each call rewrites rows
            # ctx - Tq .. ctx - 1 of its cache with the same bytes.
            LQ = LD + 2 * KV * AHD
            qkv = torch.randn((Tq, LQ), generator=torch.Generator(device=dev).manual_seed(7), device=dev)
            qn = torch.zeros(AHD, dtype=torch.int16, device=dev)
            qo_ad = torch.empty((Tq, H, AHD), device=dev)
            nsd = M.decode_splits(ctx)
            part_ad = torch.empty(Tq * H * nsd * (AHD + 2), device=dev)

            def adec(c):
                return lambda: M.attn_decode(qkv, qkv[:, LD:], qkv[:, LD + KV * AHD:], qn, qn, qo_ad, c, o1, H, KV,
                                             pd, c.max_t, 64, 1e7, 1e-6, Tq, LQ, st, part_ad, nsd)
            t_ad = time_rotating([adec(c) for c in rot], 200)
            dec[f"T{Tq}"] = {"ns": ns, "split_kernel_us": round(t_k * 1e3, 2), "with_combine_us": round(t_f * 1e3, 2),
                             "graph_step_us": round(t_g * 1e3, 2),
                             "GBps": round(kv_bytes / (t_f * 1e-3) / 1e9, 1),
                             "graph_GBps": round(kv_bytes / (t_g * 1e-3) / 1e9, 1),
                             "split_kernel_GBps": round(kv_bytes / (t_k * 1e-3) / 1e9, 1),
                             "hbm_frac": round(kv_bytes / (t_f * 1e-3) / 1e9 / PEAK_HBM, 4)}
            dec[f"T{Tq}"]["attn_decode_us"] = round(t_ad * 1e3, 2)
            if want_cpu:
                if Tq == 1:
                    hrot = host_cache(rot[0], ctx)
                dec[f"T{Tq}"]["cpu"] = cpu_decode(hrot, qh[:Tq], gh[:Tq], ctx - Tq, Tq, kv_bytes, threads)
            print(f"[bench] config2 decode T={Tq} ctx={ctx} ns={ns}: {t_f * 1e3:.1f} us "
                  f"({dec[f'T{Tq}']['GBps']} GB/s; split kernel alone {t_k * 1e3:.1f} us; "
                  f"graph-replayed step {t_g * 1e3:.1f} us = {dec[f'T{Tq}']['graph_GBps']} GB/s"
                  f"; whole attn_decode step {t_ad * 1e3:.1f} us)", flush=True)
        del rot
        extra["config2_decode_int8_90k"] = dec
        # ---------------- config 1 depth comparison / config 4: turbo at 262k ----------------
        # three turbo caches of 262144 keys (3 x 125.8 MB > the 256 MB MALL) rotate, so every decode call streams
        # its KV from HBM, as the int8 caches above do; configs[4] uses the first
        ctx = 262144
        cts = []
        for i in range(1 if a.config4_only else 3):
            c = M.DeviceKVCache(KV, ctx + 64, 1)
            fill_cache(c, ctx, seed=12 + i)
            cts.append(c)
        ct = cts[0]
        ns = M.gqa_splits(1, KV, M.decode_splits(ctx), 1)
        part = torch.empty(H * ns * (AHD + 2), device=dev)
        o1 = torch.empty((1, H, AHD), device=dev)
        pd = torch.tensor([ctx - 1], dtype=torch.int32, device=dev)

        def tdec(c):  # what attn_decode runs: partials rotated back in the split kernel, gated combine
            def f():
                M.attn_gqa_out(qo[:1], c, H, KV, pd, c.max_t, part, 1, ns, st)
                M.attn_combine(part, qg[:1], o1, H, ns, LD, 1, st)
            return f

        t_td = time_rotating([tdec(c) for c in cts], 3 if a.config4_only else 90)
        tb = 2.0 * ctx * 240
        extra["config3_decode_turbo_262k"] = {"ns": ns, "us": round(t_td * 1e3, 2),
                                              "GBps": round(tb / (t_td * 1e-3) / 1e9, 1)}
        if not a.config4_only:
            # the whole attn_decode step from the raw q/k/v row: front (+ forward WHT, turbo append of row ctx - 1,
            # the same bytes each call), split kernel, gated combine
            LQ = LD + 2 * KV * AHD
            qkv_t = torch.randn((1, LQ), generator=torch.Generator(device=dev).manual_seed(8), device=dev)
            qn_t = torch.zeros(AHD, dtype=torch.int16, device=dev)
            qo_t = torch.empty((1, H, AHD), device=dev)
            nsd = M.decode_splits(ctx)
            part_t = torch.empty(H * nsd * (AHD + 2), device=dev)

            def tstep(c):
                return lambda: M.attn_decode(qkv_t, qkv_t[:, LD:], qkv_t[:, LD + KV * AHD:], qn_t, qn_t, qo_t, c, o1, H,
                                             KV, pd, c.max_t, 64, 1e7, 1e-6, 1, LQ, st, part_t, nsd)
            extra["config3_decode_turbo_262k"]["attn_decode_us"] = round(time_rotating([tstep(c) for c in cts], 90) * 1e3, 2)
        hct = None
        if want_cpu:
            hct = host_cache(ct, ctx)
            extra["config3_decode_turbo_262k"]["cpu"] = cpu_decode(hct, qh[:1], gh[:1], ctx - 1, 1, tb, threads)
        print(f"[bench] config3 turbo decode ctx={ctx}: {t_td * 1e3:.1f} us ({tb / t_td / 1e6:.0f} GB/s)"
              + (f"; whole attn_decode step {extra['config3_decode_turbo_262k']['attn_decode_us']} us"
                 if 'attn_decode_us' in extra['config3_decode_turbo_262k'] else ""), flush=True)
        if a.decode_only:
            print(json.dumps({"decode_only": True, **extra}), flush=True)
            return
        p4 = torch.tensor([260096], dtype=torch.int32, device=dev)

        def turbo_chunk():  # a complete turbo step: FA in the rotated domain, then the inverse WHT and the gate
            M.attn_fa(qo, None, ct, out, H, KV, p4, ct.max_t, LD, T, st)
            M.turbo_out(out, qg, H, LD, T, st)
        n4 = 3 if a.config4_only else 10
        ms_t, _ = time_steps(turbo_chunk, n4, 2)
        ms_i, _ = time_steps(lambda: M.attn_fa(qo, qg, c8, out, H, KV, p4, c8.max_t, LD, T, st), n4, 2)
        f4 = flops_prefill(T, 260096)
        extra["config4_prefill_260k"] = {"turbo_ms": round(ms_t, 3), "turbo_tflops": round(f4 / ms_t / 1e9, 1),
                                         "int8_ms": round(ms_i, 3), "int8_tflops": round(f4 / ms_i / 1e9, 1),
                                         "steps": n4, "turbo_step": "attn_fa + turbo_out"}
        if want_cpu:
            extra["config4_prefill_260k"]["cpu_turbo"] = cpu_prefill(hct, qh, gh, 260096, T,
                                                                     threads, full=False)
        print(f"[bench] config4 prefill at 260096: turbo {ms_t:.2f} ms ({f4 / ms_t / 1e9:.0f} TFLOPS), "
              f"int8 {ms_i:.2f} ms ({f4 / ms_i / 1e9:.0f} TFLOPS)", flush=True)
        del ct, cts
        if a.config4_only:
            return
        # ---------------- dense int8 projections either side of the attention ----------------
        dense = {}
        for nm, O_, I_ in (("qkv", H * 2 * AHD + 2 * KV * AHD, 2048), ("o_proj", 2048, H * AHD)):
            nrot = int(600e6 // (O_ * I_)) + 1  # > the 256 MB MALL: every call streams its weights from HBM
            ws = []
            g = torch.Generator(device=dev).manual_seed(30)
            for _ in range(nrot):
                w16 = (torch.randn((O_, I_), generator=g, device=dev) * 0.02).half()
                qw = torch.empty((O_, I_), dtype=torch.int8, device=dev)
                sw = torch.empty(O_, device=dev)
                M.quantize_rows_i8(w16, qw, sw, O_, I_, st)
                ws.append((qw, sw))
            del w16
            ent = {"O": O_, "I": I_}
            for S_ in (1, 2):
                Xd = torch.randn((S_, I_), generator=g, device=dev)
                Yd = torch.empty((S_, O_), device=dev)
                t_g = time_rotating([lambda qw=qw, sw=sw: M.gemm_i8(qw, sw, Xd, Yd, S_, I_, O_, st) for qw, sw in ws], 200)
                ent[f"gemv_{S_}row_us"] = round(t_g * 1e3, 2)
                ent[f"gemv_{S_}row_GBps"] = round(O_ * I_ / (t_g * 1e-3) / 1e9, 1)
                t_r = time_graph([lambda s_, qw=qw, sw=sw: M.gemm_i8(qw, sw, Xd, Yd, S_, I_, O_, s_) for qw, sw in ws])
                ent[f"gemv_{S_}row_graph_us"] = round(t_r * 1e3, 2)
            Xd = torch.randn((T, I_), generator=g, device=dev)
            Yd = torch.empty((T, O_), device=dev)
            ms_g, _ = time_steps(lambda: M.gemm_i8(ws[0][0], ws[0][1], Xd, Yd, T, I_, O_, st), 10, 3)
            ent["gemm_2048_ms"] = round(ms_g, 4)
            ent["gemm_2048_tflops"] = round(2.0 * T * I_ * O_ / (ms_g * 1e-3) / 1e12, 1)
            dense[nm] = ent
            print(f"[bench] dense {nm} int8 [{O_}x{I_}]: GEMV 1 row {ent['gemv_1row_us']} us "
                  f"({ent['gemv_1row_GBps']} GB/s), 2 rows {ent['gemv_2row_us']} us; prefill GEMM S={T} "
                  f"{ms_g:.3f} ms ({ent['gemm_2048_tflops']} TFLOPS)", flush=True)
            # the other forms of struct Mat (kernels.cuh:186-196) on the same shape: the one-row GEMV through moex_gemv
            for fm, bpw in (("int4", 0.5), ("int6", 0.75), ("f16", 2.0)):
                nrot_f = int(600e6 // (O_ * I_ * bpw)) + 1
                mats = []
                for k in range(nrot_f):
                    w16 = (torch.randn((O_, I_), generator=g, device=dev) * 0.02).half()
                    if fm == "f16":
                        mats.append((M.Mat(f16=w16), w16))
                        continue
                    q4 = torch.empty((O_, I_ // 2), dtype=torch.uint8, device=dev)
                    s4 = torch.empty((O_, I_ // 64), dtype=torch.float32, device=dev)
                    if fm == "int4":
                        M.quantize_rows_q4(w16, q4, s4, O_, I_, st)
                        mats.append((M.Mat(q4=q4, s=s4), q4, s4))
                    else:
                        q6h = torch.empty((O_, I_ // 4), dtype=torch.uint8, device=dev)
                        M.quantize_rows_q6(w16, q4, q6h, s4, O_, I_, st)
                        mats.append((M.Mat(q6=q4, q6h=q6h, s=s4), q4, q6h, s4))
                xd1 = torch.randn((1, I_), generator=g, device=dev)
                yd1 = torch.empty((1, O_), device=dev)
                # graph-replayed: back-to-back Python calls through the Mat wrapper take longer on the host (~6.7 µs)
                # than these kernels on the GPU
                t_f = time_graph([lambda s_, m=m: M.gemv(m[0], xd1, yd1, I_, O_, s_) for m in mats])
                ent[f"gemv_{fm}_1row_graph_us"] = round(t_f * 1e3, 2)
                ent[f"gemv_{fm}_1row_graph_GBps"] = round(O_ * I_ * bpw / (t_f * 1e-3) / 1e9, 1)
                del mats
            print(f"[bench] dense {nm} GEMV 1 row graph-replayed: int8 {ent['gemv_1row_graph_us']} us, int4 "
                  f"{ent['gemv_int4_1row_graph_us']} us, int6 {ent['gemv_int6_1row_graph_us']} us, fp16 "
                  f"{ent['gemv_f16_1row_graph_us']} us ({ent['gemv_f16_1row_graph_GBps']} GB/s)", flush=True)
            del ws
        extra["dense_int8_projections"] = dense

    cpu = None
    if want_cpu:
        cpu = cpu_prefill(hc8, qh, gh, pos0, T, threads, full=False)
        cpu["sample"] += f"; nproc={os.cpu_count()}"
        print(f"[bench] cpu fp64 baseline: {cpu['value']:.4f} {cpu['unit']} on {cpu['cores']} threads "
              f"({cpu['sample']})", flush=True)

    line = {
        "metric": METRIC, "value": round(tflops, 2), "unit": "TFLOPS", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16", "data": "synthetic (seeded N(0,1) Q/gate/K/V; K/V int8-quantized by the "
                                                   "product's append kernel)",
        "config": {"workload": "configs[1]: int8-KV causal GQA FA-2 prefill chunk, T=2048 at pos0=32768 (34816 "
                               "keys), H=16, KV=2, head_dim=256, sigmoid-gated", "global_batch": 1, "seq_len": n,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_F16, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_F16, 4), "traffic": traffic, "traffic_source": traffic_src},
        "cpu_baseline": cpu,
        "wall_ms_per_step": round(wall_ms, 4),
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


def cpu_threads():
    """Host threads for the CPU baseline: every core this process may run on, but no more than the job's CPU share
    when the environment states one (OMP_NUM_THREADS; 16 on a one-GPU box)."""
    n = len(os.sched_getaffinity(0))
    share = os.environ.get("OMP_NUM_THREADS")
    if share and share.isdigit() and int(share) > 0:
        n = min(n, int(share))
    return max(1, n)


def host_cache(dc, n):
    """Host copy of the first n positions of a device cache, for the oracle."""
    from oracle import oracle as orc
    hc = orc.HostCache(KV, n, dc.turbo)
    hc.k[:] = dc.k[:, :n].cpu().numpy().view(hc.k.dtype)
    hc.v[:] = dc.v[:, :n].cpu().numpy().view(hc.v.dtype)
    hc.ks[:] = dc.ks[:, :n].cpu().numpy()
    hc.vs[:] = dc.vs[:, :n].cpu().numpy()
    return hc


def cpu_rows(hc, q, g, pos0, rows, threads, min_s=1.5):
    """The fp64 reference attention (tests/test_fa.cu:59-80 semantics, oracle/moex_oracle.c; turbo: dequantized codes
    and the inverse rotation) over (token, head) rows, threaded; returns (seconds, flops by the reference's per-row
    count 4 * D * keys); seconds is per pass over the rows."""
    import concurrent.futures as cf
    from oracle import oracle as orc
    rows = list(rows)
    nch = min(len(rows), 4 * threads)
    chunks = [rows[i::nch] for i in range(nch)]
    reps = 0
    t0 = time.perf_counter()
    with cf.ThreadPoolExecutor(threads) as ex:
        while reps == 0 or time.perf_counter() - t0 < min_s:  # short samples repeat: ~min_s of wall time at least
            list(ex.map(lambda c: orc.attn_rows_f64(q, g, LD, H, hc, pos0, c), chunks))
            reps += 1
    el = (time.perf_counter() - t0) / reps
    return el, sum(4.0 * AHD * (pos0 + t + 1) for t, _ in rows)


def sample_rows(T):
    """tests/test_fa.cu:95: tokens {0, T/3, T/2, T-2, T-1} x all heads."""
    return [(t, h) for t in sorted({0, T // 3, T // 2, T - 2, T - 1}) for h in range(H)]


def cpu_prefill(hc, q, g, pos0, T, threads, full):
    rows = [(t, h) for t in range(T) for h in range(H)] if full else sample_rows(T)
    el, fl = cpu_rows(hc, q, g, pos0, rows, threads)
    rate = fl / el
    d = {"value": round(rate / 1e12, 6), "unit": "TFLOPS", "cores": threads, "kind": "port",
         "seconds": round(el, 3)}
    if full:
        d["sample"] = f"all {T * H} (token, head) rows, fp64"
    else:
        d["sample"] = (f"the test_fa.cu:95 row sample ({len(rows)} rows of {T * H}), fp64, {el:.2f} s; "
                       f"full chunk extrapolated linearly in flops: {flops_prefill(T, pos0) / rate:.1f} s")
        d["extrapolated_full_s"] = round(flops_prefill(T, pos0) / rate, 2)
    return d


def cpu_decode(hc, q, g, pos, Tq, kv_bytes, threads):
    el, _ = cpu_rows(hc, q, g, pos, [(t, h) for t in range(Tq) for h in range(H)], threads)
    return {"value": round(kv_bytes / el / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "seconds": round(el, 3), "sample": f"all {Tq * H} (token, head) rows over {pos + Tq} keys, fp64"}


if __name__ == "__main__":
    main()
