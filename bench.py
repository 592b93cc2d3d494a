#!/usr/bin/env python3
"""Headline benchmark of libtrhip on one MI355X.

Workload (the Q4_K decode GEMV the metric is quoted on): weight 14336 x 4096 Q4_K (Llama-3-8B gate/up
shape), entries N(0, 0.02) with a seeded 1% scaled x10, encoded by tcb_amd.synth; x fp32 N(0, 1); batch 1;
c = x . deq(W)^T (GemmSet). One step is one GEMV. The weights sit in a ring of copies larger than the
256 MB MALL (>= 1.1 GiB), so each step streams its weight from HBM ("cold"); a warm figure (same copy
every step) is reported beside it. The steps are captured once into a HIP graph and replayed, so host
launch overhead does not enter the device timing; HIP events on the library's stream bracket the
replays.

Also reported: the act-quant prefill GEMM (Q4_K 14336 x 4096, M = 512 rows quantized to Q8 on the
device, int32 block sums, fp32 epilogue) in int8 TOPS = 2*M*N*K / time, and the CPU baseline: the AVX2
restatement of the reference's sdotq4k path (oracle/trq_avx2.c), all host cores, on the same bytes.

Prints one JSON line. --gpus N > 1 exits: the measurement covers one GPU.

--profile-kernel {gemv,prefill,rows,copy,read,open_q,sweep,mfma} runs only that work, eagerly, --steps times (for
rocprofv3 runs): gemv = the headline GEMV over the cold ring, prefill = one act-quant GEMM per step, rows = one M > 1
fp32 GEMM (--rows-m rows, --rows-shape dtype,N,K, --mode exact or fast) per step, copy = a plain device copy of
COPY_BYTES (torch) that calibrates the FETCH_SIZE / WRITE_SIZE counters, read = the streaming-read probe over a cold
ring of the headline's bytes, open_q = OpenQuant of the headline store, sweep = the 32-layer decode sweep (--rows-m
batch, --mode) launched eagerly, mfma = the int8 matrix-core probe without and with VALU beside it.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4_K GEMV µs + HBM GB/s (% peak) at 8B shapes; prefill GEMM int8 TOPS"
HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, datasheet
Q4K_CODE = 3
INT8_PEAK_TOPS = 5033.0      # MI355X dense int8 MFMA, datasheet (5.03 POPS)
N, K = 14336, 4096
RING_BYTES = int(1.1 * (1 << 30))
MIN_WARMUP = 1000  # untimed launches of the headline before its timed ones
COPY_BYTES = 256 << 20

# HBM bytes per launch of the headline kernel from rocprofv3 FETCH_SIZE + WRITE_SIZE over --profile-kernel gemv,
# each divided by the same counter's reading per byte of the calibration copy (profiles/gemv_q4_k_14336x4096_*.txt).
# Keyed by mode.
TRAFFIC = {"fast": 33733342, "exact": 33369237}
# Same counters over --profile-kernel prefill --mode fast (profiles/prefill_q4_k_14336x4096_M512.txt): quantizer +
# MFMA kernel.
PREFILL_TRAFFIC = {"quantize_q8": 13295334, "prefill_q4k": 81923421}


def algorithmic_bytes(n, k):
    # weights (144 B per 256-element block) + x (4K) + c written (4N)
    return n * (k // 256) * 144 + 4 * k + 4 * n


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400, help="timed GEMVs (rounded up to whole ring passes)")
    ap.add_argument("--warmup", type=int, default=4000,
                    help="untimed launches before the timed ones (at least %d: with fewer the device is not yet at its "
                         "steady clock; 72 warm-up launches measured 9.34 us per GEMV, 1008 8.48, 4032 8.28)" % MIN_WARMUP)
    ap.add_argument("--mode", choices=["exact", "fast"], default="fast",
                    help="headline mode; the other mode is measured and reported beside it")
    ap.add_argument("--prefill-m", type=int, default=512)
    ap.add_argument("--prefill-dtype", choices=["q4_k", "q6_k", "q4_0"], default="q4_k",
                    help="weights of --profile-kernel prefill (q6_k and q4_0 take random-code blocks of the same shape)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="bounded CPU-baseline sample (0 = skip)")
    ap.add_argument("--sweep", type=int, default=1, help="also time the 32-layer decode sweep (0 = skip)")
    ap.add_argument("--shapes", type=int, default=1,
                    help="also time every Llama-3-8B GEMV shape per dtype and the prefill grid (0 = skip)")
    ap.add_argument("--profile-kernel", choices=["gemv", "prefill", "rows", "copy", "read", "open_q", "sweep", "mfma"],
                    default=None,
                    help="run only this kernel --steps times, eagerly (counter runs)")
    ap.add_argument("--rows-m", type=int, default=16, help="activation rows of --profile-kernel rows (M > 1 path)")
    ap.add_argument("--merged", type=int, default=0,
                    help="--profile-kernel sweep: 1 = the merged layers ([q | k | v], [gate | up] + SwiGLU) of the bench")
    ap.add_argument("--rows-shape", default="q4_k,14336,4096",
                    help="dtype,N,K of --profile-kernel rows (q4_k or q6_k; e.g. q6_k,128256,4096 for the output head)")
    return ap.parse_args()


LAYER = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
         ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
N_LAYERS, VOCAB, HIDDEN = 32, 128256, 4096


def decode_sweep(tb, batches, mode, replays=5):
    """One token step of a 32-layer Llama-3-8B-shaped model: every linear as a quantized GEMV (q4_k), back to
    back, then the q6_k output head. Each layer owns its own device copy of the weights (4.36 GB in HBM), filled
    with random-code blocks (synth.random_blocks): throughput does not depend on the values. Batch b > 1 runs
    the M = b fp32 path. Timed as a captured graph replayed `replays` times."""
    from tcb_amd import Q4K, Q6K, _lib, synth
    L = _lib.lib()
    ctx = tb.ctx
    host = {name: synth.random_blocks(Q4K, n, k, seed=10 + i) for i, (name, n, k) in enumerate(LAYER)}
    stores = [[tb.FromQuantized(Q4K, host[name], n, k) for name, n, k in LAYER] for _ in range(N_LAYERS)]
    head = tb.FromQuantized(Q6K, synth.random_blocks(Q6K, VOCAB, HIDDEN, seed=99), VOCAB, HIDDEN)
    del host
    wbytes = sum(w.device_bytes() for layer in stores for w in layer) + head.device_bytes()
    res = {}
    for b in batches:
        xs = {4096: ctx.to_device(synth.activations(b, 4096, seed=7)), 14336: ctx.to_device(synth.activations(b, 14336, seed=8))}
        cb = ctx.alloc(b * VOCAB * 4)

        def step():
            for layer in stores:
                for (name, n, k), w in zip(LAYER, layer):
                    tb.GemmSet(b, n, k, xs[k], w, cb, mode=mode)
            tb.GemmSet(b, VOCAB, HIDDEN, xs[4096], head, cb, mode=mode)

        step()  # sizes the workspace
        ctx.sync()
        g = capture(tb, step)
        time_graph(tb, g, 1)
        ms = time_graph(tb, g, replays) / replays
        L.trhip_graph_destroy(g)
        res["batch%d" % b] = {"ms_per_token_step": round(ms, 4), "tokens_per_s": round(b / (ms * 1e-3), 1),
                              "weight_GB/s": round(wbytes / (ms * 1e-3) / 1e9, 1),
                              "hbm_frac_of_peak": round(wbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        for v in xs.values():
            v.free()
        cb.free()
    # merged layers (the reference's merged projections, lib/layers.tr:240-262): [q | k | v] and [gate | up] as one
    # store each, the gate/up product followed by the SwiGLU gate (trhip_gemm_q_swiglu)
    by = {name: i for i, (name, _, _) in enumerate(LAYER)}
    merged = []
    for layer in stores:
        qkv = layer[0].Concat([layer[by["q"]], layer[by["k"]], layer[by["v"]]])
        gu = layer[0].Concat([layer[by["gate"]], layer[by["up"]]])
        merged.append((qkv, layer[by["o"]], gu, layer[by["down"]]))
        for name in ("q", "k", "v", "gate", "up"):
            layer[by[name]].release()
    ctx.sync()
    res["merged"] = {}
    for b in batches:
        xs = {4096: ctx.to_device(synth.activations(b, 4096, seed=7)), 14336: ctx.to_device(synth.activations(b, 14336, seed=8))}
        cb = ctx.alloc(b * VOCAB * 4)

        def mstep():
            for qkv, o, gu, down in merged:
                tb.GemmSet(b, qkv.N, 4096, xs[4096], qkv, cb, mode=mode)
                tb.GemmSet(b, 4096, 4096, xs[4096], o, cb, mode=mode)
                tb.GemmSwiGLU(b, 4096, xs[4096], gu, cb, mode=mode)
                tb.GemmSet(b, 4096, 14336, xs[14336], down, cb, mode=mode)
            tb.GemmSet(b, VOCAB, HIDDEN, xs[4096], head, cb, mode=mode)

        mstep()
        ctx.sync()
        g = capture(tb, mstep)
        time_graph(tb, g, 1)
        ms = time_graph(tb, g, replays) / replays
        L.trhip_graph_destroy(g)
        res["merged"]["batch%d" % b] = {"ms_per_token_step": round(ms, 4), "tokens_per_s": round(b / (ms * 1e-3), 1),
                                        "weight_GB/s": round(wbytes / (ms * 1e-3) / 1e9, 1),
                                        "hbm_frac_of_peak": round(wbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        for v in xs.values():
            v.free()
        cb.free()
    res["merged"]["workload"] = ("same weights as merged layers: per layer [q | k | v] 6144x4096, o, [gate | up] 28672x4096 "
                                 "followed by the SwiGLU gate, down; 4 weight launches + 1 SwiGLU launch per layer")
    for m in merged:
        for w in m:
            w.release()
    head.release()
    res.update({"workload": "32 layers x (q, k, v, o, gate, up, down) q4_k + q6_k head 128256x4096, %d GEMV launches "
                            "per token step, weights %d B" % (7 * N_LAYERS + 1, wbytes),
                "mode": "fast" if mode else "exact", "weight_bytes": wbytes})
    return res


def shape_table(tb):
    """Cold-ring GEMV time for every Llama-3-8B linear shape and dtype (exact and fast), the M > 1 path at batch
    8 (q4_0) and 16 (q4_k, q6_k head), OpenQuant and the quantized embedding lookup, and the prefill grid
    M in {128, 512, 2048} x both FFN shapes. Random-code blocks (synth.random_blocks): timing only."""
    from tcb_amd import MODE_EXACT, MODE_FAST, Q4, Q4K, Q6K, Q8, _lib, synth
    L = _lib.lib()
    ctx = tb.ctx
    gemv = {}
    cases = [(Q8, 4096, 4096), (Q4, 14336, 4096), (Q4, 4096, 14336)] + \
            [(dt, n, k) for dt in (Q4K, Q6K) for n, k in ((4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336))]
    names = {Q8: "q8_0", Q4: "q4_0", Q4K: "q4_k", Q6K: "q6_k"}
    for dt, n, k in cases:
        raw = synth.random_blocks(dt, n, k, seed=5)
        ring = [tb.FromQuantized(dt, raw, n, k) for _ in range(max(2, -(-RING_BYTES // raw.nbytes)))]
        xb = ctx.to_device(synth.activations(1, k, seed=6))
        cb = ctx.alloc(n * 4)
        res = {}
        for md in (MODE_EXACT, MODE_FAST):
            tb.GemmSet(1, n, k, xb, ring[0], cb, mode=md)
            ctx.sync()
            g = capture(tb, lambda: [tb.GemmSet(1, n, k, xb, w, cb, mode=md) for w in ring])
            time_graph(tb, g, 1)
            us = time_graph(tb, g, 3) * 1e3 / (3 * len(ring))
            L.trhip_graph_destroy(g)
            res["fast" if md else "exact"] = {"us": round(us, 2), "GB/s": round(raw.nbytes / us / 1e3, 1)}
        gemv["%s %dx%d" % (names[dt], n, k)] = res
        for w in ring:
            w.release()
        xb.free()
        cb.free()
    # the M > 1 fp32 path (batched decode): q4_0 FFN shapes at batch 8, q4_k at batch 16, the q6_k output head at
    # batch 16. Like the headline: one call per weight copy over a cold ring of copies (at least 1.1 GiB), all in one
    # captured graph, time per call (a graph of a single call would mostly time the graph launch itself)
    rows = {"workload": "one call per weight copy over a cold ring of >= 1.1 GiB of copies in one graph; us per call"}
    for dt, n, k, m in ((Q4, 14336, 4096, 8), (Q4, 4096, 14336, 8), (Q4K, 14336, 4096, 16), (Q4K, 4096, 14336, 16),
                        (Q6K, 128256, 4096, 16)):
        raw = synth.random_blocks(dt, n, k, seed=12)
        ring = [tb.FromQuantized(dt, raw, n, k) for _ in range(max(2, -(-RING_BYTES // raw.nbytes)))]
        del raw
        Xb = ctx.to_device(synth.activations(m, k, seed=13))
        Cb = ctx.alloc(m * n * 4)
        res = {}
        for md in (MODE_EXACT, MODE_FAST):
            tb.GemmSet(m, n, k, Xb, ring[0], Cb, mode=md)
            ctx.sync()
            g = capture(tb, lambda: [tb.GemmSet(m, n, k, Xb, w, Cb, mode=md) for w in ring])
            time_graph(tb, g, 1)
            us = time_graph(tb, g, 3) * 1e3 / (3 * len(ring))
            L.trhip_graph_destroy(g)
            res["fast" if md else "exact"] = {"us": round(us, 1), "GB/s": round(ring[0].device_bytes() / us / 1e3, 1)}
        rows["%s %dx%d M=%d" % (names[dt], n, k, m)] = res
        Xb.free()
        Cb.free()
        for w in ring:
            w.release()
    # OpenQuant (dequantize a whole store to fp32) and the quantized embedding lookup: HBM-bound, bytes = blocks read
    # + fp32 written
    other = {}
    for dt, n, k in ((Q4K, 14336, 4096), (Q6K, 14336, 4096), (Q8, 4096, 4096)):
        w = tb.FromQuantized(dt, synth.random_blocks(dt, n, k, seed=9), n, k)
        ob = ctx.alloc(n * k * 4)
        tb.OpenQuant(ob, w)
        ctx.sync()
        g = capture(tb, lambda: tb.OpenQuant(ob, w))
        time_graph(tb, g, 2)
        us = time_graph(tb, g, 5) * 1e3 / 5
        L.trhip_graph_destroy(g)
        moved = w.device_bytes() + n * k * 4
        other["open_q %s %dx%d" % (names[dt], n, k)] = {"us": round(us, 1), "GB/s": round(moved / us / 1e3, 1)}
        ob.free()
        w.release()
    emb = tb.FromQuantized(Q6K, synth.random_blocks(Q6K, 128256, 4096, seed=11), 128256, 4096)
    for ntok in (1, 16, 512):
        ob = ctx.alloc(ntok * 4096 * 4)
        idx = np.random.default_rng(ntok).integers(0, 128256, ntok)
        tb.Embedding(ob, emb, idx)
        ctx.sync()
        e0, e1 = ctx.event(), ctx.event()
        ctx.record(e0)
        for _ in range(20):
            tb.Embedding(ob, emb, idx)
        ctx.record(e1)
        ctx.sync()
        us = ctx.elapsed_ms(e0, e1) * 1e3 / 20
        other["embedding q6_k 128256x4096, %d tokens" % ntok] = {"us": round(us, 2)}
        ob.free()
    emb.release()
    prefill = {}
    cases = [(Q4K, 14336, 4096, M) for M in (128, 512, 2048)] + [(Q4K, 4096, 14336, M) for M in (128, 512, 2048)] + \
            [(Q6K, 14336, 4096, 512), (Q4, 14336, 4096, 512)]
    for dt, n, k, M in cases:
        w = tb.FromQuantized(dt, synth.random_blocks(dt, n, k, seed=7), n, k)
        Xb = ctx.to_device(synth.activations(M, k, seed=8))
        Cb = ctx.alloc(M * n * 4)
        res = {}
        for md in ((MODE_FAST, MODE_EXACT) if dt == Q4K else (MODE_EXACT,)):
            tb.GemmActQuant(M, n, k, Xb, w, Cb, accumulate=False, mode=md)
            ctx.sync()
            g = capture(tb, lambda: tb.GemmActQuant(M, n, k, Xb, w, Cb, accumulate=False, mode=md))
            time_graph(tb, g, 2)
            ms = time_graph(tb, g, 5) / 5
            L.trhip_graph_destroy(g)
            tops = 2.0 * M * n * k / (ms * 1e-3) / 1e12
            res["fast" if md else "exact"] = {"us": round(ms * 1e3, 1), "int8_tops": round(tops, 1),
                                              "frac_of_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
        prefill["%s %dx%d M=%d" % (names[dt], n, k, M)] = res
        Xb.free()
        Cb.free()
        w.release()
    return {"gemv_cold_ring": gemv, "rows": rows, "prefill": prefill, "open_q_and_embedding": other}


def profile_kernel(a):
    """One kernel, --steps eager launches, nothing else timed or printed but one JSON line."""
    import numpy as np
    from tcb_amd import MODE_EXACT, MODE_FAST, Q4K, QuantBackend, synth
    if a.profile_kernel == "copy":
        import torch
        src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(a.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"profiled": "copy", "launches": a.steps, "bytes_read": COPY_BYTES, "bytes_written": COPY_BYTES}))
        return 0
    tb = QuantBackend(0)
    if a.profile_kernel == "mfma":
        # int8 TOPS (events) for VALU per MFMA 0..16 at one and two waves per SIMD: how much VALU work hides under
        # the matrix cores, the ceiling of the act-quant prefill kernels
        curve = {}
        for w in (1, 2):
            for v in (0, 2, 4, 6, 8, 12, 16):
                curve["%d waves/SIMD, %d VALU/MFMA" % (w, v)] = round(mfma_rate(tb, v, w, iters=20000), 1)
        print(json.dumps({"profiled": "mfma_probe", "int8_tops": curve, "peak_tops": INT8_PEAK_TOPS}))
        tb.close()
        return 0
    if a.profile_kernel == "sweep":
        # every linear of the 32-layer sweep and the head, launched eagerly (no graph), --steps token steps
        from tcb_amd import Q6K
        b = a.rows_m
        mode = MODE_FAST if a.mode == "fast" else MODE_EXACT
        host = {name: synth.random_blocks(Q4K, n, k, seed=10 + i) for i, (name, n, k) in enumerate(LAYER)}
        stores = [[tb.FromQuantized(Q4K, host[name], n, k) for name, n, k in LAYER] for _ in range(N_LAYERS)]
        head = tb.FromQuantized(Q6K, synth.random_blocks(Q6K, VOCAB, HIDDEN, seed=99), VOCAB, HIDDEN)
        xs = {4096: tb.ctx.to_device(synth.activations(b, 4096, seed=7)),
              14336: tb.ctx.to_device(synth.activations(b, 14336, seed=8))}
        cb = tb.ctx.alloc(b * VOCAB * 4)
        by = {name: i for i, (name, _, _) in enumerate(LAYER)}
        if a.merged:  # the bench's merged layers: [q | k | v], o, [gate | up] with the SwiGLU gate, down
            merged = [(layer[0].Concat([layer[by["q"]], layer[by["k"]], layer[by["v"]]]), layer[by["o"]],
                       layer[0].Concat([layer[by["gate"]], layer[by["up"]]]), layer[by["down"]]) for layer in stores]
        for _ in range(a.steps):
            if a.merged:
                for qkv, o, gu, down in merged:
                    tb.GemmSet(b, qkv.N, 4096, xs[4096], qkv, cb, mode=mode)
                    tb.GemmSet(b, 4096, 4096, xs[4096], o, cb, mode=mode)
                    tb.GemmSwiGLU(b, 4096, xs[4096], gu, cb, mode=mode)
                    tb.GemmSet(b, 4096, 14336, xs[14336], down, cb, mode=mode)
            else:
                for layer in stores:
                    for (name, n, k), w in zip(LAYER, layer):
                        tb.GemmSet(b, n, k, xs[k], w, cb, mode=mode)
            tb.GemmSet(b, VOCAB, HIDDEN, xs[4096], head, cb, mode=mode)
        tb.ctx.sync()
        print(json.dumps({"profiled": "decode_sweep_eager", "batch": b, "mode": a.mode, "token_steps": a.steps,
                          "merged": bool(a.merged)}))
        tb.close()
        return 0
    raw = synth.quant_weights(Q4K, N, K, seed=3, outliers=0.01)
    if a.profile_kernel == "gemv":
        ring = [tb.FromQuantized(Q4K, raw, N, K) for _ in range(max(2, -(-RING_BYTES // raw.nbytes)))]
        xb = tb.ctx.to_device(synth.activations(1, K, seed=4))
        cb = tb.ctx.alloc(N * 4)
        mode = MODE_FAST if a.mode == "fast" else MODE_EXACT
        for i in range(a.steps):
            tb.GemmSet(1, N, K, xb, ring[i % len(ring)], cb, mode=mode)
        tb.ctx.sync()
        print(json.dumps({"profiled": "gemv_q4_k_%s" % a.mode, "launches": a.steps,
                          "algorithmic_bytes": algorithmic_bytes(N, K)}))
    elif a.profile_kernel == "rows":
        # the M > 1 fp32 path (batched decode): exact chunk order, or the fast matrix-core kernels with --mode fast
        from tcb_amd import Q6K
        M = a.rows_m
        name, rn, rk = a.rows_shape.split(",")
        rdt, rn, rk = {"q4_k": Q4K, "q6_k": Q6K}[name], int(rn), int(rk)
        # other shapes take random-code blocks (timing only; the head's 431 MB would take minutes to encode)
        rraw = raw if (rdt, rn, rk) == (Q4K, N, K) else synth.random_blocks(rdt, rn, rk, seed=3)
        w = tb.FromQuantized(rdt, rraw, rn, rk)
        Xb = tb.ctx.to_device(synth.activations(M, rk, seed=5))
        Cb = tb.ctx.alloc(M * rn * 4)
        mode = MODE_FAST if a.mode == "fast" else MODE_EXACT
        for _ in range(a.steps):
            tb.GemmSet(M, rn, rk, Xb, w, Cb, mode=mode)
        tb.ctx.sync()
        print(json.dumps({"profiled": "rows_%s_%dx%d_%s" % (name, rn, rk, a.mode), "launches": a.steps, "M": M,
                          "weight_bytes": int(rraw.nbytes)}))
    elif a.profile_kernel == "read":
        # the streaming-read ceiling: trhip_read_probe over a cold ring of plain buffers of the headline's bytes
        nbytes = raw.nbytes // 16 * 16
        ring = [tb.ctx.alloc(nbytes) for _ in range(max(2, -(-RING_BYTES // nbytes)))]
        for b in ring:
            b.fill(1)
        for i in range(a.steps):
            tb.ctx.read_probe(ring[i % len(ring)], nbytes)
        tb.ctx.sync()
        print(json.dumps({"profiled": "read_probe", "launches": a.steps, "bytes": nbytes}))
    elif a.profile_kernel == "open_q":
        # OpenQuant: the whole headline store dequantized to fp32
        w = tb.FromQuantized(Q4K, raw, N, K)
        ob = tb.ctx.alloc(N * K * 4)
        for _ in range(a.steps):
            tb.OpenQuant(ob, w)
        tb.ctx.sync()
        print(json.dumps({"profiled": "open_q_q4_k", "launches": a.steps,
                          "bytes": int(raw.nbytes) + N * K * 4}))
    else:
        from tcb_amd import Q4, Q6K
        M = a.prefill_m
        pdt = {"q4_k": Q4K, "q6_k": Q6K, "q4_0": Q4}[a.prefill_dtype]
        w = tb.FromQuantized(pdt, raw if pdt == Q4K else synth.random_blocks(pdt, N, K, seed=3), N, K)
        Xb = tb.ctx.to_device(synth.activations(M, K, seed=5))
        Cb = tb.ctx.alloc(M * N * 4)
        mode = MODE_FAST if a.mode == "fast" else MODE_EXACT
        for _ in range(a.steps):
            tb.GemmActQuant(M, N, K, Xb, w, Cb, accumulate=False, mode=mode)
        tb.ctx.sync()
        print(json.dumps({"profiled": "prefill_%s_M%d_%s" % (a.prefill_dtype, M, a.mode), "launches": a.steps,
                          "ops": 2 * M * N * K}))
    tb.close()
    return 0


def mfma_rate(tb, valu_per_mfma, waves_per_simd, iters=40000):
    """int8 TOPS of trhip_mfma_probe: four independent v_mfma_i32_32x32x32_i8 chains per wave with valu_per_mfma
    independent fp32 FMAs beside each MFMA, one workgroup per CU."""
    from tcb_amd import _lib
    L = _lib.lib()
    ctx = tb.ctx
    L.trhip_mfma_probe(ctx.h, valu_per_mfma, waves_per_simd, 100)
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    rc = L.trhip_mfma_probe(ctx.h, valu_per_mfma, waves_per_simd, iters)
    ctx.record(e1)
    if rc:
        raise RuntimeError("mfma probe failed: %d" % rc)
    ms = ctx.elapsed_ms(e0, e1)
    cus = 256
    return 4.0 * waves_per_simd * cus * iters * 4 * 65536 / (ms * 1e-3) / 1e12


def prefill_loop_us(tb, kind, M, N, K, reps=20):
    """Microseconds per launch of trhip_prefill_probe (the prefill kernel's inner loop alone on its real grid: kind 0
    q4_k exact, 1 q4_k fast, 2 q6_k), median of reps event-timed launches after two warm-up launches."""
    from tcb_amd import _lib
    L = _lib.lib()
    ctx = tb.ctx
    for _ in range(2):
        if L.trhip_prefill_probe(ctx.h, kind, M, N, K):
            raise RuntimeError("prefill probe failed")
    ctx.sync()
    ts = []
    for _ in range(reps):
        e0, e1 = ctx.event(), ctx.event()
        ctx.record(e0)
        L.trhip_prefill_probe(ctx.h, kind, M, N, K)
        ctx.record(e1)
        ctx.sync()
        ts.append(ctx.elapsed_ms(e0, e1) * 1e3)
    ts.sort()
    return ts[len(ts) // 2]


def upload_rates(tb, raw):
    """Store creation (upload + repack) of the headline weights: GB/s of GGUF bytes from pageable host memory and
    from a trhip_host_alloc (pinned) block, median of 5."""
    import numpy as np
    ctx = tb.ctx
    out = {}
    pinned, p = ctx.host_alloc(raw.nbytes)
    pinned[:] = raw
    for name, src in (("pageable", raw), ("pinned", pinned)):
        ts = []
        for _ in range(5):
            t0 = time.perf_counter()
            w = tb.FromQuantized(Q4K_CODE, src, N, K)  # returns after the upload and repack completed (sync)
            ts.append(time.perf_counter() - t0)
            w.release()
        t = sorted(ts)[len(ts) // 2]
        out[name] = {"ms": round(t * 1e3, 2), "GB/s": round(raw.nbytes / t / 1e9, 2)}
    ctx.host_free(p)
    out["workload"] = "trhip_wstore_create of q4_k %dx%d (%d B), host to device through the upload ring + repack" % (
        N, K, raw.nbytes)
    return out


def time_graph(tb, graph, replays):
    from tcb_amd import _lib
    L = _lib.lib()
    ctx = tb.ctx
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    for _ in range(replays):
        rc = L.trhip_graph_launch(ctx.h, graph)
        if rc:
            raise RuntimeError("graph launch failed: %d" % rc)
    ctx.record(e1)
    ms = ctx.elapsed_ms(e0, e1)
    for e in (e0, e1):
        L.trhip_event_destroy(e)
    return ms


def capture(tb, body):
    import ctypes
    from tcb_amd import _lib
    L = _lib.lib()
    if L.trhip_graph_begin(tb.ctx.h):
        raise RuntimeError("graph begin failed")
    try:
        body()
    finally:
        g = _lib.P()
        rc = L.trhip_graph_end(tb.ctx.h, ctypes.byref(g))
    if rc:
        raise RuntimeError("graph end failed: %s" % L.trhip_last_error(tb.ctx.h))
    return g


def main():
    a = parse()
    if a.gpus != 1:
        print("bench.py: measures one MI355X; multi-GPU runs (--gpus %d) are not supported." % a.gpus,
              file=sys.stderr)
        return 2
    if a.profile_kernel:
        return profile_kernel(a)
    from tcb_amd import MODE_EXACT, MODE_FAST, Q4K, QuantBackend, _lib, synth

    mode = MODE_FAST if a.mode == "fast" else MODE_EXACT
    L = _lib.lib()
    tb = QuantBackend(0)
    ctx = tb.ctx

    raw = synth.quant_weights(Q4K, N, K, seed=3, outliers=0.01)
    x = synth.activations(1, K, seed=4)
    wbytes = raw.nbytes
    ring_n = max(2, -(-RING_BYTES // wbytes))
    ring = [tb.FromQuantized(Q4K, raw, N, K) for _ in range(ring_n)]
    xb = ctx.to_device(x)
    cb = ctx.alloc(N * 4)

    warm_replays = max(1, -(-max(a.warmup, MIN_WARMUP) // ring_n))
    replays = max(1, -(-a.steps // ring_n))
    steps = replays * ring_n
    abytes = algorithmic_bytes(N, K)

    def measure(md):
        # one eager call sizes any workspace before capture
        tb.GemmSet(1, N, K, xb, ring[0], cb, mode=md)
        ctx.sync()
        out = cb.download(np.float32, N)
        g_cold = capture(tb, lambda: [tb.GemmSet(1, N, K, xb, w, cb, mode=md) for w in ring])
        g_warm = capture(tb, lambda: [tb.GemmSet(1, N, K, xb, ring[0], cb, mode=md) for _ in ring])
        time_graph(tb, g_cold, warm_replays)
        ms_cold = time_graph(tb, g_cold, replays)
        time_graph(tb, g_warm, 1)
        ms_warm = time_graph(tb, g_warm, replays)
        for g in (g_cold, g_warm):
            L.trhip_graph_destroy(g)
        return out, ms_cold * 1e3 / steps, ms_warm * 1e3 / steps

    gpu_out, us_cold, us_warm = measure(mode)

    # single-launch streaming-read ceiling: the same number of bytes read once by trhip_read_probe, over a cold ring
    # of plain buffers timed the same way; no kernel that streams these bytes in one launch can be faster
    rbytes = wbytes // 16 * 16
    rring = [ctx.alloc(rbytes) for _ in range(ring_n)]
    for b in rring:
        b.fill(1)
    ctx.read_probe(rring[0], rbytes)
    ctx.sync()
    g_read = capture(tb, lambda: [ctx.read_probe(b, rbytes) for b in rring])
    time_graph(tb, g_read, warm_replays)
    us_read = time_graph(tb, g_read, replays) * 1e3 / steps
    L.trhip_graph_destroy(g_read)
    for b in rring:
        b.free()
    gbs_cold = abytes / (us_cold * 1e-6) / 1e9
    gbs_warm = abytes / (us_warm * 1e-6) / 1e9
    other = MODE_EXACT if mode == MODE_FAST else MODE_FAST
    other_out, us_other, us_other_warm = measure(other)
    exact_out = other_out if other == MODE_EXACT else gpu_out
    other_name = "exact" if other == MODE_EXACT else "fast"

    # prefill: act-quant GEMM, M rows, same weight
    prefill = None
    if a.prefill_m > 0:
        M = a.prefill_m
        X = synth.activations(M, K, seed=5)
        Xb = ctx.to_device(X)
        Cb = ctx.alloc(M * N * 4)

        def prefill_ms(md):
            tb.GemmActQuant(M, N, K, Xb, ring[0], Cb, accumulate=False, mode=md)
            ctx.sync()
            gp = capture(tb, lambda: tb.GemmActQuant(M, N, K, Xb, ring[0], Cb, accumulate=False, mode=md))
            time_graph(tb, gp, 3)
            reps = 10
            ms = time_graph(tb, gp, reps) / reps
            L.trhip_graph_destroy(gp)
            return ms

        ms = prefill_ms(mode)
        ms_other = prefill_ms(MODE_EXACT if mode == MODE_FAST else MODE_FAST)
        tops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
        ceiling = mfma_rate(tb, 0, 2)
        ceiling7 = mfma_rate(tb, 6, 2)
        loop_us = prefill_loop_us(tb, 1 if mode == MODE_FAST else 0, M, N, K)
        loop_us_q6 = prefill_loop_us(tb, 2, M, N, K)
        prefill = {"workload": "act-quant GEMM q4_k %dx%d, M=%d (quantize + int block sums + fp32 epilogue)" % (N, K, M),
                   "mode": a.mode, "us": round(ms * 1e3, 2), "int8_tops": round(tops, 2),
                   "frac_of_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                   other_name + "_mode_us": round(ms_other * 1e3, 2),
                   other_name + "_mode_frac_of_int8_peak": round(2.0 * M * N * K / (ms_other * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
                   "measured_int8_mfma_tops": round(ceiling, 1),
                   "measured_int8_mfma_tops_6valu": round(ceiling7, 1),
                   "frac_of_measured_int8": round(tops / ceiling, 4),
                   "inner_loop": {"us": round(loop_us, 2),
                                  "frac_of_int8_peak": round(2.0 * M * N * K / (loop_us * 1e-6) / 1e12 / INT8_PEAK_TOPS, 4),
                                  "q6_k_us": round(loop_us_q6, 2),
                                  "what": "trhip_prefill_probe: the kernel's per-block loop on the same grid, staging, "
                                          "barriers and stores taken out (events, median of 20)"},
                   "traffic_bytes": PREFILL_TRAFFIC if M == 512 else None,
                   "traffic_source": "rocprofv3 FETCH_SIZE + WRITE_SIZE over --profile-kernel prefill, kept in "
                                     "profiles/prefill_q4_k_14336x4096_M512.txt (not measured in this run)"}
        Xb.free()
        Cb.free()

    upload = upload_rates(tb, raw)
    sweep = decode_sweep(tb, (1, 16), mode) if a.sweep else None
    shapes = shape_table(tb) if a.shapes else None

    # CPU baseline: AVX2 restatement of the reference's sdotq4k GEMV, all host cores, same bytes
    cpu = None
    if a.cpu_seconds > 0:
        import ctypes
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import oracle as O
        threads = len(os.sched_getaffinity(0))
        copies = 16  # host ring of 16 weight copies (528 MB) so the sample streams from DRAM
        hring = [raw.copy() for _ in range(copies)]
        out = np.zeros(N, np.float32)
        P = ctypes.c_void_p
        xs = np.ascontiguousarray(x.reshape(-1))
        O.lib().trq_avx2_quant_gemv(Q4K, N, K, xs.ctypes.data_as(P), hring[0].ctypes.data_as(P), out.ctypes.data_as(P), threads)
        cpu_matches = bool(np.array_equal(out.view(np.uint32), exact_out.view(np.uint32)))
        fast_out = gpu_out if mode == MODE_FAST else other_out
        fast_err = float(np.max(np.abs(fast_out.astype(np.float64) - out) / (1.0 + np.abs(out.astype(np.float64)))))
        n_done, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < a.cpu_seconds:
            O.lib().trq_avx2_quant_gemv(Q4K, N, K, xs.ctypes.data_as(P), hring[n_done % copies].ctypes.data_as(P),
                                        out.ctypes.data_as(P), threads)
            n_done += 1
        dt = time.perf_counter() - t0
        cpu = {"value": round(abytes * n_done / dt / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": "%d GEMVs of q4_k %dx%d over a 16-copy host ring, %.1f s; AVX2 sdotq4k restatement" % (
                   n_done, N, K, dt),
               "us_per_gemv": round(dt / n_done * 1e6, 1), "gpu_exact_bits_equal_cpu": cpu_matches,
               "gpu_fast_max_rel_err_vs_cpu": fast_err}

    line = {
        "metric": METRIC,
        "value": round(gbs_cold, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm_replays * ring_n,
        "requested": {"steps": a.steps, "warmup": a.warmup,
                      "rule": "steps rounded up to whole passes of the %d-copy ring; warm-up at least %d launches" % (
                          ring_n, MIN_WARMUP)},
        "ms_per_step": round(us_cold / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "q4_k decode GEMV %dx%d batch 1, fp32 activations, %s mode, cold ring of %d copies (%.2f GiB)" % (
            N, K, a.mode, ring_n, ring_n * wbytes / (1 << 30)), "N": N, "K": K, "batch": 1, "mode": a.mode},
        "us_per_gemv": round(us_cold, 3),
        "hbm_frac_of_peak": round(gbs_cold / HBM_PEAK_GBS, 4),
        "warm": {"us_per_gemv": round(us_warm, 3), "GB/s": round(gbs_warm, 1)},
        "read_ceiling": {"us_per_launch": round(us_read, 3), "GB/s": round(rbytes / (us_read * 1e-6) / 1e9, 1),
                         "frac_of_peak": round(rbytes / (us_read * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                         "gemv_frac_of_ceiling": round(us_read / us_cold, 4),
                         "workload": "trhip_read_probe: %d bytes read once per launch, cold ring of %d buffers" % (
                             rbytes, ring_n)},
        other_name + "_mode": {"us_per_gemv": round(us_other, 3), "GB/s": round(abytes / (us_other * 1e-6) / 1e9, 1),
                               "warm_us_per_gemv": round(us_other_warm, 3)},
        "roofline": {"bound": "hbm", "achieved": round(gbs_cold, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs_cold / HBM_PEAK_GBS, 4), "traffic": TRAFFIC.get(a.mode),
                     "traffic_source": "rocprofv3 FETCH_SIZE + WRITE_SIZE over --profile-kernel gemv, kept in "
                                       "profiles/gemv_q4_k_14336x4096_traffic.txt (not measured in this run)",
                     "kernel": "gemv_q4_k_%s" % a.mode, "algorithmic_bytes_per_launch": abytes},
        "prefill": prefill,
        "store_upload": upload,
        "decode_sweep": sweep,
        "shapes": shapes,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    for w in ring:
        w.release()
    tb.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
