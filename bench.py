#!/usr/bin/env python3
"""Benchmark of the cuda_inf attention path on one MI355X.

Default workload (the decode configuration of the headline metric): flash-
decoding at 32768 tokens of context, 6 attention layers run back to back per
token, batch 1, 32 query / 8 kv heads, head_dim 64, FP8 E4M3 group-64 cache
with an fp16 tail.  Each timed step is one token: for every layer, append the
fresh K/V through the tail (and the FP8 commit when a group fills) and run
the attention.  Synthetic seeded inputs (N(0,1); K/V with 1% outliers x20;
Q with QK-RMSNorm + RoPE), resident in HBM before timing starts.

The decode loop launches k_decode_tok once per run of consecutive tokens
(up to the token that fills a group); one launch per token and one launch
per layer are timed beside it on the same tokens.

Printed: one JSON line with µs/token (warm: consecutive tokens; cold: the
256 MB Infinity Cache flushed before every token, one launch per token),
the decode kernel's roofline against 8 TB/s, a causal-prefill leg (4096
tokens), and the CPU oracle timed on this host as a baseline.

    python bench.py [--steps 256] [--warmup 10] [--ctx 32768] [--layers 6]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16
MFMA_FP8_PEAK_TFLOPS = 5000.0  # MI355X dense fp8
TRAFFIC_FILE = "profiles/decode_ctx32k_traffic.json"


def algo_bytes(Tc: int, Tt: int) -> int:
    """Algorithmic bytes of one layer's decode: FP8 K+V, fp16 group scales,
    fp16 tail K+V, q in and out."""
    return 1024 * Tc + (Tc // 64) * 8 * 2 * 2 + 2048 * Tt + 8192


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--layers", type=int, default=6)
    ap.add_argument("--nsplit", type=int, default=0,
                    help="0: matrix-core decode (one launch per layer); "
                         ">0: the reference's split+combine with this split count")
    ap.add_argument("--cold-steps", type=int, default=32)
    ap.add_argument("--prefill", type=int, default=4096, help="prefill tokens (0 = skip)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--traffic", type=float, default=None,
                    help="HBM bytes per decode token measured with rocprofv3 --pmc "
                         "(FETCH_SIZE + WRITE_SIZE, copy-kernel scaled); roofline.traffic "
                         "is this times the timed launches' tokens per launch")
    ap.add_argument("--long-ctx", type=int, default=131072,
                    help="long-context decode leg: context tokens (0 = skip)")
    ap.add_argument("--long-steps", type=int, default=8)
    ap.add_argument("--prep-steps", type=int, default=64,
                    help="decode tokens with the QK producers run inside the decode kernels "
                         "(raw q/k in; 0 = skip)")
    ap.add_argument("--block-steps", type=int, default=64,
                    help="decode tokens through the whole attention branch: INT4 q/k/v "
                         "projections, producers, attention, out_proj + residual (0 = skip)")
    ap.add_argument("--h2o-steps", type=int, default=4000,
                    help="H2O decode steps after a 1024-token prompt (0 = skip)")
    ap.add_argument("--upload-mib", type=int, default=0,
                    help="weights.bin upload leg: MiB of synthetic file (0 = skip)")
    ap.add_argument("--tokenizer", action="store_true",
                    help="host tokenizer leg (encode throughput; the reference's tokenizer.h "
                         "timed beside it under cpu_baseline)")
    ap.add_argument("--split-steps", type=int, default=32,
                    help="decode tokens through the reference's split + combine (16 splits) "
                         "at the headline context (0 = skip)")
    ap.add_argument("--calib-copy", type=int, default=0,
                    help="MiB: first run a plain device copy of this size three times "
                         "(the reference dispatch that scales rocprofv3 byte counters)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        sys.exit("bench.py measures one GPU: the attention path runs on a single MI355X; "
                 "--gpus above 1 is not supported")

    import torch
    from cuda_inf_amd import _lib, workload
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd._lib import D, NH, NKV, call

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()
    nL, ctx, K, W = a.layers, a.ctx, a.steps, a.warmup
    total_steps = W + 4 * K + 4 + a.cold_steps + a.prep_steps + a.block_steps + a.split_steps
    maxT = ctx + total_steps + 64
    log = lambda *x: print("[bench]", *x, file=sys.stderr, flush=True)  # noqa: E731
    log(f"device {torch.cuda.get_device_name(dev)}; ctx {ctx}, layers {nL}, steps {K}")

    if a.calib_copy > 0:
        n = a.calib_copy << 18
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy: 3 x {a.calib_copy} MiB read + written")
        del src, dst

    # ---- caches: ctx tokens per layer, loaded through the append loop
    layers = []
    for l in range(nL):
        L = AttnLayer(maxT, nsplit=a.nsplit, device=dev)
        g = workload.generator(1000 + l, dev)
        for c0 in range(0, ctx, 8192):
            n = min(8192, ctx - c0)
            k = workload.with_outliers(workload.normal_f16((n, NKV, D), g, dev), g)
            v = workload.with_outliers(workload.normal_f16((n, NKV, D), g, dev), g)
            call("cia_layer_append", ctypes.byref(L._s), k.data_ptr(), v.data_ptr(), n, c0,
                 stream.cuda_stream)
        layers.append(L)
    torch.cuda.synchronize()
    assert all(L.committed == ctx - ctx % 64 for L in layers)
    arr = (_lib.cia_layer * nL)(*[L._s for L in layers])

    # ---- per-token inputs for every step and layer
    g = workload.generator(7, dev)
    pos = torch.arange(ctx, ctx + total_steps, device=dev)
    q = workload.normal_f16((total_steps, nL, NH, D), g, dev)
    q = torch.stack([workload.prep_qk(q[:, l], pos) for l in range(nL)], dim=1).contiguous()
    kk = workload.with_outliers(workload.normal_f16((total_steps, nL, NKV, D), g, dev), g)
    vv = workload.with_outliers(workload.normal_f16((total_steps, nL, NKV, D), g, dev), g)
    out = torch.empty((total_steps, nL, NH, D), dtype=torch.float16, device=dev)
    qrow, krow = nL * NH * D, nL * NKV * D
    cur = {"step": 0}

    def run(steps, events=None, per=0, tpl=0):
        """steps decode tokens through cia_decode_loop_runs: per = 0 runs the
        layers of a token in one launch (k_decode_tok), 1 one launch per
        layer (k_decode); tpl = 0 runs consecutive tokens in one launch up
        to each group fill, 1 one launch per token"""
        s0 = cur["step"]
        call("cia_decode_loop_runs", arr, nL, q.data_ptr() + s0 * qrow * 2,
             kk.data_ptr() + s0 * krow * 2, vv.data_ptr() + s0 * krow * 2,
             out.data_ptr() + s0 * qrow * 2, ctx + s0, steps, 0.125, per, tpl, events,
             stream.cuda_stream)
        cur["step"] += steps

    def launches_of_steps(s0, steps):
        """k_decode_tok launches of the decode loop over steps s0.. : runs
        of tokens, each ending at the token that fills a group (the tail
        holds (ctx + s) % 64 tokens before step s)"""
        n, i = 0, 0
        while i < steps:
            i += min(steps - i, 64 - (ctx + s0 + i) % 64)
            n += 1
        return n

    def bytes_of_steps(s0, steps):
        tot = 0
        for i in range(s0, s0 + steps):
            qp = ctx + i
            Tc = ((qp + 1) // 64) * 64
            tot += algo_bytes(Tc, qp + 1 - Tc)
        return tot * nL

    # ---- warm-up, then the timed region (warm: consecutive tokens)
    run(W)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_timed = cur["step"]
    torch.cuda.synchronize()
    e0.record(stream)
    run(K)
    e1.record(stream)
    torch.cuda.synchronize()
    warm_ms = e0.elapsed_time(e1)
    us_tok = warm_ms * 1e3 / K
    timed_bytes = bytes_of_steps(s_timed, K)
    log(f"warm: {us_tok:.2f} us/token, effective {timed_bytes / (warm_ms * 1e-3) / 1e9:.0f} GB/s")

    # The decode launch (k_decode_tok: a run of consecutive tokens, all nL
    # layers of each; per layer the FP8 stream, the tail, the fresh token's
    # write and the merge, each layer scored after the one before it has
    # stored its output) is the dominant work.  The decode loop ends a run
    # at the token that fills a group (its FP8 commit), so the timed region's
    # launches are its segments between group fills; their average duration
    # is the region's span over their count (events bracket the region on
    # the kernels' own stream).
    n_launch = launches_of_steps(s_timed, K) if a.nsplit == 0 else K
    dec_us = warm_ms * 1e3 / n_launch
    dec_bytes = timed_bytes / n_launch
    achieved = dec_bytes / (dec_us * 1e-6) / 1e9

    # ---- one token per launch: HIP events recorded by the decode loop right
    # before and after each token's launch (with events the loop launches
    # token by token; each event adds its own marker overhead)
    nev = 3 * K * nL
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(nev)]
    for e in evs:  # the hipEvent_t handles exist once recorded
        e.record(stream)
    torch.cuda.synchronize()
    ev_arr = (ctypes.c_void_p * nev)(*[e.cuda_event for e in evs]) if nev else None
    run(K, ev_arr)
    torch.cuda.synchronize()
    # the loop records each layer's "before" event ahead of the launch and its
    # "after" events behind it: the last "before" (layer nL-1) and the first
    # "after" (layer 0) bracket the launch alone
    one = sorted(evs[3 * nL * r + 3 * (nL - 1)].elapsed_time(evs[3 * nL * r + 1]) * 1e3
                 for r in range(K))
    ev_us = one[len(one) // 2]
    log(f"decode launches: {n_launch} for {K} tokens, {dec_us:.2f} us and {dec_bytes / 1e6:.2f} MB "
        f"each, {achieved:.0f} GB/s; one token per launch (event-bracketed): median {ev_us:.2f} us")

    # ---- the same tokens with one launch per token (k_decode_tok, all
    # layers of the token; back to back, no events)
    run(2, tpl=1)
    torch.cuda.synchronize()
    e0.record(stream)
    run(K, tpl=1)
    e1.record(stream)
    torch.cuda.synchronize()
    ot_ms = e0.elapsed_time(e1)
    ot_bytes = bytes_of_steps(cur["step"] - K, K)
    one_token = {"us_per_token": round(ot_ms * 1e3 / K, 3),
                 "gbps": round(ot_bytes / (ot_ms * 1e-3) / 1e9, 1),
                 "kernel": f"k_decode_tok (one launch per token: {nL} layers)"}
    log(f"one launch per token: {one_token['us_per_token']:.2f} us/token "
        f"({one_token['gbps']:.0f} GB/s)")

    # ---- the same tokens with one launch per layer (k_decode; the
    # reference's per-layer launch structure)
    run(2, per=1)
    torch.cuda.synchronize()
    e0.record(stream)
    run(K, per=1)
    e1.record(stream)
    torch.cuda.synchronize()
    pl_ms = e0.elapsed_time(e1)
    pl_bytes = bytes_of_steps(cur["step"] - K, K)
    per_layer = {"us_per_token": round(pl_ms * 1e3 / K, 3),
                 "us_per_launch": round(pl_ms * 1e3 / (K * nL), 3),
                 "gbps": round(pl_bytes / (pl_ms * 1e-3) / 1e9, 1),
                 "kernel": "k_decode (one launch per layer)"}
    log(f"one launch per layer: {per_layer['us_per_token']:.2f} us/token "
        f"({per_layer['us_per_launch']:.2f} us per launch, {per_layer['gbps']:.0f} GB/s)")

    # ---- measured ceiling: a plain streaming read of the same layers'
    # committed FP8 K and V, one launch per layer, the same count of
    # back-to-back launches as the timed region
    sink = torch.zeros(1, dtype=torch.int32, device=dev)

    def plain_read(n_tok):
        for _ in range(n_tok):
            for i, L in enumerate(layers):
                nb = arr[i].committed * NKV * D  # (arr holds the live copies)
                call("cia_stream_read", L.kc8.data_ptr(), L.vc8.data_ptr(), nb, sink.data_ptr(),
                     stream.cuda_stream)

    plain_read(2)
    torch.cuda.synchronize()
    e0.record(stream)
    plain_read(K)
    e1.record(stream)
    torch.cuda.synchronize()
    floor_us = e0.elapsed_time(e1) * 1e3 / (K * nL)
    floor_bytes = 2 * arr[0].committed * NKV * D
    floor_gbps = floor_bytes / (floor_us * 1e-6) / 1e9
    log(f"plain read of the same bytes: {floor_us:.2f} us per layer, {floor_gbps:.0f} GB/s "
        f"(the decode takes {us_tok / (nL * floor_us):.2f}x its time per token)")

    # ---- cold: evict the KV from the 256 MB Infinity Cache before every token
    # by reading 1 GiB of other data (a read leaves no dirty lines behind)
    flush = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    cold = []
    for _ in range(a.cold_steps):
        flush.sum()
        torch.cuda.synchronize()
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        c0.record(stream)
        run(1)
        c1.record(stream)
        torch.cuda.synchronize()
        cold.append(c0.elapsed_time(c1) * 1e3)
    # the plain read, cold the same way (one token's worth of launches)
    floor_cold = []
    for _ in range(a.cold_steps if cold else 0):
        flush.sum()
        torch.cuda.synchronize()
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        c0.record(stream)
        plain_read(1)
        c1.record(stream)
        torch.cuda.synchronize()
        floor_cold.append(c0.elapsed_time(c1) * 1e3)
    del flush
    cold.sort()
    floor_cold.sort()
    cold_us = cold[len(cold) // 2] if cold else None
    floor_cold_us = floor_cold[len(floor_cold) // 2] if floor_cold else None
    if cold:
        log(f"cold: median {cold_us:.2f} us/token; plain read cold {floor_cold_us:.2f} us/token")
    mean_tok_bytes = timed_bytes / K

    # ---- the reference's launch shape at the same context: per layer the
    # append launch, attn_decode_split with 16 splits and attn_decode_combine
    # (engine.cu:830-852), split and combine event-bracketed separately
    split16 = None
    if a.split_steps > 4:
        ns = 16
        sbufs = []
        for l in range(nL):
            pm = torch.zeros(NH * ns, dtype=torch.float32, device=dev)
            pl = torch.zeros(NH * ns, dtype=torch.float32, device=dev)
            po = torch.zeros(NH * ns * D, dtype=torch.float32, device=dev)
            sbufs.append((pm, pl, po))
            arr[l].nsplit, arr[l].pm, arr[l].pl, arr[l].po = ns, pm.data_ptr(), pl.data_ptr(), po.data_ptr()
        n_ev = 2
        n = a.split_steps - 2 - n_ev
        run(2)
        torch.cuda.synchronize()
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        c0.record(stream)
        run(n)
        c1.record(stream)
        torch.cuda.synchronize()
        sp_us = c0.elapsed_time(c1) * 1e3 / n
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(3 * n_ev * nL)]
        for e in evs:  # the hipEvent_t handles exist once recorded
            e.record(stream)
        torch.cuda.synchronize()
        run(n_ev, (ctypes.c_void_p * len(evs))(*[e.cuda_event for e in evs]))
        torch.cuda.synchronize()
        first = sorted(evs[3 * r].elapsed_time(evs[3 * r + 1]) * 1e3 for r in range(n_ev * nL))
        second = sorted(evs[3 * r + 1].elapsed_time(evs[3 * r + 2]) * 1e3 for r in range(n_ev * nL))
        for l in range(nL):
            arr[l].nsplit = 0
        del sbufs
        s_bytes = bytes_of_steps(cur["step"] - n_ev - n, n) / n
        split16 = {"us_per_token": round(sp_us, 2), "tokens": n,
                   "gbps": round(s_bytes / (sp_us * 1e-6) / 1e9, 1),
                   "split_us_median": round(first[len(first) // 2], 2),
                   "combine_us_median": round(second[len(second) // 2], 2),
                   "launches": "append (k_append_tail / k_append_commit), k_decode split mode, "
                               "k_decode_combine_small per layer"}
        log(f"split+combine (16 splits) at {ctx}: {sp_us:.2f} us/token; split "
            f"{split16['split_us_median']} us + combine {split16['combine_us_median']} us per "
            f"layer (event-bracketed medians)")

    # ---- QK producers fused: the same layers take raw q / k, and the decode
    # kernels run per-head RMSNorm + RoPE (engine.cu:799-801) themselves
    prep = None
    if a.prep_steps > 0:
        g8 = workload.generator(17, dev)
        qw = (1.0 + 0.1 * torch.randn(D, generator=g8, device=dev)).to(torch.float16)
        kw = (1.0 + 0.1 * torch.randn(D, generator=g8, device=dev)).to(torch.float16)
        prep_ws = [torch.zeros((NH + NKV) * D, dtype=torch.float16, device=dev) for _ in range(nL)]
        for l in range(nL):
            arr[l].qw, arr[l].kw = qw.data_ptr(), kw.data_ptr()
            arr[l].eps, arr[l].theta = workload.EPS, workload.ROPE_THETA
            arr[l].prep_ws, arr[l].prep_cap = prep_ws[l].data_ptr(), 1
        run(2)
        torch.cuda.synchronize()
        n = a.prep_steps - 2
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        c0.record(stream)
        run(n)
        c1.record(stream)
        torch.cuda.synchronize()
        prep_us = c0.elapsed_time(c1) * 1e3 / n
        for l in range(nL):
            arr[l].qw = arr[l].kw = arr[l].prep_ws = None
            arr[l].prep_cap = 0
        # (runs of tokens as with prepared inputs)
        prep = {"us_per_token": round(prep_us, 2), "tokens": n,
                "over_prepared_inputs_us": round(prep_us - us_tok, 2),
                "kernels": "producers inside k_decode_tok (runs of tokens; q rows prepared "
                           "in LDS, fresh k by the tail waves, each token's RoPE by the "
                           "control wave)"}
        log(f"decode with fused QK producers: {prep_us:.2f} us/token "
            f"({prep_us - us_tok:+.2f} against prepared inputs)")

    # ---- the whole attention branch (engine.cu:792-859): INT4 q/k/v in one
    # launch, producers + attention, out_proj into the residual; synthetic
    # INT4 weights (uniform nibbles, scales 0.002-0.02)
    block = None
    if a.block_steps > 0:
        gb = torch.Generator(device=dev)
        gb.manual_seed(23)
        H = _lib.HIDDEN
        g8 = workload.generator(17, dev)
        qw = (1.0 + 0.1 * torch.randn(D, generator=g8, device=dev)).to(torch.float16)
        kw = (1.0 + 0.1 * torch.randn(D, generator=g8, device=dev)).to(torch.float16)
        keep, parr = [], (_lib.cia_attn_proj * nL)()
        for l in range(nL):
            arr[l].qw, arr[l].kw = qw.data_ptr(), kw.data_ptr()
            arr[l].eps, arr[l].theta = workload.EPS, workload.ROPE_THETA
            pw = torch.zeros((NH + NKV) * D, dtype=torch.float16, device=dev)
            arr[l].prep_ws, arr[l].prep_cap = pw.data_ptr(), 1
            keep.append(pw)
            for name, N in (("q", NH * D), ("k", NKV * D), ("v", NKV * D), ("o", H)):
                pk = torch.randint(0, 256, (N, H // 2), generator=gb, device=dev, dtype=torch.uint8)
                sc = (0.002 + 0.018 * torch.rand((N, H // 128), generator=gb, device=dev)).half()
                setattr(parr[l], name + "_packed", pk.data_ptr())
                setattr(parr[l], name + "_scales", sc.data_ptr())
                keep += [pk, sc]
            ws = torch.zeros(2 * NH * D + 2 * NKV * D, dtype=torch.float16, device=dev)
            parr[l].ws, parr[l].cap = ws.data_ptr(), 1
            keep.append(ws)
        nb = a.block_steps
        xb = torch.randn((nb, nL, H), generator=gb, device=dev).half()
        hb = torch.zeros(H, dtype=torch.float32, device=dev)

        def run_block(i0, n, events=None):
            call("cia_attn_block_loop", arr, parr, nL, xb.data_ptr() + i0 * nL * H * 2,
                 hb.data_ptr(), ctx + cur["step"], n, 0.125, events, stream.cuda_stream)
            cur["step"] += n

        n_ev = 4
        n_t = nb - 2 - n_ev
        run_block(0, 2)
        torch.cuda.synchronize()
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        c0.record(stream)
        run_block(2, n_t)
        c1.record(stream)
        torch.cuda.synchronize()
        blk_us = c0.elapsed_time(c1) * 1e3 / n_t
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(4 * n_ev * nL)]
        for e in evs:  # the hipEvent_t handles exist once recorded
            e.record(stream)
        torch.cuda.synchronize()
        run_block(2 + n_t, n_ev, (ctypes.c_void_p * len(evs))(*[e.cuda_event for e in evs]))
        torch.cuda.synchronize()
        parts = [[], [], []]
        for r in range(n_ev * nL):
            for j in range(3):
                parts[j].append(evs[4 * r + j].elapsed_time(evs[4 * r + j + 1]) * 1e3)
        med = [sorted(p)[len(p) // 2] for p in parts]
        for l in range(nL):
            arr[l].qw = arr[l].kw = arr[l].prep_ws = None
            arr[l].prep_cap = 0
        wbytes = (2 * NH * D + 2 * NKV * D) * (H // 2 + H // 64)
        block = {"us_per_token": round(blk_us, 2), "tokens": n_t,
                 "us_per_layer": round(blk_us / nL, 2),
                 "event_bracketed_us": {"qkv_proj": round(med[0], 2), "attention": round(med[1], 2),
                                        "out_proj_residual": round(med[2], 2)},
                 "int4_weight_bytes_per_layer": wbytes,
                 "launches_per_layer": 3,
                 "kernels": "k_gemv_int4 (q/k/v), k_decode (producers inside), "
                            "k_gemv_int4 (out_proj + residual)"}
        log(f"attention branch (INT4 projections + attention): {blk_us:.2f} us/token; "
            f"per layer qkv {med[0]:.2f} / attention {med[1]:.2f} / out_proj {med[2]:.2f} us")

    # ---- prefill leg: causal attention_fused over a fresh cache
    prefill = None
    if a.prefill > 0:
        S = a.prefill
        Lp = AttnLayer(S + 64, nsplit=16, device=dev)
        qp, kp, vp = workload.qkv(S, seed=0, device=dev)
        Lp.forward(qp, kp, vp, 0)  # warm-up (appends + attends)
        torch.cuda.synchronize()
        from cuda_inf_amd import kernels as Kn
        outp = torch.empty_like(qp)
        reps = 10
        p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

        def gpu_ms(fn):
            """Mean GPU time of fn's launches: one untimed call first keeps the
            GPU busy while the timed ones are enqueued, so the host's argument
            checks between calls are not counted."""
            torch.cuda.synchronize()
            fn()
            p0.record(stream)
            for _ in range(reps):
                fn()
            p1.record(stream)
            torch.cuda.synchronize()
            return p0.elapsed_time(p1) / reps

        pms = gpu_ms(lambda: Kn.attention_fused(qp, Lp.kc8, Lp.vc8, Lp.ksc, Lp.vsc, Lp.ktail,
                                                Lp.vtail, Lp.committed, outp, None, S, 0, 0.125))

        # the whole layer step of the reference: append (FP8 commit of every
        # full group, tail) and then the fused attention
        def layer_step():
            Lp._s.committed = 0
            Lp.forward(qp, kp, vp, 0, out=outp)

        lms = gpu_ms(layer_step)
        # the OCP-fp8 matrix-core variant on the same cache; its output is
        # compared with the fp16 kernel's (the tests compare both with the
        # fp32 restatement)
        out8 = torch.empty_like(qp)
        Kn.attention_fused(qp, Lp.kc8, Lp.vc8, Lp.ksc, Lp.vsc, Lp.ktail, Lp.vtail,
                           Lp.committed, outp, None, S, 0, 0.125)
        Kn.attention_fused_fp8(qp, Lp.kc8, Lp.vc8, Lp.ksc, Lp.vsc, Lp.ktail, Lp.vtail,
                               Lp.committed, out8, S, 0, 0.125)
        torch.cuda.synchronize()
        d8 = (out8.float() - outp.float()).abs()
        f8ms = gpu_ms(lambda: Kn.attention_fused_fp8(qp, Lp.kc8, Lp.vc8, Lp.ksc, Lp.vsc, Lp.ktail,
                                                     Lp.vtail, Lp.committed, out8, S, 0, 0.125))
        flops = 4.0 * D * NH * S * (S + 1) / 2
        prefill = {"tokens": S, "us": round(pms * 1e3, 1),
                   "tflops": round(flops / (pms * 1e-3) / 1e12, 2),
                   "mfma_f16_frac": round(flops / (pms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
                   "kernel": "attention_fused",
                   "layer_us_with_append": round(lms * 1e3, 1),
                   "fp8_experimental": {
                           "kernel": "attention_fused_fp8 (v_mfma_scale_f32_16x16x128_f8f6f4; "
                                     "experimental, slower than the fp16 kernel, not on the path)",
                           "us": round(f8ms * 1e3, 1),
                           "tflops": round(flops / (f8ms * 1e-3) / 1e12, 2),
                           "mfma_fp8_frac": round(flops / (f8ms * 1e-3) / 1e12
                                                  / MFMA_FP8_PEAK_TFLOPS, 4),
                           "max_abs_diff_vs_fp16": round(float(d8.max()), 5),
                           "mean_abs_diff_vs_fp16": round(float(d8.mean()), 7)}}
        log(f"prefill {S}: attention {pms * 1e3:.1f} us, {prefill['tflops']} TFLOP/s; "
            f"append + attention {lms * 1e3:.1f} us; experimental fp8 {f8ms * 1e3:.1f} us "
            f"({prefill['fp8_experimental']['tflops']} TFLOP/s), "
            f"max |fp8 - fp16| {float(d8.max()):.4f}")
        # the layer's INT4 projections over the S prompt rows (matrix-core
        # GEMM): q/k/v in one launch, out_proj into the residual
        H = _lib.HIDDEN
        gp = torch.Generator(device=dev)
        gp.manual_seed(29)
        wts = {}
        for name, N in (("q", NH * D), ("k", NKV * D), ("v", NKV * D), ("o", H)):
            wts[name] = (torch.randint(0, 256, (N, H // 2), generator=gp, device=dev,
                                       dtype=torch.uint8),
                         (0.002 + 0.018 * torch.rand((N, H // 128), generator=gp,
                                                     device=dev)).half())
        xp = torch.randn((S, H), generator=gp, device=dev).half()
        hp = torch.zeros((S, H), dtype=torch.float32, device=dev)
        pq = torch.empty((S, NH * D), dtype=torch.float16, device=dev)
        pk = torch.empty((S, NKV * D), dtype=torch.float16, device=dev)
        pv = torch.empty_like(pk)
        Kn.qkv_proj_int4(xp, wts["q"], wts["k"], wts["v"], pq, pk, pv, S, H)
        Kn.gemv_int4(pq, *wts["o"], hp, H, NH * D, S, add=True)
        torch.cuda.synchronize()
        qkv_ms = gpu_ms(lambda: Kn.qkv_proj_int4(xp, wts["q"], wts["k"], wts["v"], pq, pk, pv,
                                                 S, H))
        o_ms = gpu_ms(lambda: Kn.gemv_int4(pq, *wts["o"], hp, H, NH * D, S, add=True))
        f_qkv = 2.0 * S * H * (NH * D + 2 * NKV * D)
        f_o = 2.0 * S * H * NH * D
        prefill["int4_projections"] = {
            "kernel": "k_gemm_int4 (v_mfma_f32_16x16x32_f16, exact nibble operands, "
                      "per-group fp32 scaling)",
            "qkv_us": round(qkv_ms * 1e3, 1),
            "qkv_tflops": round(f_qkv / (qkv_ms * 1e-3) / 1e12, 1),
            "out_proj_residual_us": round(o_ms * 1e3, 1),
            "out_proj_tflops": round(f_o / (o_ms * 1e-3) / 1e12, 1),
            "mfma_f16_frac": round((f_qkv + f_o) / ((qkv_ms + o_ms) * 1e-3) / 1e12
                                   / MFMA_F16_PEAK_TFLOPS, 4)}
        log(f"prefill {S}: INT4 q/k/v {qkv_ms * 1e3:.1f} us, out_proj {o_ms * 1e3:.1f} us")

    cpu_layer, cpu_committed = layers[0], arr[0].committed

    # ---- long-context leg: matrix-core decode and the reference's split +
    # combine at the split counts of the sweep
    long_ctx = None
    if a.long_ctx > 0:
        del layers, arr
        torch.cuda.empty_cache()
        long_ctx = long_context_leg(a.long_ctx, nL, a.long_steps, dev, stream, log)

    # ---- H2O leg: 2048-slot buffer, window 256, 1024-token prompt
    h2o = h2o_leg(a.h2o_steps, dev, stream, log) if a.h2o_steps > 0 else None

    # ---- weights.bin upload: pinned double-buffered against one pageable buffer
    upload = upload_leg(a.upload_mib, dev, log) if a.upload_mib > 0 else None
    # ---- tokenizer (host): encode throughput; the reference's tokenizer.h
    # on the same text goes to the cpu_baseline block
    tokenizer, tok_ref = (tokenizer_leg(log, with_reference=not a.no_cpu) if a.tokenizer
                          else (None, None))

    # ---- CPU baseline: the oracle on this host's cores, one layer at a time
    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline(cpu_layer, cpu_committed, ctx + cur["step"] - 1, q, nL,
                           a.cpu_seconds, log)

    cpu_prefill = cpu_h2o = None
    if not a.no_cpu:
        if a.prefill > 0:
            cpu_prefill = cpu_prefill_baseline(a.prefill, a.cpu_seconds, log)
        if a.h2o_steps > 0:
            cpu_h2o = cpu_h2o_baseline(a.cpu_seconds, log)
    if cpu is not None and tok_ref is not None:
        cpu["tokenizer_reference"] = tok_ref
    if prefill is not None:
        prefill["cpu_baseline"] = cpu_prefill
    if h2o is not None:
        h2o["cpu_baseline"] = cpu_h2o

    # HBM bytes per launch: per token from the committed counters, times
    # the timed launches' tokens
    traffic = a.traffic if a.traffic is not None else measured_traffic(ctx, nL)
    if traffic is not None:
        traffic = int(round(traffic * K / n_launch))
    res = {
        "metric": "decode-attn µs/token + HBM GB/s (% of 8 TB/s) at 32k ctx; prefill MFMA util",
        "value": round(us_tok, 3),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(warm_ms / K, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 MFMA operands (P in fp16), fp32 accumulate; FP8-E4M3/fp16 cache",
        "data": "synthetic: seeded N(0,1), K/V 1% outliers x20, Q QK-RMSNorm+RoPE",
        "config": {"workload": f"flash-decoding, ctx {ctx}, {nL} attention layers/token, batch 1, "
                               f"32Q/8KV heads, d64, FP8 E4M3 group-64 KV + fp16 tail",
                   "context": ctx, "layers": nL, "decode": "matrix-core, one launch per run of "
                   "tokens up to each group fill (all layers; each layer scored after the "
                   "one before it has stored its output)"
                   if a.nsplit == 0 else f"split+combine nsplit={a.nsplit}"},
        "effective_gbps_warm": round(timed_bytes / (warm_ms * 1e-3) / 1e9, 1),
        "cold_us_per_token": round(cold_us, 3) if cold_us else None,
        "effective_gbps_cold": round(mean_tok_bytes / (cold_us * 1e-6) / 1e9, 1) if cold_us else None,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "traffic_source": TRAFFIC_FILE + " (not this run)" if traffic else None,
                     "kernel": f"k_decode_tok (one launch per run of tokens: {nL} layers each)",
                     "launches": n_launch,
                     "tokens_per_launch": round(K / n_launch, 2),
                     "algo_bytes_per_launch": int(dec_bytes),
                     "avg_launch_us": round(dec_us, 3),
                     "one_token_launch_median_us": round(ev_us, 3),
                     "measured_ceiling": {
                         "kernel": "k_stream_read (plain read of the same FP8 K+V, one "
                                   "launch per layer)",
                         "us_per_layer": round(floor_us, 3), "gbps": round(floor_gbps, 1),
                         "frac": round(achieved / floor_gbps, 4),
                         "cold_us_per_token": round(floor_cold_us, 3) if floor_cold_us else None,
                         "cold_frac": round(floor_cold_us / cold_us, 4) if floor_cold_us else None}},
        "one_token_launches": one_token,
        "per_layer_launches": per_layer,
        "prefill": prefill,
        "split16": split16,
        "qk_producers_fused": prep,
        "attention_branch": block,
        "long_context": long_ctx,
        "h2o": h2o,
        "weights_upload": upload,
        "tokenizer": tokenizer,
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


def upload_leg(mib, dev, log, runs=3):
    """weights.bin into HBM (engine.cu:678-692): cia_weights_upload (12
    reader threads, two pinned 64 MiB buffers, each copy overlapping the
    next reads) against the reference's scheme (one pageable 256 MiB
    buffer: read, then a blocking copy).  The synthetic file was just
    written, so both read it from the page cache: host memory to HBM."""
    import tempfile
    import numpy as np
    import torch
    from cuda_inf_amd.model_files import upload_file
    nbytes = mib << 20
    d = tempfile.mkdtemp(prefix="cia_upload_")
    path = os.path.join(d, "weights.bin")
    try:
        block = np.random.default_rng(1).integers(0, 256, 64 << 20, dtype=np.uint8)
        with open(path, "wb") as f:
            for off in range(0, nbytes, block.size):
                f.write(block[:min(block.size, nbytes - off)].tobytes())
        blob = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        ours, theirs = [], []
        buf = np.empty(256 << 20, np.uint8)
        for _ in range(runs):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            upload_file(path, blob)
            ours.append(time.perf_counter() - t0)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            with open(path, "rb", buffering=0) as f:
                off = 0
                while off < nbytes:
                    r = f.readinto(memoryview(buf)[:min(buf.size, nbytes - off)])
                    blob[off:off + r].copy_(torch.from_numpy(buf[:r]))
                    off += r
            torch.cuda.synchronize()
            theirs.append(time.perf_counter() - t0)
        # (the last copy wrote the file's bytes; check the tail chunk)
        tail = min(nbytes, 1 << 20)
        assert torch.equal(blob[nbytes - tail:].cpu(),
                           torch.from_numpy(np.fromfile(path, np.uint8, tail, offset=nbytes - tail)))
    finally:
        try:
            os.remove(path)
        except OSError:
            pass
        os.rmdir(d)
    o, t = float(np.median(ours)), float(np.median(theirs))
    log(f"weights upload {mib} MiB: {nbytes / o / 1e9:.1f} GB/s pinned double-buffered "
        f"({o * 1e3:.0f} ms); one pageable 256 MiB buffer {nbytes / t / 1e9:.1f} GB/s "
        f"({t * 1e3:.0f} ms)")
    return {"mib": mib, "gbps": round(nbytes / o / 1e9, 2), "ms": round(o * 1e3, 1),
            "pageable_256mib_gbps": round(nbytes / t / 1e9, 2),
            "source": "page cache (file just written)"}


def long_context_leg(ctx, nL, steps, dev, stream, log):
    """Decode at ctx tokens (6 layers): the matrix-core path and the
    reference's split + combine with 16, 64, 256 and 512 splits per head.
    Each setting: 2 warm-up tokens, then `steps` timed tokens, then 2 tokens
    with HIP events around each launch (split and combine separately); then
    a plain streaming read of the same FP8 K+V, one launch per layer."""
    import ctypes
    import torch
    from cuda_inf_amd import _lib, workload
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd._lib import D, NH, NKV, call
    settings = [0, 16, 64, 256, 512]
    n_ev = 2
    total = len(settings) * (steps + 2 + n_ev)
    layers = []
    for l in range(nL):
        L = AttnLayer(ctx + total + 64, nsplit=512, device=dev)
        g = workload.generator(2000 + l, dev)
        for c0 in range(0, ctx, 8192):
            n = min(8192, ctx - c0)
            k = workload.with_outliers(workload.normal_f16((n, NKV, D), g, dev), g)
            v = workload.with_outliers(workload.normal_f16((n, NKV, D), g, dev), g)
            call("cia_layer_append", ctypes.byref(L._s), k.data_ptr(), v.data_ptr(), n, c0,
                 stream.cuda_stream)
            torch.cuda.synchronize()
        layers.append(L)
    arr = (_lib.cia_layer * nL)(*[L._s for L in layers])
    g = workload.generator(9, dev)
    pos = torch.arange(ctx, ctx + total, device=dev)
    q = workload.normal_f16((total, nL, NH, D), g, dev)
    q = torch.stack([workload.prep_qk(q[:, l], pos) for l in range(nL)], dim=1).contiguous()
    kk = workload.with_outliers(workload.normal_f16((total, nL, NKV, D), g, dev), g)
    vv = workload.with_outliers(workload.normal_f16((total, nL, NKV, D), g, dev), g)
    out = torch.empty((total, nL, NH, D), dtype=torch.float16, device=dev)
    qrow, krow = nL * NH * D * 2, nL * NKV * D * 2
    cur = 0
    res = {"context": ctx, "layers": nL, "timed_tokens": steps}
    for ns in settings:
        for l in range(nL):
            arr[l].nsplit = ns
        times = []
        for phase, n in (("warm", 2), ("timed", steps)):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            call("cia_decode_loop", arr, nL, q.data_ptr() + cur * qrow, kk.data_ptr() + cur * krow,
                 vv.data_ptr() + cur * krow, out.data_ptr() + cur * qrow, ctx + cur, n, 0.125,
                 None, stream.cuda_stream)
            e1.record(stream)
            torch.cuda.synchronize()
            cur += n
            if phase == "timed":
                times.append(e0.elapsed_time(e1) * 1e3 / n)
        us = times[0]
        Tc = ((ctx + cur) // 64) * 64
        gbps = algo_bytes(Tc, ctx + cur - Tc) * nL / (us * 1e-6) / 1e9
        name = "matrix_core" if ns == 0 else f"split_{ns}"
        res[name] = {"us_per_token": round(us, 2), "gbps": round(gbps, 1)}
        # events before, between (split | combine) and after each layer's launches
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(3 * n_ev * nL)]
        for e in evs:  # the hipEvent_t handles exist once recorded
            e.record(stream)
        torch.cuda.synchronize()
        call("cia_decode_loop", arr, nL, q.data_ptr() + cur * qrow, kk.data_ptr() + cur * krow,
             vv.data_ptr() + cur * krow, out.data_ptr() + cur * qrow, ctx + cur, n_ev, 0.125,
             (ctypes.c_void_p * len(evs))(*[e.cuda_event for e in evs]), stream.cuda_stream)
        torch.cuda.synchronize()
        cur += n_ev
        first = sorted(evs[3 * r].elapsed_time(evs[3 * r + 1]) * 1e3 for r in range(n_ev * nL))
        second = sorted(evs[3 * r + 1].elapsed_time(evs[3 * r + 2]) * 1e3 for r in range(n_ev * nL))
        if ns == 0:
            # one launch per token: the last "before" event (layer nL-1) and
            # the first "after" event (layer 0) bracket the launch alone
            one = sorted(evs[3 * nL * t + 3 * (nL - 1)].elapsed_time(evs[3 * nL * t + 1]) * 1e3
                         for t in range(n_ev))
            res[name]["launch_us_median"] = round(one[len(one) // 2], 2)
            log(f"long context {ctx}: {name}: {us:.1f} us/token, {gbps:.0f} GB/s; "
                f"one launch {one[len(one) // 2]:.1f} us")
        else:
            res[name]["split_us_median"] = round(first[len(first) // 2], 2)
            res[name]["combine_us_median"] = round(second[len(second) // 2], 2)
            log(f"long context {ctx}: {name}: {us:.1f} us/token, {gbps:.0f} GB/s; "
                f"split {first[len(first) // 2]:.1f} us + combine {second[len(second) // 2]:.1f} us "
                f"per layer (event-bracketed)")
    # measured ceiling: the same committed FP8 K+V read plainly
    sink = torch.zeros(1, dtype=torch.int32, device=dev)

    def plain_read(n_tok):
        for _ in range(n_tok):
            for i, L in enumerate(layers):
                call("cia_stream_read", L.kc8.data_ptr(), L.vc8.data_ptr(),
                     arr[i].committed * NKV * D, sink.data_ptr(), stream.cuda_stream)

    plain_read(2)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    plain_read(steps)
    e1.record(stream)
    torch.cuda.synchronize()
    f_us = e0.elapsed_time(e1) * 1e3 / steps
    f_gbps = 2 * arr[0].committed * NKV * D * nL / (f_us * 1e-6) / 1e9
    res["plain_read"] = {"kernel": "k_stream_read", "us_per_token": round(f_us, 2),
                         "gbps": round(f_gbps, 1),
                         "matrix_core_frac": round(res["matrix_core"]["gbps"] / f_gbps, 4)}
    log(f"long context {ctx}: plain read of the same bytes {f_us:.1f} us/token, {f_gbps:.0f} GB/s")
    return res


def h2o_leg(steps, dev, stream, log, C=2048, W=256, P=1024):
    """H2O eviction decode on one layer: a C-slot per-token FP8 buffer,
    window W, a P-token prompt, then `steps` single-token steps through the
    decode loop (slot choice on the device, no host round trip), timed as a
    whole; then 64 more steps with events around the scores launch (which
    also chooses the slot and quantises the token) and the mass launch."""
    import ctypes
    import torch
    from cuda_inf_amd import _lib, workload
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd._lib import D, NH, NKV, call
    extra = 64
    total = P + steps + extra
    L = AttnLayer(total + 64, budget=C, window=W, prompt_len=P, max_batch=P, device=dev)
    g = workload.generator(7, dev)
    q = workload.normal_f16((total, NH, D), g, dev)
    k = workload.normal_f16((total, NKV, D), g, dev)
    v = workload.normal_f16((total, NKV, D), g, dev)
    out = torch.empty((total, NH, D), dtype=torch.float16, device=dev)
    L.forward(q[:P], k[:P], v[:P], 0, out=out[:P], evicted=False)
    torch.cuda.synchronize()
    qrow, krow = NH * D * 2, NKV * D * 2

    def loop(s0, n, events=None):
        call("cia_decode_loop", ctypes.byref(L._s), 1, q.data_ptr() + s0 * qrow,
             k.data_ptr() + s0 * krow, v.data_ptr() + s0 * krow, out.data_ptr() + s0 * qrow,
             s0, n, 0.125, events, stream.cuda_stream)

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    loop(P, steps)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(3 * extra)]
    for e in evs:  # the hipEvent_t handles exist once recorded
        e.record(stream)
    torch.cuda.synchronize()
    ptrs = (ctypes.c_void_p * len(evs))(*[e.cuda_event for e in evs])
    loop(P + steps, extra, ptrs)
    torch.cuda.synchronize()
    scores = sorted(evs[3 * i].elapsed_time(evs[3 * i + 1]) * 1e3 for i in range(extra))
    rest = sorted(evs[3 * i + 1].elapsed_time(evs[3 * i + 2]) * 1e3 for i in range(extra))
    # per step: FP8 K+V and fp16 scales of every live slot, its position
    # and mass (read + write), q in, out written
    step_bytes = C * (2 * NKV * D + 2 * NKV * 2 + 4 + 8) + 2 * NH * D * 2
    res = {"slots": C, "window": W, "prompt": P, "steps": steps, "us_per_step": round(us, 2),
           "gbps": round(step_bytes / (us * 1e-6) / 1e9, 1),
           "scores_place_us_median": round(scores[extra // 2], 2),
           "mass_us_median": round(rest[extra // 2], 2),
           "evictions": steps + extra + P - C,
           "policy": "slot choice and quantisation inside the scores launch (2 launches per "
                     "step, no host round trip)"}
    log(f"h2o C={C} W={W}: {us:.2f} us/step over {steps} steps; scores + placement "
        f"{res['scores_place_us_median']} us, mass {res['mass_us_median']} us (medians)")
    return res


def measured_traffic(ctx: int, nL: int):
    """HBM bytes per decode token from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, copy-kernel scaled) when it was taken on this
    workload; None otherwise."""
    p = os.path.join(os.path.dirname(os.path.abspath(__file__)), TRAFFIC_FILE)
    try:
        with open(p) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("context") != ctx or t.get("layers") != nL:
        return None
    return t.get("bytes_per_token")


def cpu_baseline(L, committed, qpos, q, nL, seconds, log):
    """The oracle's split+combine (16 splits, the reference's launch shape) on
    one layer's cache copied to the host (keys 0..qpos); reported per token of
    nL layers."""
    import numpy as np
    import torch
    import oracle
    ref = oracle.Group64Cache(L.maxT)
    ref.kc8[:] = L.kc8.cpu().numpy()
    ref.vc8[:] = L.vc8.cpu().numpy()
    ref.ksc[:] = L.ksc.cpu().view(torch.int16).numpy().view(np.uint16)
    ref.vsc[:] = L.vsc.cpu().view(torch.int16).numpy().view(np.uint16)
    ref.ktail[:] = L.ktail.cpu().view(torch.int16).numpy().view(np.uint16)
    ref.vtail[:] = L.vtail.cpu().view(torch.int16).numpy().view(np.uint16)
    ref.committed = committed
    qn = q[0, 0].cpu().view(torch.int16).numpy().view(np.uint16)
    res = {}
    ncores = min(os.cpu_count() or 1, 16)
    for threads in (1, ncores):
        n, t0 = 0, time.perf_counter()
        while True:
            oracle.attn_decode(qn, ref, qpos, nsplit=16, nthreads=threads)
            n += 1
            el = time.perf_counter() - t0
            if el > seconds / 2:
                break
        res[threads] = el / n
        log(f"cpu oracle, {threads} thread(s): {el / n * 1e3:.1f} ms per layer ({n} runs)")
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    best = min(res, key=res.get)
    return {"value": round(res[best] * nL * 1e6, 1), "unit": "us/token", "cores": best,
            "kind": "port",
            "sample": f"oracle split+combine (16 splits), one layer at {qpos + 1} keys, "
                      f"x{nL} layers; single-thread {res[1] * nL * 1e6:.0f} us/token; "
                      f"host {model} ({os.cpu_count()} cpus)"}


def _host_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def cpu_prefill_baseline(S, seconds, log):
    """The oracle's causal prefill (append with FP8 commit, then
    attention_fused) for S tokens on one host core.  The append is timed
    whole; the attention on the last query rows until about seconds / 2 have
    passed, scaled to all S rows by (query, key) pairs."""
    import numpy as np
    import oracle
    from cuda_inf_amd import workload
    q, k, v = workload.qkv(S, seed=0, device="cpu")
    qn, kn, vn = (t.view(torch_int16()).numpy().view(np.uint16) for t in (q, k, v))
    ref = oracle.Group64Cache(S + 64)
    t0 = time.perf_counter()
    ref.append(kn, vn, 0)
    t_app = time.perf_counter() - t0
    # the last n rows in one call, n doubled until the call takes a quarter of
    # the budget
    n = 4
    while True:
        rows = list(range(S - n, S))
        t0 = time.perf_counter()
        oracle.attention_fused(qn, ref, S, 0, rows=rows)
        t_att = time.perf_counter() - t0
        if t_att > seconds / 4 or n >= S:
            break
        n = min(2 * n, S)
    pairs = sum(r + 1 for r in rows)
    full_pairs = S * (S + 1) // 2
    att_full = t_att * full_pairs / pairs
    total = t_app + att_full
    log(f"cpu oracle prefill {S}: append {t_app * 1e3:.1f} ms + attention {att_full * 1e3:.0f} ms "
        f"(scaled from {len(rows)} rows), 1 thread")
    return {"value": round(total * 1e6, 1), "unit": "us/prefill", "cores": 1, "kind": "port",
            "sample": f"oracle append of {S} tokens (whole) + attention_fused on the last "
                      f"{len(rows)} query rows, scaled by (query, key) pairs to all {S} rows; "
                      f"host {_host_model()}"}


def tokenizer_leg(log, with_reference, mib=2):
    """Host-side encode throughput of cia_tok_encode on ~2 MiB of synthetic
    text with the synthetic byte-level BPE of tests/golden/tok.  Returns
    (ours, reference): where oracle/_ref/libreftok.so was built (the
    reference's tokenizer.h), the same text through it, for the
    cpu_baseline block."""
    import random
    from cuda_inf_amd.model_files import Tokenizer
    d = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests", "golden", "tok")
    rng = random.Random(3)
    words = ["the", "capital", "of", "France", "is", "Paris", "über", "straße", "中文",
             "don't", "they're", "12345", "3.14", "kato", "rien", "stion", "quai", "(x)", "--"]
    parts, n = [], 0
    while n < mib << 20:
        w = rng.choice(words) + rng.choice([" ", " ", " ", "\n", ", "])
        parts.append(w)
        n += len(w.encode())
    text = "".join(parts).encode()
    t = Tokenizer()
    if not t.load(d):
        return None, None

    def rate(fn):
        best = None
        for _ in range(3):
            t0 = time.perf_counter()
            ids = fn(text)
            el = time.perf_counter() - t0
            best = el if best is None or el < best else best
        return ids, len(text) / best / 1e6
    ids, ours = rate(t.encode)
    res = {"mb": round(len(text) / 1e6, 2), "tokens": len(ids), "mb_per_s": round(ours, 2),
           "threads": 1}
    ref_res = None
    if with_reference:
        from oracle import model_files as om
        if om.RefTokenizer.available():
            ref = om.RefTokenizer(d)
            rids, theirs = rate(ref.encode)
            ref_res = {"value": round(theirs, 2), "unit": "MB/s", "cores": 1,
                       "kind": "reference", "same_ids": rids == ids,
                       "sample": f"{len(text) / 1e6:.1f} MB of synthetic text, synthetic "
                                 f"byte-level BPE vocabulary (tests/golden/tok)"}
    log(f"tokenizer encode: {ours:.1f} MB/s on {len(text) / 1e6:.1f} MB ({len(ids)} tokens)"
        + (f"; the reference's tokenizer.h {ref_res['value']:.1f} MB/s, same ids: "
           f"{ref_res['same_ids']}" if ref_res else ""))
    return res, ref_res


def cpu_h2o_baseline(seconds, log, C=2048, W=256, P=1024):
    """The oracle's H2O layer (slot choice, per-token FP8 write, attention
    with attn_sum) on one host core: a P-token prompt (untimed), then single
    token steps for about seconds / 2."""
    import numpy as np
    import oracle
    from cuda_inf_amd import workload
    n = 4096 + P
    g = workload.generator(7, "cpu")
    q = workload.normal_f16((n, 32, 64), g, "cpu").view(torch_int16()).numpy().view(np.uint16)
    k = workload.normal_f16((n, 8, 64), g, "cpu").view(torch_int16()).numpy().view(np.uint16)
    v = workload.normal_f16((n, 8, 64), g, "cpu").view(torch_int16()).numpy().view(np.uint16)
    hc = oracle.H2OCache(C, W)
    hc.step(q[:P], k[:P], v[:P], 0, want_out=False)
    steps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds / 2 and P + steps < n:
        i = P + steps
        hc.step(q[i:i + 1], k[i:i + 1], v[i:i + 1], i)
        steps += 1
    el = time.perf_counter() - t0
    log(f"cpu oracle h2o C={C} W={W}: {el / steps * 1e6:.0f} us/step over {steps} steps, 1 thread")
    return {"value": round(el / steps * 1e6, 1), "unit": "us/step", "cores": 1, "kind": "port",
            "sample": f"oracle H2O steps {P}..{P + steps - 1} after a {P}-token prompt, "
                      f"{C} slots, window {W}; host {_host_model()}"}


def torch_int16():
    import torch
    return torch.int16


if __name__ == "__main__":
    main()
