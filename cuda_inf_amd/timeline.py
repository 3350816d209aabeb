"""Per-wave timeline of the one-launch decode (k_decode_tok) at the bench's
decode workload: 6 layers, 32 768 tokens of context, fresh tokens appended
one per step.  Uses the timestamp build (make -C cuda_inf_amd/csrc
TIMELINE=1 -> libcuda_inf_attn_tl.so); each token's launch is synchronised
and its stamps read back (s_memrealtime, 100 MHz), then medians over the
tokens of each event's time since the launch's first wave started.

    python -m cuda_inf_amd.timeline [--ctx 32768] [--layers 6] [--tokens 32]
    python -m cuda_inf_amd.timeline --run 32 [--tokens 8]

With --run N, each sample is one launch of a run of N tokens from a group
boundary (N <= 63: no commit inside), and the stamps read back are the
run's last token's (each token overwrites the one before); times are then
from that token's first layer open.  A filler call completes the group
between samples.

Printed per layer: the FP8 waves' "opened" (B1 passed), first unit's K
landed, V landed, units done, partials-in-LDS (B2) and the next layer's K
and V sent; the merge waves'
partial acknowledged, ticket, final rows fetched (last arrivers) and output
counted; the control wave's wait begun and q loaded; range 0's tail waves'
rows landed and tail done.  Each as median / max over waves (median over
tokens), in microseconds.
"""
from __future__ import annotations

import argparse
import ctypes
import statistics as st


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--layers", type=int, default=6)
    ap.add_argument("--tokens", type=int, default=32)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prep", action="store_true",
                    help="raw q / k: the QK producers run inside the kernel")
    ap.add_argument("--run", type=int, default=0,
                    help="tokens per launch (one run per sample, 2..63); 0: one launch per token")
    a = ap.parse_args()
    if a.run and not (2 <= a.run <= 63 and a.ctx % 64 == 0 and not a.prep):
        ap.error("--run needs 2 <= N <= 63, a context that is a multiple of 64 and no --prep")
    from cuda_inf_amd import _lib
    _lib.use_timeline_build()
    import numpy as np
    import torch
    from cuda_inf_amd import workload
    from cuda_inf_amd._lib import D, NH, NKV, call
    from cuda_inf_amd.layer import AttnLayer
    lib = _lib.lib()
    lib.cia_timeline_read.restype = ctypes.c_int
    lib.cia_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    dev = torch.device("cuda:0")
    s = torch.cuda.current_stream()
    nL, ctx = a.layers, a.ctx
    n = a.warmup + a.tokens
    if a.run:
        a.warmup = min(a.warmup, 2)
        n = 64 * (a.warmup + a.tokens)
    layers = []
    for l in range(nL):
        L = AttnLayer(ctx + n + 64, nsplit=0, device=dev)
        g = workload.generator(1000 + l, dev)
        for c0 in range(0, ctx, 8192):
            m = min(8192, ctx - c0)
            k = workload.with_outliers(workload.normal_f16((m, NKV, D), g, dev), g)
            v = workload.with_outliers(workload.normal_f16((m, NKV, D), g, dev), g)
            call("cia_layer_append", ctypes.byref(L._s), k.data_ptr(), v.data_ptr(), m, c0,
                 s.cuda_stream)
        layers.append(L)
    torch.cuda.synchronize()
    arr = (_lib.cia_layer * nL)(*[L._s for L in layers])
    keep = []
    if a.prep:
        g8 = workload.generator(17, dev)
        qw = (1.0 + 0.1 * torch.randn(D, generator=g8, device=dev)).to(torch.float16)
        kw = (1.0 + 0.1 * torch.randn(D, generator=g8, device=dev)).to(torch.float16)
        keep += [qw, kw]
        for l in range(nL):
            pw = torch.zeros((NH + NKV) * D, dtype=torch.float16, device=dev)
            keep.append(pw)
            arr[l].qw, arr[l].kw = qw.data_ptr(), kw.data_ptr()
            arr[l].eps, arr[l].theta = workload.EPS, workload.ROPE_THETA
            arr[l].prep_ws, arr[l].prep_cap = pw.data_ptr(), 1
    g = workload.generator(7, dev)
    pos = torch.arange(ctx, ctx + n, device=dev)
    q = workload.normal_f16((n, nL, NH, D), g, dev)
    q = torch.stack([workload.prep_qk(q[:, l], pos) for l in range(nL)], dim=1).contiguous()
    kk = workload.with_outliers(workload.normal_f16((n, nL, NKV, D), g, dev), g)
    vv = workload.with_outliers(workload.normal_f16((n, nL, NKV, D), g, dev), g)
    out = torch.empty((n, nL, NH, D), dtype=torch.float16, device=dev)
    nwg_max, nw = 8 * 44, 13
    buf = np.zeros(nwg_max * nw * 64, np.uint32)
    qrow, krow = nL * NH * D * 2, nL * NKV * D * 2
    samples = []

    def decode(i, steps):
        call("cia_decode_loop", arr, nL, q.data_ptr() + i * qrow, kk.data_ptr() + i * krow,
             vv.data_ptr() + i * krow, out.data_ptr() + i * qrow, ctx + i, steps, 0.125, None,
             s.cuda_stream)
        torch.cuda.synchronize()

    for i in (range(0, n, 64) if a.run else range(n)):
        decode(i, a.run if a.run else 1)
        if i >= (64 if a.run else 1) * a.warmup:
            _lib.check("cia_timeline_read", lib.cia_timeline_read(buf.ctypes.data, buf.nbytes))
            samples.append(buf.reshape(nwg_max, nw, 64).copy())
        if a.run:
            decode(i + a.run, 64 - a.run)  # (the rest of the group and its commit)
    ng = ctx // 64
    R = min(32, ((ng + 15) // 16 + 1) // 2 * 2)
    nwg = 8 * R
    f = ctypes.c_int(-1)
    call("cia_decode_fault", layers[0].ws_decode.data_ptr(), layers[0].ws_decode.numel(),
         ctypes.byref(f))
    print(f"timeline: ctx {ctx}, {nL} layers, {len(samples)} "
          f"{f'runs of {a.run} tokens (their last token)' if a.run else 'tokens'}, {nwg} workgroups; "
          f"fault word {f.value}")

    def rel(x, t0):
        # signed, in us (the counter wraps at 2^32 ticks of 10 ns)
        return (((x.astype(np.int64) - t0 + (1 << 31)) % (1 << 32)) - (1 << 31)) / 100.0

    def start(tl):
        # the launch's first wave, or in a run the last token's first open
        return int(tl[:, :8, 0].min()) if a.run else int(tl[:, :8, 63].min())

    rows = []
    for smp in samples:
        tl = smp[:nwg]
        t0 = start(tl)
        res = {}
        if not a.run:
            res[(0, "workgroup started")] = rel(tl[:, 0, 63], t0)
        for li in range(nL):
            b = 8 * li
            fp8 = rel(tl[:, :8, b:b + 5], t0)            # [wg][wave][5]
            mw = rel(tl[:, 9:13, b:b + 6], t0)           # merge waves
            ctl = rel(tl[:, 12, b + 6:b + 8], t0)        # control
            res[(li, "fp8 opened")] = fp8[:, :, 0]
            res[(li, "fp8 K landed")] = fp8[:, :, 1]
            res[(li, "fp8 V landed")] = fp8[:, :, 2]
            res[(li, "fp8 units done")] = fp8[:, :, 3]
            res[(li, "partials in LDS")] = fp8[:, :, 4]
            if li + 1 < nL:
                nx = rel(tl[:, :8, b + 5:b + 7], t0)
                res[(li, "fp8: next K sent")] = nx[:, :, 0]
                res[(li, "fp8: next V sent")] = nx[:, :, 1]
            res[(li, "merge: partial acked")] = mw[:, :, 2]
            res[(li, "merge: ticket")] = mw[:, :, 3]
            last = tl[:, 9:13, b + 4] != 0
            if a.run:  # (a last arriver of an earlier token of the run keeps its stamps)
                last &= rel(tl[:, 9:13, b + 4], t0) > -2.0
            res[(li, "merge: final rows (last)")] = mw[:, :, 4][last] if last.any() else np.zeros(1)
            res[(li, "merge: output counted (last)")] = mw[:, :, 5][last] if last.any() else np.zeros(1)
            if li > 0 or a.run:
                res[(li, "control: wait begun")] = ctl[:, 0]
            res[(li, "control: q loaded")] = ctl[:, 1]
            # range 0's tail waves (8-11): rows landed, tail done
            r0 = [x for x in range(nwg) if (x & 7) < 4 and (x >> 3) < 2] if R > 1 else list(range(nwg))
            tw = rel(tl[r0][:, 8:12, b + 6:b + 8], t0)
            res[(li, "tail: rows landed")] = tw[:, :, 0]
            res[(li, "tail: done")] = tw[:, :, 1]
        rows.append(res)
        buf[:] = 0
    # the workgroup that reached "partials in LDS" last in each layer of
    # the last token, with its waves' stamps of that layer
    tl = samples[-1][:nwg]
    t0 = start(tl)
    for li in range(nL):
        b = 8 * li
        b2 = rel(tl[:, :8, b + 4], t0).max(axis=1)
        wg = int(np.argmax(b2))
        print(f"  layer {li}: last workgroup to B2: {wg} (xcd {wg % 8}, slot {wg // 8}) at "
              f"{b2[wg]:.2f}; its waves (stamps 0..7 of the layer):")
        for w in range(13):
            st_ = rel(tl[wg, w, b:b + 8], t0)
            st_[tl[wg, w, b:b + 8] == 0] = np.nan
            print(f"    wave {w:2d}: " + " ".join(f"{x:7.2f}" for x in st_))
    # how often the last workgroup to B2 of layer li held a final merge of
    # layer li - 1 (its merge waves' stamp 4 set), and how much later the
    # final mergers' latest B2 is than the others' (medians over tokens)
    hits, tot, gap = 0, 0, []
    for smp in samples:
        tl = smp[:nwg]
        t0 = start(tl)
        for li in range(1, nL):
            b2 = rel(tl[:, :8, 8 * li + 4], t0).max(axis=1)
            fm = (tl[:, 9:13, 8 * (li - 1) + 4] != 0).any(axis=1)
            hits += int(fm[int(np.argmax(b2))])
            tot += 1
            if fm.any() and (~fm).any():
                gap.append(float(b2[fm].max() - b2[~fm].max()))
    if gap:
        print(f"  last workgroup to B2 held a final merge of the layer before in {hits}/{tot} layers; "
              f"final mergers' latest B2 - the others' latest: {np.median(gap):.2f} us")
    keys = list(rows[0].keys())
    for key in keys:
        med = st.median(float(np.median(r[key])) for r in rows)
        mx = st.median(float(np.max(r[key])) for r in rows)
        print(f"  layer {key[0]}  {key[1]:32s} median {med:7.2f}  max {mx:7.2f}")


if __name__ == "__main__":
    main()
