"""Child process of test_gpu_split_graph.py (run as a script, one GPU):
the drop-in cia_attn_decode_split + cia_attn_decode_combine captured into a
HIP graph on a fresh stream before this process has made any split call --
so the library's first call on the device happens under capture -- then
replayed with the program's own eager work and synchronisations between
the replays.  Every replay's partials (pm, pl, po) and output equal an eager
call's bit for bit, and so do cia_attn_decode_split_ws's with a caller
workspace.  Geometries: 32808 keys at 16 splits (range mode: the shares of a
split meet in the library's array), 2047 keys at 16 splits and 1500 at 4
(share mode: 2 and 8 workgroups per split), 32808 keys at 64 splits (no
shared splits).  Prints
one line per step; exits non-zero on the first mismatch."""
import ctypes
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402
import torch  # noqa: E402


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int32 if t.dtype == torch.float32
                                              else torch.int16).numpy().copy()


def main():
    from cuda_inf_amd import kernels as K
    from cuda_inf_amd._lib import call
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cases = [(32808, 16, 71), (2047, 16, 72), (1500, 4, 74), (32808, 64, 73)]
    layers = {}
    for ntok, _, seed in cases:
        if ntok in layers:
            continue
        L = AttnLayer(ntok + 64, nsplit=16, device=dev)
        _, k, v = qkv(ntok, seed=seed, device="cpu", outliers=True)
        kd, vd = k.to(dev), v.to(dev)
        call("cia_layer_append", ctypes.byref(L._s), kd.data_ptr(), vd.data_ptr(), ntok, 0,
             torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        layers[ntok] = L
    print("caches built", flush=True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graphs = []
    for ntok, ns, seed in cases:
        L = layers[ntok]
        qpos = ntok - 1
        q, _, _ = qkv(1, seed=seed + 100, device="cpu", past=qpos)
        qd = q.to(dev)
        bufs = {n: torch.full((32 * ns * (64 if n == "po" else 1),), float("nan"),
                              dtype=torch.float32, device=dev) for n in ("pm", "pl", "po")}
        out = torch.zeros((32, 64), dtype=torch.float16, device=dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            K.attn_decode_split(qd, L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed,
                                qpos, 0.125, bufs["pm"], bufs["pl"], bufs["po"], ns)
            K.attn_decode_combine(bufs["pm"], bufs["pl"], bufs["po"], out, ns)
        torch.cuda.synchronize()
        graphs.append((ntok, ns, qd, qpos, g, bufs, out))
        print(f"captured {ntok} keys / {ns} splits", flush=True)
    ws = torch.zeros(K.split_workspace_bytes(16), dtype=torch.uint8, device=dev)
    for ntok, ns, qd, qpos, g, bufs, out in graphs:
        L = layers[ntok]
        # the eager references: the drop-in entry, then the workspace entry
        ref = {n: torch.empty_like(b) for n, b in bufs.items()}
        ref_out = torch.empty_like(out)
        K.attn_decode_split(qd, L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed, qpos,
                            0.125, ref["pm"], ref["pl"], ref["po"], ns)
        K.attn_decode_combine(ref["pm"], ref["pl"], ref["po"], ref_out, ns)
        wsb = {n: torch.empty_like(b) for n, b in bufs.items()}
        ws_out = torch.empty_like(out)
        K.attn_decode_split(qd, L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed, qpos,
                            0.125, wsb["pm"], wsb["pl"], wsb["po"], ns, ws=ws)
        K.attn_decode_combine(wsb["pm"], wsb["pl"], wsb["po"], ws_out, ns)
        torch.cuda.synchronize()
        for n in ref:
            if not np.array_equal(bits(wsb[n]), bits(ref[n])):
                sys.exit(f"{ntok}/{ns}: workspace entry's {n} differs from the drop-in's")
        if not np.array_equal(bits(ws_out), bits(ref_out)):
            sys.exit(f"{ntok}/{ns}: workspace entry's output differs")
        for r in range(3):
            for b in bufs.values():
                b.fill_(float("nan"))
            out.zero_()
            # the program's own eager work between replays (another geometry)
            o_ntok, o_ns = (2047, 16) if ntok != 2047 else (32808, 16)
            Lo = layers[o_ntok]
            tmp = {n: torch.empty(32 * o_ns * (64 if n == "po" else 1), dtype=torch.float32,
                                  device=dev) for n in ("pm", "pl", "po")}
            K.attn_decode_split(graphs[0][2], Lo.kc8, Lo.vc8, Lo.ksc, Lo.vsc, Lo.ktail, Lo.vtail,
                                Lo.committed, o_ntok - 1, 0.125, tmp["pm"], tmp["pl"], tmp["po"],
                                o_ns)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            for n in ref:
                if not np.array_equal(bits(bufs[n]), bits(ref[n])):
                    sys.exit(f"{ntok}/{ns} replay {r}: {n} differs from the eager call")
            if not np.array_equal(bits(out), bits(ref_out)):
                sys.exit(f"{ntok}/{ns} replay {r}: output differs from the eager call")
            print(f"{ntok} keys / {ns} splits: replay {r} bit-identical", flush=True)
    print("split capture ok", flush=True)


if __name__ == "__main__":
    main()
