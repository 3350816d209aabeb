"""The decode entries under HIP graph capture: cia_attn_decode_noalloc (the
entry for callers that cannot allocate, e.g. code under capture) and
cia_attn_decode with its workspace, each captured once and replayed several
times with the program's own eager work and synchronisations between the
replays; every replay bit-identical to the eager result.  Then the decode
loop (fresh-token tail writes fused in) over 2 layers, captured and
replayed from the same cache bytes (restored before each replay: the loop
commits a group on its 4th step, from tail rows that its later steps
overwrite), each replay's outputs and cache bytes equal to the eager
loop's bit for bit."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _layer(dev, ntok, seed):
    """A layer holding ntok tokens (positions 0..ntok-1) through the append."""
    from cuda_inf_amd._lib import call
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    L = AttnLayer(ntok + 64, nsplit=0, device=dev)
    _, k, v = qkv(ntok, seed=seed, device="cpu", outliers=True)
    kd, vd = k.to(dev), v.to(dev)
    call("cia_layer_append", ctypes.byref(L._s), kd.data_ptr(), vd.data_ptr(), ntok, 0,
         torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return L


def test_decode_entries_replay_bit_identical(orc, cia, dev):
    from cuda_inf_amd import kernels as K
    from cuda_inf_amd.workload import qkv
    ntok = 33000
    L = _layer(dev, ntok, 41)
    qpos = ntok - 1
    q, _, _ = qkv(1, seed=42, device="cpu", past=qpos)
    qd = q.to(dev)
    ws = K.new_decode_workspace(ntok, dev)
    ref = torch.empty((32, 64), dtype=torch.float16, device=dev)
    # eager: both entries (the first noalloc call on a device sets up its scratch)
    K.attn_decode(qd, L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed, qpos, 0.125,
                  ref, ws)
    tmp = torch.empty_like(ref)
    K.attn_decode_noalloc(qd, L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed, qpos,
                          0.125, tmp)
    torch.cuda.synchronize()
    assert np.array_equal(_u16(tmp), _u16(ref))
    out_na = torch.empty_like(ref)
    out_ws = torch.empty_like(ref)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g_na, g_ws = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_na, stream=s):
        K.attn_decode_noalloc(qd, L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed,
                              qpos, 0.125, out_na)
    with torch.cuda.graph(g_ws, stream=s):
        K.attn_decode(qd, L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed, qpos, 0.125,
                      out_ws, ws)
    torch.cuda.synchronize()
    for r in range(4):
        out_na.zero_()
        out_ws.zero_()
        # the program's own eager work between replays
        K.attn_decode(qd, L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed, qpos, 0.125,
                      tmp, ws)
        torch.cuda.synchronize()
        assert np.array_equal(_u16(tmp), _u16(ref)), f"eager call {r}"
        print(f"graph replay {r}", flush=True)
        g_na.replay()
        g_ws.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_u16(out_na), _u16(ref)), f"noalloc replay {r}"
        assert np.array_equal(_u16(out_ws), _u16(ref)), f"workspace replay {r}"


def test_decode_loop_replay_bit_identical(orc, cia, dev):
    from cuda_inf_amd import _lib
    from cuda_inf_amd._lib import call
    from cuda_inf_amd.workload import qkv
    ctx, nL, steps = 4096 + 60, 2, 8  # the group completes on the 4th step
    names = ("kc8", "vc8", "ksc", "vsc", "ktail", "vtail")
    pair = []
    for copy in range(2):
        layers = [_layer(dev, ctx, 60 + l) for l in range(nL)]
        pair.append((layers, (_lib.cia_layer * nL)(*[L._s for L in layers])))
    # copy 1's cache bytes before the loop, restored before each replay
    saved = [{n: getattr(L, n).clone() for n in names} for L in pair[1][0]]
    qs, ks, vs = [], [], []
    for i in range(steps):
        for l in range(nL):
            q, k, v = qkv(1, seed=1000 + 10 * i + l, device="cpu", past=ctx + i)
            qs.append(q)
            ks.append(k)
            vs.append(v)
    q = torch.cat(qs).to(dev).contiguous()
    k = torch.cat(ks).to(dev).contiguous()
    v = torch.cat(vs).to(dev).contiguous()
    out_e = torch.empty((steps * nL, 32, 64), dtype=torch.float16, device=dev)
    out_g = torch.zeros_like(out_e)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())

    def loop(arr, out, stream):
        st = call("cia_decode_loop", arr, nL, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                  out.data_ptr(), ctx, steps, 0.125, None, stream.cuda_stream)
        return st

    with torch.cuda.stream(s):
        loop(pair[0][1], out_e, s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        loop(pair[1][1], out_g, s)
    torch.cuda.synchronize()
    for r in range(3):
        out_g.zero_()
        for L, sv in zip(pair[1][0], saved):
            for n in names:
                getattr(L, n).copy_(sv[n])
        torch.cuda.synchronize()
        print(f"loop replay {r}", flush=True)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_u16(out_g), _u16(out_e)), f"loop replay {r}"
        # the cache bytes the replay wrote equal the eager loop's
        for la, lb in zip(pair[0][0], pair[1][0]):
            assert la.committed == lb.committed
            for n in names:
                assert torch.equal(getattr(la, n), getattr(lb, n)), (r, n)
