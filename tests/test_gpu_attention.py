"""GPU parity of the attention kernels against the oracle (tolerance
2e-3 abs + 1e-3 rel of the fp32 oracle output).

Flash-decoding split/combine (engine.cu:396-480), the matrix-core decode, and
attention_fused (engine.cu:236-308) on the group-64 FP8 cache.
"""
import numpy as np
import pytest
import torch

from conftest import assert_close_f16

pytestmark = pytest.mark.gpu


def _u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _build(dev, orc, ntok, seed, outliers=False, nsplit=16):
    """Cache holding ntok tokens (positions 0..ntok-1), built identically on
    the GPU (AttnLayer's append loop) and in the oracle."""
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    L = AttnLayer(ntok + 64, nsplit=nsplit, device=dev)
    ref = orc.Group64Cache(ntok + 64)
    q, k, v = qkv(ntok, seed=seed, device="cpu", outliers=outliers)
    kd, vd = k.to(dev), v.to(dev)
    # append without attention: plan on host and run the writers
    from cuda_inf_amd import kernels as K
    from cuda_inf_amd.layer import kv_append_plan
    ops, c = kv_append_plan(0, ntok, 0)
    for op in ops:
        s0 = op["src_token"]
        K.kv_write_tail(kd[s0:], vd[s0:], L.ktail, L.vtail, op["slot"], op["cnt"])
        if op["commit"]:
            K.kv_commit_group(L.ktail, L.vtail, L.kc8, L.vc8, L.ksc, L.vsc, op["commit_base"],
                              op["commit_grp"])
    L._s.committed = c
    ref.append(_u16(k), _u16(v), 0)
    assert ref.committed == c
    return L, ref, q


def _decode_q(seed, qpos):
    from cuda_inf_amd.workload import qkv
    q, _, _ = qkv(1, seed=seed, device="cpu", past=qpos)
    return q


def test_decode_config0(orc, cia, dev):
    """31 committed groups + 48-token tail (2032 keys), nsplit 16."""
    from cuda_inf_amd import kernels as K
    L, ref, _ = _build(dev, orc, 2032, seed=0)
    assert L.committed == 1984
    q = _decode_q(1, 2031)
    out = torch.empty((32, 64), dtype=torch.float16, device=dev)
    K.attn_decode_split(q.to(dev), L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, 1984, 2031, 0.125,
                        L.pm, L.pl, L.po, 16)
    K.attn_decode_combine(L.pm, L.pl, L.po, out, 16)
    torch.cuda.synchronize()
    _, r32, (pm, pl, po) = orc.attn_decode(_u16(q), ref, 2031, nsplit=16)
    assert_close_f16(_u16(out), r32)
    # partials: same split ranges as the reference
    gm = L.pm.cpu().numpy()
    np.testing.assert_allclose(gm, pm, rtol=0, atol=1e-4)
    np.testing.assert_allclose(L.pl.cpu().numpy(), pl, rtol=2e-4)
    np.testing.assert_allclose(L.po.cpu().numpy().reshape(po.shape), po, rtol=2e-3, atol=2e-3)
    # and the fused prefill's last row on the same cache gives the same answer
    f16, f32 = orc.attention_fused(_u16(q), ref, 1, 2031)
    np.testing.assert_allclose(f32[0], r32, atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("nsplit", [1, 16, 64, 256, 512, 4096])
def test_decode_nsplit_sweep(orc, cia, dev, nsplit):
    from cuda_inf_amd import kernels as K
    L, ref, _ = _build(dev, orc, 1000, seed=3, outliers=True)
    q = _decode_q(4, 999)
    pm = torch.zeros(32 * nsplit, device=dev)
    pl = torch.zeros(32 * nsplit, device=dev)
    po = torch.zeros(32 * nsplit * 64, device=dev)
    out = torch.empty((32, 64), dtype=torch.float16, device=dev)
    K.attn_decode_split(q.to(dev), L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed, 999,
                        0.125, pm, pl, po, nsplit)
    K.attn_decode_combine(pm, pl, po, out, nsplit)
    torch.cuda.synchronize()
    _, r32, (rpm, rpl, _) = orc.attn_decode(_u16(q), ref, 999, nsplit=nsplit, nthreads=8)
    assert_close_f16(_u16(out), r32)
    # empty splits: l == 0 and m == -1e30 exactly where the oracle has them
    empty = rpl == 0
    assert np.array_equal(pl.cpu().numpy() == 0, empty)
    assert np.all(pm.cpu().numpy()[empty] == np.float32(-1e30))


# 65540 and 131080 keys: 2 and 4 pairs per wave; below 32768 keys a wave
# has at most one pair (33000: a few waves take two)
@pytest.mark.parametrize("ntok", [1, 63, 64, 65, 127, 128, 129, 255, 256, 257, 2032, 5000, 33000,
                                  65540, 131080])
def test_decode_matrix_cores(orc, cia, dev, ntok):
    from cuda_inf_amd import kernels as K
    L, ref, _ = _build(dev, orc, ntok, seed=ntok, outliers=True)
    ws = K.new_decode_workspace(ntok, dev)
    q = _decode_q(ntok + 1, ntok - 1)
    _, r32, _ = orc.attn_decode(_u16(q), ref, ntok - 1, nsplit=16, nthreads=8)
    for rep in range(3):  # repeated calls reuse the workspace
        out = torch.empty((32, 64), dtype=torch.float16, device=dev)
        K.attn_decode(q.to(dev), L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed,
                      ntok - 1, 0.125, out, ws)
        torch.cuda.synchronize()
        assert_close_f16(_u16(out), r32, what=f"rep {rep}")


@pytest.mark.parametrize("S,past", [(1, 0), (333, 0), (64, 0), (50, 100), (130, 64), (700, 0)])
def test_attention_fused(orc, cia, dev, S, past):
    """Prefill through the layer driver (append, then fused attention)."""
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    L = AttnLayer(past + S + 64, nsplit=16, device=dev)
    ref = orc.Group64Cache(past + S + 64)
    if past:
        q0, k0, v0 = qkv(past, seed=7, device="cpu")
        L.forward(q0.to(dev), k0.to(dev), v0.to(dev), 0)
        ref.append(_u16(k0), _u16(v0), 0)
    q, k, v = qkv(S, seed=8, device="cpu", past=past)
    out, _ = L.forward(q.to(dev), k.to(dev), v.to(dev), past)
    ref.append(_u16(k), _u16(v), past)
    torch.cuda.synchronize()
    if S == 1:
        _, r32, _ = orc.attn_decode(_u16(q), ref, past, nsplit=16)
        r32 = r32[None]
    else:
        _, r32 = orc.attention_fused(_u16(q), ref, S, past)
    assert_close_f16(_u16(out), r32)


@pytest.mark.parametrize("S,past,outliers,zero_group", [
    (2, 0, False, False), (63, 0, False, False), (65, 0, True, False), (128, 0, False, True),
    (200, 1000, True, False), (17, 4079, False, False), (1000, 37, True, True),
    (4096, 0, True, False)])
def test_prefill_matrix_cores(orc, cia, dev, S, past, outliers, zero_group):
    """The matrix-core causal prefill (attention_fused): blocks of 64 queries,
    heavy/light block pairs, FP8 groups plus the fp16 tail, lazily moved
    running max; a K/V group of zeros has scale 0.  Every query row and
    head is checked (the 4096-row case against the oracle run on the host's
    cores)."""
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    L = AttnLayer(past + S + 64, nsplit=16, device=dev)
    ref = orc.Group64Cache(past + S + 64)
    if past:
        q0, k0, v0 = qkv(past, seed=11, device="cpu", outliers=outliers)
        if zero_group and past >= 128:
            k0[64:128] = 0
            v0[64:128] = 0
        L.forward(q0.to(dev), k0.to(dev), v0.to(dev), 0)
        ref.append(_u16(k0), _u16(v0), 0)
    q, k, v = qkv(S, seed=12, device="cpu", past=past, outliers=outliers)
    if zero_group and not past:
        k[64:128] = 0
        v[64:128] = 0
    out, _ = L.forward(q.to(dev), k.to(dev), v.to(dev), past)
    ref.append(_u16(k), _u16(v), past)
    torch.cuda.synchronize()
    import os
    nth = max(1, min(16, os.cpu_count() or 1))
    _, r32 = orc.attention_fused_mt(_u16(q), ref, S, past, nthreads=nth)
    assert_close_f16(_u16(out), r32)


def test_decode_steps_through_commit(orc, cia, dev):
    """Decode steps that cross a group boundary (tail fills, commit, new tail)."""
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    n0 = 4000
    L = AttnLayer(n0 + 200, nsplit=0, device=dev)  # matrix-core decode, fused tail write
    ref = orc.Group64Cache(n0 + 200)
    q0, k0, v0 = qkv(n0, seed=11, device="cpu", outliers=True)
    L.forward(q0.to(dev), k0.to(dev), v0.to(dev), 0)
    ref.append(_u16(k0), _u16(v0), 0)
    for step in range(100):
        pos = n0 + step
        q, k, v = qkv(1, seed=1000 + step, device="cpu", past=pos, outliers=True)
        out, _ = L.forward(q.to(dev), k.to(dev), v.to(dev), pos)
        ref.append(_u16(k), _u16(v), pos)
        if step % 9 == 0 or pos % 64 in (62, 63, 0, 1):
            torch.cuda.synchronize()
            _, r32, _ = orc.attn_decode(_u16(q), ref, pos, nsplit=16, nthreads=8)
            assert_close_f16(_u16(out)[0], r32, what=f"step {step} pos {pos}")
    assert L.committed == ref.committed
    # the groups committed inside the decode launches are the reference's bytes
    c = ref.committed
    assert np.array_equal(L.kc8[:c].cpu().numpy().reshape(ref.kc8[:c].shape), ref.kc8[:c])
    assert np.array_equal(L.vc8[:c].cpu().numpy().reshape(ref.vc8[:c].shape), ref.vc8[:c])
    ng = c // 64
    assert np.array_equal(_u16(L.ksc).reshape(-1, 8)[:ng], ref.ksc[:ng])
    assert np.array_equal(_u16(L.vsc).reshape(-1, 8)[:ng], ref.vsc[:ng])
    assert np.array_equal(_u16(L.ktail).reshape(ref.ktail.shape), ref.ktail)
    assert np.array_equal(_u16(L.vtail).reshape(ref.vtail.shape), ref.vtail)


def test_decode_loop_two_layers_through_commit(orc, cia, dev):
    """cia_decode_loop (the bench's entry): 2 layers x 70 steps from 1990
    tokens, crossing a group boundary; every 7th step and the commit steps are
    checked against the oracle, then the caches byte for byte."""
    import ctypes
    from cuda_inf_amd import _lib
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    nL, n0, steps = 2, 1990, 70
    layers, refs = [], []
    for l in range(nL):
        L = AttnLayer(n0 + steps + 64, nsplit=0, device=dev)
        ref = orc.Group64Cache(n0 + steps + 64)
        _, k0, v0 = qkv(n0, seed=20 + l, device="cpu", outliers=True)
        k0d, v0d = k0.to(dev), v0.to(dev)  # alive until the append has run
        _lib.call("cia_layer_append", ctypes.byref(L._s), k0d.data_ptr(), v0d.data_ptr(), n0, 0,
                  torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        ref.append(_u16(k0), _u16(v0), 0)
        layers.append(L)
        refs.append(ref)
    torch.cuda.synchronize()
    arr = (_lib.cia_layer * nL)(*[L._s for L in layers])
    qs, ks, vs = [], [], []
    for s in range(steps):
        row = [qkv(1, seed=5000 + 10 * s + l, device="cpu", past=n0 + s, outliers=True)
               for l in range(nL)]
        qs.append(torch.cat([r[0] for r in row]))
        ks.append(torch.cat([r[1] for r in row]))
        vs.append(torch.cat([r[2] for r in row]))
    q = torch.stack(qs).contiguous()       # [steps, nL, 32, 64]
    k = torch.stack(ks).contiguous()       # [steps, nL, 8, 64]
    v = torch.stack(vs).contiguous()
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    out = torch.empty_like(qd)
    # three eager calls, with other work and a synchronisation between them
    qrow, krow = nL * 32 * 64 * 2, nL * 8 * 64 * 2
    s0 = 0
    for n in (25, 20, 25):
        _lib.call("cia_decode_loop", arr, nL, qd.data_ptr() + s0 * qrow, kd.data_ptr() + s0 * krow,
                  vd.data_ptr() + s0 * krow, out.data_ptr() + s0 * qrow, n0 + s0, n, 0.125, None,
                  torch.cuda.current_stream().cuda_stream)
        (qd.float() * 2).sum().item()
        torch.cuda.synchronize()
        s0 += n
    assert s0 == steps
    got = _u16(out)
    for s in range(steps):
        pos = n0 + s
        for l in range(nL):
            refs[l].append(_u16(k[s, l][None]), _u16(v[s, l][None]), pos)
            if s % 7 == 0 or pos % 64 in (62, 63, 0):
                _, r32, _ = orc.attn_decode(_u16(q[s, l][None]), refs[l], pos, nsplit=16, nthreads=8)
                assert_close_f16(got[s, l], r32, what=f"step {s} layer {l}")
    for l in range(nL):
        c = refs[l].committed
        assert arr[l].committed == c
        L = layers[l]
        assert np.array_equal(L.kc8[:c].cpu().numpy(), refs[l].kc8[:c])
        assert np.array_equal(L.vc8[:c].cpu().numpy(), refs[l].vc8[:c])
        assert np.array_equal(_u16(L.ksc)[:c // 64], refs[l].ksc[:c // 64])
        assert np.array_equal(_u16(L.vsc)[:c // 64], refs[l].vsc[:c // 64])
        assert np.array_equal(_u16(L.ktail), refs[l].ktail)


@pytest.mark.parametrize("S,past,outliers", [(2, 0, False), (65, 0, True), (200, 1000, True),
                                             (17, 4079, False), (1000, 37, True), (4096, 0, True)])
def test_prefill_fp8_error(orc, cia, dev, S, past, outliers):
    """The OCP-fp8 matrix-core prefill on the same cache as the fp16 kernel:
    its error against the fp32 restatement, with Q and the softmax
    numerators rounded to fp8, is printed and bounded at about twice the
    measured error of its input class (measured on MI355X: without outliers
    max 0.0012, mean 6e-5; with outliers max 0.042, mean 3e-4); the fp16
    kernel's output of the same layer stays within 2e-3 + 1e-3|ref|."""
    from cuda_inf_amd import kernels as K
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    L = AttnLayer(past + S + 64, nsplit=16, device=dev)
    ref = orc.Group64Cache(past + S + 64)
    if past:
        q0, k0, v0 = qkv(past, seed=11, device="cpu", outliers=outliers)
        L.forward(q0.to(dev), k0.to(dev), v0.to(dev), 0)
        ref.append(_u16(k0), _u16(v0), 0)
    q, k, v = qkv(S, seed=12, device="cpu", past=past, outliers=outliers)
    qd = q.to(dev)
    out16, _ = L.forward(qd, k.to(dev), v.to(dev), past)
    ref.append(_u16(k), _u16(v), past)
    out8 = torch.empty_like(qd)
    print(f"prefill fp8 S={S} past={past}", flush=True)
    K.attention_fused_fp8(qd, L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed, out8, S,
                          past, 0.125)
    torch.cuda.synchronize()
    rows = None
    if S > 1200:
        rows = np.unique(np.concatenate([np.arange(0, 70), np.arange(S - 70, S),
                                         np.arange(0, S, 37)])).astype(np.int32)
    _, r32 = orc.attention_fused(_u16(q), ref, S, past, rows=rows)
    got = out8.float().cpu().numpy()
    g16 = _u16(out16)
    if rows is not None:
        got, r32, g16 = got[rows], r32[rows], g16[rows]
    assert_close_f16(g16, r32, what="fp16 prefill")
    err = np.abs(got - r32)
    print(f"fp8 prefill S={S} past={past}: max abs err {err.max():.4g}, mean {err.mean():.4g}, "
          f"max rel {(err / (np.abs(r32) + 1e-3)).max():.3g}")
    assert np.isfinite(got).all()
    max_bound, mean_bound = (0.08, 7e-4) if outliers else (0.003, 2e-4)
    assert err.max() <= max_bound and err.mean() <= mean_bound
