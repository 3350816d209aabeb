"""Parity at the benchmark's sizes and on the remaining entry-point options:

- attention_fused with attn_sum (engine.cu:291-307): the accumulated mass bit
  for bit against the oracle (S > 1, past > 0, a tail, outliers, a non-zero
  starting attn_sum);
- cia_decode_loop at 32 768 keys, 2 layers, across the group boundary at
  32 768: every step's output within tolerance and the committed group and
  tail bytes identical, once with prepared q/k and once with the QK
  producers inside the decode kernel;
- the reference's split + combine at 131 072 keys, 16, 64, 256 and 512
  splits (the benchmark's sweep): the output and the partials;
- one 4096-token append: every committed byte and scale and the tail.
"""
import ctypes

import numpy as np
import pytest
import torch

from conftest import assert_close_f16

pytestmark = pytest.mark.gpu


def _u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _t16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev).view(torch.float16)


def _append(L, k, v, past, dev):
    from cuda_inf_amd._lib import call
    kd, vd = k.to(dev), v.to(dev)
    call("cia_layer_append", ctypes.byref(L._s), kd.data_ptr(), vd.data_ptr(), k.shape[0], past,
         torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()


def test_attention_fused_attn_sum_bit_exact(orc, cia, dev):
    from cuda_inf_amd import kernels as K
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    past, S = 1000, 150  # keys 0..1149: 17 committed groups, then a 62-key tail
    L = AttnLayer(past + S + 64, nsplit=16, device=dev)
    ref = orc.Group64Cache(past + S + 64)
    _, k0, v0 = qkv(past, seed=41, device="cpu", outliers=True)
    _append(L, k0, v0, 0, dev)
    ref.append(_u16(k0), _u16(v0), 0)
    q, k, v = qkv(S, seed=42, device="cpu", past=past, outliers=True)
    _append(L, k, v, past, dev)
    ref.append(_u16(k), _u16(v), past)
    assert L.committed == ref.committed == 1088
    T = past + S
    start = np.linspace(0.5, 3.0, T).astype(np.float32)  # accumulation onto existing mass
    asum = torch.from_numpy(start.copy()).to(dev)
    ws = torch.empty(K.mass_workspace_bytes(S), dtype=torch.uint8, device=dev)
    out = torch.empty((S, 32, 64), dtype=torch.float16, device=dev)
    K.attention_fused(q.to(dev), L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed, out,
                      asum, S, past, 0.125, ws)
    torch.cuda.synchronize()
    rsum = start.copy()
    _, r32 = orc.attention_fused(_u16(q), ref, S, past, attn_sum=rsum)
    got = asum.cpu().numpy()
    bad = np.nonzero(got.view(np.uint32) != rsum.view(np.uint32))[0]
    assert bad.size == 0, (f"{bad.size} of {T} attn_sum entries differ; first at {bad[0]}: "
                           f"{got[bad[0]]!r} vs {rsum[bad[0]]!r}")
    assert_close_f16(_u16(out), r32)


def test_attention_fused_rejects_small_mass_workspace(cia, dev):
    from cuda_inf_amd import kernels as K
    from cuda_inf_amd._lib import call, CiaError
    from cuda_inf_amd.layer import AttnLayer
    L = AttnLayer(256, nsplit=16, device=dev)
    S = 40
    q = torch.zeros((S, 32, 64), dtype=torch.float16, device=dev)
    out = torch.empty_like(q)
    asum = torch.zeros(S, dtype=torch.float32, device=dev)
    ws = torch.empty(K.mass_workspace_bytes(S) - 16, dtype=torch.uint8, device=dev)
    with pytest.raises(CiaError):
        call("cia_attention_fused", q.data_ptr(), L.kc8.data_ptr(), L.vc8.data_ptr(),
             L.ksc.data_ptr(), L.vsc.data_ptr(), L.ktail.data_ptr(), L.vtail.data_ptr(), 0,
             out.data_ptr(), asum.data_ptr(), S, 0, 0.125, ws.data_ptr(), ws.numel(),
             torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("producers", [False, True])
def test_decode_loop_32k_two_layers_through_commit(orc, cia, dev, producers):
    from cuda_inf_amd import _lib, workload
    from cuda_inf_amd.layer import AttnLayer
    nL, n0, steps = 2, 32768 - 5, 12  # tail 59 keys; the step at 32767 commits group 511
    rng = np.random.default_rng(7)
    qw = rng.uniform(0.5, 1.5, 64).astype(np.float16)
    kw = rng.uniform(0.5, 1.5, 64).astype(np.float16)
    layers, refs = [], []
    for l in range(nL):
        L = AttnLayer(n0 + steps + 64, nsplit=0, device=dev)
        ref = orc.Group64Cache(n0 + steps + 64)
        _, k0, v0 = workload.qkv(n0, seed=60 + l, device="cpu", outliers=True)
        _append(L, k0, v0, 0, dev)
        ref.append(_u16(k0), _u16(v0), 0)
        layers.append(L)
        refs.append(ref)
    print(f"decode loop 32k, producers={producers}: caches built", flush=True)
    arr = (_lib.cia_layer * nL)(*[L._s for L in layers])
    pos = np.arange(n0, n0 + steps, dtype=np.int32)
    qs, ks, vs, pqs, pks = [], [], [], [], []
    for l in range(nL):
        g = np.random.default_rng(100 + l)
        qr = (g.standard_normal((steps, 32, 64)) * 2).astype(np.float16)
        kr = (g.standard_normal((steps, 8, 64)) * 2).astype(np.float16)
        vr = g.standard_normal((steps, 8, 64)).astype(np.float16)
        if producers:
            pq, pk = orc.qk_norm_rope(qr, kr, qw, kw, pos)
            qs.append(qr.view(np.uint16))
            ks.append(kr.view(np.uint16))
        else:
            # prepared inputs: the producers' output itself
            pq, pk = orc.qk_norm_rope(qr, kr, qw, kw, pos)
            qs.append(pq)
            ks.append(pk)
        pqs.append(pq)
        pks.append(pk)
        vs.append(vr.view(np.uint16))
    q = np.stack(qs, 1)  # [steps, nL, 32, 64]
    k = np.stack(ks, 1)
    v = np.stack(vs, 1)
    qd, kd, vd = _t16(q, dev), _t16(k, dev), _t16(v, dev)
    keep = []
    if producers:
        qwd, kwd = _t16(qw, dev), _t16(kw, dev)
        keep += [qwd, kwd]
        for l in range(nL):
            pw = torch.zeros((32 + 8) * 64, dtype=torch.float16, device=dev)
            keep.append(pw)
            arr[l].qw, arr[l].kw = qwd.data_ptr(), kwd.data_ptr()
            arr[l].eps, arr[l].theta = workload.EPS, workload.ROPE_THETA
            arr[l].prep_ws, arr[l].prep_cap = pw.data_ptr(), 1
    out = torch.empty((steps, nL, 32, 64), dtype=torch.float16, device=dev)
    _lib.call("cia_decode_loop", arr, nL, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
              out.data_ptr(), n0, steps, 0.125, None, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got = _u16(out)
    for s in range(steps):
        p = n0 + s
        for l in range(nL):
            refs[l].append(pks[l][s:s + 1], vs[l][s:s + 1], p)
            _, r32, _ = orc.attn_decode(pqs[l][s], refs[l], p, nsplit=16, nthreads=8)
            assert_close_f16(got[s, l], r32, what=f"step {s} (key {p}) layer {l}")
    for l in range(nL):
        c = refs[l].committed
        assert c == 32768 and arr[l].committed == c
        L = layers[l]
        lo = 0
        assert np.array_equal(L.kc8.cpu().numpy().reshape(-1)[lo:c * 512],
                              refs[l].kc8.reshape(-1)[lo:c * 512])
        assert np.array_equal(L.vc8.cpu().numpy().reshape(-1)[lo:c * 512],
                              refs[l].vc8.reshape(-1)[lo:c * 512])
        assert np.array_equal(_u16(L.ksc).reshape(-1)[:c // 64 * 8], refs[l].ksc.reshape(-1)[:c // 64 * 8])
        assert np.array_equal(_u16(L.vsc).reshape(-1)[:c // 64 * 8], refs[l].vsc.reshape(-1)[:c // 64 * 8])
        nt = n0 + steps - c
        assert np.array_equal(_u16(L.ktail).reshape(64, -1)[:nt], refs[l].ktail.reshape(64, -1)[:nt])
        assert np.array_equal(_u16(L.vtail).reshape(64, -1)[:nt], refs[l].vtail.reshape(64, -1)[:nt])


def _check_partials(pm, pl, po, rpm, rpl, rpo):
    """A split's partial against the oracle's: empty splits exactly (m = -1e30,
    l = 0, o = 0); else m within 1e-4 (the largest scaled score), l within
    2e-4 relative, and the split's own attention output o / l within the
    output tolerance 2e-3 + 1e-3 |ref|.  (o itself is a sum over up to 8192
    keys whose terms cancel per dim; the matrix-core path rounds the softmax
    numerators to fp16, so o is compared through o / l, the quantity the
    combine uses.)"""
    gpm, gpl = pm.cpu().numpy(), pl.cpu().numpy()
    gpo = po.cpu().numpy().reshape(rpo.shape)
    empty = rpl == 0
    assert np.array_equal(gpl == 0, empty)
    assert np.all(gpm[empty] == np.float32(-1e30)) and np.all(gpo[empty] == 0)
    full = ~empty
    np.testing.assert_allclose(gpm[full], rpm[full], rtol=0, atol=1e-4)
    np.testing.assert_allclose(gpl[full], rpl[full], rtol=2e-4)
    got = gpo[full] / gpl[full][:, None]
    want = rpo[full] / rpl[full][:, None]
    err = np.abs(got - want)
    bad = err > 2e-3 + 1e-3 * np.abs(want)
    assert not bad.any(), (f"{bad.sum()} of {bad.size} split outputs o / l outside tolerance; "
                           f"max abs err {err.max():.3g}")


@pytest.fixture(scope="module")
def cache131k(orc, dev):
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    n = 131072
    L = AttnLayer(n + 64, nsplit=512, device=dev)
    ref = orc.Group64Cache(n + 64)
    for c0 in range(0, n, 16384):
        _, k, v = qkv(16384, seed=900 + c0 // 16384, device="cpu", past=c0, outliers=True)
        _append(L, k, v, c0, dev)
        ref.append(_u16(k), _u16(v), c0)
    assert L.committed == ref.committed == n
    return L, ref


@pytest.mark.parametrize("nsplit", [16, 64, 256, 512])
def test_split_combine_131k(orc, cia, dev, cache131k, nsplit):
    from cuda_inf_amd import kernels as K
    from cuda_inf_amd.workload import qkv
    L, ref = cache131k
    qpos = 131071
    q, _, _ = qkv(1, seed=77 + nsplit, device="cpu", past=qpos)
    pm = torch.zeros(32 * nsplit, device=dev)
    pl = torch.zeros(32 * nsplit, device=dev)
    po = torch.zeros(32 * nsplit * 64, device=dev)
    out = torch.empty((32, 64), dtype=torch.float16, device=dev)
    K.attn_decode_split(q.to(dev), L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed,
                        qpos, 0.125, pm, pl, po, nsplit)
    K.attn_decode_combine(pm, pl, po, out, nsplit)
    torch.cuda.synchronize()
    _, r32, (rpm, rpl, rpo) = orc.attn_decode(_u16(q), ref, qpos, nsplit=nsplit, nthreads=8)
    assert_close_f16(_u16(out), r32)
    _check_partials(pm, pl, po, rpm, rpl, rpo)


def test_decode_131k(orc, cia, dev, cache131k):
    """cia_attn_decode over the 131072-key cache (the long-context shape of the
    matrix-core leg: unequal ranges per head pair, 38 workgroups for the pair
    that owns the cache's slow 128-byte quarter, 30 for the others)."""
    from cuda_inf_amd import kernels as K
    from cuda_inf_amd.workload import qkv
    L, ref = cache131k
    qpos = L.committed - 1 + (9 if getattr(ref, "tail9", False) else 0)
    q, _, _ = qkv(1, seed=515, device="cpu", past=qpos)
    out = torch.empty((32, 64), dtype=torch.float16, device=dev)
    ws = torch.zeros(K.decode_workspace_bytes(qpos + 1), dtype=torch.uint8, device=dev)
    K.attn_decode(q.to(dev), L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed, qpos,
                  0.125, out, ws)
    torch.cuda.synchronize()
    _, r32, _ = orc.attn_decode(_u16(q), ref, qpos, nsplit=16, nthreads=8)
    assert_close_f16(_u16(out), r32)


@pytest.mark.parametrize("offset", [0, 128, 256, 384, 64])
def test_decode_pair_ranges_by_base(orc, cia, dev, offset):
    """The decode's ranges per head pair follow the cache's base address: the
    pair owning bytes 384..511 of each 512-byte block gets more workgroups.
    The same 66 560-key cache at base offsets 0, 128, 256 and 384 bytes puts
    that quarter on head pairs 3, 2, 1 and 0 in turn; a base 64 bytes off
    (not 128-byte aligned) keeps equal ranges.  Each against the oracle."""
    from cuda_inf_amd import kernels as K
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    ntok = 66560  # 1040 groups: two or more two-group units per FP8 wave
    L = AttnLayer(ntok + 64, nsplit=16, device=dev)
    ref = orc.Group64Cache(ntok + 64)
    _, k, v = qkv(ntok, seed=ntok + offset, device="cpu", outliers=True)
    _append(L, k, v, 0, dev)
    ref.append(_u16(k), _u16(v), 0)
    nb = L.kc8.numel()
    kbuf = torch.zeros(nb + 1024, dtype=torch.uint8, device=dev)
    vbuf = torch.zeros(nb + 1024, dtype=torch.uint8, device=dev)
    base = (512 - kbuf.data_ptr() % 512) % 512 + offset
    kc8 = kbuf[base:base + nb]
    vbase = (512 - vbuf.data_ptr() % 512) % 512 + offset
    vc8 = vbuf[vbase:vbase + nb]
    kc8.copy_(L.kc8.reshape(-1))
    vc8.copy_(L.vc8.reshape(-1))
    assert kc8.data_ptr() % 512 == offset and vc8.data_ptr() % 512 == offset
    qpos = ntok - 1
    q, _, _ = qkv(1, seed=7 + offset, device="cpu", past=qpos)
    out = torch.empty((32, 64), dtype=torch.float16, device=dev)
    ws = torch.zeros(K.decode_workspace_bytes(qpos + 1), dtype=torch.uint8, device=dev)
    K.attn_decode(q.to(dev), kc8, vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed, qpos,
                  0.125, out, ws)
    torch.cuda.synchronize()
    _, r32, _ = orc.attn_decode(_u16(q), ref, qpos, nsplit=16, nthreads=8)
    assert_close_f16(_u16(out), r32)


def test_split_combine_131k_tail(orc, cia, dev, cache131k):
    """The long-context shape of the split leg: 131072 committed keys and a
    9-key tail, 16 splits of 8193 keys (splits 0-14 each touch 129 groups,
    the last split holds the tail keys).  Appends to the shared cache, so it
    runs after the other 131k tests."""
    from cuda_inf_amd import kernels as K
    from cuda_inf_amd.workload import qkv
    L, ref = cache131k
    n = 131072
    if not getattr(ref, "tail9", False):
        _, k, v = qkv(9, seed=4242, device="cpu", past=n, outliers=True)
        _append(L, k, v, n, dev)
        ref.append(_u16(k), _u16(v), n)
        ref.tail9 = True
    assert L.committed == ref.committed == n
    qpos, nsplit = n + 8, 16
    q, _, _ = qkv(1, seed=991, device="cpu", past=qpos)
    pm = torch.full((32 * nsplit,), 7.0, device=dev)
    pl = torch.full((32 * nsplit,), 7.0, device=dev)
    po = torch.full((32 * nsplit * 64,), 7.0, device=dev)
    out = torch.empty((32, 64), dtype=torch.float16, device=dev)
    K.attn_decode_split(q.to(dev), L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed,
                        qpos, 0.125, pm, pl, po, nsplit)
    K.attn_decode_combine(pm, pl, po, out, nsplit)
    torch.cuda.synchronize()
    _, r32, (rpm, rpl, rpo) = orc.attn_decode(_u16(q), ref, qpos, nsplit=nsplit, nthreads=8)
    assert_close_f16(_u16(out), r32)
    _check_partials(pm, pl, po, rpm, rpl, rpo)


def test_append_4096_bit_exact(orc, cia, dev):
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    S = 4096
    L = AttnLayer(S + 64, nsplit=16, device=dev)
    ref = orc.Group64Cache(S + 64)
    _, k, v = qkv(S, seed=5, device="cpu", outliers=True)
    _append(L, k, v, 0, dev)
    ref.append(_u16(k), _u16(v), 0)
    assert L.committed == ref.committed == S
    assert np.array_equal(L.kc8.cpu().numpy(), ref.kc8)
    assert np.array_equal(L.vc8.cpu().numpy(), ref.vc8)
    assert np.array_equal(_u16(L.ksc), ref.ksc)
    assert np.array_equal(_u16(L.vsc), ref.vsc)
    assert np.array_equal(_u16(L.ktail), ref.ktail)
    assert np.array_equal(_u16(L.vtail), ref.vtail)


@pytest.mark.parametrize("ntok,nsplit", [(10109, 76), (25700, 200), (70000, 300), (2032, 7),
                                         (5000, 3), (4300, 33), (200, 1), (3000, 1), (4096, 16),
                                         (2032, 40), (777, 512), (64, 16), (131, 300), (1, 1),
                                         (33000, 16), (70001, 7)])
def test_split_partials_geometry(orc, cia, dev, ntok, nsplit):
    """Split geometries.  Matrix-core path (splits of 128 keys or more): the
    tail straddling two splits (10109 / 76, 25700 / 200, and 70000 / 300 with
    more than 8 splits per workgroup), odd workgroups per kv head (7, 3, 33),
    one workgroup per kv head (nsplit 1), no tail (4096); splits that start
    inside a group and are shared by several workgroups (33000 / 16: 33 or 34
    groups over 2 workgroups per split; 70001 / 7: 157 or 158 over 4).  Splits of fewer
    keys take the fp32 kernel: 2032 / 40, 777 / 512 and 131 / 300 (few keys,
    empty splits), 64 / 16, and no committed group (1).  Every partial against
    the oracle's, empty splits exactly (-1e30, 0, 0)."""
    from cuda_inf_amd import kernels as K
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    L = AttnLayer(ntok + 64, nsplit=16, device=dev)
    ref = orc.Group64Cache(ntok + 64)
    _, k, v = qkv(ntok, seed=ntok + nsplit, device="cpu", outliers=True)
    _append(L, k, v, 0, dev)
    ref.append(_u16(k), _u16(v), 0)
    qpos = ntok - 1
    q, _, _ = qkv(1, seed=3 * nsplit, device="cpu", past=qpos)
    pm = torch.full((32 * nsplit,), 7.0, device=dev)  # (stale values must all be replaced)
    pl = torch.full((32 * nsplit,), 7.0, device=dev)
    po = torch.full((32 * nsplit * 64,), 7.0, device=dev)
    out = torch.empty((32, 64), dtype=torch.float16, device=dev)
    K.attn_decode_split(q.to(dev), L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed,
                        qpos, 0.125, pm, pl, po, nsplit)
    K.attn_decode_combine(pm, pl, po, out, nsplit)
    torch.cuda.synchronize()
    _, r32, (rpm, rpl, rpo) = orc.attn_decode(_u16(q), ref, qpos, nsplit=nsplit, nthreads=8)
    _check_partials(pm, pl, po, rpm, rpl, rpo)
    assert_close_f16(_u16(out), r32)
