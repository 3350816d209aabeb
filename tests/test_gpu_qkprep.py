"""GPU parity of the QK producers (engine.cu:148-182, launched at 799-801):
cia_qk_norm_rope against the oracle, bit for bit."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("S,pmax,seed", [(1, 1, 0), (5, 70000, 1), (300, 131072, 2), (64, 4096, 3)])
def test_qk_norm_rope_bit_exact(orc, cia, dev, S, pmax, seed):
    from cuda_inf_amd import kernels as K
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((S, 32, 64)) * rng.uniform(0.01, 50, (S, 32, 1))).astype(np.float16)
    k = (rng.standard_normal((S, 8, 64)) * rng.uniform(0.01, 50, (S, 8, 1))).astype(np.float16)
    if S > 3:
        k[2, 1] = 0
        q[1, 5, :7] = 60000.0
    qw = rng.uniform(0.25, 2.0, 64).astype(np.float16)
    kw = rng.uniform(0.25, 2.0, 64).astype(np.float16)
    pos = rng.integers(0, pmax, S).astype(np.int32)
    rq, rk = orc.qk_norm_rope(q, k, qw, kw, pos)
    qd = torch.from_numpy(q.view(np.int16)).to(dev)
    kd = torch.from_numpy(k.view(np.int16)).to(dev)
    print(f"qk_norm_rope S={S} pmax={pmax}", flush=True)
    K.qk_norm_rope(qd, kd, torch.from_numpy(qw.view(np.int16)).to(dev),
                   torch.from_numpy(kw.view(np.int16)).to(dev), torch.from_numpy(pos).to(dev), S)
    torch.cuda.synchronize()
    gq = qd.cpu().numpy().view(np.uint16)
    gk = kd.cpu().numpy().view(np.uint16)
    for name, g, r in (("q", gq, rq), ("k", gk, rk)):
        if not np.array_equal(g, r):
            i = np.argwhere(g != r)[0]
            raise AssertionError(f"{name} differs at {tuple(i)}: {g[tuple(i)]:#06x} vs {r[tuple(i)]:#06x}")


def _raw(S, seed):
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((S, 32, 64)) * 2).astype(np.float16)
    k = (rng.standard_normal((S, 8, 64)) * 2).astype(np.float16)
    v = rng.standard_normal((S, 8, 64)).astype(np.float16)
    return q, k, v


def test_layer_with_producers_prefill_and_fused_decode(orc, cia, dev):
    """A layer given raw q/k: prefill (producers in one launch, then append
    and attention) and decode steps through cia_decode_loop (producers inside
    the decode kernels, the fresh token's tail write and a group commit
    fused), against the oracle on producer-prepared inputs: outputs within
    tolerance, cache bytes bit for bit."""
    import ctypes
    from conftest import assert_close_f16
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd._lib import call
    rng = np.random.default_rng(3)
    qw = rng.uniform(0.5, 1.5, 64).astype(np.float16)
    kw = rng.uniform(0.5, 1.5, 64).astype(np.float16)
    P, N = 1000, 90  # crosses the group boundary at 1024
    q, k, v = _raw(P + N, 4)
    pos = np.arange(P + N, dtype=np.int32)
    pq, pk = orc.qk_norm_rope(q, k, qw, kw, pos)
    L = AttnLayer(P + N + 64, nsplit=0, qk_norm=(torch.from_numpy(qw), torch.from_numpy(kw)),
                  max_batch=P, device=dev)
    ref = orc.Group64Cache(P + N + 64)
    t = lambda a: torch.from_numpy(a.view(np.int16)).to(dev).view(torch.float16)
    qd, kd, vd = t(q), t(k), t(v)
    print("producers: prefill", flush=True)
    out, _ = L.forward(qd[:P], kd[:P], vd[:P], 0)
    ref.append(pk[:P], v[:P].view(np.uint16), 0)
    torch.cuda.synchronize()
    rows = np.arange(0, P, 7).astype(np.int32)
    _, r32 = orc.attention_fused(pq[:P], ref, P, 0, rows=rows)
    assert_close_f16(out.cpu().numpy().view(np.uint16)[rows], r32[rows], what="prefill")
    outd = torch.zeros((N, 32, 64), dtype=torch.float16, device=dev)
    s = torch.cuda.current_stream()
    print("producers: decode loop", flush=True)
    call("cia_decode_loop", ctypes.byref(L._s), 1, qd[P].data_ptr(), kd[P].data_ptr(),
         vd[P].data_ptr(), outd.data_ptr(), P, N, 0.125, None, s.cuda_stream)
    torch.cuda.synchronize()
    got = outd.cpu().numpy().view(np.uint16)
    for j in range(N):
        ref.append(pk[P + j:P + j + 1], v[P + j:P + j + 1].view(np.uint16), P + j)
        if j % 9 == 0 or j == N - 1 or (P + j) % 64 in (62, 63, 0):
            _, r32, _ = orc.attn_decode(pq[P + j], ref, P + j, nsplit=16)
            assert_close_f16(got[j], r32, what=f"step {j}")
    assert L.committed == ref.committed
    c = ref.committed
    assert np.array_equal(L.kc8.cpu().numpy()[:c], ref.kc8[:c])
    assert np.array_equal(L.vc8.cpu().numpy()[:c], ref.vc8[:c])
    assert np.array_equal(L.ksc.cpu().numpy().view(np.uint16)[:c // 64], ref.ksc[:c // 64])
    nt = P + N - c
    assert np.array_equal(L.ktail.cpu().numpy().view(np.uint16)[:nt], ref.ktail[:nt])
    assert np.array_equal(L.vtail.cpu().numpy().view(np.uint16)[:nt], ref.vtail[:nt])


def test_h2o_layer_with_producers(orc, cia, dev):
    """An H2O layer given raw q/k: the producers run before placement; the
    masses and slot positions match the oracle on prepared inputs."""
    from conftest import assert_close_f16
    from cuda_inf_amd.layer import AttnLayer
    rng = np.random.default_rng(8)
    qw = rng.uniform(0.5, 1.5, 64).astype(np.float16)
    kw = rng.uniform(0.5, 1.5, 64).astype(np.float16)
    C, W, P, N = 64, 8, 32, 60
    q, k, v = _raw(P + N, 9)
    pq, pk = orc.qk_norm_rope(q, k, qw, kw, np.arange(P + N, dtype=np.int32))
    L = AttnLayer(P + N + 4, budget=C, window=W, prompt_len=P, max_batch=P,
                  qk_norm=(torch.from_numpy(qw), torch.from_numpy(kw)), device=dev)
    ref = orc.H2OCache(C, W)
    t = lambda a: torch.from_numpy(a.view(np.int16)).to(dev).view(torch.float16)
    qd, kd, vd = t(q), t(k), t(v)
    L.forward(qd[:P], kd[:P], vd[:P], 0, evicted=False)
    ref.step(pq[:P], pk[:P], v[:P].view(np.uint16), 0)
    for j in range(N):
        p = P + j
        out, ev = L.forward(qd[p:p + 1], kd[p:p + 1], vd[p:p + 1], p)
        dst, r16, r32 = ref.step(pq[p:p + 1], pk[p:p + 1], v[p:p + 1].view(np.uint16), p)
        torch.cuda.synchronize()
        assert ev == (int(dst[0]) if p >= C else -1)
        assert_close_f16(out.cpu().numpy().view(np.uint16), r32, what=f"step {j}")
    assert np.array_equal(L.hattn.cpu().numpy().view(np.uint32), ref.attn.view(np.uint32))
