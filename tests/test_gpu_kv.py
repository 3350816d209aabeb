"""GPU parity of the FP8 KV writers against the oracle: bit-exact bytes/scales.

Covers f2e4m3 (engine.cu:24-26) over all 2^32 fp32 inputs, kv_write_tail +
kv_commit_group (engine.cu:190-228) including the append loop
(engine.cu:830-845), and kv_quant_write (engine.cu:317-333).
"""
import threading

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def test_e4m3_encoder_all_fp32(orc, cia, dev):
    from cuda_inf_amd import kernels as K
    chunk = 1 << 28
    out = torch.empty(chunk, dtype=torch.uint8, device=dev)
    for c in range(1 << 4):
        first = c * chunk
        K.e4m3_encode_range(first, chunk, out)
        got = out.cpu().numpy()
        ref = np.empty(chunk, np.uint8)
        parts = 16
        step = chunk // parts

        def work(p):
            ref[p * step:(p + 1) * step] = orc.e4m3_encode_range_u32(first + p * step, step)

        th = [threading.Thread(target=work, args=(p,)) for p in range(parts)]
        [t.start() for t in th]
        [t.join() for t in th]
        if not np.array_equal(got, ref):
            bad = np.nonzero(got != ref)[0]
            i = bad[0]
            raise AssertionError(
                f"{bad.size} mismatches in chunk {c}; first bits 0x{first + i:08x}: "
                f"gpu 0x{got[i]:02x} oracle 0x{ref[i]:02x}")


def _special_tail(kind, g):
    """[64, 8, 64] fp16 tails covering the closed-form cases."""
    x = torch.randn((64, 8, 64), generator=g, dtype=torch.float64).to(torch.float16)
    if kind == "zero":
        x.zero_()
    elif kind == "negzero":
        x = torch.full_like(x, -0.0)
    elif kind == "single":
        x.zero_()
        x[17, 3, 5] = -3.25
    elif kind == "const":
        x.fill_(0.7)
    elif kind == "extremes":
        x[0, :, 0] = 65504.0
        x[1, :, 1] = -65504.0
        x[2, :, 2] = 6.0e-8   # fp16 subnormal
        x[3, :, 3] = -0.0
    elif kind == "tiny":
        x = (x.double() * 1e-6).to(torch.float16)
    elif kind == "outliers":
        m = torch.rand(x.shape, generator=g) < 0.01
        x = torch.where(m, (x.float() * 20).to(torch.float16), x)
    return x.contiguous()


@pytest.mark.parametrize("kind", ["normal", "zero", "negzero", "single", "const", "extremes",
                                  "tiny", "outliers"])
def test_commit_group_bit_exact(orc, cia, dev, kind):
    from cuda_inf_amd import kernels as K
    g = torch.Generator().manual_seed(hash(kind) % 1000)
    kt, vt = _special_tail(kind, g), _special_tail(kind if kind != "single" else "normal", g)
    T = 3 * 64
    kc8 = torch.zeros((T, 8, 64), dtype=torch.uint8, device=dev)
    vc8 = torch.zeros_like(kc8)
    ksc = torch.zeros((T // 64 + 2, 8), dtype=torch.float16, device=dev)
    vsc = torch.zeros_like(ksc)
    K.kv_commit_group(kt.to(dev), vt.to(dev), kc8, vc8, ksc, vsc, 128, 2)
    torch.cuda.synchronize()
    rk8 = np.zeros((T, 8, 64), np.uint8)
    rv8 = np.zeros_like(rk8)
    rks = np.zeros((T // 64 + 2, 8), np.uint16)
    rvs = np.zeros_like(rks)
    orc.kv_commit_group(_u16(kt), _u16(vt), rk8, rv8, rks, rvs, 128, 2)
    assert np.array_equal(kc8.cpu().numpy(), rk8)
    assert np.array_equal(vc8.cpu().numpy(), rv8)
    assert np.array_equal(_u16(ksc), rks)
    assert np.array_equal(_u16(vsc), rvs)


@pytest.mark.parametrize("S,seed", [(1, 0), (7, 1), (64, 2), (300, 3)])
def test_quant_write_bit_exact(orc, cia, dev, S, seed):
    from cuda_inf_amd import kernels as K
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((S, 8, 64), generator=g, dtype=torch.float64).to(torch.float16)
    v = torch.randn((S, 8, 64), generator=g, dtype=torch.float64).to(torch.float16)
    if S > 1:
        k[0].zero_()
        v[1, 2, :] = -0.0
        k[S - 1, 0, 7] = 60000.0
    C = 512
    dst = torch.randperm(C, generator=g)[:S].to(torch.int32)
    kf = torch.zeros((C, 8, 64), dtype=torch.uint8, device=dev)
    vf = torch.zeros_like(kf)
    ks = torch.zeros((C, 8), dtype=torch.float16, device=dev)
    vs = torch.zeros_like(ks)
    K.kv_quant_write(k.to(dev), v.to(dev), kf, vf, ks, vs, dst.to(dev), S)
    torch.cuda.synchronize()
    rkf = np.zeros((C, 8, 64), np.uint8)
    rvf = np.zeros_like(rkf)
    rks = np.zeros((C, 8), np.uint16)
    rvs = np.zeros_like(rks)
    orc.kv_quant_write(_u16(k), _u16(v), rkf, rvf, rks, rvs, dst.numpy())
    assert np.array_equal(kf.cpu().numpy(), rkf)
    assert np.array_equal(vf.cpu().numpy(), rvf)
    assert np.array_equal(_u16(ks), rks)
    assert np.array_equal(_u16(vs), rvs)


@pytest.mark.parametrize("batches", [[1] * 130, [63, 1, 64, 2, 200, 5], [2031], [64, 64, 1, 127],
                                     [50, 20], [10, 54, 3, 1, 200], [64], [5, 59, 64, 64, 7]])
def test_append_loop_bit_exact(orc, cia, dev, batches):
    """The layer driver's placement loop (batched: one launch for the groups a
    batch completes, one for the tail): committed groups, scales and the whole
    tail buffer -- stale rows included -- identical to the reference's loop."""
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    total = sum(batches)
    L = AttnLayer(total + 4, nsplit=16, device=dev)
    ref = orc.Group64Cache(total + 4)
    past = 0
    for i, S in enumerate(batches):
        q, k, v = qkv(S, seed=100 + i, device="cpu", past=past, outliers=True)
        L.forward(q.to(dev), k.to(dev), v.to(dev), past)
        ref.append(_u16(k), _u16(v), past)
        past += S
    torch.cuda.synchronize()
    assert L.committed == ref.committed
    assert np.array_equal(L.kc8.cpu().numpy(), ref.kc8)
    assert np.array_equal(L.vc8.cpu().numpy(), ref.vc8)
    assert np.array_equal(_u16(L.ksc), ref.ksc)
    assert np.array_equal(_u16(L.vsc), ref.vsc)
    assert np.array_equal(_u16(L.ktail), ref.ktail)
    assert np.array_equal(_u16(L.vtail), ref.vtail)
