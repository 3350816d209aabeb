"""GPU parity of the H2O path (engine.cu:310-384, 803-828) against the oracle.

The evicted-slot sequence must be identical and, because it depends on every
bit of the accumulated attention mass, attn_sum is compared bit for bit after
every step; attention outputs are compared within 2e-3 + 1e-3|ref|.
"""
import os

import numpy as np
import pytest
import torch

from conftest import assert_close_f16

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "h2o_c2048_w256_seed7.npz")


def _u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def test_h2o_small_stepwise(orc, cia, dev):
    """C=128, W=16, 64-token prompt, 300 decode steps: every step checked."""
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    C, W, P, N = 128, 16, 64, 300
    q, k, v = qkv(P + N, seed=21, device="cpu", prep=False)
    qn, kn, vn = _u16(q), _u16(k), _u16(v)
    L = AttnLayer(P + N + 4, budget=C, window=W, prompt_len=P, max_batch=P, device=dev)
    assert (L.budget, L.window) == (C, W)
    ref = orc.H2OCache(C, W)
    out, _ = L.forward(q[:P].to(dev), k[:P].to(dev), v[:P].to(dev), 0)
    _, r16, r32 = ref.step(qn[:P], kn[:P], vn[:P], 0)
    torch.cuda.synchronize()
    assert_close_f16(_u16(out), r32, what="prompt")
    assert np.array_equal(L.hattn.cpu().numpy().view(np.uint32), ref.attn.view(np.uint32))
    n_ev = 0
    for j in range(N):
        pos = P + j
        out, ev = L.forward(q[pos:pos + 1].to(dev), k[pos:pos + 1].to(dev), v[pos:pos + 1].to(dev),
                            pos)
        dst, r16, r32 = ref.step(qn[pos:pos + 1], kn[pos:pos + 1], vn[pos:pos + 1], pos)
        torch.cuda.synchronize()
        ref_ev = int(dst[0]) if pos >= C else -1
        assert ev == ref_ev, f"step {j}: evicted {ev}, oracle {ref_ev}"
        n_ev += ev >= 0
        got = L.hattn.cpu().numpy()
        if not np.array_equal(got.view(np.uint32), ref.attn.view(np.uint32)):
            i = int(np.argmax(got != ref.attn))
            raise AssertionError(f"step {j}: attn_sum differs at slot {i}: "
                                 f"{got[i]!r} vs {ref.attn[i]!r}")
        assert np.array_equal(L.h_slotpos.numpy(), ref.slotpos)
        assert_close_f16(_u16(out), r32, what=f"step {j}")
    assert n_ev == N + P - C


def test_h2o_eviction_golden(cia, dev):
    """2048 slots, window 256, 1024-token prompt, 4000 steps, seed 7:
    evicted-slot sequence identical to the committed oracle run."""
    from cuda_inf_amd.layer import AttnLayer
    g = np.load(GOLDEN, allow_pickle=False)
    steps, C, W, P = int(g["steps"]), int(g["C"]), int(g["W"]), int(g["prompt"])
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "make_h2o_golden", os.path.join(os.path.dirname(GOLDEN), "make_h2o_golden.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    q, k, v = mk.inputs(steps)
    assert mk.digest(q, k, v) == str(g["digest"]), "input generator changed"
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    L = AttnLayer(P + steps + 4, budget=C, window=W, prompt_len=P, max_batch=P, device=dev)
    L.forward(qd[:P], kd[:P], vd[:P], 0)
    evicted = np.full(steps, -1, np.int32)
    for j in range(steps):
        pos = P + j
        _, ev = L.forward(qd[pos:pos + 1], kd[pos:pos + 1], vd[pos:pos + 1], pos)
        evicted[j] = ev
    torch.cuda.synchronize()
    ref = g["evicted"]
    if not np.array_equal(evicted, ref):
        j = int(np.argmax(evicted != ref))
        raise AssertionError(f"first divergence at step {j}: gpu {evicted[j]} oracle {ref[j]}")
    assert np.array_equal(L.hattn.cpu().numpy().view(np.uint32), g["attn_sum"].view(np.uint32))
    assert np.array_equal(L.h_slotpos.numpy(), g["slotpos"])
