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
