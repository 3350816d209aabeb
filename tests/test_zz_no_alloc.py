"""cia_attn_decode_noalloc (the decode entry with the library's own fixed
workspace) against cia_attn_decode with a caller workspace: bit-identical
outputs on consecutive calls, the second over a smaller context (fewer
workgroups per kv head), then the larger one again; and the oracle's
tolerance on each."""
import numpy as np
import pytest
import torch

from conftest import assert_close_f16

pytestmark = pytest.mark.gpu


def _u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _cache(dev, orc, ntok, seed):
    from cuda_inf_amd import kernels as K
    from cuda_inf_amd.layer import AttnLayer, kv_append_plan
    from cuda_inf_amd.workload import qkv
    L = AttnLayer(ntok + 64, nsplit=16, device=dev)
    ref = orc.Group64Cache(ntok + 64)
    _, k, v = qkv(ntok, seed=seed, device="cpu", outliers=True)
    kd, vd = k.to(dev), v.to(dev)
    ops, c = kv_append_plan(0, ntok, 0)
    for op in ops:
        s0 = op["src_token"]
        K.kv_write_tail(kd[s0:], vd[s0:], L.ktail, L.vtail, op["slot"], op["cnt"])
        if op["commit"]:
            K.kv_commit_group(L.ktail, L.vtail, L.kc8, L.vc8, L.ksc, L.vsc, op["commit_base"],
                              op["commit_grp"])
    L._s.committed = c
    ref.append(_u16(k), _u16(v), 0)
    return L, ref


def test_noalloc_matches_workspace_entry(orc, cia, dev):
    from cuda_inf_amd import kernels as K
    from cuda_inf_amd.workload import qkv
    # 33000 keys: 32 workgroups per kv head and extra waves; 2032: two; 33000 again
    cases = [(33000, 5), (2032, 6), (33000, 7)]
    built = {}
    for ntok, seed in cases:
        if ntok not in built:
            built[ntok] = _cache(dev, orc, ntok, seed=ntok)
        L, ref = built[ntok]
        qpos = ntok - 1
        q, _, _ = qkv(1, seed=seed, device="cpu", past=qpos)
        qd = q.to(dev)
        ws = K.new_decode_workspace(ntok, dev)
        a = torch.empty((32, 64), dtype=torch.float16, device=dev)
        b = torch.empty((32, 64), dtype=torch.float16, device=dev)
        K.attn_decode(qd, L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed, qpos, 0.125,
                      a, ws)
        K.attn_decode_noalloc(qd, L.kc8, L.vc8, L.ksc, L.vsc, L.ktail, L.vtail, L.committed, qpos,
                              0.125, b)
        torch.cuda.synchronize()
        assert np.array_equal(_u16(a), _u16(b)), f"noalloc differs from the workspace entry at {ntok}"
        _, r32, _ = orc.attn_decode(_u16(q), ref, qpos, nsplit=16, nthreads=8)
        assert_close_f16(_u16(b), r32, what=f"noalloc at {ntok} keys")
