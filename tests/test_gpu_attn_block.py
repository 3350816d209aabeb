"""GPU parity of the attention branch of one layer (engine.cu:792-859):
q/k/v projections, QK producers, attention and out_proj into the residual,
through cia_attn_block_forward and cia_attn_block_loop, against the oracle
chain (oracle GEMV -> fp16, oracle producers, oracle cache and attention,
oracle GEMV of out_proj).

The residual is checked against the attention tolerance carried through
out_proj: |h - h_ref|[n] <= sum_k |Wo[n,k]| (2e-3 + 1e-3 |o_ref[k]|)
+ 1e-5 sum_k |Wo[n,k] o_ref[k]| + 4 ulp(h)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

H = 2048


def _dense(packed, scales):
    nib = np.empty((packed.shape[0], 2 * packed.shape[1]), np.int64)
    nib[:, 0::2] = packed & 0xF
    nib[:, 1::2] = packed >> 4
    return (nib - 8) * np.repeat(scales.view(np.float16).astype(np.float64), 128, axis=1)


def _setup(orc, dev, seed, P, N, **kw):
    from cuda_inf_amd.layer import AttnLayer
    rng = np.random.default_rng(seed)
    W = {}
    for name, n in (("q", 2048), ("k", 512), ("v", 512), ("o", 2048)):
        w = (rng.standard_normal((n, H)) * 0.03).astype(np.float32)
        W[name] = orc.quant_int4_g128(w)
    qw = rng.uniform(0.5, 1.5, 64).astype(np.float16)
    kw_ = rng.uniform(0.5, 1.5, 64).astype(np.float16)
    L = AttnLayer(P + N + 64, nsplit=0, qk_norm=(torch.from_numpy(qw), torch.from_numpy(kw_)),
                  max_batch=max(P, 1), device=dev, **kw)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(
        np.int16 if a.dtype == np.uint16 else a.dtype)).to(dev)
    L.set_projections(*[(t(W[n][0]), t(W[n][1])) for n in ("q", "k", "v", "o")])
    x = rng.standard_normal((P + N, H)).astype(np.float16)
    h0 = rng.standard_normal((P + N, H)).astype(np.float32)
    return L, W, qw, kw_, x, h0


def _oracle_qkv(orc, W, x, qw, kw):
    q = orc.gemv_int4(x, *W["q"]).astype(np.float16).reshape(-1, 32, 64)
    k = orc.gemv_int4(x, *W["k"]).astype(np.float16).reshape(-1, 8, 64)
    v = orc.gemv_int4(x, *W["v"]).astype(np.float16).reshape(-1, 8, 64)
    pq, pk = orc.qk_norm_rope(q, k, qw, kw, np.arange(x.shape[0], dtype=np.int32))
    return pq, pk, v.view(np.uint16)


def _check_h(got, h0, o32, Wo, what):
    Wd = np.abs(_dense(*Wo))
    o = np.abs(o32.reshape(-1, H).astype(np.float64))
    bound = (2e-3 + 1e-3 * o) @ Wd.T + 1e-5 * (o @ Wd.T) + 4 * np.spacing(np.abs(got))
    return bound


def test_attn_block_prefill_then_decode(orc, cia, dev):
    P, N = 150, 50  # the decode steps cross the group boundary at 192
    L, W, qw, kw, x, h0 = _setup(orc, dev, 21, P, N)
    xd = torch.from_numpy(x.view(np.int16)).to(dev).view(torch.float16)
    hd = torch.from_numpy(h0.copy()).to(dev)
    print("attn block: prefill", flush=True)
    L.block_forward(xd[:P], hd[:P], 0)
    for j in range(N):
        L.block_forward(xd[P + j:P + j + 1], hd[P + j:P + j + 1], P + j)
    torch.cuda.synchronize()
    got = hd.cpu().numpy()
    pq, pk, v = _oracle_qkv(orc, W, x, qw, kw)
    ref = orc.Group64Cache(P + N + 64)
    ref.append(pk[:P], v[:P], 0)
    o32 = np.zeros((P + N, 32, 64), np.float32)
    o16 = np.zeros((P + N, 32, 64), np.uint16)
    o16[:P], o32[:P] = orc.attention_fused(pq[:P], ref, P, 0)
    for j in range(N):
        ref.append(pk[P + j:P + j + 1], v[P + j:P + j + 1], P + j)
        o16[P + j], o32[P + j], _ = orc.attn_decode(pq[P + j], ref, P + j)
    assert L.committed == ref.committed == 192
    y = orc.gemv_int4(o16.reshape(-1, H), *W["o"]).astype(np.float64)
    want = h0.astype(np.float64) + y
    bound = _check_h(got, h0, o32, W["o"], "h")
    err = np.abs(got - want)
    bad = err > bound
    assert not bad.any(), (f"{bad.sum()} outside; worst {np.unravel_index(np.argmax(err - bound), err.shape)}"
                           f" err {err.max():.3g}")


def test_attn_block_loop_matches_single_calls(orc, cia, dev):
    """cia_attn_block_loop over 3 layers sharing one residual equals the same
    steps made one call at a time, bit for bit."""
    from cuda_inf_amd.layer import attn_block_loop
    P, N, nl = 100, 40, 3
    layers, xs = [], []
    for i in range(2):  # two identical stacks
        stack = []
        for l in range(nl):
            L, W, qw, kw, x, h0 = _setup(orc, dev, 30 + l, P, N)
            stack.append(L)
            if i == 0:
                xs.append(x)
        layers.append(stack)
    xd = [torch.from_numpy(x.view(np.int16)).to(dev).view(torch.float16) for x in xs]
    for stack in layers:
        for l, L in enumerate(stack):
            L.block_forward(xd[l][:P], torch.zeros((P, H), dtype=torch.float32, device=dev), 0)
    h_a = torch.zeros(H, dtype=torch.float32, device=dev)
    h_b = torch.zeros(H, dtype=torch.float32, device=dev)
    steps = torch.stack([torch.stack([xd[l][P + s] for l in range(nl)]) for s in range(N)]).contiguous()
    print("attn block loop", flush=True)
    attn_block_loop(layers[0], steps, h_a, P, N)
    for s in range(N):
        for l, L in enumerate(layers[1]):
            L.block_forward(steps[s, l].contiguous(), h_b.view(1, H), P + s)
    torch.cuda.synchronize()
    assert [L.committed for L in layers[0]] == [L.committed for L in layers[1]] == [128] * nl
    assert torch.equal(h_a, h_b)
    assert torch.isfinite(h_a).all()
