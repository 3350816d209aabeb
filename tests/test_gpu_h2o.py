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


# (C, W, prompt, steps, seed): a partial last 64-slot block (50 slots) and a
# window of 5 in the second case
@pytest.mark.parametrize("C,W,P,N,seed", [(128, 16, 64, 300, 21), (50, 5, 20, 120, 22)])
def test_h2o_small_stepwise(orc, cia, dev, C, W, P, N, seed):
    """Single-token decode steps after a prompt, every step checked: the
    evicted slot, attn_sum bits, positions and outputs."""
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    q, k, v = qkv(P + N, seed=seed, device="cpu", prep=False)
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
        assert np.array_equal(L.d_slotpos.cpu().numpy(), ref.slotpos)
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
    assert np.array_equal(L.d_slotpos.cpu().numpy(), g["slotpos"])


def test_h2o_eviction_golden_decode_loop(cia, dev):
    """The same 4000 steps through the C decode loop in two calls (2500 +
    1500): from each call's second step on, a step's slot choice reads the
    placement keys the previous step's mass launch left (8 slot workgroups
    at 2048 slots), the first step of each call scans every slot.  Final
    masses and positions bit-identical to the committed oracle run (a single
    different eviction would change both)."""
    import ctypes
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd._lib import call
    g = np.load(GOLDEN, allow_pickle=False)
    steps, C, W, P = int(g["steps"]), int(g["C"]), int(g["W"]), int(g["prompt"])
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "make_h2o_golden", os.path.join(os.path.dirname(GOLDEN), "make_h2o_golden.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    q, k, v = mk.inputs(steps)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    L = AttnLayer(P + steps + 4, budget=C, window=W, prompt_len=P, max_batch=P, device=dev)
    L.forward(qd[:P], kd[:P], vd[:P], 0)
    out = torch.zeros((P + steps, 32, 64), dtype=torch.float16, device=dev)
    s = torch.cuda.current_stream()
    for s0, n in ((P, 2500), (P + 2500, steps - 2500)):
        call("cia_decode_loop", ctypes.byref(L._s), 1, qd[s0].data_ptr(), kd[s0].data_ptr(),
             vd[s0].data_ptr(), out[s0].data_ptr(), s0, n, 0.125, None, s.cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(L.hattn.cpu().numpy().view(np.uint32), g["attn_sum"].view(np.uint32))
    assert np.array_equal(L.d_slotpos.cpu().numpy(), g["slotpos"])


# (C, W, n_live, S, past, attn kind): fill only, fill then evict, the window
# empty (fallback scan), more than one slot per thread, signed zeros and NaN
# masses, an unfused batch of evictions
PLACE_CASES = [
    (64, 8, 0, 5, 0, "ties"),
    (64, 8, 60, 10, 200, "ties"),
    (64, 1000, 64, 3, 100, "ties"),
    (3000, 256, 3000, 40, 5000, "ties"),
    (3000, 256, 2990, 16, 5000, "zeros"),
    (256, 16, 256, 7, 400, "nan"),
    (256, 32, 200, 150, 300, "ties"),
    (2048, 256, 2048, 1, 9000, "randn"),
]


@pytest.mark.parametrize("C,W,n_live,S,past,kind", PLACE_CASES)
def test_h2o_place_matches_host_rule(orc, cia, dev, C, W, n_live, S, past, kind):
    """cia_h2o_place against the oracle's restatement of engine.cu:808-826:
    slots, slot positions, attention masses and quantised bytes bit-exact."""
    from cuda_inf_amd import kernels as K
    rng = np.random.default_rng(C * 7 + S)
    if kind == "randn":
        attn = np.abs(rng.standard_normal(C)).astype(np.float32)
    else:
        attn = rng.choice(np.array([0.0, 0.25, 0.5, 1.0], np.float32), C)
    if kind == "zeros":
        attn[rng.random(C) < 0.5] = -0.0
    if kind == "nan":
        attn[rng.random(C) < 0.3] = np.nan
    attn[n_live:] = 0.0
    slotpos = np.full(C, -1, np.int32)
    slotpos[:n_live] = rng.integers(0, max(past, 1), n_live)
    k = torch.randn((S, 8, 64), dtype=torch.float64,
                    generator=torch.Generator().manual_seed(S)).to(torch.float16)
    v = torch.randn((S, 8, 64), dtype=torch.float64,
                    generator=torch.Generator().manual_seed(S + 1)).to(torch.float16)
    # oracle: the host rule on copies, the device clears picked slots
    r_slot, r_attn = slotpos.copy(), attn.copy()
    r_nl, r_dst, r_zero, r_ev = orc.h2o_pick_slots(n_live, C, W, r_slot, r_attn.copy(), S, past)
    assert r_ev >= 0
    r_attn[r_dst[r_zero == 1]] = 0.0
    rkf = np.zeros((C, 8, 64), np.uint8)
    rvf = np.zeros_like(rkf)
    rks = np.zeros((C, 8), np.uint16)
    rvs = np.zeros_like(rks)
    orc.kv_quant_write(_u16(k), _u16(v), rkf, rvf, rks, rvs, r_dst)
    # device
    d_attn = torch.from_numpy(attn.copy()).to(dev)
    d_slot = torch.from_numpy(slotpos.copy()).to(dev)
    d_dst = torch.full((S,), -7, dtype=torch.int32, device=dev)
    kf = torch.zeros((C, 8, 64), dtype=torch.uint8, device=dev)
    vf = torch.zeros_like(kf)
    ks = torch.zeros((C, 8), dtype=torch.float16, device=dev)
    vs = torch.zeros_like(ks)
    print(f"h2o_place C={C} W={W} n_live={n_live} S={S} past={past} {kind}", flush=True)
    nl = K.h2o_place(k.to(dev), v.to(dev), kf, vf, ks, vs, d_attn, d_slot, d_dst, n_live, C, W,
                     S, past)
    torch.cuda.synchronize()
    assert nl == r_nl
    assert np.array_equal(d_dst.cpu().numpy(), r_dst)
    assert np.array_equal(d_slot.cpu().numpy(), r_slot)
    assert np.array_equal(d_attn.cpu().numpy().view(np.uint32), r_attn.view(np.uint32))
    assert np.array_equal(kf.cpu().numpy(), rkf)
    assert np.array_equal(vf.cpu().numpy(), rvf)
    assert np.array_equal(_u16(ks), rks)
    assert np.array_equal(_u16(vs), rvs)


def test_h2o_place_rejects_overflow(cia, dev):
    """More evictions in one call than slots: CIA_ERR_NOSLOT before any launch."""
    from cuda_inf_amd import kernels as K
    from cuda_inf_amd._lib import CiaError
    C, S = 8, 20
    z = lambda *s, dt=torch.uint8: torch.zeros(s, dtype=dt, device=dev)
    attn = z(C, dt=torch.float32)
    with pytest.raises(CiaError, match="NOSLOT"):
        K.h2o_place(z(S, 8, 64, dt=torch.float16), z(S, 8, 64, dt=torch.float16), z(C, 8, 64),
                    z(C, 8, 64), z(C, 8, dt=torch.float16), z(C, 8, dt=torch.float16), attn,
                    z(C, dt=torch.int32), z(S, dt=torch.int32), 4, C, 2, S, 0)
    assert float(attn.abs().sum()) == 0.0


def test_h2o_decode_loop_matches_oracle(orc, cia, dev):
    """The C decode loop over an H2O layer (no readback between steps):
    C=128, W=16, 64-token prompt, 250 steps in three calls with other work
    queued between them; every output, the final masses and positions
    against the oracle."""
    import ctypes
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    from cuda_inf_amd._lib import call
    C, W, P, N = 128, 16, 64, 250
    q, k, v = qkv(P + N, seed=33, device="cpu", prep=False)
    qn, kn, vn = _u16(q), _u16(k), _u16(v)
    L = AttnLayer(P + N + 4, budget=C, window=W, prompt_len=P, max_batch=P, device=dev)
    ref = orc.H2OCache(C, W)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    out = torch.zeros((P + N, 32, 64), dtype=torch.float16, device=dev)
    L.forward(qd[:P], kd[:P], vd[:P], 0, out=out[:P], evicted=False)
    ref.step(qn[:P], kn[:P], vn[:P], 0)
    s = torch.cuda.current_stream()
    junk = torch.randn(1 << 20, device=dev)
    for s0, n in ((P, 100), (P + 100, 1), (P + 101, N - 101)):
        call("cia_decode_loop", ctypes.byref(L._s), 1, qd[s0].data_ptr(), kd[s0].data_ptr(),
             vd[s0].data_ptr(), out[s0].data_ptr(), s0, n, 0.125, None, s.cuda_stream)
        junk = junk * 1.0001 + 1.0  # eager work between the calls
    torch.cuda.synchronize()
    got = _u16(out)
    for j in range(N):
        pos = P + j
        _, r16, r32 = ref.step(qn[pos:pos + 1], kn[pos:pos + 1], vn[pos:pos + 1], pos)
        assert_close_f16(got[pos:pos + 1], r32, what=f"step {j}")
    assert L.n_live == C
    assert np.array_equal(L.hattn.cpu().numpy().view(np.uint32), ref.attn.view(np.uint32))
    assert np.array_equal(L.d_slotpos.cpu().numpy(), ref.slotpos)


@pytest.mark.parametrize("n_live,S,past,seed", [(1, 1, 0, 0), (100, 1, 150, 1), (2048, 1, 5000, 2),
                                               (300, 40, 200, 3), (4096, 17, 4000, 4)])
def test_attention_h2o_kernel(orc, cia, dev, n_live, S, past, seed):
    """cia_attention_h2o against the oracle on a filled slot buffer with
    shuffled positions (some slots in the queries' future): attn_sum bit for
    bit, outputs within 2e-3 + 1e-3|ref|; S > 16 runs several query chunks."""
    from cuda_inf_amd import kernels as K
    rng = np.random.default_rng(seed)
    C = n_live + 5
    k = torch.from_numpy(rng.standard_normal((C, 8, 64))).to(torch.float16)
    v = torch.from_numpy(rng.standard_normal((C, 8, 64))).to(torch.float16)
    q = torch.from_numpy(rng.standard_normal((S, 32, 64))).to(torch.float16)
    dst = torch.arange(C, dtype=torch.int32)
    kf = torch.zeros((C, 8, 64), dtype=torch.uint8, device=dev)
    vf = torch.zeros_like(kf)
    ks = torch.zeros((C, 8), dtype=torch.float16, device=dev)
    vs = torch.zeros_like(ks)
    K.kv_quant_write(k.to(dev), v.to(dev), kf, vf, ks, vs, dst.to(dev), C)
    # slot positions: a permutation of past-n_live+S/2 .. so the last queries
    # see more slots than the first
    slot_pos = (rng.permutation(n_live) + past - n_live + S // 2).astype(np.int32)
    slot_pos[0] = min(slot_pos[0], past)  # every query sees at least one slot
    attn0 = np.abs(rng.standard_normal(C)).astype(np.float32)
    rkf, rvf = kf.cpu().numpy(), vf.cpu().numpy()
    rks, rvs = _u16(ks), _u16(vs)
    r_attn = attn0.copy()
    sp_full = np.concatenate([slot_pos, np.full(C - n_live, 1 << 30, np.int32)])
    r16, r32 = orc.attention_h2o(_u16(q), rkf, rvf, rks, rvs, sp_full, n_live, r_attn, S, past)
    d_attn = torch.from_numpy(attn0.copy()).to(dev)
    out = torch.zeros((S, 32, 64), dtype=torch.float16, device=dev)
    ws = torch.zeros(K.h2o_workspace_bytes(S, n_live), dtype=torch.uint8, device=dev)
    print(f"attention_h2o n_live={n_live} S={S} past={past}", flush=True)
    K.attention_h2o(q.to(dev), kf, vf, ks, vs, torch.from_numpy(sp_full).to(dev), n_live, out,
                    d_attn, S, past, 0.125, ws)
    torch.cuda.synchronize()
    got = d_attn.cpu().numpy()
    if not np.array_equal(got.view(np.uint32), r_attn.view(np.uint32)):
        i = int(np.argmax(got.view(np.uint32) != r_attn.view(np.uint32)))
        raise AssertionError(f"attn_sum differs at slot {i}: {got[i]!r} vs {r_attn[i]!r}")
    assert_close_f16(_u16(out), r32, what="attention_h2o")


def test_h2o_layers_sharing_ws_mass(cia, dev):
    """Two H2O layers that share one ws_mass, run through the decode loop:
    each step's mass launch leaves the next step's placement keys in the
    shared scratch, tagged with its layer's attn_sum and position, so the
    other layer's scores launch sees a foreign tag and scans every slot.
    Evictions, masses, positions, FP8 bytes and outputs are bit-identical
    to the same two layers with a scratch each."""
    import ctypes
    from cuda_inf_amd import _lib
    from cuda_inf_amd._lib import call
    from cuda_inf_amd.layer import AttnLayer
    from cuda_inf_amd.workload import qkv
    C, W, P, N, nL = 256, 32, 256, 160, 2
    q, k, v = qkv((P + N) * nL, seed=31, device="cpu", prep=False)
    q = q.view(P + N, nL, 32, 64).to(dev)
    k = k.view(P + N, nL, 8, 64).to(dev)
    v = v.view(P + N, nL, 8, 64).to(dev)
    runs = []
    for shared in (False, True):
        layers = [AttnLayer(P + N + 4, budget=C, window=W, prompt_len=P, max_batch=P, device=dev)
                  for _ in range(nL)]
        for l, L in enumerate(layers):
            L.forward(q[:P, l].contiguous(), k[:P, l].contiguous(), v[:P, l].contiguous(), 0,
                      evicted=False)
        if shared:
            layers[1]._s.ws_mass = layers[0].ws_mass.data_ptr()
        arr = (_lib.cia_layer * nL)(*[L._s for L in layers])
        out = torch.zeros((N, nL, 32, 64), dtype=torch.float16, device=dev)
        call("cia_decode_loop", arr, nL, q[P].data_ptr(), k[P].data_ptr(), v[P].data_ptr(),
             out.data_ptr(), P, N, 0.125, None, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        runs.append((layers, out))
    (la, oa), (lb, ob) = runs
    assert torch.equal(oa.view(torch.int16), ob.view(torch.int16)), "outputs differ"
    for l in range(nL):
        for name in ("hattn", "d_slotpos", "kf", "vf", "ks", "vs"):
            x, y = getattr(la[l], name), getattr(lb[l], name)
            assert torch.equal(x.view(torch.uint8), y.view(torch.uint8)), (l, name)
