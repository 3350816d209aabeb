"""Pins the oracle's QK producers (engine.cu:148-182): the deterministic
sin/cos, the RoPE frequency table, and RMSNorm + RoPE on head rows.

The RMSNorm part and the rotation are restated independently in numpy
float32 (same operation order: the reference's tree sum of squares, IEEE
sqrt and division, fp16 after each stage); sincos_det itself is pinned by its
error against float64 sin/cos, exact values and symmetry.
"""
import numpy as np
import pytest

D = 64


def test_sincos_det_accuracy(orc):
    x = np.linspace(0.0, 2.6e5, 2_000_001, dtype=np.float32)
    s, c = orc.sincos_det(x)
    xd = x.astype(np.float64)
    assert np.abs(s - np.sin(xd)).max() < 2e-7
    assert np.abs(c - np.cos(xd)).max() < 2e-7
    # small angles: relative accuracy of sin
    t = np.logspace(-30, 0, 2000).astype(np.float32)
    st, ct = orc.sincos_det(t)
    assert np.all(np.abs(st - np.sin(t.astype(np.float64))) <= 2e-7 * np.abs(np.sin(t.astype(np.float64))) + 1e-45)
    assert np.all(np.abs(ct - np.cos(t.astype(np.float64))) < 2e-7)


def test_sincos_det_exact_points_and_symmetry(orc):
    s, c = orc.sincos_det(np.array([0.0, -0.0], np.float32))
    assert s[0] == 0.0 and not np.signbit(s[0]) and c[0] == 1.0 and s[1] == 0.0 and c[1] == 1.0
    x = np.random.default_rng(1).uniform(-1e5, 1e5, 100_000).astype(np.float32)
    s1, c1 = orc.sincos_det(x)
    s2, c2 = orc.sincos_det(-x)
    assert np.array_equal(s2.view(np.uint32), (-s1).view(np.uint32))   # odd, bit for bit
    assert np.array_equal(c2.view(np.uint32), c1.view(np.uint32))      # even, bit for bit
    assert np.abs(s1 * s1 + c1 * c1 - 1.0).max() < 1e-6


def test_rope_invf_table(orc):
    for theta in (5.0e6, 1.0e4):
        got = orc.rope_invf(theta)
        want = np.array([np.float32(theta ** (-(2.0 * i) / D)) for i in range(32)], np.float32)
        assert np.array_equal(got, want)
        assert got[0] == 1.0


def _np_norm(x16, w16, eps):
    """numpy float32 restatement of rmsnorm_head (engine.cu:148-158)."""
    x = x16.astype(np.float32)
    v = x * x
    st = D // 2
    while st:
        v = v[..., :st] + v[..., st:2 * st]
        st //= 2
    ss = v[..., 0:1]
    inv = np.float32(1.0) / np.sqrt(ss / np.float32(D) + np.float32(eps))
    return ((x * inv) * w16.astype(np.float32)).astype(np.float16)


def _np_rope(y16, pos, sn, cs):
    y = y16.astype(np.float32)
    y0, y1 = y[..., :32], y[..., 32:]
    s = sn[:, None, :]
    c = cs[:, None, :]
    return np.concatenate([(y0 * c - y1 * s), (y1 * c + y0 * s)], -1).astype(np.float16)


@pytest.mark.parametrize("seed,pmax", [(0, 4096), (1, 131072), (2, 10)])
def test_qk_norm_rope_restated(orc, seed, pmax):
    rng = np.random.default_rng(seed)
    S = 37
    q = (rng.standard_normal((S, 32, D)) * rng.uniform(0.01, 30, (S, 32, 1))).astype(np.float16)
    k = (rng.standard_normal((S, 8, D)) * rng.uniform(0.01, 30, (S, 8, 1))).astype(np.float16)
    k[3, 2] = 0  # a zero row stays zero
    qw = rng.uniform(0.5, 1.5, D).astype(np.float16)
    kw = rng.uniform(0.5, 1.5, D).astype(np.float16)
    pos = rng.integers(0, pmax, S).astype(np.int32)
    pos[0] = 0
    qo, ko = orc.qk_norm_rope(q, k, qw, kw, pos)
    invf = orc.rope_invf(5.0e6)
    ang = (pos.astype(np.float32)[:, None] * invf[None, :]).astype(np.float32)
    sn, cs = orc.sincos_det(ang)
    for x, w, o in ((q, qw, qo), (k, kw, ko)):
        want = _np_rope(_np_norm(x, w, 1e-5), pos, sn, cs)
        assert np.array_equal(o, want.view(np.uint16))
    # position 0: RoPE is the identity
    assert np.array_equal(qo[0], _np_norm(q[0], qw, 1e-5).view(np.uint16))
    assert not ko[3, 2].view(np.float16).astype(np.float32).any()  # +-0


def test_qk_norm_rope_properties(orc):
    """Unit weight: each normalised row has RMS 1; RoPE keeps pair norms."""
    rng = np.random.default_rng(5)
    S = 64
    q = (rng.standard_normal((S, 32, D)) * 3).astype(np.float16)
    k = rng.standard_normal((S, 8, D)).astype(np.float16)
    ones = np.ones(D, np.float16)
    pos = np.arange(S, dtype=np.int32) * 977
    qo, ko = orc.qk_norm_rope(q, k, ones, ones, pos)
    y = qo.view(np.float16).astype(np.float64)
    rms = np.sqrt((y * y).mean(-1))
    assert np.abs(rms - 1.0).max() < 2e-3
    n0 = _np_norm(q, ones, 1e-5).astype(np.float64)
    pair_before = n0[..., :32] ** 2 + n0[..., 32:] ** 2
    pair_after = y[..., :32] ** 2 + y[..., 32:] ** 2
    assert np.abs(pair_after - pair_before).max() < 2e-2


def test_qk_norm_rope_matches_torch_prep(orc):
    """The torch producers of the workloads (fp32 torch cos/sin and sums):
    equal up to one fp16 rounding step."""
    import torch
    from cuda_inf_amd.workload import prep_qk
    rng = np.random.default_rng(9)
    S = 50
    q = rng.standard_normal((S, 32, D)).astype(np.float16)
    k = rng.standard_normal((S, 8, D)).astype(np.float16)
    pos = (np.arange(S) * 311).astype(np.int32)
    ones = np.ones(D, np.float16)
    qo, ko = orc.qk_norm_rope(q, k, ones, ones, pos)
    tq = prep_qk(torch.from_numpy(q), torch.from_numpy(pos.astype(np.int64))).numpy()
    diff = np.abs(qo.view(np.float16).astype(np.float32) - tq.astype(np.float32))
    assert diff.max() <= 4e-3
    assert (diff > 0).mean() < 0.05
