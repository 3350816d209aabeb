"""GPU parity of the INT4 group-128 projections (engine.cu:83-109, launched
at 626-630, 792-797, 858-859) through the C-ABI, against the oracle.

The GPU sums in fp32 in its own order, the oracle in fp64; the tolerance is
written against the scale of the summation error:
    |y_gpu - y_ref| <= 1e-5 * sum_k |x[k] * w[n][k]|
(fp32 sums of a few thousand terms stay orders of magnitude inside it; one
dropped or doubled term of typical size is ~1/K of the sum of magnitudes,
about 50x the bound at K = 2048)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

REL = 1e-5


def _weights(rng, N, K, orc, kind="normal"):
    if kind == "normal":
        w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        w[rng.integers(0, N, 8), rng.integers(0, K, 8)] *= 30.0  # outliers set their groups' scales
        return orc.quant_int4_g128(w)
    if kind == "extreme":  # nibbles 0 (-8) and 15 (+7), zero-scale groups
        packed = rng.choice(np.array([0x00, 0xFF, 0x0F, 0xF0, 0x88], np.uint8), (N, K // 2))
        scales = rng.uniform(0.001, 0.5, (N, K // 128)).astype(np.float16).view(np.uint16)
        scales[:, ::3] = 0
        return packed, scales
    raise ValueError(kind)


def _t(a, dev):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to(dev)


def _check(got, ref, ab, what, extra=0.0):
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bound = REL * ab.astype(np.float64) + extra + 1e-30
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside; worst at {i}: "
                             f"got {got[i]} ref {ref[i]} absum {ab[i]}")


CASES = [
    (2048, 2048, 1, "normal", 0),   # q_proj / out_proj at decode
    (512, 2048, 1, "normal", 1),    # k_proj / v_proj
    (96, 128, 1, "normal", 2),      # one group per row
    (100, 384, 3, "normal", 3),     # ragged rows, K < 2048, three rows of x
    (33, 2176, 5, "normal", 4),     # K = 17 groups: a second, partial lane pass
    (2048, 4096, 2, "normal", 5),
    (64, 2048, 1, "extreme", 6),
    (512, 2048, 9, "normal", 7),
    (2048, 2048, 96, "normal", 8),   # matrix-core path from 56 rows of x
    (100, 384, 200, "normal", 9),    # ragged tiles in both directions
    (520, 2048, 300, "extreme", 13),
]


@pytest.mark.parametrize("N,K,M,kind,seed", CASES)
def test_gemv_int4(orc, cia, dev, N, K, M, kind, seed):
    from cuda_inf_amd import kernels as KK
    rng = np.random.default_rng(seed)
    packed, scales = _weights(rng, N, K, orc, kind)
    x = rng.standard_normal((M, K)).astype(np.float16)
    ref, ab = orc.gemv_int4(x, packed, scales, want_absum=True)
    print(f"gemv_int4 N={N} K={K} M={M} {kind}", flush=True)
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    KK.gemv_int4(_t(x, dev), _t(packed, dev), _t(scales, dev), y, N, K, M)
    torch.cuda.synchronize()
    _check(y.cpu().numpy(), ref, ab, "y")
    # out_proj + residual: y += x W^T
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    yd = torch.from_numpy(y0).to(dev)
    KK.gemv_int4(_t(x, dev), _t(packed, dev), _t(scales, dev), yd, N, K, M, add=True)
    torch.cuda.synchronize()
    _check(yd.cpu().numpy(), y0.astype(np.float64) + ref, ab, "y + residual",
           extra=2 * np.finfo(np.float32).eps * (np.abs(y0) + np.abs(ref)))


@pytest.mark.parametrize("M,seed", [(1, 10), (3, 11), (6, 12), (130, 14)])
def test_qkv_proj_int4(orc, cia, dev, M, seed):
    """q/k/v in one launch with the fp16 conversion fused: each output is
    the fp16 rounding of the same kernel's fp32 sum (compared with the fp32
    GEMV bit for bit) and within tolerance of the oracle."""
    from cuda_inf_amd import kernels as KK
    rng = np.random.default_rng(seed)
    K = 2048
    W = {n: _weights(rng, N, K, orc) for n, N in (("q", 2048), ("k", 512), ("v", 512))}
    x = (rng.standard_normal((M, K)) * 0.5).astype(np.float16)
    xd = _t(x, dev)
    Wd = {n: (_t(p, dev), _t(s, dev)) for n, (p, s) in W.items()}
    out = {n: torch.zeros((M, N), dtype=torch.float16, device=dev)
           for n, N in (("q", 2048), ("k", 512), ("v", 512))}
    print(f"qkv_proj_int4 M={M}", flush=True)
    KK.qkv_proj_int4(xd, Wd["q"], Wd["k"], Wd["v"], out["q"], out["k"], out["v"], M, K)
    torch.cuda.synchronize()
    for n in ("q", "k", "v"):
        N = out[n].shape[1]
        y = torch.zeros((M, N), dtype=torch.float32, device=dev)
        KK.gemv_int4(xd, Wd[n][0], Wd[n][1], y, N, K, M)
        torch.cuda.synchronize()
        want16 = y.cpu().numpy().astype(np.float16)
        got16 = out[n].cpu().numpy()
        assert np.array_equal(got16.view(np.uint16), want16.view(np.uint16)), n
        ref, ab = orc.gemv_int4(x, *W[n], want_absum=True)
        _check(got16.astype(np.float32), ref, ab, n,
               extra=np.abs(ref) * 2.0 ** -11 + 2.0 ** -25)
