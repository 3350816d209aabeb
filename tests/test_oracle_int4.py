"""Pins the oracle's INT4 group-128 weight format (tools/export_weights.py:
64-79) and its GEMV (engine.cu:83-109) by closed forms and by an
independent formulation: the packed bytes are unpacked with numpy into a
dense fp64 matrix and multiplied with numpy's own matrix product.
"""
import numpy as np

G = 128


def _dense(packed, scales):
    """Dequantised W [N, K] in fp64, unpacked with numpy (low nibble = even k)."""
    N, half = packed.shape
    nib = np.empty((N, 2 * half), np.int64)
    nib[:, 0::2] = packed & 0xF
    nib[:, 1::2] = packed >> 4
    sc = scales.view(np.float16).astype(np.float64)
    return (nib - 8) * np.repeat(sc, G, axis=1)


def _f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def test_quant_ties_round_half_even(orc):
    w = np.zeros((1, G), np.float32)
    vals = [7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 6.5, -6.5, 4.4, -4.6]
    w[0, :len(vals)] = vals  # amax 7 -> scale exactly 1
    packed, scales = orc.quant_int4_g128(w)
    assert scales[0, 0] == np.float16(1.0).view(np.uint16)
    nib = np.empty(G, np.int64)
    nib[0::2] = packed[0] & 0xF
    nib[1::2] = packed[0] >> 4
    want = [15, 8, 10, 10, 8, 6, 6, 12, 14, 2, 12, 3]
    assert list(nib[:len(want)]) == want
    assert np.all(nib[len(want):] == 8)


def test_quant_zero_group_and_single_elements(orc):
    K = 4 * G
    w = np.zeros((3, K), np.float32)
    packed, scales = orc.quant_int4_g128(w)
    assert np.all(packed == 0x88) and np.all(scales == 0)
    # one non-zero element per row at even k, odd k, in different groups
    for k in (0, 1, 2 * G + 37, 3 * G + 126, 3 * G + 127):
        w = np.zeros((2, K), np.float32)
        w[1, k] = -3.0
        packed, scales = orc.quant_int4_g128(w)
        assert np.all(packed[0] == 0x88) and np.all(scales[0] == 0)
        g = k // G
        want_sc = np.zeros(K // G, np.uint16)
        want_sc[g] = np.float16(np.float32(3.0) / np.float32(7.0)).view(np.uint16)
        assert np.array_equal(scales[1], want_sc)
        want = np.full(K // 2, 0x88, np.uint8)
        want[k // 2] = 0x81 if k % 2 == 0 else 0x18  # -7 -> nibble 1
        assert np.array_equal(packed[1], want)


def test_quant_error_bound_and_amax(orc):
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float32)
    w[3, 200] = 0.5  # an outlier dominates its group
    packed, scales = orc.quant_int4_g128(w)
    nib = np.empty(w.shape, np.int64)
    nib[:, 0::2] = packed & 0xF
    nib[:, 1::2] = packed >> 4
    assert nib.min() >= 1 and nib.max() <= 15
    wg = w.reshape(64, -1, G).astype(np.float64)
    amax = np.abs(wg).max(axis=2)
    s32 = (amax / 7.0).astype(np.float32).astype(np.float64)
    err = np.abs(wg - (nib.reshape(64, -1, G) - 8) * s32[..., None])
    assert np.all(err <= s32[..., None] * 0.5 * (1 + 1e-6))
    # the element of largest magnitude lands on +-7
    idx = np.abs(wg).argmax(axis=2)
    top = np.take_along_axis(nib.reshape(64, -1, G), idx[..., None], axis=2)[..., 0]
    assert np.all((top == 1) | (top == 15))
    assert np.array_equal(scales, _f16(s32.astype(np.float32)))


def test_gemv_matches_dense_fp64_product(orc):
    rng = np.random.default_rng(11)
    N, K, M = 96, 2048, 3
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    packed, scales = orc.quant_int4_g128(w)
    x = _f16(rng.standard_normal((M, K)))
    y, ab = orc.gemv_int4(x, packed, scales, want_absum=True)
    W = _dense(packed, scales)
    xf = x.view(np.float16).astype(np.float64)
    ref = xf @ W.T
    assert np.all(np.abs(y - ref) <= 1e-7 * np.abs(xf) @ np.abs(W).T + 1e-30)
    assert np.allclose(ab, np.abs(xf) @ np.abs(W).T, rtol=1e-6)


def test_gemv_closed_forms(orc):
    rng = np.random.default_rng(2)
    N, K = 16, 512
    w = (rng.standard_normal((N, K))).astype(np.float32)
    packed, scales = orc.quant_int4_g128(w)
    W = _dense(packed, scales)
    # one-hot x picks one dequantised column exactly
    for k in (0, 1, 255, 511):
        x = np.zeros((1, K), np.float32)
        x[0, k] = 1.0
        y = orc.gemv_int4(_f16(x), packed, scales)
        assert np.array_equal(y[0], W[:, k].astype(np.float32))
    # constant nibble 9 (w = +1 * scale) with one scale s: y = s * sum(x)
    packed = np.full((N, K // 2), 0x99, np.uint8)
    s = np.float16(0.375)
    scales = np.full((N, K // G), s.view(np.uint16), np.uint16)
    x = _f16(rng.standard_normal((2, K)))
    y = orc.gemv_int4(x, packed, scales)
    want = (x.view(np.float16).astype(np.float64).sum(axis=1) * float(s)).astype(np.float32)
    assert np.array_equal(y, np.repeat(want[:, None], N, axis=1))
