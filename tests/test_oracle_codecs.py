"""Pins the oracle's scalar codecs to their definitions (CPU only).

* fp32 -> fp16: all 2^32 inputs against numpy's cast (an independent IEEE
  round-to-nearest-even implementation).
* E4M3 (OCP OFP8): the 256-code table from the closed form; every decision
  threshold between neighbouring codes (midpoint ties to the even code, one
  ulp either side to the neighbours); saturation at and beyond 448 and for
  infinities; signed zero; NaN; and a brute-force nearest-code search on
  random inputs.
* exp_det: error against float64 exp and its special values.
* quant_scale: closed forms.
"""
import numpy as np
import pytest


def closed_form_e4m3(b: int) -> float:
    e, m = (b >> 3) & 0xF, b & 7
    if e == 15 and m == 7:
        v = float("nan")
    elif e == 0:
        v = m / 512.0
    else:
        v = 2.0 ** (e - 7) * (1 + m / 8.0)
    return -v if b & 0x80 else v


def test_e4m3_decode_table(orc):
    t = orc.e4m3_decode_table()
    for b in range(256):
        ref = closed_form_e4m3(b)
        if np.isnan(ref):
            assert np.isnan(t[b]) and b in (0x7F, 0xFF)
        else:
            assert t[b] == np.float32(ref), hex(b)
    assert t[0x7E] == 448.0 and t[0x01] == 2.0 ** -9 and t[0x08] == 2.0 ** -6


def _codes_sorted():
    """finite non-negative codes 0x00..0x7E and their values (increasing)."""
    codes = np.arange(0x7F)
    vals = np.array([closed_form_e4m3(int(c)) for c in codes])
    assert np.all(np.diff(vals) > 0)
    return codes, vals


def nearest_code(x: np.ndarray) -> np.ndarray:
    """Brute-force RNE SATFINITE encode by searching the code table
    (independent of the oracle's bit manipulation)."""
    codes, vals = _codes_sorted()
    ax = np.abs(x.astype(np.float64))
    sign = np.signbit(x).astype(np.uint8) << 7
    i = np.clip(np.searchsorted(vals, ax), 1, len(vals) - 1)
    lo, hi = vals[i - 1], vals[i]
    pick_hi = (ax - lo > hi - ax) | ((ax - lo == hi - ax) & ((codes[i] & 1) == 0))
    c = np.where(pick_hi, codes[i], codes[i - 1])
    c = np.where(ax >= 448.0, 0x7E, c)
    c = np.where(ax <= vals[0], 0, c)
    out = (c.astype(np.uint8) | sign)
    return np.where(np.isnan(x), 0x7F | sign, out).astype(np.uint8)


def test_e4m3_thresholds(orc):
    codes, vals = _codes_sorted()
    xs, want = [], []
    for i in range(len(vals) - 1):
        a, b = vals[i], vals[i + 1]
        mid = np.float32((a + b) / 2)
        assert float(mid) == (a + b) / 2  # exact in fp32
        even = codes[i] if codes[i] % 2 == 0 else codes[i + 1]
        for s in (1.0, -1.0):
            sb = 0x80 if s < 0 else 0
            xs += [s * mid, s * np.nextafter(mid, np.float32(np.inf)),
                   s * np.nextafter(mid, np.float32(0)), s * np.float32(a), s * np.float32(b)]
            want += [even | sb, codes[i + 1] | sb, codes[i] | sb, codes[i] | sb, codes[i + 1] | sb]
    got = orc.e4m3_encode(np.array(xs, np.float32))
    assert np.array_equal(got, np.array(want, np.uint8))


def test_e4m3_special_values(orc):
    f = np.float32
    cases = [(0.0, 0x00), (-0.0, 0x80), (448.0, 0x7E), (-448.0, 0xFE), (464.0, 0x7E),
             (480.0, 0x7E), (1e30, 0x7E), (-3e38, 0xFE), (np.inf, 0x7E), (-np.inf, 0xFE),
             (2.0 ** -10, 0x00), (-(2.0 ** -10), 0x80), (1e-30, 0x00), (-1e-45, 0x80),
             (2.0 ** -10 * 1.0001, 0x01), (3 * 2.0 ** -10, 0x02), (2.0 ** -6, 0x08),
             (float(np.nextafter(f(2.0 ** -6), f(0))), 0x08), (1.0, 0x38), (1.0625, 0x38),
             (1.0625001, 0x39), (1.1875, 0x3A)]
    xs = np.array([c[0] for c in cases], np.float32)
    got = orc.e4m3_encode(xs)
    for x, g, (_, w) in zip(xs, got, cases):
        assert g == w, f"{x!r}: 0x{g:02x} != 0x{w:02x}"
    nan = np.array([np.nan, -np.nan], np.float32)
    nan[1] = -abs(nan[1])
    assert list(orc.e4m3_encode(nan)) == [0x7F, 0xFF]


def test_e4m3_brute_force_random(orc):
    rng = np.random.default_rng(1)
    mag = np.exp2(rng.uniform(-14, 10, 2_000_000)).astype(np.float32)
    x = np.where(rng.random(mag.size) < 0.5, -mag, mag).astype(np.float32)
    x[:1000] = rng.standard_normal(1000).astype(np.float32)
    assert np.array_equal(orc.e4m3_encode(x), nearest_code(x))


def test_e4m3_monotone(orc):
    x = np.sort(np.random.default_rng(2).uniform(-500, 500, 1_000_000).astype(np.float32))
    t = orc.e4m3_decode_table()
    v = t[orc.e4m3_encode(x)]
    assert np.all(np.diff(v) >= 0)


def _f16_inputs():
    """Every fp32 exponent and sign, with all 2^10 kept-mantissa patterns and
    the rounding-relevant low bits (0, 1, half-1, half, half+1, max) for both
    the normal (13 dropped bits) and the subnormal-output regimes, plus 2^24
    random patterns.  CIA_EXHAUSTIVE=1 runs all 2^32 inputs instead."""
    e = np.arange(256, dtype=np.uint32)[:, None, None]
    top = np.arange(1024, dtype=np.uint32)[None, :, None] << 13
    low = np.array([0, 1, 0xFFF, 0x1000, 0x1001, 0x1FFF], np.uint32)[None, None, :]
    a = ((e << 23) | top | low).ravel()
    # subnormal-output region: dropped-bit count 14..24, probe its half point
    sub = []
    for ex in range(102, 113):
        shift = 126 - ex
        half = 1 << (shift - 1)
        for r in (0, 1, half - 1, half, half + 1, (1 << shift) - 1):
            m = (np.arange(0, 1 << 23, 1 << max(shift, 1), dtype=np.uint32) | r) & 0x7FFFFF
            sub.append((np.uint32(ex) << 23) | m)
    a = np.concatenate([a] + sub)
    a = np.concatenate([a, a | 0x80000000,
                        np.random.default_rng(3).integers(0, 1 << 32, 1 << 24, dtype=np.uint64)
                        .astype(np.uint32)])
    return [a]


def test_f16_exhaustive(orc):
    import os
    if os.environ.get("CIA_EXHAUSTIVE") == "1":
        step = 1 << 24
        chunks = (np.arange(s, s + step, dtype=np.uint64).astype(np.uint32)
                  for s in range(0, 1 << 32, step))
    else:
        chunks = _f16_inputs()
    for u in chunks:
        x = u.view(np.float32)
        got = orc.f32_to_f16(x)
        with np.errstate(over="ignore", invalid="ignore"):
            ref = x.astype(np.float16).view(np.uint16)
        nan = np.isnan(x)
        if not np.array_equal(got[~nan], ref[~nan]):
            i = np.nonzero((got != ref) & ~nan)[0][0]
            raise AssertionError(f"bits 0x{u[i]:08x}: 0x{got[i]:04x} vs numpy 0x{ref[i]:04x}")
        g = got[nan]
        assert np.all(((g & 0x7C00) == 0x7C00) & ((g & 0x3FF) != 0))


def test_exp_det_accuracy(orc):
    x = np.linspace(-60, 88, 3_000_001).astype(np.float32)
    x = np.concatenate([x, np.float32([0.0, -0.0, 1e-8, -1e-8, -59.999996])])
    e = orc.exp_det(x).astype(np.float64)
    r = np.exp(x.astype(np.float64))
    rel = np.abs(e - r) / r
    assert rel.max() < 2.5 * 2.0 ** -24, rel.max()
    assert orc.exp_det(np.float32([0.0]))[0] == 1.0
    assert orc.exp_det(np.float32([-60.5, -1e30, -np.inf]))[0] == 0.0
    assert np.all(orc.exp_det(np.float32([-60.5, -1e30, -np.inf])) == 0.0)
    assert np.isnan(orc.exp_det(np.float32([np.nan]))[0])
    # monotone on a fine sweep
    y = orc.exp_det(np.linspace(-20, 0, 1_000_001).astype(np.float32))
    assert np.all(np.diff(y) >= 0)


@pytest.mark.parametrize("amax", [0.0, 1.0, 448.0, 3.75, 65504.0, 6.0e-8, 1e-20])
def test_quant_scale_closed_form(orc, amax):
    a = np.float32(amax)
    want = np.float32(a / np.float32(448.0)) + np.float32(1e-12)
    assert np.float32(orc.quant_scale(float(a))) == np.float32(want)
    if amax == 0.0:
        assert orc.f32_to_f16(np.float32([orc.quant_scale(0.0)]))[0] == 0
    if amax == 448.0:
        assert orc.quant_scale(448.0) == 1.0
