"""Pins the oracle's cache writers, attention restatements and H2O mass (CPU).

* kv_commit_group / kv_quant_write (engine.cu:202-228, 317-333) against an
  independent numpy restatement (float32 IEEE arithmetic and a table-search
  E4M3 encoder), plus closed forms (zero group, single element, constant).
* kv_append (engine.cu:830-845): tail contents and committed groups equal a
  direct commit of each 64-token group.
* attention_fused / attn_decode_split+combine / attention_h2o outputs
  against fp64 softmax attention on the dequantised cache, and invariants
  (all-equal V, one key, q = 0 gives the mean of V, split counts agree,
  empty splits are skipped, decode equals the fused last row).
* The deterministic attention mass against an fp64 restatement, its total
  (one per query head), and a one-hot construction with a closed form.
"""
import numpy as np
import pytest

from test_oracle_codecs import closed_form_e4m3, nearest_code

NH, NKV, D = 32, 8, 64
TABLE = np.array([closed_form_e4m3(b) for b in range(256)], np.float64)


def f16(x):
    return np.asarray(x, np.float32).astype(np.float16)


def bits(a16):
    return np.ascontiguousarray(a16).view(np.uint16)


def rand_f16(rng, shape, scale=1.0, outliers=0.0):
    x = rng.standard_normal(shape) * scale
    if outliers:
        x = np.where(rng.random(shape) < outliers, x * 20, x)
    return f16(x)


def np_commit(tail16):
    """numpy restatement of one group commit: [64,8,64] fp16 -> bytes, scales."""
    x = tail16.astype(np.float32)
    amax = np.abs(x).max(axis=(0, 2))                       # per kv head
    sc = (amax / np.float32(448.0)).astype(np.float32) + np.float32(1e-12)
    q = (x / sc[None, :, None]).astype(np.float32)
    return nearest_code(q), sc.astype(np.float16)


@pytest.mark.parametrize("kind", ["normal", "outliers", "zero", "single", "const", "tiny"])
def test_commit_matches_numpy(orc, kind):
    rng = np.random.default_rng(hash(kind) % 997)
    k = rand_f16(rng, (64, NKV, D), outliers=0.01 if kind == "outliers" else 0)
    if kind == "zero":
        k[:] = 0
    elif kind == "single":
        k[:] = 0
        k[10, 2, 7] = -3.5
    elif kind == "const":
        k[:] = f16(0.3)
    elif kind == "tiny":
        k = f16(k.astype(np.float32) * 1e-6)
    v = rand_f16(rng, (64, NKV, D))
    kc8 = np.zeros((128, NKV, D), np.uint8)
    vc8 = np.zeros_like(kc8)
    ksc = np.zeros((4, NKV), np.uint16)
    vsc = np.zeros_like(ksc)
    orc.kv_commit_group(bits(k), bits(v), kc8, vc8, ksc, vsc, 64, 1)
    want_b, want_s = np_commit(k)
    assert np.array_equal(kc8[64:], want_b)
    assert np.array_equal(ksc[1], bits(want_s))
    assert np.all(kc8[:64] == 0) and np.all(ksc[0] == 0)
    if kind == "zero":
        assert np.all(ksc[1] == 0) and np.all(kc8[64:] == 0)
    if kind == "single":
        assert kc8[64 + 10, 2, 7] == 0xFE and np.count_nonzero(kc8[64:, 2]) == 1
    if kind == "const":
        assert np.all(kc8[64:] == 0x7E)


def test_quant_write_matches_numpy(orc):
    rng = np.random.default_rng(3)
    S, C = 40, 64
    k = rand_f16(rng, (S, NKV, D), outliers=0.02)
    v = rand_f16(rng, (S, NKV, D))
    k[3] = 0
    dst = rng.permutation(C)[:S].astype(np.int32)
    kf = np.zeros((C, NKV, D), np.uint8)
    vf = np.zeros_like(kf)
    ks = np.zeros((C, NKV), np.uint16)
    vs = np.zeros_like(ks)
    orc.kv_quant_write(bits(k), bits(v), kf, vf, ks, vs, dst)
    for j in range(S):
        x = k[j].astype(np.float32)
        amax = np.abs(x).max(axis=1)
        sc = (amax / np.float32(448.0)).astype(np.float32) + np.float32(1e-12)
        assert np.array_equal(kf[dst[j]], nearest_code((x / sc[:, None]).astype(np.float32)))
        assert np.array_equal(ks[dst[j]], bits(sc.astype(np.float16)))


def test_append_equals_direct_commits(orc):
    rng = np.random.default_rng(7)
    total = 0
    batches = [1, 70, 63, 1, 64, 129, 5]
    n = sum(batches)
    k = rand_f16(rng, (n, NKV, D))
    v = rand_f16(rng, (n, NKV, D))
    c = orc.Group64Cache(n + 64)
    for S in batches:
        c.append(bits(k[total:total + S]), bits(v[total:total + S]), total)
        total += S
    assert c.committed == (n // 64) * 64
    for g in range(n // 64):
        kb, ks = np_commit(k[64 * g:64 * g + 64])
        assert np.array_equal(c.kc8[64 * g:64 * g + 64], kb)
        assert np.array_equal(c.ksc[g], bits(ks))
    rest = n - c.committed
    assert np.array_equal(c.ktail[:rest], bits(k[c.committed:]))


# ---------------------------------------------------------------- attention
def dequant_cache(c, T):
    """fp64 K, V [T, 8, 64] from the oracle's cache (FP8 rows and the tail)."""
    K = np.zeros((T, NKV, D))
    V = np.zeros((T, NKV, D))
    for t in range(T):
        if t < c.committed:
            g = t // 64
            ks = c.ksc[g].view(np.float16).astype(np.float64)
            vs = c.vsc[g].view(np.float16).astype(np.float64)
            K[t] = TABLE[c.kc8[t]] * ks[:, None]
            V[t] = TABLE[c.vc8[t]] * vs[:, None]
        else:
            K[t] = c.ktail[t - c.committed].view(np.float16)
            V[t] = c.vtail[t - c.committed].view(np.float16)
    return K, V


def brute_attention(q16, K, V, S, past, scale=0.125):
    q = q16.astype(np.float64)
    out = np.zeros((S, NH, D))
    for i in range(S):
        T = past + i + 1
        for h in range(NH):
            s = (K[:T, h // 4] @ q[i, h]) * scale
            p = np.exp(s - s.max())
            out[i, h] = (p @ V[:T, h // 4]) / p.sum()
    return out


def make_cache(orc, rng, n, outliers=0.01):
    k = rand_f16(rng, (n, NKV, D), outliers=outliers)
    v = rand_f16(rng, (n, NKV, D), outliers=outliers)
    c = orc.Group64Cache(n + 64)
    c.append(bits(k), bits(v), 0)
    return c, k, v


@pytest.mark.parametrize("S,past", [(1, 0), (70, 0), (25, 100), (64, 64)])
def test_fused_against_fp64(orc, S, past):
    rng = np.random.default_rng(S + past)
    c, _, _ = make_cache(orc, rng, past + S)
    q = rand_f16(rng, (S, NH, D))
    o16, o32 = orc.attention_fused(bits(q), c, S, past)
    K, V = dequant_cache(c, past + S)
    ref = brute_attention(q, K, V, S, past)
    np.testing.assert_allclose(o32, ref, rtol=2e-5, atol=1e-5)
    assert np.array_equal(o16, bits(f16(o32)))


def test_fused_invariants(orc):
    rng = np.random.default_rng(11)
    S = 30
    k = rand_f16(rng, (S, NKV, D))
    v = np.broadcast_to(rand_f16(rng, (1, NKV, D)), (S, NKV, D)).copy()
    c = orc.Group64Cache(S + 64)
    c.append(bits(k), bits(v), 0)
    q = rand_f16(rng, (S, NH, D))
    _, o32 = orc.attention_fused(bits(q), c, S, 0)
    vv = v[0].astype(np.float32)
    np.testing.assert_allclose(o32, np.repeat(vv, 4, axis=0)[None].repeat(S, 0), rtol=1e-6)
    # one key: output is that key's value
    np.testing.assert_allclose(o32[0], np.repeat(vv, 4, axis=0), rtol=0, atol=0)
    # q = 0: uniform weights -> mean of V over visible keys
    v2 = rand_f16(rng, (S, NKV, D))
    c2 = orc.Group64Cache(S + 64)
    c2.append(bits(k), bits(v2), 0)
    _, o0 = orc.attention_fused(bits(np.zeros((S, NH, D), np.float16)), c2, S, 0)
    for i in (0, 9, 29):
        mean = v2[:i + 1].astype(np.float64).mean(0)
        np.testing.assert_allclose(o0[i], np.repeat(mean, 4, axis=0), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("S,past", [(40, 100), (70, 0), (1, 63)])
def test_fused_attn_sum_against_fp64(orc, S, past):
    """attention_fused's attn_sum (oracle.c:488-491, engine.cu:291-307): the
    mass each key receives, summed over the S queries and 32 heads, added
    onto the existing values; against softmax in fp64 on the dequantised
    cache, and the total added is S * 32 (each softmax sums to 1)."""
    rng = np.random.default_rng(100 + S + past)
    c, _, _ = make_cache(orc, rng, past + S)
    q = rand_f16(rng, (S, NH, D))
    T = past + S
    start = rng.uniform(0.0, 5.0, T).astype(np.float32)
    asum = start.copy()
    orc.attention_fused(bits(q), c, S, past, attn_sum=asum)
    K, V = dequant_cache(c, T)
    mass = np.zeros(T)
    for i in range(S):
        n = past + i + 1
        for h in range(NH):
            sc = (K[:n, h // 4] @ q[i, h].astype(np.float64)) * 0.125
            p = np.exp(sc - sc.max())
            mass[:n] += p / p.sum()
    added = asum.astype(np.float64) - start.astype(np.float64)
    # S * 32 fp32 adds per key into accumulators up to ~S * 32: rounding ~1e-7 relative each
    np.testing.assert_allclose(added, mass, rtol=1e-4, atol=2e-5 * S)
    assert abs(added.sum() - S * NH) < 1e-3 * S
    # keys no query can see (none here) and the visible ones: every key got mass
    assert np.all(added > 0)


def test_decode_equals_fused_last_row_and_splits_agree(orc):
    rng = np.random.default_rng(13)
    n = 1000  # 15 groups + 40 tail keys
    c, _, _ = make_cache(orc, rng, n)
    q = rand_f16(rng, (1, NH, D))
    _, f32 = orc.attention_fused(bits(q), c, 1, n - 1)
    outs = {}
    for ns in (1, 16, 256, 512, 1024, 2048):
        _, o32, (pm, pl, po) = orc.attn_decode(bits(q), c, n - 1, nsplit=ns, nthreads=4)
        outs[ns] = o32
        np.testing.assert_allclose(o32, f32[0], rtol=5e-5, atol=1e-5)
        empty = pl == 0
        chunk = -(-n // ns)
        n_nonempty = -(-n // chunk)
        assert empty.reshape(NH, ns)[:, n_nonempty:].all() and not empty.reshape(NH, ns)[:, :n_nonempty].any()
        assert np.all(pm[empty] == np.float32(-1e30))
    K, V = dequant_cache(c, n)
    ref = brute_attention(q, K, V, 1, n - 1)[0]
    np.testing.assert_allclose(outs[16], ref, rtol=2e-5, atol=1e-5)


def test_decode_mt_equals_single_thread(orc):
    rng = np.random.default_rng(17)
    c, _, _ = make_cache(orc, rng, 700)
    q = rand_f16(rng, (1, NH, D))
    a = orc.attn_decode(bits(q), c, 699, nsplit=16, nthreads=1)
    b = orc.attn_decode(bits(q), c, 699, nsplit=16, nthreads=8)
    assert np.array_equal(a[1], b[1]) and np.array_equal(a[0], b[0])


def test_fused_mt_equals_single_thread(orc):
    """The threaded head-range form of attention_fused (the reference that
    the 4096-token prefill's every row is compared with) gives the
    single-threaded oracle's bits for the heads it covers and leaves the
    others zero."""
    rng = np.random.default_rng(23)
    S, past = 90, 40
    c, _, _ = make_cache(orc, rng, past + S)
    q = rand_f16(rng, (S, NH, D))
    a16, a32 = orc.attention_fused(bits(q), c, S, past)
    b16, b32 = orc.attention_fused_mt(bits(q), c, S, past, heads=(8, 16), nthreads=5)
    assert np.array_equal(b32[:, 8:16].view(np.uint32), a32[:, 8:16].view(np.uint32))
    assert np.array_equal(b16[:, 8:16], a16[:, 8:16])
    assert not b32[:, :8].any() and not b32[:, 16:].any()
    c16, c32 = orc.attention_fused_mt(bits(q), c, S, past, nthreads=3)
    assert np.array_equal(c32.view(np.uint32), a32.view(np.uint32))


# ---------------------------------------------------------------- H2O
def h2o_setup(orc, rng, C, W, n, prompt):
    q = rand_f16(rng, (n, NH, D))
    k = rand_f16(rng, (n, NKV, D))
    v = rand_f16(rng, (n, NKV, D))
    h = orc.H2OCache(C, W)
    return h, q, k, v


def test_h2o_out_and_mass_against_fp64(orc):
    rng = np.random.default_rng(19)
    C, W = 48, 8
    h, q, k, v = h2o_setup(orc, rng, C, W, 80, 30)
    h.step(bits(q[:30]), bits(k[:30]), bits(v[:30]), 0)
    for pos in range(30, 80):
        before = h.attn.copy()
        dst, o16, o32 = h.step(bits(q[pos:pos + 1]), bits(k[pos:pos + 1]), bits(v[pos:pos + 1]), pos)
        n = h.n_live
        Kd = TABLE[h.kf[:n]] * h.ks[:n].view(np.float16).astype(np.float64)[:, :, None]
        Vd = TABLE[h.vf[:n]] * h.vs[:n].view(np.float16).astype(np.float64)[:, :, None]
        ok = h.slotpos[:n] <= pos
        mass = np.zeros(n)
        for hh in range(NH):
            s = (Kd[:, hh // 4] @ q[pos, hh].astype(np.float64)) * 0.125
            s = np.where(ok, s, -np.inf)
            p = np.exp(s - s.max())
            p /= p.sum()
            np.testing.assert_allclose(o32[0, hh], p @ Vd[:, hh // 4], rtol=2e-5, atol=1e-5)
            mass += p
        if dst[0] < C and pos >= C:
            before[dst[0]] = 0.0
        got = h.attn[:n].astype(np.float64) - before[:n].astype(np.float64)
        # 32 fp32 adds into accumulators of magnitude ~20 round at ~2e-6 each
        np.testing.assert_allclose(got, mass, rtol=1e-5, atol=1e-4)
        assert abs(got.sum() - NH) < 1e-4


def test_h2o_mass_one_hot_closed_form(orc):
    """One slot matches q, the others are orthogonal: the mass of that slot is
    32 * e^s / (e^s + n - 1) with s = 0.125 * a * k (k the dequantised 1)."""
    n, a = 40, 12.0
    k = np.zeros((n, NKV, D), np.float16)
    k[:, :, 1] = 1.0
    k[7, :, 1] = 0.0
    k[7, :, 0] = 1.0
    v = np.zeros((n, NKV, D), np.float16)
    q = np.zeros((1, NH, D), np.float16)
    q[0, :, 0] = a
    h = orc.H2OCache(64, 8)
    dst = np.arange(n, dtype=np.int32)
    orc.kv_quant_write(bits(k), bits(v), h.kf, h.vf, h.ks, h.vs, dst)
    h.slotpos[:n] = np.arange(n)
    h.n_live = n
    orc.attention_h2o(bits(q), h.kf, h.vf, h.ks, h.vs, h.slotpos, n, h.attn, 1, n - 1)
    kd = TABLE[0x7E] * np.float64(np.float16(np.float32(1.0) / np.float32(448.0) + np.float32(1e-12)))
    s = 0.125 * a * kd
    want = NH * np.exp(s) / (np.exp(s) + n - 1)
    assert abs(h.attn[7] - want) < 2e-5 * want
    others = np.delete(h.attn[:n], 7)
    np.testing.assert_allclose(others, (NH - want) / (n - 1), rtol=2e-5)


def test_h2o_mass_is_bit_reproducible(orc):
    rng = np.random.default_rng(23)
    runs = []
    for _ in range(2):
        h, q, k, v = h2o_setup(orc, np.random.default_rng(23), 32, 4, 60, 20)
        h.step(bits(q[:20]), bits(k[:20]), bits(v[:20]), 0, want_out=False)
        for pos in range(20, 60):
            h.step(bits(q[pos:pos + 1]), bits(k[pos:pos + 1]), bits(v[pos:pos + 1]), pos,
                   want_out=False)
        runs.append((h.attn.copy(), h.slotpos.copy()))
    assert np.array_equal(runs[0][0].view(np.uint32), runs[1][0].view(np.uint32))
    assert np.array_equal(runs[0][1], runs[1][1])
