"""The C-ABI library on the CPU: it loads, exports every declared symbol,
rejects bad arguments with status codes before touching a device, and its
host-only policy (append planner, H2O clamps and slot picker) follows the
reference (engine.cu:752-756, 808-845)."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("cuda_inf_attn.h", "cuda_inf_model.h")]


def declared_symbols():
    text = "".join(open(h).read() for h in HEADERS)
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cia_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(cia):
    from cuda_inf_amd import _lib
    L = _lib.lib()
    names = declared_symbols()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # the Python binding declares a signature for each of them
    assert set(names) <= set(_lib.SIGNATURES), set(names) - set(_lib.SIGNATURES)
    assert L.cia_version().startswith(b"cuda_inf_attn")


def test_status_strings(cia):
    from cuda_inf_amd import _lib
    L = _lib.lib()
    for code in range(8):
        assert L.cia_strerror(code) and L.cia_strerror(code) != b"unknown status"
    assert L.cia_strerror(99) == b"unknown status"


FAKE = 0x10000  # aligned non-null address: validation must fail before any use


@pytest.mark.parametrize("call,code", [
    (lambda L: L.cia_kv_write_tail(FAKE, FAKE, FAKE, FAKE, 60, 5, None), 3),     # slot+cnt > 64
    (lambda L: L.cia_kv_write_tail(FAKE, FAKE, FAKE, FAKE, -1, 1, None), 3),
    (lambda L: L.cia_kv_write_tail(None, FAKE, FAKE, FAKE, 0, 1, None), 1),
    (lambda L: L.cia_kv_write_tail(FAKE + 2, FAKE, FAKE, FAKE, 0, 1, None), 2),  # misaligned
    (lambda L: L.cia_kv_write_tail(None, None, None, None, 5, 0, None), 0),      # nothing to do
    (lambda L: L.cia_kv_commit_group(FAKE, FAKE, FAKE, None, FAKE, FAKE, 0, 0, None), 1),
    (lambda L: L.cia_kv_commit_group(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, -64, 0, None), 3),
    (lambda L: L.cia_attn_decode_split(*([FAKE] * 7), 64, 100, 0.125, FAKE, FAKE, FAKE, 0, None), 3),
    (lambda L: L.cia_attn_decode_split(*([FAKE] * 7), 64, 100, 0.125, FAKE, FAKE, FAKE, 5000, None), 3),
    (lambda L: L.cia_attn_decode_split(*([FAKE] * 7), 60, 100, 0.125, FAKE, FAKE, FAKE, 16, None), 3),
    (lambda L: L.cia_attn_decode_split(*([FAKE] * 7), 64, 200, 0.125, FAKE, FAKE, FAKE, 16, None), 5),
    (lambda L: L.cia_attn_decode_combine(FAKE, FAKE, FAKE, FAKE, 0, None), 3),
    (lambda L: L.cia_attn_decode(*([FAKE] * 7), 128, 100, 0.125, FAKE, FAKE, 1 << 20, None), 5),
    (lambda L: L.cia_attn_decode(*([FAKE] * 7), 64, 100, 0.125, FAKE, None, 1 << 20, None), 1),
    (lambda L: L.cia_attention_fused(*([FAKE] * 7), 0, FAKE, None, 10, 100, 0.125, None, 0, None), 5),
    (lambda L: L.cia_attention_fused(*([FAKE] * 7), 0, FAKE, None, -1, 0, 0.125, None, 0, None), 3),
    (lambda L: L.cia_attention_fused(*([None] * 7), 0, None, None, 0, 0, 0.125, None, 0, None), 0),
    # attn_sum needs a mass workspace of cia_mass_workspace_bytes(S) bytes
    (lambda L: L.cia_attention_fused(*([FAKE] * 7), 0, FAKE, FAKE, 10, 0, 0.125, None, 0, None), 1),
    (lambda L: L.cia_attention_fused(*([FAKE] * 7), 0, FAKE, FAKE, 10, 0, 0.125, FAKE,
                                     10 * 32 * 2 * 4 - 4, None), 3),
    (lambda L: L.cia_kv_quant_write(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, 3, None), 1),
    (lambda L: L.cia_kv_quant_write(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, -1, None), 3),
    (lambda L: L.cia_attention_h2o(*([FAKE] * 6), 0, FAKE, FAKE, 1, 0, 0.125, FAKE, 1 << 20, None), 3),
    (lambda L: L.cia_attention_h2o(*([FAKE] * 6), 5, FAKE, None, 1, 0, 0.125, FAKE, 1 << 20, None), 1),
    (lambda L: L.cia_attention_h2o(*([FAKE] * 6), 100, FAKE, FAKE, 1, 0, 0.125, FAKE, 64, None), 3),
    (lambda L: L.cia_h2o_place(*([FAKE] * 9), None, 8, 2, 1, 0, None), 1),
    (lambda L: L.cia_gemv_int4(FAKE, FAKE, FAKE, FAKE, 64, 100, 1, None), 3),    # K % 128
    (lambda L: L.cia_gemv_int4(FAKE, FAKE, FAKE, FAKE, 0, 128, 1, None), 3),
    (lambda L: L.cia_gemv_int4(None, None, None, None, 64, 128, 0, None), 0),     # M = 0
    (lambda L: L.cia_gemv_int4(FAKE, None, FAKE, FAKE, 64, 128, 1, None), 1),
    (lambda L: L.cia_gemv_int4(FAKE, FAKE + 8, FAKE, FAKE, 64, 128, 1, None), 2),
    (lambda L: L.cia_gemv_int4_add(FAKE + 2, FAKE, FAKE, FAKE, 64, 128, 1, None), 2),
    (lambda L: L.cia_qkv_proj_int4(FAKE, FAKE, FAKE, 64, FAKE, FAKE, FAKE, FAKE, 0, 128, 1,
                                   FAKE, FAKE, FAKE, None), 3),
    (lambda L: L.cia_qkv_proj_int4(FAKE, FAKE, FAKE, 64, FAKE, FAKE, FAKE, FAKE, 16, 128, 1,
                                   FAKE, None, FAKE, None), 1),
    (lambda L: L.cia_decode_loop_runs(FAKE, 1, *([FAKE] * 4), 100, 1, 0.125, 0, -1, None, None), 3),
    (lambda L: L.cia_decode_loop_runs(FAKE, 0, *([FAKE] * 4), 100, 1, 0.125, 0, 0, None, None), 3),
    (lambda L: L.cia_decode_loop_runs(None, 1, *([FAKE] * 4), 100, 1, 0.125, 0, 0, None, None), 1),
    (lambda L: L.cia_decode_loop_ex(FAKE, 1, *([FAKE] * 4), 100, -1, 0.125, 0, None, None), 3),
    (lambda L: L.cia_e4m3_encode_range(0, -1, FAKE, None), 3),
    (lambda L: L.cia_e4m3_encode_range(0, 16, FAKE + 8, None), 2),
])
def test_argument_validation(cia, call, code):
    from cuda_inf_amd import _lib
    assert call(_lib.lib()) == code


def simulate_append(committed, S, past):
    """Direct restatement of engine.cu:830-845 for checking the planner."""
    ops, placed = [], 0
    while placed < S:
        slot = past + placed - committed
        can = min(S - placed, 64 - slot)
        op = dict(src_token=placed, slot=slot, cnt=can, commit=slot + can == 64,
                  commit_base=committed, commit_grp=committed // 64)
        placed += can
        if op["commit"]:
            committed += 64
        ops.append(op)
    return ops, committed


def test_append_plan_matches_reference_loop(cia):
    from cuda_inf_amd.layer import kv_append_plan
    rng = np.random.default_rng(0)
    for _ in range(300):
        committed, past = 0, 0
        for _ in range(int(rng.integers(1, 8))):
            S = int(rng.choice([1, 1, 2, 63, 64, 65, int(rng.integers(1, 400))]))
            got = kv_append_plan(committed, S, past)
            want = simulate_append(committed, S, past)
            assert got == want, (committed, S, past)
            committed, past = want[1], past + S
            # invariant: committed is the largest multiple of 64 <= past
            assert committed == (past // 64) * 64


def test_append_plan_rejects_inconsistent_state(cia):
    from cuda_inf_amd import CiaError
    from cuda_inf_amd.layer import kv_append_plan
    with pytest.raises(CiaError):
        kv_append_plan(64, 1, 10)      # past < committed
    with pytest.raises(CiaError):
        kv_append_plan(0, 1, 64)       # tail would hold 64 uncommitted tokens
    with pytest.raises(CiaError):
        kv_append_plan(32, 1, 40)      # committed not a multiple of 64


@pytest.mark.parametrize("budget,window,prompt,maxT,want", [
    (48, 0, 21, 1000, (48, 24)),       # window defaults to budget/2
    (10, 0, 21, 1000, (21, 10)),       # budget raised to the prompt
    (5000, 0, 21, 1000, (1000, 500)),  # budget capped at maxT
    (48, 60, 21, 1000, (48, 47)),      # window < budget
    (48, 47, 21, 1000, (48, 47)),
    (2048, 256, 1024, 5028, (2048, 256)),
])
def test_h2o_clamp(cia, budget, window, prompt, maxT, want):
    from cuda_inf_amd.layer import h2o_clamp
    assert h2o_clamp(budget, window, prompt, maxT) == want


def test_h2o_pick_hand_cases(cia):
    from cuda_inf_amd.layer import h2o_pick_slots
    # filling: slots handed out in order, nothing evicted
    sp = np.full(4, -1, np.int32)
    at = np.zeros(4, np.float32)
    nl, dst, z, ev = h2o_pick_slots(0, 4, 2, sp, at, 3, 0)
    assert (nl, list(dst), list(z), ev) == (3, [0, 1, 2], [0, 0, 0], 0)
    # full: evict the min outside the window; ties go to the lowest slot
    sp = np.array([0, 1, 2, 3], np.int32)
    at = np.array([0.5, 0.2, 0.2, 0.1], np.float32)
    nl, dst, z, ev = h2o_pick_slots(4, 4, 2, sp, at, 1, 4)  # window keeps pos 3 (> 4-2)
    assert (list(dst), list(z), ev) == ([1], [1], 1)
    assert list(sp) == [0, 4, 2, 3] and at[1] == np.float32(1e30)
    # two tokens in one call never reuse a slot
    sp = np.array([0, 1, 2, 3], np.int32)
    at = np.array([0.3, 0.2, 0.9, 0.9], np.float32)
    nl, dst, z, ev = h2o_pick_slots(4, 4, 1, sp, at, 2, 4)
    assert list(dst) == [1, 0] and ev == 2
    # fallback: nothing outside the window -> global argmin (engine.cu:818)
    sp = np.array([8, 9, 10, 11], np.int32)
    at = np.array([0.4, 0.3, 0.9, 0.35], np.float32)
    nl, dst, z, ev = h2o_pick_slots(4, 4, 3, sp, at, 1, 12)
    assert list(dst) == [1]


def test_h2o_pick_matches_oracle(cia, orc):
    from cuda_inf_amd.layer import h2o_pick_slots
    rng = np.random.default_rng(5)
    for _ in range(200):
        C = int(rng.integers(2, 64))
        W = int(rng.integers(1, C))
        n_live = int(rng.integers(0, C + 1))
        past = int(rng.integers(n_live, 3 * C + 1))
        sp = rng.permutation(past)[:C].astype(np.int32) if past >= C else np.arange(C, dtype=np.int32)
        at = rng.choice(np.float32([0.25, 0.5, 1.0, 2.0]), C).astype(np.float32)  # many ties
        S = int(rng.integers(1, 6))
        a = h2o_pick_slots(n_live, C, W, sp.copy(), at.copy(), S, past)
        b = orc.h2o_pick_slots(n_live, C, W, sp.copy(), at.copy(), S, past)
        assert a[0] == b[0] and np.array_equal(a[1], b[1]) and np.array_equal(a[2], b[2]) \
            and a[3] == b[3]
