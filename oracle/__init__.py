"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: the HIP path is compared against it.  Only tests/,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` import
this module.  The product package ``cuda_inf_amd`` never does.

All arrays are numpy arrays; fp16 tensors are passed as ``uint16`` bit
patterns (or ``float16`` arrays, which are viewed as ``uint16``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

NH, NKV, GQA, D, KVGROUP = 32, 8, 4, 64, 64

_lib = None


def build(force: bool = False) -> str:
    """Compile liboracle.so with the Makefile beside this file."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "-B" if force else "liboracle.so"],
                       check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_I64 = ctypes.c_int64


def _declare(L):
    sig = {
        "orc_f32_to_f16": (ctypes.c_uint16, [_F]),
        "orc_f16_to_f32": (_F, [ctypes.c_uint16]),
        "orc_e4m3_encode": (ctypes.c_uint8, [_F]),
        "orc_e4m3_decode": (_F, [ctypes.c_uint8]),
        "orc_quant_scale": (_F, [_F]),
        "orc_exp_det": (_F, [_F]),
        "orc_f32_to_f16_array": (None, [_P, _P, _I64]),
        "orc_e4m3_encode_array": (None, [_P, _P, _I64]),
        "orc_e4m3_encode_range_u32": (None, [ctypes.c_uint32, _I64, _P]),
        "orc_exp_det_array": (None, [_P, _P, _I64]),
        "orc_sincos_det_array": (None, [_P, _P, _P, _I64]),
        "orc_rope_invf": (None, [_F, _P]),
        "orc_qk_norm_rope": (None, [_P, _P, _P, _P, _P, _I, _F, _F]),
        "orc_kv_write_tail": (None, [_P, _P, _P, _P, _I, _I]),
        "orc_kv_commit_group": (None, [_P, _P, _P, _P, _P, _P, _I, _I]),
        "orc_kv_append": (_I, [_P] * 8 + [_P, _I, _I]),
        "orc_attention_fused": (None, [_P] * 7 + [_I, _P, _P, _P, _I, _I, _F, _P, _I]),
        "orc_attention_fused_mt": (None, [_P] * 7 + [_I, _P, _P, _I, _I, _F, _I, _I, _I]),
        "orc_attn_decode_split": (None, [_P] * 7 + [_I, _I, _F, _P, _P, _P, _I]),
        "orc_attn_decode_combine": (None, [_P, _P, _P, _P, _P, _I]),
        "orc_attn_decode_mt": (None, [_P] * 7 + [_I, _I, _F, _P, _P, _P, _I, _P, _P, _I]),
        "orc_kv_quant_write": (None, [_P] * 7 + [_I]),
        "orc_attention_h2o": (None, [_P] * 6 + [_I, _P, _P, _P, _I, _I, _F]),
        "orc_h2o_pick_slots": (_I, [_P, _I, _I, _P, _P, _I, _I, _P, _P]),
        "orc_quant_int4_g128": (None, [_P, _I, _I, _P, _P]),
        "orc_gemv_int4": (None, [_P, _P, _P, _P, _P, _I, _I, _I]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a):
    if a is None:
        return None
    assert isinstance(a, np.ndarray) and a.flags["C_CONTIGUOUS"], "need C-contiguous ndarray"
    return a.ctypes.data


def _u16(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint16) if a.dtype == np.float16 else a


# ---------------------------------------------------------------- codecs
def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().orc_e4m3_encode_array(_p(x), _p(out), x.size)
    return out


def e4m3_encode_range_u32(first: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint8)
    lib().orc_e4m3_encode_range_u32(first, n, _p(out))
    return out


def e4m3_decode_table() -> np.ndarray:
    L = lib()
    return np.array([L.orc_e4m3_decode(b) for b in range(256)], np.float32)


def exp_det(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.float32)
    lib().orc_exp_det_array(_p(x), _p(out), x.size)
    return out


def quant_scale(amax: float) -> float:
    return lib().orc_quant_scale(amax)


def sincos_det(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    s = np.empty(x.shape, np.float32)
    c = np.empty(x.shape, np.float32)
    lib().orc_sincos_det_array(_p(x), _p(s), _p(c), x.size)
    return s, c


def rope_invf(theta: float = 5.0e6) -> np.ndarray:
    out = np.empty(32, np.float32)
    lib().orc_rope_invf(theta, _p(out))
    return out


def qk_norm_rope(q, k, qw, kw, pos, eps: float = 1e-5, theta: float = 5.0e6):
    """engine.cu:799-801 (RMSNorm of q and k, then RoPE) with the
    deterministic sin/cos; returns new fp16 bit arrays."""
    q = np.array(_u16(q), dtype=np.uint16, copy=True, order="C")
    k = np.array(_u16(k), dtype=np.uint16, copy=True, order="C")
    qw = np.ascontiguousarray(_u16(qw), dtype=np.uint16)
    kw = np.ascontiguousarray(_u16(kw), dtype=np.uint16)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    lib().orc_qk_norm_rope(_p(q), _p(k), _p(qw), _p(kw), _p(pos), int(pos.size), eps, theta)
    return q, k


# ---------------------------------------------------------------- cache
class Group64Cache:
    """Host copy of one attention layer's group-64 cache (engine.cu:596-603)."""

    def __init__(self, max_tokens: int):
        self.maxT = max_tokens
        self.kc8 = np.zeros((max_tokens, NKV, D), np.uint8)
        self.vc8 = np.zeros((max_tokens, NKV, D), np.uint8)
        ng = max_tokens // KVGROUP + 2
        self.ksc = np.zeros((ng, NKV), np.uint16)
        self.vsc = np.zeros((ng, NKV), np.uint16)
        self.ktail = np.zeros((KVGROUP, NKV, D), np.uint16)
        self.vtail = np.zeros((KVGROUP, NKV, D), np.uint16)
        self.committed = 0

    def append(self, k, v, past: int) -> int:
        k, v = _u16(k), _u16(v)
        S = k.shape[0]
        c = ctypes.c_int(self.committed)
        n = lib().orc_kv_append(_p(k), _p(v), _p(self.ktail), _p(self.vtail), _p(self.kc8),
                                _p(self.vc8), _p(self.ksc), _p(self.vsc), ctypes.byref(c), S, past)
        self.committed = c.value
        return n

    def ptrs(self):
        return (_p(self.kc8), _p(self.vc8), _p(self.ksc), _p(self.vsc),
                _p(self.ktail), _p(self.vtail))


def kv_write_tail(k, v, ktail, vtail, slot, cnt):
    k, v = _u16(k), _u16(v)
    lib().orc_kv_write_tail(_p(k), _p(v), _p(ktail), _p(vtail), slot, cnt)


def kv_commit_group(ktail, vtail, kc8, vc8, ksc, vsc, dst_tok_base, grp):
    lib().orc_kv_commit_group(_p(ktail), _p(vtail), _p(kc8), _p(vc8), _p(ksc), _p(vsc),
                              dst_tok_base, grp)


def attention_fused(q, cache: Group64Cache, S: int, past: int, scale: float = 0.125,
                    attn_sum=None, rows=None):
    """Returns (out16 [S,NH,D] uint16, out32 [S,NH,D] float32)."""
    q = _u16(q)
    out16 = np.zeros((S, NH, D), np.uint16)
    out32 = np.zeros((S, NH, D), np.float32)
    r = None if rows is None else np.ascontiguousarray(rows, dtype=np.int32)
    lib().orc_attention_fused(_p(q), *cache.ptrs(), cache.committed, _p(out16), _p(out32),
                              _p(attn_sum), S, past, scale, _p(r), 0 if r is None else r.size)
    return out16, out32


def attention_fused_mt(q, cache: Group64Cache, S: int, past: int, scale: float = 0.125,
                       heads=(0, NH), nthreads: int = 1):
    """attention_fused's outputs for query heads heads[0]..heads[1]-1 of all
    S rows on nthreads threads (no attn_sum): identical per (row, head) to
    attention_fused.  Returns (out16, out32) [S,NH,D]; other heads are 0."""
    q = _u16(q)
    out16 = np.zeros((S, NH, D), np.uint16)
    out32 = np.zeros((S, NH, D), np.float32)
    lib().orc_attention_fused_mt(_p(q), *cache.ptrs(), cache.committed, _p(out16), _p(out32),
                                 S, past, scale, int(heads[0]), int(heads[1]), int(nthreads))
    return out16, out32


def attn_decode_split(q, cache: Group64Cache, qpos: int, nsplit: int = 16, scale: float = 0.125):
    q = _u16(q)
    pm = np.zeros(NH * nsplit, np.float32)
    pl = np.zeros(NH * nsplit, np.float32)
    po = np.zeros((NH * nsplit, D), np.float32)
    lib().orc_attn_decode_split(_p(q), *cache.ptrs(), cache.committed, qpos, scale,
                                _p(pm), _p(pl), _p(po), nsplit)
    return pm, pl, po


def attn_decode_combine(pm, pl, po, nsplit: int):
    out16 = np.zeros((NH, D), np.uint16)
    out32 = np.zeros((NH, D), np.float32)
    lib().orc_attn_decode_combine(_p(pm), _p(pl), _p(po), _p(out16), _p(out32), nsplit)
    return out16, out32


def attn_decode(q, cache: Group64Cache, qpos: int, nsplit: int = 16, scale: float = 0.125,
                nthreads: int = 1):
    """split + combine; returns (out16, out32, (pm, pl, po))."""
    q = _u16(q)
    pm = np.zeros(NH * nsplit, np.float32)
    pl = np.zeros(NH * nsplit, np.float32)
    po = np.zeros((NH * nsplit, D), np.float32)
    out16 = np.zeros((NH, D), np.uint16)
    out32 = np.zeros((NH, D), np.float32)
    lib().orc_attn_decode_mt(_p(q), *cache.ptrs(), cache.committed, qpos, scale, _p(pm),
                             _p(pl), _p(po), nsplit, _p(out16), _p(out32), nthreads)
    return out16, out32, (pm, pl, po)


# ---------------------------------------------------------------- H2O
class H2OCache:
    """Host copy of one layer's H2O slot buffer (engine.cu:605-612)."""

    def __init__(self, C: int, W: int):
        self.C, self.W = C, W
        self.kf = np.zeros((C, NKV, D), np.uint8)
        self.vf = np.zeros((C, NKV, D), np.uint8)
        self.ks = np.zeros((C, NKV), np.uint16)
        self.vs = np.zeros((C, NKV), np.uint16)
        self.attn = np.zeros(C, np.float32)
        self.slotpos = np.full(C, -1, np.int32)
        self.n_live = 0

    def pick(self, S: int, past: int):
        """Slot choice; returns (dst, zeroed, evictions).  Clears attn of reused slots."""
        dst = np.zeros(S, np.int32)
        zeroed = np.zeros(S, np.int32)
        nl = ctypes.c_int(self.n_live)
        host = self.attn.copy()
        ev = lib().orc_h2o_pick_slots(ctypes.byref(nl), self.C, self.W, _p(self.slotpos),
                                      _p(host), S, past, _p(dst), _p(zeroed))
        if ev < 0:
            raise RuntimeError("h2o_pick_slots: no slot below 1e30")
        self.n_live = nl.value
        for j in range(S):
            if zeroed[j]:
                self.attn[dst[j]] = 0.0
        return dst, zeroed, ev

    def step(self, q, k, v, past: int, scale: float = 0.125, want_out: bool = True):
        """One H2O layer call (engine.cu:803-828).  Returns (dst, out16, out32)."""
        q, k, v = _u16(q), _u16(k), _u16(v)
        S = k.shape[0]
        dst, _, _ = self.pick(S, past)
        lib().orc_kv_quant_write(_p(k), _p(v), _p(self.kf), _p(self.vf), _p(self.ks),
                                 _p(self.vs), _p(dst), S)
        out16 = np.zeros((S, NH, D), np.uint16) if want_out else None
        out32 = np.zeros((S, NH, D), np.float32) if want_out else None
        lib().orc_attention_h2o(_p(q), _p(self.kf), _p(self.vf), _p(self.ks), _p(self.vs),
                                _p(self.slotpos), self.n_live, _p(out16), _p(out32),
                                _p(self.attn), S, past, scale)
        return dst, out16, out32


def kv_quant_write(k, v, kf, vf, ks, vs, dst):
    k, v = _u16(k), _u16(v)
    dst = np.ascontiguousarray(dst, dtype=np.int32)
    lib().orc_kv_quant_write(_p(k), _p(v), _p(kf), _p(vf), _p(ks), _p(vs), _p(dst), k.shape[0])


def attention_h2o(q, kf, vf, ks, vs, slot_pos, n_live, attn_sum, S, past, scale=0.125):
    q = _u16(q)
    out16 = np.zeros((S, NH, D), np.uint16)
    out32 = np.zeros((S, NH, D), np.float32)
    lib().orc_attention_h2o(_p(q), _p(kf), _p(vf), _p(ks), _p(vs), _p(slot_pos), n_live,
                            _p(out16), _p(out32), _p(attn_sum), S, past, scale)
    return out16, out32


def h2o_pick_slots(n_live, C, W, slotpos, attn_host, S, past):
    dst = np.zeros(S, np.int32)
    zeroed = np.zeros(S, np.int32)
    nl = ctypes.c_int(n_live)
    ev = lib().orc_h2o_pick_slots(ctypes.byref(nl), C, W, _p(slotpos), _p(attn_host), S, past,
                                  _p(dst), _p(zeroed))
    return nl.value, dst, zeroed, ev


# ---------------------------------------------------------------- INT4 g128
def quant_int4_g128(w):
    """tools/export_weights.py:64-79: fp32 [N, K] -> (packed u8 [N, K/2],
    scales fp16 bits [N, K/128])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    assert K % 128 == 0
    packed = np.zeros((N, K // 2), np.uint8)
    scales = np.zeros((N, K // 128), np.uint16)
    lib().orc_quant_int4_g128(_p(w), N, K, _p(packed), _p(scales))
    return packed, scales


def gemv_int4(x, packed, scales, want_absum: bool = False):
    """engine.cu:83-109: x fp16 [M, K] -> y fp32 [M, N] (fp64 accumulation)."""
    x = np.ascontiguousarray(_u16(x), dtype=np.uint16)
    if x.ndim == 1:
        x = x[None, :]
    M, K = x.shape
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(_u16(scales), dtype=np.uint16)
    N = packed.shape[0]
    assert packed.shape == (N, K // 2) and scales.shape == (N, K // 128)
    y = np.zeros((M, N), np.float32)
    ab = np.zeros((M, N), np.float32) if want_absum else None
    lib().orc_gemv_int4(_p(x), _p(packed), _p(scales), _p(y), _p(ab), N, K, M)
    return (y, ab) if want_absum else y
