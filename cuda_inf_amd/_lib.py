"""Loader of libcuda_inf_attn.so (the gfx950 attention library) via ctypes.

The library is built in-tree by ``make -C cuda_inf_amd/csrc`` (or
``__graft_entry__.build()``).  There is no fallback: if the library is
missing every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcuda_inf_attn.so")
CSRC = os.path.join(HERE, "csrc")

# Shapes (engine.cu:22-23, 35-38)
NH, NKV, GQA, D, KVGROUP = 32, 8, 4, 64, 64
NSPLIT_DEFAULT = 16
HIDDEN = 2048  # hidden size H (engine.cu:33)
NSPLIT_MAX = 4096

STATUS = {0: "CIA_OK", 1: "CIA_ERR_NULL", 2: "CIA_ERR_ALIGN", 3: "CIA_ERR_ARG",
          4: "CIA_ERR_HIP", 5: "CIA_ERR_STATE", 6: "CIA_ERR_NOSLOT",
          7: "CIA_ERR_IO"}

# Every symbol include/cuda_inf_attn.h declares, with its ctypes signature.
_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
SIGNATURES = {
    "cia_strerror": (ctypes.c_char_p, [_I]),
    "cia_last_hip_error": (_I, []),
    "cia_version": (ctypes.c_char_p, []),
    "cia_e4m3_encode_range": (_I, [ctypes.c_uint32, ctypes.c_int64, _P, _P]),
    "cia_kv_write_tail": (_I, [_P, _P, _P, _P, _I, _I, _P]),
    "cia_kv_commit_group": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _P]),
    "cia_attention_fused": (_I, [_P] * 7 + [_I, _P, _P, _I, _I, _F, _P, ctypes.c_int64, _P]),
    "cia_attention_fused_fp8": (_I, [_P] * 7 + [_I, _P, _I, _I, _F, _P]),
    "cia_attn_decode_split": (_I, [_P] * 7 + [_I, _I, _F, _P, _P, _P, _I, _P]),
    "cia_attn_decode_split_ws": (_I, [_P] * 7 + [_I, _I, _F, _P, _P, _P, _I, _P,
                                                ctypes.c_int64, _P]),
    "cia_split_workspace_bytes": (ctypes.c_int64, [_I]),
    "cia_attn_decode_combine": (_I, [_P, _P, _P, _P, _I, _P]),
    "cia_attn_decode": (_I, [_P] * 7 + [_I, _I, _F, _P, _P, ctypes.c_int64, _P]),
    "cia_decode_workspace_bytes": (ctypes.c_int64, [_I]),
    "cia_stream_read": (_I, [_P, _P, ctypes.c_int64, _P, _P]),
    "cia_attn_decode_noalloc": (_I, [_P] * 7 + [_I, _I, _F, _P, _P]),
    "cia_kv_quant_write": (_I, [_P] * 7 + [_I, _P]),
    "cia_h2o_place": (_I, [_P] * 10 + [_I, _I, _I, _I, _P]),
    "cia_attention_h2o": (_I, [_P] * 6 + [_I, _P, _P, _I, _I, _F, _P, ctypes.c_int64, _P]),
    "cia_h2o_workspace_bytes": (ctypes.c_int64, [_I, _I]),
    "cia_mass_workspace_bytes": (ctypes.c_int64, [_I]),
    "cia_qk_norm_rope": (_I, [_P, _P, _P, _P, _P, _I, _F, _F, _P]),
    "cia_gemv_int4": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "cia_gemv_int4_add": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "cia_qkv_proj_int4": (_I, [_P, _P, _P, _I, _P, _P, _P, _P, _I, _I, _I, _P, _P, _P, _P]),
    "cia_attn_block_forward": (_I, [_P, _P, _P, _P, _I, _I, _F, _P, _P]),
    "cia_attn_block_loop": (_I, [_P, _P, _I, _P, _P, _I, _I, _F, _P, _P]),
    "cia_kv_append_plan": (_I, [_P, _I, _I, _P, _I, _P]),
    "cia_h2o_clamp": (None, [_P, _P, _I, _I]),
    "cia_h2o_pick_slots": (_I, [_P, _I, _I, _P, _P, _I, _I, _P, _P]),
    "cia_layer_forward": (_I, [_P, _P, _P, _P, _P, _I, _I, _F, _P, _P]),
    "cia_layer_append": (_I, [_P, _P, _P, _I, _I, _P]),
    "cia_decode_loop": (_I, [_P, _I, _P, _P, _P, _P, _I, _I, _F, _P, _P]),
    "cia_decode_loop_ex": (_I, [_P, _I, _P, _P, _P, _P, _I, _I, _F, _I, _P, _P]),
    "cia_decode_loop_runs": (_I, [_P, _I, _P, _P, _P, _P, _I, _I, _F, _I, _I, _P, _P]),
    "cia_decode_fault": (_I, [_P, ctypes.c_int64, _P]),
    # include/cuda_inf_model.h
    "cia_index_read": (_I, [ctypes.c_char_p, _P, ctypes.c_int64, _P]),
    "cia_file_size": (_I, [ctypes.c_char_p, _P]),
    "cia_weights_upload": (_I, [ctypes.c_char_p, _P, ctypes.c_uint64, _P, _P]),
    "cia_tok_load": (_I, [ctypes.c_char_p, _P]),
    "cia_tok_free": (None, [_P]),
    "cia_tok_encode": (_I, [_P, ctypes.c_char_p, ctypes.c_int64, _P, ctypes.c_int64, _P]),
    "cia_tok_decode": (_I, [_P, _P, ctypes.c_int64, _I, _P, ctypes.c_int64, _P]),
}


class CiaError(RuntimeError):
    def __init__(self, fn: str, code: int, lib):
        msg = lib.cia_strerror(code).decode()
        extra = ""
        if code == 4:
            extra = f" (hipError {lib.cia_last_hip_error()})"
        super().__init__(f"{fn}: {STATUS.get(code, code)}: {msg}{extra}")
        self.code = code


_lib = None


def use_timeline_build() -> None:
    """Load libcuda_inf_attn_tl.so (``make -C cuda_inf_amd/csrc TIMELINE=1``:
    the same library with per-wave timestamps in the one-launch decode)
    instead of the product library.  Must be called before the first lib();
    raises if that build is missing."""
    global LIB_PATH
    if _lib is not None:
        raise RuntimeError("the library is already loaded")
    tl = os.path.join(HERE, "libcuda_inf_attn_tl.so")
    if not os.path.exists(tl):
        raise RuntimeError(f"{tl} is missing: build it with `make -C {CSRC} TIMELINE=1`")
    LIB_PATH = tl


def build(force: bool = False) -> str:
    """Compile the library with the Makefile in csrc/ (hipcc, gfx950)."""
    args = ["make", "-s", "-C", CSRC, "-j8"]
    if force:
        args.append("-B")
    subprocess.run(args, check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `make -C {CSRC}` "
                "(or __graft_entry__.build()); there is no non-HIP fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(fn: str, code: int) -> None:
    if code != 0:
        raise CiaError(fn, code, lib())


def call(fn: str, *args) -> None:
    check(fn, getattr(lib(), fn)(*args))


class cia_tensor_desc(ctypes.Structure):
    """Mirror of ``cia_tensor_desc`` in include/cuda_inf_model.h."""
    _fields_ = [("name", ctypes.c_char * 256), ("kind", ctypes.c_int32),
                ("offset", ctypes.c_uint64), ("packed", ctypes.c_uint64),
                ("scales", ctypes.c_uint64), ("d0", ctypes.c_int64), ("d1", ctypes.c_int64)]


class cia_append_op(ctypes.Structure):
    _fields_ = [("src_token", _I), ("slot", _I), ("cnt", _I), ("commit", _I),
                ("commit_base", _I), ("commit_grp", _I)]


class cia_attn_proj(ctypes.Structure):
    """Mirror of ``cia_attn_proj`` in include/cuda_inf_attn.h."""
    _fields_ = [
        ("q_packed", _P), ("q_scales", _P), ("k_packed", _P), ("k_scales", _P),
        ("v_packed", _P), ("v_scales", _P), ("o_packed", _P), ("o_scales", _P),
        ("ws", _P), ("cap", _I),
    ]


class cia_layer(ctypes.Structure):
    """Mirror of ``cia_layer`` in include/cuda_inf_attn.h."""
    _fields_ = [
        ("kc8", _P), ("vc8", _P), ("ksc", _P), ("vsc", _P), ("ktail", _P), ("vtail", _P),
        ("maxT", _I), ("committed", _I),
        ("nsplit", _I), ("pm", _P), ("pl", _P), ("po", _P), ("ws_decode", _P),
        ("budget", _I), ("window", _I),
        ("kf", _P), ("vf", _P), ("ks", _P), ("vs", _P), ("hattn", _P), ("d_slotpos", _P),
        ("d_dst", _P), ("n_live", _I), ("ws_mass", _P),
        ("qw", _P), ("kw", _P), ("eps", _F), ("theta", _F), ("prep_ws", _P), ("prep_cap", _I),
    ]
