"""The reference engine's attention kernels as Python calls on torch tensors.

Each function keeps the name, argument order and meaning of one kernel of
g023/cuda_inf ``src/engine.cu`` and runs the gfx950 implementation through the
C-ABI of libcuda_inf_attn.so on torch's current stream.  fp16 tensors may be
``torch.float16`` or ``torch.int16``/``torch.uint16`` bit patterns.  Errors
raise ``CiaError``; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import D, KVGROUP, NH, NKV, NSPLIT_DEFAULT, call

_F16 = (torch.float16, torch.int16, torch.uint16)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _dev(t: torch.Tensor, name: str, dtypes=None, numel=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    if not t.is_cuda:
        raise ValueError(f"{name}: must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if dtypes is not None and t.dtype not in dtypes:
        raise TypeError(f"{name}: dtype {t.dtype} not in {dtypes}")
    if numel is not None and t.numel() < numel:
        raise ValueError(f"{name}: needs at least {numel} elements, has {t.numel()}")
    return t.data_ptr()


def _opt(t, name, dtypes=None, numel=None):
    return None if t is None else _dev(t, name, dtypes, numel)


def e4m3_encode_range(first_bits: int, n: int, out) -> None:
    """Device E4M3 encoder on the fp32 bit patterns first_bits .. first_bits+n-1."""
    call("cia_e4m3_encode_range", first_bits, n, _dev(out, "out", (torch.uint8,), n), _stream())


# ------------------------------------------------------------ group-64 cache
def kv_write_tail(k, v, ktail, vtail, slot: int, cnt: int) -> None:
    """engine.cu:190-198: tail rows slot..slot+cnt-1 <- k, v [cnt, 8, 64]."""
    n = cnt * NKV * D
    call("cia_kv_write_tail", _dev(k, "k", _F16, n), _dev(v, "v", _F16, n),
         _dev(ktail, "ktail", _F16, KVGROUP * NKV * D), _dev(vtail, "vtail", _F16, KVGROUP * NKV * D),
         slot, cnt, _stream())


def kv_commit_group(ktail, vtail, kc8, vc8, ksc, vsc, dst_tok_base: int, grp: int) -> None:
    """engine.cu:202-228: commit the full tail group to FP8 with fp16 scales."""
    call("cia_kv_commit_group", _dev(ktail, "ktail", _F16, KVGROUP * NKV * D),
         _dev(vtail, "vtail", _F16, KVGROUP * NKV * D),
         _dev(kc8, "kc8", (torch.uint8,), (dst_tok_base + KVGROUP) * NKV * D),
         _dev(vc8, "vc8", (torch.uint8,), (dst_tok_base + KVGROUP) * NKV * D),
         _dev(ksc, "ksc", _F16, (grp + 1) * NKV), _dev(vsc, "vsc", _F16, (grp + 1) * NKV),
         dst_tok_base, grp, _stream())


# ------------------------------------------------------------ attention
def attention_fused(q, kc8, vc8, ksc, vsc, ktail, vtail, committed: int, out, attn_sum,
                    S: int, past: int, scale: float, ws=None) -> None:
    """engine.cu:236-308: causal attention of S queries at past..past+S-1."""
    T = past + S
    call("cia_attention_fused", _dev(q, "q", _F16, S * NH * D),
         _dev(kc8, "kc8", (torch.uint8,), min(T, committed) * NKV * D),
         _dev(vc8, "vc8", (torch.uint8,), min(T, committed) * NKV * D),
         _dev(ksc, "ksc", _F16), _dev(vsc, "vsc", _F16),
         _dev(ktail, "ktail", _F16, KVGROUP * NKV * D), _dev(vtail, "vtail", _F16, KVGROUP * NKV * D),
         committed, _dev(out, "out", _F16, S * NH * D),
         _opt(attn_sum, "attn_sum", (torch.float32,), T), S, past, float(scale),
         _opt(ws, "ws", None, mass_workspace_bytes(S) if attn_sum is not None else None),
         ws.numel() * ws.element_size() if ws is not None else 0, _stream())


def attention_fused_fp8(q, kc8, vc8, ksc, vsc, ktail, vtail, committed: int, out, S: int,
                        past: int, scale: float) -> None:
    """attention_fused's causal attention on the OCP-fp8 matrix cores (Q and
    the softmax numerators rounded to fp8; error reported, not bounded by
    the fp16 path's tolerance)."""
    T = past + S
    call("cia_attention_fused_fp8", _dev(q, "q", _F16, S * NH * D),
         _dev(kc8, "kc8", (torch.uint8,), min(T, committed) * NKV * D),
         _dev(vc8, "vc8", (torch.uint8,), min(T, committed) * NKV * D),
         _dev(ksc, "ksc", _F16), _dev(vsc, "vsc", _F16),
         _dev(ktail, "ktail", _F16, KVGROUP * NKV * D), _dev(vtail, "vtail", _F16, KVGROUP * NKV * D),
         committed, _dev(out, "out", _F16, S * NH * D), S, past, float(scale), _stream())


def attn_decode_split(q, kc8, vc8, ksc, vsc, ktail, vtail, committed: int, qpos: int,
                      scale: float, pm, pl, po, nsplit: int = NSPLIT_DEFAULT, ws=None) -> None:
    """engine.cu:396-464 with a runtime split count.  ws (optional): a
    workspace of split_workspace_bytes(nsplit) bytes, zeroed before its first
    use, in place of the library's fixed device array."""
    args = (_dev(q, "q", _F16, NH * D),
            _dev(kc8, "kc8", (torch.uint8,)), _dev(vc8, "vc8", (torch.uint8,)),
            _dev(ksc, "ksc", _F16), _dev(vsc, "vsc", _F16),
            _dev(ktail, "ktail", _F16, KVGROUP * NKV * D),
            _dev(vtail, "vtail", _F16, KVGROUP * NKV * D),
            committed, qpos, float(scale),
            _dev(pm, "pm", (torch.float32,), NH * nsplit),
            _dev(pl, "pl", (torch.float32,), NH * nsplit),
            _dev(po, "po", (torch.float32,), NH * nsplit * D), nsplit)
    if ws is None:
        call("cia_attn_decode_split", *args, _stream())
    else:
        call("cia_attn_decode_split_ws", *args,
             _dev(ws, "ws", (torch.uint8,), split_workspace_bytes(nsplit)), ws.numel(), _stream())


def split_workspace_bytes(nsplit: int) -> int:
    """Workspace bytes of attn_decode_split's caller-workspace form."""
    return int(_lib.lib().cia_split_workspace_bytes(nsplit))


def attn_decode_combine(pm, pl, po, out, nsplit: int = NSPLIT_DEFAULT) -> None:
    """engine.cu:467-480 with a runtime split count."""
    call("cia_attn_decode_combine", _dev(pm, "pm", (torch.float32,), NH * nsplit),
         _dev(pl, "pl", (torch.float32,), NH * nsplit),
         _dev(po, "po", (torch.float32,), NH * nsplit * D), _dev(out, "out", _F16, NH * D),
         nsplit, _stream())


def decode_workspace_bytes(max_tokens: int) -> int:
    """Scratch bytes of attn_decode for contexts of up to max_tokens keys."""
    return int(_lib.lib().cia_decode_workspace_bytes(max_tokens))


def new_decode_workspace(max_tokens: int, device="cuda") -> torch.Tensor:
    """Workspace of attn_decode: partial softmax states and per-kv-head
    arrival counters.  Zeroed here; every call leaves the counters at zero."""
    return torch.zeros(decode_workspace_bytes(max_tokens), dtype=torch.uint8, device=device)


def attn_decode(q, kc8, vc8, ksc, vsc, ktail, vtail, committed: int, qpos: int, scale: float,
                out, ws) -> None:
    """Flash-decoding on the matrix cores with the library's own split, one
    launch (replaces engine.cu:848-852's split + combine launches).  Calls
    sharing ws must be ordered on one stream."""
    call("cia_attn_decode", _dev(q, "q", _F16, NH * D),
         _dev(kc8, "kc8", (torch.uint8,)), _dev(vc8, "vc8", (torch.uint8,)),
         _dev(ksc, "ksc", _F16), _dev(vsc, "vsc", _F16),
         _dev(ktail, "ktail", _F16, KVGROUP * NKV * D), _dev(vtail, "vtail", _F16, KVGROUP * NKV * D),
         committed, qpos, float(scale), _dev(out, "out", _F16, NH * D),
         _dev(ws, "ws", (torch.uint8,), decode_workspace_bytes(qpos + 1)), ws.numel(), _stream())


def attn_decode_noalloc(q, kc8, vc8, ksc, vsc, ktail, vtail, committed: int, qpos: int,
                        scale: float, out) -> None:
    """attn_decode with the library's own fixed workspace (allocates
    nothing; calls overlapping on one GPU race)."""
    call("cia_attn_decode_noalloc", _dev(q, "q", _F16, NH * D),
         _dev(kc8, "kc8", (torch.uint8,)), _dev(vc8, "vc8", (torch.uint8,)),
         _dev(ksc, "ksc", _F16), _dev(vsc, "vsc", _F16),
         _dev(ktail, "ktail", _F16, KVGROUP * NKV * D), _dev(vtail, "vtail", _F16, KVGROUP * NKV * D),
         committed, qpos, float(scale), _dev(out, "out", _F16, NH * D), _stream())


# ------------------------------------------------------------ H2O
def kv_quant_write(k, v, kf, vf, ks, vs, dst_slots, S: int) -> None:
    """engine.cu:317-333: per-token FP8 quantisation into slots dst_slots[j]."""
    call("cia_kv_quant_write", _dev(k, "k", _F16, S * NKV * D), _dev(v, "v", _F16, S * NKV * D),
         _dev(kf, "kf", (torch.uint8,)), _dev(vf, "vf", (torch.uint8,)),
         _dev(ks, "ks", _F16), _dev(vs, "vs", _F16),
         _dev(dst_slots, "dst_slots", (torch.int32,), S), S, _stream())


def h2o_place(k, v, kf, vf, ks, vs, attn_sum, slot_pos, dst_slots, n_live: int, C: int, W: int,
              S: int, past: int) -> int:
    """engine.cu:808-826 on the device: slot choice + per-token quantisation.

    Updates attn_sum, slot_pos, dst_slots in place; returns the new n_live."""
    nl = ctypes.c_int(n_live)
    call("cia_h2o_place", _dev(k, "k", _F16, S * NKV * D), _dev(v, "v", _F16, S * NKV * D),
         _dev(kf, "kf", (torch.uint8,), C * NKV * D), _dev(vf, "vf", (torch.uint8,), C * NKV * D),
         _dev(ks, "ks", _F16, C * NKV), _dev(vs, "vs", _F16, C * NKV),
         _dev(attn_sum, "attn_sum", (torch.float32,), C),
         _dev(slot_pos, "slot_pos", (torch.int32,), C),
         _dev(dst_slots, "dst_slots", (torch.int32,), S), ctypes.byref(nl), C, W, S, past,
         _stream())
    return nl.value


def mass_workspace_bytes(S: int) -> int:
    return int(_lib.lib().cia_mass_workspace_bytes(S))


def h2o_workspace_bytes(S: int, C: int) -> int:
    return int(_lib.lib().cia_h2o_workspace_bytes(S, C))


def attention_h2o(q, kf, vf, ks, vs, slot_pos, n_live: int, out, attn_sum, S: int, past: int,
                  scale: float, ws) -> None:
    """engine.cu:337-384 with the deterministic attention-mass rule; ws is a
    uint8 device tensor of at least h2o_workspace_bytes(S, n_live) bytes."""
    call("cia_attention_h2o", _dev(q, "q", _F16, S * NH * D),
         _dev(kf, "kf", (torch.uint8,), n_live * NKV * D), _dev(vf, "vf", (torch.uint8,), n_live * NKV * D),
         _dev(ks, "ks", _F16, n_live * NKV), _dev(vs, "vs", _F16, n_live * NKV),
         _dev(slot_pos, "slot_pos", (torch.int32,), n_live), n_live,
         _dev(out, "out", _F16, S * NH * D), _dev(attn_sum, "attn_sum", (torch.float32,), n_live),
         S, past, float(scale), _dev(ws, "ws", (torch.uint8,), h2o_workspace_bytes(S, n_live)),
         ws.numel(), _stream())


# ------------------------------------------------------------ QK producers
def qk_norm_rope(q, k, qw, kw, pos, S: int, eps: float = 1e-5, theta: float = 5.0e6) -> None:
    """engine.cu:799-801 (rmsnorm_head on q and k, then rope) in place, one launch."""
    call("cia_qk_norm_rope", _dev(q, "q", _F16, S * NH * D), _dev(k, "k", _F16, S * NKV * D),
         _dev(qw, "qw", _F16, D), _dev(kw, "kw", _F16, D), _dev(pos, "pos", (torch.int32,), S),
         S, float(eps), float(theta), _stream())


# ------------------------------------------------------------ INT4 projections
def _int4(packed, scales, N: int, K: int, name: str):
    return (_dev(packed, name + ".packed", (torch.uint8,), N * K // 2),
            _dev(scales, name + ".scales", _F16, N * K // 128))


def gemv_int4(x, packed, scales, y, N: int, K: int, M: int, add: bool = False) -> None:
    """engine.cu:83-109 / 626-630: y fp32 [M, N] = x [M, K] W^T for INT4
    group-128 W (packed u8 [N, K/2], scales fp16 [N, K/128]); add=True
    accumulates into y (out_proj + residual, engine.cu:858-859)."""
    p, s = _int4(packed, scales, N, K, "w")
    call("cia_gemv_int4_add" if add else "cia_gemv_int4", _dev(x, "x", _F16, M * K), p, s,
         _dev(y, "y", (torch.float32,), M * N), N, K, M, _stream())


def qkv_proj_int4(x, wq, wk, wv, q, k, v, M: int, K: int = 2048) -> None:
    """engine.cu:792-797 in one launch: q/k/v fp16 = fp16(x W^T); wq, wk, wv
    are (packed, scales) pairs with N = q.shape[-1] / k.shape[-1] rows."""
    Nq = q.numel() // M
    Nkv = k.numel() // M
    pq, sq = _int4(*wq, Nq, K, "wq")
    pk, sk = _int4(*wk, Nkv, K, "wk")
    pv, sv = _int4(*wv, Nkv, K, "wv")
    call("cia_qkv_proj_int4", _dev(x, "x", _F16, M * K), pq, sq, Nq, pk, sk, pv, sv, Nkv, K, M,
         _dev(q, "q", _F16, M * Nq), _dev(k, "k", _F16, M * Nkv), _dev(v, "v", _F16, M * Nkv),
         _stream())
