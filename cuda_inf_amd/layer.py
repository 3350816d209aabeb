"""One attention layer of the cuda_inf engine: its device cache, the host state
the reference keeps beside it, and the attention branch of ``layer_forward``
(engine.cu:802-857), run by the C++ driver ``cia_layer_forward``.

Also exposes the host-only policy helpers (append planner, H2O clamps and
slot picker) which need no GPU.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import (D, KVGROUP, NH, NKV, NSPLIT_DEFAULT, call, cia_append_op, cia_attn_proj,
                   cia_layer)
from .kernels import decode_workspace_bytes, h2o_workspace_bytes

HIDDEN = _lib.HIDDEN


# ------------------------------------------------------------ host policy
def kv_append_plan(committed: int, S: int, past: int):
    """engine.cu:830-845 as a list of ops; returns (ops, new_committed)."""
    max_ops = S // KVGROUP + 2
    ops = (cia_append_op * max_ops)()
    c = ctypes.c_int(committed)
    n = ctypes.c_int(0)
    call("cia_kv_append_plan", ctypes.byref(c), S, past, ops, max_ops, ctypes.byref(n))
    out = [dict(src_token=o.src_token, slot=o.slot, cnt=o.cnt, commit=bool(o.commit),
                commit_base=o.commit_base, commit_grp=o.commit_grp) for o in ops[:n.value]]
    return out, c.value


def h2o_clamp(budget: int, window: int, prompt_len: int, maxT: int):
    """engine.cu:752-756; returns (budget, window)."""
    b, w = ctypes.c_int(budget), ctypes.c_int(window)
    _lib.lib().cia_h2o_clamp(ctypes.byref(b), ctypes.byref(w), prompt_len, maxT)
    return b.value, w.value


def h2o_pick_slots(n_live: int, C: int, W: int, slotpos: np.ndarray, attn_host: np.ndarray,
                   S: int, past: int):
    """engine.cu:808-823 on host arrays (updated in place).

    Returns (n_live, dst[S], zeroed[S], evictions)."""
    assert slotpos.dtype == np.int32 and attn_host.dtype == np.float32
    dst = np.zeros(S, np.int32)
    zeroed = np.zeros(S, np.int32)
    nl = ctypes.c_int(n_live)
    ev = _lib.lib().cia_h2o_pick_slots(ctypes.byref(nl), C, W, slotpos.ctypes.data,
                                       attn_host.ctypes.data, S, past, dst.ctypes.data,
                                       zeroed.ctypes.data)
    if ev < 0:
        _lib.check("cia_h2o_pick_slots", -ev)
    return nl.value, dst, zeroed, ev


# ------------------------------------------------------------ the layer
class AttnLayer:
    """Device buffers of one attention layer (engine.cu:596-613, 731-770).

    ``nsplit`` > 0 runs the reference's flash-decoding split + combine with
    that split count; ``nsplit`` = 0 runs the matrix-core decode with the
    library's own split (and the tail write fused into it).  ``budget`` > 0
    enables H2O eviction with a ``budget``-slot buffer and local ``window``
    (0 -> budget/2, clamped as the reference does against ``prompt_len``).
    ``qk_norm`` = (q weight, k weight), fp16 [64] each: q and k passed to
    ``forward`` are raw and the layer runs the QK producers (per-head
    RMSNorm with ``eps``, RoPE at ``theta``; engine.cu:799-801) itself --
    inside the decode kernels for single-token steps, else one launch into a
    ``max_batch``-token scratch.
    """

    def __init__(self, max_tokens: int, *, nsplit: int = NSPLIT_DEFAULT, budget: int = 0,
                 window: int = 0, prompt_len: int = 0, max_batch: int = 4096,
                 qk_norm=None, eps: float = 1e-5, theta: float = 5.0e6, device="cuda"):
        dev = torch.device(device)
        self.device = dev
        self.maxT = max_tokens
        u8, f16, f32, i32 = torch.uint8, torch.float16, torch.float32, torch.int32
        ng = max_tokens // KVGROUP + 2
        self.kc8 = torch.zeros((max_tokens, NKV, D), dtype=u8, device=dev)
        self.vc8 = torch.zeros((max_tokens, NKV, D), dtype=u8, device=dev)
        self.ksc = torch.zeros((ng, NKV), dtype=f16, device=dev)
        self.vsc = torch.zeros((ng, NKV), dtype=f16, device=dev)
        self.ktail = torch.zeros((KVGROUP, NKV, D), dtype=f16, device=dev)
        self.vtail = torch.zeros((KVGROUP, NKV, D), dtype=f16, device=dev)
        self.nsplit = nsplit
        ns = max(nsplit, 1)
        self.pm = torch.zeros(NH * ns, dtype=f32, device=dev)
        self.pl = torch.zeros(NH * ns, dtype=f32, device=dev)
        self.po = torch.zeros(NH * ns * D, dtype=f32, device=dev)
        self.ws_decode = torch.zeros(decode_workspace_bytes(max_tokens), dtype=u8, device=dev)
        s = cia_layer()
        for name in ("kc8", "vc8", "ksc", "vsc", "ktail", "vtail", "pm", "pl", "po", "ws_decode"):
            setattr(s, name, getattr(self, name).data_ptr())
        s.maxT, s.committed, s.nsplit = max_tokens, 0, nsplit
        self.budget = 0
        if budget > 0:
            budget, window = h2o_clamp(budget, window, prompt_len, max_tokens)
            self.budget, self.window = budget, window
            C = budget
            self.kf = torch.zeros((C, NKV, D), dtype=u8, device=dev)
            self.vf = torch.zeros((C, NKV, D), dtype=u8, device=dev)
            self.ks = torch.zeros((C, NKV), dtype=f16, device=dev)
            self.vs = torch.zeros((C, NKV), dtype=f16, device=dev)
            self.hattn = torch.zeros(C, dtype=f32, device=dev)
            self.d_slotpos = torch.full((C,), -1, dtype=i32, device=dev)
            self.d_dst = torch.zeros(max_batch, dtype=i32, device=dev)
            self.ws_mass = torch.zeros(h2o_workspace_bytes(max_batch, C), dtype=u8, device=dev)
            s.budget, s.window = budget, window
            for name in ("kf", "vf", "ks", "vs", "hattn", "d_slotpos", "d_dst", "ws_mass"):
                setattr(s, name, getattr(self, name).data_ptr())
            s.n_live = 0
        if qk_norm is not None:
            qw, kw = qk_norm
            self.qw = torch.as_tensor(qw).to(device=dev, dtype=f16).contiguous()
            self.kw = torch.as_tensor(kw).to(device=dev, dtype=f16).contiguous()
            assert self.qw.numel() == D and self.kw.numel() == D
            self.prep_ws = torch.zeros(max_batch * (NH + NKV) * D, dtype=f16, device=dev)
            s.qw, s.kw = self.qw.data_ptr(), self.kw.data_ptr()
            s.eps, s.theta = float(eps), float(theta)
            s.prep_ws, s.prep_cap = self.prep_ws.data_ptr(), max_batch
        self.max_batch = max_batch
        self._s = s

    @property
    def committed(self) -> int:
        return self._s.committed

    @property
    def n_live(self) -> int:
        return self._s.n_live

    def forward(self, q, k, v, past: int, out=None, scale: float = 0.125, evicted: bool = True):
        """Append k, v [S,8,64] at positions past.. and attend q [S,32,64].

        Returns (out [S,32,64] fp16, evicted slot of the last token or -1).
        On an H2O layer the evicted slot is read back from the device, which
        waits for the stream; ``evicted=False`` skips that (returns None)."""
        S = k.shape[0]
        if (self.budget or self._s.qw) and S > self.max_batch:
            raise ValueError(f"S={S} exceeds max_batch={self.max_batch}")
        for t, name, n in ((q, "q", S * NH * D), (k, "k", S * NKV * D), (v, "v", S * NKV * D)):
            if t.dtype != torch.float16 or not t.is_cuda or not t.is_contiguous() or t.numel() != n:
                raise ValueError(f"{name}: need a contiguous device fp16 tensor of {n} elements")
        if out is None:
            out = torch.empty((S, NH, D), dtype=torch.float16, device=self.device)
        ev = ctypes.c_int(-1)
        call("cia_layer_forward", ctypes.byref(self._s), q.data_ptr(), k.data_ptr(), v.data_ptr(),
             out.data_ptr(), S, past, float(scale), ctypes.byref(ev) if evicted else None,
             torch.cuda.current_stream().cuda_stream)
        return out, (ev.value if evicted else None)

    # -------------------------------------------------------- projections
    def set_projections(self, wq, wk, wv, wo):
        """INT4 group-128 weights of q/k/v/out_proj (engine.cu:792-797, 858):
        each a (packed u8 [N, 1024], scales fp16 [N, 16]) pair of device
        tensors, N = 2048 / 512 / 512 / 2048."""
        P = cia_attn_proj()
        self._proj_w = []
        for name, (pk, sc), N in (("q", wq, NH * D), ("k", wk, NKV * D), ("v", wv, NKV * D),
                                  ("o", wo, HIDDEN)):
            if (pk.dtype != torch.uint8 or not pk.is_cuda or not pk.is_contiguous()
                    or pk.numel() != N * HIDDEN // 2):
                raise ValueError(f"{name}_proj packed: need contiguous device uint8 [{N}, {HIDDEN // 2}]")
            if (sc.dtype not in (torch.float16, torch.int16) or not sc.is_cuda
                    or not sc.is_contiguous() or sc.numel() != N * HIDDEN // 128):
                raise ValueError(f"{name}_proj scales: need contiguous device fp16 [{N}, {HIDDEN // 128}]")
            setattr(P, name + "_packed", pk.data_ptr())
            setattr(P, name + "_scales", sc.data_ptr())
            self._proj_w += [pk, sc]
        self.proj_ws = torch.zeros(self.max_batch * (2 * NH * D + 2 * NKV * D), dtype=torch.float16,
                                   device=self.device)
        P.ws, P.cap = self.proj_ws.data_ptr(), self.max_batch
        self._p = P

    def block_forward(self, x, h, past: int, scale: float = 0.125, evicted: bool = True):
        """engine.cu:792-859: x fp16 [S, 2048] (normalised hidden state) through
        q/k/v_proj, the QK producers (when the layer has qk_norm), attention
        and out_proj, added into the residual h fp32 [S, 2048] in place.
        Returns the evicted slot of the last token on an H2O layer (or -1;
        None with evicted=False)."""
        S = x.numel() // HIDDEN
        if x.dtype != torch.float16 or not x.is_cuda or not x.is_contiguous() or x.numel() != S * HIDDEN:
            raise ValueError("x: need a contiguous device fp16 tensor [S, 2048]")
        if h.dtype != torch.float32 or not h.is_cuda or not h.is_contiguous() or h.numel() != S * HIDDEN:
            raise ValueError("h: need a contiguous device fp32 tensor [S, 2048]")
        ev = ctypes.c_int(-1)
        call("cia_attn_block_forward", ctypes.byref(self._s), ctypes.byref(self._p), x.data_ptr(),
             h.data_ptr(), S, past, float(scale), ctypes.byref(ev) if evicted else None,
             torch.cuda.current_stream().cuda_stream)
        return ev.value if evicted else None


def attn_block_loop(layers, x, h, past: int, steps: int, scale: float = 0.125, events=None):
    """cia_attn_block_loop: steps decode steps through the attention branches
    of ``layers`` (AttnLayer with projections).  x fp16 [steps, n_layers, 2048],
    h fp32 [2048] (the residual stream, added into in place)."""
    n = len(layers)
    arr = (cia_layer * n)(*[L._s for L in layers])
    parr = (cia_attn_proj * n)(*[L._p for L in layers])
    ev = None
    if events is not None:
        for e in events:  # the hipEvent_t handles exist once recorded
            e.record()
        ev = (ctypes.c_void_p * len(events))(*[e.cuda_event for e in events])
    try:
        call("cia_attn_block_loop", arr, parr, n, x.data_ptr(), h.data_ptr(), past, steps,
             float(scale), ev, torch.cuda.current_stream().cuda_stream)
    finally:
        for L, s in zip(layers, arr):  # host counters advance in the copies
            L._s.committed, L._s.n_live = s.committed, s.n_live
