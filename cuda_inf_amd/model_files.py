"""Model files around the attention path, through the C-ABI of
include/cuda_inf_model.h: the weight index and blob (``Model``, mirroring
the reference's ``Model`` of src/engine.cu:55-78 and its loading in main(),
664-692) and the byte-level BPE tokenizer (``Tokenizer``, mirroring
src/tokenizer.h's ``Tokenizer``: load / encode / decode).

The blob is one device allocation (a torch uint8 tensor) holding
weights.bin as the file lays it out; ``q4`` and ``f16`` return views into
it, so the projections read the weights where the upload put them.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import torch

from ._lib import call, check, cia_tensor_desc, lib

KIND_FP16, KIND_INT4G = 0, 1
INT4_GROUP = 128  # group size along K of an int4g tensor (tools/export_weights.py:9-12)


@dataclass(frozen=True)
class TensorDesc:
    """One index entry (tools/make_index.py:3-11; engine.cu:56 ``TDesc``)."""
    kind: int
    offset: int
    packed: int
    scales: int
    d0: int
    d1: int


def read_index(path: str) -> dict[str, TensorDesc]:
    """index.bin -> {name: TensorDesc} (engine.cu:665-675)."""
    n = ctypes.c_int64()
    p = os.fsencode(path)
    call("cia_index_read", p, None, 0, ctypes.byref(n))
    arr = (cia_tensor_desc * max(n.value, 1))()
    call("cia_index_read", p, arr, n.value, ctypes.byref(n))
    out = {}
    for i in range(n.value):
        d = arr[i]
        out[d.name.decode("utf-8", "surrogateescape")] = TensorDesc(
            d.kind, d.offset, d.packed, d.scales, d.d0, d.d1)
    return out


def upload_file(path: str, dst: torch.Tensor, stream=None) -> int:
    """Copies the file into the device tensor ``dst`` (uint8, at least the
    file's size) through pinned, double-buffered staging; returns the byte
    count once the bytes are in HBM."""
    if dst.device.type != "cuda" or dst.dtype != torch.uint8 or not dst.is_contiguous():
        raise ValueError("dst must be a contiguous uint8 device tensor")
    n = ctypes.c_uint64()
    s = stream if stream is not None else torch.cuda.current_stream(dst.device)
    with torch.cuda.device(dst.device):
        call("cia_weights_upload", os.fsencode(path), dst.data_ptr(), dst.numel(),
             ctypes.byref(n), s.cuda_stream)
    return n.value


class Model:
    """The weight blob in HBM and its index (engine.cu:59-78)."""

    def __init__(self, idx: dict[str, TensorDesc], blob: torch.Tensor):
        self.idx, self.blob = idx, blob

    @classmethod
    def load(cls, directory: str, device="cuda") -> "Model":
        """<directory>/index.bin and weights.bin, the blob uploaded in one
        allocation (engine.cu:664-692).  Every tensor must lie inside the
        blob."""
        idx = read_index(os.path.join(directory, "index.bin"))
        wp = os.path.join(directory, "weights.bin")
        size = ctypes.c_uint64()
        call("cia_file_size", os.fsencode(wp), ctypes.byref(size))
        for name, t in idx.items():
            if t.offset + t.packed + t.scales > size.value:
                raise ValueError(f"tensor {name} ends past weights.bin ({size.value} bytes)")
        blob = torch.empty(max(size.value, 1), dtype=torch.uint8, device=device)
        upload_file(wp, blob)
        return cls(idx, blob)

    def _get(self, name: str, what: str) -> TensorDesc:
        t = self.idx.get(name)
        if t is None:
            raise KeyError(f"missing {what} {name}")  # (engine.cu:67, 74)
        return t

    def q4(self, name: str):
        """(packed u8 [N, K/2], scales fp16 [N, K/128], N, K) views of an
        int4g tensor (engine.cu:65-70)."""
        t = self._get(name, "q4")
        N, K = int(t.d0), int(t.d1)
        if t.kind != KIND_INT4G or K % INT4_GROUP or t.packed != N * K // 2 or \
                t.scales != N * (K // INT4_GROUP) * 2:
            raise ValueError(f"{name} is not an int4g [{N}, {K}] tensor")
        if t.offset % 2 or (t.offset + t.packed) % 2:
            raise ValueError(f"{name}: scales not 2-byte aligned in the blob")
        packed = self.blob[t.offset:t.offset + t.packed].view(N, K // 2)
        scales = self.blob[t.offset + t.packed:t.offset + t.packed + t.scales] \
            .view(torch.float16).view(N, K // INT4_GROUP)
        return packed, scales, N, K

    def f16(self, name: str) -> torch.Tensor:
        """fp16 view [d0] or [d0, d1] of an fp16 tensor (engine.cu:71-77)."""
        t = self._get(name, "f16")
        if t.kind != KIND_FP16 or t.offset % 2:
            raise ValueError(f"{name} is not an aligned fp16 tensor")
        shape = (int(t.d0),) if t.d1 == 0 else (int(t.d0), int(t.d1))
        n = 1
        for s in shape:
            n *= s
        if 2 * n != t.packed:
            raise ValueError(f"{name}: {t.packed} bytes for shape {shape}")
        return self.blob[t.offset:t.offset + t.packed].view(torch.float16).view(shape)


class Tokenizer:
    """src/tokenizer.h's Tokenizer through the C-ABI (host only)."""

    def __init__(self):
        self._h = ctypes.c_void_p()

    def load(self, directory: str) -> bool:
        """vocab.tsv, merges.tsv, special.tsv of ``directory``; False when a
        file is missing or unreadable (tokenizer.h:42-81)."""
        self.close()
        rc = lib().cia_tok_load(os.fsencode(directory), ctypes.byref(self._h))
        if rc == 7:  # CIA_ERR_IO
            return False
        check("cia_tok_load", rc)
        return True

    def close(self) -> None:
        if self._h:
            lib().cia_tok_free(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _need(self):
        if not self._h:
            raise RuntimeError("tokenizer not loaded")

    def encode(self, text) -> list[int]:
        """Token ids of ``text`` (str, or bytes taken as UTF-8) (tokenizer.h:177-208)."""
        self._need()
        b = text.encode("utf-8") if isinstance(text, str) else bytes(text)
        ids = (ctypes.c_int32 * max(len(b), 1))()
        n = ctypes.c_int64()
        call("cia_tok_encode", self._h, b, len(b), ids, len(b), ctypes.byref(n))
        return list(ids[:n.value])

    def decode_bytes(self, ids, skip_special: bool = False) -> bytes:
        """The bytes of ``ids`` (tokenizer.h:218-231)."""
        self._need()
        ids = list(ids)
        arr = (ctypes.c_int32 * max(len(ids), 1))(*ids)
        n = ctypes.c_int64()
        call("cia_tok_decode", self._h, arr, len(ids), int(skip_special), None, 0,
             ctypes.byref(n))
        out = ctypes.create_string_buffer(max(n.value, 1))
        call("cia_tok_decode", self._h, arr, len(ids), int(skip_special), out, n.value,
             ctypes.byref(n))
        return out.raw[:n.value]

    def decode(self, ids, skip_special: bool = False) -> str:
        return self.decode_bytes(ids, skip_special).decode("utf-8", "replace")
