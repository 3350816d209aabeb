"""cuda_inf_amd -- the attention path of the cuda_inf engine (g023/cuda_inf)
rebuilt for MI355X (gfx950): FP8 E4M3 group-64 KV cache with an fp16 tail,
flash-decoding, fused causal prefill and H2O eviction.

The compute lives in libcuda_inf_attn.so (hand-written HIP for gfx950 behind
the C-ABI declared in include/cuda_inf_attn.h).  This package is the host-side
mirror of the reference's kernel-call interface:

* ``kernels``  -- one call per reference kernel, same names and arguments;
* ``layer``    -- ``AttnLayer``: one layer's cache plus the attention branch
  of ``layer_forward``, and the host policy helpers;
* ``workload`` -- seeded synthetic inputs.
"""
from ._lib import D, GQA, KVGROUP, NH, NKV, NSPLIT_DEFAULT, CiaError, build, lib  # noqa: F401

__all__ = ["D", "GQA", "KVGROUP", "NH", "NKV", "NSPLIT_DEFAULT", "CiaError", "build", "lib"]
