"""Writes tests/golden/h2o_c2048_w256_seed7.npz: the H2O eviction workload
(2048-slot per-token FP8 buffer, local window 256, 1024-token prompt, 4000
decode steps, N(0,1) q/k/v from seed 7, no norm/RoPE) run through the CPU
oracle.  Stored: the evicted slot of every decode step (-1 before the buffer
fills), the final attention mass, and a digest of the inputs.

The reference's own H2O path (engine.cu:803-828) cannot run here (CUDA), so
this fixture pins the GPU run to the oracle's deterministic restatement.

    python tests/golden/make_h2o_golden.py [--steps 4000]
"""
import argparse
import hashlib
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

C, W, PROMPT, STEPS, SEED = 2048, 256, 1024, 4000, 7
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "h2o_c2048_w256_seed7.npz")


def inputs(steps=STEPS):
    """q [N,32,64], k, v [N,8,64] fp16 for N = PROMPT + steps tokens (CPU)."""
    from cuda_inf_amd.workload import qkv
    q, k, v = qkv(PROMPT + steps, seed=SEED, device="cpu", prep=False)
    return q, k, v


def digest(q, k, v) -> str:
    h = hashlib.sha256()
    for t in (q, k, v):
        h.update(t.contiguous().view(-1).numpy().view(np.uint16).tobytes())
    return h.hexdigest()


def run_oracle(q, k, v, steps):
    import oracle
    u = lambda t: t.contiguous().numpy().view(np.uint16)  # noqa: E731
    qn, kn, vn = u(q), u(k), u(v)
    cache = oracle.H2OCache(C, W)
    cache.step(qn[:PROMPT], kn[:PROMPT], vn[:PROMPT], 0, want_out=False)
    evicted = np.full(steps, -1, np.int32)
    for j in range(steps):
        pos = PROMPT + j
        dst, zeroed, ev = cache.pick(1, pos)
        oracle.kv_quant_write(kn[pos:pos + 1], vn[pos:pos + 1], cache.kf, cache.vf, cache.ks,
                              cache.vs, dst)
        oracle.attention_h2o(qn[pos:pos + 1], cache.kf, cache.vf, cache.ks, cache.vs,
                             cache.slotpos, cache.n_live, cache.attn, 1, pos)
        if zeroed[0]:
            evicted[j] = dst[0]
    return evicted, cache.attn.copy(), cache.slotpos.copy()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=STEPS)
    a = ap.parse_args()
    q, k, v = inputs(a.steps)
    t0 = time.time()
    evicted, attn, slotpos = run_oracle(q, k, v, a.steps)
    print(f"oracle: {a.steps} steps in {time.time() - t0:.1f} s, "
          f"{int((evicted >= 0).sum())} evictions")
    np.savez(OUT, evicted=evicted, attn_sum=attn, slotpos=slotpos,
             digest=np.array(digest(q, k, v)), C=C, W=W, prompt=PROMPT, steps=a.steps, seed=SEED)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
