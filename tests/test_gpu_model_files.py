"""weights.bin / index.bin on the GPU (src/engine.cu:55-78, 664-692): a
synthetic model directory in the exporters' format (INT4 group-128
projections, fp16 tensors, filler) is uploaded by cia_weights_upload; the
device blob equals the file byte for byte (sizes across the 64 MiB staging
chunks and the 4 MiB reader slices, a ragged end, an empty file); a q4
tensor found by name feeds cia_gemv_int4 and matches the oracle's GEMV of
the same file bytes to the INT4 tests' bound
    |y_gpu - y_ref| <= 1e-5 * sum_k |x[k] * w[n][k]|."""
import os

import numpy as np
import pytest
import torch

from oracle import model_files as om

pytestmark = pytest.mark.gpu


def _model_dir(tmp, orc, rng, filler_bytes):
    recs, chunks, off = [], [], 0

    def add(name, kind, data, packed, scales, d0, d1):
        nonlocal off
        recs.append(dict(name=name, kind=kind, offset=off, packed=packed, scales=scales,
                         d0=d0, d1=d1))
        chunks.append(data)
        off += len(data)

    emb = rng.standard_normal((1000, 2048)).astype(np.float16)
    add("model.embed_tokens.weight", 0, emb.tobytes(), emb.nbytes, 0, 1000, 2048)
    for nm, N in (("q_proj", 2048), ("k_proj", 512), ("v_proj", 512), ("out_proj", 2048)):
        w = (rng.standard_normal((N, 2048)) * 0.02).astype(np.float32)
        p, s = orc.quant_int4_g128(w)
        add(f"model.layers.2.self_attn.{nm}.weight", 1, p.tobytes() + s.tobytes(), p.nbytes,
            s.nbytes, N, 2048)
    norm = rng.standard_normal(64).astype(np.float16)
    add("model.layers.2.self_attn.q_layernorm.weight", 0, norm.tobytes(), norm.nbytes, 0, 64, 0)
    filler = rng.integers(0, 256, filler_bytes, dtype=np.uint8)
    add("filler", 0, filler.tobytes(), filler_bytes, 0, filler_bytes // 2, 0)
    os.makedirs(tmp, exist_ok=True)
    with open(os.path.join(tmp, "weights.bin"), "wb") as f:
        for c in chunks:
            f.write(c)
    om.write_index(os.path.join(tmp, "index.bin"), recs)
    return recs


def test_load_model_and_project(orc, cia, dev, tmp_path):
    from cuda_inf_amd import kernels as KK
    from cuda_inf_amd.model_files import Model
    rng = np.random.default_rng(31)
    d = str(tmp_path / "m")
    # (~149 MB in all: two full 64 MiB staging chunks and a ragged third)
    _model_dir(d, orc, rng, 140_000_001)
    print("model dir written", flush=True)
    m = Model.load(d, dev)
    torch.cuda.synchronize()
    raw = np.fromfile(os.path.join(d, "weights.bin"), np.uint8)
    assert m.blob.numel() == raw.size
    assert torch.equal(m.blob.cpu(), torch.from_numpy(raw))
    packed, scales, N, K = m.q4("model.layers.2.self_attn.q_proj.weight")
    t = m.idx["model.layers.2.self_attn.q_proj.weight"]
    p_ref = raw[t.offset:t.offset + t.packed].reshape(N, K // 2)
    s_ref = raw[t.offset + t.packed:t.offset + t.packed + t.scales].view(np.uint16).reshape(N, K // 128)
    x = rng.standard_normal((3, K)).astype(np.float16)
    y = torch.zeros((3, N), dtype=torch.float32, device=dev)
    KK.gemv_int4(torch.from_numpy(x.view(np.int16)).to(dev).view(torch.float16), packed, scales,
                 y, N, K, 3)
    torch.cuda.synchronize()
    ref, ab = orc.gemv_int4(x, p_ref, s_ref, want_absum=True)
    err = np.abs(y.cpu().numpy().astype(np.float64) - ref)
    assert (err <= 1e-5 * ab + 1e-30).all(), float((err - 1e-5 * ab).max())
    norm = m.f16("model.layers.2.self_attn.q_layernorm.weight")
    t = m.idx["model.layers.2.self_attn.q_layernorm.weight"]
    assert norm.shape == (64,)
    assert np.array_equal(norm.cpu().numpy().view(np.uint8), raw[t.offset:t.offset + 128])
    with pytest.raises(KeyError, match="missing q4"):
        m.q4("model.layers.3.self_attn.q_proj.weight")
    with pytest.raises(ValueError):
        m.q4("model.embed_tokens.weight")


@pytest.mark.parametrize("size", [0, 1, 4 << 20, (4 << 20) + 3, 64 << 20, (64 << 20) + 1,
                                  (128 << 20) - 7, 200_000_001])
def test_upload_sizes(cia, dev, tmp_path, size):
    from cuda_inf_amd.model_files import upload_file
    rng = np.random.default_rng(size % 1000)
    raw = rng.integers(0, 256, size, dtype=np.uint8)
    p = str(tmp_path / "w.bin")
    raw.tofile(p)
    print(f"upload {size} bytes", flush=True)
    dst = torch.full((size + 4096,), 0xA5, dtype=torch.uint8, device=dev)
    assert upload_file(p, dst) == size
    torch.cuda.synchronize()
    got = dst.cpu()
    assert torch.equal(got[:size], torch.from_numpy(raw))
    assert bool((got[size:] == 0xA5).all())  # nothing past the file's bytes


def test_upload_rejects_small_destination(cia, dev, tmp_path):
    from cuda_inf_amd._lib import CiaError
    from cuda_inf_amd.model_files import upload_file
    p = str(tmp_path / "w.bin")
    np.zeros(1000, np.uint8).tofile(p)
    dst = torch.zeros(999, dtype=torch.uint8, device=dev)
    with pytest.raises(CiaError, match="CIA_ERR_ARG"):
        upload_file(p, dst)
