"""GGUF file -> device weights -> products, on cuda:0.

A GGUF v3 file of quantized matrices (libnuq's host quantizers, seeded
inputs) is mapped and parsed by libnuq (nuq_gguf_open), its tensor-data
section uploaded in one copy (nuq_gguf_upload), and each matrix used in place
(nuq_gguf_matrix): the device bytes must equal the file's, and every product
must be bit-identical to the same product over the same bytes uploaded
directly, and within the F32 tolerances of tests/gpu_util.py of the oracle.
"""
import numpy as np
import pytest

import nuclis_amd as nq
from nuclis_amd import gguf
from nuclis_amd.synth import gaussian
from oracle import oracle as orc
from tests.gguf_fixture import write_model
from tests.gpu_util import check_close, mass, to_gpu

pytestmark = pytest.mark.gpu

SPECS = [("blk.0.attn_q.weight", 12, 512, 2048), ("blk.0.ffn_down.weight", 14, 256, 2560),
         ("blk.0.attn_v.weight", 8, 296, 1024), ("blk.0.ffn_up.weight", 13, 256, 1280),
         ("blk.0.ffn_gate.weight", 23, 384, 2048)]


@pytest.fixture(scope="module")
def backend():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return nq.Backend(0)


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    path = tmp_path_factory.mktemp("gguf") / "model.gguf"
    mats = {}
    tensors = []
    for i, (name, enc, rows, columns) in enumerate(SPECS):
        w = nq.quantize(enc, gaussian(40 + i, (rows, columns), 0.02))
        mats[name] = (enc, rows, columns, w)
        tensors.append((name, (columns, rows), enc, w.reshape(-1)))
        if i == 1:  # an F32 vector between matrices, as norms sit in real files
            tensors.append(("blk.0.attn_norm.weight", (48,), 0, np.frombuffer(gaussian(9, 48).tobytes(), np.uint8)))
    write_model(path, tensors)
    return path, mats


def test_upload_is_byte_exact_and_products_match_direct_upload(backend, model):
    import torch
    path, mats = model
    raw = np.fromfile(path, dtype=np.uint8)
    with gguf.open(path) as doc:
        print(f"[gguf] {path.stat().st_size} bytes, {len(doc.tensors)} tensors", flush=True)
        dw = gguf.upload(backend, doc)
        assert torch.equal(dw.buffer[:doc.data_bytes].cpu(), torch.from_numpy(raw[doc.data_offset:]))
        for name, (enc, rows, columns, w) in mats.items():
            print(f"[gguf] {name} encoding {enc} {rows}x{columns}", flush=True)
            m = dw.matrix(name)
            assert (m.encoding, m.rows, m.columns, m.byte_len) == (enc, rows, columns, w.nbytes)
            assert (m.bytes.data_ptr() - dw.buffer.data_ptr()) % 32 == 0
            direct = nq.Matrix(enc, rows, columns, to_gpu(w))
            x = gaussian(3, columns)
            xg = to_gpu(x)
            a = torch.empty(rows, device="cuda")
            b = torch.empty(rows, device="cuda")
            backend.matvec(m, xg, a)
            backend.matvec(direct, xg, b)
            backend.sync()
            assert torch.equal(a, b), name
            check_close(a.cpu().numpy(), orc.matvec(enc, rows, columns, w, x), mass(enc, w, rows, columns, x)[0],
                        4e-6, name)
            for tokens in (8, 200):  # verify and prefill routes
                xt = to_gpu(gaussian(4, (tokens, columns)))
                ya = torch.empty(tokens, rows, device="cuda")
                yb = torch.empty(tokens, rows, device="cuda")
                backend.matmul(m, xt, columns, ya, rows, tokens)
                backend.matmul(direct, xt, columns, yb, rows, tokens)
                backend.sync()
                assert torch.equal(ya, yb), (name, tokens)


def test_upload_streams_a_section_larger_than_the_staging_buffers(backend, tmp_path):
    """Three F16 tensors of ~70 MB each: the copy crosses the 64 MiB staging
    chunks at offsets inside tensors, and alternates both buffers."""
    import torch
    rng = np.random.default_rng(11)
    tensors = [(f"t{i}", (4096 + 32 * i, 8600 + i), 1, rng.integers(0, 256, 2 * (4096 + 32 * i) * (8600 + i),
                                                                  dtype=np.uint8)) for i in range(3)]
    path = tmp_path / "big.gguf"
    write_model(path, tensors)
    raw = np.fromfile(path, dtype=np.uint8)
    with gguf.open(path) as doc:
        print(f"[gguf] big file {raw.size} bytes, data {doc.data_bytes}", flush=True)
        dw = gguf.upload(backend, doc)
        want = torch.from_numpy(raw[doc.data_offset:]).cuda()
        assert torch.equal(dw.buffer[:doc.data_bytes], want)
        for name, _, _, data in tensors:
            t = doc.tensors[doc.index(name)]
            assert torch.equal(dw.buffer[t.offset:t.offset + t.bytes].cpu(), torch.from_numpy(data))
