"""Device sampling on cuda:0 against the oracle: the partial top-k readback
(nuq_topk) and the history penalties (nuq_penalize), after the reference's
own device checks (inference/metal-check.zig:5530-5658, sections 9b/9c).

Bars: the top-k ids and values are bit-exact (an ordering, no arithmetic);
the exp-sum total is within 2e-6 relative of the F64 sum, the bound
metal-check asserts (sampling/root.zig:175-181 relies on it); penalties are
bit-exact (F32 division and multiply, denormals preserved).
"""
import math

import numpy as np
import pytest

import nuclis_amd as nq
from nuclis_amd.synth import gaussian
from oracle import oracle as orc
from tests.gpu_util import to_gpu

pytestmark = pytest.mark.gpu
VOCAB = 248_320  # the vocabulary metal-check uses


@pytest.fixture(scope="module")
def backend():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return nq.Backend(0)


def check_topk(backend, v, k, t):
    top = backend.topk(to_gpu(v), k, t)
    ids, vals, total, finite = orc.topk(v, k, t)
    assert top.ids == ids.tolist()
    assert np.array(top.values, np.float32).view(np.uint32).tolist() == vals.view(np.uint32).tolist()
    assert top.finite == finite
    return top, total


def test_topk_vocabulary_with_ties_matches_the_reference_sort(backend):
    v = gaussian(30, VOCAB) * 2
    v[123456] = 14.0
    v[654] = 14.0                     # two-way tie at the top: the lower id first
    v[1000 + 7 * np.arange(64)] = 12.5  # a run of equal values further down
    print("[sampling] top-k vocab ties", flush=True)
    top, _ = check_topk(backend, v, 256, 0.7)
    assert top.ids[:2] == [654, 123456]


def test_topk_exp_sum_is_within_the_reference_bound(backend):
    v = gaussian(31, VOCAB) * 2       # flat: ~1e5 terms contribute
    print("[sampling] top-k flat exp-sum", flush=True)
    top, exact = check_topk(backend, v, 256, 1.5)
    assert top.values[0] == float(v.max())
    fsum = math.fsum(math.exp((float(x) - float(v.max())) / 1.5) for x in v.astype(np.float64))
    assert abs(exact - fsum) <= 1e-9 * fsum
    assert abs(top.total - fsum) / fsum <= 2e-6, (top.total, fsum)


def test_topk_nan_raises_its_flag_and_never_enters_the_list(backend):
    v = gaussian(32, VOCAB)
    v[77777] = np.nan
    v[5] = 50.0
    top, _ = check_topk(backend, v, 256, 0.7)
    assert 77777 not in top.ids and not top.finite and top.ids[0] == 5
    w = gaussian(33, VOCAB)
    w[100] = np.inf
    top = backend.topk(to_gpu(w), 16, 1.0)
    assert not top.finite and top.ids[0] == 100


@pytest.mark.parametrize("count,k", [(1, 1), (256, 256), (4096, 256), (4097, 256), (5000, 1), (70_000, 100),
                                     (262_144, 256), (151_936, 256), (131_072, 37)])
def test_topk_chunking_and_sizes(backend, count, k):
    """One chunk, two, and the multi-pass merges up to the 262,144 limit."""
    rng = np.random.default_rng(count + k)
    v = (rng.standard_normal(count) * 3).astype(np.float32)
    v[rng.integers(0, count, max(1, count // 50))] = 1.25    # many ties
    v[rng.integers(0, count, 3)] = 0.0
    v[rng.integers(0, count, 3)] = -0.0
    check_topk(backend, v, k, 1.0)


def test_topk_with_fewer_finite_values_than_k(backend):
    v = np.full(600, np.nan, np.float32)
    v[[3, 300, 599]] = [1.0, -np.inf, 2.0]
    top, _ = check_topk(backend, v, 8, 1.0)
    assert top.ids[:3] == [599, 3, 300] and top.ids[3:] == [0xffffffff] * 5


def test_topk_is_repeatable(backend):
    v = gaussian(34, 151_936)
    a = backend.topk(to_gpu(v), 256, 0.8)
    b = backend.topk(to_gpu(v), 256, 0.8)
    assert a == b


def test_topk_shape_rejections(backend):
    v = to_gpu(gaussian(35, 1024))
    for count, k, t in ((nq.backend.TOPK_MAX_COUNT + 1, 256, 0.7), (1024, 0, 0.7), (1024, 256, 0.0),
                        (255, 256, 0.7), (1024, 257, 0.7), (1024, 16, float("nan")), (1024, 16, float("inf"))):
        with pytest.raises(nq.InvalidShape):
            backend.topk(v, k, t, count=count)


OPTIONS = [(1.0, 1.5), (1.1, 0.0), (4.0, 0.5), (0.5, -2.0)]  # (repetition, presence), metal-check.zig:5606-5611


def test_penalize_matches_the_sampler_for_every_sign(backend):
    import torch
    count = 4096
    ids = [i * 61 + 3 for i in range(64)] + [count - 1]
    words = orc.history_words(ids, count)
    wg = torch.from_numpy(words.view(np.int32)).cuda()
    for vector in range(8):
        raw = gaussian(40 + vector, count) * 4
        for i in range(64):
            raw[i * 61 + 3] = [2.5, -3.5, 0.0, -0.0, np.float32(np.finfo(np.float32).tiny) * np.float32(0.5)][i % 5]
        raw[count - 1] = -1.25
        for rep, pres in OPTIONS:
            g = to_gpu(raw)
            backend.penalize(g, wg, rep, pres)
            backend.sync()
            want = orc.penalize(raw, words, rep, pres)
            got = g.cpu().numpy()
            assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist(), (vector, rep, pres)


def test_penalize_shape_rejections_leave_logits_untouched(backend):
    import torch
    raw = gaussian(50, 4096)
    g = to_gpu(raw)
    words = torch.zeros(128, dtype=torch.int32, device="cuda")
    for count, w, rep, pres in ((0, words, 1.0, 0.0), (4096, words[:4], 1.0, 0.0), (4096, words, 0.0, 0.0),
                                (4096, words, 1.0, float("nan")), (4096, words, float("inf"), 0.0)):
        with pytest.raises(nq.InvalidShape):
            backend.penalize(g, w, rep, pres, count=count)
    backend.sync()
    assert np.array_equal(g.cpu().numpy(), raw)


def test_penalized_then_greedy_and_topk_agree_with_the_sampler(backend):
    """The device plan order (penalize, then argmax / top-k) on the hand case."""
    import torch
    logits = np.array([1.0, 2.0, 1.5, -1.0], np.float32)
    words = torch.from_numpy(orc.history_words([1, 3], 4).view(np.int32)).cuda()
    g = to_gpu(logits)
    backend.penalize(g, words, 1.0, 1.0)   # presence 1.0 -> [1, 1, 1.5, -2]
    assert backend.argmax(g) == 2
    top = backend.topk(g, 4, 1.0)
    assert top.ids == [2, 0, 1, 3] and top.values == [1.5, 1.0, 1.0, -2.0]


@pytest.mark.parametrize("encoding", [12, 14])
def test_flat_entry_points_equal_the_descriptor_forms(backend, encoding):
    """nuq_gemv / nuq_gemm / nuq_dequant_rows (raw pointer + stride) run the
    same kernels as nuq_matvec / nuq_matmul / nuq_dequant_range."""
    import ctypes
    import torch
    L = nq.lib()
    rows, columns = 512, 2048
    w = nq.quantize(encoding, gaussian(60, (rows, columns), 0.02))
    wg = to_gpu(w)
    m = nq.Matrix(encoding, rows, columns, wg)
    stride = w.shape[1]
    x = to_gpu(gaussian(61, columns))
    a, b = torch.empty(rows, device="cuda"), torch.empty(rows, device="cuda")
    backend.matvec(m, x, a)
    backend._call(L.nuq_gemv, encoding, wg.data_ptr(), stride, rows, columns, x.data_ptr(), b.data_ptr())
    xt = to_gpu(gaussian(62, (64, columns)), torch.float16)
    c, d = torch.empty(64, rows, device="cuda"), torch.empty(64, rows, device="cuda")
    backend.matmul(m, xt, columns, c, rows, 64)
    backend._call(L.nuq_gemm, encoding, wg.data_ptr(), stride, rows, columns, xt.data_ptr(), nq.F16, columns,
                  d.data_ptr(), rows, 64)
    e, f = torch.empty(rows, columns, device="cuda"), torch.empty(rows, columns, device="cuda")
    backend.dequant_rows(m, 0, rows, e)
    backend._call(L.nuq_dequant_rows, encoding, wg.data_ptr(), stride, rows, columns, f.data_ptr())
    backend.sync()
    assert torch.equal(a, b) and torch.equal(c, d) and torch.equal(e, f)
    with pytest.raises(nq.InvalidByteLength):
        backend._call(L.nuq_gemv, encoding, wg.data_ptr(), stride + 2, rows, columns, x.data_ptr(), b.data_ptr())
    with pytest.raises(nq.InvalidByteLength):
        backend._call(L.nuq_gemv, encoding, wg.data_ptr(), (1 << 63), rows, columns, x.data_ptr(), b.data_ptr())
    del ctypes
