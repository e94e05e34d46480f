"""The allocation-free entry point nuq_matvec_segments_noalloc, called
through the C ABI (ctypes on libnuq.so), against nuq_matvec_segments on the
same inputs: bit-identical outputs (same kernels, the SiLU pair's second
GEMV in the fixed per-GPU scratch instead of the context workspace), on two
calls in a row, the second with fewer rows. The context's own workspace
stays unallocated, and pairs beyond the scratch are refused before any
launch."""
import ctypes

import numpy as np
import pytest

import nuclis_amd as nq
from nuclis_amd.backend import _Segment
from nuclis_amd.synth import gaussian
from tests.gpu_util import to_gpu

pytestmark = pytest.mark.gpu


def segs(pairs):
    arr = (_Segment * len(pairs))()
    for i, (m, out) in enumerate(pairs):
        arr[i].matrix = m.c()
        arr[i].output = out.data_ptr()
    return arr


def call(fn, ctx, pairs, x, mode):
    import torch
    torch.cuda.synchronize()
    L = nq.lib()
    assert L.nuq_set_stream(ctx, torch.cuda.current_stream().cuda_stream) == 0
    rc = fn(ctx, segs(pairs), len(pairs), x.data_ptr(), mode)
    assert L.nuq_sync(ctx) == 0
    return rc


def test_noalloc_segments_match_the_allocating_entry_point():
    import torch
    L = nq.lib()
    err = ctypes.create_string_buffer(256)
    ctx = L.nuq_create(0, err, len(err))      # a fresh context: no workspace yet
    ref = nq.Backend(0)
    try:
        columns = 5120
        x = to_gpu(gaussian(81, columns))
        for rows in (17408, 4096):            # second call smaller: stale scratch must not leak
            print(f"[noalloc] silu pair {rows}x{columns}", flush=True)
            gate = nq.Matrix(12, rows, columns, to_gpu(nq.quantize(12, gaussian(82 + rows, (rows, columns), 0.02))))
            up = nq.Matrix(12, rows, columns, to_gpu(nq.quantize(12, gaussian(83 + rows, (rows, columns), 0.02))))
            got = torch.full((rows,), np.nan, device="cuda")
            want = torch.full((rows,), np.nan, device="cuda")
            assert call(L.nuq_matvec_segments_noalloc, ctx, [(gate, got), (up, got)], x,
                        nq.SEGMENT_SILU_MUL_PAIR) == 0
            ref.matvec_segments([(gate, want), (up, want)], x, nq.SEGMENT_SILU_MUL_PAIR)
            ref.sync()
            assert torch.equal(got, want)
            # plain segments (q/k/v shape) need no scratch at all
            outs = [torch.full((r,), np.nan, device="cuda") for r in (rows // 4, 1024)]
            mats = [nq.Matrix(12, r, columns, to_gpu(nq.quantize(12, gaussian(84 + r, (r, columns), 0.02))))
                    for r in (rows // 4, 1024)]
            refs = [torch.empty_like(o) for o in outs]
            assert call(L.nuq_matvec_segments_noalloc, ctx, list(zip(mats, outs)), x, nq.SEGMENT_PLAIN) == 0
            ref.matvec_segments(list(zip(mats, refs)), x, nq.SEGMENT_PLAIN)
            ref.sync()
            for o, r_ in zip(outs, refs):
                assert torch.equal(o, r_)
        assert L.nuq_workspace_bytes(ctx) == 0
        # beyond the scratch: refused, output untouched
        rows, small = nq.backend.NOALLOC_MAX_PAIR_ROWS + 16, 256
        wbig = torch.zeros(rows * 144, dtype=torch.uint8, device="cuda")
        big = nq.Matrix(12, rows, small, wbig)
        out = torch.full((rows,), 7.0, device="cuda")
        xs = to_gpu(np.ones(small, np.float32))
        rc = call(L.nuq_matvec_segments_noalloc, ctx, [(big, out), (big, out)], xs, nq.SEGMENT_SILU_MUL_PAIR)
        assert rc == nq.InvalidShape.code
        assert b"allocation-free scratch" in L.nuq_last_error(ctx)
        assert bool((out == 7.0).all())
        assert L.nuq_workspace_bytes(ctx) == 0
    finally:
        L.nuq_destroy(ctx)
        ref.close()


def test_noalloc_segments_under_graph_capture():
    """The allocation-free entry point captured in a HIP graph on a fresh
    context (no workspace, none allocated): every replay, with eager work
    and synchronizations between replays, equals the eager result."""
    import torch
    L = nq.lib()
    err = ctypes.create_string_buffer(256)
    ctx = L.nuq_create(0, err, len(err))
    try:
        rows, columns = 8192, 5120
        x = to_gpu(gaussian(85, columns))
        gate = nq.Matrix(12, rows, columns, to_gpu(nq.quantize(12, gaussian(86, (rows, columns), 0.02))))
        up = nq.Matrix(12, rows, columns, to_gpu(nq.quantize(12, gaussian(87, (rows, columns), 0.02))))
        eager = torch.full((rows,), np.nan, device="cuda")
        assert call(L.nuq_matvec_segments_noalloc, ctx, [(gate, eager), (up, eager)], x,
                    nq.SEGMENT_SILU_MUL_PAIR) == 0
        out = torch.full((rows,), np.nan, device="cuda")
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        arr = segs([(gate, out), (up, out)])
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            assert L.nuq_set_stream(ctx, stream.cuda_stream) == 0
            with torch.cuda.graph(graph, stream=stream):
                assert L.nuq_matvec_segments_noalloc(ctx, arr, 2, x.data_ptr(), nq.SEGMENT_SILU_MUL_PAIR) == 0
        for _ in range(4):
            out.fill_(np.nan)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager)
            scratch_user = torch.full((rows,), 3.0, device="cuda")  # eager work between replays
            assert call(L.nuq_matvec_segments_noalloc, ctx, [(gate, scratch_user), (up, scratch_user)], x,
                        nq.SEGMENT_SILU_MUL_PAIR) == 0
            assert torch.equal(scratch_user, eager)
        assert L.nuq_workspace_bytes(ctx) == 0
    finally:
        L.nuq_destroy(ctx)
