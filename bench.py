"""Benchmark of the quantized-weight matmul path on one MI355X.

Headline: Q4_K GEMV GB/s (% of HBM peak) at 5120 -> 17408,
M=1 (configs[1], gate/up shape), plus the prefill GEMM TFLOP/s at M=4096.

A "step" is one Q4_K GEMV over one weight copy: y = W x, W 17408 x 5120 Q4_K
(50,135,040 B), x F32 5120. Inputs are resident in HBM. The timed region
replays a HIP graph of back-to-back GEMVs that rotate over enough distinct
weight copies (>= 512 MB) that every call streams from HBM and not from the
256 MB Infinity Cache. `value` = weight bytes per step x steps / wall time;
the roofline uses the algorithmic bytes (weights + x + y) over the average
launch duration measured with HIP events on the launch stream.

cpu_baseline: the CPU oracle's matvec (the C restatement of nuclis's
cpu.matvec; the Zig reference cannot be built here) on the same matrix, timed
on this host with min(64, cores) threads for ~10 s.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--extras]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
F16_PEAK_TFLOPS = 2500.0     # MI355X dense f16 MFMA, TFLOP/s
MALL_BYTES = 256 << 20


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=2000)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--extras", action="store_true", help="also time the other configs (verify, layer, Q6_K)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--only", default="", help="comma list: gemv,prefill")
    p.add_argument("--profile-copy", action="store_true",
                   help="also run one plain 256 MiB device copy (the calibration kernel for rocprofv3 byte counters)")
    return p.parse_args()


class Timer:
    """HIP events on the stream the kernels are launched on."""

    def __init__(self, torch, stream):
        self.torch, self.stream = torch, stream
        self.start = torch.cuda.Event(enable_timing=True)
        self.end = torch.cuda.Event(enable_timing=True)

    def __enter__(self):
        self.start.record(self.stream)
        return self

    def __exit__(self, *exc):
        self.end.record(self.stream)
        self.end.synchronize()
        self.ms = self.start.elapsed_time(self.end)


def bench_upload(torch, nq, backend, total_bytes=1 << 30, reps=3):
    """GGUF file -> device: a file of Q4_K 17408x5120 matrices (about 1 GiB)
    written to a temporary directory (in the page cache), mapped and parsed
    by libnuq, then its data section uploaded (nuq_gguf_upload). Reported
    beside a plain torch copy of the same mapped bytes (pageable host
    memory). Host-to-device over PCIe: never the headline value."""
    import tempfile
    from pathlib import Path

    from nuclis_amd import gguf
    from nuclis_amd.synth import write_gguf as write_model
    w = nq.quantize(nq.Q4_K, np.full((1, 5120), 0.01, np.float32))
    mat = np.tile(w.reshape(-1), 17408)
    count = max(1, total_bytes // mat.nbytes)
    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "upload.gguf"
        write_model(path, [(f"blk.{i}.ffn_gate.weight", (5120, 17408), 12, mat) for i in range(count)])
        with gguf.open(path) as doc:
            times = []
            for _ in range(reps):
                t0 = time.perf_counter()
                dw = gguf.upload(backend, doc)
                times.append(time.perf_counter() - t0)
                del dw
            mapped = np.memmap(path, dtype=np.uint8, mode="r")[doc.data_offset:]
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            ref = torch.from_numpy(np.asarray(mapped)).cuda()
            torch.cuda.synchronize()
            plain = time.perf_counter() - t0
            nbytes = doc.data_bytes
            del ref, mapped
    best = min(times)
    return {"bytes": nbytes, "tensors": count, "seconds": [round(t, 4) for t in times],
            "gbs_best": nbytes / best / 1e9, "torch_pageable_copy_gbs": nbytes / plain / 1e9}


def bench_sampling(torch, nq, backend, stream, vocab=151936, reps=200):
    """Device sampling at the config-3 vocabulary: the partial top-k (k=256,
    sort passes + exp-sum) and the history penalties, each graph-captured and
    replayed `reps` times; microseconds per call."""
    import ctypes
    from nuclis_amd.synth import gaussian
    L = nq.lib()
    logits = torch.from_numpy(gaussian(70, vocab) * 3).cuda()
    values = torch.empty(256, device="cuda")
    indices = torch.empty(256, dtype=torch.int32, device="cuda")
    sums = torch.empty(64, device="cuda")
    flags = torch.empty(64, dtype=torch.int32, device="cuda")
    words = torch.zeros((vocab + 31) // 32, dtype=torch.int32, device="cuda")
    words[::7] = 0x01010101
    bufs = nq.backend._TopKBuffers(values.data_ptr(), indices.data_ptr(), sums.data_ptr(), flags.data_ptr())
    out = {}
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        L.nuq_set_stream(backend._h, stream.cuda_stream)
        calls = {
            "topk256": lambda: L.nuq_topk(backend._h, logits.data_ptr(), vocab, 256, 0.7, ctypes.byref(bufs)),
            "penalize": lambda: L.nuq_penalize(backend._h, logits.data_ptr(), vocab, words.data_ptr(), words.numel(),
                                               1.0, 0.0),
        }
        for name, fn in calls.items():
            assert fn() == 0
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for _ in range(reps):
                    assert fn() == 0
            graph.replay()
            torch.cuda.synchronize()
            with Timer(torch, stream) as t:
                graph.replay()
            out[f"{name}_us"] = t.ms * 1e3 / reps
    out["vocab"] = vocab
    return out


def copies_for(nbytes: int) -> int:
    return max(8, -(-2 * MALL_BYTES // nbytes))


def bench_gemv(torch, nq, backend, stream, encoding, rows, columns, steps, warmup, seed=2):
    from nuclis_amd.synth import gaussian
    w = nq.quantize(encoding, gaussian(seed, (rows, columns), 0.02))
    x = torch.from_numpy(gaussian(1, columns)).cuda()
    ncopies = copies_for(w.nbytes)
    base = torch.from_numpy(w).cuda()
    mats = [nq.Matrix(encoding, rows, columns, base if i == 0 else base.clone()) for i in range(ncopies)]
    ys = [torch.empty(rows, device="cuda") for _ in range(ncopies)]
    stream.wait_stream(torch.cuda.current_stream())  # inputs were made on the default stream
    with torch.cuda.stream(stream):
        for i in range(ncopies):
            backend.matvec(mats[i], x, ys[i])
        eager = [y.clone() for y in ys]
        # one graph = one pass over every copy
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(ncopies):
                backend.matvec(mats[i], x, ys[i])
        reps = max(1, steps // ncopies)
        wreps = max(1, warmup // ncopies)
        for _ in range(wreps):
            graph.replay()
        torch.cuda.synchronize()
        for i in range(ncopies):  # every replay must equal the eager result
            assert torch.equal(ys[i], eager[i]), "graph replay differs from eager GEMV"
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with Timer(torch, stream) as t:
            for _ in range(reps):
                graph.replay()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    launches = reps * ncopies
    weight_bytes = w.nbytes
    algo_bytes = weight_bytes + columns * 4 + rows * 4
    kernel_s = t.ms / 1e3 / launches
    return {
        "launches": launches, "copies": ncopies, "wall_s": wall, "event_ms": t.ms,
        "weight_bytes": weight_bytes, "algo_bytes": algo_bytes,
        "us_per_launch": kernel_s * 1e6,
        "weight_gbs": weight_bytes / kernel_s / 1e9,
        "algo_gbs": algo_bytes / kernel_s / 1e9,
        "wall_weight_gbs": weight_bytes * launches / wall / 1e9,
        "w": w, "x": x, "y0": eager[0],
    }


def bench_gemm(torch, nq, backend, stream, encoding, rows, columns, tokens, reps=20, warmup=3, seed=2,
               kernel=None):
    from nuclis_amd.synth import gaussian
    w = nq.quantize(encoding, gaussian(seed, (rows, columns), 0.02))
    x = torch.from_numpy(gaussian(7, (tokens, columns))).cuda().to(torch.float16)
    wg = torch.from_numpy(w).cuda()
    # rotating weight copies (>= 512 MB), so every launch streams from HBM
    # and not from the 256 MB last-level cache
    mats = [nq.Matrix(encoding, rows, columns, wg if i == 0 else wg.clone()) for i in range(copies_for(w.nbytes))]
    y = torch.empty((tokens, rows), device="cuda")
    k = nq.KERNEL_TILE if kernel is None else kernel
    stream.wait_stream(torch.cuda.current_stream())  # inputs were made on the default stream
    with torch.cuda.stream(stream):
        for i in range(warmup):
            backend.matmul_kernel(k, mats[i % len(mats)], x, columns, y, rows, tokens)
        torch.cuda.synchronize()
        with Timer(torch, stream) as t:
            for i in range(reps):
                backend.matmul_kernel(k, mats[i % len(mats)], x, columns, y, rows, tokens)
    s = t.ms / 1e3 / reps
    flops = 2.0 * tokens * rows * columns
    return {"ms": s * 1e3, "tflops": flops / s / 1e12, "flops": flops, "weight_gbs": w.nbytes / s / 1e9,
            "frac_f16_peak": flops / s / 1e12 / F16_PEAK_TFLOPS}


def bench_library_gemm(torch, stream, rows, columns, tokens, reps=20, warmup=3):
    """Context for the prefill roofline: torch's f16 GEMM (hipBLASLt) on the
    same M x N x K with f16 operands already in HBM -- no dequantization and
    F16 output, so it is an upper reference for the fused kernel, not a
    product path."""
    a = torch.randn(tokens, columns, device="cuda", dtype=torch.float16)
    b = torch.randn(rows, columns, device="cuda", dtype=torch.float16)
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            c = a @ b.T
        torch.cuda.synchronize()
        with Timer(torch, stream) as t:
            for _ in range(reps):
                c = a @ b.T
    del c
    s = t.ms / 1e3 / reps
    return {"ms": s * 1e3, "tflops": 2.0 * tokens * rows * columns / s / 1e12}


def bench_layer(torch, nq, backend, stream, reps=20):
    """Configuration 3: one decode step (q/k/v, o, gate/up, down Q4_K + Q6_K
    lm_head, M=1) captured as a HIP graph; GB/s of weight bytes per step."""
    from nuclis_amd import layer as L
    from nuclis_amd.synth import gaussian
    weights = L.quantized_weights()
    dev = L.upload(weights)
    x = torch.from_numpy(gaussian(20, L.HIDDEN)).cuda()
    stream.wait_stream(torch.cuda.current_stream())  # inputs were made on the default stream
    with torch.cuda.stream(stream):
        L.step(backend, dev, x)
        eager = dev.buffers["logits"].clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            L.step(backend, dev, x)
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(dev.buffers["logits"], eager), "graph replay differs from the eager step"
        with Timer(torch, stream) as t:
            for _ in range(reps):
                graph.replay()
        token = backend.argmax(dev.buffers["logits"])
    s = t.ms / 1e3 / reps
    nbytes = L.weight_bytes(weights)
    return {"us_per_step": s * 1e6, "weight_bytes": nbytes, "weight_gbs": nbytes / s / 1e9, "token": token}


def measured_traffic(name: str):
    """HBM bytes per launch measured with rocprofv3 (FETCH_SIZE + WRITE_SIZE,
    copy-kernel calibrated) and recorded in profiles/<name>.md; None if absent."""
    path = ROOT / "profiles" / f"{name}.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1])
    return None


def cpu_baseline(w, x_host, rows, columns, seconds):
    from oracle import oracle as orc
    threads = orc.default_threads()
    times = []
    t_end = time.perf_counter() + seconds
    while True:
        t0 = time.perf_counter()
        y = orc.matvec(12, rows, columns, w, x_host, threads=threads)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end and len(times) >= 3:
            break
    med = float(np.median(times))
    return {"value": round(w.nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{len(times)} full Q4_K 17408x5120 matvecs (oracle cpu.matvec restatement, F64 accumulate), "
                      f"median {med * 1e3:.1f} ms each; host has {os.cpu_count()} logical CPUs",
            "y": y}


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only; sharding across GPUs "
                                   "(each GPU holding whole weight rows) is not built", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    import nuclis_amd as nq
    torch.cuda.init()
    backend = nq.Backend(0)
    stream = torch.cuda.Stream()
    only = set(filter(None, args.only.split(",")))
    if args.profile_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    rows, columns = 17408, 5120
    out = {}
    g = bench_gemv(torch, nq, backend, stream, nq.Q4_K, rows, columns, args.steps, args.warmup)
    # correctness of the timed kernel against the oracle on a row sample
    from oracle import oracle as orc
    x_host = g["x"].cpu().numpy()
    sample = np.arange(0, rows, 97)
    ref = orc.matvec(12, sample.size, columns, np.ascontiguousarray(g["w"][sample]), x_host)
    got = g["y0"].cpu().numpy()[sample]
    normwise = float(np.abs(got - ref).max() / np.abs(ref).max())
    assert normwise <= 2e-3, normwise
    prefill = None
    if not only or "prefill" in only:
        prefill = bench_gemm(torch, nq, backend, stream, nq.Q4_K, 17408, 5120, 4096)
        prefill["library"] = bench_library_gemm(torch, stream, 17408, 5120, 4096)
    extras = {}
    if args.extras:
        extras["q4k_down_gemv"] = {k: v for k, v in bench_gemv(torch, nq, backend, stream, nq.Q4_K, 5120, 17408,
                                                                 args.steps, args.warmup).items()
                                   if k not in ("w", "x", "y0")}
        extras["q6k_lmhead_gemv"] = {k: v for k, v in bench_gemv(torch, nq, backend, stream, nq.Q6_K, 151936, 5120,
                                                                   64, 8).items() if k not in ("w", "x", "y0")}
        extras["decode_layer_step"] = bench_layer(torch, nq, backend, stream)
        extras["gguf_upload"] = bench_upload(torch, nq, backend)
        extras["sampling"] = bench_sampling(torch, nq, backend, stream)
        extras["q8_0_gemv"] = {k: v for k, v in bench_gemv(torch, nq, backend, stream, nq.Q8_0, 4096, 4096,
                                                             args.steps, args.warmup).items()
                               if k not in ("w", "x", "y0")}
        for name, enc in (("q5k", nq.Q5_K), ("iq4xs", nq.IQ4_XS)):
            extras[f"{name}_gate_gemv"] = {k: v for k, v in bench_gemv(torch, nq, backend, stream, enc, 17408, 5120,
                                                                       args.steps, args.warmup).items()
                                           if k not in ("w", "x", "y0")}
        if not only or "prefill" in only:
            extras["prefill_q6k_down_m4096"] = bench_gemm(torch, nq, backend, stream, nq.Q6_K, 5120, 17408, 4096)
            extras["prefill_q4k_gate_m512"] = bench_gemm(torch, nq, backend, stream, nq.Q4_K, 17408, 5120, 512)
            extras["prefill_q5k_gate_m4096"] = bench_gemm(torch, nq, backend, stream, nq.Q5_K, 17408, 5120, 4096)
            extras["prefill_iq4xs_gate_m4096"] = bench_gemm(torch, nq, backend, stream, nq.IQ4_XS, 17408, 5120, 4096)
            for kname, kid in (("rows", nq.KERNEL_ROWS), ("tile", nq.KERNEL_TILE)):
                extras[f"verify_m8_q4k_gate_{kname}"] = bench_gemm(torch, nq, backend, stream, nq.Q4_K, 17408, 5120,
                                                                   8, reps=200, warmup=20, kernel=kid)
            extras["verify_m8_q4k_down_tile"] = bench_gemm(torch, nq, backend, stream, nq.Q4_K, 5120, 17408, 8,
                                                           reps=200, warmup=20)
            extras["verify_m8_q5k_gate_tile"] = bench_gemm(torch, nq, backend, stream, nq.Q5_K, 17408, 5120, 8,
                                                           reps=200, warmup=20)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(g["w"], x_host, rows, columns, args.cpu_seconds)
        cpu.pop("y")
    kernel_s = g["us_per_launch"] / 1e6
    result = {
        "metric": "Q4_K GEMV GB/s (% of HBM peak) @5120x17408 M=1; prefill GEMM TFLOPS @M=4096",
        "value": round(g["wall_weight_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": g["launches"],
        "warmup": args.warmup,
        "ms_per_step": round(g["wall_s"] * 1e3 / g["launches"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k x f32 -> f32 (fp32 accumulate)",
        "data": "synthetic: W ~ N(0,0.02) seed 2 quantized to Q4_K by libnuq, x ~ N(0,1) seed 1",
        "config": {"workload": "configs[1]: Q4_K batch-1 GEMV gate/up 5120->17408 (N=17408, K=5120), "
                               f"{g['copies']} rotating weight copies",
                   "weight_bytes": g["weight_bytes"], "hbm_peak_frac": round(g["wall_weight_gbs"] / HBM_PEAK_GBS, 4),
                   "parity_normwise": normwise},
        "roofline": {"bound": "hbm", "achieved": round(g["algo_bytes"] / kernel_s / 1e9, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(g["algo_bytes"] / kernel_s / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("gemv_q4k_17408x5120_traffic"), "kernel": "gemv_dma_kernel<12, 4, 2>",
                     "us_per_launch": round(g["us_per_launch"], 3), "algo_bytes_per_launch": g["algo_bytes"]},
        "cpu_baseline": cpu,
    }
    if prefill is not None:
        result["prefill"] = {"workload": "configs[4]: Q4_K 17408x5120, M=4096, f16 activations",
                             "tflops": round(prefill["tflops"], 2), "ms": round(prefill["ms"], 4),
                             "roofline": {"bound": "mfma", "achieved": round(prefill["tflops"], 2),
                                          "peak": F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                          "frac": round(prefill["frac_f16_peak"], 4)},
                             "library_f16_gemm_same_shape_tflops": round(prefill["library"]["tflops"], 2)}
    if extras:
        result["extras"] = extras
    backend.close()
    print(json.dumps(result, default=float))


if __name__ == "__main__":
    main()
