"""Benchmark of the quantized-weight matmul path on one MI355X.

Headline: Q4_K GEMV GB/s (% of HBM peak) at 5120 -> 17408,
M=1 (configs[1], gate/up shape), plus the prefill GEMM TFLOP/s at M=4096.

A "step" is one Q4_K GEMV over one weight copy: y = W x, W 17408 x 5120 Q4_K
(50,135,040 B), x F32 5120. Inputs are resident in HBM. The timed region is
one replay of a HIP graph of exactly --steps back-to-back GEMVs that rotate
over enough distinct weight copies (>= 512 MB) that every call streams from
HBM and not from the 256 MB Infinity Cache, after --warmup launches of the
same rotation and a lead of at least 100 more: the lead still runs while the
region's start event and graph are queued behind it, so the region holds no
host submission latency. `value` = weight bytes x steps / the region's
duration, from HIP events on the launch stream; the roofline uses the algorithmic bytes
(weights + x + y) per launch over the same average launch duration.

Every other configuration runs by default with its own fixed repetition
count (configs[0], the configs[1] down shape, the configs[2] layer step
with its greedy token, configs[3] M=8 verify on both kernels, the F32
multi-token GEMV at 2, 3 and 8 token rows, configs[4] prefill at M=512 and
M=4096 on both matrices), each output checked against the CPU oracle (a row
or token sample) before it is reported.

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
GEMV_KERNEL = "gemv_dma_kernel<12, 4, 2, false, false>"
GEMV_DTYPE = ("q4_k codes x f32 activations as fixed point relative to each 32-value slice's maximum "
              "(power-of-two slice scale, 23 significant bits, three int8 byte planes into an exact int32 dot) "
              "-> f32 scale/accumulate")


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=2000)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--extras", action="store_true",
                   help="also time the lm_head GEMV, Q5_K / IQ4_XS, GGUF upload and sampling")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--only", default="",
                   help="comma list of: configs, prefill, gemv (the headline GEMV always runs; gemv alone runs only it)")
    p.add_argument("--case", default="",
                   help="profiling aid: only time one matmul, ENC:ROWS:COLUMNS:TOKENS (f16 activations), e.g. 14:5120:17408:4096")
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


def bench_gemv(torch, nq, backend, stream, encoding, rows, columns, steps, warmup, w_seed, x_seed=1):
    """`steps` decode GEMVs timed as one replay of a HIP graph of exactly
    `steps` launches, rotating over `copies` distinct weight copies (>= 512
    MB) so each launch streams from HBM rather than the 256 MB Infinity
    Cache; `warmup` launches of the same rotation replay untimed first. The
    timed region is bracketed by synchronizations and HIP events on the
    launch stream."""
    from nuclis_amd.synth import gaussian
    steps, warmup = max(1, steps), max(0, warmup)
    w = nq.quantize(encoding, gaussian(w_seed, (rows, columns), 0.02))
    x = torch.from_numpy(gaussian(x_seed, columns)).cuda()
    ncopies = copies_for(w.nbytes)
    base = torch.from_numpy(w).cuda()
    mats = [nq.Matrix(encoding, rows, columns, base if i == 0 else base.clone()) for i in range(ncopies)]
    ys = [torch.empty(rows, device="cuda") for _ in range(ncopies)]
    stream.wait_stream(torch.cuda.current_stream())  # inputs were made on the default stream
    with torch.cuda.stream(stream):
        for i in range(ncopies):
            backend.matvec(mats[i], x, ys[i])
        eager = [y.clone() for y in ys]

        def capture(n):
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for i in range(n):
                    backend.matvec(mats[i % ncopies], x, ys[i % ncopies])
            return graph
        timed = capture(steps)
        # The GPU's clocks settle over the first few hundred microseconds of
        # load: at least 200 launches in all replay untimed before the timed
        # region (the `warmup` requested, plus a lead reported apart). The
        # lead's replay is not waited for: the start event and the timed
        # graph are queued behind it while it runs, so the region starts on
        # a busy GPU and holds no host submission latency.
        lead = max(100, 200 - warmup)
        if warmup:
            capture(warmup).replay()
        lead_graph = capture(lead)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        lead_graph.replay()
        with Timer(torch, stream) as t:
            timed.replay()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        for i in range(min(steps, ncopies)):  # every replay must equal the eager result
            assert torch.equal(ys[i], eager[i]), "graph replay differs from the eager GEMV"
    weight_bytes = w.nbytes
    algo_bytes = weight_bytes + columns * 4 + rows * 4
    kernel_s = t.ms / 1e3 / steps
    return {
        "launches": steps, "warmup_launches": warmup, "lead_launches": lead, "copies": ncopies, "wall_s": wall, "event_ms": t.ms,
        "weight_bytes": weight_bytes, "algo_bytes": algo_bytes,
        "us_per_launch": kernel_s * 1e6,
        "weight_gbs": weight_bytes / kernel_s / 1e9,
        "algo_gbs": algo_bytes / kernel_s / 1e9,
        "wall_weight_gbs": weight_bytes * (steps + lead) / wall / 1e9,  # host clock over lead + region
        "w": w, "x": x, "y0": eager[0],
    }


def public(d):
    return {k: v for k, v in d.items() if k not in ("w", "x", "y0", "out", "xh")}


def check_gemv(orc, g, encoding, rows, columns, stride_rows=97):
    """The timed GEMV's output against the oracle on every stride_rows-th row:
    the F32 bound |d| <= 4e-6 * sum|w*x| + 1e-6 (metal-check.zig:3976)."""
    x_host = g["x"].cpu().numpy()
    sample = np.arange(0, rows, stride_rows)
    w = np.ascontiguousarray(g["w"][sample])
    ref = orc.matvec(encoding, sample.size, columns, w, x_host).astype(np.float64)
    got = g["y0"].cpu().numpy()[sample].astype(np.float64)
    dec = np.abs(orc.decode_matrix(encoding, w, sample.size, columns).astype(np.float64))
    m = dec @ np.abs(x_host.astype(np.float64))
    bound = 4e-6 * m + 1e-6
    err = np.abs(got - ref)
    assert np.all(err <= bound), f"GEMV enc {encoding} {rows}x{columns} outside the bound"
    return {"rows_checked": int(sample.size), "normwise": float(err.max() / np.abs(ref).max()),
            "worst_err_over_mass": float((err / m).max())}


MATVEC_ROWS = "matvec_rows"  # bench_gemm's `kernel` for nuq_matvec_rows (F32 activations)


def bench_gemm(torch, nq, backend, stream, encoding, rows, columns, tokens, reps=20, warmup=3, w_seed=2,
               x_seed=5, kernel=None, check=None, x_f16=True):
    """`reps` launches of the matmul entry point (one kernel route) on
    rotating weight copies (>= 512 MB), f16 activations; HIP events on the
    launch stream. `check` = (orc, token sample): the timed output is
    compared with the oracle on every row of those tokens."""
    from nuclis_amd.synth import gaussian
    w = nq.quantize(encoding, gaussian(w_seed, (rows, columns), 0.02))
    xh = gaussian(x_seed, (tokens, columns)).astype(np.float16 if x_f16 else np.float32)
    x = torch.from_numpy(xh).cuda()
    wg = torch.from_numpy(w).cuda()
    mats = [nq.Matrix(encoding, rows, columns, wg if i == 0 else wg.clone()) for i in range(copies_for(w.nbytes))]
    y = torch.full((tokens, rows), float("nan"), device="cuda")
    k = nq.KERNEL_AUTO if kernel is None else kernel

    def call(m):
        if k == MATVEC_ROWS:
            backend.matvec_rows(m, x, columns, y, rows, tokens)
        else:
            backend.matmul_kernel(k, m, x, columns, y, rows, tokens)

    stream.wait_stream(torch.cuda.current_stream())  # inputs were made on the default stream
    with torch.cuda.stream(stream):
        call(mats[0])
        torch.cuda.synchronize()
        # the warm-up launches are not waited for: the timed ones queue behind them
        for i in range(warmup):
            call(mats[i % len(mats)])
        with Timer(torch, stream) as t:
            for i in range(reps):
                call(mats[i % len(mats)])
        torch.cuda.synchronize()
    s = t.ms / 1e3 / reps
    flops = 2.0 * tokens * rows * columns
    out = {"ms": s * 1e3, "tflops": flops / s / 1e12, "flops": flops, "weight_gbs": w.nbytes / s / 1e9,
           "frac_f16_peak": flops / s / 1e12 / F16_PEAK_TFLOPS, "reps": reps}
    if check is not None:
        orc, sel, kbound = check
        got = y.cpu().numpy()[sel].astype(np.float64)
        xr = xh[sel].astype(np.float32)
        ref = orc.matmul(encoding, rows, columns, w, xr).astype(np.float64)
        dec = np.abs(orc.decode_matrix(encoding, w, rows, columns).astype(np.float64))
        m = np.abs(xr.astype(np.float64)) @ dec.T
        err = np.abs(got - ref)
        assert np.all(err <= kbound * m + 1e-6), f"matmul enc {encoding} {rows}x{columns} M={tokens} outside the bound"
        out["check"] = {"tokens_checked": int(len(sel)), "rows_checked": rows, "bound": f"{kbound:g}*sum|w*x|+1e-6",
                        "worst_err_over_mass": float((err / m).max()),
                        "normwise": float(err.max() / np.abs(ref).max())}
    return out


def token_sample(tokens):
    """First and last token of every 256-token tile (every output tile)."""
    t = sorted({s for start in range(0, tokens, 256) for s in (start, min(start + 255, tokens - 1))})
    return np.array(t)


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


def bench_layer(torch, nq, backend, stream, reps=20, check=None):
    """Configuration 3: one decode step (q/k/v, o, gate/up, down Q4_K + Q6_K
    lm_head, M=1) captured as a HIP graph; GB/s of weight bytes per step.
    `check` = the oracle module: the greedy token must equal the CPU
    composition's."""
    from nuclis_amd import layer as L
    from nuclis_amd.synth import gaussian
    weights = L.quantized_weights()
    dev = L.upload(weights)
    xh = gaussian(20, L.HIDDEN)
    x = torch.from_numpy(xh).cuda()
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
        for _ in range(5):  # lead replays, not waited for: the timed ones queue behind them
            graph.replay()
        with Timer(torch, stream) as t:
            for _ in range(reps):
                graph.replay()
        token = backend.argmax(dev.buffers["logits"])
    s = t.ms / 1e3 / reps
    nbytes = L.weight_bytes(weights)
    out = {"us_per_step": s * 1e6, "weight_bytes": nbytes, "weight_gbs": nbytes / s / 1e9, "token": token,
           "reps": reps}
    if check is not None:
        from oracle import layer_oracle
        ref = layer_oracle.cpu_step(L.SHAPES, weights, xh)
        want = check.argmax(ref)
        assert token == want, f"layer step greedy token {token} != oracle {want}"
        out["oracle_token"] = want
    del dev
    return out


TRAFFIC_PROFILE = "gemv_q4k_17408x5120_traffic"


def measured_traffic(name: str):
    """HBM bytes per launch from a rocprofv3 --pmc run (FETCH_SIZE +
    WRITE_SIZE, copy-kernel calibrated) recorded in profiles/<name>.md; None
    if absent. Counters cannot be read inside this process, so this figure is
    the profiled run's, not this run's."""
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
    from nuclis_amd.synth import CONFIGS
    from oracle import oracle as orc
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

    def want(name):
        return not only or name in only

    if args.case:
        e, r, c, t = (int(v) for v in args.case.split(":"))
        d = bench_gemm(torch, nq, backend, stream, e, r, c, t, reps=10, warmup=2)
        print(json.dumps({"case": args.case, "ms": d["ms"], "tflops": d["tflops"]}))
        backend.close()
        return

    # headline: configs[1] gate/up GEMV, exactly --steps launches timed
    enc, rows, columns, seed = CONFIGS["c2_gate"]
    g = bench_gemv(torch, nq, backend, stream, enc, rows, columns, args.steps, args.warmup, seed)
    gcheck = check_gemv(orc, g, enc, rows, columns)
    configs = {}
    fixed = 200  # launches per secondary GEMV line, whatever --steps is
    if want("configs"):
        for key, name in (("configs[0] q8_0 4096x4096", "c1_q8_0"), ("configs[1] q4_k down 5120x17408", "c2_down")):
            e, r, c, sd = CONFIGS[name]
            d = bench_gemv(torch, nq, backend, stream, e, r, c, fixed, 50, sd)
            d["check"] = check_gemv(orc, d, e, r, c)
            d["roofline_frac"] = d["algo_gbs"] / HBM_PEAK_GBS
            configs[key] = public(d)
        configs["configs[2] layer step + q6_k lm_head"] = bench_layer(torch, nq, backend, stream, check=orc)
        e, r, c, sd = CONFIGS["c2_gate"]
        e2, r2, c2, sd2 = CONFIGS["c2_down"]
        # the register-dequant multi-row GEMV (KERNEL_ROWS, F32 arithmetic)
        # against the MFMA tile, both on f16 activations
        for kname, kid in (("rows", nq.KERNEL_ROWS), ("tile", nq.KERNEL_TILE)):
            for label, (ee, rr, cc, ss) in (("gate 17408x5120", (e, r, c, sd)), ("down 5120x17408", (e2, r2, c2, sd2))):
                d = bench_gemm(torch, nq, backend, stream, ee, rr, cc, 8, reps=100 if kname == "rows" else 200,
                               warmup=20, w_seed=ss, x_seed=4, kernel=kid,
                               check=(orc, np.arange(8), 4e-6 if kname == "rows" else 2e-4))
                d["algo_gbs"] = (rr * cc // 256 * 144 + 8 * cc * 2 + 8 * rr * 4) / d["ms"] / 1e6
                configs[f"configs[3] verify M=8 q4_k {label} {kname}"] = d
        # the routed multi-token GEMV (T = 2, 3 F32 token rows, matvecRows)
        for tokens in (2, 3):
            d = bench_gemm(torch, nq, backend, stream, e, r, c, tokens, reps=200, warmup=20, w_seed=sd, x_seed=4,
                           kernel=nq.KERNEL_AUTO, x_f16=False, check=(orc, np.arange(tokens), 4e-6))
            d["ratio_to_m1"] = d["ms"] * 1e3 / g["us_per_launch"]
            configs[f"multi-token T={tokens} f32 q4_k gate 17408x5120 (auto route)"] = d
        # matvecRows at its largest token count (F32, two passes of 4 tokens)
        d = bench_gemm(torch, nq, backend, stream, e, r, c, 8, reps=100, warmup=10, w_seed=sd, x_seed=4,
                       kernel=MATVEC_ROWS, x_f16=False, check=(orc, np.arange(8), 4e-6))
        d["ratio_to_m1"] = d["ms"] * 1e3 / g["us_per_launch"]
        configs["multi-token T=8 f32 q4_k gate 17408x5120 (matvecRows)"] = d
    prefill = None
    if want("prefill"):
        e, r, c, sd = CONFIGS["c5_gate"]
        prefill = bench_gemm(torch, nq, backend, stream, e, r, c, 4096, w_seed=sd,
                             check=(orc, token_sample(4096), 2e-4))
        prefill["library"] = bench_library_gemm(torch, stream, r, c, 4096)
        if want("configs"):
            for label, name, tokens in (("q4_k gate 17408x5120 M=512", "c5_gate", 512),
                                        ("q6_k down 5120x17408 M=4096", "c5_down", 4096),
                                        ("q6_k down 5120x17408 M=512", "c5_down", 512)):
                e, r, c, sd = CONFIGS[name]
                configs[f"configs[4] prefill {label}"] = bench_gemm(torch, nq, backend, stream, e, r, c, tokens,
                                                                    w_seed=sd, check=(orc, token_sample(tokens), 2e-4))
    extras = {}
    if args.extras:
        extras["q6k_lmhead_gemv"] = public(bench_gemv(torch, nq, backend, stream, nq.Q6_K, 151936, 5120, 64, 8, 17))
        extras["gguf_upload"] = bench_upload(torch, nq, backend)
        extras["sampling"] = bench_sampling(torch, nq, backend, stream)
        for name, enc in (("q5k", nq.Q5_K), ("iq4xs", nq.IQ4_XS)):
            extras[f"{name}_gate_gemv"] = public(bench_gemv(torch, nq, backend, stream, enc, 17408, 5120, fixed, 50, 2))
        if want("prefill"):
            extras["prefill_q5k_gate_m4096"] = bench_gemm(torch, nq, backend, stream, nq.Q5_K, 17408, 5120, 4096)
            extras["prefill_iq4xs_gate_m4096"] = bench_gemm(torch, nq, backend, stream, nq.IQ4_XS, 17408, 5120, 4096)
            extras["verify_m8_q5k_gate_tile"] = bench_gemm(torch, nq, backend, stream, nq.Q5_K, 17408, 5120, 8,
                                                           reps=200, warmup=20, x_seed=4)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(g["w"], g["x"].cpu().numpy(), rows, columns, args.cpu_seconds)
        cpu.pop("y")
    kernel_s = g["us_per_launch"] / 1e6
    value = g["weight_gbs"]
    result = {
        "metric": "Q4_K GEMV GB/s (% of HBM peak) @5120x17408 M=1; prefill GEMM TFLOPS @M=4096",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": g["launches"],
        "warmup": g["warmup_launches"],
        "ms_per_step": round(g["event_ms"] / g["launches"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": GEMV_DTYPE,
        "data": f"synthetic: W ~ N(0,0.02) seed {seed} quantized to Q4_K by libnuq, x ~ N(0,1) seed 1",
        "config": {"workload": "configs[1]: Q4_K batch-1 GEMV gate/up 5120->17408 (N=17408, K=5120), "
                               f"{g['copies']} rotating weight copies; value = weight bytes x steps / "
                               "event-timed region (one graph replay of exactly `steps` launches)",
                   "weight_bytes": g["weight_bytes"], "hbm_peak_frac": round(value / HBM_PEAK_GBS, 4),
                   "lead_launches": g["lead_launches"],
                   "wall_weight_gbs": round(g["wall_weight_gbs"], 2), "parity": gcheck},
        "roofline": {"bound": "hbm", "achieved": round(g["algo_bytes"] / kernel_s / 1e9, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(g["algo_bytes"] / kernel_s / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(TRAFFIC_PROFILE),
                     "traffic_source": f"profiles/{TRAFFIC_PROFILE}.md (rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE, "
                                       "copy-kernel calibrated; a profiled run, not this one)",
                     "kernel": GEMV_KERNEL,
                     "us_per_launch": round(g["us_per_launch"], 3), "algo_bytes_per_launch": g["algo_bytes"]},
        "cpu_baseline": cpu,
    }
    if prefill is not None:
        result["prefill"] = {"workload": "configs[4]: Q4_K 17408x5120, M=4096, f16 activations",
                             "tflops": round(prefill["tflops"], 2), "ms": round(prefill["ms"], 4),
                             "roofline": {"bound": "mfma", "achieved": round(prefill["tflops"], 2),
                                          "peak": F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                          "frac": round(prefill["frac_f16_peak"], 4)},
                             "check": prefill.get("check"),
                             "library_f16_gemm_same_shape_tflops": round(prefill["library"]["tflops"], 2)}
    if configs:
        result["configs"] = configs
    if extras:
        result["extras"] = extras
    backend.close()
    print(json.dumps(result, default=float))


if __name__ == "__main__":
    main()
