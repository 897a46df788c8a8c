#!/usr/bin/env python3
"""Benchmark of the dequant-GEMV hot path on one MI355X.

Workload (one "step"): the INT4 group-64 one-row product y = x . deq(W) on the
Llama-3-8B gate/up projection shape, K = 4096 -> N = 14336, with x ~ N(0,1) fp32 and
W ~ N(0, 0.02) quantized on the device by kt_quantize (the reference layout: qdata
[K x N/2], fp32 scales and u8 zeros [K/64 x N]) plus the column-run copy that the
one-row kernel streams (kt_qweight_pack). Inputs are resident in HBM before timing.
The weight is cloned until one pass over the copies streams more than twice the 256 MB
Infinity Cache; `--steps` launches rotating over the copies are recorded in one HIP
graph and replayed once between synchronizations (HIP events on the launch stream),
after `--warmup` launches recorded and replayed the same way.

value = algorithmic bytes of a step / measured step time (GB/s). Algorithmic bytes
per product = K*bytesPerRow + 4*groups*N + groups*N (zeros) + 4*K (x) + 4*N (y).

The JSON line also carries:
  roofline      -- the headline kernel itself against 8 TB/s; traffic (HBM bytes per
                   launch) from rocprofv3 PMC runs recorded under profiles/;
  cpu_baseline  -- the oracle (C restatement of MatMul.multiplyQuantized, M == 1
                   unit schedule, work-stealing threads) on the same product on this
                   host: faithful and FMA-contracted builds, all threads and one, the
                   median of 5 samples after 3 warm-up calls;
  extra         -- the rest of the workload family: C2, the Qwen2-0.5B layer step
                   (grouped launches, and the decoder's one chained launch with the
                   norms, SwiGLU and residual adds fused) and each projection alone at
                   g64 and g32; C1, the
                   INT8 2048 x 2048 GEMV at g64 and g32; C5's g32 rows at M = 1; the
                   INT8 group-32 prefill GEMM at M = 512 on the 2048-wide layer's four
                   shapes and their sum, each beside the vendor library's plain bf16
                   GEMM (torch.matmul -> hipBLASLt, no dequantization) timed the same
                   way; the M sweep (1, 16, 128, 512, 2048) of the INT8 2048 -> 8192
                   product; the Llama-3-8B projection shapes (4096->4096, 4096->1024,
                   4096->14336, 14336->4096), INT4 and INT8 g64 at M = 1, 8, 64, 512;
                   kt_quantize on 4096 x 14336; and the Llama-style 1B INT4 decoder end
                   to end (1024-token prefill, greedy decode steps). Every timed graph
                   reads each of its weight copies (> 2x MALL).

--only dominant | copy | quantize | gemm | decode runs just the headline product (or a
256 MB device copy, the calibration of the HBM byte counters, or kt_quantize INT4 and
INT8 g64 on 4096 x 14336, or the INT8 g32 M = 512 GEMM on 2048 -> 8192, or the 1B
decoder's prefill and decode steps) for rocprofv3 runs.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "dequant-GEMV GB/s (% HBM peak) at M=1; dequant-GEMM TFLOP/s at M=512"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16/bf16
MALL_BYTES = 256 << 20

# the headline: K, N, bits, group size of the Llama-3-8B gate/up projection
HEADLINE = (4096, 14336, 4, 64)
QWEN = [("q", 896, 896), ("k", 896, 128), ("v", 896, 128), ("o", 896, 896), ("gate", 896, 4864),
        ("up", 896, 4864), ("down", 4864, 896), ("lm_head", 896, 151936)]


def layout(k, n, bits, g):
    groups = (k + g - 1) // g
    bpr = (n + n % 2) // 2 if bits == 4 else n
    return groups, bpr


def gemv_bytes(m, k, n, bits, g):
    groups, bpr = layout(k, n, bits, g)
    return k * bpr + 4 * groups * n + (groups * n if bits == 4 else 0) + 4 * m * k + 4 * m * n


class Weight:
    """One quantized weight in torch-allocated device memory, passed through the C ABI."""

    def __init__(self, torch, kt_lib, k, n, bits, g, seed, stream):
        self.k, self.n, self.bits, self.g = k, n, bits, g
        groups, bpr = layout(k, n, bits, g)
        gen = torch.Generator(device="cuda").manual_seed(seed)
        w = torch.randn((k, n), generator=gen, device="cuda", dtype=torch.float32) * 0.02
        self.q = torch.empty(k * bpr, dtype=torch.uint8, device="cuda")
        self.s = torch.empty(groups * n, dtype=torch.float32, device="cuda")
        self.z = torch.empty(groups * n, dtype=torch.uint8, device="cuda") if bits == 4 else None
        torch.cuda.synchronize()
        kt_lib.call("kt_quantize", w.data_ptr(), k, n, bits, g, self.q.data_ptr(), self.s.data_ptr(),
                    self.z.data_ptr() if self.z is not None else None, stream)
        del w
        self.p = None
        self.struct = None
        self._bind(kt_lib)

    def _bind(self, kt_lib):
        self.struct = kt_lib.QWeight(self.q.data_ptr(), self.s.data_ptr(),
                                     self.z.data_ptr() if self.z is not None else None,
                                     self.k, self.n, self.bits, self.g,
                                     self.p.data_ptr() if self.p is not None else None)

    def pack(self, torch, kt_lib, stream):
        """Adds the column-run copy (kt_qweight_pack) that the one-row kernel streams."""
        nbytes = ctypes.c_int64()
        kt_lib.call("kt_qweight_packed_bytes", self.k, self.n, self.bits, self.g, ctypes.byref(nbytes))
        self.p = torch.empty(nbytes.value, dtype=torch.uint8, device="cuda")
        self._bind(kt_lib)
        kt_lib.call("kt_qweight_pack", ctypes.byref(self.struct), self.p.data_ptr(), stream)
        return self

    def clone(self, kt_lib):
        c = object.__new__(Weight)
        c.k, c.n, c.bits, c.g = self.k, self.n, self.bits, self.g
        c.q = self.q.clone()
        c.s = self.s.clone()
        c.z = self.z.clone() if self.z is not None else None
        c.p = self.p.clone() if self.p is not None else None
        c._bind(kt_lib)
        return c

    def without_copy(self, kt_lib):
        """The same weight (shared tensors) without its column-run copy: the kernels for
        the reference layout."""
        c = object.__new__(Weight)
        c.k, c.n, c.bits, c.g = self.k, self.n, self.bits, self.g
        c.q, c.s, c.z, c.p = self.q, self.s, self.z, None
        c._bind(kt_lib)
        return c

    @property
    def nbytes(self):
        return self.q.numel() + 4 * self.s.numel() + (self.z.numel() if self.z is not None else 0)


def qmatmul(kt_lib, x, m, w, y, stream):
    kt_lib.call("kt_qmatmul", x.data_ptr(), m, ctypes.byref(w.struct), y.data_ptr(), 0, ctypes.c_float(1.0), stream)


def qmatmul_group(kt_lib, x, m, ws, ys, stream):
    """Products of one input with up to four weights in one launch (kt_qmatmul_group)."""
    n = len(ws)
    structs = (kt_lib.QWeight * n)(*[w.struct for w in ws])
    outs = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
    kt_lib.call("kt_qmatmul_group", x.data_ptr(), m, structs, n, outs, None, 0, ctypes.c_float(1.0), stream)


def time_graph_launches(torch, stream_obj, fn, copies, launches, replays=3):
    """Average duration of one launch: `launches` back-to-back launches (rotating weight
    copies) captured in one graph, HIP events on the launch stream around the replays."""
    launches = max(launches, len(copies))  # every copy is read in each replay
    gph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gph, stream=stream_obj):
        for i in range(launches):
            fn(copies[i % len(copies)])
    gph.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream_obj)
    for _ in range(replays):
        gph.replay()
    t1.record(stream_obj)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / (replays * launches)


def host_threads() -> int:
    """The cores this process may use: its affinity set, capped by OMP_NUM_THREADS when the
    host sets it (the share of a multi-GPU host's cores that belongs to one GPU)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cap = os.environ.get("OMP_NUM_THREADS", "")
    if cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(1, n)


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(seconds: float = 10.0):
    """The oracle's M == 1 product (C restatement of MatMul.multiplyQuantized, the M == 1
    unit schedule on work-stealing threads) on the headline workload, on this host.
    Four modes: faithful (-ffp-contract=off, the reference's rounding) and fast (FMA
    contraction, AVX2), each on all of the host's threads and on one; each mode is 3
    warm-up calls, then 5 samples of repeated calls, and the median sample is reported."""
    import numpy as np

    import oracle

    oracle.build()
    k, n, bits, g = HEADLINE
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((k, n), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    _, q = oracle.quantize(w, bits, g)
    del w
    x = rng.standard_normal((1, k), dtype=np.float32)
    nbytes = gemv_bytes(1, k, n, bits, g)
    threads = host_threads()
    per_sample = seconds / 20.0

    def measure(t, fast):
        for _ in range(3):
            oracle.multiply_quantized(x, q, 1, threads=t, fast=fast)
        t0 = time.perf_counter()
        oracle.multiply_quantized(x, q, 1, threads=t, fast=fast)
        reps = max(1, int(per_sample / max(time.perf_counter() - t0, 1e-6)))
        samples = []
        for _ in range(5):
            t0 = time.perf_counter()
            for _ in range(reps):
                oracle.multiply_quantized(x, q, 1, threads=t, fast=fast)
            samples.append((time.perf_counter() - t0) / reps)
        sec = sorted(samples)[2]
        return {"GB/s": round(nbytes / sec / 1e9, 3), "ms_per_call": round(sec * 1e3, 3), "calls_per_sample": reps}

    faithful = measure(threads, False)
    return {
        "value": faithful["GB/s"],
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"INT4 g64 M=1 4096x14336 ({nbytes} algorithmic bytes per call), C restatement of "
                  f"MatMul.multiplyQuantized's M=1 unit schedule built -O3 -ffp-contract=off, {threads} threads, "
                  "median of 5 samples after 3 warm-up calls",
        "cpu_model": cpu_model(),
        "host_cpus": os.cpu_count(),
        "modes": {
            f"faithful_{threads}t": faithful,
            "faithful_1t": measure(1, False),
            f"fast_{threads}t": measure(threads, True),
            "fast_1t": measure(1, True),
        },
    }


def traffic_from_profiles():
    """HBM bytes per launch of the headline kernel measured with rocprofv3 --pmc
    (profiles/), if recorded."""
    path = ROOT / "profiles" / "traffic_gemv_packed_int4_4096x14336.json"
    if path.exists():
        try:
            return json.loads(path.read_text()).get("bytes_per_launch")
        except (ValueError, OSError):
            return None
    return None


def decoder_figures(torch, stream_obj) -> dict:
    """The Llama-style 1B INT4 decoder (16 layers, d 2048, 32 q / 8 kv heads of 64,
    SwiGLU 8192, vocab 32000, RMSNorm, RoPE theta 5e5; weights ~N(0, 0.02) quantized
    g64 on the device): prefill of a 1024-token prompt (ids seed 2), then 127 greedy
    decode steps replayed from one recorded HIP graph. HIP events on the launch stream;
    the second of two runs is reported."""
    import numpy as np
    import kotensor_amd as kt
    from kotensor_amd import _lib
    ks = kt.Stream(handle=stream_obj.cuda_stream)
    model = kt.Transformer(32000, 2048, 16, 32, 8192, 8, norm_eps=1e-5, rope_theta=500000.0,
                           quantization=kt.Quantization.INT4, seed=1, stream=ks)
    prompt = np.random.default_rng(2).integers(0, 32000, 1024).tolist()
    steps = 127
    # bytes a decode step streams: every projection and the head, not the embedding
    # table (one row of it is gathered)
    streamed = model.weight_bytes - model.weights["embedding"].size_in_bytes
    out = {}
    for _ in range(2):
        cache, buffers = model.new_cache(1024 + steps + 1, ks), model.new_inference_buffers(1024 + steps + 1)
        torch.cuda.synchronize()
        e = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        e[0].record(stream_obj)
        model.prefill(prompt, cache, buffers, ks)
        e[1].record(stream_obj)
        # the first greedy token and one eager step (which sizes the workspaces), then
        # the recorded step replayed
        _lib.call("kt_argmax", buffers.logits.ptr, model.vocabulary_size, buffers.tokens.ptr, ks.handle)
        model.decode_step(cache, buffers, ks)
        graph = model.capture_decode(cache, buffers, ks)
        e[2].record(stream_obj)
        graph.replay(steps - 1)
        e[3].record(stream_obj)
        torch.cuda.synchronize()
        graph.destroy()
        prefill_ms = e[0].elapsed_time(e[1])
        decode_ms = e[2].elapsed_time(e[3]) / (steps - 1)
        out = {"prefill_tokens": 1024, "prefill_ms": round(prefill_ms, 3),
               "prefill_tok/s": round(1024 / (prefill_ms * 1e-3), 1),
               "decode_ms_per_token": round(decode_ms, 4), "decode_tok/s": round(1e3 / decode_ms, 1),
               "decode_weight_GB/s": round(streamed / (decode_ms * 1e-3) / 1e9, 1),
               "decode_weight_bytes": streamed, "decode_steps_timed": steps - 1, "graph_replay": True}
        del cache, buffers
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip the 8B GEMV and M=512 GEMM figures")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--plain", action="store_true",
                    help="with --only gemm: weights without the column-run copy (the reference-layout GEMM)")
    ap.add_argument("--only", choices=["dominant", "copy", "quantize", "gemm", "decode", "c1", "rows", "narrow"],
                    help="run one kernel for a rocprofv3 run")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    import kotensor_amd  # noqa: F401  (loads libkotensor_hip.so after torch's HIP runtime)
    from kotensor_amd import _lib as kt_lib

    torch.cuda.set_device(0)
    # A dedicated stream: every launch, event and graph capture below runs on it.
    stream_obj = torch.cuda.Stream()
    with torch.cuda.stream(stream_obj):
        if args.only:
            return run_only(args, torch, kt_lib, stream_obj)
        return run(args, torch, kt_lib, stream_obj)


def run_only(args, torch, kt_lib, stream_obj) -> int:
    """One kernel, args.steps times, for hardware-counter runs (one dispatch per launch)."""
    stream = ctypes.c_void_p(stream_obj.cuda_stream)
    if args.only == "copy":
        # calibration: 256 MiB read + 256 MiB written per launch
        src = torch.empty(64 << 20, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"only": "copy", "bytes_read": src.numel() * 4, "bytes_written": dst.numel() * 4,
                          "launches": args.steps}), flush=True)
        return 0
    if args.only == "quantize":
        # kt_quantize INT4 then INT8, g64, on 4096 x 14336, three distinct fp32 inputs in rotation
        kq, nq = 4096, 14336
        srcs = [torch.randn((kq, nq), device="cuda", dtype=torch.float32) * 0.02 for _ in range(3)]
        done = {}
        for bits in (4, 8):
            groups, bpr = layout(kq, nq, bits, 64)
            qq = torch.empty(kq * bpr, dtype=torch.uint8, device="cuda")
            sq = torch.empty(groups * nq, dtype=torch.float32, device="cuda")
            zq = torch.empty(groups * nq, dtype=torch.uint8, device="cuda") if bits == 4 else None
            torch.cuda.synchronize()
            for i in range(args.steps):
                kt_lib.call("kt_quantize", srcs[i % 3].data_ptr(), kq, nq, bits, 64, qq.data_ptr(), sq.data_ptr(),
                            zq.data_ptr() if zq is not None else None, stream)
            torch.cuda.synchronize()
            done[f"int{bits}"] = 4 * kq * nq + kq * bpr + (5 if bits == 4 else 4) * groups * nq
        print(json.dumps({"only": "quantize", "kernel": "quant4_vec, quant8_vec 4096x14336 g64",
                          "algorithmic_bytes": done, "launches_each": args.steps}), flush=True)
        return 0
    if args.only == "gemm":
        # the INT8 g32 prefill GEMM at M = 512 on 2048 -> 8192 (column-run copy), weight
        # copies in rotation
        wg = Weight(torch, kt_lib, 2048, 8192, 8, 32, seed=9, stream=stream)
        if not args.plain:
            wg.pack(torch, kt_lib, stream)
        cg = [wg] + [wg.clone(kt_lib) for _ in range(max(1, -(-2 * MALL_BYTES // (2 * wg.nbytes))) - 1)]
        xg = torch.randn((512, 2048), device="cuda", dtype=torch.float32)
        yg = torch.empty((512, 8192), device="cuda", dtype=torch.float32)
        torch.cuda.synchronize()
        for i in range(args.steps):
            qmatmul(kt_lib, xg, 512, cg[i % len(cg)], yg, stream)
        torch.cuda.synchronize()
        kernel = "gemm_kernel" if args.plain else "gemm_packed_kernel"
        print(json.dumps({"only": "gemm", "kernel": f"{kernel} int8 g32 M=512 2048x8192",
                          "flops": 2 * 512 * 2048 * 8192, "launches": args.steps}), flush=True)
        return 0
    if args.only == "decode":
        # the Llama-style 1B INT4 decoder: 1024-token prefill and 127 greedy steps, twice
        print(json.dumps({"only": "decode", **decoder_figures(torch, stream_obj)}), flush=True)
        return 0
    if args.only in ("c1", "rows", "narrow"):
        # c1: the INT8 g64 one-row product on 2048 x 2048; rows: M = 8 and narrow: M = 64 on
        # the Llama-3-8B gate/up shape, INT4 g64; packed weights in rotation
        k, n, bits, g, m = {"c1": (2048, 2048, 8, 64, 1), "rows": (4096, 14336, 4, 64, 8),
                            "narrow": (4096, 14336, 4, 64, 64)}[args.only]
        cs = weight_copies(torch, kt_lib, k, n, bits, g, 5, stream, packed=True)
        x = torch.randn((m, k), device="cuda", dtype=torch.float32)
        y = torch.empty((m, n), device="cuda", dtype=torch.float32)
        torch.cuda.synchronize()
        for i in range(args.steps):
            qmatmul(kt_lib, x, m, cs[i % len(cs)], y, stream)
        torch.cuda.synchronize()
        print(json.dumps({"only": args.only, "shape": f"{k}x{n} int{bits} g{g} M={m}",
                          "algorithmic_bytes": gemv_bytes(m, k, n, bits, g), "flops": 2 * m * k * n,
                          "launches": args.steps}), flush=True)
        return 0
    k, n, bits, g = HEADLINE
    copies = weight_copies(torch, kt_lib, k, n, bits, g, 8, stream, packed=True)
    x = torch.randn((1, k), device="cuda", dtype=torch.float32)
    y = torch.empty((1, n), device="cuda", dtype=torch.float32)
    torch.cuda.synchronize()
    for i in range(args.steps):
        qmatmul(kt_lib, x, 1, copies[i % len(copies)], y, stream)
    torch.cuda.synchronize()
    print(json.dumps({"only": "dominant", "kernel": "gemv_packed_single INT4 g64 M=1 4096x14336",
                      "algorithmic_bytes": gemv_bytes(1, k, n, bits, g), "launches": args.steps}), flush=True)
    return 0


def progress(what):
    """One line on stderr per finished section (stdout carries only the JSON line)."""
    print(f"[bench] {what}", file=sys.stderr, flush=True)


def weight_copies(torch, kt_lib, k, n, bits, g, seed, stream, packed):
    """A quantized weight and enough clones that one pass over them streams more than
    twice the MALL; packed adds each one's column-run copy (what M == 1 reads)."""
    w = Weight(torch, kt_lib, k, n, bits, g, seed, stream)
    if packed:
        w.pack(torch, kt_lib, stream)
    count = max(2, -(-2 * MALL_BYTES // w.nbytes))
    out = [w] + [w.clone(kt_lib) for _ in range(count - 1)]
    torch.cuda.synchronize()
    return out


def time_exact_steps(torch, stream_obj, fn, copies, steps, warmup):
    """Exactly `steps` launches (rotating the weight copies), recorded in one graph and
    replayed once between synchronizations, HIP events on the launch stream around the
    replay; `warmup` launches replayed the same way before. Returns ms per launch."""
    warm = torch.cuda.CUDAGraph()
    with torch.cuda.graph(warm, stream=stream_obj):
        for i in range(max(1, warmup)):
            fn(copies[i % len(copies)])
    timed = torch.cuda.CUDAGraph()
    with torch.cuda.graph(timed, stream=stream_obj):
        for i in range(steps):
            fn(copies[i % len(copies)])
    warm.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream_obj)
    timed.replay()
    t1.record(stream_obj)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps


def gemv_row(torch, kt_lib, stream_obj, k, n, bits, g, seed, launches=64):
    """Average launch time of the one-row product on the packed copy, back to back."""
    stream = ctypes.c_void_p(stream_obj.cuda_stream)
    cs = weight_copies(torch, kt_lib, k, n, bits, g, seed, stream, packed=True)
    x = torch.randn((1, k), device="cuda", dtype=torch.float32)
    y = torch.empty((1, n), device="cuda", dtype=torch.float32)
    for w in cs[:2]:
        qmatmul(kt_lib, x, 1, w, y, stream)
    ms = time_graph_launches(torch, stream_obj, lambda w: qmatmul(kt_lib, x, 1, w, y, stream), cs, launches)
    nbytes = gemv_bytes(1, k, n, bits, g)
    gbs = nbytes / (ms * 1e-3) / 1e9
    del cs
    return {"avg_us": round(ms * 1e3, 3), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "bytes": nbytes}


def chain_steps(kt_lib, ws, bufs):
    """The five kt_qmatmul_chain steps of one Qwen2-0.5B layer and the head, in the
    decoder's order (TransformerBlock.kt:40-46): o accumulated into x, norm2 and the
    SwiGLU gate/up pair, down accumulated into x, norm1 and q/k/v, the final norm and the
    head. Returns (the step array, the arrays it points into)."""
    b = bufs
    spec = [(b["ctx"], None, ws[3:4], [b["x"]], 1, 0),
            (b["x"], b["norm2"], ws[4:6], [b["gate"], b["up"]], 0, 1),
            (b["gate"], None, ws[6:7], [b["x"]], 1, 0),
            (b["x"], b["norm1"], ws[0:3], [b["q"], b["k"], b["v"]], 0, 0),
            (b["x"], b["normf"], ws[7:8], [b["logits"]], 0, 0)]
    steps = (kt_lib.QMatmulStep * len(spec))()
    keep = []
    for s, (x, nw, wl, outs, acc, swiglu) in zip(steps, spec):
        wa = (kt_lib.QWeight * len(wl))(*[w.struct for w in wl])
        oa = (ctypes.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
        keep += [wa, oa]
        s.x, s.norm_weight, s.eps = x.data_ptr(), nw.data_ptr() if nw is not None else None, 1e-6
        s.normed = b["normed"].data_ptr()
        s.weights = ctypes.cast(wa, ctypes.POINTER(kt_lib.QWeight))
        s.count = len(wl)
        s.outputs = ctypes.cast(oa, ctypes.POINTER(ctypes.c_void_p))
        s.biases, s.accumulate, s.alpha, s.swiglu_gate = None, acc, 1.0, swiglu
    return steps, keep


def qwen_step(torch, kt_lib, stream_obj, bits, g, steps, chained=False):
    """One Qwen2-0.5B layer's projections and the head at M = 1 on packed weights: q/k/v
    and gate/up as one grouped launch each, o, down and the head one launch each; or,
    chained, the decoder's single kt_qmatmul_chain launch over the same weights with the
    norms, the SwiGLU gate and the residual adds fused. One graph per weight copy,
    replayed. Returns (ms per step, bytes per step, copies)."""
    stream = ctypes.c_void_p(stream_obj.cuda_stream)
    base = [Weight(torch, kt_lib, k, n, bits, g, seed=1 + i, stream=stream).pack(torch, kt_lib, stream)
            for i, (_, k, n) in enumerate(QWEN)]
    set_bytes = sum(w.nbytes for w in base)
    copies = max(2, -(-2 * MALL_BYTES // set_bytes))
    sets = [base] + [[w.clone(kt_lib) for w in base] for _ in range(copies - 1)]
    xs = {k: torch.randn((1, k), device="cuda", dtype=torch.float32) for k in (896, 4864)}
    ys = [torch.empty((1, n), device="cuda", dtype=torch.float32) for _, _, n in QWEN]
    bufs = {name: torch.randn(n, device="cuda", dtype=torch.float32) * 0.1 + (1.0 if name.startswith("norm") else 0.0)
            for name, n in (("x", 896), ("ctx", 896), ("normed", 896), ("norm1", 896), ("norm2", 896),
                            ("normf", 896), ("gate", 4864), ("up", 4864), ("q", 896), ("k", 128), ("v", 128),
                            ("logits", 151936))}
    chains = [chain_steps(kt_lib, ws, bufs) for ws in sets] if chained else None
    torch.cuda.synchronize()

    def step(r):
        ws = sets[r]
        if chained:
            kt_lib.call("kt_qmatmul_chain", chains[r][0], 5, stream)
            return
        qmatmul_group(kt_lib, xs[896], 1, ws[0:3], ys[0:3], stream)
        qmatmul(kt_lib, xs[896], 1, ws[3], ys[3], stream)
        qmatmul_group(kt_lib, xs[896], 1, ws[4:6], ys[4:6], stream)
        qmatmul(kt_lib, xs[4864], 1, ws[6], ys[6], stream)
        qmatmul(kt_lib, xs[896], 1, ws[7], ys[7], stream)

    for r in range(copies):
        step(r)
    torch.cuda.synchronize()
    graphs = []
    for r in range(copies):
        gph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gph, stream=stream_obj):
            step(r)
        graphs.append(gph)
    for i in range(4 * copies):
        graphs[i % copies].replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream_obj)
    for i in range(steps):
        graphs[i % copies].replay()
    t1.record(stream_obj)
    torch.cuda.synchronize()
    del graphs, sets, base, chains
    return t0.elapsed_time(t1) / steps, sum(gemv_bytes(1, k, n, bits, g) for _, k, n in QWEN), copies


def run(args, torch, kt_lib, stream_obj) -> int:
    stream = ctypes.c_void_p(stream_obj.cuda_stream)
    gen = torch.Generator(device="cuda").manual_seed(0)

    # ---- the headline: INT4 g64 one-row product on the Llama-3-8B gate/up shape, packed
    k, n, bits, g = HEADLINE
    head = weight_copies(torch, kt_lib, k, n, bits, g, 7, stream, packed=True)
    x = torch.randn((1, k), generator=gen, device="cuda", dtype=torch.float32)
    y = torch.empty((1, n), device="cuda", dtype=torch.float32)
    for w in head:
        qmatmul(kt_lib, x, 1, w, y, stream)
    torch.cuda.synchronize()
    ms_per_step = time_exact_steps(torch, stream_obj, lambda w: qmatmul(kt_lib, x, 1, w, y, stream), head,
                                   args.steps, args.warmup)
    step_bytes = gemv_bytes(1, k, n, bits, g)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(value / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(),
                "kernel": "gemv_packed_single<4,4,true,0> (INT4 g64 M=1 4096x14336, packed copy)",
                "algorithmic_bytes": step_bytes, "avg_us": round(ms_per_step * 1e3, 3)}
    copies_head = len(head)
    del head
    progress(f"headline {ms_per_step * 1e3:.3f} us/step, {value:.1f} GB/s")

    extra = {}
    if not args.no_extra:
        # C2: the Qwen2-0.5B layer step (grouped launches) and each projection alone,
        # group 64 (primary) and 32 (secondary)
        c2 = {}
        for gg in (64, 32):
            ms, b, cp = qwen_step(torch, kt_lib, stream_obj, 4, gg, 200)
            gbs = b / (ms * 1e-3) / 1e9
            row = {"step": {"ms": round(ms, 5), "bytes": b, "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                            "launches": 5, "weight_copies": cp}}
            ms, b, cp = qwen_step(torch, kt_lib, stream_obj, 4, gg, 200, chained=True)
            gbs = b / (ms * 1e-3) / 1e9
            row["step_chained"] = {"ms": round(ms, 5), "bytes": b, "GB/s": round(gbs, 1),
                                   "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "launches": 1, "weight_copies": cp,
                                   "fused": "norm1, norm2, final norm, SwiGLU gate, two residual adds"}
            for name, kk, nn in [("q_o", 896, 896), ("k_v", 896, 128), ("gate_up", 896, 4864), ("down", 4864, 896),
                                 ("lm_head", 896, 151936)]:
                row[f"{name}_{kk}x{nn}"] = gemv_row(torch, kt_lib, stream_obj, kk, nn, 4, gg, 3)
            c2[f"g{gg}"] = row
        extra["c2_qwen2_0.5b_int4_m1"] = c2
        progress("C2 rows")

        # C1: INT8 GEMV 2048 x 2048 (group 64 and 32); per launch, back to back
        extra["c1_int8_gemv_2048x2048"] = {f"g{gg}": gemv_row(torch, kt_lib, stream_obj, 2048, 2048, 8, gg, 5, 128)
                                          for gg in (64, 32)}

        # C5 at M = 1, group 32 secondaries: gate/up and the head, INT4 and INT8
        progress("C1 rows")
        extra["c5_m1_g32"] = {f"int{bb}_{kk}x{nn}": gemv_row(torch, kt_lib, stream_obj, kk, nn, bb, 32, 17)
                              for bb in (4, 8) for kk, nn in [(4096, 14336), (4096, 128256)]}
        # INT8 prefill GEMM at M = 512, group 32, on the four projection shapes of a
        # 2048-wide layer, weights with their column-run copy (the column-run GEMM);
        # "layer" is their flops over their summed time (one of each). The same weights
        # without the copy (the reference-layout GEMM) are timed beside them.
        tot_flops = tot_ms = 0.0
        for (k, n) in [(2048, 2048), (2048, 512), (2048, 8192), (8192, 2048)]:
            wg = Weight(torch, kt_lib, k, n, 8, 32, seed=9, stream=stream).pack(torch, kt_lib, stream)
            ng = max(2, -(-2 * MALL_BYTES // (2 * wg.nbytes)))
            cg = [wg] + [wg.clone(kt_lib) for _ in range(ng - 1)]
            xg = torch.randn((512, k), generator=gen, device="cuda", dtype=torch.float32)
            yg = torch.empty((512, n), device="cuda", dtype=torch.float32)
            for w in cg:
                qmatmul(kt_lib, xg, 512, w, yg, stream)
            ag = time_graph_launches(torch, stream_obj, lambda w: qmatmul(kt_lib, xg, 512, w, yg, stream), cg, 32)
            plain = [w.without_copy(kt_lib) for w in cg]
            for w in plain[:2]:  # eager calls size the stream's workspace before recording
                qmatmul(kt_lib, xg, 512, w, yg, stream)
            ap = time_graph_launches(torch, stream_obj, lambda w: qmatmul(kt_lib, xg, 512, w, yg, stream), plain, 32)
            flops = 2.0 * 512 * k * n
            tflops = flops / (ag * 1e-3) / 1e12
            tot_flops += flops
            tot_ms += ag
            # the vendor library's plain bf16 GEMM of the same shape (no dequantization),
            # timed the same way, for scale
            wb = [torch.randn((k, n), generator=gen, device="cuda", dtype=torch.bfloat16)
                  for _ in range(max(2, -(-2 * MALL_BYTES // (2 * k * n))))]
            xb = xg.to(torch.bfloat16)
            yb = torch.empty((512, n), device="cuda", dtype=torch.bfloat16)
            for w in wb[:2]:  # eager calls first: the library sets up its handle outside capture
                torch.matmul(xb, w, out=yb)
            torch.cuda.synchronize()
            ab = time_graph_launches(torch, stream_obj, lambda w: torch.matmul(xb, w, out=yb), wb, 32)
            tb = flops / (ab * 1e-3) / 1e12
            tpl = flops / (ap * 1e-3) / 1e12
            extra[f"int8_g32_gemm_m512_{k}x{n}"] = {
                "TFLOP/s": round(tflops, 1), "frac_mfma": round(tflops / MFMA_PEAK_TFLOPS, 4),
                "avg_us": round(ag * 1e3, 3), "copies": ng, "kernel": "column-run GEMM (packed copy)",
                "reference_layout_gemm": {"TFLOP/s": round(tpl, 1), "frac_mfma": round(tpl / MFMA_PEAK_TFLOPS, 4),
                                          "avg_us": round(ap * 1e3, 3)},
                "hipblaslt_bf16_same_shape": {"TFLOP/s": round(tb, 1), "frac_mfma": round(tb / MFMA_PEAK_TFLOPS, 4),
                                              "avg_us": round(ab * 1e3, 3)}}
            del cg, wg, wb, plain
        layer = tot_flops / (tot_ms * 1e-3) / 1e12
        progress("C3 M=512 GEMM rows")
        extra["int8_g32_gemm_m512_layer"] = {"TFLOP/s": round(layer, 1), "frac_mfma": round(layer / MFMA_PEAK_TFLOPS, 4),
                                             "avg_us": round(tot_ms * 1e3, 3)}

        # the M sweep of the INT8 g32 2048 -> 8192 product (M = 1, 16: the decode kernels;
        # 128 and up: the GEMM), weights with their column-run copy: time per launch,
        # TFLOP/s and GB/s of algorithmic bytes
        wm = Weight(torch, kt_lib, 2048, 8192, 8, 32, seed=11, stream=stream).pack(torch, kt_lib, stream)
        nm = max(2, -(-2 * MALL_BYTES // (2 * wm.nbytes)))
        cm = [wm] + [wm.clone(kt_lib) for _ in range(nm - 1)]
        sweep = {}
        for mm in (1, 16, 128, 512, 2048):
            xm = torch.randn((mm, 2048), generator=gen, device="cuda", dtype=torch.float32)
            ym = torch.empty((mm, 8192), device="cuda", dtype=torch.float32)
            for w in cm[:2]:
                qmatmul(kt_lib, xm, mm, w, ym, stream)
            am = time_graph_launches(torch, stream_obj, lambda w: qmatmul(kt_lib, xm, mm, w, ym, stream), cm, 32)
            flops = 2.0 * mm * 2048 * 8192
            sweep[str(mm)] = {"avg_us": round(am * 1e3, 3), "TFLOP/s": round(flops / (am * 1e-3) / 1e12, 1),
                              "GB/s": round(gemv_bytes(mm, 2048, 8192, 8, 32) / (am * 1e-3) / 1e9, 1)}
        extra["int8_g32_m_sweep_2048x8192"] = sweep
        progress("C3 M sweep")
        del cm, wm

        # Llama-3-8B projection shapes (q/o 4096 -> 4096, k/v 4096 -> 1024, gate/up
        # 4096 -> 14336, down 14336 -> 4096), INT4 and INT8 at group 64, M = 1, 8, 16, 64, 512
        l8 = {}
        for bits in (4, 8):
            for (k, n) in [(4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)]:
                wl = Weight(torch, kt_lib, k, n, bits, 64, seed=13, stream=stream).pack(torch, kt_lib, stream)
                nl = max(2, -(-2 * MALL_BYTES // wl.nbytes))
                cl = [wl] + [wl.clone(kt_lib) for _ in range(nl - 1)]
                row = {}
                for mm in (1, 8, 16, 64, 512):
                    xl = torch.randn((mm, k), generator=gen, device="cuda", dtype=torch.float32)
                    yl = torch.empty((mm, n), device="cuda", dtype=torch.float32)
                    for w in cl[:2]:
                        qmatmul(kt_lib, xl, mm, w, yl, stream)
                    al = time_graph_launches(torch, stream_obj, lambda w: qmatmul(kt_lib, xl, mm, w, yl, stream), cl, 32)
                    gbs = gemv_bytes(mm, k, n, bits, 64) / (al * 1e-3) / 1e9
                    tfl = 2.0 * mm * k * n / (al * 1e-3) / 1e12
                    row[str(mm)] = {"avg_us": round(al * 1e3, 3), "GB/s": round(gbs, 1),
                                    "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "TFLOP/s": round(tfl, 1),
                                    "frac_mfma": round(tfl / MFMA_PEAK_TFLOPS, 4)}
                l8[f"int{bits}_g64_{k}x{n}"] = row
                del cl, wl
        extra["llama8b_projections_m_sweep"] = l8
        progress("C5 M sweep")

        # kt_quantize on the gate/up shape 4096 x 14336 at group 64 (reads the fp32 weight,
        # writes the packed weight, scales and zeros), three distinct inputs (> 2x MALL);
        # each call ends with the NaN flag's readback, so the figure is per call, event to
        # event on the stream, not per kernel
        qz = {}
        kq, nq = 4096, 14336
        srcs = [torch.randn((kq, nq), generator=gen, device="cuda", dtype=torch.float32) * 0.02 for _ in range(3)]
        for bits in (4, 8):
            groups, bpr = layout(kq, nq, bits, 64)
            qq = torch.empty(kq * bpr, dtype=torch.uint8, device="cuda")
            sq = torch.empty(groups * nq, dtype=torch.float32, device="cuda")
            zq = torch.empty(groups * nq, dtype=torch.uint8, device="cuda") if bits == 4 else None

            def quantize_once(src, bits=bits, qq=qq, sq=sq, zq=zq):
                kt_lib.call("kt_quantize", src.data_ptr(), kq, nq, bits, 64, qq.data_ptr(), sq.data_ptr(),
                            zq.data_ptr() if zq is not None else None, stream)

            for src in srcs:
                quantize_once(src)
            torch.cuda.synchronize()
            times = []
            for i in range(12):
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record(stream_obj)
                quantize_once(srcs[i % len(srcs)])
                e1.record(stream_obj)
                torch.cuda.synchronize()
                times.append(e0.elapsed_time(e1))
            tq = sorted(times)[len(times) // 2]
            bq = 4 * kq * nq + kq * bpr + 4 * groups * nq + (groups * nq if bits == 4 else 0)
            gq = bq / (tq * 1e-3) / 1e9
            qz[f"int{bits}_g64_{kq}x{nq}"] = {"median_us_per_call": round(tq * 1e3, 3), "bytes": bq,
                                              "GB/s": round(gq, 1), "frac_hbm": round(gq / HBM_PEAK_GBS, 4)}
        extra["quantize_llama8b_gate_4096x14336"] = qz
        progress("quantize")
        del srcs

        extra["llama1b_int4_decoder"] = decoder_figures(torch, stream_obj)
        progress("C4 decoder")

    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: x ~ N(0,1) fp32, W ~ N(0,0.02) fp32 quantized on device (seeded)",
        "config": {"workload": "llama-3-8b gate/up projection 4096x14336, INT4 g64, M=1 (one dequant-GEMV "
                               "launch per step)",
                   "launches_per_step": 1,
                   "weights": "uint4 + fp32 scales + u8 zeros (reference layout) with the column-run copy the "
                              "one-row kernel streams", "group_size": g, "m": 1,
                   "step_bytes": step_bytes, "weight_copies": copies_head, "graph_replay": True},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
