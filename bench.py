#!/usr/bin/env python3
"""Benchmark of the dequant-GEMV hot path on one MI355X.

Workload (one "step"): the INT4 (g64) M = 1 projections of a Qwen2-0.5B-shaped
decoder layer plus its lm_head -- q/o 896->896, k/v 896->128, gate/up 896->4864,
down 4864->896, lm_head 896->151936 -- with x ~ N(0,1) fp32 and W ~ N(0, 0.02)
quantized on the device by kt_quantize (the reference layout: qdata [K x N/2],
fp32 scales and u8 zeros [K/64 x N]). Inputs are resident in HBM before timing.
q/k/v (one input) and gate/up (one input) each go out as one grouped launch
(kt_qmatmul_group), o, down and lm_head as one launch each. Each step uses a
different copy of the weight set so that the timed loop streams more than twice
the 256 MB Infinity Cache; a step's launches are captured in a HIP graph (one graph
per weight copy) and replayed.

value = algorithmic bytes of a step / measured step time (GB/s). Algorithmic bytes
per GEMV = K*bytesPerRow + 4*groups*N + groups*N (zeros) + 4*K (x) + 4*N (y).

The JSON line also carries:
  roofline      -- the dominant kernel (the lm_head GEMV): back-to-back launches in a
                   graph on the launch stream, HIP events around the timed replays,
                   against 8 TB/s; traffic from rocprofv3 PMC runs (profiles/);
  cpu_baseline  -- the oracle (C restatement of MatMul.multiplyQuantized, M == 1
                   unit schedule, work-stealing threads) on the same workload;
  extra         -- the two targets of the workload family: INT4 GEMV on the
                   Llama-3-8B FFN shape (4096->14336) and the INT8 group-32 prefill
                   GEMM at M = 512 on the 2048-wide layer's four projection shapes
                   (2048->2048, 2048->512, 2048->8192, 8192->2048) and their sum, each
                   with its fraction of the MFMA peak and, for scale, the vendor library's
                   plain bf16 GEMM (torch.matmul -> hipBLASLt, no dequantization) on the
                   same shape timed the same way; the M sweep (1, 16, 128, 512, 2048) of
                   the INT8 2048 -> 8192 product; the Llama-3-8B projection shapes
                   (4096->4096, 4096->1024, 4096->14336, 14336->4096), INT4 and INT8 g64
                   at M = 1, 8, 64, 512; kt_quantize on 4096 x 14336 (per call,
                   including its NaN-flag readback); and the Llama-style 1B INT4
                   decoder end to end (1024-token prefill, greedy decode steps).
                   Every timed graph reads each of its weight copies (> 2x MALL).

--only dominant | copy | quantize | gemm runs just the lm_head GEMV (or a 256 MB device
copy, the calibration of the HBM byte counters, or kt_quantize INT4 and INT8 g64 on
4096 x 14336, or the INT8 g32 M = 512 GEMM on 2048 -> 8192) for rocprofv3 runs.
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
        self.struct = None
        self._bind(kt_lib)

    def _bind(self, kt_lib):
        self.struct = kt_lib.QWeight(self.q.data_ptr(), self.s.data_ptr(),
                                     self.z.data_ptr() if self.z is not None else None,
                                     self.k, self.n, self.bits, self.g)

    def clone(self, kt_lib):
        c = object.__new__(Weight)
        c.k, c.n, c.bits, c.g = self.k, self.n, self.bits, self.g
        c.q = self.q.clone()
        c.s = self.s.clone()
        c.z = self.z.clone() if self.z is not None else None
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


def cpu_baseline(seconds: float = 10.0):
    """The oracle's M == 1 kernel on the same Qwen set, on this host's cores."""
    import numpy as np

    import oracle

    oracle.build()
    threads = max(1, min(16, os.cpu_count() or 1))
    rng = np.random.default_rng(1)
    weights = []
    for _, k, n in QWEN:
        w = (rng.standard_normal((k, n), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
        st, q = oracle.quantize(w, 4, 64)
        weights.append((k, n, q))
    xs = {k: np.random.default_rng(0).standard_normal((1, k), dtype=np.float32) for k in (896, 4864)}
    step_bytes = sum(gemv_bytes(1, k, n, 4, 64) for _, k, n in QWEN)
    steps = 0
    t0 = time.perf_counter()
    while True:
        for k, n, q in weights:
            oracle.multiply_quantized(xs[k], q, 1, threads=threads)
        steps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= seconds:
            break
    return {
        "value": round(step_bytes * steps / elapsed / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{steps} passes of the 8 Qwen2-0.5B INT4 g64 M=1 projections ({elapsed:.1f} s), "
                  "C restatement of MatMul.multiplyQuantized's M=1 unit schedule, -O3 -ffp-contract=off",
    }


def traffic_from_profiles():
    """HBM bytes per lm_head launch measured with rocprofv3 --pmc (profiles/), if recorded."""
    path = ROOT / "profiles" / "traffic_gemv_int4_lm_head.json"
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
    ap.add_argument("--only", choices=["dominant", "copy", "quantize", "gemm"],
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
        # the INT8 g32 prefill GEMM at M = 512 on 2048 -> 8192, weight copies in rotation
        wg = Weight(torch, kt_lib, 2048, 8192, 8, 32, seed=9, stream=stream)
        cg = [wg] + [wg.clone(kt_lib) for _ in range(max(1, -(-2 * MALL_BYTES // wg.nbytes)) - 1)]
        xg = torch.randn((512, 2048), device="cuda", dtype=torch.float32)
        yg = torch.empty((512, 8192), device="cuda", dtype=torch.float32)
        torch.cuda.synchronize()
        for i in range(args.steps):
            qmatmul(kt_lib, xg, 512, cg[i % len(cg)], yg, stream)
        torch.cuda.synchronize()
        print(json.dumps({"only": "gemm", "kernel": "gemm_kernel int8 g32 M=512 2048x8192",
                          "flops": 2 * 512 * 2048 * 8192, "launches": args.steps}), flush=True)
        return 0
    w = Weight(torch, kt_lib, 896, 151936, 4, 64, seed=8, stream=stream)
    copies = [w] + [w.clone(kt_lib) for _ in range(max(1, -(-2 * MALL_BYTES // w.nbytes)) - 1)]
    x = torch.randn((1, 896), device="cuda", dtype=torch.float32)
    y = torch.empty((1, 151936), device="cuda", dtype=torch.float32)
    torch.cuda.synchronize()
    for i in range(args.steps):
        qmatmul(kt_lib, x, 1, copies[i % len(copies)], y, stream)
    torch.cuda.synchronize()
    print(json.dumps({"only": "dominant", "kernel": "lm_head 896x151936 int4 g64 M=1",
                      "algorithmic_bytes": gemv_bytes(1, 896, 151936, 4, 64), "launches": args.steps}), flush=True)
    return 0


def run(args, torch, kt_lib, stream_obj) -> int:
    stream = ctypes.c_void_p(stream_obj.cuda_stream)
    bits, g = 4, 64

    # ---- weights: one quantized set, cloned until the rotation exceeds 2x the MALL
    base = [Weight(torch, kt_lib, k, n, bits, g, seed=1 + i, stream=stream) for i, (_, k, n) in enumerate(QWEN)]
    set_bytes = sum(w.nbytes for w in base)
    copies = max(2, -(-2 * MALL_BYTES // set_bytes))
    sets = [base] + [[w.clone(kt_lib) for w in base] for _ in range(copies - 1)]
    gen = torch.Generator(device="cuda").manual_seed(0)
    xs = {k: torch.randn((1, k), generator=gen, device="cuda", dtype=torch.float32) for k in (896, 4864)}
    ys = [torch.empty((1, n), device="cuda", dtype=torch.float32) for _, _, n in QWEN]
    torch.cuda.synchronize()

    def step(ws):
        # q, k, v share x; gate, up share x: one grouped launch each
        qmatmul_group(kt_lib, xs[896], 1, ws[0:3], ys[0:3], stream)
        qmatmul(kt_lib, xs[896], 1, ws[3], ys[3], stream)
        qmatmul_group(kt_lib, xs[896], 1, ws[4:6], ys[4:6], stream)
        qmatmul(kt_lib, xs[4864], 1, ws[6], ys[6], stream)
        qmatmul(kt_lib, xs[896], 1, ws[7], ys[7], stream)

    # eager warm-up (allocates the library's per-stream workspace before capture)
    for r in range(copies):
        step(sets[r])
    torch.cuda.synchronize()
    graphs = []
    for r in range(copies):
        gph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gph, stream=stream_obj):
            step(sets[r])
        graphs.append(gph)
    torch.cuda.synchronize()
    for i in range(args.warmup):
        graphs[i % copies].replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream_obj)
    for i in range(args.steps):
        graphs[i % copies].replay()
    t1.record(stream_obj)
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / args.steps
    step_bytes = sum(gemv_bytes(1, k, n, bits, g) for _, k, n in QWEN)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    # ---- dominant kernel: the lm_head GEMV, back-to-back launches on the launch stream
    head = [s[-1] for s in sets]
    head_y = ys[-1]
    head_bytes = gemv_bytes(1, 896, 151936, bits, g)
    avg_ms = time_graph_launches(torch, stream_obj, lambda w: qmatmul(kt_lib, xs[896], 1, w, head_y, stream), head, 60)
    achieved = head_bytes / (avg_ms * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(),
                "kernel": "gemv_wide_kernel<4,4,true> (lm_head 896x151936 int4 g64 M=1)",
                "algorithmic_bytes": head_bytes, "avg_us": round(avg_ms * 1e3, 3)}

    extra = {}
    if not args.no_extra:
        # INT4 GEMV on the Llama-3-8B FFN shape, 16 copies (> 2x MALL)
        w8 = Weight(torch, kt_lib, 4096, 14336, 4, 64, seed=7, stream=stream)
        n8 = max(2, -(-2 * MALL_BYTES // w8.nbytes))
        c8 = [w8] + [w8.clone(kt_lib) for _ in range(n8 - 1)]
        x8 = torch.randn((1, 4096), generator=gen, device="cuda", dtype=torch.float32)
        y8 = torch.empty((1, 14336), device="cuda", dtype=torch.float32)
        for w in c8:
            qmatmul(kt_lib, x8, 1, w, y8, stream)
        a8 = time_graph_launches(torch, stream_obj, lambda w: qmatmul(kt_lib, x8, 1, w, y8, stream), c8, 64)
        b8 = gemv_bytes(1, 4096, 14336, 4, 64)
        extra["int4_gemv_llama8b_ffn_4096x14336"] = {
            "GB/s": round(b8 / (a8 * 1e-3) / 1e9, 1), "frac_hbm": round(b8 / (a8 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "avg_us": round(a8 * 1e3, 3), "bytes": b8, "copies": n8}
        del c8, w8
        # INT8 prefill GEMM at M = 512, group 32, on the four projection shapes of a
        # 2048-wide layer; "layer" is their flops over their summed time (one of each).
        tot_flops = tot_ms = 0.0
        for (k, n) in [(2048, 2048), (2048, 512), (2048, 8192), (8192, 2048)]:
            wg = Weight(torch, kt_lib, k, n, 8, 32, seed=9, stream=stream)
            ng = max(2, -(-2 * MALL_BYTES // wg.nbytes))
            cg = [wg] + [wg.clone(kt_lib) for _ in range(ng - 1)]
            xg = torch.randn((512, k), generator=gen, device="cuda", dtype=torch.float32)
            yg = torch.empty((512, n), device="cuda", dtype=torch.float32)
            for w in cg:
                qmatmul(kt_lib, xg, 512, w, yg, stream)
            ag = time_graph_launches(torch, stream_obj, lambda w: qmatmul(kt_lib, xg, 512, w, yg, stream), cg, 32)
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
            extra[f"int8_g32_gemm_m512_{k}x{n}"] = {
                "TFLOP/s": round(tflops, 1), "frac_mfma": round(tflops / MFMA_PEAK_TFLOPS, 4),
                "avg_us": round(ag * 1e3, 3), "copies": ng,
                "hipblaslt_bf16_same_shape": {"TFLOP/s": round(tb, 1), "frac_mfma": round(tb / MFMA_PEAK_TFLOPS, 4),
                                              "avg_us": round(ab * 1e3, 3)}}
            del cg, wg, wb
        layer = tot_flops / (tot_ms * 1e-3) / 1e12
        extra["int8_g32_gemm_m512_layer"] = {"TFLOP/s": round(layer, 1), "frac_mfma": round(layer / MFMA_PEAK_TFLOPS, 4),
                                             "avg_us": round(tot_ms * 1e3, 3)}

        # the M sweep of the INT8 g32 2048 -> 8192 product (M = 1, 16: the decode kernels;
        # 128 and up: the GEMM): time per launch, TFLOP/s and GB/s of algorithmic bytes
        wm = Weight(torch, kt_lib, 2048, 8192, 8, 32, seed=11, stream=stream)
        nm = max(2, -(-2 * MALL_BYTES // wm.nbytes))
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
        del cm, wm

        # Llama-3-8B projection shapes (q/o 4096 -> 4096, k/v 4096 -> 1024, gate/up
        # 4096 -> 14336, down 14336 -> 4096), INT4 and INT8 at group 64, M = 1, 8, 64, 512
        l8 = {}
        for bits in (4, 8):
            for (k, n) in [(4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)]:
                wl = Weight(torch, kt_lib, k, n, bits, 64, seed=13, stream=stream)
                nl = max(2, -(-2 * MALL_BYTES // wl.nbytes))
                cl = [wl] + [wl.clone(kt_lib) for _ in range(nl - 1)]
                row = {}
                for mm in (1, 8, 64, 512):
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
        del srcs

        extra["llama1b_int4_decoder"] = decoder_figures(torch, stream_obj)

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
        "config": {"workload": "qwen2-0.5b int4 g64 M=1 projection GEMVs (q,k,v,o,gate,up,down,lm_head)",
                   "launches_per_step": 5,
                   "weights": "uint4 + fp32 scales + u8 zeros, reference layout", "group_size": g, "m": 1,
                   "step_bytes": step_bytes, "weight_copies": copies, "graph_replay": True},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
