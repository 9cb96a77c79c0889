"""Benchmark of the NF4 quantized-linear hot path on one MI355X.

Headline (BASELINE.json metric, configs[1]): the decode GEMV
y[1, 11008] = x[1, 4096] . deq(W), W the reference's [4096, 11008] packed NF4
weight with double-quantized scales (as Nf4Linear::from_values builds it,
src/qwennet.rs:198-205), f32 activations and accumulation.  One step = one
GEMV launch over one batch.  Weights are resident in HBM and rotated over
enough copies (>= 512 MiB, twice the 256 MiB Infinity Cache) that every step
streams its weight from HBM ("cold").  value = algorithmic bytes per step *
steps / timed seconds.

Also reported in the same JSON line (not the headline): warm GEMV, NF4
dequantize and quantize of the config-1 4096x4096 matrix, each with its
kernel's roofline fraction, and the CPU baseline (the oracle's restatement
of the reference's CPU path, timed on this host).

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "NF4 dequant/GEMV GB/s and prefill GEMM TFLOP/s, % of MI355X roofline"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6
MALL_BYTES = 256 << 20


def gemv_bytes(d_in: int, d_out: int, dq: bool, x_bytes: int = 4, y_bytes: int = 4) -> int:
    """Algorithmic HBM bytes of one GEMV: packed codes + scales + x + y."""
    n = d_in * d_out
    nb = (n + 63) // 64
    scales = nb + 4 if dq else 4 * nb
    return (n + 1) // 2 + scales + d_in * x_bytes + d_out * y_bytes


def kernel_ms(torch, fn, iters: int) -> float:
    """Average GPU time of fn() measured with event pairs on the launch stream.

    A long sleep kernel is queued first so that every launch below is already
    enqueued when the GPU reaches it: the event pairs then bracket the kernel
    itself, not host-side launch latency."""
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    torch.cuda.synchronize()
    torch.cuda._sleep(200_000_000)
    for i in range(iters):
        starts[i].record()
        fn(i)
        ends[i].record()
    torch.cuda.synchronize()
    times = sorted(s.elapsed_time(e) for s, e in zip(starts, ends))
    return times[len(times) // 2]


def bench_gemv(torch, Q, L, args) -> dict:
    d_in, d_out = 4096, 11008
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(0x4E463458)
    w = torch.randn(d_in * d_out, device=dev, generator=g) * 0.02
    base = Q.PackedNf4Tensor.quantize(w).with_double_quantization()
    del w
    nbytes = gemv_bytes(d_in, d_out, dq=True)
    copies = max(2, -(-(2 * MALL_BYTES) // nbytes))  # >= 512 MiB of weights
    layers = []
    for _ in range(copies):
        p = Q.PackedNf4Tensor(base.codes.clone(), len(base), dq_codes=base.dq_codes.clone(),
                              scale_of_scales=base.scale_of_scales.clone())
        layers.append(Q.Nf4Linear.from_packed(p, d_in, d_out))
    x = torch.randn(1, d_in, device=dev, generator=g)
    y = torch.empty(1, d_out, device=dev)
    ws_bytes = L.lib().unifur_nf4_linear_workspace_size(1, d_in, d_out, L.F32, 0)
    ws = torch.zeros(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    structs = [lay.weight_struct() for lay in layers]
    lib = L.lib()

    def launch(i: int) -> None:
        st = lib.unifur_nf4_linear_forward(x.data_ptr(), L.F32, 1, ctypes.byref(structs[i % copies]), None, None,
                                           y.data_ptr(), L.F32, ws.data_ptr(), ws_bytes,
                                           torch.cuda.current_stream().cuda_stream)
        if st != 0:
            L.check(st)

    # sanity: GEMV of copy 0 against torch's f32 matvec of the dequantized weight
    launch(0)
    ref = x @ layers[0].dequantized_weight()
    torch.cuda.synchronize()
    rel = float((y - ref).abs().max() / ref.abs().max())
    if not rel < 1e-4:
        raise RuntimeError(f"GEMV sanity check failed: max rel error {rel:.3e}")

    for i in range(args.warmup):
        launch(i)
    steps = args.steps
    # Whole-job timing: K launches replayed from a HIP graph (launch-bound
    # otherwise: one GEMV is a few microseconds), falling back to eager.
    graph = None
    try:
        graph = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(graph, stream=s):
                for i in range(copies):
                    launch(i)
        torch.cuda.current_stream().wait_stream(s)
        graph.replay()
        torch.cuda.synchronize()
    except Exception as e:  # noqa: BLE001 - report and time eagerly
        print(f"# graph capture unavailable ({e}); timing eager launches", file=sys.stderr)
        graph = None
    reps = -(-steps // copies) if graph is not None else 0
    if graph is not None:
        steps = reps * copies
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    if graph is not None:
        for _ in range(reps):
            graph.replay()
    else:
        for i in range(steps):
            launch(i)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    cold_ms = kernel_ms(torch, lambda i: launch(i % copies), 2 * copies)
    warm_ms = kernel_ms(torch, lambda i: launch(0), 2 * copies)
    # re-check after the timed work
    launch(1)
    torch.cuda.synchronize()
    if not float((y - ref).abs().max() / ref.abs().max()) < 1e-4:
        raise RuntimeError("GEMV result drifted during timing")
    return {
        "steps": steps, "elapsed_s": elapsed, "bytes": nbytes, "copies": copies,
        "value_gbs": nbytes * steps / elapsed / 1e9, "ms_per_step": elapsed * 1e3 / steps,
        "kernel_cold_ms": cold_ms, "kernel_warm_ms": warm_ms, "graph": graph is not None,
    }


def bench_codec(torch, Q, L) -> dict:
    """Config 1 (4096 x 4096 f32): quantize and dequantize kernels."""
    n = 4096 * 4096
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(0x4E463457)
    copies = 4
    vals = [torch.randn(n, device=dev, generator=g) * 0.02 for _ in range(copies)]
    packs = [Q.PackedNf4Tensor.quantize(v) for v in vals]
    outs = [torch.empty(n, device=dev) for _ in range(copies)]
    q_ms = kernel_ms(torch, lambda i: Q.PackedNf4Tensor.quantize(vals[i % copies]), 16)
    lib = L.lib()
    structs = [p.scales_struct() for p in packs]

    def deq(i: int) -> None:
        p = packs[i % copies]
        L.check(lib.unifur_nf4_dequantize(p.codes.data_ptr(), ctypes.byref(structs[i % copies]), n,
                                          outs[i % copies].data_ptr(), L.F32,
                                          torch.cuda.current_stream().cuda_stream))

    d_ms = kernel_ms(torch, deq, 16)
    codec_bytes = 4 * n + n // 2 + 4 * (n // 64)  # f32 values + packed codes + f32 absmax
    return {"quantize_ms": q_ms, "dequant_ms": d_ms, "bytes": codec_bytes,
            "quantize_gbs": codec_bytes / q_ms / 1e6, "dequant_gbs": codec_bytes / d_ms / 1e6}


def cpu_baseline(sample_s: float) -> dict:
    """The reference's CPU path restated (oracle): serial dequantize of the
    whole weight, then an f32 matmul on all host cores, timed on the config-2
    GEMV for about `sample_s` seconds."""
    import numpy as np

    from oracle import oracle as O

    d_in, d_out = 4096, 11008
    v = O.fill_normal(0x4E463458, 0.02, d_in * d_out)
    packed, absmax = O.quantize_packed(v)
    q, sos = O.double_quantize(absmax)
    x = O.fill_normal(0x59, 1.0, d_in).reshape(1, d_in)
    threads = len(os.sched_getaffinity(0))
    iters = 0
    t0 = time.perf_counter()
    while True:
        w = O.dequantize_packed(packed, v.size, None, q, sos)      # 1 thread, as the reference
        O.linear_f32(x, w, d_in, d_out, threads=threads)            # all cores
        iters += 1
        if time.perf_counter() - t0 >= sample_s:
            break
    dt = (time.perf_counter() - t0) / iters
    del w
    _ = np.zeros(1)
    return {"value": gemv_bytes(d_in, d_out, dq=True) / dt / 1e9, "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"{iters} x (1-thread dequantize of the 4096x11008 DQ weight + {threads}-thread f32 "
                      f"GEMV), {dt * 1e3:.1f} ms each, oracle/nf4_oracle.c restatement of "
                      f"PackedNf4Tensor::dequantize + burn linear"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2400)
    ap.add_argument("--warmup", type=int, default=96)
    ap.add_argument("--cpu-sample-s", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(see DESIGN.md for how the NF4 path would shard); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    from unifur_amd import _lib as L
    from unifur_amd import quantize as Q

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    L.lib()
    gemv = bench_gemv(torch, Q, L, args)
    codec = bench_codec(torch, Q, L)
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_sample_s)

    achieved = gemv["bytes"] / gemv["kernel_cold_ms"] / 1e6
    line = {
        "metric": METRIC,
        "value": round(gemv["value_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": gemv["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(gemv["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "config 2: NF4 decode GEMV x[1x4096] f32 . W[4096x11008] (Wt of the logical "
                        "11008x4096), block 64, double-quantized scales, y f32; "
                        f"{gemv['copies']} weight copies rotated (cold HBM)",
            "timing": "HIP-graph replay of the launches" if gemv["graph"] else "eager launches",
            "d_in": 4096, "d_out": 11008, "rows": 1, "block_size": 64, "double_quantized": True,
            "bytes_per_step": gemv["bytes"],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "gemv_kernel<1,16,f32,dq>",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
        },
        "cpu_baseline": cpu,
        "secondary": {
            "gemv_warm": {"kernel_ms": round(gemv["kernel_warm_ms"], 5),
                          "gbs": round(gemv["bytes"] / gemv["kernel_warm_ms"] / 1e6, 1)},
            "dequantize_f32_config1": {"kernel_ms": round(codec["dequant_ms"], 5),
                                       "gbs": round(codec["dequant_gbs"], 1),
                                       "frac": round(codec["dequant_gbs"] / HBM_PEAK_GBS, 4)},
            "quantize_config1": {"kernel_ms": round(codec["quantize_ms"], 5),
                                 "gbs": round(codec["quantize_gbs"], 1),
                                 "frac": round(codec["quantize_gbs"] / HBM_PEAK_GBS, 4)},
        },
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
