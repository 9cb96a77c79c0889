"""Benchmark of the NF4 quantized-linear hot path on one MI355X.

Headline (BASELINE.json metric, configs[1]): the decode GEMV
y[1, 11008] = x[1, 4096] . deq(W), W the reference's [4096, 11008] NF4
weight (logical 11008 x 4096, blocks of 64 along d_out) with double-quantized
scales, as Nf4Linear::from_values builds it (src/qwennet.rs:198-205), held on
the device in the column-striped layout; f32 activations and accumulation.
One step = one GEMV launch.  The weights are resident in HBM and rotated over
enough copies (>= 512 MiB, twice the 256 MiB Infinity Cache) that every step
streams its weight from HBM ("cold").  value = algorithmic bytes per step *
steps / timed seconds, the steps replayed from a HIP graph.

The same JSON line carries the GEMV kernel's roofline (HIP events on its
launch stream), the CPU baseline (the oracle's restatement of the
reference's CPU path, timed on this host) and secondary figures for every
BASELINE config: quantize / dequantize (config 1), the MFMA prefill GEMM
with LoRA (config 3, TFLOP/s), the SwiGLU block at T = 1, 16, 512
(config 4) and the Qwen2-0.5B-shaped projection set (config 5: whole-model
quantize pass, per-token decode at batch 1 and 32).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
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
F32_MFMA_PEAK_TFLOPS = 157.3
MALL_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_gemv_config2.txt")


def gemv_bytes(d_in: int, d_out: int, dq: bool, x_bytes: int = 4, y_bytes: int = 4, rows: int = 1) -> int:
    """Algorithmic HBM bytes of one GEMV: packed codes + scales + x + y."""
    n = d_in * d_out
    nb = (n + 63) // 64
    scales = nb + 4 if dq else 4 * nb
    return (n + 1) // 2 + scales + rows * (d_in * x_bytes + d_out * y_bytes)


def event_ms(torch, fn, iters: int) -> float:
    """Median GPU time of fn(i) from one event pair per launch on the launch
    stream.  A long sleep kernel is queued first so that every launch is
    enqueued before the GPU reaches it: the pairs bracket the kernels, not
    host launch latency."""
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


def capture(torch, fn, n: int):
    """A HIP graph of fn(0) .. fn(n - 1) on a side stream (None if capture fails)."""
    try:
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            # one eager pass on the capture stream first: the library sizes its
            # per-stream workspace (hipMalloc) outside the capture
            for i in range(n):
                fn(i)
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=s):
                for i in range(n):
                    fn(i)
        torch.cuda.current_stream().wait_stream(s)
        g.replay()
        torch.cuda.synchronize()
        return g
    except Exception as e:  # noqa: BLE001 - report and time eagerly
        print(f"# graph capture unavailable ({e}); timing eager launches", file=sys.stderr)
        return None


def replay_event_ms(torch, graph, launches: int, reps: int = 20) -> float:
    """Per-launch GPU time of a graph of `launches` kernels: one HIP event pair
    on the replay stream around `reps` back-to-back replays."""
    graph.replay()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (reps * launches)


def steady_ms(torch, graph, launches: int, reps: int = 10, runs: int = 5, warm_s: float = 0.05) -> float:
    """Per-launch GPU time of a graph at steady state: the graph is replayed
    for at least warm_s seconds first (a pass timed straight after capture
    meets the clocks still ramping: config 3 read 79 us per call there against
    70 us a few passes later on the same box), then the median of `runs`
    event-timed passes of `reps` back-to-back replays (replay_event_ms)."""
    t0 = time.perf_counter()
    while True:
        graph.replay()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= warm_s:
            break
    times = sorted(replay_event_ms(torch, graph, launches, reps) for _ in range(runs))
    return times[len(times) // 2]


def _i64(v: int) -> int:
    return v - (1 << 64) if v >= 1 << 63 else v


_GAMMA, _MIX1, _MIX2 = _i64(0x9E3779B97F4A7C15), _i64(0xBF58476D1CE4E5B9), _i64(0x94D049BB133111EB)


def _lsr(z, s: int):
    return (z >> s) & ((1 << (64 - s)) - 1)  # logical shift of int64 bits


def _splitmix64(z):
    z = (z ^ _lsr(z, 30)) * _MIX1
    z = (z ^ _lsr(z, 27)) * _MIX2
    return z ^ _lsr(z, 31)


def seeded_normal(torch, seed: int, sigma: float, n: int, device="cuda"):
    """n float32 values ~ N(0, sigma^2), the tests' input generator: value i is
    the Box-Muller transform of the SplitMix64 outputs at seed + (2 i + 1) gamma
    and seed + (2 i + 2) gamma (gamma = 0x9E3779B97F4A7C15), u1 in (0, 1],
    u2 in [0, 1), evaluated in float64 -- counter-based, so computed here on
    the device with wrapping int64 arithmetic."""
    out = torch.empty(n, dtype=torch.float32, device=device)
    base = _i64(seed % (1 << 64))
    step = 1 << 24
    for s0 in range(0, n, step):
        i = torch.arange(s0, min(n, s0 + step), dtype=torch.int64, device=device)
        a = _splitmix64(base + (2 * i + 1) * _GAMMA)
        b = _splitmix64(base + (2 * i + 2) * _GAMMA)
        u1 = (_lsr(a, 11) + 1).double() * (1.0 / 9007199254740992.0)
        u2 = _lsr(b, 11).double() * (1.0 / 9007199254740992.0)
        z = torch.sqrt(-2.0 * torch.log(u1)) * torch.cos(6.283185307179586476925286766559 * u2)
        out[s0:s0 + i.numel()] = (z * sigma).float()
    return out


class Rng:
    """Seeded inputs of one workload: each draw is seeded_normal of its own
    seed (the workload's seed plus a draw counter)."""

    def __init__(self, torch, seed: int, device="cuda"):
        self.torch, self.seed, self.device, self.count = torch, seed, device, 0

    def normal(self, *shape, sigma: float = 1.0):
        n = 1
        for d in shape:
            n *= d
        self.count += 1
        return seeded_normal(self.torch, (self.seed << 16) + self.count, sigma, n, self.device).view(*shape)


def rand_weights(torch, Q, d_in, d_out, rng, dq=True, striped=True):
    w = rng.normal(d_in * d_out, sigma=0.02)
    p = Q.PackedNf4Tensor.quantize(w)
    if dq:
        p = p.with_double_quantization()
    del w
    return Q.Nf4Linear.from_packed(p, d_in, d_out, striped=striped)


def clone_linear(Q, lin):
    """A second device copy of a striped double-quantized layer (same bytes)."""
    return Q.Nf4Linear._from_striped(lin._codes.clone(), lin._scales.clone(), lin._sos.clone(), lin.d_input(),
                                     lin.d_output())


# --------------------------------------------------------------- config 2 --

def bench_gemv(torch, Q, L, args) -> dict:
    d_in, d_out = 4096, 11008
    dev = torch.device("cuda:0")
    g = Rng(torch, 0x4E463458)
    base = rand_weights(torch, Q, d_in, d_out, g)
    nbytes = gemv_bytes(d_in, d_out, dq=True)
    copies = max(2, -(-(2 * MALL_BYTES) // nbytes))  # >= 512 MiB of weights
    layers = [base] + [Q.Nf4Linear.from_packed(base.packed(), d_in, d_out) for _ in range(copies - 1)]
    x = g.normal(1, d_in)
    y = torch.empty(1, d_out, device=dev)
    structs = [lay.weight_struct() for lay in layers]
    lib = L.lib()

    def launch(i: int) -> None:
        st = lib.unifur_nf4_linear_forward(x.data_ptr(), L.F32, 1, ctypes.byref(structs[i % copies]), None, None,
                                           y.data_ptr(), L.F32, None, 0, torch.cuda.current_stream().cuda_stream)
        if st != 0:
            L.check(st)

    # sanity: against torch's f32 matvec of the dequantized weight
    launch(0)
    ref = x @ layers[0].dequantized_weight()
    torch.cuda.synchronize()
    rel = float((y - ref).abs().max() / ref.abs().max())
    if not rel < 1e-4:
        raise RuntimeError(f"GEMV sanity check failed: max rel error {rel:.3e}")
    for i in range(args.warmup):
        launch(i)
    graph = capture(torch, launch, copies)
    steps = args.steps
    torch.cuda.synchronize()
    # exactly `steps` launches, rotating over the copies: one graph of them
    # Each measurement times exactly `steps` launches between two
    # synchronizations, with HIP events recorded on the launch stream right
    # before and after them (the GPU time of the K steps, launch gaps between
    # them included; the host's own launch and wake-up latency around the
    # replay is not a step's -- its wall time is reported beside it).  It is
    # repeated (at least 5 times and ~0.2 s in all) and the median taken, so
    # that a short run (the driver's --steps 20 is ~0.2 ms of GPU work) is not
    # one sample of jitter.
    timed = capture(torch, launch, steps) if graph is not None else None
    samples, walls = [], []
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if timed is not None:
        timed.replay()  # once untimed (graph upload)
        torch.cuda.synchronize()
    while len(samples) < 5 or (sum(walls) < 0.2 and len(samples) < 1000):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record()
        if timed is not None:
            timed.replay()
        else:
            for i in range(steps):
                launch(i)
        ev1.record()
        torch.cuda.synchronize()
        walls.append(time.perf_counter() - t0)
        samples.append(ev0.elapsed_time(ev1) / 1e3)
    if timed is not None:
        del timed
    samples.sort()
    walls.sort()
    elapsed = samples[len(samples) // 2]
    # per-launch kernel time: HIP events on the launch stream around graph
    # replays of the rotating launches (cold), and of one weight (warm)
    cold_ms = replay_event_ms(torch, graph, copies) if graph is not None else event_ms(
        torch, lambda i: launch(i % copies), 4 * copies)
    warm = capture(torch, lambda i: launch(0), copies)
    warm_ms = replay_event_ms(torch, warm, copies) if warm is not None else event_ms(torch, lambda i: launch(0), 4 * copies)
    launch(1)
    torch.cuda.synchronize()
    if not float((y - ref).abs().max() / ref.abs().max()) < 1e-4:
        raise RuntimeError("GEMV result drifted during timing")
    out = {"steps": steps, "elapsed_s": elapsed, "bytes": nbytes, "copies": copies, "repeats": len(samples),
           "value_gbs": nbytes * steps / elapsed / 1e9, "ms_per_step": elapsed * 1e3 / steps,
           "host_wall_ms_per_step": walls[len(walls) // 2] * 1e3 / steps,
           "kernel_cold_ms": cold_ms, "kernel_warm_ms": warm_ms, "graph": graph is not None}
    # bf16 activations (same weight bytes, x half the size)
    xb = x.to(torch.bfloat16)

    def launch_b(i: int) -> None:
        L.check(lib.unifur_nf4_linear_forward(xb.data_ptr(), L.BF16, 1, ctypes.byref(structs[i % copies]), None,
                                              None, y.data_ptr(), L.F32, None, 0,
                                              torch.cuda.current_stream().cuda_stream))
    gb = capture(torch, launch_b, copies)
    out["kernel_cold_ms_bf16x"] = replay_event_ms(torch, gb, copies) if gb is not None else event_ms(
        torch, launch_b, 4 * copies)
    del gb
    # plain f32 block scales (PackedScales::F32, the variant without double
    # quantization): 25,422,848 bytes per launch, rotated cold likewise
    gp = Rng(torch, 0x4E463459)
    base_p = rand_weights(torch, Q, d_in, d_out, gp, dq=False)
    nbytes_p = gemv_bytes(d_in, d_out, dq=False)
    copies_p = max(2, -(-(2 * MALL_BYTES) // nbytes_p))
    layers_p = [base_p] + [Q.Nf4Linear.from_packed(base_p.packed(), d_in, d_out) for _ in range(copies_p - 1)]
    structs_p = [lay.weight_struct() for lay in layers_p]

    def launch_p(i: int) -> None:
        L.check(lib.unifur_nf4_linear_forward(x.data_ptr(), L.F32, 1, ctypes.byref(structs_p[i % copies_p]), None,
                                              None, y.data_ptr(), L.F32, None, 0,
                                              torch.cuda.current_stream().cuda_stream))
    launch_p(0)
    ref_p = x @ layers_p[0].dequantized_weight()
    torch.cuda.synchronize()
    if not float((y - ref_p).abs().max() / ref_p.abs().max()) < 1e-4:
        raise RuntimeError("plain-scale GEMV sanity check failed")
    gpl = capture(torch, launch_p, copies_p)
    plain_ms = replay_event_ms(torch, gpl, copies_p) if gpl is not None else event_ms(torch, launch_p, 4 * copies_p)
    out["plain_scales"] = {"kernel_ms": plain_ms, "bytes": nbytes_p, "copies": copies_p}
    del gpl, layers_p, structs_p
    return out


def bench_gemv_stripes(torch, Q, L) -> dict:
    """The config-2 GEMV (d_in 4096, DQ, f32 x) at d_out of 544, 688, 768 and
    1024 stripes of 16 columns (2.125, 2.69, 3 and 4 workgroups per CU of the
    256; every point past 512 stripes, so all take the 4-wave kernel): the
    fixed and per-stripe cost of a launch, and whether config 2's 2.69
    stripes per CU cost like a whole 3, cold weights, per-launch time by HIP
    events around graph replays."""
    d_in = 4096
    dev = torch.device("cuda:0")
    g = Rng(torch, 0x4E463459)
    lib = L.lib()
    out = {}
    for d_out in (8704, 11008, 12288, 16384):
        base = rand_weights(torch, Q, d_in, d_out, g)
        nbytes = gemv_bytes(d_in, d_out, dq=True)
        copies = max(2, -(-(2 * MALL_BYTES) // nbytes))
        layers = [base] + [Q.Nf4Linear.from_packed(base.packed(), d_in, d_out) for _ in range(copies - 1)]
        structs = [lay.weight_struct() for lay in layers]
        x = g.normal(1, d_in)
        y = torch.empty(1, d_out, device=dev)

        def launch(i: int, structs=structs, x=x, y=y, copies=copies) -> None:
            L.check(lib.unifur_nf4_linear_forward(x.data_ptr(), L.F32, 1, ctypes.byref(structs[i % copies]), None,
                                                  None, y.data_ptr(), L.F32, None, 0,
                                                  torch.cuda.current_stream().cuda_stream))
        for i in range(copies):
            launch(i)
        graph = capture(torch, launch, copies)
        ms = replay_event_ms(torch, graph, copies) if graph is not None else event_ms(torch, launch, 4 * copies)
        stripes = d_out // 16
        out[f"d_out_{d_out}"] = {"stripes": stripes, "stripes_per_cu": round(stripes / 256, 3),
                                 "kernel_us": round(ms * 1e3, 3), "gbs": round(nbytes / ms / 1e6, 1),
                                 "ns_per_stripe": round(ms * 1e6 / stripes, 2)}
        del layers, structs, graph
    # the line through the whole-number points (3 and 4 per CU), and what it
    # predicts below them: a launch paced by its fullest CU would cost the
    # same at 544 and 688 stripes as at 768
    a, b = out["d_out_12288"], out["d_out_16384"]
    slope = (b["kernel_us"] - a["kernel_us"]) / (b["stripes"] - a["stripes"])
    icpt = a["kernel_us"] - slope * a["stripes"]
    out["fit_3_and_4_per_cu"] = {"fixed_us": round(icpt, 3), "ns_per_stripe": round(slope * 1e3, 3),
                                 "marginal_gbs": round(gemv_bytes(d_in, 16 * 1024, dq=True) / 1024 / slope / 1e3, 1),
                                 "predicted_544_us": round(icpt + slope * 544, 3),
                                 "measured_544_us": out["d_out_8704"]["kernel_us"],
                                 "predicted_688_us": round(icpt + slope * 688, 3),
                                 "measured_688_us": out["d_out_11008"]["kernel_us"]}
    return out


# ----------------------------------------------------------- HBM ceiling --

_PROBE = None


def probe_lib():
    """The bench's streaming probes (unifur_amd/bench_probe, built beside the
    library by unifur_amd.build; not part of libunifur_nf4.so)."""
    global _PROBE
    if _PROBE is None:
        from unifur_amd import build as B
        if not os.path.exists(B.PROBE_LIB):
            raise RuntimeError(f"{B.PROBE_LIB} is not built: run python -m unifur_amd.build")
        lib = ctypes.CDLL(B.PROBE_LIB)
        P, U64, U32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32
        lib.unifur_bench_stream_probe.argtypes = [P, U64, P, P, U32, P]
        lib.unifur_bench_stream_mixed.argtypes = [P, P, U64, U32, U32, P]
        _PROBE = lib
    return _PROBE


def _probe_check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(f"stream probe failed with status {rc}")


def bench_ceiling(torch, L, nbytes: int, write_ratio: int = 0) -> dict:
    """What this part streams for buffers of the GEMV's size, timed as the
    GEMV is (graph replay over copies rotated past the Infinity Cache, one
    event pair around the replays): the bench's streaming probe (16-byte
    accesses, grid-stride) as a plain read of nbytes and as a copy of
    nbytes / 2 (nbytes moved), the best over a few grid sizes.  With
    write_ratio R > 0, also a write-dominated stream of nbytes in all:
    nbytes R / (R + 1) written and 1 / (R + 1) of it read (R = 8 is the
    dequantize's mix, 8.9 MB read for 67 MB written at 4096 x 4096)."""
    dev = torch.device("cuda:0")
    nbytes = nbytes // 64 * 64
    copies = max(2, -(-(2 * MALL_BYTES) // nbytes))
    bufs = [torch.ones(nbytes // 4, device=dev) for _ in range(copies)]
    dsts = [torch.empty(nbytes // 4, device=dev) for _ in range(copies)]
    sink = torch.zeros(64, dtype=torch.int32, device=dev)
    lib = probe_lib()
    out = {"bytes": nbytes, "copies": copies, "kernel": "bench_probe/stream_probe.hip"}
    kinds = [("read", nbytes), ("copy", nbytes)]
    if write_ratio:
        unit = 16 * write_ratio * 256  # the probe writes whole 256-unit blocks
        w_bytes = nbytes * write_ratio // (write_ratio + 1) // unit * unit
        kinds.append(("write_dominated", w_bytes + w_bytes // write_ratio))
    for name, moved in kinds:
        best = None
        for grid in (256, 512, 1024, 2048, 4096):
            def fn(i: int, grid=grid, name=name) -> None:
                st = torch.cuda.current_stream().cuda_stream
                if name == "read":
                    _probe_check(lib.unifur_bench_stream_probe(bufs[i % copies].data_ptr(), nbytes, None,
                                                               sink.data_ptr(), grid, st))
                elif name == "copy":
                    _probe_check(lib.unifur_bench_stream_probe(bufs[i % copies].data_ptr(), nbytes // 2,
                                                               dsts[i % copies].data_ptr(), sink.data_ptr(), grid, st))
                else:
                    _probe_check(lib.unifur_bench_stream_mixed(bufs[i % copies].data_ptr(), dsts[i % copies].data_ptr(),
                                                               w_bytes, write_ratio, grid, st))
            gr = capture(torch, fn, copies)
            ms = replay_event_ms(torch, gr, copies) if gr is not None else event_ms(torch, fn, 2 * copies)
            if best is None or ms < best[0]:
                best = (ms, grid)
        out[f"{name}_us"] = round(best[0] * 1e3, 2)
        out[f"{name}_gbs"] = round(moved / best[0] / 1e6, 1)
        out[f"{name}_workgroups"] = best[1]
    if int(sink.count_nonzero()) != 0:
        raise RuntimeError("stream probe sink written: the read was not of the expected data")
    del bufs, dsts
    return out


# --------------------------------------------------------------- config 1 --

def bench_codec(torch, Q, L) -> dict:
    """Config 1 (4096 x 4096 f32): quantize and dequantize kernels."""
    n = 4096 * 4096
    dev = torch.device("cuda:0")
    g = Rng(torch, 0x4E463457)
    copies = 8  # 8 x (64 MiB + 8 MiB) > the Infinity Cache
    vals = [g.normal(n, sigma=0.02) for _ in range(copies)]
    packs = [Q.PackedNf4Tensor.quantize(v) for v in vals]
    outs = [torch.empty(n, device=dev) for _ in range(copies)]
    lib = L.lib()

    def quant(i: int) -> None:
        p = packs[i % copies]
        L.check(lib.unifur_nf4_quantize(vals[i % copies].data_ptr(), n, p.codes.data_ptr(), p.absmax.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream))

    structs = [p.scales_struct() for p in packs]

    def deq(i: int) -> None:
        p = packs[i % copies]
        L.check(lib.unifur_nf4_dequantize(p.codes.data_ptr(), ctypes.byref(structs[i % copies]), n,
                                          outs[i % copies].data_ptr(), L.F32,
                                          torch.cuda.current_stream().cuda_stream))

    gq, gd = capture(torch, quant, copies), capture(torch, deq, copies)
    q_ms = replay_event_ms(torch, gq, copies) if gq is not None else event_ms(torch, quant, 4 * copies)
    d_ms = replay_event_ms(torch, gd, copies) if gd is not None else event_ms(torch, deq, 4 * copies)
    codec_bytes = 4 * n + n // 2 + 4 * (n // 64)  # f32 values + packed codes + f32 absmax
    out = {"quantize_ms": q_ms, "dequant_ms": d_ms, "bytes": codec_bytes,
           "quantize_gbs": codec_bytes / q_ms / 1e6, "dequant_gbs": codec_bytes / d_ms / 1e6}
    del gq, gd
    # the variants: dequantize to bf16 (codes + f32 absmax in, 2 B out per
    # value: 42,991,616 B), double quantization of the block scales, and the
    # dequantize from double-quantized scales (u8 codes + scale of scales)
    outs_b = [torch.empty(n, dtype=torch.bfloat16, device=dev) for _ in range(copies)]

    def deq_b(i: int) -> None:
        p = packs[i % copies]
        L.check(lib.unifur_nf4_dequantize(p.codes.data_ptr(), ctypes.byref(structs[i % copies]), n,
                                          outs_b[i % copies].data_ptr(), L.BF16,
                                          torch.cuda.current_stream().cuda_stream))
    nb = n // 64
    qs = [torch.empty(nb, dtype=torch.uint8, device=dev) for _ in range(copies)]
    sos = [torch.empty(1, device=dev) for _ in range(copies)]

    def dq(i: int) -> None:
        L.check(lib.unifur_nf4_double_quantize(packs[i % copies].absmax.data_ptr(), nb, qs[i % copies].data_ptr(),
                                               sos[i % copies].data_ptr(), torch.cuda.current_stream().cuda_stream))
    for i in range(copies):
        dq(i)
    dq_structs = [L.Scales(L.SCALES_DOUBLE_QUANTIZED, None, qs[i].data_ptr(), sos[i].data_ptr()) for i in range(copies)]

    def deq_dq(i: int) -> None:
        p = packs[i % copies]
        L.check(lib.unifur_nf4_dequantize(p.codes.data_ptr(), ctypes.byref(dq_structs[i % copies]), n,
                                          outs[i % copies].data_ptr(), L.F32,
                                          torch.cuda.current_stream().cuda_stream))
    gdb, gdq, gdd = capture(torch, deq_b, copies), capture(torch, dq, copies), capture(torch, deq_dq, copies)
    out["dequant_bf16_ms"] = replay_event_ms(torch, gdb, copies) if gdb is not None else event_ms(torch, deq_b, 4 * copies)
    out["dequant_bf16_bytes"] = n // 2 + 4 * nb + 2 * n
    out["double_quantize_ms"] = replay_event_ms(torch, gdq, copies) if gdq is not None else event_ms(torch, dq, 4 * copies)
    out["double_quantize_bytes"] = 4 * nb + nb + 4
    out["dequant_dq_ms"] = replay_event_ms(torch, gdd, copies) if gdd is not None else event_ms(torch, deq_dq, 4 * copies)
    out["dequant_dq_bytes"] = n // 2 + nb + 4 + 4 * n
    return out


# --------------------------------------------------------------- config 3 --

def bench_gemm(torch, Q, L) -> dict:
    """Config 3: X bf16 [2048, 4096] . NF4 W [4096, 4096] + LoRA r 16 (scale 2), bf16 Y."""
    M, K, N, r = 2048, 4096, 4096, 16
    dev = torch.device("cuda:0")
    g = Rng(torch, 0x4E463457 + 3)
    lin = rand_weights(torch, Q, K, N, g)
    x = g.normal(M, K).to(torch.bfloat16)
    a = g.normal(K, r, sigma=0.01)
    b = g.normal(r, N, sigma=0.01)
    ql = Q.QloraLinear(lin, Q.LoraAdapter.from_parts(a, b, 2.0))
    y = ql.forward(x)
    ref = (x.float() @ lin.dequantized_weight()) + (x.float() @ a) @ b * 2.0
    err = float((y.float() - ref).abs().max() / ref.abs().max())
    if not err < 1e-2:
        raise RuntimeError(f"GEMM sanity check failed: {err:.3e}")
    flops = 2 * M * N * K + 2 * M * K * r + 2 * M * r * N
    w = lin.weight_struct()
    lo = ql.adapter.struct()
    lib = L.lib()
    ws_bytes = lib.unifur_nf4_linear_workspace_size(M, K, N, L.BF16, r)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)

    def launch(i: int) -> None:
        L.check(lib.unifur_nf4_qlora_forward(x.data_ptr(), L.BF16, M, ctypes.byref(w), ctypes.byref(lo), y.data_ptr(),
                                             L.BF16, ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream))

    for i in range(3):
        launch(i)
    graph = capture(torch, launch, 8)
    ms = steady_ms(torch, graph, 8) if graph is not None else event_ms(torch, launch, 16)
    # the base GEMM kernel alone (no LoRA: one launch)
    ybase = torch.empty(M, N, dtype=torch.bfloat16, device=dev)

    def base(i: int) -> None:
        L.check(lib.unifur_nf4_linear_forward(x.data_ptr(), L.BF16, M, ctypes.byref(w), None, None, ybase.data_ptr(),
                                              L.BF16, None, 0, torch.cuda.current_stream().cuda_stream))
    gbase = capture(torch, base, 8)
    base_ms = steady_ms(torch, gbase, 8) if gbase is not None else event_ms(torch, base, 16)
    base_flops = 2 * M * N * K
    # the fused kernel (NF4 tiles dequantized on chip, LoRA in the epilogue):
    # what the least workspace selects, with the adapter and without
    fused = {}
    for name, lo_ in (("qlora", lo), ("base", None)):
        rank = r if lo_ is not None else 0
        lean = lib.unifur_nf4_linear_min_workspace_size(M, K, N, L.BF16, rank)
        wl = torch.zeros(lean, dtype=torch.uint8, device=dev)
        yf = torch.empty(M, N, dtype=torch.bfloat16, device=dev)

        def fused_launch(i: int, lo_=lo_, wl=wl, lean=lean, yf=yf) -> None:
            L.check(lib.unifur_nf4_linear_forward(x.data_ptr(), L.BF16, M, ctypes.byref(w), None,
                                                  ctypes.byref(lo_) if lo_ is not None else None, yf.data_ptr(),
                                                  L.BF16, wl.data_ptr(), lean, torch.cuda.current_stream().cuda_stream))
        fused_launch(0)
        torch.cuda.synchronize()
        if name == "qlora":
            ferr = float((yf.float() - ref).abs().max() / ref.abs().max())
            if not ferr < 1e-2:
                raise RuntimeError(f"fused GEMM sanity check failed: {ferr:.3e}")
        gf = capture(torch, fused_launch, 8)
        f_ms = steady_ms(torch, gf, 8) if gf is not None else event_ms(torch, fused_launch, 16)
        f_flops = flops if name == "qlora" else base_flops
        fused[name] = {"ms": round(f_ms, 5), "tflops": round(f_flops / f_ms / 1e9, 1),
                       "frac": round(f_flops / f_ms / 1e9 / BF16_PEAK_TFLOPS, 4)}
    # f32 activations at the same shapes (the reference's precision): the f32
    # MFMA kernel over NF4 tiles dequantized exactly in LDS, with the adapter,
    # and the backward's dX for f32 dY through its transposed form
    x32 = x.float()
    y32 = torch.empty(M, N, device=dev)
    ws32 = lib.unifur_nf4_linear_workspace_size(M, K, N, L.F32, r)
    w32 = torch.zeros(max(ws32, 1), dtype=torch.uint8, device=dev)

    def f32_launch(i: int) -> None:
        L.check(lib.unifur_nf4_qlora_forward(x32.data_ptr(), L.F32, M, ctypes.byref(w), ctypes.byref(lo),
                                             y32.data_ptr(), L.F32, w32.data_ptr(), ws32,
                                             torch.cuda.current_stream().cuda_stream))
    f32_launch(0)
    torch.cuda.synchronize()
    e32 = float((y32 - ref).abs().max() / ref.abs().max())
    if not e32 < 1e-3:
        raise RuntimeError(f"f32 GEMM sanity check failed: {e32:.3e}")
    g32 = capture(torch, f32_launch, 4)
    ms32 = steady_ms(torch, g32, 4, reps=5) if g32 is not None else event_ms(torch, f32_launch, 8)
    dy32 = g.normal(M, N)
    dx32 = torch.empty(M, K, device=dev)
    wsb = lib.unifur_nf4_linear_backward_workspace_size(M, K, N, L.F32, 0)
    wb = torch.zeros(max(wsb, 1), dtype=torch.uint8, device=dev)

    def dx_launch(i: int) -> None:
        L.check(lib.unifur_nf4_linear_backward(dy32.data_ptr(), L.F32, M, ctypes.byref(w), None, None, L.F32,
                                               dx32.data_ptr(), L.F32, None, None, wb.data_ptr(), wsb,
                                               torch.cuda.current_stream().cuda_stream))
    dx_launch(0)
    gdx = capture(torch, dx_launch, 4)
    msdx = steady_ms(torch, gdx, 4, reps=5) if gdx is not None else event_ms(torch, dx_launch, 8)
    f32 = {"path": "f32 MFMA (v_mfma_f32_32x32x2f32) over NF4 tiles dequantized exactly in LDS",
           "qlora_ms": round(ms32, 5), "qlora_tflops": round(flops / ms32 / 1e9, 1),
           "frac_of_f32_mfma_peak": round(flops / ms32 / 1e9 / F32_MFMA_PEAK_TFLOPS, 4),
           "backward_dx_ms": round(msdx, 5), "backward_dx_tflops": round(base_flops / msdx / 1e9, 1),
           "max_rel_err": e32}
    return {"ms": ms, "tflops": flops / ms / 1e9, "frac": flops / ms / 1e9 / BF16_PEAK_TFLOPS,
            "base_kernel_ms": base_ms, "base_tflops": base_flops / base_ms / 1e9, "max_rel_err": err,
            "fused": fused, "f32": f32}


# --------------------------------------------------------------- config 4 --

def bench_swiglu(torch, Q, L, tokens) -> dict:
    hidden, inter = 4096, 11008
    dev = torch.device("cuda:0")
    g = Rng(torch, 0x4E463457 + 4)
    wbytes = 2 * gemv_bytes(hidden, inter, True, 0, 0) + gemv_bytes(inter, hidden, True, 0, 0)
    # rotate >= 512 MiB of packed weights (twice the 256 MiB Infinity Cache):
    # 8 blocks of 69.7 MB, so every step streams its weights from HBM
    copies = max(2, -(-(2 * MALL_BYTES) // wbytes))
    base = [rand_weights(torch, Q, hidden, inter, g), rand_weights(torch, Q, hidden, inter, g),
            rand_weights(torch, Q, inter, hidden, g)]
    blocks = [Q.QwenMlp(*base)] + [Q.QwenMlp(*[clone_linear(Q, w) for w in base]) for _ in range(copies - 1)]
    out = {}
    for T in tokens:
        x = g.normal(T, hidden).to(torch.bfloat16)
        ys = [None] * copies

        def run(i: int) -> None:
            ys[i % copies] = blocks[i % copies].forward(x)

        for i in range(copies):
            run(i)
        graph = capture(torch, run, copies)
        ms = steady_ms(torch, graph, copies) if graph is not None else event_ms(torch, run, 2 * copies)
        flops = T * 270_532_608
        out[f"T{T}"] = {"ms": round(ms, 5), "weight_gbs": round(wbytes / ms / 1e6, 1),
                        "tflops": round(flops / ms / 1e9, 2)}
    # T = 512 (like every prefill batch up to 512 rows) takes the fused MFMA
    # kernels by default -- no expanded weight copies: gate and up in one
    # pair launch storing silu(g) * u (344 output tiles over whole d_in),
    # then down with its 64 output tiles splitting d_in four ways (split-K).
    # The least workspace the library reports (sized for gate and up of
    # different scale kinds) holds this same plan.
    if "T512" in out:
        out["T512"]["path"] = "fused MFMA kernels: gate/up pair launch + down, split-K (default workspace)"
    out["rotation"] = f"{copies} blocks of {wbytes} B rotated (cold HBM)"
    return out


# --------------------------------------------------------------- config 5 --

QWEN_PROJ = [("q", 896, 896), ("k", 896, 128), ("v", 896, 128), ("o", 896, 896),
             ("gate", 896, 4864), ("up", 896, 4864), ("down", 4864, 896)]


def bench_qwen(torch, Q, L, layers: int = 24) -> dict:
    dev = torch.device("cuda:0")
    g = Rng(torch, 0x4E463457 + 5)
    # whole-model quantize pass: quantize + double-quantize + stripe, 168 weights
    vals = [(g.normal(di * do, sigma=0.02), di, do)
            for _ in range(layers) for (_, di, do) in QWEN_PROJ]
    torch.cuda.synchronize()

    def quantize_all():  # the grouped pass: three launches per 48 weights
        return Q.quantize_linears(vals)

    def quantize_each():  # Nf4Linear::from_values per weight, as the reference's loop
        return [Q.Nf4Linear.from_values(v, di, do) for (v, di, do) in vals]

    def best_of_three(fn):
        # steady state: the best of three passes (the pass right after the
        # warm-up one regrows the allocator's cache and runs several times slower)
        fn()  # warm
        best, res = float("inf"), None
        for _ in range(3):
            res = None
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            res = fn()
            torch.cuda.synchronize()
            best = min(best, time.perf_counter() - t0)
        return best, res

    q_each_s, _ = best_of_three(quantize_each)
    q_s, lins = best_of_three(quantize_all)
    # the grouped pass's kernels alone: its launches timed with HIP events
    q_kernel_ms = event_ms(torch, lambda i: Q.quantize_linears(vals), 3)
    params = sum(di * do for (_, di, do) in vals)
    q_bytes = 4 * params + params // 2 + 4 * (params // 64)  # f32 in, codes + f32 absmax out (config 5 unit)
    # the same pass from bf16 checkpoint tensors as they lie ([out, in], PyTorch
    # order: qwen_linear's input), transposed inside the quantize kernel
    ckpt = [v.view(di, do).t().contiguous().to(torch.bfloat16) for (v, di, do) in vals]
    del vals
    torch.cuda.synchronize()
    c_s, _ = best_of_three(lambda: Q.quantize_checkpoint_linears(ckpt))
    c_kernel_ms = event_ms(torch, lambda i: Q.quantize_checkpoint_linears(ckpt), 3)
    c_bytes = 2 * params + params // 2 + 4 * (params // 64)  # bf16 in
    del ckpt
    out = {"quantize_pass_ms": round(q_s * 1e3, 3), "quantize_pass_gbs": round(q_bytes / q_s / 1e9, 1),
           "quantize_pass_per_weight_ms": round(q_each_s * 1e3, 3), "quantize_pass_events_ms": round(q_kernel_ms, 3),
           "quantize_pass_bf16_checkpoint_ms": round(c_s * 1e3, 3),
           "quantize_pass_bf16_checkpoint_events_ms": round(c_kernel_ms, 3),
           "quantize_pass_bf16_checkpoint_gbs": round(c_bytes / c_s / 1e9, 1),
           "params": params}
    wbytes = sum(gemv_bytes(lin.d_input(), lin.d_output(), True, 0, 0) for lin in lins)
    # the 184.5 MB model fits the 256 MiB Infinity Cache: rotate model copies
    # (>= 512 MiB in all) so that every token step reads its weights from HBM
    mcopies = max(2, -(-(2 * MALL_BYTES) // wbytes))
    models = [lins] + [[clone_linear(Q, lin) for lin in lins] for _ in range(mcopies - 1)]
    # batch 1 in f32 (the reference's precision), batch 32 in bf16 and in f32
    for b, xdt, tag in ((1, torch.float32, "b1"), (32, torch.bfloat16, "b32"), (32, torch.float32, "b32_f32")):
        xs = {di: g.normal(b, di).to(xdt) for (_, di, _) in QWEN_PROJ}

        def step(i: int) -> None:
            for lin in models[i % mcopies]:
                lin.forward(xs[lin.d_input()])

        step(0)
        graph = capture(torch, step, mcopies)
        ms = steady_ms(torch, graph, mcopies) if graph is not None else event_ms(torch, step, 2 * mcopies)
        out[f"decode_{tag}"] = {"ms_per_token_step": round(ms, 4), "weight_gbs": round(wbytes / ms / 1e6, 1),
                                "tokens_per_s": round(b / ms * 1e3, 1)}

        # the same weights as a decoder layer drives them: q, k, v in one
        # shared-input launch, o, and the SwiGLU block (gate/up pair + down)
        layer_sets = [[(m[7 * l:7 * l + 3], m[7 * l + 3], Q.QwenMlp(*m[7 * l + 4:7 * l + 7])) for l in range(layers)]
                      for m in models]

        def layer_step(i: int) -> None:
            for qkv, o, mlp in layer_sets[i % mcopies]:
                Q.forward_shared_input(xs[896], qkv)
                o.forward(xs[896])
                mlp.forward(xs[896])

        layer_step(0)
        graph = capture(torch, layer_step, mcopies)
        ms = steady_ms(torch, graph, mcopies) if graph is not None else event_ms(torch, layer_step, 2 * mcopies)
        out[f"decode_{tag}_layer_launches"] = {"ms_per_token_step": round(ms, 4),
                                              "weight_gbs": round(wbytes / ms / 1e6, 1),
                                              "tokens_per_s": round(b / ms * 1e3, 1), "launches": 4 * layers}

        # QwenDecoderLayer::step's NF4 chain through the two stage entry
        # points per layer (input norm + q/k/v; o + residual, post norm +
        # SwiGLU + residual), each layer's output feeding the next; q stands
        # in for the attention output (the attention itself is not on the NF4
        # path and is not timed)
        norms = [(g.normal(896, sigma=0.1), g.normal(896, sigma=0.1))
                 for _ in range(layers)]
        from unifur_amd import qwennet as N
        dec_sets = [[N.QwenDecoderLayer(*m[7 * l:7 * l + 4], Q.QwenMlp(*m[7 * l + 4:7 * l + 7]), *norms[l], 1e-6)
                     for l in range(layers)] for m in models]
        x0 = xs[896]

        def decoder_step(i: int) -> None:
            h = x0
            for lay in dec_sets[i % mcopies]:
                q, _, _ = lay.project(h)
                h = lay.attn_out_mlp(h, q)

        decoder_step(0)
        graph = capture(torch, decoder_step, mcopies)
        ms = steady_ms(torch, graph, mcopies) if graph is not None else event_ms(torch, decoder_step, 2 * mcopies)
        out[f"decode_{tag}_decoder_stages"] = {"ms_per_token_step": round(ms, 4),
                                              "weight_gbs": round(wbytes / ms / 1e6, 1),
                                              "tokens_per_s": round(b / ms * 1e3, 1),
                                              "calls_per_layer": 2,
                                              "activations": "f32" if xdt == torch.float32 else "bf16"}
    out["weight_bytes"] = wbytes
    out["rotation"] = f"{mcopies} model copies of {wbytes} B rotated (cold HBM)"
    return out


# ------------------------------------------------------- next: backward ----

def bench_backward(torch, Q, L) -> dict:
    """Adapter-only training step of one config-3 layer in reverse: dy bf16
    [2048, 4096] through the 4096 x 4096 DQ weight with the r = 16 adapter:
    dx (bf16) and both adapter gradients (f32)."""
    M, K, N, r = 2048, 4096, 4096, 16
    dev = torch.device("cuda:0")
    g = Rng(torch, 0x4E463457 + 7)
    lin = rand_weights(torch, Q, K, N, g)
    x = g.normal(M, K).to(torch.bfloat16)
    dy = g.normal(M, N).to(torch.bfloat16)
    a = g.normal(K, r, sigma=0.01)
    b = g.normal(r, N, sigma=0.01)
    ql = Q.QloraLinear(lin, Q.LoraAdapter.from_parts(a, b, 2.0))
    lib = L.lib()
    ws_bytes = lib.unifur_nf4_linear_backward_workspace_size(M, K, N, L.BF16, r)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
    dx = torch.empty(M, K, dtype=torch.bfloat16, device=dev)
    ga = torch.empty(K, r, device=dev)
    gb = torch.empty(r, N, device=dev)
    w, lo = lin.weight_struct(), ql.adapter.struct()

    def step(i: int) -> None:
        L.check(lib.unifur_nf4_linear_backward(dy.data_ptr(), L.BF16, M, ctypes.byref(w), ctypes.byref(lo),
                                               x.data_ptr(), L.BF16, dx.data_ptr(), L.BF16, ga.data_ptr(),
                                               gb.data_ptr(), ws.data_ptr(), ws_bytes,
                                               torch.cuda.current_stream().cuda_stream))

    def grads_only(i: int) -> None:
        L.check(lib.unifur_nf4_linear_backward(dy.data_ptr(), L.BF16, M, ctypes.byref(w), ctypes.byref(lo),
                                               x.data_ptr(), L.BF16, None, L.BF16, ga.data_ptr(),
                                               gb.data_ptr(), ws.data_ptr(), ws_bytes,
                                               torch.cuda.current_stream().cuda_stream))

    # the same step with the least workspace: dx through the fused NF4 kernel
    # over W's rows (no expanded weight, no BLAS call)
    lean_bytes = lib.unifur_nf4_linear_backward_min_workspace_size(M, K, N, L.BF16, r, L.LAYOUT_STRIPED)
    lean = torch.zeros(lean_bytes, dtype=torch.uint8, device=dev)

    def step_lean(i: int) -> None:
        L.check(lib.unifur_nf4_linear_backward(dy.data_ptr(), L.BF16, M, ctypes.byref(w), ctypes.byref(lo),
                                               x.data_ptr(), L.BF16, dx.data_ptr(), L.BF16, ga.data_ptr(),
                                               gb.data_ptr(), lean.data_ptr(), lean_bytes,
                                               torch.cuda.current_stream().cuda_stream))

    res = {}
    for name, fn in (("ms", step), ("grads_only_ms", grads_only), ("lean_ms", step_lean)):
        for i in range(3):
            fn(i)
        graph = capture(torch, fn, 4)
        res[name] = steady_ms(torch, graph, 4) if graph is not None else event_ms(torch, fn, 8)
    ms = res["ms"]
    flops = 2 * M * N * K + 2 * K * r * N + 4 * M * r * (K + N)
    # the adapter gradients read x and dy twice each (bf16)
    grads_bytes = 2 * 2 * M * (K + N)
    return {"ms": round(ms, 5), "tflops": round(flops / ms / 1e9, 1),
            "frac": round(flops / ms / 1e9 / BF16_PEAK_TFLOPS, 4),
            "grads_only_ms": round(res["grads_only_ms"], 5),
            "grads_only_gbs": round(grads_bytes / res["grads_only_ms"] / 1e6, 1),
            "fused_dx": {"ms": round(res["lean_ms"], 5), "tflops": round(flops / res["lean_ms"] / 1e9, 1),
                         "workspace_bytes": lean_bytes, "default_workspace_bytes": ws_bytes,
                         "path": "least workspace: dx through the fused NF4 MFMA kernel over W's rows"}}


# ------------------------------------------------------ next: embedding ----

def bench_embedding(torch, Q, L) -> dict:
    """Nf4Embedding::forward on the Qwen2-0.5B vocabulary table (151936 x 896,
    double quantized): the gather-dequantize of 32 and 2048 token ids against
    the reference's sequence, a whole-table dequantize per forward
    (src/qwennet.rs:279-290) timed with the same dequantize kernel."""
    from unifur_amd import qwennet as QN
    n_emb, d = 151936, 896
    dev = torch.device("cuda:0")
    rng = Rng(torch, 0x4E463457 + 6)
    g = torch.Generator(device=dev)  # token ids
    g.manual_seed(0x4E463457 + 6)
    emb = QN.Nf4Embedding.from_values(rng.normal(n_emb * d, sigma=0.02), n_emb, d)
    out = {"table": f"{n_emb}x{d}", "resident_bytes": emb.resident_bytes()}
    for t in (32, 2048):
        ids = torch.randint(0, n_emb, (t,), device=dev, generator=g)
        rows = torch.empty(t, d, device=dev)
        s = emb.packed.scales_struct()

        def gather(i: int) -> None:
            L.check(L.lib().unifur_nf4_embedding_forward(
                emb.packed.codes.data_ptr(), ctypes.byref(s), n_emb, d, ids.data_ptr(), L.IDS_I64, t,
                rows.data_ptr(), L.F32, torch.cuda.current_stream().cuda_stream))

        gather(0)
        graph = capture(torch, gather, 16)
        ms = steady_ms(torch, graph, 16) if graph is not None else event_ms(torch, gather, 16)
        moved = t * (d // 2 + d // 64 + 4 * d) + 8 * t
        out[f"gather_T{t}_us"] = round(ms * 1e3, 2)
        out[f"gather_T{t}_gbs"] = round(moved / ms / 1e6, 1)
    full = torch.empty(n_emb * d, device=dev)
    sf = emb.packed.scales_struct()

    def whole(i: int) -> None:
        L.check(L.lib().unifur_nf4_dequantize(emb.packed.codes.data_ptr(), ctypes.byref(sf), n_emb * d,
                                              full.data_ptr(), L.F32, torch.cuda.current_stream().cuda_stream))

    whole(0)
    out["whole_table_dequantize_us"] = round(event_ms(torch, whole, 5) * 1e3, 1)
    return out


# ------------------------------------------------------------- CPU baseline --

def cpu_baseline(sample_s: float) -> dict:
    """The reference's CPU path restated (oracle): serial dequantize of the
    whole weight, then an f32 matmul on all host cores, timed on the config-2
    GEMV for about `sample_s` seconds."""
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
    # the same step with the matmul on one thread too (the dequantize already is)
    t0 = time.perf_counter()
    w = O.dequantize_packed(packed, v.size, None, q, sos)
    O.linear_f32(x, w, d_in, d_out, threads=1)
    dt1 = time.perf_counter() - t0
    return {"value": round(gemv_bytes(d_in, d_out, dq=True) / dt / 1e9, 4), "unit": "GB/s", "cores": threads,
            "value_one_thread": round(gemv_bytes(d_in, d_out, dq=True) / dt1 / 1e9, 4),
            "cpu_model": cpu_model(), "kind": "port",
            "sample": f"{iters} x config-2 GEMV (1-thread dequantize of the 4096x11008 DQ weight + {threads}-thread "
                      f"f32 GEMV), {dt * 1e3:.1f} ms each; oracle/nf4_oracle.c restatement of "
                      f"PackedNf4Tensor::dequantize + burn linear"}


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it: model name, vendor, family /
    model / stepping, and the logical CPUs this process may use."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" not in line:
                    if fields:
                        break  # the first processor's block is enough
                    continue
                k, v = (t.strip() for t in line.split(":", 1))
                fields.setdefault(k, v)
    except OSError:
        return "unknown"
    name = fields.get("model name", "unknown")
    ident = ", ".join(f"{k} {fields[k]}" for k in ("vendor_id", "cpu family", "model", "stepping") if k in fields)
    return f"{name} ({ident}; {len(os.sched_getaffinity(0))} logical CPUs usable)"


def cpu_beside() -> dict:
    """The reference's CPU path (the oracle's restatement) beside the GPU
    figures of configs 1 and 3, on this host: quantize and dequantize of the
    4096 x 4096 config-1 tensor on one thread (the reference's loops are
    serial), and the config-3 QLoRA layer as the reference runs it --
    serial dequantize, then an all-core f32 matmul plus the adapter -- with
    the oracle's row loop (a 32-row sample of X, scaled to the 2048 rows) and
    with a blocked sgemm of the matrixmultiply scheme (all 2048 rows)."""
    from oracle import oracle as O
    threads = len(os.sched_getaffinity(0))
    out = {"cores": threads, "cpu_model": cpu_model()}
    n = 4096 * 4096
    v = O.fill_normal(0x4E463458, 0.02, n)
    t0 = time.perf_counter()
    packed, absmax = O.quantize_packed(v)
    tq = time.perf_counter() - t0
    t0 = time.perf_counter()
    w = O.dequantize_packed(packed, n, absmax)
    td = time.perf_counter() - t0
    unit = 76_546_048  # config-1 bytes (read + write) of either direction
    out["quantize_config1"] = {"s": round(tq, 4), "gbs": round(unit / tq / 1e9, 3), "threads": 1}
    out["dequantize_config1"] = {"s": round(td, 4), "gbs": round(unit / td / 1e9, 3), "threads": 1}
    M, K, N, r, rows = 2048, 4096, 4096, 16, 32
    x = O.fill_normal(0x5A, 1.0, rows * K).reshape(rows, K)
    a = O.fill_normal(0x41, 0.01, K * r).reshape(K, r)
    b = O.fill_normal(0x42, 0.01, r * N).reshape(r, N)
    t0 = time.perf_counter()
    O.dequantize_packed(packed, n, absmax)                           # per forward, serial
    t1 = time.perf_counter()
    t_deq = t1 - t0
    O.linear_f32(x, w, K, N, threads=threads)                        # base, all cores
    xa = O.linear_f32(x, a, K, r, threads=threads)                   # adapter: (x A) B * scaling
    O.linear_f32(xa, b, r, N, threads=threads)
    t2 = time.perf_counter()
    total = (t1 - t0) + (t2 - t1) * (M / rows)
    flops = 2 * M * N * K + 2 * M * K * r + 2 * M * r * N
    out["qlora_gemm_config3"] = {"s": round(total, 3), "tflops": round(flops / total / 1e12, 5),
                                 "sample": f"{rows} of {M} rows timed, scaled", "threads": threads,
                                 "gemm": "the oracle's OpenMP row loop (oracle/nf4_oracle.c nf4o_linear_f32), "
                                         "not cache-blocked like matrixmultiply's sgemm"}
    # the same layer with a blocked f32 GEMM (oracle/cpu_sgemm.c: the packed
    # Goto/BLIS scheme of the matrixmultiply crate burn-ndarray runs on),
    # all 2048 rows timed
    xf = O.fill_normal(0x5A, 1.0, M * K).reshape(M, K)
    w2 = w.reshape(K, N)
    t0 = time.perf_counter()
    O.dequantize_packed(packed, n, absmax)                           # per forward, serial
    O.sgemm_blocked(xf, w2, threads)
    O.sgemm_blocked(O.sgemm_blocked(xf, a, threads), b, threads)
    total_b = time.perf_counter() - t0
    out["qlora_gemm_config3_blocked"] = {
        "s": round(total_b, 3), "tflops": round(flops / total_b / 1e12, 5),
        "sample": f"all {M} rows; serial dequantize as above", "threads": threads,
        "gemm": "oracle/cpu_sgemm.c: cache-blocked packed sgemm, 6x16 AVX2/FMA register tile "
                "(the scheme of matrixmultiply 0.3.x)"}
    del xf
    # the matmuls on one thread (a 4-row sample, scaled)
    rows1 = 4
    t0 = time.perf_counter()
    O.linear_f32(x[:rows1], w, K, N, threads=1)
    xa1 = O.linear_f32(x[:rows1], a, K, r, threads=1)
    O.linear_f32(xa1, b, r, N, threads=1)
    t2 = time.perf_counter()
    total1 = t_deq + (t2 - t0) * (M / rows1)
    out["qlora_gemm_config3_one_thread"] = {"s": round(total1, 3), "tflops": round(flops / total1 / 1e12, 5),
                                            "sample": f"{rows1} of {M} rows timed, scaled; dequantize as above",
                                            "threads": 1}
    return out


def read_traffic():
    """HBM bytes per GEMV launch from the committed rocprofv3 PMC summary."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


PARTS = {
    "gemm": lambda torch, Q, L: bench_gemm(torch, Q, L),
    "swiglu": lambda torch, Q, L: bench_swiglu(torch, Q, L, (1, 16, 512)),
    "qwen": lambda torch, Q, L: bench_qwen(torch, Q, L),
    "embedding": lambda torch, Q, L: bench_embedding(torch, Q, L),
    "backward": lambda torch, Q, L: bench_backward(torch, Q, L),
    "ceiling": lambda torch, Q, L: {f"{mib}MiB": bench_ceiling(torch, L, mib << 20) for mib in (22, 69, 256)},
    "gemv_stripes": lambda torch, Q, L: bench_gemv_stripes(torch, Q, L),
}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4800)
    ap.add_argument("--warmup", type=int, default=96)
    ap.add_argument("--cpu-sample-s", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--quick", action="store_true", help="headline GEMV and codec only")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 20 device copies of 256 MiB (the reference kernel for scaling HBM byte counters)")
    ap.add_argument("--parts", nargs="+", choices=sorted(PARTS),
                    help="only these secondary workloads, one JSON object of their figures (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(every kernel runs on one GPU's share of a layer); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    from unifur_amd import _lib as L
    from unifur_amd import quantize as Q

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    if args.copy_calibration:
        # a plain copy of known size: 256 MiB read + 256 MiB written per launch
        a = torch.ones(64 << 20, device="cuda")
        b = torch.empty_like(a)
        for _ in range(20):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": a.numel() * 4, "copy_calibration_bytes_written": b.numel() * 4,
                          "launches": 20}))
        return 0
    L.lib()
    if args.parts:
        print(json.dumps({name: PARTS[name](torch, Q, L) for name in args.parts}))
        return 0
    gemv = bench_gemv(torch, Q, L, args)
    ceiling = bench_ceiling(torch, L, gemv["bytes"])
    codec = bench_codec(torch, Q, L)
    ceiling1 = bench_ceiling(torch, L, codec["bytes"], write_ratio=8)
    secondary = {
        "hbm_ceiling_gemv_size": ceiling,
        "hbm_ceiling_config1_size": ceiling1,
        "gemv_warm": {"kernel_ms": round(gemv["kernel_warm_ms"], 5),
                      "gbs": round(gemv["bytes"] / gemv["kernel_warm_ms"] / 1e6, 1)},
        "gemv_bf16_activations_cold": {
            "kernel_ms": round(gemv["kernel_cold_ms_bf16x"], 5),
            "gbs": round(gemv_bytes(4096, 11008, True, 2, 4) / gemv["kernel_cold_ms_bf16x"] / 1e6, 1)},
        "gemv_plain_scales_cold": {
            "kernel_ms": round(gemv["plain_scales"]["kernel_ms"], 5), "bytes": gemv["plain_scales"]["bytes"],
            "gbs": round(gemv["plain_scales"]["bytes"] / gemv["plain_scales"]["kernel_ms"] / 1e6, 1),
            "frac": round(gemv["plain_scales"]["bytes"] / gemv["plain_scales"]["kernel_ms"] / 1e6 / HBM_PEAK_GBS, 4)},
        "dequantize_bf16_config1": {
            "kernel_ms": round(codec["dequant_bf16_ms"], 5), "bytes": codec["dequant_bf16_bytes"],
            "gbs": round(codec["dequant_bf16_bytes"] / codec["dequant_bf16_ms"] / 1e6, 1)},
        "dequantize_f32_double_quantized_config1": {
            "kernel_ms": round(codec["dequant_dq_ms"], 5), "bytes": codec["dequant_dq_bytes"],
            "gbs": round(codec["dequant_dq_bytes"] / codec["dequant_dq_ms"] / 1e6, 1)},
        "double_quantize_config1": {"kernel_ms": round(codec["double_quantize_ms"], 5),
                                    "bytes": codec["double_quantize_bytes"]},
        "dequantize_f32_config1": {"kernel_ms": round(codec["dequant_ms"], 5), "gbs": round(codec["dequant_gbs"], 1),
                                   "frac": round(codec["dequant_gbs"] / HBM_PEAK_GBS, 4),
                                   "frac_of_write_dominated_ceiling":
                                       round(codec["dequant_gbs"] / ceiling1["write_dominated_gbs"], 4)},
        "quantize_config1": {"kernel_ms": round(codec["quantize_ms"], 5), "gbs": round(codec["quantize_gbs"], 1),
                             "frac": round(codec["quantize_gbs"] / HBM_PEAK_GBS, 4),
                             "frac_of_read_ceiling": round(codec["quantize_gbs"] / ceiling1["read_gbs"], 4)},
    }
    if not args.quick:
        gemm = bench_gemm(torch, Q, L)
        secondary["prefill_qlora_gemm_config3"] = {
            "path": "default workspace: W (+ s A B) expanded to bf16, then hipBLASLt",
            "ms": round(gemm["ms"], 5), "tflops": round(gemm["tflops"], 1), "frac": round(gemm["frac"], 4),
            "base_gemm_kernel_ms": round(gemm["base_kernel_ms"], 5), "base_tflops": round(gemm["base_tflops"], 1),
            "max_rel_err": gemm["max_rel_err"]}
        secondary["prefill_fused_gemm_config3"] = dict(
            path="least workspace: the fused MFMA kernel (NF4 tiles dequantized in LDS, LoRA in the epilogue)",
            **gemm["fused"])
        secondary["prefill_f32_activations_config3_shapes"] = gemm["f32"]
        secondary["swiglu_config4"] = bench_swiglu(torch, Q, L, (1, 16, 512))
        secondary["qwen05b_config5"] = bench_qwen(torch, Q, L)
        secondary["embedding_qwen05b"] = bench_embedding(torch, Q, L)
        secondary["qlora_backward_config3"] = bench_backward(torch, Q, L)
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_sample_s)
    if not args.no_cpu and not args.quick:
        secondary["cpu_port_beside"] = cpu_beside()

    achieved = gemv["bytes"] / gemv["kernel_cold_ms"] / 1e6
    line = {
        "metric": METRIC,
        "value": round(gemv["value_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": gemv["steps"],
        "steps_requested": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gemv["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "config 2: NF4 decode GEMV x[1x4096] f32 . W[4096x11008] (Wt of the logical 11008x4096), "
                        "block 64, double-quantized scales, y f32; weight held striped; "
                        f"{gemv['copies']} weight copies rotated (cold HBM)",
            "timing": ("HIP-graph replay of the launches" if gemv["graph"] else "eager launches") +
                      f"; median of {gemv['repeats']} runs of exactly {gemv['steps']} steps, each between two "
                      "synchronizations and timed by HIP events on the launch stream "
                      f"(host wall time {gemv['host_wall_ms_per_step'] * 1e3:.3f} us per step)",
            "d_in": 4096, "d_out": 11008, "rows": 1, "block_size": 64, "double_quantized": True,
            "bytes_per_step": gemv["bytes"],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "gemv_striped_kernel<1,4,2,f32,dq,·,·,2>",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": read_traffic(),
            "frac_of_measured_read": round(achieved / ceiling["read_gbs"], 4),
            "measured_read_gbs": ceiling["read_gbs"],
        },
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
