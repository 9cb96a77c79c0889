"""The library's calls captured in a HIP graph replay to the eager result.

bench.py times the prefill, SwiGLU, backward and decode paths from graph
replays, so each path here is captured once (after an eager call that sizes
the workspaces and picks the BLAS kernels), replayed several times with
eager work and synchronizations between the replays, and every replay is
compared with the eager result bit for bit: a captured memset node or any
state that only the first replay sees would show up as a mismatch.
"""
from __future__ import annotations

import pytest
import torch

from unifur_amd import quantize as Q

from test_gpu_gemm import lora_parts
from test_gpu_linear import acts, make_linear

pytestmark = pytest.mark.gpu


def replay_matches(fn, outs_fn, reps=4):
    """fn() launches the work (outputs written in place); outs_fn() returns
    the output tensors.  Eager first, then capture and replay."""
    fn()
    torch.cuda.synchronize()
    want = [o.clone() for o in outs_fn()]
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # the capture stream's own eager call (workspace sized outside capture)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(reps):
        for o in outs_fn():
            o.fill_(float("nan"))  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, w in zip(outs_fn(), want):
            assert torch.equal(o, w), "graph replay differs from the eager result"


def test_prefill_qlora_replays(device, oracle):
    M, K, N, r = 300, 1024, 512, 16
    lin, _ = make_linear(oracle, K, N, 2000, device)
    lin.bias = torch.from_numpy(oracle.fill_normal(2001, 0.1, N)).to(device)
    _, _, ad = lora_parts(oracle, K, N, r, 2002, device)
    _, xt = acts(oracle, M, K, 2003, torch.bfloat16, device)
    ql = Q.QloraLinear(lin, ad)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=device)

    def run():
        y.copy_(ql.forward(xt, out_dtype=torch.bfloat16))

    replay_matches(run, lambda: [y])


def test_swiglu_prefill_and_decode_replay(device, oracle):
    hidden, inter = 512, 1408
    g, _ = make_linear(oracle, hidden, inter, 2010, device)
    u, _ = make_linear(oracle, hidden, inter, 2011, device)
    d, _ = make_linear(oracle, inter, hidden, 2012, device)
    mlp = Q.QwenMlp(g, u, d)
    _, xb = acts(oracle, 256, hidden, 2013, torch.bfloat16, device)
    _, x1 = acts(oracle, 1, hidden, 2014, torch.float32, device)
    yb = torch.empty(256, hidden, device=device)
    y1 = torch.empty(1, hidden, device=device)

    def run():
        yb.copy_(mlp.forward(xb, out_dtype=torch.float32))
        y1.copy_(mlp.forward(x1))

    replay_matches(run, lambda: [yb, y1])


def test_backward_replays(device, oracle):
    M, K, N, r = 256, 512, 384, 8
    lin, _ = make_linear(oracle, K, N, 2020, device)
    _, _, ad = lora_parts(oracle, K, N, r, 2021, device)
    _, xt = acts(oracle, M, K, 2022, torch.bfloat16, device)
    _, dyt = acts(oracle, M, N, 2023, torch.bfloat16, device)
    ql = Q.QloraLinear(lin, ad)
    outs = [torch.empty(M, K, device=device), torch.empty(K, r, device=device), torch.empty(r, N, device=device)]

    def run():
        dx, ga, gb = ql.backward(xt, dyt, dx_dtype=torch.float32)
        for o, v in zip(outs, (dx, ga, gb)):
            o.copy_(v)

    replay_matches(run, lambda: outs)


def test_skinny_split_and_gemv_replay(device, oracle):
    # the skinny kernel's split-d_in hand-off (arrival counters) and the GEMV
    lin, _ = make_linear(oracle, 11008, 4096, 2030, device, striped=True)
    _, x16 = acts(oracle, 16, 11008, 2031, torch.bfloat16, device)
    _, x1 = acts(oracle, 1, 11008, 2032, torch.float32, device)
    y16 = torch.empty(16, 4096, device=device)
    y1 = torch.empty(1, 4096, device=device)

    def run():
        y16.copy_(lin.forward(x16, out_dtype=torch.float32))
        y1.copy_(lin.forward(x1))

    replay_matches(run, lambda: [y16, y1])
