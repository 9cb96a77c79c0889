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


@pytest.mark.parametrize("rank", [0, 16])
def test_fused_dx_backward_replays(device, oracle, rank):
    """The bounded-workspace backward (dX through the fused NF4 kernel over
    the weight's rows; its adapter operands or split-K partials in the
    caller's workspace) replays to the eager bits."""
    M, K, N = 96, 512, 1024
    lin, _ = make_linear(oracle, K, N, 2060 + rank, device)
    _, xt = acts(oracle, M, K, 2061, torch.bfloat16, device)
    _, dyt = acts(oracle, M, N, 2062, torch.bfloat16, device)
    from unifur_amd import _lib as L
    need = L.lib().unifur_nf4_linear_backward_min_workspace_size(M, K, N, L.BF16, rank, L.LAYOUT_STRIPED)
    # room for the split-K partials without the adapter, the minimum with it
    ws = torch.zeros(max(need, 2 << 20) if rank == 0 else need, dtype=torch.uint8, device=device)
    dx = torch.empty(M, K, device=device)
    if rank:
        _, _, ad = lora_parts(oracle, K, N, rank, 2063, device)
        ql = Q.QloraLinear(lin, ad)
        ga = torch.empty(K, rank, device=device)
        gb = torch.empty(rank, N, device=device)

        def run():
            d, a_, b_ = ql.backward(xt, dyt, dx_dtype=torch.float32, workspace=ws)
            dx.copy_(d)
            ga.copy_(a_)
            gb.copy_(b_)

        replay_matches(run, lambda: [dx, ga, gb])
    else:
        def run():
            dx.copy_(lin.backward(dyt, dx_dtype=torch.float32, workspace=ws))

        replay_matches(run, lambda: [dx])


@pytest.mark.parametrize("rank", [0, 16])
def test_f32_mfma_forward_and_dx_replay(device, oracle, rank):
    """f32 activations past the skinny rows and f32 dY: the f32 MFMA GEMM
    (and with an adapter its x A / dY B^T row products, whose slab sums
    use arrival counters) replays to the eager bits."""
    M, K, N = 300, 1024, 512
    lin, _ = make_linear(oracle, K, N, 2070 + rank, device)
    lin.bias = torch.from_numpy(oracle.fill_normal(2071, 0.1, N)).to(device)
    _, xt = acts(oracle, M, K, 2072, torch.float32, device)
    _, dyt = acts(oracle, M, N, 2073, torch.float32, device)
    layer = lin
    if rank:
        _, _, ad = lora_parts(oracle, K, N, rank, 2074, device)
        layer = Q.QloraLinear(lin, ad)
    y = torch.empty(M, N, device=device)
    dx = torch.empty(M, K, device=device)

    def run():
        y.copy_(layer.forward(xt, out_dtype=torch.float32))
        if rank:
            dx.copy_(layer.backward(xt, dyt, dx_dtype=torch.float32)[0])
        else:
            dx.copy_(layer.backward(dyt, dx_dtype=torch.float32))

    replay_matches(run, lambda: [y, dx])


def test_grouped_quantize_pass_replays(device, oracle):
    """The grouped quantize pass (f32 values and bf16 checkpoint tensors,
    more weights than one launch group takes) replays to the eager bytes."""
    shapes = [(64 * (1 + i % 3), 64 * (1 + i % 4)) for i in range(53)]
    vals = [(torch.from_numpy(oracle.fill_normal(2080 + i, 0.02, di * do)).to(device), di, do)
            for i, (di, do) in enumerate(shapes)]
    ckpt = [v.view(di, do).t().contiguous().to(torch.bfloat16) for (v, di, do) in vals]
    outs = []

    def run():
        lins = Q.quantize_linears(vals) + Q.quantize_checkpoint_linears(ckpt)
        if not outs:
            outs.extend([torch.empty_like(t) for lin in lins for t in (lin._codes, lin._scales, lin._sos)])
        for o, t in zip(outs, [t for lin in lins for t in (lin._codes, lin._scales, lin._sos)]):
            o.copy_(t)

    # as replay_matches, with zeros instead of NaN between the replays (the
    # code and scale buffers are bytes)
    run()
    torch.cuda.synchronize()
    want = [o.clone() for o in outs]
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        run()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=st):
            run()
    torch.cuda.current_stream().wait_stream(st)
    for _ in range(4):
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, w in zip(outs, want):
            assert torch.equal(o, w), "graph replay differs from the eager result"


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


def _hip():
    import ctypes
    h = ctypes.CDLL("libamdhip64.so.7")  # the runtime torch and the library already share
    P = ctypes.c_void_p
    h.hipStreamCreateWithFlags.argtypes = [ctypes.POINTER(P), ctypes.c_uint]
    h.hipStreamBeginCapture.argtypes = [P, ctypes.c_int]
    h.hipStreamEndCapture.argtypes = [P, ctypes.POINTER(P)]
    h.hipGraphGetNodes.argtypes = [P, P, ctypes.POINTER(ctypes.c_size_t)]
    h.hipGraphInstantiate.argtypes = [ctypes.POINTER(P), P, P, P, ctypes.c_size_t]
    h.hipGraphLaunch.argtypes = [P, P]
    h.hipStreamSynchronize.argtypes = [P]
    for f in ("hipGraphDestroy", "hipGraphExecDestroy", "hipStreamDestroy"):
        getattr(h, f).argtypes = [P]
    return h


def test_internal_workspace_under_capture(device, oracle):
    # The internal workspace (workspace == NULL) of a stream: a call under
    # capture that would have to create or grow it is refused with
    # UNIFUR_NF4_ERR_WORKSPACE and records nothing; a graph captured from a
    # small call keeps replaying correctly after eager calls on the same
    # stream have grown the workspace past it (outgrown buffers stay alive).
    import ctypes
    from unifur_amd import _lib as L
    h = _hip()
    lib = L.lib()
    P = ctypes.c_void_p
    relaxed = 2  # hipStreamCaptureModeRelaxed
    s = P()
    assert h.hipStreamCreateWithFlags(ctypes.byref(s), 1) == 0  # a new stream: no workspace yet
    try:
        lin, _ = make_linear(oracle, 1024, 512, 2040, device)
        _, x1 = acts(oracle, 2, 1024, 2041, torch.float32, device)
        _, xb = acts(oracle, 300, 1024, 2042, torch.bfloat16, device)
        w = lin.weight_struct()
        y1 = torch.empty(2, 512, device=device)
        yb = torch.empty(300, 512, device=device)
        torch.cuda.synchronize()

        def small():
            return lib.unifur_nf4_linear_forward(x1.data_ptr(), L.F32, 2, ctypes.byref(w), None, None,
                                                 y1.data_ptr(), L.F32, None, 0, s)

        def large():
            return lib.unifur_nf4_linear_forward(xb.data_ptr(), L.BF16, 300, ctypes.byref(w), None, None,
                                                 yb.data_ptr(), L.F32, None, 0, s)

        graph = P()
        assert h.hipStreamBeginCapture(s, relaxed) == 0
        st = small()
        assert h.hipStreamEndCapture(s, ctypes.byref(graph)) == 0
        n = ctypes.c_size_t(0)
        assert h.hipGraphGetNodes(graph, None, ctypes.byref(n)) == 0
        h.hipGraphDestroy(graph)
        assert st == L.ERR_WORKSPACE and b"capturing" in lib.unifur_nf4_last_error()
        assert n.value == 0, "a refused call recorded graph nodes"

        # eager call sizes the workspace, then capture the small call
        assert small() == 0
        assert h.hipStreamSynchronize(s) == 0
        want = y1.clone()
        assert h.hipStreamBeginCapture(s, relaxed) == 0
        assert small() == 0
        assert h.hipStreamEndCapture(s, ctypes.byref(graph)) == 0
        ex = P()
        assert h.hipGraphInstantiate(ctypes.byref(ex), graph, None, None, 0) == 0
        # a larger call of the same stream under capture is refused too
        assert h.hipStreamBeginCapture(s, relaxed) == 0
        st = large()
        g2 = P()
        assert h.hipStreamEndCapture(s, ctypes.byref(g2)) == 0
        h.hipGraphDestroy(g2)
        assert st == L.ERR_WORKSPACE
        # eagerly it grows the workspace; the captured graph still replays
        assert large() == 0
        assert h.hipStreamSynchronize(s) == 0
        want_b = yb.clone()
        for _ in range(3):
            y1.fill_(float("nan"))
            torch.cuda.synchronize()
            assert h.hipGraphLaunch(ex, s) == 0
            assert h.hipStreamSynchronize(s) == 0
            assert torch.equal(y1, want), "replay after the workspace grew differs"
            assert large() == 0
            assert h.hipStreamSynchronize(s) == 0
            assert torch.equal(yb, want_b)
        h.hipGraphExecDestroy(ex)
        h.hipGraphDestroy(graph)
    finally:
        assert h.hipStreamSynchronize(s) == 0
        h.hipStreamDestroy(s)


@pytest.mark.parametrize("rows,dt", [(1, torch.float32), (2, torch.bfloat16), (32, torch.bfloat16),
                                     (12, torch.float32)])
def test_decoder_stages_replay(device, oracle, rows, dt):
    """QwenDecoderLayer::step's two stages (src/qwennet.rs:1112-1129) at a
    reduced shape, captured together as a decode loop would capture them:
    the folded norms, residual epilogues, the norm kernel and the skinny
    splits' arrival counters all replay to the eager bits."""
    from unifur_amd import qwennet as N
    hid, qd, kvd, inter = 256, 256, 64, 704
    lins = {}
    for i, (name, di, do) in enumerate((("q", hid, qd), ("k", hid, kvd), ("v", hid, kvd), ("o", qd, hid),
                                        ("gate", hid, inter), ("up", hid, inter), ("down", inter, hid))):
        lins[name], _ = make_linear(oracle, di, do, 2400 + i, device)
    g_in = torch.from_numpy(oracle.fill_normal(2410, 0.1, hid)).to(device)
    g_post = torch.from_numpy(oracle.fill_normal(2411, 0.1, hid)).to(device)
    lay = N.QwenDecoderLayer(lins["q"], lins["k"], lins["v"], lins["o"],
                             Q.QwenMlp(lins["gate"], lins["up"], lins["down"]), g_in, g_post, 1e-6)
    _, xt = acts(oracle, rows, hid, 2412 + rows, dt, device)
    q = torch.empty(rows, qd, dtype=dt, device=device)
    y = torch.empty(rows, hid, dtype=dt, device=device)

    def run():
        qq, _, _ = lay.project(xt)
        q.copy_(qq)
        y.copy_(lay.attn_out_mlp(xt, q))  # q stands in for the attention output

    replay_matches(run, lambda: [q, y])
