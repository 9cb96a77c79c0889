"""GPU parity of the MFMA prefill GEMM (bf16 activations, more than four
rows): NF4 weight dequantized into LDS as bf16, f32 accumulation, fused bias
and scaled LoRA epilogue.

The reference value is the float64 product of the same (bf16-valued) inputs
with the oracle's dequantized weight, which is bit-identical to the
reference's dequantized f32 weight (src/quantize.rs:355-366).  The bf16
tolerance of BASELINE.json's north star applies: normwise error and
max|y - r| / max|r| both <= 1e-2.  Rounding the dequantized weight to bf16
bounds the normwise error by 2^-9 plus accumulation error, so a dropped term,
a wrong scale or a transposed tile fails it by orders of magnitude.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from unifur_amd import _lib as L
from unifur_amd import quantize as Q

from test_gpu_linear import TOL_BF16, acts, check, make_linear

pytestmark = pytest.mark.gpu


def lora_parts(oracle, d_in, d_out, r, seed, device, scaling=2.0, sigma=0.01):
    # config 3's adapters: A, B ~ N(0, 0.01^2)
    a = oracle.fill_normal(seed, sigma, d_in * r).reshape(d_in, r)
    b = oracle.fill_normal(seed + 1, sigma, r * d_out).reshape(r, d_out)
    ad = Q.LoraAdapter.from_parts(torch.from_numpy(a).to(device), torch.from_numpy(b).to(device), scaling)
    return a, b, ad


@pytest.mark.parametrize("striped", [True, False])
def test_config3_prefill_qlora(device, oracle, striped):
    # X bf16 [2048, 4096], W NF4 4096 -> 4096 with double
    # quantization, LoRA r = 16, scale 2, bf16 output.
    M, K, N, r = 2048, 4096, 4096, 16
    lin, wdeq = make_linear(oracle, K, N, 0x4E463457 + 3, device, dq=True, striped=striped)
    x, xt = acts(oracle, M, K, 0x58 + 3, torch.bfloat16, device)
    a, b, ad = lora_parts(oracle, K, N, r, 0x41 + 3, device)
    ql = Q.QloraLinear(lin, ad)
    ref = oracle.linear_ref_f64(x, wdeq) + oracle.lora_ref_f64(x, a, b, 2.0)
    y = ql.forward(xt, out_dtype=torch.bfloat16)
    assert y.dtype == torch.bfloat16 and y.shape == (M, N)
    check(y, ref, x, wdeq, TOL_BF16, "mfma config3 qlora bf16-out")
    yf = ql.forward(xt, out_dtype=torch.float32)
    check(yf, ref, x, wdeq, TOL_BF16, "mfma config3 qlora f32-out")
    # deterministic: no atomics, fixed accumulation order
    assert torch.equal(ql.forward(xt, out_dtype=torch.float32), yf)


@pytest.mark.parametrize("striped", [True, False])
@pytest.mark.parametrize("M", [5, 64, 127, 128, 129, 300])
@pytest.mark.parametrize("dq", [True, False])
def test_ragged_rows_and_scale_kinds(device, oracle, M, dq, striped):
    K, N = 512, 384
    lin, wdeq = make_linear(oracle, K, N, 100 + M, device, dq=dq, striped=striped)
    x, xt = acts(oracle, M, K, 200 + M, torch.bfloat16, device)
    ref = oracle.linear_ref_f64(x, wdeq)
    check(lin.forward(xt, out_dtype=torch.float32), ref, x, wdeq, TOL_BF16, f"mfma M={M} dq={dq}")


@pytest.mark.parametrize("striped", [True, False])
@pytest.mark.parametrize("shape", [(896, 4864), (4864, 896), (896, 128), (64, 128), (11008, 4096)])
def test_qwen_and_edge_shapes(device, oracle, shape, striped):
    K, N = shape
    M = 32
    lin, wdeq = make_linear(oracle, K, N, 300 + K + N, device, striped=striped)
    x, xt = acts(oracle, M, K, 301, torch.bfloat16, device)
    check(lin.forward(xt, out_dtype=torch.bfloat16), oracle.linear_ref_f64(x, wdeq), x, wdeq, TOL_BF16,
          f"mfma {shape}")


@pytest.mark.parametrize("striped", [True, False])
@pytest.mark.parametrize("r", [1, 8, 16, 40, 64])
def test_bias_and_lora_ranks(device, oracle, r, striped):
    M, K, N = 200, 1024, 512
    lin, wdeq = make_linear(oracle, K, N, 400 + r, device, striped=striped)
    bias = oracle.fill_normal(401, 0.1, N)
    lin.bias = torch.from_numpy(bias).to(device)
    x, xt = acts(oracle, M, K, 402, torch.bfloat16, device)
    a, b, ad = lora_parts(oracle, K, N, r, 403 + r, device, scaling=16.0 / r)
    ref = oracle.linear_ref_f64(x, wdeq, bias) + oracle.lora_ref_f64(x, a, b, 16.0 / r)
    check(Q.QloraLinear(lin, ad).forward(xt, out_dtype=torch.float32), ref, x, wdeq, TOL_BF16,
          f"mfma bias+lora r={r}")
    # a fresh adapter (B = 0) adds exactly nothing (src/quantize.rs:1059-1081)
    fresh = Q.LoraAdapter.new(Q.LoraConfig.new(K, N, r), device=device)
    assert torch.equal(Q.QloraLinear(lin, fresh).forward(xt), lin.forward(xt))


def zero_linear(K, N, device, striped):
    """An NF4 layer whose every block is zero (absmax 0): deq(W) = 0."""
    p = Q.PackedNf4Tensor.quantize(torch.zeros(K * N, device=device)).with_double_quantization()
    lin = Q.Nf4Linear.from_packed(p, K, N, striped=striped)
    assert float(lin.dequantized_weight().abs().max()) == 0.0
    return lin


@pytest.mark.parametrize("striped", [True, False])
@pytest.mark.parametrize("work", ["default", "least"])
@pytest.mark.parametrize("r", [3, 16, 40])
def test_adapter_term_alone_over_a_zero_weight(device, oracle, r, work, striped):
    """Over an all-zero base weight y is the adapter term (x A) B s alone
    (src/quantize.rs:619-624), so its error is taken against that term: with
    a normal base weight the adapter is a few per cent of y, and a wrong
    factor row or column could hide inside the bf16 bar.  The default
    workspace merges s A B into the expanded weight (rank 16: factors staged
    through LDS; other ranks: per-wave fragment loads); the least workspace
    takes the fused kernel's epilogue."""
    M, K, N = 256, 1024, 512
    lin = zero_linear(K, N, device, striped)
    s = 16.0 / r
    x, xt = acts(oracle, M, K, 0x77, torch.bfloat16, device)
    a, b, ad = lora_parts(oracle, K, N, r, 0x78 + r, device, scaling=s, sigma=0.05)
    ref = oracle.lora_ref_f64(x, a, b, s)
    lib = L.lib()
    size = lib.unifur_nf4_linear_workspace_size if work == "default" else lib.unifur_nf4_linear_min_workspace_size
    need = size(M, K, N, L.BF16, r)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=device)
    w, lo = lin.weight_struct(), ad.struct()
    y = torch.empty(M, N, device=device)
    L.check(lib.unifur_nf4_linear_forward(xt.data_ptr(), L.BF16, M, ctypes.byref(w), None, ctypes.byref(lo),
                                          y.data_ptr(), L.F32, ws.data_ptr(), need,
                                          torch.cuda.current_stream().cuda_stream))
    got = y.cpu().numpy().astype(np.float64)
    # per element against the sum of |products| of the adapter term
    bound = (np.abs(x) @ np.abs(a)) @ np.abs(b) * s
    nw = float(np.max(np.abs(got - ref) / bound))
    lit = float(np.max(np.abs(got - ref)) / np.max(np.abs(ref)))
    print(f"adapter alone r={r} {work} striped={striped}: normwise {nw:.3e} literal {lit:.3e}", flush=True)
    assert nw <= TOL_BF16 and lit <= TOL_BF16


@pytest.mark.parametrize("K", [64, 128, 192, 320])
def test_rank16_adapter_expand_at_one_and_two_k_tiles_per_workgroup(device, oracle, K):
    """Rank 16 stages the factors through LDS in the expand (96 rows take
    the expanded path); d_in of 1, 2, 3 and 5 64-row tiles give workgroups
    of one, two, one and one tile (four tiles: the tests at d_in 1024),
    each against the adapter term alone."""
    M, N, r = 96, 384, 16
    lin = zero_linear(K, N, device, True)
    x, xt = acts(oracle, M, K, 0x79 + K, torch.bfloat16, device)
    a, b, ad = lora_parts(oracle, K, N, r, 0x7A + K, device, scaling=1.0, sigma=0.05)
    ref = oracle.lora_ref_f64(x, a, b, 1.0)
    y = Q.QloraLinear(lin, ad).forward(xt, out_dtype=torch.float32).cpu().numpy().astype(np.float64)
    bound = (np.abs(x) @ np.abs(a)) @ np.abs(b)
    nw = float(np.max(np.abs(y - ref) / bound))
    print(f"rank-16 expand K={K}: normwise {nw:.3e}", flush=True)
    assert nw <= TOL_BF16


def test_misaligned_activations_take_the_generic_path(device, oracle):
    # X not 16-byte aligned: the generic dequantize + f32 matmul serves it,
    # with the same result to the bf16 tolerance.
    M, K, N = 16, 256, 128
    lin, wdeq = make_linear(oracle, K, N, 500, device)
    x, _ = acts(oracle, M, K, 501, torch.bfloat16, device)
    buf = torch.zeros(M * K + 1, dtype=torch.bfloat16, device=device)
    buf[1:] = torch.from_numpy(x.reshape(-1)).to(torch.bfloat16)
    xv = buf[1:].view(M, K)
    assert xv.data_ptr() % 16 != 0
    y = torch.empty(M, N, device=device)
    w = lin.weight_struct()
    stream = torch.cuda.current_stream().cuda_stream
    L.check(L.lib().unifur_nf4_linear_forward(xv.data_ptr(), L.BF16, M, ctypes.byref(w), None, None, y.data_ptr(),
                                              L.F32, None, 0, stream))
    check(y, oracle.linear_ref_f64(x, wdeq), x, wdeq, TOL_BF16, "misaligned x")
    aligned = lin.forward(torch.from_numpy(x).to(device).to(torch.bfloat16), out_dtype=torch.float32)
    check(aligned, oracle.linear_ref_f64(x, wdeq), x, wdeq, TOL_BF16, "aligned x")


def _qlora_with_workspace(device, oracle, M, K, N, r, need, seed, striped=True):
    lin, wdeq = make_linear(oracle, K, N, seed, device, striped=striped)
    x, xt = acts(oracle, M, K, seed + 1, torch.bfloat16, device)
    a, b, ad = lora_parts(oracle, K, N, r, seed + 2, device)
    bias = oracle.fill_normal(seed + 3, 0.1, N)
    bt = torch.from_numpy(bias).to(device)
    ws = torch.zeros(need, dtype=torch.uint8, device=device)
    w, lo = lin.weight_struct(), ad.struct()
    stream = torch.cuda.current_stream().cuda_stream
    ref = oracle.linear_ref_f64(x, wdeq, bias) + oracle.lora_ref_f64(x, a, b, 2.0)
    outs = []
    for _ in range(2):
        y = torch.empty(M, N, device=device)
        L.check(L.lib().unifur_nf4_linear_forward(xt.data_ptr(), L.BF16, M, ctypes.byref(w),
                                                  bt.data_ptr(),
                                                  ctypes.byref(lo), y.data_ptr(), L.F32, ws.data_ptr(), need, stream))
        check(y, ref, x, wdeq, TOL_BF16, f"prefill workspace {need}")
        outs.append(y)
    assert torch.equal(outs[0], outs[1])
    assert int(ws[:65536].count_nonzero()) == 0


@pytest.mark.parametrize("striped", [True, False])
def test_workspace_sizes_select_expanded_or_fused_prefill(device, oracle, striped):
    # the default size holds the bf16 expansion of W (d_in d_out 2 bytes) and
    # the BLAS scratch; the minimum only the fused kernel's LoRA operands
    M, K, N, r = 256, 512, 256, 16
    full = L.lib().unifur_nf4_linear_workspace_size(M, K, N, L.BF16, r)
    lean = L.lib().unifur_nf4_linear_min_workspace_size(M, K, N, L.BF16, r)
    assert full >= 65536 + K * N * 2
    assert lean < K * N * 2 and lean <= 65536 + M * 16 * 2 + 16 * K * 2 + N * 16 * 2 + 3 * 256
    assert L.lib().unifur_nf4_linear_min_workspace_size(4, K, N, L.F32, 0) == \
        L.lib().unifur_nf4_linear_workspace_size(4, K, N, L.F32, 0)
    _qlora_with_workspace(device, oracle, M, K, N, r, full, 600, striped)   # expanded + BLAS
    _qlora_with_workspace(device, oracle, M, K, N, r, lean, 610, striped)   # fused kernel
    with pytest.raises(RuntimeError):
        _qlora_with_workspace(device, oracle, M, K, N, r, lean - 256, 620, striped)


@pytest.mark.parametrize("M", [65, 128, 300, 2048])
def test_fused_prefill_kernel_config3_shapes(device, oracle, M):
    # the fused MFMA kernel (what a caller with bounded scratch gets) at the
    # config-3 weight shape, with bias and LoRA, against the same reference
    K, N, r = 4096, 4096, 16
    lean = L.lib().unifur_nf4_linear_min_workspace_size(M, K, N, L.BF16, r)
    _qlora_with_workspace(device, oracle, M, K, N, r, lean, 700 + M)


@pytest.mark.parametrize("striped", [True, False])
@pytest.mark.parametrize("K", [64, 128, 192, 256, 320, 448])
def test_fused_prefill_few_k_steps(device, oracle, K, striped):
    # 1-7 K steps of 64 per workgroup: the dequantizing waves' prologue
    # (one or two steps) and their last 0-3 steps after the 4-step main loop
    M, N, r = 300, 256, 8
    lean = L.lib().unifur_nf4_linear_min_workspace_size(M, K, N, L.BF16, r)
    _qlora_with_workspace(device, oracle, M, K, N, r, lean, 900 + K, striped=striped)


@pytest.mark.parametrize("ydt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shift", [0, 1, 2])
def test_fused_prefill_output_alignment(device, oracle, ydt, shift):
    # The fused kernel stores four outputs at once when y is 16-byte aligned
    # and one at a time otherwise; an output offset by `shift` elements (and
    # rows past a 256-row tile) must give the aligned result bit for bit.
    M, K, N, r = 300, 512, 384, 8
    lin, wdeq = make_linear(oracle, K, N, 800 + shift, device)
    x, xt = acts(oracle, M, K, 801, torch.bfloat16, device)
    a, b, ad = lora_parts(oracle, K, N, r, 802, device)
    bias = oracle.fill_normal(803, 0.1, N)
    bt = torch.from_numpy(bias).to(device)
    need = L.lib().unifur_nf4_linear_min_workspace_size(M, K, N, L.BF16, r)
    ws = torch.zeros(need, dtype=torch.uint8, device=device)
    w, lo = lin.weight_struct(), ad.struct()
    st = torch.cuda.current_stream().cuda_stream
    code = L.BF16 if ydt == torch.bfloat16 else L.F32

    def run(y_ptr):
        L.check(L.lib().unifur_nf4_linear_forward(xt.data_ptr(), L.BF16, M, ctypes.byref(w), bt.data_ptr(),
                                                  ctypes.byref(lo), y_ptr, code, ws.data_ptr(), need, st))

    y0 = torch.empty(M, N, dtype=ydt, device=device)
    run(y0.data_ptr())
    buf = torch.full((M * N + 8,), float("nan"), dtype=ydt, device=device)
    run(buf[shift:].data_ptr())
    y1 = buf[shift:shift + M * N].view(M, N)
    assert torch.equal(y0, y1)
    assert torch.isnan(buf[:shift]).all() and torch.isnan(buf[shift + M * N:]).all()
    ref = oracle.linear_ref_f64(x, wdeq, bias) + oracle.lora_ref_f64(x, a, b, ad.scaling())
    check(y0, ref, x, wdeq, TOL_BF16, f"fused prefill y {ydt} shift {shift}")


# ---- split-K of the fused kernel (no adapter; a workspace with room for the
# f32 partials but not for the expanded weight) ----

@pytest.mark.parametrize("M,K,N", [(300, 4096, 512), (512, 11008, 1024), (130, 2048, 256), (64 + 8, 4096, 128)])
@pytest.mark.parametrize("ydt", [torch.bfloat16, torch.float32])
def test_fused_split_k(device, oracle, M, K, N, ydt):
    lin, wdeq = make_linear(oracle, K, N, 3300 + M, device)
    bias = oracle.fill_normal(3301, 0.1, N)
    bt = torch.from_numpy(bias).to(device)
    x, xt = acts(oracle, M, K, 3302 + M, torch.bfloat16, device)
    lean = L.lib().unifur_nf4_linear_min_workspace_size(M, K, N, L.BF16, 0)
    full = L.lib().unifur_nf4_linear_workspace_size(M, K, N, L.BF16, 0)
    split_room = lean + 8 * M * N * 4 + 4096  # partials of up to 8 slabs
    assert split_room < full
    w = lin.weight_struct()
    st = torch.cuda.current_stream().cuda_stream
    code = L.BF16 if ydt == torch.bfloat16 else L.F32
    ref = oracle.linear_ref_f64(x, wdeq, bias)
    outs = {}
    for name, need in (("split", split_room), ("whole", lean)):
        ws = torch.zeros(need, dtype=torch.uint8, device=device)
        y = torch.empty(M, N, dtype=ydt, device=device)
        L.check(L.lib().unifur_nf4_linear_forward(xt.data_ptr(), L.BF16, M, ctypes.byref(w), bt.data_ptr(), None,
                                                  y.data_ptr(), code, ws.data_ptr(), need, st))
        check(y, ref, x, wdeq, TOL_BF16, f"fused {name} M={M} K={K} N={N}")
        y2 = torch.empty_like(y)
        L.check(L.lib().unifur_nf4_linear_forward(xt.data_ptr(), L.BF16, M, ctypes.byref(w), bt.data_ptr(), None,
                                                  y2.data_ptr(), code, ws.data_ptr(), need, st))
        assert torch.equal(y, y2)  # slabs added in a fixed order
        assert int(ws[:65536].count_nonzero()) == 0
        outs[name] = y.float()
    # both sum the same products, in another order: within f32 rounding (plus
    # one bf16 rounding of the output)
    tol = 1e-2 if ydt == torch.bfloat16 else 1e-4
    assert float((outs["split"] - outs["whole"]).abs().max() / outs["whole"].abs().max()) < tol


@pytest.mark.parametrize("T", [256, 512])
def test_fused_swiglu_split_k(device, oracle, T):
    # a 7B-shaped MLP at reduced width: down (inter -> hidden) has few tiles
    # and splits d_in; the gate/up pair (16 K steps) runs over whole d_in
    hidden, inter = 1024, 2816
    ws_, deqs = [], []
    for i, (din, dout) in enumerate([(hidden, inter), (hidden, inter), (inter, hidden)]):
        lin, wd = make_linear(oracle, din, dout, 3400 + i, device)
        ws_.append(lin)
        deqs.append(wd)
    x, xt = acts(oracle, T, hidden, 3410 + T, torch.bfloat16, device)
    lean = L.lib().unifur_nf4_swiglu_min_workspace_size(T, hidden, inter, L.BF16)
    # up to 512 rows the default workspace is the fused kernels' with the
    # split-K partials (down's two slabs of f32 here), not an expanded weight
    room = L.lib().unifur_nf4_swiglu_workspace_size(T, hidden, inter, L.BF16)
    assert lean + 2 * T * hidden * 4 <= room < lean + 2 * T * hidden * 4 + 4096
    g, u, d = (l.weight_struct() for l in ws_)
    st = torch.cuda.current_stream().cuda_stream
    h = oracle.silu_f64(x.astype(np.float64) @ deqs[0]) * (x.astype(np.float64) @ deqs[1])
    ref = oracle.swiglu_ref_f64(x, *deqs)
    outs = []
    for need in (room, lean):
        ws = torch.zeros(need, dtype=torch.uint8, device=device)
        y = torch.empty(T, hidden, device=device)
        L.check(L.lib().unifur_nf4_swiglu_forward(xt.data_ptr(), L.BF16, T, ctypes.byref(g), ctypes.byref(u),
                                                  ctypes.byref(d), y.data_ptr(), L.F32, ws.data_ptr(), need, st))
        check(y, ref, h, deqs[2], TOL_BF16, f"fused swiglu T={T} workspace {need}")
        outs.append(y)
    assert float((outs[0] - outs[1]).abs().max() / outs[1].abs().max()) < 1e-2


def swiglu_call(g, u, d, xt, T, hidden, need, device):
    ws = torch.zeros(need, dtype=torch.uint8, device=device)
    y = torch.empty(T, hidden, device=device)
    L.check(L.lib().unifur_nf4_swiglu_forward(xt.data_ptr(), L.BF16, T, ctypes.byref(g), ctypes.byref(u),
                                              ctypes.byref(d), y.data_ptr(), L.F32, ws.data_ptr(), need,
                                              torch.cuda.current_stream().cuda_stream))
    return y, ws


def swiglu_layers(oracle, device, hidden, inter, seed, kinds=(True, True, True), striped=None):
    lins = [make_linear(oracle, din, dout, seed + i, device, dq=dq, striped=striped)
            for i, ((din, dout), dq) in enumerate(zip([(hidden, inter), (hidden, inter), (inter, hidden)], kinds))]
    return [l for l, _ in lins], [w for _, w in lins]


@pytest.mark.parametrize("striped,dq", [(True, True), (False, True), (True, False)])
def test_fused_swiglu_pair(device, oracle, striped, dq):
    # gate and up of one scale kind run as one pair launch whose epilogue
    # forms silu(g) * u.  Here its grid has few output tiles over 64 K steps:
    # with the default workspace it splits d_in and a reduction adds the
    # slabs (in slab order) before the product; with the least workspace it
    # runs over whole d_in.  Both against the oracle, and each deterministic.
    hidden, inter, T = 4096, 1024, 256
    lins, (wg, wu, wd) = swiglu_layers(oracle, device, hidden, inter, 3500, (dq, dq, dq), striped)
    x, xt = acts(oracle, T, hidden, 3510, torch.bfloat16, device)
    ref = oracle.swiglu_ref_f64(x, wg, wu, wd)
    h = oracle.silu_f64(x.astype(np.float64) @ wg) * (x.astype(np.float64) @ wu)
    room = L.lib().unifur_nf4_swiglu_workspace_size(T, hidden, inter, L.BF16)
    lean = L.lib().unifur_nf4_swiglu_min_workspace_size(T, hidden, inter, L.BF16)
    assert room >= lean + 2 * T * 2 * inter * 4  # the pair's partials: gate and up, two or more slabs
    g, u, d = (l.weight_struct() for l in lins)
    outs = {}
    for name, need in (("split", room), ("whole", lean)):
        y, ws = swiglu_call(g, u, d, xt, T, hidden, need, device)
        check(y, ref, h, wd, TOL_BF16, f"pair {name} striped={striped} dq={dq}")
        y2, _ = swiglu_call(g, u, d, xt, T, hidden, need, device)
        assert torch.equal(y, y2)
        assert int(ws[:65536].count_nonzero()) == 0
        outs[name] = y
    assert float((outs["split"] - outs["whole"]).abs().max() / outs["whole"].abs().max()) < 1e-2


def test_fused_swiglu_mixed_scale_kinds(device, oracle):
    # gate double-quantized, up with f32 scales: no pair launch -- gate and
    # up are two launches (f32 outputs, split over d_in with the default
    # workspace) and the elementwise kernel forms silu(g) * u
    hidden, inter, T = 4096, 1024, 256
    lins, (wg, wu, wd) = swiglu_layers(oracle, device, hidden, inter, 3520, (True, False, True))
    x, xt = acts(oracle, T, hidden, 3530, torch.bfloat16, device)
    ref = oracle.swiglu_ref_f64(x, wg, wu, wd)
    h = oracle.silu_f64(x.astype(np.float64) @ wg) * (x.astype(np.float64) @ wu)
    g, u, d = (l.weight_struct() for l in lins)
    for need in (L.lib().unifur_nf4_swiglu_workspace_size(T, hidden, inter, L.BF16),
                 L.lib().unifur_nf4_swiglu_min_workspace_size(T, hidden, inter, L.BF16)):
        y, _ = swiglu_call(g, u, d, xt, T, hidden, need, device)
        check(y, ref, h, wd, TOL_BF16, f"mixed kinds workspace {need}")


@pytest.mark.parametrize("T,hidden,inter,pair", [(512, 4096, 9600, True), (512, 2048, 19200, False)])
def test_fused_swiglu_tail_round(device, oracle, T, hidden, inter, pair):
    # 300 output tiles: one whole round of 256 tiles, then a last round of 44.
    # With the default workspace the whole round runs whole and the last
    # round's tiles split d_in (4 ways for the pair launch, 2 for gate and up
    # as separate launches), an ordered reduction of just those tiles; with
    # the least workspace every tile runs whole (up to 512 rows the default
    # workspace is the fused kernels', not the expanded weights).  Both
    # against the oracle.
    kinds = (True, True, True) if pair else (True, False, True)
    lins, (wg, wu, wd) = swiglu_layers(oracle, device, hidden, inter, 3600 + T, kinds)
    x, xt = acts(oracle, T, hidden, 3610, torch.bfloat16, device)
    ref = oracle.swiglu_ref_f64(x, wg, wu, wd)
    h = oracle.silu_f64(x.astype(np.float64) @ wg) * (x.astype(np.float64) @ wu)
    room = L.lib().unifur_nf4_swiglu_workspace_size(T, hidden, inter, L.BF16)
    lean = L.lib().unifur_nf4_swiglu_min_workspace_size(T, hidden, inter, L.BF16)
    assert room > lean
    g, u, d = (l.weight_struct() for l in lins)
    outs = {}
    for name, need in (("tail", room), ("whole", lean)):
        y, ws = swiglu_call(g, u, d, xt, T, hidden, need, device)
        check(y, ref, h, wd, TOL_BF16, f"swiglu tail round {name} T={T} pair={pair}")
        y2, _ = swiglu_call(g, u, d, xt, T, hidden, need, device)
        assert torch.equal(y, y2)
        outs[name] = y
    assert float((outs["tail"] - outs["whole"]).abs().max() / outs["whole"].abs().max()) < 1e-2


@pytest.mark.parametrize("hidden", [64, 192, 256, 320])
def test_fused_swiglu_pair_few_k_steps(device, oracle, hidden):
    # the gate/up pair launch at 1-5 K steps of 64 (d_in = hidden): the
    # dequantizing waves' prologue and their last 1-3 steps in PAIR mode,
    # with the default and the least workspace, against the oracle
    inter, T = 384, 300
    lins, (wg, wu, wd) = swiglu_layers(oracle, device, hidden, inter, 3700 + hidden)
    x, xt = acts(oracle, T, hidden, 3710 + hidden, torch.bfloat16, device)
    ref = oracle.swiglu_ref_f64(x, wg, wu, wd)
    h = oracle.silu_f64(x.astype(np.float64) @ wg) * (x.astype(np.float64) @ wu)
    g, u, d = (l.weight_struct() for l in lins)
    for need in (L.lib().unifur_nf4_swiglu_workspace_size(T, hidden, inter, L.BF16),
                 L.lib().unifur_nf4_swiglu_min_workspace_size(T, hidden, inter, L.BF16)):
        y, _ = swiglu_call(g, u, d, xt, T, hidden, need, device)
        check(y, ref, h, wd, TOL_BF16, f"pair hidden={hidden} workspace {need}")


def test_prefill_past_two_gib_of_activations(device, oracle):
    """262,200 bf16 rows of 4096 (2.15 GB of activations): past the fused
    kernel's 2^31-byte reach of X offsets.  The default workspace keeps the
    expanded weight and the BLAS GEMM (64-bit offsets), the least workspace
    takes the generic path; for the linear with an adapter and for the SwiGLU
    block, rows sampled at the start, the middle, the 2^31-byte boundary and
    the end against the float64 oracle within the bf16 bar."""
    M, K, N, r = 262_200, 4096, 256, 8
    assert (M + 256) * K * 2 >= 1 << 31
    g = torch.Generator(device=device).manual_seed(0x2617)
    xt = torch.randn(M, K, generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)
    idx = np.array([0, 1, 7, M // 2, (1 << 31) // (2 * K) - 1, (1 << 31) // (2 * K), M - 2, M - 1])
    xs = xt[torch.from_numpy(idx).to(device)].float().cpu().numpy().astype(np.float64)
    lin, wdeq = make_linear(oracle, K, N, 0x2618, device, striped=True)
    a, b, ad = lora_parts(oracle, K, N, r, 0x2619, device, scaling=2.0)
    ref = oracle.linear_ref_f64(xs, wdeq) + oracle.lora_ref_f64(xs, a, b, 2.0)
    lib = L.lib()
    w, lo = lin.weight_struct(), ad.struct()
    for size in (lib.unifur_nf4_linear_workspace_size, lib.unifur_nf4_linear_min_workspace_size):
        need = size(M, K, N, L.BF16, r)
        print(f"{M} rows, workspace {need} B", flush=True)
        ws = torch.zeros(need, dtype=torch.uint8, device=device)
        y = torch.empty(M, N, device=device)
        L.check(lib.unifur_nf4_linear_forward(xt.data_ptr(), L.BF16, M, ctypes.byref(w), None, ctypes.byref(lo),
                                              y.data_ptr(), L.F32, ws.data_ptr(), need,
                                              torch.cuda.current_stream().cuda_stream))
        check(y[torch.from_numpy(idx).to(device)], ref, xs, wdeq, TOL_BF16, f"{M} rows, workspace {need}")
        del ws, y
    # the SwiGLU block over the same rows (gate/up 4096 -> 256, down 256 -> 4096)
    gl, wg = make_linear(oracle, K, N, 0x261A, device, striped=True)
    ul, wu = make_linear(oracle, K, N, 0x261B, device, striped=True)
    dl, wd = make_linear(oracle, N, K, 0x261C, device, striped=True)
    ref = oracle.swiglu_ref_f64(xs, wg, wu, wd)
    h = oracle.silu_f64(xs @ wg) * (xs @ wu)
    y = Q.QwenMlp(gl, ul, dl).forward(xt, out_dtype=torch.float32)
    check(y[torch.from_numpy(idx).to(device)], ref, h, wd, TOL_BF16, f"swiglu {M} rows")
