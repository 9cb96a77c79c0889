"""GPU parity of the NF4 linear backward for adapter-only training: the
vector-Jacobian products of Nf4Linear::forward / QloraLinear::forward
(src/qwennet.rs:238-241, :325-345; LoraAdapter::forward (x A) B s,
src/quantize.rs:619-624) that burn's autodiff takes under
src/qwentrain.rs:421-470, the base weight frozen:

    dx     = dy W^T + ((dy s) B^T) A^T
    grad_b = (x A)^T (dy s)
    grad_a = x^T ((dy s) B^T)

Each is checked against the float64 evaluation of those formulas
(``oracle.linear_backward_ref_f64``, pinned against torch.autograd and
central differences in tests/test_oracle.py) with the
oracle's dequantized weight (bit-identical to the reference's), by the larger of the
per-element normwise error (max_i |got_i - ref_i| over that element's sum of
absolute products) and the literal max|got - ref| / max|ref|: f32 dy through the f32
dequantized weight within 1e-5; bf16 dy through the bf16-expanded weight
within 1e-2 (the forward GEMM's bar); the adapter gradients, summed in f32,
within 1e-5 whatever the input types.  A transposed factor, a dropped
scaling or a wrong reduction axis fails these by orders of magnitude.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from unifur_amd import _lib as L
from unifur_amd import quantize as Q

from oracle.oracle import linear_backward_ref_f64 as refs
from test_gpu_gemm import lora_parts
from test_gpu_linear import acts, make_linear

pytestmark = pytest.mark.gpu


def normwise(got, ref, bound):
    """max over elements of |got_i - ref_i| / bound_i (the per-element
    normwise error of test_gpu_linear.check), or the BASELINE-literal
    max|got - ref| / max|ref| when that is larger: both are held to the
    tolerance."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    per_elem = float(np.max(np.abs(got - ref) / np.maximum(np.asarray(bound, np.float64), 1e-30)))
    literal = float(np.max(np.abs(got - ref)) / max(float(np.max(np.abs(ref))), 1e-30))
    return max(per_elem, literal)


@pytest.mark.parametrize("case", [
    # (M, K, N, r, dy dtype, x dtype, striped, dq)
    (37, 256, 384, 8, torch.float32, torch.float32, True, True),
    (37, 256, 384, 8, torch.float32, torch.bfloat16, False, False),
    (300, 512, 256, 16, torch.bfloat16, torch.bfloat16, True, True),
    (300, 512, 256, 16, torch.bfloat16, torch.float32, False, True),
    (5, 1024, 128, 64, torch.bfloat16, torch.bfloat16, True, False),
    (129, 896, 4864, 16, torch.bfloat16, torch.bfloat16, True, True),
    (64, 100, 70, 3, torch.float32, torch.float32, False, True),  # ragged: generic path, d_out % 64 != 0
    (257, 1024, 512, 32, torch.bfloat16, torch.float32, True, True),  # rank bucket 32, mixed input types
    (16384, 256, 136, 16, torch.bfloat16, torch.bfloat16, False, True),  # unsplit row products, 32 row slabs
])
def test_qlora_backward(device, oracle, case):
    M, K, N, r, dyt, xt_dtype, striped, dq = case
    lin, wdeq = make_linear(oracle, K, N, 1400 + M + K, device, dq=dq, striped=striped and N % 64 == 0)
    s = 16.0 / r
    a, b, ad = lora_parts(oracle, K, N, r, 1401 + r, device, scaling=s)
    x, xt = acts(oracle, M, K, 1402, xt_dtype, device)
    dy, dyt_ = acts(oracle, M, N, 1403, dyt, device)
    ql = Q.QloraLinear(lin, ad)
    dx, ga, gb = ql.backward(xt, dyt_, dx_dtype=torch.float32)
    rdx, bdx, rga, bga, rgb, bgb = refs(x, dy, wdeq, a, b, s)
    tol_dx = 1e-2 if dyt == torch.bfloat16 else 1e-5
    e_dx, e_ga, e_gb = normwise(dx.cpu(), rdx, bdx), normwise(ga.cpu(), rga, bga), normwise(gb.cpu(), rgb, bgb)
    print(f"backward {case}: dx {e_dx:.2e} grad_a {e_ga:.2e} grad_b {e_gb:.2e}", flush=True)
    assert e_dx <= tol_dx and e_ga <= 1e-5 and e_gb <= 1e-5
    assert ga.shape == (K, r) and gb.shape == (r, N) and dx.shape == (M, K)
    # deterministic: fixed reduction order
    dx2, ga2, gb2 = ql.backward(xt, dyt_, dx_dtype=torch.float32)
    assert torch.equal(dx, dx2) and torch.equal(ga, ga2) and torch.equal(gb, gb2)


@pytest.mark.parametrize("dyt", [torch.float32, torch.bfloat16])
def test_base_backward_without_adapter(device, oracle, dyt):
    M, K, N = 200, 512, 384
    lin, wdeq = make_linear(oracle, K, N, 1500, device)
    dy, dyt_ = acts(oracle, M, N, 1501, dyt, device)
    dx = lin.backward(dyt_, dx_dtype=torch.float32)
    ref = np.asarray(dy, np.float64) @ np.asarray(wdeq, np.float64).T
    bound = np.abs(np.asarray(dy, np.float64)) @ np.abs(np.asarray(wdeq, np.float64)).T
    assert normwise(dx.cpu(), ref, bound) <= (1e-2 if dyt == torch.bfloat16 else 1e-5)
    # bf16 out is that result rounded
    dxb = lin.backward(dyt_, dx_dtype=torch.bfloat16)
    assert normwise(dxb.float().cpu(), ref, bound) <= 1e-2


def test_config3_backward(device, oracle):
    # the config-3 shapes in reverse: dy bf16 [2048, 4096] through the
    # 4096 x 4096 DQ weight with the r = 16 adapter (scale 2)
    M, K, N, r = 2048, 4096, 4096, 16
    lin, wdeq = make_linear(oracle, K, N, 0x4E463457 + 3, device, dq=True, striped=True)
    a, b, ad = lora_parts(oracle, K, N, r, 0x41 + 3, device)
    x, xt = acts(oracle, M, K, 0x58 + 3, torch.bfloat16, device)
    dy, dyt_ = acts(oracle, M, N, 0x59 + 3, torch.bfloat16, device)
    dx, ga, gb = Q.QloraLinear(lin, ad).backward(xt, dyt_, dx_dtype=torch.bfloat16)
    rdx, bdx, rga, bga, rgb, bgb = refs(x, dy, wdeq, a, b, 2.0)
    assert normwise(dx.float().cpu(), rdx, bdx) <= 1e-2
    assert normwise(ga.cpu(), rga, bga) <= 1e-5 and normwise(gb.cpu(), rgb, bgb) <= 1e-5


def test_gradients_only_and_empty_batch(device, oracle):
    M, K, N, r = 50, 256, 128, 4
    lin, wdeq = make_linear(oracle, K, N, 1600, device)
    a, b, ad = lora_parts(oracle, K, N, r, 1601, device)
    x, xt = acts(oracle, M, K, 1602, torch.float32, device)
    dy, dyt_ = acts(oracle, M, N, 1603, torch.float32, device)
    dx, ga, gb = Q.QloraLinear(lin, ad).backward(xt, dyt_, want_dx=False)
    assert dx is None
    _, _, rga, bga, rgb, bgb = refs(x, dy, wdeq, a, b, 2.0)
    assert normwise(ga.cpu(), rga, bga) <= 1e-5 and normwise(gb.cpu(), rgb, bgb) <= 1e-5
    # no rows: zero gradients, nothing else touched
    dx0, ga0, gb0 = Q.QloraLinear(lin, ad).backward(xt[:0], dyt_[:0])
    assert dx0.shape == (0, K) and not ga0.any() and not gb0.any()
    # gradients without the adapter or without x are refused
    w = lin.weight_struct()
    g = torch.empty(K, r, device=device)
    st = torch.cuda.current_stream().cuda_stream
    assert L.lib().unifur_nf4_linear_backward(dyt_.data_ptr(), L.F32, M, ctypes.byref(w), None, xt.data_ptr(), L.F32,
                                              None, L.F32, g.data_ptr(), None, None, 0, st) == L.ERR_INVALID
    lo = ad.struct()
    assert L.lib().unifur_nf4_linear_backward(dyt_.data_ptr(), L.F32, M, ctypes.byref(w), ctypes.byref(lo), None,
                                              L.F32, None, L.F32, g.data_ptr(), None, None, 0, st) == L.ERR_INVALID


@pytest.mark.parametrize("case", [
    # (M, K = d_in, N = d_out, r, dq, dx dtype): K a multiple of 128 (the
    # fused kernel's output tiles), N of 64
    (2048, 4096, 4096, 16, True, torch.bfloat16),   # the config-3 shapes in reverse
    (300, 896, 4864, 16, True, torch.float32),      # a config-5 down-projection-shaped weight, ragged rows
    (65, 1024, 512, 8, False, torch.float32),       # f32 block scales, one row tile
    (257, 512, 1024, 64, True, torch.bfloat16),     # rank 64, rows past a 256-row tile
])
def test_fused_dx_with_the_minimum_workspace(device, oracle, case):
    """A workspace too small for the expanded weight: dx through the fused
    NF4 MFMA kernel over the striped weight's rows (the adapter term in its
    epilogue), against the same float64 formulas and bars as the expanded
    path, and the gradients unchanged."""
    M, K, N, r, dq, dxt = case
    lin, wdeq = make_linear(oracle, K, N, 1700 + M, device, dq=dq, striped=True)
    s = 16.0 / r
    a, b, ad = lora_parts(oracle, K, N, r, 1701 + r, device, scaling=s)
    x, xt = acts(oracle, M, K, 1702, torch.bfloat16, device)
    dy, dyt_ = acts(oracle, M, N, 1703, torch.bfloat16, device)
    lib = L.lib()
    need = lib.unifur_nf4_linear_backward_min_workspace_size(M, K, N, L.BF16, r, L.LAYOUT_STRIPED)
    full = lib.unifur_nf4_linear_backward_workspace_size(M, K, N, L.BF16, r)
    # the default size holds the expanded bf16 weight; the minimum does not
    # (its scratch: the adapter's operands and the gradients')
    assert need <= full - K * N * 2, (need, full)
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=device)
    ql = Q.QloraLinear(lin, ad)
    dx, ga, gb = ql.backward(xt, dyt_, dx_dtype=dxt, workspace=ws[:need])
    rdx, bdx, rga, bga, rgb, bgb = refs(x, dy, wdeq, a, b, s)
    e_dx = normwise(dx.float().cpu(), rdx, bdx)
    e_ga, e_gb = normwise(ga.cpu(), rga, bga), normwise(gb.cpu(), rgb, bgb)
    print(f"fused dx {case}: dx {e_dx:.2e} grad_a {e_ga:.2e} grad_b {e_gb:.2e} (workspace {need} B)", flush=True)
    assert e_dx <= 1e-2 and e_ga <= 1e-5 and e_gb <= 1e-5
    # deterministic, and the expanded path agrees to the bf16 bar
    dx2, _, _ = ql.backward(xt, dyt_, dx_dtype=dxt, workspace=ws[:need])
    assert torch.equal(dx, dx2)
    dxe, _, _ = ql.backward(xt, dyt_, dx_dtype=dxt)
    assert normwise(dx.float().cpu(), dxe.float().cpu().numpy(), bdx) <= 2e-2
    if need >= 256:
        with pytest.raises(RuntimeError):
            ql.backward(xt, dyt_, dx_dtype=dxt, workspace=ws[:need - 256])


@pytest.mark.parametrize("work", ["default", "least"])
@pytest.mark.parametrize("r", [3, 16])
def test_dx_adapter_term_alone_over_a_zero_weight(device, oracle, r, work):
    """Over an all-zero base weight dx is the adapter's term
    ((dy s) B^T) A^T alone, so its error is taken against that term (with a
    normal base weight the term is a few per cent of dx).  Default
    workspace: s A B merged into the expanded weight; least: the fused dX
    kernel's epilogue."""
    from test_gpu_gemm import zero_linear
    M, K, N = 192, 512, 1024
    lin = zero_linear(K, N, device, striped=True)
    s = 16.0 / r
    a, b, ad = lora_parts(oracle, K, N, r, 1781 + r, device, scaling=s, sigma=0.05)
    x, xt = acts(oracle, M, K, 1782, torch.bfloat16, device)
    dy, dyt_ = acts(oracle, M, N, 1783, torch.bfloat16, device)
    ws = None
    if work == "least":
        need = L.lib().unifur_nf4_linear_backward_min_workspace_size(M, K, N, L.BF16, r, L.LAYOUT_STRIPED)
        ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=device)[:need]
    dx, ga, gb = Q.QloraLinear(lin, ad).backward(xt, dyt_, dx_dtype=torch.float32, workspace=ws)
    rdx, bdx, rga, bga, rgb, bgb = refs(x, dy, np.zeros((K, N)), a, b, s)
    e = (normwise(dx.cpu(), rdx, bdx), normwise(ga.cpu(), rga, bga), normwise(gb.cpu(), rgb, bgb))
    print(f"dx adapter alone r={r} {work}: dx {e[0]:.2e} grad_a {e[1]:.2e} grad_b {e[2]:.2e}", flush=True)
    assert e[0] <= 1e-2 and e[1] <= 1e-5 and e[2] <= 1e-5


def test_min_workspace_for_a_row_major_weight(device, oracle):
    """Only a striped weight takes the fused dX kernel: for a row-major one
    the least workspace is the default size, and a backward given exactly
    that succeeds (through the expanded weight) within the bars."""
    M, K, N, r = 96, 512, 1024, 8
    lib = L.lib()
    need = lib.unifur_nf4_linear_backward_min_workspace_size(M, K, N, L.BF16, r, L.LAYOUT_ROW_MAJOR)
    assert need == lib.unifur_nf4_linear_backward_workspace_size(M, K, N, L.BF16, r)
    assert need > lib.unifur_nf4_linear_backward_min_workspace_size(M, K, N, L.BF16, r, L.LAYOUT_STRIPED)
    lin, wdeq = make_linear(oracle, K, N, 1760, device, striped=False)
    s = 2.0
    a, b, ad = lora_parts(oracle, K, N, r, 1761, device, scaling=s)
    x, xt = acts(oracle, M, K, 1762, torch.bfloat16, device)
    dy, dyt_ = acts(oracle, M, N, 1763, torch.bfloat16, device)
    ws = torch.zeros(need, dtype=torch.uint8, device=device)
    dx, ga, gb = Q.QloraLinear(lin, ad).backward(xt, dyt_, dx_dtype=torch.float32, workspace=ws)
    rdx, bdx, rga, bga, rgb, bgb = refs(x, dy, wdeq, a, b, s)
    e = (normwise(dx.cpu(), rdx, bdx), normwise(ga.cpu(), rga, bga), normwise(gb.cpu(), rgb, bgb))
    print(f"row-major min workspace {need} B: dx {e[0]:.2e} grad_a {e[1]:.2e} grad_b {e[2]:.2e}", flush=True)
    assert e[0] <= 1e-2 and e[1] <= 1e-5 and e[2] <= 1e-5


@pytest.mark.parametrize("M,work", [(64, 0), (64, 4 << 20), (512, 0)])
def test_fused_dx_without_adapter(device, oracle, M, work):
    """The base dx = dy W^T through the fused kernel: with no scratch at all
    (whole d_out per tile) and with room for its split-K partials (64 rows
    leave most CUs idle: d_out split, partials added in order)."""
    K, N = 1024, 4096
    lin, wdeq = make_linear(oracle, K, N, 1750 + M, device)
    dy, dyt_ = acts(oracle, M, N, 1751, torch.bfloat16, device)
    need = L.lib().unifur_nf4_linear_backward_min_workspace_size(M, K, N, L.BF16, 0, L.LAYOUT_STRIPED)
    assert need <= 65536  # the workspace's fixed counter region only
    size = max(work, need)
    ws = torch.zeros(size, dtype=torch.uint8, device=device)
    dx = lin.backward(dyt_, dx_dtype=torch.float32, workspace=ws)
    ref = np.asarray(dy, np.float64) @ np.asarray(wdeq, np.float64).T
    bound = np.abs(np.asarray(dy, np.float64)) @ np.abs(np.asarray(wdeq, np.float64)).T
    e = normwise(dx.cpu(), ref, bound)
    print(f"fused dx base M={M} workspace={work}: {e:.2e}", flush=True)
    assert e <= 1e-2
    assert torch.equal(dx, lin.backward(dyt_, dx_dtype=torch.float32, workspace=ws))


@pytest.mark.parametrize("M,K,N,r,work", [
    (33, 128, 64, 4, 0),          # one output tile, one K step
    (33, 128, 128, 3, 0),         # two K steps, odd rank
    (1, 256, 192, 0, 0),          # one row, three K steps, no adapter
    (20, 128, 256, 8, 0),         # four K steps: two after the prologue
    (20, 256, 320, 0, 0),         # five K steps: three after the prologue
    (40, 384, 1344, 0, 4 << 20),  # no adapter, split over d_out (21 K steps: a ragged last slab)
])
def test_fused_dx_edge_shapes(device, oracle, M, K, N, r, work):
    """The fused dX kernel's producer prologue with one and two K steps, a
    single output tile, one row, and a split whose last slab is short."""
    lin, wdeq = make_linear(oracle, K, N, 1800 + K + N, device)
    dy, dyt_ = acts(oracle, M, N, 1801, torch.bfloat16, device)
    need = L.lib().unifur_nf4_linear_backward_min_workspace_size(M, K, N, L.BF16, r, L.LAYOUT_STRIPED)
    ws = torch.zeros(max(need, work, 256), dtype=torch.uint8, device=device)
    ws = ws[:max(need, work)] if max(need, work) > 0 else ws[:1]
    dy64, w64 = np.asarray(dy, np.float64), np.asarray(wdeq, np.float64)
    if r:
        s = 16.0 / r
        a, b, ad = lora_parts(oracle, K, N, r, 1802, device, scaling=s)
        x, xt = acts(oracle, M, K, 1803, torch.bfloat16, device)
        dx, _, _ = Q.QloraLinear(lin, ad).backward(xt, dyt_, dx_dtype=torch.float32, workspace=ws)
        rdx, bdx, _, _, _, _ = refs(x, dy, wdeq, a, b, s)
    else:
        dx = lin.backward(dyt_, dx_dtype=torch.float32, workspace=ws)
        rdx, bdx = dy64 @ w64.T, np.abs(dy64) @ np.abs(w64).T
    e = normwise(dx.cpu(), rdx, bdx)
    print(f"fused dx edge M={M} K={K} N={N} r={r} workspace={ws.numel()}: {e:.2e}", flush=True)
    assert e <= 1e-2
