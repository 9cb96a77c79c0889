"""GPU parity of the f32 MFMA path (nf4_gemm_f32.hip): Nf4Linear::forward /
QloraLinear::forward (src/qwennet.rs:238-241, :325-345) with f32 activations
past the skinny kernel's rows, the backward's dX for f32 dY (the autodiff
under src/qwentrain.rs:421-470), and the SwiGLU block (src/qwennet.rs:816-819)
with f32 activations -- the reference's own f32 arithmetic, now on
v_mfma_f32_32x32x2f32 with the weight dequantized exactly in LDS instead of
an f32 copy of the whole weight.

Each case is checked against the float64 product of the same inputs with the
oracle's dequantized weight at the f32 bar (1e-5, normwise over the summed
terms and the literal max|y - r| / max|r|), bf16 outputs at 1e-2, and the
workspace each call asks for is checked to hold no f32 copy of the weight.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from unifur_amd import _lib as L
from unifur_amd import quantize as Q

from oracle.oracle import linear_backward_ref_f64
from test_gpu_gemm import lora_parts
from test_gpu_linear import TOL_BF16, TOL_F32, acts, check, make_linear

pytestmark = pytest.mark.gpu


def normwise(got, ref, bound):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    per_elem = float(np.max(np.abs(got - ref) / np.maximum(np.asarray(bound, np.float64), 1e-30)))
    literal = float(np.max(np.abs(got - ref)) / max(float(np.max(np.abs(ref))), 1e-30))
    return max(per_elem, literal)


@pytest.mark.parametrize("case", [
    # (rows, d_in, d_out, striped, dq, lora rank, y dtype, bias)
    (2048, 4096, 4096, True, True, 16, torch.float32, False),   # the config-3 shapes with f32 activations
    (100, 256, 320, False, True, 0, torch.float32, True),       # row-major, a half-width last column tile
    (129, 100, 192, True, False, 8, torch.bfloat16, True),      # d_in 100: a partial K step; f32 scales; bf16 out
    (65, 4096, 64, True, True, 0, torch.float32, False),        # one 64-column block
    (300, 896, 4864, True, True, 4, torch.float32, False),      # a config-5 gate-shaped weight
    (257, 512, 1024, False, False, 64, torch.float32, True),    # rank 64, row-major, f32 scales
])
def test_f32_forward(device, oracle, case):
    M, K, N, striped, dq, r, yt, with_bias = case
    print(f"f32 forward {case}", flush=True)
    lin, wdeq = make_linear(oracle, K, N, 6000 + M + K, device, dq=dq, striped=striped)
    assert lin.is_striped() == striped
    x, xt = acts(oracle, M, K, 6001, torch.float32, device)
    bias = None
    if with_bias:
        bias = oracle.fill_normal(6002, 0.1, N)
        lin.bias = torch.from_numpy(bias).to(device)
    ref = oracle.linear_ref_f64(x, wdeq, bias)
    if r:
        a, b, ad = lora_parts(oracle, K, N, r, 6003 + r, device, scaling=16.0 / r)
        y = Q.QloraLinear(lin, ad).forward(xt, out_dtype=yt)
        ref = ref + oracle.lora_ref_f64(x, a, b, 16.0 / r)
        bound_extra = (np.abs(x) @ np.abs(a)) @ np.abs(b) * (16.0 / r)
    else:
        y = lin.forward(xt, out_dtype=yt)
        bound_extra = 0.0
    assert y.dtype == yt and y.shape == (M, N)
    tol = TOL_F32 if yt == torch.float32 else TOL_BF16
    bound = np.abs(x) @ np.abs(wdeq) + bound_extra
    e = normwise(y.float().cpu().numpy(), ref, bound)
    print(f"  error {e:.2e}", flush=True)
    assert e <= tol
    # no f32 copy of the weight in the workspace
    if K * N >= 1 << 16:
        need = L.lib().unifur_nf4_linear_workspace_size(M, K, N, L.F32, r)
        assert need < K * N * 4, need


@pytest.mark.parametrize("case", [
    # (rows, d_in, d_out, rank, striped, dq, dx dtype)
    (2048, 4096, 4096, 16, True, True, torch.float32),    # the config-3 shapes in reverse, f32 dY
    (100, 100, 192, 4, True, True, torch.float32),        # d_in 100: a partial output tile
    (300, 896, 4864, 0, True, True, torch.float32),       # no adapter, config-5 gate shape in reverse
    (77, 512, 384, 8, False, False, torch.bfloat16),      # row-major, f32 scales, bf16 dX
])
def test_f32_backward_dx(device, oracle, case):
    M, K, N, r, striped, dq, dxt = case
    print(f"f32 backward {case}", flush=True)
    lin, wdeq = make_linear(oracle, K, N, 6100 + M + K, device, dq=dq, striped=striped)
    dy, dyt = acts(oracle, M, N, 6101, torch.float32, device)
    if r:
        s = 16.0 / r
        a, b, ad = lora_parts(oracle, K, N, r, 6102 + r, device, scaling=s)
        x, xt = acts(oracle, M, K, 6103, torch.float32, device)
        dx, ga, gb = Q.QloraLinear(lin, ad).backward(xt, dyt, dx_dtype=dxt)
        rdx, bdx, rga, bga, rgb, bgb = linear_backward_ref_f64(x, dy, wdeq, a, b, s)
        assert normwise(ga.cpu(), rga, bga) <= 1e-5 and normwise(gb.cpu(), rgb, bgb) <= 1e-5
    else:
        dx = lin.backward(dyt, dx_dtype=dxt)
        d64, w64 = np.asarray(dy, np.float64), np.asarray(wdeq, np.float64)
        rdx, bdx = d64 @ w64.T, np.abs(d64) @ np.abs(w64).T
    tol = TOL_F32 if dxt == torch.float32 else TOL_BF16
    e = normwise(dx.float().cpu().numpy(), rdx, bdx)
    print(f"  dx error {e:.2e}", flush=True)
    assert e <= tol and dx.shape == (M, K)
    if K * N >= 1 << 20:  # where an f32 weight copy would dominate the adapter gradients' scratch
        need = L.lib().unifur_nf4_linear_backward_workspace_size(M, K, N, L.F32, r)
        assert need < K * N * 4, need


@pytest.mark.parametrize("rows", [100, 512])
def test_f32_swiglu(device, oracle, rows):
    hidden, inter = 512, 1024
    lg, wg = make_linear(oracle, hidden, inter, 6200, device)
    lu, wu = make_linear(oracle, hidden, inter, 6201, device)
    ld, wd = make_linear(oracle, inter, hidden, 6202, device)
    x, xt = acts(oracle, rows, hidden, 6203, torch.float32, device)
    y = Q.QwenMlp(lg, lu, ld).forward(xt)
    ref = oracle.swiglu_ref_f64(x, wg, wu, wd)
    h = oracle.silu_f64(x @ wg) * (x @ wu)
    bound = np.abs(h) @ np.abs(wd)
    e = normwise(y.cpu().numpy(), ref, bound)
    print(f"f32 swiglu rows {rows}: {e:.2e}", flush=True)
    assert e <= TOL_F32
