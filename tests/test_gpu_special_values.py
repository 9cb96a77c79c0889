"""Non-finite weights through every linear path.

With f32 block scales a block holding an infinity has an infinite absmax,
so its dequantized values are +-inf (level * inf) and NaN where the level is
0 (0 * inf), as the reference's PackedNf4Tensor::dequantize gives them
(src/quantize.rs:355-366; the oracle restates it bit for bit); with double
quantization the infinity reaches every block scale (the second test).  Nf4Linear::forward
(src/qwennet.rs:238-241) then sums x_k W[k][j]: a column meeting NaN, or
both +inf and -inf, is NaN, one meeting infinities of one sign only is that
infinity -- whatever the order of the sum.  So the pattern of non-finite
outputs is fixed, and each path must reproduce it exactly while its finite
outputs keep their bar against the float64 product."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from unifur_amd import _lib as L
from unifur_amd import quantize as Q

from test_gpu_linear import TOL_BF16, TOL_F32, acts

pytestmark = pytest.mark.gpu


def weight_with_inf_blocks(oracle, d_in, d_out, seed, dq, striped, device):
    v = oracle.fill_normal(seed, 0.02, d_in * d_out)
    # rows 3 and d_in - 2: an infinity in one 64-column block each (one
    # positive, one negative), so those blocks dequantize to +-inf / NaN
    v[3 * d_out + 70] = np.inf
    v[(d_in - 2) * d_out + 5] = -np.inf
    packed, absmax = oracle.quantize_packed(v)
    if dq:
        q, sos = oracle.double_quantize(absmax)
        wdeq = oracle.dequantize_packed(packed, v.size, None, q, sos)
    else:
        wdeq = oracle.dequantize_packed(packed, v.size, absmax)
    p = Q.PackedNf4Tensor.quantize(torch.from_numpy(v).to(device))
    if dq:
        p = p.with_double_quantization()
    return Q.Nf4Linear.from_packed(p, d_in, d_out, striped=striped), wdeq.reshape(d_in, d_out)


PATHS = [
    (1, torch.float32, "default"),     # striped GEMV
    (3, torch.bfloat16, "default"),    # GEMV, bf16 x
    (16, torch.bfloat16, "default"),   # skinny MFMA
    (24, torch.float32, "default"),    # skinny, f32 operands
    (128, torch.bfloat16, "default"),  # expanded weight + BLAS GEMM
    (128, torch.bfloat16, "least"),    # fused MFMA kernel
    (100, torch.float32, "default"),   # f32 MFMA GEMM
]


def run_linear(lin, xt, rows, d_in, d_out, xdt, work, device):
    lib = L.lib()
    dt = L.BF16 if xdt == torch.bfloat16 else L.F32
    size = lib.unifur_nf4_linear_workspace_size if work == "default" else lib.unifur_nf4_linear_min_workspace_size
    need = size(rows, d_in, d_out, dt, 0)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=device)
    w = lin.weight_struct()
    y = torch.empty(rows, d_out, device=device)
    L.check(lib.unifur_nf4_linear_forward(xt.data_ptr(), dt, rows, ctypes.byref(w), None, None, y.data_ptr(), L.F32,
                                          ws.data_ptr(), need, torch.cuda.current_stream().cuda_stream))
    return y.cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("rows,xdt,work", PATHS)
def test_infinite_blocks_propagate_as_the_reference_sums_them(device, oracle, rows, xdt, work):
    """f32 block scales: the two blocks holding an infinity dequantize to
    NaN (level 0) and +-inf, the other blocks stay finite."""
    d_in, d_out = 256, 192
    print(f"non-finite weight: rows {rows} {xdt} {work}", flush=True)
    lin, wdeq = weight_with_inf_blocks(oracle, d_in, d_out, 0x1AF0 + rows, False, True, device)
    assert np.isinf(wdeq).any() and np.isnan(wdeq).any()
    x, xt = acts(oracle, rows, d_in, 0x1AF1 + rows, xdt, device)
    with np.errstate(invalid="ignore", over="ignore"):
        ref = x.astype(np.float64) @ wdeq.astype(np.float64)
        bound = np.abs(x.astype(np.float64)) @ np.abs(wdeq.astype(np.float64))
    got = run_linear(lin, xt, rows, d_in, d_out, xdt, work, device)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "NaN outputs differ"
    assert np.array_equal(np.isposinf(got), np.isposinf(ref)) and np.array_equal(np.isneginf(got), np.isneginf(ref))
    fin = np.isfinite(ref)
    assert fin.any() and not fin.all()
    tol = TOL_F32 if xdt == torch.float32 else TOL_BF16
    nw = float(np.max(np.abs(got[fin] - ref[fin]) / bound[fin]))
    print(f"  {int((~fin).sum())} non-finite outputs, finite normwise {nw:.2e}", flush=True)
    assert nw <= tol


@pytest.mark.parametrize("rows,xdt,work", PATHS)
def test_double_quantized_infinite_block_poisons_every_output(device, oracle, rows, xdt, work):
    """With double quantization an infinite absmax makes the scale of scales
    infinite and every u8 scale code 0 (s / inf; inf / inf is NaN, which
    encodes as 0), so every block scale is (0 / 255) * inf = NaN
    (src/quantize.rs:126-149, :349): the whole weight, and every output, is
    NaN -- on the reference's CPU path and on each of these paths."""
    d_in, d_out = 256, 192
    print(f"non-finite DQ weight: rows {rows} {xdt} {work}", flush=True)
    lin, wdeq = weight_with_inf_blocks(oracle, d_in, d_out, 0x1AF8 + rows, True, True, device)
    assert np.isnan(wdeq).all()
    x, xt = acts(oracle, rows, d_in, 0x1AF9 + rows, xdt, device)
    assert np.isnan(run_linear(lin, xt, rows, d_in, d_out, xdt, work, device)).all()


@pytest.mark.parametrize("rows,xdt,work", PATHS)
def test_non_finite_activations_propagate(device, oracle, rows, xdt, work):
    """x with an infinity and a NaN in two of its rows and finite weights
    (double-quantized): inf * w is +-inf, inf * 0 (a weight of level 0) NaN,
    and a NaN reaches its row's every output -- the pattern the float64
    product gives, whatever the order of the sum; the untouched rows keep
    their bar."""
    from test_gpu_linear import make_linear
    d_in, d_out = 256, 192
    print(f"non-finite x: rows {rows} {xdt} {work}", flush=True)
    lin, wdeq = make_linear(oracle, d_in, d_out, 0x1B00 + rows, device, striped=True)
    x, _ = acts(oracle, rows, d_in, 0x1B01 + rows, xdt, device)
    x = x.copy()
    x[0, 5] = np.inf
    x[rows - 1, 77] = np.nan
    if rows > 2:
        x[1, 200] = -np.inf
    xt = torch.from_numpy(x).to(device).to(xdt)
    with np.errstate(invalid="ignore", over="ignore"):
        ref = x.astype(np.float64) @ wdeq.astype(np.float64)
        bound = np.abs(x.astype(np.float64)) @ np.abs(wdeq.astype(np.float64))
    got = run_linear(lin, xt, rows, d_in, d_out, xdt, work, device)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "NaN outputs differ"
    assert np.array_equal(np.isposinf(got), np.isposinf(ref)) and np.array_equal(np.isneginf(got), np.isneginf(ref))
    fin = np.isfinite(ref)
    assert not fin.all()
    if fin.any():
        tol = TOL_F32 if xdt == torch.float32 else TOL_BF16
        assert float(np.max(np.abs(got[fin] - ref[fin]) / bound[fin])) <= tol
