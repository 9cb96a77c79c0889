"""GPU parity of the shared-input launch (QwenFullAttention's q, k, v
projections of one hidden state, src/qwennet.rs:927-956): each output against
the float64 product with the oracle's dequantized weight, to the tolerance of
its activation type (f32 1e-5, bf16 1e-2), for the fused GEMV (<= 4 rows) and
skinny (5..64 bf16 rows) launches and for the calls that fall back to one
linear at a time (more rows, a row-major weight, mixed scale kinds)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from unifur_amd import _lib as L
from unifur_amd import quantize as Q

from test_gpu_linear import TOL_BF16, TOL_F32, acts, check, make_linear

pytestmark = pytest.mark.gpu


def qkv(oracle, device, hidden=896, kv=128, kinds=(True, True, True), striped=(True, True, True), seed=1700):
    outs = []
    for i, d_out in enumerate((hidden, kv, kv)):
        lin, wdeq = make_linear(oracle, hidden, d_out, seed + i, device, dq=kinds[i], striped=striped[i])
        b = oracle.fill_normal(seed + 10 + i, 0.1, d_out)
        lin.bias = torch.from_numpy(b).to(device)
        outs.append((lin, wdeq, b))
    return outs


@pytest.mark.parametrize("rows,dt", [(1, torch.float32), (2, torch.float32), (4, torch.float32), (1, torch.bfloat16),
                                     (7, torch.bfloat16), (32, torch.bfloat16), (64, torch.bfloat16),
                                     (100, torch.bfloat16), (9, torch.float32)])
def test_qkv_shared_input(device, oracle, rows, dt):
    layers = qkv(oracle, device)
    x, xt = acts(oracle, rows, 896, 1750 + rows, dt, device)
    ys = Q.forward_shared_input(xt, [l for l, _, _ in layers], out_dtype=torch.float32)
    tol = TOL_F32 if dt == torch.float32 else TOL_BF16
    for (lin, wdeq, b), y in zip(layers, ys):
        assert y.shape == (rows, lin.d_output())
        check(y, oracle.linear_ref_f64(x, wdeq, b), x, wdeq, tol, f"qkv rows={rows} d_out={lin.d_output()}")


@pytest.mark.parametrize("rows,dt", [(1, torch.float32), (3, torch.float32), (16, torch.bfloat16),
                                     (40, torch.bfloat16)])
def test_qkv_shared_input_grid_off_the_xcds(device, oracle, rows, dt):
    """hidden 960 and kv 64: 60 + 4 + 4 = 68 stripes, so the launch's
    workgroups (68, or 68 / stripes per wave) are not a multiple of the 8
    XCDs and keep their plain order, while the workgroups of k and v take
    their weight slots (1 and 2) by the selects over the argument block."""
    layers = qkv(oracle, device, hidden=960, kv=64, seed=1900)
    x, xt = acts(oracle, rows, 960, 1950 + rows, dt, device)
    ys = Q.forward_shared_input(xt, [l for l, _, _ in layers], out_dtype=torch.float32)
    tol = TOL_F32 if dt == torch.float32 else TOL_BF16
    for (lin, wdeq, b), y in zip(layers, ys):
        check(y, oracle.linear_ref_f64(x, wdeq, b), x, wdeq, tol, f"qkv 960/64 rows={rows} d_out={lin.d_output()}")


@pytest.mark.parametrize("variant", ["mixed_kinds", "row_major", "two", "one"])
def test_fallbacks_and_counts(device, oracle, variant):
    kinds, striped, n = (True, True, True), (True, True, True), 3
    if variant == "mixed_kinds":
        kinds = (True, False, True)
    if variant == "row_major":
        striped = (True, False, True)
    if variant == "two":
        n = 2
    if variant == "one":
        n = 1
    layers = qkv(oracle, device, kinds=kinds, striped=striped, seed=1800)[:n]
    x, xt = acts(oracle, 3, 896, 1801, torch.float32, device)
    ys = Q.forward_shared_input(xt, [l for l, _, _ in layers])
    for (lin, wdeq, b), y in zip(layers, ys):
        check(y, oracle.linear_ref_f64(x, wdeq, b), x, wdeq, TOL_F32, f"{variant} d_out={lin.d_output()}")


def test_bad_arguments(device, oracle):
    layers = qkv(oracle, device, seed=1900)
    other, _ = make_linear(oracle, 128, 64, 1910, device)
    x, xt = acts(oracle, 2, 896, 1901, torch.float32, device)
    with pytest.raises(ValueError):
        Q.forward_shared_input(xt, [layers[0][0], other])
    with pytest.raises(ValueError):
        Q.forward_shared_input(xt, [l for l, _, _ in layers] + [layers[0][0]])
    assert L.lib().unifur_nf4_linear_multi_workspace_size(1, 896, None, 3, L.F32) == 0
