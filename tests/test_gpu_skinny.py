"""GPU parity of the skinny MFMA path: 5..64 bf16 activation rows over a
striped NF4 weight (the medium batches between the decode GEMV and the
prefill GEMM: speculative decode, small batches, config 4 at T = 16).

The weight operand is bf16(level * scale), x is bf16: the bf16 tolerance of
BASELINE.json's north star applies (normwise and max|y - r| / max|r| both
<= 1e-2 against the float64 product with the oracle's dequantized weight).
Token counts straddle the 16-token MFMA tiles; d_in values leave partial
64-row chunks and partial 16-row lane groups (d_in % 64 = 8, 40), which is
where a transposed-operand index mistake would show.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from unifur_amd import _lib as L
from unifur_amd import quantize as Q

from test_gpu_gemm import lora_parts
from test_gpu_linear import TOL_BF16, TOL_F32, acts, check, make_linear

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T", [5, 8, 16, 17, 31, 32, 33, 48, 63, 64])
@pytest.mark.parametrize("dq", [True, False])
def test_token_counts_and_scale_kinds(device, oracle, T, dq):
    K, N = 1024, 512
    lin, wdeq = make_linear(oracle, K, N, 700 + T, device, dq=dq, striped=True)
    x, xt = acts(oracle, T, K, 701 + T, torch.bfloat16, device)
    ref = oracle.linear_ref_f64(x, wdeq)
    check(lin.forward(xt, out_dtype=torch.float32), ref, x, wdeq, TOL_BF16, f"skinny T={T} dq={dq}")
    check(lin.forward(xt, out_dtype=torch.bfloat16), ref, x, wdeq, TOL_BF16, f"skinny T={T} dq={dq} bf16-out")


# d_out 11008 and 8192 put four and two stripes on each wave (one activation
# load feeds them all); the others one
@pytest.mark.parametrize("shape", [(904, 192), (200, 128), (40, 64), (8, 64), (896, 4864), (4864, 896),
                                   (4096, 1024), (904, 11008), (200, 8192)])
@pytest.mark.parametrize("T", [7, 32, 64])
def test_ragged_d_in_and_qwen_shapes(device, oracle, shape, T):
    K, N = shape
    lin, wdeq = make_linear(oracle, K, N, 800 + K + N + T, device, striped=True)
    x, xt = acts(oracle, T, K, 801 + T, torch.bfloat16, device)
    check(lin.forward(xt, out_dtype=torch.float32), oracle.linear_ref_f64(x, wdeq), x, wdeq, TOL_BF16,
          f"skinny {shape} T={T}")


@pytest.mark.parametrize("r", [1, 16, 64])
@pytest.mark.parametrize("T", [12, 40])
def test_bias_and_lora(device, oracle, r, T):
    K, N = 512, 256
    lin, wdeq = make_linear(oracle, K, N, 900 + r, device, striped=True)
    bias = oracle.fill_normal(901, 0.1, N)
    lin.bias = torch.from_numpy(bias).to(device)
    x, xt = acts(oracle, T, K, 902 + T, torch.bfloat16, device)
    a, b, ad = lora_parts(oracle, K, N, r, 903 + r, device, scaling=16.0 / r)
    ref = oracle.linear_ref_f64(x, wdeq, bias) + oracle.lora_ref_f64(x, a, b, 16.0 / r)
    y = Q.QloraLinear(lin, ad).forward(xt, out_dtype=torch.float32)
    check(y, ref, x, wdeq, TOL_BF16, f"skinny bias+lora r={r} T={T}")
    # fixed accumulation order: bit-identical on a second call
    assert torch.equal(Q.QloraLinear(lin, ad).forward(xt, out_dtype=torch.float32), y)


def test_misaligned_or_odd_d_in_falls_back_with_the_same_result(device, oracle):
    # d_in % 8 != 0 cannot take 16-byte activation loads: another path
    # serves it, within the same tolerance
    K, N, T = 100, 64, 9
    lin, wdeq = make_linear(oracle, K, N, 950, device, striped=True)
    x, xt = acts(oracle, T, K, 951, torch.bfloat16, device)
    check(lin.forward(xt, out_dtype=torch.float32), oracle.linear_ref_f64(x, wdeq), x, wdeq, TOL_BF16,
          "odd d_in")


def _swiglu_parts(oracle, hidden, inter, seed, device, kinds=(True, True, True)):
    ws, deqs = [], []
    for i, (din, dout) in enumerate([(hidden, inter), (hidden, inter), (inter, hidden)]):
        lin, wd = make_linear(oracle, din, dout, seed + i, device, dq=kinds[i], striped=True)
        ws.append(lin)
        deqs.append(wd)
    return ws, deqs


@pytest.mark.parametrize("T", [5, 16, 33, 64])
@pytest.mark.parametrize("kinds", [(True, True, True), (True, False, True), (False, False, False)])
def test_swiglu_pair_and_mixed_scale_kinds(device, oracle, T, kinds):
    hidden, inter = 256, 704
    (g, u, d), (wg, wu, wd) = _swiglu_parts(oracle, hidden, inter, 1000 + T, device, kinds)
    x, xt = acts(oracle, T, hidden, 1010 + T, torch.bfloat16, device)
    ref = oracle.swiglu_ref_f64(x, wg, wu, wd)
    mlp = Q.QwenMlp(g, u, d)
    y = mlp.forward(xt, out_dtype=torch.float32)
    # the down projection reads bf16(silu(g) * u); bound with |h| from the reference
    h = oracle.silu_f64(x.astype(np.float64) @ wg) * (x.astype(np.float64) @ wu)
    check(y, ref, h, wd, TOL_BF16, f"skinny swiglu T={T} kinds={kinds}")
    assert torch.equal(mlp.forward(xt, out_dtype=torch.float32), y)


def test_user_workspace_covers_mixed_kinds(device, oracle):
    hidden, inter, T = 256, 704, 24
    (g, u, d), (wg, wu, wd) = _swiglu_parts(oracle, hidden, inter, 1100, device, (True, False, True))
    x, xt = acts(oracle, T, hidden, 1101, torch.bfloat16, device)
    need = L.lib().unifur_nf4_swiglu_workspace_size(T, hidden, inter, L.BF16)
    assert need >= 65536 + T * inter * (2 + 4 + 4)
    ws = torch.zeros(need, dtype=torch.uint8, device=device)
    y = torch.empty(T, hidden, device=device)
    gs, us, ds = g.weight_struct(), u.weight_struct(), d.weight_struct()
    stream = torch.cuda.current_stream().cuda_stream
    L.check(L.lib().unifur_nf4_swiglu_forward(xt.data_ptr(), L.BF16, T, ctypes.byref(gs), ctypes.byref(us),
                                              ctypes.byref(ds), y.data_ptr(), L.F32, ws.data_ptr(), need, stream))
    h = oracle.silu_f64(x.astype(np.float64) @ wg) * (x.astype(np.float64) @ wu)
    check(y, oracle.swiglu_ref_f64(x, wg, wu, wd), h, wd, TOL_BF16, "skinny swiglu user workspace")


@pytest.mark.parametrize("T", [9, 24, 64])
def test_swiglu_pair_with_grouped_stripes(device, oracle, T):
    # intermediate 10240 (640 stripes): the gate/up pair runs four stripes per
    # wave at one token tile and two at more
    hidden, inter = 128, 10240
    (g, u, d), (wg, wu, wd) = _swiglu_parts(oracle, hidden, inter, 1200 + T, device)
    x, xt = acts(oracle, T, hidden, 1210 + T, torch.bfloat16, device)
    y = Q.QwenMlp(g, u, d).forward(xt, out_dtype=torch.float32)
    h = oracle.silu_f64(x.astype(np.float64) @ wg) * (x.astype(np.float64) @ wu)
    check(y, oracle.swiglu_ref_f64(x, wg, wu, wd), h, wd, TOL_BF16, f"skinny swiglu grouped T={T}")


@pytest.mark.parametrize("T", [16, 64])
def test_split_d_in_hand_off_with_user_workspace(device, oracle, T):
    # d_out 4096 over d_in 11008: four stripes per wave leave 64 stripe groups,
    # so d_in is split over workgroups and the last slab to arrive adds the
    # partial sums; the arrival counters must be left zeroed for the next call
    K, N = 11008, 4096
    lin, wdeq = make_linear(oracle, K, N, 1300 + T, device, striped=True)
    x, xt = acts(oracle, T, K, 1301 + T, torch.bfloat16, device)
    need = L.lib().unifur_nf4_linear_workspace_size(T, K, N, L.BF16, 0)
    assert need > 65536  # the counters and the partials
    ws = torch.zeros(need, dtype=torch.uint8, device=device)
    w = lin.weight_struct()
    stream = torch.cuda.current_stream().cuda_stream
    ref = oracle.linear_ref_f64(x, wdeq)
    outs = []
    for _ in range(2):
        y = torch.empty(T, N, device=device)
        L.check(L.lib().unifur_nf4_linear_forward(xt.data_ptr(), L.BF16, T, ctypes.byref(w), None, None, y.data_ptr(),
                                                  L.F32, ws.data_ptr(), need, stream))
        check(y, ref, x, wdeq, TOL_BF16, f"skinny split T={T}")
        assert int(ws[:65536].count_nonzero()) == 0
        outs.append(y)
    assert torch.equal(outs[0], outs[1])  # slabs added in a fixed order


# ---- f32 activations (v_mfma_f32_16x16x4_f32, exact f32 weight operand) ----
# The reference's own precision: the f32 bar (1e-5) of BASELINE.json's north
# star.  33..64 rows run as launches of at most 32 rows.

@pytest.mark.parametrize("T", [5, 8, 16, 17, 31, 32, 33, 48, 64])
@pytest.mark.parametrize("dq", [True, False])
def test_f32_token_counts_and_scale_kinds(device, oracle, T, dq):
    K, N = 1024, 512
    lin, wdeq = make_linear(oracle, K, N, 2700 + T, device, dq=dq, striped=True)
    x, xt = acts(oracle, T, K, 2701 + T, torch.float32, device)
    ref = oracle.linear_ref_f64(x, wdeq)
    check(lin.forward(xt), ref, x, wdeq, TOL_F32, f"skinny f32 T={T} dq={dq}")
    check(lin.forward(xt, out_dtype=torch.bfloat16), ref, x, wdeq, TOL_BF16, f"skinny f32 T={T} bf16-out")


@pytest.mark.parametrize("shape", [(904, 192), (40, 64), (896, 896), (896, 128), (896, 4864), (4864, 896),
                                   (904, 11008)])
@pytest.mark.parametrize("T", [7, 32, 64])
def test_f32_ragged_d_in_and_qwen_shapes(device, oracle, shape, T):
    K, N = shape
    lin, wdeq = make_linear(oracle, K, N, 2800 + K + N + T, device, striped=True)
    x, xt = acts(oracle, T, K, 2801 + T, torch.float32, device)
    y = lin.forward(xt)
    check(y, oracle.linear_ref_f64(x, wdeq), x, wdeq, TOL_F32, f"skinny f32 {shape} T={T}")
    assert torch.equal(lin.forward(xt), y)  # slabs added in a fixed order


@pytest.mark.parametrize("T", [12, 40])
def test_f32_bias_and_lora(device, oracle, T):
    K, N, r = 512, 256, 16
    lin, wdeq = make_linear(oracle, K, N, 2900, device, striped=True)
    bias = oracle.fill_normal(2901, 0.1, N)
    lin.bias = torch.from_numpy(bias).to(device)
    x, xt = acts(oracle, T, K, 2902 + T, torch.float32, device)
    a, b, ad = lora_parts(oracle, K, N, r, 2903, device, scaling=2.0)
    ref = oracle.linear_ref_f64(x, wdeq, bias) + oracle.lora_ref_f64(x, a, b, 2.0)
    y = Q.QloraLinear(lin, ad).forward(xt)
    bound_x = np.abs(x) @ np.abs(wdeq) + np.abs(x) @ np.abs(a) @ np.abs(b) * 2.0
    from oracle import oracle as O
    nw = O.normwise_error(y.cpu().numpy(), ref, x, bound_x)
    assert nw <= TOL_F32 and O.max_rel_error(y.cpu().numpy(), ref) <= TOL_F32, nw


@pytest.mark.parametrize("T", [5, 16, 32])
@pytest.mark.parametrize("kinds", [(True, True, True), (True, False, True)])
def test_f32_swiglu_keeps_an_f32_middle(device, oracle, T, kinds):
    hidden, inter = 896, 4864  # config 5's MLP
    (g, u, d), (wg, wu, wd) = _swiglu_parts(oracle, hidden, inter, 3000 + T, device, kinds)
    x, xt = acts(oracle, T, hidden, 3010 + T, torch.float32, device)
    y = Q.QwenMlp(g, u, d).forward(xt)
    h = oracle.silu_f64(x.astype(np.float64) @ wg) * (x.astype(np.float64) @ wu)
    check(y, oracle.swiglu_ref_f64(x, wg, wu, wd), h, wd, TOL_F32, f"skinny f32 swiglu T={T} kinds={kinds}")


@pytest.mark.parametrize("T", [6, 32])
def test_f32_shared_input_qkv(device, oracle, T):
    lins = [make_linear(oracle, 896, n, 3100 + n, device, striped=True) for n in (896, 128, 128)]
    x, xt = acts(oracle, T, 896, 3101 + T, torch.float32, device)
    ys = Q.forward_shared_input(xt, [l for l, _ in lins])
    for (lin, wdeq), y in zip(lins, ys):
        check(y, oracle.linear_ref_f64(x, wdeq), x, wdeq, TOL_F32, f"skinny f32 qkv T={T} d_out={lin.d_output()}")
