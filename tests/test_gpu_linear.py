"""GPU parity of the NF4 linear path (GEMV, generic GEMM, QLoRA, SwiGLU).

The reference value is the float64 product of the same inputs with the
oracle's dequantized weight (bit-identical to the reference's dequantized
f32 weight).  Tolerances, from BASELINE.json's north star:
  * f32 activations / f32 output: normwise error <= 1e-5 and
    max|y - r| / max|r| <= 1e-5;
  * bf16 activations or bf16 output: both <= 1e-2.
Normwise error is max_n |y_n - r_n| / sum_k |x_k| |W_kn| (elementwise
relative error is unbounded near zero outputs).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from unifur_amd import quantize as Q

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5
TOL_BF16 = 1e-2


def make_linear(oracle, d_in, d_out, seed, device, dq=True, sigma=0.02, striped=None):
    """Nf4Linear from seeded [d_in, d_out] values; returns (layer, W_deq f32).
    striped=None lets the layer pick (striped when d_out % 64 == 0)."""
    v = oracle.fill_normal(seed, sigma, d_in * d_out)
    packed, absmax = oracle.quantize_packed(v)
    if dq:
        q, sos = oracle.double_quantize(absmax)
        wdeq = oracle.dequantize_packed(packed, v.size, None, q, sos)
    else:
        wdeq = oracle.dequantize_packed(packed, v.size, absmax)
    p = Q.PackedNf4Tensor.quantize(torch.from_numpy(v).to(device))
    if dq:
        p = p.with_double_quantization()
    assert np.array_equal(p.codes.cpu().numpy(), packed)
    lin = Q.Nf4Linear.from_packed(p, d_in, d_out, striped=striped)
    # either layout gives back the reference's packed bytes
    assert np.array_equal(lin.packed().codes.cpu().numpy(), packed)
    return lin, wdeq.reshape(d_in, d_out)


def check(y, ref, x, wdeq, tol, tag):
    y = y.float().cpu().numpy().reshape(ref.shape)
    bound = np.abs(np.asarray(x, np.float64)) @ np.abs(np.asarray(wdeq, np.float64))
    from oracle import oracle as O
    nw = O.normwise_error(y, ref, x, bound)
    lit = O.max_rel_error(y, ref)
    print(f"{tag}: normwise {nw:.3e} literal {lit:.3e}", flush=True)
    assert nw <= tol and lit <= tol, f"{tag}: normwise {nw:.3e}, literal {lit:.3e} > {tol}"


def acts(oracle, rows, d_in, seed, dtype, device):
    x = oracle.fill_normal(seed, 1.0, rows * d_in).reshape(rows, d_in)
    if dtype == torch.bfloat16:
        x = oracle.round_bf16(x).reshape(rows, d_in)
    return x, torch.from_numpy(x).to(device).to(dtype)


def test_orientation_known_answer(device, oracle):
    # src/qwennet.rs:2196-2211: W [[1,2,3],[4,5,6]] as [in=2, out=3], x = [1, -1]
    v = np.arange(1, 7, dtype=np.float32)
    lin = Q.Nf4Linear.from_values(torch.from_numpy(v).to(device), 2, 3)
    w = lin.dequantized_weight().cpu().numpy().astype(np.float64)
    y = lin.forward(torch.tensor([[1.0, -1.0]], device=device)).cpu().numpy()
    assert np.allclose(y, [w[0] - w[1]], rtol=0, atol=1e-6)
    # the dequantized weight keeps each row's largest value exact (absmax endpoint)
    assert w[1, 2] == pytest.approx(6.0, abs=6 * 2 / 255)


@pytest.mark.parametrize("striped", [True, False])
@pytest.mark.parametrize("dq", [True, False])
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
def test_gemv_config2_4096_to_11008(device, oracle, dq, x_dtype, striped):
    # x[1, 4096] ~ N(0,1), W logical 11008x4096 stored [4096, 11008]
    lin, wdeq = make_linear(oracle, 4096, 11008, 0x4E463457 + 1, device, dq=dq, striped=striped)
    assert lin.is_striped() == striped
    x, xt = acts(oracle, 1, 4096, 0x58 + 1, x_dtype, device)
    ref = oracle.linear_ref_f64(x, wdeq)
    y = lin.forward(xt, out_dtype=torch.float32)
    tol = TOL_F32 if x_dtype == torch.float32 else TOL_BF16
    check(y, ref, x, wdeq, tol, f"gemv dq={dq} x={x_dtype}")
    yb = lin.forward(xt, out_dtype=torch.bfloat16)
    check(yb, ref, x, wdeq, TOL_BF16, f"gemv bf16-out dq={dq}")
    # deterministic: the split-K reduction runs in a fixed order
    assert torch.equal(lin.forward(xt, out_dtype=torch.float32), y)


@pytest.mark.parametrize("striped", [True, False])
@pytest.mark.parametrize("rows", [1, 2, 3, 4])
@pytest.mark.parametrize("shape", [(896, 4864), (4864, 896), (896, 128), (256, 64), (4096, 4096), (100, 192),
                                   (11008, 4096), (64, 128), (192, 256), (320, 896)])
def test_gemv_rows_and_shapes(device, oracle, rows, shape, striped):
    d_in, d_out = shape
    lin, wdeq = make_linear(oracle, d_in, d_out, 11 + d_in + d_out, device, striped=striped)
    x, xt = acts(oracle, rows, d_in, 5 + rows, torch.float32, device)
    check(lin.forward(xt), oracle.linear_ref_f64(x, wdeq), x, wdeq, TOL_F32, f"gemv rows={rows} {shape}")


@pytest.mark.parametrize("rows", [1, 2, 3, 4])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_striped_gemv_one_row_per_lane(device, oracle, rows, dt):
    # The striped GEMV takes two rows per lane (paired loads) when d_in is
    # even and x is aligned for the pairs; an odd d_in, or x one element off
    # that alignment, takes one row per lane.  Both against the oracle.
    tol = TOL_F32 if dt == torch.float32 else TOL_BF16
    lin, wdeq = make_linear(oracle, 1001, 192, 0x1001, device, striped=True)
    x, xt = acts(oracle, rows, 1001, 0x1002 + rows, dt, device)
    check(lin.forward(xt, out_dtype=torch.float32), oracle.linear_ref_f64(x, wdeq), x, wdeq, tol,
          f"odd d_in rows={rows} {dt}")
    lin, wdeq = make_linear(oracle, 1024, 192, 0x1003, device, striped=True)
    x, xt = acts(oracle, rows, 1024, 0x1004 + rows, dt, device)
    buf = torch.empty(rows * 1024 + 1, dtype=dt, device=device)
    xs = buf[1:].view(rows, 1024)
    xs.copy_(xt)
    assert xs.data_ptr() % (8 if dt == torch.float32 else 4) != 0
    ref = oracle.linear_ref_f64(x, wdeq)
    y = lin.forward(xs, out_dtype=torch.float32)
    check(y, ref, x, wdeq, tol, f"x off alignment rows={rows} {dt}")
    y2 = lin.forward(xt, out_dtype=torch.float32)  # aligned: two rows per lane
    check(y2, ref, x, wdeq, tol, f"aligned rows={rows} {dt}")


@pytest.mark.parametrize("striped", [True, False])
def test_gemv_bias_and_qlora(device, oracle, striped):
    d_in, d_out, r = 4096, 4096, 16
    lin, wdeq = make_linear(oracle, d_in, d_out, 21, device, dq=True, striped=striped)
    bias = oracle.fill_normal(22, 0.1, d_out)
    lin.bias = torch.from_numpy(bias).to(device)
    x, xt = acts(oracle, 2, d_in, 23, torch.float32, device)
    ref = oracle.linear_ref_f64(x, wdeq, bias)
    check(lin.forward(xt), ref, x, wdeq, TOL_F32, "gemv bias")
    a = oracle.fill_normal(0x41, 0.01, d_in * r).reshape(d_in, r)
    b = oracle.fill_normal(0x42, 0.01, r * d_out).reshape(r, d_out)
    ad = Q.LoraAdapter.from_parts(torch.from_numpy(a).to(device), torch.from_numpy(b).to(device), 2.0)
    ql = Q.QloraLinear(lin, ad)
    ref_l = ref + oracle.lora_ref_f64(x, a, b, 2.0)
    check(ql.forward(xt), ref_l, x, wdeq, TOL_F32, "gemv qlora")
    # a fresh adapter (B = 0) is an exact no-op (src/quantize.rs:1059-1081)
    fresh = Q.LoraAdapter.new(Q.LoraConfig.new(d_in, d_out, r), device=device)
    assert torch.equal(Q.QloraLinear(lin, fresh).forward(xt), lin.forward(xt))


@pytest.mark.parametrize("shape,rows,dt", [((8, 6), 4, torch.float32), ((100, 70), 1, torch.float32),
                                          ((96, 130), 5, torch.bfloat16), ((256, 512), 9, torch.float32),
                                          ((4096, 4096), 16, torch.float32)])
def test_generic_path_dequantize_then_matmul(device, oracle, shape, rows, dt):
    # d_out not a multiple of 64, or f32 activations with more than 4 rows:
    # the reference's own dequantize + f32 matmul sequence.
    d_in, d_out = shape
    lin, wdeq = make_linear(oracle, d_in, d_out, 31 + d_in, device, dq=True, sigma=1.0)
    x, xt = acts(oracle, rows, d_in, 33, dt, device)
    tol = TOL_F32 if dt == torch.float32 else TOL_BF16
    check(lin.forward(xt, out_dtype=torch.float32), oracle.linear_ref_f64(x, wdeq), x, wdeq, tol,
          f"generic {shape} rows={rows}")


@pytest.mark.parametrize("striped", [True, False])
@pytest.mark.parametrize("rows", [1, 2, 3, 4, 7])
def test_swiglu_small(device, oracle, rows, striped):
    hidden, inter = 256, 512
    g, wg = make_linear(oracle, hidden, inter, 41, device, striped=striped)
    u, wu = make_linear(oracle, hidden, inter, 42, device, striped=striped)
    d, wd = make_linear(oracle, inter, hidden, 43, device, striped=striped)
    mlp = Q.QwenMlp(g, u, d)
    x, xt = acts(oracle, rows, hidden, 44, torch.float32, device)
    ref = oracle.swiglu_ref_f64(x, wg, wu, wd)
    h = oracle.silu_f64(x.astype(np.float64) @ wg) * (x.astype(np.float64) @ wu)
    check(mlp.forward(xt), ref, h, wd, TOL_F32, f"swiglu rows={rows}")


@pytest.mark.parametrize("striped", [True, False])
@pytest.mark.parametrize("T", [1, 16, 512])
def test_swiglu_config4(device, oracle, T, striped):
    # hidden 4096, intermediate 11008, bf16 x, T = 1, 16, 512
    # (T = 1: GEMV pair; T = 16 and 512: the MFMA GEMMs with a bf16 middle)
    g, wg = make_linear(oracle, 4096, 11008, 0x4E463457 + 4, device, striped=striped)
    u, wu = make_linear(oracle, 4096, 11008, 0x4E463457 + 5, device, striped=striped)
    d, wd = make_linear(oracle, 11008, 4096, 0x4E463457 + 6, device, striped=striped)
    x, xt = acts(oracle, T, 4096, 0x58 + 4, torch.bfloat16, device)
    ref = oracle.swiglu_ref_f64(x, wg, wu, wd)
    h = oracle.silu_f64(x.astype(np.float64) @ wg) * (x.astype(np.float64) @ wu)
    y = Q.QwenMlp(g, u, d).forward(xt, out_dtype=torch.float32)
    check(y, ref, h, wd, TOL_BF16, f"swiglu config4 T={T} striped={striped}")


@pytest.mark.parametrize("T", [200, 600])
@pytest.mark.parametrize("striped", [True, False])
def test_swiglu_prefill_expanded_and_fused(device, oracle, striped, T):
    # more than 64 rows: with the default workspace up to 512 rows take the
    # fused MFMA kernels (split-K where their grid is small), more rows expand
    # each weight to bf16 for the BLAS GEMM; with the minimum workspace the
    # fused kernels over whole d_in run; all within the bf16 tolerance
    from unifur_amd import _lib as L
    import ctypes
    hidden, inter = 1024, 2816
    g, wg = make_linear(oracle, hidden, inter, 61, device, striped=striped)
    u, wu = make_linear(oracle, hidden, inter, 62, device, striped=striped)
    d, wd = make_linear(oracle, inter, hidden, 63, device, striped=striped)
    x, xt = acts(oracle, T, hidden, 64, torch.bfloat16, device)
    ref = oracle.swiglu_ref_f64(x, wg, wu, wd)
    h = oracle.silu_f64(x.astype(np.float64) @ wg) * (x.astype(np.float64) @ wu)
    full = L.lib().unifur_nf4_swiglu_workspace_size(T, hidden, inter, L.BF16)
    lean = L.lib().unifur_nf4_swiglu_min_workspace_size(T, hidden, inter, L.BF16)
    if T > 512:
        assert full > lean + 2 * hidden * inter * 2  # the expanded gate and up weights
    else:
        assert lean < full < lean + hidden * inter * 2  # split-K partials, no expanded weight
    gs, us, ds = g.weight_struct(), u.weight_struct(), d.weight_struct()
    stream = torch.cuda.current_stream().cuda_stream
    for need in (full, lean):
        ws = torch.zeros(need, dtype=torch.uint8, device=device)
        y = torch.empty(T, hidden, device=device)
        L.check(L.lib().unifur_nf4_swiglu_forward(xt.data_ptr(), L.BF16, T, ctypes.byref(gs), ctypes.byref(us),
                                                  ctypes.byref(ds), y.data_ptr(), L.F32, ws.data_ptr(), need, stream))
        check(y, ref, h, wd, TOL_BF16, f"swiglu T={T} workspace {need}")


def test_swiglu_decode_repeated_on_one_workspace(device, oracle):
    # Decode SwiGLU calls of two shapes and both pair row counts, one after
    # another on one zero-filled caller workspace: each matches the oracle
    # and leaves the workspace's counter region zero (its contract).
    from unifur_amd import _lib as L
    import ctypes
    shapes = [(896, 4864, 71), (256, 512, 75)]
    mlps = []
    for hidden, inter, seed in shapes:
        g, wg = make_linear(oracle, hidden, inter, seed, device, striped=True)
        u, wu = make_linear(oracle, hidden, inter, seed + 1, device, striped=True)
        d, wd = make_linear(oracle, inter, hidden, seed + 2, device, striped=True)
        mlps.append((hidden, inter, (g, u, d), (wg, wu, wd)))
    need = max(L.lib().unifur_nf4_swiglu_workspace_size(2, h_, i_, L.F32) for h_, i_, _ in shapes)
    ws = torch.zeros(need, dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream().cuda_stream
    for call, (k, rows) in enumerate([(0, 1), (1, 2), (0, 2), (1, 1), (0, 1)]):
        hidden, inter, (g, u, d), (wg, wu, wd) = mlps[k]
        x, xt = acts(oracle, rows, hidden, 80 + call, torch.float32, device)
        gs, us, ds = g.weight_struct(), u.weight_struct(), d.weight_struct()
        y = torch.empty(rows, hidden, device=device)
        L.check(L.lib().unifur_nf4_swiglu_forward(xt.data_ptr(), L.F32, rows, ctypes.byref(gs), ctypes.byref(us),
                                                  ctypes.byref(ds), y.data_ptr(), L.F32, ws.data_ptr(), need,
                                                  stream))
        ref = oracle.swiglu_ref_f64(x, wg, wu, wd)
        h = oracle.silu_f64(x.astype(np.float64) @ wg) * (x.astype(np.float64) @ wu)
        check(y, ref, h, wd, TOL_F32, f"swiglu call {call} shape {hidden}x{inter} rows={rows}")
        assert int(ws[:64 << 10].count_nonzero()) == 0, f"counter region not left zero after call {call}"


def test_workspace_shared_by_generic_then_gemv_calls(device, oracle):
    # A generic-path call writes an f32 weight copy into the workspace; the
    # GEMV's split-K arrival counters live in a region nothing else touches,
    # so a later GEMV on the same workspace is still correct.
    from unifur_amd import _lib as L
    import ctypes
    small, wsmall = make_linear(oracle, 64, 70, 51, device, sigma=1.0)    # generic (70 % 64 != 0)
    big, wbig = make_linear(oracle, 4096, 4096, 52, device, striped=False)  # row-major GEMV, split-K
    need = max(L.lib().unifur_nf4_linear_workspace_size(1, 64, 70, 0, 0),
               L.lib().unifur_nf4_linear_workspace_size(1, 4096, 4096, 0, 0))
    ws = torch.zeros(need, dtype=torch.uint8, device=device)
    xs, xst = acts(oracle, 1, 64, 53, torch.float32, device)
    xb, xbt = acts(oracle, 1, 4096, 54, torch.float32, device)
    stream = torch.cuda.current_stream().cuda_stream
    for _ in range(3):
        for lin, xt, x, wd in ((small, xst, xs, wsmall), (big, xbt, xb, wbig)):
            y = torch.empty(1, lin.d_output(), device=device)
            w = lin.weight_struct()
            L.check(L.lib().unifur_nf4_linear_forward(xt.data_ptr(), L.F32, 1, ctypes.byref(w), None, None,
                                                      y.data_ptr(), L.F32, ws.data_ptr(), need, stream))
            check(y, oracle.linear_ref_f64(x, wd), x, wd, TOL_F32, f"shared ws {lin.d_output()}")
    assert int(ws[:65536].count_nonzero()) == 0, "counter region must be left zeroed"
