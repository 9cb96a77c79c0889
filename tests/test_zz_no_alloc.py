"""The allocation-free linear entry point (unifur_nf4_linear_forward_noalloc).

It has no counterpart in the reference: it is unifur_nf4_linear_forward for
callers that cannot allocate, running on a static per-GPU scratch.  Each case
calls it through the C ABI twice in a row -- the second call with a smaller
input, so that it runs on the scratch the first call left behind -- and
compares every output bit for bit with unifur_nf4_linear_forward given its
least workspace (unifur_nf4_linear_min_workspace_size: the same kernels), or,
for prefill calls without an adapter (the fused kernel's split-K partials
fit the scratch), given the scratch's 16 MiB; prefill cases are also checked
against the float64 product within the bf16 bar.  Calls alternating between
two streams are checked to come out in order.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from unifur_amd import _lib as L
from unifur_amd import quantize as Q

from test_gpu_gemm import lora_parts
from test_gpu_linear import TOL_BF16, acts, check, make_linear

pytestmark = pytest.mark.gpu


def _dt(t: torch.dtype) -> int:
    return L.BF16 if t == torch.bfloat16 else L.F32


SCRATCH = 16 << 20  # the allocation-free entry point's static scratch


def existing(lin, x, lora, y_dtype, bias=None, workspace=None):
    """unifur_nf4_linear_forward with the least workspace it accepts, or with
    ``workspace`` bytes."""
    lib = L.lib()
    w = lin.weight_struct()
    rows, d_in = x.shape
    rank = lora.rank if lora is not None else 0
    need = lib.unifur_nf4_linear_min_workspace_size(rows, d_in, lin.d_output(), _dt(x.dtype), rank)
    if workspace is not None:
        need = workspace
    ws = torch.zeros(max(int(need), 1), dtype=torch.uint8, device=x.device)
    y = torch.empty(rows, lin.d_output(), dtype=y_dtype, device=x.device)
    L.check(lib.unifur_nf4_linear_forward(x.data_ptr(), _dt(x.dtype), rows, ctypes.byref(w),
                                          bias.data_ptr() if bias is not None else None,
                                          ctypes.byref(lora) if lora is not None else None, y.data_ptr(),
                                          _dt(y_dtype), ws.data_ptr(), int(need),
                                          torch.cuda.current_stream().cuda_stream))
    return y


def noalloc(lin, x, lora, y_dtype, bias=None):
    lib = L.lib()
    w = lin.weight_struct()
    rows = x.shape[0]
    y = torch.empty(rows, lin.d_output(), dtype=y_dtype, device=x.device)
    L.check(lib.unifur_nf4_linear_forward_noalloc(x.data_ptr(), _dt(x.dtype), rows, ctypes.byref(w),
                                                  bias.data_ptr() if bias is not None else None,
                                                  ctypes.byref(lora) if lora is not None else None, y.data_ptr(),
                                                  _dt(y_dtype), torch.cuda.current_stream().cuda_stream))
    return y


@pytest.mark.parametrize("case", [
    # (rows of the first call, rows of the second, d_in, d_out, x dtype, y dtype, lora rank, striped)
    (4, 1, 4096, 11008, torch.float32, torch.float32, 0, True),      # config-2 GEMV
    (3, 1, 1024, 512, torch.bfloat16, torch.float32, 8, False),      # row-major GEMV with an adapter
    (48, 16, 4096, 11008, torch.bfloat16, torch.bfloat16, 0, True),  # skinny MFMA, split d_in
    (300, 100, 1024, 768, torch.bfloat16, torch.bfloat16, 16, True),  # fused prefill GEMM with LoRA
    (2048, 256, 4096, 4096, torch.bfloat16, torch.bfloat16, 16, True),  # config 3, then a smaller batch
    (20, 7, 512, 384, torch.float32, torch.float32, 4, False),      # generic dequantize + f32 GEMM
])
def test_noalloc_matches_linear_forward_twice(device, oracle, case):
    m1, m2, k, n, xt, yt, r, striped = case
    print(f"noalloc case {case}", flush=True)
    lin, wdeq = make_linear(oracle, k, n, 5000 + k + n, device, dq=True, striped=striped)
    lora = None
    if r:
        a, b, ad = lora_parts(oracle, k, n, r, 5001 + r, device)
        lora = ad.struct()
    bias = torch.from_numpy(oracle.fill_normal(5002, 0.1, n)).to(device)
    for m, seed in ((m1, 5003), (m2, 5004)):
        x, xd = acts(oracle, m, k, seed, xt, device)
        want = existing(lin, xd, lora, yt, bias)
        got = noalloc(lin, xd, lora, yt, bias)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"rows {m}: noalloc output differs from linear_forward"
        if m == m1 and m >= 300:
            ref = oracle.linear_ref_f64(x, wdeq, oracle.fill_normal(5002, 0.1, n))
            if r:
                ref = ref + oracle.lora_ref_f64(x, a, b, ad.scaling())
            check(got, ref, x, wdeq, TOL_BF16, f"noalloc rows {m}")


@pytest.mark.parametrize("rows", [(100, 40), (300, 130)])
def test_noalloc_split_k_without_adapter(device, oracle, rows):
    """Without an adapter the fused kernel's split-K partials fit the scratch
    (100 x 4096 x 4096 takes two d_in slabs): bit for bit what
    unifur_nf4_linear_forward gives with a 16 MiB workspace, and within the
    bf16 bar of the float64 product, twice in a row."""
    k = n = 4096
    print(f"noalloc split-K rows {rows}", flush=True)
    lin, wdeq = make_linear(oracle, k, n, 5200, device, dq=True, striped=True)
    bias = torch.from_numpy(oracle.fill_normal(5201, 0.1, n)).to(device)
    for m, seed in zip(rows, (5202, 5203)):
        x, xd = acts(oracle, m, k, seed, torch.bfloat16, device)
        got = noalloc(lin, xd, None, torch.bfloat16, bias)
        want = existing(lin, xd, None, torch.bfloat16, bias, workspace=SCRATCH)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"rows {m}: noalloc differs from linear_forward with a 16 MiB workspace"
        check(got, oracle.linear_ref_f64(x, wdeq, oracle.fill_normal(5201, 0.1, n)), x, wdeq, TOL_BF16,
              f"noalloc split-K rows {m}")


def test_noalloc_calls_on_two_streams_are_ordered(device, oracle):
    """Calls from two streams share the GPU's scratch; the entry point makes a
    call on another stream than the previous call's wait for it on the GPU,
    so six fused-prefill calls with an adapter (its x A operands live in the
    scratch), alternating between two streams with no host synchronisation,
    each give linear_forward's bits."""
    m, k, n, r = 300, 1024, 768, 16
    lin, _ = make_linear(oracle, k, n, 5300, device, dq=True, striped=True)
    _, _, ad = lora_parts(oracle, k, n, r, 5301, device)
    lora = ad.struct()
    xs = [acts(oracle, m, k, 5302 + i, torch.bfloat16, device)[1] for i in range(6)]
    want = [existing(lin, x, lora, torch.bfloat16) for x in xs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    got = []
    for i, x in enumerate(xs):
        with torch.cuda.stream(streams[i % 2]):
            got.append(noalloc(lin, x, lora, torch.bfloat16))
    torch.cuda.synchronize()
    for i, (g, w) in enumerate(zip(got, want)):
        assert torch.equal(g, w), f"call {i} (stream {i % 2}) differs from linear_forward"


def test_noalloc_refuses_what_does_not_fit(device, oracle):
    # f32 activations over 64 rows off the 16-byte alignment take the generic
    # path: the whole weight dequantized to f32 (4096 * 11008 * 4 bytes) does
    # not fit the scratch
    lin, _ = make_linear(oracle, 4096, 11008, 5100, device)
    _, x = acts(oracle, 101, 4096, 5101, torch.float32, device)
    xm = x.view(-1)[1:1 + 100 * 4096]  # 4 bytes past the allocation's alignment
    w = lin.weight_struct()
    y = torch.empty(100, 11008, device=device)
    lib = L.lib()
    stream = torch.cuda.current_stream().cuda_stream
    st = lib.unifur_nf4_linear_forward_noalloc(xm.data_ptr(), L.F32, 100, ctypes.byref(w), None, None, y.data_ptr(),
                                               L.F32, stream)
    assert st == L.ERR_WORKSPACE and b"16777216" in lib.unifur_nf4_last_error()
    # aligned, the same call runs on the f32 MFMA kernel without weight-sized
    # scratch, as the entry point with a workspace does
    L.check(lib.unifur_nf4_linear_forward_noalloc(x.data_ptr(), L.F32, 100, ctypes.byref(w), None, None,
                                                  y.data_ptr(), L.F32, stream))
    y2 = torch.empty_like(y)
    L.check(lib.unifur_nf4_linear_forward(x.data_ptr(), L.F32, 100, ctypes.byref(w), None, None, y2.data_ptr(),
                                          L.F32, None, 0, stream))
    assert torch.equal(y, y2)
    # 5..64 f32 rows run on MFMA over the striped weight and fit: the same
    # result as the entry point with a workspace
    y8 = torch.empty(8, 11008, device=device)
    L.check(lib.unifur_nf4_linear_forward_noalloc(x.data_ptr(), L.F32, 8, ctypes.byref(w), None, None, y8.data_ptr(),
                                                  L.F32, stream))
    ref8 = torch.empty_like(y8)
    L.check(lib.unifur_nf4_linear_forward(x.data_ptr(), L.F32, 8, ctypes.byref(w), None, None, ref8.data_ptr(), L.F32,
                                          None, 0, stream))
    assert torch.equal(y8, ref8)
    # and bad arguments are refused like the existing entry point's
    assert lib.unifur_nf4_linear_forward_noalloc(None, L.F32, 1, ctypes.byref(w), None, None, y.data_ptr(), L.F32,
                                                 None) == L.ERR_INVALID
    assert lib.unifur_nf4_linear_forward_noalloc(x.data_ptr(), 7, 1, ctypes.byref(w), None, None, y.data_ptr(),
                                                 L.F32, None) == L.ERR_INVALID
    # an empty batch does nothing
    assert lib.unifur_nf4_linear_forward_noalloc(None, L.F32, 0, ctypes.byref(w), None, None, None, L.F32,
                                                 None) == L.OK


@pytest.mark.parametrize("seed", range(12))
def test_noalloc_sweep(device, oracle, seed):
    """Drawn shapes, types, ranks and layouts, two calls in a row (the second
    smaller) on the shared scratch, each within its path's bar of the
    float64 product (1e-5 for f32 activations and output, 1e-2 otherwise)."""
    from test_gpu_linear import TOL_F32
    r = np.random.default_rng(0xA110 + seed)
    k = int(r.choice([64, 192, 512, 896, 1000, 2048]))
    n = int(r.choice([64, 128, 384, 896, 1024, 2048]))
    m1 = int(r.choice([1, 3, 4, 16, 33, 64, 65, 129, 300, 513]))
    m2 = max(1, int(m1 * r.uniform(0.2, 0.9)))
    xt = torch.bfloat16 if r.integers(2) else torch.float32
    yt = torch.bfloat16 if r.integers(2) else torch.float32
    rank = int(r.choice([0, 0, 1, 8, 16, 40]))
    striped = None if r.integers(2) else False
    print(f"noalloc sweep seed {seed}: rows {m1} then {m2}, {k} -> {n}, x {xt} y {yt} rank {rank} "
          f"striped {striped}", flush=True)
    lin, wdeq = make_linear(oracle, k, n, 0xA111 + seed, device, dq=bool(r.integers(2)), striped=striped)
    lora, a, b, s = None, None, None, 0.0
    if rank:
        s = 16.0 / rank
        a, b, ad = lora_parts(oracle, k, n, rank, 0xA112 + seed, device, scaling=s)
        lora = ad.struct()
    tol = TOL_F32 if (xt == torch.float32 and yt == torch.float32) else TOL_BF16
    for m, xs in ((m1, 0xA113 + seed), (m2, 0xA114 + seed)):
        x, xd = acts(oracle, m, k, xs, xt, device)
        got = noalloc(lin, xd, lora, yt).float().cpu().numpy().astype(np.float64)
        ref = oracle.linear_ref_f64(x, wdeq)
        bound = np.abs(x.astype(np.float64)) @ np.abs(wdeq.astype(np.float64))
        if rank:
            ref = ref + oracle.lora_ref_f64(x, a, b, s)
            bound = bound + (np.abs(x.astype(np.float64)) @ np.abs(a)) @ np.abs(b) * s
        nw = float(np.max(np.abs(got - ref) / np.maximum(bound, 1e-30)))
        lit = float(np.max(np.abs(got - ref)) / max(float(np.max(np.abs(ref))), 1e-30))
        print(f"  rows {m}: normwise {nw:.2e} literal {lit:.2e} (tol {tol})", flush=True)
        assert nw <= tol and lit <= tol
