"""Seeded sweeps over shapes, types and options of every GPU entry point,
against the oracle: the fixed tests pin each path at its chosen shapes, these
draw the shapes (ragged rows, d_in off the 64-row chunk, d_out off the 64-column
block, every rank bucket, both scale kinds, both layouts, both workspace
sizes), so that a path's plan is exercised away from the shapes it was tuned
on.  Each case is drawn from its own seed, prints its parameters before it
runs, and is held to the bar of its path:

* codec (src/quantize.rs:259-366): codes, absmax, DQ codes, scale of scales
  and dequantized f32 bit-exact;
* grouped quantize pass (QwenTrunk::to_nf4, src/qwennet.rs:1185-1269): the
  bytes of the per-weight path, which the codec tests pin;
* linear / QLoRA forward (src/qwennet.rs:238-241, :325-345; LoraAdapter::
  forward, src/quantize.rs:619-624): the float64 product of the same inputs
  with the oracle's dequantized weight, per-element normwise error over
  |x||W| + |x||A||B|s (+|b|) and max|y - r| / max|r|, both <= 1e-5 for f32
  activations and f32 output, <= 1e-2 when activations or output are bf16;
* backward (the VJP of the above under src/qwentrain.rs:421-470): dx within
  1e-5 for f32 dy and 1e-2 for bf16 dy, the adapter gradients within 1e-5;
* SwiGLU (QwenMlp::forward, src/qwennet.rs:816-819): as the linear, with the
  bound |h||W_down|.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from unifur_amd import _lib as L
from unifur_amd import quantize as Q

from oracle.oracle import linear_backward_ref_f64 as backward_refs
from test_gpu_backward import normwise
from test_gpu_codec import assert_matches_oracle, gpu_roundtrip
from test_gpu_gemm import lora_parts
from test_gpu_linear import TOL_BF16, TOL_F32, acts, check, make_linear
from test_gpu_quantize_linears import per_weight, same_bytes

pytestmark = pytest.mark.gpu

ROWS = [1, 2, 3, 4, 5, 7, 16, 17, 31, 32, 33, 48, 63, 64, 65, 100, 127, 129, 256, 300, 513]
D_IN = [24, 64, 72, 128, 192, 320, 448, 512, 896, 1000, 1024, 1536, 2048]
D_OUT = [16, 48, 64, 100, 128, 136, 192, 384, 512, 640, 896, 1024, 2048]
RANKS = [1, 2, 4, 8, 16, 24, 40, 64]


def _stream():
    return torch.cuda.current_stream().cuda_stream


def linear_case(seed):
    r = np.random.default_rng(seed)
    rows, d_in, d_out = int(r.choice(ROWS)), int(r.choice(D_IN)), int(r.choice(D_OUT))
    return dict(rows=rows, d_in=d_in, d_out=d_out, x_bf16=bool(r.integers(2)), y_bf16=bool(r.integers(2)),
                dq=bool(r.integers(2)), striped=None if r.integers(2) else False,
                rank=int(r.choice(RANKS)) if r.integers(3) else 0, bias=bool(r.integers(2)),
                least=bool(r.integers(2)))


@pytest.mark.parametrize("seed", range(128))
def test_linear_forward_sweep(device, oracle, seed):
    c = linear_case(0x5EE0 + seed)
    print(f"sweep linear seed {seed}: {c}", flush=True)
    lin, wdeq = make_linear(oracle, c["d_in"], c["d_out"], 0x5EE1 + seed, device, dq=c["dq"], striped=c["striped"])
    x, xt = acts(oracle, c["rows"], c["d_in"], 0x5EE2 + seed, torch.bfloat16 if c["x_bf16"] else torch.float32,
                 device)
    bias = oracle.fill_normal(0x5EE3 + seed, 0.1, c["d_out"]) if c["bias"] else None
    ref = oracle.linear_ref_f64(x, wdeq, bias)
    bound = np.abs(x.astype(np.float64)) @ np.abs(wdeq.astype(np.float64))
    if bias is not None:
        bound = bound + np.abs(bias)
    lo = None
    if c["rank"]:
        s = 16.0 / c["rank"]
        a, b, ad = lora_parts(oracle, c["d_in"], c["d_out"], c["rank"], 0x5EE4 + seed, device, scaling=s)
        ref = ref + oracle.lora_ref_f64(x, a, b, s)
        bound = bound + (np.abs(x.astype(np.float64)) @ np.abs(a)) @ np.abs(b) * s
        lo = ad.struct()
    w = lin.weight_struct()
    bt = torch.from_numpy(bias).to(device) if bias is not None else None
    xd = L.BF16 if c["x_bf16"] else L.F32
    lib = L.lib()
    size = lib.unifur_nf4_linear_min_workspace_size if c["least"] else lib.unifur_nf4_linear_workspace_size
    need = size(c["rows"], c["d_in"], c["d_out"], xd, c["rank"])
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=device)
    y = torch.empty(c["rows"], c["d_out"], dtype=torch.bfloat16 if c["y_bf16"] else torch.float32, device=device)
    L.check(lib.unifur_nf4_linear_forward(xt.data_ptr(), xd, c["rows"], ctypes.byref(w),
                                          bt.data_ptr() if bt is not None else None,
                                          ctypes.byref(lo) if lo is not None else None, y.data_ptr(),
                                          L.BF16 if c["y_bf16"] else L.F32, ws.data_ptr(), need, _stream()))
    got = y.float().cpu().numpy().astype(np.float64)
    tol = TOL_BF16 if (c["x_bf16"] or c["y_bf16"]) else TOL_F32
    nw = float(np.max(np.abs(got - ref) / np.maximum(bound, 1e-30)))
    lit = float(np.max(np.abs(got - ref)) / max(float(np.max(np.abs(ref))), 1e-30))
    print(f"  normwise {nw:.2e} literal {lit:.2e} (tol {tol})", flush=True)
    assert nw <= tol and lit <= tol, c


def backward_case(seed):
    r = np.random.default_rng(seed)
    return dict(rows=int(r.choice(ROWS)), d_in=int(r.choice(D_IN[1:])), d_out=int(r.choice(D_OUT)),
                dy_bf16=bool(r.integers(2)), x_bf16=bool(r.integers(2)), dq=bool(r.integers(2)),
                striped=None if r.integers(2) else False, rank=int(r.choice(RANKS)), least=bool(r.integers(2)))


@pytest.mark.parametrize("seed", range(64))
def test_backward_sweep(device, oracle, seed):
    c = backward_case(0xBAC0 + seed)
    print(f"sweep backward seed {seed}: {c}", flush=True)
    M, K, N, r = c["rows"], c["d_in"], c["d_out"], c["rank"]
    lin, wdeq = make_linear(oracle, K, N, 0xBAC1 + seed, device, dq=c["dq"], striped=c["striped"])
    s = 16.0 / r
    a, b, ad = lora_parts(oracle, K, N, r, 0xBAC2 + seed, device, scaling=s)
    x, xt = acts(oracle, M, K, 0xBAC3 + seed, torch.bfloat16 if c["x_bf16"] else torch.float32, device)
    dy, dyt = acts(oracle, M, N, 0xBAC4 + seed, torch.bfloat16 if c["dy_bf16"] else torch.float32, device)
    ws = None
    if c["least"]:
        layout = L.LAYOUT_STRIPED if lin.is_striped() else L.LAYOUT_ROW_MAJOR
        need = L.lib().unifur_nf4_linear_backward_min_workspace_size(
            M, K, N, L.BF16 if c["dy_bf16"] else L.F32, r, layout)
        ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=device)[:need]
    dx, ga, gb = Q.QloraLinear(lin, ad).backward(xt, dyt, dx_dtype=torch.float32, workspace=ws)
    rdx, bdx, rga, bga, rgb, bgb = backward_refs(x, dy, wdeq, a, b, s)
    e = (normwise(dx.cpu(), rdx, bdx), normwise(ga.cpu(), rga, bga), normwise(gb.cpu(), rgb, bgb))
    tol_dx = TOL_BF16 if c["dy_bf16"] else TOL_F32
    print(f"  dx {e[0]:.2e} grad_a {e[1]:.2e} grad_b {e[2]:.2e}", flush=True)
    assert e[0] <= tol_dx and e[1] <= TOL_F32 and e[2] <= TOL_F32, c


@pytest.mark.parametrize("seed", range(40))
def test_swiglu_sweep(device, oracle, seed):
    r = np.random.default_rng(0x5A10 + seed)
    T = int(r.choice([1, 2, 3, 4, 5, 16, 31, 33, 64, 65, 200, 512, 600]))
    hidden = int(r.choice([64, 256, 512, 896, 1024]))
    inter = int(r.choice([128, 192, 512, 1024, 1408, 2816]))
    x_bf16, dq, striped, least = (bool(r.integers(2)) for _ in range(4))
    print(f"sweep swiglu seed {seed}: T {T} hidden {hidden} inter {inter} bf16 x {x_bf16} dq {dq} "
          f"striped {striped} least {least}", flush=True)
    g, wg = make_linear(oracle, hidden, inter, 0x5A11 + seed, device, dq=dq, striped=None if striped else False)
    u, wu = make_linear(oracle, hidden, inter, 0x5A12 + seed, device, dq=dq, striped=None if striped else False)
    d, wd = make_linear(oracle, inter, hidden, 0x5A13 + seed, device, dq=dq, striped=None if striped else False)
    x, xt = acts(oracle, T, hidden, 0x5A14 + seed, torch.bfloat16 if x_bf16 else torch.float32, device)
    ref = oracle.swiglu_ref_f64(x, wg, wu, wd)
    h = oracle.silu_f64(x.astype(np.float64) @ wg) * (x.astype(np.float64) @ wu)
    xd = L.BF16 if x_bf16 else L.F32
    lib = L.lib()
    size = lib.unifur_nf4_swiglu_min_workspace_size if least else lib.unifur_nf4_swiglu_workspace_size
    need = size(T, hidden, inter, xd)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=device)
    y = torch.empty(T, hidden, device=device)
    gs, us, ds = g.weight_struct(), u.weight_struct(), d.weight_struct()
    L.check(lib.unifur_nf4_swiglu_forward(xt.data_ptr(), xd, T, ctypes.byref(gs), ctypes.byref(us), ctypes.byref(ds),
                                          y.data_ptr(), L.F32, ws.data_ptr(), need, _stream()))
    check(y, ref, h, wd, TOL_BF16 if x_bf16 else TOL_F32, f"sweep swiglu seed {seed}")


@pytest.mark.parametrize("seed", range(16))
def test_codec_sweep(device, oracle, seed):
    r = np.random.default_rng(0xC0DE + seed)
    n = int(r.integers(1, 300_000))
    kind = int(r.integers(4))
    v = oracle.fill_normal(0xC0DF + seed, float(10.0 ** r.uniform(-6, 3)), n)
    if kind == 1:  # whole blocks of zeros
        for b in r.choice((n + 63) // 64, size=min(8, (n + 63) // 64), replace=False):
            v[64 * b:64 * b + 64] = 0.0
    elif kind == 2:  # specials in place
        idx = r.choice(n, size=min(16, n), replace=False)
        v[idx] = r.choice(np.array([np.nan, np.inf, -np.inf, -0.0, 1e-40, -1e-45], np.float32), size=idx.size)
    elif kind == 3:  # a wide dynamic range within blocks
        v = (v * np.float32(10.0) ** r.integers(-30, 30, size=n).astype(np.float32)).astype(np.float32)
    print(f"sweep codec seed {seed}: n {n} kind {kind}", flush=True)
    assert_matches_oracle(v, gpu_roundtrip(v, device), oracle, f"sweep codec seed {seed}")


@pytest.mark.parametrize("seed", range(6))
def test_grouped_quantize_sweep(device, oracle, seed):
    r = np.random.default_rng(0x6A0 + seed)
    count = int(r.integers(1, 60))
    shapes = [(int(r.choice([1, 2, 64, 100, 128, 896, 1000])), int(64 * r.integers(1, 20))) for _ in range(count)]
    print(f"sweep grouped quantize seed {seed}: {count} weights, {sum(a * b for a, b in shapes)} values",
          flush=True)
    ws = [(torch.from_numpy(oracle.fill_normal(0x6A1 + 97 * seed + i, 0.02, di * do)).to(device), di, do)
          for i, (di, do) in enumerate(shapes)]
    for (v, di, do), g in zip(ws, Q.quantize_linears(ws)):
        same_bytes(g, per_weight(v, di, do))


@pytest.mark.parametrize("seed", range(8))
def test_checkpoint_pass_sweep(device, oracle, seed):
    """The grouped checkpoint pass over drawn [out, in] shapes and element
    types: the oracle's transpose2d + quantize + double quantization in the
    striped permutation (qwen_linear, src/qwennet.rs:1687-1726)."""
    from test_gpu_layout import striped_codes_np, striped_scales_np
    from test_gpu_quantize_linears import checkpoint_tensors
    r = np.random.default_rng(0xC4E0 + seed)
    dtype = [torch.float32, torch.bfloat16, torch.float16][int(r.integers(3))]
    count = int(r.integers(1, 70))
    shapes = [(int(r.choice([1, 3, 8, 9, 64, 100, 130, 896])), int(64 * r.integers(1, 16))) for _ in range(count)]
    print(f"sweep checkpoint seed {seed}: {count} tensors of {dtype}", flush=True)
    host, dev = checkpoint_tensors(oracle, shapes, 0xC4E1 + 131 * seed, dtype, device)
    got = Q.quantize_checkpoint_linears(dev)
    for i, ((di, do), v, g) in enumerate(zip(shapes, host, got)):
        packed, absmax = oracle.quantize_packed(oracle.transpose(v.reshape(-1), do, di))
        q, sos = oracle.double_quantize(absmax)
        assert (g.d_input(), g.d_output()) == (di, do)
        assert np.array_equal(g._codes.cpu().numpy(), striped_codes_np(packed, di, do)), f"tensor {i} {(di, do)}"
        assert np.array_equal(g._scales.cpu().numpy(), striped_scales_np(q, di, do)), f"tensor {i} {(di, do)}"
        assert g._sos.cpu().numpy().view(np.uint32)[0] == np.float32(sos).view(np.uint32), f"tensor {i}"


@pytest.mark.parametrize("seed", range(32))
def test_decoder_stages_sweep(device, oracle, seed):
    """QwenDecoderLayer::step's NF4 stages (src/qwennet.rs:1112-1129) over
    drawn layer shapes, rows and types: input norm + q/k/v, then o +
    residual, post norm + SwiGLU + residual, against the float64 oracle."""
    from unifur_amd import qwennet as N
    from test_gpu_decoder import EPS, assert_close, out_mlp_bound
    r = np.random.default_rng(0xDEC0 + seed)
    hidden = int(r.choice([64, 128, 256, 448, 896]))
    q_out, kv_out = int(r.choice([64, 128, 256, 896])), int(r.choice([64, 128]))
    inter = int(r.choice([128, 256, 704, 1408]))
    rows = int(r.choice([1, 2, 3, 4, 5, 9, 16, 32, 40, 64, 80]))
    dt = torch.bfloat16 if r.integers(2) else torch.float32
    dq, striped = bool(r.integers(2)), None if r.integers(2) else False
    print(f"sweep decoder seed {seed}: hidden {hidden} q {q_out} kv {kv_out} inter {inter} rows {rows} {dt} "
          f"dq {dq} striped {striped}", flush=True)
    shapes = {"q": (hidden, q_out), "k": (hidden, kv_out), "v": (hidden, kv_out), "o": (q_out, hidden),
              "gate": (hidden, inter), "up": (hidden, inter), "down": (inter, hidden)}
    lins, w = {}, {}
    for i, (name, (d_in, d_out)) in enumerate(shapes.items()):
        lins[name], w[name] = make_linear(oracle, d_in, d_out, 0xDEC1 + 16 * seed + i, device, dq=dq, striped=striped)
    g_in = oracle.fill_normal(0xDEC2 + seed, 0.1, hidden)
    g_post = oracle.fill_normal(0xDEC3 + seed, 0.1, hidden)
    lay = N.QwenDecoderLayer(lins["q"], lins["k"], lins["v"], lins["o"],
                             Q.QwenMlp(lins["gate"], lins["up"], lins["down"]),
                             torch.from_numpy(g_in).to(device), torch.from_numpy(g_post).to(device), EPS)
    tol = TOL_F32 if dt == torch.float32 else TOL_BF16
    x, xt = acts(oracle, rows, hidden, 0xDEC4 + seed, dt, device)
    refs = oracle.decoder_attn_in_ref_f64(x, g_in, EPS, w["q"], w["k"], w["v"])
    n = np.abs(oracle.rms_norm_f64(x, g_in, EPS))
    for name, got, ref in zip("qkv", lay.project(xt), refs):
        assert_close(got.float().cpu().numpy(), ref, n @ np.abs(w[name]), tol, f"sweep attn_in {name}")
    ctx, ct = acts(oracle, rows, q_out, 0xDEC5 + seed, dt, device)
    y = lay.attn_out_mlp(xt, ct)
    _, ref = oracle.decoder_attn_out_mlp_ref_f64(x, ctx, g_post, EPS, w["o"], w["gate"], w["up"], w["down"])
    assert_close(y.float().cpu().numpy(), ref, out_mlp_bound(oracle, x, ctx, w, g_post), tol, "sweep attn_out_mlp")


@pytest.mark.parametrize("seed", range(10))
def test_embedding_sweep(device, oracle, seed):
    """Nf4Embedding::forward (src/qwennet.rs:244-291) over drawn table shapes,
    scale kinds, id types and counts: every gathered row bit for bit the
    oracle's dequantized row (f32), and its RNE rounding (bf16)."""
    from unifur_amd import qwennet as QN
    from test_gpu_embedding import bf16_rne, table
    r = np.random.default_rng(0xE3B0 + seed)
    n_emb, d = int(r.integers(1, 5000)), int(r.choice([1, 3, 8, 64, 100, 257, 896, 1000]))
    dq, ids_dtype = bool(r.integers(2)), [torch.int32, torch.int64][int(r.integers(2))]
    count = int(r.integers(1, 3000))
    print(f"sweep embedding seed {seed}: table {n_emb} x {d} dq {dq} ids {count} {ids_dtype}", flush=True)
    v, deq = table(oracle, n_emb, d, 0xE3B1 + seed, dq=dq)
    p = Q.PackedNf4Tensor.quantize(torch.from_numpy(v).to(device))
    if dq:
        p = p.with_double_quantization()
    emb = QN.Nf4Embedding(p, n_emb, d)
    ids = r.integers(0, n_emb, size=count)
    got = emb.forward(torch.from_numpy(ids).to(ids_dtype).to(device))
    assert np.array_equal(got.cpu().numpy().view(np.uint32), deq[ids].view(np.uint32))
    gb = emb.forward(torch.from_numpy(ids).to(ids_dtype).to(device), dtype=torch.bfloat16)
    assert np.array_equal(gb.cpu().view(torch.int16).numpy().view(np.uint16), bf16_rne(deq[ids]))
