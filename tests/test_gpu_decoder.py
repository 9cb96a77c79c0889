"""GPU parity of the decoder-layer decode stages (QwenDecoderLayer::step,
src/qwennet.rs:1112-1129) at the config-5 shapes (hidden 896, 14 heads / 2 KV
heads of dim 64, intermediate 4864): ``unifur_nf4_decoder_attn_in`` (input
norm + q/k/v) and ``unifur_nf4_decoder_attn_out_mlp`` (o + residual, post
norm + SwiGLU + residual), each against the float64 oracle on the same inputs,
then the composed chain over several decode positions and two layers with a
KV-cache attention written here in numpy (the attention is the caller's part,
not the NF4 path).  Tolerances: f32 1e-5, bf16 1e-2, normwise over the
accumulated terms and the literal max|y - r| / max|r|."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from unifur_amd import _lib as L
from unifur_amd import quantize as Q
from unifur_amd import qwennet as N

from test_gpu_linear import TOL_BF16, TOL_F32, acts, make_linear

pytestmark = pytest.mark.gpu

HIDDEN, HEADS, KV, DIM, INTER = 896, 14, 2, 64, 4864
EPS = 1e-6


def make_layer(oracle, device, seed, dq=True, striped=None):
    shapes = {"q": (HIDDEN, HEADS * DIM), "k": (HIDDEN, KV * DIM), "v": (HIDDEN, KV * DIM),
              "o": (HEADS * DIM, HIDDEN), "gate": (HIDDEN, INTER), "up": (HIDDEN, INTER), "down": (INTER, HIDDEN)}
    lins, w = {}, {}
    for i, (name, (d_in, d_out)) in enumerate(shapes.items()):
        lins[name], w[name] = make_linear(oracle, d_in, d_out, seed + i, device, dq=dq, striped=striped)
    g_in = oracle.fill_normal(seed + 20, 0.1, HIDDEN)
    g_post = oracle.fill_normal(seed + 21, 0.1, HIDDEN)
    layer = N.QwenDecoderLayer(lins["q"], lins["k"], lins["v"], lins["o"],
                               Q.QwenMlp(lins["gate"], lins["up"], lins["down"]),
                               torch.from_numpy(g_in).to(device), torch.from_numpy(g_post).to(device), EPS)
    return layer, w, g_in, g_post


def errors(y, ref, bound):
    from oracle import oracle as O
    y = np.asarray(y, np.float64).reshape(ref.shape)
    return O.normwise_error(y, ref, None, bound), O.max_rel_error(y, ref)


def assert_close(y, ref, bound, tol, tag):
    nw, lit = errors(y, ref, bound)
    print(f"{tag}: normwise {nw:.3e} literal {lit:.3e}", flush=True)
    assert nw <= tol and lit <= tol, f"{tag}: normwise {nw:.3e}, literal {lit:.3e} > {tol}"


def out_mlp_bound(oracle, x, ctx, w, g_post):
    """Scale of the terms summed into y: |x| + |ctx| |Wo| + |h| |Wd| with h
    the float64 silu(gate n) * up n of x1's norm n."""
    x1, _ = oracle.decoder_attn_out_mlp_ref_f64(x, ctx, g_post, EPS, w["o"], w["gate"], w["up"], w["down"])
    n = oracle.rms_norm_f64(x1, g_post, EPS)
    h = oracle.silu_f64(n @ w["gate"]) * (n @ w["up"])
    return np.abs(x) + np.abs(ctx) @ np.abs(w["o"]) + np.abs(h) @ np.abs(w["down"])


@pytest.fixture(scope="module")
def layer(oracle, device):
    return make_layer(oracle, device, 0x4E463457 + 5)


@pytest.mark.parametrize("rows,dt", [(1, torch.float32), (2, torch.float32), (3, torch.float32), (4, torch.float32),
                                     (1, torch.bfloat16), (32, torch.bfloat16), (9, torch.float32),
                                     (80, torch.bfloat16), (5, torch.bfloat16), (40, torch.float32)])
def test_attn_in(device, oracle, layer, rows, dt):
    lay, w, g_in, _ = layer
    x, xt = acts(oracle, rows, HIDDEN, 0x58 + 5 + rows, dt, device)
    q, k, v = lay.project(xt)
    refs = oracle.decoder_attn_in_ref_f64(x, g_in, EPS, w["q"], w["k"], w["v"])
    n = np.abs(oracle.rms_norm_f64(x, g_in, EPS))
    tol = TOL_F32 if dt == torch.float32 else TOL_BF16
    for name, got, ref in zip("qkv", (q, k, v), refs):
        assert got.dtype == dt and got.shape == (rows, w[name].shape[1])
        assert_close(got.float().cpu().numpy(), ref, n @ np.abs(w[name]), tol, f"attn_in {name} rows={rows} {dt}")


def test_attn_in_fused_paths_need_no_workspace(layer):
    lay, _, _, _ = layer
    s = lay.layer_struct()
    for rows in (1, 2, 4):
        assert L.lib().unifur_nf4_decoder_attn_in_workspace_size(rows, s, L.F32) == 0
    assert L.lib().unifur_nf4_decoder_attn_in_workspace_size(32, s, L.BF16) > 0


@pytest.mark.parametrize("rows,dt", [(1, torch.float32), (2, torch.float32), (3, torch.float32), (4, torch.float32),
                                     (2, torch.bfloat16), (32, torch.bfloat16), (64, torch.bfloat16),
                                     (7, torch.float32), (80, torch.bfloat16), (5, torch.bfloat16),
                                     (40, torch.float32)])
def test_attn_out_mlp(device, oracle, layer, rows, dt):
    lay, w, _, g_post = layer
    x, xt = acts(oracle, rows, HIDDEN, 0x5800 + rows, dt, device)
    ctx, ct = acts(oracle, rows, HEADS * DIM, 0x5900 + rows, dt, device)
    ctx = ctx * 0.5
    ct = ct * 0.5
    y = lay.attn_out_mlp(xt, ct)
    _, ref = oracle.decoder_attn_out_mlp_ref_f64(x, ctx, g_post, EPS, w["o"], w["gate"], w["up"], w["down"])
    tol = TOL_F32 if dt == torch.float32 else TOL_BF16
    assert y.dtype == dt and y.shape == xt.shape
    assert_close(y.float().cpu().numpy(), ref, out_mlp_bound(oracle, x, ctx, w, g_post), tol,
                 f"attn_out_mlp rows={rows} {dt}")


@pytest.mark.parametrize("rows,dt", [(32, torch.bfloat16), (16, torch.float32)])
def test_attn_out_mlp_misaligned_ctx_fits_the_queried_workspace(device, oracle, layer, rows, dt):
    """A ctx one element off the 16-byte alignment moves o off the skinny
    kernel: a workspace of exactly the queried size still serves the call."""
    import ctypes
    lay, w, _, g_post = layer
    x, xt = acts(oracle, rows, HIDDEN, 0x5A00 + rows, dt, device)
    ctx, ct = acts(oracle, rows, HEADS * DIM, 0x5B00 + rows, dt, device)
    buf = torch.empty(rows * HEADS * DIM + 1, dtype=dt, device=device)
    buf[1:].copy_(ct.reshape(-1))
    ct_off = buf[1:].view(rows, HEADS * DIM)
    s = lay.layer_struct()
    code = L.BF16 if dt == torch.bfloat16 else L.F32
    need = L.lib().unifur_nf4_decoder_attn_out_mlp_workspace_size(rows, s, code)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=device)
    y = torch.empty_like(xt)
    L.check(L.lib().unifur_nf4_decoder_attn_out_mlp(xt.data_ptr(), ct_off.data_ptr(), code, rows, ctypes.byref(s),
                                                     y.data_ptr(), ws.data_ptr(), need,
                                                     torch.cuda.current_stream().cuda_stream))
    _, ref = oracle.decoder_attn_out_mlp_ref_f64(x, ctx, g_post, EPS, w["o"], w["gate"], w["up"], w["down"])
    tol = TOL_F32 if dt == torch.float32 else TOL_BF16
    assert_close(y.float().cpu().numpy(), ref, out_mlp_bound(oracle, x, ctx, w, g_post), tol,
                 f"attn_out_mlp misaligned ctx rows={rows} {dt}")


def test_attn_out_mlp_in_place(device, oracle, layer):
    lay, w, _, g_post = layer
    x, xt = acts(oracle, 1, HIDDEN, 0x5A00, torch.float32, device)
    ctx, ct = acts(oracle, 1, HEADS * DIM, 0x5A01, torch.float32, device)
    y = lay.attn_out_mlp(xt, ct, out=xt)  # y may be x
    assert y.data_ptr() == xt.data_ptr()
    _, ref = oracle.decoder_attn_out_mlp_ref_f64(x, ctx, g_post, EPS, w["o"], w["gate"], w["up"], w["down"])
    assert_close(y.cpu().numpy(), ref, out_mlp_bound(oracle, x, ctx, w, g_post), TOL_F32, "in place")


def attend_np(q, k_cache, v_cache):
    """Single-query attention over the cached positions with adjacent-repeat
    GQA (head h reads KV head h // (HEADS / KV)), scaled dot products and a
    softmax, in float64: the caller's part of the step."""
    q = np.asarray(q, np.float64).reshape(HEADS, DIM)
    k = np.stack(k_cache).reshape(-1, KV, DIM)
    v = np.stack(v_cache).reshape(-1, KV, DIM)
    grp = HEADS // KV
    ctx = np.empty((HEADS, DIM))
    for h in range(HEADS):
        s = k[:, h // grp, :] @ q[h] / np.sqrt(DIM)
        p = np.exp(s - s.max())
        p /= p.sum()
        ctx[h] = p @ v[:, h // grp, :]
    return ctx.reshape(1, HEADS * DIM)


def test_composed_decode_chain(device, oracle):
    """Two layers, four decode positions: the GPU chain (its own q/k/v in its
    own caches) against the float64 oracle chain (its own caches), token by
    token, through the layer outputs."""
    layers = [make_layer(oracle, device, 0x6000 + 40 * i) for i in range(2)]
    caches_gpu = [([], []) for _ in layers]
    caches_ref = [([], []) for _ in layers]
    for pos in range(4):
        x = oracle.fill_normal(0x6100 + pos, 1.0, HIDDEN).reshape(1, HIDDEN)
        xg = torch.from_numpy(x.astype(np.float32)).to(device)
        xr = x.astype(np.float64)
        for li, (lay, w, g_in, g_post) in enumerate(layers):
            q, k, v = lay.project(xg)
            caches_gpu[li][0].append(k.cpu().numpy().astype(np.float64))
            caches_gpu[li][1].append(v.cpu().numpy().astype(np.float64))
            ctx = attend_np(q.cpu().numpy(), *caches_gpu[li])
            xg = lay.attn_out_mlp(xg, torch.from_numpy(ctx.astype(np.float32)).to(device))

            qr, kr, vr = oracle.decoder_attn_in_ref_f64(xr, g_in, EPS, w["q"], w["k"], w["v"])
            caches_ref[li][0].append(kr)
            caches_ref[li][1].append(vr)
            ctx_r = attend_np(qr, *caches_ref[li])
            bound = out_mlp_bound(oracle, xr, ctx_r, w, g_post)
            _, xr = oracle.decoder_attn_out_mlp_ref_f64(xr, ctx_r, g_post, EPS, w["o"], w["gate"], w["up"],
                                                        w["down"])
            assert_close(xg.cpu().numpy(), xr, bound, TOL_F32, f"chain pos={pos} layer={li}")


def test_row_major_and_f32_scales(device, oracle):
    """Row-major weights with f32 scales take the general path (norm kernel,
    linears, add kernels); same results."""
    lay, w, g_in, g_post = make_layer(oracle, device, 0x6500, dq=False, striped=False)
    x, xt = acts(oracle, 2, HIDDEN, 0x6501, torch.float32, device)
    q, k, v = lay.project(xt)
    n = np.abs(oracle.rms_norm_f64(x, g_in, EPS))
    for name, got, ref in zip("qkv", (q, k, v), oracle.decoder_attn_in_ref_f64(x, g_in, EPS, w["q"], w["k"], w["v"])):
        assert_close(got.cpu().numpy(), ref, n @ np.abs(w[name]), TOL_F32, f"row-major attn_in {name}")
    ctx, ct = acts(oracle, 2, HEADS * DIM, 0x6502, torch.float32, device)
    y = lay.attn_out_mlp(xt, ct)
    _, ref = oracle.decoder_attn_out_mlp_ref_f64(x, ctx, g_post, EPS, w["o"], w["gate"], w["up"], w["down"])
    assert_close(y.cpu().numpy(), ref, out_mlp_bound(oracle, x, ctx, w, g_post), TOL_F32, "row-major attn_out_mlp")


def test_bad_arguments(device, oracle, layer):
    lay, _, _, _ = layer
    x = torch.zeros(1, HIDDEN, device=device)
    with pytest.raises(ValueError):
        lay.attn_out_mlp(x, torch.zeros(1, 100, device=device))
    with pytest.raises(ValueError):
        lay.project(torch.zeros(1, 100, device=device))
    s = lay.layer_struct()
    s.post_norm = None
    st = torch.cuda.current_stream().cuda_stream
    r = L.lib().unifur_nf4_decoder_attn_out_mlp(x.data_ptr(), x.data_ptr(), L.F32, 1, s, x.data_ptr(), None, 0, st)
    assert r == L.ERR_INVALID and b"norm" in L.lib().unifur_nf4_last_error()
    s = lay.layer_struct()
    s.o = lay.layer_struct().k  # [896, 128]: o must map back to hidden
    r = L.lib().unifur_nf4_decoder_attn_in(x.data_ptr(), L.F32, 1, s, x.data_ptr(), x.data_ptr(), x.data_ptr(),
                                           None, 0, st)
    assert r == L.ERR_INVALID
