"""GPU parity of the grouped quantize pass (unifur_nf4_quantize_linears):
QwenTrunk::to_nf4 (src/qwennet.rs:1185-1269) runs Nf4Linear::from_values
(src/qwennet.rs:196-205) on every projection in turn; the grouped pass must
write, for each weight, exactly the bytes of the per-weight path -- quantize
(src/quantize.rs:259-279), double quantization (:281-309), then the striped
layout -- whose codec is pinned bit-exact against the oracle by the codec
tests.  Shapes cover the config-5 projections, spans that cross rows or end
inside a 1024-value span, one-row weights, groups of more than 48 weights,
and blocks of zeros, NaN, infinities and subnormals.  The checkpoint form
(unifur_nf4_quantize_checkpoint_linears) takes the PyTorch-order [out, in]
tensors (f32 or bf16) that qwen_linear receives (src/qwennet.rs:1687-1726)
and must write the bytes of the transposed copies, tested the same ways.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from unifur_amd import _lib as L
from unifur_amd import quantize as Q

pytestmark = pytest.mark.gpu


def per_weight(values, d_in, d_out):
    return Q.Nf4Linear.from_values(values, d_in, d_out)


def same_bytes(a: Q.Nf4Linear, b: Q.Nf4Linear):
    assert a.is_striped() and b.is_striped()
    assert torch.equal(a._codes, b._codes), "striped codes differ"
    assert torch.equal(a._scales, b._scales), "u8 scales differ"
    assert torch.equal(a._sos.view(torch.int32), b._sos.view(torch.int32)), "scale of scales differs"


def weights(oracle, shapes, seed):
    out = []
    for i, (di, do) in enumerate(shapes):
        v = torch.from_numpy(oracle.fill_normal(seed + i, 0.02, di * do)).cuda()
        out.append((v, di, do))
    return out


def test_config5_projection_shapes(device, oracle):
    shapes = [(896, 896), (896, 128), (896, 128), (896, 896), (896, 4864), (896, 4864), (4864, 896)]
    ws = weights(oracle, shapes, 3000)
    got = Q.quantize_linears(ws)
    for (v, di, do), g in zip(ws, got):
        same_bytes(g, per_weight(v, di, do))


def test_config5_all_weights_against_the_oracle(device, oracle):
    # QwenTrunk::to_nf4 over the config-5 projection set (src/qwennet.rs:1196-1269):
    # 24 layers x {q, k, v, o, gate, up, down}, 168 weights ~ N(0, 0.02^2), in
    # ONE grouped call; every weight's striped codes, u8 scales and scale of
    # scales equal the oracle's PackedNf4Tensor::quantize +
    # with_double_quantization (src/quantize.rs:259-309) in the documented
    # striped permutation, byte for byte.
    from test_gpu_layout import striped_codes_np, striped_scales_np
    per_layer = [(896, 896), (896, 128), (896, 128), (896, 896), (896, 4864), (896, 4864), (4864, 896)]
    shapes = per_layer * 24
    host, dev = [], []
    for i, (di, do) in enumerate(shapes):
        v = oracle.fill_normal(0x4E463457 + 5 + 0x10000 * i, 0.02, di * do)
        host.append(v)
        dev.append((torch.from_numpy(v).to(device), di, do))
    got = Q.quantize_linears(dev)
    torch.cuda.synchronize()
    assert len(got) == 168
    for i, ((di, do), v, g) in enumerate(zip(shapes, host, got)):
        packed, absmax = oracle.quantize_packed(v)
        q, sos = oracle.double_quantize(absmax)
        assert g.is_striped()
        assert np.array_equal(g._codes.cpu().numpy(), striped_codes_np(packed, di, do)), f"weight {i}: codes"
        assert np.array_equal(g._scales.cpu().numpy(), striped_scales_np(q, di, do)), f"weight {i}: u8 scales"
        assert g._sos.cpu().numpy().view(np.uint32)[0] == np.float32(sos).view(np.uint32), f"weight {i}: sos"
    print(f"config 5: {sum(a * b for a, b in shapes)} values in 168 weights byte-exact", flush=True)


def test_partial_spans_tiny_and_many(device, oracle):
    # 50 weights (two groups), spans crossing rows and ending mid-span
    shapes = [(1, 64), (3, 128), (17, 192), (5, 64), (33, 320), (2, 1024), (7, 960)] * 7 + [(1, 64)]
    ws = weights(oracle, shapes, 3100)
    got = Q.quantize_linears(ws)
    assert len(got) == len(shapes)
    for (v, di, do), g in zip(ws, got):
        same_bytes(g, per_weight(v, di, do))


def test_special_values(device, oracle):
    di, do = 9, 256
    v = oracle.fill_normal(3200, 0.02, di * do).copy()
    v[0:64] = 0.0                                     # zero block: codes 7, scale 0
    v[64:128] = np.float32(1e-40)                     # subnormal block: exact division path
    v[128] = np.nan                                   # NaN -> code 0, ignored by absmax
    v[200] = np.inf                                   # Inf block
    v[300:364] = np.nan                               # all-NaN block: absmax 0
    v[400] = -0.0
    v[500] = np.float32(3.0e38)                       # large absmax: exact path
    t = torch.from_numpy(v).cuda()
    got = Q.quantize_linears([(t, di, do)])[0]
    same_bytes(got, per_weight(t, di, do))
    # all-zero weight: max 0, every u8 scale 0, scale of scales 0
    z = torch.zeros(4 * 128, device="cuda")
    gz = Q.quantize_linears([(z, 4, 128)])[0]
    same_bytes(gz, per_weight(z, 4, 128))
    assert float(gz._sos) == 0.0 and not gz._scales.any()


def test_forward_matches_and_argument_errors(device, oracle):
    ws = weights(oracle, [(256, 384)], 3300)
    got = Q.quantize_linears(ws)[0]
    ref = per_weight(*ws[0])
    x = torch.from_numpy(oracle.fill_normal(3301, 1.0, 3 * 256)).cuda().view(3, 256)
    assert torch.equal(got.forward(x), ref.forward(x))
    assert torch.equal(got.dequantized_weight(), ref.dequantized_weight())
    with pytest.raises(ValueError):
        Q.quantize_linears([(torch.zeros(8 * 100, device="cuda"), 8, 100)])  # d_out % 64 != 0
    lib = L.lib()
    P = ctypes.c_void_p * 1
    U = ctypes.c_uint64 * 1
    buf = torch.zeros(1024, dtype=torch.uint8, device="cuda")
    vals = torch.zeros(64, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    # misaligned values
    assert lib.unifur_nf4_quantize_linears(P(vals.data_ptr() + 4), U(1), U(64), 1, P(buf.data_ptr()),
                                           P(buf.data_ptr() + 256), P(buf.data_ptr() + 512), None, 0,
                                           st) == L.ERR_INVALID
    # a NULL array
    assert lib.unifur_nf4_quantize_linears(None, U(1), U(64), 1, P(buf.data_ptr()), P(buf.data_ptr() + 256),
                                           P(buf.data_ptr() + 512), None, 0, st) == L.ERR_INVALID
    assert lib.unifur_nf4_quantize_linears(None, None, None, 0, None, None, None, None, 0, st) == 0


# ------------------------------------------------- checkpoint [out, in] form --

def checkpoint_tensors(oracle, shapes, seed, dtype, device):
    """[out = d_out, in = d_in] tensors; bf16 ones hold exactly the oracle's
    RNE rounding of the f32 draw, f16 ones numpy's (host: the f32 values the
    reference decodes from them)."""
    host, dev = [], []
    for i, (di, do) in enumerate(shapes):
        v = oracle.fill_normal(seed + 0x10000 * i, 0.02, di * do)
        if dtype == torch.float16:
            h = v.astype(np.float16)  # binary16 draws; f32 as f16_to_f32 decodes them
            host.append(oracle.decode_checkpoint(h.view(np.uint16), "f16").reshape(do, di))
            dev.append(torch.from_numpy(h.reshape(do, di)).to(device))
            continue
        if dtype == torch.bfloat16:
            v = oracle.round_bf16(v)
        v = v.reshape(do, di)
        host.append(v)
        dev.append(torch.from_numpy(v).to(device).to(dtype))
    return host, dev


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_checkpoint_config5_all_weights_against_the_oracle(device, oracle, dtype):
    """All 168 config-5 projections from checkpoint tensors as they lie, in
    one call: each weight's striped codes, u8 scales and scale of scales equal
    the oracle's transpose2d + PackedNf4Tensor::quantize +
    with_double_quantization in the striped permutation."""
    from test_gpu_layout import striped_codes_np, striped_scales_np
    per_layer = [(896, 896), (896, 128), (896, 128), (896, 896), (896, 4864), (896, 4864), (4864, 896)]
    shapes = per_layer * 24
    host, dev = checkpoint_tensors(oracle, shapes, 0x4E463457 + 5, dtype, device)
    got = Q.quantize_checkpoint_linears(dev)
    torch.cuda.synchronize()
    assert len(got) == 168
    for i, ((di, do), v, g) in enumerate(zip(shapes, host, got)):
        tv = oracle.transpose(v.reshape(-1), do, di)  # [in, out]
        packed, absmax = oracle.quantize_packed(tv)
        q, sos = oracle.double_quantize(absmax)
        assert g.is_striped() and (g.d_input(), g.d_output()) == (di, do)
        assert np.array_equal(g._codes.cpu().numpy(), striped_codes_np(packed, di, do)), f"weight {i}: codes"
        assert np.array_equal(g._scales.cpu().numpy(), striped_scales_np(q, di, do)), f"weight {i}: u8 scales"
        assert g._sos.cpu().numpy().view(np.uint32)[0] == np.float32(sos).view(np.uint32), f"weight {i}: sos"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_checkpoint_ragged_shapes_match_the_transposed_pass(device, oracle, dtype):
    """d_in not a multiple of 64 (a partial source tile), of 8 or 4 (the
    element-load path), one-row and one-column weights, two groups: the same
    bytes as the f32 pass over the transposed copies."""
    shapes = [(1, 64), (7, 128), (100, 192), (130, 64), (64, 64), (3, 960), (65, 320)] * 7 + [(896, 128)]
    host, dev = checkpoint_tensors(oracle, shapes, 3400, dtype, device)
    got = Q.quantize_checkpoint_linears(dev)
    ref = Q.quantize_linears([(t.float().t().contiguous().view(-1), di, do) for t, (di, do) in zip(dev, shapes)])
    for g, r in zip(got, ref):
        same_bytes(g, r)


def test_checkpoint_special_values(device, oracle):
    do, di = 256, 9  # [out, in]
    v = oracle.fill_normal(3500, 0.02, di * do).reshape(do, di).copy()
    v[0:64, 0] = 0.0        # a zero block (column 0 of the transposed weight, rows 0-63)
    v[64:128, 1] = 1e-40    # a subnormal block
    v[3, 2] = np.nan
    v[130, 3] = np.inf
    v[192:256, 4] = np.nan  # an all-NaN block
    v[5, 5] = -0.0
    v[70, 6] = 3.0e38       # large absmax: the exact path
    t = torch.from_numpy(v).cuda()
    got = Q.quantize_checkpoint_linears([t])[0]
    same_bytes(got, Q.quantize_linears([(t.t().contiguous().view(-1), di, do)])[0])


def test_checkpoint_f16_special_values(device, oracle):
    """binary16 sources with infinities, NaNs (quiet and signalling), signed
    zeros and subnormals, in a zero, a subnormal-only and an all-NaN block:
    the same bytes as the f32 pass over the oracle's decode, transposed."""
    do, di = 192, 16  # [out, in]
    h = oracle.fill_normal(3600, 0.05, di * do).astype(np.float16).reshape(do, di).copy()
    hb = h.view(np.uint16)
    hb[0:64, 0] = 0x0000                                   # a zero block
    hb[64:128, 1] = np.arange(64, dtype=np.uint16) + 1     # subnormals only
    hb[128:192, 2] = 0x7D01                                # signalling NaNs: an all-NaN block
    hb[3, 3], hb[4, 3], hb[5, 3] = 0x7C00, 0xFC00, 0x7E55  # +inf, -inf, a quiet NaN with a payload
    hb[6, 4], hb[7, 4] = 0x8000, 0x8001                    # -0, the smallest negative subnormal
    hb[8, 5] = 0x7BFF                                      # the largest finite half
    t = torch.from_numpy(h).to(device)
    f = oracle.decode_checkpoint(hb.reshape(-1), "f16").reshape(do, di)
    ref_t = torch.from_numpy(np.ascontiguousarray(f.T)).to(device).view(-1)
    got = Q.quantize_checkpoint_linears([t])[0]
    same_bytes(got, Q.quantize_linears([(ref_t, di, do)])[0])
    # the single-tensor entry point, before double quantization, is the oracle's
    packed_ref, absmax_ref = oracle.quantize_packed(np.ascontiguousarray(f.T).reshape(-1))
    codes = torch.empty(do * di // 2, dtype=torch.uint8, device=device)
    absmax = torch.empty(do * di // 64, dtype=torch.float32, device=device)
    L.check(L.lib().unifur_nf4_quantize_transposed(t.data_ptr(), L.F16, do, di, codes.data_ptr(),
                                                   absmax.data_ptr(), Q._stream()))
    assert np.array_equal(codes.cpu().numpy(), packed_ref)
    assert np.array_equal(absmax.cpu().numpy().view(np.uint32), absmax_ref.view(np.uint32))


def test_checkpoint_argument_errors(device):
    a = torch.zeros(64, 8, device="cuda")
    b = torch.zeros(64, 8, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        Q.quantize_checkpoint_linears([a, b])  # mixed dtypes in one call
    with pytest.raises(ValueError):
        Q.quantize_checkpoint_linears([torch.zeros(100, 8, device="cuda")])  # out % 64 != 0
    lib = L.lib()
    P = ctypes.c_void_p * 1
    U = ctypes.c_uint64 * 1
    buf = torch.zeros(1024, dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    # bf16 values off their 2-byte alignment, and a bad dtype
    assert lib.unifur_nf4_quantize_checkpoint_linears(P(b.data_ptr() + 1), L.BF16, U(8), U(64), 1, P(buf.data_ptr()),
                                                      P(buf.data_ptr() + 256), P(buf.data_ptr() + 512), None, 0,
                                                      st) == L.ERR_INVALID
    assert lib.unifur_nf4_quantize_checkpoint_linears(P(a.data_ptr()), 5, U(8), U(64), 1, P(buf.data_ptr()),
                                                      P(buf.data_ptr() + 256), P(buf.data_ptr() + 512), None, 0,
                                                      st) == L.ERR_INVALID
