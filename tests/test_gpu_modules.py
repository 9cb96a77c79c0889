"""GPU parity of the module-level NF4 entry points: the fused transpose +
quantize of checkpoint linears (src/qwennet.rs:1687-1726), the simulated
QLoRA layer and its merge (src/quantize.rs:637-727), module quantization
(src/quantize.rs:418-511), the dense f32 linear, and the QwenLinear
residency switch (src/qwennet.rs:293-435).

Codes, scales and dequantized values are compared bit for bit with the
oracle; products against float64 at the north star's tolerances (f32 1e-5,
bf16 1e-2; normwise and literal, as in the linear-path tests).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from unifur_amd import quantize as Q
from unifur_amd import qwennet as QN

from test_gpu_linear import TOL_BF16, TOL_F32, acts, check

pytestmark = pytest.mark.gpu


def checkpoint_linear(oracle, out_f, in_f, seed, dtype):
    """A decoded checkpoint tensor [out, in] (numpy f32 values, device tensor)."""
    v = oracle.fill_normal(seed, 0.05, out_f * in_f).reshape(out_f, in_f)
    if dtype == torch.float16:
        # binary16 draws (numpy's RNE narrowing), and the f32 values the
        # reference decodes from them (f16_to_f32, src/import.rs:283-317)
        h = v.astype(np.float16)
        return oracle.decode_checkpoint(h.view(np.uint16), "f16").reshape(out_f, in_f), torch.from_numpy(h).to("cuda:0")
    if dtype == torch.bfloat16:
        v = oracle.round_bf16(v).reshape(out_f, in_f)
    return v, torch.from_numpy(v).to("cuda:0").to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(64, 1), (64, 7), (128, 64), (192, 100), (896, 896), (4864, 130)])
def test_quantize_transposed_is_transpose_then_quantize(device, oracle, dtype, shape):
    out_f, in_f = shape
    v, t = checkpoint_linear(oracle, out_f, in_f, 0x7A + out_f + in_f, dtype)
    packed_ref, absmax_ref = oracle.quantize_packed(oracle.transpose(v.reshape(-1), out_f, in_f))
    lin, nbytes = QN.qwen_linear(t, QN.WeightStore.NF4)
    assert lin.kind == QN.QwenLinear.NF4
    assert (lin.d_input(), lin.d_output()) == (in_f, out_f)
    p = lin.inner.packed()
    assert np.array_equal(p.codes.cpu().numpy(), packed_ref)
    q_ref, sos_ref = oracle.double_quantize(absmax_ref)
    assert np.array_equal(p.dq_codes.cpu().numpy(), q_ref)
    assert p.scale_of_scales.cpu().numpy()[0].view(np.uint32) == np.float32(sos_ref).view(np.uint32)
    assert nbytes == oracle.estimated_resident_bytes(out_f * in_f, True)
    # the raw entry point, before double quantization: absmax bit-exact
    codes = torch.empty((out_f * in_f + 1) // 2, dtype=torch.uint8, device=device)
    absmax = torch.empty((out_f * in_f + 63) // 64, dtype=torch.float32, device=device)
    from unifur_amd import _lib as L
    L.check(L.lib().unifur_nf4_quantize_transposed(t.data_ptr(), Q._src_dtype_code(dtype), out_f, in_f,
                                                   codes.data_ptr(), absmax.data_ptr(), Q._stream()))
    assert np.array_equal(codes.cpu().numpy(), packed_ref)
    assert np.array_equal(absmax.cpu().numpy().view(np.uint32), absmax_ref.view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(100, 96), (70, 129), (1, 64), (130, 1)])
def test_qwen_linear_with_ragged_out_features_falls_back_to_separate_transpose(device, oracle, dtype, shape):
    """out % 64 != 0: the library transposes (unifur_nf4_transpose_checkpoint,
    bf16 decoded exactly) and the flat buffer is quantized; codes, DQ codes and
    scale of scales equal the oracle's transpose + quantize + double quantize."""
    out_f, in_f = shape
    v, t = checkpoint_linear(oracle, out_f, in_f, 0x7B + out_f, dtype)
    tv = oracle.transpose(v.reshape(-1), out_f, in_f)
    packed_ref, absmax_ref = oracle.quantize_packed(tv)
    q_ref, sos_ref = oracle.double_quantize(absmax_ref)
    lin, nbytes = QN.qwen_linear(t, QN.WeightStore.NF4)
    p = lin.inner.packed()
    assert np.array_equal(p.codes.cpu().numpy(), packed_ref)
    assert np.array_equal(p.dq_codes.cpu().numpy(), q_ref)
    assert p.scale_of_scales.cpu().numpy()[0].view(np.uint32) == np.float32(sos_ref).view(np.uint32)
    assert not lin.inner.is_striped()
    assert nbytes == oracle.estimated_resident_bytes(out_f * in_f, True)
    # the transpose entry point itself: bit for bit the oracle's transpose2d
    from unifur_amd import _lib as L
    dst = torch.empty(out_f * in_f, dtype=torch.float32, device=device)
    L.check(L.lib().unifur_nf4_transpose_checkpoint(t.data_ptr(), Q._src_dtype_code(dtype), out_f, in_f, dst.data_ptr(),
                                                    Q._stream()))
    assert np.array_equal(dst.cpu().numpy().view(np.uint32), tv.view(np.uint32))


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_transpose_checkpoint_decodes_every_half_bit_pattern(device, oracle, dtype):
    """All 65536 binary16 (or bfloat16) patterns, NaN payloads, infinities
    and subnormals included, as a [256, 256] checkpoint tensor: the f32
    transpose is bit for bit the oracle's decode (read_tensor_f32,
    src/import.rs:255-317) then transpose2d."""
    from unifur_amd import _lib as L
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    t = torch.from_numpy(bits.view(np.int16)).to(device).view(torch.float16 if dtype == "f16" else torch.bfloat16)
    ref = oracle.transpose(oracle.decode_checkpoint(bits, dtype), 256, 256)
    dst = torch.empty(1 << 16, dtype=torch.float32, device=device)
    L.check(L.lib().unifur_nf4_transpose_checkpoint(t.data_ptr(), Q._src_dtype_code(t.dtype), 256, 256,
                                                    dst.data_ptr(), Q._stream()))
    assert np.array_equal(dst.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_qwen_linear_f32_store_and_forward(device, oracle):
    out_f, in_f = 256, 192
    v, t = checkpoint_linear(oracle, out_f, in_f, 0x7C, torch.float32)
    lin, nbytes = QN.qwen_linear(t, QN.WeightStore.F32)
    assert lin.kind == QN.QwenLinear.F32 and nbytes == 4 * out_f * in_f
    assert lin.resident_bytes() == nbytes
    x, xt = acts(oracle, 9, in_f, 0x7D, torch.float32, device)
    w = v.T.astype(np.float64)
    check(lin.forward(xt), x.astype(np.float64) @ w, x, v.T, TOL_F32, "qwen f32 linear")
    # to_nf4 of the in-memory [in, out] weight equals quantizing it directly
    nf4 = lin.to_nf4()
    assert nf4.kind == QN.QwenLinear.NF4
    packed_ref, _ = oracle.quantize_packed(np.ascontiguousarray(v.T).reshape(-1))
    assert np.array_equal(nf4.inner.packed().codes.cpu().numpy(), packed_ref)
    assert nf4.resident_bytes() == oracle.estimated_resident_bytes(out_f * in_f, True)
    assert nf4.to_nf4() is nf4


def test_qwen_linear_lora_attachment_rules(device):
    t = torch.randn(128, 64, device=device)
    f32, _ = QN.qwen_linear(t, QN.WeightStore.F32)
    with pytest.raises(ValueError, match="NF4-resident"):
        f32.with_lora(QN.QwenLoraConfig())
    nf4 = f32.to_nf4()
    with pytest.raises(ValueError, match="positive"):
        nf4.with_lora(QN.QwenLoraConfig(rank=0))
    with pytest.raises(ValueError, match="finite"):
        nf4.with_lora(QN.QwenLoraConfig(alpha=float("nan")))
    q = nf4.with_lora(QN.QwenLoraConfig(rank=8, alpha=16.0))
    assert q.kind == QN.QwenLinear.QLORA
    assert q.inner.adapter.scaling() == 2.0
    assert q.resident_bytes() == nf4.resident_bytes() + 4 * (64 + 128) * 8
    with pytest.raises(ValueError, match="already"):
        q.with_lora(QN.QwenLoraConfig())
    with pytest.raises(ValueError, match="de-adapted"):
        q.to_nf4()
    # a fresh adapter is an exact no-op
    x = torch.randn(3, 64, device=device)
    assert torch.equal(q.forward(x), nf4.forward(x))


def test_projections_to_nf4_records_classes(device):
    projs = {f"layers.{i}.{c}": QN.qwen_linear(torch.randn(128, 64, device=device), QN.WeightStore.F32)[0]
             for i in range(2) for c in ("q_proj", "o_proj")}
    report = QN.Nf4ResidencyReport()
    out = QN.projections_to_nf4(projs, report)
    assert all(v.kind == QN.QwenLinear.NF4 for v in out.values())
    per = Q.PackedNf4Tensor.estimated_resident_bytes(128 * 64, True)
    assert report.packed_bytes == 4 * per and report.f32_kept_bytes == 0
    assert [(r.cls, r.tensors, r.packed_bytes) for r in report.by_class] == [("q_proj", 2, 2 * per),
                                                                               ("o_proj", 2, 2 * per)]


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows", [1, 5, 64, 300])
def test_dense_linear_bias_and_lora(device, oracle, x_dtype, rows):
    d_in, d_out, r = 320, 192, 8
    w = oracle.fill_normal(0x90 + rows, 0.05, d_in * d_out).reshape(d_in, d_out)
    bias = oracle.fill_normal(0x91, 0.1, d_out)
    a = oracle.fill_normal(0x92, 0.05, d_in * r).reshape(d_in, r)
    b = oracle.fill_normal(0x93, 0.05, r * d_out).reshape(r, d_out)
    dense = Q.DenseLinear(torch.from_numpy(w).to(device), torch.from_numpy(bias).to(device))
    ad = Q.LoraAdapter.from_parts(torch.from_numpy(a).to(device), torch.from_numpy(b).to(device), 1.5)
    x, xt = acts(oracle, rows, d_in, 0x94 + rows, x_dtype, device)
    tol = TOL_F32 if x_dtype == torch.float32 else TOL_BF16
    check(dense.forward(xt, out_dtype=torch.float32), oracle.linear_ref_f64(x, w, bias), x, w, tol, "dense")
    ref = oracle.linear_ref_f64(x, w, bias) + oracle.lora_ref_f64(x, a, b, 1.5)
    check(dense._forward(xt, ad, torch.float32), ref, x, w, tol, "dense+lora")


def test_qlora_simulated_is_the_base_layer_at_init(device, oracle):
    # src/quantize.rs:1059-1081: with B = 0 the layer is exactly its quantized base
    g = torch.Generator().manual_seed(3)
    cfg = Q.LoraConfig.new(Q.BLOCK_SIZE, 8, 2)
    base = Q.DenseLinear(*Q._linear_init(Q.BLOCK_SIZE, 8, g, device))
    w_np = base.weight.cpu().numpy().reshape(-1)
    q = Q.QLoRALinear.from_linear(base, cfg, True, device, g)
    packed, absmax = oracle.quantize_packed(w_np)
    dqc, sos = oracle.double_quantize(absmax)
    want = oracle.dequantize_packed(packed, w_np.size, None, dqc, sos)
    assert np.array_equal(q.base.weight.cpu().numpy().reshape(-1).view(np.uint32), want.view(np.uint32))
    assert torch.equal(q.base.bias, base.bias)
    x = torch.rand(2, Q.BLOCK_SIZE, generator=g).to(device) * 2 - 1
    assert torch.equal(q.forward(x), q.base.forward(x))
    nf4_bits, f32_bits = q.resident_bits()
    assert nf4_bits * 7.0 < f32_bits
    assert nf4_bits == 4.0 * 512 + 8.0 * 8 + 32.0 and f32_bits == 32.0 * 512


@pytest.mark.parametrize("shape", [(Q.BLOCK_SIZE, 8), (896, 4864)])
def test_qlora_merge_preserves_outputs(device, oracle, shape):
    # src/quantize.rs:1084-1099 at its own shape and at a Qwen projection
    d_in, d_out = shape
    g = torch.Generator().manual_seed(5)
    q = Q.QLoRALinear.new(d_in, d_out, Q.LoraConfig.new(d_in, d_out, 2), False, device, g)
    q.adapter().b.copy_((torch.rand(2, d_out, generator=g) * 0.6 - 0.3).to(device))
    x = (torch.rand(5, d_in, generator=g) * 2 - 1).to(device)
    before = q.forward(x)
    merged = q.merged()
    after = merged.forward(x)
    # the reference's bound is absolute at K = 64 (outputs of order 1); at
    # K = 896 the two summation orders differ by f32 rounding of larger
    # outputs, so the bound scales with them
    assert float((before - after).abs().max()) < 1e-5 * max(1.0, float(before.abs().max()))
    # the merged weight itself, against float64
    w = q.base.weight.cpu().double().numpy()
    a, b = q.adapter().a.cpu().double().numpy(), q.adapter().b.cpu().double().numpy()
    ref = w + (a @ b) * q.adapter().scaling()
    got = merged.weight.cpu().double().numpy()
    assert np.max(np.abs(got - ref)) <= TOL_F32 * max(np.max(np.abs(ref)), 1.0)
    assert torch.equal(merged.bias, q.base.bias)


def test_quantize_module_touches_only_weight_shaped_params(device, oracle):
    # src/quantize.rs:1102-1130: skipped modules bit-identical, others on the grid
    g = torch.Generator().manual_seed(7)
    module = {
        "blocks.0.attn.weight": torch.randn(64, 96, generator=g),
        "blocks.0.attn.bias": torch.randn(96, generator=g),
        "blocks.0.norm.weight": torch.randn(1, 32, generator=g),     # fewer than 64 values
        "label_embeddings.weight": torch.randn(10, 64, generator=g),  # skipped by name
        "head.weight": torch.randn(130, 7, generator=g),            # ragged last block
    }
    module = {k: v.to(device) for k, v in module.items()}
    out, count = Q.quantize_module(module, True, skip=["label_embeddings"])
    assert count == 64 * 96 + 130 * 7
    for k in ("blocks.0.attn.bias", "blocks.0.norm.weight", "label_embeddings.weight"):
        assert out[k] is module[k]
    for k in ("blocks.0.attn.weight", "head.weight"):
        v = module[k].cpu().numpy().reshape(-1)
        packed, absmax = oracle.quantize_packed(v)
        dqc, sos = oracle.double_quantize(absmax)
        want = oracle.dequantize_packed(packed, v.size, None, dqc, sos)
        got = out[k].cpu().numpy().reshape(-1)
        assert out[k].shape == module[k].shape
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), k


def test_quantized_weights_stay_on_the_grid(device, oracle):
    # src/quantize.rs:1133-1160
    g = torch.Generator().manual_seed(11)
    t = torch.randn(4, Q.BLOCK_SIZE, generator=g)
    restored = Q.quantize_dequantize_tensor(t.to(device), False).cpu().numpy().reshape(-1)
    levels = oracle.levels()
    for blk, chunk in enumerate(t.numpy().reshape(-1, Q.BLOCK_SIZE)):
        am = float(np.max(np.abs(chunk)))
        for i in range(Q.BLOCK_SIZE):
            r = restored[blk * Q.BLOCK_SIZE + i]
            assert np.any(np.abs(levels * np.float32(am) - r) <= 1e-6 * max(am, 1.0))
