"""The load path end to end: a safetensors shard of [out, in] linears in
F32, BF16 and F16 (read by range, src/import.rs:243-280) to resident NF4
through the library's checkpoint pass, each weight byte for byte the
oracle's decode (read_tensor_f32) + transpose2d + PackedNf4Tensor::quantize
+ with_double_quantization (qwen_linear, src/qwennet.rs:1687-1726)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from unifur_amd import safetensors_io as S

from test_safetensors_io import write_shard

pytestmark = pytest.mark.gpu


def test_shard_to_resident_nf4(device, oracle, tmp_path):
    specs = [("model.layers.0.self_attn.q_proj.weight", "BF16", 896, 896),
             ("model.layers.0.self_attn.k_proj.weight", "BF16", 128, 896),
             ("model.layers.0.mlp.gate_proj.weight", "F16", 4864, 896),
             ("model.layers.0.mlp.down_proj.weight", "F16", 896, 4864),
             ("model.layers.0.extra.weight", "F32", 192, 100),
             ("model.layers.0.ragged.weight", "BF16", 100, 64)]  # out % 64 != 0: the separate transpose
    tensors, want = [], {}
    for i, (name, dt, out_f, in_f) in enumerate(specs):
        v = oracle.fill_normal(0x5A7 + i, 0.02, out_f * in_f)
        if dt == "F32":
            raw, f = v.astype("<f4").tobytes(), v
        elif dt == "BF16":
            f = oracle.round_bf16(v)
            raw = (f.view(np.uint32) >> 16).astype("<u2").tobytes()
        else:
            h = v.astype(np.float16)
            raw, f = h.astype("<f2").tobytes(), oracle.decode_checkpoint(h.view(np.uint16), "f16")
        tensors.append((name, dt, [out_f, in_f], raw))
        want[name] = (f, out_f, in_f)
    path = write_shard(tmp_path, tensors)
    idx = S.open_index(path)
    names = [s[0] for s in specs]
    got = S.load_checkpoint_linears(path, idx, names, device=device)
    torch.cuda.synchronize()
    for name, (lin, nbytes) in zip(names, got):
        f, out_f, in_f = want[name]
        print(f"load {name} {out_f}x{in_f}", flush=True)
        packed, absmax = oracle.quantize_packed(oracle.transpose(f, out_f, in_f))
        q, sos = oracle.double_quantize(absmax)
        p = lin.inner.packed()
        assert (lin.d_input(), lin.d_output()) == (in_f, out_f)
        assert np.array_equal(p.codes.cpu().numpy(), packed), f"{name}: codes"
        assert np.array_equal(p.dq_codes.cpu().numpy(), q), f"{name}: u8 scales"
        assert p.scale_of_scales.cpu().numpy()[0].view(np.uint32) == np.float32(sos).view(np.uint32), name
        assert nbytes == oracle.estimated_resident_bytes(out_f * in_f, True)
        assert lin.inner.is_striped() == (out_f % 64 == 0)


def test_non_finite_checkpoint_is_refused(device, tmp_path):
    bad = np.zeros((64, 8), np.float16)
    bad[3, 3] = np.inf
    path = write_shard(tmp_path, [("w", "F16", [64, 8], bad.astype("<f2").tobytes())])
    idx = S.open_index(path)
    with pytest.raises(ValueError, match="non-finite"):
        S.load_checkpoint_linears(path, idx, ["w"], device=device)
