"""Host-side logic of the module-level mirrors (no device needed): adapter
configuration checks (src/qwennet.rs:732-746), residency accounting
(src/qwennet.rs:1636-1680), and the quantizer's parameter filter
(src/quantize.rs:452-476)."""
from __future__ import annotations

import math

import pytest

from unifur_amd import quantize as Q
from unifur_amd import qwennet as QN


def test_qwen_lora_config_defaults_and_validation():
    c = QN.QwenLoraConfig()
    assert (c.rank, c.alpha) == (16, 16.0)
    c.validate()
    for bad in (QN.QwenLoraConfig(rank=0), QN.QwenLoraConfig(alpha=0.0), QN.QwenLoraConfig(alpha=-1.0),
                QN.QwenLoraConfig(alpha=math.inf), QN.QwenLoraConfig(alpha=math.nan)):
        with pytest.raises(ValueError):
            bad.validate()


def test_residency_report_accounting():
    r = QN.Nf4ResidencyReport()
    r.record("q_proj", 100, QN.WeightStore.NF4)
    r.record("q_proj", 50, QN.WeightStore.F32)
    r.record_f32("norm", 8)
    r.record("mlp", 30, QN.WeightStore.NF4)
    r.note_scratch(1000)
    r.note_scratch(10)
    assert (r.packed_bytes, r.f32_kept_bytes, r.total_resident_bytes()) == (130, 58, 188)
    assert r.peak_scratch_bytes == 1000
    rows = {c.cls: (c.tensors, c.packed_bytes, c.f32_bytes) for c in r.by_class}
    assert rows == {"q_proj": (2, 100, 50), "norm": (1, 0, 8), "mlp": (1, 30, 0)}
    assert [c.cls for c in r.by_class] == ["q_proj", "norm", "mlp"]  # first-seen order


def test_quantizer_parameter_filter():
    q = Q.Nf4Quantizer(True).skipping("label_embeddings")
    assert q.should_quantize("blocks.0.attn.weight", (64, 96))
    assert not q.should_quantize("blocks.0.attn.bias", (96,))           # rank 1
    assert not q.should_quantize("blocks.0.norm.weight", (1, 63))       # < 64 values
    assert q.should_quantize("blocks.0.norm.weight", (1, 64))
    assert not q.should_quantize("label_embeddings.weight", (10, 64))   # module path skipped
    assert not q.should_quantize("model.my_label_embeddings_2.weight", (10, 64))  # substring of a part
    assert q.should_quantize("label.weight", (10, 64))
    # the parameter's own name is not part of the module path
    assert Q.Nf4Quantizer(False).skipping("weight").should_quantize("a.weight", (8, 8))
