"""Host-side mirror of the NF4 residency types of unifur's ``src/qwennet.rs``.

=====================================  ==========================================
this module                            reference (s-b-repo/unifur)
=====================================  ==========================================
``QwenLoraConfig``                     ``QwenLoraConfig`` (src/qwennet.rs:703-747)
``QwenLinear``                         ``QwenLinear`` (src/qwennet.rs:293-435)
``WeightStore``                        ``WeightStore`` (src/qwennet.rs:1598-1607)
``Nf4ResidencyReport``                 ``Nf4ResidencyReport`` (src/qwennet.rs:1609-1681)
``qwen_linear``                        ``qwen_linear`` (src/qwennet.rs:1683-1726)
``projections_to_nf4``                 ``QwenTrunk::to_nf4`` (src/qwennet.rs:1185-1269), projections only
=====================================  ==========================================

Every computation is a call into ``libunifur_nf4.so`` (through
``unifur_amd.quantize``); the checkpoint transpose of the loader is fused into
the quantize kernel (``unifur_nf4_quantize_transposed``).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field
from enum import Enum
from typing import Optional

import torch

from . import _lib as L
from . import quantize as Q


@dataclass
class QwenLoraConfig:
    """Adapter hyperparameters: rank 16, alpha 16 by default."""
    rank: int = 16
    alpha: float = 16.0

    def validate(self) -> None:
        if self.rank < 1:
            raise ValueError(f"lora rank must be positive, not {self.rank}")
        if not (math.isfinite(self.alpha) and self.alpha > 0.0):
            raise ValueError(f"lora alpha must be positive and finite, not {self.alpha}")


class QwenLinear:
    """Residency switch of a projection: F32 (``DenseLinear``), Nf4
    (``Nf4Linear``) or Qlora (``QloraLinear``); all forward to the same
    function and differ only in memory."""

    F32, NF4, QLORA = "F32", "Nf4", "Qlora"

    def __init__(self, kind: str, inner):
        if kind not in (self.F32, self.NF4, self.QLORA):
            raise ValueError(f"unknown residency {kind}")
        self.kind = kind
        self.inner = inner

    def forward(self, x: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        return self.inner.forward(x, out_dtype)

    __call__ = forward

    def d_input(self) -> int:
        return self.inner.base.d_input() if self.kind == self.QLORA else self.inner.d_input()

    def d_output(self) -> int:
        return self.inner.base.d_output() if self.kind == self.QLORA else self.inner.d_output()

    def resident_bytes(self) -> int:
        """src/qwennet.rs:357-370."""
        if self.kind == self.F32:
            return 4 * self.inner.weight.numel()
        if self.kind == self.NF4:
            return self.inner.resident_bytes()
        ad = self.inner.adapter
        return self.inner.base.resident_bytes() + 4 * (ad.in_features() + ad.out_features()) * ad.rank()

    def to_nf4(self) -> "QwenLinear":
        """src/qwennet.rs:378-413: an f32 weight ([d_in, d_out], already in
        the packed order) into NF4 residency with double quantization; the
        bias stays f32.  A weight carrying an adapter is an error."""
        if self.kind == self.F32:
            d_in, d_out = self.inner.weight.shape
            nf4 = Q.Nf4Linear.from_values(self.inner.weight.contiguous().view(-1), d_in, d_out)
            nf4.bias = self.inner.bias
            return QwenLinear(self.NF4, nf4)
        if self.kind == self.NF4:
            return self
        raise ValueError("a weight carrying an adapter must be de-adapted before conversion")

    def with_lora(self, config: QwenLoraConfig, device="cuda",
                  generator: Optional[torch.Generator] = None) -> "QwenLinear":
        """src/qwennet.rs:419-434: attach a fresh (B = 0, exact no-op) adapter
        to an NF4-resident base; f32 bases and double attachment are errors."""
        config.validate()
        if self.kind == self.NF4:
            base = self.inner
            cfg = Q.LoraConfig.new(base.d_input(), base.d_output(), config.rank).with_alpha(config.alpha)
            return QwenLinear(self.QLORA, Q.QloraLinear(base, Q.LoraAdapter.new(cfg, device, generator)))
        if self.kind == self.F32:
            raise ValueError("LoRA adapters attach to NF4-resident weights only")
        raise ValueError("weight already carries a LoRA adapter")


class WeightStore(Enum):
    F32 = "F32"
    NF4 = "Nf4"


@dataclass
class ClassResidency:
    cls: str
    tensors: int = 0
    packed_bytes: int = 0
    f32_bytes: int = 0


@dataclass
class Nf4ResidencyReport:
    """Resident-memory accounting of a load (src/qwennet.rs:1609-1681)."""
    packed_bytes: int = 0
    f32_kept_bytes: int = 0
    by_class: list = field(default_factory=list)
    peak_scratch_bytes: int = 0

    def total_resident_bytes(self) -> int:
        return self.packed_bytes + self.f32_kept_bytes

    def class_mut(self, cls: str) -> ClassResidency:
        for row in self.by_class:
            if row.cls == cls:
                return row
        row = ClassResidency(cls)
        self.by_class.append(row)
        return row

    def record(self, cls: str, nbytes: int, store: WeightStore) -> None:
        row = self.class_mut(cls)
        if store == WeightStore.NF4:
            self.packed_bytes += nbytes
            row.packed_bytes += nbytes
        else:
            self.f32_kept_bytes += nbytes
            row.f32_bytes += nbytes
        row.tensors += 1

    def record_f32(self, cls: str, nbytes: int) -> None:
        self.f32_kept_bytes += nbytes
        row = self.class_mut(cls)
        row.f32_bytes += nbytes
        row.tensors += 1

    def note_scratch(self, nbytes: int) -> None:
        self.peak_scratch_bytes = max(self.peak_scratch_bytes, nbytes)


def qwen_linear(tensor: torch.Tensor, store: WeightStore) -> tuple:
    """src/qwennet.rs:1687-1726: one decoded checkpoint linear [out, in]
    (f32 or bf16, on the device) into a QwenLinear in the requested storage,
    with the resident bytes of the chosen form.  Nf4: transposed to
    [in, out] and quantized in one kernel, then double-quantized."""
    if tensor.dim() != 2:
        raise ValueError(f"tensor of shape {tuple(tensor.shape)} is not rank-2")
    Q._require_cuda(tensor, "tensor")
    rows, cols = tensor.shape  # [out, in]
    if store == WeightStore.F32:
        w = tensor.float().t().contiguous()
        return QwenLinear(QwenLinear.F32, Q.DenseLinear(w)), 4 * tensor.numel()
    n = rows * cols
    if rows % 64 == 0:
        codes = torch.empty((n + 1) // 2, dtype=torch.uint8, device=tensor.device)
        absmax = torch.empty((n + 63) // 64, dtype=torch.float32, device=tensor.device)
        L.check(L.lib().unifur_nf4_quantize_transposed(tensor.data_ptr(), Q._dtype_code(tensor.dtype), rows, cols,
                                                       codes.data_ptr(), absmax.data_ptr(), Q._stream()))
        packed = Q.PackedNf4Tensor(codes, n, absmax=absmax)
    else:  # blocks straddle rows of the transposed buffer: transpose, then quantize
        packed = Q.PackedNf4Tensor.quantize(tensor.float().t().contiguous().view(-1))
    packed = packed.with_double_quantization()
    nbytes = packed.resident_bytes()
    return QwenLinear(QwenLinear.NF4, Q.Nf4Linear.from_packed(packed, cols, rows)), nbytes


def projections_to_nf4(projections: dict, report: Optional[Nf4ResidencyReport] = None) -> dict:
    """QwenTrunk::to_nf4 (src/qwennet.rs:1196-1269) over a mapping of
    projection names to QwenLinear: every F32 projection to NF4 residency,
    recorded per class (the last dotted component, e.g. ``q_proj``)."""
    out = {}
    for name, lin in projections.items():
        conv = lin.to_nf4()
        if report is not None:
            report.record(name.split(".")[-1], conv.resident_bytes(), WeightStore.NF4)
        out[name] = conv
    return out
