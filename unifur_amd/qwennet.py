"""Host-side mirror of the NF4 residency types of unifur's ``src/qwennet.rs``.

=====================================  ==========================================
this module                            reference (s-b-repo/unifur)
=====================================  ==========================================
``QwenLoraConfig``                     ``QwenLoraConfig`` (src/qwennet.rs:703-747)
``QwenLinear``                         ``QwenLinear`` (src/qwennet.rs:293-435)
``Nf4Embedding``                       ``Nf4Embedding`` (src/qwennet.rs:244-291)
``WeightStore``                        ``WeightStore`` (src/qwennet.rs:1598-1607)
``Nf4ResidencyReport``                 ``Nf4ResidencyReport`` (src/qwennet.rs:1609-1681)
``qwen_linear``                        ``qwen_linear`` (src/qwennet.rs:1683-1726)
``projections_to_nf4``                 ``QwenTrunk::to_nf4`` (src/qwennet.rs:1185-1269), projections only
``QwenDecoderLayer``                   ``QwenDecoderLayer::step`` (src/qwennet.rs:1112-1129), the NF4
                                       projections and norms around a caller-supplied attention
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


class Nf4Embedding:
    """NF4-resident embedding table (src/qwennet.rs:244-291): the
    ``[n_embedding, d_model]`` table as one packed tensor with double
    quantization.  ``forward`` gathers and dequantizes only the selected rows
    (the reference dequantizes the whole table per call, then gathers);
    the rows are the reference's f32 values bit for bit."""

    def __init__(self, packed: Q.PackedNf4Tensor, n_embedding: int, d_model: int):
        if len(packed) != n_embedding * d_model:
            raise ValueError(f"packed table holds {len(packed)} values, not {n_embedding} x {d_model}")
        self.packed = packed
        self.n_embedding = int(n_embedding)
        self.d_model = int(d_model)

    @staticmethod
    def from_values(values: torch.Tensor, n_embedding: int, d_model: int) -> "Nf4Embedding":
        """src/qwennet.rs:265-271: quantize the row-major table, then double quantization."""
        v = values.reshape(-1)
        if v.numel() != n_embedding * d_model:
            raise ValueError(f"{v.numel()} values for a {n_embedding} x {d_model} table")
        return Nf4Embedding(Q.PackedNf4Tensor.quantize(v.contiguous()).with_double_quantization(), n_embedding,
                            d_model)

    def resident_bytes(self) -> int:
        """src/qwennet.rs:274-276."""
        return self.packed.resident_bytes()

    def dequantized_weight(self) -> torch.Tensor:
        """src/qwennet.rs:279-286: the whole ``[n_embedding, d_model]`` f32 table."""
        return self.packed.dequantize().view(self.n_embedding, self.d_model)

    def forward(self, ids: torch.Tensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """src/qwennet.rs:288-290: ``ids`` int64 or int32 of any shape ->
        ``[*ids.shape, d_model]``.  An id outside ``[0, n_embedding)`` yields
        a row of NaN (burn would panic)."""
        if ids.dtype not in (torch.int64, torch.int32):
            raise ValueError("ids must be int64 or int32")
        if not ids.is_cuda:
            raise ValueError("ids must be a device tensor")
        flat = ids.reshape(-1).contiguous()
        out = torch.empty(flat.numel(), self.d_model, dtype=dtype, device=flat.device)
        s = self.packed.scales_struct()
        L.check(L.lib().unifur_nf4_embedding_forward(
            self.packed.codes.data_ptr(), ctypes.byref(s), self.n_embedding, self.d_model, flat.data_ptr(),
            L.IDS_I64 if flat.dtype == torch.int64 else L.IDS_I32, flat.numel(), out.data_ptr(),
            L.BF16 if dtype == torch.bfloat16 else L.F32, torch.cuda.current_stream().cuda_stream))
        return out.view(*ids.shape, self.d_model)


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
    (f32, bf16 or f16, on the device) into a QwenLinear in the requested storage,
    with the resident bytes of the chosen form.  Nf4: transposed to
    [in, out], quantized and double-quantized -- for out % 64 == 0 in one
    grouped pass straight into the striped resident form
    (quantize_checkpoint_linears: transpose, quantize and the scales' max in
    the kernels, three launches); otherwise the blocks straddle rows of the
    transposed buffer, which the library transposes first
    (unifur_nf4_transpose_checkpoint) and quantizes flat."""
    if tensor.dim() != 2:
        raise ValueError(f"tensor of shape {tuple(tensor.shape)} is not rank-2")
    Q._require_cuda(tensor, "tensor")
    rows, cols = tensor.shape  # [out, in]
    if tensor.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise ValueError("checkpoint linears are f32, bf16 or f16")
    src = tensor.contiguous()
    if store == WeightStore.F32:  # linear_param (src/qwennet.rs:1396-1420): the transposed f32 weight
        w = torch.empty(cols, rows, dtype=torch.float32, device=src.device)
        L.check(L.lib().unifur_nf4_transpose_checkpoint(src.data_ptr(), Q._src_dtype_code(src.dtype), rows, cols,
                                                        w.data_ptr(), Q._stream()))
        return QwenLinear(QwenLinear.F32, Q.DenseLinear(w)), 4 * tensor.numel()
    if rows % 64 == 0:
        lin = Q.quantize_checkpoint_linears([src])[0]
    else:
        flat = torch.empty(rows * cols, dtype=torch.float32, device=src.device)
        L.check(L.lib().unifur_nf4_transpose_checkpoint(src.data_ptr(), Q._src_dtype_code(src.dtype), rows, cols,
                                                        flat.data_ptr(), Q._stream()))
        lin = Q.Nf4Linear.from_packed(Q.PackedNf4Tensor.quantize(flat).with_double_quantization(), cols, rows)
    return QwenLinear(QwenLinear.NF4, lin), lin.resident_bytes()


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


# ------------------------------------------------------- decoder-layer decode --

class QwenDecoderLayer:
    """The NF4 projection chain of one full-attention decoder layer's decode
    step, ``QwenDecoderLayer::step`` (src/qwennet.rs:1112-1129):

        n = input_norm(x); q, k, v = n Wq, n Wk, n Wv      (project, :927-951)
        ctx = attend(q, k, v)                               (the caller's attention)
        x1 = x + ctx Wo
        y = x1 + down(silu(gate(post_norm(x1))) * up(post_norm(x1)))

    ``input_norm`` / ``post_norm`` are QwenRmsNorm weights [hidden] applied as
    ``w + 1`` with epsilon ``eps`` (src/qwennet.rs:104-109).  The per-head QK
    norms, rotary and the attention itself belong to ``attend``: they are not
    on the NF4 path.  Two library calls per step:
    ``unifur_nf4_decoder_attn_in`` and ``unifur_nf4_decoder_attn_out_mlp``."""

    def __init__(self, q_proj: "Q.Nf4Linear", k_proj: "Q.Nf4Linear", v_proj: "Q.Nf4Linear",
                 o_proj: "Q.Nf4Linear", mlp: "Q.QwenMlp", input_norm: torch.Tensor, post_norm: torch.Tensor,
                 eps: float = 1e-6):
        hidden = q_proj.d_input()
        if k_proj.d_input() != hidden or v_proj.d_input() != hidden:
            raise ValueError("q, k and v must share d_input (hidden)")
        if o_proj.d_output() != hidden or mlp.gate_proj.d_input() != hidden:
            raise ValueError("o and the MLP must map hidden back to hidden")
        for name, t in (("input_norm", input_norm), ("post_norm", post_norm)):
            Q._require_cuda(t, name)
            if t.dtype != torch.float32 or t.numel() != hidden:
                raise ValueError(f"{name} must be float32 [hidden]")
        self.q_proj, self.k_proj, self.v_proj, self.o_proj = q_proj, k_proj, v_proj, o_proj
        self.mlp = mlp
        self.input_norm, self.post_norm, self.eps = input_norm, post_norm, float(eps)

    def hidden(self) -> int:
        return self.q_proj.d_input()

    def layer_struct(self) -> L.DecoderLayer:
        m = self.mlp
        return L.DecoderLayer(self.q_proj.weight_struct(), self.k_proj.weight_struct(), self.v_proj.weight_struct(),
                              self.o_proj.weight_struct(), m.gate_proj.weight_struct(), m.up_proj.weight_struct(),
                              m.down_proj.weight_struct(), self.input_norm.data_ptr(), self.post_norm.data_ptr(),
                              self.eps)

    def _rows(self, x: torch.Tensor, width: int, name: str) -> int:
        Q._require_cuda(x, name)
        if x.shape[-1] != width:
            raise ValueError(f"{name} has last dim {x.shape[-1]}, expected {width}")
        return x.numel() // width

    def project(self, x: torch.Tensor):
        """q, k, v of input_norm(x) (before the per-head QK norms)."""
        rows = self._rows(x, self.hidden(), "x")
        lead = x.shape[:-1]
        q = torch.empty(*lead, self.q_proj.d_output(), dtype=x.dtype, device=x.device)
        k = torch.empty(*lead, self.k_proj.d_output(), dtype=x.dtype, device=x.device)
        v = torch.empty(*lead, self.v_proj.d_output(), dtype=x.dtype, device=x.device)
        layer = self.layer_struct()
        L.check(L.lib().unifur_nf4_decoder_attn_in(x.data_ptr(), Q._dtype_code(x.dtype), rows, ctypes.byref(layer),
                                                    q.data_ptr(), k.data_ptr(), v.data_ptr(), None, 0,
                                                    Q._stream()))
        return q, k, v

    def attn_out_mlp(self, x: torch.Tensor, ctx: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x + ctx Wo, then its MLP residual: the step's output."""
        rows = self._rows(x, self.hidden(), "x")
        if self._rows(ctx, self.o_proj.d_input(), "ctx") != rows or ctx.dtype != x.dtype:
            raise ValueError("ctx must hold one row per row of x, in x's dtype")
        y = torch.empty_like(x) if out is None else out
        if y.shape != x.shape or y.dtype != x.dtype or not y.is_contiguous():
            raise ValueError("out must be a contiguous tensor shaped and typed like x")
        layer = self.layer_struct()
        L.check(L.lib().unifur_nf4_decoder_attn_out_mlp(x.data_ptr(), ctx.data_ptr(), Q._dtype_code(x.dtype), rows,
                                                         ctypes.byref(layer), y.data_ptr(), None, 0, Q._stream()))
        return y

    def step(self, x: torch.Tensor, attend) -> torch.Tensor:
        """One decode step: ``attend(q, k, v) -> ctx`` supplies the attention."""
        q, k, v = self.project(x)
        return self.attn_out_mlp(x, attend(q, k, v))
