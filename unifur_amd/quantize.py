"""Host-side mirror of unifur's NF4 API over the MI355X library.

Names, argument meaning and error behaviour follow the reference's Rust
types so that code written against them reads the same:

=====================================  ==========================================
this module                            reference (s-b-repo/unifur)
=====================================  ==========================================
``BLOCK_SIZE``, ``nf4_levels()``       ``BLOCK_SIZE``, ``NF4_LEVELS`` (src/quantize.rs:37, :49-66)
``PackedNf4Tensor``                    ``PackedNf4Tensor`` (src/quantize.rs:249-400)
``Nf4Tensor``                          ``Nf4Tensor`` (src/quantize.rs:79-201)
``quantize_dequantize_tensor``         ``quantize_dequantize_tensor`` (src/quantize.rs:404-416)
``LoraConfig``, ``LoraAdapter``        ``LoraConfig``, ``LoraAdapter`` (src/quantize.rs:513-635)
``Nf4Linear``                          ``Nf4Linear`` (src/qwennet.rs:161-242)
``QloraLinear``                        ``QloraLinear`` (src/qwennet.rs:311-345)
``QwenMlp``                            ``QwenMlp`` (src/qwennet.rs:786-820)
=====================================  ==========================================

Device memory and streams come from PyTorch (tensors on ``cuda``); every
computation is a call into ``libunifur_nf4.so``.  There is no CPU or torch
fallback: without the built library, or without a GPU, calls raise.
"""
from __future__ import annotations

import ctypes
import itertools
import math
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib as L

BLOCK_SIZE = L.BLOCK_SIZE


def nf4_levels() -> list[float]:
    """NF4_LEVELS as the library holds them (src/quantize.rs:49-66)."""
    out = (ctypes.c_float * 16)()
    L.check(L.lib().unifur_nf4_levels(out))
    return list(out)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return L.F32
    if dtype == torch.bfloat16:
        return L.BF16
    raise ValueError(f"unsupported dtype {dtype}; the NF4 path takes float32 or bfloat16")


def _src_dtype_code(dtype: torch.dtype) -> int:
    """A checkpoint tensor's element type: the three read_tensor_f32 decodes
    (src/import.rs:255-272)."""
    if dtype == torch.float16:
        return L.F16
    if dtype in (torch.float32, torch.bfloat16):
        return _dtype_code(dtype)
    raise ValueError(f"unsupported checkpoint dtype {dtype}; checkpoints are float32, bfloat16 or float16")


def _require_cuda(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a CUDA (HIP) device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


class PackedNf4Tensor:
    """Packed NF4 storage: two codes per byte, low nibble first, per-block
    f32 absmax or double-quantized u8 scales (src/quantize.rs:235-257)."""

    def __init__(self, codes: torch.Tensor, length: int, absmax: Optional[torch.Tensor] = None,
                 dq_codes: Optional[torch.Tensor] = None, scale_of_scales: Optional[torch.Tensor] = None):
        self.codes = codes
        self._len = int(length)
        self.absmax = absmax
        self.dq_codes = dq_codes
        self.scale_of_scales = scale_of_scales  # 1-element f32 device tensor

    # -- construction -------------------------------------------------------------
    @staticmethod
    def quantize(values: torch.Tensor) -> "PackedNf4Tensor":
        """PackedNf4Tensor::quantize (src/quantize.rs:262-279) on a flat f32 view."""
        _require_cuda(values, "values")
        if values.dtype != torch.float32:
            raise ValueError("quantize takes float32 values, as the reference's &[f32]")
        n = values.numel()
        nb = (n + BLOCK_SIZE - 1) // BLOCK_SIZE
        codes = torch.empty((n + 1) // 2, dtype=torch.uint8, device=values.device)
        absmax = torch.empty(nb, dtype=torch.float32, device=values.device)
        L.check(L.lib().unifur_nf4_quantize(values.data_ptr(), n, codes.data_ptr(), absmax.data_ptr(), _stream()))
        return PackedNf4Tensor(codes, n, absmax=absmax)

    def with_double_quantization(self) -> "PackedNf4Tensor":
        """src/quantize.rs:284-309; idempotent."""
        if self.is_double_quantized():
            return self
        nb = self.num_blocks()
        dq = torch.empty(nb, dtype=torch.uint8, device=self.codes.device)
        sos = torch.empty(1, dtype=torch.float32, device=self.codes.device)
        L.check(L.lib().unifur_nf4_double_quantize(self.absmax.data_ptr(), nb, dq.data_ptr(), sos.data_ptr(),
                                                   _stream()))
        return PackedNf4Tensor(self.codes, self._len, dq_codes=dq, scale_of_scales=sos)

    # -- accessors -------------------------------------------------------------------
    def is_double_quantized(self) -> bool:
        return self.dq_codes is not None

    def __len__(self) -> int:
        return self._len

    def len(self) -> int:
        return self._len

    def is_empty(self) -> bool:
        return self._len == 0

    def num_blocks(self) -> int:
        return int(L.lib().unifur_nf4_num_blocks(self._len))

    def scales_struct(self) -> L.Scales:
        if self.is_double_quantized():
            return L.Scales(L.SCALES_DOUBLE_QUANTIZED, None, self.dq_codes.data_ptr(),
                            self.scale_of_scales.data_ptr())
        return L.Scales(L.SCALES_F32, self.absmax.data_ptr(), None, None)

    def dequantize(self, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """src/quantize.rs:355-366: f32 bit-identical to the reference, or bf16
        (that f32 rounded to nearest even)."""
        out = torch.empty(self._len, dtype=dtype, device=self.codes.device)
        s = self.scales_struct()
        L.check(L.lib().unifur_nf4_dequantize(self.codes.data_ptr(), ctypes.byref(s), self._len, out.data_ptr(),
                                              _dtype_code(dtype), _stream()))
        return out

    def resident_bytes(self) -> int:
        """src/quantize.rs:370-376."""
        return PackedNf4Tensor.estimated_resident_bytes(self._len, self.is_double_quantized())

    def bits_per_value(self) -> float:
        """src/quantize.rs:382-388."""
        return float(L.lib().unifur_nf4_bits_per_value(self._len, int(self.is_double_quantized())))

    @staticmethod
    def estimated_resident_bytes(length: int, double_quantized: bool) -> int:
        """src/quantize.rs:391-399."""
        return int(L.lib().unifur_nf4_estimated_resident_bytes(length, int(double_quantized)))


class Nf4Tensor:
    """The reference's simulated form (src/quantize.rs:79-201): one code per
    byte (``codes``, u8[len], the concatenated ``Nf4Block::codes``), the f32
    absmax of every block (kept after double quantization, as the
    reference's blocks keep theirs), and with double quantization the u8
    scale codes and the scale of scales.

    Its codes are those of the packed codec (PackedNf4Tensor::quantize takes
    them from Nf4Tensor::quantize, src/quantize.rs:262-265), unpacked on the
    device; its dequantize packs them back and runs the packed dequantize,
    which is bit-identical to Nf4Tensor::dequantize (src/quantize.rs:353-354)."""

    def __init__(self, codes: torch.Tensor, absmax: torch.Tensor, dq_codes: Optional[torch.Tensor] = None,
                 scale_of_scales: Optional[torch.Tensor] = None):
        self.codes = codes
        self.absmax = absmax
        self.dq_codes = dq_codes
        self.scale_of_scales = scale_of_scales

    @staticmethod
    def quantize(values: torch.Tensor) -> "Nf4Tensor":
        """Nf4Tensor::quantize (src/quantize.rs:99-124)."""
        p = PackedNf4Tensor.quantize(values)
        codes = torch.empty(len(p), dtype=torch.uint8, device=values.device)
        L.check(L.lib().unifur_nf4_unpack_codes(p.codes.data_ptr(), len(p), codes.data_ptr(), _stream()))
        return Nf4Tensor(codes, p.absmax)

    def with_double_quantization(self) -> "Nf4Tensor":
        """src/quantize.rs:128-149: recomputed from the kept absmax values,
        so applying it twice gives the same codes."""
        nb = self.num_blocks()
        dq = torch.empty(nb, dtype=torch.uint8, device=self.codes.device)
        sos = torch.empty(1, dtype=torch.float32, device=self.codes.device)
        L.check(L.lib().unifur_nf4_double_quantize(self.absmax.data_ptr(), nb, dq.data_ptr(), sos.data_ptr(),
                                                   _stream()))
        return Nf4Tensor(self.codes, self.absmax, dq_codes=dq, scale_of_scales=sos)

    def is_double_quantized(self) -> bool:
        return self.dq_codes is not None

    def len(self) -> int:
        return self.codes.numel()

    def __len__(self) -> int:
        return self.codes.numel()

    def is_empty(self) -> bool:
        return self.codes.numel() == 0

    def num_blocks(self) -> int:
        return self.absmax.numel()

    def packed(self) -> PackedNf4Tensor:
        """The same codes two per byte, with this tensor's scales."""
        n = self.len()
        bytes_ = torch.empty((n + 1) // 2, dtype=torch.uint8, device=self.codes.device)
        L.check(L.lib().unifur_nf4_pack_codes(self.codes.data_ptr(), n, bytes_.data_ptr(), _stream()))
        if self.is_double_quantized():
            return PackedNf4Tensor(bytes_, n, dq_codes=self.dq_codes, scale_of_scales=self.scale_of_scales)
        return PackedNf4Tensor(bytes_, n, absmax=self.absmax)

    def dequantize(self, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """Nf4Tensor::dequantize (src/quantize.rs:177-185)."""
        return self.packed().dequantize(dtype)

    def bits_per_value(self) -> float:
        """src/quantize.rs:190-200: quotes a 4-bit payload it does not pack."""
        return float(L.lib().unifur_nf4_simulated_bits_per_value(self.len(), int(self.is_double_quantized())))


def quantize_dequantize_tensor(tensor: torch.Tensor, double_quantization: bool) -> torch.Tensor:
    """src/quantize.rs:404-416: the NF4 round trip of a rank-2 tensor, on its
    flat row-major buffer."""
    if tensor.dim() != 2:
        raise ValueError("quantize_dequantize_tensor takes a rank-2 tensor")
    q = PackedNf4Tensor.quantize(tensor.contiguous().view(-1))
    if double_quantization:
        q = q.with_double_quantization()
    return q.dequantize().view(tensor.shape)


# ---------------------------------------------------------------------- LoRA --

@dataclass
class LoraConfig:
    """src/quantize.rs:513-548."""
    in_features: int
    out_features: int
    rank: int
    alpha: float

    @staticmethod
    def new(in_features: int, out_features: int, rank: int) -> "LoraConfig":
        r = max(rank, 1)
        return LoraConfig(in_features, out_features, r, float(r))

    def with_alpha(self, alpha: float) -> "LoraConfig":
        return LoraConfig(self.in_features, self.out_features, self.rank, float(alpha))

    def scaling(self) -> float:
        return self.alpha / max(self.rank, 1)

    def num_parameters(self) -> int:
        return self.rank * (self.in_features + self.out_features)


class LoraAdapter:
    """src/quantize.rs:550-635: a [in, rank], b [rank, out] (f32), scaling."""

    def __init__(self, a: torch.Tensor, b: torch.Tensor, scaling: float):
        _require_cuda(a, "lora a")
        _require_cuda(b, "lora b")
        if a.dtype != torch.float32 or b.dtype != torch.float32:
            raise ValueError("LoRA factors are float32, as the reference's")
        if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[0]:
            raise ValueError(f"LoRA factor shapes {tuple(a.shape)} and {tuple(b.shape)} do not chain")
        self.a = a
        self.b = b
        self._scaling = float(scaling)

    @staticmethod
    def new(config: LoraConfig, device="cuda", generator: Optional[torch.Generator] = None) -> "LoraAdapter":
        """A ~ N(0, 1/rank), B = 0: an exact no-op until trained."""
        std = 1.0 / math.sqrt(max(config.rank, 1))
        a = torch.randn(config.in_features, config.rank, generator=generator, dtype=torch.float32) * std
        b = torch.zeros(config.rank, config.out_features, dtype=torch.float32)
        return LoraAdapter(a.to(device), b.to(device), config.scaling())

    @staticmethod
    def from_parts(a: torch.Tensor, b: torch.Tensor, scaling: float) -> "LoraAdapter":
        return LoraAdapter(a.contiguous(), b.contiguous(), scaling)

    def in_features(self) -> int:
        return self.a.shape[0]

    def out_features(self) -> int:
        return self.b.shape[1]

    def rank(self) -> int:
        return self.a.shape[1]

    def scaling(self) -> float:
        return self._scaling

    def struct(self) -> L.Lora:
        return L.Lora(self.a.data_ptr(), self.b.data_ptr(), self.rank(), self._scaling)


# ------------------------------------------------------------------- linears --

def _weight_struct(packed: PackedNf4Tensor, d_in: int, d_out: int) -> L.Weight:
    return L.Weight(packed.codes.data_ptr(), packed.scales_struct(), d_in, d_out, L.LAYOUT_ROW_MAJOR)


class Nf4Linear:
    """A frozen NF4-resident linear with weight [d_input, d_output]
    (src/qwennet.rs:161-242); forward never materialises the weight.

    The packed weight is held on the device in the column-striped layout
    when d_output % 64 == 0 (``striped=None`` picks it then): a byte
    permutation of the reference's packed codes and scales, same size, that
    the decode GEMV streams contiguously.  ``packed()`` rebuilds the
    reference-layout tensor bit for bit."""

    def __init__(self, packed: PackedNf4Tensor, d_input: int, d_output: int, bias: Optional[torch.Tensor] = None,
                 striped: Optional[bool] = None):
        if len(packed) != d_input * d_output:
            raise ValueError(f"packed weight holds {len(packed)} values, [{d_input}, {d_output}] needs "
                             f"{d_input * d_output}")
        if bias is not None:
            _require_cuda(bias, "bias")
            if bias.dtype != torch.float32 or bias.numel() != d_output:
                raise ValueError("bias must be float32 [d_output]")
        if striped is None:
            striped = d_output % 64 == 0
        if striped and d_output % 64 != 0:
            raise ValueError("the striped layout needs d_output % 64 == 0")
        self._d_in = int(d_input)
        self._d_out = int(d_output)
        self.bias = bias
        self._striped = bool(striped)
        self._len = len(packed)
        self._dq = packed.is_double_quantized()
        self._sos = packed.scale_of_scales
        if self._striped:
            src = _weight_struct(packed, d_input, d_output)
            self._codes = torch.empty_like(packed.codes)
            self._scales = torch.empty_like(packed.dq_codes if self._dq else packed.absmax)
            L.check(L.lib().unifur_nf4_stripe_weight(ctypes.byref(src), self._codes.data_ptr(),
                                                     self._scales.data_ptr(), _stream()))
            self._packed = None
        else:
            self._codes = packed.codes
            self._scales = packed.dq_codes if self._dq else packed.absmax
            self._packed = packed

    @staticmethod
    def from_packed(packed: PackedNf4Tensor, d_input: int, d_output: int,
                    bias: Optional[torch.Tensor] = None, striped: Optional[bool] = None) -> "Nf4Linear":
        return Nf4Linear(packed, d_input, d_output, bias, striped)

    @staticmethod
    def from_values(values: torch.Tensor, d_input: int, d_output: int, striped: Optional[bool] = None) -> "Nf4Linear":
        """src/qwennet.rs:198-205: quantize [d_input, d_output] row-major values,
        always with double quantization."""
        return Nf4Linear(PackedNf4Tensor.quantize(values.contiguous().view(-1)).with_double_quantization(),
                         d_input, d_output, striped=striped)

    @classmethod
    def _from_striped(cls, codes: torch.Tensor, dq_codes: torch.Tensor, scale_of_scales: torch.Tensor, d_input: int,
                      d_output: int) -> "Nf4Linear":
        """A layer over already-striped, double-quantized device buffers."""
        self = cls.__new__(cls)
        self._d_in, self._d_out = int(d_input), int(d_output)
        self.bias = None
        self._striped = True
        self._len = self._d_in * self._d_out
        self._dq = True
        self._sos = scale_of_scales
        self._codes = codes
        self._scales = dq_codes
        self._packed = None
        return self

    @classmethod
    def _from_group(cls, group: tuple, i: int, d_input: int, d_output: int) -> "Nf4Linear":
        """Layer i of a grouped quantize pass: group = (codes, code offsets,
        dq codes, scale offsets, scales of scales), one allocation each for
        the whole pass.  Its slices of them are made on first use (slicing
        three views per layer up front cost a 168-weight pass more host time
        than its launches)."""
        self = cls.__new__(cls)
        self._d_in, self._d_out = d_input, d_output
        self.bias = None
        self._striped = True
        self._len = d_input * d_output
        self._dq = True
        self._packed = None
        self._group = (group, i)
        return self

    def __getattr__(self, name: str):
        # reached only for attributes not set: the slices of a grouped pass
        if name in ("_codes", "_scales", "_sos"):
            g = self.__dict__.get("_group")
            if g is not None:
                (codes, c_off, dq, s_off, sos), i = g
                self._codes = codes[c_off[i]:c_off[i + 1]]
                self._scales = dq[s_off[i]:s_off[i + 1]]
                self._sos = sos[i:i + 1]
                del self._group
                return self.__dict__[name]
        raise AttributeError(f"{type(self).__name__!r} object has no attribute {name!r}")

    def d_input(self) -> int:
        return self._d_in

    def d_output(self) -> int:
        return self._d_out

    def is_striped(self) -> bool:
        return self._striped

    def resident_bytes(self) -> int:
        return PackedNf4Tensor.estimated_resident_bytes(self._len, self._dq)

    def packed(self) -> PackedNf4Tensor:
        """The reference-layout packed tensor (rebuilt on the device from the
        striped copy when the layer holds that)."""
        if self._packed is not None:
            return self._packed
        codes = torch.empty_like(self._codes)
        scales = torch.empty_like(self._scales)
        w = self.weight_struct()
        L.check(L.lib().unifur_nf4_unstripe_weight(ctypes.byref(w), codes.data_ptr(), scales.data_ptr(), _stream()))
        if self._dq:
            return PackedNf4Tensor(codes, self._len, dq_codes=scales, scale_of_scales=self._sos)
        return PackedNf4Tensor(codes, self._len, absmax=scales)

    def dequantized_weight(self) -> torch.Tensor:
        """src/qwennet.rs:230-236."""
        return self.packed().dequantize().view(self._d_in, self._d_out)

    def weight_struct(self) -> L.Weight:
        if self._dq:
            sc = L.Scales(L.SCALES_DOUBLE_QUANTIZED, None, self._scales.data_ptr(), self._sos.data_ptr())
        else:
            sc = L.Scales(L.SCALES_F32, self._scales.data_ptr(), None, None)
        return L.Weight(self._codes.data_ptr(), sc, self._d_in, self._d_out,
                        L.LAYOUT_STRIPED if self._striped else L.LAYOUT_ROW_MAJOR)

    def _forward(self, x: torch.Tensor, lora: Optional[LoraAdapter], out_dtype: Optional[torch.dtype]):
        _require_cuda(x, "x")
        if x.shape[-1] != self._d_in:
            raise ValueError(f"x has last dim {x.shape[-1]}, the layer takes {self._d_in}")
        rows = x.numel() // self._d_in
        out_dtype = out_dtype or x.dtype
        y = torch.empty(*x.shape[:-1], self._d_out, dtype=out_dtype, device=x.device)
        w = self.weight_struct()
        lo = lora.struct() if lora is not None else None
        L.check(L.lib().unifur_nf4_linear_forward(
            x.data_ptr(), _dtype_code(x.dtype), rows, ctypes.byref(w),
            self.bias.data_ptr() if self.bias is not None else None,
            ctypes.byref(lo) if lo is not None else None,
            y.data_ptr(), _dtype_code(out_dtype), None, 0, _stream()))
        return y

    def forward(self, x: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """src/qwennet.rs:238-241: y = x W (+ bias) over the last dim of x."""
        return self._forward(x, None, out_dtype)

    __call__ = forward

    def _backward(self, dy: torch.Tensor, lora: Optional[LoraAdapter], x: Optional[torch.Tensor], want_dx: bool,
                  dx_dtype: Optional[torch.dtype], workspace: Optional[torch.Tensor] = None):
        _require_cuda(dy, "dy")
        if dy.shape[-1] != self._d_out:
            raise ValueError(f"dy has last dim {dy.shape[-1]}, the layer gives {self._d_out}")
        rows = dy.numel() // self._d_out
        if lora is not None:
            if x is None:
                raise ValueError("the adapter gradients need the forward input x")
            _require_cuda(x, "x")
            if x.shape[-1] != self._d_in or x.numel() // self._d_in != rows:
                raise ValueError("x must be [..., d_input] with the rows of dy")
        dx = None
        if want_dx:
            dx = torch.empty(*dy.shape[:-1], self._d_in, dtype=dx_dtype or dy.dtype, device=dy.device)
        ga = gb = None
        lo = None
        if lora is not None:
            lo = lora.struct()
            ga = torch.empty(self._d_in, lora.rank(), dtype=torch.float32, device=dy.device)
            gb = torch.empty(lora.rank(), self._d_out, dtype=torch.float32, device=dy.device)
        w = self.weight_struct()
        L.check(L.lib().unifur_nf4_linear_backward(
            dy.data_ptr(), _dtype_code(dy.dtype), rows, ctypes.byref(w),
            ctypes.byref(lo) if lo is not None else None,
            x.data_ptr() if x is not None else None, _dtype_code(x.dtype) if x is not None else L.F32,
            dx.data_ptr() if dx is not None else None, _dtype_code(dx.dtype) if dx is not None else L.F32,
            ga.data_ptr() if ga is not None else None, gb.data_ptr() if gb is not None else None,
            workspace.data_ptr() if workspace is not None else None,
            workspace.numel() * workspace.element_size() if workspace is not None else 0, _stream()))
        return dx, ga, gb

    def backward(self, dy: torch.Tensor, dx_dtype: Optional[torch.dtype] = None,
                 workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
        """dL/dx = dy W^T for dy = dL/dy: the gradient burn's autodiff
        takes through the detached dequantized weight (src/qwennet.rs:238-241
        under src/qwentrain.rs:421-470); the frozen weight gets none.
        workspace: optional device buffer (the library's per-stream cache
        when None); one below the default size, down to
        unifur_nf4_linear_backward_min_workspace_size, takes the fused dX
        kernel."""
        return self._backward(dy, None, None, True, dx_dtype, workspace)[0]


# weights per launch sequence of the library's grouped quantize pass
_QGROUP = 48


def quantize_linears(weights) -> list:
    """Nf4Linear.from_values on every (values, d_input, d_output) of
    ``weights`` -- the quantize pass of QwenTrunk::to_nf4
    (src/qwennet.rs:1185-1269) -- in one grouped pass (three launches per 48
    weights): values are f32 [d_input * d_output] row-major on the device,
    d_output % 64 == 0; the layers come back striped and double quantized,
    their buffers slices of one allocation each for codes, scales and scales
    of scales."""
    return _quantize_grouped(weights, checkpoint=False)


def quantize_checkpoint_linears(tensors) -> list:
    """The same pass from checkpoint linears as they lie: each tensor is the
    PyTorch-order [out, in] weight (f32, bf16 or f16, on the device), as
    qwen_linear (src/qwennet.rs:1687-1726) receives it, transposed to
    [in, out] on the fly (transpose2d, src/qwennet.rs:1375-1390) inside the
    grouped quantize kernel; out % 64 == 0.  Byte for byte what
    quantize_linears gives for the transposed f32 copies."""
    ws = []
    for t in tensors:
        shape = t.shape
        if len(shape) != 2:
            raise ValueError(f"tensor of shape {tuple(shape)} is not rank-2")
        ws.append((t, shape[1], shape[0]))
    return _quantize_grouped(ws, checkpoint=True)


def _quantize_grouped(weights, checkpoint: bool) -> list:
    n = len(weights)
    if n == 0:
        return []
    dims = [(int(di), int(do)) for (_, di, do) in weights]
    for (di, do) in dims:
        if di <= 0 or do % 64 != 0 or do <= 0:
            raise ValueError("quantize_linears needs d_input > 0 and d_output a positive multiple of 64")
    dev = weights[0][0].device
    # back to back: code sizes are multiples of 32 bytes (d_output % 64 == 0),
    # so every slice stays 8-byte aligned; u8 scales need no alignment.  The
    # buffers are allocated from the shapes alone, then the values are checked
    # and launched a group at a time (the library's grouped pass takes 48
    # weights per launch sequence), so that the first kernels start while the
    # later groups are still being checked; each layer makes its views of
    # the three buffers when first used.
    c_sizes = [di * do // 2 for (di, do) in dims]
    s_sizes = [di * do // 64 for (di, do) in dims]
    codes = torch.empty(sum(c_sizes), dtype=torch.uint8, device=dev)
    dq = torch.empty(sum(s_sizes), dtype=torch.uint8, device=dev)
    sos = torch.empty(n, dtype=torch.float32, device=dev)
    c_off = list(itertools.accumulate(c_sizes, initial=0))
    s_off = list(itertools.accumulate(s_sizes, initial=0))
    cb, db, sb = codes.data_ptr(), dq.data_ptr(), sos.data_ptr()
    keep = []  # contiguous copies made here stay alive until their launch is queued
    stream = _stream()
    lib = L.lib()
    src_dtype = None
    for g0 in range(0, n, _QGROUP):
        idx = range(g0, min(n, g0 + _QGROUP))
        v_ptrs = []
        for i in idx:
            v = weights[i][0]
            di, do = dims[i]
            if not v.is_cuda:
                raise ValueError("values must be a CUDA (HIP) device tensor")
            if checkpoint:
                dt = v.dtype
                if dt is not src_dtype:
                    if dt is not torch.float32 and dt is not torch.bfloat16 and dt is not torch.float16:
                        raise ValueError(f"checkpoint linears must be f32, bf16 or f16 [{do}, {di}]")
                    if src_dtype is not None:
                        raise ValueError("checkpoint linears of one call share a dtype")
                    src_dtype = dt
                if v.shape != (do, di):
                    raise ValueError(f"checkpoint linears must be f32, bf16 or f16 [{do}, {di}]")
                if not v.is_contiguous():
                    v = v.contiguous()
                    keep.append(v)
            else:
                if v.dtype != torch.float32 or v.numel() != di * do:
                    raise ValueError(f"values must be float32 with {di} x {do} elements")
                if not v.is_contiguous() or v.data_ptr() % 16 != 0:
                    v = v.contiguous().clone()
                    keep.append(v)
            v_ptrs.append(v.data_ptr())
        m = len(v_ptrs)
        P = ctypes.c_void_p * m
        U = ctypes.c_uint64 * m
        tail = (U(*[dims[i][0] for i in idx]), U(*[dims[i][1] for i in idx]), m,
                P(*[cb + c_off[i] for i in idx]), P(*[db + s_off[i] for i in idx]), P(*[sb + 4 * i for i in idx]),
                None, 0, stream)
        if checkpoint:
            L.check(lib.unifur_nf4_quantize_checkpoint_linears(P(*v_ptrs), _src_dtype_code(src_dtype), *tail))
        else:
            L.check(lib.unifur_nf4_quantize_linears(P(*v_ptrs), *tail))
    group = (codes, c_off, dq, s_off, sos)
    return [Nf4Linear._from_group(group, i, di, do) for i, (di, do) in enumerate(dims)]


def forward_shared_input(x: torch.Tensor, layers, out_dtype: Optional[torch.dtype] = None) -> list:
    """y_i = layers[i].forward(x) for up to three Nf4Linears sharing d_input,
    as QwenFullAttention applies q_proj, k_proj and v_proj to one hidden state
    (src/qwennet.rs:927-956): decode-sized batches over striped weights of one
    scale kind take a single launch that reads x once for all of them."""
    _require_cuda(x, "x")
    layers = list(layers)
    if not 1 <= len(layers) <= 3:
        raise ValueError("forward_shared_input takes one to three layers")
    d_in = layers[0].d_input()
    if any(l.d_input() != d_in for l in layers) or x.shape[-1] != d_in:
        raise ValueError("the layers must share d_input with x's last dim")
    rows = x.numel() // d_in
    out_dtype = out_dtype or x.dtype
    ys = [torch.empty(*x.shape[:-1], l.d_output(), dtype=out_dtype, device=x.device) for l in layers]
    ws = (L.Weight * len(layers))(*[l.weight_struct() for l in layers])
    biases = (ctypes.c_void_p * len(layers))(*[l.bias.data_ptr() if l.bias is not None else None for l in layers])
    outs = (ctypes.c_void_p * len(layers))(*[y.data_ptr() for y in ys])
    L.check(L.lib().unifur_nf4_linear_forward_multi(x.data_ptr(), _dtype_code(x.dtype), rows, ws, biases, outs,
                                                    _dtype_code(out_dtype), len(layers), None, 0, _stream()))
    return ys


class QloraLinear:
    """Frozen packed NF4 base plus a LoRA adapter (src/qwennet.rs:311-345):
    forward(x) = base(x) + (x a) b * scaling, fused into one launch chain."""

    def __init__(self, base: Nf4Linear, adapter: LoraAdapter):
        if adapter.in_features() != base.d_input() or adapter.out_features() != base.d_output():
            raise ValueError("adapter shape does not match the base layer")
        self.base = base
        self.adapter = adapter

    def forward(self, x: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        return self.base._forward(x, self.adapter, out_dtype)

    __call__ = forward

    def backward(self, x: torch.Tensor, dy: torch.Tensor, want_dx: bool = True,
                 dx_dtype: Optional[torch.dtype] = None, workspace: Optional[torch.Tensor] = None):
        """Vector-Jacobian products of forward for dy = dL/dy: returns
        (dx, grad_a, grad_b), dx = dy W^T + ((dy s) B^T) A^T,
        grad_b = (x A)^T (dy s), grad_a = x^T ((dy s) B^T) (f32); dx is None
        when want_dx is False.  The base weight is frozen.  workspace as in
        Nf4Linear.backward."""
        return self.base._backward(dy, self.adapter, x, want_dx, dx_dtype, workspace)


class QwenMlp:
    """down(silu(gate(x)) * up(x)) with three bias-free NF4 linears
    (src/qwennet.rs:786-820)."""

    def __init__(self, gate_proj: Nf4Linear, up_proj: Nf4Linear, down_proj: Nf4Linear):
        hidden, inter = gate_proj.d_input(), gate_proj.d_output()
        if (up_proj.d_input(), up_proj.d_output()) != (hidden, inter) or \
                (down_proj.d_input(), down_proj.d_output()) != (inter, hidden):
            raise ValueError("gate/up must be [hidden, intermediate] and down [intermediate, hidden]")
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj

    def forward(self, x: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        _require_cuda(x, "x")
        hidden = self.gate_proj.d_input()
        if x.shape[-1] != hidden:
            raise ValueError(f"x has last dim {x.shape[-1]}, the block takes {hidden}")
        rows = x.numel() // hidden
        out_dtype = out_dtype or x.dtype
        y = torch.empty(*x.shape[:-1], hidden, dtype=out_dtype, device=x.device)
        g, u, d = (self.gate_proj.weight_struct(), self.up_proj.weight_struct(), self.down_proj.weight_struct())
        L.check(L.lib().unifur_nf4_swiglu_forward(
            x.data_ptr(), _dtype_code(x.dtype), rows, ctypes.byref(g), ctypes.byref(u), ctypes.byref(d),
            y.data_ptr(), _dtype_code(out_dtype), None, 0, _stream()))
        return y

    __call__ = forward


# ------------------------------------------------------- dense f32 linears --

class DenseLinear:
    """A plain linear with an f32-resident weight [d_input, d_output] and
    optional bias: Burn's ``Linear`` as the reference uses it for the F32 arm
    of ``QwenLinear`` (src/qwennet.rs:293-355) and for the output of
    ``QLoRALinear::merged`` (src/quantize.rs:716-726).  Forward runs the
    library's f32 GEMM (``unifur_nf4_dense_linear_forward``)."""

    def __init__(self, weight: torch.Tensor, bias: Optional[torch.Tensor] = None):
        _require_cuda(weight, "weight")
        if weight.dtype != torch.float32 or weight.dim() != 2:
            raise ValueError("weight must be float32 [d_input, d_output]")
        if bias is not None:
            _require_cuda(bias, "bias")
            if bias.dtype != torch.float32 or bias.numel() != weight.shape[1]:
                raise ValueError("bias must be float32 [d_output]")
        self.weight = weight
        self.bias = bias

    def d_input(self) -> int:
        return self.weight.shape[0]

    def d_output(self) -> int:
        return self.weight.shape[1]

    def _forward(self, x: torch.Tensor, lora: Optional["LoraAdapter"], out_dtype: Optional[torch.dtype]):
        _require_cuda(x, "x")
        d_in, d_out = self.weight.shape
        if x.shape[-1] != d_in:
            raise ValueError(f"x has last dim {x.shape[-1]}, the layer takes {d_in}")
        rows = x.numel() // d_in
        out_dtype = out_dtype or x.dtype
        y = torch.empty(*x.shape[:-1], d_out, dtype=out_dtype, device=x.device)
        lo = lora.struct() if lora is not None else None
        L.check(L.lib().unifur_nf4_dense_linear_forward(
            x.data_ptr(), _dtype_code(x.dtype), rows, self.weight.data_ptr(), d_in, d_out,
            self.bias.data_ptr() if self.bias is not None else None,
            ctypes.byref(lo) if lo is not None else None, y.data_ptr(), _dtype_code(out_dtype), None, 0,
            _stream()))
        return y

    def forward(self, x: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        return self._forward(x, None, out_dtype)

    __call__ = forward


def _linear_init(d_in: int, d_out: int, generator: Optional[torch.Generator], device) -> tuple:
    """Burn's default ``LinearConfig`` initialisation (Kaiming-uniform with
    gain 1/sqrt(3), i.e. U(-1/sqrt(d_in), 1/sqrt(d_in)) for weight and bias)."""
    bound = 1.0 / math.sqrt(max(d_in, 1))
    w = (torch.rand(d_in, d_out, generator=generator) * 2 - 1) * bound
    b = (torch.rand(d_out, generator=generator) * 2 - 1) * bound
    return w.to(device), b.to(device)


def _quantize_dequantize_flat(values: torch.Tensor, double_quantization: bool) -> torch.Tensor:
    q = PackedNf4Tensor.quantize(values.contiguous().view(-1))
    if double_quantization:
        q = q.with_double_quantization()
    return q.dequantize().view(values.shape)


class QLoRALinear:
    """The simulated QLoRA layer of src/quantize.rs:637-727: an f32-stored
    base whose weight holds NF4-grid values (``quantize_dequantize_tensor``),
    an f32 bias, and a LoRA adapter.  ``resident_bits`` reports what the base
    would occupy packed; ``merged`` folds ``scaling * A B`` into the weight.
    (The NF4-resident form is ``QloraLinear`` above.)"""

    def __init__(self, base: DenseLinear, adapter: LoraAdapter, quantized_values: int, double_quantized: bool):
        self.base = base
        self._adapter = adapter
        self.quantized_values = int(quantized_values)
        self.double_quantized = bool(double_quantized)

    @staticmethod
    def from_linear(base: DenseLinear, config: LoraConfig, double_quantization: bool, device="cuda",
                    generator: Optional[torch.Generator] = None) -> "QLoRALinear":
        """src/quantize.rs:653-676: quantize the base weight to NF4 (values
        kept dequantized in f32), keep the bias, attach a fresh adapter."""
        n = base.weight.numel()
        q = _quantize_dequantize_flat(base.weight, double_quantization)
        return QLoRALinear(DenseLinear(q, base.bias), LoraAdapter.new(config, device, generator), n,
                           double_quantization)

    @staticmethod
    def new(in_features: int, out_features: int, config: LoraConfig, double_quantization: bool, device="cuda",
            generator: Optional[torch.Generator] = None) -> "QLoRALinear":
        """src/quantize.rs:679-690: a fresh biased linear, quantized and adapted."""
        w, b = _linear_init(in_features, out_features, generator, device)
        return QLoRALinear.from_linear(DenseLinear(w, b), config, double_quantization, device, generator)

    def forward(self, x: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """base(x) + adapter(x) (src/quantize.rs:692-694), one fused launch chain."""
        return self.base._forward(x, self._adapter, out_dtype)

    __call__ = forward

    def adapter(self) -> LoraAdapter:
        return self._adapter

    def resident_bits(self) -> tuple:
        """src/quantize.rs:700-713: (packed NF4 bits, f32 bits) of the base weight."""
        blocks = float((self.quantized_values + BLOCK_SIZE - 1) // BLOCK_SIZE)
        scale_bits = 8.0 * blocks + 32.0 if self.double_quantized else 32.0 * blocks
        return 4.0 * self.quantized_values + scale_bits, 32.0 * self.quantized_values

    def merged(self) -> DenseLinear:
        """src/quantize.rs:716-726: a plain linear with W + scaling * (A B)."""
        out = torch.empty_like(self.base.weight)
        d_in, d_out = self.base.weight.shape
        lo = self._adapter.struct()
        L.check(L.lib().unifur_nf4_lora_merge(self.base.weight.data_ptr(), d_in, d_out, ctypes.byref(lo),
                                              out.data_ptr(), _stream()))
        return DenseLinear(out, self.base.bias)


# ---------------------------------------------------- module-level quantize --

class Nf4Quantizer:
    """src/quantize.rs:418-493: quantize every weight-shaped parameter of a
    module to the NF4 grid in place.  Parameters of rank < 2, with fewer than
    BLOCK_SIZE values, or under a module whose path contains a ``skip``
    needle are left alone.  A module is a mapping of dotted parameter names
    to device tensors; the module path of ``a.b.weight`` is ``[a, b]``."""

    def __init__(self, double_quantization: bool):
        self.double_quantization = bool(double_quantization)
        self.skip: list[str] = []
        self.quantized_values = 0
        self.skipped_params = 0

    def skipping(self, name: str) -> "Nf4Quantizer":
        self.skip.append(name)
        return self

    def is_skipped(self, path: list) -> bool:
        return any(needle in part for needle in self.skip for part in path)

    def should_quantize(self, name: str, shape) -> bool:
        """The map_float decision (src/quantize.rs:469-475), host-side."""
        numel = 1
        for d in shape:
            numel *= int(d)
        path = name.split(".")[:-1]
        return len(shape) >= 2 and numel >= BLOCK_SIZE and not self.is_skipped(path)

    def map_float(self, name: str, param: torch.Tensor) -> torch.Tensor:
        if not self.should_quantize(name, tuple(param.shape)):
            self.skipped_params += 1
            return param
        if param.dtype != torch.float32:
            raise ValueError(f"{name}: the quantizer takes float32 parameters")
        self.quantized_values += param.numel()
        return _quantize_dequantize_flat(param, self.double_quantization)


def quantize_module(module: dict, double_quantization: bool, skip=()) -> tuple:
    """src/quantize.rs:498-511: (quantized module, values quantized)."""
    mapper = Nf4Quantizer(double_quantization)
    for s in skip:
        mapper.skipping(s)
    out = {name: mapper.map_float(name, p) for name, p in module.items()}
    return out, mapper.quantized_values
