"""ctypes binding of libunifur_nf4.so (the C ABI in include/unifur_nf4.h).

Loading fails loudly when the library has not been built: there is no
fallback implementation of any entry point.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libunifur_nf4.so")

OK = 0
ERR_INVALID = -1
ERR_HIP = -2
ERR_WORKSPACE = -3

F32 = 0
BF16 = 1
F16 = 2  # checkpoint sources only

IDS_I32 = 0
IDS_I64 = 1

SCALES_F32 = 0
SCALES_DOUBLE_QUANTIZED = 1

LAYOUT_ROW_MAJOR = 0
LAYOUT_STRIPED = 1

BLOCK_SIZE = 64


class Scales(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("absmax", ctypes.c_void_p),
        ("dq_codes", ctypes.c_void_p),
        ("scale_of_scales", ctypes.c_void_p),
    ]


class Weight(ctypes.Structure):
    _fields_ = [
        ("packed", ctypes.c_void_p),
        ("scales", Scales),
        ("d_in", ctypes.c_uint64),
        ("d_out", ctypes.c_uint64),
        ("layout", ctypes.c_int32),
    ]


class DecoderLayer(ctypes.Structure):
    _fields_ = [
        ("q", Weight),
        ("k", Weight),
        ("v", Weight),
        ("o", Weight),
        ("gate", Weight),
        ("up", Weight),
        ("down", Weight),
        ("input_norm", ctypes.c_void_p),
        ("post_norm", ctypes.c_void_p),
        ("eps", ctypes.c_float),
    ]


class Lora(ctypes.Structure):
    _fields_ = [
        ("a", ctypes.c_void_p),
        ("b", ctypes.c_void_p),
        ("rank", ctypes.c_uint32),
        ("scaling", ctypes.c_float),
    ]


# Every symbol include/unifur_nf4.h declares, with its ctypes signature.
_P = ctypes.c_void_p
_U64 = ctypes.c_uint64
_I = ctypes.c_int
SIGNATURES = {
    "unifur_nf4_last_error": (ctypes.c_char_p, []),
    "unifur_nf4_levels": (_I, [ctypes.POINTER(ctypes.c_float)]),
    "unifur_nf4_num_blocks": (_U64, [_U64]),
    "unifur_nf4_packed_bytes": (_U64, [_U64]),
    "unifur_nf4_estimated_resident_bytes": (_U64, [_U64, _I]),
    "unifur_nf4_bits_per_value": (ctypes.c_double, [_U64, _I]),
    "unifur_nf4_simulated_bits_per_value": (ctypes.c_double, [_U64, _I]),
    "unifur_nf4_quantize": (_I, [_P, _U64, _P, _P, _P]),
    "unifur_nf4_double_quantize": (_I, [_P, _U64, _P, _P, _P]),
    "unifur_nf4_dequantize": (_I, [_P, ctypes.POINTER(Scales), _U64, _P, _I, _P]),
    "unifur_nf4_unpack_codes": (_I, [_P, _U64, _P, _P]),
    "unifur_nf4_pack_codes": (_I, [_P, _U64, _P, _P]),
    "unifur_nf4_quantize_transposed": (_I, [_P, _I, _U64, _U64, _P, _P, _P]),
    "unifur_nf4_quantize_linears_workspace_size": (_U64, [_P, _P, ctypes.c_uint32]),
    "unifur_nf4_quantize_linears": (_I, [_P, _P, _P, ctypes.c_uint32, _P, _P, _P, _P, _U64, _P]),
    "unifur_nf4_transpose_checkpoint": (_I, [_P, _I, _U64, _U64, _P, _P]),
    "unifur_nf4_quantize_checkpoint_linears": (_I, [_P, _I, _P, _P, ctypes.c_uint32, _P, _P, _P, _P, _U64, _P]),
    "unifur_nf4_dense_linear_workspace_size": (_U64, [_U64, ctypes.c_uint32]),
    "unifur_nf4_dense_linear_forward": (_I, [_P, _I, _U64, _P, _U64, _U64, _P, ctypes.POINTER(Lora), _P, _I, _P,
                                             _U64, _P]),
    "unifur_nf4_lora_merge": (_I, [_P, _U64, _U64, ctypes.POINTER(Lora), _P, _P]),
    "unifur_nf4_stripe_weight": (_I, [ctypes.POINTER(Weight), _P, _P, _P]),
    "unifur_nf4_unstripe_weight": (_I, [ctypes.POINTER(Weight), _P, _P, _P]),
    "unifur_nf4_embedding_forward": (_I, [_P, ctypes.POINTER(Scales), _U64, _U64, _P, _I, _U64, _P, _I, _P]),
    "unifur_nf4_linear_workspace_size": (_U64, [_U64, _U64, _U64, _I, ctypes.c_uint32]),
    "unifur_nf4_linear_multi_workspace_size": (_U64, [_U64, _U64, _P, ctypes.c_uint32, _I]),
    "unifur_nf4_linear_forward_multi": (_I, [_P, _I, _U64, ctypes.POINTER(Weight), _P, _P, _I,
                                             ctypes.c_uint32, _P, _U64, _P]),
    "unifur_nf4_linear_backward_workspace_size": (_U64, [_U64, _U64, _U64, _I, ctypes.c_uint32]),
    "unifur_nf4_linear_backward_min_workspace_size": (_U64, [_U64, _U64, _U64, _I, ctypes.c_uint32, _I]),
    "unifur_nf4_linear_backward": (_I, [_P, _I, _U64, ctypes.POINTER(Weight), ctypes.POINTER(Lora), _P, _I,
                                        _P, _I, _P, _P, _P, _U64, _P]),
    "unifur_nf4_linear_min_workspace_size": (_U64, [_U64, _U64, _U64, _I, ctypes.c_uint32]),
    "unifur_nf4_linear_forward": (_I, [_P, _I, _U64, ctypes.POINTER(Weight), _P, ctypes.POINTER(Lora), _P, _I,
                                       _P, _U64, _P]),
    "unifur_nf4_linear_forward_noalloc": (_I, [_P, _I, _U64, ctypes.POINTER(Weight), _P, ctypes.POINTER(Lora), _P,
                                               _I, _P]),
    "unifur_nf4_qlora_forward": (_I, [_P, _I, _U64, ctypes.POINTER(Weight), ctypes.POINTER(Lora), _P, _I, _P,
                                      _U64, _P]),
    "unifur_nf4_decoder_attn_in_workspace_size": (_U64, [_U64, ctypes.POINTER(DecoderLayer), _I]),
    "unifur_nf4_decoder_attn_in": (_I, [_P, _I, _U64, ctypes.POINTER(DecoderLayer), _P, _P, _P, _P, _U64, _P]),
    "unifur_nf4_decoder_attn_out_mlp_workspace_size": (_U64, [_U64, ctypes.POINTER(DecoderLayer), _I]),
    "unifur_nf4_decoder_attn_out_mlp": (_I, [_P, _P, _I, _U64, ctypes.POINTER(DecoderLayer), _P, _P, _U64, _P]),
    "unifur_nf4_swiglu_workspace_size": (_U64, [_U64, _U64, _U64, _I]),
    "unifur_nf4_swiglu_min_workspace_size": (_U64, [_U64, _U64, _U64, _I]),
    "unifur_nf4_swiglu_forward": (_I, [_P, _I, _U64, ctypes.POINTER(Weight), ctypes.POINTER(Weight),
                                       ctypes.POINTER(Weight), _P, _I, _P, _U64, _P]),
}

_lib = None


class Nf4Error(RuntimeError):
    """A non-zero status from the library, with its message."""

    def __init__(self, status: int, message: str):
        super().__init__(f"unifur_nf4 status {status}: {message}")
        self.status = status


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m unifur_amd.build` (hipcc, gfx950). "
                "There is no fallback implementation.")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != OK:
        msg = lib().unifur_nf4_last_error().decode(errors="replace")
        raise Nf4Error(status, msg)
