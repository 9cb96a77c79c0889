"""unifur_amd -- MI355X-native NF4 quantized-linear path of unifur.

The compute lives in ``libunifur_nf4.so`` (hand-written gfx950 HIP kernels
behind the C ABI of ``include/unifur_nf4.h``); ``unifur_amd.quantize``
mirrors the reference's Rust API over it.  Build with
``python -m unifur_amd.build``.
"""
from ._lib import LIB_PATH, Nf4Error, lib  # noqa: F401

__all__ = ["LIB_PATH", "Nf4Error", "lib"]
