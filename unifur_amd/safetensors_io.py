"""Checkpoint shards to the device, for the load path that ends in packed NF4.

Host side of src/import.rs (the safetensors reader) and of the WeightStore
reads in src/qwennet.rs:1538-1565: a shard's header is parsed and checked
without touching its weights (``open_index``, src/import.rs:134-227), and a
tensor is read by its byte range only (``read_tensor_f32``,
src/import.rs:243-280).  Where the reference then decodes the bytes to f32 on
the CPU, transposes and quantizes, here the raw F32 / BF16 / F16 bytes go to
the device as they are and the library decodes, transposes and quantizes
them in one pass (``quantize.quantize_checkpoint_linears``), so the on-disk
format turns into the resident striped, double-quantized NF4 form without an
f32 copy on either side.

Errors raise ``ValueError`` naming the file and tensor, as the reference's
``ensure!`` / ``bail!`` do.
"""
from __future__ import annotations

import enum
import json
import os
import struct
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

# The header cap of the format (src/import.rs:36-37): a corrupt length word
# is refused before anything is allocated for it.
MAX_HEADER_BYTES = 100_000_000


class ImportDtype(enum.Enum):
    """The element types the reader takes (src/import.rs:39-66)."""
    F32 = "F32"
    F16 = "F16"
    BF16 = "BF16"

    @staticmethod
    def parse(s: str) -> "ImportDtype":
        try:
            return ImportDtype(s)
        except ValueError:
            raise ValueError(f"unsupported safetensors dtype {s!r}: only F32/F16/BF16 decode "
                             "(no silent casts)") from None

    def size(self) -> int:
        return 4 if self is ImportDtype.F32 else 2

    def torch_dtype(self) -> torch.dtype:
        return {ImportDtype.F32: torch.float32, ImportDtype.F16: torch.float16,
                ImportDtype.BF16: torch.bfloat16}[self]


@dataclass
class TensorMeta:
    """A tensor's place in a shard: [start, end) within the data section
    (src/import.rs:68-88)."""
    name: str
    dtype: ImportDtype
    shape: list
    start: int
    end: int

    def byte_len(self) -> int:
        n = 1
        for d in self.shape:
            n *= int(d)
        return n * self.dtype.size()


class SafetensorsIndex:
    """Header-only view of a shard (src/import.rs:97-131)."""

    def __init__(self, tensors: list, data_start: int, file_len: int):
        self.tensors = tensors
        self.data_start = data_start
        self._file_len = file_len
        self._by_name = {t.name: t for t in tensors}

    def __len__(self) -> int:
        return len(self.tensors)

    def len(self) -> int:
        return len(self.tensors)

    def is_empty(self) -> bool:
        return not self.tensors

    def find(self, name: str) -> Optional[TensorMeta]:
        return self._by_name.get(name)

    def file_len(self) -> int:
        return self._file_len

    def covered_bytes(self) -> int:
        return sum(max(0, t.end - t.start) for t in self.tensors)


def open_index(path) -> SafetensorsIndex:
    """Parse and check the header of ``path`` (src/import.rs:134-227): the
    length word within the cap and the file, every entry's dtype, offsets in
    order and in the file, each range as long as shape x dtype, and the
    ranges tiling the data section exactly (no overlap, hole or trailing
    bytes)."""
    path = os.fspath(path)
    file_len = os.path.getsize(path)
    with open(path, "rb") as f:
        word = f.read(8)
        if len(word) != 8:
            raise ValueError(f"{path}: too short for a header length")
        header_len = struct.unpack("<Q", word)[0]
        if header_len > MAX_HEADER_BYTES:
            raise ValueError(f"header of {path} claims {header_len} bytes, over the format's "
                             f"{MAX_HEADER_BYTES}-byte limit")
        data_start = 8 + header_len
        if data_start > file_len:
            raise ValueError(f"header ({data_start} bytes) runs past end of {path} ({file_len} bytes)")
        raw = f.read(header_len)
    try:
        header = json.loads(raw)
    except (json.JSONDecodeError, UnicodeDecodeError) as e:
        raise ValueError(f"{path}: header JSON does not parse: {e}") from None
    if not isinstance(header, dict):
        raise ValueError(f"{path}: header JSON is not an object")
    tensors = []
    for name in sorted(header):
        if name == "__metadata__":  # sidecar metadata, not a tensor
            continue
        entry = header[name]
        try:
            dtype_s = str(entry["dtype"])
            shape = [int(d) for d in entry["shape"]]
            start, end = (int(o) for o in entry["data_offsets"])
        except (KeyError, TypeError, ValueError):
            raise ValueError(f"{path}: header entry for tensor {name!r} does not parse") from None
        dtype = ImportDtype.parse(dtype_s)
        if start > end:
            raise ValueError(f"tensor {name!r} has inverted offsets [{start}, {end})")
        if data_start + end > file_len:
            raise ValueError(f"tensor {name!r} range [{start}, {end}) runs past end of file")
        meta = TensorMeta(name, dtype, shape, start, end)
        if end - start != meta.byte_len():
            raise ValueError(f"tensor {name!r} range length {end - start} != shape x dtype {meta.byte_len()}")
        tensors.append(meta)
    if not tensors:
        raise ValueError(f"no tensors in {path}")
    cursor = 0
    for t in sorted(tensors, key=lambda t: (t.start, t.end)):
        if t.start != cursor:
            raise ValueError(f"tensor {t.name!r} starts at {t.start}, but the previous range ends at {cursor} "
                             f"(overlapping or non-contiguous offsets in {path})")
        cursor = t.end
    if data_start + cursor != file_len:
        raise ValueError(f"tensor data ends at byte {data_start + cursor} of {path}, which is {file_len} bytes long")
    return SafetensorsIndex(tensors, data_start, file_len)


def _non_finite_mask_bits(raw: np.ndarray, dtype: ImportDtype) -> bool:
    """Whether any element of the raw little-endian bytes is Inf or NaN, from
    the exponent bits alone (all ones), without decoding the values."""
    if dtype is ImportDtype.F32:
        u = raw.view("<u4")
        return bool(np.any((u & np.uint32(0x7F800000)) == np.uint32(0x7F800000)))
    u = raw.view("<u2")
    e = np.uint16(0x7F80) if dtype is ImportDtype.BF16 else np.uint16(0x7C00)
    return bool(np.any((u & e) == e))


def read_tensor_device(path, index: SafetensorsIndex, name: str, device="cuda",
                       require_finite: bool = False) -> torch.Tensor:
    """One named tensor's bytes, read by their range only (as
    read_tensor_f32, src/import.rs:243-280) and placed on the device in the
    file's element type and shape -- undecoded: the library's checkpoint
    kernels decode F32 / BF16 / F16 exactly.  ``require_finite`` refuses Inf
    and NaN as the WeightStore's checked reads do (src/qwennet.rs:1540-1560)."""
    meta = index.find(name)
    if meta is None:
        raise ValueError(f"tensor {name!r} not in {os.fspath(path)}")
    n = meta.end - meta.start
    with open(os.fspath(path), "rb") as f:
        f.seek(index.data_start + meta.start)
        raw = f.read(n)
    if len(raw) != n:
        raise ValueError(f"read {len(raw)} of {n} bytes for tensor {name!r}")
    host = np.frombuffer(raw, dtype=np.uint8)
    if require_finite and _non_finite_mask_bits(host, meta.dtype):
        raise ValueError(f"tensor {name!r} contains non-finite values")
    t = torch.from_numpy(host.copy()).to(device)
    return t.view(meta.dtype.torch_dtype()).reshape(meta.shape)


def load_checkpoint_linears(path, index: SafetensorsIndex, names, device="cuda", require_finite: bool = True):
    """qwen_linear's NF4 arm (src/qwennet.rs:1687-1726) over named rank-2
    [out, in] linears of one shard: each tensor is read by its range, the
    ones with out % 64 == 0 go through one grouped checkpoint pass per
    element type (decode, transpose, quantize and double quantize on the
    device, straight into the striped resident form), the others through
    ``qwennet.qwen_linear``.  Returns (QwenLinear, resident bytes) per name,
    in order."""
    from . import quantize as Q
    from . import qwennet as QN

    tensors = []
    for name in names:
        t = read_tensor_device(path, index, name, device, require_finite)
        if t.dim() != 2:
            raise ValueError(f"tensor {name!r} is not rank-2")
        tensors.append(t)
    out = [None] * len(tensors)
    by_dtype = {}
    for i, t in enumerate(tensors):
        if t.shape[0] % 64 == 0:
            by_dtype.setdefault(t.dtype, []).append(i)
        else:
            out[i] = QN.qwen_linear(t, QN.WeightStore.NF4)
    for idx in by_dtype.values():
        lins = Q.quantize_checkpoint_linears([tensors[i] for i in idx])
        for i, lin in zip(idx, lins):
            out[i] = (QN.QwenLinear(QN.QwenLinear.NF4, lin), lin.resident_bytes())
    return out
