"""The checkpoint shard reader (unifur_amd/safetensors_io.py) on the CPU:
the header checks and ranged reads of src/import.rs, restated as its own
tests restate them (src/import.rs:402-571: known encodings, three dtypes,
corrupt headers, ranges that must tile the data section, an oversized
length word), plus the finite check of the WeightStore's reads
(src/qwennet.rs:1540-1560).  Tensors are placed on the CPU here; the GPU
test of the whole load path is tests/test_gpu_safetensors_load.py."""
from __future__ import annotations

import json
import struct

import numpy as np
import pytest
import torch

from unifur_amd import safetensors_io as S


def write_shard(tmp_path, tensors, name="shard.safetensors", trailing=b""):
    """A shard from (name, dtype, shape, raw bytes), offsets in order."""
    header, data, off = {}, b"", 0
    for n, dt, shape, raw in tensors:
        header[n] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        off += len(raw)
        data += raw
    return write_raw(tmp_path, header, data + trailing, name)


def write_raw(tmp_path, header, data, name="raw.safetensors"):
    h = json.dumps(header).encode()
    p = tmp_path / name
    p.write_bytes(struct.pack("<Q", len(h)) + h + data)
    return p


def f32le(values):
    return np.asarray(values, "<f4").tobytes()


def u16le(values):
    return np.asarray(values, "<u2").tobytes()


THREE = [("w.f32", "F32", [2, 2], f32le([1.0, 2.0, 3.0, 4.0])),
         ("w.bf16", "BF16", [3], u16le([0x3F80, 0xC000, 0x7F80])),
         ("w.f16", "F16", [2], u16le([0x3C00, 0x0001]))]


def test_header_indexes_without_touching_weights(tmp_path):
    idx = S.open_index(write_shard(tmp_path, THREE))
    assert len(idx) == 3 and not idx.is_empty()
    m = idx.find("w.bf16")
    assert m.shape == [3] and m.dtype is S.ImportDtype.BF16 and m.byte_len() == 6
    assert idx.find("missing") is None
    assert idx.covered_bytes() == 16 + 6 + 4


def test_ranged_reads_give_the_files_elements(tmp_path, oracle):
    p = write_shard(tmp_path, THREE)
    idx = S.open_index(p)
    f = S.read_tensor_device(p, idx, "w.f32", device="cpu")
    assert f.dtype == torch.float32 and f.shape == (2, 2) and f.flatten().tolist() == [1.0, 2.0, 3.0, 4.0]
    b = S.read_tensor_device(p, idx, "w.bf16", device="cpu")
    assert b.dtype == torch.bfloat16 and b.view(torch.int16).numpy().view(np.uint16).tolist() == [0x3F80, 0xC000,
                                                                                                  0x7F80]
    # the values the reference decodes from them (src/import.rs:453-470)
    assert oracle.decode_checkpoint(b.view(torch.int16).numpy().view(np.uint16), "bf16").tolist() == [
        1.0, -2.0, float("inf")]
    h = S.read_tensor_device(p, idx, "w.f16", device="cpu")
    assert h.dtype == torch.float16
    assert oracle.decode_checkpoint(h.view(torch.int16).numpy().view(np.uint16), "f16").tolist() == [1.0, 2.0 ** -24]
    with pytest.raises(ValueError):
        S.read_tensor_device(p, idx, "nope", device="cpu")


def test_corrupt_headers_are_refused(tmp_path):
    with pytest.raises(ValueError, match="unsupported safetensors dtype"):
        S.open_index(write_shard(tmp_path, [("w.q", "Q4_K", [4], b"\0" * 4)], "q.st"))
    with pytest.raises(ValueError, match="shape x dtype"):
        S.open_index(write_shard(tmp_path, [("w.bad", "F32", [2], f32le([1.0, 2.0, 3.0]))], "bad.st"))
    full = write_shard(tmp_path, [("w.ok", "F32", [2], f32le([1.0, 2.0]))], "ok.st")
    cut = tmp_path / "cut.st"
    cut.write_bytes(full.read_bytes()[:-3])
    with pytest.raises(ValueError):
        S.open_index(cut)
    with pytest.raises(ValueError, match="no tensors"):
        S.open_index(write_raw(tmp_path, {"__metadata__": {"format": "pt"}}, b"", "meta.st"))
    with pytest.raises(ValueError, match="inverted"):
        S.open_index(write_raw(tmp_path, {"a": {"dtype": "F32", "shape": [0], "data_offsets": [4, 0]}}, b"\0" * 4,
                               "inv.st"))


def test_ranges_must_tile_the_data_section(tmp_path):
    data = f32le([1.0, 2.0, 3.0, 4.0])
    ok = write_raw(tmp_path, {"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
                              "b": {"dtype": "F32", "shape": [2], "data_offsets": [8, 16]},
                              "__metadata__": {"format": "pt"}}, data, "ok.st")
    assert S.open_index(ok).len() == 2
    cases = {
        "overlap": {"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 12]},
                    "b": {"dtype": "F32", "shape": [2], "data_offsets": [8, 16]}},
        "hole": {"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]},
                 "b": {"dtype": "F32", "shape": [2], "data_offsets": [8, 16]}},
        "trailing": {"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 12]}},
    }
    for name, header in cases.items():
        with pytest.raises(ValueError):
            S.open_index(write_raw(tmp_path, header, data, name + ".st"))


def test_oversized_header_length_is_refused_before_reading_it(tmp_path):
    p = tmp_path / "huge.st"
    p.write_bytes(struct.pack("<Q", S.MAX_HEADER_BYTES + 1))
    with pytest.raises(ValueError, match="limit"):
        S.open_index(p)


@pytest.mark.parametrize("dtype,bad", [("F32", f32le([1.0, float("nan")])), ("F32", f32le([float("-inf"), 0.0])),
                                       ("BF16", u16le([0x3F80, 0x7FC0])), ("F16", u16le([0x7C00, 0x3C00])),
                                       ("F16", u16le([0x3C00, 0xFE01]))])
def test_checked_reads_refuse_non_finite_values(tmp_path, dtype, bad):
    p = write_shard(tmp_path, [("w", dtype, [2], bad)])
    idx = S.open_index(p)
    with pytest.raises(ValueError, match="non-finite"):
        S.read_tensor_device(p, idx, "w", device="cpu", require_finite=True)
    assert S.read_tensor_device(p, idx, "w", device="cpu").numel() == 2  # unchecked reads pass them through


def test_finite_values_pass_the_check(tmp_path):
    # the largest finite value of each type is not mistaken for Inf
    p = write_shard(tmp_path, [("a", "F32", [1], f32le([3.4028235e38])), ("b", "BF16", [1], u16le([0x7F7F])),
                               ("c", "F16", [1], u16le([0x7BFF]))])
    idx = S.open_index(p)
    for n in ("a", "b", "c"):
        assert S.read_tensor_device(p, idx, n, device="cpu", require_finite=True).numel() == 1
