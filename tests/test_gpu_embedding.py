"""GPU parity of the NF4 embedding gather (Nf4Embedding::forward,
src/qwennet.rs:244-291): rows of the dequantized table, bit-exact.

The oracle dequantizes the whole table exactly as the reference does
(src/quantize.rs:355-366, pinned by the codec tests) and gathers with numpy;
the library dequantizes only the gathered rows.  f32 rows must match bit for
bit, bf16 rows must be the round-to-nearest-even of those f32 values.  Shapes
include d_model values that are not multiples of 64 or of 8, where a row
starts inside a block and the scalar path serves it.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from unifur_amd import _lib as L
from unifur_amd import quantize as Q
from unifur_amd import qwennet as QN

pytestmark = pytest.mark.gpu


def bf16_rne(f: np.ndarray) -> np.ndarray:
    u = f.astype(np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(f)
    r[nan] = 0x7FC0
    return r


def table(oracle, n_emb, d, seed, dq=True):
    v = oracle.fill_normal(seed, 0.02, n_emb * d)
    packed, absmax = oracle.quantize_packed(v)
    if dq:
        q, sos = oracle.double_quantize(absmax)
        deq = oracle.dequantize_packed(packed, v.size, None, q, sos)
    else:
        deq = oracle.dequantize_packed(packed, v.size, absmax, None, None)
    return v, deq.reshape(n_emb, d)


@pytest.mark.parametrize("shape", [(1000, 64), (257, 100), (50, 8), (151, 896), (3, 7), (64, 1)])
@pytest.mark.parametrize("ids_dtype", [torch.int64, torch.int32])
def test_rows_bit_exact(device, oracle, shape, ids_dtype):
    n_emb, d = shape
    v, deq = table(oracle, n_emb, d, 0xE0 + n_emb + d)
    emb = QN.Nf4Embedding.from_values(torch.from_numpy(v).to(device), n_emb, d)
    rng = np.random.default_rng(n_emb * 7 + d)
    ids = rng.integers(0, n_emb, size=(3, 17))
    ids[0, :3] = [0, n_emb - 1, 0]  # first and last rows, a repeat
    got = emb.forward(torch.from_numpy(ids).to(ids_dtype).to(device))
    assert got.shape == (3, 17, d) and got.dtype == torch.float32
    want = deq[ids]
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))
    gb = emb.forward(torch.from_numpy(ids).to(ids_dtype).to(device), dtype=torch.bfloat16)
    assert np.array_equal(gb.cpu().view(torch.int16).numpy().view(np.uint16), bf16_rne(want))
    # the whole-table path of the reference gives the same rows
    full = emb.dequantized_weight().cpu().numpy()
    assert np.array_equal(full.view(np.uint32), deq.view(np.uint32))


def test_plain_scales_and_misaligned_output(device, oracle):
    # f32 absmax scales (no double quantization) through the ABI, and an
    # output that is 4- but not 16-byte aligned (scalar path)
    n_emb, d = 300, 64
    v, deq = table(oracle, n_emb, d, 0xE7, dq=False)
    p = Q.PackedNf4Tensor.quantize(torch.from_numpy(v).to(device))
    ids = torch.tensor([5, 299, 0, 5, 123], dtype=torch.int64, device=device)
    buf = torch.zeros(ids.numel() * d + 1, dtype=torch.float32, device=device)
    out = buf[1:]
    assert out.data_ptr() % 16 != 0
    s = p.scales_struct()
    L.check(L.lib().unifur_nf4_embedding_forward(p.codes.data_ptr(), ctypes.byref(s), n_emb, d, ids.data_ptr(),
                                                 L.IDS_I64, ids.numel(), out.data_ptr(), L.F32,
                                                 torch.cuda.current_stream().cuda_stream))
    want = deq[ids.cpu().numpy()]
    assert np.array_equal(out.view(ids.numel(), d).cpu().numpy().view(np.uint32), want.view(np.uint32))
    assert float(buf[0]) == 0.0  # nothing written before the output


def test_out_of_range_ids_give_nan_rows(device, oracle):
    n_emb, d = 40, 72
    v, deq = table(oracle, n_emb, d, 0xE9)
    emb = QN.Nf4Embedding.from_values(torch.from_numpy(v).to(device), n_emb, d)
    ids = torch.tensor([3, -1, n_emb, 39, 2**40], dtype=torch.int64, device=device)
    got = emb.forward(ids).cpu().numpy()
    assert np.isnan(got[[1, 2, 4]]).all()
    assert np.array_equal(got[[0, 3]].view(np.uint32), deq[[3, 39]].view(np.uint32))
    got32 = emb.forward(torch.tensor([-5, 7], dtype=torch.int32, device=device)).cpu().numpy()
    assert np.isnan(got32[0]).all() and np.array_equal(got32[1].view(np.uint32), deq[7].view(np.uint32))


def test_empty_and_argument_errors(device, oracle):
    n_emb, d = 10, 64
    v, _ = table(oracle, n_emb, d, 0xEA)
    emb = QN.Nf4Embedding.from_values(torch.from_numpy(v).to(device), n_emb, d)
    assert emb.forward(torch.empty(0, 4, dtype=torch.int64, device=device)).shape == (0, 4, d)
    assert emb.resident_bytes() == n_emb * d // 2 + n_emb * d // 64 + 4  # packed + u8 scales + sos
    s = emb.packed.scales_struct()
    ids = torch.zeros(2, dtype=torch.int64, device=device)
    out = torch.empty(2, d, device=device)
    lib = L.lib()
    st = torch.cuda.current_stream().cuda_stream
    assert lib.unifur_nf4_embedding_forward(emb.packed.codes.data_ptr(), ctypes.byref(s), n_emb, d, ids.data_ptr(),
                                            7, 2, out.data_ptr(), L.F32, st) == L.ERR_INVALID
    assert lib.unifur_nf4_embedding_forward(emb.packed.codes.data_ptr(), ctypes.byref(s), n_emb, d, None,
                                            L.IDS_I64, 2, out.data_ptr(), L.F32, st) == L.ERR_INVALID
    with pytest.raises(ValueError):
        emb.forward(torch.zeros(2, dtype=torch.float32, device=device))
