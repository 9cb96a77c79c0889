"""GPU checks of the column-striped device layout of a linear weight.

The striped layout (include/unifur_nf4.h, UNIFUR_NF4_LAYOUT_STRIPED) is this
build's own resident form, not a reference format: its contract is that it
is a pure byte permutation of the reference's packed codes and scales.  So:
  * the bytes equal an independent numpy statement of the permutation;
  * unstriping gives back the reference's bytes bit for bit;
  * every linear path computes the same function on either layout (the
    numerics are pinned in test_gpu_linear / test_gpu_gemm).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from unifur_amd import _lib as L
from unifur_amd import quantize as Q

pytestmark = pytest.mark.gpu


def striped_codes_np(packed: np.ndarray, k: int, n: int) -> np.ndarray:
    """striped[(s*K + k)*8 + j] = row_major[k*N/2 + s*8 + j]."""
    return packed.reshape(k, n // 16, 8).transpose(1, 0, 2).reshape(-1)


def striped_scales_np(scales: np.ndarray, k: int, n: int) -> np.ndarray:
    """striped[b*K + k] = row_major[k*N/64 + b]."""
    return scales.reshape(k, n // 64).T.reshape(-1)


@pytest.mark.parametrize("dq", [True, False])
@pytest.mark.parametrize("shape", [(1, 64), (3, 64), (65, 128), (4096, 11008), (11008, 4096), (896, 128),
                                   (130, 4096 + 64)])
def test_stripe_is_the_documented_permutation_and_round_trips(device, oracle, shape, dq):
    k, n = shape
    v = oracle.fill_normal(9000 + k + n, 0.02, k * n)
    packed, absmax = oracle.quantize_packed(v)
    p = Q.PackedNf4Tensor.quantize(torch.from_numpy(v).to(device))
    if dq:
        p = p.with_double_quantization()
        q, _ = oracle.double_quantize(absmax)
    lin = Q.Nf4Linear.from_packed(p, k, n, striped=True)
    assert lin.is_striped()
    torch.cuda.synchronize()
    assert np.array_equal(lin._codes.cpu().numpy(), striped_codes_np(packed, k, n))
    sc = lin._scales.cpu().numpy()
    if dq:
        assert np.array_equal(sc, striped_scales_np(q, k, n))
    else:
        assert np.array_equal(sc.view(np.uint32), striped_scales_np(absmax, k, n).view(np.uint32))
    back = lin.packed()
    assert np.array_equal(back.codes.cpu().numpy(), packed)
    if dq:
        assert np.array_equal(back.dq_codes.cpu().numpy(), q)
    else:
        assert np.array_equal(back.absmax.cpu().numpy().view(np.uint32), absmax.view(np.uint32))
    # and the dequantized weight of the layer is the reference's, bit for bit
    deq = oracle.dequantize_packed(packed, k * n, None if dq else absmax, q if dq else None,
                                   oracle.double_quantize(absmax)[1] if dq else None)
    assert np.array_equal(lin.dequantized_weight().cpu().numpy().reshape(-1).view(np.uint32), deq.view(np.uint32))


def test_striped_layout_rejects_bad_shapes_and_alignment(device):
    p = Q.PackedNf4Tensor.quantize(torch.randn(100 * 96, device=device))
    with pytest.raises(ValueError):
        Q.Nf4Linear.from_packed(p, 100, 96, striped=True)  # 96 % 64 != 0
    lin = Q.Nf4Linear.from_packed(p, 100, 96)
    assert not lin.is_striped()
    # a striped weight with misaligned codes is refused by the library
    w = Q.Nf4Linear.from_packed(Q.PackedNf4Tensor.quantize(torch.randn(64 * 64, device=device)), 64, 64)
    ws = w.weight_struct()
    ws.packed += 4
    x = torch.randn(1, 64, device=device)
    y = torch.empty(1, 64, device=device)
    st = L.lib().unifur_nf4_linear_forward(x.data_ptr(), L.F32, 1, ctypes.byref(ws), None, None, y.data_ptr(), L.F32,
                                           None, 0, torch.cuda.current_stream().cuda_stream)
    assert st == L.ERR_INVALID and b"8-byte" in L.lib().unifur_nf4_last_error()
