"""GPU parity of the simulated NF4 form and of the rank-2 round trip.

* ``Nf4Tensor`` (src/quantize.rs:79-201) holds one code per byte: its codes,
  absmax, double-quantized codes and scale of scales, dequantized f32 and
  bits per value are compared bit for bit with the oracle's restatement of
  Nf4Tensor::quantize / with_double_quantization / dequantize
  (oracle/nf4_oracle.c nf4o_quantize_sim, nf4o_double_quantize,
  nf4o_dequantize_sim), which the oracle tests pin against the reference's
  own known answers.
* ``quantize_dequantize_tensor`` (src/quantize.rs:402-416) runs
  Nf4Tensor::quantize (+ with_double_quantization) and dequantize on the
  flat row-major buffer: at config 1 (4096 x 4096 ~ N(0, 0.02^2), seed
  0x4E463457 + 1) and at ragged shapes the result equals the oracle's chain
  bit for bit, with plain and with double-quantized scales.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from unifur_amd import quantize as Q

pytestmark = pytest.mark.gpu


def u32(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def check_simulated(values: np.ndarray, oracle, device, tag: str):
    codes, absmax = oracle.quantize_sim(values)
    q, sos = oracle.double_quantize(absmax)
    n = values.size
    t = Q.Nf4Tensor.quantize(torch.from_numpy(np.ascontiguousarray(values, np.float32)).to(device))
    assert t.len() == n and len(t) == n and t.is_empty() == (n == 0)
    assert t.num_blocks() == oracle.num_blocks(n)
    assert not t.is_double_quantized()
    assert np.array_equal(t.codes.cpu().numpy(), codes), f"{tag}: codes differ"
    assert np.array_equal(u32(t.absmax.cpu().numpy()), u32(absmax)), f"{tag}: absmax differs"
    assert np.array_equal(u32(t.dequantize().cpu().numpy()), u32(oracle.dequantize_sim(codes, absmax))), \
        f"{tag}: dequantized f32 differs"
    assert t.bits_per_value() == oracle.bits_per_value_sim(n, False)
    d = t.with_double_quantization()
    assert d.is_double_quantized()
    assert np.array_equal(d.dq_codes.cpu().numpy(), q), f"{tag}: DQ codes differ"
    assert u32(d.scale_of_scales.cpu().numpy())[0] == u32(np.float32(sos))[()], f"{tag}: scale of scales differs"
    want = oracle.dequantize_sim(codes, None, q, sos)
    assert np.array_equal(u32(d.dequantize().cpu().numpy()), u32(want)), f"{tag}: DQ dequantized f32 differs"
    assert d.bits_per_value() == oracle.bits_per_value_sim(n, True)
    # recomputed from the kept absmax: a second application changes nothing
    dd = d.with_double_quantization()
    assert torch.equal(dd.dq_codes, d.dq_codes) and torch.equal(dd.scale_of_scales, d.scale_of_scales)
    # the packed form of the same codes is the packed codec's bytes
    packed, _ = oracle.quantize_packed(values)
    assert np.array_equal(t.packed().codes.cpu().numpy(), packed), f"{tag}: packing differs"


@pytest.mark.parametrize("n", [1, 63, 64, 69, 384, 1000, 4097])
def test_simulated_form_ragged(device, oracle, n):
    v = oracle.fill_normal(7000 + n, 0.02, n).copy()
    if n >= 128:
        v[64:128] = 0.0  # a zero block: code 7, absmax 0 (src/quantize.rs:106-110)
    check_simulated(v, oracle, device, f"n={n}")


def test_simulated_form_fixtures(device, oracle, fixtures):
    # the golden vectors include NaN / Inf / -0 / subnormal blocks
    names, z = fixtures
    for nm in names:
        check_simulated(z[nm + ".values"], oracle, device, nm)
        # and the fixture's own one-code-per-byte vector (a second, numpy restatement)
        t = Q.Nf4Tensor.quantize(torch.from_numpy(np.ascontiguousarray(z[nm + ".values"], np.float32)).to(device))
        assert np.array_equal(t.codes.cpu().numpy(), z[nm + ".codes"]), nm


def test_simulated_form_config1(device, oracle):
    v = oracle.fill_normal(0x4E463457 + 1, 0.02, 4096 * 4096)
    check_simulated(v, oracle, device, "config 1")


def test_simulated_form_empty_and_code_conversions(device, oracle):
    t = Q.Nf4Tensor.quantize(torch.zeros(0, dtype=torch.float32, device=device))
    assert t.is_empty() and t.num_blocks() == 0 and t.bits_per_value() == 0.0
    assert t.dequantize().numel() == 0
    # unpack -> pack is the identity on packed bytes, pack takes codes mod 16
    from unifur_amd import _lib as L
    st = torch.cuda.current_stream().cuda_stream
    for n in (1, 2, 7, 64, 1001):
        b = torch.randint(0, 256, ((n + 1) // 2,), dtype=torch.uint8, device=device)
        if n % 2:
            b[-1] &= 0x0F  # an odd length's last byte has a zero high nibble
        c = torch.empty(n, dtype=torch.uint8, device=device)
        L.check(L.lib().unifur_nf4_unpack_codes(b.data_ptr(), n, c.data_ptr(), st))
        cn = c.cpu().numpy()
        bn = b.cpu().numpy()
        assert np.array_equal(cn[0::2], bn & 15) and np.array_equal(cn[1::2], (bn >> 4)[: n // 2])
        back = torch.empty_like(b)
        L.check(L.lib().unifur_nf4_pack_codes((c + 16).data_ptr(), n, back.data_ptr(), st))
        assert torch.equal(back, b)
    assert L.lib().unifur_nf4_unpack_codes(None, 4, None, st) == L.ERR_INVALID
    assert L.lib().unifur_nf4_pack_codes(None, 0, None, st) == L.OK


@pytest.mark.parametrize("shape", [(4096, 4096), (37, 41), (1, 64), (3, 1000)])
@pytest.mark.parametrize("dq", [False, True])
def test_quantize_dequantize_tensor_matches_oracle(device, oracle, shape, dq):
    r, c = shape
    seed = 0x4E463457 + 1 if shape == (4096, 4096) else 7100 + r * c
    v = oracle.fill_normal(seed, 0.02, r * c)
    codes, absmax = oracle.quantize_sim(v)
    if dq:
        q, sos = oracle.double_quantize(absmax)
        want = oracle.dequantize_sim(codes, None, q, sos)
    else:
        want = oracle.dequantize_sim(codes, absmax)
    t = torch.from_numpy(v).to(device).view(r, c)
    got = Q.quantize_dequantize_tensor(t, dq)
    assert got.shape == (r, c) and got.dtype == torch.float32
    assert np.array_equal(u32(got.cpu().numpy().reshape(-1)), u32(want))
    # a non-contiguous view is taken in its row-major order, as burn's into_data
    tt = torch.from_numpy(v.reshape(r, c).T.copy()).to(device).t()
    assert np.array_equal(u32(Q.quantize_dequantize_tensor(tt, dq).cpu().numpy().reshape(-1)), u32(want))
    with pytest.raises(ValueError):
        Q.quantize_dequantize_tensor(t.view(-1), dq)
