"""GPU parity of the NF4 codec: libunifur_nf4.so vs the CPU oracle, bit-exact.

Codes, packed bytes, absmax, double-quantized codes and scale of scales, and
dequantized f32 are compared bit for bit (src/quantize.rs semantics); bf16
dequantization must equal the oracle's f32 result rounded to nearest even.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from unifur_amd import quantize as Q

pytestmark = pytest.mark.gpu


def u32(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def gpu_roundtrip(values: np.ndarray, device):
    x = torch.from_numpy(np.ascontiguousarray(values, np.float32)).to(device)
    p = Q.PackedNf4Tensor.quantize(x)
    d = p.with_double_quantization()
    out = {
        "packed": p.codes.cpu().numpy(),
        "absmax": p.absmax.cpu().numpy(),
        "dq_codes": d.dq_codes.cpu().numpy(),
        "dq_sos": d.scale_of_scales.cpu().numpy(),
        "deq_plain": p.dequantize().cpu().numpy(),
        "deq_dq": d.dequantize().cpu().numpy(),
        "deq_plain_bf16": p.dequantize(torch.bfloat16).float().cpu().numpy(),
        "deq_dq_bf16": d.dequantize(torch.bfloat16).float().cpu().numpy(),
    }
    torch.cuda.synchronize()
    return out


def assert_matches_oracle(values: np.ndarray, got: dict, oracle, tag: str):
    packed, absmax = oracle.quantize_packed(values)
    q, sos = oracle.double_quantize(absmax)
    n = values.size
    deq = oracle.dequantize_packed(packed, n, absmax)
    deq_dq = oracle.dequantize_packed(packed, n, None, q, sos)
    assert np.array_equal(got["packed"], packed), f"{tag}: packed bytes differ"
    assert np.array_equal(u32(got["absmax"]), u32(absmax)), f"{tag}: absmax differs"
    assert np.array_equal(got["dq_codes"], q), f"{tag}: DQ codes differ"
    assert u32(got["dq_sos"])[0] == u32(np.float32(sos))[()], f"{tag}: scale of scales differs"
    assert np.array_equal(u32(got["deq_plain"]), u32(deq)), f"{tag}: dequantized f32 differs"
    assert np.array_equal(u32(got["deq_dq"]), u32(deq_dq)), f"{tag}: DQ dequantized f32 differs"
    fin = np.isfinite(deq)
    assert np.array_equal(u32(got["deq_plain_bf16"])[fin], u32(oracle.round_bf16(deq))[fin]), f"{tag}: bf16"
    fin = np.isfinite(deq_dq)
    assert np.array_equal(u32(got["deq_dq_bf16"])[fin], u32(oracle.round_bf16(deq_dq))[fin]), f"{tag}: bf16 DQ"


def test_golden_fixtures_bit_exact(device, fixtures, oracle):
    names, z = fixtures
    for nm in names:
        v = z[f"{nm}.values"]
        print(f"fixture {nm} n={v.size}", flush=True)
        got = gpu_roundtrip(v, device)
        for key in ("packed", "absmax", "dq_codes", "deq_plain", "deq_dq"):
            expect = z[f"{nm}.{key}"]
            g = got[key]
            if g.dtype == np.float32:
                assert np.array_equal(u32(g), u32(expect)), f"{nm}.{key}"
            else:
                assert np.array_equal(g, expect), f"{nm}.{key}"
        assert u32(got["dq_sos"])[0] == u32(z[f"{nm}.dq_sos"])[0], nm
        assert_matches_oracle(v, got, oracle, nm)


def test_config1_round_trip_4096x4096_bit_exact(device, oracle):
    # one f32 weight 4096 x 4096 ~ N(0, 0.02^2), block 64
    v = oracle.fill_normal(0x4E463457 + 0, 0.02, 4096 * 4096)
    print("config1 4096x4096", flush=True)
    assert_matches_oracle(v, gpu_roundtrip(v, device), oracle, "config1")


@pytest.mark.parametrize("n", [1, 2, 3, 63, 64, 65, 127, 1023, 1024, 1025, 2047, 4097, 100003])
def test_ragged_lengths_bit_exact(device, oracle, n):
    v = oracle.fill_normal(1000 + n, 1.3, n)
    v[:: max(1, n // 7)] = 0.0
    assert_matches_oracle(v, gpu_roundtrip(v, device), oracle, f"n={n}")


def test_misaligned_buffers_take_the_scalar_path(device, oracle):
    n = 5000
    v = oracle.fill_normal(77, 0.5, n)
    base = torch.zeros(n + 8, dtype=torch.float32, device=device)
    base[1:1 + n] = torch.from_numpy(v).to(device)
    x = base[1:1 + n]  # 4-byte offset: not 16-byte aligned
    codes_buf = torch.zeros((n + 1) // 2 + 8, dtype=torch.uint8, device=device)
    codes = codes_buf[1:1 + (n + 1) // 2]  # odd byte offset
    absmax = torch.zeros((n + 63) // 64, dtype=torch.float32, device=device)
    from unifur_amd import _lib as L
    L.check(L.lib().unifur_nf4_quantize(x.data_ptr(), n, codes.data_ptr(), absmax.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream))
    packed, am = oracle.quantize_packed(v)
    assert np.array_equal(codes.cpu().numpy(), packed)
    assert np.array_equal(u32(absmax.cpu().numpy()), u32(am))
    p = Q.PackedNf4Tensor(codes, n, absmax=absmax)
    out_buf = torch.zeros(n + 8, dtype=torch.float32, device=device)
    out = out_buf[1:1 + n]
    s = p.scales_struct()
    import ctypes
    L.check(L.lib().unifur_nf4_dequantize(codes.data_ptr(), ctypes.byref(s), n, out.data_ptr(), L.F32,
                                          torch.cuda.current_stream().cuda_stream))
    assert np.array_equal(u32(out.cpu().numpy()), u32(oracle.dequantize_packed(packed, n, am)))


def test_empty_tensor_and_idempotent_double_quantization(device):
    p = Q.PackedNf4Tensor.quantize(torch.zeros(0, dtype=torch.float32, device=device))
    assert p.is_empty() and p.num_blocks() == 0 and p.dequantize().numel() == 0
    x = torch.randn(640, device=device)
    d1 = Q.PackedNf4Tensor.quantize(x).with_double_quantization()
    d2 = d1.with_double_quantization()
    assert d2 is d1 and d1.is_double_quantized()
    assert d1.resident_bytes() == 320 + 10 + 4  # src/quantize.rs:793-822
    assert Q.PackedNf4Tensor.quantize(x).resident_bytes() == 320 + 40


def test_every_f32_in_unit_interval_gets_the_scan_code(device):
    """All 2.13e9 f32 values u in [-1, 1]: with absmax == 1 the code must be
    #{t : u >= T_t}, the reference's scan (thresholds pinned on the CPU)."""
    from tests.test_oracle import THRESHOLD_BITS
    T = torch.tensor(np.array(THRESHOLD_BITS, np.uint32).view(np.float32), device=device)
    per = 63
    chunk = per * (1 << 20)  # values per launch
    stream = torch.cuda.current_stream().cuda_stream
    from unifur_amd import _lib as L
    nblk = chunk // per
    buf = torch.empty(nblk, 64, dtype=torch.float32, device=device)
    codes = torch.empty(nblk * 32, dtype=torch.uint8, device=device)
    absmax = torch.empty(nblk, dtype=torch.float32, device=device)
    checked = 0
    for sign in (0, 0x80000000):
        start, stop = 0, 0x3F800000 + 1  # +0 .. 1.0 (or -0 .. -1.0)
        lo = start
        while lo < stop:
            hi = min(lo + chunk, stop)
            m = hi - lo
            pat = torch.arange(lo, hi, dtype=torch.int64, device=device) | sign
            u = pat.to(torch.int32).view(torch.float32) if sign == 0 else \
                (pat - (1 << 32)).to(torch.int32).view(torch.float32)
            buf.zero_()
            buf[:, 0] = 1.0
            flat = buf[:, 1:]
            full = torch.zeros(nblk * per, dtype=torch.float32, device=device)
            full[:m] = u
            flat.copy_(full.view(nblk, per))
            L.check(L.lib().unifur_nf4_quantize(buf.data_ptr(), nblk * 64, codes.data_ptr(), absmax.data_ptr(),
                                                stream))
            lo_n = (codes & 0xF).to(torch.int64)
            hi_n = (codes >> 4).to(torch.int64)
            c = torch.stack([lo_n, hi_n], dim=1).view(nblk, 64)[:, 1:].reshape(-1)[:m]
            expect = torch.searchsorted(T, u, right=True)
            bad = torch.nonzero(c != expect)
            assert bad.numel() == 0, f"u bits {hex(int(pat[bad[0, 0]]))}: got {int(c[bad[0,0]])}"
            checked += m
            lo = hi
        print(f"sign {hex(sign)} done, {checked} values", flush=True)
    assert checked == 2 * (0x3F800000 + 1)


THRESHOLD_BITS = [
    0xbf591cd8, 0xbf1c5270, 0xbeeb847f, 0xbeadea76, 0xbe703cec, 0xbe0d38bb, 0xbd3a7870, 0x3d22fb00,
    0x3df64863, 0x3e5067e1, 0x3e9582d5, 0x3ec753fa, 0x3f006d04, 0x3f248db0, 0x3f5c89da,
]


def near_threshold_blocks(seed: int, nblocks: int) -> np.ndarray:
    """Blocks whose values sit within a few ulp of threshold * absmax, for
    absmax over the whole normal range and its ends (subnormal, 2^126 and
    beyond, zero, with inf and NaN entries): the values the kernel's fast
    reciprocal classification must hand to the exact division."""
    rng = np.random.default_rng(seed)
    T = np.array(THRESHOLD_BITS, np.uint32).view(np.float32)
    exps = rng.integers(-130, 128, nblocks)
    m = (rng.uniform(1.0, 2.0, nblocks) * np.exp2(exps.astype(np.float64))).astype(np.float32)
    m[:8] = np.array([0.0, 1e-45, 1e-40, 1.1754944e-38, 8.507059e37, 1.7e38, 3.4028235e38, 1.0], np.float32)
    m[~np.isfinite(m)] = np.float32(3.0e38)
    blocks = np.zeros((nblocks, 64), np.float32)
    blocks[:, 0] = m
    with np.errstate(over="ignore", invalid="ignore"):
        for j in range(1, 64):
            t = T[rng.integers(0, 15, nblocks)]
            v = (t.astype(np.float64) * m.astype(np.float64)).astype(np.float32)
            k = rng.integers(-6, 7, nblocks)
            for step in range(6):  # nudge by up to 6 ulp either way
                v = np.where(k > step, np.nextafter(v, np.float32(np.inf)), v)
                v = np.where(-k > step, np.nextafter(v, np.float32(-np.inf)), v)
            blocks[:, j] = np.where(np.abs(v) <= m, v, np.float32(0.0))
    blocks[8, 5] = np.inf
    blocks[9, 7] = -np.inf
    blocks[10, 3] = np.nan
    blocks[11] = 0.0
    return blocks.ravel()


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_values_next_to_thresholds_at_every_scale_bit_exact(device, oracle, seed):
    v = near_threshold_blocks(seed, 4096)
    x = torch.from_numpy(v).to(device)
    p = Q.PackedNf4Tensor.quantize(x)
    packed, absmax = oracle.quantize_packed(v)
    got = p.codes.cpu().numpy()
    bad = np.nonzero(got != packed)[0]
    assert bad.size == 0, f"seed {seed}: {bad.size} code bytes differ, first at byte {bad[:5]}"
    assert np.array_equal(u32(p.absmax.cpu().numpy()), u32(absmax))
