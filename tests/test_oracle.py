"""Pin the CPU oracle (oracle/nf4_oracle.c) before trusting it.

Each check is chosen so that a plausible restatement mistake fails it:
the reference's own known-answer tests (file:line cited per test), the
published codebook, the exact real-arithmetic nearest level, an
independently derived threshold table, closed forms of double quantization,
and bit-exact agreement with fixtures written by an independent numpy
restatement (tests/golden/make_golden.py).
"""
from __future__ import annotations

import json
import os
import struct

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# Exact decision thresholds of the reference's nearest_level_code, found by
# enumerating every f32 in [-1, 1] against the literal scan (an independent
# derivation, not this oracle): scan(u) = #{t : u >= T_t}.
THRESHOLD_BITS = [
    0xbf591cd8, 0xbf1c5270, 0xbeeb847f, 0xbeadea76, 0xbe703cec, 0xbe0d38bb, 0xbd3a7870, 0x3d22fb00,
    0x3df64863, 0x3e5067e1, 0x3e9582d5, 0x3ec753fa, 0x3f006d04, 0x3f248db0, 0x3f5c89da,
]


def f32_from_bits(b: int) -> float:
    return struct.unpack("<f", struct.pack("<I", b))[0]


def bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def scan_codes(oracle, u: np.ndarray) -> np.ndarray:
    """Codes of arbitrary u in [-1, 1] through the oracle quantizer: each
    64-block starts with 1.0, so absmax == 1 and v / absmax == v exactly."""
    u = np.asarray(u, np.float32)
    n = u.size
    per = 63
    nb = (n + per - 1) // per
    buf = np.zeros((nb, 64), np.float32)
    buf[:, 0] = 1.0
    flat = np.zeros(nb * per, np.float32)
    flat[:n] = u
    buf[:, 1:] = flat.reshape(nb, per)
    codes, absmax = oracle.quantize_sim(buf.ravel())
    assert np.all(absmax == 1.0)
    return codes.reshape(nb, 64)[:, 1:].ravel()[:n]


# ------------------------------------------------------------------ codebook --

def test_levels_are_the_published_nf4_codebook(oracle):
    # src/quantize.rs:839-866
    with open(os.path.join(GOLDEN, "nf4_codebook.json")) as f:
        published = json.load(f)["published_f64"]
    expect = np.array(published, np.float64).astype(np.float32)
    assert np.array_equal(bits(oracle.levels()), bits(expect))


def test_levels_are_sorted_symmetric_and_contain_zero(oracle):
    # src/quantize.rs:824-837
    lv = oracle.levels()
    assert np.all(np.diff(lv) > 0)
    assert lv[0] == -1.0 and lv[-1] == 1.0 and 0.0 in lv and lv.size == 16


# --------------------------------------------------------------- level scan --

def test_scan_equals_exact_nearest_level_away_from_midpoints(oracle):
    # Mathematics fixes the nearest level for any u not within an ulp of a
    # midpoint; the f32 distance compare may differ only there.
    rng = np.random.default_rng(7)
    u = np.concatenate([rng.uniform(-1, 1, 400_000), rng.normal(0, 0.1, 100_000).clip(-1, 1),
                        oracle.levels()]).astype(np.float32)
    got = scan_codes(oracle, u)
    lv = oracle.levels().astype(np.float64)
    d = np.abs(u.astype(np.float64)[:, None] - lv[None, :])
    exact = np.argmin(d, axis=1)
    mids = (lv[1:] + lv[:-1]) / 2
    near_mid = np.min(np.abs(u.astype(np.float64)[:, None] - mids[None, :]), axis=1) <= \
        2 * np.spacing(np.abs(u).astype(np.float32)).astype(np.float64) + 1e-12
    assert np.array_equal(got[~near_mid], exact[~near_mid])
    assert np.all(np.abs(got[near_mid].astype(int) - exact[near_mid]) <= 1)


def test_scan_thresholds_match_the_enumerated_table(oracle):
    # Bisect over f32 bit patterns for the first u with code >= t.
    def key(f):
        b = struct.unpack("<I", struct.pack("<f", f))[0]
        return b if b < 0x80000000 else -(b & 0x7FFFFFFF)

    def from_key(k):
        return f32_from_bits(k) if k >= 0 else f32_from_bits((-k) | 0x80000000)

    lo0, hi0 = key(-1.0), key(1.0)
    lv = oracle.levels()
    for t in range(1, 16):
        lo, hi = lo0, hi0
        while lo < hi:
            mid = (lo + hi) // 2
            if oracle.nearest_level_code(from_key(mid)) >= t:
                hi = mid
            else:
                lo = mid + 1
        T = from_key(lo)
        assert struct.unpack("<I", struct.pack("<f", T))[0] == THRESHOLD_BITS[t - 1], t
        # and within one ulp of the f32 midpoint of the adjacent levels
        midpoint = np.float32((np.float32(lv[t - 1]) + np.float32(lv[t])) / np.float32(2))
        assert abs(float(T) - float(midpoint)) <= float(np.spacing(np.float32(abs(midpoint))))


def test_scan_is_monotone_with_15_changes_and_nan_is_zero(oracle):
    u = np.linspace(-1, 1, 200_001, dtype=np.float32)
    c = scan_codes(oracle, u).astype(int)
    assert np.all(np.diff(c) >= 0) and np.count_nonzero(np.diff(c)) == 15
    T = np.array([f32_from_bits(b) for b in THRESHOLD_BITS], np.float32)
    assert np.array_equal(c, np.searchsorted(T, u, side="right"))
    assert oracle.nearest_level_code(float("nan")) == 0


# ------------------------------------------------- reference known answers --

def test_exact_values_survive_a_roundtrip(oracle):
    # src/quantize.rs:868-879
    values = (oracle.levels() * np.float32(0.75)).astype(np.float32)
    codes, absmax = oracle.quantize_sim(values)
    restored = oracle.dequantize_sim(codes, absmax)
    assert np.all(np.abs(restored - values) < 1e-6)


def test_absmax_endpoints_are_exact(oracle):
    # src/quantize.rs:881-894
    v = np.full(64, 0.01, np.float32)
    v[7], v[9] = -4.25, 2.0
    codes, absmax = oracle.quantize_sim(v)
    assert oracle.dequantize_sim(codes, absmax)[7] == np.float32(-4.25)


def test_quantization_error_bounded_and_beats_uniform(oracle):
    # src/quantize.rs:896-955, src/verify.rs:1045-1066
    lv = oracle.levels()
    max_gap = np.max(np.diff(lv))
    v = np.random.default_rng(3).standard_normal(64 * 32).astype(np.float32)
    codes, absmax = oracle.quantize_sim(v)
    r = oracle.dequantize_sim(codes, absmax)
    bound = np.repeat(0.5 * max_gap * absmax, 64) + 1e-6
    assert np.all(np.abs(r - v) <= bound)
    nf4_err = float(np.sum((v - r) ** 2))
    am = np.maximum(absmax, 1e-12).repeat(64)
    step = 2 * am / 15
    uni = np.round((v + am) / step) * step - am
    assert nf4_err < float(np.sum((v - uni) ** 2))


def test_zero_blocks_are_exact(oracle):
    # src/quantize.rs:957-964, src/verify.rs:1068-1078
    codes, absmax = oracle.quantize_sim(np.zeros(128, np.float32))
    assert np.all(oracle.dequantize_sim(codes, absmax) == 0) and np.all(codes == 7)
    v = np.zeros(64, np.float32)
    v[3] = 2.5
    codes, absmax = oracle.quantize_sim(v)
    assert oracle.dequantize_sim(codes, absmax)[0] == 0.0


def test_ragged_last_block(oracle):
    # src/quantize.rs:966-973
    v = (np.arange(69, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    codes, absmax = oracle.quantize_sim(v)
    assert absmax.size == 2 and oracle.dequantize_sim(codes, absmax).size == 69


def test_quantized_weights_stay_on_the_grid(oracle):
    # src/quantize.rs:1132-1163
    v = np.random.default_rng(5).standard_normal(4 * 64).astype(np.float32)
    codes, absmax = oracle.quantize_sim(v)
    r = oracle.dequantize_sim(codes, absmax)
    grid = oracle.levels()[None, :] * np.repeat(absmax, 64)[:, None]
    assert np.all(np.min(np.abs(grid - r[:, None]), axis=1) <= 1e-6 * np.maximum(np.repeat(absmax, 64), 1))


@pytest.mark.parametrize("n", [1000, 63, 384, 2048])
def test_packed_roundtrip_matches_simulated_exactly(oracle, n):
    # src/quantize.rs:755-791, src/verify.rs:1086-1120
    v = (np.random.default_rng(n).standard_normal(n) * 1.7).astype(np.float32)
    if n >= 192:
        v[64:128] = 0
    codes, absmax = oracle.quantize_sim(v)
    packed, absmax_p = oracle.quantize_packed(v)
    assert np.array_equal(bits(absmax), bits(absmax_p))
    expect = codes if n % 2 == 0 else np.concatenate([codes, [0]]).astype(np.uint8)
    assert np.array_equal(packed, expect[0::2] | (expect[1::2] << 4))
    q, sos = oracle.double_quantize(absmax)
    assert np.array_equal(bits(oracle.dequantize_packed(packed, n, absmax_p)),
                          bits(oracle.dequantize_sim(codes, absmax)))
    assert np.array_equal(bits(oracle.dequantize_packed(packed, n, None, q, sos)),
                          bits(oracle.dequantize_sim(codes, None, q, sos)))


def test_residency_known_answer(oracle):
    # src/quantize.rs:793-822: 640 values = 10 blocks
    assert oracle.estimated_resident_bytes(640, False) == 320 + 40
    assert oracle.estimated_resident_bytes(640, True) == 320 + 10 + 4
    assert abs(oracle.bits_per_value_packed(640, False) - 4.5) < 1e-9
    assert oracle.bits_per_value_packed(640, True) < 4.2
    assert abs(oracle.bits_per_value_sim(64 * 64, False) - 4.5) < 1e-9
    assert oracle.bits_per_value_sim(64 * 64, True) < 4.2
    assert oracle.bits_per_value_sim(0, True) == 0.0


def test_double_quantization_keeps_accuracy(oracle):
    # src/quantize.rs:975-1009
    v = np.random.default_rng(11).standard_normal(64 * 64).astype(np.float32)
    codes, absmax = oracle.quantize_sim(v)
    q, sos = oracle.double_quantize(absmax)
    e_plain = np.sum((oracle.dequantize_sim(codes, absmax) - v) ** 2)
    e_dq = np.sum((oracle.dequantize_sim(codes, None, q, sos) - v) ** 2)
    assert e_dq < 1.1 * e_plain


# ------------------------------------------------ double quantization forms --

def test_double_quantization_closed_forms(oracle):
    a = np.array([0.5, 2.0, 1.0, 0.0], np.float32)
    q, sos = oracle.double_quantize(a)
    assert sos == np.float32(2.0) and q[1] == 255 and q[3] == 0 and q[2] == 128  # 127.5 -> away
    q0, sos0 = oracle.double_quantize(np.zeros(5, np.float32))
    assert sos0 == 0 and np.all(q0 == 0)
    # +inf absmax: every finite block -> 0, the inf block -> NaN -> 0
    qi, sosi = oracle.double_quantize(np.array([1.0, np.inf], np.float32))
    assert np.isinf(sosi) and qi[0] == 0 and qi[1] == 0


def test_double_quantization_rounds_ties_away_from_zero(oracle):
    # find t with fl(t * 255) == k + 0.5 exactly, for even k (so that
    # round-half-even would give k, and half-away gives k + 1)
    found = 0
    for k in range(0, 254, 2):
        t = np.float32((k + 0.5) / 255)
        if np.float32(t * np.float32(255)) == np.float32(k + 0.5):
            q, _ = oracle.double_quantize(np.array([1.0, t], np.float32))
            assert q[1] == k + 1
            found += 1
    assert found > 5


def test_dq_scale_formula_order(oracle):
    # ((q / 255) * sos), two f32 roundings in that order
    for q in (1, 17, 128, 254, 255):
        for sos in (0.02, 3.7, 1e-30):
            expect = np.float32(np.float32(np.float32(q) / np.float32(255)) * np.float32(sos))
            assert oracle.dq_scale(q, sos) == expect


# ---------------------------------------------------------------- fixtures --

def test_oracle_matches_independent_numpy_fixtures(oracle, fixtures):
    names, z = fixtures
    assert len(names) >= 10
    for nm in names:
        v = z[f"{nm}.values"]
        codes, absmax = oracle.quantize_sim(v)
        packed, _ = oracle.quantize_packed(v)
        q, sos = oracle.double_quantize(absmax)
        assert np.array_equal(codes, z[f"{nm}.codes"]), nm
        assert np.array_equal(packed, z[f"{nm}.packed"]), nm
        assert np.array_equal(bits(absmax), bits(z[f"{nm}.absmax"])), nm
        assert np.array_equal(q, z[f"{nm}.dq_codes"]), nm
        assert bits(np.float32(sos))[()] == bits(z[f"{nm}.dq_sos"])[0], nm
        assert np.array_equal(bits(oracle.dequantize_packed(packed, v.size, absmax)),
                              bits(z[f"{nm}.deq_plain"])), nm
        assert np.array_equal(bits(oracle.dequantize_packed(packed, v.size, None, q, sos)),
                              bits(z[f"{nm}.deq_dq"])), nm


# --------------------------------------------------------- linear and misc --

def test_linear_orientation_known_answer(oracle):
    # src/qwennet.rs:2196-2211: W [[1,2,3],[4,5,6]] as [in=2, out=3], x = [1, -1]
    y = oracle.linear_f32(np.array([1.0, -1.0]), np.arange(1, 7, dtype=np.float32), 2, 3)
    assert np.array_equal(y, [[-3.0, -3.0, -3.0]])


def test_linear_f32_matches_f64_product(oracle):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((3, 300)).astype(np.float32)
    w = rng.standard_normal((300, 70)).astype(np.float32)
    b = rng.standard_normal(70).astype(np.float32)
    y = oracle.linear_f32(x, w, 300, 70, bias=b, threads=2)
    ref = oracle.linear_ref_f64(x, w, b)
    assert oracle.normwise_error(y, ref, x, np.abs(x) @ np.abs(w)) < 1e-5


def test_error_metrics_known_answers(oracle):
    # normwise: the largest |y - r| over the bound of the same element, not
    # over the largest bound; literal: the largest |y - r| over the largest |r|
    y = np.array([[1.0, 2.5], [0.0, -4.0]])
    r = np.array([[1.0, 2.0], [0.1, -4.0]])
    bound = np.array([[10.0, 5.0], [0.2, 8.0]])
    assert oracle.normwise_error(y, r, None, bound) == pytest.approx(0.5)   # 0.1 / 0.2
    assert oracle.max_rel_error(y, r) == pytest.approx(0.125)              # 0.5 / 4
    assert oracle.normwise_error(r, r, None, bound) == 0.0
    assert oracle.max_rel_error(np.zeros(3), np.zeros(3)) == 0.0            # no division by zero
    assert oracle.num_blocks(0) == 0 and oracle.num_blocks(64) == 1 and oracle.num_blocks(65) == 2


@pytest.mark.parametrize("m,k,n", [(2, 3, 3), (7, 300, 70), (97, 513, 2050), (6, 256, 16), (1, 1, 1), (5, 0, 4)])
def test_sgemm_blocked_matches_f64_product(oracle, m, k, n):
    # the CPU baseline's blocked sgemm: ragged edges of every block size
    # (MR 6, NR 16, KC 256, MC 96, NC 2048), a second k block, empty k
    rng = np.random.default_rng(m * 1000 + k + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    c = oracle.sgemm_blocked(a, b, threads=3)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    bound = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    assert c.shape == (m, n)
    assert np.all(np.abs(c - ref) <= 1e-5 * np.maximum(bound, 1e-30))
    # orientation: the known answer of nf4o_linear_f32's test
    y = oracle.sgemm_blocked(np.array([[1.0, -1.0]]), np.arange(1, 7, dtype=np.float32).reshape(2, 3))
    assert np.array_equal(y, [[-3.0, -3.0, -3.0]])


def test_checkpoint_f16_decode_all_bit_patterns(oracle):
    # f16_to_f32 (src/import.rs:283-317) over every binary16 pattern
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = oracle.decode_checkpoint(bits, "f16").view(np.uint32)
    ieee = bits.view(np.float16).astype(np.float32).view(np.uint32)  # exact widening
    exp, mant = (bits.astype(np.uint32) >> 10) & 0x1F, bits.astype(np.uint32) & 0x3FF
    nan = (exp == 0x1F) & (mant != 0)
    assert np.array_equal(got[~nan], ieee[~nan])
    # NaN: payload moved up 13 bits and the quiet bit forced (a signalling
    # input cannot trap downstream)
    assert np.array_equal(got[nan], ieee[nan] | np.uint32(0x00400000))
    assert np.all((got[nan] & np.uint32(0x7FC00000)) == np.uint32(0x7FC00000))
    # subnormals: mant * 2^-24 exactly, from the mathematics rather than numpy
    sub = (exp == 0) & (mant != 0)
    vals = got[sub].view(np.float32).astype(np.float64)
    sign = np.where(bits[sub] & 0x8000, -1.0, 1.0)
    assert np.array_equal(vals, sign * mant[sub].astype(np.float64) * 2.0 ** -24)
    known = {0x3C00: 1.0, 0xC000: -2.0, 0x7BFF: 65504.0, 0x0001: 2.0 ** -24, 0x03FF: 1023 * 2.0 ** -24,
             0x0400: 2.0 ** -14, 0x3555: 0.333251953125}
    for b, v in known.items():
        assert float(oracle.decode_checkpoint(np.array([b]), "f16")[0]) == v, hex(b)
    inf = oracle.decode_checkpoint(np.array([0x7C00, 0xFC00, 0x8000]), "f16")
    assert inf[0] == np.inf and inf[1] == -np.inf and inf[2] == 0.0 and np.signbit(inf[2])


def test_checkpoint_bf16_decode_all_bit_patterns(oracle):
    # bf16_to_f32 (src/import.rs:321-327): the top 16 bits of the f32
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = oracle.decode_checkpoint(bits, "bf16").view(np.uint32)
    assert np.array_equal(got, bits.astype(np.uint32) << 16)


def test_silu_closed_forms(oracle):
    z = np.array([0.0, 30.0, -30.0, 1.0, -2.5, 1e-3], np.float32)
    s = oracle.silu(z)
    assert s[0] == 0 and s[1] == np.float32(30.0) and abs(s[2]) < 1e-11
    ref = oracle.silu_f64(z)
    assert np.all(np.abs(s - ref) <= 4 * np.spacing(np.abs(ref).astype(np.float32)) + 1e-12)


def test_rms_norm_closed_forms(oracle):
    """QwenRmsNorm (src/qwennet.rs:104-109): known answers that catch a sum
    taken for the mean, eps added outside the root, or w used for w + 1."""
    x = np.array([[3.0, 4.0]])
    np.testing.assert_allclose(oracle.rms_norm_f64(x, [0.0, 0.0], 0.0), x / np.sqrt(12.5), rtol=1e-15)
    # eps inside the root: mean 1, eps 3 -> 1 / sqrt(4)
    np.testing.assert_allclose(oracle.rms_norm_f64([[1.0, 1.0]], [0.0, 0.0], 3.0), [[0.5, 0.5]], rtol=1e-15)
    # the weight enters as w + 1: a constant row normalises to sign * (w + 1)
    w = np.array([0.5, -0.25, 2.0])
    np.testing.assert_allclose(oracle.rms_norm_f64([[-7.0, -7.0, -7.0]], w, 0.0), [-(w + 1.0)], rtol=1e-15)
    # unit mean square with w = 0, eps = 0, for any row; scale invariant
    r = np.random.default_rng(5).normal(size=(4, 37))
    n = oracle.rms_norm_f64(r, np.zeros(37), 0.0)
    np.testing.assert_allclose(np.mean(n * n, axis=-1), 1.0, rtol=1e-12)
    np.testing.assert_allclose(oracle.rms_norm_f64(9.0 * r, np.zeros(37), 0.0), n, rtol=1e-12)
    assert np.all(oracle.rms_norm_f64(np.zeros((1, 5)), np.zeros(5), 1e-6) == 0.0)


def test_decoder_stage_references_compose(oracle):
    """The decoder-step references: residuals are identities when the
    projections are zero, and the attention-input stage is the norm followed
    by the three products."""
    rng = np.random.default_rng(11)
    h, inter, qd = 8, 12, 6
    x = rng.normal(size=(2, h))
    ctx = rng.normal(size=(2, qd))
    g = rng.normal(size=h)
    z = lambda a, b: np.zeros((a, b))
    x1, y = oracle.decoder_attn_out_mlp_ref_f64(x, ctx, g, 1e-6, z(qd, h), z(h, inter), z(h, inter), z(inter, h))
    np.testing.assert_array_equal(x1, x)
    np.testing.assert_array_equal(y, x)
    wo = rng.normal(size=(qd, h))
    x1, y = oracle.decoder_attn_out_mlp_ref_f64(x, ctx, g, 1e-6, wo, rng.normal(size=(h, inter)),
                                                rng.normal(size=(h, inter)), z(inter, h))
    np.testing.assert_allclose(x1, x + ctx @ wo, rtol=1e-14)
    np.testing.assert_array_equal(y, x1)
    wq, wk, wv = (rng.normal(size=(h, d)) for d in (4, 2, 2))
    q, k, v = oracle.decoder_attn_in_ref_f64(x, g, 1e-6, wq, wk, wv)
    n = oracle.rms_norm_f64(x, g, 1e-6)
    for got, w in ((q, wq), (k, wk), (v, wv)):
        np.testing.assert_allclose(got, n @ w, rtol=1e-14)


def test_transpose_is_an_involution_with_index_identity(oracle):
    a = np.arange(130 * 67, dtype=np.float32)
    t = oracle.transpose(a, 130, 67)
    assert np.array_equal(t.reshape(67, 130), a.reshape(130, 67).T)
    assert np.array_equal(oracle.transpose(t, 67, 130), a)


def test_generator_is_deterministic_with_normal_moments(oracle):
    a = oracle.fill_normal(123, 0.02, 1_000_000)
    assert np.array_equal(bits(a), bits(oracle.fill_normal(123, 0.02, 1_000_000)))
    assert not np.array_equal(a, oracle.fill_normal(124, 0.02, 1_000_000))
    assert abs(a.mean()) < 1e-4 and abs(a.std() - 0.02) < 1e-4


def test_round_bf16_is_round_to_nearest_even(oracle):
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -3.0, np.inf], np.float32)
    r = oracle.round_bf16(x)
    assert list(r) == [1.0, 1.0, 1.0 + 2 ** -6, -3.0, np.inf]


def test_thresholds_sit_far_from_bucket_edges_and_from_each_other():
    # The GPU quantizer classifies v * rcp(absmax), which is within 2^-22 of
    # fl(v / absmax), through a table over floor(16 u), and divides exactly
    # only within 2^-20 of the threshold inside the bucket.  That is exact if
    # every threshold is more than 2^-20 + 2^-22 from each bucket edge j / 16
    # and the thresholds are more than 1/16 apart (one per bucket).
    T = np.array(THRESHOLD_BITS, np.uint32).view(np.float32).astype(np.float64)
    edge = np.abs(T * 16 - np.round(T * 16)) / 16
    assert edge.min() > 2.0 ** -20 + 2.0 ** -22
    assert edge.min() > 2.0 ** -10  # in fact more than 2^-10
    assert np.diff(np.sort(T)).min() > 1.0 / 16


# ---------------------------------------- SwiGLU, LoRA and backward refs --

def test_swiglu_ref_known_answers(oracle):
    """QwenMlp::forward (src/qwennet.rs:816-819) is down(silu(gate x) * up x):
    silu goes through the gate product only, down is applied last."""
    one = np.array([[1.0]])
    y = oracle.swiglu_ref_f64(one, one, 2.0 * one, one)
    # silu(1) * 2 = 2 / (1 + e^-1); with gate and up swapped: silu(2) * 1
    assert abs(y[0, 0] - 1.4621171572600098) < 1e-15
    assert abs(oracle.swiglu_ref_f64(one, 2.0 * one, one, one)[0, 0] - 1.7615941559557649) < 1e-15
    rng = np.random.default_rng(21)
    x = rng.normal(size=(3, 5))
    wg, wu, wd = rng.normal(size=(5, 7)), rng.normal(size=(5, 7)), rng.normal(size=(7, 4))
    assert np.all(oracle.swiglu_ref_f64(x, wg, np.zeros((5, 7)), wd) == 0.0)  # up = 0
    assert np.all(oracle.swiglu_ref_f64(x, np.zeros((5, 7)), wu, wd) == 0.0)  # silu(0) = 0
    # orientation of down: hidden 2 -> intermediate 1 -> hidden 2
    y = oracle.swiglu_ref_f64([[1.0, 0.0]], [[1.0], [0.0]], [[2.0], [0.0]], [[3.0, -1.0]])
    h = 2.0 / (1.0 + np.exp(-1.0))
    np.testing.assert_allclose(y, [[3.0 * h, -h]], rtol=1e-15)


def test_swiglu_ref_matches_torch_float64(oracle):
    """Against an independent evaluation (torch's silu on the CPU, float64)."""
    import torch
    rng = np.random.default_rng(22)
    x = rng.normal(size=(6, 32))
    wg, wu, wd = (rng.normal(scale=0.2, size=s) for s in ((32, 48), (32, 48), (48, 32)))
    t = lambda a: torch.from_numpy(a)
    ref = (torch.nn.functional.silu(t(x) @ t(wg)) * (t(x) @ t(wu))) @ t(wd)
    np.testing.assert_allclose(oracle.swiglu_ref_f64(x, wg, wu, wd), ref.numpy(), rtol=1e-12, atol=1e-14)
    swapped = (torch.nn.functional.silu(t(x) @ t(wu)) * (t(x) @ t(wg))) @ t(wd)
    assert np.max(np.abs(oracle.swiglu_ref_f64(x, wg, wu, wd) - swapped.numpy())) > 1e-2


def test_lora_ref_scaling_and_dense_identity(oracle):
    """src/quantize.rs:1027-1047: LoraConfig::new(12, 6, 3).with_alpha(6)
    scales by alpha / rank = 2, and the factored (x A) B s equals x (s A B)."""
    from unifur_amd.quantize import LoraConfig
    cfg = LoraConfig.new(12, 6, 3).with_alpha(6.0)
    assert cfg.scaling() == 2.0
    assert LoraConfig.new(16, 8, 4).scaling() == 1.0  # alpha defaults to the rank
    rng = np.random.default_rng(23)
    x = rng.uniform(-1, 1, size=(4, 12))
    a = rng.normal(scale=1 / np.sqrt(3), size=(12, 3))
    b = rng.uniform(-0.5, 0.5, size=(3, 6))
    factored = oracle.lora_ref_f64(x, a, b, cfg.scaling())
    np.testing.assert_allclose(factored, x @ (cfg.scaling() * (a @ b)), rtol=1e-12, atol=1e-14)
    # B = 0 at init: an exact no-op (src/quantize.rs:1011-1025)
    assert np.all(oracle.lora_ref_f64(x, a, np.zeros((3, 6)), 2.0) == 0.0)


def test_lora_ref_hand_computed(oracle):
    """x A = [1, 2], (x A) B = [2, 1], times 0.5; B A order would give
    [1.5, 2], A transposed [1.5, 0.5]."""
    x = np.array([[1.0, 0.0]])
    a = np.array([[1.0, 2.0], [3.0, 4.0]])
    b = np.array([[0.0, 1.0], [1.0, 0.0]])
    np.testing.assert_array_equal(oracle.lora_ref_f64(x, a, b, 0.5), [[1.0, 0.5]])


def _qlora_forward_f64(x, w, a, b, s):
    return x @ w + (x @ a) @ b * s


def test_backward_ref_matches_autograd(oracle):
    """The VJP formulas against torch.autograd of the float64 forward
    x W + ((x A) B) s on the CPU, with s != 1 and non-square factors so that
    a missing or doubled s, or a dropped transpose, cannot agree."""
    import torch
    rng = np.random.default_rng(24)
    M, K, N, r, s = 5, 7, 6, 3, 2.5
    x, w = rng.normal(size=(M, K)), rng.normal(size=(K, N))
    a, b, dy = rng.normal(size=(K, r)), rng.normal(size=(r, N)), rng.normal(size=(M, N))
    tx, ta, tb = (torch.tensor(v, requires_grad=True) for v in (x, a, b))
    y = _qlora_forward_f64(tx, torch.from_numpy(w), ta, tb, s)
    y.backward(torch.from_numpy(dy))
    dx, _, ga, _, gb, _ = oracle.linear_backward_ref_f64(x, dy, w, a, b, s)
    for got, want in ((dx, tx.grad), (ga, ta.grad), (gb, tb.grad)):
        np.testing.assert_allclose(got, want.numpy(), rtol=1e-12, atol=1e-12)
    # the same check rejects the plausible mistakes
    g = dy * s
    wrong = {
        "s twice in dx": dy @ w.T + ((g * s) @ b.T) @ a.T,
        "s dropped in grad_a": x.T @ (dy @ b.T),
        "s twice in grad_b": (x @ a).T @ (g * s),
    }
    assert np.max(np.abs(wrong["s twice in dx"] - tx.grad.numpy())) > 1e-3
    assert np.max(np.abs(wrong["s dropped in grad_a"] - ta.grad.numpy())) > 1e-3
    assert np.max(np.abs(wrong["s twice in grad_b"] - tb.grad.numpy())) > 1e-3


def test_backward_ref_matches_central_differences(oracle):
    """The forward is linear in x, in A and in B separately, so a central
    difference of <dy, y> is exact up to rounding: every entry of each
    gradient is checked that way."""
    rng = np.random.default_rng(25)
    M, K, N, r, s = 3, 5, 4, 2, 0.75
    x, w = rng.normal(size=(M, K)), rng.normal(size=(K, N))
    a, b, dy = rng.normal(size=(K, r)), rng.normal(size=(r, N)), rng.normal(size=(M, N))
    dx, _, ga, _, gb, _ = oracle.linear_backward_ref_f64(x, dy, w, a, b, s)
    loss = lambda x_, a_, b_: float(np.sum(dy * _qlora_forward_f64(x_, w, a_, b_, s)))
    h = 1e-3
    for arr, grad, which in ((x, dx, 0), (a, ga, 1), (b, gb, 2)):
        for idx in np.ndindex(arr.shape):
            args_p = [x.copy(), a.copy(), b.copy()]
            args_m = [x.copy(), a.copy(), b.copy()]
            args_p[which][idx] += h
            args_m[which][idx] -= h
            fd = (loss(*args_p) - loss(*args_m)) / (2 * h)
            assert abs(fd - grad[idx]) < 1e-9 * max(1.0, abs(fd)), (which, idx)


def test_backward_ref_bounds_dominate(oracle):
    """Each bound is the sum of the absolute products: never below the
    magnitude of its gradient, equal to it for non-negative inputs."""
    rng = np.random.default_rng(26)
    M, K, N, r, s = 4, 6, 5, 2, 3.0
    args = [rng.normal(size=sh) for sh in ((M, K), (M, N), (K, N), (K, r), (r, N))]
    dx, bdx, ga, bga, gb, bgb = oracle.linear_backward_ref_f64(*args, s)
    for g, bd in ((dx, bdx), (ga, bga), (gb, bgb)):
        assert np.all(np.abs(g) <= bd * (1 + 1e-12))
    pos = [np.abs(v) for v in args]
    dx, bdx, ga, bga, gb, bgb = oracle.linear_backward_ref_f64(*pos, s)
    for g, bd in ((dx, bdx), (ga, bga), (gb, bgb)):
        np.testing.assert_allclose(g, bd, rtol=1e-12)
