"""Write tests/golden/nf4_fixtures.npz: NF4 codec input/output vectors.

The reference (Rust, Burn 0.21) cannot be built here, and its own NF4 tests
draw unseeded random inputs, so it holds no NF4 golden vectors beyond the
published codebook.  These fixtures therefore come from a SECOND, independent
restatement of src/quantize.rs written here in numpy float32 (vectorised
argmin scan, numpy reductions), not from the C oracle: the oracle and the HIP
library are both checked against them bit for bit.

Inputs come from numpy's PCG64 (not the oracle's generator) and include the
reference tests' shapes (src/quantize.rs:755-791, :793-822, :868-894,
:957-973; src/verify.rs:1068-1078) plus NaN / Inf / -0 / subnormal blocks.

Run:  python tests/golden/make_golden.py   (rewrites the .npz in place)
"""
from __future__ import annotations

import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
BLOCK = 64

# The published NF4 codebook as float64 (src/quantize.rs:841-858, the
# bitsandbytes / QLoRA appendix values); cast to f32 it must equal NF4_LEVELS.
PUBLISHED_F64 = [
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634,
    0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
    0.7229568362236023, 1.0,
]
LEVELS = np.array(PUBLISHED_F64, dtype=np.float64).astype(np.float32)


def np_quantize(values: np.ndarray):
    v = np.asarray(values, np.float32).ravel()
    n = v.size
    nb = (n + BLOCK - 1) // BLOCK
    pad = np.full(nb * BLOCK, np.float32(0.0), np.float32)
    pad[:n] = v
    blocks = pad.reshape(nb, BLOCK)
    # absmax = fold(0, max(acc, |v|)) with NaN-ignoring max; the zero padding
    # of the last block cannot raise it.
    absmax = np.fmax.reduce(np.abs(blocks), axis=1, initial=np.float32(0.0)).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        u = np.where(absmax[:, None] == 0, np.float32(0.0), blocks / absmax[:, None]).astype(np.float32)
        d = np.abs(u[..., None] - LEVELS).astype(np.float32)  # [nb, 64, 16]
    # strict-< scan with first index winning == first argmin; NaN rows -> 0
    nan_row = np.isnan(d).all(axis=-1)
    codes = np.argmin(np.where(np.isnan(d), np.float32(np.inf), d), axis=-1).astype(np.uint8)
    codes[nan_row] = 0
    codes = codes.ravel()[:n]
    return codes, absmax


def np_pack(codes: np.ndarray) -> np.ndarray:
    c = np.asarray(codes, np.uint8)
    if c.size % 2:
        c = np.concatenate([c, np.zeros(1, np.uint8)])
    return (c[0::2] | (c[1::2] << 4)).astype(np.uint8)


def np_double_quantize(absmax: np.ndarray):
    a = np.asarray(absmax, np.float32)
    m = np.fmax.reduce(a, initial=np.float32(0.0)).astype(np.float32)
    if m == 0:
        return np.zeros(a.size, np.uint8), np.float32(m)
    with np.errstate(invalid="ignore"):
        x = ((a / m).astype(np.float32) * np.float32(255.0)).astype(np.float32)
        fl = np.floor(x)
        r = fl + ((x - fl) >= np.float32(0.5))  # half away from zero (x >= 0)
    r = np.where(np.isnan(r), 0, np.clip(r, 0, 255))
    return r.astype(np.uint8), np.float32(m)


def np_dequantize(codes, n, scales_per_block):
    c = np.asarray(codes, np.uint8)[:n]
    s = np.repeat(np.asarray(scales_per_block, np.float32), BLOCK)[:n]
    return (LEVELS[c] * s).astype(np.float32)


def dq_scales(q, sos):
    return ((np.asarray(q, np.uint8).astype(np.float32) / np.float32(255.0)).astype(np.float32)
            * np.float32(sos)).astype(np.float32)


def cases() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(20240917)
    out: dict[str, np.ndarray] = {}
    for n in (1000, 63, 384):  # src/quantize.rs:755-791
        v = (rng.standard_normal(n) * 1.7).astype(np.float32)
        if n >= 128 + 64:
            v[64:128] = 0.0
        out[f"normal_{n}"] = v
    out["normal_640"] = rng.standard_normal(640).astype(np.float32)  # :793-822
    out["ramp_69"] = (np.arange(69, dtype=np.float32) * np.float32(0.01)).astype(np.float32)  # :966-973
    out["grid_16"] = (LEVELS * np.float32(0.75)).astype(np.float32)  # :868-879
    e = np.full(64, np.float32(0.01), np.float32)
    e[7], e[9] = -4.25, 2.0
    out["endpoint_64"] = e  # :881-894
    z = np.zeros(128, np.float32)
    z[64 + 3] = 2.5
    out["zeros_mixed_128"] = z  # src/verify.rs:1068-1078
    out["normal_4096"] = rng.standard_normal(4096).astype(np.float32)  # :975-1009
    out["weights_96x128"] = (rng.standard_normal(96 * 128) * 0.02).astype(np.float32)
    s = (rng.standard_normal(64 * 8) * 3.0).astype(np.float32)
    s[0:64][5] = np.nan                      # NaN ignored by absmax, coded 0
    s[64:128][10] = np.inf                   # absmax inf: finite -> 7, inf -> 0
    s[64:128][11] = -np.inf
    s[128:192] = np.nan                      # all-NaN block: absmax 0, codes 7
    s[192:256] = -0.0                        # negative zeros
    s[256:320] = (rng.standard_normal(64) * 1e-40).astype(np.float32)  # subnormals
    s[320:384][::2] = 0.0
    s[384:448] = np.float32(1e30) * rng.standard_normal(64).astype(np.float32)
    s[448:512] = np.float32(-7.5)            # constant block
    out["specials_512"] = s
    return out


def main() -> None:
    arrays: dict[str, np.ndarray] = {}
    for name, v in cases().items():
        codes, absmax = np_quantize(v)
        q, sos = np_double_quantize(absmax)
        arrays[f"{name}.values"] = v
        arrays[f"{name}.codes"] = codes
        arrays[f"{name}.packed"] = np_pack(codes)
        arrays[f"{name}.absmax"] = absmax
        arrays[f"{name}.dq_codes"] = q
        arrays[f"{name}.dq_sos"] = np.array([sos], np.float32)
        with np.errstate(invalid="ignore", over="ignore"):
            arrays[f"{name}.deq_plain"] = np_dequantize(codes, v.size, absmax)
            arrays[f"{name}.deq_dq"] = np_dequantize(codes, v.size, dq_scales(q, sos))
    np.savez_compressed(os.path.join(HERE, "nf4_fixtures.npz"), **arrays)
    with open(os.path.join(HERE, "nf4_codebook.json"), "w") as f:
        json.dump({"source": "src/quantize.rs:841-858 (bitsandbytes get_4bit_type('nf4'))",
                   "published_f64": PUBLISHED_F64}, f, indent=1)
    print(f"wrote {len(arrays)} arrays")


if __name__ == "__main__":
    main()
