"""Python face of the CPU oracle (test infrastructure only).

Loads ``oracle/libnf4_oracle.so`` (the C restatement of unifur's
``src/quantize.rs`` NF4 codec, built by ``oracle/Makefile``) and adds the
float64 reference products the GEMV/GEMM/MLP parity tests compare against.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, as the checker or the timed CPU
baseline.  The product (``unifur_amd``) never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libnf4_oracle.so")
_lib = None

BLOCK = 64

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)


def build() -> str:
    """Compile the C restatement with its own Makefile (gcc, no GPU)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.nf4o_levels.argtypes = [_f32p]
        L.nf4o_nearest_level_code.argtypes = [ctypes.c_float]
        L.nf4o_nearest_level_code.restype = ctypes.c_uint8
        for name in ("nf4o_quantize_sim", "nf4o_quantize_packed"):
            getattr(L, name).argtypes = [_f32p, ctypes.c_size_t, _u8p, _f32p]
        L.nf4o_double_quantize.argtypes = [_f32p, ctypes.c_size_t, _u8p, _f32p]
        L.nf4o_dq_scale.argtypes = [ctypes.c_uint8, ctypes.c_float]
        L.nf4o_dq_scale.restype = ctypes.c_float
        for name in ("nf4o_dequantize_sim", "nf4o_dequantize_packed"):
            getattr(L, name).argtypes = [_u8p, ctypes.c_size_t, _f32p, _u8p, ctypes.c_float, _f32p]
        L.nf4o_estimated_resident_bytes.argtypes = [ctypes.c_size_t, ctypes.c_int]
        L.nf4o_estimated_resident_bytes.restype = ctypes.c_size_t
        for name in ("nf4o_bits_per_value_sim", "nf4o_bits_per_value_packed"):
            getattr(L, name).argtypes = [ctypes.c_size_t, ctypes.c_int]
            getattr(L, name).restype = ctypes.c_double
        L.nf4o_transpose.argtypes = [_f32p, ctypes.c_size_t, ctypes.c_size_t, _f32p]
        L.nf4o_silu.argtypes = [ctypes.c_float]
        L.nf4o_silu.restype = ctypes.c_float
        L.nf4o_silu_vec.argtypes = [_f32p, ctypes.c_size_t, _f32p]
        L.nf4o_linear_f32.argtypes = [_f32p, ctypes.c_size_t, _f32p, ctypes.c_size_t,
                                      ctypes.c_size_t, _f32p, _f32p, ctypes.c_int]
        L.nf4o_sgemm_blocked.argtypes = [_f32p, ctypes.c_size_t, ctypes.c_size_t, _f32p, ctypes.c_size_t,
                                         _f32p, ctypes.c_int]
        L.nf4o_sgemm_blocked.restype = ctypes.c_int
        L.nf4o_fill_normal.argtypes = [ctypes.c_uint64, ctypes.c_double, ctypes.c_size_t, _f32p]
        L.nf4o_round_bf16.argtypes = [_f32p, ctypes.c_size_t, _f32p]
        _u16p = ctypes.POINTER(ctypes.c_uint16)
        for name in ("nf4o_f16_to_f32", "nf4o_bf16_to_f32"):
            getattr(L, name).argtypes = [_u16p, ctypes.c_size_t, _f32p]
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def num_blocks(n: int) -> int:
    return (n + BLOCK - 1) // BLOCK


# --------------------------------------------------------------- codec ----

def levels() -> np.ndarray:
    out = np.empty(16, np.float32)
    lib().nf4o_levels(_p(out, _f32p))
    return out


def nearest_level_code(v: float) -> int:
    return int(lib().nf4o_nearest_level_code(ctypes.c_float(v)))


def quantize_sim(values) -> tuple[np.ndarray, np.ndarray]:
    """Nf4Tensor::quantize -> (codes u8[n], absmax f32[nb])."""
    v = _f32(values).ravel()
    codes = np.empty(v.size, np.uint8)
    absmax = np.empty(num_blocks(v.size), np.float32)
    lib().nf4o_quantize_sim(_p(v, _f32p), v.size, _p(codes, _u8p), _p(absmax, _f32p))
    return codes, absmax


def quantize_packed(values) -> tuple[np.ndarray, np.ndarray]:
    """PackedNf4Tensor::quantize -> (packed u8[ceil(n/2)], absmax f32[nb])."""
    v = _f32(values).ravel()
    packed = np.empty((v.size + 1) // 2, np.uint8)
    absmax = np.empty(num_blocks(v.size), np.float32)
    lib().nf4o_quantize_packed(_p(v, _f32p), v.size, _p(packed, _u8p), _p(absmax, _f32p))
    return packed, absmax


def double_quantize(absmax) -> tuple[np.ndarray, np.float32]:
    """with_double_quantization -> (q u8[nb], scale_of_scales f32)."""
    a = _f32(absmax).ravel()
    q = np.empty(a.size, np.uint8)
    sos = np.zeros(1, np.float32)
    lib().nf4o_double_quantize(_p(a, _f32p), a.size, _p(q, _u8p), _p(sos, _f32p))
    return q, sos[0]


def dq_scale(q: int, sos: float) -> np.float32:
    return np.float32(lib().nf4o_dq_scale(ctypes.c_uint8(q), ctypes.c_float(sos)))


def _dequant(fn, codes, n, absmax, dq_codes, sos):
    out = np.empty(n, np.float32)
    a = _f32(absmax if absmax is not None else np.zeros(num_blocks(n), np.float32))
    dq = None if dq_codes is None else np.ascontiguousarray(dq_codes, np.uint8)
    fn(_p(codes, _u8p), n, _p(a, _f32p), None if dq is None else _p(dq, _u8p),
       ctypes.c_float(0.0 if sos is None else float(sos)), _p(out, _f32p))
    return out


def dequantize_sim(codes, absmax=None, dq_codes=None, sos=None) -> np.ndarray:
    c = np.ascontiguousarray(codes, np.uint8)
    return _dequant(lib().nf4o_dequantize_sim, c, c.size, absmax, dq_codes, sos)


def dequantize_packed(packed, n, absmax=None, dq_codes=None, sos=None) -> np.ndarray:
    p = np.ascontiguousarray(packed, np.uint8)
    return _dequant(lib().nf4o_dequantize_packed, p, n, absmax, dq_codes, sos)


def estimated_resident_bytes(n: int, dq: bool) -> int:
    return int(lib().nf4o_estimated_resident_bytes(n, int(dq)))


def bits_per_value_sim(n: int, dq: bool) -> float:
    return float(lib().nf4o_bits_per_value_sim(n, int(dq)))


def bits_per_value_packed(n: int, dq: bool) -> float:
    return float(lib().nf4o_bits_per_value_packed(n, int(dq)))


def transpose(data, rows: int, cols: int) -> np.ndarray:
    d = _f32(data).ravel()
    out = np.empty(rows * cols, np.float32)
    lib().nf4o_transpose(_p(d, _f32p), rows, cols, _p(out, _f32p))
    return out


def silu(x) -> np.ndarray:
    v = _f32(x)
    out = np.empty_like(v)
    lib().nf4o_silu_vec(_p(v, _f32p), v.size, _p(out, _f32p))
    return out


def linear_f32(x, w, d_in: int, d_out: int, bias=None, threads: int = 0) -> np.ndarray:
    """Restated burn linear in f32 (the timed CPU baseline's matmul)."""
    xv = _f32(x).reshape(-1, d_in)
    wv = _f32(w).reshape(d_in, d_out)
    b = None if bias is None else _f32(bias)
    y = np.empty((xv.shape[0], d_out), np.float32)
    lib().nf4o_linear_f32(_p(xv, _f32p), xv.shape[0], _p(wv, _f32p), d_in, d_out,
                          None if b is None else _p(b, _f32p), _p(y, _f32p), int(threads))
    return y


def sgemm_blocked(a, b, threads: int = 0) -> np.ndarray:
    """a [m, k] @ b [k, n] in f32 by the blocked, packed CPU sgemm
    (oracle/cpu_sgemm.c): the CPU baseline's stand-in for the matrixmultiply
    crate that burn-ndarray's matmul runs on.  Not a parity reference."""
    av = np.ascontiguousarray(a, np.float32)
    bv = np.ascontiguousarray(b, np.float32)
    if av.ndim != 2 or bv.ndim != 2 or av.shape[1] != bv.shape[0]:
        raise ValueError(f"sgemm_blocked: shapes {av.shape} and {bv.shape} do not chain")
    c = np.empty((av.shape[0], bv.shape[1]), np.float32)
    if lib().nf4o_sgemm_blocked(_p(av, _f32p), av.shape[0], av.shape[1], _p(bv, _f32p), bv.shape[1],
                                _p(c, _f32p), int(threads)) != 0:
        raise MemoryError("sgemm_blocked: packing buffers")
    return c


def fill_normal(seed: int, sigma: float, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().nf4o_fill_normal(ctypes.c_uint64(seed), float(sigma), n, _p(out, _f32p))
    return out


def decode_checkpoint(bits, dtype: str) -> np.ndarray:
    """Checkpoint elements (u16 bit patterns) to f32 as read_tensor_f32 does
    (src/import.rs:255-272): ``dtype`` "f16" (f16_to_f32, src/import.rs:283-317)
    or "bf16" (bf16_to_f32, src/import.rs:321-327)."""
    b = np.ascontiguousarray(bits, np.uint16)
    out = np.empty(b.shape, np.float32)
    fn = {"f16": lib().nf4o_f16_to_f32, "bf16": lib().nf4o_bf16_to_f32}[dtype]
    fn(b.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), b.size, _p(out, _f32p))
    return out


def round_bf16(x) -> np.ndarray:
    v = _f32(x)
    out = np.empty_like(v)
    lib().nf4o_round_bf16(_p(v, _f32p), v.size, _p(out, _f32p))
    return out


# ------------------------------------------------- float64 references ----

def linear_ref_f64(x, w_deq, bias=None) -> np.ndarray:
    """y = x @ W (+ b) in float64 on exactly the inputs the GPU sees."""
    y = np.asarray(x, np.float64) @ np.asarray(w_deq, np.float64)
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    return y


def lora_ref_f64(x, a, b, scaling) -> np.ndarray:
    """LoraAdapter::forward (src/quantize.rs:619-624): (x @ A) @ B * scaling."""
    x64 = np.asarray(x, np.float64)
    return (x64 @ np.asarray(a, np.float64)) @ np.asarray(b, np.float64) * float(scaling)


def linear_backward_ref_f64(x, dy, w_deq, a, b, scaling):
    """Vector-Jacobian products of y = x W + ((x A) B) s, the function of
    QloraLinear::forward (src/qwennet.rs:325-345) with LoraAdapter::forward
    (src/quantize.rs:619-624), that burn's autodiff takes under
    src/qwentrain.rs:421-470 with the base weight frozen, in float64:

        dx     = dy W^T + ((dy s) B^T) A^T
        grad_a = x^T ((dy s) B^T)
        grad_b = (x A)^T (dy s)

    Returns (dx, dx_bound, grad_a, grad_a_bound, grad_b, grad_b_bound); each
    bound is the same sum of products over absolute values, the scale of the
    accumulated terms for a normwise error."""
    x = np.asarray(x, np.float64)
    dy = np.asarray(dy, np.float64)
    w = np.asarray(w_deq, np.float64)
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    g = dy * float(scaling)
    dx = dy @ w.T + (g @ b.T) @ a.T
    dx_bound = np.abs(dy) @ np.abs(w).T + (np.abs(g) @ np.abs(b).T) @ np.abs(a).T
    gb = (x @ a).T @ g
    gb_bound = (np.abs(x) @ np.abs(a)).T @ np.abs(g)
    ga = x.T @ (g @ b.T)
    ga_bound = np.abs(x).T @ (np.abs(g) @ np.abs(b).T)
    return dx, dx_bound, ga, ga_bound, gb, gb_bound


def silu_f64(z):
    z = np.asarray(z, np.float64)
    return z / (1.0 + np.exp(-z))


def swiglu_ref_f64(x, wg, wu, wd) -> np.ndarray:
    """QwenMlp::forward (src/qwennet.rs:816-819): down(silu(gate x) * up x)."""
    x64 = np.asarray(x, np.float64)
    h = silu_f64(x64 @ np.asarray(wg, np.float64)) * (x64 @ np.asarray(wu, np.float64))
    return h @ np.asarray(wd, np.float64)


def rms_norm_f64(x, w, eps) -> np.ndarray:
    """QwenRmsNorm::forward (src/qwennet.rs:104-109) over the last dim:
    x * (mean(x^2) + eps)^(-1/2) * (w + 1), in float64."""
    x64 = np.asarray(x, np.float64)
    ms = np.mean(x64 * x64, axis=-1, keepdims=True)
    return x64 * (ms + float(eps)) ** -0.5 * (np.asarray(w, np.float64) + 1.0)


def decoder_attn_in_ref_f64(x, input_norm, eps, wq, wk, wv):
    """QwenDecoderLayer::step up to the attention (src/qwennet.rs:1112-1121,
    QwenFullAttention::project :927-951 before the QK norms): q, k, v of
    input_norm(x), each with its dequantized weight [hidden, d_out]."""
    n = rms_norm_f64(x, input_norm, eps)
    return linear_ref_f64(n, wq), linear_ref_f64(n, wk), linear_ref_f64(n, wv)


def decoder_attn_out_mlp_ref_f64(x, ctx, post_norm, eps, wo, wg, wu, wd):
    """QwenDecoderLayer::step after the attention (src/qwennet.rs:1122-1128):
    x1 = x + ctx Wo; x1 + QwenMlp(post_norm(x1)).  Returns (x1, y)."""
    x1 = np.asarray(x, np.float64) + linear_ref_f64(ctx, wo)
    return x1, x1 + swiglu_ref_f64(rms_norm_f64(x1, post_norm, eps), wg, wu, wd)


def normwise_error(y, ref, x, w_abs_bound) -> float:
    """max_n |y_n - r_n| / max(sum_k |x_k| |W_kn|, tiny), per output row.

    ``w_abs_bound`` is |x| @ |W| (float64), the scale of the accumulated
    terms; elementwise relative error is unbounded near zero outputs."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.maximum(np.asarray(w_abs_bound, np.float64), 1e-30)
    return float(np.max(np.abs(y - ref) / den))


def max_rel_error(y, ref) -> float:
    """BASELINE-literal max|y - r| / max|r|."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-30))
