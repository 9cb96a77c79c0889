"""The C ABI library on a CPU-only host: it loads, exports every symbol that
include/unifur_nf4.h declares, and its host-only accounting agrees with the
oracle.  No kernel is launched here."""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "unifur_nf4.h")


def declared_symbols() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(unifur_nf4_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from unifur_amd import _lib
    return _lib.lib()


def test_library_exports_every_declared_symbol(lib):
    from unifur_amd import _lib
    syms = declared_symbols()
    assert len(syms) >= 15
    for s in syms:
        assert hasattr(lib, s), f"{s} declared in unifur_nf4.h but not exported"
    assert set(syms) == set(_lib.SIGNATURES), "ctypes binding and header disagree"


def test_library_exports_nothing_beyond_the_header(lib):
    """The product library's exported C symbols are exactly the header's: the
    bench's measurement kernels live in their own library."""
    import subprocess
    from unifur_amd import _lib
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.split() and line.split()[-1].startswith("unifur_")}
    assert exported == set(declared_symbols()), sorted(exported ^ set(declared_symbols()))


def test_levels_match_oracle(lib, oracle):
    out = (ctypes.c_float * 16)()
    assert lib.unifur_nf4_levels(out) == 0
    assert np.array_equal(np.array(out, np.float32).view(np.uint32), oracle.levels().view(np.uint32))


@pytest.mark.parametrize("n", [0, 1, 2, 63, 64, 65, 69, 127, 128, 640, 1000, 4096 * 11008])
def test_accounting_matches_oracle(lib, oracle, n):
    assert lib.unifur_nf4_num_blocks(n) == (n + 63) // 64
    assert lib.unifur_nf4_packed_bytes(n) == (n + 1) // 2
    for dq in (0, 1):
        assert lib.unifur_nf4_estimated_resident_bytes(n, dq) == oracle.estimated_resident_bytes(n, dq)
        assert lib.unifur_nf4_bits_per_value(n, dq) == oracle.bits_per_value_packed(n, dq)
        assert lib.unifur_nf4_simulated_bits_per_value(n, dq) == oracle.bits_per_value_sim(n, dq)


def test_invalid_arguments_fail_before_any_device_work(lib):
    from unifur_amd import _lib
    st = lib.unifur_nf4_quantize(None, 10, None, None, None)
    assert st == _lib.ERR_INVALID and b"NULL" in lib.unifur_nf4_last_error()
    s = _lib.Scales(7, None, None, None)
    assert lib.unifur_nf4_dequantize(None, ctypes.byref(s), 10, None, 0, None) == _lib.ERR_INVALID
    assert b"scales kind" in lib.unifur_nf4_last_error()
    w = _lib.Weight(None, _lib.Scales(0, None, None, None), 4, 4)
    assert lib.unifur_nf4_linear_forward(None, 0, 1, ctypes.byref(w), None, None, None, 0, None, 0,
                                         None) == _lib.ERR_INVALID
    assert lib.unifur_nf4_linear_forward(None, 5, 1, ctypes.byref(w), None, None, None, 0, None, 0,
                                         None) == _lib.ERR_INVALID
    assert lib.unifur_nf4_qlora_forward(None, 0, 1, ctypes.byref(w), None, None, 0, None, 0,
                                        None) == _lib.ERR_INVALID


def test_shapes_past_any_device_are_refused(lib):
    """An element count over 2^48 (rows x a width, or a weight's d_in x
    d_out) is past any device: the size queries answer UINT64_MAX instead
    of a byte count that wrapped 64 bits, and the calls refuse the shape
    before any device work."""
    from unifur_amd import _lib
    top = (1 << 64) - 1
    big = (1 << 31) - 1  # each dimension within its own 2^31 bound
    assert lib.unifur_nf4_linear_workspace_size(big, big, big, 0, 0) == top
    assert lib.unifur_nf4_linear_min_workspace_size(big, 4096, big, 1, 16) == top
    assert lib.unifur_nf4_linear_backward_workspace_size(big, big, 4096, 1, 0) == top
    assert lib.unifur_nf4_linear_backward_min_workspace_size(big, big, 4096, 1, 0, 1) == top
    assert lib.unifur_nf4_swiglu_workspace_size(big, 4096, big, 1) == top
    assert lib.unifur_nf4_swiglu_min_workspace_size(big, big, 11008, 1) == top
    d_out = (ctypes.c_uint64 * 1)(big)
    assert lib.unifur_nf4_linear_multi_workspace_size(big, big, d_out, 1, 0) == top
    assert lib.unifur_nf4_quantize_linears_workspace_size((ctypes.c_uint64 * 1)(big), d_out, 1) == top
    # at the bound a weight of exactly 2^48 values still gets its byte count
    # (one row: the GEMV's counter region), one block more does not
    assert 0 < lib.unifur_nf4_linear_workspace_size(1, 1 << 24, 1 << 24, 0, 0) < top
    assert lib.unifur_nf4_linear_workspace_size(1, (1 << 24) + 64, 1 << 24, 0, 0) == top
    # a call with such a shape fails on the host (the pointers are never read)
    fake = 1 << 20
    w = _lib.Weight(fake, _lib.Scales(_lib.SCALES_F32, fake, None, None), big, 1 << 20, 0)
    assert lib.unifur_nf4_linear_forward(fake, _lib.F32, big, ctypes.byref(w), None, None, fake, _lib.F32, None, 0,
                                         None) == _lib.ERR_INVALID
    assert b"2^48" in lib.unifur_nf4_last_error()
    assert lib.unifur_nf4_embedding_forward(fake, None, 1 << 30, 1 << 20, fake, 0, 1, fake, _lib.F32,
                                            None) == _lib.ERR_INVALID
    assert b"2^48" in lib.unifur_nf4_last_error()


def test_workspace_sizes_are_consistent(lib):
    # GEMV path: counters + split-K partials; generic path: an f32 weight copy
    small = lib.unifur_nf4_linear_workspace_size(1, 4096, 11008, 0, 0)
    assert 0 < small < 4096 * 11008 * 4
    generic = lib.unifur_nf4_linear_workspace_size(1, 100, 70, 0, 0)
    assert generic >= 100 * 70 * 4
    assert lib.unifur_nf4_linear_workspace_size(0, 10, 10, 0, 0) == 0
    # every non-empty plan starts with the 64 KiB counter region
    assert lib.unifur_nf4_linear_workspace_size(1, 64, 64, 0, 0) >= 65536
    assert lib.unifur_nf4_swiglu_workspace_size(1, 4096, 11008, 1) >= 11008 * 4


def test_backward_and_prefill_workspace_sizes(lib):
    # host-only planning, including empty batches (no division by a zero
    # tile count)
    for rows in (0, 1, 5, 64, 65, 2048):
        bw = lib.unifur_nf4_linear_backward_workspace_size(rows, 4096, 4096, 1, 16)
        assert bw >= 65536
        if rows:  # bf16 dy: the expanded bf16 weight is part of it
            assert bw >= 4096 * 4096 * 2
        assert lib.unifur_nf4_linear_backward_workspace_size(rows, 100, 70, 0, 3) >= 65536
    # f32 dy over whole 64-column blocks: the f32 MFMA kernel, no weight copy
    assert 65536 <= lib.unifur_nf4_linear_backward_workspace_size(8, 256, 128, 0, 0) < 256 * 128 * 4
    # ... with d_out off the blocks: the generic path's f32 dequantized weight
    assert lib.unifur_nf4_linear_backward_workspace_size(8, 256, 100, 0, 0) >= 256 * 100 * 4
    # f32 activations past 64 rows: no weight copy either
    assert lib.unifur_nf4_linear_workspace_size(2048, 4096, 4096, 0, 16) < 4096 * 4096 * 4
    # prefill: the default holds the bf16 expansion, the minimum does not
    full = lib.unifur_nf4_linear_workspace_size(2048, 4096, 4096, 1, 16)
    lean = lib.unifur_nf4_linear_min_workspace_size(2048, 4096, 4096, 1, 16)
    assert lean < 4096 * 4096 * 2 <= full
    assert lib.unifur_nf4_swiglu_min_workspace_size(512, 4096, 11008, 1) < \
        lib.unifur_nf4_swiglu_workspace_size(512, 4096, 11008, 1)
