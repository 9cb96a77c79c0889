// nf4_common.hpp -- shared device-side definitions for the NF4 kernels.
//
// Layout facts every kernel relies on (they are the reference's, see
// src/quantize.rs:36-66 and :240-247):
//   * a tensor of n values is cut into ceil(n/64) blocks of 64 consecutive
//     values (the last block may be short);
//   * codes are packed two per byte, value 2i in the low nibble of byte i;
//   * a block's scale is its f32 absmax, or with double quantization
//     ((float)q / 255.0f) * scale_of_scales.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace unifur {

constexpr int kBlock = 64;

// NF4_LEVELS (src/quantize.rs:49-66) as the f32 bit patterns the decimal
// literals round to; identical to the reference's table bit for bit.
__host__ __device__ constexpr uint32_t level_bits(int c) {
  constexpr uint32_t bits[16] = {
      0xbf800000u, 0xbf3239b1u, 0xbf066b30u, 0xbeca32a0u, 0xbe91a24du, 0xbe3d353fu,
      0xbdba7871u, 0x00000000u, 0x3da2faffu, 0x3e24cae3u, 0x3e7c04ddu, 0x3ead033au,
      0x3ee1a4b8u, 0x3f1007abu, 0x3f3913b3u, 0x3f800000u};
  return bits[c];
}

__device__ __forceinline__ float level(int c) { return __uint_as_float(level_bits(c)); }

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

// Two f32 -> packed bf16x2, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  f32x2 v = {lo, hi};
  bf16x2 r = __builtin_convertvector(v, bf16x2);
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b16) { return __uint_as_float(b16 << 16); }

// binary16 bits -> f32, exact, as the reference's checkpoint decode
// (f16_to_f32, src/import.rs:283-317): a subnormal renormalised (its value
// mant * 2^-24), infinities kept, a NaN's payload kept with the quiet bit set.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16, exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
  uint32_t out;
  if (exp == 0u) {
    if (mant == 0u) {
      out = sign;
    } else {
      const uint32_t s = (uint32_t)__builtin_clz(mant) - 21u;  // shifts that bring the leading one to bit 10
      out = sign | ((113u - s) << 23) | (((mant << s) & 0x3ffu) << 13);
    }
  } else if (exp == 0x1fu) {
    out = sign | 0x7f800000u | (mant == 0u ? 0u : (((mant << 13) | 0x00400000u) & 0x007fffffu));
  } else {
    out = sign | ((exp + 112u) << 23) | (mant << 13);
  }
  return __uint_as_float(out);
}

// Element types a checkpoint tensor may arrive in (src/import.rs:255-272),
// each decoded to f32 exactly.
enum { kSrcF32 = 0, kSrcBf16 = 1, kSrcF16 = 2 };
template <int SRC>
__device__ __forceinline__ float decode_src(const void* base, uint64_t idx) {
  if constexpr (SRC == kSrcF32) return static_cast<const float*>(base)[idx];
  else if constexpr (SRC == kSrcBf16) return bf16_bits_to_f32(static_cast<const uint16_t*>(base)[idx]);
  else return f16_bits_to_f32(static_cast<const uint16_t*>(base)[idx]);
}
template <int SRC>
__device__ __forceinline__ float decode_half(uint32_t h16) {
  if constexpr (SRC == kSrcBf16) return bf16_bits_to_f32(h16);
  else return f16_bits_to_f32(h16);
}

// v_perm_b32: result byte i = byte sel[i] of the 8-byte value {a:b}
// (bytes 0-3 come from b, 4-7 from a, selector 0x0c yields 0x00).
__device__ __forceinline__ uint32_t perm_b32(uint32_t a, uint32_t b, uint32_t sel) {
  return __builtin_amdgcn_perm(a, b, sel);
}

// DPP move with every lane written: CTRL is a pattern whose source lane is
// always in the wave (quad_perm, row_mirror 0x140, row_half_mirror 0x141,
// row_newbcast 0x150 + j) and all rows and banks are enabled.  bound_ctrl
// (a lane with no source lane reads 0 -- there is none here) tells the
// compiler that no lane keeps the old value, so a move whose result is not
// folded into its user (v_max_u32_dpp, v_add_f32_dpp) needs no initialising
// v_mov_b32 of the destination, which the form without it costs per use.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {
  static_assert(CTRL <= 0xFF || CTRL == 0x140 || CTRL == 0x141 || (CTRL >= 0x150 && CTRL <= 0x15F),
                "a DPP pattern with out-of-range source lanes");
  return __builtin_amdgcn_update_dpp(0u, v, CTRL, 0xF, 0xF, true);
}

// Split-K hand-off between workgroups.  Partial sums are written with
// agent-scope atomic stores (coherent across the XCDs' L2s) and the writer
// waits for them to complete before it counts itself in; the last arrival
// reads them back with agent-scope atomic loads.  This is the release /
// acquire sequence of the AMDGPU memory model for agent scope without its
// L2 write-back and invalidate, which only non-atomic data would need.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_all_memory() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);  // vmcnt = expcnt = lgkmcnt = 0: every store acknowledged
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

}  // namespace unifur
