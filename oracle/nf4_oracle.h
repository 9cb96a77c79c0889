/*
 * nf4_oracle.h -- CPU restatement of unifur's NF4 quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the parity checker for the HIP library
 * under unifur_amd/.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker or the timed CPU
 * baseline -- never as the product path.
 *
 * Every function follows the reference crate `diffusionblocks`
 * (s-b-repo/unifur, Rust, Burn 0.21) line by line; each declaration cites
 * the file:line it restates.  Arithmetic is IEEE binary32, round to nearest
 * even per operation, no contraction (built with -ffp-contract=off), which is
 * what Rust emits for the same source.
 */
#ifndef UNIFUR_NF4_ORACLE_H
#define UNIFUR_NF4_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* BLOCK_SIZE (src/quantize.rs:36-37). */
#define NF4O_BLOCK 64

/* Copy the 16 NF4 levels (src/quantize.rs:49-66) into out[16]. */
void nf4o_levels(float out[16]);

/* nearest_level_code (src/quantize.rs:208-219): linear scan, strict `<`,
 * first index wins, NaN -> 0. */
uint8_t nf4o_nearest_level_code(float v);

/* Nf4Tensor::quantize (src/quantize.rs:99-124): one code per byte
 * (codes[n]) and one f32 absmax per 64-value block (absmax[ceil(n/64)]). */
void nf4o_quantize_sim(const float *values, size_t n, uint8_t *codes, float *absmax);

/* PackedNf4Tensor::quantize (src/quantize.rs:262-279): codes packed two per
 * byte, low nibble = even index, into packed[ceil(n/2)]. */
void nf4o_quantize_packed(const float *values, size_t n, uint8_t *packed, float *absmax);

/* Nf4Tensor::with_double_quantization (src/quantize.rs:129-149) and
 * PackedNf4Tensor::with_double_quantization (src/quantize.rs:284-309):
 * q[nb] u8 codes of absmax / max * 255 rounded half away from zero,
 * *scale_of_scales = max. */
void nf4o_double_quantize(const float *absmax, size_t nb, uint8_t *q, float *scale_of_scales);

/* Nf4Tensor::block_scale (src/quantize.rs:169-175) /
 * PackedNf4Tensor::block_scale (src/quantize.rs:341-352). */
float nf4o_dq_scale(uint8_t q, float scale_of_scales);

/* Nf4Tensor::dequantize (src/quantize.rs:178-185).  dq_codes == NULL
 * selects f32 absmax scales, else the double-quantized scales. */
void nf4o_dequantize_sim(const uint8_t *codes, size_t n, const float *absmax,
                         const uint8_t *dq_codes, float scale_of_scales, float *out);

/* PackedNf4Tensor::dequantize (src/quantize.rs:329-366). */
void nf4o_dequantize_packed(const uint8_t *packed, size_t n, const float *absmax,
                            const uint8_t *dq_codes, float scale_of_scales, float *out);

/* PackedNf4Tensor::estimated_resident_bytes (src/quantize.rs:391-399). */
size_t nf4o_estimated_resident_bytes(size_t len, int double_quantized);

/* Nf4Tensor::bits_per_value (src/quantize.rs:189-200). */
double nf4o_bits_per_value_sim(size_t len, int double_quantized);

/* PackedNf4Tensor::bits_per_value (src/quantize.rs:378-383). */
double nf4o_bits_per_value_packed(size_t len, int double_quantized);

/* transpose2d (src/qwennet.rs:1375-1390): [rows, cols] -> [cols, rows]. */
void nf4o_transpose(const float *data, size_t rows, size_t cols, float *out);

/* tensor_ext::silu (src/tensor_ext.rs:87-90): x * sigmoid(x), with the
 * logistic evaluated as 1 / (1 + exp(-x)) in f32. */
float nf4o_silu(float x);
void nf4o_silu_vec(const float *x, size_t n, float *out);

/* burn::tensor::module::linear as Nf4Linear::forward uses it
 * (src/qwennet.rs:238-241): y[r][o] = sum_i x[r][i] * w[i][o] (+ bias[o]),
 * w row-major [d_in, d_out].  f32 accumulation in increasing i, one thread:
 * the ordering is the restatement's, the reference's sgemm order is not
 * reproducible.  Used as the timed CPU baseline, not as the parity value
 * (parity compares against an f64 product of the same inputs). */
void nf4o_linear_f32(const float *x, size_t rows, const float *w, size_t d_in, size_t d_out,
                     const float *bias, float *y, int threads);

/* CPU baseline only (oracle/cpu_sgemm.c): c[m][n] = a[m][k] b[k][n], all
 * row-major, by a cache-blocked packed sgemm (6 x 16 FMA register tile, the
 * scheme of the matrixmultiply crate burn-ndarray runs on) on `threads`
 * OpenMP threads (0: the default).  Returns 0, or -1 if its packing buffers
 * cannot be allocated. */
int nf4o_sgemm_blocked(const float *a, size_t m, size_t k, const float *b, size_t n, float *c, int threads);

/* Counter-based seeded N(0, sigma^2) generator shared by tests and bench
 * inputs: element i draws two SplitMix64 outputs at counters 2i+1, 2i+2,
 * Box-Muller in f64, times sigma, rounded to f32. */
void nf4o_fill_normal(uint64_t seed, double sigma, size_t n, float *out);

/* Round f32 to bf16 (RNE) and back to f32, elementwise. */
void nf4o_round_bf16(const float *in, size_t n, float *out);

/* Checkpoint element decode (src/import.rs:255-272): binary16 bits to f32 as
 * f16_to_f32 (src/import.rs:283-317: exact; NaN payload kept, quiet bit set),
 * bfloat16 bits to f32 as bf16_to_f32 (src/import.rs:321-327). */
void nf4o_f16_to_f32(const uint16_t *in, size_t n, float *out);
void nf4o_bf16_to_f32(const uint16_t *in, size_t n, float *out);

#ifdef __cplusplus
}
#endif
#endif
