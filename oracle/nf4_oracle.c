/*
 * nf4_oracle.c -- CPU restatement of unifur's NF4 quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and timed CPU baseline); the
 * product path is the HIP library under unifur_amd/ and never calls this.
 *
 * Pinning status of each function (how tests/test_oracle.py checks it):
 *   nf4o_levels              published codebook known-answer test
 *                            (src/quantize.rs:839-866) + sortedness/zero
 *   nf4o_nearest_level_code  brute force vs exact real-arithmetic nearest
 *                            level, thresholds within 1 ulp of midpoints,
 *                            exact threshold table re-derived by bisection
 *   nf4o_quantize_*          reference known-answer tests (grid values,
 *                            absmax endpoint, zero blocks, ragged block,
 *                            error bound, on-grid) + golden fixtures from an
 *                            independent numpy restatement
 *   nf4o_double_quantize     closed forms (max block -> 255, zero tensor,
 *                            idempotence, half-away-from-zero tie) + fixtures
 *   nf4o_dequantize_*        packed == simulated bit-identity
 *                            (src/quantize.rs:755-791) + fixtures
 *   nf4o_*resident*, bits    residency known-answer test (src/quantize.rs:793-822)
 *   nf4o_linear_f32          orientation known-answer test
 *                            (src/qwennet.rs:2196-2211) + f64 product
 *   nf4o_silu                closed-form limits and an f64 evaluation
 *   nf4o_transpose           involution and index identity
 *   nf4o_fill_normal         determinism and moments (input generator only)
 *   nf4o_f16_to_f32          all 65536 bit patterns: IEEE widening (numpy) for
 *                            every non-NaN, subnormals against mant * 2^-24 in
 *                            f64, NaNs with the quiet bit forced, known answers
 *   nf4o_bf16_to_f32         all 65536 bit patterns against bits << 16
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp).
 */
#include "nf4_oracle.h"

#include <math.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* NF4_LEVELS (src/quantize.rs:49-66), written as the same decimal literals
 * the reference uses so the f32 rounding is the compiler's, as in Rust. */
static const float LEVELS[16] = {
    -1.0f,
    -0.6961928f,
    -0.52507305f,
    -0.3949175f,
    -0.28444138f,
    -0.18477343f,
    -0.091050036f,
    0.0f,
    0.0795803f,
    0.1609302f,
    0.2461123f,
    0.33791524f,
    0.44070983f,
    0.562617f,
    0.72295684f,
    1.0f,
};

void nf4o_levels(float out[16]) { memcpy(out, LEVELS, sizeof(LEVELS)); }

/* Rust f32::max: if one operand is NaN the other is returned (IEEE maxNum). */
static float rust_max(float a, float b) { return fmaxf(a, b); }

uint8_t nf4o_nearest_level_code(float v) {
    /* src/quantize.rs:208-219 */
    size_t best = 0;
    float best_dist = INFINITY;
    for (size_t i = 0; i < 16; ++i) {
        float d = fabsf(v - LEVELS[i]);
        if (d < best_dist) {
            best_dist = d;
            best = i;
        }
    }
    return (uint8_t)best;
}

void nf4o_quantize_sim(const float *values, size_t n, uint8_t *codes, float *absmax) {
    /* src/quantize.rs:99-124: chunks of BLOCK_SIZE, absmax = fold(0, max(acc, |v|)),
     * code = scan(0) for an all-zero block, else scan(v / absmax). */
    size_t nb = (n + NF4O_BLOCK - 1) / NF4O_BLOCK;
    for (size_t b = 0; b < nb; ++b) {
        size_t start = b * NF4O_BLOCK;
        size_t end = start + NF4O_BLOCK < n ? start + NF4O_BLOCK : n;
        float amax = 0.0f;
        for (size_t i = start; i < end; ++i) amax = rust_max(amax, fabsf(values[i]));
        for (size_t i = start; i < end; ++i)
            codes[i] = amax == 0.0f ? nf4o_nearest_level_code(0.0f)
                                    : nf4o_nearest_level_code(values[i] / amax);
        absmax[b] = amax;
    }
}

void nf4o_quantize_packed(const float *values, size_t n, uint8_t *packed, float *absmax) {
    /* src/quantize.rs:262-279: codes from the simulated quantizer, packed per
     * block in pairs, low nibble first; an odd tail leaves the high nibble 0.
     * Blocks hold an even count except the last, so byte k = codes[2k..2k+1]. */
    size_t nb = (n + NF4O_BLOCK - 1) / NF4O_BLOCK;
    uint8_t block_codes[NF4O_BLOCK];
    size_t out = 0;
    for (size_t b = 0; b < nb; ++b) {
        size_t start = b * NF4O_BLOCK;
        size_t len = start + NF4O_BLOCK < n ? NF4O_BLOCK : n - start;
        nf4o_quantize_sim(values + start, len, block_codes, &absmax[b]);
        for (size_t p = 0; p < len; p += 2) {
            uint8_t low = block_codes[p];
            uint8_t high = p + 1 < len ? block_codes[p + 1] : 0;
            packed[out++] = (uint8_t)(low | (high << 4));
        }
    }
}

void nf4o_double_quantize(const float *absmax, size_t nb, uint8_t *q, float *scale_of_scales) {
    /* src/quantize.rs:284-309 (= :129-149 on the same values). */
    float max_scale = 0.0f;
    for (size_t b = 0; b < nb; ++b) max_scale = rust_max(max_scale, absmax[b]);
    for (size_t b = 0; b < nb; ++b) {
        if (max_scale == 0.0f) {
            q[b] = 0;
            continue;
        }
        /* (s / max_scale * 255.0).round().clamp(0.0, 255.0) as u8:
         * two f32 RN ops, round half away from zero, clamp keeps NaN,
         * `as u8` saturates and maps NaN to 0. */
        float r = roundf((absmax[b] / max_scale) * 255.0f);
        if (r != r) {
            q[b] = 0;
        } else {
            if (r < 0.0f) r = 0.0f;
            if (r > 255.0f) r = 255.0f;
            q[b] = (uint8_t)r;
        }
    }
    *scale_of_scales = max_scale;
}

float nf4o_dq_scale(uint8_t q, float scale_of_scales) {
    /* codes[i] as f32 / 255.0 * scale_of_scales (src/quantize.rs:173, :349) */
    return ((float)q / 255.0f) * scale_of_scales;
}

static float block_scale(size_t b, const float *absmax, const uint8_t *dq_codes, float sos) {
    return dq_codes ? nf4o_dq_scale(dq_codes[b], sos) : absmax[b];
}

void nf4o_dequantize_sim(const uint8_t *codes, size_t n, const float *absmax,
                         const uint8_t *dq_codes, float scale_of_scales, float *out) {
    /* src/quantize.rs:178-185 */
    size_t nb = (n + NF4O_BLOCK - 1) / NF4O_BLOCK;
    for (size_t b = 0; b < nb; ++b) {
        float scale = block_scale(b, absmax, dq_codes, scale_of_scales);
        size_t start = b * NF4O_BLOCK;
        size_t end = start + NF4O_BLOCK < n ? start + NF4O_BLOCK : n;
        for (size_t i = start; i < end; ++i) out[i] = LEVELS[codes[i]] * scale;
    }
}

void nf4o_dequantize_packed(const uint8_t *packed, size_t n, const float *absmax,
                            const uint8_t *dq_codes, float scale_of_scales, float *out) {
    /* src/quantize.rs:329-337 (code), :355-366 (dequantize) */
    size_t nb = (n + NF4O_BLOCK - 1) / NF4O_BLOCK;
    for (size_t b = 0; b < nb; ++b) {
        float scale = block_scale(b, absmax, dq_codes, scale_of_scales);
        size_t start = b * NF4O_BLOCK;
        size_t end = start + NF4O_BLOCK < n ? start + NF4O_BLOCK : n;
        for (size_t i = start; i < end; ++i) {
            uint8_t byte = packed[i / 2];
            uint8_t code = (i % 2 == 0) ? (byte & 0x0F) : (byte >> 4);
            out[i] = LEVELS[code] * scale;
        }
    }
}

size_t nf4o_estimated_resident_bytes(size_t len, int double_quantized) {
    /* src/quantize.rs:391-399 */
    size_t blocks = (len + NF4O_BLOCK - 1) / NF4O_BLOCK;
    size_t scale_bytes = double_quantized ? blocks + 4 : 4 * blocks;
    return (len + 1) / 2 + scale_bytes;
}

double nf4o_bits_per_value_sim(size_t len, int double_quantized) {
    /* src/quantize.rs:189-200 */
    if (len == 0) return 0.0;
    double blocks = (double)((len + NF4O_BLOCK - 1) / NF4O_BLOCK);
    double payload = 4.0 * (double)len;
    double scales = double_quantized ? 8.0 * blocks + 32.0 : 32.0 * blocks;
    return (payload + scales) / (double)len;
}

double nf4o_bits_per_value_packed(size_t len, int double_quantized) {
    /* src/quantize.rs:378-383 */
    if (len == 0) return 0.0;
    return 8.0 * (double)nf4o_estimated_resident_bytes(len, double_quantized) / (double)len;
}

void nf4o_transpose(const float *data, size_t rows, size_t cols, float *out) {
    /* src/qwennet.rs:1375-1390, 64x64 tiles */
    const size_t B = 64;
    for (size_t r0 = 0; r0 < rows; r0 += B) {
        size_t rend = r0 + B < rows ? r0 + B : rows;
        for (size_t c0 = 0; c0 < cols; c0 += B) {
            size_t cend = c0 + B < cols ? c0 + B : cols;
            for (size_t r = r0; r < rend; ++r)
                for (size_t c = c0; c < cend; ++c) out[c * rows + r] = data[r * cols + c];
        }
    }
}

float nf4o_silu(float x) {
    /* src/tensor_ext.rs:87-90 */
    float s = 1.0f / (1.0f + expf(-x));
    return x * s;
}

void nf4o_silu_vec(const float *x, size_t n, float *out) {
    for (size_t i = 0; i < n; ++i) out[i] = nf4o_silu(x[i]);
}

void nf4o_linear_f32(const float *x, size_t rows, const float *w, size_t d_in, size_t d_out,
                     const float *bias, float *y, int threads) {
    /* src/qwennet.rs:238-241 -> burn linear: y = x W (+ b), W [d_in, d_out].
     * Columns are split over threads; each thread walks i in order. */
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
    const size_t CB = 256;
    size_t nchunks = (d_out + CB - 1) / CB;
#pragma omp parallel for collapse(2) schedule(static)
    for (size_t r = 0; r < rows; ++r) {
        for (size_t ch = 0; ch < nchunks; ++ch) {
            size_t o0 = ch * CB;
            size_t o1 = o0 + CB < d_out ? o0 + CB : d_out;
            float acc[256];
            for (size_t o = o0; o < o1; ++o) acc[o - o0] = 0.0f;
            const float *xr = x + r * d_in;
            for (size_t i = 0; i < d_in; ++i) {
                float xi = xr[i];
                const float *wr = w + i * d_out;
                for (size_t o = o0; o < o1; ++o) acc[o - o0] += xi * wr[o];
            }
            for (size_t o = o0; o < o1; ++o)
                y[r * d_out + o] = bias ? acc[o - o0] + bias[o] : acc[o - o0];
        }
    }
}

static uint64_t splitmix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

void nf4o_fill_normal(uint64_t seed, double sigma, size_t n, float *out) {
    const uint64_t gamma = 0x9E3779B97F4A7C15ULL;
    const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) {
        uint64_t a = splitmix64(seed + (2 * (uint64_t)i + 1) * gamma);
        uint64_t b = splitmix64(seed + (2 * (uint64_t)i + 2) * gamma);
        double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0); /* (0, 1] */
        double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);         /* [0, 1) */
        double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
        out[i] = (float)(z * sigma);
    }
}

/* Checkpoint element decode (read_tensor_f32, src/import.rs:243-280): f16
 * bits to f32 as f16_to_f32 (src/import.rs:283-317) -- zero kept signed, a
 * subnormal renormalised by the same shift loop, infinity kept, a NaN's
 * payload moved up 13 bits with the quiet bit forced -- and bf16 bits to f32
 * as bf16_to_f32 (src/import.rs:321-327): the top 16 bits. */
void nf4o_f16_to_f32(const uint16_t *in, size_t n, float *out) {
    for (size_t i = 0; i < n; ++i) {
        const uint32_t bits = in[i];
        const uint32_t sign = (bits >> 15) & 1u, exp = (bits >> 10) & 0x1fu, mant = bits & 0x3ffu;
        uint32_t o;
        if (exp == 0) {
            if (mant == 0) {
                o = sign << 31;
            } else {
                uint32_t m = mant, e = 127u - 14u;
                while ((m & 0x400u) == 0) {
                    m <<= 1;
                    e -= 1u;
                }
                m &= 0x3ffu;
                o = (sign << 31) | (e << 23) | (m << 13);
            }
        } else if (exp == 0x1fu) {
            const uint32_t payload = mant == 0 ? 0u : (((mant << 13) | 0x00400000u) & 0x007fffffu);
            o = (sign << 31) | (0xffu << 23) | payload;
        } else {
            o = (sign << 31) | ((exp + (127u - 15u)) << 23) | (mant << 13);
        }
        memcpy(&out[i], &o, 4);
    }
}

void nf4o_bf16_to_f32(const uint16_t *in, size_t n, float *out) {
    for (size_t i = 0; i < n; ++i) {
        const uint32_t o = (uint32_t)in[i] << 16;
        memcpy(&out[i], &o, 4);
    }
}

void nf4o_round_bf16(const float *in, size_t n, float *out) {
    for (size_t i = 0; i < n; ++i) {
        uint32_t u;
        memcpy(&u, &in[i], 4);
        if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) {
            u |= 0x00400000u; /* quiet NaN stays NaN */
        } else {
            u += 0x7FFFu + ((u >> 16) & 1u);
        }
        u &= 0xFFFF0000u;
        memcpy(&out[i], &u, 4);
    }
}
