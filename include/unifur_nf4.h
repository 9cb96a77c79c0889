/*
 * unifur_nf4.h -- C ABI of the MI355X-native NF4 quantized-linear library
 * (libunifur_nf4.so, hand-written gfx950 HIP kernels).
 *
 * It replaces the NF4 path of unifur (crate `diffusionblocks`): the codec in
 * src/quantize.rs and the NF4-resident linear layers in src/qwennet.rs.  Each
 * entry point names the reference item it stands in for (file:line).  The
 * reference has no FFI for this path today (it is in-process Rust); these are
 * the symbols its FFI crate would bind.
 *
 * Conventions (all entry points):
 *   - Data buffers are DEVICE pointers owned by the caller; `stream` is a
 *     hipStream_t (NULL = the default stream).  Every call is stream-ordered:
 *     it only enqueues work and returns; results are ready when the stream
 *     has reached the call.
 *   - Return value: UNIFUR_NF4_OK (0) or a negative status; the message of the
 *     last failure on the calling thread is unifur_nf4_last_error().
 *   - The library holds no global mutable state except an optional internal
 *     workspace cache (used only when a call passes workspace == NULL) and
 *     the branch streams below, each guarded by a mutex and keyed by
 *     (device, stream).
 *   - A call may run part of its work on a library-owned branch stream
 *     (default priority), forked from `stream` and joined back into it with
 *     events before the call's last launch on `stream`: the call stays
 *     ordered on `stream`, and a graph capture of `stream` records the fork
 *     and the join.  The branch is created on the first such call outside
 *     capture; under capture without one the work stays on `stream`.
 *   - Layout of a quantized tensor of `len` values (src/quantize.rs:221-257):
 *     ceil(len/64) blocks of 64 consecutive values; `packed` holds
 *     ceil(len/2) bytes, value 2i in the low nibble of byte i; scales are one
 *     f32 absmax per block, or with double quantization one u8 code per block
 *     and one f32 scale of scales.
 *   - A linear weight is the reference's [d_in, d_out] row-major matrix
 *     (y = x W, src/qwennet.rs:2196-2211), so its 64-value blocks run along
 *     d_out.  On the device it may also be held in the column-striped
 *     layout (UNIFUR_NF4_LAYOUT_STRIPED), a byte permutation of the same
 *     codes and scales that the decode kernels stream contiguously.
 *   - Shapes past any device -- rows, d_in or d_out above 2^31-1, or an
 *     element count rows x width or d_in x d_out above 2^48 -- are refused:
 *     the workspace-size queries return UINT64_MAX for them (never a byte
 *     count that wrapped) and the calls fail with UNIFUR_NF4_ERR_INVALID.
 */
#ifndef UNIFUR_NF4_H
#define UNIFUR_NF4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* BLOCK_SIZE (src/quantize.rs:36-37). */
#define UNIFUR_NF4_BLOCK_SIZE 64

enum {
  UNIFUR_NF4_OK = 0,
  UNIFUR_NF4_ERR_INVALID = -1,     /* bad argument (null pointer, shape, dtype) */
  UNIFUR_NF4_ERR_HIP = -2,         /* a HIP runtime call or launch failed */
  UNIFUR_NF4_ERR_WORKSPACE = -3,   /* workspace smaller than required */
};

/* Element types of activations and outputs (F32, BF16), and of checkpoint
 * sources (also F16). */
enum { UNIFUR_NF4_F32 = 0, UNIFUR_NF4_BF16 = 1,
       /* checkpoint sources only (quantize_transposed, transpose_checkpoint,
        * quantize_checkpoint_linears): binary16 decoded exactly as
        * f16_to_f32, src/import.rs:283-317 */
       UNIFUR_NF4_F16 = 2 };

/* Index types of embedding lookups. */
enum { UNIFUR_NF4_IDS_I32 = 0, UNIFUR_NF4_IDS_I64 = 1 };

/* PackedScales (src/quantize.rs:221-233). */
enum { UNIFUR_NF4_SCALES_F32 = 0, UNIFUR_NF4_SCALES_DOUBLE_QUANTIZED = 1 };

typedef struct unifur_nf4_scales {
  int32_t kind;                 /* UNIFUR_NF4_SCALES_* */
  const float *absmax;          /* F32: one f32 per block */
  const uint8_t *dq_codes;      /* DOUBLE_QUANTIZED: one u8 per block */
  const float *scale_of_scales; /* DOUBLE_QUANTIZED: one f32 (device pointer) */
} unifur_nf4_scales;

/* Device layouts of a linear weight's codes and scales (d_in = K, d_out = N):
 *   ROW_MAJOR  the reference's: packed[ceil(K*N/2)] in value order, scales
 *              one per 64-value block in value order (src/quantize.rs:240-257);
 *   STRIPED    N % 64 == 0: 16-column stripe s of all K rows contiguous,
 *              packed[(s*K + k)*8 + j] = row-major packed[k*N/2 + s*8 + j], and
 *              scales block-major, scale[b*K + k] = row-major scale[k*N/64 + b].
 *              unifur_nf4_stripe_weight / unifur_nf4_unstripe_weight convert. */
enum { UNIFUR_NF4_LAYOUT_ROW_MAJOR = 0, UNIFUR_NF4_LAYOUT_STRIPED = 1 };

/* The packed weight an Nf4Linear holds (src/qwennet.rs:161-178). */
typedef struct unifur_nf4_weight {
  const uint8_t *packed;
  unifur_nf4_scales scales;
  uint64_t d_in;
  uint64_t d_out;
  int32_t layout; /* UNIFUR_NF4_LAYOUT_* */
} unifur_nf4_weight;

/* LoraAdapter factors (src/quantize.rs:556-565): a [d_in, rank] and
 * b [rank, d_out], f32 row-major; forward adds (x a) b * scaling. */
typedef struct unifur_nf4_lora {
  const float *a;
  const float *b;
  uint32_t rank;
  float scaling;
} unifur_nf4_lora;

/* Message of the calling thread's last failure ("" if none). */
const char *unifur_nf4_last_error(void);

/* ---- host-only accounting ------------------------------------------------ */

/* NF4_LEVELS (src/quantize.rs:49-66), copied into out[16]. */
int unifur_nf4_levels(float out[16]);

/* Nf4Tensor::num_blocks / PackedNf4Tensor::num_blocks (src/quantize.rs:165-167, :325-327). */
uint64_t unifur_nf4_num_blocks(uint64_t len);

/* Bytes of the packed code array, ceil(len/2) (src/quantize.rs:250-251). */
uint64_t unifur_nf4_packed_bytes(uint64_t len);

/* PackedNf4Tensor::estimated_resident_bytes (src/quantize.rs:391-399); equal to
 * resident_bytes() of a tensor of that length (src/quantize.rs:370-376). */
uint64_t unifur_nf4_estimated_resident_bytes(uint64_t len, int double_quantized);

/* PackedNf4Tensor::bits_per_value (src/quantize.rs:382-388). */
double unifur_nf4_bits_per_value(uint64_t len, int double_quantized);

/* Nf4Tensor::bits_per_value (src/quantize.rs:190-200), the simulated form. */
double unifur_nf4_simulated_bits_per_value(uint64_t len, int double_quantized);

/* ---- codec (bit-exact to the reference) ------------------------------------ */

/* PackedNf4Tensor::quantize (src/quantize.rs:262-279), which takes its codes
 * from Nf4Tensor::quantize (src/quantize.rs:99-124): per block absmax, codes
 * of v/absmax by the nearest-level scan (src/quantize.rs:208-219), packed.
 * values[len] -> packed[ceil(len/2)], absmax[ceil(len/64)]. */
int unifur_nf4_quantize(const float *values, uint64_t len, uint8_t *packed, float *absmax, void *stream);

/* PackedNf4Tensor::with_double_quantization (src/quantize.rs:284-309), same
 * formula as Nf4Tensor::with_double_quantization (src/quantize.rs:129-149):
 * absmax[num_blocks] -> dq_codes[num_blocks], *scale_of_scales (device). */
int unifur_nf4_double_quantize(const float *absmax, uint64_t num_blocks, uint8_t *dq_codes,
                               float *scale_of_scales, void *stream);

/* PackedNf4Tensor::dequantize (src/quantize.rs:355-366), bit-identical to
 * Nf4Tensor::dequantize (src/quantize.rs:178-185): out[len] =
 * NF4_LEVELS[code] * block scale, as f32 (bit-exact) or bf16 (that f32
 * rounded to nearest even). */
int unifur_nf4_dequantize(const uint8_t *packed, const unifur_nf4_scales *scales, uint64_t len, void *out,
                          int out_dtype, void *stream);

/* The simulated form's storage, Nf4Block::codes (src/quantize.rs:68-77): one
 * code per byte.  unpack_codes writes codes[len] from packed[ceil(len/2)]
 * (value i from nibble i % 2 of byte i / 2, src/quantize.rs:329-337), the
 * codes Nf4Tensor::quantize (src/quantize.rs:99-124) holds; pack_codes is
 * the pairing loop of PackedNf4Tensor::quantize (src/quantize.rs:266-273),
 * low nibble first, a zero high nibble after an odd length's last code.
 * Codes are taken modulo 16. */
int unifur_nf4_unpack_codes(const uint8_t *packed, uint64_t len, uint8_t *codes, void *stream);
int unifur_nf4_pack_codes(const uint8_t *codes, uint64_t len, uint8_t *packed, void *stream);

/* Nf4Embedding::forward (src/qwennet.rs:288-290): out[t][:] = row ids[t] of
 * the dequantized [n_embedding, d_model] table, held as one packed tensor
 * with its scales (Nf4Embedding::from_values, src/qwennet.rs:265-271); f32
 * bit-identical to the reference's dequantized table, or bf16.  Only the
 * gathered rows are dequantized (the reference dequantizes the whole table
 * per call, src/qwennet.rs:280-286).  ids: n_ids device indices, int32 or
 * int64 (UNIFUR_NF4_IDS_*); an id outside [0, n_embedding) yields a row of
 * NaN, where burn's embedding would panic. */
int unifur_nf4_embedding_forward(const uint8_t *packed, const unifur_nf4_scales *scales, uint64_t n_embedding,
                                 uint64_t d_model, const void *ids, int ids_dtype, uint64_t n_ids, void *out,
                                 int out_dtype, void *stream);

/* Loader step of qwen_linear (src/qwennet.rs:1687-1726): a checkpoint weight
 * src [out_features, in_features] row-major (PyTorch order), f32, bf16 or
 * f16 (src_dtype UNIFUR_NF4_F32 / _BF16 / _F16; bf16 and f16 decoded exactly
 * as read_tensor_f32 does, src/import.rs:255-272, :283-327), is transposed to
 * [in_features, out_features] (transpose2d, src/qwennet.rs:1375-1390) and
 * quantized (PackedNf4Tensor::quantize, src/quantize.rs:262-279) in one pass:
 * packed/absmax are bit-identical to quantizing the transposed copy.
 * out_features % 64 == 0; packed 8-byte aligned. */
int unifur_nf4_quantize_transposed(const void *src, int src_dtype, uint64_t out_features, uint64_t in_features,
                                   uint8_t *packed, float *absmax, void *stream);

/* transpose2d (src/qwennet.rs:1375-1390) of a decoded checkpoint linear:
 * dst [in_features, out_features] f32 = the transpose of src [out_features,
 * in_features] (f32, or bf16 / f16 decoded exactly, src/import.rs:255-327), for
 * weights whose out_features is not a multiple of 64 (their blocks straddle
 * the rows of the transposed buffer, so they are quantized flat after this).
 * out_features <= 65535 * 64. */
int unifur_nf4_transpose_checkpoint(const void *src, int src_dtype, uint64_t out_features, uint64_t in_features,
                                    float *dst, void *stream);

/* The quantize pass over a model's linears (QwenTrunk::to_nf4,
 * src/qwennet.rs:1185-1269, which runs Nf4Linear::from_values,
 * src/qwennet.rs:196-205 -- PackedNf4Tensor::quantize then
 * with_double_quantization, src/quantize.rs:259-309 -- on each weight in
 * turn): n row-major f32 weights values[i] [d_in[i], d_out[i]] quantized with
 * double quantization straight into the striped resident form, three
 * launches per group of up to 48 weights.  packed[i] receives
 * d_in*d_out/2 bytes of striped codes, dq_codes[i] the u8 scales
 * [d_out/64][d_in], scale_of_scales[i] one f32 (device): byte for byte what
 * unifur_nf4_quantize + unifur_nf4_double_quantize + unifur_nf4_stripe_weight
 * write for that weight.  The pointer and shape arrays are host memory;
 * d_out % 64 == 0, values 16-byte and packed 8-byte aligned.  Workspace:
 * unifur_nf4_quantize_linears_workspace_size bytes (NULL: internal). */
uint64_t unifur_nf4_quantize_linears_workspace_size(const uint64_t *d_in, const uint64_t *d_out, uint32_t n);
int unifur_nf4_quantize_linears(const float *const *values, const uint64_t *d_in, const uint64_t *d_out, uint32_t n,
                                uint8_t *const *packed, uint8_t *const *dq_codes, float *const *scale_of_scales,
                                void *workspace, uint64_t workspace_bytes, void *stream);

/* The same pass from checkpoint tensors as they lie (qwen_linear,
 * src/qwennet.rs:1687-1726, over each decoded linear of the checkpoint):
 * values[i] is the PyTorch-order [d_out[i], d_in[i]] weight in src_dtype
 * (f32, or bf16 / f16 decoded exactly as src/import.rs:255-327 does), transposed on
 * the fly (transpose2d, src/qwennet.rs:1375-1390) -- packed[i], dq_codes[i]
 * and scale_of_scales[i] are byte for byte what unifur_nf4_quantize_linears
 * writes for the transposed f32 copy.  d_out % 64 == 0, values aligned to
 * their dtype (rows of a multiple of 16 bytes take the vector loads), packed
 * 8-byte aligned.  Workspace as unifur_nf4_quantize_linears. */
int unifur_nf4_quantize_checkpoint_linears(const void *const *values, int src_dtype, const uint64_t *d_in,
                                           const uint64_t *d_out, uint32_t n, uint8_t *const *packed,
                                           uint8_t *const *dq_codes, float *const *scale_of_scales, void *workspace,
                                           uint64_t workspace_bytes, void *stream);

/* ---- device layout of a linear weight ------------------------------------------ */

/* Row-major -> striped.  src->layout must be ROW_MAJOR, d_out % 64 == 0 and
 * src->packed 8-byte aligned.  Writes ceil(d_in*d_out/2) bytes to dst_packed
 * and the per-block scales (u8 DQ codes or f32 absmax, as src->scales.kind) to
 * dst_scales; a double-quantized weight keeps its scale_of_scales.  No
 * counterpart in the reference (which has one layout); it stands in for the
 * load-time [out, in] -> [in, out] transpose of src/qwennet.rs:1375-1390 as the
 * place where the resident form is fixed. */
int unifur_nf4_stripe_weight(const unifur_nf4_weight *src, uint8_t *dst_packed, void *dst_scales, void *stream);

/* Striped -> row-major (the reference's bytes, bit for bit), the inverse. */
int unifur_nf4_unstripe_weight(const unifur_nf4_weight *src, uint8_t *dst_packed, void *dst_scales, void *stream);

/* ---- linear layers ----------------------------------------------------------- */

/* Device workspace bytes unifur_nf4_linear_forward needs for these
 * arguments.  A caller-provided workspace must be zero-filled before its
 * first use; every call leaves it ready for the next one. */
uint64_t unifur_nf4_linear_workspace_size(uint64_t rows, uint64_t d_in, uint64_t d_out, int x_dtype,
                                          uint32_t lora_rank);

/* The least workspace a call with these arguments accepts.  Batches of more
 * than 64 bf16 rows normally expand the weight (plus the LoRA update) to
 * bf16 in the workspace -- d_in * d_out * 2 bytes, plus the BLAS GEMM's
 * scratch -- and multiply with a BLAS GEMM; given a workspace smaller than
 * unifur_nf4_linear_workspace_size but at least this size, they take the
 * fused MFMA kernel instead, which dequantizes W tiles on chip and needs no
 * weight-sized scratch.  A batch of more than 2 GiB of activations is past
 * the fused kernel's reach and takes the generic path (the weight
 * dequantized to f32 in the workspace) when given less than the default
 * size.  Has no counterpart in the reference (which allocates freely); it
 * is for callers with bounded device memory. */
uint64_t unifur_nf4_linear_min_workspace_size(uint64_t rows, uint64_t d_in, uint64_t d_out, int x_dtype,
                                              uint32_t lora_rank);

/* Nf4Linear::forward (src/qwennet.rs:238-241): y = x deq(W) (+ bias), and with
 * lora != NULL QloraLinear::forward (src/qwennet.rs:325-345): base(x) +
 * (x a) b * scaling.  x [rows, d_in] (f32 or bf16), y [rows, d_out]
 * (f32 or bf16), bias [d_out] f32 or NULL.  workspace == NULL selects the
 * internal workspace cache. */
int unifur_nf4_linear_forward(const void *x, int x_dtype, uint64_t rows, const unifur_nf4_weight *w,
                              const float *bias, const unifur_nf4_lora *lora, void *y, int y_dtype,
                              void *workspace, uint64_t workspace_bytes, void *stream);

/* n <= 3 linears over one input: y[i] = x w[i] (+ bias[i]) with a shared
 * d_in -- the q, k and v projections of QwenFullAttention::forward
 * (src/qwennet.rs:927-956), each an Nf4Linear.  For decode-sized batches
 * (<= 4 rows, or 5..64 bf16 rows) over striped weights of one scale kind
 * a single kernel launch serves all of them and each activation load feeds
 * every weight; other calls run the linears in turn.  w points to n
 * weights, bias to n pointers (or is NULL; entries may be NULL), y to n
 * outputs [rows, w[i].d_out]. */
uint64_t unifur_nf4_linear_multi_workspace_size(uint64_t rows, uint64_t d_in, const uint64_t *d_out, uint32_t n,
                                                int x_dtype);
int unifur_nf4_linear_forward_multi(const void *x, int x_dtype, uint64_t rows, const unifur_nf4_weight *w,
                                    const float *const *bias, void *const *y, int y_dtype, uint32_t n,
                                    void *workspace, uint64_t workspace_bytes, void *stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): unifur_nf4_linear_forward without a workspace argument.
 * It allocates nothing -- no hipMalloc / hipFree, no allocating library
 * call -- and uses a static device scratch of 16 MiB per GPU (held until the
 * process ends).  Batches of more than 64 bf16 rows take the fused MFMA
 * kernel, never the expanded weight, with its split-K partials where they
 * fit the scratch (bit-identical to unifur_nf4_linear_forward given a 16 MiB
 * workspace; with the least workspace the fused kernel runs over whole d_in
 * and its f32 sums may differ in order).  A call whose scratch need exceeds 16 MiB fails with
 * UNIFUR_NF4_ERR_WORKSPACE and a message naming the size.  All calls on one
 * GPU share that scratch.  The library orders eager calls: a call on another
 * stream than the previous call's waits on the GPU for that call's work (an
 * event the library records after each call's launches), and calls from
 * several host threads enqueue one at a time, so overlapping calls run one
 * after the other.  Calls made under stream capture are not ordered against
 * other calls: the caller must keep a captured graph's replays from
 * overlapping other calls on the same GPU. */
int unifur_nf4_linear_forward_noalloc(const void *x, int x_dtype, uint64_t rows, const unifur_nf4_weight *w,
                                      const float *bias, const unifur_nf4_lora *lora, void *y, int y_dtype,
                                      void *stream);

/* QloraLinear::forward (src/qwennet.rs:325-345); identical to
 * unifur_nf4_linear_forward with a non-NULL lora. */
int unifur_nf4_qlora_forward(const void *x, int x_dtype, uint64_t rows, const unifur_nf4_weight *w,
                             const unifur_nf4_lora *lora, void *y, int y_dtype, void *workspace,
                             uint64_t workspace_bytes, void *stream);

/* Backward of Nf4Linear::forward / QloraLinear::forward for adapter-only
 * training (src/qwentrain.rs:421-470 runs burn's autodiff through the
 * detached dequantized weight; the packed base weight is #[module(skip)],
 * src/qwennet.rs:168-178, so it has no gradient).  Given dy [rows, d_out]
 * (f32 or bf16) and, with lora, x [rows, d_in] (f32 or bf16):
 *   dx     [rows, d_in]   = dy W^T + ((dy scaling) B^T) A^T   (dx may be NULL)
 *   grad_b [rank, d_out]  = (x A)^T (dy scaling)             (f32, may be NULL)
 *   grad_a [d_in, rank]   = x^T ((dy scaling) B^T)           (f32, may be NULL)
 * the vector-Jacobian products of LoraAdapter::forward ((x A) B scaling,
 * src/quantize.rs:619-624) and of the base product.  bf16 dy goes through
 * the weight expanded to bf16 (with the adapter merged) and a BLAS GEMM;
 * f32 dy through an f32 MFMA GEMM over the NF4 tiles dequantized exactly on
 * chip, W's rows as its outputs and the adapter term in its epilogue (no
 * weight copy; shapes it does not take use an f32 dequantized copy of the
 * weight).  The adapter gradients are
 * summed over the rows in a fixed order (deterministic); when dx takes the
 * BLAS path they run on the branch stream beside its GEMM.
 * A workspace smaller than the default size but at least the minimum size
 * below selects, for a striped weight with bf16 dy, d_in a multiple of 128
 * and 16-byte aligned dy and dx, the fused NF4 MFMA kernel for dx: W's rows
 * are its outputs and each W tile is dequantized on chip, so the only
 * scratch is the adapter's bf16 operands (dx gains ((dy scaling) B^T) A^T
 * in the kernel's epilogue, the adapter unmerged); for other layouts
 * (layout is the weight's UNIFUR_NF4_LAYOUT_*) and shapes the minimum is the
 * default size. */
uint64_t unifur_nf4_linear_backward_workspace_size(uint64_t rows, uint64_t d_in, uint64_t d_out, int dy_dtype,
                                                   uint32_t lora_rank);
uint64_t unifur_nf4_linear_backward_min_workspace_size(uint64_t rows, uint64_t d_in, uint64_t d_out, int dy_dtype,
                                                       uint32_t lora_rank, int layout);
int unifur_nf4_linear_backward(const void *dy, int dy_dtype, uint64_t rows, const unifur_nf4_weight *w,
                               const unifur_nf4_lora *lora, const void *x, int x_dtype, void *dx, int dx_dtype,
                               float *grad_a, float *grad_b, void *workspace, uint64_t workspace_bytes,
                               void *stream);

/* Linear with an f32-resident weight w [d_in, d_out] row-major: the F32 arm of
 * QwenLinear (src/qwennet.rs:293-355) and the dequantized base of the
 * simulated QLoraLinear (src/quantize.rs:637-700); y = x w (+ bias)
 * (+ (x a) b * scaling).  Same conventions as unifur_nf4_linear_forward. */
uint64_t unifur_nf4_dense_linear_workspace_size(uint64_t rows, uint32_t lora_rank);
int unifur_nf4_dense_linear_forward(const void *x, int x_dtype, uint64_t rows, const float *w, uint64_t d_in,
                                    uint64_t d_out, const float *bias, const unifur_nf4_lora *lora, void *y,
                                    int y_dtype, void *workspace, uint64_t workspace_bytes, void *stream);

/* QLoraLinear::merged (src/quantize.rs:716-726): out = w + (a b) * scaling,
 * LoraAdapter::delta_weight (src/quantize.rs:626-634) folded into an f32
 * weight [d_in, d_out]. */
int unifur_nf4_lora_merge(const float *w, uint64_t d_in, uint64_t d_out, const unifur_nf4_lora *lora, float *out,
                          void *stream);

/* Workspace bytes of unifur_nf4_swiglu_forward (same contract as above). */
uint64_t unifur_nf4_swiglu_workspace_size(uint64_t rows, uint64_t hidden, uint64_t intermediate, int x_dtype);
/* The least workspace unifur_nf4_swiglu_forward accepts (the fused MFMA
 * kernels for more than 64 bf16 rows; see unifur_nf4_linear_min_workspace_size). */
uint64_t unifur_nf4_swiglu_min_workspace_size(uint64_t rows, uint64_t hidden, uint64_t intermediate, int x_dtype);

/* QwenMlp::forward (src/qwennet.rs:816-819): y = down(silu(gate x) * up x),
 * silu(z) = z * sigmoid(z) (src/tensor_ext.rs:87-90).  gate and up are
 * [hidden, intermediate], down is [intermediate, hidden]; x [rows, hidden],
 * y [rows, hidden]. */
int unifur_nf4_swiglu_forward(const void *x, int x_dtype, uint64_t rows, const unifur_nf4_weight *gate,
                              const unifur_nf4_weight *up, const unifur_nf4_weight *down, void *y, int y_dtype,
                              void *workspace, uint64_t workspace_bytes, void *stream);

/* ---- decoder-layer decode ------------------------------------------------ */

/* The NF4 projections and norms of one decoder layer with a full-attention
 * mixer: QwenDecoderLayer (src/qwennet.rs:1064-1129) whose QwenFullAttention
 * (src/qwennet.rs:856-956, attn_output_gate = false) and QwenMlp
 * (src/qwennet.rs:786-820) hold Nf4Linear projections.  q, k, v, gate and up
 * are [hidden, *], o is [q.d_out, hidden], down [gate.d_out, hidden].
 * input_norm and post_norm are the QwenRmsNorm weights [hidden] (f32, applied
 * as w + 1, src/qwennet.rs:104-109) with epsilon eps. */
typedef struct unifur_nf4_decoder_layer {
  unifur_nf4_weight q, k, v, o;
  unifur_nf4_weight gate, up, down;
  const float *input_norm;
  const float *post_norm;
  float eps;
} unifur_nf4_decoder_layer;

/* QwenDecoderLayer::step up to the attention (src/qwennet.rs:1112-1121 with
 * QwenFullAttention::project, :927-951): n = input_norm(x), then
 * q = n Wq, k = n Wk, v = n Wv -- before the per-head norms, rotary and the
 * attention itself, which stay with the caller.  x [rows, hidden]; q, k, v
 * [rows, d_out of their weight]; all of dtype.  Decode batches (<= 4 rows)
 * over striped weights of one scale kind take one launch with the norm
 * folded in, and so do 5..64 bf16 (5..32 f32) rows over striped weights with
 * double-quantized scales and a 16-byte aligned x; other calls norm x into
 * the workspace first.  The workspace size covers those other calls. */
uint64_t unifur_nf4_decoder_attn_in_workspace_size(uint64_t rows, const unifur_nf4_decoder_layer *layer, int dtype);
int unifur_nf4_decoder_attn_in(const void *x, int dtype, uint64_t rows, const unifur_nf4_decoder_layer *layer,
                               void *q, void *k, void *v, void *workspace, uint64_t workspace_bytes, void *stream);

/* QwenDecoderLayer::step after the attention (src/qwennet.rs:1122-1128):
 * x1 = x + ctx Wo, then y = x1 + down(silu(gate(n)) * up(n)) with
 * n = post_norm(x1).  x, y [rows, hidden]; ctx [rows, o.d_in] (the merged
 * attention heads); all of dtype; y may be x.  Decode batches over striped
 * weights add the residuals in the projections' epilogues and fold the norm
 * into the gate/up launch (up to 4 rows; 5..64 bf16 or 5..32 f32 rows with
 * double-quantized scales), else norm x1 once first. */
uint64_t unifur_nf4_decoder_attn_out_mlp_workspace_size(uint64_t rows, const unifur_nf4_decoder_layer *layer,
                                                        int dtype);
int unifur_nf4_decoder_attn_out_mlp(const void *x, const void *ctx, int dtype, uint64_t rows,
                                    const unifur_nf4_decoder_layer *layer, void *y, void *workspace,
                                    uint64_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* UNIFUR_NF4_H */
