/*
 * eredu_hip.h -- C ABI of the MI355X (gfx950) quantized-linear library.
 *
 * Drop-in boundary for the reference's quantized-linear hot path.  Every entry
 * point:
 *   - takes device pointers that it borrows (never frees, never retains),
 *   - enqueues its kernels on `stream` (NULL = the device's null stream) and
 *     returns without synchronising, like MLX's lazy evaluation hands work to
 *     its stream,
 *   - returns 0 on success and non-zero on failure, with a message readable
 *     from eq_last_error() on the calling thread (the mlx-c convention:
 *     safemlx-sys/src/mlx-c/mlx/c/ops.cpp:2585-2617 returns 0/1 and the message
 *     goes to a thread-local slot, safemlx/src/error.rs:239-269).
 * Arguments are validated before anything is launched; a rejected call
 * launches nothing.
 */
#ifndef EREDU_HIP_H
#define EREDU_HIP_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t without pulling HIP headers into C/FFI callers. */
typedef struct ihipStream_t* eq_stream_t;

/* Element types of activations, scales/biases and dense outputs. */
enum eq_dtype { EQ_DTYPE_F32 = 0, EQ_DTYPE_F16 = 1, EQ_DTYPE_BF16 = 2, EQ_DTYPE_U8 = 3 /* MXFP4 scales */ };

/* GGML block types handled on the device (codes of eredu-gguf/src/format.rs:297-330). */
enum eq_ggml_type {
    EQ_GGML_Q4_0 = 2, EQ_GGML_Q4_1 = 3, EQ_GGML_Q5_0 = 6, EQ_GGML_Q5_1 = 7, EQ_GGML_Q8_0 = 8,
    EQ_GGML_Q2_K = 10, EQ_GGML_Q3_K = 11, EQ_GGML_Q4_K = 12, EQ_GGML_Q5_K = 13, EQ_GGML_Q6_K = 14,
    EQ_GGML_IQ4_NL = 20, EQ_GGML_IQ4_XS = 23 /* dequantize and native linear only: no affine form */
};

/* Byte order of multi-byte block fields (eredu-gguf/src/format.rs:5-23 Endian). */
enum eq_endian { EQ_ENDIAN_LITTLE = 0, EQ_ENDIAN_BIG = 1 };

/* Which dense-dequant definition to follow for GGML blocks:
 * AFFINE = convert_affine then AffineTensor::dequantize (eredu-gguf/src/convert.rs:43-56,81-101);
 * NATIVE = the checkpoint-native decoders (safemlx/src/native_quantization.rs:3445-3469,
 * 3499-3509,3539-3542), the affine route for types without one (Q5_K and Q6_K dequantize
 * through IQuantTensor::dequantize_f32, native_quantization.rs:792-830).
 * The two differ only for Q4_K (f16 rounding of d*sc and -dmin*m) and for Q8_0 when
 * -128 d overflows f16. */
enum eq_dequant_definition { EQ_DEQUANT_AFFINE = 0, EQ_DEQUANT_NATIVE = 1 };

/* Message of the last failed call on this thread ("" if none). */
const char* eq_last_error(void);

/* Library ABI version (major * 100 + minor). */
int eq_version(void);

/*
 * Group-wise quantized matmul (affine or MXFP4).
 * Replaces mlx_quantized_matmul (safemlx-sys/src/mlx-c/mlx/c/ops.h:809-819) as
 * called by safemlx::ops::quantized_matmul_with_mode
 * (safemlx/src/ops/quantization.rs:190-226).
 *
 *   transpose = true : w is [N, K*bits/32] u32 (rows of W packed along K),
 *                      scales/biases [N, K/group_size];  y = x . W^T
 *   transpose = false: w is [K, N*bits/32] u32 (packed along N),
 *                      scales/biases [K, N/group_size];  y = x . W
 *   W[r, c] = scale[r, c/gs] * q[r, c] + bias[r, c/gs], q read LSB-first from
 *   the u32 words (eredu-gguf/src/convert.rs:87-99,413-427).
 * x is [M, K] of x_dtype (leading batch dims flattened into M), y is [M, N] of
 * x_dtype.  biases may be NULL (treated as zero).  mode "affine" (or NULL):
 * bits in {2, 3, 4, 5, 6, 8} (3/5/6-bit codes form an LSB-first bit stream
 * and may straddle words; a packed row holds whole words); group_size 16 or a
 * positive multiple of 32 (eredu-checkpoint/src/lib.rs:103-122).
 * mode "mxfp4" (safemlx/src/ops/quantization.rs:16-46): group_size 32, bits
 * 4, scale_dtype EQ_DTYPE_U8 (E8M0 bytes, 2^(e - 127), 255 = NaN), biases
 * NULL; W[r, c] = 2^(e[r, c/32] - 127) * e2m1(q[r, c]) with the E2M1 code
 * bit 3 = sign, magnitudes 0, .5, 1, 1.5, 2, 3, 4, 6.
 * Accumulation is f32.  Calls the matrix-core prefill kernel takes (M > 16,
 * or fewer rows than that which the decode kernel would multiply in several
 * passes over the weights) may split K through f32 partials in the library
 * workspace of `stream`, which cannot grow while `stream` is capturing: such
 * a capture fails with a message until one eager call of that shape has run
 * on the stream (it never records another plan than the eager call's).
 */
int eq_quantized_matmul(void* y, const void* x, const uint32_t* w, const void* scales,
                        const void* biases, int64_t M, int64_t N, int64_t K, bool transpose,
                        int group_size, int bits, const char* mode, int x_dtype,
                        int scale_dtype, eq_stream_t stream);

/* One problem of a grouped quantized matmul: y[M, N] = x[M, K] . W^T (or . W). */
typedef struct eq_qmm_problem {
    void* y;
    const void* x;
    const uint32_t* w;
    const void* scales;
    const void* biases; /* may be NULL */
    int64_t N;
    int64_t K;
} eq_qmm_problem;

/*
 * Grouped quantized matmul: `count` independent problems that share M,
 * transpose, group_size, bits, mode and dtypes, with the results of `count`
 * eq_quantized_matmul calls (bit for bit: each problem runs the same kernel
 * code either way).  Decode-shaped groups (transpose, 16-bit x, 4/8-bit
 * codes, M <= 16 rows that one pass of the decode kernel multiplies: 8 at
 * 4-bit group 64, 16 at 8-bit group 64, 4 at group 32) run as one persistent
 * launch per 8 problems, which streams the weights of all of them back to
 * back instead of paying a kernel launch per projection; rows that would
 * take the decode kernel several passes go, as in eq_quantized_matmul, to
 * the prefill kernel one problem at a time.
 * No single counterpart in the reference's C ABI: it stands for the
 * consecutive mlx_quantized_matmul calls (safemlx-sys/src/mlx-c/mlx/c/ops.h:809-819)
 * that a decoder layer issues on one input, e.g. the q/k/v projections of
 * eredu-architectures/src/llama.rs:272-295 or the gate/up pair of :414-423.
 */
int eq_quantized_matmul_batched(const eq_qmm_problem* problems, int count, int64_t M, bool transpose,
                                int group_size, int bits, const char* mode, int x_dtype, int scale_dtype,
                                eq_stream_t stream);

/*
 * Affine dequantize: out[r, c] = scale[r, c/gs] * q[r, c] + bias[r, c/gs],
 * computed in f32 (one multiply, one add) and written as out_dtype; "mxfp4":
 * out[r, c] = 2^(e[r, c/32] - 127) * e2m1(q[r, c]) (scale_dtype EQ_DTYPE_U8,
 * biases NULL).
 * Replaces mlx_dequantize (safemlx-sys/src/mlx-c/mlx/c/ops.h:359-369) as called
 * by safemlx::ops::dequantize_with_mode (safemlx/src/ops/quantization.rs:256-289).
 * w is [rows, cols*bits/32] u32; scales/biases [rows, cols/gs]; biases may be NULL.
 */
int eq_dequantize(void* out, const uint32_t* w, const void* scales, const void* biases,
                  int64_t rows, int64_t cols, int group_size, int bits, const char* mode,
                  int scale_dtype, int out_dtype, eq_stream_t stream);

/*
 * GGML blocks -> MLX affine (u32 codes, f16 scale bits, f16 bias bits),
 * byte-identical to eredu_gguf::convert_affine (eredu-gguf/src/convert.rs:318-564)
 * with (bits, group size) of convert.rs:142-152: Q2_K (2, 16), Q3_K (3, 16),
 * Q4_0 / Q4_1 / Q4_K (4, 32), Q5_0 / Q5_1 / Q5_K (5, 32), Q6_K (6, 16),
 * Q8_0 (8, 32).  `rows` x `cols` is the MLX shape (GGUF dims reversed,
 * format.rs:449-452); cols is a multiple of the block length (32, or 256 for
 * the K types); raw holds rows*cols/block_values blocks (raw_len bytes,
 * checked like convert.rs:319-324).  Outputs: weights [rows, cols*bits/32],
 * scales/biases [rows, cols/group_size].
 */
int eq_gguf_convert_affine(uint32_t* weights, uint16_t* scales, uint16_t* biases,
                           const uint8_t* raw, int64_t raw_len, int ggml_type, int64_t rows,
                           int64_t cols, int endian, eq_stream_t stream);

/*
 * GGML type 39 (MXFP4) blocks of a [rows, cols] tensor -> MLX's MXFP4 pair:
 * weights [rows, cols / 8] u32 (E2M1 codes, 8 per word LSB-first) and scales
 * [rows, cols / 32] E8M0 bytes.  A block is the scale byte and 16 code bytes
 * (low nibbles values 0..15, high nibbles 16..31); no value changes.
 * Replaces the MXFP4 branch of eredu_gguf::convert (eredu-gguf/src/convert.rs:
 * 241, 247-276).  cols must be a multiple of 32, raw_len = rows * cols / 32 * 17.
 */
int eq_gguf_convert_mxfp4(uint32_t* weights, uint8_t* scales, const uint8_t* raw, int64_t raw_len, int64_t rows,
                          int64_t cols, eq_stream_t stream);

/*
 * GGML blocks -> dense [rows, cols] of out_dtype (EQ_DTYPE_BF16 or EQ_DTYPE_F32),
 * following `definition` (eq_dequant_definition; IQ4_NL / IQ4_XS have one
 * definition, factor * level, eredu-gguf/src/iquant.rs:271-301).  bf16 output
 * is the round-to-nearest-even image of the reference's f32 result.
 * Replaces IQuantTensor::dequantize_f32 (eredu-gguf/src/convert.rs:43-56) and
 * NativeQuantizedTensor::dequantize's CPU decoders
 * (safemlx/src/native_quantization.rs:3417-3542).
 */
int eq_gguf_dequantize(void* out, const uint8_t* raw, int64_t raw_len, int ggml_type,
                       int64_t rows, int64_t cols, int endian, int definition, int out_dtype,
                       eq_stream_t stream);

/*
 * Native GGUF embedding: out[t, :] = row tokens[t] of the [rows, cols] GGUF
 * tensor (raw blocks as stored, raw_len bytes) decoded by the native
 * definition (as eq_gguf_dequantize with EQ_DEQUANT_NATIVE), as out_dtype
 * (EQ_DTYPE_F32, the reference's output, or EQ_DTYPE_BF16, its
 * round-to-nearest-even image).  tokens: n_tokens device int32 ids; an id
 * outside [0, rows) gives a row of +0 (the ids are not read on the host).
 * The picked rows' blocks are copied into the library's per-stream
 * workspace (n_tokens * row bytes; the first call on a stream may allocate)
 * and decoded there.  out 16-byte aligned.  Replaces
 * NativeQuantizedTensor::embedding (safemlx/src/native_quantization.rs:
 * 774-789; its CPU streaming path :915-939 with decode_native_row :948-996,
 * whose out-of-range id is an error).
 */
int eq_gguf_embedding(void* out, const uint8_t* raw, int64_t raw_len, int ggml_type, int64_t rows, int64_t cols,
                      const int32_t* tokens, int64_t n_tokens, int endian, int out_dtype, eq_stream_t stream);

/*
 * Native GGUF grouped linear (mixture-of-experts): y[r, :] = x[r, :] . W[ids[r]]^T
 * for r < routes, with W an expert bank [experts, N, K] of Q4_K, Q5_K, Q6_K,
 * Q5_1, Q8_0, IQ4_NL or IQ4_XS blocks as stored (raw_len bytes, experts * N
 * rows of K values); x [routes, K] and y [routes, N] bf16; ids device int32,
 * an id outside [0, experts) gives a row of +0.  Up to 16 routes: one
 * launch of eq_gguf_linear's M = 1 kernels for all routes, each route's
 * expert matrix picked on the device from ids (native definition, f32
 * factors).
 * More routes (N % 128 == 0, K % 64 == 0): the whole bank is re-packed into
 * the workspace as eq_gguf_linear's prefill does and the routes run as one
 * gathered product (sorted_ids: ascending ids promised, the grouped
 * matrix-core kernel; unsorted ids under the promise give wrong rows but
 * stay in bounds).  The re-packed bank takes experts * N * (K * b / 8 +
 * 4 * K / gs) bytes of the stream's workspace (b = 4 for Q4_K, 8 for the
 * others; gs = 32, or 16 for Q6_K), every expert whether ids reference it or
 * not, plus routes * K * 2 bytes of gathered rows; the workspace only grows
 * and is kept until the process ends, so one call on a wide bank holds that
 * memory for the process's lifetime.  Replaces native_grouped_linear (safemlx/src/native_quantization.rs:
 * 1039-1072; its CPU loop :1002-1037) as eredu's MoE calls it
 * (eredu/src/backend/mlx/nn/moe.rs:1080-1092).  x 16-byte, y 8-byte aligned, a
 * Q4_K bank 16-byte aligned.
 */
int eq_gguf_grouped_linear(void* y, const void* x, const uint8_t* raw, int64_t raw_len, int ggml_type,
                           int64_t experts, int64_t N, int64_t K, const int32_t* ids, int64_t routes, int endian,
                           int x_dtype, bool sorted_ids, eq_stream_t stream);

/*
 * Native GGUF linear: y[M, N] = x[M, K] . W^T with W the GGUF tensor (MLX
 * shape [N, K], raw Q4_K, Q5_K, Q6_K, Q5_1, Q8_0, IQ4_NL or IQ4_XS blocks as stored, raw_len
 * bytes) decoded by the native definition (Q4_K: d*sc*q - dmin*m, Q5_K the
 * same with 5-bit q, Q6_K: d*sc*(q - 32), Q5_1: d*q + m, Q8_0: d*q, IQ4_NL /
 * IQ4_XS: factor*level; factors in f32, not rounded to f16) without an
 * affine expansion; f32 accumulation,
 * bf16 x and y.  Replaces NativeQuantizedTensor::linear with transpose = true
 * (safemlx/src/native_quantization.rs:741-772; its Metal kernels for these
 * formats at :1320-1400,1856), whose CUDA/CPU builds decode on the host
 * (:846-913).  x 16-byte aligned; a Q4_K payload 16-byte aligned.
 * Above 8 activation rows (prefill) the blocks are re-packed per call, in
 * slices of at most 128 MiB held in the library's per-stream workspace, to the
 * affine triple (f16 scale and bias; IQ4: levels as bytes with an f16
 * factor) and multiplied on the bf16 matrix cores, weights dequantized to
 * bf16 as MLX's quantized matmul does; the first such call on a stream may
 * allocate that workspace.
 */
int eq_gguf_linear(void* y, const void* x, const uint8_t* raw, int64_t raw_len, int ggml_type, int64_t M,
                   int64_t N, int64_t K, int endian, int x_dtype, eq_stream_t stream);

/*
 * Gathered quantized matmul (routed experts): for b in [0, batch),
 *   y[b] = x[lhs[b]] . dequant(w[rhs[b]])^T   (transpose)
 *   y[b] = x[lhs[b]] . dequant(w[rhs[b]])     (!transpose)
 * x [x_batches, M, K], w / scales / biases [w_batches, N, K*bits/32 | K/gs]
 * (transpose) or [w_batches, K, N*bits/32 | N/gs], y [batch, M, N].  The int32
 * index arrays live on the device; a null lhs_indices means b (x_batches ==
 * batch) or 0 (x_batches == 1), likewise rhs_indices.  A batch whose index is
 * out of range gets zero output rows.  sorted_indices promises rhs_indices in
 * ascending order (MLX's meaning); with it and many routes per expert
 * (transpose, M = 1, bf16 x, 4/8-bit) each expert's routes run as one MFMA
 * GEMM -- same results within the matmul rule; unsorted indices under the
 * promise give wrong rows (never an out-of-bounds access).  Replaces mlx_gather_qmm
 * (safemlx-sys/src/bindings.rs:3309) under safemlx::ops::gather_qmm_with_mode
 * (safemlx/src/ops/quantization.rs:298-379), as called by eredu's routed
 * experts (eredu/src/backend/mlx/nn/moe.rs:121-139).
 */
int eq_gather_qmm(void* y, const void* x, const uint32_t* w, const void* scales, const void* biases,
                  const int32_t* lhs_indices, const int32_t* rhs_indices, int64_t batch, int64_t x_batches,
                  int64_t w_batches, int64_t M, int64_t N, int64_t K, bool transpose, int group_size, int bits,
                  const char* mode, int x_dtype, int scale_dtype, bool sorted_indices, eq_stream_t stream);

/*
 * Affine group quantization of w [rows, cols] (dtype: f32, f16 or bf16) along
 * its rows: codes [rows, cols * bits / 32] u32 packed LSB-first, scales and
 * biases [rows, cols / group_size] in w's dtype, with MLX's affine rule --
 * scale = (max - min) / (2^bits - 1) signed toward the larger magnitude, the
 * edge value made exactly representable, bias = edge, codes rounded from the
 * stored scale and bias.  Replaces mlx_quantize (ops.h:801-808) under
 * safemlx::ops::quantize_with_mode (safemlx/src/ops/quantization.rs:100-159).
 * bits and group_size as for eq_quantized_matmul.  "mxfp4" (group 32, bits
 * 4, biases NULL): scales are u8 E8M0 bytes, the smallest power of two 2^e,
 * e in [-127, 127], with max|w| / 2^e <= 6 (a group with a NaN or infinity:
 * 255, an all-zero group: 0), and each code the nearest E2M1 value of
 * w / 2^e, ties to the even code, sign bit set for w < 0.  Nothing
 * saturates, unlike the OCP MX v1.0 rule (2^(floor(log2 max|w|) - 2), then a
 * clamp to 6); MLX's own quantizer is not available to check against.
 */
int eq_quantize(uint32_t* w_out, void* scales, void* biases, const void* w, int64_t rows, int64_t cols,
                int group_size, int bits, const char* mode, int dtype, eq_stream_t stream);

/* Activation prologues of eq_quantized_matmul_batched_prologue. */
enum eq_prologue_kind { EQ_PROLOGUE_SILU_MUL = 1, EQ_PROLOGUE_RMS_NORM = 2 };

typedef struct eq_activation_prologue {
    int kind;            /* enum eq_prologue_kind */
    const void* second;  /* SILU_MUL: up (x is the gate); RMS_NORM: residual added to x (may be NULL) */
    const void* weight;  /* RMS_NORM: norm weight [K] */
    void* hidden_out;    /* RMS_NORM: x + residual [K] (may be NULL; must not overlap x or the residual) */
    float eps;           /* RMS_NORM */
} eq_activation_prologue;

/*
 * eq_quantized_matmul_batched with the shared input row transformed first:
 *   SILU_MUL:  x' = silu(x) * second            (Mlp::hidden before down_proj,
 *              eredu-architectures/src/llama.rs:414-422)
 *   RMS_NORM:  h = x + second (rounded to bf16, stored to hidden_out),
 *              x' = h * rsqrt(mean(h^2) + eps) * weight
 *              (the residual add and pre-norm of TransformerBlock::forward,
 *              llama.rs:477-495)
 * then y_i = x' . W_i^T.  Results equal eq_silu_mul / eq_rms_norm followed by
 * eq_quantized_matmul_batched (RMS_NORM up to the order of the sum of
 * squares).  No counterpart in the reference's C ABI: it folds the MLX ops a
 * decoder layer runs before its projections into their launch.  Supported:
 * M = 1, 1-8 problems sharing x, transpose = true, bf16 x and scales, group
 * size 64, 4/8-bit, N % 16 == 0, K % 64 == 0, K <= 4096 for RMS_NORM;
 * anything else is rejected (use the separate entry points).
 */
int eq_quantized_matmul_batched_prologue(const eq_qmm_problem* problems, int count, int64_t M,
                                         bool transpose, int group_size, int bits, const char* mode,
                                         int x_dtype, int scale_dtype,
                                         const eq_activation_prologue* prologue, eq_stream_t stream);

/*
 * The gate/up projection of a SwiGLU MLP with the activation folded into the
 * launch (batch 1):
 *   out[f] = silu(g_f) * u_f,  g_f = bf16(x' . Wg[f]),  u_f = bf16(x' . Wu[f]),
 * each op rounded to bf16 as in eq_silu_mul (Mlp::hidden,
 * eredu-architectures/src/llama.rs:414-422), x' = x or, with `prologue`
 * (kind EQ_PROLOGUE_RMS_NORM only; NULL for none), the residual add + RMSNorm
 * of eq_quantized_matmul_batched_prologue.  w / scales / biases hold the two
 * projections interleaved in blocks of 8 rows: rows 16t .. 16t + 7 are gate
 * rows 8t .. 8t + 7 and rows 16t + 8 .. 16t + 15 are up rows 8t .. 8t + 7
 * ([2F, K] in the affine layout of eq_quantized_matmul, transpose = true);
 * the same packed rows, moved, so that a decode workgroup's 16-row tile
 * holds both halves of 8 outputs.  Results equal eq_quantized_matmul_batched
 * on the two projections followed by eq_silu_mul, bit for bit.  No
 * counterpart in the reference's C ABI (it folds the MLX ops between the
 * gate/up and down projections into one launch).  Supported: bf16 x and
 * scales, group size 64, 4/8-bit, F % 8 == 0, K a multiple of the decode
 * kernel's code block (512 values at 4 bits, 256 at 8), K <= 4096 with the
 * prologue; x and w 16-byte aligned; out (F values) must not overlap any
 * input.
 */
int eq_quantized_matmul_swiglu(void* out, const void* x, const uint32_t* w, const void* scales, const void* biases,
                               int64_t F, int64_t K, int group_size, int bits, const char* mode, int x_dtype,
                               int scale_dtype, const eq_activation_prologue* prologue, eq_stream_t stream);

/*
 * Decode-step operations around the quantized projections of a Llama-shaped
 * decoder at batch 1 (configs[4] of the measurement plan).  bf16 only
 * (dtype must be EQ_DTYPE_BF16); no counterpart in the quantized-linear C ABI
 * of the reference -- these replace the MLX calls a decoder layer makes
 * between its projections.
 */

/* hidden[rows, dim] += residual (when residual is not NULL, each sum rounded
 * to bf16, in place); out = hidden * rsqrt(mean(hidden^2) + eps) * weight.
 * Replaces the block's residual adds and nn::RmsNorm (fast::rms_norm,
 * safemlx/src/fast.rs:1119) in TransformerBlock::forward
 * (eredu-architectures/src/llama.rs:477-495).  dim % 8 == 0, 16-byte aligned. */
int eq_rms_norm(void* out, void* hidden, const void* residual, const void* weight, int64_t rows,
                int64_t dim, float eps, int dtype, eq_stream_t stream);

/* One decode position of grouped-query attention with a KV cache:
 *   q [n_heads, 128], k_new / v_new [n_kv_heads, 128] (the projections' outputs);
 *   q and k_new rotated by RoPE (half-split pairs, angle pos / freqs[i],
 *   freqs[64] f32 = the Llama3Rope frequencies, eredu/src/backend/mlx/nn/rope.rs:105-186);
 *   rotated k_new and v_new stored at row pos of k_cache / v_cache
 *   [n_kv_heads, max_seq, 128];
 *   out [n_heads, 128] = softmax(scale * q . K[0..pos]^T) . V[0..pos], head h
 *   reading KV head h / (n_heads / n_kv_heads).
 * Replaces Attention::attend (llama.rs:296-330): rotary forward, cache
 * update_for_attention and fast::scaled_dot_product_attention.  head_dim must
 * be 128 and n_heads / n_kv_heads at most 4.  Two launches: 64 softmax
 * states per query head (state y over the 32-position chunks y, y + 64, ...
 * of the cache), then their combination.  The states (n_heads * 64 * 520
 * bytes, whatever the position) live in the
 * library workspace of `stream` (grow-only, never freed while the process
 * runs); it cannot grow while `stream` is capturing, so a capture needs an
 * earlier call with at least this head count on that stream (else the call
 * fails), or eq_rope_attention_decode_noalloc. */
int eq_rope_attention_decode(void* out, const void* q, const void* k_new, const void* v_new,
                             void* k_cache, void* v_cache, const float* freqs, int64_t pos,
                             int64_t max_seq, int n_heads, int n_kv_heads, int head_dim, float scale,
                             int dtype, eq_stream_t stream);

/* eq_rope_attention_decode without any device allocation: no counterpart in
 * the reference.  For callers that cannot allocate device memory -- code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  Same arguments, validation and results (the same kernels); the
 * attention softmax states live in a library-owned static device array of
 * 8 MiB per GPU, held until the process ends, instead of the stream's
 * workspace.  A call needing more than that -- n_heads * 64 * 520 bytes, i.e.
 * more than 252 query heads -- is rejected with a message.  Every call on one
 * GPU shares that GPU's array: calls that overlap in time on one GPU (two
 * streams, or two processes' graphs) race and must be serialised by the
 * caller.  The first call on each device resolves the array's address. */
int eq_rope_attention_decode_noalloc(void* out, const void* q, const void* k_new, const void* v_new,
                                     void* k_cache, void* v_cache, const float* freqs, int64_t pos,
                                     int64_t max_seq, int n_heads, int n_kv_heads, int head_dim, float scale,
                                     int dtype, eq_stream_t stream);

/* eq_rope_attention_decode at a position read from device memory when the
 * kernel runs (pos: one int32 in device memory), so that one captured HIP
 * graph decodes successive positions: the reference advances its cache
 * offset every token (eredu/src/runtime/generation/streaming.rs:1038-1050,
 * through Attention::attend, llama.rs:296-330).  Same shapes, rules, kernels
 * and results as eq_rope_attention_decode at that position (the same
 * launches; the kernels take their chunk counts from the position).  The
 * softmax states live in the library workspace of `stream` (n_heads * 64 *
 * 520 bytes), so a capture needs an earlier call with this head count on that
 * stream.  A position outside [0, max_seq) writes no cache row and gives
 * zeros.  max_seq <= 131072. */
int eq_rope_attention_decode_at(void* out, const void* q, const void* k_new, const void* v_new,
                                void* k_cache, void* v_cache, const float* freqs, const int32_t* pos,
                                int64_t max_seq, int n_heads, int n_kv_heads, int head_dim, float scale,
                                int dtype, eq_stream_t stream);

/* pos[0] += 1 on `stream` (pos: one int32 in device memory): the end of a
 * decode step whose position lives on the device, the cache offset advance of
 * the reference's token loop (streaming.rs:1038-1050). */
int eq_advance_position(int32_t* pos, eq_stream_t stream);

/* out[n] = silu(gate) * up, silu(x) = x * sigmoid(x), each op rounded to bf16
 * (Mlp::hidden, llama.rs:414-422; eredu/src/backend/mlx/nn/layers.rs:21).
 * n % 8 == 0, 16-byte aligned. */
int eq_silu_mul(void* out, const void* gate, const void* up, int64_t n, int dtype, eq_stream_t stream);

/* out[t, :] = table[tokens[t], :] (zeros for an id outside [0, vocab)); tokens
 * is device memory (Decoder::embed, llama.rs:576-582). */
int eq_embedding(void* out, const void* table, const int32_t* tokens, int64_t n_tokens, int64_t vocab,
                 int64_t dim, int dtype, eq_stream_t stream);

/* out[r] = first index of the largest value of logits[r, 0..n) (greedy
 * decoding of the model's logits, llama.rs:649-658); NaNs are skipped (a row
 * of NaNs gives 0).  Rows of 16384 or more 16-byte aligned values (up to 4096
 * rows) are split over several workgroups that meet at arrival counters of
 * `stream` (allocated on the stream's first such call; under capture before
 * that, one workgroup per row is used). */
int eq_argmax(int32_t* out, const void* logits, int64_t rows, int64_t n, int dtype, eq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* EREDU_HIP_H */
