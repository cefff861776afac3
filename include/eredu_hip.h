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
enum eq_dtype { EQ_DTYPE_F32 = 0, EQ_DTYPE_F16 = 1, EQ_DTYPE_BF16 = 2 };

/* GGML block types handled on the device (codes of eredu-gguf/src/format.rs:297-330). */
enum eq_ggml_type { EQ_GGML_Q4_0 = 2, EQ_GGML_Q8_0 = 8, EQ_GGML_Q4_K = 12 };

/* Byte order of multi-byte block fields (eredu-gguf/src/format.rs:5-23 Endian). */
enum eq_endian { EQ_ENDIAN_LITTLE = 0, EQ_ENDIAN_BIG = 1 };

/* Which dense-dequant definition to follow for GGML blocks:
 * AFFINE = convert_affine then AffineTensor::dequantize (eredu-gguf/src/convert.rs:43-56,81-101);
 * NATIVE = the checkpoint-native decoders (safemlx/src/native_quantization.rs:3445-3469,3539-3542).
 * The two differ only for Q4_K (f16 rounding of d*sc and -dmin*m). */
enum eq_dequant_definition { EQ_DEQUANT_AFFINE = 0, EQ_DEQUANT_NATIVE = 1 };

/* Message of the last failed call on this thread ("" if none). */
const char* eq_last_error(void);

/* Library ABI version (major * 100 + minor). */
int eq_version(void);

/*
 * Group-wise affine quantized matmul.
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
 * x_dtype.  biases may be NULL (treated as zero).  mode must be "affine" (or
 * NULL).  bits in {2, 4, 8}; group_size in {32, 64, 128}.  Accumulation is f32.
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
 * code either way).  Decode-shaped groups (M <= 16, transpose, bf16 x) run as
 * one persistent launch per 8 problems, which streams the weights of all of
 * them back to back instead of paying a kernel launch per projection.
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
 * computed in f32 (one multiply, one add) and written as out_dtype.
 * Replaces mlx_dequantize (safemlx-sys/src/mlx-c/mlx/c/ops.h:359-369) as called
 * by safemlx::ops::dequantize_with_mode (safemlx/src/ops/quantization.rs:256-289).
 * w is [rows, cols*bits/32] u32; scales/biases [rows, cols/gs]; biases may be NULL.
 */
int eq_dequantize(void* out, const uint32_t* w, const void* scales, const void* biases,
                  int64_t rows, int64_t cols, int group_size, int bits, const char* mode,
                  int scale_dtype, int out_dtype, eq_stream_t stream);

/*
 * GGML blocks -> MLX affine (u32 codes, f16 scale bits, f16 bias bits),
 * byte-identical to eredu_gguf::convert_affine (eredu-gguf/src/convert.rs:318-465)
 * for Q4_0 (bits 4), Q8_0 (bits 8) and Q4_K (bits 4), all group 32.
 * `rows` x `cols` is the MLX shape (GGUF dims reversed, format.rs:449-452);
 * raw holds rows*cols/block_values blocks (raw_len bytes, checked like
 * convert.rs:319-324).  Outputs: weights [rows, cols*bits/32],
 * scales/biases [rows, cols/32].
 */
int eq_gguf_convert_affine(uint32_t* weights, uint16_t* scales, uint16_t* biases,
                           const uint8_t* raw, int64_t raw_len, int ggml_type, int64_t rows,
                           int64_t cols, int endian, eq_stream_t stream);

/*
 * GGML blocks -> dense [rows, cols] of out_dtype (EQ_DTYPE_BF16 or EQ_DTYPE_F32),
 * following `definition` (eq_dequant_definition).  bf16 output is the
 * round-to-nearest-even image of the reference's f32 result.
 * Replaces IQuantTensor::dequantize_f32 (eredu-gguf/src/convert.rs:43-56) and
 * NativeQuantizedTensor::dequantize's CPU decoders
 * (safemlx/src/native_quantization.rs:3417-3542).
 */
int eq_gguf_dequantize(void* out, const uint8_t* raw, int64_t raw_len, int ggml_type,
                       int64_t rows, int64_t cols, int endian, int definition, int out_dtype,
                       eq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* EREDU_HIP_H */
