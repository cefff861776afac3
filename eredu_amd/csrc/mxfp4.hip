// MXFP4 mode of quantize / dequantize / quantized_matmul / gather_qmm
// (safemlx QuantizationMode::MxFp4, safemlx/src/ops/quantization.rs:16-46,
// tested there by test_mxfp4_quantize_dequantize_and_matmul, :489-545):
// E2M1 codes packed 8 per u32 LSB-first, one E8M0 scale byte per 32 values
// along the packed dimension, no biases.  W[n, k] = e2m1(q[n, k]) * 2^(s - 127).
//
// Quantizer (MLX's own is not in the snapshot, so its exponent choice is a
// restatement of the format's definition, not a copy of MLX): per group of
// 32, the shared exponent is the smallest e with max|v| / 2^e <= 6 (no
// element saturates), clamped to the E8M0 range; each value is v / 2^e
// rounded to the nearest E2M1 magnitude, ties to the even code, with v's
// sign.  A group of zeros takes the smallest scale; a group whose largest
// magnitude is infinite or NaN takes the NaN scale (255).
//
// The matmul kernels accumulate in f32; the decode shape (transpose, bf16 x,
// M <= 16) runs the any-width decode kernel of qmv_any.hip with an E2M1
// decode, everything else the general kernels below.
#include "eq_common.hpp"

namespace eq {
namespace {

// E2M1 code of v / 2^e (inv = 2^-e): 7 comparisons against the midpoints of
// 0, 0.5, 1, 1.5, 2, 3, 4, 6; a midpoint goes to the neighbour with mantissa
// bit 0 (0.25 -> 0, 0.75 -> 1, 1.25 -> 1, 1.75 -> 2, 2.5 -> 2, 3.5 -> 4, 5 -> 4).
__device__ __forceinline__ uint32_t e2m1_code(float v, float inv) {
    const float a = fabsf(v) * inv;
    const uint32_t m = uint32_t(a > 0.25f) + uint32_t(a >= 0.75f) + uint32_t(a > 1.25f) + uint32_t(a >= 1.75f) +
                       uint32_t(a > 2.5f) + uint32_t(a >= 3.5f) + uint32_t(a > 5.0f);
    return m | (v < 0.f ? 8u : 0u);
}

// E8M0 byte of the shared exponent of a group whose largest magnitude is amax.
__device__ __forceinline__ uint32_t mxfp4_scale_byte(float amax) {
    if (!(amax < __builtin_huge_valf())) return 255u;  // inf or NaN
    if (!(amax > 0.f)) return 0u;
    // e = ceil(log2(amax / 6)), read from the bits of r = amax / 6 (a power of
    // two gives its exponent, anything above it the next one)
    const float r = amax / 6.0f;
    const uint32_t bits = __float_as_uint(r);
    const int ex = int((bits >> 23) & 0xffu), mant = int(bits & 0x7fffffu);
    int e;
    if (ex == 0) e = (r > __uint_as_float(0x00400000u)) ? -126 : -127;  // below 2^-126
    else e = (mant == 0) ? ex - 127 : ex - 126;
    e = e < -127 ? -127 : (e > 127 ? 127 : e);
    return uint32_t(e + 127);
}

// One thread per group of 32 values of w [rows, cols] (row-major).
template <typename T>
__global__ __launch_bounds__(256) void mxfp4_quantize_kernel(uint32_t* __restrict__ wq, uint8_t* __restrict__ sc,
                                                             const typename T::storage* __restrict__ w,
                                                             int64_t groups) {
    const int64_t gi = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (gi >= groups) return;
    const typename T::storage* p = w + gi * 32;
    float v[32];
    float amax = 0.f;
    bool nan = false;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        v[i] = load_param<T>(p, i);
        amax = fmaxf(amax, fabsf(v[i]));
        nan = nan || v[i] != v[i];
    }
    const uint32_t s = mxfp4_scale_byte(nan ? __builtin_nanf("") : amax);
    sc[gi] = uint8_t(s);
    // 2^-e as f32 (e = s - 127 in [-127, 127]): exact
    const int e = int(s) - 127;
    const float inv = s == 255u ? 0.f : (e >= -126 ? __uint_as_float(uint32_t(127 - e) << 23) : 0x1p127f);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) word |= e2m1_code(v[8 * j + i], inv) << (4 * i);
        wq[gi * 4 + j] = word;
    }
}

// One thread per code word (8 values).
template <typename OT>
__global__ __launch_bounds__(256) void mxfp4_dequant_kernel(typename OT::storage* __restrict__ out,
                                                            const uint32_t* __restrict__ w,
                                                            const uint8_t* __restrict__ sc, int64_t words) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= words) return;
    const uint32_t word = w[i];
    const float s = e8m0_to_f32(sc[i >> 2]);
#pragma unroll
    for (int c = 0; c < 8; c++) store_out<OT>(out, i * 8 + c, e2m1_to_f32((word >> (4 * c)) & 15u) * s);
}

// One thread per code word (8 values; consecutive lanes, consecutive words)
// with 16-byte streaming stores: the codes convert in hardware
// (v_cvt_scalef32_pk_{bf16,f32}_fp4 with the scale's f32 image, exact); f16
// outputs round from the exact f32 values.  out 16-byte aligned.
template <typename OT>
__global__ __launch_bounds__(256) void mxfp4_dequant_vec_kernel(typename OT::storage* __restrict__ out,
                                                                const uint32_t* __restrict__ w,
                                                                const uint8_t* __restrict__ sc, int64_t words) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= words) return;
    const uint32_t q = w[i];
    const float s = e8m0_to_f32(sc[i >> 2]);
    uint4* dst = reinterpret_cast<uint4*>(out + i * 8);
    if constexpr (__is_same(OT, BF16T)) {
        uint32_t p[4];
        e2m1x8_to_bf16(q, s, p);
        store_stream16(dst, make_uint4(p[0], p[1], p[2], p[3]));
    } else {
        const auto a = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(q, s, 0);
        const auto b = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(q, s, 1);
        const auto c = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(q, s, 2);
        const auto d = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(q, s, 3);
        const float v[8] = {a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
        if constexpr (__is_same(OT, F32T)) {
            store_stream16(dst, make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                           __float_as_uint(v[3])));
            store_stream16(dst + 1, make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]),
                                               __float_as_uint(v[7])));
        } else {
            uint32_t h[4];
#pragma unroll
            for (int k = 0; k < 4; k++)
                h[k] = uint32_t(__builtin_bit_cast(uint16_t, static_cast<_Float16>(v[2 * k]))) |
                       (uint32_t(__builtin_bit_cast(uint16_t, static_cast<_Float16>(v[2 * k + 1]))) << 16);
            store_stream16(dst, make_uint4(h[0], h[1], h[2], h[3]));
        }
    }
}

constexpr int kMxRows = 4;  // weight rows (waves) per workgroup of the transposed kernel
constexpr int kMxM = 4;     // activation rows per pass

// transpose = true: a wave per (output batch, weight row n); lanes take groups
// of 32 codes (one 16-byte load and one scale byte each).
template <typename XT>
__global__ __launch_bounds__(64 * kMxRows) void mxfp4_qmm_t_kernel(typename XT::storage* __restrict__ y,
                                                                   const typename XT::storage* __restrict__ x,
                                                                   const uint32_t* __restrict__ w,
                                                                   const uint8_t* __restrict__ sc, GatherIdx g,
                                                                   int64_t b0, int M, int N, int K) {
    const int lane = threadIdx.x & 63;
    const int64_t n = int64_t(blockIdx.x) * kMxRows + (threadIdx.x >> 6);
    const int64_t b = b0 + blockIdx.y;
    if (n >= N) return;
    int64_t xb, wb;
    const bool ok = gather_batch(g, b, xb, wb);
    const int G = K / 32;
    const uint32_t* wr = w + (wb * N + n) * int64_t(K / 8);
    const uint8_t* sr = sc + (wb * N + n) * int64_t(G);
    const typename XT::storage* xr = x + xb * int64_t(M) * K;
    for (int m0 = 0; m0 < M; m0 += kMxM) {
        float acc[kMxM] = {0.f, 0.f, 0.f, 0.f};
        if (ok) {
            for (int gi = lane; gi < G; gi += 64) {
                const uint32_t qw[4] = {wr[gi * 4], wr[gi * 4 + 1], wr[gi * 4 + 2], wr[gi * 4 + 3]};
                const float s = e8m0_to_f32(sr[gi]);
                float wv[32];
#pragma unroll
                for (int c = 0; c < 32; c++) wv[c] = e2m1_to_f32((qw[c >> 3] >> (4 * (c & 7))) & 15u);
#pragma unroll
                for (int i = 0; i < kMxM; i++) {
                    if (m0 + i >= M) break;
                    const typename XT::storage* xp = xr + int64_t(m0 + i) * K + gi * 32;
                    float t = 0.f;
#pragma unroll
                    for (int c = 0; c < 32; c++) t = fmaf(load_param<XT>(xp, c), wv[c], t);
                    acc[i] = fmaf(s, t, acc[i]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < kMxM; i++) {
            if (m0 + i >= M) break;
            const float v = wave_sum(acc[i]);
            if (lane == 0) store_out<XT>(y, (b * M + m0 + i) * int64_t(N) + n, v);
        }
    }
}

// transpose = false: W [K, N] packed along N.  A thread per (output batch,
// 8-column word j, activation row m): walks the K rows of its word.
template <typename XT>
__global__ __launch_bounds__(256) void mxfp4_qmm_n_kernel(typename XT::storage* __restrict__ y,
                                                          const typename XT::storage* __restrict__ x,
                                                          const uint32_t* __restrict__ w,
                                                          const uint8_t* __restrict__ sc, GatherIdx g, int64_t b0,
                                                          int M, int N, int K) {
    const int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x;
    const int Nw = N / 8, G = N / 32;
    const int64_t b = b0 + blockIdx.y;
    if (t >= int64_t(Nw) * M) return;
    const int j = int(t % Nw), m = int(t / Nw);
    int64_t xb, wb;
    const bool ok = gather_batch(g, b, xb, wb);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (ok) {
        const uint32_t* wr = w + wb * int64_t(K) * Nw + j;
        const uint8_t* sr = sc + wb * int64_t(K) * G + j / 4;
        const typename XT::storage* xr = x + (xb * M + m) * int64_t(K);
        for (int k = 0; k < K; k++) {
            const uint32_t q = wr[int64_t(k) * Nw];
            const float xs = load_param<XT>(xr, k) * e8m0_to_f32(sr[int64_t(k) * G]);
#pragma unroll
            for (int c = 0; c < 8; c++) acc[c] = fmaf(xs, e2m1_to_f32((q >> (4 * c)) & 15u), acc[c]);
        }
    }
#pragma unroll
    for (int c = 0; c < 8; c++) store_out<XT>(y, (b * M + m) * int64_t(N) + j * 8 + c, acc[c]);
}

}  // namespace

int mxfp4_quantize(uint32_t* w_out, uint8_t* scales, const void* w, int64_t rows, int64_t cols, int dtype,
                   hipStream_t st) {
    const int64_t groups = rows * (cols / 32);
    if (groups == 0) return 0;
    if ((groups + 255) / 256 > INT32_MAX) {
        set_error("tensor too large");
        return 1;
    }
    const dim3 grid(unsigned((groups + 255) / 256));
    with_dtype(dtype, [&](auto tt) {
        typedef decltype(tt) T;
        mxfp4_quantize_kernel<T><<<grid, 256, 0, st>>>(w_out, scales, static_cast<const typename T::storage*>(w),
                                                       groups);
    });
    return check_launch("quantize (mxfp4)");
}

int mxfp4_dequantize(void* out, const uint32_t* w, const uint8_t* scales, int64_t rows, int64_t cols, int out_dtype,
                     hipStream_t st) {
    const int64_t words = rows * (cols / 8);
    if (words == 0) return 0;
    if ((words + 255) / 256 > INT32_MAX) {
        set_error("tensor too large");
        return 1;
    }
    const bool vec = aligned(out, 16);
    const dim3 grid(unsigned((words + 255) / 256));
    with_dtype(out_dtype, [&](auto ot) {
        typedef decltype(ot) OT;
        typedef typename OT::storage OS;
        if (vec) mxfp4_dequant_vec_kernel<OT><<<grid, 256, 0, st>>>(static_cast<OS*>(out), w, scales, words);
        else mxfp4_dequant_kernel<OT><<<grid, 256, 0, st>>>(static_cast<OS*>(out), w, scales, words);
    });
    return check_launch("dequantize (mxfp4)");
}

int mxfp4_matmul(void* y, const void* x, const uint32_t* w, const uint8_t* scales, const GatherIdx& g,
                 int64_t batch, int64_t M, int64_t N, int64_t K, bool transpose, int x_dtype, bool sorted,
                 const WsSource* ws, hipStream_t st) {
    if (M == 0 || batch == 0) return 0;
    uint16_t* yb = static_cast<uint16_t*>(y);
    const uint16_t* xb = static_cast<const uint16_t*>(x);
    const bool plain = batch == 1 && g.lhs == nullptr && g.rhs == nullptr;
    const bool bf16_t = transpose && x_dtype == EQ_DTYPE_BF16;
    const bool mfma_ok = bf16_t && aligned(x, 16) && aligned(w, 16);
    // prefill (and M > 4, where the decode kernel's passes of 4 rows, each
    // reading W again, cost more than one MFMA tile of 128 rows): the MFMA qmm
    if (mfma_ok && plain && M > 4 && N % 128 == 0 && K % 64 == 0 && aligned(y, 8) &&
        launch_qmm_mfma_mxfp4(yb, xb, w, scales, int(M), int(N), int(K), ws, st))
        return take_refusal() ? 1 : check_launch("quantized_matmul (mxfp4 qmm)");
    // the decode shape: the any-width decode kernel with E2M1 codes
    if (bf16_t && plain && M <= 16 && launch_qmv_any_mxfp4(yb, xb, w, scales, int(M), int(N), int(K), st))
        return check_launch("quantized_matmul (mxfp4 decode)");
    // many routes over sorted experts: one MFMA GEMM per expert's rows
    if (mfma_ok && M == 1 && sorted && g.rhs && batch >= 64 && batch >= 2 * g.w_batches && batch <= INT32_MAX &&
        g.w_batches <= INT32_MAX && N % 128 == 0 && K % 64 == 0 && aligned(y, 8) &&
        int64_t(N) * K / 2 < (int64_t(1) << 31) && batch * K * 2 < (int64_t(1) << 31) &&
        launch_qmm_grouped_mxfp4(yb, xb, w, scales, g.lhs, g.rhs, int(batch), g.x_batches, int(g.w_batches), int(N),
                                 int(K), st))
        return check_launch("gather_qmm (mxfp4 grouped qmm)");
    // transpose = false, few rows: the split-K VALU kernel of the affine path
    if (!transpose && x_dtype == EQ_DTYPE_BF16 && M <= 8 &&
        launch_qmm_n_small(4, EQ_DTYPE_U8, yb, xb, w, scales, nullptr, g, batch, int(M), int(N), int(K), 32, ws, st))
        return check_launch("quantized_matmul (mxfp4 qmm_n)");
    if (!transpose && x_dtype == EQ_DTYPE_BF16 && plain && M > 8 && M <= kQmmNRowsMax &&
        launch_qmm_n_rows(4, EQ_DTYPE_U8, yb, xb, w, scales, nullptr, M, int(N), int(K), 32, ws, st))
        return check_launch("quantized_matmul (mxfp4 qmm_n rows)");
    // routed-expert decode: one activation row per route
    if (mfma_ok && M == 1) {
        for (int64_t b0 = 0; b0 < batch; b0 += kMaxGridY) {
            const unsigned nb = unsigned(batch - b0 < kMaxGridY ? batch - b0 : kMaxGridY);
            launch_gather_qmv_mxfp4(yb, xb, w, scales, g, b0, nb, int(N), int(K), st);
        }
        return check_launch("gather_qmm (mxfp4 qmv)");
    }
    if ((N + kMxRows - 1) / kMxRows > INT32_MAX || (N / 8) * M / 256 >= INT32_MAX) {
        set_error("dimension too large for the MXFP4 kernels");
        return 1;
    }
    bool launched = false;
    with_dtype(x_dtype, [&](auto xt) {
        typedef decltype(xt) XT;
        typedef typename XT::storage XS;
        for (int64_t b0 = 0; b0 < batch; b0 += kMaxGridY) {
            const unsigned nb = unsigned(batch - b0 < kMaxGridY ? batch - b0 : kMaxGridY);
            if (transpose) {
                const dim3 grid(unsigned((N + kMxRows - 1) / kMxRows), nb);
                mxfp4_qmm_t_kernel<XT><<<grid, 64 * kMxRows, 0, st>>>(static_cast<XS*>(y), static_cast<const XS*>(x),
                                                                      w, scales, g, b0, int(M), int(N), int(K));
            } else {
                const int64_t threads = (N / 8) * M;
                const dim3 grid(unsigned((threads + 255) / 256), nb);
                mxfp4_qmm_n_kernel<XT><<<grid, 256, 0, st>>>(static_cast<XS*>(y), static_cast<const XS*>(x), w, scales,
                                                             g, b0, int(M), int(N), int(K));
            }
        }
        launched = true;
    });
    if (!launched) {
        set_error("no MXFP4 kernel for this activation dtype");
        return 1;
    }
    return check_launch("quantized_matmul (mxfp4)");
}

}  // namespace eq
