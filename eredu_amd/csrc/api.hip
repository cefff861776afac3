// C ABI entry points, argument validation and dispatch, plus the general
// (any activation/scale dtype, any layout) quantized matmul and dequantize
// kernels that back the shapes the matrix-core paths do not take.
//
// Dispatch of eq_quantized_matmul:
//   transpose, bf16 x, bits 4/8, bf16/f16 scales, group size 32/64/128:
//     M <= 16  -> qmv (qmv.hip), the decode path (N % 16 == 0), unless the
//                 rows need several passes over the weights (decode_rows)
//     M  > 16  -> qmm_mfma (qmm.hip), the prefill path (N % 128 == 0, K % 64 == 0)
//   transpose = false, bf16 x, bits 4/8, M <= 8 -> qmm_n (qmm_n.hip)
// Everything else -- f32/f16 activations, f32 scales, bits 2/3/5/6 (3/5/6-bit
// codes form an LSB-first bit stream), group size 16 or a multiple of 32
// other than 32/64/128, the remaining transpose = false shapes, ragged N --
// runs the f32 kernels below.  There is no host fallback: a shape no kernel
// takes is an error.
#include <cstring>
#include <vector>
#include <type_traits>

#include "eq_common.hpp"

#ifndef EQ_QMV_ONE_PASS
#define EQ_QMV_ONE_PASS 1  // 1: multi-pass decode calls go to the prefill kernel when it can take them; 0: M <= 16 to qmv
#endif

namespace eq {

// Whether an M-row call of 4/8-bit codes (transpose, 16-bit x) takes the
// decode kernels: up to 16 rows, unless they would read the weights in
// several passes (a pass multiplies 16 / groups-per-span rows: 8 at 4-bit
// group 64, 4 at 4-bit group 32, 16 at 8-bit group 64) and the prefill
// kernel, which reads them once for any M, can take the call (qmm_shape).
// Measured on the Llama-3-8B shapes: two passes of 4-bit group 64 or of
// 8-bit group 32 1.0-1.6x slower than the prefill kernel; two passes of
// 4-bit group 32 within 0.9-1.1x of it, three or more 1.3-2.1x slower.
static bool decode_rows(int64_t M, int bits, int group_size, bool qmm_shape) {
    if (M > 16) return false;
    if (!EQ_QMV_ONE_PASS || !qmm_shape) return true;
    const int rows = qmv_rows_per_pass(bits, group_size);
    const int passes = (int(M) + rows - 1) / rows;
    return passes < (bits == 4 && group_size < 64 ? 3 : 2);
}

static thread_local std::string g_last_error;

static thread_local bool g_refused = false;

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }
void note_refusal() { g_refused = true; }
bool take_refusal() {
    const bool r = g_refused;
    g_refused = false;
    return r;
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error(std::string(what) + ": kernel launch failed: " + hipGetErrorString(e));
        return 1;
    }
    return 0;
}

namespace {

// ------------------------------------------------------------ general kernels

// transpose = true: one wave per output feature n (qmm_t_rows), activations
// in chunks of 8 rows.
template <int BITS, typename XT, typename ST>
__global__ __launch_bounds__(64 * kGenRowsPerWG) void qmm_t_general(
    typename XT::storage* __restrict__ y, const typename XT::storage* __restrict__ x,
    const uint32_t* __restrict__ w, const typename ST::storage* __restrict__ s,
    const typename ST::storage* __restrict__ b, int64_t M, int64_t N, int64_t K, int gs) {
    const int64_t n = int64_t(blockIdx.x) * kGenRowsPerWG + (threadIdx.x >> 6);
    if (n >= N) return;
    qmm_t_rows<BITS, XT, ST>(y, x, w, s, b, M, N, K, gs, n, threadIdx.x & 63);
}

// transpose = false: W is [K, N] packed along N.  One thread per output
// column n and chunk of 8 activation rows (qmm_n_cols).
template <int BITS, typename XT, typename ST>
__global__ __launch_bounds__(256) void qmm_n_general(typename XT::storage* __restrict__ y,
                                                     const typename XT::storage* __restrict__ x,
                                                     const uint32_t* __restrict__ w,
                                                     const typename ST::storage* __restrict__ s,
                                                     const typename ST::storage* __restrict__ b, int64_t M,
                                                     int64_t N, int64_t K, int gs) {
    const int64_t n = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (n >= N) return;
    qmm_n_cols<BITS, XT, ST>(y, x, w, s, b, M, N, K, gs, n, int64_t(blockIdx.y) * kGenMChunk);
}

// out[r, c] = f32(s) * q + f32(b), one rounding each (convert.rs:81-101).
// One thread per code word; its PACK codes share a group (gs >= 32 >= PACK).
// VEC (out 16-byte aligned): the word's outputs leave as 8- or 16-byte
// stores instead of PACK scalar ones.
// GS: the group size when it is a compile-time power of two (32, 64, 128),
// else 0 and `gs` holds it.  Rows hold whole groups, so the group of element
// e (row-major) is e / gs.
template <int BITS, typename ST, typename OT, bool VEC, int GS = 0>
__global__ __launch_bounds__(256) void dequant_kernel(typename OT::storage* __restrict__ out,
                                                      const uint32_t* __restrict__ w,
                                                      const typename ST::storage* __restrict__ s,
                                                      const typename ST::storage* __restrict__ b, int64_t rows,
                                                      int64_t cols, int gs) {
    constexpr int PACK = 32 / BITS;
    typedef typename OT::storage OS;
    const int64_t words = rows * cols / PACK;
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= words) return;
    const uint32_t word = w[i];
    const int64_t base = i * PACK;  // element index of the word's first code
    const int64_t g = GS ? base / GS : base / gs;
    const float sc = load_param<ST>(s, g);
    const float bi = b ? load_param<ST>(b, g) : 0.f;
    OS v[PACK];
#pragma unroll
    for (int p = 0; p < PACK; p++)
        v[p] = to_storage<OT>(__fadd_rn(sc * float((word >> (p * BITS)) & ((1u << BITS) - 1u)), bi));
    if constexpr (VEC) {
        constexpr int BYTES = PACK * int(sizeof(OS));
        if constexpr (BYTES % 16 == 0) {
#pragma unroll
            for (int q = 0; q < BYTES / 16; q++)
                store_stream16(reinterpret_cast<uint4*>(out + base) + q, reinterpret_cast<const uint4*>(v)[q]);
        } else {
#pragma unroll
            for (int q = 0; q < BYTES / 8; q++)
                store_stream8(reinterpret_cast<uint2*>(out + base) + q, reinterpret_cast<const uint2*>(v)[q]);
        }
    } else {
#pragma unroll
        for (int p = 0; p < PACK; p++) out[base + p] = v[p];
    }
}

// 3-, 5- and 6-bit codes (an LSB-first bit stream, eredu-gguf/src/convert.rs:413-427):
// one thread per CPT codes -- 32 (BITS words) for 3 and 5 bits, 16 (3 words)
// for 6 bits.  A packed row holds whole words, so cols is a multiple of CPT
// and a thread's codes lie in one row; at group size 16 they span two groups.
template <int BITS, typename ST, typename OT>
__global__ __launch_bounds__(256) void dequant_odd_kernel(typename OT::storage* __restrict__ out,
                                                          const uint32_t* __restrict__ w,
                                                          const typename ST::storage* __restrict__ s,
                                                          const typename ST::storage* __restrict__ b, int64_t rows,
                                                          int64_t cols, int gs) {
    constexpr int CPT = BITS == 6 ? 16 : 32, WPT = CPT * BITS / 32;
    const int64_t units = rows * cols / CPT;
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= units) return;
    uint32_t wd[WPT + 1];
#pragma unroll
    for (int j = 0; j < WPT; j++) wd[j] = w[i * WPT + j];
    wd[WPT] = 0u;
    const int64_t base = i * CPT;
    const int64_t r = base / cols, c0 = base % cols;
    const int64_t g0 = r * (cols / gs);
#pragma unroll
    for (int p = 0; p < CPT; p++) {
        constexpr uint32_t mask = (1u << BITS) - 1u;
        const int bit = p * BITS, wi = bit >> 5, sh = bit & 31;
        uint32_t q = wd[wi] >> sh;
        if (sh + BITS > 32) q |= wd[wi + 1] << (32 - sh);
        q &= mask;
        const int64_t g = g0 + (c0 + p) / gs;
        const float sc = load_param<ST>(s, g);
        const float bi = b ? load_param<ST>(b, g) : 0.f;
        out[base + p] = to_storage<OT>(__fadd_rn(sc * float(q), bi));
    }
}

// --------------------------------------------------------------- dispatch

}  // namespace
}  // namespace eq

using namespace eq;

// Affine group quantizer (the MLX quantize that safemlx::ops::quantize_with_mode
// calls, safemlx/src/ops/quantization.rs:100-159), one thread per group of
// `gs` values along a row: min and max; scale = (max - min) / (2^bits - 1)
// (at least 1e-7), signed toward the larger magnitude; the edge value
// (min or max) made exactly representable (scale = edge / rint(edge /
// scale)); bias = edge; scale and bias stored in the input's dtype and the
// codes q = clamp(rint((w - bias) / scale), 0, 2^bits - 1) computed with the
// stored values, packed LSB-first.
template <int BITS, typename T>
__global__ __launch_bounds__(256) void quantize_kernel(uint32_t* __restrict__ wq, typename T::storage* __restrict__ sc,
                                                       typename T::storage* __restrict__ bi,
                                                       const typename T::storage* __restrict__ w, int64_t groups,
                                                       int gs) {
    const int64_t gidx = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (gidx >= groups) return;
    const typename T::storage* v = w + gidx * gs;
    constexpr int n_bins = (1 << BITS) - 1;
    float mn = load_param<T>(v, 0), mx = mn;
    for (int i = 1; i < gs; i++) {
        const float x = load_param<T>(v, i);
        mn = x < mn ? x : mn;
        mx = x > mx ? x : mx;
    }
    float scale = (mx - mn) / float(n_bins);
    if (scale < 1e-7f) scale = 1e-7f;
    const bool neg = fabsf(mn) > fabsf(mx);
    scale = neg ? scale : -scale;
    const float edge = neg ? mn : mx;
    const float q0 = rintf(edge / scale);
    if (q0 != 0.0f) scale = edge / q0;
    store_out<T>(sc, gidx, scale);
    store_out<T>(bi, gidx, edge);
    const float s_st = load_param<T>(sc, gidx), b_st = load_param<T>(bi, gidx);
    uint32_t* dst = wq + gidx * (gs * BITS / 32);
    for (int w0 = 0; w0 < gs * BITS / 32; w0++) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 32 / BITS; e++) {
            const float x = load_param<T>(v, w0 * (32 / BITS) + e);
            float q = s_st != 0.0f ? rintf((x - b_st) / s_st) : 0.0f;
            q = q >= 0.0f ? q : 0.0f;
            q = q > float(n_bins) ? float(n_bins) : q;
            word |= uint32_t(q) << (BITS * e);
        }
        dst[w0] = word;
    }
}

// quantize_kernel for 3-, 5- and 6-bit codes: one thread per unit of `gpu`
// consecutive groups (2 when one group's codes do not fill whole words, group
// size 16 at 3 or 5 bits), the same arithmetic per group, codes appended to an
// LSB-first bit stream (eredu-gguf/src/convert.rs:413-427 `pack`).
template <int BITS, typename T>
__global__ __launch_bounds__(256) void quantize_odd_kernel(uint32_t* __restrict__ wq,
                                                           typename T::storage* __restrict__ sc,
                                                           typename T::storage* __restrict__ bi,
                                                           const typename T::storage* __restrict__ w, int64_t units,
                                                           int gs, int gpu) {
    const int64_t unit = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (unit >= units) return;
    constexpr int n_bins = (1 << BITS) - 1;
    uint32_t* dst = wq + unit * (int64_t(gs) * gpu * BITS / 32);
    uint64_t acc = 0;
    int nacc = 0, wo = 0;
    for (int gi = 0; gi < gpu; gi++) {
        const int64_t gidx = unit * gpu + gi;
        const typename T::storage* v = w + gidx * gs;
        float mn = load_param<T>(v, 0), mx = mn;
        for (int i = 1; i < gs; i++) {
            const float x = load_param<T>(v, i);
            mn = x < mn ? x : mn;
            mx = x > mx ? x : mx;
        }
        float scale = (mx - mn) / float(n_bins);
        if (scale < 1e-7f) scale = 1e-7f;
        const bool neg = fabsf(mn) > fabsf(mx);
        scale = neg ? scale : -scale;
        const float edge = neg ? mn : mx;
        const float q0 = rintf(edge / scale);
        if (q0 != 0.0f) scale = edge / q0;
        store_out<T>(sc, gidx, scale);
        store_out<T>(bi, gidx, edge);
        const float s_st = load_param<T>(sc, gidx), b_st = load_param<T>(bi, gidx);
        for (int i = 0; i < gs; i++) {
            const float x = load_param<T>(v, i);
            float q = s_st != 0.0f ? rintf((x - b_st) / s_st) : 0.0f;
            q = q >= 0.0f ? q : 0.0f;
            q = q > float(n_bins) ? float(n_bins) : q;
            acc |= uint64_t(uint32_t(q)) << nacc;
            nacc += BITS;
            if (nacc >= 32) {
                dst[wo++] = uint32_t(acc);
                acc >>= 32;
                nacc -= 32;
            }
        }
    }
}

// quantize_kernel with the group held in registers: one thread per group of
// GS values, loaded with 16-byte loads (w 16-byte aligned), the same
// arithmetic in the same order (bit-identical results), codes stored as
// 16- or 8-byte words (wq 16-byte aligned).
template <int BITS, typename T, int GS>
__global__ __launch_bounds__(256) void quantize_vec_kernel(uint32_t* __restrict__ wq,
                                                           typename T::storage* __restrict__ sc,
                                                           typename T::storage* __restrict__ bi,
                                                           const typename T::storage* __restrict__ w, int64_t groups) {
    typedef typename T::storage S;
    constexpr int PER16 = 16 / int(sizeof(S)), WORDS = GS * BITS / 32, PACK = 32 / BITS;
    const int64_t gidx = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (gidx >= groups) return;
    float x[GS];
    const uint4* src = reinterpret_cast<const uint4*>(w + gidx * GS);
#pragma unroll
    for (int q = 0; q < GS / PER16; q++) {
        const uint4 u = src[q];
        const S* e = reinterpret_cast<const S*>(&u);
#pragma unroll
        for (int j = 0; j < PER16; j++) {
            if constexpr (sizeof(S) == 4) x[q * PER16 + j] = __builtin_bit_cast(float, e[j]);
            else x[q * PER16 + j] = load_param<T>(e, j);
        }
    }
    constexpr int n_bins = (1 << BITS) - 1;
    float mn = x[0], mx = mn;
#pragma unroll
    for (int i = 1; i < GS; i++) {
        mn = x[i] < mn ? x[i] : mn;
        mx = x[i] > mx ? x[i] : mx;
    }
    float scale = (mx - mn) / float(n_bins);
    if (scale < 1e-7f) scale = 1e-7f;
    const bool neg = fabsf(mn) > fabsf(mx);
    scale = neg ? scale : -scale;
    const float edge = neg ? mn : mx;
    const float q0 = rintf(edge / scale);
    if (q0 != 0.0f) scale = edge / q0;
    const S s_bits = to_storage<T>(scale), b_bits = to_storage<T>(edge);
    sc[gidx] = s_bits;
    bi[gidx] = b_bits;
    const float s_st = load_param<T>(&s_bits, 0), b_st = load_param<T>(&b_bits, 0);
    uint32_t words[WORDS];
#pragma unroll
    for (int w0 = 0; w0 < WORDS; w0++) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < PACK; e++) {
            float q = s_st != 0.0f ? rintf((x[w0 * PACK + e] - b_st) / s_st) : 0.0f;
            q = q >= 0.0f ? q : 0.0f;
            q = q > float(n_bins) ? float(n_bins) : q;
            word |= uint32_t(q) << (BITS * e);
        }
        words[w0] = word;
    }
    uint32_t* dst = wq + gidx * WORDS;
    if constexpr (WORDS % 4 == 0) {
#pragma unroll
        for (int q = 0; q < WORDS / 4; q++) reinterpret_cast<uint4*>(dst)[q] = reinterpret_cast<const uint4*>(words)[q];
    } else {
#pragma unroll
        for (int q = 0; q < WORDS / 2; q++) reinterpret_cast<uint2*>(dst)[q] = reinterpret_cast<const uint2*>(words)[q];
    }
}

extern "C" const char* eq_last_error(void) { return g_last_error.c_str(); }

extern "C" int eq_version(void) { return 100; }

// eq_quantized_matmul with the scratch memory of split-K launches taken from
// `ws` (null: the library workspace).
static int quantized_matmul_impl(void* y, const void* x, const uint32_t* w, const void* scales, const void* biases,
                                 int64_t M, int64_t N, int64_t K, bool transpose, int group_size, int bits,
                                 const char* mode, int x_dtype, int scale_dtype, const WsSource* ws,
                                 eq_stream_t stream) {
    QuantMode qm;
    if (parse_mode(mode, qm)) return 1;
    if (qm == kModeMxFp4 ? check_mxfp4(group_size, bits, scale_dtype, biases) : check_gs_bits(group_size, bits))
        return 1;
    if (!valid_dtype(x_dtype) || (qm == kModeAffine && !valid_dtype(scale_dtype))) {
        set_error("invalid dtype code");
        return 1;
    }
    if (M < 0 || N <= 0 || K <= 0) {
        set_error("invalid shape: M >= 0, N > 0 and K > 0 required");
        return 1;
    }
    // The packed (quantized) dimension must hold whole groups
    // (MLX: "last dimension is not divisible by group size").
    const int64_t packed_dim = transpose ? K : N;
    if (packed_dim % group_size != 0) {
        set_error("the quantized dimension (" + std::to_string(packed_dim) + ") is not divisible by group_size " +
                  std::to_string(group_size));
        return 1;
    }
    if (!check_packed_row(packed_dim, bits)) return 1;
    if (!y || !x || !w || !scales) {
        set_error("null pointer argument");
        return 1;
    }
    if (M == 0) return 0;
    if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) {
        set_error("dimension exceeds 2^31 - 1");
        return 1;
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (qm == kModeMxFp4) {
        const GatherIdx one{nullptr, nullptr, 1, 1};
        return mxfp4_matmul(y, x, w, static_cast<const uint8_t*>(scales), one, 1, M, N, K, transpose, x_dtype, false, ws,
                            st);
    }

    // matrix-core kernels: bf16 or f16 activations (the output in the same type)
    const bool x16 = x_dtype == EQ_DTYPE_BF16 || x_dtype == EQ_DTYPE_F16;
    const bool mfma_ok = transpose && x16 && (bits == 4 || bits == 8) &&
                         (scale_dtype == EQ_DTYPE_BF16 || scale_dtype == EQ_DTYPE_F16) && aligned(x, 16) &&
                         aligned(w, 16);
    // prefill on the matrix cores: 4/8-bit codes directly, 2/3/5/6-bit codes
    // re-packed to bytes slice by slice in the workspace
    const bool odd_ok = transpose && x16 && (bits == 2 || bits == 3 || bits == 5 || bits == 6) &&
                        (scale_dtype == EQ_DTYPE_BF16 || scale_dtype == EQ_DTYPE_F16) && aligned(x, 16) &&
                        aligned(w, 4);
    const bool qmm_shape = N % 128 == 0 && K % 64 == 0 && aligned(y, 8);
    const bool qmv_rows = decode_rows(M, bits, group_size, qmm_shape);
    if (mfma_ok && qmv_rows && N % 16 == 0) {
        if (launch_qmv_mfma(bits, group_size, scale_dtype, static_cast<uint16_t*>(y), static_cast<const uint16_t*>(x),
                            w, scales, biases, int(M), int(N), int(K), st, x_dtype))
            return check_launch("quantized_matmul (qmv)");
    }
    if ((mfma_ok ? !qmv_rows : odd_ok && M > 16) && qmm_shape) {
        if (launch_qmm_mfma(bits, group_size, scale_dtype, static_cast<uint16_t*>(y), static_cast<const uint16_t*>(x),
                            w, scales, biases, int(M), int(N), int(K), ws, st, -1, x_dtype))
            return take_refusal() ? 1 : check_launch("quantized_matmul (qmm)");
    }
    if (transpose && x_dtype == EQ_DTYPE_BF16 && M <= 16 &&
        launch_qmv_any(bits, group_size, scale_dtype, static_cast<uint16_t*>(y), static_cast<const uint16_t*>(x), w,
                       scales, biases, int(M), int(N), int(K), st))
        return check_launch("quantized_matmul (qmv_any)");
    if (!transpose && x_dtype == EQ_DTYPE_BF16 && M <= 8) {
        const GatherIdx one{nullptr, nullptr, 1, 1};
        if (launch_qmm_n_small(bits, scale_dtype, static_cast<uint16_t*>(y), static_cast<const uint16_t*>(x), w,
                               scales, biases, one, 1, int(M), int(N), int(K), group_size, ws, st))
            return check_launch("quantized_matmul (qmm_n)");
    }
    if (!transpose && x_dtype == EQ_DTYPE_BF16 && M > 8 && M <= kQmmNRowsMax &&
        launch_qmm_n_rows(bits, scale_dtype, static_cast<uint16_t*>(y), static_cast<const uint16_t*>(x), w, scales,
                          biases, M, int(N), int(K), group_size, ws, st))
        return check_launch("quantized_matmul (qmm_n rows)");

    bool launched = false;
    with_bits(bits, [&](auto bc) {
        constexpr int B = decltype(bc)::value;
        with_dtype(x_dtype, [&](auto xt) {
            typedef decltype(xt) XT;
            with_dtype(scale_dtype, [&](auto stt) {
                typedef decltype(stt) ST;
                typedef typename XT::storage XS;
                typedef typename ST::storage SS;
                if (transpose) {
                    const dim3 grid(unsigned((N + kGenRowsPerWG - 1) / kGenRowsPerWG));
                    qmm_t_general<B, XT, ST><<<grid, 64 * kGenRowsPerWG, 0, st>>>(
                        static_cast<XS*>(y), static_cast<const XS*>(x), w, static_cast<const SS*>(scales),
                        static_cast<const SS*>(biases), M, N, K, group_size);
                } else {
                    // grid.y is at most 65535: activation rows in pieces of 65535 * kGenMChunk
                    const int64_t piece = int64_t(kMaxGridY) * kGenMChunk;
                    for (int64_t m0 = 0; m0 < M; m0 += piece) {
                        const int64_t mc = M - m0 < piece ? M - m0 : piece;
                        const dim3 grid(unsigned((N + 255) / 256), unsigned((mc + kGenMChunk - 1) / kGenMChunk));
                        qmm_n_general<B, XT, ST><<<grid, 256, 0, st>>>(
                            static_cast<XS*>(y) + m0 * N, static_cast<const XS*>(x) + m0 * K, w,
                            static_cast<const SS*>(scales), static_cast<const SS*>(biases), mc, N, K, group_size);
                    }
                }
                launched = true;
            });
        });
    });
    if (!launched) {
        set_error("no kernel for this combination");
        return 1;
    }
    return check_launch("quantized_matmul (general)");
}

extern "C" int eq_quantized_matmul(void* y, const void* x, const uint32_t* w, const void* scales, const void* biases,
                                   int64_t M, int64_t N, int64_t K, bool transpose, int group_size, int bits,
                                   const char* mode, int x_dtype, int scale_dtype, eq_stream_t stream) {
    clear_error();
    return quantized_matmul_impl(y, x, w, scales, biases, M, N, K, transpose, group_size, bits, mode, x_dtype,
                                 scale_dtype, nullptr, stream);
}

extern "C" int eq_quantized_matmul_batched(const eq_qmm_problem* problems, int count, int64_t M, bool transpose,
                                           int group_size, int bits, const char* mode, int x_dtype, int scale_dtype,
                                           eq_stream_t stream) {
    clear_error();
    QuantMode qm;
    if (parse_mode(mode, qm)) return 1;
    if (qm == kModeMxFp4 ? (group_size != 32 || bits != 4) : check_gs_bits(group_size, bits) != 0) {
        if (qm == kModeMxFp4) check_mxfp4(group_size, bits, scale_dtype, nullptr);
        return 1;
    }
    if (!valid_dtype(x_dtype) || !(qm == kModeAffine ? valid_dtype(scale_dtype) : scale_dtype == EQ_DTYPE_U8)) {
        set_error("invalid dtype code");
        return 1;
    }
    if (count < 0 || M < 0 || (count > 0 && problems == nullptr)) {
        set_error("invalid problem list");
        return 1;
    }
    for (int i = 0; i < count; i++) {
        const eq_qmm_problem& p = problems[i];
        if (p.N <= 0 || p.K <= 0 || p.N > INT32_MAX || p.K > INT32_MAX) {
            set_error("problem " + std::to_string(i) + ": N and K must be in [1, 2^31 - 1]");
            return 1;
        }
        const int64_t packed_dim = transpose ? p.K : p.N;
        if (packed_dim % group_size != 0) {
            set_error("problem " + std::to_string(i) + ": the quantized dimension (" + std::to_string(packed_dim) +
                      ") is not divisible by group_size " + std::to_string(group_size));
            return 1;
        }
        if (!check_packed_row(packed_dim, bits)) {
            set_error("problem " + std::to_string(i) + ": " + eq_last_error());
            return 1;
        }
        if (!p.y || !p.x || !p.w || !p.scales) {
            set_error("problem " + std::to_string(i) + ": null pointer argument");
            return 1;
        }
    }
    if (M == 0 || count == 0) return 0;
    if (M > INT32_MAX) {
        set_error("dimension exceeds 2^31 - 1");
        return 1;
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    // Decode-shaped groups go to one grouped launch per kQmvMaxProblems
    // problems, when every problem would take the decode kernels alone.
    bool grouped = qm == kModeAffine && transpose && (x_dtype == EQ_DTYPE_BF16 || x_dtype == EQ_DTYPE_F16) &&
                   (bits == 4 || bits == 8) && (scale_dtype == EQ_DTYPE_BF16 || scale_dtype == EQ_DTYPE_F16) && M <= 16;
    std::vector<QmvSpec> specs;
    for (int i = 0; i < count && grouped; i++) {
        const eq_qmm_problem& p = problems[i];
        grouped = p.N % 16 == 0 && aligned(p.x, 16) && aligned(p.w, 16) &&
                  decode_rows(M, bits, group_size, p.N % 128 == 0 && p.K % 64 == 0 && aligned(p.y, 8));
        specs.push_back(QmvSpec{static_cast<const uint16_t*>(p.x), p.w, p.scales, p.biases, static_cast<uint16_t*>(p.y),
                                int(p.N), int(p.K), int(p.N)});
    }
    if (grouped && launch_qmv_batched(bits, group_size, scale_dtype, specs.data(), count, int(M), st, x_dtype))
        return check_launch("quantized_matmul_batched (qmv)");
    // Otherwise one call per problem (same results: every problem runs the
    // same kernels either way).
    for (int i = 0; i < count; i++) {
        const eq_qmm_problem& p = problems[i];
        const int r = eq_quantized_matmul(p.y, p.x, p.w, p.scales, p.biases, M, p.N, p.K, transpose, group_size, bits,
                                          mode, x_dtype, scale_dtype, stream);
        if (r != 0) {
            const std::string msg = "problem " + std::to_string(i) + ": " + eq_last_error();
            set_error(msg);
            return r;
        }
    }
    return 0;
}

// A device byte range [p, p + bytes).
struct ByteRange {
    const void* p;
    int64_t bytes;
};

static bool ranges_overlap(const ByteRange& a, const ByteRange& b) {
    if (!a.p || !b.p || a.bytes <= 0 || b.bytes <= 0) return false;
    const uintptr_t x = reinterpret_cast<uintptr_t>(a.p), y = reinterpret_cast<uintptr_t>(b.p);
    return x < y + uintptr_t(b.bytes) && y < x + uintptr_t(a.bytes);
}

extern "C" int eq_quantized_matmul_batched_prologue(const eq_qmm_problem* problems, int count, int64_t M,
                                                    bool transpose, int group_size, int bits, const char* mode,
                                                    int x_dtype, int scale_dtype,
                                                    const eq_activation_prologue* prologue, eq_stream_t stream) {
    clear_error();
    if (check_mode(mode) || check_gs_bits(group_size, bits)) return 1;
    if (!prologue || (prologue->kind != EQ_PROLOGUE_SILU_MUL && prologue->kind != EQ_PROLOGUE_RMS_NORM)) {
        set_error("prologue: kind must be EQ_PROLOGUE_SILU_MUL or EQ_PROLOGUE_RMS_NORM");
        return 1;
    }
    const eq_activation_prologue& pr = *prologue;
    if (count < 1 || count > 8 || !problems) {
        set_error("prologue: 1 to 8 problems");
        return 1;
    }
    if (M != 1 || !transpose || x_dtype != EQ_DTYPE_BF16 || scale_dtype != EQ_DTYPE_BF16 || group_size != 64 ||
        (bits != 4 && bits != 8)) {
        set_error("prologue: supported for M = 1, transpose = true, bf16 activations and scales, group size 64, "
                  "4- or 8-bit codes");
        return 1;
    }
    const void* x = problems[0].x;
    const int64_t K = problems[0].K;
    std::vector<QmvSpec> specs;
    for (int i = 0; i < count; i++) {
        const eq_qmm_problem& p = problems[i];
        if (!p.y || !p.x || !p.w || !p.scales) {
            set_error("problem " + std::to_string(i) + ": null pointer argument");
            return 1;
        }
        if (p.x != x || p.K != K) {
            set_error("prologue: all problems must share one input x");
            return 1;
        }
        if (p.N <= 0 || p.N > INT32_MAX || p.N % 16 != 0 || !aligned(p.w, 16)) {
            set_error("problem " + std::to_string(i) + ": N must be a positive multiple of 16, w 16-byte aligned");
            return 1;
        }
        specs.push_back(QmvSpec{static_cast<const uint16_t*>(p.x), p.w, p.scales, p.biases, static_cast<uint16_t*>(p.y),
                                int(p.N), int(p.K), int(p.N)});
    }
    if (K <= 0 || K % 64 != 0 || K > INT32_MAX || !aligned(x, 16)) {
        set_error("prologue: K must be a positive multiple of 64 and x 16-byte aligned");
        return 1;
    }
    const int64_t bytes = K * 2;
    if (pr.kind == EQ_PROLOGUE_SILU_MUL) {
        if (!pr.second || !aligned(pr.second, 16)) {
            set_error("prologue: silu_mul needs a 16-byte aligned second input");
            return 1;
        }
    } else {
        if (K > 4096) {
            set_error("prologue: rms_norm takes rows of at most 4096 values");
            return 1;
        }
        if (!pr.weight || !aligned(pr.weight, 16) || (pr.second && !aligned(pr.second, 16)) ||
            (pr.hidden_out && !aligned(pr.hidden_out, 16))) {
            set_error("prologue: rms_norm needs a weight and 16-byte aligned vectors");
            return 1;
        }
        if (!(pr.eps >= 0.f)) {
            set_error("prologue: eps must be >= 0");
            return 1;
        }
    }
    // Every workgroup reads x, the second input, the norm weight and the
    // weights of every problem while others write y_i and hidden_out: no
    // written range may overlap a read one or another written one.
    std::vector<ByteRange> reads{{x, bytes}, {pr.second, bytes}};
    if (pr.kind == EQ_PROLOGUE_RMS_NORM) reads.push_back({pr.weight, bytes});
    std::vector<ByteRange> writes;
    for (int i = 0; i < count; i++) {
        const eq_qmm_problem& p = problems[i];
        const int64_t G = K / group_size;
        reads.push_back({p.w, p.N * K * bits / 8});
        reads.push_back({p.scales, p.N * G * 2});
        reads.push_back({p.biases, p.N * G * 2});
        writes.push_back({p.y, p.N * 2});
    }
    if (pr.kind == EQ_PROLOGUE_RMS_NORM) writes.push_back({pr.hidden_out, bytes});
    for (size_t i = 0; i < writes.size(); i++) {
        for (const ByteRange& r : reads)
            if (ranges_overlap(writes[i], r)) {
                set_error("prologue: an output (y or hidden_out) overlaps an input (x, the second input, the norm "
                          "weight or a problem's weights, scales or biases)");
                return 1;
            }
        for (size_t j = i + 1; j < writes.size(); j++)
            if (ranges_overlap(writes[i], writes[j])) {
                set_error("prologue: outputs (y of each problem, hidden_out) must not overlap each other");
                return 1;
            }
    }
    QmvPrologue q{pr.kind, static_cast<const uint16_t*>(pr.second), static_cast<const uint16_t*>(pr.weight),
                  static_cast<uint16_t*>(pr.hidden_out), pr.eps};
    if (!launch_qmv_prologue(bits, group_size, scale_dtype, specs.data(), count, q,
                             reinterpret_cast<hipStream_t>(stream))) {
        set_error("prologue: these problems do not fit one decode launch (at most 8, shared LDS budget)");
        return 1;
    }
    return check_launch("quantized_matmul_batched_prologue");
}

extern "C" int eq_quantized_matmul_swiglu(void* out, const void* x, const uint32_t* w, const void* scales,
                                          const void* biases, int64_t F, int64_t K, int group_size, int bits,
                                          const char* mode, int x_dtype, int scale_dtype,
                                          const eq_activation_prologue* prologue, eq_stream_t stream) {
    clear_error();
    if (check_mode(mode) || check_gs_bits(group_size, bits)) return 1;
    if (prologue && prologue->kind != EQ_PROLOGUE_RMS_NORM) {
        set_error("swiglu: the prologue, when given, must be EQ_PROLOGUE_RMS_NORM");
        return 1;
    }
    if (x_dtype != EQ_DTYPE_BF16 || scale_dtype != EQ_DTYPE_BF16 || group_size != 64 || (bits != 4 && bits != 8)) {
        set_error("swiglu: supported for bf16 activations and scales, group size 64, 4- or 8-bit codes");
        return 1;
    }
    if (!out || !x || !w || !scales) {
        set_error("swiglu: null pointer argument");
        return 1;
    }
    if (F <= 0 || F % 8 != 0 || 2 * F > INT32_MAX || K <= 0 || K % 64 != 0 || K > INT32_MAX) {
        set_error("swiglu: F must be a positive multiple of 8 and K a positive multiple of 64");
        return 1;
    }
    if (!aligned(x, 16) || !aligned(w, 16)) {
        set_error("swiglu: x and w must be 16-byte aligned");
        return 1;
    }
    const int64_t bytes = K * 2;
    if (prologue) {
        const eq_activation_prologue& pr = *prologue;
        if (K > 4096) {
            set_error("swiglu: the rms_norm prologue takes rows of at most 4096 values");
            return 1;
        }
        if (!pr.weight || !aligned(pr.weight, 16) || (pr.second && !aligned(pr.second, 16)) ||
            (pr.hidden_out && !aligned(pr.hidden_out, 16))) {
            set_error("swiglu: rms_norm needs a weight and 16-byte aligned vectors");
            return 1;
        }
        if (!(pr.eps >= 0.f)) {
            set_error("swiglu: eps must be >= 0");
            return 1;
        }
    }
    // every workgroup reads x (and the prologue's inputs) and the weights
    // while others write out (and hidden_out)
    const int64_t G = K / group_size, N = 2 * F;
    std::vector<ByteRange> reads{{x, bytes}, {w, N * K * bits / 8}, {scales, N * G * 2}, {biases, N * G * 2}};
    std::vector<ByteRange> writes{{out, F * 2}};
    if (prologue) {
        reads.push_back({prologue->second, bytes});
        reads.push_back({prologue->weight, bytes});
        writes.push_back({prologue->hidden_out, bytes});
    }
    for (size_t i = 0; i < writes.size(); i++) {
        for (const ByteRange& r : reads)
            if (ranges_overlap(writes[i], r)) {
                set_error("swiglu: an output (out or hidden_out) overlaps an input");
                return 1;
            }
        for (size_t j = i + 1; j < writes.size(); j++)
            if (ranges_overlap(writes[i], writes[j])) {
                set_error("swiglu: out and hidden_out must not overlap");
                return 1;
            }
    }
    const QmvSpec spec{static_cast<const uint16_t*>(x), w, scales, biases, static_cast<uint16_t*>(out), int(N), int(K),
                       int(N)};
    QmvPrologue q{};
    if (prologue)
        q = QmvPrologue{prologue->kind, static_cast<const uint16_t*>(prologue->second),
                        static_cast<const uint16_t*>(prologue->weight), static_cast<uint16_t*>(prologue->hidden_out),
                        prologue->eps};
    if (!launch_qmv_swiglu(bits, spec, prologue ? &q : nullptr, reinterpret_cast<hipStream_t>(stream))) {
        set_error("swiglu: this shape does not fit one decode launch (K a multiple of the code block, shared LDS "
                  "budget)");
        return 1;
    }
    return check_launch("quantized_matmul_swiglu");
}

extern "C" int eq_quantize(uint32_t* w_out, void* scales, void* biases, const void* w, int64_t rows, int64_t cols,
                           int group_size, int bits, const char* mode, int dtype, eq_stream_t stream) {
    clear_error();
    QuantMode qm;
    if (parse_mode(mode, qm)) return 1;
    if (qm == kModeMxFp4) {
        // E2M1 codes and E8M0 scale bytes, no biases (the biases argument must be null)
        if (check_mxfp4(group_size, bits, EQ_DTYPE_U8, biases)) return 1;
        if (!valid_dtype(dtype)) {
            set_error("invalid dtype code");
            return 1;
        }
        if (rows < 0 || cols < 0 || cols % 32 != 0) {
            set_error("cols must be a non-negative multiple of group_size");
            return 1;
        }
        if (rows == 0 || cols == 0) return 0;
        if (!w_out || !scales || !w) {
            set_error("null pointer argument");
            return 1;
        }
        return mxfp4_quantize(w_out, static_cast<uint8_t*>(scales), w, rows, cols, dtype,
                              reinterpret_cast<hipStream_t>(stream));
    }
    if (check_gs_bits(group_size, bits)) return 1;
    if (!valid_dtype(dtype)) {
        set_error("invalid dtype code");
        return 1;
    }
    if (rows < 0 || cols < 0 || (cols % group_size) != 0) {
        set_error("cols must be a non-negative multiple of group_size");
        return 1;
    }
    if (!check_packed_row(cols, bits)) return 1;
    if (rows == 0 || cols == 0) return 0;
    if (!w_out || !scales || !biases || !w) {
        set_error("null pointer argument");
        return 1;
    }
    const int64_t groups = rows * (cols / group_size);
    if ((groups + 255) / 256 > INT32_MAX) {
        set_error("tensor too large");
        return 1;
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const dim3 grid(unsigned((groups + 255) / 256));
    with_bits(bits, [&](auto bc) {
        constexpr int B = decltype(bc)::value;
        with_dtype(dtype, [&](auto tt) {
            typedef decltype(tt) T;
            typedef typename T::storage S;
            S* sp = static_cast<S*>(scales);
            S* bp = static_cast<S*>(biases);
            const S* wp = static_cast<const S*>(w);
            if constexpr (32 % B != 0) {
                // a unit of whole words: one group, or two at group size 16
                const int gpu = (int64_t(group_size) * B) % 32 == 0 ? 1 : 2;
                const int64_t units = groups / gpu;
                quantize_odd_kernel<B, T><<<dim3(unsigned((units + 255) / 256)), 256, 0, st>>>(w_out, sp, bp, wp, units,
                                                                                             group_size, gpu);
            } else if (aligned(w, 16) && aligned(w_out, 16) && fast_group_size(group_size)) {
                if (group_size == 32) quantize_vec_kernel<B, T, 32><<<grid, 256, 0, st>>>(w_out, sp, bp, wp, groups);
                else if (group_size == 64) quantize_vec_kernel<B, T, 64><<<grid, 256, 0, st>>>(w_out, sp, bp, wp, groups);
                else quantize_vec_kernel<B, T, 128><<<grid, 256, 0, st>>>(w_out, sp, bp, wp, groups);
            } else {
                quantize_kernel<B, T><<<grid, 256, 0, st>>>(w_out, sp, bp, wp, groups, group_size);
            }
        });
    });
    return check_launch("quantize");
}

extern "C" int eq_dequantize(void* out, const uint32_t* w, const void* scales, const void* biases, int64_t rows,
                             int64_t cols, int group_size, int bits, const char* mode, int scale_dtype,
                             int out_dtype, eq_stream_t stream) {
    clear_error();
    QuantMode qm;
    if (parse_mode(mode, qm)) return 1;
    if (qm == kModeMxFp4) {
        if (check_mxfp4(group_size, bits, scale_dtype, biases)) return 1;
        if (!valid_dtype(out_dtype)) {
            set_error("invalid dtype code");
            return 1;
        }
        if (rows < 0 || cols < 0 || cols % 32 != 0) {
            set_error("cols must be a non-negative multiple of group_size");
            return 1;
        }
        if (rows == 0 || cols == 0) return 0;
        if (!out || !w || !scales) {
            set_error("null pointer argument");
            return 1;
        }
        return mxfp4_dequantize(out, w, static_cast<const uint8_t*>(scales), rows, cols, out_dtype,
                                reinterpret_cast<hipStream_t>(stream));
    }
    if (check_gs_bits(group_size, bits)) return 1;
    if (!valid_dtype(scale_dtype) || !valid_dtype(out_dtype)) {
        set_error("invalid dtype code");
        return 1;
    }
    if (rows < 0 || cols < 0 || (cols % group_size) != 0) {
        set_error("cols must be a non-negative multiple of group_size");
        return 1;
    }
    if (!check_packed_row(cols, bits)) return 1;
    if (rows == 0 || cols == 0) return 0;
    if (!out || !w || !scales) {
        set_error("null pointer argument");
        return 1;
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int64_t words = rows * cols * bits / 32;
    const dim3 grid(unsigned((words + 255) / 256));
    with_bits(bits, [&](auto bc) {
        constexpr int B = decltype(bc)::value;
        with_dtype(scale_dtype, [&](auto stt) {
            typedef decltype(stt) ST;
            with_dtype(out_dtype, [&](auto ot) {
                typedef decltype(ot) OT;
                typedef typename OT::storage OS;
                typedef typename ST::storage SS;
                if constexpr (32 % B != 0) {
                    constexpr int CPT = B == 6 ? 16 : 32;
                    const int64_t units = rows * cols / CPT;
                    dequant_odd_kernel<B, ST, OT><<<dim3(unsigned((units + 255) / 256)), 256, 0, st>>>(
                        static_cast<OS*>(out), w, static_cast<const SS*>(scales), static_cast<const SS*>(biases), rows,
                        cols, group_size);
                } else if (aligned(out, 16)) {
                    auto go = [&](auto kernel) {
                        kernel<<<grid, 256, 0, st>>>(static_cast<OS*>(out), w, static_cast<const SS*>(scales),
                                                     static_cast<const SS*>(biases), rows, cols, group_size);
                    };
                    if (group_size == 32) go(dequant_kernel<B, ST, OT, true, 32>);
                    else if (group_size == 64) go(dequant_kernel<B, ST, OT, true, 64>);
                    else if (group_size == 128) go(dequant_kernel<B, ST, OT, true, 128>);
                    else go(dequant_kernel<B, ST, OT, true>);
                } else
                    dequant_kernel<B, ST, OT, false><<<grid, 256, 0, st>>>(
                        static_cast<OS*>(out), w, static_cast<const SS*>(scales), static_cast<const SS*>(biases), rows,
                        cols, group_size);
            });
        });
    });
    return check_launch("dequantize");
}
