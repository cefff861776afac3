// Prefill-shaped quantized matmul (M > 16, bf16 activations, transpose = true)
// on gfx950 matrix cores.
//
// y = x . W^T with W[n, k] = s[n, k/gs] * q[n, k] + b[n, k/gs]
// (safemlx/src/ops/quantization.rs:190-226, QuantizedLinear's layout).
//
// Tiling: a workgroup of 4 waves owns a 128 (m) x 128 (n) output tile and
// walks K in steps of 64.  Per step it loads the activation tile (16 KB bf16)
// and the packed weight tile (4 or 8 KB) with 16-byte coalesced loads into
// registers one step ahead, dequantizes the weights in registers
// (w = s*q + b in f32, rounded once to bf16) and writes both tiles to LDS
// (rows padded by 16 bytes against bank conflicts).  Each wave computes a
// 64 x 64 sub-tile with 2 x 2 v_mfma_f32_32x32x16_bf16 accumulators in f32.
// Workgroup ids are remapped so that the workgroups one XCD receives share
// weight tiles in that XCD's L2.
#include "eq_common.hpp"

namespace eq {

typedef uint32_t q_u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBN = 128, kBK = 64, kLdsK = kBK + 8;

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

template <int BITS, int GS, typename ST>
__global__ __launch_bounds__(256) void qmm_mfma_kernel(uint16_t* __restrict__ y, const uint16_t* __restrict__ x,
                                                       const uint32_t* __restrict__ w,
                                                       const typename ST::storage* __restrict__ scales,
                                                       const typename ST::storage* __restrict__ biases, int M,
                                                       int N, int K, int mtiles) {
    __shared__ __attribute__((aligned(16))) uint16_t xs[kBM * kLdsK];
    __shared__ __attribute__((aligned(16))) uint16_t ws[kBN * kLdsK];

    int bid = blockIdx.x;
    const int nwg = gridDim.x;
    if ((nwg & 7) == 0) bid = (bid & 7) * (nwg >> 3) + (bid >> 3);  // consecutive tiles per XCD
    const int tn = bid / mtiles, tm = bid % mtiles;
    const int m0 = tm * kBM, n0 = tn * kBN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int lrow = tid >> 1, lhalf = tid & 1;
    const int G = K / GS;
    constexpr int WPT = BITS;  // words per thread per K step: 32 codes * BITS / 32

    const uint16_t* xsrc = x + int64_t(min(m0 + lrow, M - 1)) * K + lhalf * 32;
    const uint32_t* wsrc = w + int64_t(n0 + lrow) * (int64_t(K) * BITS / 32) + lhalf * WPT;
    const typename ST::storage* srow = scales + int64_t(n0 + lrow) * G;
    const typename ST::storage* brow = biases ? biases + int64_t(n0 + lrow) * G : nullptr;

    q_u32x4 xr[4];
    q_u32x4 wr[WPT / 4];
    float sc, bi;
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 4; i++) xr[i] = *reinterpret_cast<const q_u32x4*>(xsrc + k0 + 8 * i);
#pragma unroll
        for (int i = 0; i < WPT / 4; i++)
            wr[i] = *reinterpret_cast<const q_u32x4*>(wsrc + (int64_t(k0) * BITS / 32) + 4 * i);
        const int g = (k0 + lhalf * 32) / GS;
        sc = load_param<ST>(srow, g);
        bi = brow ? load_param<ST>(brow, g) : 0.f;
    };
    auto lstore = [&]() {
        q_u32x4* xd = reinterpret_cast<q_u32x4*>(xs + lrow * kLdsK + lhalf * 32);
#pragma unroll
        for (int i = 0; i < 4; i++) xd[i] = xr[i];
        uint32_t o[16];
        if (BITS == 4) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t word = wr[j >> 2][j & 3];
                const uint32_t lo = word & 0x0f0f0f0fu, hi = (word >> 4) & 0x0f0f0f0fu;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float ce = float((lo >> (8 * i)) & 0xffu);  // code 8j + 2i
                    const float co = float((hi >> (8 * i)) & 0xffu);  // code 8j + 2i + 1
                    o[4 * j + i] = pack_bf16x2(fmaf(sc, ce, bi), fmaf(sc, co, bi));
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const uint32_t word = wr[j >> 2][j & 3];
                const float c0 = float(word & 0xffu), c1 = float((word >> 8) & 0xffu);
                const float c2 = float((word >> 16) & 0xffu), c3 = float(word >> 24);
                o[2 * j] = pack_bf16x2(fmaf(sc, c0, bi), fmaf(sc, c1, bi));
                o[2 * j + 1] = pack_bf16x2(fmaf(sc, c2, bi), fmaf(sc, c3, bi));
            }
        }
        q_u32x4* wdst = reinterpret_cast<q_u32x4*>(ws + lrow * kLdsK + lhalf * 32);
#pragma unroll
        for (int i = 0; i < 4; i++) wdst[i] = q_u32x4{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x16{};

    const int l32 = lane & 31, lk = (lane >> 5) * 8;
    gload(0);
    for (int k0 = 0; k0 < K; k0 += kBK) {
        lstore();
        __syncthreads();
        if (k0 + kBK < K) gload(k0 + kBK);
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 16) {
            bf16x8 a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; i++)
                a[i] = *reinterpret_cast<const bf16x8*>(xs + (wm + 32 * i + l32) * kLdsK + kk + lk);
#pragma unroll
            for (int j = 0; j < 2; j++)
                b[j] = *reinterpret_cast<const bf16x8*>(ws + (wn + 32 * j + l32) * kLdsK + kk + lk);
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

    // D layout of 32x32 MFMA: register r of lane l is row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int n = n0 + wn + 32 * j + l32;
                if (m < M) y[int64_t(m) * N + n] = uint16_t(f32_to_bf16_bits(acc[i][j][r]));
            }
}

template <int BITS, int GS, typename ST>
static void launch_qmm_t(uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s, const void* b, int M,
                         int N, int K, hipStream_t st) {
    const int mtiles = (M + kBM - 1) / kBM, ntiles = N / kBN;
    typedef typename ST::storage S;
    qmm_mfma_kernel<BITS, GS, ST><<<dim3(unsigned(mtiles * ntiles)), dim3(256), 0, st>>>(
        y, x, w, static_cast<const S*>(s), static_cast<const S*>(b), M, N, K, mtiles);
}

template <int BITS, typename ST>
static bool launch_qmm_gs(int gs, uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s, const void* b,
                          int M, int N, int K, hipStream_t st) {
    switch (gs) {
    case 32: launch_qmm_t<BITS, 32, ST>(y, x, w, s, b, M, N, K, st); return true;
    case 64: launch_qmm_t<BITS, 64, ST>(y, x, w, s, b, M, N, K, st); return true;
    case 128: launch_qmm_t<BITS, 128, ST>(y, x, w, s, b, M, N, K, st); return true;
    default: return false;
    }
}

// Preconditions checked by the dispatcher (api.hip): x bf16, transpose,
// N % 128 == 0, K % 64 == 0, K % gs == 0, 16-byte aligned x and w,
// scale dtype bf16 or f16.
bool launch_qmm_mfma(int bits, int gs, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w,
                     const void* s, const void* b, int M, int N, int K, hipStream_t st) {
    if (bits == 4) {
        if (scale_dtype == EQ_DTYPE_BF16) return launch_qmm_gs<4, BF16T>(gs, y, x, w, s, b, M, N, K, st);
        if (scale_dtype == EQ_DTYPE_F16) return launch_qmm_gs<4, F16T>(gs, y, x, w, s, b, M, N, K, st);
    } else if (bits == 8) {
        if (scale_dtype == EQ_DTYPE_BF16) return launch_qmm_gs<8, BF16T>(gs, y, x, w, s, b, M, N, K, st);
        if (scale_dtype == EQ_DTYPE_F16) return launch_qmm_gs<8, F16T>(gs, y, x, w, s, b, M, N, K, st);
    }
    return false;
}

}  // namespace eq
