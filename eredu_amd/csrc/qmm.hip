// Prefill-shaped quantized matmul (M > 16, bf16 activations, transpose = true)
// on gfx950 matrix cores.
//
// y = x . W^T with W[n, k] = s[n, k/gs] * q[n, k] + b[n, k/gs]
// (safemlx/src/ops/quantization.rs:190-226, QuantizedLinear's layout).
//
// Work layout.  A workgroup of 4 waves owns a 128 (m) x 256 (n) output tile
// and walks K in chunks of 64.  Wave w owns the 64 columns [64w, 64w + 64) and
// all 128 rows: 4 x 2 tiles of v_mfma_f32_32x32x16_bf16 with f32 accumulators.
//
//  * Weights never touch LDS.  Each wave dequantizes only its own columns,
//    straight from a 16-byte load per lane into the B-operand registers:
//    lane l reads row n = l % 32 of a 32-column block, 32 consecutive codes
//    starting at k = 32 * (l / 32); code word t of those feeds MFMA step t.
//    w = s*q + b is one f32 FMA per code and one v_cvt_pk_bf16_f32 per pair,
//    and is used by the 4 row blocks of the tile.
//  * Activations go through LDS (shared by the 4 waves), double buffered:
//    the chunk k+1 is loaded into registers while chunk k is computed, then
//    written to the other buffer.  16-byte chunks of a row are stored at
//    chunk c ^ (row & 7), so the rows of one A operand read different banks.
//    A operand of step t for lane (m, kb) = x[m][k0 + 32 kb + 8 t .. + 8],
//    matching the codes the B lane (n, kb) holds for step t.
//  * All global reads are buffer loads: rows past M or N and chunks past K
//    read as zero, so any M and N work.
//  * Tiles are assigned so that the workgroups one XCD receives cover few
//    row blocks of x (which then stay in that XCD's L2).
#include "eq_common.hpp"

namespace eq {

typedef uint32_t q_u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 q_bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kBM = 128, kBN = 256, kBK = 64;
constexpr int kQmmThreads = 256;
constexpr int kLdsBuf = kBM * kBK * 2;  // bytes per activation buffer

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const q_bf16x2 p = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};  // RNE (v_cvt_pk_bf16_f32)
    return __builtin_bit_cast(uint32_t, p);
}

// 8 codes in k order -> 4 registers of bf16 pairs (s*q + b).
template <int BITS>
__device__ __forceinline__ q_u32x4 dequant8(const uint32_t* words, float s, float b);
template <>
__device__ __forceinline__ q_u32x4 dequant8<4>(const uint32_t* words, float s, float b) {
    const uint32_t w = words[0];
    uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;  // codes 2i | 2i+1 in byte i
    // (opaque to the optimiser, so that each code converts with one
    // v_cvt_f32_ubyte{0..3} instead of a bit-field extract plus a convert)
    asm volatile("" : "+v"(lo), "+v"(hi));
    q_u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; i++)
        r[i] = pack_bf16x2(fmaf(s, float((lo >> (8 * i)) & 0xffu), b), fmaf(s, float((hi >> (8 * i)) & 0xffu), b));
    return r;
}
template <>
__device__ __forceinline__ q_u32x4 dequant8<8>(const uint32_t* words, float s, float b) {
    q_u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t w = words[i >> 1];
        const int sh = (i & 1) * 16;
        r[i] = pack_bf16x2(fmaf(s, float((w >> sh) & 0xffu), b), fmaf(s, float((w >> (sh + 8)) & 0xffu), b));
    }
    return r;
}

// Codes and parameters of one chunk for one wave: 2 column blocks x 32 codes.
template <int BITS>
struct QmmB {
    static constexpr int WORDS = BITS;  // 32 codes * BITS / 32
    uint32_t w[2][WORDS];
    uint16_t s[2], b[2];
};

template <int BITS, int GS>
__device__ __forceinline__ void qmm_load_b(QmmB<BITS>& B, __amdgpu_buffer_rsrc_t wr, __amdgpu_buffer_rsrc_t sr,
                                           __amdgpu_buffer_rsrc_t br, const uint32_t* woff, const uint32_t* soff,
                                           int k0) {
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t wo = woff[j] + uint32_t(k0) * BITS / 8;
#pragma unroll
        for (int i = 0; i < QmmB<BITS>::WORDS / 4; i++) {
            const q_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(wr, wo + 16 * i, 0, 0);
            B.w[j][4 * i] = v[0], B.w[j][4 * i + 1] = v[1], B.w[j][4 * i + 2] = v[2], B.w[j][4 * i + 3] = v[3];
        }
        const uint32_t so = soff[j] + uint32_t(k0 / GS) * 2u;
        B.s[j] = __builtin_amdgcn_raw_buffer_load_b16(sr, so, 0, 0);
        B.b[j] = __builtin_amdgcn_raw_buffer_load_b16(br, so, 0, 0);
    }
}

template <typename ST>
__device__ __forceinline__ float qmm_param(uint16_t bits);
template <>
__device__ __forceinline__ float qmm_param<BF16T>(uint16_t bits) { return bf16_bits_to_f32(bits); }
template <>
__device__ __forceinline__ float qmm_param<F16T>(uint16_t bits) { return f16_bits_to_f32(bits); }

template <int BITS, int GS, typename ST>
__global__ __launch_bounds__(kQmmThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void qmm_mfma_kernel(
    uint16_t* __restrict__ y, const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases, int M, int N, int K, int mtiles,
    int ntiles) {
    __shared__ __attribute__((aligned(16))) char lds[2 * kLdsBuf];

    // Tile of this workgroup: the workgroups of one XCD (id % 8) take a
    // contiguous run of row-major tiles, i.e. few row blocks of x.
    const int T = mtiles * ntiles;
    int bid = blockIdx.x;
    if ((T & 7) == 0) bid = (bid & 7) * (T >> 3) + (bid >> 3);
    const int tm = bid / ntiles, tn = bid % ntiles;
    const int m0 = tm * kBM, n0 = tn * kBN;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, kb = lane >> 5;
    const int G = K / GS;

    const __amdgpu_buffer_rsrc_t xr = raw_rsrc(x, uint32_t(M) * uint32_t(K) * 2u);
    const __amdgpu_buffer_rsrc_t wr = raw_rsrc(w, uint32_t(N) * uint32_t(K) * BITS / 8u);
    const __amdgpu_buffer_rsrc_t sr = raw_rsrc(scales, uint32_t(N) * uint32_t(G) * 2u);
    const __amdgpu_buffer_rsrc_t br = biases ? raw_rsrc(biases, uint32_t(N) * uint32_t(G) * 2u) : sr;
    const float bias_on = biases ? 1.f : 0.f;

    // Activation staging: thread tid copies the 16-byte chunks q = tid + 256 i
    // (row q / 8, chunk q % 8) of each 128 x 64 tile.
    uint32_t a_goff[4], a_loff[4];
    bool a_in[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int q = tid + kQmmThreads * i, row = q >> 3, c = q & 7;
        a_in[i] = m0 + row < M;
        a_goff[i] = (uint32_t(m0 + row) * uint32_t(K) + uint32_t(8 * c)) * 2u;
        a_loff[i] = uint32_t(row * (kBK * 2) + ((c ^ (row & 7)) << 4));
    }
    auto load_a = [&](q_u32x4* r, int k0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = (tid + kQmmThreads * i) & 7;
            const bool in = a_in[i] && k0 + 8 * c < K;
            r[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, in ? a_goff[i] + uint32_t(k0) * 2u : kOutOfRange, 0, 0);
        }
    };
    auto store_a = [&](const q_u32x4* r, int buf) {
#pragma unroll
        for (int i = 0; i < 4; i++) *reinterpret_cast<q_u32x4*>(lds + buf * kLdsBuf + a_loff[i]) = r[i];
    };

    // Weight rows of this lane: columns n0 + 64 wave + 32 j + l32, codes from 32 kb.
    uint32_t woff[2], soff[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t n = uint32_t(n0 + 64 * wave + 32 * j + l32);
        woff[j] = n * uint32_t(K) * BITS / 8u + uint32_t(32 * kb) * BITS / 8u;
        soff[j] = (n * uint32_t(G)) * 2u + uint32_t((32 * kb) / GS) * 2u;
    }
    // (a lane's 32 codes lie in one group: group sizes are multiples of 32 and
    // chunks start at multiples of 64)

    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x16{};

    const int nchunks = (K + kBK - 1) / kBK;
    q_u32x4 areg[4];
    QmmB<BITS> bcur, bnxt;
    load_a(areg, 0);
    qmm_load_b<BITS, GS>(bcur, wr, sr, br, woff, soff, 0);
    store_a(areg, 0);
    __syncthreads();

    // A-operand LDS offsets of this lane for step t: row 32 mi + l32, chunk (4 kb + t) ^ (row & 7).
    uint32_t aoff[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
        for (int t = 0; t < 4; t++)
            aoff[mi][t] = uint32_t((32 * mi + l32) * (kBK * 2) + (((4 * kb + t) ^ (l32 & 7)) << 4));

    for (int c = 0; c < nchunks; c++) {
        const int buf = c & 1;
        // codes of this lane past a ragged end of K get zero scale and bias
        const float live = c * kBK + 32 * kb < K ? 1.f : 0.f;
        const bool more = c + 1 < nchunks;
        // Prefetch chunk c + 1 (re-reads chunk c on the last iteration: in cache).
        const int kn = more ? (c + 1) * kBK : c * kBK;
        load_a(areg, kn);
        qmm_load_b<BITS, GS>(bnxt, wr, sr, br, woff, soff, kn);
        if (opaque_one()) {
            asm volatile("" ::: "memory");
            q_u32x4 bq[2][4];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const float s = qmm_param<ST>(bcur.s[j]) * live;
                const float b = qmm_param<ST>(bcur.b[j]) * bias_on * live;
#pragma unroll
                for (int t = 0; t < 4; t++) bq[j][t] = dequant8<BITS>(&bcur.w[j][t * BITS / 4], s, b);
            }
#pragma unroll
            for (int t = 0; t < 4; t++) {
                bf16x8 a[4];
#pragma unroll
                for (int mi = 0; mi < 4; mi++)
                    a[mi] = *reinterpret_cast<const bf16x8*>(lds + buf * kLdsBuf + aoff[mi][t]);
#pragma unroll
                for (int mi = 0; mi < 4; mi++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[mi][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            a[mi], __builtin_bit_cast(bf16x8, bq[j][t]), acc[mi][j], 0, 0, 0);
            }
        }
        if (more) store_a(areg, buf ^ 1);
        __syncthreads();
        bcur = bnxt;
    }

    // D layout of the 32x32 MFMA: register r of lane l is row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + 64 * wave + 32 * j + l32;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + 32 * mi + 8 * (r >> 2) + 4 * kb + (r & 3);
                if (m < M && n < N) y[int64_t(m) * N + n] = uint16_t(f32_to_bf16_bits(acc[mi][j][r]));
            }
        }
}

template <int BITS, int GS, typename ST>
static void launch_qmm_t(uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s, const void* b, int M,
                         int N, int K, hipStream_t st) {
    const int mtiles = (M + kBM - 1) / kBM, ntiles = (N + kBN - 1) / kBN;
    qmm_mfma_kernel<BITS, GS, ST><<<dim3(unsigned(mtiles * ntiles)), dim3(kQmmThreads), 0, st>>>(
        y, x, w, static_cast<const uint16_t*>(s), static_cast<const uint16_t*>(b), M, N, K, mtiles, ntiles);
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
// K % gs == 0, 16-byte aligned x and w, scale dtype bf16 or f16, buffers
// below 2^31 bytes.
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
