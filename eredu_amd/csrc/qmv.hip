// Decode-shaped quantized matmul (M <= 16, bf16 activations, transpose = true)
// on gfx950 matrix cores.
//
// y[m, n] = sum_g s[n,g] * sum_{k in g} x[m,k] q[n,k] + b[n,g] * sum_{k in g} x[m,k]
// (the affine contract of safemlx/src/ops/quantization.rs:190-226 with W = [N, K]).
//
// Layout of the work.  A workgroup owns 16 output features (rows of W) and its
// waves split K by whole quantization groups.  Each wave runs
// v_mfma_f32_16x16x32_bf16 with A = activations (16 rows, M of them real) and
// B = codes of the 16 rows, one MFMA per 32 codes:
//   lane l: column n = l % 16, k-slot block kq = l / 16.
//   Per group a lane loads the gs/4 consecutive codes of row n starting at
//   kq*gs/4 (a single 4/8/16/32-byte load), so every MFMA sums codes of one
//   group only and the per-group scale can be applied to its result.
// 4-bit codes become bf16 (128 + q) with one byte permute and one and-or per
// pair; 8-bit codes go through v_cvt_f32_ubyte.  A second MFMA against a
// constant all-ones B gives sum_k x per group in the same accumulator layout,
// which carries both the bias term and the removal of the +128 offset.
// Per group each lane then does acc += s * t + (b - 128 s) * xs in f32.
// Waves reduce through LDS; the result is rounded once to bf16.
//
// The weight stream is read exactly once with coalesced loads; activations
// (at most 16 x K bf16) stay in L1/L2.
#include "eq_common.hpp"

namespace eq {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int N> struct WordVec;
template <> struct WordVec<1> {
    static __device__ __forceinline__ void load(const uint32_t* p, uint32_t* o) { o[0] = *p; }
};
template <> struct WordVec<2> {
    static __device__ __forceinline__ void load(const uint32_t* p, uint32_t* o) {
        const u32x2 v = *reinterpret_cast<const u32x2*>(p);
        o[0] = v[0]; o[1] = v[1];
    }
};
template <> struct WordVec<4> {
    static __device__ __forceinline__ void load(const uint32_t* p, uint32_t* o) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(p);
        o[0] = v[0]; o[1] = v[1]; o[2] = v[2]; o[3] = v[3];
    }
};
template <> struct WordVec<8> {
    static __device__ __forceinline__ void load(const uint32_t* p, uint32_t* o) {
        WordVec<4>::load(p, o);
        WordVec<4>::load(p + 4, o + 4);
    }
};

// 8 consecutive 4-bit codes (one word, LSB first) -> 8 bf16 values 128 + q,
// in k order: pair i holds codes 2i (low half) and 2i+1 (high half).
__device__ __forceinline__ bf16x8 unpack4_bf16_offset128(uint32_t w) {
    const uint32_t t = w >> 4;
    u32x4 p;
    // byte 0 <- w.byte i (low nibble = code 2i), byte 2 <- t.byte i (low nibble = code 2i+1)
    p[0] = __builtin_amdgcn_perm(t, w, 0x0c040c00u);
    p[1] = __builtin_amdgcn_perm(t, w, 0x0c050c01u);
    p[2] = __builtin_amdgcn_perm(t, w, 0x0c060c02u);
    p[3] = __builtin_amdgcn_perm(t, w, 0x0c070c03u);
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = (p[i] & 0x000f000fu) | 0x43004300u;  // bf16 0x43XX = 128 + X
    return __builtin_bit_cast(bf16x8, p);
}

// 8 consecutive 8-bit codes (two words) -> 8 bf16 values q, exact.
__device__ __forceinline__ bf16x8 unpack8_bf16(uint32_t w0, uint32_t w1) {
    u32x4 p;
    const uint32_t w[2] = {w0, w1};
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t f0 = __float_as_uint(float(w[h] & 0xffu));
        const uint32_t f1 = __float_as_uint(float((w[h] >> 8) & 0xffu));
        const uint32_t f2 = __float_as_uint(float((w[h] >> 16) & 0xffu));
        const uint32_t f3 = __float_as_uint(float(w[h] >> 24));
        // high halves of the f32 images are the exact bf16 images (<= 8 significant bits)
        p[2 * h] = __builtin_amdgcn_perm(f1, f0, 0x07060302u);
        p[2 * h + 1] = __builtin_amdgcn_perm(f3, f2, 0x07060302u);
    }
    return __builtin_bit_cast(bf16x8, p);
}

constexpr int kQmvMaxWaves = 16;
constexpr int kQmvUnroll = 4;

template <int BITS, int GS, typename ST, int MREG>
__global__ __launch_bounds__(64 * kQmvMaxWaves) void qmv_mfma_kernel(
    uint16_t* __restrict__ y, const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const typename ST::storage* __restrict__ scales, const typename ST::storage* __restrict__ biases, int M,
    int N, int K, int groups_per_wave) {
    constexpr int CPL = GS / 4;             // codes per lane per group
    constexpr int WPL = CPL * BITS / 32;    // words per lane per group
    constexpr int STEPS = CPL / 8;          // MFMAs per group
    constexpr int WPG = GS * BITS / 32;     // words per group per row
    __shared__ float red[kQmvMaxWaves][16][16];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nwaves = blockDim.x >> 6;
    const int ln = lane & 15;
    const int kq = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int G = K / GS;
    const int g_begin = wave * groups_per_wave;
    const int g_end = min(G, g_begin + groups_per_wave);

    const uint32_t* wrow = w + int64_t(n0 + ln) * (int64_t(K) * BITS / 32) + kq * WPL;
    const bool x_live = ln < M;
    const uint16_t* xrow = x + int64_t(x_live ? ln : 0) * K + kq * CPL;
    const typename ST::storage* srow = scales + int64_t(n0 + ln) * G;
    const typename ST::storage* brow = biases ? biases + int64_t(n0 + ln) * G : nullptr;

    u32x4 ones_bits = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
    const bf16x8 ones = __builtin_bit_cast(bf16x8, ones_bits);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};

    for (int g0 = g_begin; g0 < g_end; g0 += kQmvUnroll) {
        uint32_t wd[kQmvUnroll][WPL];
        bf16x8 xa[kQmvUnroll][STEPS];
        float sc[kQmvUnroll], bi[kQmvUnroll];
#pragma unroll
        for (int u = 0; u < kQmvUnroll; u++) {
            const int g = g0 + u;
            if (g < g_end) {
                WordVec<WPL>::load(wrow + int64_t(g) * WPG, wd[u]);
                sc[u] = load_param<ST>(srow, g);
                bi[u] = brow ? load_param<ST>(brow, g) : 0.f;
#pragma unroll
                for (int j = 0; j < STEPS; j++) {
                    if (x_live)
                        xa[u][j] = *reinterpret_cast<const bf16x8*>(xrow + g * GS + 8 * j);
                    else
                        xa[u][j] = bf16x8{};
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kQmvUnroll; u++) {
            if (g0 + u < g_end) {
                f32x4 t = {0.f, 0.f, 0.f, 0.f};
                f32x4 xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < STEPS; j++) {
                    bf16x8 bq;
                    if (BITS == 4)
                        bq = unpack4_bf16_offset128(wd[u][j]);
                    else
                        bq = unpack8_bf16(wd[u][2 * j], wd[u][2 * j + 1]);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[u][j], bq, t, 0, 0, 0);
                    xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[u][j], ones, xs, 0, 0, 0);
                }
                const float beff = BITS == 4 ? bi[u] - 128.f * sc[u] : bi[u];
#pragma unroll
                for (int r = 0; r < MREG; r++) acc[r] = fmaf(sc[u], t[r], fmaf(beff, xs[r], acc[r]));
            }
        }
    }

    // D layout: lane holds rows m = 4*kq + r of column n = ln.
#pragma unroll
    for (int r = 0; r < MREG; r++) {
        const int m = 4 * kq + r;
        if (m < M) red[wave][m][ln] = acc[r];
    }
    __syncthreads();
    for (int t = threadIdx.x; t < 16 * M; t += blockDim.x) {
        const int m = t >> 4, n = t & 15;
        float v = 0.f;
        for (int i = 0; i < nwaves; i++) v += red[i][m][n];
        y[int64_t(m) * N + n0 + n] = uint16_t(f32_to_bf16_bits(v));
    }
}

// Host-side launcher; returns false if this shape/dtype is not covered.
template <int BITS, int GS, typename ST>
static void launch_qmv_t(uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s, const void* b, int M,
                         int N, int K, hipStream_t st) {
    const int G = K / GS;
    int waves = G / 4;
    waves = waves < 1 ? 1 : (waves > kQmvMaxWaves ? kQmvMaxWaves : waves);
    const int gpw = (G + waves - 1) / waves;
    waves = (G + gpw - 1) / gpw;
    const dim3 grid(unsigned(N / 16)), block(unsigned(64 * waves));
    typedef typename ST::storage S;
    if (M == 1)
        qmv_mfma_kernel<BITS, GS, ST, 1><<<grid, block, 0, st>>>(y, x, w, static_cast<const S*>(s),
                                                                 static_cast<const S*>(b), M, N, K, gpw);
    else
        qmv_mfma_kernel<BITS, GS, ST, 4><<<grid, block, 0, st>>>(y, x, w, static_cast<const S*>(s),
                                                                 static_cast<const S*>(b), M, N, K, gpw);
}

template <int BITS, typename ST>
static bool launch_qmv_gs(int gs, uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s, const void* b,
                          int M, int N, int K, hipStream_t st) {
    switch (gs) {
    case 32: launch_qmv_t<BITS, 32, ST>(y, x, w, s, b, M, N, K, st); return true;
    case 64: launch_qmv_t<BITS, 64, ST>(y, x, w, s, b, M, N, K, st); return true;
    case 128: launch_qmv_t<BITS, 128, ST>(y, x, w, s, b, M, N, K, st); return true;
    default: return false;
    }
}

// Entry used by the dispatcher (api.hip).  Preconditions checked there:
// x bf16, transpose, 1 <= M <= 16, N % 16 == 0, K % gs == 0, 16-byte aligned
// x and weight rows, scale dtype bf16 or f16.
bool launch_qmv_mfma(int bits, int gs, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w,
                     const void* s, const void* b, int M, int N, int K, hipStream_t st) {
    if (bits == 4) {
        if (scale_dtype == EQ_DTYPE_BF16) return launch_qmv_gs<4, BF16T>(gs, y, x, w, s, b, M, N, K, st);
        if (scale_dtype == EQ_DTYPE_F16) return launch_qmv_gs<4, F16T>(gs, y, x, w, s, b, M, N, K, st);
    } else if (bits == 8) {
        if (scale_dtype == EQ_DTYPE_BF16) return launch_qmv_gs<8, BF16T>(gs, y, x, w, s, b, M, N, K, st);
        if (scale_dtype == EQ_DTYPE_F16) return launch_qmv_gs<8, F16T>(gs, y, x, w, s, b, M, N, K, st);
    }
    return false;
}

}  // namespace eq
