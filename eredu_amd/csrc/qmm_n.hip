// x . W with W [K, N] packed along N -- quantized_matmul with transpose =
// false (safemlx/src/ops/quantization.rs:190-226; the safemlx default) --
// for M <= 8 activation rows per batch: the values product of the quantized
// KV attention (eredu/src/backend/mlx/nn/tensor.rs:133-142, scores [.., 1, T]
// times values [.., T, D]) and small-batch x . W in general.
//
// y[m, n] = sum_k x[m, k] (s[k, n / gs] q[k, n] + b[k, n / gs])
//         = sum_k (x[m, k] s[k, g]) q[k, n] + sum_k x[m, k] b[k, g]:
// the bias term is shared by the columns of a group, so a code costs one
// convert and one FMA per activation row.
#include "eq_common.hpp"

#ifndef EQ_QMMN_UNROLL
#define EQ_QMMN_UNROLL 4  // rows per lane and step (M = 1 kernel)
#endif
#ifndef EQ_QMMN_TARGET
#define EQ_QMMN_TARGET 1024  // workgroups the K split aims for (M = 1 kernel)
#endif
#ifndef EQ_QMMN_ROWS
#define EQ_QMMN_ROWS 4  // minimum rows per lane and split (M = 1 kernel)
#endif
#ifndef EQ_QMMN_TLMAX
#define EQ_QMMN_TLMAX 32  // lanes across the columns (M = 1 kernel): 64, 32, 16, 8 or 4
#endif

namespace eq {
namespace {

// Workgroup = TW word columns x KP = 256 / TW row phases.  Lane (jw, p) owns
// the code word j = blockIdx.x * TW + jw of every row (32 / BITS consecutive
// columns, inside one group since gs >= 32) and walks rows kb + p, kb + p +
// KP, ... of its K split [kb, ke) (blockIdx.y); consecutive lanes read
// consecutive words of a row.  The phases are summed through LDS; with more
// than one split the sums go to ws[split][batch][M][N] for qmm_n_finish.
template <int BITS, typename ST, bool MANY, int TW>
__global__ __launch_bounds__(256) void qmm_n_small(uint16_t* __restrict__ y, float* __restrict__ ws,
                                                   const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
                                                   const typename ST::storage* __restrict__ s,
                                                   const typename ST::storage* __restrict__ bz, GatherIdx g, int M,
                                                   int N, int K, int gs, int kchunk, int64_t b0,
                                                   int64_t batch_total) {
    constexpr int KP = 256 / TW, CPW = 32 / BITS, MC = MANY ? 8 : 1;
    __shared__ float red[256 * CPW];
    const int tid = threadIdx.x, jw = tid % TW, p = tid / TW;
    const int Nw = N / CPW, G = N / gs;
    const int j = blockIdx.x * TW + jw;
    const int64_t b = b0 + blockIdx.z;
    const int split = blockIdx.y;
    const int kb = split * kchunk, ke = min(K, kb + kchunk);
    float acc[MC][CPW], xbias[MC];
#pragma unroll
    for (int m = 0; m < MC; m++) {
        xbias[m] = 0.f;
#pragma unroll
        for (int c = 0; c < CPW; c++) acc[m][c] = 0.f;
    }
    int64_t xbt, wbt;
    if (gather_batch(g, b, xbt, wbt) && j < Nw) {
        const uint16_t* xr = x + xbt * M * K;
        const uint32_t* wr = w + wbt * int64_t(K) * Nw + j;
        const typename ST::storage* sr = s + wbt * int64_t(K) * G + j * CPW / gs;
        const typename ST::storage* br = bz ? bz + wbt * int64_t(K) * G + j * CPW / gs : nullptr;
#pragma unroll 2
        for (int k = kb + p; k < ke; k += KP) {
            const uint32_t word = wr[int64_t(k) * Nw];
            const float sc = load_param<ST>(sr, int64_t(k) * G);
            const float bi = br ? load_param<ST>(br, int64_t(k) * G) : 0.f;
            float q[CPW];
            if constexpr (BITS == 4) {
                const uint32_t lo = word & 0x0f0f0f0fu, hi = (word >> 4) & 0x0f0f0f0fu;  // codes 0,2,4,6 / 1,3,5,7
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    q[2 * i] = float((lo >> (8 * i)) & 0xffu);
                    q[2 * i + 1] = float((hi >> (8 * i)) & 0xffu);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) q[i] = float((word >> (8 * i)) & 0xffu);
            }
#pragma unroll
            for (int m = 0; m < MC; m++) {
                if (m >= M) break;
                const float xv = bf16_bits_to_f32(xr[int64_t(m) * K + k]);
                const float xs = xv * sc;
                xbias[m] = fmaf(xv, bi, xbias[m]);
#pragma unroll
                for (int c = 0; c < CPW; c++) acc[m][c] = fmaf(xs, q[c], acc[m][c]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MC; m++) {
        if (m >= M) break;
#pragma unroll
        for (int c = 0; c < CPW; c++) red[(p * TW + jw) * CPW + c] = acc[m][c] + xbias[m];
        __syncthreads();
        for (int t = tid; t < TW * CPW; t += 256) {
            float v = 0.f;
#pragma unroll
            for (int q = 0; q < KP; q++) v += red[q * TW * CPW + t];
            const int n = blockIdx.x * TW * CPW + t;
            if (n < N) {
                if (ws) ws[((int64_t(split) * batch_total + b) * M + m) * N + n] = v;
                else y[(b * M + m) * N + n] = uint16_t(f32_to_bf16_bits(v));
            }
        }
        __syncthreads();
    }
}

// M = 1: lane (jl, p) of TL lanes across columns x KP = 256 / TL row phases
// owns four code words of a row (one 16-byte load: CPL = 128 / BITS columns
// of one group) and rows kb + p, kb + p + KP, ...; EQ_QMMN_UNROLL rows' loads
// are issued before any is used.  A workgroup covers KP x (rows per lane)
// rows of TL x CPL columns, so its partial sums are few against the codes
// read.
template <int BITS, typename ST, int TL>
__global__ __launch_bounds__(256) void qmm_n_m1(uint16_t* __restrict__ y, float* __restrict__ ws,
                                                const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
                                                const typename ST::storage* __restrict__ s,
                                                const typename ST::storage* __restrict__ bz, GatherIdx g, int N, int K,
                                                int gs, int kchunk, int64_t b0, int64_t batch_total) {
    constexpr int KP = 256 / TL, CPL = 128 / BITS, U = EQ_QMMN_UNROLL;
    __shared__ float red[256 * CPL];
    const int tid = threadIdx.x, jl = tid % TL, p = tid / TL;
    const int Nq = N / CPL, G = N / gs;  // 16-byte words per row, groups per row
    // Workgroups reach the 8 XCDs round-robin by linear id, each XCD with its
    // own L2; the (tile, split) pairs are numbered split-major and dealt out
    // so that the tiles of one split -- which read the same scale and bias
    // rows -- share an XCD: unit = x * floor(T / 8) + min(x, T % 8) + id / 8
    // for id on XCD x = id % 8 (a bijection of [0, T) for any T).
    const int tiles = gridDim.x, total = gridDim.x * gridDim.y;
    const int lin = blockIdx.x + gridDim.x * blockIdx.y, xcd = lin & 7;
    const int unit = xcd * (total >> 3) + min(xcd, total & 7) + (lin >> 3);
    const int jq = (unit % tiles) * TL + jl;
    const int64_t b = b0 + blockIdx.z;
    const int split = unit / tiles;
    const int kb = split * kchunk, ke = min(K, kb + kchunk);
    float acc[CPL], xbias = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; c++) acc[c] = 0.f;
    int64_t xbt, wbt;
    if (gather_batch(g, b, xbt, wbt) && jq < Nq) {
        const uint16_t* xr = x + xbt * K;
        const uint4* wr = reinterpret_cast<const uint4*>(w + wbt * int64_t(K) * (N * BITS / 32)) + jq;
        const typename ST::storage* sr = s + wbt * int64_t(K) * G + jq * CPL / gs;
        const typename ST::storage* br = bz ? bz + wbt * int64_t(K) * G + jq * CPL / gs : nullptr;
        auto row = [&](uint4 wv, float sc, float bi, float xv) {
            const float xs = xv * sc;
            xbias = fmaf(xv, bi, xbias);
            const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
            for (int t = 0; t < 4; t++) {
                if constexpr (BITS == 4) {
                    const uint32_t lo = wd[t] & 0x0f0f0f0fu, hi = (wd[t] >> 4) & 0x0f0f0f0fu;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        acc[8 * t + 2 * i] = fmaf(xs, float((lo >> (8 * i)) & 0xffu), acc[8 * t + 2 * i]);
                        acc[8 * t + 2 * i + 1] = fmaf(xs, float((hi >> (8 * i)) & 0xffu), acc[8 * t + 2 * i + 1]);
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[4 * t + i] = fmaf(xs, float((wd[t] >> (8 * i)) & 0xffu), acc[4 * t + i]);
                }
            }
        };
        // U rows per step, all loads first; rows past the split re-read its
        // last row with a zero activation (no contribution)
        for (int k = kb + p; k < ke; k += U * KP) {
            uint4 wv[U];
            float sc[U], bi[U], xv[U];
#pragma unroll
            for (int i = 0; i < U; i++) {
                const int kk = k + i * KP;
                const int kl = kk < ke ? kk : ke - 1;
                wv[i] = load_stream16(wr + int64_t(kl) * Nq);
                sc[i] = load_param<ST>(sr, int64_t(kl) * G);
                bi[i] = br ? load_param<ST>(br, int64_t(kl) * G) : 0.f;
                xv[i] = kk < ke ? bf16_bits_to_f32(xr[kl]) : 0.f;
            }
#pragma unroll
            for (int i = 0; i < U; i++) row(wv[i], sc[i], bi[i], xv[i]);
        }
    }
#pragma unroll
    for (int c = 0; c < CPL; c++) red[(p * TL + jl) * CPL + c] = acc[c] + xbias;
    __syncthreads();
    for (int t = tid; t < TL * CPL; t += 256) {
        float v = 0.f;
#pragma unroll 8
        for (int q = 0; q < KP; q++) v += red[q * TL * CPL + t];
        const int n = (unit % tiles) * TL * CPL + t;
        if (n < N) {
            if (ws) ws[(int64_t(split) * batch_total + b) * N + n] = v;
            else y[b * N + n] = uint16_t(f32_to_bf16_bits(v));
        }
    }
}

// y[e] = bf16(sum over splits of ws[split][e]), e over batch * M * N: 8 lanes
// per element, each summing every 8th split with independent partial sums,
// then a shuffle sum over the 8 lanes.
__global__ __launch_bounds__(256) void qmm_n_finish(uint16_t* __restrict__ y, const float* __restrict__ ws,
                                                    int64_t mn, int splits) {
    const int64_t e = (int64_t(blockIdx.x) * 256 + threadIdx.x) >> 3;
    const int sub = threadIdx.x & 7;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (e < mn) {
        int sp = sub;
        for (; sp + 24 < splits; sp += 32) {
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] += ws[int64_t(sp + 8 * i) * mn + e];
        }
        for (; sp < splits; sp += 8) v[0] += ws[int64_t(sp) * mn + e];
    }
    float t = (v[0] + v[1]) + (v[2] + v[3]);
    t += __shfl_xor(t, 4);
    t += __shfl_xor(t, 2);
    t += __shfl_xor(t, 1);
    if (e < mn && sub == 0) y[e] = uint16_t(f32_to_bf16_bits(t));
}

constexpr int64_t kMaxBatchesPerLaunch = 65535;  // grid z

template <int BITS, typename ST, bool MANY, int TW>
void launch_n(uint16_t* y, float* ws, const uint16_t* x, const uint32_t* w, const void* s, const void* b,
              const GatherIdx& g, int64_t batch, int M, int N, int K, int gs, int splits, int kchunk,
              hipStream_t st) {
    typedef typename ST::storage SS;
    const int Nw = N / (32 / BITS);
    for (int64_t b0 = 0; b0 < batch; b0 += kMaxBatchesPerLaunch) {
        const unsigned nb = unsigned(batch - b0 < kMaxBatchesPerLaunch ? batch - b0 : kMaxBatchesPerLaunch);
        const dim3 grid(unsigned((Nw + TW - 1) / TW), unsigned(splits), nb);
        qmm_n_small<BITS, ST, MANY, TW><<<grid, 256, 0, st>>>(y, ws, x, w, static_cast<const SS*>(s),
                                                               static_cast<const SS*>(b), g, M, N, K, gs, kchunk,
                                                               b0, batch);
    }
}

template <int BITS, typename ST>
void launch_n_bits(uint16_t* y, float* ws, const uint16_t* x, const uint32_t* w, const void* s, const void* b,
                   const GatherIdx& g, int64_t batch, int M, int N, int K, int gs, int splits, int kchunk, int tw,
                   hipStream_t st) {
#define EQ_N(MANY, TW) launch_n<BITS, ST, MANY, TW>(y, ws, x, w, s, b, g, batch, M, N, K, gs, splits, kchunk, st)
    if (M == 1) {
        if (tw == 64) EQ_N(false, 64);
        else if (tw == 32) EQ_N(false, 32);
        else EQ_N(false, 16);
    } else {
        if (tw == 64) EQ_N(true, 64);
        else if (tw == 32) EQ_N(true, 32);
        else EQ_N(true, 16);
    }
#undef EQ_N
}

template <int BITS, typename ST, int TL>
void launch_m1(uint16_t* y, float* ws, const uint16_t* x, const uint32_t* w, const void* s, const void* b,
               const GatherIdx& g, int64_t batch, int N, int K, int gs, int splits, int kchunk, hipStream_t st) {
    typedef typename ST::storage SS;
    const int Nq = N / (128 / BITS);
    for (int64_t b0 = 0; b0 < batch; b0 += kMaxBatchesPerLaunch) {
        const unsigned nb = unsigned(batch - b0 < kMaxBatchesPerLaunch ? batch - b0 : kMaxBatchesPerLaunch);
        const dim3 grid(unsigned((Nq + TL - 1) / TL), unsigned(splits), nb);
        qmm_n_m1<BITS, ST, TL><<<grid, 256, 0, st>>>(y, ws, x, w, static_cast<const SS*>(s),
                                                     static_cast<const SS*>(b), g, N, K, gs, kchunk, b0, batch);
    }
}

template <int BITS, typename ST>
void launch_m1_tl(int tl, uint16_t* y, float* ws, const uint16_t* x, const uint32_t* w, const void* s,
                  const void* b, const GatherIdx& g, int64_t batch, int N, int K, int gs, int splits, int kchunk,
                  hipStream_t st) {
    if (tl == 64) launch_m1<BITS, ST, 64>(y, ws, x, w, s, b, g, batch, N, K, gs, splits, kchunk, st);
    else if (tl == 32) launch_m1<BITS, ST, 32>(y, ws, x, w, s, b, g, batch, N, K, gs, splits, kchunk, st);
    else if (tl == 16) launch_m1<BITS, ST, 16>(y, ws, x, w, s, b, g, batch, N, K, gs, splits, kchunk, st);
    else if (tl == 8) launch_m1<BITS, ST, 8>(y, ws, x, w, s, b, g, batch, N, K, gs, splits, kchunk, st);
    else launch_m1<BITS, ST, 4>(y, ws, x, w, s, b, g, batch, N, K, gs, splits, kchunk, st);
}

// K split so that the launch has about `target` workgroups, each lane at
// least `min_rows` rows of its split; returns (splits, kchunk).
void pick_splits(int64_t tiles, int K, int kp, int min_rows, int64_t target, int& splits, int& kchunk) {
    int64_t sp = (target + tiles - 1) / tiles;
    const int64_t max_sp = (int64_t(K) + int64_t(min_rows) * kp - 1) / (int64_t(min_rows) * kp);
    if (sp > max_sp) sp = max_sp;
    if (sp > 65535) sp = 65535;
    if (sp < 1) sp = 1;
    kchunk = int((K + sp - 1) / sp);
    splits = int((K + kchunk - 1) / kchunk);
}

}  // namespace

bool launch_qmm_n_small(int bits, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s,
                        const void* b, const GatherIdx& g, int64_t batch, int M, int N, int K, int gs,
                        const WsSource* src, hipStream_t st) {
    if ((bits != 4 && bits != 8) || (scale_dtype != EQ_DTYPE_BF16 && scale_dtype != EQ_DTYPE_F16) || M < 1 ||
        M > 8 || batch < 1 || gs < 32)
        return false;
    const int64_t mn = batch * M * int64_t(N);
    // M = 1 with rows of whole 16-byte words: qmm_n_m1 (up to EQ_QMMN_TLMAX
    // lanes across the columns, at least EQ_QMMN_ROWS rows per lane and
    // split); else qmm_n_small.
    const int cpl = 128 / bits;
    const bool m1 = M == 1 && N % cpl == 0 && aligned(w, 16);
    int tl = 0, kp = 0, splits = 1, kchunk = K;
    int64_t tiles = 0;
    if (m1) {
        const int Nq = N / cpl;
        tl = Nq >= 64 && EQ_QMMN_TLMAX >= 64   ? 64
             : Nq >= 32 && EQ_QMMN_TLMAX >= 32 ? 32
             : Nq >= 16 && EQ_QMMN_TLMAX >= 16 ? 16
             : Nq >= 8 && EQ_QMMN_TLMAX >= 8   ? 8
                                               : 4;
        kp = 256 / tl;
        tiles = int64_t((Nq + tl - 1) / tl) * batch;
        pick_splits(tiles, K, kp, EQ_QMMN_ROWS, EQ_QMMN_TARGET, splits, kchunk);
    } else {
        const int Nw = N / (32 / bits);
        tl = Nw >= 64 ? 64 : Nw >= 32 ? 32 : 16;
        kp = 256 / tl;
        tiles = int64_t((Nw + tl - 1) / tl) * batch;
        pick_splits(tiles, K, kp, 4, 1024, splits, kchunk);
    }
    float* ws = nullptr;
    if (splits > 1 && src && size_t(splits) * size_t(mn) * 4u > src->cap) {
        // a fixed scratch region holds fewer splits: re-plan for what fits
        const int64_t fit = int64_t(src->cap / (size_t(mn) * 4u));
        if (fit >= 2) {
            kchunk = int((K + fit - 1) / fit);
            splits = int((K + kchunk - 1) / kchunk);
        } else {
            splits = 1;
            kchunk = K;
        }
    }
    if (splits > 1) {
        ws = static_cast<float*>(ws_acquire(src, size_t(splits) * size_t(mn) * 4u, st));
        if (!ws) {
            splits = 1;
            kchunk = K;
        }
    }
#define EQ_N_DISPATCH(BITS, ST)                                                                                  \
    (m1 ? launch_m1_tl<BITS, ST>(tl, y, ws, x, w, s, b, g, batch, N, K, gs, splits, kchunk, st)                 \
        : launch_n_bits<BITS, ST>(y, ws, x, w, s, b, g, batch, M, N, K, gs, splits, kchunk, tl, st))
    if (bits == 4) {
        if (scale_dtype == EQ_DTYPE_BF16) EQ_N_DISPATCH(4, BF16T);
        else EQ_N_DISPATCH(4, F16T);
    } else {
        if (scale_dtype == EQ_DTYPE_BF16) EQ_N_DISPATCH(8, BF16T);
        else EQ_N_DISPATCH(8, F16T);
    }
#undef EQ_N_DISPATCH
    if (splits > 1)
        qmm_n_finish<<<dim3(unsigned((mn * 8 + 255) / 256)), dim3(256), 0, st>>>(y, ws, mn, splits);
    return true;
}

}  // namespace eq
