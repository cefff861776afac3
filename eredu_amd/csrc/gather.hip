// gather_qmm: for each output batch b,
//   y[b] = x[lhs[b]] . dequant(w[rhs[b]])^T   (transpose = true)
//   y[b] = x[lhs[b]] . dequant(w[rhs[b]])     (transpose = false)
// with x [x_batches, M, K], w / scales / biases [w_batches, ...] and y
// [batch, M, N]: MLX's gather_qmm under safemlx::ops::gather_qmm_with_mode
// (safemlx/src/ops/quantization.rs:298-379), as eredu's routed experts call
// it (eredu/src/backend/mlx/nn/moe.rs:121-139: x [routes, 1, K], lhs =
// arange(routes), rhs = the expert of each route).
//
// The indices stay on the device: each workgroup reads its batch's pair.  An
// index outside its operand's batches makes that batch's output rows zero
// and reads nothing (MLX leaves such gathers undefined).
//
// Kernels: the routed-expert decode (transpose = true, one bf16 activation
// row per batch, 4/8-bit codes, N % 16 == 0, K a whole number of the decode
// kernel's blocks) runs qmv.hip's persistent decode kernel, up to 8 batches
// per launch, with each batch's x row and expert found from the indices on
// the device (launch_qmv_gather).  gather_qmv -- the other decode shapes: the team
// layout of a workgroup (T teams of 256 / T lanes, 4 weight rows per team,
// lanes splitting a row's 16-byte code chunks, so a chunk's activations are
// loaded once for 4 rows); 4-bit sums run on v_dot2c_f32_bf16 with codes as
// the exact bf16 values 128 + q.  Everything else: the general kernels'
// bodies (one wave per output feature, or one thread per output column),
// offset per batch; transpose = false with M <= 8, bf16 x and 4/8-bit codes
// takes qmm_n_small (qmm_n.hip) with these indices.
#include "eq_common.hpp"

namespace eq {
namespace {

// grid (ceil(N / kGenRowsPerWG), batches of this launch); b = b0 + blockIdx.y.
template <int BITS, typename XT, typename ST>
__global__ __launch_bounds__(64 * kGenRowsPerWG) void gather_t_general(
    typename XT::storage* __restrict__ y, const typename XT::storage* __restrict__ x,
    const uint32_t* __restrict__ w, const typename ST::storage* __restrict__ s,
    const typename ST::storage* __restrict__ bz, GatherIdx g, int64_t b0, int64_t M, int64_t N, int64_t K, int gs) {
    const int64_t b = b0 + blockIdx.y;
    const int64_t n = int64_t(blockIdx.x) * kGenRowsPerWG + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (n >= N) return;
    int64_t xb, wb;
    y += b * M * N;
    if (!gather_batch(g, b, xb, wb)) {
        for (int64_t m = lane; m < M; m += 64) store_out<XT>(y, m * N + n, 0.f);
        return;
    }
    const int64_t G = K / gs;
    qmm_t_rows<BITS, XT, ST>(y, x + xb * M * K, w + wb * N * (K * BITS / 32), s + wb * N * G,
                             bz ? bz + wb * N * G : nullptr, M, N, K, gs, n, lane);
}

// grid (ceil(N / 256), ceil(M / kGenMChunk), batches of this launch).
template <int BITS, typename XT, typename ST>
__global__ __launch_bounds__(256) void gather_n_general(
    typename XT::storage* __restrict__ y, const typename XT::storage* __restrict__ x,
    const uint32_t* __restrict__ w, const typename ST::storage* __restrict__ s,
    const typename ST::storage* __restrict__ bz, GatherIdx g, int64_t b0, int64_t M, int64_t N, int64_t K, int gs) {
    const int64_t b = b0 + blockIdx.z;
    const int64_t n = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t m0 = int64_t(blockIdx.y) * kGenMChunk;
    if (n >= N) return;
    int64_t xb, wb;
    y += b * M * N;
    if (!gather_batch(g, b, xb, wb)) {
        for (int64_t m = m0; m < M && m < m0 + kGenMChunk; m++) store_out<XT>(y, m * N + n, 0.f);
        return;
    }
    const int64_t G = N / gs;
    qmm_n_cols<BITS, XT, ST>(y, x + xb * M * K, w + wb * K * (N * BITS / 32), s + wb * K * G,
                             bz ? bz + wb * K * G : nullptr, M, N, K, gs, n, m0);
}

constexpr int kGqRows = 4;  // weight rows per team

// 8 consecutive 4-bit codes (one word, LSB first) as 4 bf16 pairs (128 +
// c_2i, 128 + c_2i+1), the order of the activation words.
__device__ __forceinline__ void unpack4_pairs(uint32_t w, uint32_t* p) {
    const uint32_t t = w >> 4;
    p[0] = (__builtin_amdgcn_perm(t, w, 0x0c040c00u) & 0x000f000fu) | kNibbleMagic;
    p[1] = (__builtin_amdgcn_perm(t, w, 0x0c050c01u) & 0x000f000fu) | kNibbleMagic;
    p[2] = (__builtin_amdgcn_perm(t, w, 0x0c060c02u) & 0x000f000fu) | kNibbleMagic;
    p[3] = (__builtin_amdgcn_perm(t, w, 0x0c070c03u) & 0x000f000fu) | kNibbleMagic;
}

// grid (ceil(N / (4 T)), batches of this launch); 256 lanes.  Chunk c of a
// row = 16 bytes of codes = CPC codes inside one group (CPC <= GS).  Per
// row and chunk: scale * sum(x q) + bias * sum(x), sum(x) shared by the rows.
// MXFP4 (ST = E8M0T): the chunk is one group of 32 E2M1 codes, decoded to
// bf16 with the scale folded in (e2m1x8_to_bf16), no bias.
template <int BITS, int GS, typename ST, int T>
__global__ __launch_bounds__(256) void gather_qmv(uint16_t* __restrict__ y, const uint16_t* __restrict__ x,
                                                  const uint32_t* __restrict__ w,
                                                  const typename ST::storage* __restrict__ s,
                                                  const typename ST::storage* __restrict__ bz, GatherIdx g,
                                                  int64_t b0, int N, int K) {
    constexpr int S = 256 / T, WPT = S / 64, CPC = 128 / BITS;
    static_assert(CPC <= GS, "a chunk lies inside one group");
    __shared__ float red[4 * kGqRows];
    const int64_t b = b0 + blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sl = tid % S, team = tid / S;
    const int row0 = blockIdx.x * T * kGqRows, r0 = row0 + team * kGqRows;
    const int G = K / GS, nch = K / CPC;
    const int64_t row_words = int64_t(K) * BITS / 32;
    float acc[kGqRows];
#pragma unroll
    for (int r = 0; r < kGqRows; r++) acc[r] = 0.f;
    int64_t xb, wb;
    if (gather_batch(g, b, xb, wb)) {
        const uint16_t* xr = x + xb * K;
        const uint32_t* wr = w + wb * N * row_words;
        const typename ST::storage* sr = s + wb * N * G;
        const typename ST::storage* br = bz ? bz + wb * N * G : nullptr;
#pragma unroll 1
        for (int c = sl; c < nch; c += S) {
            const int grp = c * CPC / GS;
            uint4 qv[kGqRows];
            float sc[kGqRows], bi[kGqRows];
#pragma unroll
            for (int r = 0; r < kGqRows; r++) {
                const int n = min(r0 + r, N - 1);  // rows past N read row N - 1; their sums are not stored
                qv[r] = load_stream16(wr + n * row_words + c * 4);
                sc[r] = load_param<ST>(sr, int64_t(n) * G + grp);
                bi[r] = br ? load_param<ST>(br, int64_t(n) * G + grp) : 0.f;
            }
            const uint4* xa = reinterpret_cast<const uint4*>(xr + int64_t(c) * CPC);
            if constexpr (__is_same(ST, E8M0T)) {
                uint32_t xw[16];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint4 v = xa[i];
                    xw[4 * i] = v.x, xw[4 * i + 1] = v.y, xw[4 * i + 2] = v.z, xw[4 * i + 3] = v.w;
                }
#pragma unroll
                for (int r = 0; r < kGqRows; r++) {
                    const uint32_t qw[4] = {qv[r].x, qv[r].y, qv[r].z, qv[r].w};
                    float e = 0.f;  // sum x 2^(s - 127) e2m1(q)
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        uint32_t p[4];
                        e2m1x8_to_bf16(qw[t], sc[r], p);
#pragma unroll
                        for (int j = 0; j < 4; j++) e = dot2_bf16(xw[4 * t + j], p[j], e);
                    }
                    acc[r] += e;
                }
            } else if constexpr (BITS == 4) {
                uint32_t xw[16];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint4 v = xa[i];
                    xw[4 * i] = v.x, xw[4 * i + 1] = v.y, xw[4 * i + 2] = v.z, xw[4 * i + 3] = v.w;
                }
                float sx = 0.f;
#pragma unroll
                for (int i = 0; i < 16; i++) sx = dot2_bf16(xw[i], kBf16Ones, sx);
#pragma unroll
                for (int r = 0; r < kGqRows; r++) {
                    const uint32_t qw[4] = {qv[r].x, qv[r].y, qv[r].z, qv[r].w};
                    float e = 0.f;  // sum x (128 + q)
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        uint32_t p[4];
                        unpack4_pairs(qw[t], p);
#pragma unroll
                        for (int j = 0; j < 4; j++) e = dot2_bf16(xw[4 * t + j], p[j], e);
                    }
                    acc[r] += sc[r] * (e - 128.f * sx) + bi[r] * sx;
                }
            } else {
                const uint4 xv[2] = {xa[0], xa[1]};
                float f[16];
                bf16x8_to_f32(xv[0], f);
                bf16x8_to_f32(xv[1], f + 8);
                float sx = 0.f;
                sx = dot2_bf16(xv[0].x, kBf16Ones, dot2_bf16(xv[0].y, kBf16Ones, sx));
                sx = dot2_bf16(xv[0].z, kBf16Ones, dot2_bf16(xv[0].w, kBf16Ones, sx));
                sx = dot2_bf16(xv[1].x, kBf16Ones, dot2_bf16(xv[1].y, kBf16Ones, sx));
                sx = dot2_bf16(xv[1].z, kBf16Ones, dot2_bf16(xv[1].w, kBf16Ones, sx));
#pragma unroll
                for (int r = 0; r < kGqRows; r++) {
                    const uint32_t qw[4] = {qv[r].x, qv[r].y, qv[r].z, qv[r].w};
                    float e = 0.f;
#pragma unroll
                    for (int j = 0; j < 16; j++) e = fmaf(f[j], float((qw[j >> 2] >> (8 * (j & 3))) & 0xffu), e);
                    acc[r] += sc[r] * e + bi[r] * sx;
                }
            }
        }
    }
    // team sums: waves by shuffles, then the team's waves through LDS
#pragma unroll
    for (int r = 0; r < kGqRows; r++) {
        const float v = wave_sum(acc[r]);
        if (lane == 0) red[wave * kGqRows + r] = v;
    }
    __syncthreads();
    if (tid < T * kGqRows) {
        const int tm = tid / kGqRows, r = tid % kGqRows;
        float v = 0.f;
#pragma unroll
        for (int i = 0; i < WPT; i++) v += red[(tm * WPT + i) * kGqRows + r];
        const int n = row0 + tm * kGqRows + r;
        if (n < N) y[b * N + n] = uint16_t(f32_to_bf16_bits(v));
    }
}

template <int BITS, int GS, typename ST>
void launch_gather_qmv(uint16_t* y, const uint16_t* x, const uint32_t* w, const typename ST::storage* s,
                       const typename ST::storage* bz, const GatherIdx& g, int64_t b0, unsigned nb, int N, int K,
                       hipStream_t st) {
    const int nch = K / (128 / BITS);
    const int teams = nch <= 64 ? 4 : nch <= 128 ? 2 : 1;
    const unsigned gx = unsigned((N + teams * kGqRows - 1) / (teams * kGqRows));
    const dim3 grid(gx, nb);
    if (teams == 4) gather_qmv<BITS, GS, ST, 4><<<grid, 256, 0, st>>>(y, x, w, s, bz, g, b0, N, K);
    else if (teams == 2) gather_qmv<BITS, GS, ST, 2><<<grid, 256, 0, st>>>(y, x, w, s, bz, g, b0, N, K);
    else gather_qmv<BITS, GS, ST, 1><<<grid, 256, 0, st>>>(y, x, w, s, bz, g, b0, N, K);
}

template <int BITS, typename ST>
void launch_gather_qmv_gs(int gs, uint16_t* y, const uint16_t* x, const uint32_t* w, const typename ST::storage* s,
                          const typename ST::storage* bz, const GatherIdx& g, int64_t b0, unsigned nb, int N, int K,
                          hipStream_t st) {
    if (gs == 32) launch_gather_qmv<BITS, 32, ST>(y, x, w, s, bz, g, b0, nb, N, K, st);
    else if (gs == 64) launch_gather_qmv<BITS, 64, ST>(y, x, w, s, bz, g, b0, nb, N, K, st);
    else launch_gather_qmv<BITS, 128, ST>(y, x, w, s, bz, g, b0, nb, N, K, st);
}

}  // namespace

void launch_gather_qmv_mxfp4(uint16_t* y, const uint16_t* x, const uint32_t* w, const uint8_t* s, const GatherIdx& g,
                             int64_t b0, unsigned nb, int N, int K, hipStream_t st) {
    launch_gather_qmv<4, 32, E8M0T>(y, x, w, s, nullptr, g, b0, nb, N, K, st);
}

}  // namespace eq

using namespace eq;

namespace eq {

int gather_qmm_launch(void* y, const void* x, const uint32_t* w, const void* scales, const void* biases,
                      const int32_t* lhs_indices, const int32_t* rhs_indices, int64_t batch, int64_t x_batches,
                      int64_t w_batches, int64_t M, int64_t N, int64_t K, bool transpose, int group_size, int bits,
                      QuantMode qm, int x_dtype, int scale_dtype, bool sorted_indices, const WsSource* src,
                      hipStream_t st) {
    const GatherIdx g{lhs_indices, rhs_indices, x_batches, w_batches};
    if (qm == kModeMxFp4)
        return mxfp4_matmul(y, x, w, static_cast<const uint8_t*>(scales), g, batch, M, N, K, transpose, x_dtype,
                            sorted_indices, nullptr, st);

    // many routes over sorted experts: one MFMA GEMM per expert's rows
    const bool grouped = transpose && M == 1 && sorted_indices && rhs_indices && x_dtype == EQ_DTYPE_BF16 &&
                         scale_dtype != EQ_DTYPE_F32 && (bits == 4 || bits == 8) && batch >= 64 &&
                         batch >= 2 * w_batches && batch <= INT32_MAX && w_batches <= INT32_MAX && N % 128 == 0 &&
                         K % 64 == 0 && aligned(x, 16) && aligned(w, 16) && aligned(y, 8) &&
                         int64_t(N) * K * bits / 8 < (int64_t(1) << 31) && batch * K * 2 < (int64_t(1) << 31);
    if (grouped && launch_qmm_grouped(bits, group_size, scale_dtype, static_cast<uint16_t*>(y),
                                      static_cast<const uint16_t*>(x), w, scales, biases, lhs_indices, rhs_indices,
                                      int(batch), x_batches, int(w_batches), int(N), int(K), st, src))
        return check_launch("gather_qmm (grouped qmm)");
    const bool fast = transpose && M == 1 && x_dtype == EQ_DTYPE_BF16 && scale_dtype != EQ_DTYPE_F32 &&
                      (bits == 4 || bits == 8) && fast_group_size(group_size) && aligned(x, 16) && aligned(w, 16);
    if (!transpose && M <= 8 && x_dtype == EQ_DTYPE_BF16 &&
        launch_qmm_n_small(bits, scale_dtype, static_cast<uint16_t*>(y), static_cast<const uint16_t*>(x), w, scales,
                           biases, g, batch, int(M), int(N), int(K), group_size, nullptr, st))
        return check_launch("gather_qmm (qmm_n)");
    // the routed decode on the persistent decode kernel (qmv.hip) where its
    // shapes fit: codes streamed as the dense decode streams them
    if (fast && launch_qmv_gather(bits, group_size, scale_dtype, static_cast<uint16_t*>(y),
                                  static_cast<const uint16_t*>(x), w, scales, biases, g, batch, int(N), int(K), st))
        return check_launch("gather_qmm (qmv)");
    for (int64_t b0 = 0; b0 < batch; b0 += kMaxGridY) {
        const unsigned nb = unsigned(batch - b0 < kMaxGridY ? batch - b0 : kMaxGridY);
        if (fast) {
            uint16_t* yy = static_cast<uint16_t*>(y);
            const uint16_t* xx = static_cast<const uint16_t*>(x);
            const uint16_t* ss = static_cast<const uint16_t*>(scales);
            const uint16_t* bb = static_cast<const uint16_t*>(biases);
            if (scale_dtype == EQ_DTYPE_BF16) {
                if (bits == 4) launch_gather_qmv_gs<4, BF16T>(group_size, yy, xx, w, ss, bb, g, b0, nb, int(N), int(K), st);
                else launch_gather_qmv_gs<8, BF16T>(group_size, yy, xx, w, ss, bb, g, b0, nb, int(N), int(K), st);
            } else {
                if (bits == 4) launch_gather_qmv_gs<4, F16T>(group_size, yy, xx, w, ss, bb, g, b0, nb, int(N), int(K), st);
                else launch_gather_qmv_gs<8, F16T>(group_size, yy, xx, w, ss, bb, g, b0, nb, int(N), int(K), st);
            }
            continue;
        }
        with_bits(bits, [&](auto bc) {
            constexpr int B = decltype(bc)::value;
            with_dtype(x_dtype, [&](auto xt) {
                typedef decltype(xt) XT;
                with_dtype(scale_dtype, [&](auto stt) {
                    typedef decltype(stt) ST;
                    typedef typename XT::storage XS;
                    typedef typename ST::storage SS;
                    if (transpose) {
                        const dim3 grid(unsigned((N + kGenRowsPerWG - 1) / kGenRowsPerWG), nb);
                        gather_t_general<B, XT, ST><<<grid, 64 * kGenRowsPerWG, 0, st>>>(
                            static_cast<XS*>(y), static_cast<const XS*>(x), w, static_cast<const SS*>(scales),
                            static_cast<const SS*>(biases), g, b0, M, N, K, group_size);
                    } else {
                        const dim3 grid(unsigned((N + 255) / 256), unsigned((M + kGenMChunk - 1) / kGenMChunk), nb);
                        gather_n_general<B, XT, ST><<<grid, 256, 0, st>>>(
                            static_cast<XS*>(y), static_cast<const XS*>(x), w, static_cast<const SS*>(scales),
                            static_cast<const SS*>(biases), g, b0, M, N, K, group_size);
                    }
                });
            });
        });
    }
    return check_launch("gather_qmm");
}

}  // namespace eq

extern "C" int eq_gather_qmm(void* y, const void* x, const uint32_t* w, const void* scales, const void* biases,
                             const int32_t* lhs_indices, const int32_t* rhs_indices, int64_t batch, int64_t x_batches,
                             int64_t w_batches, int64_t M, int64_t N, int64_t K, bool transpose, int group_size,
                             int bits, const char* mode, int x_dtype, int scale_dtype, bool sorted_indices,
                             eq_stream_t stream) {
    // sorted_indices: an ordering hint.  With it (and many routes) the
    // grouped MFMA path runs; its results equal the other paths' within the
    // matmul rule for sorted indices (unsorted indices under the hint give
    // wrong rows, as in MLX, but every access stays in bounds).
    clear_error();
    QuantMode qm;
    if (parse_mode(mode, qm)) return 1;
    if (qm == kModeMxFp4 ? check_mxfp4(group_size, bits, scale_dtype, biases) : check_gs_bits(group_size, bits))
        return 1;
    if (!valid_dtype(x_dtype) || (qm == kModeAffine && !valid_dtype(scale_dtype))) {
        set_error("invalid dtype code");
        return 1;
    }
    if (batch < 0 || x_batches < 1 || w_batches < 1 || M < 0 || N <= 0 || K <= 0) {
        set_error("invalid shape: batch >= 0, x_batches >= 1, w_batches >= 1, M >= 0, N > 0 and K > 0 required");
        return 1;
    }
    const int64_t packed_dim = transpose ? K : N;
    if (packed_dim % group_size != 0) {
        set_error("the quantized dimension (" + std::to_string(packed_dim) + ") is not divisible by group_size " +
                  std::to_string(group_size));
        return 1;
    }
    if (!check_packed_row(packed_dim, bits)) return 1;
    if (!lhs_indices && x_batches != batch && x_batches != 1) {
        set_error("without lhs_indices, x must have one batch or as many as the output");
        return 1;
    }
    if (!rhs_indices && w_batches != batch && w_batches != 1) {
        set_error("without rhs_indices, w must have one batch or as many as the output");
        return 1;
    }
    if (batch == 0 || M == 0) return 0;
    if (!y || !x || !w || !scales) {
        set_error("null pointer argument");
        return 1;
    }
    if (N > INT32_MAX || K > INT32_MAX) {
        set_error("dimension exceeds 2^31 - 1");
        return 1;
    }
    if (!transpose && (M + kGenMChunk - 1) / kGenMChunk > kMaxGridY) {
        set_error("M exceeds " + std::to_string(kMaxGridY * kGenMChunk) + " rows per batch (transpose = false)");
        return 1;
    }
    return gather_qmm_launch(y, x, w, scales, biases, lhs_indices, rhs_indices, batch, x_batches, w_batches, M, N, K,
                             transpose, group_size, bits, qm, x_dtype, scale_dtype, sorted_indices, nullptr,
                             reinterpret_cast<hipStream_t>(stream));
}
