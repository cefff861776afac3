// Decode (M <= 16, transpose = true, bf16 activations) for the widths the
// matrix-core kernels do not take: 2-, 3-, 5- and 6-bit codes at any group
// size, and 4- / 8-bit codes at group sizes other than 32, 64 and 128
// (eredu-checkpoint admits bits 2..8 and group 16 or any multiple of 32,
// eredu-checkpoint/src/lib.rs:103-122).
//
// y[m, n] = sum_g s[n, g] sum_{k in g} x[m, k] q[n, k] + b[n, g] sum_{k in g} x[m, k]
//
// A wave owns one weight row at a time; its lanes take 32-code segments of
// the row (segment j = lane, lane + 64, ...).  A segment is BITS consecutive
// words of the LSB-first code stream (eredu-gguf/src/convert.rs:413-427), so
// one BITS*4-byte load per segment (a wave load covers 64 consecutive
// segments).  Codes below 128 (BITS <= 6, and 4-bit) are summed against the
// activations with bf16 dot2 on code pairs OR-ed into 0x4300 (the exact bf16
// values 128 + q): sum x q = dot - 128 sum x.  8-bit codes take an f32 convert
// and FMA each.  The workgroup stages the activations in LDS once (16-byte
// chunks swizzled so that the four chunks a lane reads for one segment, read
// by 16 lanes at a time, fall in distinct banks) together with their sums
// over every 16 values, and its waves then walk rows (workgroups persist
// over rows).
#include "eq_common.hpp"

namespace eq {
namespace {

typedef uint32_t qa_u32x4 __attribute__((ext_vector_type(4)));

constexpr int kAnyWaves = 4;  // waves (rows in flight) per workgroup
constexpr int kAnyMaxM = 4;   // activation rows per launch

struct QmvAnyArgs {
    uint16_t* y;
    const uint16_t* x;
    const uint32_t* w;
    const void* s;
    const void* b;  // may be null
    int M, N, K, gs;
    int xs_lds;     // LDS byte offset of the 16-value sums
};

// Position of 16-byte chunk q of an activation row in LDS: the chunks of
// segment j (4j .. 4j + 3) are permuted by f(j) = (j ^ (j >> 2)) & 3, so that
// lanes j = 4a + c reading chunk 4j + r hit bank group 4c + (r ^ c ^ a).
__device__ __forceinline__ int any_chunk_slot(int q) {
    const int j = q >> 2;
    return (q & ~3) | ((q ^ j ^ (j >> 2)) & 3);
}

// Code c (0..31) of a segment of BITS words (c compile-time after unrolling).
template <int BITS>
__device__ __forceinline__ uint32_t seg_code(const uint32_t* wv, int c) {
    const int bit = c * BITS, wi = bit >> 5, sh = bit & 31;
    constexpr uint32_t mask = (1u << BITS) - 1u;
    if (sh + BITS <= 32) return (wv[wi] >> sh) & mask;
    return __builtin_amdgcn_alignbit(wv[wi + 1], wv[wi], sh) & mask;
}

template <typename ST> __device__ __forceinline__ float any_param(uint32_t v);
template <> __device__ __forceinline__ float any_param<BF16T>(uint32_t v) { return bf16_bits_to_f32(v & 0xffffu); }
template <> __device__ __forceinline__ float any_param<F16T>(uint32_t v) { return f16_bits_to_f32(v & 0xffffu); }

// Loads the BITS words of segment `off` (byte offset) into wv.
template <int BITS>
__device__ __forceinline__ void load_segment(uint32_t* wv, __amdgpu_buffer_rsrc_t r, uint32_t off) {
    if constexpr (BITS == 2) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
        wv[0] = v[0], wv[1] = v[1];
    } else if constexpr (BITS == 3) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b96(r, off, 0, 0);
        wv[0] = v[0], wv[1] = v[1], wv[2] = v[2];
    } else {
#pragma unroll
        for (int i = 0; i < BITS / 4; i++) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16u * i, 0, 0);
            wv[4 * i] = v[0], wv[4 * i + 1] = v[1], wv[4 * i + 2] = v[2], wv[4 * i + 3] = v[3];
        }
        if constexpr (BITS % 4 == 1) {
            wv[BITS - 1] = __builtin_amdgcn_raw_buffer_load_b32(r, off + 16u * (BITS / 4), 0, 0);
        } else if constexpr (BITS % 4 == 2) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off + 16u * (BITS / 4), 0, 0);
            wv[BITS - 2] = v[0], wv[BITS - 1] = v[1];
        }
    }
}

// GS16: group size 16 (two groups per segment); otherwise a segment lies in
// one group (group size a multiple of 32).  MX: MXFP4 (BITS 4, group 32,
// E8M0 scale bytes, no biases): the codes convert in hardware to bf16 pairs
// with the group's scale folded in (e2m1x8_to_bf16), y = sum x . v.
template <int BITS, typename ST, int MC, bool GS16, bool MX = false>
__global__ __launch_bounds__(64 * kAnyWaves) void qmv_any_kernel(const QmvAnyArgs a) {
    static_assert(!MX || (BITS == 4 && !GS16), "MXFP4 is 4-bit, group 32");
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = a.M, N = a.N, K = a.K, gs = a.gs;
    const int G = K / gs, nseg = K / 32, cpr = K / 8;  // chunks of 8 values per row
    float* xs16 = reinterpret_cast<float*>(smem + a.xs_lds);

    // Stage x and its 16-value sums (two adjacent threads hold the chunks of one 16).
    {
        const __amdgpu_buffer_rsrc_t xr = raw_rsrc(a.x, uint32_t(M) * uint32_t(K) * 2u);
        const int total = M * cpr;
        for (int c0 = 0; c0 < total; c0 += 64 * kAnyWaves) {  // wave-uniform trip count
            const int c = c0 + tid;
            const bool live = c < total;
            const int m = live ? c / cpr : 0, q = c - m * cpr;
            const qa_u32x4 v = __builtin_bit_cast(
                qa_u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, live ? uint32_t(c) * 16u : kOutOfRange, 0, 0));
            float sum = 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++) sum += bf16_bits_to_f32(v[i] & 0xffffu) + bf16_bits_to_f32(v[i] >> 16);
            sum += __shfl_xor(sum, 1);
            if (live) {
                *reinterpret_cast<qa_u32x4*>(smem + m * K * 2 + any_chunk_slot(q) * 16) = v;
                if ((q & 1) == 0) xs16[m * (K / 16) + (q >> 1)] = sum;
            }
        }
    }
    __syncthreads();

    const uint32_t row_bytes = uint32_t(K) * BITS / 8;
    const __amdgpu_buffer_rsrc_t wr = raw_rsrc(a.w, uint32_t(N) * row_bytes);
    const __amdgpu_buffer_rsrc_t sr = raw_rsrc(a.s, uint32_t(N) * uint32_t(G) * (MX ? 1u : 2u));
    const __amdgpu_buffer_rsrc_t br = raw_rsrc(a.b ? a.b : a.s, a.b ? uint32_t(N) * uint32_t(G) * 2u : 0u);
    constexpr uint32_t kMagic = 0x43004300u;  // bf16 (128, 128)

    for (int n = blockIdx.x * kAnyWaves + wave; n < N; n += gridDim.x * kAnyWaves) {
        float acc[MC];
#pragma unroll
        for (int m = 0; m < MC; m++) acc[m] = 0.f;
#pragma unroll 2
        for (int j = lane; j < nseg; j += 64) {
            uint32_t wv[BITS];
            load_segment<BITS>(wv, wr, uint32_t(n) * row_bytes + uint32_t(j) * (4u * BITS));
            // parameters of the segment's group(s)
            float s0, b0 = 0.f, s1 = 0.f, b1 = 0.f;
            if constexpr (MX) {
                s0 = e8m0_to_f32(__builtin_amdgcn_raw_buffer_load_b8(sr, uint32_t(n) * uint32_t(G) + uint32_t(j), 0, 0));
            } else if constexpr (GS16) {
                const uint32_t po = (uint32_t(n) * uint32_t(G) + 2u * uint32_t(j)) * 2u;
                const uint32_t sv = __builtin_amdgcn_raw_buffer_load_b32(sr, po, 0, 0);
                const uint32_t bv = __builtin_amdgcn_raw_buffer_load_b32(br, po, 0, 0);
                s0 = any_param<ST>(sv), s1 = any_param<ST>(sv >> 16);
                b0 = any_param<ST>(bv), b1 = any_param<ST>(bv >> 16);
            } else {
                const uint32_t po = (uint32_t(n) * uint32_t(G) + uint32_t((32 * j) / gs)) * 2u;
                s0 = any_param<ST>(__builtin_amdgcn_raw_buffer_load_b16(sr, po, 0, 0));
                b0 = any_param<ST>(__builtin_amdgcn_raw_buffer_load_b16(br, po, 0, 0));
            }
            // code pairs as bf16 (128 + q0, 128 + q1)
            uint32_t pk[16];
            if constexpr (MX) {
#pragma unroll
                for (int r = 0; r < 4; r++) e2m1x8_to_bf16(wv[r], s0, pk + 4 * r);
            } else if constexpr (BITS < 8) {
#pragma unroll
                for (int i = 0; i < 16; i++) pk[i] = seg_code<BITS>(wv, 2 * i) | (seg_code<BITS>(wv, 2 * i + 1) << 16) | kMagic;
            }
#pragma unroll
            for (int m = 0; m < MC; m++) {
                if (m >= M) break;
                uint32_t xw[16];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const qa_u32x4 v =
                        *reinterpret_cast<const qa_u32x4*>(smem + m * K * 2 + any_chunk_slot(4 * j + r) * 16);
                    xw[4 * r] = v[0], xw[4 * r + 1] = v[1], xw[4 * r + 2] = v[2], xw[4 * r + 3] = v[3];
                }
                const float xa = xs16[m * (K / 16) + 2 * j], xb = xs16[m * (K / 16) + 2 * j + 1];
                float t0 = 0.f, t1 = 0.f;  // sum x q over values 0..15 and 16..31 of the segment
                if constexpr (MX) {
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        t0 = dot2_bf16(xw[i], pk[i], t0);
                        t1 = dot2_bf16(xw[8 + i], pk[8 + i], t1);
                    }
                } else if constexpr (BITS < 8) {
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        t0 = dot2_bf16(xw[i], pk[i], t0);
                        t1 = dot2_bf16(xw[8 + i], pk[8 + i], t1);
                    }
                    t0 = fmaf(-128.f, xa, t0);
                    t1 = fmaf(-128.f, xb, t1);
                } else {
#pragma unroll
                    for (int i = 0; i < 16; i++) {
                        const uint32_t q0 = seg_code<BITS>(wv, 2 * i), q1 = seg_code<BITS>(wv, 2 * i + 1);
                        float& t = i < 8 ? t0 : t1;
                        t = fmaf(bf16_bits_to_f32(xw[i] & 0xffffu), float(q0), t);
                        t = fmaf(bf16_bits_to_f32(xw[i] >> 16), float(q1), t);
                    }
                }
                if constexpr (MX) {
                    acc[m] += t0 + t1;
                } else if constexpr (GS16) {
                    acc[m] += fmaf(s0, t0, b0 * xa) + fmaf(s1, t1, b1 * xb);
                } else {
                    acc[m] += fmaf(s0, t0 + t1, b0 * (xa + xb));
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MC; m++) {
            if (m >= M) break;
            const float v = wave_sum(acc[m]);
            if (lane == 0) a.y[int64_t(m) * N + n] = uint16_t(f32_to_bf16_bits(v));
        }
    }
}

int any_lds_bytes(int M, int K) { return M * K * 2 + M * (K / 16) * 4; }

}  // namespace

bool launch_qmv_any(int bits, int gs, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w,
                    const void* s, const void* b, int M, int N, int K, hipStream_t st) {
    if (M < 1 || M > 16 || K % 32 != 0 || !(gs == 16 || gs % 32 == 0) || K % gs != 0 ||
        (scale_dtype != EQ_DTYPE_BF16 && scale_dtype != EQ_DTYPE_F16) || !aligned(x, 16) || !aligned(w, 4) ||
        !aligned(s, gs == 16 ? 4 : 2) || (b && !aligned(b, gs == 16 ? 4 : 2)))
        return false;
    if (bits != 2 && bits != 3 && bits != 4 && bits != 5 && bits != 6 && bits != 8) return false;
    const int64_t row_bytes = int64_t(K) * bits / 8;
    if (int64_t(N) * row_bytes >= (int64_t(1) << 31) || int64_t(N) * (K / gs) * 2 >= (int64_t(1) << 31) ||
        int64_t(kAnyMaxM) * K * 2 >= (int64_t(1) << 31))
        return false;
    const int mc_max = any_lds_bytes(kAnyMaxM, K) <= 65536 ? kAnyMaxM : (any_lds_bytes(1, K) <= 65536 ? 1 : 0);
    if (mc_max == 0) return false;
    const int64_t rows_wg = kAnyWaves;
    const int64_t grid = (N + rows_wg - 1) / rows_wg < int64_t(device_cu_count()) * 4
                             ? (N + rows_wg - 1) / rows_wg
                             : int64_t(device_cu_count()) * 4;
    for (int m0 = 0; m0 < M; m0 += mc_max) {
        const int mc = M - m0 < mc_max ? M - m0 : mc_max;
        QmvAnyArgs a{y + int64_t(m0) * N, x + int64_t(m0) * K, w, s, b, mc, N, K, gs, mc * K * 2};
        const size_t lds = size_t(any_lds_bytes(mc, K));
        auto go = [&](auto kernel) { kernel<<<dim3(unsigned(grid)), dim3(64 * kAnyWaves), lds, st>>>(a); };
        auto pick = [&](auto bits_tag, auto st_tag) {
            constexpr int B = decltype(bits_tag)::value;
            typedef decltype(st_tag) T;
            if (gs == 16) {
                if (mc == 1) go(qmv_any_kernel<B, T, 1, true>);
                else go(qmv_any_kernel<B, T, kAnyMaxM, true>);
            } else {
                if (mc == 1) go(qmv_any_kernel<B, T, 1, false>);
                else go(qmv_any_kernel<B, T, kAnyMaxM, false>);
            }
        };
        auto with_st = [&](auto bits_tag) {
            if (scale_dtype == EQ_DTYPE_BF16) pick(bits_tag, BF16T{});
            else pick(bits_tag, F16T{});
        };
        switch (bits) {
        case 2: with_st(std::integral_constant<int, 2>{}); break;
        case 3: with_st(std::integral_constant<int, 3>{}); break;
        case 4: with_st(std::integral_constant<int, 4>{}); break;
        case 5: with_st(std::integral_constant<int, 5>{}); break;
        case 6: with_st(std::integral_constant<int, 6>{}); break;
        default: with_st(std::integral_constant<int, 8>{}); break;
        }
    }
    return true;
}

bool launch_qmv_any_mxfp4(uint16_t* y, const uint16_t* x, const uint32_t* w, const uint8_t* s, int M, int N, int K,
                          hipStream_t st) {
    if (M < 1 || M > 16 || K % 32 != 0 || !aligned(x, 16) || !aligned(w, 4)) return false;
    if (int64_t(N) * K / 2 >= (int64_t(1) << 31) || int64_t(kAnyMaxM) * K * 2 >= (int64_t(1) << 31)) return false;
    const int mc_max = any_lds_bytes(kAnyMaxM, K) <= 65536 ? kAnyMaxM : (any_lds_bytes(1, K) <= 65536 ? 1 : 0);
    if (mc_max == 0) return false;
    const int64_t rows_wg = kAnyWaves;
    const int64_t grid = (N + rows_wg - 1) / rows_wg < int64_t(device_cu_count()) * 4 ? (N + rows_wg - 1) / rows_wg
                                                                                      : int64_t(device_cu_count()) * 4;
    for (int m0 = 0; m0 < M; m0 += mc_max) {
        const int mc = M - m0 < mc_max ? M - m0 : mc_max;
        QmvAnyArgs a{y + int64_t(m0) * N, x + int64_t(m0) * K, w, s, nullptr, mc, N, K, 32, mc * K * 2};
        const size_t lds = size_t(any_lds_bytes(mc, K));
        if (mc == 1) qmv_any_kernel<4, BF16T, 1, false, true><<<dim3(unsigned(grid)), dim3(64 * kAnyWaves), lds, st>>>(a);
        else qmv_any_kernel<4, BF16T, kAnyMaxM, false, true><<<dim3(unsigned(grid)), dim3(64 * kAnyWaves), lds, st>>>(a);
    }
    return true;
}

}  // namespace eq
