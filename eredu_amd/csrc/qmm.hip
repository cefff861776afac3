// Prefill-shaped quantized matmul (M > 16, bf16 activations, transpose = true)
// on gfx950 matrix cores.
//
// y = x . W^T with W[n, k] = s[n, k/gs] * q[n, k] + b[n, k/gs]
// (safemlx/src/ops/quantization.rs:190-226, QuantizedLinear's layout).
//
// Work layout.  A workgroup of 8 waves owns a 128 (m) x 256 (n) output tile
// and walks K (or one split of it) in chunks of 64.  The waves form two
// K-groups of 4 that take alternate chunks (even, odd), each with its own
// double-buffered activation tile in LDS, so that every SIMD runs two waves
// (one's dequantization and memory waits overlap the other's MFMAs) while a
// wave keeps a large output block; at the end the second K-group adds its
// sums into the first through LDS.  Wave w of a K-group owns the 64 columns
// [64w, 64w + 64) and all 128 rows: 4 x 2 tiles of v_mfma_f32_32x32x16_bf16
// with f32 accumulators.
//
//  * Weights never touch LDS.  Each wave dequantizes only its own columns,
//    straight from 16-byte loads into the B-operand registers: lane l reads
//    row n = l % 32 of a 32-column block, 32 consecutive codes starting at
//    k = 32 * (l / 32); code word t of those feeds MFMA step t.  w = s*q + b is
//    one f32 FMA per code and one v_cvt_pk_bf16_f32 per pair, and is used by
//    the 4 row blocks of the tile.
//  * Activations go through LDS (shared by the 4 waves), double buffered.
//    16-byte chunks of a row are stored at chunk c ^ (row & 7), so the rows of
//    one A operand read different banks.  A operand of step t for lane
//    (m, kb) = x[m][k0 + 32 kb + 8 t .. + 8], matching the codes the B lane
//    (n, kb) holds for step t.
//  * Pipeline: before chunk c is computed, the activations of chunk c + 1
//    (from L2, into registers; written to the other LDS buffer after the
//    compute) and the codes and parameters of chunk c + 2 (from HBM, into a
//    three-slot register ring) are requested.  The loop is unrolled by three
//    so that no slot is ever copied (a copy of a register that is still
//    loading makes the wave wait for every load in flight).  Chunk offsets go
//    into the scalar offset operand of the buffer loads, so issuing a chunk
//    takes no vector instruction.
//  * All global reads are buffer loads: rows past M or N read as zero, so any
//    M and N work (K is a multiple of 64, checked by the dispatcher).
//  * Split K: when the output has too few tiles to fill the GPU, each tile's K
//    is split over several workgroups that write f32 partial tiles to a
//    workspace; a second kernel sums the splits in a fixed order (results do
//    not depend on timing) and rounds once to bf16.
//  * Tiles are assigned so that the workgroups one XCD receives cover few
//    row blocks of x (which then stay in that XCD's L2).
#include <mutex>

#include "eq_common.hpp"

namespace eq {

typedef uint32_t q_u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 q_bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kBM = 128, kBN = 256, kBK = 64;
constexpr int kQmmThreads = 512;        // two K-groups of 4 waves
constexpr int kLdsBuf = kBM * kBK * 2;  // bytes per activation buffer
constexpr int kRing = 3;                // register slots of the load ring

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

// One ring slot: this lane's codes and parameters (2 column blocks x 32 codes).
template <int BITS>
struct QmmSlot {
    static constexpr int WORDS = BITS;  // 32 codes * BITS / 32
    q_u32x4 w[2][WORDS / 4];
    uint32_t s[2], b[2];
};

// Reads every register of a slot in an empty asm statement (the never-taken
// side of an opaque_one() guard): every path then retires the slot's loads,
// which keeps the compiler's wait analysis exact at the join.
template <int BITS>
__device__ __forceinline__ void qmm_retire(const QmmSlot<BITS>& s) {
#pragma unroll
    for (int j = 0; j < 2; j++) {
#pragma unroll
        for (int i = 0; i < QmmSlot<BITS>::WORDS / 4; i++) asm volatile("" ::"v"(s.w[j][i]));
        asm volatile("" ::"v"(s.s[j]), "v"(s.b[j]));
    }
}

template <typename ST>
__device__ __forceinline__ float qmm_param(uint32_t bits);
template <>
__device__ __forceinline__ float qmm_param<BF16T>(uint32_t bits) { return bf16_bits_to_f32(bits & 0xffffu); }
template <>
__device__ __forceinline__ float qmm_param<F16T>(uint32_t bits) { return f16_bits_to_f32(bits & 0xffffu); }

struct QmmArgs {
    uint16_t* y;
    float* ws;  // split K: f32 partial tiles, [split][M][N]
    const uint16_t* x;
    const uint32_t* w;
    const uint16_t* s;
    const uint16_t* b;  // may be null
    int M, N, K, mtiles, ntiles, splits, cps;  // cps: chunks per split
};

template <int BITS, int GS, typename ST, bool SPLIT>
__global__ __launch_bounds__(kQmmThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void qmm_mfma_kernel(
    const QmmArgs args) {
    __shared__ __attribute__((aligned(16))) char lds_all[2 * 2 * kLdsBuf];  // [K-group][buffer]
    const int M = args.M, N = args.N, K = args.K;

    // Tile and split of this workgroup: the workgroups of one XCD (id % 8)
    // take a contiguous run of row-major tiles, i.e. few row blocks of x.
    const int T = args.mtiles * args.ntiles * args.splits;
    int bid = blockIdx.x;
    if ((T & 7) == 0) bid = (bid & 7) * (T >> 3) + (bid >> 3);
    const int split = bid % args.splits, tile = bid / args.splits;
    const int tm = tile / args.ntiles, tn = tile % args.ntiles;
    const int m0 = tm * kBM, n0 = tn * kBN;
    const int nchunks = K / kBK;
    const int c_begin = split * args.cps, c_end = min(nchunks, c_begin + args.cps);
    const int nloc = c_end - c_begin;  // >= 1 (the planner leaves no split empty)

    const int lane = threadIdx.x & 63;
    const int kgrp = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 8);  // K-group: chunks 2i + kgrp
    const int tid = threadIdx.x & 255;                                         // thread within the K-group
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);                 // column quarter
    const int l32 = lane & 31, kb = lane >> 5;
    char* lds = lds_all + kgrp * 2 * kLdsBuf;
    const int steps = (nloc + 1) / 2;  // chunks per K-group (the second may have one fewer)
    const int G = K / GS;

    const __amdgpu_buffer_rsrc_t xr = raw_rsrc(args.x, uint32_t(M) * uint32_t(K) * 2u);
    const __amdgpu_buffer_rsrc_t wr = raw_rsrc(args.w, uint32_t(N) * uint32_t(K) * BITS / 8u);
    const __amdgpu_buffer_rsrc_t sr = raw_rsrc(args.s, uint32_t(N) * uint32_t(G) * 2u);
    const __amdgpu_buffer_rsrc_t br = raw_rsrc(args.b ? args.b : args.s, args.b ? uint32_t(N) * uint32_t(G) * 2u : 0u);

    // Lane offsets (chunk 0); rows past M and columns past N read zero.
    // Activations: thread tid copies the 16-byte chunks q = tid + 256 i
    // (row q / 8, chunk q % 8) of each 128 x 64 tile.
    uint32_t a_goff[4], a_loff[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int q = tid + 256 * i, row = q >> 3, c = q & 7;
        a_goff[i] = m0 + row < M ? (uint32_t(m0 + row) * uint32_t(K) + uint32_t(8 * c)) * 2u : kOutOfRange;
        a_loff[i] = uint32_t(row * (kBK * 2) + ((c ^ (row & 7)) << 4));
    }
    // Weight rows of this lane: columns n0 + 64 wave + 32 j + l32, codes from 32 kb.
    uint32_t woff[2], soff[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t n = uint32_t(n0 + 64 * wave + 32 * j + l32);
        woff[j] = int(n) < N ? n * uint32_t(K) * BITS / 8u + uint32_t(32 * kb) * BITS / 8u : kOutOfRange;
        soff[j] = int(n) < N ? (n * uint32_t(G)) * 2u + uint32_t((32 * kb) / GS) * 2u : kOutOfRange;
    }
    // (a lane's 32 codes lie in one group: group sizes are multiples of 32 and
    // chunks start at multiples of 64, so its group is k0 / GS + 32 kb / GS)

    // Loads of this K-group's chunk i, i.e. chunk 2i + kgrp of the split (past
    // the split's end: the last chunk again, in cache and never computed).
    auto chunk_k0 = [&](int i) __attribute__((always_inline)) {
        return (c_begin + min(2 * i + kgrp, nloc - 1)) * kBK;
    };
    auto load_a = [&](q_u32x4* r, int i) __attribute__((always_inline)) {
        const uint32_t ks = __builtin_amdgcn_readfirstlane(uint32_t(chunk_k0(i)) * 2u);
#pragma unroll
        for (int q = 0; q < 4; q++) r[q] = __builtin_amdgcn_raw_buffer_load_b128(xr, a_goff[q], ks, 0);
    };
    auto load_b = [&](QmmSlot<BITS>& S, int i) __attribute__((always_inline)) {
        const int k0 = chunk_k0(i);
        const uint32_t kw = __builtin_amdgcn_readfirstlane(uint32_t(k0) * BITS / 8u);
        const uint32_t kp = __builtin_amdgcn_readfirstlane(uint32_t(k0 / GS) * 2u);
#pragma unroll
        for (int j = 0; j < 2; j++) {
#pragma unroll
            for (int q = 0; q < QmmSlot<BITS>::WORDS / 4; q++)
                S.w[j][q] = __builtin_amdgcn_raw_buffer_load_b128(wr, woff[j] + 16 * q, kw, 0);
            S.s[j] = __builtin_amdgcn_raw_buffer_load_b16(sr, soff[j], kp, 0);
            S.b[j] = __builtin_amdgcn_raw_buffer_load_b16(br, soff[j], kp, 0);
        }
    };
    auto store_a = [&](const q_u32x4* r, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 4; q++) *reinterpret_cast<q_u32x4*>(lds + buf * kLdsBuf + a_loff[q]) = r[q];
    };

    // A operand of this lane for step t and row block mi: row 32 mi + l32,
    // chunk (4 kb + t) ^ (row & 7) (row & 7 = l32 & 7 for every mi).
    uint32_t aoff[4];
#pragma unroll
    for (int t = 0; t < 4; t++) aoff[t] = uint32_t(l32 * (kBK * 2) + (((4 * kb + t) ^ (l32 & 7)) << 4));

    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x16{};

    auto compute = [&](const QmmSlot<BITS>& S, int buf) __attribute__((always_inline)) {
        asm volatile("" ::: "memory");
        q_u32x4 bq[2][4];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const float s = qmm_param<ST>(S.s[j]);
            const float b = qmm_param<ST>(S.b[j]);
#pragma unroll
            for (int t = 0; t < 4; t++)
                bq[j][t] = dequant8<BITS>(reinterpret_cast<const uint32_t*>(&S.w[j][0]) + t * BITS / 4, s, b);
        }
        const char* base = lds + buf * kLdsBuf;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            bf16x8 a[4];
#pragma unroll
            for (int mi = 0; mi < 4; mi++)
                a[mi] = *reinterpret_cast<const bf16x8*>(base + aoff[t] + mi * 32 * (kBK * 2));
#pragma unroll
            for (int mi = 0; mi < 4; mi++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[mi][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, bq[j][t]), a[mi],
                                                                         acc[mi][j], 0, 0, 0);
        }
    };

    // Prologue: chunk 0's activations in LDS; codes of chunks 0 and 1 requested.
    QmmSlot<BITS> ring[kRing];
    q_u32x4 areg[4];
    load_a(areg, 0);
    load_b(ring[0], 0);
    load_b(ring[1], 1);
    store_a(areg, 0);
    __syncthreads();

    // Step i: request chunk i + 1's activations and chunk i + 2's codes,
    // compute chunk i (LDS buffer i & 1), store chunk i + 1's activations into
    // the other buffer, synchronise.
    for (int i0 = 0;; i0 += kRing) {
#pragma unroll
        for (int r = 0; r < kRing; r++) {
            const int i = i0 + r;
            load_a(areg, i + 1);
            load_b(ring[(r + 2) % kRing], i + 2);
            if (opaque_one() && 2 * i + kgrp < nloc) compute(ring[r], i & 1);
            else qmm_retire(ring[r]);
            if (i + 1 >= steps) goto done;
            store_a(areg, (i + 1) & 1);
            __syncthreads();
        }
    }
done:
    // The second K-group's sums go to LDS (half the row blocks at a time:
    // 64 KiB), the first adds them.  Layout: [wave][mi & 1][j][q][lane] x 16 B,
    // q = the run of 4 accumulator registers.
#pragma unroll
    for (int half = 0; half < 2; half++) {
        __syncthreads();
        f32x4* red = reinterpret_cast<f32x4*>(lds_all);
        if (kgrp == 1) {
#pragma unroll
            for (int mh = 0; mh < 2; mh++)
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        red[(((wave * 2 + mh) * 2 + j) * 4 + q) * 64 + lane] =
                            f32x4{acc[2 * half + mh][j][4 * q], acc[2 * half + mh][j][4 * q + 1],
                                  acc[2 * half + mh][j][4 * q + 2], acc[2 * half + mh][j][4 * q + 3]};
        }
        __syncthreads();
        if (kgrp == 0) {
#pragma unroll
            for (int mh = 0; mh < 2; mh++)
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const f32x4 v = red[(((wave * 2 + mh) * 2 + j) * 4 + q) * 64 + lane];
#pragma unroll
                        for (int e = 0; e < 4; e++) acc[2 * half + mh][j][4 * q + e] += v[e];
                    }
        }
    }
    if (kgrp == 1) return;

    // The MFMA computed y^T blocks (weights as the first operand): register r
    // of lane l holds row m = 32 mi + l % 32 and column n = 32 j + 8 (r / 4) +
    // 4 (l / 32) + r % 4, so each run of 4 registers is 4 adjacent columns of
    // one row.  Columns past N are whole waves (N % 128 == 0).
    if (n0 + 64 * wave >= N) return;
#pragma unroll
    for (int mi = 0; mi < 4; mi++) {
        const int m = m0 + 32 * mi + l32;
        if (m < M) {
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int n = n0 + 64 * wave + 32 * j + 8 * q + 4 * kb;
                    const f32x4 v = {acc[mi][j][4 * q], acc[mi][j][4 * q + 1], acc[mi][j][4 * q + 2], acc[mi][j][4 * q + 3]};
                    if constexpr (SPLIT) {
                        *reinterpret_cast<f32x4*>(args.ws + (int64_t(split) * M + m) * N + n) = v;
                    } else {
                        const uint32_t lo = pack_bf16x2(v[0], v[1]), hi = pack_bf16x2(v[2], v[3]);
                        *reinterpret_cast<uint2*>(args.y + int64_t(m) * N + n) = make_uint2(lo, hi);
                    }
                }
        }
    }
}

// y = bf16(sum over splits of the partial tiles), splits summed in order.
__global__ __launch_bounds__(256) void qmm_split_reduce(uint16_t* __restrict__ y, const float* __restrict__ ws,
                                                         int64_t mn, int splits, bool vec) {
    typedef float f32x4_t __attribute__((ext_vector_type(4)));
    const int64_t i = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
    if (i >= mn) return;
    if (vec && i + 4 <= mn) {
        f32x4_t v = *reinterpret_cast<const f32x4_t*>(ws + i);
        for (int s = 1; s < splits; s++) {
            const f32x4_t u = *reinterpret_cast<const f32x4_t*>(ws + int64_t(s) * mn + i);
            v = f32x4_t{v[0] + u[0], v[1] + u[1], v[2] + u[2], v[3] + u[3]};
        }
        typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
        *reinterpret_cast<u16x4*>(y + i) = u16x4{uint16_t(f32_to_bf16_bits(v[0])), uint16_t(f32_to_bf16_bits(v[1])),
                                                 uint16_t(f32_to_bf16_bits(v[2])), uint16_t(f32_to_bf16_bits(v[3]))};
    } else {
        for (int64_t e = i; e < mn; e++) {
            float v = ws[e];
            for (int s = 1; s < splits; s++) v += ws[int64_t(s) * mn + e];
            y[e] = uint16_t(f32_to_bf16_bits(v));
        }
    }
}

// Per-device f32 workspace for split K, grown on demand outside stream
// capture (a capturing caller whose workspace is too small gets no split).
static float* qmm_workspace(size_t bytes, hipStream_t st) {
    static std::mutex mu;
    static float* ptr[64] = {};
    static size_t cap[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (cap[dev] >= bytes) return ptr[dev];
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
    // the old buffer may still be in use by queued work: synchronise first
    if (ptr[dev]) {
        if (hipDeviceSynchronize() != hipSuccess) return nullptr;
        (void)hipFree(ptr[dev]);
        ptr[dev] = nullptr;
        cap[dev] = 0;
    }
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) return nullptr;
    ptr[dev] = static_cast<float*>(p);
    cap[dev] = bytes;
    return ptr[dev];
}

// Compute units of the current device.
static int qmm_cu_count() {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) return 256;
    return v;
}

template <int BITS, int GS, typename ST>
static void launch_qmm_t(uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s, const void* b, int M,
                         int N, int K, hipStream_t st) {
    QmmArgs a{};
    a.y = y, a.x = x, a.w = w, a.s = static_cast<const uint16_t*>(s), a.b = static_cast<const uint16_t*>(b);
    a.M = M, a.N = N, a.K = K;
    a.mtiles = (M + kBM - 1) / kBM, a.ntiles = (N + kBN - 1) / kBN;
    const int tiles = a.mtiles * a.ntiles, nchunks = K / kBK;
    // Split K so that the grid covers the CUs, at least 8 chunks per split (4
    // per K-group).
    int splits = (qmm_cu_count() + tiles / 2) / tiles;
    splits = splits < 1 ? 1 : splits;
    splits = splits > nchunks / 8 ? nchunks / 8 : splits;
    splits = splits < 1 ? 1 : splits;
    if (splits > 1) {
        a.cps = (nchunks + splits - 1) / splits;
        splits = (nchunks + a.cps - 1) / a.cps;  // no empty split
        a.ws = qmm_workspace(size_t(splits) * size_t(M) * size_t(N) * 4u, st);
        if (!a.ws) splits = 1;
    }
    a.splits = splits;
    if (splits == 1) {
        a.cps = nchunks;
        qmm_mfma_kernel<BITS, GS, ST, false><<<dim3(unsigned(tiles)), dim3(kQmmThreads), 0, st>>>(a);
        return;
    }
    qmm_mfma_kernel<BITS, GS, ST, true><<<dim3(unsigned(tiles * splits)), dim3(kQmmThreads), 0, st>>>(a);
    const int64_t mn = int64_t(M) * N;
    qmm_split_reduce<<<dim3(unsigned((mn / 4 + 255) / 256 + 1)), dim3(256), 0, st>>>(y, a.ws, mn, splits,
                                                                                    aligned(y, 8));
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
// K % 64 == 0 and K % gs == 0, 16-byte aligned x and w, scale dtype bf16 or
// f16, buffers below 2^31 bytes.
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
