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

namespace eq {
namespace {

typedef uint32_t qn_u32x4 __attribute__((ext_vector_type(4)));

// Raw bits of a scale or bias (bf16 / f16 in the low half, or f32) -> f32.
template <typename ST> __device__ __forceinline__ float param_bits(uint32_t v);
template <> __device__ __forceinline__ float param_bits<BF16T>(uint32_t v) { return bf16_bits_to_f32(v & 0xffffu); }
template <> __device__ __forceinline__ float param_bits<F16T>(uint32_t v) { return f16_bits_to_f32(v & 0xffffu); }
template <> __device__ __forceinline__ float param_bits<F32T>(uint32_t v) { return __uint_as_float(v); }

// Workgroup = TW word columns x KP = 256 / TW row phases.  Lane (jw, p) owns
// the code word j = blockIdx.x * TW + jw of every row (32 / BITS consecutive
// columns, inside one group since gs >= 32) and walks rows kb + p, kb + p +
// KP, ... of its K split [kb, ke) (blockIdx.y); consecutive lanes read
// consecutive words of a row.  The phases are summed through LDS; with more
// than one split the sums go to ws[split][batch][M][N] for qmm_n_finish.
// MXFP4 (ST = E8M0T, no biases): the codes convert to their E2M1 values
// (v_cvt_scalef32_pk_f32_fp4 at scale 1) and x s carries 2^(e - 127).
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
            if constexpr (__is_same(ST, E8M0T)) {
                const auto v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, 0);
                const auto v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, 1);
                const auto v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, 2);
                const auto v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, 3);
                q[0] = v0[0], q[1] = v0[1], q[2] = v1[0], q[3] = v1[1];
                q[4] = v2[0], q[5] = v2[1], q[6] = v3[0], q[7] = v3[1];
            } else if constexpr (BITS == 4) {
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

// M = 1.  A workgroup owns a tile of C = 4 CPL columns (lane cl of 4 reads
// 16 bytes = CPL codes of a row, so a wave reads 16 rows x 64 contiguous
// bytes per load) and a run of R rows [kb, ke) of one batch; its 64 row phases
// p take rows kb + p, kb + p + 64, ...
//  * Staged in LDS first: xs[r][gi] = x[k] s[k, g] (f32) for the tile's NG
//    groups, and sum_k x[k] b[k, g] per group (the bias term, shared by the
//    columns of a group).  Those loads go out before the first codes, so the
//    L2 trip of the staging overlaps the HBM trip of the codes.
//  * Per row a lane then adds xs * q into CPL column sums (one convert and one
//    FMA per code); its rows' codes are requested U rows ahead.
//  * The 64 phases are summed through LDS.  With one run per tile the sums
//    are y.  With several (split K) a run's sums go to ws[split][batch][N] and,
//    when the launch has arrival counters, the workgroup that finishes a tile
//    last adds the runs in split order (device-scope stores and loads: the
//    runs of a tile may run on different XCDs) and writes y; without
//    counters qmm_n_finish does that in a second launch.
struct QmmN1Args {
    uint16_t* y;
    float* ws;            // split K: [splits][batch_total][N] run sums
    unsigned* counters;   // per (batch in launch, column tile); null: qmm_n_finish sums the runs
    const uint16_t* x;
    const uint32_t* w;
    const void* s;
    const void* b;        // may be null
    GatherIdx g;
    int N, K, gs, R, splits, ctiles;
    int64_t b0, batch_total;
};

constexpr int kQmmN1Phases = 64;   // row phases per workgroup
constexpr int kQmmN1Stage = 512;   // staged (row, group) products per workgroup, at most
constexpr int kQmmN1Unroll = 4;    // rows per lane and load block

template <int BITS, typename ST>
__global__ __launch_bounds__(256) void qmm_n_m1(const QmmN1Args a) {
    typedef typename ST::storage SS;
    constexpr int CPL = 128 / BITS, C = 4 * CPL, RP = kQmmN1Phases, U = kQmmN1Unroll;
    constexpr int RS = C + 4;  // row stride of the phase sums (spreads the phases over banks)
    constexpr int E = kQmmN1Stage / 256;
    static_assert(kQmmN1Stage <= RP * RS, "the staged products share the phase-sum buffer");
    __shared__ __attribute__((aligned(16))) float lds[RP * RS];  // staged products, then phase sums
    __shared__ float xbias_w[4][4];                                // [wave][group in tile]
    __shared__ float colpart[256];
    __shared__ unsigned ticket;
    const int tid = threadIdx.x, cl = tid & 3, p = tid >> 2, lane = tid & 63, wave = tid >> 6;
    const int N = a.N, K = a.K, gs = a.gs, G = N / gs;
    // Workgroups reach the 8 XCDs round-robin by linear id, each XCD with its
    // own L2; (tile, split) pairs are numbered split-major and dealt out so
    // that the tiles of one run -- which read the same x, scale and bias
    // rows -- share an XCD: unit = x * floor(T / 8) + min(x, T % 8) + id / 8
    // for id on XCD x = id % 8 (a bijection of [0, T) for any T).
    const int total = gridDim.x, lin = blockIdx.x, xcd = lin & 7;
    const int unit = xcd * (total >> 3) + min(xcd, total & 7) + (lin >> 3);
    const int tile = unit % a.ctiles, split = unit / a.ctiles;
    const int64_t b = a.b0 + blockIdx.z;
    const int kb = split * a.R, ke = min(K, kb + a.R);
    const int n0 = tile * C, g0 = n0 / gs;
    const int NG = C >= gs ? C / gs : 1;  // groups in the tile (1, 2 or 4)
    int64_t xbt, wbt;
    const bool ok = gather_batch(a.g, b, xbt, wbt);
    if (!ok) xbt = wbt = 0;  // read in-range rows, contribute nothing
    const int rows = ok ? ke - kb : 0;

    // Staging loads: element e = r * NG + gi (row kb + r, group g0 + gi).
    // Buffer loads, unconditional: elements past the run (or of a failed
    // gather) read as zero through out-of-range offsets, so no load sits
    // behind a branch (which would make the wave wait for it on the spot).
    const uint16_t* xp = a.x + xbt * K;
    const SS* sp = static_cast<const SS*>(a.s) + wbt * int64_t(K) * G;
    const SS* bp = a.b ? static_cast<const SS*>(a.b) + wbt * int64_t(K) * G : sp;
    const __amdgpu_buffer_rsrc_t xr = raw_rsrc(xp, uint32_t(K) * 2u);
    const __amdgpu_buffer_rsrc_t sr = raw_rsrc(sp, uint32_t(K) * uint32_t(G) * uint32_t(sizeof(SS)));
    const __amdgpu_buffer_rsrc_t br = raw_rsrc(bp, a.b ? uint32_t(K) * uint32_t(G) * uint32_t(sizeof(SS)) : 0u);
    const int ne = a.R * NG;
    uint32_t xv[E], sv[E], bv[E];
#pragma unroll
    for (int i = 0; i < E; i++) {
        const int e = tid + 256 * i;
        const int r = e / NG, gi = e % NG;
        const bool live = e < ne && r < rows && g0 + gi < G;
        const uint32_t xo = live ? uint32_t(kb + r) * 2u : kOutOfRange;
        const uint32_t po = live ? (uint32_t(kb + r) * uint32_t(G) + uint32_t(g0 + gi)) * uint32_t(sizeof(SS)) : kOutOfRange;
        xv[i] = __builtin_amdgcn_raw_buffer_load_b16(xr, xo, 0, 0);
        if constexpr (sizeof(SS) == 2) {
            sv[i] = __builtin_amdgcn_raw_buffer_load_b16(sr, po, 0, 0);
            bv[i] = __builtin_amdgcn_raw_buffer_load_b16(br, po, 0, 0);
        } else {
            sv[i] = __builtin_amdgcn_raw_buffer_load_b32(sr, po, 0, 0);
            bv[i] = __builtin_amdgcn_raw_buffer_load_b32(br, po, 0, 0);
        }
    }

    // The first block of codes.
    const uint32_t row_bytes = uint32_t(N) * BITS / 8;
    const __amdgpu_buffer_rsrc_t wr =
        raw_rsrc(a.w + wbt * int64_t(K) * (N * BITS / 32), uint32_t(K) * row_bytes);
    const int col = n0 + cl * CPL;
    const bool col_ok = col < N;
    const int nr = (a.R + RP - 1) / RP;  // row slots per lane
    auto load_block = [&](qn_u32x4* v, int i0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int r = p + (i0 + u) * RP;
            const uint32_t off =
                (col_ok && r < rows) ? uint32_t(kb + r) * row_bytes + uint32_t(col) * BITS / 8 : kOutOfRange;
            v[u] = __builtin_bit_cast(qn_u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0));
        }
    };
    qn_u32x4 wa[U], wb[U];
    load_block(wa, 0);

    // Finish the staging: products to LDS, this thread's bias part (group tid % NG).
    float* xs = lds;
    float xb = 0.f;
#pragma unroll
    for (int i = 0; i < E; i++) {
        const int e = tid + 256 * i;
        // dead elements read zero: x1 = 0 makes both terms vanish
        const float x1 = bf16_bits_to_f32(xv[i]);
        if (e < ne) xs[e] = x1 * param_bits<ST>(sv[i]);
        xb = fmaf(x1, param_bits<ST>(bv[i]), xb);
    }
    // sum the bias parts of each group: lanes of one group are NG apart
    for (int o = 32; o >= NG; o >>= 1) xb += __shfl_xor(xb, o);
    if (lane < NG) xbias_w[wave][lane] = xb;
    __syncthreads();

    // Main loop: the next block's codes are requested before this one is used
    // (past the last row slot the loads go out of range and touch nothing).
    const int gil = col_ok ? col / gs - g0 : 0;
    float acc[CPL];
#pragma unroll
    for (int c = 0; c < CPL; c++) acc[c] = 0.f;
    auto compute = [&](const qn_u32x4* v, int i0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int r = p + (i0 + u) * RP;
            const float x1 = r < a.R ? xs[r * NG + gil] : 0.f;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint32_t wd = v[u][t];
                if constexpr (BITS == 4) {
                    const uint32_t lo = wd & 0x0f0f0f0fu, hi = (wd >> 4) & 0x0f0f0f0fu;  // codes 0,2,4,6 / 1,3,5,7
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        acc[8 * t + 2 * i] = fmaf(x1, float((lo >> (8 * i)) & 0xffu), acc[8 * t + 2 * i]);
                        acc[8 * t + 2 * i + 1] = fmaf(x1, float((hi >> (8 * i)) & 0xffu), acc[8 * t + 2 * i + 1]);
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[4 * t + i] = fmaf(x1, float((wd >> (8 * i)) & 0xffu), acc[4 * t + i]);
                }
            }
        }
    };
    for (int i0 = 0; i0 < nr; i0 += 2 * U) {
        load_block(wb, i0 + U);
        compute(wa, i0);
        load_block(wa, i0 + 2 * U);
        if (i0 + U < nr) compute(wb, i0 + U);
    }

    // Phase sums through LDS (the staged products are dead: barrier first).
    __syncthreads();
#pragma unroll
    for (int c = 0; c < CPL; c += 4)
        *reinterpret_cast<float4*>(lds + p * RS + cl * CPL + c) = make_float4(acc[c], acc[c + 1], acc[c + 2], acc[c + 3]);
    __syncthreads();
    {
        constexpr int H = 256 / C;  // threads per column
        const int c = tid % C, h = tid / C;
        float v = 0.f;
#pragma unroll 8
        for (int q = h * (RP / H); q < (h + 1) * (RP / H); q++) v += lds[q * RS + c];
        colpart[tid] = v;
    }
    __syncthreads();
    float v = 0.f;
    const int n = n0 + tid;
    if (tid < C) {
        constexpr int H = 256 / C;
#pragma unroll
        for (int h = 0; h < H; h++) v += colpart[h * C + tid];
        const int gi = (n < N ? n / gs : g0) - g0;
#pragma unroll
        for (int w = 0; w < 4; w++) v += xbias_w[w][gi];
    }
    if (a.splits == 1) {
        if (tid < C && n < N) a.y[b * N + n] = uint16_t(f32_to_bf16_bits(v));
        return;
    }
    float* wsb = a.ws + b * int64_t(N);  // run s of this batch at wsb + s * batch_total * N
    const int64_t sstride = a.batch_total * int64_t(N);
    if (!a.counters) {
        if (tid < C && n < N) wsb[split * sstride + n] = v;
        return;
    }
    if (tid < C && n < N) __hip_atomic_store(wsb + split * sstride + n, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!last_arriver(a.counters + blockIdx.z * a.ctiles + tile, unsigned(a.splits), &ticket)) return;
    if (tid < C && n < N) {
        float t = 0.f;
        int s0 = 0;
        for (; s0 + 8 <= a.splits; s0 += 8) {
            float r8[8];
#pragma unroll
            for (int i = 0; i < 8; i++)
                r8[i] = __hip_atomic_load(wsb + (s0 + i) * sstride + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int i = 0; i < 8; i++) t += r8[i];
        }
        for (; s0 < a.splits; s0++)
            t += __hip_atomic_load(wsb + s0 * sstride + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        a.y[b * N + n] = uint16_t(f32_to_bf16_bits(t));
    }
}

// ------------------------------------------------ M = 1, 4-bit codes, on MFMA
//
// The same product on v_mfma_f32_16x16x32_bf16, with the codes transposed on
// their way out of LDS.  A workgroup owns a tile of 128 columns (8 slices of
// 16) and a run of rows [kb, ke), walked in chunks of kQnmRows rows.  Per
// chunk:
//  * the codes (rows x 64 bytes) are copied to LDS, rows kQnmWStride bytes
//    apart (the 16 rows of one transposing read then fall in different banks);
//  * the activation side is staged per (row, group of the tile):
//    xs = x[k] s[k, g] as two bf16 values hi = bf16(xs), lo = bf16(xs - hi)
//    (together about 16 significant bits), in the order of the unpacked codes
//    below; the run's sums of hi + lo and of x[k] b[k, g] are kept per group.
// The loads of the next two chunks are in flight while a chunk is computed.
//
// The 8 waves of a workgroup own one 16-column slice each (with 4 waves, two
// adjacent slices of one group; 8 measured 3-6 % faster on MI355X).
// ds_read_b64_tr_b4 transposes a 16 x 16 block of nibbles within each
// 16-lane group: lane (g, i) names row
// 16g + i of a 64-row block at the slice's 8 bytes and receives column i's
// codes of rows 16g .. 16g + 15.  Its first word is the B operand of one MFMA
// (rows 16g + 0..7 for lane block g), its second of the next (rows
// 16g + 8..15); the codes unpack as bf16 128 + q in row order 0,2,4,6,1,3,5,7
// and the staged pairs are stored in that order.  A operand row 0 = hi, row
// 1 = lo, the other rows zero, so C rows 0 + 1 = sum_k xs (128 + q), and
//   y[n] = C0 + C1 - 128 sum_k (hi + lo) + sum_k x b.
// Runs of one tile are combined as in qmm_n_m1.
#ifndef EQ_QNM_WAVES
#define EQ_QNM_WAVES 8
#endif
constexpr int kQnmWaves = EQ_QNM_WAVES;              // waves per workgroup: 8 / kQnmWaves slices each
constexpr int kQnmThreads = 64 * kQnmWaves;
constexpr int kQnmCols = 128;                        // columns per tile
constexpr int kQnmRows = 256;                        // rows per chunk
constexpr int kQnmWStride = 80;                      // LDS bytes per code row
constexpr int kQnmWBytes = kQnmRows * kQnmWStride;   // code buffer
constexpr int kQnmABytes = 4 * 2 * kQnmRows * 2;     // staged pairs: [group][hi, lo][row] bf16

// 8 codes of one 32-bit word (nibble j = row j) -> bf16 128 + q in row order
// 0,2,4,6,1,3,5,7: two masks, a shift, four byte permutes against 0x43.
__device__ __forceinline__ bf16x8 qnm_unpack(uint32_t w) {
    const uint32_t c43 = 0x43434343u;
    const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
    qn_u32x4 p;
    p[0] = __builtin_amdgcn_perm(c43, lo, 0x04010400u);  // [b0, 43, b1, 43]
    p[1] = __builtin_amdgcn_perm(c43, lo, 0x04030402u);
    p[2] = __builtin_amdgcn_perm(c43, hi, 0x04010400u);
    p[3] = __builtin_amdgcn_perm(c43, hi, 0x04030402u);
    return __builtin_bit_cast(bf16x8, p);
}

template <typename ST, int GS>
__global__ __launch_bounds__(kQnmThreads) void qmm_n_m1_mfma(const QmmN1Args a) {
    typedef typename ST::storage SS;
    typedef int qn_v2i __attribute__((ext_vector_type(2)));
    constexpr int NT = kQnmThreads, NW = kQnmWaves, SPW = 8 / NW;  // threads, waves, slices per wave
    constexpr int C = kQnmCols, RC = kQnmRows, NG = C >= GS ? C / GS : 1;
    constexpr int E = (RC * NG + NT - 1) / NT;  // staged elements per thread and chunk
    static_assert(NG <= 4 && (NW == 4 || NW == 8), "group sizes 32, 64, 128; 4 or 8 waves");
    __shared__ __attribute__((aligned(16))) char wl[2][kQnmWBytes];
    __shared__ __attribute__((aligned(16))) char al[2][kQnmABytes];
    __shared__ float sums[2][NW][NG];  // [sum of hi + lo, sum of x b][wave][group]
    __shared__ float colv[C];
    __shared__ unsigned ticket;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int N = a.N, K = a.K, G = N / GS;
    // (tile, split) numbering as in qmm_n_m1 (the tiles of one run share an XCD)
    const int total = gridDim.x, lin = blockIdx.x, xcd = lin & 7;
    const int unit = xcd * (total >> 3) + min(xcd, total & 7) + (lin >> 3);
    const int tile = unit % a.ctiles, split = unit / a.ctiles;
    const int64_t b = a.b0 + blockIdx.z;
    const int kb = split * a.R, ke = min(K, kb + a.R);
    const int n0 = tile * C, g0 = n0 / GS;
    int64_t xbt, wbt;
    const bool ok = gather_batch(a.g, b, xbt, wbt);
    if (!ok) xbt = wbt = 0;
    const int rows = ok ? max(0, ke - kb) : 0;
    const int nch = (a.R + RC - 1) / RC;

    const uint32_t row_bytes = uint32_t(N) / 2u;
    const __amdgpu_buffer_rsrc_t wr = raw_rsrc(a.w + wbt * int64_t(K) * (N / 8), uint32_t(K) * row_bytes);
    const SS* sp = static_cast<const SS*>(a.s) + wbt * int64_t(K) * G;
    const SS* bp = a.b ? static_cast<const SS*>(a.b) + wbt * int64_t(K) * G : sp;
    const __amdgpu_buffer_rsrc_t xr = raw_rsrc(a.x + xbt * K, uint32_t(K) * 2u);
    const __amdgpu_buffer_rsrc_t sr = raw_rsrc(sp, uint32_t(K) * uint32_t(G) * uint32_t(sizeof(SS)));
    const __amdgpu_buffer_rsrc_t br = raw_rsrc(bp, a.b ? uint32_t(K) * uint32_t(G) * uint32_t(sizeof(SS)) : 0u);

    // Code copy: thread t moves 16 bytes (32 columns) of rows t / 4 + (NT / 4) j.
    constexpr int CPR = RC / (NT / 4);  // copies per thread and chunk
    const int cr = tid >> 2, cb = (tid & 3) * 16;
    const bool ccol = n0 + 2 * cb < N;
    auto load_codes = [&](qn_u32x4* v, int c) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < CPR; j++) {
            const int r = c * RC + cr + (NT / 4) * j;
            const uint32_t off = (ccol && r < rows) ? uint32_t(kb + r) * row_bytes + uint32_t(n0 / 2 + cb) : kOutOfRange;
            v[j] = __builtin_bit_cast(qn_u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0));
        }
    };
    auto store_codes = [&](const qn_u32x4* v, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < CPR; j++)
            *reinterpret_cast<qn_u32x4*>(&wl[buf][(cr + (NT / 4) * j) * kQnmWStride + cb]) = v[j];
    };
    // Staging: element e = tid + NT i is (row e / NG of the chunk, group e % NG).
    auto load_stage = [&](uint32_t* xv, uint32_t* sv, uint32_t* bv, int c) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < E; i++) {
            const int e = tid + NT * i;
            const int r = c * RC + e / NG, gi = e % NG;
            const bool live = e < RC * NG && r < rows && g0 + gi < G;
            const uint32_t xo = live ? uint32_t(kb + r) * 2u : kOutOfRange;
            const uint32_t po =
                live ? (uint32_t(kb + r) * uint32_t(G) + uint32_t(g0 + gi)) * uint32_t(sizeof(SS)) : kOutOfRange;
            xv[i] = __builtin_amdgcn_raw_buffer_load_b16(xr, xo, 0, 0);
            if constexpr (sizeof(SS) == 2) {
                sv[i] = __builtin_amdgcn_raw_buffer_load_b16(sr, po, 0, 0);
                bv[i] = __builtin_amdgcn_raw_buffer_load_b16(br, po, 0, 0);
            } else {
                sv[i] = __builtin_amdgcn_raw_buffer_load_b32(sr, po, 0, 0);
                bv[i] = __builtin_amdgcn_raw_buffer_load_b32(br, po, 0, 0);
            }
        }
    };
    float s_xs = 0.f, s_xb = 0.f;  // this thread's run sums for group tid % NG
    auto store_stage = [&](const uint32_t* xv, const uint32_t* sv, const uint32_t* bv, int buf)
                           __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < E; i++) {
            const int e = tid + NT * i;
            if (RC * NG % NT != 0 && e >= RC * NG) break;  // (the last round covers part of the threads)
            const int rr = e / NG, gi = e % NG;
            // dead elements read zero: every term below is zero for them
            const float x1 = bf16_bits_to_f32(xv[i]);
            const float xs = x1 * param_bits<ST>(sv[i]);
            const uint32_t hi = f32_to_bf16_bits(xs);
            const uint32_t lo = f32_to_bf16_bits(xs - bf16_bits_to_f32(hi));
            s_xs += bf16_bits_to_f32(hi) + bf16_bits_to_f32(lo);
            s_xb = fmaf(x1, param_bits<ST>(bv[i]), s_xb);
            const int j = rr & 7, slot = (j & 1) ? 4 + (j >> 1) : (j >> 1);
            uint16_t* dst = reinterpret_cast<uint16_t*>(al[buf]) + (gi * 2) * RC + (rr & ~7) + slot;
            dst[0] = uint16_t(hi);
            dst[RC] = uint16_t(lo);
        }
    };

    // Two chunks' loads are in flight while a chunk is computed: register sets
    // 0 and 1 take the even and odd chunks (the loop is unrolled by two so that
    // no set is ever copied).
    qn_u32x4 cv0[CPR], cv1[CPR];
    uint32_t xv0[E], sv0[E], bv0[E], xv1[E], sv1[E], bv1[E];
    load_stage(xv0, sv0, bv0, 0);  // (L2) first, so that the staging does not wait for the codes
    load_codes(cv0, 0);
    load_stage(xv1, sv1, bv1, 1);
    load_codes(cv1, 1);

    // A operand: lane row m = lane % 16 (0 = hi, 1 = lo, others zero), lane block g.
    const int g = lane >> 4, m = lane & 15;
    const int gi_w = (n0 + (C / NW) * wave) / GS - g0;  // this wave's group in the tile
    const uint32_t a_off = m < 2 ? uint32_t(((gi_w * 2 + m) * RC + 16 * g) * 2) : 0u;
    f32x4 acc[SPW];
#pragma unroll
    for (int s2 = 0; s2 < SPW; s2++) acc[s2] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int c, int buf) __attribute__((always_inline)) {
        const int crows = rows - c * RC;
#pragma unroll
        for (int rd = 0; rd < RC / 64; rd++) {
            if (64 * rd >= crows) break;  // (wave-uniform)
            const bf16x8 za = __builtin_bit_cast(bf16x8, qn_u32x4{0u, 0u, 0u, 0u});
            const bf16x8 aa = m < 2 ? *reinterpret_cast<const bf16x8*>(al[buf] + a_off + rd * 128) : za;
            const bf16x8 ab = m < 2 ? *reinterpret_cast<const bf16x8*>(al[buf] + a_off + rd * 128 + 16) : za;
#pragma unroll
            for (int s2 = 0; s2 < SPW; s2++) {
                const int sl = SPW * wave + s2;
                const qn_v2i v = __builtin_amdgcn_ds_read_tr4_b64_v2i32(
                    (__attribute__((address_space(3))) qn_v2i*)(&wl[buf][(64 * rd + 16 * g + m) * kQnmWStride + sl * 8]));
                acc[s2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aa, qnm_unpack(uint32_t(v.x)), acc[s2], 0, 0, 0);
                acc[s2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, qnm_unpack(uint32_t(v.y)), acc[s2], 0, 0, 0);
            }
        }
    };
    for (int c = 0; c < nch; c += 2) {
        store_stage(xv0, sv0, bv0, 0);
        store_codes(cv0, 0);
        lds_barrier();
        load_stage(xv0, sv0, bv0, c + 2);  // past the run: out of range, no traffic
        load_codes(cv0, c + 2);
        compute(c, 0);
        if (c + 1 >= nch) break;  // (uniform)
        store_stage(xv1, sv1, bv1, 1);
        store_codes(cv1, 1);
        lds_barrier();
        load_stage(xv1, sv1, bv1, c + 3);
        load_codes(cv1, c + 3);
        compute(c + 1, 1);
    }

    // Group sums of the run: lanes of one group are NG apart.
#pragma unroll
    for (int o = 32; o >= NG; o >>= 1) {
        s_xs += __shfl_xor(s_xs, o);
        s_xb += __shfl_xor(s_xb, o);
    }
    if (lane < NG) {
        sums[0][wave][lane] = s_xs;
        sums[1][wave][lane] = s_xb;
    }
    __syncthreads();
    if (lane < 16) {
        float sx = 0.f, sb = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) sx += sums[0][w][gi_w], sb += sums[1][w][gi_w];
        const float corr = fmaf(-128.f, sx, sb);
#pragma unroll
        for (int s2 = 0; s2 < SPW; s2++) colv[(SPW * wave + s2) * 16 + lane] = (acc[s2][0] + acc[s2][1]) + corr;
    }
    __syncthreads();
    const int n = n0 + tid;
    const float v = tid < C ? colv[tid] : 0.f;
    if (a.splits == 1) {
        if (tid < C && n < N) a.y[b * N + n] = uint16_t(f32_to_bf16_bits(v));
        return;
    }
    float* wsb = a.ws + b * int64_t(N);
    const int64_t sstride = a.batch_total * int64_t(N);
    if (!a.counters) {
        if (tid < C && n < N) wsb[split * sstride + n] = v;
        return;
    }
    if (tid < C && n < N) __hip_atomic_store(wsb + split * sstride + n, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!last_arriver(a.counters + blockIdx.z * a.ctiles + tile, unsigned(a.splits), &ticket)) return;
    if (tid < C && n < N) {
        float t = 0.f;
        int s0 = 0;
        for (; s0 + 8 <= a.splits; s0 += 8) {
            float r8[8];
#pragma unroll
            for (int i = 0; i < 8; i++)
                r8[i] = __hip_atomic_load(wsb + (s0 + i) * sstride + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int i = 0; i < 8; i++) t += r8[i];
        }
        for (; s0 < a.splits; s0++)
            t += __hip_atomic_load(wsb + s0 * sstride + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        a.y[b * N + n] = uint16_t(f32_to_bf16_bits(t));
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


// M = 1 through qmm_n_m1_mfma (4-bit codes) or qmm_n_m1 (8-bit); false,
// launching nothing, when neither takes the problem (rows not whole 16-byte
// words, a batch's codes of 2^31 bytes or more, or no workspace for the K
// split its row runs need).
bool launch_qmm_n_m1(int bits, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w,
                     const void* s, const void* b, const GatherIdx& g, int64_t batch, int N, int K, int gs,
                     const WsSource* src, hipStream_t st) {
    const int cpl = 128 / bits;
    if (N % cpl != 0 || !aligned(w, 16) || int64_t(N) * K * bits / 8 >= (int64_t(1) << 31) || N % gs != 0)
        return false;
    const bool mfma = bits == 4 && (gs == 32 || gs == 64 || gs == 128);
    const int C = mfma ? kQnmCols : 4 * cpl;
    const int ng = C >= gs ? C / gs : 1;
    const int ctiles = (N + C - 1) / C;
    const int64_t tiles = int64_t(ctiles) * batch;
    // K split: at most one workgroup per CU in all (tiles x splits), runs of
    // whole 64-row blocks, at most 128 runs per tile (the last workgroup of a
    // tile reads all of them); the VALU kernel stages at most kQmmN1Stage
    // (row, group) products.  Measured on MI355X at 4096 x 4096, 14336 x 4096
    // and 4096 x 14336: a second workgroup on some CUs (1.3 - 4 per CU) costs
    // more than the longer runs of one.
    int64_t sp = device_cu_count() / tiles;
    if (sp > 128) sp = 128;
    if (sp < 1) sp = 1;
    int R = int((K + sp - 1) / sp);
    R = (R + 63) / 64 * 64;
    if (!mfma && R > kQmmN1Stage / ng) R = kQmmN1Stage / ng;
    const int splits = (K + R - 1) / R;
    if (int64_t(ctiles) * splits > INT32_MAX) return false;
    QmmN1Args a{};
    a.y = y, a.x = x, a.w = w, a.s = s, a.b = b, a.g = g;
    a.N = N, a.K = K, a.gs = gs, a.R = R, a.splits = splits, a.ctiles = ctiles;
    a.batch_total = batch;
    int64_t per_launch = kMaxBatchesPerLaunch;
    if (splits > 1) {
        a.ws = static_cast<float*>(ws_acquire(src, size_t(splits) * size_t(batch) * size_t(N) * 4u, st));
        if (!a.ws) return false;
        a.counters = ws_counters(src, st);
        // one counter per (batch in the launch, column tile), in the lower half of the counter block
        if (a.counters) {
            const int64_t fit = (kWsCounters / 2) / ctiles;
            if (fit < 1) a.counters = nullptr;
            else if (fit < per_launch) per_launch = fit;
        }
    }
    auto go = [&](auto kernel, int threads) {
        for (int64_t b0 = 0; b0 < batch; b0 += per_launch) {
            const unsigned nb = unsigned(batch - b0 < per_launch ? batch - b0 : per_launch);
            a.b0 = b0;
            kernel<<<dim3(unsigned(ctiles * splits), 1, nb), dim3(threads), 0, st>>>(a);
        }
    };
    auto with_gs = [&](auto st_tag) {
        typedef decltype(st_tag) T;
        if (gs == 32) go(qmm_n_m1_mfma<T, 32>, kQnmThreads);
        else if (gs == 64) go(qmm_n_m1_mfma<T, 64>, kQnmThreads);
        else go(qmm_n_m1_mfma<T, 128>, kQnmThreads);
    };
    if (mfma) {
        if (scale_dtype == EQ_DTYPE_BF16) with_gs(BF16T{});
        else with_gs(F16T{});
    } else if (bits == 4) {
        if (scale_dtype == EQ_DTYPE_BF16) go(qmm_n_m1<4, BF16T>, 256);
        else go(qmm_n_m1<4, F16T>, 256);
    } else {
        if (scale_dtype == EQ_DTYPE_BF16) go(qmm_n_m1<8, BF16T>, 256);
        else go(qmm_n_m1<8, F16T>, 256);
    }
    if (splits > 1 && !a.counters) {
        const int64_t mn = batch * int64_t(N);
        qmm_n_finish<<<dim3(unsigned((mn * 8 + 255) / 256)), dim3(256), 0, st>>>(y, a.ws, mn, splits);
    }
    return true;
}

}  // namespace

bool launch_qmm_n_small(int bits, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s,
                        const void* b, const GatherIdx& g, int64_t batch, int M, int N, int K, int gs,
                        const WsSource* src, hipStream_t st) {
    if ((bits != 4 && bits != 8) ||
        (scale_dtype != EQ_DTYPE_BF16 && scale_dtype != EQ_DTYPE_F16 && scale_dtype != EQ_DTYPE_U8) || M < 1 ||
        M > 8 || batch < 1 || gs < 32 || (scale_dtype == EQ_DTYPE_U8 && (bits != 4 || gs != 32 || b)))
        return false;
    if (M == 1 && scale_dtype != EQ_DTYPE_U8 &&
        launch_qmm_n_m1(bits, scale_dtype, y, x, w, s, b, g, batch, N, K, gs, src, st))
        return true;
    const int64_t mn = batch * M * int64_t(N);
    int tl = 0, kp = 0, splits = 1, kchunk = K;
    int64_t tiles = 0;
    {
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
#define EQ_N_DISPATCH(BITS, ST) launch_n_bits<BITS, ST>(y, ws, x, w, s, b, g, batch, M, N, K, gs, splits, kchunk, tl, st)
    if (scale_dtype == EQ_DTYPE_U8) {
        EQ_N_DISPATCH(4, E8M0T);
    } else if (bits == 4) {
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

bool launch_qmm_n_rows(int bits, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s,
                       const void* b, int64_t M, int N, int K, int gs, const WsSource* src, hipStream_t st) {
    if (M < 1) return false;
    const int64_t full = M / 8, rest = M % 8;
    if (full > 0) {
        // the rows as `full` batches of 8 over one weight matrix
        const GatherIdx g{nullptr, nullptr, full, 1};
        if (!launch_qmm_n_small(bits, scale_dtype, y, x, w, s, b, g, full, 8, N, K, gs, src, st)) return false;
    }
    if (rest > 0) {
        const GatherIdx g{nullptr, nullptr, 1, 1};
        if (!launch_qmm_n_small(bits, scale_dtype, y + full * 8 * N, x + full * 8 * K, w, s, b, g, 1, int(rest), N, K,
                                gs, src, st))
            return false;
    }
    return true;
}

}  // namespace eq
