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
// with f32 accumulators.  Outputs with too few such tiles to fill the GPU
// without splitting K into short pieces take 64 x 128 tiles instead (wave w:
// columns [32w, 32w + 32), all 64 rows, 2 x 1 MFMA tiles; the planner,
// qmm_plan, chooses).
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
//  * MXFP4 (scale type E8M0T: group 32, E8M0 scale bytes, no biases): the
//    same tiles and pipeline; each lane's 32 codes become B operands through
//    v_cvt_scalef32_pk_bf16_fp4 with the group's scale folded in (exact).
#include <mutex>

#include "eq_common.hpp"

namespace eq {

typedef uint32_t q_u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBN = 256, kBK = 64;  // the default tile (rows, columns) and the K chunk
constexpr int kQmmThreads = 512;               // two K-groups of 4 waves
constexpr int kRing = 3;                       // slots of the load rings (codes in registers, activations in LDS)

typedef _Float16 q_f16x8 __attribute__((ext_vector_type(8)));

// Activation types of the prefill kernel: the 16-bit type both MFMA operands
// take (the dequantized weights are rounded to it), the MFMA and the output.
template <typename XT>
struct QmmAct;
template <>
struct QmmAct<BF16T> {
    __device__ static __forceinline__ uint32_t pack(float a, float b) { return pack_bf16x2(a, b); }
    __device__ static __forceinline__ f32x16 mfma(q_u32x4 wq, bf16x8 a, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, wq), a, c, 0, 0, 0);
    }
    __device__ static __forceinline__ uint16_t out(float v) { return uint16_t(f32_to_bf16_bits(v)); }
};
template <>
struct QmmAct<F16T> {
    // two f32 -> one word of f16 (a low), round to nearest even (v_cvt_pk_f16_f32)
    __device__ static __forceinline__ uint32_t pack(float a, float b) {
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
    }
    __device__ static __forceinline__ f32x16 mfma(q_u32x4 wq, bf16x8 a, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(q_f16x8, wq), __builtin_bit_cast(q_f16x8, a),
                                                      c, 0, 0, 0);
    }
    __device__ static __forceinline__ uint16_t out(float v) { return uint16_t(f32_to_f16_bits(v)); }
};

// 8 codes in k order -> 4 registers of 16-bit pairs (s*q + b) in XT.
template <int BITS, typename XT = BF16T>
__device__ __forceinline__ q_u32x4 dequant8(const uint32_t* words, float s, float b) {
    q_u32x4 r;
    if constexpr (BITS == 4) {
        const uint32_t w = words[0];
        uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;  // codes 2i | 2i+1 in byte i
        // (opaque to the optimiser, so that each code converts with one
        // v_cvt_f32_ubyte{0..3} instead of a bit-field extract plus a convert)
        asm volatile("" : "+v"(lo), "+v"(hi));
#pragma unroll
        for (int i = 0; i < 4; i++)
            r[i] = QmmAct<XT>::pack(fmaf(s, float((lo >> (8 * i)) & 0xffu), b),
                                    fmaf(s, float((hi >> (8 * i)) & 0xffu), b));
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t w = words[i >> 1];
            const int sh = (i & 1) * 16;
            r[i] = QmmAct<XT>::pack(fmaf(s, float((w >> sh) & 0xffu), b), fmaf(s, float((w >> (sh + 8)) & 0xffu), b));
        }
    }
    return r;
}

// One ring slot: this lane's codes (TN column blocks x 32 codes) and, unless
// the parameters come in windows, the scale and bias of each block.
template <int BITS, bool PARAMS, int TN = 2>
struct QmmSlot {
    static constexpr int WORDS = BITS;  // 32 codes * BITS / 32
    q_u32x4 w[TN][WORDS / 4];
    uint32_t s[TN], b[TN];
};
template <int BITS, int TN>
struct QmmSlot<BITS, false, TN> {
    static constexpr int WORDS = BITS;
    q_u32x4 w[TN][WORDS / 4];
};

// Reads every register of a slot in an empty asm statement (the never-taken
// side of an opaque_one() guard): every path then retires the slot's loads,
// which keeps the compiler's wait analysis exact at the join.
template <int BITS, bool PARAMS, int TN>
__device__ __forceinline__ void qmm_retire(const QmmSlot<BITS, PARAMS, TN>& s) {
#pragma unroll
    for (int j = 0; j < TN; j++) {
#pragma unroll
        for (int i = 0; i < QmmSlot<BITS, PARAMS, TN>::WORDS / 4; i++) asm volatile("" ::"v"(s.w[j][i]));
        if constexpr (PARAMS) asm volatile("" ::"v"(s.s[j]), "v"(s.b[j]));
    }
}

// s_waitcnt vmcnt(N), other counters untouched.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
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
    int M, N, K, ldy, mtiles, ntiles, splits, cps;  // cps: chunks per split; ldy: y row stride
    // Grouped (routed experts, no split K): row tile tm of the grid is entry
    // groups[tm] = {expert, first row, rows, row offset} of a device-built
    // list; x and y rows [first, first + rows) belong to the expert, whose
    // weights, scales and biases follow the previous expert's.  An expert
    // below zero marks an unused entry.  Null: one plain problem.
    const int4* groups;
};

// PW (parameter windows, group size 64 with an even number of groups per row
// and an even first chunk per split): instead of two 2-byte loads per column
// block and step, which touch one cache line per row each, the workgroup
// stages the scales and biases of 12 consecutive groups (6 steps of each
// K-group) of its 256 columns in LDS, each row's 24 bytes loaded by two lanes
// (every wave loads 32 rows of each), and every lane reads its column's word
// of a step from there.
//
// TM x TN: 32-row blocks and 32-column blocks of each wave's output block;
// the workgroup's tile is 32 TM rows x 128 TN columns (4 x 2: 128 x 256, the
// default; 2 x 1: 64 x 128, for outputs with too few large tiles to fill the
// GPU, which then need no split of K or fewer splits).
template <int BITS, int GS, typename ST, bool SPLIT, bool PW, typename XT = BF16T, int TM = 4, int TN = 2>
__global__ __launch_bounds__(kQmmThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void qmm_mfma_kernel(
    const QmmArgs args) {
    constexpr int BM = 32 * TM, BN = 128 * TN, LBUF = BM * kBK * 2;  // LBUF: bytes per K-group buffer
    static_assert((TM == 4 && TN == 2) || (TM == 2 && TN == 1) || (TM == 4 && TN == 1), "tile shapes");
    // Activation ring: three buffers per K-group.  Separate arrays, so that
    // the compiler's LDS alias scopes tell the buffers apart and a read of one
    // does not wait for the loads still landing in another.
    __shared__ __attribute__((aligned(16))) char abuf0[2 * LBUF], abuf1[2 * LBUF], abuf2[2 * LBUF];
    constexpr bool MX = __is_same(ST, E8M0T);
    constexpr uint32_t PB = MX ? 1u : 2u;  // bytes per scale / bias
    static_assert(!MX || (BITS == 4 && GS == 32 && !PW), "MXFP4: 4-bit codes, group 32");
    static_assert(!MX || std::is_same<XT, BF16T>::value, "MXFP4 prefill takes bf16 activations");
    const int N = args.N, K = args.K, G = K / GS;
    int M = args.M;

    // Tile and split of this workgroup: the workgroups of one XCD (id % 8)
    // take a contiguous run of row-major tiles, i.e. few row blocks of x.
    const int T = args.mtiles * args.ntiles * args.splits;
    int bid = blockIdx.x;
    if ((T & 7) == 0) bid = (bid & 7) * (T >> 3) + (bid >> 3);
    const int split = bid % args.splits, tile = bid / args.splits;
    const int tm = tile / args.ntiles, tn = tile % args.ntiles;
    int m0 = tm * BM;
    const int n0 = tn * BN;
    const uint16_t* xp = args.x;
    const uint32_t* wp = args.w;
    const char* sp = reinterpret_cast<const char*>(args.s);
    const char* bp = reinterpret_cast<const char*>(args.b);
    uint16_t* yp = args.y;
    if (args.groups) {
        const int4 gd = args.groups[tm];
        if (gd.x < 0) return;  // unused entry: the whole workgroup leaves before any barrier
        xp += int64_t(gd.y) * K;
        yp += int64_t(gd.y) * args.ldy;
        M = gd.z;
        m0 = gd.w;
        wp += int64_t(gd.x) * N * (K * BITS / 32);
        sp += int64_t(gd.x) * N * G * PB;
        if (bp) bp += int64_t(gd.x) * N * G * PB;
    }
    const int nchunks = K / kBK;
    const int c_begin = split * args.cps, c_end = min(nchunks, c_begin + args.cps);
    const int nloc = c_end - c_begin;  // >= 1 (the planner leaves no split empty)

    const int lane = threadIdx.x & 63;
    const int kgrp = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 8);  // K-group: chunks 2i + kgrp
    const int tid = threadIdx.x & 255;                                         // thread within the K-group
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);                 // column quarter
    const int l32 = lane & 31, kb = lane >> 5;
    const int gofs = kgrp * LBUF;  // this K-group's part of each ring buffer
    const int steps = (nloc + 1) / 2;  // chunks per K-group (the second may have one fewer)

    const __amdgpu_buffer_rsrc_t xr = raw_rsrc(xp, uint32_t(M) * uint32_t(K) * 2u);
    const uint32_t row_bytes = uint32_t(K) * BITS / 8u;  // (the launcher keeps N * row_bytes below 2^31)
    const __amdgpu_buffer_rsrc_t wr = raw_rsrc(wp, uint32_t(N) * row_bytes);
    const __amdgpu_buffer_rsrc_t sr = raw_rsrc(sp, uint32_t(N) * uint32_t(G) * PB);
    const __amdgpu_buffer_rsrc_t br = raw_rsrc(bp ? bp : sp, bp ? uint32_t(N) * uint32_t(G) * PB : 0u);
    // Parameter windows in LDS: [buffer][scale, bias][column * 6 + word], word
    // w of a column holding groups 2w (low half) and 2w + 1 of the window.
    __shared__ __attribute__((aligned(16))) uint32_t pbuf[2][2][BN * 6];

    // Lane offsets (chunk 0); rows past M and columns past N read zero.
    // Activations go straight from memory to LDS: load i of wave w fills the
    // 1 KiB (8 rows of 128 B) at (TM w + i) KiB of the BM x 64 tile, lane l
    // the 16 B at 16 l, i.e. row 8 (TM w + i) + l / 8, slot l % 8.  Slot p of
    // row r holds the row's 16-byte chunk p ^ ((r / 2) & 7), so the lane loads
    // chunk (l % 8) ^ ((row / 2) & 7).  (A 16-lane group of an A-operand read
    // takes rows r .. r + 15 at one chunk; 64 banks of 4 bytes span two rows,
    // so the rows of one parity must land in 8 different 16-byte bank groups.)
    uint32_t a_goff[4];  // (the first TM used; a bound of TM fails clang's host pass when a lambda captures it)
#pragma unroll
    for (int i = 0; i < TM; i++) {
        const int row = 8 * (TM * wave + i) + (lane >> 3), c = (lane & 7) ^ ((row >> 1) & 7);
        a_goff[i] = m0 + row < M ? (uint32_t(m0 + row) * uint32_t(K) + uint32_t(8 * c)) * 2u : kOutOfRange;
    }
    // Weight rows of this lane: columns n0 + 32 TN wave + 32 j + l32, codes from 32 kb.
    uint32_t woff[TN], soff[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const uint32_t n = uint32_t(n0 + 32 * TN * wave + 32 * j + l32);
        woff[j] = int(n) < N ? n * row_bytes + uint32_t(32 * kb) * BITS / 8u : kOutOfRange;
        // (not used with parameter windows, which have their own offsets)
        soff[j] = int(n) < N ? (n * uint32_t(G)) * PB + uint32_t((32 * kb) / GS) * PB : kOutOfRange;
    }
    // (a lane's 32 codes lie in one group when the group size is a multiple of
    // 32 -- chunks start at multiples of 64, so its group is k0 / GS + 32 kb /
    // GS -- and in groups 2 kb, 2 kb + 1 of the chunk at group size 16)

    // Loads of this K-group's chunk i, i.e. chunk 2i + kgrp of the split (past
    // the split's end: the last chunk again, in cache and never computed).
    auto chunk_k0 = [&](int i) __attribute__((always_inline)) {
        return (c_begin + min(2 * i + kgrp, nloc - 1)) * kBK;
    };
    auto load_a = [&](char* buf, int i) __attribute__((always_inline)) {
        const uint32_t ks = __builtin_amdgcn_readfirstlane(uint32_t(chunk_k0(i)) * 2u);
#pragma unroll
        for (int q = 0; q < TM; q++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xr, (__attribute__((address_space(3))) void*)(buf + gofs + (TM * wave + q) * 1024), 16,
                a_goff[q], ks, 0, 0);
    };
    typedef QmmSlot<BITS, !PW, TN> Slot;
    constexpr int NW = Slot::WORDS / 4;  // 16-byte code loads per column block
    auto load_b = [&](Slot& S, int i) __attribute__((always_inline)) {
        const int k0 = chunk_k0(i);
        const uint32_t kw = __builtin_amdgcn_readfirstlane(uint32_t(k0) * BITS / 8u);
        const uint32_t kp = __builtin_amdgcn_readfirstlane(uint32_t(k0 / GS) * PB);
#pragma unroll
        for (int j = 0; j < TN; j++) {
#pragma unroll
            for (int q = 0; q < NW; q++) S.w[j][q] = __builtin_amdgcn_raw_buffer_load_b128(wr, woff[j] + 16 * q, kw, 0);
            if constexpr (MX) {
                S.s[j] = __builtin_amdgcn_raw_buffer_load_b8(sr, soff[j], kp, 0);
                S.b[j] = 0u;
            } else if constexpr (GS == 16) {
                // the lane's 32 codes span two groups: both parameters in one word
                S.s[j] = __builtin_amdgcn_raw_buffer_load_b32(sr, soff[j], kp, 0);
                S.b[j] = __builtin_amdgcn_raw_buffer_load_b32(br, soff[j], kp, 0);
            } else if constexpr (!PW) {
                S.s[j] = __builtin_amdgcn_raw_buffer_load_b16(sr, soff[j], kp, 0);
                S.b[j] = __builtin_amdgcn_raw_buffer_load_b16(br, soff[j], kp, 0);
            }
        }
    };
    // Parameter window w (steps 6w .. 6w + 5, groups 12w .. 12w + 11 of the
    // split): wave v of the workgroup (v = 4 kgrp + wave < BN / 32) loads rows
    // 32 v .. 32 v + 31 of the tile, lane l the 12 bytes (6 groups) at half
    // l % 2 of row 32 v + l / 2, into registers (one step) and then into LDS.
    typedef uint32_t q_u32x3 __attribute__((ext_vector_type(3)));
    q_u32x3 pst[2];
    const int prow = 32 * (4 * kgrp + wave) + (lane >> 1);
    const bool pw_wave = 4 * kgrp + wave < BN / 32;  // (wave-uniform)
    const uint32_t poff = n0 + prow < N ? uint32_t(n0 + prow) * uint32_t(G) * PB + uint32_t(c_begin) * 2u +
                                              uint32_t(lane & 1) * 12u
                                        : kOutOfRange;
    auto load_pw = [&](int w) __attribute__((always_inline)) {
        if (!pw_wave) return;
        const uint32_t kq = __builtin_amdgcn_readfirstlane(uint32_t(12 * w) * 2u);
        pst[0] = __builtin_amdgcn_raw_buffer_load_b96(sr, poff, kq, 0);
        pst[1] = __builtin_amdgcn_raw_buffer_load_b96(br, poff, kq, 0);
    };
    auto store_pw = [&](int buf) __attribute__((always_inline)) {
        if (!pw_wave) return;
#pragma unroll
        for (int a = 0; a < 2; a++) {
            uint32_t* d = &pbuf[buf][a][prow * 6 + (lane & 1) * 3];
            d[0] = pst[a][0];
            d[1] = pst[a][1];
            d[2] = pst[a][2];
        }
    };
    // Before a barrier: this wave's activation loads for the next step have
    // landed (only the newest step's loads, codes then activations, may still
    // be in flight; memory operations complete in order).  (Per step: TN NW
    // code loads, 2 TN parameter loads -- TN for MXFP4, none with windows, whose
    // loads come first in their step and so land before its barrier -- and TM
    // activation loads.)
    auto wait_a = [&]() __attribute__((always_inline)) {
        constexpr int n = TN * NW + (MX ? TN : PW ? 0 : 2 * TN) + TM;
        wait_vmcnt<n>();
    };
    auto barrier = [&]() __attribute__((always_inline)) { asm volatile("s_barrier" ::: "memory"); };

    // A operand of this lane for step t and row block mi: row 32 mi + l32,
    // chunk 4 kb + t in slot (4 kb + t) ^ ((row / 2) & 7) (the same for every mi).
    uint32_t aoff[4];
#pragma unroll
    for (int t = 0; t < 4; t++) aoff[t] = uint32_t(l32 * (kBK * 2) + (((4 * kb + t) ^ ((l32 >> 1) & 7)) << 4));

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = f32x16{};

    // Codes of one chunk -> the B operands of its 4 MFMA steps (TN column blocks).
    auto dequant = [&](const Slot& S, const uint32_t* sbits, const uint32_t* bbits, q_u32x4 (&bq)[TN][4])
                       __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < TN; j++) {
            if constexpr (MX) {
                const float s = e8m0_to_f32(sbits[j]);
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    uint32_t p[4];
                    e2m1x8_to_bf16(S.w[j][0][t], s, p);
                    bq[j][t] = q_u32x4{p[0], p[1], p[2], p[3]};
                }
            } else {
                // (group 16: codes 0..15 of the lane's 32 take the low halves, 16..31 the high)
                const float s0 = qmm_param<ST>(sbits[j]), b0 = qmm_param<ST>(bbits[j]);
                const float s1 = GS == 16 ? qmm_param<ST>(sbits[j] >> 16) : s0;
                const float b1 = GS == 16 ? qmm_param<ST>(bbits[j] >> 16) : b0;
#pragma unroll
                for (int t = 0; t < 4; t++)
                    bq[j][t] = dequant8<BITS, XT>(reinterpret_cast<const uint32_t*>(&S.w[j][0]) + t * BITS / 4,
                                                  t < 2 ? s0 : s1, t < 2 ? b0 : b1);
            }
        }
    };
    // The chunk's 4 TM TN MFMAs (4 steps x TM row blocks x TN column blocks),
    // A operands from this K-group's part of the activation buffer.
    auto mma = [&](const q_u32x4 (&bq)[TN][4], const char* buf) __attribute__((always_inline)) {
        const char* base = buf + gofs;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            bf16x8 a[TM];
#pragma unroll
            for (int mi = 0; mi < TM; mi++)
                a[mi] = *reinterpret_cast<const bf16x8*>(base + aoff[t] + mi * 32 * (kBK * 2));
#pragma unroll
            for (int mi = 0; mi < TM; mi++)
#pragma unroll
                for (int j = 0; j < TN; j++) acc[mi][j] = QmmAct<XT>::mfma(bq[j][t], a[mi], acc[mi][j]);
        }
    };
    // Scale and bias words of this K-group's chunk at unrolled step r (0 ..
    // U; U is the next window's first step) of the current window.
    auto params = [&](const Slot& S, int r, int pw_cur, uint32_t* sb, uint32_t* bb) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < TN; j++) {
            if constexpr (PW) {
                const int col = 32 * TN * wave + 32 * j + l32;
                const int buf = r < 6 ? pw_cur : pw_cur ^ 1, w = r < 6 ? r : r - 6;
                sb[j] = pbuf[buf][0][col * 6 + w] >> (16 * kgrp);
                bb[j] = pbuf[buf][1][col * 6 + w] >> (16 * kgrp);
            } else {
                sb[j] = S.s[j];
                bb[j] = S.b[j];
            }
        }
    };

    // Prologue: the first parameter window, codes and activations of chunks
    // 0 and 1 requested; the window stored to LDS.
    Slot ring[kRing];
    if constexpr (PW) load_pw(0);
    load_b(ring[0], 0);
    load_a(abuf0, 0);
    load_b(ring[1], 1);
    load_a(abuf1, 1);
    if constexpr (PW) {
        store_pw(0);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the window's LDS stores are done
    }
    wait_a();
    barrier();

    // Step i: request chunk i + 2's codes and activations (into the buffer
    // every wave finished reading before the last barrier) and, with windows,
    // at i % 6 == 0 the next window (stored to the other LDS window at
    // i % 6 == 1, ahead of that step's barrier); then the two K-groups work
    // in opposite phase, so that on every SIMD one wave issues MFMAs while the
    // other dequantizes: the first (KG = 0) multiplies its chunk of step i
    // (dequantized in step i - 1) and then dequantizes its chunk of step
    // i + 1, the second dequantizes its chunk of step i and then multiplies
    // it.  Wait for chunk i + 1's activations, synchronise.  The schedule is
    // a constant of each copy of the loop, so each has its own register plan.
    // With 8-bit codes (twice the code registers) the second K-group lets
    // the compiler interleave its dequantization with its MFMAs (SCHED 2)
    // instead of keeping them apart.  4-bit codes at group sizes 16 and 32
    // with biases, whose per-step parameter loads sit in the ring, and 8-bit
    // codes without windows keep the in-step order for both K-groups (SCHED 2
    // for both; opposite phase measured 2-5 % slower there, against 4-16 %
    // faster for 4-bit group 64 with windows, group 128 and MXFP4, and up to
    // 8 % for 8-bit group 64 with windows).
    //   SCHED 0: multiply step i, then dequantize step i + 1 (anti-phase first K-group)
    //   SCHED 1: dequantize step i, then multiply it, kept apart (anti-phase second K-group)
    //   SCHED 2: dequantize step i and multiply it, interleaved by the compiler
    constexpr int U = PW ? 2 * kRing : kRing;
    constexpr bool kAnti = (BITS == 4 && (PW || GS == 128 || MX)) || (BITS == 8 && PW);
    constexpr int kSecond = BITS == 8 ? 2 : 1;  // the second K-group's schedule in opposite phase
    auto main_loop = [&](auto sched_c) __attribute__((always_inline)) {
        constexpr int SCHED = decltype(sched_c)::value;
        q_u32x4 bq[TN][4];  // dequantized B operands
        if constexpr (SCHED == 0) {
            uint32_t sb[TN], bb[TN];
            params(ring[0], 0, 0, sb, bb);
            dequant(ring[0], sb, bb, bq);
        }
        for (int i0 = 0;; i0 += U) {
            const int pw_cur = (i0 / U) & 1;  // this iteration's parameter window buffer
#pragma unroll
            for (int r = 0; r < U; r++) {
                const int i = i0 + r;
                if constexpr (PW)
                    if (r == 0) load_pw(i0 / U + 1);
                char* const bufs[3] = {abuf0, abuf1, abuf2};
                load_b(ring[(r + 2) % kRing], i + 2);
                load_a(bufs[(r + 2) % 3], i + 2);
                if constexpr (SCHED == 0) {
                    // (the first K-group has a chunk at every step)
                    mma(bq, bufs[r % 3]);
                    __builtin_amdgcn_sched_barrier(0);
                    if (opaque_one() && i + 1 < steps) {
                        uint32_t sb[TN], bb[TN];
                        params(ring[(r + 1) % kRing], r + 1, pw_cur, sb, bb);
                        dequant(ring[(r + 1) % kRing], sb, bb, bq);
                    } else {
                        qmm_retire(ring[(r + 1) % kRing]);
                    }
                } else {
                    if (opaque_one() && 2 * i + kgrp < nloc) {
                        uint32_t sb[TN], bb[TN];
                        params(ring[r % kRing], r, pw_cur, sb, bb);
                        dequant(ring[r % kRing], sb, bb, bq);
                        if constexpr (SCHED == 1) __builtin_amdgcn_sched_barrier(0);
                        mma(bq, bufs[r % 3]);
                    } else {
                        qmm_retire(ring[r % kRing]);
                    }
                }
                if (i + 1 >= steps) return;
                if constexpr (PW) {
                    if (r == 1) {
                        store_pw(pw_cur ^ 1);
                        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0) before the barrier
                    }
                }
                wait_a();
                barrier();
            }
        }
    };
    if constexpr (kAnti) {
        if (kgrp == 0) main_loop(std::integral_constant<int, 0>{});
        else main_loop(std::integral_constant<int, kSecond>{});
    } else {
        main_loop(std::integral_constant<int, 2>{});
    }
    // Every load has landed (the ring buffers are reused below).
    __builtin_amdgcn_s_waitcnt(0);
    // The second K-group's sums go to LDS, one row block (16 TN KiB, at most
    // a buffer's 2 LBUF bytes) at a time through alternating buffers, and the
    // first adds them.  Layout: [wave][j][q][lane] x 16 B, q = the run of 4
    // accumulator registers.
    static_assert(4 * TN * 4 * 64 * 16 <= 2 * LBUF, "a row block's sums fit one buffer");
    __syncthreads();
#pragma unroll
    for (int mi = 0; mi < TM; mi++) {
        f32x4* red = reinterpret_cast<f32x4*>(mi == 1 ? abuf1 : mi == 2 ? abuf2 : abuf0);
        if (kgrp == 1) {
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int q = 0; q < 4; q++)
                    red[((wave * TN + j) * 4 + q) * 64 + lane] =
                        f32x4{acc[mi][j][4 * q], acc[mi][j][4 * q + 1], acc[mi][j][4 * q + 2], acc[mi][j][4 * q + 3]};
        }
        __syncthreads();
        if (kgrp == 0) {
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const f32x4 v = red[((wave * TN + j) * 4 + q) * 64 + lane];
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[mi][j][4 * q + e] += v[e];
                }
        }
    }
    if (kgrp == 1) return;

    // The MFMA computed y^T blocks (weights as the first operand): register r
    // of lane l holds row m = 32 mi + l % 32 and column n = 32 j + 8 (r / 4) +
    // 4 (l / 32) + r % 4, so each run of 4 registers is 4 adjacent columns of
    // one row.  Columns past N are whole waves (N % 128 == 0).
    if (n0 + 32 * TN * wave >= N) return;
#pragma unroll
    for (int mi = 0; mi < TM; mi++) {
        const int m = m0 + 32 * mi + l32;
        if (m < M) {
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int n = n0 + 32 * TN * wave + 32 * j + 8 * q + 4 * kb;
                    const f32x4 v = {acc[mi][j][4 * q], acc[mi][j][4 * q + 1], acc[mi][j][4 * q + 2], acc[mi][j][4 * q + 3]};
                    if constexpr (SPLIT) {
                        *reinterpret_cast<f32x4*>(args.ws + (int64_t(split) * M + m) * N + n) = v;
                    } else {
                        const uint32_t lo = QmmAct<XT>::pack(v[0], v[1]), hi = QmmAct<XT>::pack(v[2], v[3]);
                        *reinterpret_cast<uint2*>(yp + int64_t(m) * args.ldy + n) = make_uint2(lo, hi);
                    }
                }
        }
    }
}

// y = bf16(sum over splits of the partial tiles), splits summed in order.
// y[m, n] (row stride ldy) = bf16(sum over splits of ws[split, m, n]), the
// partials dense [splits, M, N] f32; four outputs per thread (vec: y 8-byte
// aligned and N, ldy multiples of 4, so the four stay in one row).
template <typename XT = BF16T>
__global__ __launch_bounds__(256) void qmm_split_reduce(uint16_t* __restrict__ y, const float* __restrict__ ws,
                                                         int64_t mn, int64_t n, int64_t ldy, int splits, bool vec) {
    typedef float f32x4_t __attribute__((ext_vector_type(4)));
    const int64_t i = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
    if (i >= mn) return;
    if (vec && i + 4 <= mn) {
        f32x4_t v = *reinterpret_cast<const f32x4_t*>(ws + i);
        for (int s = 1; s < splits; s++) {
            const f32x4_t u = *reinterpret_cast<const f32x4_t*>(ws + int64_t(s) * mn + i);
            v = f32x4_t{v[0] + u[0], v[1] + u[1], v[2] + u[2], v[3] + u[3]};
        }
        const int64_t row = i / n, col = i - row * n;
        typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
        *reinterpret_cast<u16x4*>(y + row * ldy + col) =
            u16x4{QmmAct<XT>::out(v[0]), QmmAct<XT>::out(v[1]), QmmAct<XT>::out(v[2]), QmmAct<XT>::out(v[3])};
    } else {
        for (int64_t e = i; e < mn && e < i + 4; e++) {
            float v = ws[e];
            for (int s = 1; s < splits; s++) v += ws[int64_t(s) * mn + e];
            const int64_t row = e / n;
            y[row * ldy + (e - row * n)] = QmmAct<XT>::out(v);
        }
    }
}

// Compute units of the current device.
static int qmm_cu_count() {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) return 256;
    return v;
}

#ifndef EQ_QMM_SMALL_TILES
#define EQ_QMM_SMALL_TILES 1  // 0: 128 x 256 tiles only; 1: the planner's choice; 2: 64 x 128 whenever it may split
#endif

// Tile shape and split of K of one launch.  128 x 256 tiles when there are
// at least 3/4 as many as CUs, or when K split to fill the CUs still leaves
// each split 32 chunks or more; otherwise 64 x 128 tiles (four times as many,
// each dequantized code used by 64 rows instead of 128) when the large tiles
// would split K 8 ways or more, or at group size 64 (parameter windows,
// whose dequantization is the cheapest per code).  K is split so that the
// grid fills the CUs without exceeding them (a second round would double
// the time), at least 8 chunks per split (4 per K-group).  Measured: at
// M = 512, N = 4096, K = 4096, 4-bit group 64, the large tiles split K 4
// ways (f32 partials of 4 x M x N, a reduction pass, a short pipeline per
// workgroup) in 37.7 us, the small tiles need no split: 34.4 us; at group 16
// (the 2/3/5/6-bit re-packed codes included) the small tiles' per-code
// work made them 2-8 % slower there; at M = 128 (8-16 large-tile splits)
// and N = 1024 they are 1.2-1.5x faster.
#ifndef EQ_QMM_MID_TILES
#define EQ_QMM_MID_TILES 1  // 0: no 128 x 128 tiles
#endif
struct QmmPlan {
    bool small;  // 64 x 128 tiles
    bool mid;    // 128 x 128 tiles
    int mtiles, ntiles, splits;
};
static int qmm_splits(int tiles, int slots, int nchunks) {
    int s = slots / (tiles > 0 ? tiles : 1);
    s = s > nchunks / 8 ? nchunks / 8 : s;
    return s < 1 ? 1 : s;
}
static QmmPlan qmm_plan(int M, int N, int K, int gs, int bits, bool may_split) {
    QmmPlan p{};
    const int cu = qmm_cu_count(), nchunks = K / kBK;
    const int big = ((M + 127) / 128) * ((N + 255) / 256);
    const int big_splits = may_split ? qmm_splits(big, cu, nchunks) : 1;
    const bool big_ok = 4 * big >= 3 * cu || nchunks / big_splits >= 32;
    const bool small_ok = big_splits >= 8 || gs == 64;
    p.small = EQ_QMM_SMALL_TILES == 2 ? may_split : EQ_QMM_SMALL_TILES == 1 && !big_ok && small_ok;
    // 128 x 128 tiles (group size 64) in place of the small tiles, or of large
    // tiles that split K, when their own split leaves each piece at least 24
    // chunks, fills 3/4 of the CUs and writes f32 partials of at most twice
    // the weight bytes: every code then feeds 128 rows, as in the large tile,
    // with twice the large tile's workgroups.
    if (EQ_QMM_MID_TILES && EQ_QMM_SMALL_TILES == 1 && may_split && gs == 64 && (p.small || big_splits > 1)) {
        const int mid = ((M + 127) / 128) * ((N + 127) / 128);
        const int ms = qmm_splits(mid, cu, nchunks);
        const bool fills = 4 * mid * ms >= 3 * cu;
        const bool long_k = nchunks / ms >= 24;
        const bool partials_ok =
            ms == 1 || double(ms) * M * N * 4.0 <= 2.0 * double(N) * double(K) * bits / 8.0;
        if (fills && long_k && partials_ok && (p.small || ms < big_splits)) {
            p.small = false;
            p.mid = true;
        }
    }
    p.mtiles = p.small ? (M + 63) / 64 : (M + 127) / 128;
    p.ntiles = (p.small || p.mid) ? (N + 127) / 128 : (N + 255) / 256;
    p.splits = !may_split ? 1 : (p.small || p.mid) ? qmm_splits(p.mtiles * p.ntiles, cu, nchunks) : big_splits;
    return p;
}

// One launch (plus the split reduction): every buffer below 2^31 bytes.
template <int BITS, int GS, typename ST, typename XT = BF16T>
static bool launch_qmm_piece(uint16_t* y, int ldy, const uint16_t* x, const uint32_t* w, const void* s, const void* b,
                             int M, int N, int K, bool may_split, const WsSource* src, hipStream_t st) {
    QmmArgs a{};
    a.y = y, a.x = x, a.w = w, a.s = static_cast<const uint16_t*>(s), a.b = static_cast<const uint16_t*>(b);
    a.M = M, a.N = N, a.K = K, a.ldy = ldy;
    const QmmPlan plan = qmm_plan(M, N, K, GS, BITS, may_split);
    a.mtiles = plan.mtiles, a.ntiles = plan.ntiles;
    const int tiles = a.mtiles * a.ntiles, nchunks = K / kBK;
    int splits = plan.splits;
    if (splits > 1) {
        a.cps = (nchunks + splits - 1) / splits;
        a.cps += a.cps & 1;  // even, so that parameter windows stay 4-byte aligned
        splits = (nchunks + a.cps - 1) / a.cps;  // no empty split
        // a fixed scratch region may hold fewer splits than planned
        const size_t per_split = size_t(M) * size_t(N) * 4u;
        if (src && splits > 1 && size_t(splits) * per_split > src->cap) {
            const int fit = int(src->cap / per_split);
            if (fit >= 2) {
                a.cps = (nchunks + fit - 1) / fit;
                a.cps += a.cps & 1;
                splits = (nchunks + a.cps - 1) / a.cps;
            } else {
                splits = 1;
            }
        }
        if (splits > 1) {
            a.ws = static_cast<float*>(ws_acquire(src, size_t(splits) * per_split, st));
            if (!a.ws && !src) {
                // The library workspace cannot grow (the stream is capturing,
                // or the allocation failed).  Running unsplit would be a
                // different plan with a different summation order than the
                // same call made eagerly, so the call fails instead.
                set_error("quantized_matmul (qmm): the split-K plan needs " +
                          std::to_string(size_t(splits) * per_split) +
                          " bytes of workspace on this stream, which cannot grow while the stream is capturing "
                          "(make one call of this shape on the stream before capturing)");
                note_refusal();
                return false;
            }
            if (!a.ws) splits = 1;
        }
    }
    a.splits = splits;
    if (splits == 1) a.cps = nchunks;
    // parameter windows: group size 64, rows of an even number of groups
    const bool pw = GS == 64 && (K / GS) % 2 == 0 && a.cps % 2 == 0;
    const dim3 grid(unsigned(tiles * splits)), block(kQmmThreads);
    auto go = [&](auto tm, auto tn) {
        constexpr int TM = decltype(tm)::value, TN = decltype(tn)::value;
        if (splits == 1) {
            if (pw) qmm_mfma_kernel<BITS, GS, ST, false, GS == 64, XT, TM, TN><<<grid, block, 0, st>>>(a);
            else qmm_mfma_kernel<BITS, GS, ST, false, false, XT, TM, TN><<<grid, block, 0, st>>>(a);
        } else {
            if (pw) qmm_mfma_kernel<BITS, GS, ST, true, GS == 64, XT, TM, TN><<<grid, block, 0, st>>>(a);
            else qmm_mfma_kernel<BITS, GS, ST, true, false, XT, TM, TN><<<grid, block, 0, st>>>(a);
        }
    };
    if (plan.small) go(std::integral_constant<int, 2>{}, std::integral_constant<int, 1>{});
    else if (plan.mid) go(std::integral_constant<int, 4>{}, std::integral_constant<int, 1>{});
    else go(std::integral_constant<int, 4>{}, std::integral_constant<int, 2>{});
    if (splits == 1) return true;
    const int64_t mn = int64_t(M) * N;
    qmm_split_reduce<XT><<<dim3(unsigned((mn / 4 + 255) / 256 + 1)), dim3(256), 0, st>>>(
        y, a.ws, mn, N, ldy, splits, aligned(y, 8) && N % 4 == 0 && ldy % 4 == 0);
    return true;
}

// Buffer offsets in the kernel are 32-bit: a weight matrix of 2^31 bytes or
// more runs in row pieces (multiples of the 256-column tile), an activation
// matrix that large in row pieces (multiples of the 128-row tile).
// y's row stride is ldy (N when negative); split K only when y is one whole
// piece of stride N.
template <int BITS, int GS, typename ST, typename XT = BF16T>
static void launch_qmm_t(uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s, const void* b, int M,
                         int N, int K, const WsSource* src, hipStream_t st, int ldy = -1) {
    if (ldy < 0) ldy = N;
    const int64_t limit = (int64_t(1) << 31) - 1;
    const int64_t row_bytes = int64_t(K) * BITS / 8;
    const int64_t G = K / GS;
    int64_t n_piece = limit / row_bytes / kBN * kBN;
    int64_t m_piece = limit / (int64_t(K) * 2) / kBM * kBM;
    n_piece = n_piece < kBN ? kBN : n_piece;
    m_piece = m_piece < kBM ? kBM : m_piece;
    const bool whole = n_piece >= N && m_piece >= M;
    for (int64_t m0 = 0; m0 < M; m0 += m_piece) {
        const int mc = int(M - m0 < m_piece ? M - m0 : m_piece);
        for (int64_t n0 = 0; n0 < N; n0 += n_piece) {
            const int nc = int(N - n0 < n_piece ? N - n0 : n_piece);
            constexpr int64_t PB = __is_same(ST, E8M0T) ? 1 : 2;
            const char* sp = static_cast<const char*>(s) + n0 * G * PB;
            const char* bp = b ? static_cast<const char*>(b) + n0 * G * PB : nullptr;
            // (only a whole problem splits K, so a refusal comes before any launch)
            if (!launch_qmm_piece<BITS, GS, ST, XT>(y + m0 * ldy + n0, ldy, x + m0 * K, w + n0 * (row_bytes / 4), sp, bp,
                                                mc, nc, K, whole, src, st))
                return;
        }
    }
}

template <int BITS, typename ST, typename XT = BF16T>
static bool launch_qmm_gs(int gs, uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s, const void* b,
                          int M, int N, int K, const WsSource* src, hipStream_t st, int ldy = -1) {
    switch (gs) {
    case 16: launch_qmm_t<BITS, 16, ST, XT>(y, x, w, s, b, M, N, K, src, st, ldy); return true;
    case 32: launch_qmm_t<BITS, 32, ST, XT>(y, x, w, s, b, M, N, K, src, st, ldy); return true;
    case 64: launch_qmm_t<BITS, 64, ST, XT>(y, x, w, s, b, M, N, K, src, st, ldy); return true;
    case 128: launch_qmm_t<BITS, 128, ST, XT>(y, x, w, s, b, M, N, K, src, st, ldy); return true;
    default: return false;
    }
}

// ------------------------------------------------------- grouped (experts)

// First index i of a[0, n) with a[i] >= v (a sorted ascending; for unsorted
// input the result is still in [0, n]).
__device__ __forceinline__ int lower_bound_i32(const int32_t* __restrict__ a, int n, int v) {
    int lo = 0, hi = n;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (a[mid] < v) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// Sorted expert indices -> the grouped tile list: expert e owns rows
// [lower_bound(e), lower_bound(e + 1)) and takes ceil(rows / kBM) entries
// {e, first, rows, kBM t}.  One workgroup of 1024 threads, experts in passes
// of 1024 with a block scan of the entry counts; entries at or past `cap`
// are dropped and the list's remaining entries are marked unused.
__global__ __launch_bounds__(1024) void qmm_group_tiles(int4* __restrict__ out, const int32_t* __restrict__ rhs,
                                                        int batch, int experts, int cap) {
    __shared__ int scan[1024];
    __shared__ int carry;
    const int tid = threadIdx.x;
    if (tid == 0) carry = 0;
    __syncthreads();
    for (int e0 = 0; e0 < experts; e0 += 1024) {
        const int e = e0 + tid;
        int first = 0, rows = 0;
        if (e < experts) {
            first = lower_bound_i32(rhs, batch, e);
            const int end = lower_bound_i32(rhs, batch, e + 1);
            rows = end > first ? end - first : 0;
        }
        const int nt = (rows + kBM - 1) / kBM;
        scan[tid] = nt;
        __syncthreads();
        for (int o = 1; o < 1024; o <<= 1) {  // inclusive scan
            const int v = tid >= o ? scan[tid - o] : 0;
            __syncthreads();
            scan[tid] += v;
            __syncthreads();
        }
        const int base = carry + scan[tid] - nt;
        for (int t = 0; t < nt; t++)
            if (base + t < cap) out[base + t] = make_int4(e, first, rows, t * kBM);
        __syncthreads();
        if (tid == 1023) carry += scan[1023];
        __syncthreads();
    }
    for (int i = carry + tid; i < cap; i += 1024) out[i] = make_int4(-1, 0, 0, 0);
}

// xg[b] = x[lhs[b]] (K bf16 per row, 16-byte copies); an out-of-range index
// gives a zero row.  One workgroup per row.
__global__ __launch_bounds__(256) void qmm_gather_rows(uint16_t* __restrict__ xg, const uint16_t* __restrict__ x,
                                                       const int32_t* __restrict__ lhs, int64_t x_batches, int K) {
    const int64_t b = blockIdx.x;
    const int64_t src = lhs ? int64_t(lhs[b]) : (x_batches == 1 ? 0 : b);
    uint4* dst = reinterpret_cast<uint4*>(xg + b * K);
    const bool ok = src >= 0 && src < x_batches;
    const uint4* from = reinterpret_cast<const uint4*>(x + (ok ? src : 0) * K);
    for (int i = threadIdx.x; i < K / 8; i += 256) dst[i] = ok ? from[i] : make_uint4(0, 0, 0, 0);
}

// y = 0 (n bf16 values, n a multiple of 4, y 8-byte aligned).
__global__ __launch_bounds__(256) void qmm_zero(uint16_t* __restrict__ y, int64_t n) {
    for (int64_t i = (int64_t(blockIdx.x) * 256 + threadIdx.x) * 4; i < n; i += int64_t(gridDim.x) * 1024)
        *reinterpret_cast<uint2*>(y + i) = make_uint2(0, 0);
}

template <int BITS, int GS, typename ST>
static bool launch_qmm_grouped_t(uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s, const void* b,
                                 const int32_t* lhs, const int32_t* rhs, int batch, int64_t x_batches, int experts,
                                 int N, int K, hipStream_t st, const WsSource* src = nullptr) {
    const int cap = experts + (batch + kBM - 1) / kBM;  // sum over experts of ceil(rows / kBM)
    // one launch with 32-bit offsets: each expert's codes and the gathered rows below 2^31 bytes
    if (int64_t(N) * K * BITS / 8 >= (int64_t(1) << 31) || int64_t(batch) * K * 2 >= (int64_t(1) << 31)) return false;
    const size_t xg_bytes = (size_t(batch) * size_t(K) * 2u + 255u) & ~size_t(255);
    void* ws = ws_acquire(src, xg_bytes + size_t(cap) * sizeof(int4), st);
    if (!ws) return false;
    uint16_t* xg = reinterpret_cast<uint16_t*>(ws);
    int4* list = reinterpret_cast<int4*>(reinterpret_cast<char*>(ws) + xg_bytes);
    const int64_t yn = int64_t(batch) * N;
    qmm_zero<<<dim3(unsigned(yn / 1024 < 4096 ? yn / 1024 + 1 : 4096)), dim3(256), 0, st>>>(y, yn);
    qmm_gather_rows<<<dim3(unsigned(batch)), dim3(256), 0, st>>>(xg, x, lhs, x_batches, K);
    qmm_group_tiles<<<dim3(1), dim3(1024), 0, st>>>(list, rhs, batch, experts, cap);
    QmmArgs a{};
    a.y = y, a.x = xg, a.w = w, a.s = static_cast<const uint16_t*>(s), a.b = static_cast<const uint16_t*>(b);
    a.M = batch, a.N = N, a.K = K, a.ldy = N;
    a.mtiles = cap, a.ntiles = (N + kBN - 1) / kBN, a.splits = 1, a.cps = K / kBK;
    a.groups = list;
    const bool pw = GS == 64 && (K / GS) % 2 == 0 && a.cps % 2 == 0;
    const dim3 grid(unsigned(a.mtiles * a.ntiles)), block(kQmmThreads);
    if (pw) qmm_mfma_kernel<BITS, GS, ST, false, GS == 64, BF16T, 4, 2><<<grid, block, 0, st>>>(a);
    else qmm_mfma_kernel<BITS, GS, ST, false, false, BF16T, 4, 2><<<grid, block, 0, st>>>(a);
    return true;
}

template <int BITS, typename ST>
static bool launch_qmm_grouped_gs(int gs, uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s,
                                  const void* b, const int32_t* lhs, const int32_t* rhs, int batch,
                                  int64_t x_batches, int experts, int N, int K, const WsSource* src, hipStream_t st) {
    switch (gs) {
    case 16:
        return launch_qmm_grouped_t<BITS, 16, ST>(y, x, w, s, b, lhs, rhs, batch, x_batches, experts, N, K, st, src);
    case 32:
        return launch_qmm_grouped_t<BITS, 32, ST>(y, x, w, s, b, lhs, rhs, batch, x_batches, experts, N, K, st, src);
    case 64:
        return launch_qmm_grouped_t<BITS, 64, ST>(y, x, w, s, b, lhs, rhs, batch, x_batches, experts, N, K, st, src);
    case 128:
        return launch_qmm_grouped_t<BITS, 128, ST>(y, x, w, s, b, lhs, rhs, batch, x_batches, experts, N, K, st, src);
    default: return false;
    }
}

bool launch_qmm_grouped(int bits, int gs, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w,
                        const void* s, const void* b, const int32_t* lhs, const int32_t* rhs, int batch,
                        int64_t x_batches, int experts, int N, int K, hipStream_t st, const WsSource* src) {
    if (bits == 4) {
        if (scale_dtype == EQ_DTYPE_BF16)
            return launch_qmm_grouped_gs<4, BF16T>(gs, y, x, w, s, b, lhs, rhs, batch, x_batches, experts, N, K, src,
                                                   st);
        if (scale_dtype == EQ_DTYPE_F16)
            return launch_qmm_grouped_gs<4, F16T>(gs, y, x, w, s, b, lhs, rhs, batch, x_batches, experts, N, K, src,
                                                  st);
    } else if (bits == 8) {
        if (scale_dtype == EQ_DTYPE_BF16)
            return launch_qmm_grouped_gs<8, BF16T>(gs, y, x, w, s, b, lhs, rhs, batch, x_batches, experts, N, K, src,
                                                   st);
        if (scale_dtype == EQ_DTYPE_F16)
            return launch_qmm_grouped_gs<8, F16T>(gs, y, x, w, s, b, lhs, rhs, batch, x_batches, experts, N, K, src,
                                                  st);
    }
    return false;
}

bool launch_qmm_mfma_mxfp4(uint16_t* y, const uint16_t* x, const uint32_t* w, const uint8_t* s, int M, int N, int K,
                           const WsSource* ws, hipStream_t st) {
    launch_qmm_t<4, 32, E8M0T>(y, x, w, s, nullptr, M, N, K, ws, st);
    return true;
}

bool launch_qmm_grouped_mxfp4(uint16_t* y, const uint16_t* x, const uint32_t* w, const uint8_t* s,
                              const int32_t* lhs, const int32_t* rhs, int batch, int64_t x_batches, int experts, int N,
                              int K, hipStream_t st) {
    return launch_qmm_grouped_t<4, 32, E8M0T>(y, x, w, s, nullptr, lhs, rhs, batch, x_batches, experts, N, K, st);
}

// ------------------------------------------- prefill at 2, 3, 5 and 6 bits
//
// The codes of these widths are an LSB-first bit stream (a 32-code unit of a
// row is exactly BITS words).  For M > 16 they are re-packed, a slice of
// weight rows at a time, to one byte per code in the stream's workspace and
// multiplied by the 8-bit matrix-core kernel with the same scales and biases
// and group size: the code values, and so the products, are unchanged.

// One thread per 32-code unit: BITS words in, 8 words (32 byte codes) out.
template <int BITS>
__global__ __launch_bounds__(256) void qmm_codes_to_bytes(const uint32_t* __restrict__ w, uint4* __restrict__ out,
                                                          int64_t units) {
    const int64_t u = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (u >= units) return;
    uint32_t in[BITS];
#pragma unroll
    for (int i = 0; i < BITS; i++) in[i] = w[u * BITS + i];
    uint32_t o[8];
#pragma unroll
    for (int q = 0; q < 8; q++) {
        uint32_t v = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int bit = (4 * q + e) * BITS, wd = bit >> 5, sh = bit & 31;
            uint32_t c = in[wd] >> sh;
            if (sh + BITS > 32) c |= in[wd + 1] << (32 - sh);
            v |= (c & ((1u << BITS) - 1u)) << (8 * e);
        }
        o[q] = v;
    }
    out[2 * u] = make_uint4(o[0], o[1], o[2], o[3]);
    out[2 * u + 1] = make_uint4(o[4], o[5], o[6], o[7]);
}

template <typename ST, typename XT = BF16T>
static bool launch_qmm_odd_t(int bits, int gs, uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s,
                             const void* b, int M, int N, int K, const WsSource* src, hipStream_t st, int ldy = -1) {
    if (gs != 16 && gs != 32 && gs != 64 && gs != 128) return false;
    if (ldy < 0) ldy = N;
    // rows per slice: their byte codes within 64 MiB, a multiple of the 256-column tile
    int64_t nc = (int64_t(64) << 20) / K / kBN * kBN;
    nc = nc < kBN ? kBN : nc;
    nc = nc > N ? N : nc;
    const size_t code_bytes = (size_t(nc) * size_t(K) + 255) & ~size_t(255);
    // room after the codes for the split-K partials of a slice the planner would split
    const int splits = qmm_plan(M, int(nc), K, gs, 8, true).splits;
    const size_t part_bytes = splits > 1 ? size_t(splits) * size_t(M) * size_t(nc) * 4u : 0;
    size_t want = code_bytes + part_bytes;
    char* base = static_cast<char*>(ws_acquire(src, want, st));
    if (!base && !src) {
        // the library workspace cannot grow (capture): fail rather than run
        // another plan than the same call made eagerly
        set_error("quantized_matmul (qmm, " + std::to_string(bits) + "-bit): the plan needs " + std::to_string(want) +
                  " bytes of workspace on this stream, which cannot grow while the stream is capturing "
                  "(make one call of this shape on the stream before capturing)");
        note_refusal();
        return true;
    }
    if (!base) base = static_cast<char*>(ws_acquire(src, want = code_bytes, st));
    if (!base) return false;
    const size_t cap = src ? src->cap : want;
    WsSource rest{base + code_bytes, cap > code_bytes ? cap - code_bytes : 0, nullptr};
    const int64_t G = K / gs;
    constexpr int64_t PB = 2;
    for (int64_t n0 = 0; n0 < N; n0 += nc) {
        const int ncs = int(N - n0 < nc ? N - n0 : nc);
        const int64_t units = int64_t(ncs) * (K / 32);
        const dim3 grid(unsigned((units + 255) / 256));
        const uint32_t* wr = w + n0 * (int64_t(K) * bits / 32);
        uint4* codes = reinterpret_cast<uint4*>(base);
        switch (bits) {
        case 2: qmm_codes_to_bytes<2><<<grid, 256, 0, st>>>(wr, codes, units); break;
        case 3: qmm_codes_to_bytes<3><<<grid, 256, 0, st>>>(wr, codes, units); break;
        case 5: qmm_codes_to_bytes<5><<<grid, 256, 0, st>>>(wr, codes, units); break;
        default: qmm_codes_to_bytes<6><<<grid, 256, 0, st>>>(wr, codes, units); break;
        }
        const char* sp = static_cast<const char*>(s) + n0 * G * PB;
        const char* bp = b ? static_cast<const char*>(b) + n0 * G * PB : nullptr;
        const uint32_t* w8 = reinterpret_cast<const uint32_t*>(base);
        const WsSource* parts = rest.cap > 0 ? &rest : nullptr;
        if (!parts) {
            // no room for partials: a fixed region of exactly the codes, no split
            static const WsSource none{nullptr, 0, nullptr};
            parts = &none;
        }
        switch (gs) {
        case 16: launch_qmm_t<8, 16, ST, XT>(y + n0, x, w8, sp, bp, M, ncs, K, parts, st, ldy); break;
        case 32: launch_qmm_t<8, 32, ST, XT>(y + n0, x, w8, sp, bp, M, ncs, K, parts, st, ldy); break;
        case 64: launch_qmm_t<8, 64, ST, XT>(y + n0, x, w8, sp, bp, M, ncs, K, parts, st, ldy); break;
        default: launch_qmm_t<8, 128, ST, XT>(y + n0, x, w8, sp, bp, M, ncs, K, parts, st, ldy); break;
        }
    }
    return true;
}

bool launch_qmm_mfma(int bits, int gs, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w,
                     const void* s, const void* b, int M, int N, int K, const WsSource* ws, hipStream_t st,
                     int ldy, int x_dtype) {
    auto by_x = [&](auto stt) -> bool {
        typedef decltype(stt) ST;
        auto go = [&](auto xt) -> bool {
            typedef decltype(xt) XT;
            if (bits == 4) return launch_qmm_gs<4, ST, XT>(gs, y, x, w, s, b, M, N, K, ws, st, ldy);
            if (bits == 8) return launch_qmm_gs<8, ST, XT>(gs, y, x, w, s, b, M, N, K, ws, st, ldy);
            if (bits == 2 || bits == 3 || bits == 5 || bits == 6)
                return launch_qmm_odd_t<ST, XT>(bits, gs, y, x, w, s, b, M, N, K, ws, st, ldy);
            return false;
        };
        if (x_dtype == EQ_DTYPE_BF16) return go(BF16T{});
        if (x_dtype == EQ_DTYPE_F16) return go(F16T{});
        return false;
    };
    if (scale_dtype == EQ_DTYPE_BF16) return by_x(BF16T{});
    if (scale_dtype == EQ_DTYPE_F16) return by_x(F16T{});
    return false;
}

}  // namespace eq
