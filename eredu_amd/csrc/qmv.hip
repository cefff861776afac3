// Decode-shaped quantized matmul (small M, bf16 activations, transpose = true)
// on gfx950 matrix cores.
//
// y[m, n] = sum_g s[n,g] * sum_{k in g} x[m,k] q[n,k] + b[n,g] * sum_{k in g} x[m,k]
// (the affine contract of safemlx/src/ops/quantization.rs:190-226 with W = [N, K]).
//
// The weight stream is the whole cost, so the layout of the work is chosen for
// it.  A workgroup owns 16 output features (rows of W); its waves split K into
// "spans".  In one span every lane issues ONE 16-byte load of packed codes:
// lane l reads row n = l % 16 at byte offset 16 * (l / 16) of the span, so a
// wave load covers 64 contiguous bytes of each of 16 rows (128 codes per row
// at 4 bits, 64 at 8 bits).  The codes then feed v_mfma_f32_16x16x32_bf16
// directly in the lane layout they were loaded in: B[k][n] = codes of row n,
// with the k-slot block of lane l equal to l / 16.
//
// Per-group scales must be applied to per-group partial sums, but one MFMA
// sums 32 k-slots that straddle 2 or 4 quantization groups (when a span holds
// P = span / gs > 1 groups).  The A operand separates them at no cost: its 16
// rows are split into P blocks of 16/P rows, block p carrying the activations
// of the k-slots that belong to group p of the span and zeros elsewhere.  Row
// (p, m) of the MFMA result is then the group-p partial dot product of
// activation row m, and lanes of the result own exactly one group each.  This
// limits one launch to M <= 16/P activation rows; larger M is split into
// chunks by the launcher.
//
// 4-bit codes become bf16 (128 + q) with one byte permute and one and-or per
// pair; 8-bit codes go through v_cvt_f32_ubyte.  A second MFMA against an
// all-ones B gives sum_k x per group in the same layout, which carries both
// the bias term and the removal of the +128 offset:
//   acc += s * t + (b - 128 s) * xs         (f32, per span)
// Waves combine through LDS; the result is rounded once to bf16.
#include <algorithm>
#include <atomic>
#include <type_traits>
#include <vector>

#include "eq_common.hpp"

namespace eq {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Loop-invariant constants kept in VGPRs (opaque to the optimiser), so that
// (p & mask) | bias compiles to one v_and_or_b32: on gfx9 a VOP3 instruction
// takes no literal operands.  The code images depend on the activation type
// XT the MFMA multiplies in: bf16 0x43XX = 128 + XX (unit ulp for XX < 128),
// f16 0x64XX = 1024 + XX (unit ulp for XX < 1024).
struct UnpackConsts {
    uint32_t nib_mask;  // 0x000f000f
    uint32_t bf16_128;  // 0x43004300 (bf16) or 0x64006400 (f16): the offset's image in both halves
    uint32_t c43;       // 0x43434343 or 0x64646464 (uniform): its high byte in every byte
};
template <typename XT = BF16T>
__device__ __forceinline__ UnpackConsts make_unpack_consts() {
    UnpackConsts c;
    asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(c.nib_mask));
    if constexpr (std::is_same<XT, F16T>::value) {
        asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(c.bf16_128));
        asm volatile("s_mov_b32 %0, 0x64646464" : "=s"(c.c43));
    } else {
        asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(c.bf16_128));
        asm volatile("s_mov_b32 %0, 0x43434343" : "=s"(c.c43));
    }
    return c;
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Activation types of the decode kernels: the offset the 16-bit code images
// carry, the all-ones operand, the MFMA, and the output rounding.
template <typename XT>
struct QmvAct;
template <>
struct QmvAct<BF16T> {
    static constexpr uint32_t kOnes = 0x3f803f80u;  // bf16 1.0 pairs
    template <int BITS>
    static constexpr float offset() { return BITS == 4 ? 128.f : 0.f; }  // 8-bit codes convert exactly
    __device__ static __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    __device__ static __forceinline__ uint16_t out(float v) { return uint16_t(f32_to_bf16_bits(v)); }
};
template <>
struct QmvAct<F16T> {
    static constexpr uint32_t kOnes = 0x3c003c00u;  // f16 1.0 pairs
    template <int BITS>
    static constexpr float offset() { return 1024.f; }  // 1024 + q, both widths
    __device__ static __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    }
    __device__ static __forceinline__ uint16_t out(float v) { return uint16_t(f32_to_f16_bits(v)); }
};

// 8 consecutive 4-bit codes (one word, LSB first) -> 8 bf16 values 128 + q,
// in k order: pair i holds codes 2i (low half) and 2i+1 (high half).
// 9 VALU ops: one shift, four byte permutes, four and-or.
__device__ __forceinline__ bf16x8 unpack4_bf16_offset128(uint32_t w, const UnpackConsts& c) {
    const uint32_t t = w >> 4;
    u32x4 p;
    // byte 0 <- w.byte i (low nibble = code 2i), byte 2 <- t.byte i (low nibble = code 2i+1)
    p[0] = __builtin_amdgcn_perm(t, w, 0x0c040c00u);
    p[1] = __builtin_amdgcn_perm(t, w, 0x0c050c01u);
    p[2] = __builtin_amdgcn_perm(t, w, 0x0c060c02u);
    p[3] = __builtin_amdgcn_perm(t, w, 0x0c070c03u);
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = (p[i] & c.nib_mask) | c.bf16_128;
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

// 8 consecutive 8-bit codes (two words) -> 8 f16 values 1024 + q, exact, in k
// order: four byte permutes against the constant 0x64 bytes.
__device__ __forceinline__ bf16x8 unpack8_f16_offset1024(uint32_t w0, uint32_t w1, uint32_t c64) {
    u32x4 p;
    p[0] = __builtin_amdgcn_perm(c64, w0, 0x04010400u);  // [w0.b0, 64, w0.b1, 64]
    p[1] = __builtin_amdgcn_perm(c64, w0, 0x04030402u);
    p[2] = __builtin_amdgcn_perm(c64, w1, 0x04010400u);
    p[3] = __builtin_amdgcn_perm(c64, w1, 0x04030402u);
    return __builtin_bit_cast(bf16x8, p);
}

// 8 consecutive 4-bit codes -> 8 bf16 values 128 + q in the slot order
// (c0, c2, c4, c6, c1, c3, c5, c7): 7 VALU ops (two masks, a shift, four byte
// permutes against the constant 0x43 bytes).  The activations of the A
// operand must be permuted the same way (qmv_permute_x8).
__device__ __forceinline__ bf16x8 unpack4_bf16_offset128_perm(uint32_t w, uint32_t c43) {
    const uint32_t lo = w & 0x0f0f0f0fu;         // bytes: c0 c2 c4 c6
    const uint32_t hi = (w >> 4) & 0x0f0f0f0fu;  // bytes: c1 c3 c5 c7
    u32x4 p;
    p[0] = __builtin_amdgcn_perm(c43, lo, 0x04010400u);  // [lo.b0, 43, lo.b1, 43]
    p[1] = __builtin_amdgcn_perm(c43, lo, 0x04030402u);  // [lo.b2, 43, lo.b3, 43]
    p[2] = __builtin_amdgcn_perm(c43, hi, 0x04010400u);
    p[3] = __builtin_amdgcn_perm(c43, hi, 0x04030402u);
    return __builtin_bit_cast(bf16x8, p);
}

// 8 activations [x0 .. x7] (16 bytes) -> [x0, x2, x4, x6, x1, x3, x5, x7].
__device__ __forceinline__ u32x4 qmv_permute_x8(u32x4 v) {
    u32x4 o;
    o[0] = __builtin_amdgcn_perm(v[1], v[0], 0x05040100u);
    o[1] = __builtin_amdgcn_perm(v[3], v[2], 0x05040100u);
    o[2] = __builtin_amdgcn_perm(v[1], v[0], 0x07060302u);
    o[3] = __builtin_amdgcn_perm(v[3], v[2], 0x07060302u);
    return o;
}

#ifndef EQ_QMV_WAVES
#define EQ_QMV_WAVES 8
#endif
#ifndef EQ_QMV_UNROLL
#define EQ_QMV_UNROLL 4
#endif
#ifndef EQ_QMV_SPANS_PER_WAVE
#define EQ_QMV_SPANS_PER_WAVE 8
#endif
constexpr int kQmvMaxWaves = EQ_QMV_WAVES;            // waves per workgroup (upper bound)
constexpr int kQmvUnroll = EQ_QMV_UNROLL;             // spans per load block
constexpr int kQmvSpansPerWave = EQ_QMV_SPANS_PER_WAVE;  // target spans per wave

template <int BITS, int GS>
struct QmvGeom {
    static constexpr int CPL = 128 / BITS;                  // codes per lane per span (16 bytes)
    static constexpr int SPAN = 4 * CPL;                    // codes per row per span
    static constexpr int P = SPAN > GS ? SPAN / GS : 1;     // quantization groups per span
    static constexpr int MB = 16 / P;                       // A-operand rows per group block
    // Activation rows one pass of the LDS kernel takes: MB, or with four
    // groups per span (4-bit, group 32) two sets of MB rows, each set its own
    // MFMAs on the same unpacked codes.
    static constexpr int RPL = P == 4 ? 2 * MB : MB;
    static constexpr int STEPS = CPL / 8;                   // MFMAs per span
    static constexpr int SPAN_WORDS = SPAN * BITS / 32;     // = 16
};


// Raw 16-bit parameter bits -> f32 (bf16 or f16 scales/biases).
template <typename ST> __device__ __forceinline__ float param_bits_to_f32(uint32_t b);
template <> __device__ __forceinline__ float param_bits_to_f32<BF16T>(uint32_t b) { return bf16_bits_to_f32(b); }
template <> __device__ __forceinline__ float param_bits_to_f32<F16T>(uint32_t b) { return f16_bits_to_f32(b); }

// Per-lane state of one wave's walk over its spans (byte offsets into the
// buffers; span j adds j * the per-span stride).
struct QmvLane {
    __amdgpu_buffer_rsrc_t wr, xr, sr, br;
    uint32_t woff;    // codes: row n0 + l%16, 16-byte chunk l/16 of span 0
    uint32_t xoff;    // activations of this lane's A slots at span 0 (out of range for dead rows)
    uint32_t xstep;   // activation bytes per span (0 for dead rows)
    uint32_t soff;    // scales/biases of this lane's row
    int r_p;          // this lane's result group within a span
};

// Scale/bias words of one block: the NU * SPAN / GS consecutive groups of a
// row that the block's spans cover (at least one word).
template <int BITS, int GS, int NU>
struct QmvParamWords {
    static constexpr int GROUPS = (NU * QmvGeom<BITS, GS>::SPAN) / GS > 0 ? (NU * QmvGeom<BITS, GS>::SPAN) / GS : 1;
    static constexpr int WORDS = (GROUPS + 1) / 2;
};

// Registers of one block of NU spans.  With VEC the block's scales and biases
// arrive as one vector load each (row and block starts aligned to the load),
// otherwise as one 16-bit load per span.
template <int BITS, int GS, int NU, bool VEC>
struct QmvBlock {
    static constexpr bool VECP = VEC && NU > 1;
    static constexpr int PWORDS = VECP ? QmvParamWords<BITS, GS, NU>::WORDS : NU;
    bf16x8 xa[NU][QmvGeom<BITS, GS>::STEPS];
    u32x4 wd[NU];
    uint32_t sw[PWORDS], bw[PWORDS];
};

// Reads every register of a block in an empty asm statement, which makes the
// compiler wait for the block's loads.  A compute guarded by opaque_one()
// is followed by `else qmv_retire(block)`: the else path never runs, but
// without it the compiler's wait analysis sees a path on which the block's
// loads are still in flight after the guard, and the next load into those
// registers then waits for every outstanding load, prefetches included.
__device__ __forceinline__ void qmv_retire_reg(const u32x4& v) { asm volatile("" ::"v"(v)); }
__device__ __forceinline__ void qmv_retire_reg(const bf16x8& v) { asm volatile("" ::"v"(v)); }
__device__ __forceinline__ void qmv_retire_reg(uint32_t v) { asm volatile("" ::"v"(v)); }
template <int BITS, int GS, int NU, bool VEC>
__device__ __forceinline__ void qmv_retire(const QmvBlock<BITS, GS, NU, VEC>& b) {
#pragma unroll
    for (int u = 0; u < NU; u++) {
        qmv_retire_reg(b.wd[u]);
#pragma unroll
        for (int t = 0; t < QmvGeom<BITS, GS>::STEPS; t++) qmv_retire_reg(b.xa[u][t]);
    }
#pragma unroll
    for (int i = 0; i < QmvBlock<BITS, GS, NU, VEC>::PWORDS; i++) {
        qmv_retire_reg(b.sw[i]);
        qmv_retire_reg(b.bw[i]);
    }
}

// Loads `W` consecutive 32-bit words at byte offset `off` (16-, 8- or 4-byte loads).
template <int W>
__device__ __forceinline__ void load_words(uint32_t* d, __amdgpu_buffer_rsrc_t r, uint32_t off) {
    if constexpr (W >= 4) {
#pragma unroll
        for (int i = 0; i < W / 4; i++) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * i, 0, 0);
            d[4 * i] = v[0], d[4 * i + 1] = v[1], d[4 * i + 2] = v[2], d[4 * i + 3] = v[3];
        }
    } else if constexpr (W == 2) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
        d[0] = v[0], d[1] = v[1];
    } else {
        d[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    }
}

// Loads spans [j0, j0 + NU) (issue order scale/bias bits, activations, codes).
// When a group is longer than a span (8-bit codes, group 128) j0 must be even
// or NU == 1, so that group(j0 + u) = group(j0) + u * SPAN / GS.
template <int BITS, int GS, int NU, bool VEC>
__device__ __forceinline__ void qmv_load(QmvBlock<BITS, GS, NU, VEC>& b, const QmvLane& L, int j0) {
    typedef QmvGeom<BITS, GS> Geo;
    typedef QmvBlock<BITS, GS, NU, VEC> B;
    if constexpr (B::VECP) {
        // the block's groups of this lane's row (the lane's own group is picked later)
        const uint32_t so = L.soff + uint32_t((j0 * Geo::SPAN) / GS) * 2u;
        load_words<B::PWORDS>(b.sw, L.sr, so);
        load_words<B::PWORDS>(b.bw, L.br, so);
    } else {
        const uint32_t so = L.soff + (uint32_t((j0 * Geo::SPAN) / GS) + uint32_t(L.r_p)) * 2u;
#pragma unroll
        for (int u = 0; u < NU; u++) {
            b.sw[u] = __builtin_amdgcn_raw_buffer_load_b16(L.sr, so + (u * Geo::SPAN) / GS * 2, 0, 0);
            b.bw[u] = __builtin_amdgcn_raw_buffer_load_b16(L.br, so + (u * Geo::SPAN) / GS * 2, 0, 0);
        }
    }
    const uint32_t xo = L.xoff + uint32_t(j0) * L.xstep;
#pragma unroll
    for (int u = 0; u < NU; u++)
#pragma unroll
        for (int t = 0; t < Geo::STEPS; t++)
            b.xa[u][t] = __builtin_bit_cast(
                bf16x8, __builtin_amdgcn_raw_buffer_load_b128(L.xr, xo + u * Geo::SPAN * 2 + 16 * t, 0, 0));
    const uint32_t wo = L.woff + uint32_t(j0) * 64u;
#pragma unroll
    for (int u = 0; u < NU; u++) b.wd[u] = __builtin_amdgcn_raw_buffer_load_b128(L.wr, wo + u * 64, 0, 0);
}

// acc += s * (x . (128 + q)) + (b - 128 s) * sum(x) per span (4-bit); the 8-bit
// codes are exact, so acc += s * (x . q) + b * sum(x).
// Element e of a row of 16-bit parameters held in 32-bit words, as f32.
// Group element e = base + r_p of the 16-bit parameters held in 32-bit words,
// as f32, for a lane whose result group r_p lies in [0, P): base (a
// compile-time multiple of P) fixes the word up to the choice among P/2
// words, and r_p's low bit picks the half.
template <typename ST, int P>
__device__ __forceinline__ float pick_param(const uint32_t* words, int base, int r_p) {
    uint32_t w;
    if (P <= 1) {
        w = words[base >> 1];
        w = (base & 1) ? (w >> 16) : w;
        return param_bits_to_f32<ST>(w & 0xffffu);
    }
    w = words[base >> 1];
    if (P == 4) w = (r_p >> 1) ? words[(base >> 1) + 1] : w;
    if constexpr (std::is_same<ST, BF16T>::value)  // bf16 bits of the chosen half into an f32's top half
        return __uint_as_float(__builtin_amdgcn_perm(0u, w, (r_p & 1) ? 0x03020c0cu : 0x01000c0cu));
    else
        return param_bits_to_f32<ST>((w >> ((r_p & 1) * 16)) & 0xffffu);
}

// One span of one 16-row tile: the group-split MFMAs on the A operand xa
// (activations) and the codes wd, then acc += s * t + b' * xs with the span's
// scale s and bias b of this lane's result group:
// 4-bit: t = x . (128 + q), b' = b - 128 s; 8-bit: t = x . q, b' = b.
// With f16 activations (XT = F16T) the code images are f16 1024 + q for both
// widths and t = x . (1024 + q), b' = b - 1024 s.
template <int BITS, int GS, typename ST, int MREG, bool PERM = false, typename XT = BF16T>
__device__ __forceinline__ void qmv_span(f32x4& acc, const bf16x8* xa, const u32x4& wd, float sc, float bi,
                                         const UnpackConsts& uc, bf16x8 ones) {
    typedef QmvGeom<BITS, GS> Geo;
    typedef QmvAct<XT> A;
    f32x4 t4 = {0.f, 0.f, 0.f, 0.f};
    f32x4 xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < Geo::STEPS; t++) {
        bf16x8 bq;
        if (BITS == 4)
            bq = PERM ? unpack4_bf16_offset128_perm(wd[t], uc.c43) : unpack4_bf16_offset128(wd[t], uc);
        else if constexpr (std::is_same<XT, F16T>::value)
            bq = unpack8_f16_offset1024(wd[2 * t], wd[2 * t + 1], uc.c43);
        else
            bq = unpack8_bf16(wd[2 * t], wd[2 * t + 1]);
        t4 = A::mfma(xa[t], bq, t4);
        xs = A::mfma(xa[t], ones, xs);
    }
    constexpr float off = A::template offset<BITS>();
    const float beff = off != 0.f ? fmaf(-off, sc, bi) : bi;
#pragma unroll
    for (int r = 0; r < MREG; r++) acc[r] = fmaf(sc, t4[r], fmaf(beff, xs[r], acc[r]));
}

// qmv_span for two sets of four activation rows (group size 32, 4-bit codes,
// MREG 8): rows 0-3 through the A operand xa, rows 4-7 through xa2, on the
// same unpacked codes; acc holds rows 0-3 and acc2 rows 4-7.
template <int BITS, int GS, typename ST, bool PERM, typename XT>
__device__ __forceinline__ void qmv_span2(f32x4& acc, f32x4& acc2, const bf16x8* xa, const bf16x8* xa2,
                                          const u32x4& wd, float sc, float bi, const UnpackConsts& uc, bf16x8 ones) {
    typedef QmvGeom<BITS, GS> Geo;
    typedef QmvAct<XT> A;
    static_assert(BITS == 4 && Geo::P == 4, "two row sets: 4-bit codes, four groups per span");
    f32x4 t4 = {0.f, 0.f, 0.f, 0.f}, xs = {0.f, 0.f, 0.f, 0.f};
    f32x4 t4b = {0.f, 0.f, 0.f, 0.f}, xsb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < Geo::STEPS; t++) {
        const bf16x8 bq = PERM ? unpack4_bf16_offset128_perm(wd[t], uc.c43) : unpack4_bf16_offset128(wd[t], uc);
        t4 = A::mfma(xa[t], bq, t4);
        xs = A::mfma(xa[t], ones, xs);
        t4b = A::mfma(xa2[t], bq, t4b);
        xsb = A::mfma(xa2[t], ones, xsb);
    }
    constexpr float off = A::template offset<BITS>();
    const float beff = off != 0.f ? fmaf(-off, sc, bi) : bi;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        acc[r] = fmaf(sc, t4[r], fmaf(beff, xs[r], acc[r]));
        acc2[r] = fmaf(sc, t4b[r], fmaf(beff, xsb[r], acc2[r]));
    }
}

// Scale and bias of span u of a block for this lane's result group r_p.
template <int BITS, int GS, typename ST, int NU, bool VEC>
__device__ __forceinline__ void qmv_params(const uint32_t* sw, const uint32_t* bw, int u, int r_p, float bias_on,
                                           float& sc, float& bi) {
    typedef QmvGeom<BITS, GS> Geo;
    if constexpr (VEC && NU > 1) {
        // this lane's group, counted from the block's first: (u * SPAN) / GS + r_p
        sc = pick_param<ST, Geo::P>(sw, (u * Geo::SPAN) / GS, r_p);
        bi = pick_param<ST, Geo::P>(bw, (u * Geo::SPAN) / GS, r_p) * bias_on;
    } else {
        sc = param_bits_to_f32<ST>(sw[u] & 0xffffu);
        bi = param_bits_to_f32<ST>(bw[u] & 0xffffu) * bias_on;
    }
}

template <int BITS, int GS, typename ST, int MREG, int NU, bool VEC, typename XT = BF16T>
__device__ __forceinline__ void qmv_compute(f32x4& acc, const QmvBlock<BITS, GS, NU, VEC>& b, int r_p,
                                            float bias_on, const UnpackConsts& uc, bf16x8 ones) {
    // Loads issued before this block stay before it (no load may be sunk
    // across a memory clobber).
    asm volatile("" ::: "memory");
#pragma unroll
    for (int u = 0; u < NU; u++) {
        float sc, bi;
        qmv_params<BITS, GS, ST, NU, VEC>(b.sw, b.bw, u, r_p, bias_on, sc, bi);
        qmv_span<BITS, GS, ST, MREG, false, XT>(acc, b.xa[u], b.wd[u], sc, bi, uc, ones);
    }
}

// MREG: result registers that can hold a live activation row (1 when M == 1).
// Buffer sizes (M*K*2, N*K*bits/8, N*G*2 bytes) are below 2^31 (the launcher
// splits N otherwise).
//
// Occupancy target 2 waves per SIMD: the two register blocks of the
// double-buffered span pipeline must both stay live (the default target of
// higher occupancy makes the scheduler serialise the prefetch instead).
template <int BITS, int GS, typename ST, int MREG, bool VEC, typename XT>
__global__ __launch_bounds__(64 * kQmvMaxWaves) __attribute__((amdgpu_waves_per_eu(1, 2))) void qmv_mfma_kernel(
    uint16_t* __restrict__ y, const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases, int M, int N, int K, int ldy,
    int spans_per_wave) {
    typedef QmvGeom<BITS, GS> Geo;
    constexpr int CPL = Geo::CPL, SPAN = Geo::SPAN, P = Geo::P, MB = Geo::MB;
    constexpr int U = kQmvUnroll;
    static_assert(U % 2 == 0, "blocks must start at even spans");
    __shared__ float red[kQmvMaxWaves][16][16];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int nwaves = blockDim.x >> 6;
    const int ln = lane & 15;
    const int kq = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int G = K / GS;
    const int S_full = K / SPAN;               // spans wholly inside the row
    const int S = (K + SPAN - 1) / SPAN;       // including a ragged last span
    const int j_begin = wave * spans_per_wave;
    const int j_end = min(S, j_begin + spans_per_wave);
    const int j_full_end = min(S_full, j_end);
    const uint32_t row_bytes = uint32_t(K) * BITS / 8;

    // A operand: lane row ln is activation row ln % MB of group block ln / MB; it is
    // live when that block is the group of this lane's k-slots (block kq * P / 4).
    const int a_m = ln % MB;
    const bool a_live = (ln / MB) == (kq * P / 4) && a_m < M;
    // Result lanes: block kq holds result rows 4kq..4kq+3, all in group block kq * P / 4.
    const int r_p = kq * P / 4;

    QmvLane L;
    L.wr = raw_rsrc(w, uint32_t(N) * row_bytes);
    L.xr = raw_rsrc(x, uint32_t(M) * uint32_t(K) * 2u);
    L.sr = raw_rsrc(scales, uint32_t(N) * uint32_t(G) * 2u);
    L.br = biases ? raw_rsrc(biases, uint32_t(N) * uint32_t(G) * 2u) : L.sr;
    L.woff = uint32_t(n0 + ln) * row_bytes + uint32_t(kq) * 16u;
    L.xoff = a_live ? (uint32_t(a_m) * uint32_t(K) + uint32_t(kq * CPL)) * 2u : kOutOfRange;
    L.xstep = a_live ? SPAN * 2 : 0;
    L.soff = uint32_t(n0 + ln) * uint32_t(G) * 2u;
    L.r_p = r_p;
    const float bias_on = biases ? 1.f : 0.f;

    const UnpackConsts uc = make_unpack_consts<XT>();
    constexpr uint32_t k1 = QmvAct<XT>::kOnes;
    u32x4 ones_bits = {k1, k1, k1, k1};
    const bf16x8 ones = __builtin_bit_cast(bf16x8, ones_bits);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};

    // Full blocks, double-buffered: the loads of block i + 1 are in flight
    // while block i is computed.  Each compute sits in a basic block of its
    // own (opaque_one) so that the prefetch issued before it stays there.  The
    // loop body handles a pair of blocks; every prefetch is unconditional (past
    // the last block it re-reads the last block, which is still in L2).
    const int nblk = max(0, (j_full_end - j_begin) / U);
    if (nblk > 0) {
        QmvBlock<BITS, GS, U, VEC> ba, bb;
        qmv_load<BITS, GS, U, VEC>(ba, L, j_begin);
        for (int i = 0; i + 1 < nblk; i += 2) {
            qmv_load<BITS, GS, U, VEC>(bb, L, j_begin + (i + 1) * U);
            if (opaque_one()) qmv_compute<BITS, GS, ST, MREG, U, VEC, XT>(acc, ba, r_p, bias_on, uc, ones);
            else qmv_retire(ba);
            qmv_load<BITS, GS, U, VEC>(ba, L, j_begin + min(i + 2, nblk - 1) * U);
            if (opaque_one()) qmv_compute<BITS, GS, ST, MREG, U, VEC, XT>(acc, bb, r_p, bias_on, uc, ones);
            else qmv_retire(bb);
        }
        if (nblk & 1) qmv_compute<BITS, GS, ST, MREG, U, VEC, XT>(acc, ba, r_p, bias_on, uc, ones);  // block nblk - 1
    }
    // Remaining whole spans one at a time.
    for (int j = j_begin + nblk * U; j < j_full_end; j++) {
        QmvBlock<BITS, GS, 1, VEC> b1;
        qmv_load<BITS, GS, 1, VEC>(b1, L, j);
        qmv_compute<BITS, GS, ST, MREG, 1, VEC, XT>(acc, b1, r_p, bias_on, uc, ones);
    }
    // A ragged last span (K % SPAN != 0): chunks past the end of the row see
    // zero activations (their codes belong to the next row, or read as zero
    // past the buffer), and a group past the end has zero scale and bias.
    if (j_end > S_full && S_full >= j_begin) {
        const int j = S_full;
        const bool chunk_in = j * SPAN + kq * CPL < K;
        const bool g_in = j * SPAN + r_p * GS < K;
        QmvLane T = L;
        if (!chunk_in) T.xoff = kOutOfRange, T.xstep = 0;
        if (!g_in) T.soff = kOutOfRange;
        QmvBlock<BITS, GS, 1, VEC> b1;
        qmv_load<BITS, GS, 1, VEC>(b1, T, j);
        qmv_compute<BITS, GS, ST, MREG, 1, VEC, XT>(acc, b1, r_p, bias_on, uc, ones);
    }

    // Result lane (n = ln, block kq) register r is row 4kq + r = (group block, m) with
    // m = (4kq + r) % MB; fold the P group blocks (lane blocks 4/P apart) together.
#pragma unroll
    for (int r = 0; r < MREG; r++) {
        if (P >= 4) acc[r] += __shfl_xor(acc[r], 16);
        if (P >= 2) acc[r] += __shfl_xor(acc[r], 32);
    }
    if (r_p == 0) {
#pragma unroll
        for (int r = 0; r < MREG; r++) {
            const int m = 4 * kq + r;
            if (m < M) red[wave][m][ln] = acc[r];
        }
    }
    __syncthreads();
    for (int t = threadIdx.x; t < 16 * M; t += blockDim.x) {
        const int m = t >> 4, n = t & 15;
        float v = 0.f;
        for (int i = 0; i < nwaves; i++) v += red[i][m][n];
        y[int64_t(m) * ldy + n0 + n] = QmvAct<XT>::out(v);
    }
}

// ---------------------------------------------------------------------------
// Persistent variant with activations in LDS.
//
// The grid holds about one workgroup per CU.  A workgroup first copies the
// activations of every problem it serves into LDS, once, and then walks 16-row
// tiles (tile, tile + gridDim.x, ...), possibly of several independent
// problems (a grouped launch, e.g. the q/k/v projections of one token).  Its
// waves split each tile's K into spans exactly as above, but the A operands
// now come from LDS (ds_read, counted apart from the weight loads), so the
// register blocks of the weight pipeline hold only codes and scale words and
// the texture path carries almost nothing but the weight stream.  Per tile the
// waves combine their partial sums through a double-buffered LDS slot (fixed
// summation order, so results are reproducible).
//
// LDS layout (bytes): per staged activation matrix M rows of kpad bf16
// (kpad = K rounded up to 64, zero-filled past K), 16-byte chunk c of row m
// stored at chunk c ^ (m & 7) so that the rows of one A operand fall in
// different banks; then a zero block read by dead A rows; then the reduction
// slots.

constexpr int kQmvMaxProblems = 8;

struct QmvProblem {
    const uint16_t* x;
    const uint32_t* w;
    const uint16_t* s;
    const uint16_t* b;   // may be null
    uint16_t* y;
    int N, K, ldy;
    int spw;             // spans per wave
    int x_lds;           // LDS byte offset of its activations
    int kpad;            // activation row length in LDS (multiple of 64)
    float inv_cpr;       // 1 / (kpad / 8): row of a 16-byte LDS chunk by multiplication
};

// Field order: every workgroup starts by reading its arguments through the
// scalar cache, where one round of requests covers 8 lines of 64 bytes (a
// larger first round is split by the compiler into two dependent ones).  The
// header, the routed/prologue fields and problems 0-3 sit in the first 512
// bytes, which the kernel requests together at entry; problems 4-7 (launches
// of more than four problems) are read when used.
struct QmvBatch {
    int count;               // problems
    int M;                   // activation rows (all problems)
    int total_tiles;
    int nstage;              // distinct activation matrices to stage
    int tile0[kQmvMaxProblems];  // first global tile of each problem; INT_MAX past count
    int zero_lds, zero_bytes;
    int red_lds;             // 2 x waves x M x 16 floats
    // K phases (one problem, one tile per workgroup, activations too long for
    // LDS): LDS holds phase_spans spans of the rows at a time, phase p
    // covering spans [p * phase_spans, (p + 1) * phase_spans); 0 = no phases.
    int phase_spans;
    int stage[kQmvMaxProblems];  // problem whose x each staged matrix is
    // Activation prologue (M = 1, one staged input): 1 = silu(x) * pro_second,
    // 2 = RMSNorm(x + pro_second) * pro_weight, the sum also written to
    // pro_hidden_out by workgroup 0.  Applied while staging.
    const uint16_t* pro_second;
    const uint16_t* pro_weight;
    uint16_t* pro_hidden_out;
    float pro_eps;
    // Routed problems (gather_qmm's decode; kernels with GATHER): problem i
    // is output batch g_b0 + i, its x row and its expert's codes, scales and
    // biases at the bases in p[i] plus the batch's index (g_lhs / g_rhs; null:
    // the batch itself, or 0 when there is one batch) times g_x_stride
    // elements, g_w_stride words and g_s_stride parameters.  An index outside
    // its operand's batches gives a zero row.
    int g_b0;
    const int32_t* g_lhs;
    const int32_t* g_rhs;
    int64_t g_xb, g_wb, g_x_stride, g_w_stride, g_s_stride;
    QmvProblem p[kQmvMaxProblems];
};
constexpr int kQmvArgLines = 8;  // 64-byte lines requested at entry
static_assert(offsetof(QmvBatch, p) + 4 * sizeof(QmvProblem) <= 64 * kQmvArgLines,
              "the header and problems 0-3 fit the lines requested at entry");


// Routed problems: the x and expert indices of each problem of the launch,
// resolved once per workgroup from device memory into LDS (routes[2 pi] =
// x batch, routes[2 pi + 1] = expert; -1 for both when either index is out
// of range), so that the tiles' address computations read LDS.
template <bool GATHER>
__device__ __forceinline__ void qmv_load_routes(const QmvBatch& batch, int* routes) {
    if constexpr (GATHER) {
        const int pi = int(threadIdx.x);
        if (pi < batch.count) {
            const int64_t bb = int64_t(batch.g_b0) + pi;
            const int64_t xb = batch.g_lhs ? int64_t(batch.g_lhs[bb]) : (batch.g_xb == 1 ? 0 : bb);
            const int64_t wb = batch.g_rhs ? int64_t(batch.g_rhs[bb]) : (batch.g_wb == 1 ? 0 : bb);
            const bool live = xb >= 0 && xb < batch.g_xb && wb >= 0 && wb < batch.g_wb;
            routes[2 * pi] = live ? int(xb) : -1;
            routes[2 * pi + 1] = live ? int(wb) : -1;
        }
        __syncthreads();
    }
}

// The operands of problem pi: p[pi]'s pointers, offset by the route's
// indices with GATHER; live is false for a route whose index is out of
// range (its loads then read zero).
struct QmvPtrs {
    const uint16_t* x;
    const uint32_t* w;
    const uint16_t* s;
    const uint16_t* b;
    bool live;
};
template <bool GATHER>
__device__ __forceinline__ QmvPtrs qmv_ptrs(const QmvBatch& batch, int pi, const int* routes) {
    const QmvProblem& pr = batch.p[pi];
    QmvPtrs r{pr.x, pr.w, pr.s, pr.b, true};
    if constexpr (GATHER) {
        const int xb = __builtin_amdgcn_readfirstlane(routes[2 * pi]);
        const int wb = __builtin_amdgcn_readfirstlane(routes[2 * pi + 1]);
        r.live = xb >= 0;
        const int64_t xo = r.live ? xb : 0, wo = r.live ? wb : 0;
        r.x += xo * batch.g_x_stride;
        r.w += wo * batch.g_w_stride;
        r.s += wo * batch.g_s_stride;
        if (r.b) r.b += wo * batch.g_s_stride;
    }
    return r;
}

// Registers of one block of NU spans of the LDS variant: codes and scale words.
template <int BITS, int GS, int NU, bool VEC>
struct QmvWBlock {
    static constexpr int PWORDS = (VEC && NU > 1) ? QmvParamWords<BITS, GS, NU>::WORDS : NU;
    u32x4 wd[NU];
    uint32_t sw[PWORDS], bw[PWORDS];
};

template <int BITS, int GS, int NU, bool VEC>
__device__ __forceinline__ void qmv_retire(const QmvWBlock<BITS, GS, NU, VEC>& b) {
#pragma unroll
    for (int u = 0; u < NU; u++) qmv_retire_reg(b.wd[u]);
#pragma unroll
    for (int i = 0; i < QmvWBlock<BITS, GS, NU, VEC>::PWORDS; i++) {
        qmv_retire_reg(b.sw[i]);
        qmv_retire_reg(b.bw[i]);
    }
}

struct QmvTileLane {
    __amdgpu_buffer_rsrc_t wr, sr, br;
    uint32_t woff, soff;  // this lane's code chunk / scale row within the tile, at span 0
    int r_p;
};

template <int BITS, int GS, int NU, bool VEC>
__device__ __forceinline__ void qmv_wload(QmvWBlock<BITS, GS, NU, VEC>& b, const QmvTileLane& L, int j0) {
    typedef QmvGeom<BITS, GS> Geo;
    if constexpr (VEC && NU > 1) {
        const uint32_t so = L.soff + uint32_t((j0 * Geo::SPAN) / GS) * 2u;
        load_words<QmvWBlock<BITS, GS, NU, VEC>::PWORDS>(b.sw, L.sr, so);
        load_words<QmvWBlock<BITS, GS, NU, VEC>::PWORDS>(b.bw, L.br, so);
    } else {
        const uint32_t so = L.soff + (uint32_t((j0 * Geo::SPAN) / GS) + uint32_t(L.r_p)) * 2u;
#pragma unroll
        for (int u = 0; u < NU; u++) {
            b.sw[u] = __builtin_amdgcn_raw_buffer_load_b16(L.sr, so + (u * Geo::SPAN) / GS * 2, 0, 0);
            b.bw[u] = __builtin_amdgcn_raw_buffer_load_b16(L.br, so + (u * Geo::SPAN) / GS * 2, 0, 0);
        }
    }
    const uint32_t wo = L.woff + uint32_t(j0) * 64u;
#pragma unroll
    for (int u = 0; u < NU; u++) b.wd[u] = __builtin_amdgcn_raw_buffer_load_b128(L.wr, wo + u * 64, 0, 0);
}

// qmv_wload for the ring: the wave-uniform part of each offset (block j0)
// goes into the scalar offset operand, so that issuing a block takes no
// vector instruction.  A lane offset at kOutOfRange still reads zero.
template <int W>
__device__ __forceinline__ void load_words_s(uint32_t* d, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    if constexpr (W >= 4) {
#pragma unroll
        for (int i = 0; i < W / 4; i++) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16 * i, soff, 0);
            d[4 * i] = v[0], d[4 * i + 1] = v[1], d[4 * i + 2] = v[2], d[4 * i + 3] = v[3];
        }
    } else if constexpr (W == 2) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
        d[0] = v[0], d[1] = v[1];
    } else {
        d[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
    }
}

template <int BITS, int GS, int NU>
__device__ __forceinline__ void qmv_wload_ring(QmvWBlock<BITS, GS, NU, true>& b, const QmvTileLane& L, int j0) {
    typedef QmvGeom<BITS, GS> Geo;
    static_assert(NU > 1, "vector parameter loads");
    const uint32_t so = __builtin_amdgcn_readfirstlane(uint32_t((j0 * Geo::SPAN) / GS) * 2u);
    load_words_s<QmvWBlock<BITS, GS, NU, true>::PWORDS>(b.sw, L.sr, L.soff, so);
    load_words_s<QmvWBlock<BITS, GS, NU, true>::PWORDS>(b.bw, L.br, L.soff, so);
    const uint32_t wo = __builtin_amdgcn_readfirstlane(uint32_t(j0) * 64u);
#pragma unroll
    for (int u = 0; u < NU; u++) b.wd[u] = __builtin_amdgcn_raw_buffer_load_b128(L.wr, L.woff + u * 64, wo, 0);
}

// A operands of span j0 + u are read from LDS at xa_t + j0 * xstep + u * SPAN * 2
// (dead rows have xstep 0 and xa_t in the zero block, which covers NU spans).
// MREG 8: the second row set's A operands at xa_t2 + j0 * xstep2 (acc2).
// PERM4: the staged activations of 4-bit codes are permuted per 8-element
// chunk (qmv_permute_x8); false: in k order (codes unpacked in k order).
template <int BITS, int GS, typename ST, int MREG, int NU, bool VEC, typename XT = BF16T, bool PERM4 = true>
__device__ __forceinline__ void qmv_wcompute(f32x4& acc, const QmvWBlock<BITS, GS, NU, VEC>& b, const char* smem,
                                             const uint32_t* xa_t, uint32_t xstep, int j0, int r_p,
                                             float bias_on, const UnpackConsts& uc, bf16x8 ones,
                                             f32x4* acc2 = nullptr, const uint32_t* xa_t2 = nullptr,
                                             uint32_t xstep2 = 0) {
    typedef QmvGeom<BITS, GS> Geo;
    asm volatile("" ::: "memory");
    uint32_t xb[Geo::STEPS], xb2[MREG == 8 ? Geo::STEPS : 1];
#pragma unroll
    for (int t = 0; t < Geo::STEPS; t++) xb[t] = xa_t[t] + uint32_t(j0) * xstep;
    if constexpr (MREG == 8) {
#pragma unroll
        for (int t = 0; t < Geo::STEPS; t++) xb2[t] = xa_t2[t] + uint32_t(j0) * xstep2;
    }
#pragma unroll
    for (int u = 0; u < NU; u++) {
        bf16x8 xa[Geo::STEPS];
#pragma unroll
        for (int t = 0; t < Geo::STEPS; t++)
            xa[t] = *reinterpret_cast<const bf16x8*>(smem + xb[t] + u * Geo::SPAN * 2);
        float sc, bi;
        qmv_params<BITS, GS, ST, NU, VEC>(b.sw, b.bw, u, r_p, bias_on, sc, bi);
        if constexpr (MREG == 8) {
            bf16x8 xa2[Geo::STEPS];
#pragma unroll
            for (int t = 0; t < Geo::STEPS; t++)
                xa2[t] = *reinterpret_cast<const bf16x8*>(smem + xb2[t] + u * Geo::SPAN * 2);
            qmv_span2<BITS, GS, ST, BITS == 4 && PERM4, XT>(acc, *acc2, xa, xa2, b.wd[u], sc, bi, uc, ones);
        } else {
            qmv_span<BITS, GS, ST, MREG, BITS == 4 && PERM4, XT>(acc, xa, b.wd[u], sc, bi, uc, ones);
        }
    }
}

#ifndef EQ_QMV_LDS_WAVES
#define EQ_QMV_LDS_WAVES 4
#endif
#ifndef EQ_QMV_RING
#define EQ_QMV_RING 2
#endif
#ifndef EQ_QMV_WAVES_PER_CU
#define EQ_QMV_WAVES_PER_CU 8
#endif
constexpr int kQmvLdsMaxWaves = 8;              // waves per workgroup of the LDS variant, at most
constexpr int kQmvLdsWaves = EQ_QMV_LDS_WAVES;  // the planner's choice
// Span stride between a wave's consecutive blocks in a tile.  TAIL = false
// kernels (every K a whole number of blocks) interleave the waves' blocks
// along K -- wave w takes blocks w, w + NW, ... -- so that a workgroup's
// concurrent loads walk each row of its tile front to back together instead
// of four separate quarters of every row: fewer DRAM pages open at once
// (measured on the headline step: 3363 -> 3439 GB/s; gate/up 16.9 -> 16.2 us,
// down 9.7 -> 9.5 us per launch).  TAIL kernels give each wave one contiguous
// range (their ragged spans sit at the end of it).
template <bool TAIL>
constexpr int qmv_block_stride() { return !TAIL ? kQmvUnroll * kQmvLdsWaves : kQmvUnroll; }

// Register blocks in the load ring of the LDS variant: loads run RING - 1
// blocks ahead of the block being computed.  Measured on MI355X (decode
// shapes of an 8B model), two blocks and four waves per workgroup beat
// deeper rings and eight waves: more requests in flight per CU only queue.
// With 32-wide groups a block carries twice the scale words; rings deeper
// than three would not fit the 256 registers of two waves per SIMD.
template <int BITS, int GS>
struct QmvRing {
    static constexpr int D = (BITS == 4 && GS == 32 && EQ_QMV_RING > 3) ? 3 : EQ_QMV_RING;
};

// Per-wave view of one tile: span range, buffers, offsets, A-operand addresses.
template <int BITS, int GS>
struct QmvTileView {
    QmvTileLane L;
    int n0, j_begin, j_end, j_full_end, nblk, S_full, K;
    float bias_on;
    uint32_t xa_t[QmvGeom<BITS, GS>::STEPS];
    uint32_t xstep;
    // the second row set (rows MB .. 2 MB - 1 of the group blocks; MREG 8)
    uint32_t xa_t2[QmvGeom<BITS, GS>::STEPS];
    uint32_t xstep2;
};

// TAIL = false: every problem's K is a multiple of U * SPAN, so a wave's
// range is whole blocks; a wave without blocks in a tile gets one virtual
// block instead (loads out of range read zero, activations from the zero
// block), so that every tile takes at least one block from the ring.
template <int BITS, int GS, bool TAIL, bool GATHER = false>
__device__ __forceinline__ QmvTileView<BITS, GS> qmv_tile_view(const QmvBatch& batch, int pi, int tile, int wave,
                                                              int ln, int kq, int a_m, bool a_live, int r_p,
                                                              const int* routes = nullptr, bool a_live2 = false) {
    typedef QmvGeom<BITS, GS> Geo;
    const QmvProblem& pr = batch.p[pi];
    const QmvPtrs op = qmv_ptrs<GATHER>(batch, pi, routes);
    QmvTileView<BITS, GS> v;
    const int N = pr.N, K = pr.K, G = K / GS;
    v.K = K;
    v.n0 = (tile - batch.tile0[pi]) * 16;
    v.S_full = K / Geo::SPAN;
    const int S = (K + Geo::SPAN - 1) / Geo::SPAN;
    v.j_begin = qmv_block_stride<TAIL>() != kQmvUnroll ? wave * kQmvUnroll : wave * pr.spw;
    v.j_end = min(S, v.j_begin + pr.spw);
    v.j_full_end = min(v.S_full, v.j_end);
    v.nblk = max(0, (v.j_full_end - v.j_begin) / kQmvUnroll);
    if constexpr (qmv_block_stride<TAIL>() != kQmvUnroll) {
        // blocks wave, wave + NW, ... of the tile's v.S_full / U (whole K)
        const int nb = v.S_full / kQmvUnroll;
        v.nblk = nb > wave ? (nb - wave + kQmvLdsWaves - 1) / kQmvLdsWaves : 0;
        v.j_end = v.j_full_end = v.S_full;
    }
    const uint32_t row_bytes = uint32_t(K) * BITS / 8;
    const uint32_t live = op.live ? 1u : 0u;  // (a dead route's loads read zero)
    v.L.wr = raw_rsrc(op.w, live * uint32_t(N) * row_bytes);
    v.L.sr = raw_rsrc(op.s, live * uint32_t(N) * uint32_t(G) * 2u);
    v.L.br = op.b ? raw_rsrc(op.b, live * uint32_t(N) * uint32_t(G) * 2u) : v.L.sr;
    v.L.woff = uint32_t(v.n0 + ln) * row_bytes + uint32_t(kq) * 16u;
    v.L.soff = uint32_t(v.n0 + ln) * uint32_t(G) * 2u;
    v.L.r_p = r_p;
    v.bias_on = op.b ? 1.f : 0.f;
#pragma unroll
    for (int t = 0; t < Geo::STEPS; t++)
        v.xa_t[t] = a_live ? uint32_t(pr.x_lds + a_m * pr.kpad * 2 + (((kq * Geo::CPL / 8 + t) ^ (a_m & 7)) * 16))
                           : uint32_t(batch.zero_lds);
    v.xstep = a_live ? Geo::SPAN * 2 : 0;
    {
        const int a_m2 = a_m + Geo::MB;
#pragma unroll
        for (int t = 0; t < Geo::STEPS; t++)
            v.xa_t2[t] = a_live2
                             ? uint32_t(pr.x_lds + a_m2 * pr.kpad * 2 + (((kq * Geo::CPL / 8 + t) ^ (a_m2 & 7)) * 16))
                             : uint32_t(batch.zero_lds);
        v.xstep2 = a_live2 ? Geo::SPAN * 2 : 0;
    }
    if (!TAIL && v.nblk == 0) {
        v.nblk = 1;
        v.j_begin = v.j_end = v.j_full_end = 0;
        v.S_full = 1 << 20;  // no ragged span
        v.L.woff = v.L.soff = kOutOfRange;
#pragma unroll
        for (int t = 0; t < Geo::STEPS; t++) v.xa_t[t] = v.xa_t2[t] = uint32_t(batch.zero_lds);
        v.xstep = v.xstep2 = 0;
    }
    return v;
}

// Problem of global tile t: the number of later problems whose first tile
// is at or below t, counted without a loop (scalar compares and selects).
__device__ __forceinline__ int qmv_problem_of(const QmvBatch& batch, int t, int /*hint*/) {
    int pi = 0;
#pragma unroll
    for (int i = 1; i < kQmvMaxProblems; i++) pi += t >= batch.tile0[i] ? 1 : 0;
    return __builtin_amdgcn_readfirstlane(pi);
}

// The load side of a wave: the full blocks of its span range in each tile of
// its workgroup (tile, tile + gridDim.x, ...), one after the other.  Once the
// stream is exhausted its loads go out of range (they read zero and touch no
// memory), so that the ring keeps issuing loads without a data-dependent
// branch around them: a conditional load would make the compiler wait for
// every load before the join.
struct QmvStream {
    QmvTileLane L;
    int tile, pi, j, j_stop;
    bool done;
};

template <int BITS, int GS, bool TAIL, bool GATHER = false>
__device__ __forceinline__ void qmv_stream_seek(const QmvBatch& batch, QmvStream& st, int tile, int wave, int ln,
                                                int kq, int r_p, const int* routes = nullptr) {
    if constexpr (!TAIL) {
        // every tile has a block (real or virtual)
        if (tile < batch.total_tiles) {
            st.pi = qmv_problem_of(batch, tile, st.pi);
            const QmvTileView<BITS, GS> v = qmv_tile_view<BITS, GS, TAIL, GATHER>(batch, st.pi, tile, wave, ln, kq, 0, false, r_p, routes);
            st.L = v.L;
            st.tile = tile;
            st.j = v.j_begin;
            st.j_stop = v.j_begin + v.nblk * qmv_block_stride<TAIL>();
            return;
        }
        st.done = true;
        st.j = 0;
        st.L.woff = st.L.soff = kOutOfRange;
        return;
    }
    for (; tile < batch.total_tiles; tile += gridDim.x) {
        st.pi = qmv_problem_of(batch, tile, st.pi);
        const QmvTileView<BITS, GS> v = qmv_tile_view<BITS, GS, TAIL, GATHER>(batch, st.pi, tile, wave, ln, kq, 0, false, r_p, routes);
        if (v.nblk > 0) {
            st.L = v.L;
            st.tile = tile;
            st.j = v.j_begin;
            st.j_stop = v.j_begin + v.nblk * qmv_block_stride<TAIL>();
            return;
        }
    }
    st.done = true;
    st.j = 0;
    st.L.woff = st.L.soff = kOutOfRange;
}

template <int BITS, int GS, bool TAIL, bool GATHER = false>
__device__ __forceinline__ void qmv_stream_next(const QmvBatch& batch, QmvStream& st, int wave, int ln, int kq,
                                                int r_p, const int* routes = nullptr) {
    if (st.done) return;
    if (st.j + qmv_block_stride<TAIL>() < st.j_stop) {
        st.j += qmv_block_stride<TAIL>();
        return;
    }
    qmv_stream_seek<BITS, GS, TAIL, GATHER>(batch, st, st.tile + gridDim.x, wave, ln, kq, r_p, routes);
}

// silu(g) * u on 8 bf16 values with the decoder's roundings: sigmoid, the
// product with g and the product with u each rounded to bf16
// (eredu/src/backend/mlx/nn/layers.rs:21; Mlp::hidden,
// eredu-architectures/src/llama.rs:414-422).
__device__ __forceinline__ u32x4 qmv_silu_mul8(const u32x4 g, const u32x4 u) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t o = 0;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const float x = bf16_bits_to_f32((g[i] >> (16 * h)) & 0xffffu);
            const float up = bf16_bits_to_f32((u[i] >> (16 * h)) & 0xffffu);
            const float sg = silu_sigmoid_bf16(x);
            const float sl = float(static_cast<__bf16>(x * sg));
            o |= uint32_t(__builtin_bit_cast(uint16_t, static_cast<__bf16>(sl * up))) << (16 * h);
        }
        r[i] = o;
    }
    return r;
}

// qmv_silu_mul8 on one pair of bf16 values (bits), the result's bits.
__device__ __forceinline__ uint16_t qmv_silu_mul1(uint32_t g, uint32_t u) {
    const float x = bf16_bits_to_f32(g & 0xffffu);
    const float up = bf16_bits_to_f32(u & 0xffffu);
    const float sg = silu_sigmoid_bf16(x);
    const float sl = float(static_cast<__bf16>(x * sg));
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(sl * up));
}

// a + b on 8 bf16 values, each sum rounded to bf16 (the residual add).
__device__ __forceinline__ u32x4 qmv_add8(const u32x4 a, const u32x4 b) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float lo = bf16_bits_to_f32(a[i] & 0xffffu) + bf16_bits_to_f32(b[i] & 0xffffu);
        const float hi = bf16_bits_to_f32(a[i] >> 16) + bf16_bits_to_f32(b[i] >> 16);
        r[i] = f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
    }
    return r;
}

__device__ __forceinline__ float qmv_sumsq8(const u32x4 a) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float lo = bf16_bits_to_f32(a[i] & 0xffffu), hi = bf16_bits_to_f32(a[i] >> 16);
        ss = fmaf(lo, lo, ss);
        ss = fmaf(hi, hi, ss);
    }
    return ss;
}

// w * (a * inv) on 8 bf16 values, rounded to bf16 (RMSNorm's scaling).
__device__ __forceinline__ u32x4 qmv_norm8(const u32x4 a, const u32x4 w, float inv) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float lo = bf16_bits_to_f32(w[i] & 0xffffu) * (bf16_bits_to_f32(a[i] & 0xffffu) * inv);
        const float hi = bf16_bits_to_f32(w[i] >> 16) * (bf16_bits_to_f32(a[i] >> 16) * inv);
        r[i] = f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
    }
    return r;
}

// PRO: activation prologue (QmvBatch::pro_*), 0 none, 1 silu-mul, 2 RMSNorm.
// With PRO = 2 the staged row (K <= 2 * 16 * 64 * NW values) is one round of
// at most 2 chunks per thread, kept in registers across the workgroup's sum
// of squares.
// EPI: epilogue, 0 none, 1 SwiGLU: the (one) problem's matrix holds, in each
// 16-row tile t, gate rows 8t .. 8t + 7 then up rows 8t .. 8t + 7, and the
// tile writes y[8t + i] = silu(bf16(gate_i)) * bf16(up_i) with the roundings
// of qmv_silu_mul8 (M = 1).
// DIRECT (launches planned in K phases): each phase's activations go from
// memory straight to LDS (one buffer_load ... lds per KiB, every piece of
// the phase in flight at once, the XOR swizzle chosen through the source
// addresses), in k order, so 4-bit codes are unpacked in k order too.
template <int BITS, int GS, typename ST, int MREG, bool VEC, bool TAIL, int PRO = 0, typename XT = BF16T,
          int EPI = 0, bool GATHER = false, bool DIRECT = false>
__global__ __launch_bounds__(64 * kQmvLdsMaxWaves) __attribute__((amdgpu_waves_per_eu(1, 2))) void qmv_lds_kernel(
    const QmvBatch batch) {
    typedef QmvGeom<BITS, GS> Geo;
    constexpr int CPL = Geo::CPL, SPAN = Geo::SPAN, P = Geo::P, MB = Geo::MB, STEPS = Geo::STEPS;
    constexpr int U = kQmvUnroll;
    constexpr int D = QmvRing<BITS, GS>::D;
    static_assert(U % 2 == 0, "blocks must start at even spans");
    static_assert(D >= 2, "the ring needs two blocks");
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // The grid is launched with exactly kQmvLdsWaves waves per workgroup.
    constexpr int NW = kQmvLdsWaves;
    static_assert(NW >= 4, "the cross-wave sum assumes 16 * 16 <= 64 * NW threads");
    const int nwaves = NW;
    const int ln = lane & 15;
    const int kq = lane >> 4;
    const int M = batch.M;
    const int r_p = kq * P / 4;  // result group block of this lane
    prefetch_args<kQmvArgLines, offsetof(QmvBatch, total_tiles) / 4>(batch);
    if (int(blockIdx.x) >= batch.total_tiles) return;
    __shared__ int routes[GATHER ? 2 * kQmvMaxProblems : 1];
    qmv_load_routes<GATHER>(batch, routes);

    // Activation staging, one round: eight 16-byte chunks per thread are loaded
    // before any is written, so a round costs one trip to L2.  For 4-bit codes
    // each 8-element chunk is stored as [x0, x2, x4, x6, x1, x3, x5, x7], the
    // order in which unpack4_bf16_offset128_perm delivers the codes.
    const int zero_lds = __builtin_amdgcn_readfirstlane(batch.zero_lds);
    static_assert(PRO == 0 || MREG == 1, "activation prologues are for one activation row");
    static_assert(MREG != 8 || (Geo::RPL == 8 && !TAIL && VEC), "two row sets: group 32, whole blocks, vector parameters");
    static_assert(PRO == 0 || std::is_same<XT, BF16T>::value, "activation prologues are for bf16 rows");
    constexpr int NCH = PRO == 2 ? 2 : 8;  // chunks per thread and staging round
    u32x4 x2v[PRO != 0 ? NCH : 1];         // second input (up, residual); with PRO = 2 also the norm weight
    u32x4 nwv[PRO == 2 ? NCH : 1];
    auto stage_load = [&](int r, int c0, u32x4* v, int* dst, int k0 = 0) __attribute__((always_inline)) {
        const QmvProblem& pr = batch.p[batch.stage[r]];
        const QmvPtrs op = qmv_ptrs<GATHER>(batch, batch.stage[r], routes);
        const __amdgpu_buffer_rsrc_t xr = raw_rsrc(op.x, op.live ? uint32_t(M) * uint32_t(pr.K) * 2u : 0u);
        // (the prologue's inputs: with PRO = 2 a missing residual reads zero)
        const __amdgpu_buffer_rsrc_t x2r =
            raw_rsrc(PRO != 0 && batch.pro_second ? batch.pro_second : pr.x,
                     PRO != 0 && batch.pro_second ? uint32_t(pr.K) * 2u : 0u);
        const __amdgpu_buffer_rsrc_t nwr = raw_rsrc(PRO == 2 ? batch.pro_weight : pr.x, PRO == 2 ? uint32_t(pr.K) * 2u : 0u);
        const int K = pr.K, kpad = pr.kpad, x_lds = pr.x_lds;
        const float inv_cpr = pr.inv_cpr;
        const int cpr = kpad / 8;  // 16-byte chunks per LDS row
        const int total = M * cpr;
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            const int c = c0 + i * 64 * NW;
            // c / cpr exactly: c < 2^15 (the staged rows fit in LDS), so the
            // product's error (below 2^-19) is far from the distance, at least
            // 0.5 / cpr >= 2^-15, of (c + 0.5) / cpr to an integer
            const int m = MREG == 1 ? 0 : int((float(c) + 0.5f) * inv_cpr), cc = c - m * cpr;
            const bool live = c < total;
            const uint32_t off = (live & (k0 + cc * 8 < K))
                                     ? (uint32_t(m) * uint32_t(K) + uint32_t(k0 + cc * 8)) * 2u : kOutOfRange;
            v[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0);
            if constexpr (PRO != 0) x2v[i] = __builtin_amdgcn_raw_buffer_load_b128(x2r, off, 0, 0);
            if constexpr (PRO == 2) nwv[i] = __builtin_amdgcn_raw_buffer_load_b128(nwr, off, 0, 0);
            // chunks past the end read zero and land in the zero block
            dst[i] = live ? x_lds + m * kpad * 2 + ((cc ^ (m & 7)) * 16) : zero_lds;
        }
    };
    auto stage_store = [&](u32x4* v, const int* dst, int c0) __attribute__((always_inline)) {
        if constexpr (PRO == 1) {
#pragma unroll
            for (int i = 0; i < NCH; i++) v[i] = qmv_silu_mul8(v[i], x2v[i]);
        } else if constexpr (PRO == 2) {
            // hidden = x + residual (workgroup 0 writes it out), then the
            // workgroup's sum of squares, then w * (hidden * inv)
            float ss = 0.f;
            const int K0 = batch.p[batch.stage[0]].K;
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                v[i] = qmv_add8(v[i], x2v[i]);
                ss += qmv_sumsq8(v[i]);
                const int c = c0 + i * 64 * NW;
                if (blockIdx.x == 0 && batch.pro_hidden_out && c * 8 < K0)
                    *reinterpret_cast<u32x4*>(batch.pro_hidden_out + c * 8) = v[i];
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
            float* pred = reinterpret_cast<float*>(smem + batch.red_lds);
            if (lane == 0) pred[wave] = ss;
            __syncthreads();
            float tot = 0.f;
#pragma unroll
            for (int w = 0; w < NW; w++) tot += pred[w];
            const float inv = 1.0f / sqrtf(tot / float(K0) + batch.pro_eps);
#pragma unroll
            for (int i = 0; i < NCH; i++) v[i] = qmv_norm8(v[i], nwv[i], inv);
        }
#pragma unroll
        for (int i = 0; i < NCH; i++)
            *reinterpret_cast<u32x4*>(smem + dst[i]) = BITS == 4 ? qmv_permute_x8(v[i]) : v[i];
    };

    // The first staging round, then the first D - 1 weight blocks, are
    // requested before anything waits, so the L2 trip of the activations and
    // the HBM trip of the weights overlap.
    // Order of the first requests: the activations, then the weight blocks.
    // Loads complete in order, so the activations can be stored (and the
    // workgroup synchronised) while the weights are still on their way.
    static_assert(!DIRECT || (PRO == 0 && EPI == 0 && !GATHER && !TAIL && (MREG == 4 || MREG == 8)),
                  "direct staging: K-phase launches (one plain problem, whole blocks, up to 16 rows)");
    // DIRECT: slot sl of the phase buffer (row m = sl / cpr, slot p) holds
    // the 16-byte chunk p ^ (m & 7) of the phase, one wave load per 1 KiB;
    // the launcher takes this variant only when M * cpr is a multiple of 64
    // (phases of whole interleave strides make it so), so every piece lies
    // inside the activation region.
    auto stage_direct = [&](int k0) __attribute__((always_inline)) {
        const QmvProblem& pr = batch.p[0];
        const __amdgpu_buffer_rsrc_t xr = raw_rsrc(pr.x, uint32_t(M) * uint32_t(pr.K) * 2u);
        const int cpr = pr.kpad / 8, pieces = M * cpr / 64;
        const float inv_cpr = pr.inv_cpr;
        for (int pc = wave; pc < pieces; pc += NW) {
            const int sl = pc * 64 + lane;
            // sl / cpr exactly (sl < 2^15, as in stage_load)
            const int m = int((float(sl) + 0.5f) * inv_cpr), cc = (sl - m * cpr) ^ (m & 7);
            const uint32_t off =
                k0 + cc * 8 < pr.K ? (uint32_t(m) * uint32_t(pr.K) + uint32_t(k0 + cc * 8)) * 2u : kOutOfRange;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xr, (__attribute__((address_space(3))) void*)(smem + pr.x_lds + pc * 1024), 16, off, 0, 0, 0);
        }
    };
    u32x4 xv[NCH];
    int xdst[NCH];
    if constexpr (DIRECT) stage_direct(0);
    else stage_load(0, threadIdx.x, xv, xdst);
    QmvStream ls;
    ls.pi = qmv_problem_of(batch, blockIdx.x, 0);
    ls.L = qmv_tile_view<BITS, GS, TAIL, GATHER>(batch, ls.pi, blockIdx.x, wave, ln, kq, 0, false, r_p, routes).L;
    ls.tile = blockIdx.x;
    ls.j = ls.j_stop = 0;
    ls.done = false;
    qmv_stream_seek<BITS, GS, TAIL, GATHER>(batch, ls, blockIdx.x, wave, ln, kq, r_p, routes);
    typedef QmvWBlock<BITS, GS, U, VEC> RingBlock;
    RingBlock ring[D];
    auto ring_load = [&](RingBlock& b) __attribute__((always_inline)) {
        if constexpr (VEC) qmv_wload_ring<BITS, GS, U>(b, ls.L, ls.j);
        else qmv_wload<BITS, GS, U, VEC>(b, ls.L, ls.j);
    };
#pragma unroll
    for (int d = 0; d < D - 1; d++) {
        ring_load(ring[d]);
        qmv_stream_next<BITS, GS, TAIL, GATHER>(batch, ls, wave, ln, kq, r_p, routes);
    }
    if constexpr (!DIRECT) stage_store(xv, xdst, int(threadIdx.x));
    if constexpr (PRO != 2 && !DIRECT) {  // (the planner keeps a normalized row to one round)
        for (int r = 0; r < batch.nstage; r++) {
            const QmvProblem& pr = batch.p[batch.stage[r]];
            const int total = M * (pr.kpad / 8);
            for (int c0 = int(threadIdx.x) + (r == 0 ? NCH * 64 * NW : 0); c0 < total; c0 += NCH * 64 * NW) {
                stage_load(r, c0, xv, xdst);
                stage_store(xv, xdst, c0);
            }
        }
    }
    static_assert(U * SPAN * 2 + 64 <= 16 * 64 * NW, "one pass clears the zero block");
    if (int(threadIdx.x) < batch.zero_bytes / 16)
        *reinterpret_cast<u32x4*>(smem + zero_lds + threadIdx.x * 16) = u32x4{0u, 0u, 0u, 0u};
    if constexpr (DIRECT) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's pieces have landed
    __syncthreads();

    const UnpackConsts uc = make_unpack_consts<XT>();
    constexpr uint32_t k1 = QmvAct<XT>::kOnes;
    u32x4 ones_bits = {k1, k1, k1, k1};
    const bf16x8 ones = __builtin_bit_cast(bf16x8, ones_bits);
    // A operand row ln is activation row ln % MB of group block ln / MB; live when
    // that block is the group of this lane's k-slots (block kq * P / 4).
    const int a_m = ln % MB;
    const bool a_live = (ln / MB) == (kq * P / 4) && a_m < M;
    const bool a_live2 = MREG == 8 && (ln / MB) == (kq * P / 4) && a_m + MB < M;  // the second row set
    float* red = reinterpret_cast<float*>(smem + batch.red_lds);

    // The compute side walks the same tiles; per tile it takes its V.nblk
    // blocks from the ring, then the spans that do not fill a block.
    int tile = blockIdx.x;
    int pi = qmv_problem_of(batch, tile, 0);
    QmvTileView<BITS, GS> V = qmv_tile_view<BITS, GS, TAIL, GATHER>(batch, pi, tile, wave, ln, kq, a_m, a_live, r_p,
                                                                    routes, a_live2);
    int left = V.nblk, jc = V.j_begin, iter = 0;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    f32x4 acc2 = {0.f, 0.f, 0.f, 0.f};  // rows MB .. 2 MB - 1 (MREG 8)

    // Ends the current tile: leftover spans, the cross-wave sum, the store;
    // then moves to the next tile.  False when the workgroup has no more.
    auto finish = [&]() __attribute__((always_inline)) -> bool {
        if constexpr (TAIL) {
        for (int j = jc; j < V.j_full_end; j++) {
            QmvWBlock<BITS, GS, 1, VEC> b1;
            qmv_wload<BITS, GS, 1, VEC>(b1, V.L, j);
            qmv_wcompute<BITS, GS, ST, MREG, 1, VEC, XT>(acc, b1, smem, V.xa_t, V.xstep, j, r_p, V.bias_on, uc, ones);
        }
        // Ragged last span: chunks past K see the zero block, groups past K
        // have zero scale and bias.
        if (V.j_end > V.S_full && V.S_full >= V.j_begin) {
            const int j = V.S_full;
            const bool chunk_in = j * SPAN + kq * CPL < V.K;
            const bool g_in = j * SPAN + r_p * GS < V.K;
            QmvTileLane T = V.L;
            if (!g_in) T.soff = kOutOfRange;
            uint32_t xt[STEPS];
#pragma unroll
            for (int t = 0; t < STEPS; t++)
                xt[t] = chunk_in ? V.xa_t[t] : uint32_t(batch.zero_lds) - uint32_t(j) * V.xstep;
            QmvWBlock<BITS, GS, 1, VEC> b1;
            qmv_wload<BITS, GS, 1, VEC>(b1, T, j);
            qmv_wcompute<BITS, GS, ST, MREG, 1, VEC, XT>(acc, b1, smem, xt, V.xstep, j, r_p, V.bias_on, uc, ones);
        }
        }
        // Fold the P group blocks, then combine the waves through LDS (two
        // slots: a wave may fill the next tile's slot while this one is read).
        constexpr int R1 = MREG < 4 ? MREG : 4;  // registers of the first row set
#pragma unroll
        for (int r = 0; r < R1; r++) {
            if (P >= 4) acc[r] += __shfl_xor(acc[r], 16);
            if (P >= 2) acc[r] += __shfl_xor(acc[r], 32);
            if constexpr (MREG == 8) {
                acc2[r] += __shfl_xor(acc2[r], 16);
                acc2[r] += __shfl_xor(acc2[r], 32);
            }
        }
        float* slot = red + (iter & 1) * (nwaves * M * 16);
        if (r_p == 0) {
#pragma unroll
            for (int r = 0; r < R1; r++) {
                const int m = 4 * kq + r;
                if (m < M) slot[(wave * M + m) * 16 + ln] = acc[r];
                if constexpr (MREG == 8) {
                    if (m + MB < M) slot[(wave * M + m + MB) * 16 + ln] = acc2[r];
                }
            }
        }
        const int tile1 = tile + int(gridDim.x);
        const bool has1 = tile1 < batch.total_tiles;
        __syncthreads();
        // Straight-line on purpose (16 M <= 64 NW threads, NW unrolled): a loop
        // holding a global store makes the compiler wait for every load in
        // flight before entering it, prefetches included.
        if (int(threadIdx.x) < 16 * M) {
            const QmvProblem& pr = batch.p[pi];
            const int m = threadIdx.x >> 4, n = threadIdx.x & 15;
            float v = 0.f;
#pragma unroll
            for (int i = 0; i < NW; i++) v += slot[(i * M + m) * 16 + n];
            if constexpr (EPI == 1) {
                static_assert(MREG == 1 && std::is_same<XT, BF16T>::value, "SwiGLU epilogue: one bf16 row");
                // row n + 8 (the up row of gate row n), from the lane holding it
                const float u = __shfl(v, int(threadIdx.x) | 8);
                if (n < 8) pr.y[(V.n0 >> 1) + n] = qmv_silu_mul1(f32_to_bf16_bits(v), f32_to_bf16_bits(u));
            } else {
                pr.y[int64_t(m) * pr.ldy + V.n0 + n] = QmvAct<XT>::out(v);
            }
        }
        iter++;
        acc = f32x4{0.f, 0.f, 0.f, 0.f};
        acc2 = f32x4{0.f, 0.f, 0.f, 0.f};
        tile = tile1;
        if (!has1) return false;
        pi = qmv_problem_of(batch, tile, pi);
        V = qmv_tile_view<BITS, GS, TAIL, GATHER>(batch, pi, tile, wave, ln, kq, a_m, a_live, r_p, routes, a_live2);
        left = V.nblk;
        jc = V.j_begin;
        return true;
    };

    if constexpr (TAIL) {
        while (left == 0)
            if (!finish()) return;
    }
    // K phases (batch.phase_spans > 0; one problem, one tile per workgroup, no
    // tail): LDS holds the rows' spans [phase_base, phase_end).  Every wave has
    // the same number of blocks in each phase but the last, so all of them
    // reach each phase change, where the workgroup stages the next phase's
    // activations (the ring's weight loads stay in flight across it).
    int phase_base = 0, phase_end = batch.phase_spans > 0 ? batch.phase_spans : 0x7fffffff;
    auto restage = [&]() __attribute__((always_inline)) {
        __syncthreads();  // every wave is done with the previous phase's activations
        if constexpr (DIRECT) {
            stage_direct(phase_end * SPAN);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        } else {
            const int total = M * (batch.p[0].kpad / 8);
            for (int c0 = int(threadIdx.x); c0 < total; c0 += NCH * 64 * NW) {
                stage_load(0, c0, xv, xdst, phase_end * SPAN);
                stage_store(xv, xdst, c0);
            }
        }
        __syncthreads();
        phase_base = phase_end;
        phase_end += batch.phase_spans;
    };
    for (;;) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            ring_load(ring[(d + D - 1) % D]);
            qmv_stream_next<BITS, GS, TAIL, GATHER>(batch, ls, wave, ln, kq, r_p, routes);
            if constexpr (!TAIL && PRO == 0) {
                if (jc >= phase_end) restage();
            }
            if (opaque_one()) {
                qmv_wcompute<BITS, GS, ST, MREG, U, VEC, XT, !DIRECT>(acc, ring[d], smem, V.xa_t, V.xstep,
                                                                    jc - phase_base, r_p, V.bias_on, uc, ones, &acc2,
                                                                    V.xa_t2, V.xstep2);
            } else {
                qmv_retire(ring[d]);
            }
            jc += qmv_block_stride<TAIL>();
            if (--left == 0) {
                if constexpr (TAIL) {
                    do {
                        if (!finish()) return;
                    } while (left == 0);
                } else {
                    if (!finish()) return;  // every tile has a block
                }
            }
        }
    }
}

template <int BITS, int GS, typename ST, bool VEC, typename XT>
static void launch_qmv_v(uint16_t* y, const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                         int M, int N, int K, int ldy, int spw, int waves, hipStream_t st) {
    typedef QmvGeom<BITS, GS> Geo;
    const dim3 grid(unsigned(N / 16)), block(unsigned(64 * waves));
    // One launch takes at most MB activation rows; larger M runs in row chunks
    // (each chunk reads the weights again).
    for (int m0 = 0; m0 < M; m0 += Geo::MB) {
        const int mc = M - m0 < Geo::MB ? M - m0 : Geo::MB;
        uint16_t* yc = y + int64_t(m0) * ldy;
        const uint16_t* xc = x + int64_t(m0) * K;
        if (mc == 1)
            qmv_mfma_kernel<BITS, GS, ST, 1, VEC, XT><<<grid, block, 0, st>>>(yc, xc, w, s, b, mc, N, K, ldy, spw);
        else
            qmv_mfma_kernel<BITS, GS, ST, 4, VEC, XT><<<grid, block, 0, st>>>(yc, xc, w, s, b, mc, N, K, ldy, spw);
    }
}

// LDS available to one workgroup on the current device (cached per device).
static int device_lds_bytes() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 65536;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v <= 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
            v = 65536;
        cache[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

#ifndef EQ_QMV_DIRECT_PHASES
#define EQ_QMV_DIRECT_PHASES 1  // 0: K-phase launches stage through registers
#endif

// Launch plan of the persistent LDS variant.
struct QmvLdsPlan {
    QmvBatch B;
    int lds, grid, waves;
    bool vec;
    bool tail;  // some K is not a multiple of a block (U spans)
};

// Plans the persistent LDS variant for `count` problems sharing bits, group
// size, scale type and M (<= MB).  Returns false when the problems do not fit
// it (too many, LDS too small, buffers of 2^31 bytes or more, N % 16 != 0).
template <int BITS, int GS, typename ST>
static bool plan_qmv_lds(const QmvSpec* specs, int count, int M, QmvLdsPlan& plan, bool share_x = true) {
    typedef QmvGeom<BITS, GS> Geo;
    constexpr int W = kQmvLdsWaves, U = kQmvUnroll;
    static_assert(W >= 1 && W <= kQmvLdsMaxWaves, "waves per workgroup");
    if (count < 1 || count > kQmvMaxProblems || M < 1 || M > Geo::RPL) return false;
    QmvBatch& B = plan.B;
    B = QmvBatch{};
    for (int i = 0; i < kQmvMaxProblems; i++) B.tile0[i] = INT_MAX;
    B.count = count;
    B.M = M;
    const int pbytes = QmvParamWords<BITS, GS, U>::WORDS * 4;
    const int align = pbytes < 16 ? pbytes : 16;
    bool vec = true, tail = false;
    int lds = 0, tiles = 0;
    for (int i = 0; i < count; i++) {
        const QmvSpec& q = specs[i];
        QmvProblem& p = B.p[i];
        const int64_t G = q.K / GS;
        if (q.N % 16 != 0 || q.K % GS != 0 || q.K <= 0 || q.N <= 0) return false;
        if (int64_t(q.N) * q.K * BITS / 8 >= (int64_t(1) << 31) || int64_t(M) * q.K * 2 >= (int64_t(1) << 31) ||
            int64_t(q.N) * G * 2 >= (int64_t(1) << 31))
            return false;
        p.x = q.x, p.w = q.w, p.s = static_cast<const uint16_t*>(q.s), p.b = static_cast<const uint16_t*>(q.b);
        p.y = q.y, p.N = q.N, p.K = q.K, p.ldy = q.ldy;
        const int S = (q.K + Geo::SPAN - 1) / Geo::SPAN;
        // spans per wave: a multiple of U (blocks start at multiples of U)
        p.spw = ((S + W - 1) / W + U - 1) / U * U;
        tail = tail || q.K % (U * Geo::SPAN) != 0;
        B.tile0[i] = tiles;
        tiles += q.N / 16;
        p.kpad = (q.K + 63) / 64 * 64;
        p.inv_cpr = 1.0f / float(p.kpad / 8);
        vec = vec && (G * 2) % align == 0 && aligned(q.s, align) && (q.b == nullptr || aligned(q.b, align));
        // stage each distinct activation matrix once
        p.x_lds = -1;
        for (int j = 0; j < i && share_x; j++)
            if (B.p[j].x == q.x && B.p[j].K == q.K) p.x_lds = B.p[j].x_lds;
        if (p.x_lds < 0) {
            p.x_lds = lds;
            B.stage[B.nstage++] = i;
            lds += M * p.kpad * 2;
        }
    }
    B.total_tiles = tiles;
    B.phase_spans = 0;
    const int zero_bytes = (U * Geo::SPAN * 2 + 64 + 15) / 16 * 16;
    const int red_bytes = 2 * W * M * 16 * 4;
    // Per-CU workgroups of the grid (EQ_QMV_WAVES_PER_CU waves per CU).
    const int per_cu = EQ_QMV_WAVES_PER_CU / W > 0 ? EQ_QMV_WAVES_PER_CU / W : 1;
    const int cap = per_cu * device_cu_count();
    if (lds + zero_bytes + red_bytes > device_lds_bytes()) {
        // Activations too long for LDS: stage them in K phases, for one
        // problem with whole blocks and at most one tile per workgroup, the
        // phase length a whole number of the waves' interleave stride.
        const QmvSpec& q = specs[0];
        const int S = q.K / Geo::SPAN, stride = U * W;
        if (count != 1 || tail || tiles > cap || S % stride != 0 || S / U < W) return false;
        const int nstrides = S / stride;
        int ps = 0;
        for (int P = 2; P <= nstrides && ps == 0; P++) {
            const int per = (nstrides + P - 1) / P;  // strides per phase (the last may have fewer)
            if (M * per * stride * Geo::SPAN * 2 + zero_bytes + red_bytes <= device_lds_bytes()) ps = per * stride;
        }
        if (ps == 0) return false;
        QmvProblem& p = B.p[0];
        p.kpad = ps * Geo::SPAN;
        p.inv_cpr = 1.0f / float(p.kpad / 8);
        B.phase_spans = ps;
        lds = M * p.kpad * 2;
    }
    B.zero_lds = lds;
    B.zero_bytes = zero_bytes;
    lds += B.zero_bytes;
    B.red_lds = lds;
    lds += red_bytes;

    if (lds > device_lds_bytes()) return false;
    if (M > Geo::MB && (!vec || tail)) return false;  // two row sets: whole blocks, vector parameters
    plan.lds = lds;
    plan.vec = vec;
    plan.tail = tail;
    plan.waves = W;
    plan.grid = tiles < cap ? tiles : cap;
    return true;
}

template <int BITS, int GS, typename ST, typename XT = BF16T>
static void run_qmv_lds(const QmvLdsPlan& plan, hipStream_t st) {
    auto go = [&](auto kernel) {
        // (a refusal surfaces as a launch error)
        if (plan.lds > 65536)
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      plan.lds);
        kernel<<<dim3(unsigned(plan.grid)), dim3(64 * plan.waves), size_t(plan.lds), st>>>(plan.B);
    };
    if constexpr (QmvGeom<BITS, GS>::RPL > QmvGeom<BITS, GS>::MB) {
        if (plan.B.M > QmvGeom<BITS, GS>::MB) {  // (the planner checked vec and whole blocks)
            if (EQ_QMV_DIRECT_PHASES && plan.B.phase_spans > 0 && plan.B.p[0].x_lds == 0 &&
                (plan.B.M * (plan.B.p[0].kpad / 8)) % 64 == 0)
                go(qmv_lds_kernel<BITS, GS, ST, 8, true, false, 0, XT, 0, false, true>);
            else
                go(qmv_lds_kernel<BITS, GS, ST, 8, true, false, 0, XT>);
            return;
        }
    }
    if (plan.B.M == 1) {
        if (plan.vec && !plan.tail) go(qmv_lds_kernel<BITS, GS, ST, 1, true, false, 0, XT>);
        else if (plan.vec) go(qmv_lds_kernel<BITS, GS, ST, 1, true, true, 0, XT>);
        else go(qmv_lds_kernel<BITS, GS, ST, 1, false, true, 0, XT>);
    } else {
        if (EQ_QMV_DIRECT_PHASES && plan.B.phase_spans > 0 && plan.vec && !plan.tail &&
            plan.B.p[0].x_lds == 0 && (plan.B.M * (plan.B.p[0].kpad / 8)) % 64 == 0)
            go(qmv_lds_kernel<BITS, GS, ST, 4, true, false, 0, XT, 0, false, true>);
        else if (plan.vec && !plan.tail) go(qmv_lds_kernel<BITS, GS, ST, 4, true, false, 0, XT>);
        else if (plan.vec) go(qmv_lds_kernel<BITS, GS, ST, 4, true, true, 0, XT>);
        else go(qmv_lds_kernel<BITS, GS, ST, 4, false, true, 0, XT>);
    }
}

// Activation rows per launch of the LDS kernel for these problems: RPL when
// the two-row-set kernel takes them (every K whole blocks, vector parameter
// loads), else MB.
template <int BITS, int GS>
static int qmv_launch_rows(const QmvSpec* specs, int count) {
    typedef QmvGeom<BITS, GS> Geo;
    if (Geo::RPL == Geo::MB) return Geo::MB;
    const int pbytes = QmvParamWords<BITS, GS, kQmvUnroll>::WORDS * 4;
    const int align = pbytes < 16 ? pbytes : 16;
    for (int i = 0; i < count; i++) {
        const QmvSpec& q = specs[i];
        const int64_t G = q.K / GS;
        if (q.K % (kQmvUnroll * Geo::SPAN) != 0 || (G * 2) % align != 0 || !aligned(q.s, align) ||
            (q.b != nullptr && !aligned(q.b, align)))
            return Geo::MB;
    }
    return Geo::RPL;
}

template <int BITS, int GS, typename ST, typename XT>
static bool launch_qmv_lds(const QmvSpec* specs, int count, int M, hipStream_t st) {
    QmvLdsPlan plan;
    if (!plan_qmv_lds<BITS, GS, ST>(specs, count, M, plan)) return false;
    run_qmv_lds<BITS, GS, ST, XT>(plan, st);
    return true;
}

// Grouped decode launch: problems in groups of kQmvMaxProblems, activation
// rows in chunks of qmv_launch_rows; every launch is planned before any is
// issued.
template <int BITS, int GS, typename ST, typename XT>
static bool launch_qmv_group_t(const QmvSpec* specs, int count, int M, hipStream_t st) {
    std::vector<QmvLdsPlan> plans;
    QmvSpec chunk[kQmvMaxProblems];
    const int rows = qmv_launch_rows<BITS, GS>(specs, count);
    for (int m0 = 0; m0 < M; m0 += rows) {
        const int mc = M - m0 < rows ? M - m0 : rows;
        for (int i0 = 0; i0 < count; i0 += kQmvMaxProblems) {
            const int n = count - i0 < kQmvMaxProblems ? count - i0 : kQmvMaxProblems;
            for (int i = 0; i < n; i++) {
                chunk[i] = specs[i0 + i];
                chunk[i].x += int64_t(m0) * chunk[i].K;
                chunk[i].y += int64_t(m0) * chunk[i].ldy;
            }
            plans.emplace_back();
            if (!plan_qmv_lds<BITS, GS, ST>(chunk, n, mc, plans.back())) return false;
        }
    }
    for (const QmvLdsPlan& plan : plans) run_qmv_lds<BITS, GS, ST, XT>(plan, st);
    return true;
}

template <int BITS, int GS, typename ST, typename XT>
static void launch_qmv_t(uint16_t* y, const uint16_t* x, const uint32_t* w, const void* sv, const void* bv, int M,
                         int N, int K, hipStream_t st) {
    typedef QmvGeom<BITS, GS> Geo;
    // Persistent LDS variant, in chunks of at most qmv_launch_rows activation
    // rows; the rows it does not take (activations too large for LDS) go to
    // the kernel above.
    int m0 = 0;
    const QmvSpec q0{x, w, sv, bv, y, N, K, N};
    const int rows = qmv_launch_rows<BITS, GS>(&q0, 1);
    for (; m0 < M; m0 += rows) {
        const int mc = M - m0 < rows ? M - m0 : rows;
        const QmvSpec q{x + int64_t(m0) * K, w, sv, bv, y + int64_t(m0) * N, N, K, N};
        if (!launch_qmv_lds<BITS, GS, ST, XT>(&q, 1, mc, st)) break;
    }
    if (m0 >= M) return;
    x += int64_t(m0) * K;
    y += int64_t(m0) * N;
    M -= m0;
    const uint16_t* s = static_cast<const uint16_t*>(sv);
    const uint16_t* b = static_cast<const uint16_t*>(bv);
    const int spans = (K + Geo::SPAN - 1) / Geo::SPAN;
    // About kQmvSpansPerWave spans per wave, at most kQmvMaxWaves waves; spans
    // per wave a multiple of the block length, so that every block starts at a
    // multiple of kQmvUnroll (aligned scale loads; even spans, see qmv_load).
    int waves = (spans + kQmvSpansPerWave - 1) / kQmvSpansPerWave;
    waves = waves < 1 ? 1 : (waves > kQmvMaxWaves ? kQmvMaxWaves : waves);
    const int spw = ((spans + waves - 1) / waves + kQmvUnroll - 1) / kQmvUnroll * kQmvUnroll;
    waves = (spans + spw - 1) / spw;
    // Vector scale/bias loads need rows and pointers aligned to the load size.
    const int G = K / GS;
    const int pbytes = QmvParamWords<BITS, GS, kQmvUnroll>::WORDS * 4;
    const int align = pbytes < 16 ? pbytes : 16;
    const bool vec = (G * 2) % align == 0 && aligned(s, align) && (b == nullptr || aligned(b, align));
    // Buffer offsets are 32-bit: launch in row chunks of < 2^31 bytes of codes.
    const int64_t row_bytes = int64_t(K) * BITS / 8;
    int64_t rows_per_launch = ((int64_t(1) << 31) - 1) / row_bytes / 16 * 16;
    if (rows_per_launch < 16) rows_per_launch = 16;
    for (int64_t n0 = 0; n0 < N; n0 += rows_per_launch) {
        const int nc = int(N - n0 < rows_per_launch ? N - n0 : rows_per_launch);
        const uint32_t* wc = w + n0 * (row_bytes / 4);
        const uint16_t* sc = s + n0 * G;
        const uint16_t* bc = b ? b + n0 * G : nullptr;
        // y rows are strided by N; a row chunk writes columns [n0, n0 + nc) of y.
        if (vec)
            launch_qmv_v<BITS, GS, ST, true, XT>(y + n0, x, wc, sc, bc, M, nc, K, N, spw, waves, st);
        else
            launch_qmv_v<BITS, GS, ST, false, XT>(y + n0, x, wc, sc, bc, M, nc, K, N, spw, waves, st);
        if (N - n0 <= rows_per_launch) break;
    }
}

template <int BITS, typename ST, typename XT>
static bool launch_qmv_gs(int gs, uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s, const void* b,
                          int M, int N, int K, hipStream_t st) {
    switch (gs) {
    case 32: launch_qmv_t<BITS, 32, ST, XT>(y, x, w, s, b, M, N, K, st); return true;
    case 64: launch_qmv_t<BITS, 64, ST, XT>(y, x, w, s, b, M, N, K, st); return true;
    case 128: launch_qmv_t<BITS, 128, ST, XT>(y, x, w, s, b, M, N, K, st); return true;
    default: return false;
    }
}

// Calls f(bits, scale type, activation type) as compile-time values for the
// combinations the decode kernels take; false for the others.
template <typename F>
static bool with_qmv_types(int bits, int scale_dtype, int x_dtype, F&& f) {
    auto by_x = [&](auto bc, auto st) -> bool {
        if (x_dtype == EQ_DTYPE_BF16) return f(bc, st, BF16T{});
        if (x_dtype == EQ_DTYPE_F16) return f(bc, st, F16T{});
        return false;
    };
    auto by_s = [&](auto bc) -> bool {
        if (scale_dtype == EQ_DTYPE_BF16) return by_x(bc, BF16T{});
        if (scale_dtype == EQ_DTYPE_F16) return by_x(bc, F16T{});
        return false;
    };
    if (bits == 4) return by_s(std::integral_constant<int, 4>{});
    if (bits == 8) return by_s(std::integral_constant<int, 8>{});
    return false;
}

int qmv_rows_per_pass(int bits, int gs) {
    const int span = 4 * (128 / bits);  // QmvGeom<BITS, GS>::SPAN
    const int groups = gs > 0 && span > gs ? span / gs : 1;
    return 16 / groups;
}

// Entry used by the dispatcher (api.hip).  Preconditions checked there:
// x bf16 or f16 (y in x's type), transpose, 1 <= M <= 16, N % 16 == 0,
// K % gs == 0, 16-byte aligned x and weight pointers, scale dtype bf16 or f16.
bool launch_qmv_mfma(int bits, int gs, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w,
                     const void* s, const void* b, int M, int N, int K, hipStream_t st, int x_dtype) {
    return with_qmv_types(bits, scale_dtype, x_dtype, [&](auto bc, auto stt, auto xt) {
        return launch_qmv_gs<decltype(bc)::value, decltype(stt), decltype(xt)>(gs, y, x, w, s, b, M, N, K, st);
    });
}

template <int BITS, typename ST, typename XT>
static bool launch_qmv_group_gs(int gs, const QmvSpec* specs, int count, int M, hipStream_t st) {
    switch (gs) {
    case 32: return launch_qmv_group_t<BITS, 32, ST, XT>(specs, count, M, st);
    case 64: return launch_qmv_group_t<BITS, 64, ST, XT>(specs, count, M, st);
    case 128: return launch_qmv_group_t<BITS, 128, ST, XT>(specs, count, M, st);
    default: return false;
    }
}

// Preconditions as for launch_qmv_mfma, for every problem.
// One decode launch (M = 1) whose shared activation row gets a prologue
// while it is staged (QmvBatch::pro_*).  False, launching nothing, when the
// problems do not fit: more than kQmvMaxProblems, different inputs, N % 16,
// RMSNorm rows longer than one staging round.
template <int BITS, int GS, typename ST, int PRO>
static bool launch_qmv_pro_t(const QmvSpec* specs, int count, const QmvPrologue& pro, hipStream_t st) {
    QmvLdsPlan plan;
    if (!plan_qmv_lds<BITS, GS, ST>(specs, count, 1, plan) || plan.B.nstage != 1 || plan.B.phase_spans != 0)
        return false;
    const int K = specs[0].K;
    if (PRO == 2 && K > 2 * 8 * 64 * kQmvLdsWaves) return false;
    plan.B.pro_second = pro.second;
    plan.B.pro_weight = pro.weight;
    plan.B.pro_hidden_out = pro.hidden_out;
    plan.B.pro_eps = pro.eps;
    auto go = [&](auto kernel) {
        if (plan.lds > 65536)
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      plan.lds);
        kernel<<<dim3(unsigned(plan.grid)), dim3(64 * plan.waves), size_t(plan.lds), st>>>(plan.B);
    };
    if (plan.vec && !plan.tail) go(qmv_lds_kernel<BITS, GS, ST, 1, true, false, PRO>);
    else if (plan.vec) go(qmv_lds_kernel<BITS, GS, ST, 1, true, true, PRO>);
    else go(qmv_lds_kernel<BITS, GS, ST, 1, false, true, PRO>);
    return true;
}

bool launch_qmv_prologue(int bits, int gs, int scale_dtype, const QmvSpec* specs, int count, const QmvPrologue& pro,
                         hipStream_t st) {
    if (gs != 64 || scale_dtype != EQ_DTYPE_BF16 || count < 1) return false;
    if (pro.kind == 1) {
        if (bits == 4) return launch_qmv_pro_t<4, 64, BF16T, 1>(specs, count, pro, st);
        if (bits == 8) return launch_qmv_pro_t<8, 64, BF16T, 1>(specs, count, pro, st);
    } else if (pro.kind == 2) {
        if (bits == 4) return launch_qmv_pro_t<4, 64, BF16T, 2>(specs, count, pro, st);
        if (bits == 8) return launch_qmv_pro_t<8, 64, BF16T, 2>(specs, count, pro, st);
    }
    return false;
}

// The SwiGLU launch: one problem (an interleaved gate/up matrix, N = 2F),
// one activation row, whole blocks, optionally the RMSNorm prologue.
template <int BITS, int PRO>
static bool launch_qmv_swiglu_t(const QmvSpec& spec, const QmvPrologue* pro, hipStream_t st) {
    QmvLdsPlan plan;
    if (!plan_qmv_lds<BITS, 64, BF16T>(&spec, 1, 1, plan) || plan.B.nstage != 1 || plan.B.phase_spans != 0 ||
        !plan.vec || plan.tail)
        return false;
    if (PRO == 2) {
        if (spec.K > 2 * 8 * 64 * kQmvLdsWaves) return false;
        plan.B.pro_second = pro->second;
        plan.B.pro_weight = pro->weight;
        plan.B.pro_hidden_out = pro->hidden_out;
        plan.B.pro_eps = pro->eps;
    }
    auto kernel = qmv_lds_kernel<BITS, 64, BF16T, 1, true, false, PRO, BF16T, 1>;
    if (plan.lds > 65536)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  plan.lds);
    kernel<<<dim3(unsigned(plan.grid)), dim3(64 * plan.waves), size_t(plan.lds), st>>>(plan.B);
    return true;
}

bool launch_qmv_swiglu(int bits, const QmvSpec& spec, const QmvPrologue* pro, hipStream_t st) {
    if (pro && pro->kind != 2) return false;
    if (bits == 4) return pro ? launch_qmv_swiglu_t<4, 2>(spec, pro, st) : launch_qmv_swiglu_t<4, 0>(spec, pro, st);
    if (bits == 8) return pro ? launch_qmv_swiglu_t<8, 2>(spec, pro, st) : launch_qmv_swiglu_t<8, 0>(spec, pro, st);
    return false;
}

// Routed decode (gather_qmm, transpose, one bf16 activation row per output
// batch): output batches in launches of up to kQmvMaxProblems problems whose
// activation rows all fit LDS at once; every K a whole number of blocks and
// vector-aligned parameters.  False, launching nothing, when the call does
// not fit that (the caller then runs the general routed kernel).
template <int BITS, int GS, typename ST>
static bool launch_qmv_gather_t(uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s, const void* b,
                                const GatherIdx& g, int64_t batch, int N, int K, hipStream_t st) {
    const int kpad = (K + 63) / 64 * 64;
    int per = (device_lds_bytes() - 16384) / (kpad * 2);
    per = per > kQmvMaxProblems ? kQmvMaxProblems : per;
    // at most two launches: many routes run faster as the single launch of
    // the general routed kernel (4096 routes of 768 x 2048: 0.7 against 6.6 ms)
    if (per < 1 || batch < 1 || batch > 2 * per) return false;
    const int64_t G = K / GS;
    std::vector<QmvLdsPlan> plans;
    for (int64_t b0 = 0; b0 < batch; b0 += per) {
        const int count = int(batch - b0 < per ? batch - b0 : per);
        QmvSpec specs[kQmvMaxProblems];
        for (int i = 0; i < count; i++)
            specs[i] = QmvSpec{x, w, s, b, y + (b0 + i) * int64_t(N), N, K, N};
        QmvLdsPlan plan;
        if (!plan_qmv_lds<BITS, GS, ST>(specs, count, 1, plan, false) || !plan.vec || plan.tail ||
            plan.B.phase_spans != 0)
            return false;
        plan.B.g_lhs = g.lhs;
        plan.B.g_rhs = g.rhs;
        plan.B.g_xb = g.x_batches;
        plan.B.g_wb = g.w_batches;
        plan.B.g_x_stride = K;
        plan.B.g_w_stride = int64_t(N) * (int64_t(K) * BITS / 32);
        plan.B.g_s_stride = int64_t(N) * G;
        plan.B.g_b0 = int(b0);
        plans.push_back(plan);
    }
    auto kernel = qmv_lds_kernel<BITS, GS, ST, 1, true, false, 0, BF16T, 0, true>;
    for (const QmvLdsPlan& plan : plans) {
        if (plan.lds > 65536)
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, plan.lds);
        kernel<<<dim3(unsigned(plan.grid)), dim3(64 * plan.waves), size_t(plan.lds), st>>>(plan.B);
    }
    return true;
}

bool launch_qmv_gather(int bits, int gs, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w,
                       const void* s, const void* b, const GatherIdx& g, int64_t batch, int N, int K,
                       hipStream_t st) {
    if (N % 16 != 0 || batch > INT32_MAX || (bits != 4 && bits != 8)) return false;
    auto by_gs = [&](auto bc, auto stt) -> bool {
        constexpr int B = decltype(bc)::value;
        typedef decltype(stt) ST;
        switch (gs) {
        case 32: return launch_qmv_gather_t<B, 32, ST>(y, x, w, s, b, g, batch, N, K, st);
        case 64: return launch_qmv_gather_t<B, 64, ST>(y, x, w, s, b, g, batch, N, K, st);
        case 128: return launch_qmv_gather_t<B, 128, ST>(y, x, w, s, b, g, batch, N, K, st);
        default: return false;
        }
    };
    if (scale_dtype == EQ_DTYPE_BF16)
        return bits == 4 ? by_gs(std::integral_constant<int, 4>{}, BF16T{}) : by_gs(std::integral_constant<int, 8>{}, BF16T{});
    if (scale_dtype == EQ_DTYPE_F16)
        return bits == 4 ? by_gs(std::integral_constant<int, 4>{}, F16T{}) : by_gs(std::integral_constant<int, 8>{}, F16T{});
    return false;
}

bool launch_qmv_batched(int bits, int gs, int scale_dtype, const QmvSpec* specs, int count, int M, hipStream_t st,
                        int x_dtype) {
    return with_qmv_types(bits, scale_dtype, x_dtype, [&](auto bc, auto stt, auto xt) {
        return launch_qmv_group_gs<decltype(bc)::value, decltype(stt), decltype(xt)>(gs, specs, count, M, st);
    });
}

}  // namespace eq
