// GGML block dequant and convert on gfx950.
//
// Restates, per block and bit for bit, eredu-gguf/src/convert.rs:318-564
// (convert_affine for Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q8_0 / Q2_K / Q3_K / Q4_K /
// Q5_K / Q6_K), AffineTensor::dequantize (convert.rs:81-101) and the native
// decoders of safemlx/src/native_quantization.rs:3445-3469 (Q4_K), :3499-3509
// (Q5_1) and :3539-3542 (Q8_0).
//
// All kernels are HBM-bound byte work.  Q4_0 (18 B) and Q8_0 (34 B) blocks are
// not 4-byte aligned, so a workgroup stages its 256 blocks through LDS with
// 16-byte coalesced loads and each thread then decodes one block from LDS.
// Q4_K superblocks (144 B) are 16-byte aligned and are read directly, one
// thread per 32-value group for the affine convert.  Dense output is written
// by four lanes per 32-value block or group (8 values each), so that wave
// stores are contiguous.  Every product in these decoders is exact in f32
// (an 11-bit f16 significand times a code of at most 8 bits), so each output
// carries exactly one rounding, as on the reference's CPU.
#include <atomic>

#include "eq_common.hpp"

namespace eq {
namespace {

// Routes of a mixture-of-experts call in one launch of the native linear
// kernels: route r = blockIdx.y reads x row r, writes y row r, and takes the
// expert matrix raw + ids[r] * stride.  An id outside [0, experts) reads
// expert 0 (every access stays in the bank) and its row is written as +0.  ids null: one matrix, one route (grid.y = 1).
struct ExpertSel {
    const int32_t* ids = nullptr;
    int64_t stride = 0;
    int experts = 0;
    int routes = 1;
};

__device__ __forceinline__ const uint8_t* select_expert(const uint8_t* raw, const ExpertSel& sel) {
    if (!sel.ids) return raw;
    int e = sel.ids[blockIdx.y];
    e = (e < 0 || e >= sel.experts) ? 0 : e;
    return raw + int64_t(e) * sel.stride;
}

// Row offset of this block's route (0 without ids).
__device__ __forceinline__ int64_t route_row(const ExpertSel& sel) { return sel.ids ? int64_t(blockIdx.y) : 0; }

// False for a route whose id is outside the bank: its row is written as +0.
__device__ __forceinline__ bool route_ok(const ExpertSel& sel) {
    if (!sel.ids) return true;
    const int e = sel.ids[blockIdx.y];
    return e >= 0 && e < sel.experts;
}

constexpr int kBlocksPerWG = 256;

__device__ __forceinline__ uint32_t bswap16(uint32_t v) { return ((v & 0xffu) << 8) | ((v >> 8) & 0xffu); }

// Four low nibbles of the bytes of x, compressed into 16 bits (byte i's low
// nibble lands in bits 4i..4i+3): the 4-bit LSB-first pack of convert.rs:413-427
// for codes taken byte by byte.
__device__ __forceinline__ uint32_t lo_nibbles(uint32_t x) {
    x &= 0x0f0f0f0fu;
    x |= x >> 4;
    return (x & 0xffu) | ((x >> 8) & 0xff00u);
}
__device__ __forceinline__ uint32_t hi_nibbles(uint32_t x) { return lo_nibbles(x >> 4); }

// Copies `nb` blocks of `bytes` each (starting at block blk0) into LDS.
// Full workgroups on a 16-byte-aligned payload use 16-byte loads; a ragged
// tail uses 2-byte loads (block sizes here are even), so nothing past the
// payload is ever read.
template <int BYTES, int NB = kBlocksPerWG>
__device__ __forceinline__ void stage_blocks(uint16_t* lds, const uint8_t* raw, int64_t blk0, int nb,
                                             bool vec_ok) {
    static_assert(NB * BYTES % 16 == 0, "a workgroup's blocks must start 16-byte aligned");
    const uint8_t* src = raw + blk0 * BYTES;
    if (vec_ok && nb == NB) {
        constexpr int kVec = NB * BYTES / 16;
        const uint4* s4 = reinterpret_cast<const uint4*>(src);
        uint4* d4 = reinterpret_cast<uint4*>(lds);
        for (int i = threadIdx.x; i < kVec; i += blockDim.x) d4[i] = s4[i];
    } else {
        const uint16_t* s2 = reinterpret_cast<const uint16_t*>(src);
        const int n2 = nb * BYTES / 2;
        for (int i = threadIdx.x; i < n2; i += blockDim.x) lds[i] = s2[i];
    }
    __syncthreads();
}

__device__ __forceinline__ uint32_t lds_u32(const uint16_t* p) { return uint32_t(p[0]) | (uint32_t(p[1]) << 16); }

// ------------------------------------------------------------- Q4_0 / Q8_0

// Decodes one Q4_0 block from LDS: f16 d, and the 16 quant bytes as 4 words.
template <bool BIG>
__device__ __forceinline__ void q4_0_block(const uint16_t* b, uint32_t& d, uint32_t q[4]) {
    d = BIG ? bswap16(b[0]) : b[0];
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = lds_u32(b + 1 + 2 * i);
}

template <bool BIG>
__global__ __launch_bounds__(256) void q4_0_to_affine(const uint8_t* __restrict__ raw, int64_t nblocks,
                                                      bool vec_ok, uint4* __restrict__ w,
                                                      uint16_t* __restrict__ s, uint16_t* __restrict__ bias) {
    __shared__ uint16_t lds[kBlocksPerWG * 18 / 2];
    const int64_t blk0 = int64_t(blockIdx.x) * kBlocksPerWG;
    const int nb = int(min<int64_t>(kBlocksPerWG, nblocks - blk0));
    stage_blocks<18>(lds, raw, blk0, nb, vec_ok);
    const int t = threadIdx.x;
    if (t >= nb) return;
    uint32_t d, q[4];
    q4_0_block<BIG>(lds + t * 9, d, q);
    const int64_t blk = blk0 + t;
    // codes[0..16) = low nibbles, codes[16..32) = high nibbles (convert.rs:355-358)
    w[blk] = make_uint4(lo_nibbles(q[0]) | (lo_nibbles(q[1]) << 16), lo_nibbles(q[2]) | (lo_nibbles(q[3]) << 16),
                        hi_nibbles(q[0]) | (hi_nibbles(q[1]) << 16), hi_nibbles(q[2]) | (hi_nibbles(q[3]) << 16));
    s[blk] = uint16_t(d);
    bias[blk] = uint16_t(f32_to_f16_bits(-8.0f * f16_bits_to_f32(d)));  // convert.rs:352
}

template <bool BIG>
__global__ __launch_bounds__(256) void q8_0_to_affine(const uint8_t* __restrict__ raw, int64_t nblocks,
                                                      bool vec_ok, uint4* __restrict__ w,
                                                      uint16_t* __restrict__ s, uint16_t* __restrict__ bias) {
    __shared__ uint16_t lds[kBlocksPerWG * 34 / 2];
    const int64_t blk0 = int64_t(blockIdx.x) * kBlocksPerWG;
    const int nb = int(min<int64_t>(kBlocksPerWG, nblocks - blk0));
    stage_blocks<34>(lds, raw, blk0, nb, vec_ok);
    const int t = threadIdx.x;
    if (t >= nb) return;
    const uint16_t* b = lds + t * 17;
    const uint32_t d = BIG ? bswap16(b[0]) : b[0];
    uint32_t q[8];
#pragma unroll
    for (int i = 0; i < 8; i++) q[i] = lds_u32(b + 1 + 2 * i) ^ 0x80808080u;  // convert.rs:381
    const int64_t blk = blk0 + t;
    w[2 * blk] = make_uint4(q[0], q[1], q[2], q[3]);
    w[2 * blk + 1] = make_uint4(q[4], q[5], q[6], q[7]);
    s[blk] = uint16_t(d);
    bias[blk] = uint16_t(f32_to_f16_bits(-128.0f * f16_bits_to_f32(d)));  // convert.rs:380
}

// Dense output: a block's (or Q4_K group's) 32 values are decoded by four
// consecutive lanes, 8 values each, so that one wave store writes a
// contiguous kilobyte (bf16) or two (f32).
template <typename OUT>
__device__ __forceinline__ void store8(typename OUT::storage* out, int64_t base, const float v[8]);
template <>
__device__ __forceinline__ void store8<BF16T>(uint16_t* out, int64_t base, const float v[8]) {
    uint32_t p[4];
#pragma unroll
    for (int j = 0; j < 4; j++) p[j] = pack_bf16x2(v[2 * j], v[2 * j + 1]);
    store_stream16(out + base, make_uint4(p[0], p[1], p[2], p[3]));
}
template <>
__device__ __forceinline__ void store8<F32T>(float* out, int64_t base, const float v[8]) {
    store_stream16(out + base, make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                          __float_as_uint(v[3])));
    store_stream16(out + base + 4, make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]),
                                              __float_as_uint(v[7])));
}

// Q4_0 dense: affine route only (Q4_0 has no native decoder, format.rs:423-428):
// w = f32(d) * code + f32(f16(-8 d)).  Quarter c of a block holds values
// [8c, 8c + 8): low nibbles of quant bytes [8c, 8c + 8) for c < 2, high
// nibbles of bytes [8(c - 2), ...) for c >= 2 (convert.rs:355-358).
template <bool BIG, typename OUT>
__global__ __launch_bounds__(256) void q4_0_dense(const uint8_t* __restrict__ raw, int64_t nblocks, bool vec_ok,
                                                  typename OUT::storage* __restrict__ out) {
    __shared__ uint16_t lds[kBlocksPerWG * 18 / 2];
    const int64_t blk0 = int64_t(blockIdx.x) * kBlocksPerWG;
    const int nb = int(min<int64_t>(kBlocksPerWG, nblocks - blk0));
    stage_blocks<18>(lds, raw, blk0, nb, vec_ok);
    const int c = threadIdx.x & 3;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int lb = k * 64 + (threadIdx.x >> 2);
        if (lb >= nb) break;
        const uint16_t* blk = lds + lb * 9;
        const uint32_t d = BIG ? bswap16(blk[0]) : blk[0];
        const float scale = f16_bits_to_f32(d);
        const float bias = f16_bits_to_f32(f32_to_f16_bits(-8.0f * scale));
        const int sh = (c >> 1) * 4;
        const uint32_t q0 = lds_u32(blk + 1 + 4 * (c & 1)), q1 = lds_u32(blk + 3 + 4 * (c & 1));
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = scale * float(((i < 4 ? q0 : q1) >> (8 * (i & 3) + sh)) & 15u) + bias;
        store8<OUT>(out, (blk0 + lb) * 32 + 8 * c, v);
    }
}

// Q8_0 dense.  Affine route: f32(d) * (q ^ 0x80) + f32(f16(-128 d));
// native route: f32(d) * int8(q).  Identical unless -128 d overflows f16.
template <bool BIG, bool NATIVE, typename OUT>
__global__ __launch_bounds__(256) void q8_0_dense(const uint8_t* __restrict__ raw, int64_t nblocks, bool vec_ok,
                                                  typename OUT::storage* __restrict__ out) {
    __shared__ uint16_t lds[kBlocksPerWG * 34 / 2];
    const int64_t blk0 = int64_t(blockIdx.x) * kBlocksPerWG;
    const int nb = int(min<int64_t>(kBlocksPerWG, nblocks - blk0));
    stage_blocks<34>(lds, raw, blk0, nb, vec_ok);
    const int c = threadIdx.x & 3;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int lb = k * 64 + (threadIdx.x >> 2);
        if (lb >= nb) break;
        const uint16_t* blk = lds + lb * 17;
        const uint32_t dbits = BIG ? bswap16(blk[0]) : blk[0];
        const float d = f16_bits_to_f32(dbits);
        const float bias = f16_bits_to_f32(f32_to_f16_bits(-128.0f * d));
        const uint32_t q0 = lds_u32(blk + 1 + 4 * c), q1 = lds_u32(blk + 3 + 4 * c);
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t byte = ((i < 4 ? q0 : q1) >> (8 * (i & 3))) & 0xffu;
            if (NATIVE)
                v[i] = d * float(int8_t(byte));
            else
                v[i] = d * float(byte ^ 0x80u) + bias;
        }
        store8<OUT>(out, (blk0 + lb) * 32 + 8 * c, v);
    }
}

// ------------------------------------------------------------------- Q4_K

struct Q4KGroup {
    float d, dmin;
    uint32_t sc, m;
    uint32_t q[8];  // the 32 quant bytes holding this group's nibbles
};

// 6-bit scale and min of group g from the 12 scale bytes s[0..12) = bytes of
// h[1], h[2], h[3] (scale_min, convert.rs:429-438).
__device__ __forceinline__ void q4k_scale_min(const uint32_t h[4], int g, uint32_t& sc, uint32_t& m) {
    auto sbyte = [&](int i) -> uint32_t { return (h[1 + (i >> 2)] >> (8 * (i & 3))) & 0xffu; };
    if (g < 4) {
        sc = sbyte(g) & 63u;
        m = sbyte(g + 4) & 63u;
    } else {
        sc = (sbyte(g + 4) & 15u) | ((sbyte(g - 4) >> 6) << 4);
        m = (sbyte(g + 4) >> 4) | ((sbyte(g) >> 6) << 4);
    }
}

// One 32-value group g of a 144-byte superblock (convert.rs:439-465,
// native_quantization.rs:3445-3469): header = d, dmin, 12 scale bytes; group g
// takes the low (g even) or high (g odd) nibbles of quant bytes [(g/2)*32, +32).
template <bool BIG>
__device__ __forceinline__ Q4KGroup load_q4k_group(const uint8_t* __restrict__ raw, int64_t sb, int g, bool vec_ok) {
    const uint8_t* p = raw + sb * 144;
    uint32_t h[4], q[8];
    if (vec_ok) {
        const uint4 hv = *reinterpret_cast<const uint4*>(p);
        const uint4 qa = *reinterpret_cast<const uint4*>(p + 16 + (g >> 1) * 32);
        const uint4 qb = *reinterpret_cast<const uint4*>(p + 32 + (g >> 1) * 32);
        h[0] = hv.x; h[1] = hv.y; h[2] = hv.z; h[3] = hv.w;
        q[0] = qa.x; q[1] = qa.y; q[2] = qa.z; q[3] = qa.w;
        q[4] = qb.x; q[5] = qb.y; q[6] = qb.z; q[7] = qb.w;
    } else {
        const uint16_t* p2 = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
        for (int i = 0; i < 4; i++) h[i] = uint32_t(p2[2 * i]) | (uint32_t(p2[2 * i + 1]) << 16);
        const uint16_t* q2 = p2 + 8 + (g >> 1) * 16;
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = uint32_t(q2[2 * i]) | (uint32_t(q2[2 * i + 1]) << 16);
    }
    Q4KGroup r;
    const uint32_t dbits = BIG ? bswap16(h[0] & 0xffffu) : (h[0] & 0xffffu);
    const uint32_t mbits = BIG ? bswap16(h[0] >> 16) : (h[0] >> 16);
    r.d = f16_bits_to_f32(dbits);
    r.dmin = f16_bits_to_f32(mbits);
    q4k_scale_min(h, g, r.sc, r.m);
#pragma unroll
    for (int i = 0; i < 8; i++) r.q[i] = q[i];
    return r;
}

template <bool BIG>
__global__ __launch_bounds__(256) void q4k_to_affine(const uint8_t* __restrict__ raw, int64_t ngroups, bool vec_ok,
                                                     uint4* __restrict__ w, uint16_t* __restrict__ s,
                                                     uint16_t* __restrict__ bias) {
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= ngroups) return;
    const int g = int(idx & 7);
    const Q4KGroup r = load_q4k_group<BIG>(raw, idx >> 3, g, vec_ok);
    uint32_t wd[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t a = r.q[2 * j], b = r.q[2 * j + 1];
        wd[j] = (g & 1) ? (hi_nibbles(a) | (hi_nibbles(b) << 16)) : (lo_nibbles(a) | (lo_nibbles(b) << 16));
    }
    w[idx] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
    s[idx] = uint16_t(f32_to_f16_bits(r.d * float(r.sc)));       // convert.rs:449
    bias[idx] = uint16_t(f32_to_f16_bits(-r.dmin * float(r.m)));  // convert.rs:450
}

// Q4_K dense: thread idx decodes quarter c = idx % 4 (values [8c, 8c + 8),
// quant bytes [8c, 8c + 8) of the group's 32) of group (idx / 4) % 8 of
// superblock idx / 32.
template <bool BIG, bool NATIVE, typename OUT>
__global__ __launch_bounds__(256) void q4k_dense(const uint8_t* __restrict__ raw, int64_t nquarters, bool vec_ok,
                                                 typename OUT::storage* __restrict__ out) {
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= nquarters) return;
    const int c = int(idx & 3), g = int((idx >> 2) & 7);
    // the superblock's 16-byte header (same address for its 32 lanes) and this
    // quarter's 8 quant bytes
    const uint8_t* p = raw + (idx >> 5) * 144;
    const int qo = 16 + (g >> 1) * 32 + 8 * c;
    uint32_t h[4], q0, q1;
    if (vec_ok) {
        const uint4 hv = *reinterpret_cast<const uint4*>(p);
        const uint2 qv = *reinterpret_cast<const uint2*>(p + qo);
        h[0] = hv.x, h[1] = hv.y, h[2] = hv.z, h[3] = hv.w;
        q0 = qv.x, q1 = qv.y;
    } else {
        const uint16_t* p2 = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
        for (int i = 0; i < 4; i++) h[i] = uint32_t(p2[2 * i]) | (uint32_t(p2[2 * i + 1]) << 16);
        const uint16_t* q2 = reinterpret_cast<const uint16_t*>(p + qo);
        q0 = uint32_t(q2[0]) | (uint32_t(q2[1]) << 16);
        q1 = uint32_t(q2[2]) | (uint32_t(q2[3]) << 16);
    }
    uint32_t sc, m;
    q4k_scale_min(h, g, sc, m);
    const float d = f16_bits_to_f32(BIG ? bswap16(h[0] & 0xffffu) : (h[0] & 0xffffu));
    const float dmin = f16_bits_to_f32(BIG ? bswap16(h[0] >> 16) : (h[0] >> 16));
    const int sh = (g & 1) * 4;
    float v[8];
    if (NATIVE) {
        // d * sc * q - dmin * m, left to right (native_quantization.rs:3466)
        const float ds = d * float(sc);
        const float dm = dmin * float(m);
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = ds * float(((i < 4 ? q0 : q1) >> (8 * (i & 3) + sh)) & 15u) - dm;
    } else {
        // f32(f16(d sc)) * q + f32(f16(-dmin m)) (convert.rs:81-101 on the q45k output)
        const float scale = f16_bits_to_f32(f32_to_f16_bits(d * float(sc)));
        const float bias = f16_bits_to_f32(f32_to_f16_bits(-dmin * float(m)));
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = scale * float(((i < 4 ? q0 : q1) >> (8 * (i & 3) + sh)) & 15u) + bias;
    }
    store8<OUT>(out, (idx >> 2) * 32 + 8 * c, v);
}

// --------------------------- Q4_1 / Q5_0 / Q5_1 / Q2_K / Q3_K / Q5_K / Q6_K
//
// Blocks of 20 / 22 / 24 / 84 / 110 / 176 / 210 bytes, staged through LDS
// like Q4_0.  The unit of work is 32 consecutive values: a whole block of
// the 32-value types, an eighth of a 256-value superblock.  A unit packs to
// exactly `bits` u32 words and holds one (group 32) or two (group 16)
// affine groups, so each thread of the convert writes whole words and whole
// groups, and each quarter-lane of the dense decode writes 8 values of one
// group.

template <int T>
struct KQuant;
// levels: the codes index the IQ4 level table instead of being affine codes.
template <> struct KQuant<EQ_GGML_Q4_1> { static constexpr int bytes = 20, units = 1, bits = 4, gs = 32; static constexpr bool levels = false; };
template <> struct KQuant<EQ_GGML_Q5_0> { static constexpr int bytes = 22, units = 1, bits = 5, gs = 32; static constexpr bool levels = false; };
template <> struct KQuant<EQ_GGML_Q5_1> { static constexpr int bytes = 24, units = 1, bits = 5, gs = 32; static constexpr bool levels = false; };
template <> struct KQuant<EQ_GGML_Q2_K> { static constexpr int bytes = 84, units = 8, bits = 2, gs = 16; static constexpr bool levels = false; };
template <> struct KQuant<EQ_GGML_Q3_K> { static constexpr int bytes = 110, units = 8, bits = 3, gs = 16; static constexpr bool levels = false; };
template <> struct KQuant<EQ_GGML_Q5_K> { static constexpr int bytes = 176, units = 8, bits = 5, gs = 32; static constexpr bool levels = false; };
template <> struct KQuant<EQ_GGML_Q6_K> { static constexpr int bytes = 210, units = 8, bits = 6, gs = 16; static constexpr bool levels = false; };
template <> struct KQuant<EQ_GGML_IQ4_NL> { static constexpr int bytes = 18, units = 1, bits = 4, gs = 32; static constexpr bool levels = true; };
template <> struct KQuant<EQ_GGML_IQ4_XS> { static constexpr int bytes = 136, units = 8, bits = 4, gs = 32; static constexpr bool levels = true; };

// The 16 levels of IQ4_NL / IQ4_XS (the GGML format's kvalues_iq4nl; the
// reference's KVALUES_IQ4NL, eredu-gguf/src/iquant_tables.rs:1920), each plus
// 128 (1 .. 241) as the bytes of four words: entries 4w .. 4w + 3 in word w.
constexpr uint32_t kIq4Lut0 = 1u | (24u << 8) | (45u << 16) | (63u << 24);      // -127 -104 -83 -65
constexpr uint32_t kIq4Lut1 = 79u | (93u << 8) | (106u << 16) | (118u << 24);   //  -49  -35 -22 -10
constexpr uint32_t kIq4Lut2 = 129u | (141u << 8) | (153u << 16) | (166u << 24); //    1   13  25  38
constexpr uint32_t kIq4Lut3 = 181u | (197u << 8) | (217u << 16) | (241u << 24); //   53   69  89 113

// Nibble codes in byte lanes -> level + 128 in the same lanes: two byte
// permutes pick from entries 0..7 and 8..15, bit 3 of each code chooses.
__device__ __forceinline__ uint32_t iq4_level_bytes(uint32_t c) {
    const uint32_t sel = c & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(kIq4Lut1, kIq4Lut0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(kIq4Lut3, kIq4Lut2, sel);
    const uint32_t m = ((c >> 3) & 0x01010101u) * 0xffu;
    return (hi & m) | (lo & ~m);
}

// f16 field at byte offset o of a block in LDS.
template <bool BIG>
__device__ __forceinline__ uint32_t lds_half(const uint8_t* b, int o) {
    return BIG ? (uint32_t(b[o]) << 8) | b[o + 1] : uint32_t(b[o]) | (uint32_t(b[o + 1]) << 8);
}

// 8 bytes at an even LDS offset as two words: byte j in byte j % 4 of lo (j < 4)
// or hi.  Blocks of 22 / 110 / 210 bytes sit at 2-byte alignment in LDS, so
// the words are assembled from 16-bit reads.
__device__ __forceinline__ void lds_8b(const uint8_t* p, uint32_t& lo, uint32_t& hi) {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
    lo = uint32_t(q[0]) | (uint32_t(q[1]) << 16);
    hi = uint32_t(q[2]) | (uint32_t(q[3]) << 16);
}

// Bits 0..3 of t moved to bit 0 of bytes 0..3 (the four shifted copies of t
// do not overlap, so the product carries nothing).
__device__ __forceinline__ uint32_t spread4(uint32_t t) { return ((t & 15u) * 0x204081u) & 0x01010101u; }

// Codes of values i0 .. i0 + 7 (i0 a multiple of 8) of unit u of a block, as
// byte lanes: value i0 + j in byte j % 4 of c0 (j < 4) or c1.  Every code of
// a byte lane is extracted by one shift and mask of the word.
template <int T, bool BIG>
__device__ __forceinline__ void kq_codes8(const uint8_t* b, int u, int i0, uint32_t& c0, uint32_t& c1) {
    uint32_t a0, a1, h0, h1;
    if constexpr (T == EQ_GGML_IQ4_NL || T == EQ_GGML_IQ4_XS) {
        // level indices: byte 2 + i (IQ4_NL) or 8 + 16 ib + i (IQ4_XS, unit = group ib)
        // holds value i in its low nibble and value 16 + i in its high (iquant.rs:271-301)
        lds_8b(b + (T == EQ_GGML_IQ4_NL ? 2 : 8 + 16 * u) + (i0 & 15), a0, a1);
        const int sh = (i0 >> 4) * 4;
        c0 = (a0 >> sh) & 0x0f0f0f0fu;
        c1 = (a1 >> sh) & 0x0f0f0f0fu;
    } else if constexpr (T == EQ_GGML_Q4_1) {
        // low nibbles of bytes 4..20 are values 0..15, high nibbles 16..31 (convert.rs:367-370)
        lds_8b(b + 4 + (i0 & 15), a0, a1);
        const int sh = (i0 >> 4) * 4;
        c0 = (a0 >> sh) & 0x0f0f0f0fu;
        c1 = (a1 >> sh) & 0x0f0f0f0fu;
    } else if constexpr (T == EQ_GGML_Q5_0 || T == EQ_GGML_Q5_1) {
        // nibbles as Q4_1 at 6 / 8, plus bit i of the u32 at 2 / 4 as bit 4 (convert.rs:553-562):
        // bits i0 .. i0 + 7 are byte i0 / 8 of that word in its byte order
        constexpr int qh = T == EQ_GGML_Q5_0 ? 2 : 4, qs = qh + 4;
        lds_8b(b + qs + (i0 & 15), a0, a1);
        const int sh = (i0 >> 4) * 4;
        const uint32_t hb = b[qh + (BIG ? 3 - (i0 >> 3) : (i0 >> 3))];
        c0 = ((a0 >> sh) & 0x0f0f0f0fu) | (spread4(hb) << 4);
        c1 = ((a1 >> sh) & 0x0f0f0f0fu) | (spread4(hb >> 4) << 4);
    } else if constexpr (T == EQ_GGML_Q2_K) {
        // group g = 2u + i/16 takes 2 bits at shift 2 ((g % 8) / 2) = 2 (u % 4) of byte
        // 16 + (g / 8) 32 + (g % 2) 16 + i % 16 = 16 + (u / 4) 32 + i (convert.rs:501-505)
        lds_8b(b + 16 + (u >> 2) * 32 + i0, a0, a1);
        const int sh = (u & 3) * 2;
        c0 = (a0 >> sh) & 0x03030303u;
        c1 = (a1 >> sh) & 0x03030303u;
    } else if constexpr (T == EQ_GGML_Q3_K) {
        // as Q2_K at byte 32, plus bit g / 2 = u of hm[(g % 2) 16 + i % 16] = hm[i] as bit 2
        // (convert.rs:531-539)
        lds_8b(b + 32 + (u >> 2) * 32 + i0, a0, a1);
        lds_8b(b + i0, h0, h1);
        const int sh = (u & 3) * 2;
        c0 = ((a0 >> sh) & 0x03030303u) | (((h0 >> u) & 0x01010101u) << 2);
        c1 = ((a1 >> sh) & 0x03030303u) | (((h1 >> u) & 0x01010101u) << 2);
    } else if constexpr (T == EQ_GGML_Q5_K) {
        // unit = group g: nibble g % 2 of qs[(g / 2) 32 + i] at 48, bit g of qh[i] at 16
        // as bit 4 (convert.rs:453-461)
        lds_8b(b + 48 + (u >> 1) * 32 + i0, a0, a1);
        lds_8b(b + 16 + i0, h0, h1);
        const int sh = (u & 1) * 4;
        c0 = ((a0 >> sh) & 0x0f0f0f0fu) | (((h0 >> u) & 0x01010101u) << 4);
        c1 = ((a1 >> sh) & 0x0f0f0f0fu) | (((h1 >> u) & 0x01010101u) << 4);
    } else {
        // Q6_K: unit u is value run k = u % 4 of half h = u / 4: nibble k / 2 of
        // ql[h 64 + (k % 2) 32 + i], bits 2k, 2k + 1 of qh[128 + h 32 + i] as bits 4, 5
        // (convert.rs:472-477)
        const int h = u >> 2, k = u & 3;
        lds_8b(b + h * 64 + (k & 1) * 32 + i0, a0, a1);
        lds_8b(b + 128 + h * 32 + i0, h0, h1);
        const int sh = (k >> 1) * 4;
        c0 = ((a0 >> sh) & 0x0f0f0f0fu) | (((h0 >> (2 * k)) & 0x03030303u) << 4);
        c1 = ((a1 >> sh) & 0x0f0f0f0fu) | (((h1 >> (2 * k)) & 0x03030303u) << 4);
    }
}

// 6-bit scale and min of group g from the 12 scale bytes at s (scale_min,
// convert.rs:429-438), as q4k_scale_min but from LDS bytes.
__device__ __forceinline__ void scale_min_bytes(const uint8_t* s, int g, uint32_t& sc, uint32_t& m) {
    if (g < 4) {
        sc = s[g] & 63u;
        m = s[g + 4] & 63u;
    } else {
        sc = (s[g + 4] & 15u) | ((uint32_t(s[g - 4]) >> 6) << 4);
        m = (uint32_t(s[g + 4]) >> 4) | ((uint32_t(s[g]) >> 6) << 4);
    }
}

// f16 bits of the scale and the bias of group g of a block.
template <int T, bool BIG>
__device__ __forceinline__ void kq_group(const uint8_t* b, int g, uint32_t& sb, uint32_t& bb) {
    if constexpr (T == EQ_GGML_Q4_1 || T == EQ_GGML_Q5_1) {
        sb = lds_half<BIG>(b, 0);  // d and m as stored (convert.rs:364-365, 548-551)
        bb = lds_half<BIG>(b, 2);
    } else if constexpr (T == EQ_GGML_Q5_0) {
        sb = lds_half<BIG>(b, 0);
        bb = f32_to_f16_bits(-16.0f * f16_bits_to_f32(sb));  // convert.rs:549
    } else if constexpr (T == EQ_GGML_Q2_K) {
        const float d = f16_bits_to_f32(lds_half<BIG>(b, 80)), dm = f16_bits_to_f32(lds_half<BIG>(b, 82));
        sb = f32_to_f16_bits(d * float(b[g] & 15u));  // convert.rs:496-499
        bb = f32_to_f16_bits(-dm * float(uint32_t(b[g]) >> 4));
    } else if constexpr (T == EQ_GGML_Q3_K) {
        // 6-bit code: low 4 bits from byte 96 + g % 8 (nibble g / 8), high 2 bits
        // from byte 104 + g % 4 (bits 2 (g / 4)) (convert.rs:514-520)
        const uint32_t enc = ((uint32_t(b[96 + (g & 7)]) >> (4 * (g >> 3))) & 15u) |
                             (((uint32_t(b[104 + (g & 3)]) >> (2 * (g >> 2))) & 3u) << 4);
        const float sc = f16_bits_to_f32(lds_half<BIG>(b, 108)) * float(int(enc) - 32);
        sb = f32_to_f16_bits(sc);  // convert.rs:524-526
        bb = f32_to_f16_bits(-4.0f * sc);
    } else if constexpr (T == EQ_GGML_Q5_K) {
        uint32_t sc, m;
        scale_min_bytes(b + 4, g, sc, m);
        sb = f32_to_f16_bits(f16_bits_to_f32(lds_half<BIG>(b, 0)) * float(sc));  // convert.rs:449-450
        bb = f32_to_f16_bits(-f16_bits_to_f32(lds_half<BIG>(b, 2)) * float(m));
    } else {
        // Q6_K: int8 scale byte 192 + g, d at 208 (convert.rs:469, 479-482)
        const float sc = f16_bits_to_f32(lds_half<BIG>(b, 208)) * float(int8_t(b[192 + g]));
        sb = f32_to_f16_bits(sc);
        bb = f32_to_f16_bits(-32.0f * sc);
    }
}

// Group factors in f32 without f16 rounding: the native definition (and, for
// the IQ4 types, the only one).
template <int T, bool BIG>
__device__ __forceinline__ void kq_native_group(const uint8_t* b, int g, float& scale, float& bias) {
    if constexpr (T == EQ_GGML_Q5_1) {
        scale = f16_bits_to_f32(lds_half<BIG>(b, 0));  // native_quantization.rs:3499-3509
        bias = f16_bits_to_f32(lds_half<BIG>(b, 2));
    } else if constexpr (T == EQ_GGML_Q5_K) {
        uint32_t sc, m;
        scale_min_bytes(b + 4, g, sc, m);
        scale = f16_bits_to_f32(lds_half<BIG>(b, 0)) * float(sc);
        bias = -(f16_bits_to_f32(lds_half<BIG>(b, 2)) * float(m));
    } else if constexpr (T == EQ_GGML_IQ4_NL) {
        scale = f16_bits_to_f32(lds_half<BIG>(b, 0));  // iquant.rs:273
        bias = 0.f;
    } else if constexpr (T == EQ_GGML_IQ4_XS) {
        // 6-bit ls: nibble g % 2 of byte 4 + g / 2, bits 2g, 2g + 1 of the u16 at 2 (iquant.rs:287-290)
        const uint32_t ls = ((uint32_t(b[4 + (g >> 1)]) >> (4 * (g & 1))) & 15u) |
                            (((lds_half<BIG>(b, 2) >> (2 * g)) & 3u) << 4);
        scale = f16_bits_to_f32(lds_half<BIG>(b, 0)) * float(int(ls) - 32);
        bias = 0.f;
    } else {
        static_assert(T == EQ_GGML_Q6_K, "native linear covers Q5_1, Q5_K, Q6_K, IQ4_NL and IQ4_XS here");
        scale = f16_bits_to_f32(lds_half<BIG>(b, 208)) * float(int8_t(b[192 + g]));
        bias = -32.0f * scale;
    }
}

// Stores the `BITS` words of one unit at w (w is 4 * BITS-byte aligned times
// the unit index from a 16-byte-aligned base).
template <int BITS>
__device__ __forceinline__ void store_unit(uint32_t* w, const uint32_t* wd) {
    if constexpr (BITS == 4) {
        *reinterpret_cast<uint4*>(w) = make_uint4(wd[0], wd[1], wd[2], wd[3]);
    } else if constexpr (BITS == 2 || BITS == 6) {
#pragma unroll
        for (int j = 0; j < BITS; j += 2) *reinterpret_cast<uint2*>(w + j) = make_uint2(wd[j], wd[j + 1]);
    } else {
#pragma unroll
        for (int j = 0; j < BITS; j++) w[j] = wd[j];
    }
}

// Four 2-bit codes in byte lanes -> 8 bits, code j at bits 2j.
__device__ __forceinline__ uint32_t crumbs(uint32_t x) {
    x |= x >> 6;
    return (x | (x >> 12)) & 0xffu;
}

// LSB-first pack (convert.rs:413-427) of a unit's 32 codes, given as eight
// byte-lane words, into BITS words.  Widths 3, 5 and 6 go four codes (one
// 4 BITS-bit chunk) at a time; every shift is a constant once unrolled.
template <int BITS>
__device__ __forceinline__ void pack_unit(const uint32_t cw[8], uint32_t wd[BITS]) {
    if constexpr (BITS == 4) {
#pragma unroll
        for (int j = 0; j < 4; j++) wd[j] = lo_nibbles(cw[2 * j]) | (lo_nibbles(cw[2 * j + 1]) << 16);
    } else if constexpr (BITS == 2) {
#pragma unroll
        for (int j = 0; j < 2; j++)
            wd[j] = crumbs(cw[4 * j]) | (crumbs(cw[4 * j + 1]) << 8) | (crumbs(cw[4 * j + 2]) << 16) |
                    (crumbs(cw[4 * j + 3]) << 24);
    } else {
#pragma unroll
        for (int j = 0; j < BITS; j++) wd[j] = 0;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const uint32_t x = cw[q];
            const uint32_t chunk = (x & 0xffu) | (((x >> 8) & 0xffu) << BITS) | (((x >> 16) & 0xffu) << (2 * BITS)) |
                                   ((x >> 24) << (3 * BITS));
            const int off = q * 4 * BITS, sh = off & 31;
            wd[off >> 5] |= chunk << sh;
            if (sh + 4 * BITS > 32) wd[(off >> 5) + 1] |= chunk >> (32 - sh);
        }
    }
}

template <int T, bool BIG>
__global__ __launch_bounds__(256) void kq_to_affine(const uint8_t* __restrict__ raw, int64_t nblocks, bool vec_ok,
                                                    uint32_t* __restrict__ w, uint16_t* __restrict__ s,
                                                    uint16_t* __restrict__ bias) {
    using P = KQuant<T>;
    constexpr int NB = 256 / P::units, G = 32 / P::gs;
    __shared__ __attribute__((aligned(16))) uint16_t lds[NB * P::bytes / 2];
    const int64_t blk0 = int64_t(blockIdx.x) * NB;
    const int nb = int(min<int64_t>(NB, nblocks - blk0));
    stage_blocks<P::bytes, NB>(lds, raw, blk0, nb, vec_ok);
    const int lb = threadIdx.x / P::units, u = threadIdx.x % P::units;
    if (lb >= nb) return;
    const uint8_t* b = reinterpret_cast<const uint8_t*>(lds) + lb * P::bytes;
    uint32_t cw[8], wd[P::bits];
#pragma unroll
    for (int q = 0; q < 4; q++) kq_codes8<T, BIG>(b, u, 8 * q, cw[2 * q], cw[2 * q + 1]);
    pack_unit<P::bits>(cw, wd);
    const int64_t unit = (blk0 + lb) * P::units + u;
    store_unit<P::bits>(w + unit * P::bits, wd);
#pragma unroll
    for (int j = 0; j < G; j++) {
        uint32_t sb, bb;
        kq_group<T, BIG>(b, u * G + j, sb, bb);
        s[unit * G + j] = uint16_t(sb);
        bias[unit * G + j] = uint16_t(bb);
    }
}

// One byte per value and f16 group factors: the 8-bit affine form the
// prefill kernels take, written straight from the blocks (no packed-code pass
// in between).  Affine types: the code itself, with the scale and bias of
// kq_group (the affine conversion's, so s * byte + bias is its value
// exactly).  IQ4_NL / IQ4_XS: level + 128, with s = f16(factor) and bias
// -128 s (exact), so that s * byte + bias = s * level (the factor's f16
// rounding is the only change; IQ4_NL's d is f16 already).
template <int T, bool BIG>
__global__ __launch_bounds__(256) void kq_to_bytes(const uint8_t* __restrict__ raw, int64_t nblocks, bool vec_ok,
                                                   uint4* __restrict__ w, uint16_t* __restrict__ s,
                                                   uint16_t* __restrict__ bias) {
    using P = KQuant<T>;
    constexpr int NB = 256 / P::units, G = 32 / P::gs;
    __shared__ __attribute__((aligned(16))) uint16_t lds[NB * P::bytes / 2];
    const int64_t blk0 = int64_t(blockIdx.x) * NB;
    const int nb = int(min<int64_t>(NB, nblocks - blk0));
    stage_blocks<P::bytes, NB>(lds, raw, blk0, nb, vec_ok);
    const int lb = threadIdx.x / P::units, u = threadIdx.x % P::units;
    if (lb >= nb) return;
    const uint8_t* b = reinterpret_cast<const uint8_t*>(lds) + lb * P::bytes;
    uint32_t cw[8];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        kq_codes8<T, BIG>(b, u, 8 * q, cw[2 * q], cw[2 * q + 1]);
        if constexpr (P::levels) {
            cw[2 * q] = iq4_level_bytes(cw[2 * q]);
            cw[2 * q + 1] = iq4_level_bytes(cw[2 * q + 1]);
        }
    }
    const int64_t unit = (blk0 + lb) * P::units + u;
    w[2 * unit] = make_uint4(cw[0], cw[1], cw[2], cw[3]);
    w[2 * unit + 1] = make_uint4(cw[4], cw[5], cw[6], cw[7]);
    if constexpr (P::levels) {
        float factor, zero;
        kq_native_group<T, BIG>(b, u, factor, zero);
        const uint32_t sb = f32_to_f16_bits(factor);
        s[unit] = uint16_t(sb);
        bias[unit] = uint16_t(f32_to_f16_bits(-128.f * f16_bits_to_f32(sb)));
    } else {
#pragma unroll
        for (int j = 0; j < G; j++) {
            uint32_t sb, bb;
            kq_group<T, BIG>(b, u * G + j, sb, bb);
            s[unit * G + j] = uint16_t(sb);
            bias[unit * G + j] = uint16_t(bb);
        }
    }
}

// Dense decode by the affine route, f32(scale) * code + f32(bias)
// (convert.rs:81-101); for these types it is also the native definition
// (Q5_1's native decoder d * q + m uses the same unrounded d and m,
// native_quantization.rs:3499-3509).  Lane quarter c of unit lu decodes values
// [8c, 8c + 8); each code converts from its byte lane in one instruction.
template <int T, bool BIG, typename OUT>
__global__ __launch_bounds__(256) void kq_dense(const uint8_t* __restrict__ raw, int64_t nblocks, bool vec_ok,
                                                typename OUT::storage* __restrict__ out) {
    using P = KQuant<T>;
    constexpr int NB = 256 / P::units;
    __shared__ __attribute__((aligned(16))) uint16_t lds[NB * P::bytes / 2];
    const int64_t blk0 = int64_t(blockIdx.x) * NB;
    const int nb = int(min<int64_t>(NB, nblocks - blk0));
    stage_blocks<P::bytes, NB>(lds, raw, blk0, nb, vec_ok);
    const int c = threadIdx.x & 3;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int lu = k * 64 + (threadIdx.x >> 2);
        const int lb = lu / P::units, u = lu % P::units;
        if (lb >= nb) break;
        const uint8_t* b = reinterpret_cast<const uint8_t*>(lds) + lb * P::bytes;
        uint32_t c0, c1;
        kq_codes8<T, BIG>(b, u, 8 * c, c0, c1);
        float scale, bv;
        if constexpr (P::levels) {
            // w = factor * level, level = (level + 128) - 128 exactly; the
            // product is exact in f32, as in the reference (iquant.rs:275, 294),
            // and carries its sign of zero (a zero factor)
            kq_native_group<T, BIG>(b, (u * 32 + 8 * c) / P::gs, scale, bv);
            c0 = iq4_level_bytes(c0);
            c1 = iq4_level_bytes(c1);
        } else {
            uint32_t sb, bb;
            kq_group<T, BIG>(b, (u * 32 + 8 * c) / P::gs, sb, bb);
            scale = f16_bits_to_f32(sb), bv = f16_bits_to_f32(bb);
        }
        float v[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if constexpr (P::levels) {
                v[i] = scale * (float((c0 >> (8 * i)) & 0xffu) - 128.f);
                v[4 + i] = scale * (float((c1 >> (8 * i)) & 0xffu) - 128.f);
            } else {
                v[i] = scale * float((c0 >> (8 * i)) & 0xffu) + bv;
                v[4 + i] = scale * float((c1 >> (8 * i)) & 0xffu) + bv;
            }
        }
        store8<OUT>(out, ((blk0 + lb) * P::units + u) * 32 + 8 * c, v);
    }
}

// ------------------------------------------------- native linear (M small)
//
// NativeQuantizedTensor::linear with transpose = true
// (safemlx/src/native_quantization.rs:741-772, its CPU stream at :858-913):
// y[m, n] = sum_k x[m, k] W[n, k], W decoded by the native definition (Q4_K:
// d sc q - dmin m; Q8_0: d q), accumulated in f32, y in bf16.  No affine
// expansion: the blocks are read once, straight from the payload, and the
// per-group factors are applied to sums of x q and of x (d sc sum(x q) -
// dmin m sum(x)).  kLinRows activation rows per launch.
constexpr int kLinRows = 8;


// An empty asm that makes v opaque to the optimizer: values derived from it
// are recomputed after this point instead of hoisted and kept live, and loads
// whose address depends on it are not issued before it.
__device__ __forceinline__ void opaque(uint32_t& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void opaque(int& v) { asm volatile("" : "+v"(v)); }

// Workgroup layout of the linear kernels: 256 lanes in T teams of S = 256 / T
// lanes; a team takes kTeamRows consecutive rows and splits their columns into
// chunks c = s, s + S, ... (s = the lane's index in the team), so the
// activation values of a chunk are loaded once for all of the team's rows.
// T is picked on the host so that S is about the number of chunks per row.
constexpr int kTeamRows = 4;

// A lane's partial sums, one per (activation row m, team row r).  With one
// activation row (MANY = false) they live in registers; with 2..kLinRows in
// the workgroup's LDS, one word per lane and pair (consecutive lanes in
// consecutive words, so no bank conflicts), which lets the loop over
// activation rows stay rolled with one row's values live at a time.
template <bool MANY>
struct LinAcc {
    float v[kTeamRows];
    __device__ __forceinline__ LinAcc(float*) {}
    __device__ __forceinline__ float& at(int, int r) { return v[r]; }
};
template <>
struct LinAcc<true> {
    float* base;
    __device__ __forceinline__ LinAcc(float* lds) : base(lds + threadIdx.x) {}
    __device__ __forceinline__ float& at(int m, int r) { return base[(m * kTeamRows + r) * 256]; }
};

// Sum of the team's lanes' partials for each (activation row, team row):
// waves reduce by shuffles, lane 0 of each wave writes red, then one lane per
// pair adds the team's waves and writes y.  Ends with a barrier so red can be
// reused.
template <int T, bool MANY>
__device__ __forceinline__ void team_reduce(LinAcc<MANY>& acc, float* red, uint16_t* __restrict__ y, int M, int N,
                                            int row0, bool keep) {
    constexpr int S = 256 / T, WPT = S / 64;  // waves per team
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll 1
    for (int m = 0; m < (MANY ? M : 1); m++) {
#pragma unroll
        for (int r = 0; r < kTeamRows; r++) {
            const float v = wave_sum(acc.at(m, r));
            if (lane == 0) red[wave * kLinRows * kTeamRows + m * kTeamRows + r] = v;
        }
    }
    __syncthreads();
    const int per_team = M * kTeamRows;
    if (tid < T * per_team) {
        const int team = tid / per_team, j = tid % per_team, m = j / kTeamRows, r = j % kTeamRows;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < WPT; w++) v += red[(team * WPT + w) * kLinRows * kTeamRows + m * kTeamRows + r];
        const int n = row0 + team * kTeamRows + r;
        if (n < N) y[int64_t(m) * N + n] = uint16_t(f32_to_bf16_bits(keep ? v : 0.f));
    }
    __syncthreads();
}

// Q4_K: a chunk is one 16-byte run of codes (16 of group 2p in the low
// nibbles, 16 of group 2p + 1 in the high) plus its superblock's 16-byte
// header (d, dmin, the 12 scale/min bytes); rows are whole superblocks of
// 144 = 9 x 16 bytes, so both loads are aligned.  Per row and chunk:
// d sc sum(x q) - dmin m sum(x) for each group, sum(x) shared by the rows;
// sum(x q) by bf16 dot products with the codes as 128 + q.  (Chunks of a
// whole group pair, 32 code bytes, halve the scale decoding but measured
// slower: fewer waves in flight.)
template <bool BIG, int T, bool MANY>
__global__ __launch_bounds__(256) void q4k_linear(uint16_t* __restrict__ y, const uint16_t* __restrict__ x,
                                                  const uint8_t* __restrict__ raw, int M, int N, int K,
                                                  ExpertSel sel) {
    raw = select_expert(raw, sel);
    x += route_row(sel) * K;
    y += route_row(sel) * N;
    const bool keep = route_ok(sel);
    constexpr int S = 256 / T;
    __shared__ float red[4 * kLinRows * kTeamRows];
    __shared__ float lacc[MANY ? kLinRows * kTeamRows * 256 : 1];
    const int s = threadIdx.x % S, team = threadIdx.x / S;
    const int nsb = K / 256, nch = nsb * 8;
    const int64_t row_bytes = int64_t(nsb) * 144;
    for (int row0 = blockIdx.x * T * kTeamRows; row0 < N; row0 += gridDim.x * T * kTeamRows) {
        const int r0 = row0 + team * kTeamRows;
        LinAcc<MANY> acc(lacc);
#pragma unroll 1
        for (int m = 0; m < (MANY ? M : 1); m++)
#pragma unroll
            for (int r = 0; r < kTeamRows; r++) acc.at(m, r) = 0.f;
#pragma unroll 1
        for (int c = s; c < nch; c += S) {
            const int sb = c >> 3, q = c & 7, p = q >> 1;
            uint4 hv[kTeamRows], qv[kTeamRows];
#pragma unroll
            for (int r = 0; r < kTeamRows; r++) {
                const int n = min(r0 + r, N - 1);  // rows past N read row N - 1; their sums are not stored
                const uint8_t* blk = raw + int64_t(n) * row_bytes + sb * 144;
                hv[r] = load_stream16(blk);
                qv[r] = load_stream16(blk + 16 + q * 16);
            }
            float ds[kTeamRows][2], dm[kTeamRows][2];
#pragma unroll
            for (int r = 0; r < kTeamRows; r++) {
                const uint32_t h[4] = {hv[r].x, hv[r].y, hv[r].z, hv[r].w};
                uint32_t sc0, m0, sc1, m1;
                q4k_scale_min(h, 2 * p, sc0, m0);
                q4k_scale_min(h, 2 * p + 1, sc1, m1);
                const float d = f16_bits_to_f32(BIG ? bswap16(h[0] & 0xffffu) : (h[0] & 0xffffu));
                const float dmin = f16_bits_to_f32(BIG ? bswap16(h[0] >> 16) : (h[0] >> 16));
                ds[r][0] = d * float(sc0), dm[r][0] = dmin * float(m0);
                ds[r][1] = d * float(sc1), dm[r][1] = dmin * float(m1);
            }
            const int k0 = sb * 256 + 2 * p * 32 + (q & 1) * 16;  // group 2p; group 2p + 1 at k0 + 32
#pragma unroll 1
            for (int m = 0; m < (MANY ? M : 1); m++) {
                int kk = k0;
                if (MANY) {  // the codes are re-extracted per activation row, not kept live
                    opaque(kk);
#pragma unroll
                    for (int r = 0; r < kTeamRows; r++) opaque(qv[r].x), opaque(qv[r].y), opaque(qv[r].z), opaque(qv[r].w);
                }
                // x words: xw[0..7] = group 2p values (x0, x1) .. (x14, x15), xw[8..15] group 2p + 1
                const uint4* xa = reinterpret_cast<const uint4*>(x + int64_t(m) * K + kk);
                const uint4* xb = reinterpret_cast<const uint4*>(x + int64_t(m) * K + kk + 32);
                const uint4 xv[4] = {xa[0], xa[1], xb[0], xb[1]};
                uint32_t xw[16];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    xw[4 * i] = xv[i].x, xw[4 * i + 1] = xv[i].y, xw[4 * i + 2] = xv[i].z, xw[4 * i + 3] = xv[i].w;
                }
                float sx0 = 0.f, sx1 = 0.f;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    sx0 = dot2_bf16(xw[i], kBf16Ones, sx0);
                    sx1 = dot2_bf16(xw[8 + i], kBf16Ones, sx1);
                }
#pragma unroll
                for (int r = 0; r < kTeamRows; r++) {
                    const uint32_t qw[4] = {qv[r].x, qv[r].y, qv[r].z, qv[r].w};
                    // sum x (128 + q) per group; byte j holds code j of group 2p
                    // (low nibble) and of group 2p + 1 (high nibble)
                    float e0 = 0.f, e1 = 0.f;
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const uint32_t lo2 = __builtin_amdgcn_perm(0u, qw[t], 0x0c010c00u);  // bytes 0, 1 -> halves
                        const uint32_t hi2 = __builtin_amdgcn_perm(0u, qw[t], 0x0c030c02u);  // bytes 2, 3 -> halves
                        e0 = dot2_bf16(xw[2 * t], (lo2 & 0x000f000fu) | kNibbleMagic, e0);
                        e0 = dot2_bf16(xw[2 * t + 1], (hi2 & 0x000f000fu) | kNibbleMagic, e0);
                        e1 = dot2_bf16(xw[8 + 2 * t], ((lo2 >> 4) & 0x000f000fu) | kNibbleMagic, e1);
                        e1 = dot2_bf16(xw[8 + 2 * t + 1], ((hi2 >> 4) & 0x000f000fu) | kNibbleMagic, e1);
                    }
                    const float sxq0 = e0 - 128.f * sx0, sxq1 = e1 - 128.f * sx1;
                    acc.at(m, r) += (ds[r][0] * sxq0 - dm[r][0] * sx0) + (ds[r][1] * sxq1 - dm[r][1] * sx1);
                }
            }
        }
        team_reduce<T, MANY>(acc, red, y, M, N, row0, route_ok(sel));
    }
}

// ------------------------------------- native linear for Q5_K / Q6_K / Q5_1
//
// NativeQuantizedTensor::linear, transpose = true, for the other encodings
// eredu keeps native (safemlx/src/native_quantization.rs:741-772; its Metal
// kernels q5k / q6k / q5_1 _linear_metal, :1320-1400, 1856): y[m, n] =
// sum_k x[m, k] W[n, k] with W decoded in f32 without f16 rounding of the
// group factors -- Q6_K d sc (q - 32), Q5_K d sc q - dmin m, Q5_1 d q + m --
// as those kernels decode.  A workgroup stages the payload of R consecutive
// weight rows (contiguous bytes) through LDS with 16-byte loads; wave w takes
// rows w, w + 4, ... and its lanes split each row's 32-value units.  Per unit
// the codes come from kq_codes8 as byte lanes, are turned into bf16 pairs
// 128 + q by byte permutes, and meet x in v_dot2c_f32_bf16; per group
// sum x q = e - 128 sum x.  Up to kLinRows activation rows per launch.

constexpr int kKqStageVec = 8;  // 16-byte pieces per lane of one staged row group

// Persistent workgroups walk row groups grp, grp + gridDim.x, ...; a full
// group on a 16-byte-aligned payload is fetched into registers one group
// ahead (its loads in flight while the current group is multiplied), a
// ragged or unaligned one is staged with 2-byte loads when its turn comes.
// Sums of x over every group of K are taken once per launch into LDS.
template <int T, bool BIG, bool MANY, int W>
__global__ __launch_bounds__(64 * W) void kq_linear(uint16_t* __restrict__ y, const uint16_t* __restrict__ x,
                                                    const uint8_t* __restrict__ raw, int M, int N, int K, int R,
                                                    bool vec_ok, ExpertSel sel) {
    raw = select_expert(raw, sel);
    x += route_row(sel) * K;
    y += route_row(sel) * N;
    const bool keep = route_ok(sel);
    using P = KQuant<T>;
    constexpr int G = 32 / P::gs, VG = 32 / G, NT = 64 * W;  // groups per unit, values per group
    extern __shared__ __attribute__((aligned(16))) uint16_t kq_lds[];
    const int row_bytes = K / (32 * P::units) * P::bytes, U = K / 32, ngk = K / VG;
    const int gbytes = R * row_bytes;
    float* sxs = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(kq_lds) + ((gbytes + 15) & ~15));
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wpr = R >= W ? 1 : W / R;  // waves per row (R is a power of two)
    __shared__ float red[W * kLinRows];
    const uint32_t c43 = 0x43434343u;
    for (int i = threadIdx.x; i < M * ngk; i += NT) {
        const uint4* xp = reinterpret_cast<const uint4*>(x + int64_t(i / ngk) * K + int64_t(i % ngk) * VG);
        float sx = 0.f;
#pragma unroll
        for (int j = 0; j < VG / 8; j++) {
            const uint4 v = xp[j];
            sx = dot2_bf16(v.x, kBf16Ones, sx);
            sx = dot2_bf16(v.y, kBf16Ones, sx);
            sx = dot2_bf16(v.z, kBf16Ones, sx);
            sx = dot2_bf16(v.w, kBf16Ones, sx);
        }
        sxs[i] = sx;
    }
    const int64_t ngroups = (int64_t(N) + R - 1) / R;
    auto pipelined = [&](int64_t gi) { return vec_ok && (gi + 1) * R <= N; };
    uint4 buf[kKqStageVec];
    auto fetch = [&](int64_t gi) {
        const uint4* src = reinterpret_cast<const uint4*>(raw + gi * gbytes);
#pragma unroll
        for (int i = 0; i < kKqStageVec; i++) {
            const int idx = threadIdx.x + i * NT;
            if (idx < gbytes / 16) buf[i] = load_stream16(src + idx);
        }
    };
    int64_t grp = blockIdx.x;
    if (grp < ngroups && pipelined(grp)) fetch(grp);
    for (; grp < ngroups; grp += gridDim.x) {
        const int64_t n0 = grp * R;
        const int nr = int(min<int64_t>(R, N - n0));
        if (pipelined(grp)) {
#pragma unroll
            for (int i = 0; i < kKqStageVec; i++) {
                const int idx = threadIdx.x + i * NT;
                if (idx < gbytes / 16) reinterpret_cast<uint4*>(kq_lds)[idx] = buf[i];
            }
        } else {
            const uint16_t* src = reinterpret_cast<const uint16_t*>(raw + n0 * row_bytes);
            for (int i = threadIdx.x; i < nr * row_bytes / 2; i += NT) kq_lds[i] = src[i];
        }
        __syncthreads();
        const int64_t next = grp + gridDim.x;
        if (next < ngroups && pipelined(next)) fetch(next);
        // wpr waves per row when the group has fewer rows than waves: each
        // takes every wpr-th run of 64 units, and their sums meet in red
        for (int rb = 0; rb < nr; rb += W / wpr) {
            const int r = rb + wave / wpr, part = wave % wpr;
            const uint8_t* row = reinterpret_cast<const uint8_t*>(kq_lds) + r * row_bytes;
            float acc[kLinRows];
#pragma unroll
            for (int m = 0; m < kLinRows; m++) acc[m] = 0.f;
            for (int u = (r < nr ? part * 64 + lane : U); u < U; u += 64 * wpr) {
                const uint8_t* b = row + (u / P::units) * P::bytes;
                const int uu = u % P::units;
                uint32_t cp[16];  // bf16 pairs (128 + q) of values 2j, 2j + 1
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    uint32_t c0, c1;
                    kq_codes8<T, BIG>(b, uu, 8 * q, c0, c1);
                    if constexpr (P::levels) {
                        // level + 128 (up to 241: exact in bf16, past the 0x43 trick's
                        // range) converted per byte
                        const uint32_t l0 = iq4_level_bytes(c0), l1 = iq4_level_bytes(c1);
                        cp[4 * q] = pack_bf16x2(float(l0 & 0xffu), float((l0 >> 8) & 0xffu));
                        cp[4 * q + 1] = pack_bf16x2(float((l0 >> 16) & 0xffu), float(l0 >> 24));
                        cp[4 * q + 2] = pack_bf16x2(float(l1 & 0xffu), float((l1 >> 8) & 0xffu));
                        cp[4 * q + 3] = pack_bf16x2(float((l1 >> 16) & 0xffu), float(l1 >> 24));
                    } else {
                        cp[4 * q] = __builtin_amdgcn_perm(c43, c0, 0x04010400u);
                        cp[4 * q + 1] = __builtin_amdgcn_perm(c43, c0, 0x04030402u);
                        cp[4 * q + 2] = __builtin_amdgcn_perm(c43, c1, 0x04010400u);
                        cp[4 * q + 3] = __builtin_amdgcn_perm(c43, c1, 0x04030402u);
                    }
                }
                float sc[G], bi[G];
#pragma unroll
                for (int g = 0; g < G; g++) kq_native_group<T, BIG>(b, uu * G + g, sc[g], bi[g]);
#pragma unroll
                for (int m = 0; m < (MANY ? kLinRows : 1); m++) {
                    if (m >= M) break;
                    const uint4* xp = reinterpret_cast<const uint4*>(x + int64_t(m) * K + int64_t(u) * 32);
                    uint32_t xw[16];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const uint4 v = xp[i];
                        xw[4 * i] = v.x, xw[4 * i + 1] = v.y, xw[4 * i + 2] = v.z, xw[4 * i + 3] = v.w;
                    }
#pragma unroll
                    for (int g = 0; g < G; g++) {
                        float e = 0.f;
#pragma unroll
                        for (int j = 0; j < VG / 2; j++) e = dot2_bf16(xw[g * VG / 2 + j], cp[g * VG / 2 + j], e);
                        const float sx = sxs[m * ngk + u * G + g];
                        acc[m] += sc[g] * (e - 128.f * sx) + bi[g] * sx;
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < (MANY ? kLinRows : 1); m++) {
                if (m >= M) break;
                const float v = wave_sum(acc[m]);
                if (wpr == 1) {
                    if (lane == 0 && r < nr) y[int64_t(m) * N + n0 + r] = uint16_t(f32_to_bf16_bits(keep ? v : 0.f));
                } else if (lane == 0) {
                    red[wave * kLinRows + m] = v;
                }
            }
            if (wpr > 1) {
                __syncthreads();
                const int t = threadIdx.x, rr = rb + t / (MANY ? kLinRows : 1), m = t % (MANY ? kLinRows : 1);
                if (t < (W / wpr) * (MANY ? kLinRows : 1) && rr < nr && m < M) {
                    float v = 0.f;
                    for (int q = 0; q < wpr; q++) v += red[((rr - rb) * wpr + q) * kLinRows + m];
                    y[int64_t(m) * N + n0 + rr] = uint16_t(f32_to_bf16_bits(keep ? v : 0.f));
                }
                __syncthreads();
            }
        }
        __syncthreads();  // the rows are read before the next group is staged
    }
}

// ------------------------------------------- native Q4_K linear on MFMA
//
// The same product as q4k_linear for up to 8 activation rows per launch, on
// v_mfma_f32_16x16x32_bf16.  A workgroup takes a tile of 16 weight rows and
// its W waves split each row's superblocks into contiguous ranges.  Per
// superblock, lane (n = lane % 16, kq = lane / 16) loads the 16-byte header
// of tile row n (d, dmin, the 12 scale/min bytes) and code chunks kq and
// kq + 4, 16 bytes each (bytes 16 kq and 64 + 16 kq of the 128 code bytes).
// Chunk 2p + h holds values 16 h .. 16 h + 15 of groups 2p (low nibbles) and
// 2p + 1 (high nibbles), so lane kq sees groups 2a, 2a + 1 (chunk kq) and
// 4 + 2a, 5 + 2a (chunk kq + 4), a = kq / 2, values 16 (kq % 2) .. + 15.
//
// Eight MFMA steps per superblock.  Step s takes chunk cc = s / 4, nibble
// plane o = s % 2 and bytes 8 hb .. 8 hb + 7 (hb = (s / 2) % 2): eight codes of
// group 4 cc + 2a + o as bf16 128 + q, in byte order (B operand).  The four
// lane blocks of one step cover two groups (a = 0, 1), so the A operand
// splits its 16 rows as (a, m), row 8a + m = activation row m, non-zero only
// in the lane blocks of its own a (other lanes read a zero block of LDS).
// Result lane (n, kq) then holds rows 4kq .. 4kq + 3 = (a = kq / 2,
// m = 4 (kq % 2) + i) of the step's group: one accumulator per (cc, o).  Per
// group and row:
//   sum x (d sc q - dmin m) = d sc (t - 128 xs) - dmin m xs,
// t = sum x (128 + q) from the MFMAs, xs = sum x over the group, computed once
// per workgroup while the activations are staged into LDS.
//
// LDS: activation row m at m * xstride (xstride = 2K + 16, so the rows of one
// A read fall in different banks), then xs [M][K / 32] f32, then a zero
// block, then the cross-wave partial sums.
// Launch shapes (waves per workgroup W, superblocks in the load ring D; loads
// run D - 1 superblocks ahead), measured on MI355X at the decode shapes of an
// 8B model with payloads rotating past the caches: rows of 56 superblocks
// (K = 14336) run best with W = 8, D = 2; rows of 16 (K = 4096) with W = 4,
// D = 4 (more workgroups per CU, each wave a longer run).  A 16-row tile is
// the whole grid's unit, so the short rows want the smaller workgroups.
constexpr int kQ4kMaxWaves = 8;
constexpr int kQ4kMaxRows = 8;           // activation rows per launch
constexpr int kQ4kZeroBytes = 512;       // zero block: the largest step offset (336) plus a read

typedef uint32_t q4k_u32x4 __attribute__((ext_vector_type(4)));

struct Q4kMfmaArgs {
    uint16_t* y;
    const uint16_t* x;
    const uint8_t* raw;
    ExpertSel sel;  // raw + the picked expert's offset (none by default)
    int M, N, K;  // M <= kQ4kMaxRows; y [M, ldy] (columns [0, N)), x [M, K]
    int ldy;
    int sbw;      // superblocks per wave
    int xstride;  // LDS bytes per staged activation row
    int xs_lds, zero_lds, red_lds;
};

// One superblock of one lane: the header and its two code chunks.
struct Q4kSb {
    q4k_u32x4 h, c0, c1;
};

// Eight codes of one nibble plane (o = 0 low, 1 high) of bytes b0 .. b7
// (words w0, w1) as bf16 128 + q, in byte order: mask, then byte permutes
// against the constant 0x43 bytes (0x43XX = 128 + XX as bf16).
__device__ __forceinline__ bf16x8 q4k_plane8(uint32_t w0, uint32_t w1, int o) {
    const uint32_t c43 = 0x43434343u;
    const uint32_t l0 = (o ? w0 >> 4 : w0) & 0x0f0f0f0fu;
    const uint32_t l1 = (o ? w1 >> 4 : w1) & 0x0f0f0f0fu;
    q4k_u32x4 p;
    p[0] = __builtin_amdgcn_perm(c43, l0, 0x04010400u);  // [b0, 43, b1, 43]
    p[1] = __builtin_amdgcn_perm(c43, l0, 0x04030402u);  // [b2, 43, b3, 43]
    p[2] = __builtin_amdgcn_perm(c43, l1, 0x04010400u);
    p[3] = __builtin_amdgcn_perm(c43, l1, 0x04030402u);
    return __builtin_bit_cast(bf16x8, p);
}

__device__ __forceinline__ void q4k_retire(const Q4kSb& b) { asm volatile("" ::"v"(b.h), "v"(b.c0), "v"(b.c1)); }

// MREG: result registers per lane that can hold a live activation row (1 when M == 1, else 4).
template <bool BIG, int MREG, int W, int D>
__global__ __launch_bounds__(64 * W) void q4k_mfma_linear(const Q4kMfmaArgs args) {
    static_assert(D >= 2, "the ring needs two superblocks");
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ln = lane & 15, kq = lane >> 4, a = kq >> 1;
    const int M = args.M, N = args.N, K = args.K;
    const int n0 = blockIdx.x * 16;
    const int nsb = K / 256, G = K / 32;
    const uint32_t row_bytes = uint32_t(nsb) * 144u;

    // This wave's superblocks [sb0, sb0 + cnt).
    const int sb0 = min(nsb, wave * args.sbw);
    const int cnt = min(nsb, sb0 + args.sbw) - sb0;

    // Weight loads: rows past N read zero (offsets out of range, fixed step 0).
    const bool row_live = n0 + ln < N;
    const __amdgpu_buffer_rsrc_t wr = raw_rsrc(select_expert(args.raw, args.sel), uint32_t(N) * row_bytes);
    const uint32_t hoff = row_live ? uint32_t(n0 + ln) * row_bytes : kOutOfRange;
    const uint32_t hstep = row_live ? 144u : 0u;
    auto load_sb = [&](Q4kSb& b, int j) __attribute__((always_inline)) {
        // superblocks past the wave's range read zero
        const uint32_t o = j < cnt ? hoff + uint32_t(sb0 + j) * hstep : kOutOfRange;
        b.h = __builtin_bit_cast(q4k_u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, o, 0, 0));
        b.c0 = __builtin_bit_cast(q4k_u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, o + 16u + 16u * kq, 0, 0));
        b.c1 = __builtin_bit_cast(q4k_u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, o + 80u + 16u * kq, 0, 0));
    };

    // Stage x (natural order, row m at m * xstride) and the group sums xs.
    // A round takes NCH 16-byte chunks per thread; four consecutive threads
    // hold the four chunks of one group.  The first round's loads go out
    // before the first D - 1 superblocks of the ring, the stores after them:
    // loads complete in order, so the stores wait for the activations only.
    constexpr int NCH = 4;
    const __amdgpu_buffer_rsrc_t xr = raw_rsrc(args.x + route_row(args.sel) * K, uint32_t(M) * uint32_t(K) * 2u);
    const int cpr = K / 8, total = M * cpr;
    auto stage_load = [&](int c0, q4k_u32x4* v) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            const int c = c0 + i * 64 * W + int(threadIdx.x);
            const int m = c < total ? c / cpr : 0, cc = c - m * cpr;
            const uint32_t off = c < total ? (uint32_t(m) * uint32_t(K) + uint32_t(cc) * 8u) * 2u : kOutOfRange;
            v[i] = __builtin_bit_cast(q4k_u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
        }
    };
    auto stage_store = [&](int c0, const q4k_u32x4* v) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            const int c = c0 + i * 64 * W + int(threadIdx.x);
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < 4; e++) s += bf16_bits_to_f32(v[i][e] & 0xffffu) + bf16_bits_to_f32(v[i][e] >> 16);
            s += __shfl_xor(s, 1);
            s += __shfl_xor(s, 2);
            if (c < total) {
                const int m = c / cpr, cc = c - m * cpr;
                *reinterpret_cast<q4k_u32x4*>(smem + m * args.xstride + cc * 16) = v[i];
                if ((cc & 3) == 0) reinterpret_cast<float*>(smem + args.xs_lds)[m * G + (cc >> 2)] = s;
            }
        }
    };
    q4k_u32x4 xv[NCH];
    stage_load(0, xv);
    Q4kSb ring[D];
#pragma unroll
    for (int d = 0; d < D - 1; d++) load_sb(ring[d], d);
    stage_store(0, xv);
    for (int c0 = NCH * 64 * W; c0 < total; c0 += NCH * 64 * W) {  // wave-uniform trip count
        stage_load(c0, xv);
        stage_store(c0, xv);
    }
    if (int(threadIdx.x) < kQ4kZeroBytes / 16)
        *reinterpret_cast<q4k_u32x4*>(smem + args.zero_lds + threadIdx.x * 16) = q4k_u32x4{0u, 0u, 0u, 0u};
    __syncthreads();

    // A operand: lane row ln = (ln / 8, m = ln % 8), live in the lane blocks of
    // its own a; its 16-byte read for step s of superblock sb is at
    // xa + 512 sb + 256 cc + 64 o + 16 hb.
    const int a_m = ln & 7;
    const bool a_live = (ln >> 3) == a && a_m < M;
    const uint32_t xa = a_live ? uint32_t(a_m * args.xstride + 128 * a + 32 * (kq & 1)) : uint32_t(args.zero_lds);
    const uint32_t xstep = a_live ? 512u : 0u;
    // Group sums of this lane's result rows m_i = 4 (kq % 2) + i (rows past M read row 0:
    // their results are not stored): groups 4cc + 2a + o of superblock sb at
    // xsb[i] + 32 sb + 16 cc + 4 o.
    uint32_t xsb[MREG];
#pragma unroll
    for (int i = 0; i < MREG; i++) {
        const int m = 4 * (kq & 1) + i;
        xsb[i] = uint32_t(args.xs_lds + ((m < M ? m : 0) * G + 2 * a) * 4);
    }

    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const Q4kSb& b, int j) __attribute__((always_inline)) {
        const int sb = sb0 + j;
        // activations first: the LDS reads overlap the unpacking
        const uint32_t xb = xa + uint32_t(sb) * xstep;
        bf16x8 av[8];
#pragma unroll
        for (int s = 0; s < 8; s++)
            av[s] = *reinterpret_cast<const bf16x8*>(smem + xb + 256 * (s >> 2) + 64 * (s & 1) + 16 * ((s >> 1) & 1));
        float xs[MREG][4];
#pragma unroll
        for (int i = 0; i < MREG; i++) {
            const float* p = reinterpret_cast<const float*>(smem + xsb[i] + 32u * uint32_t(sb));
            xs[i][0] = p[0], xs[i][1] = p[1], xs[i][2] = p[4], xs[i][3] = p[5];  // (cc, o) = (0,0) (0,1) (1,0) (1,1)
        }
        f32x4 t[4];
#pragma unroll
        for (int g = 0; g < 4; g++) t[g] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const int cc = s >> 2, o = s & 1, hb = (s >> 1) & 1;
            const q4k_u32x4& cw = cc ? b.c1 : b.c0;
            const bf16x8 bq = q4k_plane8(cw[2 * hb], cw[2 * hb + 1], o);
            t[2 * cc + o] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[s], bq, t[2 * cc + o], 0, 0, 0);
        }
        // Factors of groups 2a + o (bytes 2a + o of the scale words h1, h2) and
        // 4 + 2a + o (low 6 bits from h3, top 2 from h1 / h2): scale_min of
        // convert.rs:429-438.
        const uint32_t h0 = b.h[0];
        const float d = f16_bits_to_f32(BIG ? bswap16(h0 & 0xffffu) : (h0 & 0xffffu));
        const float dmin = f16_bits_to_f32(BIG ? bswap16(h0 >> 16) : (h0 >> 16));
        const uint32_t H1 = b.h[1] >> (16 * a), H2 = b.h[2] >> (16 * a), H3 = b.h[3] >> (16 * a);
#pragma unroll
        for (int o = 0; o < 2; o++) {
            const uint32_t s1 = H1 >> (8 * o), s2 = H2 >> (8 * o), s3 = H3 >> (8 * o);
            const uint32_t sc0 = s1 & 63u, mn0 = s2 & 63u;
            const uint32_t sc1 = (s3 & 15u) | (((s1 >> 6) & 3u) << 4);
            const uint32_t mn1 = ((s3 >> 4) & 15u) | (((s2 >> 6) & 3u) << 4);
            const float ds0 = d * float(sc0), ds1 = d * float(sc1);
            const float be0 = fmaf(-128.f, ds0, -dmin * float(mn0));
            const float be1 = fmaf(-128.f, ds1, -dmin * float(mn1));
#pragma unroll
            for (int i = 0; i < MREG; i++) {
                acc[i] = fmaf(ds0, t[o][i], fmaf(be0, xs[i][o], acc[i]));
                acc[i] = fmaf(ds1, t[2 + o][i], fmaf(be1, xs[i][2 + o], acc[i]));
            }
        }
    };

    // The ring: loads run D - 1 superblocks ahead; each compute sits in a
    // basic block of its own, so the loads issued before it stay there.
    for (int j = 0; j < cnt; j += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            load_sb(ring[(d + D - 1) % D], j + d + D - 1);
            if (j + d < cnt) compute(ring[d], j + d);
            else q4k_retire(ring[d]);
        }
    }

    // Fold the two a halves (lane blocks kq and kq ^ 2 hold the same rows),
    // then sum the waves through LDS in a fixed order.
#pragma unroll
    for (int i = 0; i < MREG; i++) acc[i] += __shfl_xor(acc[i], 32);
    float* red = reinterpret_cast<float*>(smem + args.red_lds);
    if (kq < 2) {
#pragma unroll
        for (int i = 0; i < MREG; i++) {
            const int m = 4 * kq + i;
            if (m < M) red[(wave * kQ4kMaxRows + m) * 16 + ln] = acc[i];
        }
    }
    __syncthreads();
    if (int(threadIdx.x) < 16 * M) {
        const int m = threadIdx.x >> 4, n = threadIdx.x & 15;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < W; w++) v += red[(w * kQ4kMaxRows + m) * 16 + n];
        if (n0 + n < N) args.y[(route_row(args.sel) + m) * args.ldy + n0 + n] =
                uint16_t(f32_to_bf16_bits(route_ok(args.sel) ? v : 0.f));
    }
}

// Q8_0: 34-byte blocks are not 4-byte aligned, so a wave first copies a run
// of up to 256 blocks of its row into LDS (16-byte loads when the run is
// 16-byte aligned, else 2-byte loads), then each lane takes whole blocks.
template <bool BIG>
__global__ __launch_bounds__(256) void q8_0_linear(uint16_t* __restrict__ y, const uint16_t* __restrict__ x,
                                                   const uint8_t* __restrict__ raw, int M, int N, int K,
                                                   ExpertSel sel) {
    raw = select_expert(raw, sel);
    x += route_row(sel) * K;
    y += route_row(sel) * N;
    const bool keep = route_ok(sel);
    constexpr int kRun = 256;
    __shared__ uint16_t lds[4][kRun * 17];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = K / 32;
    uint16_t* mine = lds[wave];
    for (int n = blockIdx.x * 4 + wave; n < N; n += gridDim.x * 4) {
        float acc[kLinRows];
#pragma unroll
        for (int m = 0; m < kLinRows; m++) acc[m] = 0.f;
        for (int b0 = 0; b0 < nb; b0 += kRun) {
            const int cnt = min(kRun, nb - b0);
            const uint8_t* src = raw + (int64_t(n) * nb + b0) * 34;
            __builtin_amdgcn_wave_barrier();
            if ((reinterpret_cast<uintptr_t>(src) & 15u) == 0 && (cnt * 34) % 16 == 0) {
                for (int i = lane; i < cnt * 34 / 16; i += 64)
                    reinterpret_cast<uint4*>(mine)[i] = reinterpret_cast<const uint4*>(src)[i];
            } else {
                for (int i = lane; i < cnt * 17; i += 64) mine[i] = reinterpret_cast<const uint16_t*>(src)[i];
            }
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS stores have landed
            __builtin_amdgcn_wave_barrier();
            for (int lb = lane; lb < cnt; lb += 64) {
                const uint16_t* blk = mine + lb * 17;
                const float d = f16_bits_to_f32(BIG ? bswap16(blk[0]) : blk[0]);
                uint32_t qw[8];
#pragma unroll
                for (int i = 0; i < 8; i++) qw[i] = lds_u32(blk + 1 + 2 * i);
                // codes as q + 128 (sign bit flipped: one unsigned byte convert
                // each), sum x q = sum x (q + 128) - 128 sum x
#pragma unroll
                for (int i = 0; i < 8; i++) qw[i] ^= 0x80808080u;
                const int k0 = (b0 + lb) * 32;
#pragma unroll
                for (int m = 0; m < kLinRows; m++) {
                    if (m >= M) break;
                    const uint4* xa = reinterpret_cast<const uint4*>(x + int64_t(m) * K + k0);
                    float s = 0.f, sx = 0.f;
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const uint4 xv = xa[v];
                        sx = dot2_bf16(xv.x, kBf16Ones, sx);
                        sx = dot2_bf16(xv.y, kBf16Ones, sx);
                        sx = dot2_bf16(xv.z, kBf16Ones, sx);
                        sx = dot2_bf16(xv.w, kBf16Ones, sx);
                        float f[8];
                        bf16x8_to_f32(xv, f);
#pragma unroll
                        for (int j = 0; j < 8; j++) {
                            const int e = v * 8 + j;
                            s = fmaf(f[j], float((qw[e >> 2] >> (8 * (e & 3))) & 0xffu), s);
                        }
                    }
                    acc[m] = fmaf(d, s - 128.f * sx, acc[m]);
                }
            }
        }
#pragma unroll
        for (int m = 0; m < kLinRows; m++) {
            if (m >= M) break;
            const float v = wave_sum(acc[m]);
            if (lane == 0) y[int64_t(m) * N + n] = uint16_t(f32_to_bf16_bits(keep ? v : 0.f));
        }
    }
}

struct Geometry {
    int values, bytes, bits, gs;
    bool affine = true;  // has an affine form (convert.rs:142-152); the IQ4 types do not
};

bool geometry(int type, Geometry& g) {
    switch (type) {  // eredu-gguf/src/format.rs:368-400, convert.rs:142-152
    case EQ_GGML_Q4_0: g = {32, 18, 4, 32}; return true;
    case EQ_GGML_Q4_1: g = {32, 20, 4, 32}; return true;
    case EQ_GGML_Q5_0: g = {32, 22, 5, 32}; return true;
    case EQ_GGML_Q5_1: g = {32, 24, 5, 32}; return true;
    case EQ_GGML_Q8_0: g = {32, 34, 8, 32}; return true;
    case EQ_GGML_Q2_K: g = {256, 84, 2, 16}; return true;
    case EQ_GGML_Q3_K: g = {256, 110, 3, 16}; return true;
    case EQ_GGML_Q4_K: g = {256, 144, 4, 32}; return true;
    case EQ_GGML_Q5_K: g = {256, 176, 5, 32}; return true;
    case EQ_GGML_Q6_K: g = {256, 210, 6, 16}; return true;
    case EQ_GGML_IQ4_NL: g = {32, 18, 4, 32, false}; return true;
    case EQ_GGML_IQ4_XS: g = {256, 136, 4, 32, false}; return true;
    default: return false;
    }
}

// Shared argument checks of the two GGUF entry points (convert.rs:158-176,319-324).
int validate(const uint8_t* raw, int64_t raw_len, int type, int64_t rows, int64_t cols, int endian,
             Geometry& geo, int64_t& nblocks) {
    if (!geometry(type, geo)) {
        set_error("unsupported GGML tensor type " + std::to_string(type) +
                  " (device path covers Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS)");
        return 1;
    }
    if (endian != EQ_ENDIAN_LITTLE && endian != EQ_ENDIAN_BIG) {
        set_error("invalid endian " + std::to_string(endian));
        return 1;
    }
    if (rows <= 0 || cols <= 0) {
        set_error("quantized scalar is invalid: rows and cols must be positive");
        return 1;
    }
    if (cols % geo.gs != 0) {
        set_error("last dimension is not divisible by group size " + std::to_string(geo.gs));
        return 1;
    }
    if (cols % geo.values != 0) {
        set_error("row width " + std::to_string(cols) + " is not divisible by block length " +
                  std::to_string(geo.values));
        return 1;
    }
    if (rows > INT64_MAX / cols) {
        set_error("tensor element count overflows");
        return 1;
    }
    nblocks = rows * cols / geo.values;
    if (raw_len != nblocks * geo.bytes) {
        set_error("payload length does not match descriptor: got " + std::to_string(raw_len) + " bytes, expected " +
                  std::to_string(nblocks * geo.bytes));
        return 1;
    }
    if (!raw) {
        set_error("null payload pointer");
        return 1;
    }
    return 0;
}

// Calls f(type tag, byte-order tag) for the types of KQuant; false, calling
// nothing, for the others.
template <typename F>
bool with_kq(int type, bool big, F&& f) {
    auto go = [&](auto t) {
        if (big)
            f(t, std::true_type{});
        else
            f(t, std::false_type{});
        return true;
    };
    switch (type) {
    case EQ_GGML_Q4_1: return go(std::integral_constant<int, EQ_GGML_Q4_1>{});
    case EQ_GGML_Q5_0: return go(std::integral_constant<int, EQ_GGML_Q5_0>{});
    case EQ_GGML_Q5_1: return go(std::integral_constant<int, EQ_GGML_Q5_1>{});
    case EQ_GGML_Q2_K: return go(std::integral_constant<int, EQ_GGML_Q2_K>{});
    case EQ_GGML_Q3_K: return go(std::integral_constant<int, EQ_GGML_Q3_K>{});
    case EQ_GGML_Q5_K: return go(std::integral_constant<int, EQ_GGML_Q5_K>{});
    case EQ_GGML_Q6_K: return go(std::integral_constant<int, EQ_GGML_Q6_K>{});
    case EQ_GGML_IQ4_NL: return go(std::integral_constant<int, EQ_GGML_IQ4_NL>{});
    case EQ_GGML_IQ4_XS: return go(std::integral_constant<int, EQ_GGML_IQ4_XS>{});
    default: return false;
    }
}

// The convert kernels of an affine type (geometry checked by the caller).
void launch_convert_affine(int ggml_type, bool big, const uint8_t* raw, int64_t nblocks, bool vec_ok,
                           uint32_t* weights, uint16_t* scales, uint16_t* biases, hipStream_t st) {
    uint4* w4 = reinterpret_cast<uint4*>(weights);
    if (with_kq(ggml_type, big, [&](auto t, auto b) {
            constexpr int T = decltype(t)::value;
            constexpr int NB = 256 / KQuant<T>::units;
            if constexpr (!KQuant<T>::levels)
                kq_to_affine<T, decltype(b)::value><<<dim3(unsigned((nblocks + NB - 1) / NB)), 256, 0, st>>>(
                    raw, nblocks, vec_ok, weights, scales, biases);
        }))
        return;
    if (ggml_type == EQ_GGML_Q4_K) {
        const int64_t ngroups = nblocks * 8;
        const dim3 grid(unsigned((ngroups + 255) / 256));
        if (big)
            q4k_to_affine<true><<<grid, 256, 0, st>>>(raw, ngroups, vec_ok, w4, scales, biases);
        else
            q4k_to_affine<false><<<grid, 256, 0, st>>>(raw, ngroups, vec_ok, w4, scales, biases);
    } else {
        const dim3 grid(unsigned((nblocks + kBlocksPerWG - 1) / kBlocksPerWG));
        if (ggml_type == EQ_GGML_Q4_0) {
            if (big)
                q4_0_to_affine<true><<<grid, 256, 0, st>>>(raw, nblocks, vec_ok, w4, scales, biases);
            else
                q4_0_to_affine<false><<<grid, 256, 0, st>>>(raw, nblocks, vec_ok, w4, scales, biases);
        } else {
            if (big)
                q8_0_to_affine<true><<<grid, 256, 0, st>>>(raw, nblocks, vec_ok, w4, scales, biases);
            else
                q8_0_to_affine<false><<<grid, 256, 0, st>>>(raw, nblocks, vec_ok, w4, scales, biases);
        }
    }
}

// Native linear at M > kLinRows on the matrix cores: a slice of weight rows
// at a time is converted to the affine triple (convert_affine, f16 group
// factors; 5- and 6-bit codes and IQ4 levels as bytes, kq_to_bytes) in the
// stream's workspace and
// multiplied by the affine prefill kernels, writing its columns of y.  The affine route is the dense fallback of the
// reference's native linear on its non-Metal backends for Q5_K / Q6_K
// (native_quantization.rs:846-862 via IQuantTensor::dequantize_f32); for
// Q4_K, Q5_1 and Q8_0 it differs from the native decoders only by the f16
// rounding of the group factors (none for Q5_1, and for Q8_0 only when
// -128 d overflows f16).  False, launching nothing, when the shape does not
// suit the prefill kernels or no workspace can be had.
bool launch_native_prefill(int ggml_type, bool big, const Geometry& geo, uint16_t* y, const uint16_t* x,
                           const uint8_t* raw, int64_t M, int64_t N, int64_t K, hipStream_t st) {
    if (N % 128 != 0 || K % 64 != 0 || !aligned(y, 8)) return false;
    // one byte per value for the widths the matrix-core kernel takes as bytes
    // (Q5_1 / Q5_K / Q6_K) and for the IQ4 levels: kq_to_bytes
    const bool as_bytes = !geo.affine || (geo.bits != 4 && geo.bits != 8);
    const int bits = as_bytes ? 8 : geo.bits;
    const int64_t row_bytes = K / geo.values * geo.bytes;
    const int64_t wbytes_row = K * bits / 8, pbytes_row = K / geo.gs * 2;
    // rows per slice: the slice's triple within 128 MiB (a 4096 x 14336
    // projection's in one slice at every width), a multiple of 256 rows
    int64_t nc = (int64_t(128) << 20) / (wbytes_row + 2 * pbytes_row) / 256 * 256;
    nc = nc < 256 ? 256 : nc;
    nc = nc > N ? N : nc;
    // slices of equal size (a short last slice would leave most CUs idle)
    const int64_t nslices = (N + nc - 1) / nc;
    nc = ((N + nslices - 1) / nslices + 255) / 256 * 256;
    nc = nc > N ? N : nc;
    auto up = [](size_t v) { return (v + 255) & ~size_t(255); };
    const size_t wsz = up(size_t(nc * wbytes_row)), psz = up(size_t(nc * pbytes_row));
    const size_t triple = wsz + 2 * psz;
    // behind the triple: the 2/3/5/6-bit path's byte codes and split-K partials
    const size_t rest = size_t(nc) * size_t(K) + size_t(4) * size_t(M) * size_t(nc) * 4u + 512;
    size_t want = triple + rest;
    char* base = static_cast<char*>(ws_acquire(nullptr, want, st));
    if (!base) base = static_cast<char*>(ws_acquire(nullptr, want = triple, st));
    if (!base) return false;
    uint32_t* w = reinterpret_cast<uint32_t*>(base);
    uint16_t* s = reinterpret_cast<uint16_t*>(base + wsz);
    uint16_t* b = reinterpret_cast<uint16_t*>(base + wsz + psz);
    const WsSource tail{base + triple, want - triple, nullptr};
    const bool vec_ok = aligned(raw, 16);
    for (int64_t n0 = 0; n0 < N; n0 += nc) {
        const int64_t ncs = N - n0 < nc ? N - n0 : nc;
        const uint8_t* rs = raw + n0 * row_bytes;
        const int64_t nb = ncs * K / geo.values;
        const bool v16 = vec_ok && (n0 * row_bytes) % 16 == 0;
        if (!as_bytes) {
            launch_convert_affine(ggml_type, big, rs, nb, v16, w, s, b, st);
        } else if (!with_kq(ggml_type, big, [&](auto t, auto bt) {
                       constexpr int T = decltype(t)::value;
                       constexpr int NB = 256 / KQuant<T>::units;
                       kq_to_bytes<T, decltype(bt)::value><<<dim3(unsigned((nb + NB - 1) / NB)), 256, 0, st>>>(
                           rs, nb, v16, reinterpret_cast<uint4*>(w), s, b);
                   })) {
            return false;
        }
        if (!launch_qmm_mfma(bits, geo.gs, EQ_DTYPE_F16, y + n0, x, w, s, b, int(M), int(ncs), int(K), &tail, st,
                             int(N)))
            return false;
    }
    return true;
}

}  // namespace
}  // namespace eq

using namespace eq;

extern "C" int eq_gguf_convert_affine(uint32_t* weights, uint16_t* scales, uint16_t* biases, const uint8_t* raw,
                                      int64_t raw_len, int ggml_type, int64_t rows, int64_t cols, int endian,
                                      eq_stream_t stream) {
    clear_error();
    Geometry geo;
    int64_t nblocks;
    if (validate(raw, raw_len, ggml_type, rows, cols, endian, geo, nblocks)) return 1;
    if (!geo.affine) {
        set_error("tensor encoding has no affine conversion (GGML type " + std::to_string(ggml_type) + ")");
        return 1;
    }
    if (!weights || !scales || !biases) {
        set_error("null output pointer");
        return 1;
    }
    if (!aligned(weights, 16) || !aligned(scales, 2) || !aligned(biases, 2)) {
        set_error("weights must be 16-byte aligned and scales/biases 2-byte aligned");
        return 1;
    }
    launch_convert_affine(ggml_type, endian == EQ_ENDIAN_BIG, raw, nblocks, aligned(raw, 16), weights, scales,
                          biases, reinterpret_cast<hipStream_t>(stream));
    return check_launch("gguf convert_affine");
}

namespace {
template <typename OUT>
void launch_dense(int type, bool big, bool native, const uint8_t* raw, int64_t nblocks, bool vec_ok,
                  typename OUT::storage* out, hipStream_t st) {
    if (with_kq(type, big, [&](auto t, auto b) {
            constexpr int T = decltype(t)::value;
            constexpr int NB = 256 / KQuant<T>::units;
            kq_dense<T, decltype(b)::value, OUT><<<dim3(unsigned((nblocks + NB - 1) / NB)), 256, 0, st>>>(
                raw, nblocks, vec_ok, out);
        }))
        return;
    if (type == EQ_GGML_Q4_K) {
        const int64_t nq = nblocks * 32;  // 8 groups x 4 quarters per superblock
        const dim3 grid(unsigned((nq + 255) / 256));
        if (big) {
            if (native) q4k_dense<true, true, OUT><<<grid, 256, 0, st>>>(raw, nq, vec_ok, out);
            else q4k_dense<true, false, OUT><<<grid, 256, 0, st>>>(raw, nq, vec_ok, out);
        } else {
            if (native) q4k_dense<false, true, OUT><<<grid, 256, 0, st>>>(raw, nq, vec_ok, out);
            else q4k_dense<false, false, OUT><<<grid, 256, 0, st>>>(raw, nq, vec_ok, out);
        }
        return;
    }
    const dim3 grid(unsigned((nblocks + kBlocksPerWG - 1) / kBlocksPerWG));
    if (type == EQ_GGML_Q4_0) {
        if (big) q4_0_dense<true, OUT><<<grid, 256, 0, st>>>(raw, nblocks, vec_ok, out);
        else q4_0_dense<false, OUT><<<grid, 256, 0, st>>>(raw, nblocks, vec_ok, out);
    } else {
        if (big) {
            if (native) q8_0_dense<true, true, OUT><<<grid, 256, 0, st>>>(raw, nblocks, vec_ok, out);
            else q8_0_dense<true, false, OUT><<<grid, 256, 0, st>>>(raw, nblocks, vec_ok, out);
        } else {
            if (native) q8_0_dense<false, true, OUT><<<grid, 256, 0, st>>>(raw, nblocks, vec_ok, out);
            else q8_0_dense<false, false, OUT><<<grid, 256, 0, st>>>(raw, nblocks, vec_ok, out);
        }
    }
}

// LDS layout of q4k_mfma_linear for mc activation rows of length K; returns
// the total bytes.
int64_t q4k_mfma_layout(int64_t K, int mc, Q4kMfmaArgs& a) {
    const int64_t xstride = 2 * K + 16;
    int64_t off = mc * xstride;
    a.xstride = int(xstride);
    a.xs_lds = int(off);
    off += int64_t(mc) * (K / 32) * 4;
    a.zero_lds = int(off);
    off += kQ4kZeroBytes;
    a.red_lds = int(off);
    off += int64_t(kQ4kMaxWaves) * kQ4kMaxRows * 16 * 4;
    return off;
}

// LDS available to one workgroup on the current device (cached per device).
int lds_limit() {
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

// Native Q4_K linear on MFMA: activation rows in chunks of at most
// kQ4kMaxRows (fewer when their staged rows would not fit in LDS), weight rows
// in chunks of < 2^31 payload bytes (32-bit buffer offsets).  False, launching
// nothing, when even one activation row does not fit in LDS.
bool launch_q4k_mfma(uint16_t* y, const uint16_t* x, const uint8_t* raw, int64_t M, int64_t N, int64_t K, bool big,
                     hipStream_t st, ExpertSel sel = ExpertSel{}) {
    Q4kMfmaArgs a{};
    a.sel = sel;
    int mcap = kQ4kMaxRows;
    while (mcap > 0 && q4k_mfma_layout(K, mcap, a) > lds_limit()) mcap--;
    if (mcap == 0) return false;
    const int64_t nsb = K / 256, row_bytes = nsb * 144;
    int64_t rows_cap = ((int64_t(1) << 31) - 1) / row_bytes / 16 * 16;
    if (rows_cap < 16 || (sel.ids && rows_cap < N)) return false;
    for (int64_t m0 = 0; m0 < M; m0 += mcap) {
        const int mc = int(M - m0 < mcap ? M - m0 : mcap);
        const int lds = int(q4k_mfma_layout(K, mc, a));
        for (int64_t n0 = 0; n0 < N; n0 += rows_cap) {
            const int64_t nc = N - n0 < rows_cap ? N - n0 : rows_cap;
            a.y = y + m0 * N + n0;
            a.x = x + m0 * K;
            a.raw = raw + n0 * row_bytes;
            a.M = mc, a.N = int(nc), a.K = int(K), a.ldy = int(N);
            const bool wide = nsb >= 32;  // W = 8, D = 2; else W = 4, D = 4
            const int W = wide ? 8 : 4;
            a.sbw = int((nsb + W - 1) / W);
            auto go = [&](auto kernel) {
                // (a refusal surfaces as a launch error)
                if (lds > 65536)
                    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, lds);
                kernel<<<dim3(unsigned((nc + 15) / 16), unsigned(sel.routes)), dim3(64 * W), size_t(lds), st>>>(a);
            };
            auto pick = [&](auto big_tag) {
                constexpr bool B = decltype(big_tag)::value;
                if (wide) {
                    if (mc == 1) go(q4k_mfma_linear<B, 1, 8, 2>);
                    else go(q4k_mfma_linear<B, 4, 8, 2>);
                } else {
                    if (mc == 1) go(q4k_mfma_linear<B, 1, 4, 4>);
                    else go(q4k_mfma_linear<B, 4, 4, 4>);
                }
            };
            if (big) pick(std::true_type{});
            else pick(std::false_type{});
        }
    }
    return true;
}
}  // namespace

namespace eq {
namespace {
// GGML type 39 (MXFP4) -> MLX MXFP4 (eredu-gguf/src/convert.rs:247-276): block
// = 1 E8M0 byte + 16 code bytes, low nibbles values 0..15, high nibbles
// 16..31; out: the scale byte and 4 words of 8 codes each, LSB-first.  One
// thread per block (byte loads: 17-byte blocks are not aligned).
__global__ __launch_bounds__(256) void mxfp4_from_ggml(uint32_t* __restrict__ w, uint8_t* __restrict__ s,
                                                      const uint8_t* __restrict__ raw, int64_t nblocks) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= nblocks) return;
    const uint8_t* b = raw + i * 17;
    s[i] = b[0];
    uint32_t lo[2] = {0u, 0u}, hi[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint32_t q = b[1 + j];
        lo[j >> 3] |= (q & 15u) << (4 * (j & 7));
        hi[j >> 3] |= (q >> 4) << (4 * (j & 7));
    }
    w[i * 4 + 0] = lo[0];
    w[i * 4 + 1] = lo[1];
    w[i * 4 + 2] = hi[0];
    w[i * 4 + 3] = hi[1];
}
}  // namespace
}  // namespace eq

extern "C" int eq_gguf_convert_mxfp4(uint32_t* weights, uint8_t* scales, const uint8_t* raw, int64_t raw_len,
                                     int64_t rows, int64_t cols, eq_stream_t stream) {
    clear_error();
    if (rows < 0 || cols < 0 || cols % 32 != 0) {
        set_error("MXFP4 row width is not divisible by 32");
        return 1;
    }
    const int64_t nblocks = rows * (cols / 32);
    if (raw_len != nblocks * 17) {
        set_error("payload length does not match descriptor");
        return 1;
    }
    if (nblocks == 0) return 0;
    if (!weights || !scales || !raw) {
        set_error("null pointer argument");
        return 1;
    }
    if ((nblocks + 255) / 256 > INT32_MAX) {
        set_error("tensor too large");
        return 1;
    }
    mxfp4_from_ggml<<<dim3(unsigned((nblocks + 255) / 256)), dim3(256), 0, reinterpret_cast<hipStream_t>(stream)>>>(
        weights, scales, raw, nblocks);
    return check_launch("gguf convert (mxfp4)");
}

extern "C" int eq_gguf_dequantize(void* out, const uint8_t* raw, int64_t raw_len, int ggml_type, int64_t rows,
                                  int64_t cols, int endian, int definition, int out_dtype, eq_stream_t stream) {
    clear_error();
    Geometry geo;
    int64_t nblocks;
    if (validate(raw, raw_len, ggml_type, rows, cols, endian, geo, nblocks)) return 1;
    if (definition != EQ_DEQUANT_AFFINE && definition != EQ_DEQUANT_NATIVE) {
        set_error("invalid dequant definition " + std::to_string(definition));
        return 1;
    }
    if (out_dtype != EQ_DTYPE_BF16 && out_dtype != EQ_DTYPE_F32) {
        set_error("dense GGUF output must be bf16 or f32");
        return 1;
    }
    if (!out || !aligned(out, 16)) {
        set_error("output must be a non-null 16-byte aligned pointer");
        return 1;
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const bool vec_ok = aligned(raw, 16);
    const bool big = endian == EQ_ENDIAN_BIG;
    const bool native = definition == EQ_DEQUANT_NATIVE;
    if (out_dtype == EQ_DTYPE_BF16)
        launch_dense<BF16T>(ggml_type, big, native, raw, nblocks, vec_ok, static_cast<uint16_t*>(out), st);
    else
        launch_dense<F32T>(ggml_type, big, native, raw, nblocks, vec_ok, static_cast<float*>(out), st);
    return check_launch("gguf dequantize");
}

namespace eq {
namespace {

// Rows of a tensor's blocks picked by device token ids into a contiguous
// buffer, one workgroup per token (16-byte copies when every row starts
// 16-byte aligned).  An id outside [0, rows) copies nothing; its output row
// is cleared after the decode by embedding_clear_rows.
__global__ __launch_bounds__(256) void embedding_gather_rows(uint8_t* __restrict__ dst,
                                                             const uint8_t* __restrict__ raw,
                                                             const int32_t* __restrict__ tokens, int64_t rows,
                                                             int64_t row_bytes, bool vec) {
    const int64_t t = blockIdx.x;
    const int32_t id = tokens[t];
    if (id < 0 || id >= rows) return;
    const uint8_t* src = raw + int64_t(id) * row_bytes;
    uint8_t* d = dst + t * row_bytes;
    if (vec) {
        const int64_t n16 = row_bytes / 16;
        for (int64_t i = threadIdx.x; i < n16; i += blockDim.x)
            reinterpret_cast<uint4*>(d)[i] = reinterpret_cast<const uint4*>(src)[i];
    } else {
        for (int64_t i = threadIdx.x; i < row_bytes; i += blockDim.x) d[i] = src[i];
    }
}

// Zeroes (+0) the output row of every id outside [0, rows).
template <typename E>
__global__ __launch_bounds__(256) void embedding_clear_rows(E* __restrict__ out, const int32_t* __restrict__ tokens,
                                                            int64_t rows, int64_t cols) {
    const int64_t t = blockIdx.x;
    const int32_t id = tokens[t];
    if (id >= 0 && id < rows) return;
    for (int64_t i = threadIdx.x; i < cols; i += blockDim.x) out[t * cols + i] = E(0);
}

}  // namespace
}  // namespace eq

extern "C" int eq_gguf_embedding(void* out, const uint8_t* raw, int64_t raw_len, int ggml_type, int64_t rows,
                                 int64_t cols, const int32_t* tokens, int64_t n_tokens, int endian, int out_dtype,
                                 eq_stream_t stream) {
    clear_error();
    Geometry geo;
    int64_t nblocks;
    if (validate(raw, raw_len, ggml_type, rows, cols, endian, geo, nblocks)) return 1;
    if (out_dtype != EQ_DTYPE_BF16 && out_dtype != EQ_DTYPE_F32) {
        set_error("embedding output must be bf16 or f32");
        return 1;
    }
    if (n_tokens < 0 || n_tokens > INT32_MAX) {
        set_error("token count must be in [0, 2^31 - 1]");
        return 1;
    }
    if (n_tokens == 0) return 0;
    if (!out || !tokens || !aligned(out, 16) || !aligned(tokens, 4)) {
        set_error("out must be a non-null 16-byte aligned pointer and tokens a non-null int32 pointer");
        return 1;
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int64_t row_bytes = cols / geo.values * geo.bytes;
    uint8_t* picked = static_cast<uint8_t*>(ws_acquire(nullptr, size_t(n_tokens) * size_t(row_bytes), st));
    if (!picked) {
        set_error("could not obtain " + std::to_string(n_tokens * row_bytes) +
                  " bytes of workspace for the picked rows (first call on a stream under graph capture?)");
        return 1;
    }
    const bool vec = aligned(raw, 16) && row_bytes % 16 == 0;
    embedding_gather_rows<<<dim3(unsigned(n_tokens)), 256, 0, st>>>(picked, raw, tokens, rows, row_bytes, vec);
    const bool big = endian == EQ_ENDIAN_BIG;
    const int64_t nb = n_tokens * (cols / geo.values);
    if (out_dtype == EQ_DTYPE_BF16) {
        launch_dense<BF16T>(ggml_type, big, true, picked, nb, row_bytes % 16 == 0, static_cast<uint16_t*>(out), st);
        embedding_clear_rows<uint16_t><<<dim3(unsigned(n_tokens)), 256, 0, st>>>(static_cast<uint16_t*>(out), tokens,
                                                                                 rows, cols);
    } else {
        launch_dense<F32T>(ggml_type, big, true, picked, nb, row_bytes % 16 == 0, static_cast<float*>(out), st);
        embedding_clear_rows<float><<<dim3(unsigned(n_tokens)), 256, 0, st>>>(static_cast<float*>(out), tokens, rows,
                                                                              cols);
    }
    return check_launch("gguf embedding");
}

namespace eq {
namespace {

// The native linear's launches after argument checks: `sel` picks the
// matrix of an expert bank on the device (none: raw is the matrix).
int native_linear_run(void* y, const void* x, const uint8_t* raw, int ggml_type, const Geometry& geo, bool kq,
                      int64_t M, int64_t N, int64_t K, bool big, ExpertSel sel, hipStream_t st) {
    if (M > kLinRows && !sel.ids && launch_native_prefill(ggml_type, big, geo, static_cast<uint16_t*>(y),
                                        static_cast<const uint16_t*>(x), raw, M, N, K, st))
        return check_launch("gguf linear (prefill)");
    if (kq) {
        // R weight rows per workgroup, staged whole in LDS: 8 while they fit
        // in 64 KB, fewer for long rows, one row up to the device's LDS
        // R weight rows per group: as many as fit the register stage (up to
        // 8, kKqStageVec 16-byte pieces per lane), then sums of x for up to
        // kLinRows activation rows behind them in LDS.  A row longer than the
        // stage takes groups of one row staged with 2-byte loads.
        constexpr int W = 4;
        const int64_t row_bytes = K / geo.values * geo.bytes;
        const int64_t stage = int64_t(kKqStageVec) * 16 * 64 * W;
        int R = 8;
        while (R > 1 && R * row_bytes > stage) R /= 2;
        const int64_t rows_lds = (R * row_bytes + 15) / 16 * 16;
        const int64_t sx_row = (K / geo.gs) * 4;  // sums of x of one activation row
        if (rows_lds + sx_row > lds_limit()) {
            set_error("native linear: one weight row (" + std::to_string(row_bytes) + " bytes) exceeds LDS");
            return 1;
        }
        int mcap = kLinRows;  // activation rows per launch: as many as LDS holds, up to kLinRows
        while (rows_lds + mcap * sx_row > lds_limit()) mcap--;
        const bool vec_ok = aligned(raw, 16) && sel.stride % 16 == 0 && (R * row_bytes) % 16 == 0 &&
                            R * row_bytes <= stage;
        const int64_t groups = (N + R - 1) / R;
        const int64_t cap = int64_t(device_cu_count()) * 4;  // 2, 8, 32 per CU measured slower
        const unsigned grid = unsigned(groups < cap ? groups : cap);
        if (!with_kq(ggml_type, big, [&](auto t, auto b) {
                constexpr int T = decltype(t)::value;
                if constexpr (T == EQ_GGML_Q5_1 || T == EQ_GGML_Q5_K || T == EQ_GGML_Q6_K || T == EQ_GGML_IQ4_NL ||
                              T == EQ_GGML_IQ4_XS) {
                    constexpr bool B = decltype(b)::value;
                    for (int64_t m0 = 0; m0 < M; m0 += mcap) {
                        const int mc = int(M - m0 < mcap ? M - m0 : mcap);
                        const int lds = int(rows_lds + mc * sx_row);
                        auto go = [&](auto kernel) {
                            if (lds > 65536)
                                (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                          hipFuncAttributeMaxDynamicSharedMemorySize, lds);
                            kernel<<<dim3(grid, unsigned(sel.routes)), 64 * W, size_t(lds), st>>>(
                                static_cast<uint16_t*>(y) + m0 * N,
                                                                  static_cast<const uint16_t*>(x) + m0 * K, raw, mc,
                                                                  int(N), int(K), R, vec_ok, sel);
                        };
                        if (mc == 1)
                            go(kq_linear<T, B, false, W>);
                        else
                            go(kq_linear<T, B, true, W>);
                    }
                }
            }))
            return 1;
        return check_launch("gguf linear");
    }
    if (ggml_type == EQ_GGML_Q4_K &&
        launch_q4k_mfma(static_cast<uint16_t*>(y), static_cast<const uint16_t*>(x), raw, M, N, K, big, st, sel))
        return check_launch("gguf linear");
    // Q4_K: 32-code chunks per row -> teams per workgroup; Q8_0: a wave per row
    const int64_t nch = K / 32;
    const int teams = nch <= 64 ? 4 : nch <= 128 ? 2 : 1;
    const int64_t rows_per_wg = ggml_type == EQ_GGML_Q4_K ? int64_t(teams) * kTeamRows : 4;
    const int64_t wgs = (N + rows_per_wg - 1) / rows_per_wg;
    const unsigned grid = unsigned(wgs < 8192 ? wgs : 8192);
    for (int64_t m0 = 0; m0 < M; m0 += kLinRows) {
        const int mc = int(M - m0 < kLinRows ? M - m0 : kLinRows);
        uint16_t* yy = static_cast<uint16_t*>(y) + m0 * N;
        const uint16_t* xx = static_cast<const uint16_t*>(x) + m0 * K;
        const int n = int(N), k = int(K);
#define EQ_LIN_MANY(KERNEL, T, MANY)                                                        \
    (big ? KERNEL<true, T, MANY><<<dim3(grid, unsigned(sel.routes)), 256, 0, st>>>(yy, xx, raw, mc, n, k, sel) \
         : KERNEL<false, T, MANY><<<dim3(grid, unsigned(sel.routes)), 256, 0, st>>>(yy, xx, raw, mc, n, k, sel))
#define EQ_LIN_T(KERNEL, T) (mc == 1 ? EQ_LIN_MANY(KERNEL, T, false) : EQ_LIN_MANY(KERNEL, T, true))
#define EQ_LIN(KERNEL) \
    (teams == 4 ? EQ_LIN_T(KERNEL, 4) : teams == 2 ? EQ_LIN_T(KERNEL, 2) : EQ_LIN_T(KERNEL, 1))
        if (ggml_type == EQ_GGML_Q4_K) {
            EQ_LIN(q4k_linear);
        } else {
            if (big) q8_0_linear<true><<<dim3(grid, unsigned(sel.routes)), 256, 0, st>>>(yy, xx, raw, mc, n, k, sel);
            else q8_0_linear<false><<<dim3(grid, unsigned(sel.routes)), 256, 0, st>>>(yy, xx, raw, mc, n, k, sel);
        }
#undef EQ_LIN_MANY
#undef EQ_LIN_T
#undef EQ_LIN
    }
    return check_launch("gguf linear");
}

}  // namespace
}  // namespace eq

extern "C" int eq_gguf_linear(void* y, const void* x, const uint8_t* raw, int64_t raw_len, int ggml_type, int64_t M,
                              int64_t N, int64_t K, int endian, int x_dtype, eq_stream_t stream) {
    clear_error();
    const bool kq = ggml_type == EQ_GGML_Q5_1 || ggml_type == EQ_GGML_Q5_K || ggml_type == EQ_GGML_Q6_K ||
                    ggml_type == EQ_GGML_IQ4_NL || ggml_type == EQ_GGML_IQ4_XS;
    if (ggml_type != EQ_GGML_Q4_K && ggml_type != EQ_GGML_Q8_0 && !kq) {
        set_error("native GGUF linear covers Q4_K, Q5_K, Q6_K, Q5_1, Q8_0, IQ4_NL and IQ4_XS");
        return 1;
    }
    Geometry geo;
    int64_t nblocks;
    if (validate(raw, raw_len, ggml_type, N, K, endian, geo, nblocks)) return 1;
    if (x_dtype != EQ_DTYPE_BF16) {
        set_error("native GGUF linear takes bf16 activations");
        return 1;
    }
    if (M < 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) {
        set_error("dimension exceeds 2^31 - 1");
        return 1;
    }
    if (M == 0) return 0;
    if (!y || !x) {
        set_error("null pointer argument");
        return 1;
    }
    if (!aligned(x, 16) || (ggml_type == EQ_GGML_Q4_K && !aligned(raw, 16))) {
        set_error("x (and a Q4_K payload) must be 16-byte aligned");
        return 1;
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const bool big = endian == EQ_ENDIAN_BIG;
    return native_linear_run(y, x, raw, ggml_type, geo, kq, M, N, K, big, ExpertSel{}, st);
}

namespace eq {
namespace {

// Routes at or below this count take one launch of the native linear
// kernels (a grid row per route, the route's expert picked on the device);
// above it the bank is re-packed
// once and the routes run as one gathered (grouped when sorted) matrix
// product.
constexpr int64_t kGroupedCopyRoutes = 16;

}  // namespace
}  // namespace eq

extern "C" int eq_gguf_grouped_linear(void* y, const void* x, const uint8_t* raw, int64_t raw_len, int ggml_type,
                                      int64_t experts, int64_t N, int64_t K, const int32_t* ids, int64_t routes,
                                      int endian, int x_dtype, bool sorted_ids, eq_stream_t stream) {
    clear_error();
    const bool native = ggml_type == EQ_GGML_Q4_K || ggml_type == EQ_GGML_Q8_0 || ggml_type == EQ_GGML_Q5_1 ||
                        ggml_type == EQ_GGML_Q5_K || ggml_type == EQ_GGML_Q6_K || ggml_type == EQ_GGML_IQ4_NL ||
                        ggml_type == EQ_GGML_IQ4_XS;
    if (!native) {
        set_error("native GGUF grouped linear covers Q4_K, Q5_K, Q6_K, Q5_1, Q8_0, IQ4_NL and IQ4_XS");
        return 1;
    }
    if (experts <= 0 || N <= 0 || experts > INT32_MAX || N > INT32_MAX || K > INT32_MAX ||
        experts * N > INT64_MAX / (K > 0 ? K : 1)) {
        set_error("invalid expert bank shape");
        return 1;
    }
    Geometry geo;
    int64_t nblocks;
    if (validate(raw, raw_len, ggml_type, experts * N, K, endian, geo, nblocks)) return 1;
    if (x_dtype != EQ_DTYPE_BF16) {
        set_error("native GGUF grouped linear takes bf16 activations");
        return 1;
    }
    if (routes < 0 || routes > INT32_MAX) {
        set_error("route count must be in [0, 2^31 - 1]");
        return 1;
    }
    if (routes == 0) return 0;
    if (!y || !x || !ids || !aligned(ids, 4)) {
        set_error("null pointer argument");
        return 1;
    }
    if (!aligned(x, 16) || !aligned(y, 8) || (ggml_type == EQ_GGML_Q4_K && !aligned(raw, 16))) {
        set_error("x (and a Q4_K payload) must be 16-byte and y 8-byte aligned");
        return 1;
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const bool big = endian == EQ_ENDIAN_BIG;
    const int64_t row_bytes = K / geo.values * geo.bytes, matrix_bytes = N * row_bytes;
    uint16_t* yy = static_cast<uint16_t*>(y);
    const uint16_t* xx = static_cast<const uint16_t*>(x);
    if (routes <= kGroupedCopyRoutes) {
        // decode: one launch of the native M = 1 kernels, route r = grid row r,
        // its expert picked on the device
        if (native_linear_run(yy, xx, raw, ggml_type, geo, ggml_type != EQ_GGML_Q4_K && ggml_type != EQ_GGML_Q8_0, 1,
                              N, K, big, ExpertSel{ids, matrix_bytes, int(experts), int(routes)}, st))
            return 1;
    } else {
        // prefill: the bank re-packed once (as the native prefill does), then the gathered product
        if (N % 128 != 0 || K % 64 != 0) {
            set_error("more than " + std::to_string(kGroupedCopyRoutes) +
                      " routes need N % 128 == 0 and K % 64 == 0");
            return 1;
        }
        const bool as_bytes = !geo.affine || (geo.bits != 4 && geo.bits != 8);
        const int bits = as_bytes ? 8 : geo.bits;
        auto up = [](size_t v) { return (v + 255) & ~size_t(255); };
        const size_t wsz = up(size_t(experts * N) * size_t(K) * bits / 8);
        const size_t psz = up(size_t(experts * N) * size_t(K / geo.gs) * 2);
        const size_t triple = wsz + 2 * psz;
        const int64_t cap = experts + (routes + 127) / 128;  // entries of the grouped tile list
        const size_t rest = up(size_t(routes) * size_t(K) * 2) + size_t(cap) * 16 + 256;
        char* base = static_cast<char*>(ws_acquire(nullptr, triple + rest, st));
        if (!base) {
            set_error("could not obtain workspace for the re-packed expert bank");
            return 1;
        }
        uint32_t* w = reinterpret_cast<uint32_t*>(base);
        uint16_t* s = reinterpret_cast<uint16_t*>(base + wsz);
        uint16_t* b = reinterpret_cast<uint16_t*>(base + wsz + psz);
        const WsSource tail{base + triple, rest, nullptr};
        const bool v16 = aligned(raw, 16);
        if (!as_bytes) {
            launch_convert_affine(ggml_type, big, raw, nblocks, v16, w, s, b, st);
        } else if (!with_kq(ggml_type, big, [&](auto t, auto bt) {
                       constexpr int T = decltype(t)::value;
                       constexpr int NB = 256 / KQuant<T>::units;
                       kq_to_bytes<T, decltype(bt)::value><<<dim3(unsigned((nblocks + NB - 1) / NB)), 256, 0, st>>>(
                           raw, nblocks, v16, reinterpret_cast<uint4*>(w), s, b);
                   })) {
            set_error("no re-pack kernel for this encoding");
            return 1;
        }
        if (gather_qmm_launch(y, x, w, s, b, nullptr, ids, routes, routes, experts, 1, N, K, true, geo.gs, bits,
                              kModeAffine, EQ_DTYPE_BF16, EQ_DTYPE_F16, sorted_ids, &tail, st))
            return 1;
        // the rows of ids outside the bank are +0 (the decode kernels write them so themselves)
        embedding_clear_rows<uint16_t><<<dim3(unsigned(routes)), 256, 0, st>>>(yy, ids, experts, N);
    }
    return check_launch("gguf grouped linear");
}
