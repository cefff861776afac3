/*
 * eq_oracle.c -- CPU restatement of the reference's quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this file.  It is the checker for the HIP kernels (tests/, the
 * __graft_entry__ smoke check) and the timed CPU baseline in bench.py.
 *
 * Every function cites the reference file:line it restates.  Paths are
 * relative to the jbg/eredu checkout.
 *
 * Parity status of each function (how it is pinned, see tests/test_oracle.py):
 *   or_f32_to_f16 / or_f16_to_f32   pinned: numpy float16 (IEEE RNE) on 2^16
 *                                    f16 patterns and 2^20 random f32s.
 *   or_f32_to_bf16                   pinned: torch bfloat16 RNE conversion.
 *   or_gguf_convert_affine           pinned: mlx-v0.32.0.oracle fixture rows
 *                                    (Q4_0, Q4_1, Q8_0, Q2_K, Q3_K, Q4_K,
 *                                    Q5_K, Q6_K byte-exact), the boundary
 *                                    blocks and Q5_0/Q5_1 repack tests of
 *                                    eredu-gguf/tests/oracle.rs, and closed
 *                                    forms from ggml's published decoders
 *                                    (tests/test_oracle_kquants.py).
 *   or_gguf_dequant_f32 (affine)     pinned: fixture "dequantized" column
 *                                    (exact after f16 rounding; Q6_K within
 *                                    the reference test's tolerance and exact
 *                                    under MLX's two-rounding f16 arithmetic),
 *                                    the Q5_0/Q5_1 rows' f16 weights (exact).
 *   or_iq4_dequant_f32               pinned: llama-c0bc8591-iq.oracle rows 20, 23
 *                                    (llama.cpp's f16 outputs, exact), zero
 *                                    blocks, byte-order swap (iquant.rs tests).
 *   or_gguf_dequant_f32 (native)     pinned: closed form d*sc*q - dmin*m in
 *                                    f64, and the <=1e-6 native-vs-affine
 *                                    tests' sample blocks.
 *   or_affine_dequant_f32            pinned: fixture dequant column through
 *                                    the converted tensor; closed form.
 *   or_qmm_f32                       pinned: fp64 numpy closed form (tolerance),
 *                                    pure-Python brute force on tiny shapes.
 *   or_quantize_affine               parity unpinned: input generator and the
 *                                    checker of the device quantizer
 *                                    (MLX v0.32.0 quantize is not available);
 *                                    bounded by test_quantize_dequantize's
 *                                    max|w - w_hat| <= 127/2^bits rule.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- floats */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary16 -> binary32, exact (half 2.7.1 f16::to_f32, Cargo.lock:1267). */
float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ffu;
    if (exp == 0x1f) return u2f(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: man * 2^-24 */
        float v = (float)man * u2f(0x33800000u); /* 2^-24, exact */
        return (h & 0x8000u) ? -v : v;
    }
    return u2f(sign | ((exp + 112) << 23) | (man << 13));
}

/* binary32 -> binary16 bits with round-to-nearest-even, overflow to inf,
 * NaN kept quiet with the top payload bits (half 2.7.1 f16::from_f32, used by
 * eredu-gguf/src/convert.rs:409-411 `hbits`). */
uint16_t or_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xff;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff) {
        if (man == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | (man >> 13));
    }
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        /* result is subnormal (or zero) in f16 */
        if (e < -10) return (uint16_t)sign; /* below half the smallest subnormal */
        uint32_t m = man | 0x800000u;       /* implicit one */
        uint32_t shift = (uint32_t)(14 - e); /* 24-bit significand -> 10-bit field */
        uint32_t half_bits = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half_bits & 1))) half_bits += 1;
        return (uint16_t)(sign | half_bits);
    }
    uint32_t half_bits = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half_bits & 1))) half_bits += 1; /* may carry into inf: correct */
    return (uint16_t)(sign | half_bits);
}

/* binary32 -> bfloat16 bits, round-to-nearest-even; NaN stays a quiet NaN. */
uint16_t or_f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7f800000u) == 0x7f800000u && (x & 0x7fffffu))
        return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

float or_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* Scale/activation dtypes shared with include/eredu_hip.h (EQ_DTYPE_*). */
enum { OR_F32 = 0, OR_F16 = 1, OR_BF16 = 2 };

static float load_scalar(const void* p, int dtype, int64_t i) {
    switch (dtype) {
    case OR_F16: return or_f16_to_f32(((const uint16_t*)p)[i]);
    case OR_BF16: return or_bf16_to_f32(((const uint16_t*)p)[i]);
    default: return ((const float*)p)[i];
    }
}

/* ----------------------------------------------------------- GGUF types */

enum {
    OR_Q4_0 = 2, OR_Q4_1 = 3, OR_Q5_0 = 6, OR_Q5_1 = 7, OR_Q8_0 = 8,
    OR_Q2_K = 10, OR_Q3_K = 11, OR_Q4_K = 12, OR_Q5_K = 13, OR_Q6_K = 14,
    OR_IQ4_NL = 20, OR_IQ4_XS = 23
};

static uint16_t rd16(const uint8_t* b, int big_endian) {
    /* eredu-gguf/src/format.rs:12-17 Endian::u16 */
    return big_endian ? (uint16_t)((b[0] << 8) | b[1]) : (uint16_t)(b[0] | (b[1] << 8));
}

static uint32_t rd32(const uint8_t* b, int big_endian) {
    /* eredu-gguf/src/format.rs:18-23 Endian::u32 (the Q5_0/Q5_1 high-bit word) */
    return big_endian ? ((uint32_t)b[0] << 24) | ((uint32_t)b[1] << 16) | ((uint32_t)b[2] << 8) | b[3]
                      : (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
}

/* LSB-first bit packing of `n` codes of `bits` each into u32 words
 * (eredu-gguf/src/convert.rs:413-427 `pack`).  `out` must be zeroed. */
static void pack_codes(const uint8_t* codes, int n, int bits, uint32_t* out) {
    uint32_t mask = (1u << bits) - 1u;
    for (int i = 0; i < n; i++) {
        int off = i * bits, w = off / 32, s = off % 32;
        out[w] |= ((uint32_t)codes[i] & mask) << s;
        if (s + bits > 32) out[w + 1] |= (uint32_t)codes[i] >> (32 - s);
    }
}

/* Q4_K 6-bit scale/min unpack (eredu-gguf/src/convert.rs:429-438 `scale_min`). */
static void q4k_scale_min(const uint8_t* s, int i, uint8_t* sc, uint8_t* m) {
    if (i < 4) {
        *sc = s[i] & 63;
        *m = s[i + 4] & 63;
    } else {
        *sc = (uint8_t)((s[i + 4] & 15) | ((s[i - 4] >> 6) << 4));
        *m = (uint8_t)((s[i + 4] >> 4) | ((s[i] >> 6) << 4));
    }
}

/* Values and bytes per block (eredu-gguf/src/format.rs:368-400). */
int or_gguf_block_geometry(int type, int* values, int* bytes) {
    switch (type) {
    case OR_Q4_0: *values = 32; *bytes = 18; return 0;
    case OR_Q4_1: *values = 32; *bytes = 20; return 0;
    case OR_Q5_0: *values = 32; *bytes = 22; return 0;
    case OR_Q5_1: *values = 32; *bytes = 24; return 0;
    case OR_Q8_0: *values = 32; *bytes = 34; return 0;
    case OR_Q2_K: *values = 256; *bytes = 84; return 0;
    case OR_Q3_K: *values = 256; *bytes = 110; return 0;
    case OR_Q4_K: *values = 256; *bytes = 144; return 0;
    case OR_Q5_K: *values = 256; *bytes = 176; return 0;
    case OR_Q6_K: *values = 256; *bytes = 210; return 0;
    case OR_IQ4_NL: *values = 32; *bytes = 18; return 0;
    case OR_IQ4_XS: *values = 256; *bytes = 136; return 0;
    default: return 1;
    }
}

/* (bits, group size) of the affine form (eredu-gguf/src/convert.rs:142-152). */
int or_gguf_affine_config(int type, int* bits, int* gs) {
    switch (type) {
    case OR_Q2_K: *bits = 2; *gs = 16; return 0;
    case OR_Q3_K: *bits = 3; *gs = 16; return 0;
    case OR_Q4_0: case OR_Q4_1: case OR_Q4_K: *bits = 4; *gs = 32; return 0;
    case OR_Q5_0: case OR_Q5_1: case OR_Q5_K: *bits = 5; *gs = 32; return 0;
    case OR_Q6_K: *bits = 6; *gs = 16; return 0;
    case OR_Q8_0: *bits = 8; *gs = 32; return 0;
    default: return 1;
    }
}

/*
 * One block of the types added after Q4_0/Q8_0/Q4_K: its codes (in value
 * order) and the f16 scale/bias bits of each group.  The whole block is then
 * packed as one LSB-first stream; every group of these types ends on a word
 * boundary except Q3_K's, and convert.rs packs Q3_K per block too.
 *   Q4_1  convert.rs:362-373  scale = d, bias = m (raw halves), nibbles at 4
 *   Q5_0  convert.rs:544-564  scale = d, bias = f16(-16 d), qh u32 at 2, qs at 6
 *   Q5_1  convert.rs:544-564  scale = d, bias = m, qh u32 at 4, qs at 8
 *   Q5_K  convert.rs:439-465  as Q4_K + bit g of qh[i] (b[16..48]) as bit 4,
 *                             qs at 48
 *   Q6_K  convert.rs:467-489  two 128-value halves: ql (64 B), qh (32 B),
 *                             int8 scales at 192 + 8 half; d at 208;
 *                             scale = f16(d sc), bias = f16(-32 d sc)
 *   Q2_K  convert.rs:491-508  scale byte g: low nibble * d, high nibble * dmin
 *                             (bias negated); d at 80, dmin at 82
 *   Q3_K  convert.rs:510-542  6-bit signed scales (enc - 32) from 12 bytes at 96,
 *                             bias = f16(-4 d sc); high bit from hm; d at 108
 */
static void kquant_block(int type, int be, const uint8_t* p, uint8_t* codes, uint16_t* s, uint16_t* b) {
    if (type == OR_Q4_1) {
        s[0] = rd16(p, be);
        b[0] = rd16(p + 2, be);
        for (int i = 0; i < 16; i++) {
            codes[i] = p[4 + i] & 15;
            codes[16 + i] = p[4 + i] >> 4;
        }
    } else if (type == OR_Q5_0 || type == OR_Q5_1) {
        const int q50 = type == OR_Q5_0;
        uint16_t d = rd16(p, be);
        s[0] = d;
        b[0] = q50 ? or_f32_to_f16(-16.0f * or_f16_to_f32(d)) : rd16(p + 2, be);
        uint32_t qh = rd32(p + (q50 ? 2 : 4), be);
        const uint8_t* qs = p + (q50 ? 6 : 8);
        for (int j = 0; j < 16; j++) {
            codes[j] = (uint8_t)((qs[j] & 15) | (((qh >> j) & 1) << 4));
            codes[j + 16] = (uint8_t)((qs[j] >> 4) | (((qh >> (j + 16)) & 1) << 4));
        }
    } else if (type == OR_Q5_K) {
        float d = or_f16_to_f32(rd16(p, be));
        float dm = or_f16_to_f32(rd16(p + 2, be));
        const uint8_t* qh = p + 16;
        const uint8_t* qs = p + 48;
        for (int g = 0; g < 8; g++) {
            uint8_t sc, m;
            q4k_scale_min(p + 4, g, &sc, &m);
            s[g] = or_f32_to_f16(d * (float)sc);
            b[g] = or_f32_to_f16(-dm * (float)m);
            for (int i = 0; i < 32; i++) {
                uint8_t q = qs[(g / 2) * 32 + i];
                uint8_t lo = (g % 2 == 0) ? (q & 15) : (q >> 4);
                codes[g * 32 + i] = (uint8_t)(lo | ((qh[i] >> g) & 1) << 4);
            }
        }
    } else if (type == OR_Q6_K) {
        float d = or_f16_to_f32(rd16(p + 208, be));
        for (int half = 0; half < 2; half++) {
            const uint8_t* ql = p + half * 64;
            const uint8_t* qh = p + 128 + half * 32;
            uint8_t* v = codes + half * 128;
            for (int i = 0; i < 32; i++) {
                v[i] = (uint8_t)((ql[i] & 15) | ((qh[i] & 3) << 4));
                v[i + 32] = (uint8_t)((ql[i + 32] & 15) | (((qh[i] >> 2) & 3) << 4));
                v[i + 64] = (uint8_t)((ql[i] >> 4) | (((qh[i] >> 4) & 3) << 4));
                v[i + 96] = (uint8_t)((ql[i + 32] >> 4) | (((qh[i] >> 6) & 3) << 4));
            }
            for (int g = 0; g < 8; g++) {
                float sc = d * (float)(int8_t)p[192 + half * 8 + g];
                s[half * 8 + g] = or_f32_to_f16(sc);
                b[half * 8 + g] = or_f32_to_f16(-32.0f * sc);
            }
        }
    } else if (type == OR_Q2_K) {
        float d = or_f16_to_f32(rd16(p + 80, be));
        float dm = or_f16_to_f32(rd16(p + 82, be));
        for (int g = 0; g < 16; g++) {
            s[g] = or_f32_to_f16(d * (float)(p[g] & 15));
            b[g] = or_f32_to_f16(-dm * (float)(p[g] >> 4));
            int qo = (g / 8) * 32 + (g % 2) * 16, shift = ((g % 8) / 2) * 2;
            for (int i = 0; i < 16; i++) codes[g * 16 + i] = (p[16 + qo + i] >> shift) & 3;
        }
    } else { /* OR_Q3_K */
        const uint8_t* hm = p;
        const uint8_t* qs = p + 32;
        const uint8_t* src = p + 96;
        uint8_t enc[16];
        for (int i = 0; i < 4; i++) {
            enc[i] = (uint8_t)((src[i] & 15) | ((src[8 + i] & 3) << 4));
            enc[4 + i] = (uint8_t)((src[4 + i] & 15) | (((src[8 + i] >> 2) & 3) << 4));
            enc[8 + i] = (uint8_t)((src[i] >> 4) | (((src[8 + i] >> 4) & 3) << 4));
            enc[12 + i] = (uint8_t)((src[4 + i] >> 4) | (((src[8 + i] >> 6) & 3) << 4));
        }
        float d = or_f16_to_f32(rd16(p + 108, be));
        for (int g = 0; g < 16; g++) {
            float sc = d * (float)((int)enc[g] - 32);
            s[g] = or_f32_to_f16(sc);
            b[g] = or_f32_to_f16(-4.0f * sc);
            int qo = (g / 8) * 32 + (g % 2) * 16, shift = ((g % 8) / 2) * 2;
            for (int i = 0; i < 16; i++)
                codes[g * 16 + i] = (uint8_t)(((qs[qo + i] >> shift) & 3) |
                                              ((hm[(g % 2) * 16 + i] >> (g / 2)) & 1) << 2);
        }
    }
}

/*
 * GGML blocks -> MLX affine (u32 codes, f16 scales, f16 biases).
 * eredu-gguf/src/convert.rs:318-404 (`convert_affine`/`affine`):
 *   Q4_0  :349-361   scale = d, bias = f16(-8 d), codes lo nibbles then hi
 *   Q8_0  :377-385   scale = d, bias = f16(-128 d), codes = byte ^ 0x80, 8-bit
 *   Q4_K  :439-465   scale = f16(d sc), bias = f16(-dmin m), 8 groups of 32
 *   the others in kquant_block above.
 * Outputs per block: values * bits / 32 words and values / group size groups
 * (or_gguf_affine_config).  Returns 0, or 1 for an unsupported type.
 */
int or_gguf_convert_affine(int type, int big_endian, const uint8_t* raw, int64_t nblocks,
                           uint32_t* w, uint16_t* s, uint16_t* b) {
    uint8_t codes[256];
    int values, bytes, bits, gs;
    if (or_gguf_block_geometry(type, &values, &bytes) || or_gguf_affine_config(type, &bits, &gs)) return 1;
    if (type != OR_Q4_0 && type != OR_Q8_0 && type != OR_Q4_K) {
        const int wpb = values * bits / 32, gpb = values / gs;
        for (int64_t blk = 0; blk < nblocks; blk++) {
            kquant_block(type, big_endian, raw + blk * bytes, codes, s + blk * gpb, b + blk * gpb);
            memset(w + blk * wpb, 0, sizeof(uint32_t) * wpb);
            pack_codes(codes, values, bits, w + blk * wpb);
        }
        return 0;
    }
    for (int64_t blk = 0; blk < nblocks; blk++) {
        if (type == OR_Q4_0) {
            const uint8_t* p = raw + blk * 18;
            uint16_t d = rd16(p, big_endian);
            s[blk] = d;
            b[blk] = or_f32_to_f16(-8.0f * or_f16_to_f32(d));
            for (int i = 0; i < 16; i++) {
                codes[i] = p[2 + i] & 15;
                codes[16 + i] = p[2 + i] >> 4;
            }
            memset(w + blk * 4, 0, 16);
            pack_codes(codes, 32, 4, w + blk * 4);
        } else if (type == OR_Q8_0) {
            const uint8_t* p = raw + blk * 34;
            uint16_t d = rd16(p, big_endian);
            s[blk] = d;
            b[blk] = or_f32_to_f16(-128.0f * or_f16_to_f32(d));
            for (int i = 0; i < 32; i++) codes[i] = p[2 + i] ^ 0x80;
            memset(w + blk * 8, 0, 32);
            pack_codes(codes, 32, 8, w + blk * 8);
        } else if (type == OR_Q4_K) {
            const uint8_t* p = raw + blk * 144;
            float d = or_f16_to_f32(rd16(p, big_endian));
            float dm = or_f16_to_f32(rd16(p + 2, big_endian));
            const uint8_t* sm = p + 4;
            const uint8_t* qs = p + 16;
            for (int g = 0; g < 8; g++) {
                uint8_t sc, m;
                q4k_scale_min(sm, g, &sc, &m);
                s[blk * 8 + g] = or_f32_to_f16(d * (float)sc);
                b[blk * 8 + g] = or_f32_to_f16(-dm * (float)m);
                for (int i = 0; i < 32; i++) {
                    uint8_t q = qs[(g / 2) * 32 + i];
                    codes[i] = (g % 2 == 0) ? (q & 15) : (q >> 4);
                }
                memset(w + blk * 32 + g * 4, 0, 16);
                pack_codes(codes, 32, 4, w + blk * 32 + g * 4);
            }
        } else {
            return 1;
        }
    }
    return 0;
}

/*
 * Generic affine dequantize to f32: w = f32(scale) * code + f32(bias), one f32
 * multiply then one f32 add (eredu-gguf/src/convert.rs:81-101
 * `AffineTensor::dequantize`; the MLX `dequantize` contract of
 * safemlx/src/ops/quantization.rs:228-289).  LSB-first codes that may straddle
 * words (any bits in 2..8).  Scales/biases are [rows, cols/gs] of `scale_dtype`;
 * biases may be NULL (treated as zero).
 */
void or_affine_dequant_f32(const uint32_t* w, const void* scales, const void* biases, int scale_dtype,
                           int64_t rows, int64_t cols, int gs, int bits, float* out) {
    uint32_t mask = (1u << bits) - 1u;
    int64_t words_per_row = cols * bits / 32;
    int64_t groups_per_row = cols / gs;
    for (int64_t r = 0; r < rows; r++) {
        const uint32_t* wr = w + r * words_per_row;
        for (int64_t c = 0; c < cols; c++) {
            int64_t bit = c * bits, word = bit / 32, shift = bit % 32;
            uint32_t code = wr[word] >> shift;
            if (shift + bits > 32) code |= wr[word + 1] << (32 - shift);
            code &= mask;
            int64_t g = r * groups_per_row + c / gs;
            float sc = load_scalar(scales, scale_dtype, g);
            float bi = biases ? load_scalar(biases, scale_dtype, g) : 0.0f;
            out[r * cols + c] = sc * (float)code + bi; /* built with -ffp-contract=off, as Rust */
        }
    }
}

/* The 16 non-uniform 4-bit levels of IQ4_NL / IQ4_XS: the GGML format's
 * table (kvalues_iq4nl; the reference's copy is KVALUES_IQ4NL,
 * eredu-gguf/src/iquant_tables.rs:1920). */
static const int8_t kIq4Levels[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/*
 * IQ4_NL / IQ4_XS blocks -> f32, the reference's decode_f32 for these types
 * (eredu-gguf/src/iquant.rs:271-301):
 *   IQ4_NL (32 values, 18 B): d = f16 at 0; byte 2 + i holds value i (low
 *     nibble) and value 16 + i (high nibble); w = d * level[nibble].
 *   IQ4_XS (256 values, 136 B): d = f16 at 0, scales_high u16 at 2, scales_low
 *     bytes 4..8, codes at 8; group ib (32 values): 6-bit ls = nibble ib % 2 of
 *     scales_low[ib / 2] | bits 2 ib, 2 ib + 1 of scales_high << 4;
 *     dl = d * (ls - 32); codes 8 + 16 ib + i as in IQ4_NL; w = dl * level.
 * Every product is exact in f32 (the levels need 8 bits, dl at most 17).
 * Returns 0, or 1 for another type.
 */
int or_iq4_dequant_f32(int type, int big_endian, const uint8_t* raw, int64_t nblocks, float* out) {
    if (type == OR_IQ4_NL) {
        for (int64_t blk = 0; blk < nblocks; blk++) {
            const uint8_t* p = raw + blk * 18;
            float d = or_f16_to_f32(rd16(p, big_endian));
            for (int i = 0; i < 16; i++) {
                out[blk * 32 + i] = d * (float)kIq4Levels[p[2 + i] & 15];
                out[blk * 32 + 16 + i] = d * (float)kIq4Levels[p[2 + i] >> 4];
            }
        }
        return 0;
    }
    if (type == OR_IQ4_XS) {
        for (int64_t blk = 0; blk < nblocks; blk++) {
            const uint8_t* p = raw + blk * 136;
            float d = or_f16_to_f32(rd16(p, big_endian));
            uint16_t sh = rd16(p + 2, big_endian);
            for (int ib = 0; ib < 8; ib++) {
                int low = (p[4 + ib / 2] >> (4 * (ib % 2))) & 15;
                int high = (sh >> (2 * ib)) & 3;
                float dl = d * (float)((low | (high << 4)) - 32);
                const uint8_t* q = p + 8 + 16 * ib;
                for (int i = 0; i < 16; i++) {
                    out[blk * 256 + 32 * ib + i] = dl * (float)kIq4Levels[q[i] & 15];
                    out[blk * 256 + 32 * ib + 16 + i] = dl * (float)kIq4Levels[q[i] >> 4];
                }
            }
        }
        return 0;
    }
    return 1;
}

/*
 * Dense dequant of GGML blocks to f32.
 * definition 0 ("affine route"): convert_affine then AffineTensor::dequantize
 *   (eredu-gguf/src/convert.rs:43-56,81-101).
 * definition 1 ("native route"): safemlx/src/native_quantization.rs
 *   :3445-3469 decode_q4k_block   w = d*sc*q - dmin*m  (f32, left to right)
 *   :3499-3509 decode_q5_1_block  w = d*q + m (equal to the affine route:
 *                                 scale and bias are d and m unrounded)
 *   :3539-3542 decode_q8_0_block  w = d*int8(q)
 *   Q4_0, Q4_1, Q5_0, Q2_K and Q3_K have no native form (format.rs:423-428)
 *   and Q5_K / Q6_K dequantize through the affine form; both definitions use
 *   the affine route for them.
 */
int or_gguf_dequant_f32(int type, int big_endian, int definition, const uint8_t* raw, int64_t nblocks,
                        float* out) {
    int values, bytes;
    if (or_gguf_block_geometry(type, &values, &bytes)) return 1;
    if (type == OR_IQ4_NL || type == OR_IQ4_XS) return or_iq4_dequant_f32(type, big_endian, raw, nblocks, out);
    if (definition == 1 && type == OR_Q4_K) {
        for (int64_t blk = 0; blk < nblocks; blk++) {
            const uint8_t* p = raw + blk * 144;
            float d = or_f16_to_f32(rd16(p, big_endian));
            float dm = or_f16_to_f32(rd16(p + 2, big_endian));
            for (int g = 0; g < 8; g++) {
                uint8_t sc, m;
                q4k_scale_min(p + 4, g, &sc, &m);
                for (int i = 0; i < 32; i++) {
                    uint8_t q = p[16 + (g / 2) * 32 + i];
                    q = (g % 2 == 0) ? (q & 15) : (q >> 4);
                    out[blk * 256 + g * 32 + i] = d * (float)sc * (float)q - dm * (float)m;
                }
            }
        }
        return 0;
    }
    if (definition == 1 && type == OR_Q8_0) {
        for (int64_t blk = 0; blk < nblocks; blk++) {
            const uint8_t* p = raw + blk * 34;
            float d = or_f16_to_f32(rd16(p, big_endian));
            for (int i = 0; i < 32; i++) out[blk * 32 + i] = d * (float)(int8_t)p[2 + i];
        }
        return 0;
    }
    if (definition == 1 && type == OR_Q5_1) {
        for (int64_t blk = 0; blk < nblocks; blk++) {
            const uint8_t* p = raw + blk * 24;
            float d = or_f16_to_f32(rd16(p, big_endian));
            float m = or_f16_to_f32(rd16(p + 2, big_endian));
            uint32_t high = rd32(p + 4, big_endian);
            for (int i = 0; i < 32; i++) {
                uint8_t packed = p[8 + i % 16];
                uint32_t q = (uint32_t)(i < 16 ? (packed & 15) : (packed >> 4)) | (((high >> i) & 1) << 4);
                out[blk * 32 + i] = d * (float)q + m;
            }
        }
        return 0;
    }
    /* Every other (type, definition): the affine route.  Q5_K and Q6_K have
     * no CPU decoder of their own in the reference; their native dequantize
     * is IQuantTensor::dequantize_f32 = convert_affine + dequantize
     * (safemlx/src/native_quantization.rs:792-830, convert.rs:43-56). */
    int bits, gs;
    or_gguf_affine_config(type, &bits, &gs);
    uint32_t w[64];
    uint16_t s[16], b[16];
    for (int64_t blk = 0; blk < nblocks; blk++) {
        or_gguf_convert_affine(type, big_endian, raw + blk * bytes, 1, w, s, b);
        or_affine_dequant_f32(w, s, b, OR_F16, 1, values, gs, bits, out + blk * values);
    }
    return 0;
}

/*
 * Affine group quantizer used ONLY to generate matmul inputs (the role of MLX
 * `quantize`, safemlx/src/ops/quantization.rs:121-159).  Per group of `gs`:
 *   scale = (max - min) / (2^bits - 1), stored in `scale_dtype`;
 *   the edge value of larger magnitude becomes the bias (stored rounded), and
 *   the scale is re-derived so that edge maps exactly onto a code;
 *   q = clamp(round((w - bias) / scale), 0, 2^bits - 1).
 * Output codes are packed LSB-first.  Input w is f32 [rows, cols].
 */
void or_quantize_affine(const float* wsrc, int64_t rows, int64_t cols, int gs, int bits, int scale_dtype,
                        uint32_t* wq, void* scales, void* biases) {
    int n_bins = (1 << bits) - 1;
    int64_t words_per_row = cols * bits / 32;
    memset(wq, 0, sizeof(uint32_t) * (size_t)(rows * words_per_row));
    uint8_t* codes = (uint8_t*)malloc((size_t)cols);
    for (int64_t r = 0; r < rows; r++) {
        for (int64_t g0 = 0; g0 < cols; g0 += gs) {
            const float* v = wsrc + r * cols + g0;
            float mn = v[0], mx = v[0];
            for (int i = 1; i < gs; i++) { if (v[i] < mn) mn = v[i]; if (v[i] > mx) mx = v[i]; }
            float scale = (mx - mn) / (float)n_bins;
            if (scale < 1e-7f) scale = 1e-7f;
            int neg = fabsf(mn) > fabsf(mx);
            scale = neg ? scale : -scale;
            float edge = neg ? mn : mx;
            float q0 = rintf(edge / scale);
            if (q0 != 0.0f) scale = edge / q0;
            float bias = edge;
            /* store rounded to the parameter dtype, then quantize with the
             * stored values so dequantization reproduces the codes' intent */
            int64_t gi = r * (cols / gs) + g0 / gs;
            float s_st, b_st;
            if (scale_dtype == OR_BF16) {
                ((uint16_t*)scales)[gi] = or_f32_to_bf16(scale);
                ((uint16_t*)biases)[gi] = or_f32_to_bf16(bias);
                s_st = or_bf16_to_f32(((uint16_t*)scales)[gi]);
                b_st = or_bf16_to_f32(((uint16_t*)biases)[gi]);
            } else if (scale_dtype == OR_F16) {
                ((uint16_t*)scales)[gi] = or_f32_to_f16(scale);
                ((uint16_t*)biases)[gi] = or_f32_to_f16(bias);
                s_st = or_f16_to_f32(((uint16_t*)scales)[gi]);
                b_st = or_f16_to_f32(((uint16_t*)biases)[gi]);
            } else {
                ((float*)scales)[gi] = scale;
                ((float*)biases)[gi] = bias;
                s_st = scale;
                b_st = bias;
            }
            for (int i = 0; i < gs; i++) {
                float q = s_st != 0.0f ? rintf((v[i] - b_st) / s_st) : 0.0f;
                if (!(q >= 0.0f)) q = 0.0f;
                if (q > (float)n_bins) q = (float)n_bins;
                codes[g0 + i] = (uint8_t)q;
            }
        }
        uint32_t* wr = wq + r * words_per_row;
        for (int64_t c = 0; c < cols; c++) {
            int64_t off = c * bits, w = off / 32, sh = off % 32;
            wr[w] |= ((uint32_t)codes[c]) << sh;
            if (sh + bits > 32) wr[w + 1] |= (uint32_t)codes[c] >> (32 - sh);
        }
    }
    free(codes);
}

/*
 * Restated MLX CPU quantized matmul, transpose=true (W is [N, K]):
 *   y[m, n] = sum_k x[m, k] * (s[n, k/gs] * q[n, k] + b[n, k/gs])
 * Structure of MLX's CPU `_qmm_t` (dispatched from
 * mlx/backend/cpu/quantized.cpp; visible context:
 * safemlx-sys/src/mlx-c/patches/mlx-affine-group16.patch:1-22): per output
 * row n, walk the groups, dequantize each code on the fly and accumulate.
 * This restatement accumulates in f32 (the contract the hot path is held to).
 * Activations and scales are read as `x_dtype` / `scale_dtype`; the result is
 * written as f32.  Rows of the output are split over `threads` POSIX threads.
 */
typedef struct {
    float* y; const void* x; const uint32_t* w; const void* s; const void* b;
    int64_t M, N, K; int gs, bits, x_dtype, scale_dtype; int64_t n0, n1;
} qmm_job;

static void* qmm_worker(void* arg) {
    qmm_job* j = (qmm_job*)arg;
    int pack = 32 / j->bits;
    uint32_t mask = (1u << j->bits) - 1u;
    int64_t wpr = j->K * j->bits / 32, gpr = j->K / j->gs;
    float* xf = (float*)malloc(sizeof(float) * (size_t)(j->M * j->K));
    for (int64_t i = 0; i < j->M * j->K; i++) xf[i] = load_scalar(j->x, j->x_dtype, i);
    for (int64_t n = j->n0; n < j->n1; n++) {
        const uint32_t* wr = j->w + n * wpr;
        for (int64_t m = 0; m < j->M; m++) {
            const float* xr = xf + m * j->K;
            float acc = 0.0f;
            int64_t k = 0;
            for (int64_t g = 0; g < gpr; g++) {
                float sc = load_scalar(j->s, j->scale_dtype, n * gpr + g);
                float bi = j->b ? load_scalar(j->b, j->scale_dtype, n * gpr + g) : 0.0f;
                for (int kw = 0; kw < j->gs / pack; kw++) {
                    uint32_t word = wr[k / pack];
                    for (int p = 0; p < pack; p++, k++) {
                        acc += xr[k] * (sc * (float)(word & mask) + bi);
                        word >>= j->bits;
                    }
                }
            }
            j->y[m * j->N + n] = acc;
        }
    }
    free(xf);
    return NULL;
}

int or_qmm_t_f32(float* y, const void* x, const uint32_t* w, const void* scales, const void* biases,
                 int64_t M, int64_t N, int64_t K, int gs, int bits, int x_dtype, int scale_dtype,
                 int threads) {
    if (bits != 2 && bits != 4 && bits != 8) return 1;
    if (K % gs || gs % (32 / bits)) return 1;
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    qmm_job jobs[256];
    int64_t per = (N + threads - 1) / threads;
    int started = 0;
    for (int t = 0; t < threads; t++) {
        int64_t n0 = t * per, n1 = n0 + per > N ? N : n0 + per;
        if (n0 >= n1) break;
        jobs[t] = (qmm_job){y, x, w, scales, biases, M, N, K, gs, bits, x_dtype, scale_dtype, n0, n1};
        if (threads == 1) { qmm_worker(&jobs[t]); continue; }
        pthread_create(&tid[t], NULL, qmm_worker, &jobs[t]);
        started++;
    }
    for (int t = 0; t < started; t++) pthread_join(tid[t], NULL);
    return 0;
}
