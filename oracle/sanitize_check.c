/*
 * sanitize_check.c -- TEST INFRASTRUCTURE ONLY: drives every exported function
 * of eq_oracle.c on seeded inputs under AddressSanitizer and
 * UndefinedBehaviorSanitizer (`make -C oracle sanitize`, run by
 * tests/test_oracle_sanitize.py).  Buffers are allocated at their exact sizes,
 * so a read or write one element past an input or output is reported.  The
 * values computed are not checked here (the other oracle tests do that); the
 * exit status is 0 unless a sanitizer fires or a call reports an error.  With
 * the argument `planted` it makes one out-of-bounds write on purpose, so the
 * test can show the build reports it.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
uint16_t or_f32_to_bf16(float f);
float or_bf16_to_f32(uint16_t b);
int or_gguf_block_geometry(int type, int* values, int* bytes);
int or_gguf_affine_config(int type, int* bits, int* gs);
int or_gguf_convert_affine(int type, int big_endian, const uint8_t* raw, int64_t nblocks, uint32_t* w, uint16_t* s,
                           uint16_t* b);
void or_affine_dequant_f32(const uint32_t* w, const void* scales, const void* biases, int scale_dtype, int64_t rows,
                           int64_t cols, int gs, int bits, float* out);
int or_gguf_dequant_f32(int type, int big_endian, int definition, const uint8_t* raw, int64_t nblocks, float* out);
void or_quantize_affine(const float* wsrc, int64_t rows, int64_t cols, int gs, int bits, int scale_dtype,
                        uint32_t* wq, void* scales, void* biases);
int or_qmm_t_f32(float* y, const void* x, const uint32_t* w, const void* scales, const void* biases, int64_t M,
                 int64_t N, int64_t K, int gs, int bits, int x_dtype, int scale_dtype, int threads);

static uint64_t rng = 0x9e3779b97f4a7c15ull;
static uint32_t next_u32(void) {
    rng ^= rng << 13;
    rng ^= rng >> 7;
    rng ^= rng << 17;
    return (uint32_t)(rng >> 11);
}
static float next_f32(void) { return ((float)(next_u32() & 0xffffff) / 8388608.0f - 1.0f) * 0.05f; }

static void* xmalloc(size_t n) {
    void* p = malloc(n ? n : 1);
    if (!p) {
        fprintf(stderr, "out of memory\n");
        exit(2);
    }
    return p;
}

static int fail(const char* what) {
    fprintf(stderr, "sanitize_check: %s returned an error\n", what);
    return 1;
}

/* A mistake planted on purpose (`sanitize_check planted`): a Q4_K conversion
 * into a weight buffer one word short, which the sanitizer must report. */
static int planted(void) {
    uint8_t raw[144];
    for (int i = 0; i < 144; i++) raw[i] = (uint8_t)next_u32();
    uint32_t* w = xmalloc(31 * sizeof(uint32_t));
    uint16_t s[8], b[8];
    int rc = or_gguf_convert_affine(12, 0, raw, 1, w, s, b);
    free(w);
    return rc;
}

int main(int argc, char** argv) {
    if (argc > 1 && strcmp(argv[1], "planted") == 0) return planted();
    int bad = 0;
    /* floats: every f16 pattern and a spread of f32 */
    for (uint32_t h = 0; h < 65536; h++) (void)or_f16_to_f32((uint16_t)h);
    for (int i = 0; i < 1 << 16; i++) {
        union { uint32_t u; float f; } v = {next_u32()};
        (void)or_f32_to_f16(v.f);
        (void)or_bf16_to_f32(or_f32_to_bf16(v.f));
    }
    /* every GGML type with an affine form, both byte orders and definitions */
    const int types[] = {2, 3, 6, 7, 8, 10, 11, 12, 13, 14};
    for (size_t t = 0; t < sizeof(types) / sizeof(types[0]); t++) {
        int values, bytes, bits, gs;
        if (or_gguf_block_geometry(types[t], &values, &bytes) || or_gguf_affine_config(types[t], &bits, &gs))
            return fail("geometry");
        const int64_t nblocks = 5;
        uint8_t* raw = xmalloc((size_t)(nblocks * bytes));
        for (int64_t i = 0; i < nblocks * bytes; i++) raw[i] = (uint8_t)next_u32();
        const int64_t words = nblocks * values * bits / 32, groups = nblocks * values / gs;
        uint32_t* w = xmalloc((size_t)words * sizeof(uint32_t));
        uint16_t* s = xmalloc((size_t)groups * sizeof(uint16_t));
        uint16_t* b = xmalloc((size_t)groups * sizeof(uint16_t));
        float* out = xmalloc((size_t)(nblocks * values) * sizeof(float));
        for (int be = 0; be < 2; be++) {
            bad |= or_gguf_convert_affine(types[t], be, raw, nblocks, w, s, b) ? fail("convert_affine") : 0;
            for (int def = 0; def < 2; def++)
                bad |= or_gguf_dequant_f32(types[t], be, def, raw, nblocks, out) ? fail("dequant_f32") : 0;
        }
        or_affine_dequant_f32(w, s, b, 1, nblocks, (int64_t)values, gs, bits, out);
        or_affine_dequant_f32(w, s, NULL, 1, nblocks, (int64_t)values, gs, bits, out);
        free(raw), free(w), free(s), free(b), free(out);
    }
    /* quantizer and matmul at every width the matmul restatement takes */
    const int widths[][2] = {{2, 32}, {3, 32}, {4, 64}, {5, 32}, {6, 16}, {8, 128}};
    for (size_t i = 0; i < sizeof(widths) / sizeof(widths[0]); i++) {
        const int bits = widths[i][0], gs = widths[i][1];
        const int64_t M = 3, N = 5, K = 256;
        float* wsrc = xmalloc((size_t)(N * K) * sizeof(float));
        for (int64_t j = 0; j < N * K; j++) wsrc[j] = next_f32();
        uint32_t* wq = xmalloc((size_t)(N * K * bits / 32) * sizeof(uint32_t));
        for (int dt = 0; dt < 3; dt++) {
            const size_t psz = dt == 0 ? 4 : 2;
            void* sc = xmalloc((size_t)(N * K / gs) * psz);
            void* bi = xmalloc((size_t)(N * K / gs) * psz);
            or_quantize_affine(wsrc, N, K, gs, bits, dt, wq, sc, bi);
            if (bits == 2 || bits == 4 || bits == 8) {
                uint16_t* x = xmalloc((size_t)(M * K) * sizeof(uint16_t));
                for (int64_t j = 0; j < M * K; j++) x[j] = or_f32_to_bf16(next_f32() * 20.0f);
                float* y = xmalloc((size_t)(M * N) * sizeof(float));
                bad |= or_qmm_t_f32(y, x, wq, sc, bi, M, N, K, gs, bits, 2, dt, 1) ? fail("qmm_t 1") : 0;
                bad |= or_qmm_t_f32(y, x, wq, sc, bi, M, N, K, gs, bits, 2, dt, 4) ? fail("qmm_t 4") : 0;
                free(x), free(y);
            }
            free(sc), free(bi);
        }
        free(wsrc), free(wq);
    }
    if (!bad) printf("sanitize_check: ok\n");
    return bad;
}
