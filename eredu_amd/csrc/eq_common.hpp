// Shared device helpers and host error plumbing for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstring>
#include <string>
#include <type_traits>

#include "../../include/eredu_hip.h"

namespace eq {

// ------------------------------------------------------------------ host side

// Thread-local message of the last failed call (the mlx-c convention of
// safemlx/src/error.rs:239-269: status code plus a per-thread message).
void set_error(const std::string& msg);
void clear_error();

// Checks the launch status of the kernels just enqueued.
int check_launch(const char* what);

// A launcher that takes a shape but cannot run its plan (its scratch memory
// cannot be provided) sets the message and records a refusal instead of
// running another plan; the entry point then fails.  take_refusal() reads
// and clears it.
void note_refusal();
bool take_refusal();

// Compute units of the current device (cached per device; 256 if the query fails).
int device_cu_count();

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// One matrix-vector problem of a (possibly grouped) decode launch:
// y[M, ldy] (columns [0, N)) = x[M, K] . W^T, W = [N, K] packed along K.
struct QmvSpec {
    const uint16_t* x;
    const uint32_t* w;
    const void* s;
    const void* b;  // may be null
    uint16_t* y;
    int N, K, ldy;
};

// Decode (small-M) launchers of qmv.hip.  launch_qmv_mfma takes one problem;
// launch_qmv_batched takes several sharing M, bits, group size and scale type
// and returns false, launching nothing, if the grouped path cannot take them
// all (the caller then issues them one by one).
// x_dtype (EQ_DTYPE_BF16 or EQ_DTYPE_F16) is the activation type, which y shares.
bool launch_qmv_mfma(int bits, int gs, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w,
                     const void* s, const void* b, int M, int N, int K, hipStream_t st, int x_dtype = EQ_DTYPE_BF16);
bool launch_qmv_batched(int bits, int gs, int scale_dtype, const QmvSpec* specs, int count, int M, hipStream_t st,
                        int x_dtype = EQ_DTYPE_BF16);
// Routed decode for gather_qmm (qmv.hip): y[b] = x[lhs(b)] . W[rhs(b)]^T for
// `batch` output batches of one bf16 row each, 4/8-bit codes, group 32/64/128,
// bf16 or f16 parameters, N % 16 == 0, the indices read on the device; false,
// launching nothing, when the shapes do not fit the decode kernel.
struct GatherIdx;
bool launch_qmv_gather(int bits, int gs, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w,
                       const void* s, const void* b, const GatherIdx& g, int64_t batch, int N, int K,
                       hipStream_t st);
// Activation rows one pass of launch_qmv_mfma's kernels multiplies for 4/8-bit
// codes at group size gs (a 16-row MFMA operand holds 16 / (groups per span)
// rows): 8 for 4-bit group 64, 16 for 8-bit group 64; more rows read the
// weights once per pass.
int qmv_rows_per_pass(int bits, int gs);
// Decode for the other widths (qmv_any.hip): transpose, bf16 x, M <= 16, bits
// 2..8, group 16 or a multiple of 32, K a multiple of 32; false, launching
// nothing, when it does not take the problem.
bool launch_qmv_any(int bits, int gs, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w,
                    const void* s, const void* b, int M, int N, int K, hipStream_t st);
// The same kernel for MXFP4 codes (E8M0 scale bytes, no biases).
bool launch_qmv_any_mxfp4(uint16_t* y, const uint16_t* x, const uint32_t* w, const uint8_t* s, int M, int N, int K,
                          hipStream_t st);

// Activation prologue of a decode launch: kind 1 = silu(x) * second,
// kind 2 = RMSNorm(x + second) * weight (second may be null), x + second
// written to hidden_out (may be null).  launch_qmv_prologue takes M = 1
// problems sharing one input; false, launching nothing, when it cannot.
struct QmvPrologue {
    int kind;
    const uint16_t* second;
    const uint16_t* weight;
    uint16_t* hidden_out;
    float eps;
};
bool launch_qmv_prologue(int bits, int gs, int scale_dtype, const QmvSpec* specs, int count, const QmvPrologue& pro,
                         hipStream_t st);
// One interleaved gate/up problem (group 64, bf16) with the SwiGLU epilogue,
// optionally after the RMSNorm prologue (pro: null or kind 2).
bool launch_qmv_swiglu(int bits, const QmvSpec& spec, const QmvPrologue* pro, hipStream_t st);

// ---------------------------------------------------------------- device side

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Buffer resource (V#) of a raw byte range: loads through it are range-checked
// by the hardware, and an offset at or past `bytes` reads as zero.  Buffer
// loads are also ordered against scheduling barriers, which plain loads from
// read-only pointers are not.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
// A wave-uniform 1 that the compiler cannot see through.  `if (opaque_one())`
// puts the guarded code in a basic block of its own: instruction selection
// and the machine scheduler work per block, so a block of prefetch loads
// placed before it is issued before it (within one block the schedulers
// would sink the loads down to their uses and serialise the pipeline).
__device__ __forceinline__ int opaque_one() {
    int v;
    asm volatile("s_mov_b32 %0, 1" : "=s"(v));
    return v;
}

// An offset past every buffer the kernels build (all are < 2^31 bytes), leaving
// room for the immediate offsets added to it.
constexpr uint32_t kOutOfRange = 0xC0000000u;

// ------------------------------------------------- cross-workgroup hand-off
//
// Each XCD has its own L2, and those caches are not kept coherent with each
// other for ordinary loads and stores; device-scope atomics are.  A kernel
// whose workgroups combine results within one launch does it through
// device-scope atomics and an arrival counter (last_arriver).  Measured on
// MI355X, such a hand-off (store completion, the counter's round trip, the
// last workgroup's reads) costs more than a kernel boundary in a HIP graph,
// so the kernels here use it only where the combined data is a few words.

// s_waitcnt vmcnt(0): every vector memory operation of this wave, stores
// included, has completed.
__device__ __forceinline__ void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Workgroup barrier for LDS hand-offs that leaves global loads in flight:
// this wave's LDS operations complete (lgkmcnt(0)), then s_barrier.
// __syncthreads() also carries a workgroup-scope fence, which the compiler
// implements by waiting for every outstanding memory operation (vmcnt(0)),
// prefetches included.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Counts this workgroup at `counter` after all its threads' device-scope
// stores have completed; true in the workgroup that arrives last of
// `expected`, which also resets the counter to zero for the next launch.
// Every workgroup must call it exactly once (it has two barriers), with the
// same `ticket` slot of LDS.
__device__ __forceinline__ bool last_arriver(unsigned* counter, unsigned expected, unsigned* ticket) {
    wait_vmem_all();
    __syncthreads();
    if (threadIdx.x == 0) *ticket = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const bool last = *ticket == expected - 1;
    if (last && threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return last;
}

// Pulls the 64-byte lines of a kernel's by-value argument block (the first
// MAX_LINES of them) into the scalar cache with independent loads and one
// wait.  The block is cold at each dispatch; without this, code that indexes
// it with computed values (a problem table walked per tile) pays one memory
// round trip per line, in sequence, before its first useful load.  The
// compiler issues at most 8 such loads before a wait, so more lines cost a
// second round trip (measured: ~0.4 us for 8 lines, ~0.75 us for 11).
// W0 is the word read from the first line: the one the kernel's own first
// test reads, so that the two are one load.
template <int MAX_LINES = 8, int W0 = 0, typename T>
__device__ __forceinline__ void prefetch_args(const T& args) {
    constexpr int lines = int(sizeof(T) + 63) / 64 < MAX_LINES ? int(sizeof(T) + 63) / 64 : MAX_LINES;
    static_assert(W0 >= 0 && W0 < 16, "a word of the first line");
    const uint32_t* p = reinterpret_cast<const uint32_t*>(&args);
    uint32_t acc = p[W0];
#pragma unroll
    for (int i = 1; i < lines; i++) acc ^= p[16 * i];
    asm volatile("" ::"s"(acc));
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// f32 -> bf16 bits, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t x = __float_as_uint(f);
    if ((x & 0x7f800000u) == 0x7f800000u && (x & 0x7fffffu)) return (x >> 16) | 0x40u;
    x += 0x7fffu + ((x >> 16) & 1u);
    return x >> 16;
}

// sigmoid(x) = 1 / (1 + e^-x) rounded to bf16 (the decoder's SiLU rounds it):
// e^-x as 2^(-x log2 e) with v_exp_f32 and the reciprocal with v_rcp_f32 --
// each within ~1 f32 ulp, far below the bf16 rounding that follows; the
// rounding to bf16 is the hardware RNE conversion.
__device__ __forceinline__ float silu_sigmoid_bf16(float x) {
    const float e = __builtin_amdgcn_exp2f(-x * 1.44269504088896341f);
    return float(static_cast<__bf16>(__builtin_amdgcn_rcpf(1.0f + e)));
}

// f32 -> IEEE binary16 bits with round-to-nearest-even, overflow to infinity
// and NaN quieted with the top payload bits kept: the rounding of the `half`
// crate's f16::from_f32 that eredu-gguf/src/convert.rs:409-411 uses.  Finite
// and infinite inputs take the hardware conversion (v_cvt_f16_f32 under the
// default round-to-nearest-even mode with f16 subnormals kept); NaN takes the
// crate's bit pattern, which the hardware does not promise.  The empty asm
// keeps f the rounded f32 it is: without it the compiler folds a product into
// the conversion (v_fma_mix with a +0 addend), rounding once instead of twice
// and turning a -0 product into +0.
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    const uint32_t x = __float_as_uint(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return ((x >> 16) & 0x8000u) | 0x7e00u | ((x & 0x7fffffu) >> 13);
    asm volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Scalar parameter loads for each scale/activation element type.
struct BF16T { typedef uint16_t storage; };
struct F16T { typedef uint16_t storage; };
struct F32T { typedef float storage; };
// MXFP4 scales: E8M0 bytes (load_param gives 2^(e - 127)).
struct E8M0T { typedef uint8_t storage; };

// --------------------------------------------------------------- dispatch

template <typename F>
inline bool with_dtype(int dt, F&& f) {
    switch (dt) {
    case EQ_DTYPE_F32: f(F32T{}); return true;
    case EQ_DTYPE_F16: f(F16T{}); return true;
    case EQ_DTYPE_BF16: f(BF16T{}); return true;
    default: return false;
    }
}

template <typename F>
inline bool with_bits(int bits, F&& f) {
    switch (bits) {
    case 2: f(std::integral_constant<int, 2>{}); return true;
    case 3: f(std::integral_constant<int, 3>{}); return true;
    case 4: f(std::integral_constant<int, 4>{}); return true;
    case 5: f(std::integral_constant<int, 5>{}); return true;
    case 6: f(std::integral_constant<int, 6>{}); return true;
    case 8: f(std::integral_constant<int, 8>{}); return true;
    default: return false;
    }
}

inline bool valid_dtype(int d) { return d == EQ_DTYPE_F32 || d == EQ_DTYPE_F16 || d == EQ_DTYPE_BF16; }
inline bool valid_scale_dtype(int d) { return valid_dtype(d) || d == EQ_DTYPE_U8; }

enum QuantMode { kModeAffine = 0, kModeMxFp4 = 1 };

// "affine" (or null) / "mxfp4"; anything else is an error.
inline int parse_mode(const char* mode, QuantMode& out) {
    if (mode == nullptr || std::strcmp(mode, "affine") == 0) {
        out = kModeAffine;
        return 0;
    }
    if (std::strcmp(mode, "mxfp4") == 0) {
        out = kModeMxFp4;
        return 0;
    }
    set_error(std::string("invalid quantization mode '") + mode + "'");
    return 1;
}

// Entry points that take the affine encoding only.
inline int check_mode(const char* mode) {
    QuantMode m;
    if (parse_mode(mode, m)) return 1;
    if (m == kModeMxFp4) {
        set_error("quantization mode 'mxfp4' is not supported by this entry point (affine only)");
        return 1;
    }
    return 0;
}

// MXFP4's fixed geometry (safemlx/src/ops/quantization.rs:37-45): group size
// 32, 4-bit codes, u8 scales, no biases.
inline int check_mxfp4(int group_size, int bits, int scale_dtype, const void* biases) {
    if (group_size != 32 || bits != 4) {
        set_error("MXFP4 requires group_size=32 and bits=4, got group_size=" + std::to_string(group_size) +
                  " bits=" + std::to_string(bits));
        return 1;
    }
    if (scale_dtype != EQ_DTYPE_U8) {
        set_error("MXFP4 scales are E8M0 bytes (EQ_DTYPE_U8)");
        return 1;
    }
    if (biases != nullptr) {
        set_error("MXFP4 has no biases");
        return 1;
    }
    return 0;
}

// MXFP4 host entry points (mxfp4.hip); arguments validated by the callers
// (geometry by check_mxfp4, pointers, shapes).
int mxfp4_quantize(uint32_t* w_out, uint8_t* scales, const void* w, int64_t rows, int64_t cols, int dtype,
                   hipStream_t st);
int mxfp4_dequantize(void* out, const uint32_t* w, const uint8_t* scales, int64_t rows, int64_t cols, int out_dtype,
                     hipStream_t st);


// Group size / bits rules of the affine contract (eredu-checkpoint/src/lib.rs:103-122,
// safemlx/src/ops/quantization.rs:62-64): bits 2, 3, 4, 5, 6 or 8; group size 16
// or a positive multiple of 32.  The fast kernels take bits 4 / 8 at group
// sizes 32, 64 and 128; every other combination runs on the general kernels.
inline int check_gs_bits(int group_size, int bits) {
    if (bits != 2 && bits != 3 && bits != 4 && bits != 5 && bits != 6 && bits != 8) {
        set_error("bits must be one of 2, 3, 4, 5, 6 or 8, got " + std::to_string(bits));
        return 1;
    }
    if (group_size != 16 && (group_size <= 0 || group_size % 32 != 0)) {
        set_error("group_size must be 16 or a positive multiple of 32, got " + std::to_string(group_size));
        return 1;
    }
    return 0;
}

// Group sizes the fast (templated) kernels are built for.
inline bool fast_group_size(int gs) { return gs == 32 || gs == 64 || gs == 128; }

// A packed row of `dim` codes must fill whole u32 words (quantized_packed_dimension
// is dim * bits / 32); false, with the error set, otherwise.
inline bool check_packed_row(int64_t dim, int bits) {
    if ((dim * bits) % 32 != 0) {
        set_error("a packed row of " + std::to_string(dim) + " " + std::to_string(bits) +
                  "-bit codes does not fill whole 32-bit words");
        return false;
    }
    return true;
}

template <typename T> __device__ __forceinline__ float load_param(const typename T::storage* p, int64_t i);
template <> __device__ __forceinline__ float load_param<BF16T>(const uint16_t* p, int64_t i) { return bf16_bits_to_f32(p[i]); }
template <> __device__ __forceinline__ float load_param<F16T>(const uint16_t* p, int64_t i) { return f16_bits_to_f32(p[i]); }
template <> __device__ __forceinline__ float load_param<F32T>(const float* p, int64_t i) { return p[i]; }

template <typename T> __device__ __forceinline__ void store_out(typename T::storage* p, int64_t i, float v);
template <> __device__ __forceinline__ void store_out<BF16T>(uint16_t* p, int64_t i, float v) { p[i] = static_cast<uint16_t>(f32_to_bf16_bits(v)); }
template <> __device__ __forceinline__ void store_out<F16T>(uint16_t* p, int64_t i, float v) { p[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v)); }
template <> __device__ __forceinline__ void store_out<F32T>(float* p, int64_t i, float v) { p[i] = v; }

// The storage bits store_out writes (RNE to the output type).
template <typename T> __device__ __forceinline__ typename T::storage to_storage(float v);
template <> __device__ __forceinline__ uint16_t to_storage<BF16T>(float v) { return static_cast<uint16_t>(f32_to_bf16_bits(v)); }
template <> __device__ __forceinline__ uint16_t to_storage<F16T>(float v) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v)); }
template <> __device__ __forceinline__ float to_storage<F32T>(float v) { return v; }

// ------------------------------------------------------ small vector helpers

// 16-byte streaming load: the weight blocks are read once, so they are not
// kept in the caches the activation rows are re-read from.
__device__ __forceinline__ uint4 load_stream16(const void* p) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 16- / 8-byte streaming stores for large outputs written once (dense
// dequantized tensors): the GGUF dense dequant ran 4-15 % faster with them,
// the affine dequantize 5 %; the affine re-pack (packed codes, a third of
// the bytes) ran slower, so it keeps plain stores.
__device__ __forceinline__ void store_stream16(void* p, uint4 v) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4*>(p));
}
__device__ __forceinline__ void store_stream8(void* p, uint2 v) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    __builtin_nontemporal_store(u32x2{v.x, v.y}, reinterpret_cast<u32x2*>(p));
}

__device__ __forceinline__ void bf16x8_to_f32(const uint4 v, float* f) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(&v);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f[2 * i] = bf16_bits_to_f32(p[i] & 0xffffu);
        f[2 * i + 1] = bf16_bits_to_f32(p[i] >> 16);
    }
}

// Two f32 -> one word of bf16 (a low, b high), round to nearest even, in one
// v_cvt_pk_bf16_f32; equal to f32_to_bf16_bits on every input but NaN (any
// quiet NaN).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// a.x b.x + a.y b.y + c over bf16 pairs (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

// MXFP4 (safemlx QuantizationMode::MxFp4, safemlx/src/ops/quantization.rs:16-46;
// the OCP microscaling FP4 format): E2M1 codes -- bit 3 sign, bits 2-1
// exponent, bit 0 mantissa; magnitudes 0, 0.5, 1, 1.5, 2, 3, 4, 6 -- packed 8
// per u32 LSB-first like 4-bit affine codes, and one E8M0 scale byte per 32
// values: 2^(e - 127), e = 255 is NaN.
__device__ __forceinline__ float e2m1_to_f32(uint32_t c) {
    const uint32_t m = c & 7u;
    // m >= 2: 2^(m/2 - 1) * (1 + (m & 1) / 2) as f32 bits; m = 1: 0.5; m = 0: 0
    uint32_t bits = ((126u + (m >> 1)) << 23) | ((m & 1u) << 22);
    bits = m >= 2u ? bits : (m == 1u ? 0x3F000000u : 0u);
    return __uint_as_float(bits | ((c & 8u) << 28));
}
__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
    e &= 0xffu;
    return __uint_as_float(e == 255u ? 0x7FC00000u : (e == 0u ? 0x00400000u : e << 23));
}
template <> __device__ __forceinline__ float load_param<E8M0T>(const uint8_t* p, int64_t i) { return e8m0_to_f32(p[i]); }

// The 8 E2M1 codes of a word (LSB-first) times `scale`, as 4 bf16 pairs in
// code order (c0, c1), (c2, c3), ...: v_cvt_scalef32_pk_bf16_fp4, which reads
// only the exponent field of `scale` (2^(field - 127), field 255 giving NaN).
// With scale = e8m0_to_f32(e) that is 2^(e - 127) for every byte e, byte 0's
// subnormal image included; the products are exact in bf16 (two significant
// bits) down to its subnormals.
__device__ __forceinline__ void e2m1x8_to_bf16(uint32_t w, float scale, uint32_t* p) {
    p[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0));
    p[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1));
    p[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2));
    p[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3));
}

// Two 4-bit codes n0, n1 as the bf16 pair (128 + n0, 128 + n1): 128 = 0x4300
// has a unit ulp, so OR-ing n into the mantissa is exact.
constexpr uint32_t kNibbleMagic = 0x43004300u;
constexpr uint32_t kBf16Ones = 0x3f803f80u;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}


// ------------------------------------------------------------ gather / batch

// Batch indirection of gather_qmm (and of batched transpose = false launches):
// output batch b reads x batch lhs[b] and weight batch rhs[b].
struct GatherIdx {
    const int32_t* lhs;  // null: batch b reads x batch b (or 0 when x has one)
    const int32_t* rhs;  // null: batch b reads w batch b (or 0 when w has one)
    int64_t x_batches, w_batches;
};

// MXFP4 matmul (mxfp4.hip): y[b] = x[lhs(b)] . dequant(w[rhs(b)])^T (or
// without the transpose) for every output batch b of `batch`; the plain
// matmul is batch 1 with no indices.  sorted: ascending rhs indices promised
// (gather_qmm's hint).  Split-K scratch from `ws` (null: the library
// workspace).  Validated by the callers.
struct WsSource;
int mxfp4_matmul(void* y, const void* x, const uint32_t* w, const uint8_t* scales, const GatherIdx& g,
                 int64_t batch, int64_t M, int64_t N, int64_t K, bool transpose, int x_dtype, bool sorted,
                 const WsSource* ws, hipStream_t st);

// The operand batches of output batch b; false if an index is out of range.
__device__ __forceinline__ bool gather_batch(const GatherIdx& g, int64_t b, int64_t& xb, int64_t& wb) {
    xb = g.lhs ? int64_t(g.lhs[b]) : (g.x_batches == 1 ? 0 : b);
    wb = g.rhs ? int64_t(g.rhs[b]) : (g.w_batches == 1 ? 0 : b);
    return xb >= 0 && xb < g.x_batches && wb >= 0 && wb < g.w_batches;
}

// Where a launch's scratch memory comes from: a fixed region (ptr, cap) that
// the caller owns, or, for a null WsSource*, the library's workspace of the
// current device and `st` (workspace.hip: grow-only, never freed while the
// process runs, one buffer per stream).
struct WsSource {
    void* ptr;
    size_t cap;
    unsigned* counters;  // kWsCounters zeroed 32-bit words that kernels leave zeroed
};

// Arrival counters of one stream (or fixed region): last-arriver kernels
// count their workgroups here and reset each counter they used, so the words
// are zero between launches.
constexpr int kWsCounters = 16384;

// At least `bytes` of device scratch, 256-byte aligned, or null when none can
// be provided (fixed region too small, or the library buffer would have to
// grow while `st` is capturing).  Launches that use it are ordered on `st`.
void* ws_acquire(const WsSource* src, size_t bytes, hipStream_t st);

// The kWsCounters arrival counters of `src` (null: the library's, one
// zero-filled buffer per device and stream, used for nothing else), or null
// when they cannot be provided (first use while `st` is capturing).
unsigned* ws_counters(const WsSource* src, hipStream_t st);

// Routed experts over sorted expert indices (gather_qmm with sorted_indices,
// transpose, one activation row per route, bf16 x, 4/8-bit, bf16/f16
// scales): y [batch, N] zeroed, rows x[lhs[b]] gathered into the workspace,
// a device-built list of (expert, 128-row tile) entries, and one MFMA qmm
// launch over the list, so each expert's weights are read once per 128
// routes instead of once per route.  N a multiple of 128, K of 64, x and w
// 16-byte aligned, y 8-byte aligned.  False (nothing launched) when the
// workspace cannot be provided or the combination has no kernel.
bool launch_qmm_grouped(int bits, int gs, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w,
                        const void* s, const void* b, const int32_t* lhs, const int32_t* rhs, int batch,
                        int64_t x_batches, int experts, int N, int K, hipStream_t st,
                        const WsSource* src = nullptr);

// Everything of eq_gather_qmm after argument validation (gather.hip); `src`
// (or the stream's workspace when null) holds the grouped path's scratch.
int gather_qmm_launch(void* y, const void* x, const uint32_t* w, const void* scales, const void* biases,
                      const int32_t* lhs_indices, const int32_t* rhs_indices, int64_t batch, int64_t x_batches,
                      int64_t w_batches, int64_t M, int64_t N, int64_t K, bool transpose, int group_size, int bits,
                      QuantMode qm, int x_dtype, int scale_dtype, bool sorted_indices, const WsSource* src,
                      hipStream_t st);

// Prefill qmm (qmm.hip): M > 16, x bf16, transpose, 4/8-bit, bf16/f16 scales,
// N % 128 == 0, K % 64 == 0, 16-byte aligned x and w, 8-byte aligned y.  Any
// buffer size: launches are split so that every buffer offset fits 32 bits.
// Split K takes its partial tiles from `ws` (null: the library workspace);
// without room for them the launch runs unsplit.  Bits 4 and 8 at group 16,
// 32, 64 or 128; bits 2, 3, 5 and 6 (4-byte aligned w) re-pack their codes
// to bytes in `ws` slice by slice and run the 8-bit kernel (false when no
// workspace can be had).  y's row stride is ldy (N when negative; split K
// only when it is N).
bool launch_qmm_mfma(int bits, int gs, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w,
                     const void* s, const void* b, int M, int N, int K, const WsSource* ws, hipStream_t st,
                     int ldy = -1, int x_dtype = EQ_DTYPE_BF16);

// The same two launchers for MXFP4 codes (E8M0 scale bytes, no biases).
bool launch_qmm_mfma_mxfp4(uint16_t* y, const uint16_t* x, const uint32_t* w, const uint8_t* s, int M, int N, int K,
                           const WsSource* ws, hipStream_t st);
bool launch_qmm_grouped_mxfp4(uint16_t* y, const uint16_t* x, const uint32_t* w, const uint8_t* s,
                              const int32_t* lhs, const int32_t* rhs, int batch, int64_t x_batches, int experts, int N,
                              int K, hipStream_t st);

// Routed-expert decode for MXFP4 (gather.hip's per-route kernel): transpose,
// M = 1, bf16 x, 16-byte aligned x and w; batches b0 .. b0 + nb of g.
void launch_gather_qmv_mxfp4(uint16_t* y, const uint16_t* x, const uint32_t* w, const uint8_t* s, const GatherIdx& g,
                             int64_t b0, unsigned nb, int N, int K, hipStream_t st);

// x . W for W [K, N] packed along N (transpose = false), M <= 8 activation
// rows per batch, bf16 x and y, bf16/f16 scales, 4- or 8-bit codes, or MXFP4
// (scale_dtype EQ_DTYPE_U8, bits 4, gs 32, b null); batches through g (y
// [batch, M, N]).  False (nothing launched) for other combinations.
bool launch_qmm_n_small(int bits, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s,
                        const void* b, const GatherIdx& g, int64_t batch, int M, int N, int K, int gs,
                        const WsSource* ws, hipStream_t st);

// The same for one product of any M (batch 1, no indices): launches of 8
// activation rows per batch (the rows as M / 8 batches over one weight
// matrix), then the remaining rows.  Each launch reads W once, so the codes
// are read ceil(M / 8) times: for the small M of transpose = false callers.
constexpr int64_t kQmmNRowsMax = int64_t(1) << 20;
bool launch_qmm_n_rows(int bits, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w, const void* s,
                       const void* b, int64_t M, int N, int K, int gs, const WsSource* ws, hipStream_t st);

// ------------------------------------------------------------ general bodies

// LSB-first code c of a packed row (codes of 2, 4 or 8 bits never straddle words).
template <int BITS>
__device__ __forceinline__ uint32_t code_at(const uint32_t* row, int64_t c) {
    if constexpr (32 % BITS == 0) {
        constexpr int PACK = 32 / BITS;
        return (row[c / PACK] >> ((c % PACK) * BITS)) & ((1u << BITS) - 1u);
    } else {
        // 3-, 5- and 6-bit codes: an LSB-first bit stream whose codes may
        // straddle two words (eredu-gguf/src/convert.rs:413-427 `pack`)
        const int64_t bit = c * BITS;
        const int sh = int(bit & 31);
        uint32_t v = row[bit >> 5] >> sh;
        if (sh + BITS > 32) v |= row[(bit >> 5) + 1] << (32 - sh);
        return v & ((1u << BITS) - 1u);
    }
}

constexpr int kGenRowsPerWG = 4;
constexpr int kGenMChunk = 8;
constexpr int64_t kMaxGridY = 65535;  // largest grid y / z dimension of a launch

// transpose = true, output feature n by one wave (lane = 0..63): lanes stride
// over K, activations in chunks of kGenMChunk rows, f32 arithmetic
// throughout, y[m, n] written by lane 0.
template <int BITS, typename XT, typename ST>
__device__ __forceinline__ void qmm_t_rows(typename XT::storage* __restrict__ y,
                                           const typename XT::storage* __restrict__ x, const uint32_t* __restrict__ w,
                                           const typename ST::storage* __restrict__ s,
                                           const typename ST::storage* __restrict__ b, int64_t M, int64_t N,
                                           int64_t K, int gs, int64_t n, int lane) {
    const int64_t G = K / gs;
    const uint32_t* row = w + n * (K * BITS / 32);
    for (int64_t m0 = 0; m0 < M; m0 += kGenMChunk) {
        float acc[kGenMChunk];
#pragma unroll
        for (int i = 0; i < kGenMChunk; i++) acc[i] = 0.f;
        for (int64_t k = lane; k < K; k += 64) {
            const int64_t g = k / gs;
            const float wv = load_param<ST>(s, n * G + g) * float(code_at<BITS>(row, k)) +
                             (b ? load_param<ST>(b, n * G + g) : 0.f);
#pragma unroll
            for (int i = 0; i < kGenMChunk; i++)
                if (m0 + i < M) acc[i] = fmaf(load_param<XT>(x, (m0 + i) * K + k), wv, acc[i]);
        }
#pragma unroll
        for (int i = 0; i < kGenMChunk; i++) {
            float v = acc[i];
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
            if (lane == 0 && m0 + i < M) store_out<XT>(y, (m0 + i) * N + n, v);
        }
    }
}

// transpose = false (W [K, N] packed along N): output column n for the
// activation rows m0 .. m0 + kGenMChunk - 1, walking K.
template <int BITS, typename XT, typename ST>
__device__ __forceinline__ void qmm_n_cols(typename XT::storage* __restrict__ y,
                                           const typename XT::storage* __restrict__ x, const uint32_t* __restrict__ w,
                                           const typename ST::storage* __restrict__ s,
                                           const typename ST::storage* __restrict__ b, int64_t M, int64_t N,
                                           int64_t K, int gs, int64_t n, int64_t m0) {
    const int64_t G = N / gs;
    float acc[kGenMChunk];
#pragma unroll
    for (int i = 0; i < kGenMChunk; i++) acc[i] = 0.f;
    for (int64_t k = 0; k < K; k++) {
        const uint32_t* row = w + k * (N * BITS / 32);
        const float wv = load_param<ST>(s, k * G + n / gs) * float(code_at<BITS>(row, n)) +
                         (b ? load_param<ST>(b, k * G + n / gs) : 0.f);
#pragma unroll
        for (int i = 0; i < kGenMChunk; i++)
            if (m0 + i < M) acc[i] = fmaf(load_param<XT>(x, (m0 + i) * K + k), wv, acc[i]);
    }
#pragma unroll
    for (int i = 0; i < kGenMChunk; i++)
        if (m0 + i < M) store_out<XT>(y, (m0 + i) * N + n, acc[i]);
}

}  // namespace eq
