// Shared device helpers and host error plumbing for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/eredu_hip.h"

namespace eq {

// ------------------------------------------------------------------ host side

// Thread-local message of the last failed call (the mlx-c convention of
// safemlx/src/error.rs:239-269: status code plus a per-thread message).
void set_error(const std::string& msg);
void clear_error();

// Checks the launch status of the kernels just enqueued.
int check_launch(const char* what);

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
bool launch_qmv_mfma(int bits, int gs, int scale_dtype, uint16_t* y, const uint16_t* x, const uint32_t* w,
                     const void* s, const void* b, int M, int N, int K, hipStream_t st);
bool launch_qmv_batched(int bits, int gs, int scale_dtype, const QmvSpec* specs, int count, int M, hipStream_t st);

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

// Pulls every 64-byte line of a kernel's by-value argument block into the
// scalar cache with independent loads and one wait.  The block is cold at
// each dispatch; without this, code that indexes it with computed values
// (a problem table walked per tile) pays one memory round trip per line, in
// sequence, before its first useful load.
template <typename T>
__device__ __forceinline__ void prefetch_args(const T& args) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(&args);
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < int(sizeof(T) + 63) / 64; i++) acc ^= p[16 * i];
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
// crate's f16::from_f32 that eredu-gguf/src/convert.rs:409-411 uses.  Done in
// integer arithmetic so the result does not depend on the hardware mode bits.
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    uint32_t x = __float_as_uint(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) return sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u);
    int e = static_cast<int>(exp) - 112;  // rebias 127 -> 15
    if (e >= 0x1f) return sign | 0x7c00u;
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t m = man | 0x800000u;
        uint32_t shift = static_cast<uint32_t>(14 - e);
        uint32_t h = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (h & 1u))) h += 1u;
        return sign | h;
    }
    uint32_t h = (static_cast<uint32_t>(e) << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return sign | h;
}

// Scalar parameter loads for each scale/activation element type.
struct BF16T { typedef uint16_t storage; };
struct F16T { typedef uint16_t storage; };
struct F32T { typedef float storage; };

template <typename T> __device__ __forceinline__ float load_param(const typename T::storage* p, int64_t i);
template <> __device__ __forceinline__ float load_param<BF16T>(const uint16_t* p, int64_t i) { return bf16_bits_to_f32(p[i]); }
template <> __device__ __forceinline__ float load_param<F16T>(const uint16_t* p, int64_t i) { return f16_bits_to_f32(p[i]); }
template <> __device__ __forceinline__ float load_param<F32T>(const float* p, int64_t i) { return p[i]; }

template <typename T> __device__ __forceinline__ void store_out(typename T::storage* p, int64_t i, float v);
template <> __device__ __forceinline__ void store_out<BF16T>(uint16_t* p, int64_t i, float v) { p[i] = static_cast<uint16_t>(f32_to_bf16_bits(v)); }
template <> __device__ __forceinline__ void store_out<F16T>(uint16_t* p, int64_t i, float v) { p[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v)); }
template <> __device__ __forceinline__ void store_out<F32T>(float* p, int64_t i, float v) { p[i] = v; }

}  // namespace eq
