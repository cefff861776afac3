// Decode-step kernels around the quantized projections of a Llama-shaped
// decoder layer at batch 1 (bf16 activations):
//
//   eq_rms_norm            hidden += residual; out = RMSNorm(hidden) * weight
//                          (TransformerBlock::forward, eredu-architectures/src/llama.rs:477-495;
//                          nn::RmsNorm / fast::rms_norm, safemlx/src/fast.rs:1119)
//   eq_rope_attention_decode
//                          RoPE of q and the new k at `pos` (Llama3Rope::forward,
//                          eredu/src/backend/mlx/nn/rope.rs:188-216), the new k/v
//                          written into the cache (update_for_attention), then
//                          softmax(scale q.k) . v over positions 0..pos with grouped
//                          KV heads (Attention::attend, llama.rs:296-330;
//                          fast::scaled_dot_product_attention)
//   eq_silu_mul            silu(gate) * up (Mlp::hidden, llama.rs:414-422;
//                          silu = x * sigmoid(x), eredu/src/backend/mlx/nn/layers.rs:21)
//   eq_embedding           rows of a bf16 table by device token ids (Decoder::embed)
//   eq_argmax              index of the largest logit (greedy decoding)
//
// Everything here is a small fraction of a decode step's bytes (the packed
// projections are ~97 %); the kernels aim at few launches and full-width
// loads, not at MFMA.
#include <math.h>

#include <mutex>

#include "eq_common.hpp"

namespace eq {
namespace {

constexpr int kHeadDim = 128;  // head width of the attention fast path
constexpr int kAttnChunk = 32; // cache positions per attention workgroup
constexpr int kRowPad = kHeadDim + 8;  // LDS row of keys/values: 272 B, so 32 rows spread over 16 banks

__device__ __forceinline__ float bf16_round(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

// Sum over a block of 1024 threads (16 waves); every thread gets the total.
__device__ __forceinline__ float block_sum_1024(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) t += red[i];  // same order in every thread
    __syncthreads();
    return t;
}

// One row per workgroup of 1024 threads; dim % 8 == 0 (16-byte vectors).
__global__ __launch_bounds__(1024) void rms_norm_kernel(uint16_t* __restrict__ out, uint16_t* __restrict__ x,
                                                        const uint16_t* __restrict__ residual,
                                                        const uint16_t* __restrict__ weight, int dim, float eps) {
    __shared__ float red[16];
    const int64_t row = blockIdx.x;
    uint16_t* xr = x + row * dim;
    const uint16_t* rr = residual ? residual + row * dim : nullptr;
    uint16_t* orow = out + row * dim;
    const int nvec = dim / 8;
    float ss = 0.f;
    for (int v = threadIdx.x; v < nvec; v += 1024) {
        uint4 a = reinterpret_cast<const uint4*>(xr)[v];
        if (rr) {
            const uint4 b = reinterpret_cast<const uint4*>(rr)[v];
            uint32_t* pa = reinterpret_cast<uint32_t*>(&a);
            const uint32_t* pb = reinterpret_cast<const uint32_t*>(&b);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float lo = bf16_bits_to_f32(pa[i] & 0xffffu) + bf16_bits_to_f32(pb[i] & 0xffffu);
                const float hi = bf16_bits_to_f32(pa[i] >> 16) + bf16_bits_to_f32(pb[i] >> 16);
                pa[i] = f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
            }
            reinterpret_cast<uint4*>(xr)[v] = a;
        }
        const uint32_t* pa = reinterpret_cast<const uint32_t*>(&a);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float lo = bf16_bits_to_f32(pa[i] & 0xffffu), hi = bf16_bits_to_f32(pa[i] >> 16);
            ss = fmaf(lo, lo, ss);
            ss = fmaf(hi, hi, ss);
        }
    }
    const float total = block_sum_1024(ss, red);
    const float inv = 1.0f / sqrtf(total / float(dim) + eps);
    for (int v = threadIdx.x; v < nvec; v += 1024) {
        const uint4 a = reinterpret_cast<const uint4*>(xr)[v];  // this thread's own (updated) values
        const uint4 w = reinterpret_cast<const uint4*>(weight)[v];
        const uint32_t* pa = reinterpret_cast<const uint32_t*>(&a);
        const uint32_t* pw = reinterpret_cast<const uint32_t*>(&w);
        uint4 o;
        uint32_t* po = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float lo = bf16_bits_to_f32(pw[i] & 0xffffu) * (bf16_bits_to_f32(pa[i] & 0xffffu) * inv);
            const float hi = bf16_bits_to_f32(pw[i] >> 16) * (bf16_bits_to_f32(pa[i] >> 16) * inv);
            po[i] = f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
        }
        reinterpret_cast<uint4*>(orow)[v] = o;
    }
}

// Non-traditional (half-split) rotation of one head held in LDS as f32:
// out[i] = x[i] cos - x[i+h] sin, out[i+h] = x[i+h] cos + x[i] sin, angle
// pos / freqs[i] (Llama3Rope::forward).  128 threads per head.
__device__ __forceinline__ void rope_pair(float* head, const float* __restrict__ freqs, float pos, int i) {
    const float a = pos / freqs[i];
    float s, c;
    sincosf(a, &s, &c);
    const float x1 = head[i], x2 = head[i + kHeadDim / 2];
    head[i] = x1 * c - x2 * s;
    head[i + kHeadDim / 2] = x2 * c + x1 * s;
}

// One workgroup (256 threads, 4 waves) per (KV head, chunk of 32 positions):
// the query heads of the group (q rotated here), the chunk's keys and values
// staged in LDS, partial softmax state (max, sum, weighted values) written
// to the workspace for the combine pass.  The chunk that holds `pos` also
// rotates the new key and stores it and the new value into the cache; no
// other workgroup reads position `pos`.
__global__ __launch_bounds__(256) void attn_partial_kernel(float* __restrict__ ws, const uint16_t* __restrict__ q,
                                                           const uint16_t* __restrict__ k_new,
                                                           const uint16_t* __restrict__ v_new,
                                                           uint16_t* __restrict__ k_cache,
                                                           uint16_t* __restrict__ v_cache,
                                                           const float* __restrict__ freqs, int pos, int max_seq,
                                                           int n_heads, int n_kv_heads, int nchunks, float scale) {
    __shared__ float qs[4][kHeadDim];                            // rotated queries of this group
    __shared__ __attribute__((aligned(16))) uint16_t ks[kAttnChunk][kRowPad];
    __shared__ __attribute__((aligned(16))) uint16_t vs[kAttnChunk][kRowPad];
    __shared__ float knew[kHeadDim];
    const int g = blockIdx.x, c = blockIdx.y;
    const int group = n_heads / n_kv_heads;  // <= 4
    const int p0 = c * kAttnChunk, np = min(kAttnChunk, pos + 1 - p0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float fpos = float(pos);

    // queries of the group, rotated
    for (int i = tid; i < group * kHeadDim; i += 256)
        qs[i / kHeadDim][i % kHeadDim] = bf16_bits_to_f32(q[(int64_t(g) * group + i / kHeadDim) * kHeadDim + i % kHeadDim]);
    const bool has_new = pos >= p0 && pos < p0 + kAttnChunk;
    if (has_new && tid < kHeadDim) knew[tid] = bf16_bits_to_f32(k_new[int64_t(g) * kHeadDim + tid]);
    __syncthreads();
    for (int i = tid; i < group * (kHeadDim / 2); i += 256) rope_pair(qs[i / (kHeadDim / 2)], freqs, fpos, i % (kHeadDim / 2));
    if (has_new && tid < kHeadDim / 2) rope_pair(knew, freqs, fpos, tid);
    __syncthreads();

    // keys and values of the chunk (16-byte pieces); position pos from the new ones
    uint16_t* kc = k_cache + int64_t(g) * max_seq * kHeadDim;
    uint16_t* vc = v_cache + int64_t(g) * max_seq * kHeadDim;
    for (int i = tid; i < np * (kHeadDim / 8); i += 256) {
        const int p = i / (kHeadDim / 8), v = i % (kHeadDim / 8);
        uint4 kk, vv;
        if (p0 + p == pos) {
            uint32_t* pk = reinterpret_cast<uint32_t*>(&kk);
#pragma unroll
            for (int e = 0; e < 4; e++)
                pk[e] = f32_to_bf16_bits(knew[8 * v + 2 * e]) | (f32_to_bf16_bits(knew[8 * v + 2 * e + 1]) << 16);
            vv = reinterpret_cast<const uint4*>(v_new + int64_t(g) * kHeadDim)[v];
            reinterpret_cast<uint4*>(kc + int64_t(pos) * kHeadDim)[v] = kk;
            reinterpret_cast<uint4*>(vc + int64_t(pos) * kHeadDim)[v] = vv;
        } else {
            kk = reinterpret_cast<const uint4*>(kc + int64_t(p0 + p) * kHeadDim)[v];
            vv = reinterpret_cast<const uint4*>(vc + int64_t(p0 + p) * kHeadDim)[v];
        }
        reinterpret_cast<uint4*>(&ks[p][0])[v] = kk;
        reinterpret_cast<uint4*>(&vs[p][0])[v] = vv;
    }
    __syncthreads();

    // wave h: query head g*group + h.  Scores: lane = position (p < 32) x half
    // of the dimensions (lane / 32), summed over the pair.
    for (int h = wave; h < group; h += 4) {
        const int p = lane & 31, half = lane >> 5;
        float s = 0.f;
        if (p < np) {
            const uint32_t* kr = reinterpret_cast<const uint32_t*>(&ks[p][half * (kHeadDim / 2)]);
            const float* qh = &qs[h][half * (kHeadDim / 2)];
#pragma unroll 8
            for (int d = 0; d < kHeadDim / 4; d++) {
                const uint32_t kk = kr[d];
                s = fmaf(qh[2 * d], bf16_bits_to_f32(kk & 0xffffu), s);
                s = fmaf(qh[2 * d + 1], bf16_bits_to_f32(kk >> 16), s);
            }
        }
        s += __shfl_xor(s, 32);
        s = p < np ? s * scale : -INFINITY;
        float m = s;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        const float e = p < np ? expf(s - m) : 0.f;
        float l = e;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) l += __shfl_xor(l, o);
        // weighted values: lane owns dimensions 2 lane, 2 lane + 1
        float o0 = 0.f, o1 = 0.f;
        for (int pp = 0; pp < np; pp++) {
            const float w = __shfl(e, pp);
            const uint32_t vv = reinterpret_cast<const uint32_t*>(&vs[pp][0])[lane];
            o0 = fmaf(w, bf16_bits_to_f32(vv & 0xffffu), o0);
            o1 = fmaf(w, bf16_bits_to_f32(vv >> 16), o1);
        }
        float* dst = ws + (int64_t(g * group + h) * nchunks + c) * (kHeadDim + 2);
        if (lane == 0) {
            dst[0] = m;
            dst[1] = l;
        }
        dst[2 + 2 * lane] = o0;
        dst[3 + 2 * lane] = o1;
    }
}

// One workgroup of 128 threads per query head: the chunks' partial states
// merged in chunk order, divided by the total weight, rounded to bf16.
__global__ __launch_bounds__(128) void attn_combine_kernel(uint16_t* __restrict__ out, const float* __restrict__ ws,
                                                           int nchunks) {
    const int h = blockIdx.x, d = threadIdx.x;
    const float* base = ws + int64_t(h) * nchunks * (kHeadDim + 2);
    float mx = -INFINITY;
    for (int c = 0; c < nchunks; c++) mx = fmaxf(mx, base[c * (kHeadDim + 2)]);
    float l = 0.f, o = 0.f;
    for (int c = 0; c < nchunks; c++) {
        const float* p = base + c * (kHeadDim + 2);
        const float f = expf(p[0] - mx);
        l = fmaf(f, p[1], l);
        o = fmaf(f, p[2 + d], o);
    }
    out[int64_t(h) * kHeadDim + d] = uint16_t(f32_to_bf16_bits(o / l));
}

// silu(gate) * up with the reference's roundings: sigmoid, the product with
// gate and the product with up each round to bf16.  8 values per thread.
__global__ __launch_bounds__(256) void silu_mul_kernel(uint16_t* __restrict__ out, const uint16_t* __restrict__ gate,
                                                       const uint16_t* __restrict__ up, int64_t nvec) {
    const int64_t v = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (v >= nvec) return;
    const uint4 gg = reinterpret_cast<const uint4*>(gate)[v];
    const uint4 uu = reinterpret_cast<const uint4*>(up)[v];
    const uint32_t* pg = reinterpret_cast<const uint32_t*>(&gg);
    const uint32_t* pu = reinterpret_cast<const uint32_t*>(&uu);
    uint4 o;
    uint32_t* po = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t r = 0;
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const float x = bf16_bits_to_f32((pg[i] >> (16 * hh)) & 0xffffu);
            const float u = bf16_bits_to_f32((pu[i] >> (16 * hh)) & 0xffffu);
            const float sg = bf16_round(1.0f / (1.0f + expf(-x)));
            const float sl = bf16_round(x * sg);
            r |= f32_to_bf16_bits(sl * u) << (16 * hh);
        }
        po[i] = r;
    }
    reinterpret_cast<uint4*>(out)[v] = o;
}

// Row tokens[t] of the table (zeros for an id outside [0, vocab)).
__global__ __launch_bounds__(256) void embedding_kernel(uint16_t* __restrict__ out, const uint16_t* __restrict__ table,
                                                        const int32_t* __restrict__ tokens, int64_t vocab,
                                                        int64_t dim) {
    const int64_t t = blockIdx.y;
    const int32_t id = tokens[t];
    const int64_t nvec = dim / 8;
    for (int64_t v = int64_t(blockIdx.x) * 256 + threadIdx.x; v < nvec; v += int64_t(gridDim.x) * 256) {
        uint4 r = make_uint4(0, 0, 0, 0);
        if (id >= 0 && id < vocab) r = reinterpret_cast<const uint4*>(table + int64_t(id) * dim)[v];
        reinterpret_cast<uint4*>(out + t * dim)[v] = r;
    }
}

// First index of the largest value of each row (1024 threads per row).
__global__ __launch_bounds__(1024) void argmax_kernel(int32_t* __restrict__ out, const uint16_t* __restrict__ logits,
                                                      int64_t n) {
    __shared__ float bv[16];
    __shared__ int64_t bi[16];
    const uint16_t* row = logits + int64_t(blockIdx.x) * n;
    float best = -INFINITY;
    int64_t idx = n;  // none yet
    for (int64_t i = threadIdx.x; i < n; i += 1024) {
        const float v = bf16_bits_to_f32(row[i]);
        if (v > best || idx == n) {
            best = v;
            idx = i;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o);
        const int64_t oi = __shfl_xor(idx, o);
        if (ov > best || (ov == best && oi < idx)) {
            best = ov;
            idx = oi;
        }
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) {
        bv[wave] = best;
        bi[wave] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = bv[0];
        int64_t k = bi[0];
        for (int w = 1; w < 16; w++)
            if (bv[w] > b || (bv[w] == b && bi[w] < k)) {
                b = bv[w];
                k = bi[w];
            }
        out[blockIdx.x] = int32_t(k < n ? k : 0);
    }
}

// Per-device f32 workspace of the attention partials, grown outside stream
// capture (a capturing call whose workspace is too small fails).
float* attn_workspace(size_t bytes, hipStream_t st) {
    static std::mutex mu;
    static float* ptr[64] = {};
    static size_t cap[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (cap[dev] >= bytes) return ptr[dev];
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
    if (ptr[dev]) {
        if (hipDeviceSynchronize() != hipSuccess) return nullptr;
        (void)hipFree(ptr[dev]);
        ptr[dev] = nullptr;
        cap[dev] = 0;
    }
    void* p = nullptr;
    const size_t want = bytes < (size_t(4) << 20) ? (size_t(4) << 20) : bytes;
    if (hipMalloc(&p, want) != hipSuccess) return nullptr;
    ptr[dev] = static_cast<float*>(p);
    cap[dev] = want;
    return ptr[dev];
}

bool bf16_only(int dtype, const char* what) {
    if (dtype != EQ_DTYPE_BF16) {
        set_error(std::string(what) + ": only bf16 is implemented");
        return false;
    }
    return true;
}

}  // namespace
}  // namespace eq

using namespace eq;

extern "C" int eq_rms_norm(void* out, void* x, const void* residual, const void* weight, int64_t rows, int64_t dim,
                           float eps, int dtype, eq_stream_t stream) {
    clear_error();
    if (!bf16_only(dtype, "eq_rms_norm")) return 1;
    if (!out || !x || !weight) {
        set_error("eq_rms_norm: null pointer argument");
        return 1;
    }
    if (rows < 0 || dim <= 0 || dim % 8 != 0 || dim > (int64_t(1) << 24) || rows > INT32_MAX) {
        set_error("eq_rms_norm: dim must be a positive multiple of 8 (at most 2^24), rows in [0, 2^31)");
        return 1;
    }
    if (!aligned(out, 16) || !aligned(x, 16) || !aligned(weight, 16) || (residual && !aligned(residual, 16))) {
        set_error("eq_rms_norm: pointers must be 16-byte aligned");
        return 1;
    }
    if (!(eps >= 0.f)) {
        set_error("eq_rms_norm: eps must be >= 0");
        return 1;
    }
    if (rows == 0) return 0;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    rms_norm_kernel<<<dim3(unsigned(rows)), dim3(1024), 0, st>>>(
        static_cast<uint16_t*>(out), static_cast<uint16_t*>(x), static_cast<const uint16_t*>(residual),
        static_cast<const uint16_t*>(weight), int(dim), eps);
    return check_launch("eq_rms_norm");
}

extern "C" int eq_rope_attention_decode(void* out, const void* q, const void* k_new, const void* v_new,
                                        void* k_cache, void* v_cache, const float* freqs, int64_t pos,
                                        int64_t max_seq, int n_heads, int n_kv_heads, int head_dim, float scale,
                                        int dtype, eq_stream_t stream) {
    clear_error();
    if (!bf16_only(dtype, "eq_rope_attention_decode")) return 1;
    if (!out || !q || !k_new || !v_new || !k_cache || !v_cache || !freqs) {
        set_error("eq_rope_attention_decode: null pointer argument");
        return 1;
    }
    if (head_dim != kHeadDim) {
        set_error("eq_rope_attention_decode: head_dim must be 128");
        return 1;
    }
    if (n_kv_heads <= 0 || n_heads <= 0 || n_heads % n_kv_heads != 0 || n_heads / n_kv_heads > 4 ||
        n_kv_heads > 65535) {
        set_error("eq_rope_attention_decode: n_heads must be 1-4 times n_kv_heads");
        return 1;
    }
    if (pos < 0 || max_seq <= 0 || pos >= max_seq || max_seq > (int64_t(1) << 24)) {
        set_error("eq_rope_attention_decode: need 0 <= pos < max_seq <= 2^24");
        return 1;
    }
    if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(v_new, 16)) {
        set_error("eq_rope_attention_decode: cache and value pointers must be 16-byte aligned");
        return 1;
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int nchunks = int((pos + kAttnChunk) / kAttnChunk);
    const size_t ws_bytes = size_t(n_heads) * size_t(nchunks) * (kHeadDim + 2) * sizeof(float);
    float* ws = attn_workspace(ws_bytes, st);
    if (!ws) {
        set_error("eq_rope_attention_decode: no workspace (first call must not be under stream capture)");
        return 1;
    }
    attn_partial_kernel<<<dim3(unsigned(n_kv_heads), unsigned(nchunks)), dim3(256), 0, st>>>(
        ws, static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k_new), static_cast<const uint16_t*>(v_new),
        static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), freqs, int(pos), int(max_seq), n_heads,
        n_kv_heads, nchunks, scale);
    attn_combine_kernel<<<dim3(unsigned(n_heads)), dim3(kHeadDim), 0, st>>>(static_cast<uint16_t*>(out), ws, nchunks);
    return check_launch("eq_rope_attention_decode");
}

extern "C" int eq_silu_mul(void* out, const void* gate, const void* up, int64_t n, int dtype, eq_stream_t stream) {
    clear_error();
    if (!bf16_only(dtype, "eq_silu_mul")) return 1;
    if (!out || !gate || !up) {
        set_error("eq_silu_mul: null pointer argument");
        return 1;
    }
    if (n < 0 || n % 8 != 0 || !aligned(out, 16) || !aligned(gate, 16) || !aligned(up, 16)) {
        set_error("eq_silu_mul: n must be a multiple of 8 and pointers 16-byte aligned");
        return 1;
    }
    if (n == 0) return 0;
    const int64_t nvec = n / 8;
    if ((nvec + 255) / 256 > INT32_MAX) {
        set_error("eq_silu_mul: n too large");
        return 1;
    }
    silu_mul_kernel<<<dim3(unsigned((nvec + 255) / 256)), dim3(256), 0, reinterpret_cast<hipStream_t>(stream)>>>(
        static_cast<uint16_t*>(out), static_cast<const uint16_t*>(gate), static_cast<const uint16_t*>(up), nvec);
    return check_launch("eq_silu_mul");
}

extern "C" int eq_embedding(void* out, const void* table, const int32_t* tokens, int64_t n_tokens, int64_t vocab,
                            int64_t dim, int dtype, eq_stream_t stream) {
    clear_error();
    if (!bf16_only(dtype, "eq_embedding")) return 1;
    if (!out || !table || !tokens) {
        set_error("eq_embedding: null pointer argument");
        return 1;
    }
    if (n_tokens < 0 || n_tokens > 65535 || vocab <= 0 || dim <= 0 || dim % 8 != 0 || !aligned(out, 16) ||
        !aligned(table, 16)) {
        set_error("eq_embedding: need 0 <= n_tokens <= 65535, dim a positive multiple of 8, 16-byte aligned rows");
        return 1;
    }
    if (n_tokens == 0) return 0;
    const int64_t nvec = dim / 8;
    const unsigned gx = unsigned(nvec < 256 * 64 ? (nvec + 255) / 256 : 64);
    embedding_kernel<<<dim3(gx, unsigned(n_tokens)), dim3(256), 0, reinterpret_cast<hipStream_t>(stream)>>>(
        static_cast<uint16_t*>(out), static_cast<const uint16_t*>(table), tokens, vocab, dim);
    return check_launch("eq_embedding");
}

extern "C" int eq_argmax(int32_t* out, const void* logits, int64_t rows, int64_t n, int dtype, eq_stream_t stream) {
    clear_error();
    if (!bf16_only(dtype, "eq_argmax")) return 1;
    if (!out || !logits) {
        set_error("eq_argmax: null pointer argument");
        return 1;
    }
    if (rows < 0 || rows > INT32_MAX || n <= 0 || n > INT32_MAX) {
        set_error("eq_argmax: need 0 <= rows and 0 < n < 2^31");
        return 1;
    }
    if (rows == 0) return 0;
    argmax_kernel<<<dim3(unsigned(rows)), dim3(1024), 0, reinterpret_cast<hipStream_t>(stream)>>>(
        out, static_cast<const uint16_t*>(logits), n);
    return check_launch("eq_argmax");
}
