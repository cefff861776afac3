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
constexpr int kMaxChunks = 4096;       // positions up to kMaxChunks * kAttnChunk = 131072

__device__ __forceinline__ float bf16_round(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

// Sum over the block (blockDim.x a multiple of 64, at most 1024); every
// thread gets the same total (the waves' sums added in wave order).
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}

// bf16 pair sums a + b, each rounded to bf16 (the residual add).
__device__ __forceinline__ uint4 add_bf16x8(uint4 a, const uint4 b) {
    uint32_t* pa = reinterpret_cast<uint32_t*>(&a);
    const uint32_t* pb = reinterpret_cast<const uint32_t*>(&b);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float lo = bf16_bits_to_f32(pa[i] & 0xffffu) + bf16_bits_to_f32(pb[i] & 0xffffu);
        const float hi = bf16_bits_to_f32(pa[i] >> 16) + bf16_bits_to_f32(pb[i] >> 16);
        pa[i] = f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
    }
    return a;
}

__device__ __forceinline__ float sumsq_bf16x8(const uint4 a) {
    const uint32_t* pa = reinterpret_cast<const uint32_t*>(&a);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float lo = bf16_bits_to_f32(pa[i] & 0xffffu), hi = bf16_bits_to_f32(pa[i] >> 16);
        ss = fmaf(lo, lo, ss);
        ss = fmaf(hi, hi, ss);
    }
    return ss;
}

__device__ __forceinline__ uint4 norm_bf16x8(const uint4 a, const uint4 w, float inv) {
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
    return o;
}

// One row per workgroup; dim % 8 == 0 (16-byte vectors).  VPT > 0: every
// thread keeps its (at most VPT) vectors in registers between the two passes;
// VPT == 0: any dim, the row is read again in the second pass.
template <int VPT>
__global__ __launch_bounds__(1024) void rms_norm_kernel(uint16_t* __restrict__ out, uint16_t* __restrict__ x,
                                                        const uint16_t* __restrict__ residual,
                                                        const uint16_t* __restrict__ weight, int dim, float eps) {
    __shared__ float red[16];
    const int64_t row = blockIdx.x;
    uint4* xr = reinterpret_cast<uint4*>(x + row * dim);
    const uint4* rr = residual ? reinterpret_cast<const uint4*>(residual + row * dim) : nullptr;
    uint4* orow = reinterpret_cast<uint4*>(out + row * dim);
    const uint4* wr = reinterpret_cast<const uint4*>(weight);
    const int nvec = dim / 8, step = blockDim.x;
    float ss = 0.f;
    if constexpr (VPT > 0) {
        uint4 a[VPT], w[VPT];
#pragma unroll
        for (int j = 0; j < VPT; j++) {
            const int v = threadIdx.x + j * step;
            if (v < nvec) {
                a[j] = xr[v];
                w[j] = wr[v];
                if (rr) {
                    a[j] = add_bf16x8(a[j], rr[v]);
                    xr[v] = a[j];
                }
                ss += sumsq_bf16x8(a[j]);
            }
        }
        const float inv = 1.0f / sqrtf(block_sum(ss, red) / float(dim) + eps);
#pragma unroll
        for (int j = 0; j < VPT; j++) {
            const int v = threadIdx.x + j * step;
            if (v < nvec) orow[v] = norm_bf16x8(a[j], w[j], inv);
        }
    } else {
        for (int v = threadIdx.x; v < nvec; v += step) {
            uint4 a = xr[v];
            if (rr) {
                a = add_bf16x8(a, rr[v]);
                xr[v] = a;
            }
            ss += sumsq_bf16x8(a);
        }
        const float inv = 1.0f / sqrtf(block_sum(ss, red) / float(dim) + eps);
        for (int v = threadIdx.x; v < nvec; v += step) orow[v] = norm_bf16x8(xr[v], wr[v], inv);  // own values
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
//
// pos_p, when not null, names the position in device memory (read when the
// kernel runs) and the grid covers every chunk of max_seq: workgroups of
// chunks past the position leave at once, and a position outside
// [0, max_seq) does nothing.  nchunks is the chunk stride of ws per head.
__global__ __launch_bounds__(256) void attn_partial_kernel(float* __restrict__ ws, const uint16_t* __restrict__ q,
                                                           const uint16_t* __restrict__ k_new,
                                                           const uint16_t* __restrict__ v_new,
                                                           uint16_t* __restrict__ k_cache,
                                                           uint16_t* __restrict__ v_cache,
                                                           const float* __restrict__ freqs, int pos_arg,
                                                           const int32_t* __restrict__ pos_p, int max_seq,
                                                           int n_heads, int n_kv_heads, int nchunks, float scale) {
    __shared__ float qs[4][kHeadDim];                            // rotated queries of this group
    __shared__ __attribute__((aligned(16))) uint16_t ks[kAttnChunk][kRowPad];
    __shared__ __attribute__((aligned(16))) uint16_t vs[kAttnChunk][kRowPad];
    __shared__ float knew[kHeadDim];
    const int g = blockIdx.x, c = blockIdx.y;
    const int pos = pos_p ? __builtin_amdgcn_readfirstlane(*pos_p) : pos_arg;
    if (pos < 0 || pos >= max_seq || c * kAttnChunk > pos) return;
    const int group = n_heads / n_kv_heads;  // <= 4
    const int p0 = c * kAttnChunk, np = min(kAttnChunk, pos + 1 - p0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float fpos = float(pos);

    // queries of the group, the new key (if this chunk holds pos) and the
    // chunk's cached keys and values, all requested before any waits
    for (int i = tid; i < group * kHeadDim; i += 256)
        qs[i / kHeadDim][i % kHeadDim] = bf16_bits_to_f32(q[(int64_t(g) * group + i / kHeadDim) * kHeadDim + i % kHeadDim]);
    const bool has_new = pos >= p0 && pos < p0 + kAttnChunk;
    if (has_new && tid < kHeadDim) knew[tid] = bf16_bits_to_f32(k_new[int64_t(g) * kHeadDim + tid]);
    uint16_t* kc = k_cache + int64_t(g) * max_seq * kHeadDim;
    uint16_t* vc = v_cache + int64_t(g) * max_seq * kHeadDim;
    for (int i = tid; i < np * (kHeadDim / 8); i += 256) {
        const int p = i / (kHeadDim / 8), v = i % (kHeadDim / 8);
        if (p0 + p == pos) continue;
        reinterpret_cast<uint4*>(&ks[p][0])[v] = reinterpret_cast<const uint4*>(kc + int64_t(p0 + p) * kHeadDim)[v];
        reinterpret_cast<uint4*>(&vs[p][0])[v] = reinterpret_cast<const uint4*>(vc + int64_t(p0 + p) * kHeadDim)[v];
    }
    __syncthreads();
    for (int i = tid; i < group * (kHeadDim / 2); i += 256) rope_pair(qs[i / (kHeadDim / 2)], freqs, fpos, i % (kHeadDim / 2));
    if (has_new && tid < kHeadDim / 2) rope_pair(knew, freqs, fpos, tid);
    __syncthreads();
    // position pos: the rotated new key (rounded to bf16) and the new value,
    // into LDS and into the cache
    if (has_new && tid < kHeadDim / 8) {
        const int p = pos - p0, v = tid;
        uint4 kk;
        uint32_t* pk = reinterpret_cast<uint32_t*>(&kk);
#pragma unroll
        for (int e = 0; e < 4; e++)
            pk[e] = f32_to_bf16_bits(knew[8 * v + 2 * e]) | (f32_to_bf16_bits(knew[8 * v + 2 * e + 1]) << 16);
        const uint4 vv = reinterpret_cast<const uint4*>(v_new + int64_t(g) * kHeadDim)[v];
        reinterpret_cast<uint4*>(kc + int64_t(pos) * kHeadDim)[v] = kk;
        reinterpret_cast<uint4*>(vc + int64_t(pos) * kHeadDim)[v] = vv;
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

// pos[0] += 1 (the next decode position), one thread.
__global__ void advance_position_kernel(int32_t* pos) { pos[0] += 1; }

// One workgroup of 256 threads per query head: the chunks' partial states
// (max, weight sum, weighted values) merged -- their maxima and rescale
// factors computed in parallel into LDS, then two halves of the threads sum
// alternate chunks for each dimension with independent loads -- divided by
// the total weight, rounded to bf16.
// With pos_p (device position) the chunk count comes from the position
// (zeros for one outside [0, max_seq)); ws holds `stride` chunks per head.
__global__ __launch_bounds__(256) void attn_combine_kernel(uint16_t* __restrict__ out, const float* __restrict__ ws,
                                                           int nchunks_arg, const int32_t* __restrict__ pos_p,
                                                           int max_seq, int stride) {
    __shared__ float fac[kMaxChunks];
    __shared__ float red[4];
    __shared__ float part[128];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int nchunks = nchunks_arg;
    if (pos_p) {
        const int pos = __builtin_amdgcn_readfirstlane(*pos_p);
        nchunks = pos >= 0 && pos < max_seq ? pos / kAttnChunk + 1 : 0;
        if (nchunks == 0) {
            if (tid < kHeadDim) out[int64_t(h) * kHeadDim + tid] = 0;
            return;
        }
    }
    const float* base = ws + int64_t(h) * stride * (kHeadDim + 2);
    float m = -INFINITY;
    for (int c = tid; c < nchunks; c += 256) m = fmaxf(m, base[c * (kHeadDim + 2)]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if (lane == 0) red[wave] = m;
    __syncthreads();
    const float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float l = 0.f;
    for (int c = tid; c < nchunks; c += 256) {
        const float f = expf(base[c * (kHeadDim + 2)] - mx);
        fac[c] = f;
        l = fmaf(f, base[c * (kHeadDim + 2) + 1], l);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o);
    if (lane == 0) red[wave] = l;
    __syncthreads();
    const float lsum = (red[0] + red[1]) + (red[2] + red[3]);
    const int d = tid & (kHeadDim - 1), half = tid >> 7;
    float o = 0.f;
#pragma unroll 8
    for (int c = half; c < nchunks; c += 2) o = fmaf(fac[c], base[c * (kHeadDim + 2) + 2 + d], o);
    if (half == 1) part[d] = o;
    __syncthreads();
    if (half == 0) out[int64_t(h) * kHeadDim + d] = uint16_t(f32_to_bf16_bits((o + part[d]) / lsum));
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
            const float sg = silu_sigmoid_bf16(x);
            const float sl = float(static_cast<__bf16>(x * sg));
            r |= uint32_t(__builtin_bit_cast(uint16_t, static_cast<__bf16>(sl * u))) << (16 * hh);
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

// First index of the largest value of each row (1024 threads per row):
// each thread scans 16-byte pieces (8 values) of the row in index order,
// four pieces in flight, then (value, index) pairs merge with ties to the
// lower index.
__device__ __forceinline__ void argmax_take(float v, int64_t i, float& best, int64_t& idx) {
    if (v > best || (v == best && i < idx)) {
        best = v;
        idx = i;
    }
}
__global__ __launch_bounds__(1024) void argmax_kernel(int32_t* __restrict__ out, const uint16_t* __restrict__ logits,
                                                      int64_t n, bool vec) {
    __shared__ float bv[16];
    __shared__ int64_t bi[16];
    const uint16_t* row = logits + int64_t(blockIdx.x) * n;
    float best = -INFINITY;
    int64_t idx = INT64_MAX;
    int64_t tail = 0;
    if (vec) {
        const int64_t nv = n / 8;
        const uint4* rv = reinterpret_cast<const uint4*>(row);
        int64_t v = threadIdx.x;
        for (; v + 3 * 1024 < nv; v += 4 * 1024) {
            uint4 a[4];
#pragma unroll
            for (int u = 0; u < 4; u++) a[u] = rv[v + u * 1024];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint32_t* pa = reinterpret_cast<const uint32_t*>(&a[u]);
#pragma unroll
                for (int e = 0; e < 8; e++)
                    argmax_take(bf16_bits_to_f32((pa[e >> 1] >> (16 * (e & 1))) & 0xffffu), (v + u * 1024) * 8 + e,
                                best, idx);
            }
        }
        for (; v < nv; v += 1024) {
            const uint4 a = rv[v];
            const uint32_t* pa = reinterpret_cast<const uint32_t*>(&a);
#pragma unroll
            for (int e = 0; e < 8; e++)
                argmax_take(bf16_bits_to_f32((pa[e >> 1] >> (16 * (e & 1))) & 0xffffu), v * 8 + e, best, idx);
        }
        tail = nv * 8;
    }
    for (int64_t i = tail + threadIdx.x; i < n; i += 1024) argmax_take(bf16_bits_to_f32(row[i]), i, best, idx);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o);
        const int64_t oi = __shfl_xor(idx, o);
        argmax_take(ov, oi, best, idx);
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
        for (int w = 1; w < 16; w++) argmax_take(bv[w], bi[w], b, k);
        out[blockIdx.x] = int32_t(k < n ? k : 0);
    }
}

bool bf16_only(int dtype, const char* what) {
    if (dtype != EQ_DTYPE_BF16) {
        set_error(std::string(what) + ": only bf16 is implemented");
        return false;
    }
    return true;
}

}  // namespace
// Multi-workgroup argmax of one row per blockIdx.y: workgroup blockIdx.x
// scans its slice (a multiple of 8 values, 16-byte pieces), reduces to its
// first largest value, and folds it into the row's 64-bit key with an atomic
// maximum -- key = (order-preserving image of the value) << 32 | (2^32 - 1 -
// index), so the largest value wins and, among equal values, the lowest
// index.  The last workgroup of the row (arrival counter) reads and clears the
// key and writes the index.  NaNs are skipped as argmax_take skips them; a
// row with nothing but NaNs gives index 0.
__global__ __launch_bounds__(256) void argmax_wide_kernel(int32_t* __restrict__ out,
                                                          const uint16_t* __restrict__ logits, int64_t n, int slice,
                                                          unsigned* __restrict__ counters,
                                                          unsigned long long* __restrict__ keys) {
    __shared__ float bv[4];
    __shared__ int64_t bi[4];
    __shared__ unsigned ticket;
    const int64_t row = blockIdx.y;
    const uint16_t* r = logits + row * n;
    const int64_t lo = int64_t(blockIdx.x) * slice, hi = lo + slice < n ? lo + slice : n;
    float best = -INFINITY;
    int64_t idx = INT64_MAX;
    const uint4* rv = reinterpret_cast<const uint4*>(r);
    for (int64_t v = lo / 8 + threadIdx.x; v < hi / 8; v += 256) {
        const uint4 a = rv[v];
        const uint32_t* pa = reinterpret_cast<const uint32_t*>(&a);
#pragma unroll
        for (int e = 0; e < 8; e++) argmax_take(bf16_bits_to_f32((pa[e >> 1] >> (16 * (e & 1))) & 0xffffu), v * 8 + e, best, idx);
    }
    for (int64_t i = hi / 8 * 8 + threadIdx.x; i < hi; i += 256) argmax_take(bf16_bits_to_f32(r[i]), i, best, idx);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o);
        const int64_t oi = __shfl_xor(idx, o);
        argmax_take(ov, oi, best, idx);
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) bv[wave] = best, bi[wave] = idx;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) argmax_take(bv[w], bi[w], best, idx);
        if (idx < n) {
            const uint32_t b = __float_as_uint(best);
            const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
            const unsigned long long key = (static_cast<unsigned long long>(ord) << 32) | (0xFFFFFFFFu - uint32_t(idx));
            __hip_atomic_fetch_max(keys + row, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (!last_arriver(counters + row, gridDim.x, &ticket)) return;
    if (threadIdx.x == 0) {
        const unsigned long long key = __hip_atomic_exchange(keys + row, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        out[row] = key ? int32_t(0xFFFFFFFFu - uint32_t(key & 0xFFFFFFFFull)) : 0;
    }
}

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
    const int nvec = int(dim / 8);
    const int block = nvec >= 1024 ? 1024 : (nvec + 63) / 64 * 64;
    const int vpt = (nvec + block - 1) / block;
    auto go = [&](auto kern) {
        kern<<<dim3(unsigned(rows)), dim3(unsigned(block)), 0, st>>>(
            static_cast<uint16_t*>(out), static_cast<uint16_t*>(x), static_cast<const uint16_t*>(residual),
            static_cast<const uint16_t*>(weight), int(dim), eps);
    };
    if (vpt == 1) go(rms_norm_kernel<1>);
    else if (vpt == 2) go(rms_norm_kernel<2>);
    else if (vpt <= 4) go(rms_norm_kernel<4>);
    else go(rms_norm_kernel<0>);
    return check_launch("eq_rms_norm");
}

// Validation shared by the two attention entry points; the number of
// position chunks on success.
static bool attention_args_ok(const char* name, const void* out, const void* q, const void* k_new,
                              const void* v_new, const void* k_cache, const void* v_cache, const float* freqs,
                              int64_t pos, int64_t max_seq, int n_heads, int n_kv_heads, int head_dim, int dtype) {
    const std::string who(name);
    if (!bf16_only(dtype, name)) return false;
    if (!out || !q || !k_new || !v_new || !k_cache || !v_cache || !freqs) {
        set_error(who + ": null pointer argument");
        return false;
    }
    if (head_dim != kHeadDim) {
        set_error(who + ": head_dim must be 128");
        return false;
    }
    if (n_kv_heads <= 0 || n_heads <= 0 || n_heads % n_kv_heads != 0 || n_heads / n_kv_heads > 4 ||
        n_kv_heads > 65535) {
        set_error(who + ": n_heads must be 1-4 times n_kv_heads");
        return false;
    }
    if (pos < 0 || max_seq <= 0 || pos >= max_seq || pos >= int64_t(kMaxChunks) * kAttnChunk) {
        set_error(who + ": need 0 <= pos < max_seq and pos < 131072");
        return false;
    }
    if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(v_new, 16)) {
        set_error(who + ": cache and value pointers must be 16-byte aligned");
        return false;
    }
    return true;
}

// The two attention passes: per-chunk partial softmax states into ws, then
// their combination per query head.
static void launch_attention(float* ws, void* out, const void* q, const void* k_new, const void* v_new, void* k_cache,
                             void* v_cache, const float* freqs, int64_t pos, int64_t max_seq, int n_heads,
                             int n_kv_heads, int nchunks, float scale, hipStream_t st) {
    attn_partial_kernel<<<dim3(unsigned(n_kv_heads), unsigned(nchunks)), dim3(256), 0, st>>>(
        ws, static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k_new), static_cast<const uint16_t*>(v_new),
        static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), freqs, int(pos), nullptr, int(max_seq),
        n_heads, n_kv_heads, nchunks, scale);
    attn_combine_kernel<<<dim3(unsigned(n_heads)), dim3(256), 0, st>>>(static_cast<uint16_t*>(out), ws, nchunks,
                                                                       nullptr, int(max_seq), nchunks);
}

static size_t attention_scratch_bytes(int64_t pos, int n_heads, int& nchunks) {
    nchunks = int((pos + kAttnChunk) / kAttnChunk);
    return size_t(n_heads) * size_t(nchunks) * (kHeadDim + 2) * sizeof(float);
}

extern "C" int eq_rope_attention_decode(void* out, const void* q, const void* k_new, const void* v_new,
                                        void* k_cache, void* v_cache, const float* freqs, int64_t pos,
                                        int64_t max_seq, int n_heads, int n_kv_heads, int head_dim, float scale,
                                        int dtype, eq_stream_t stream) {
    clear_error();
    if (!attention_args_ok("eq_rope_attention_decode", out, q, k_new, v_new, k_cache, v_cache, freqs, pos, max_seq,
                           n_heads, n_kv_heads, head_dim, dtype))
        return 1;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    int nchunks = 0;
    const size_t ws_bytes = attention_scratch_bytes(pos, n_heads, nchunks);
    float* ws = static_cast<float*>(ws_acquire(nullptr, ws_bytes, st));
    if (!ws) {
        set_error("eq_rope_attention_decode: no workspace (its stream's workspace cannot grow while capturing: "
                  "make one call of at least this position on the stream before capturing)");
        return 1;
    }
    launch_attention(ws, out, q, k_new, v_new, k_cache, v_cache, freqs, pos, max_seq, n_heads, n_kv_heads, nchunks,
                     scale, st);
    return check_launch("eq_rope_attention_decode");
}

extern "C" int eq_rope_attention_decode_at(void* out, const void* q, const void* k_new, const void* v_new,
                                           void* k_cache, void* v_cache, const float* freqs, const int32_t* pos,
                                           int64_t max_seq, int n_heads, int n_kv_heads, int head_dim, float scale,
                                           int dtype, eq_stream_t stream) {
    clear_error();
    const char* who = "eq_rope_attention_decode_at";
    if (!pos) {
        set_error(std::string(who) + ": null pointer argument");
        return 1;
    }
    // the shape rules of the by-value entry point, checked at position 0 (the
    // position itself is read by the kernel; one outside [0, max_seq) gives zeros)
    if (!attention_args_ok(who, out, q, k_new, v_new, k_cache, v_cache, freqs, 0, max_seq, n_heads, n_kv_heads,
                           head_dim, dtype))
        return 1;
    if (max_seq > int64_t(kMaxChunks) * kAttnChunk) {
        set_error(std::string(who) + ": max_seq must be at most 131072");
        return 1;
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    // every chunk of max_seq has a slot; the kernels read the position
    const int nchunks = int((max_seq + kAttnChunk - 1) / kAttnChunk);
    const size_t ws_bytes = size_t(n_heads) * size_t(nchunks) * (kHeadDim + 2) * sizeof(float);
    float* ws = static_cast<float*>(ws_acquire(nullptr, ws_bytes, st));
    if (!ws) {
        set_error(std::string(who) + ": no workspace (its stream's workspace cannot grow while capturing: make one "
                  "call with this max_seq on the stream before capturing)");
        return 1;
    }
    attn_partial_kernel<<<dim3(unsigned(n_kv_heads), unsigned(nchunks)), dim3(256), 0, st>>>(
        ws, static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k_new), static_cast<const uint16_t*>(v_new),
        static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), freqs, 0, pos, int(max_seq), n_heads,
        n_kv_heads, nchunks, scale);
    attn_combine_kernel<<<dim3(unsigned(n_heads)), dim3(256), 0, st>>>(static_cast<uint16_t*>(out), ws, 0, pos,
                                                                       int(max_seq), nchunks);
    return check_launch(who);
}

extern "C" int eq_advance_position(int32_t* pos, eq_stream_t stream) {
    clear_error();
    if (!pos) {
        set_error("eq_advance_position: null pointer argument");
        return 1;
    }
    advance_position_kernel<<<1, 1, 0, reinterpret_cast<hipStream_t>(stream)>>>(pos);
    return check_launch("eq_advance_position");
}

// ---------------------------------------------------- allocation-free variant

// Scratch of eq_rope_attention_decode_noalloc: the attention partials
// (n_heads * chunks * 520 bytes).  Every GPU the library runs on holds its own
// copy until the process ends.  The array's name is a host-side stand-in in
// host code; the device address comes from attention_scratch_address().
constexpr size_t kAttnScratchBytes = size_t(8) << 20;
static __device__ __align__(256) char scratch[kAttnScratchBytes];

// Device address of `scratch` on the current device, resolved on the first
// call on each device (with that device current) and kept.
static void* attention_scratch_address() {
    static std::mutex mu;
    static void* addr[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        set_error("eq_rope_attention_decode_noalloc: no current device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            set_error(std::string("eq_rope_attention_decode_noalloc: scratch address lookup failed: ") +
                      hipGetErrorString(e));
            return nullptr;
        }
        addr[dev] = p;
    }
    return addr[dev];
}

extern "C" int eq_rope_attention_decode_noalloc(void* out, const void* q, const void* k_new, const void* v_new,
                                                void* k_cache, void* v_cache, const float* freqs, int64_t pos,
                                                int64_t max_seq, int n_heads, int n_kv_heads, int head_dim,
                                                float scale, int dtype, eq_stream_t stream) {
    clear_error();
    if (!attention_args_ok("eq_rope_attention_decode_noalloc", out, q, k_new, v_new, k_cache, v_cache, freqs, pos,
                           max_seq, n_heads, n_kv_heads, head_dim, dtype))
        return 1;
    int nchunks = 0;
    const size_t ws_bytes = attention_scratch_bytes(pos, n_heads, nchunks);
    if (ws_bytes > kAttnScratchBytes) {
        set_error("eq_rope_attention_decode_noalloc: n_heads * (pos / 32 + 1) * 520 = " + std::to_string(ws_bytes) +
                  " bytes of scratch, more than the " + std::to_string(kAttnScratchBytes) +
                  " this entry point holds (use eq_rope_attention_decode)");
        return 1;
    }
    void* ws = attention_scratch_address();
    if (!ws) return 1;
    launch_attention(static_cast<float*>(ws), out, q, k_new, v_new, k_cache, v_cache, freqs, pos, max_seq, n_heads,
                     n_kv_heads, nchunks, scale, reinterpret_cast<hipStream_t>(stream));
    return check_launch("eq_rope_attention_decode_noalloc");
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
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    // Long rows: several workgroups per row (a key and a counter per row in
    // the stream's arrival counters); otherwise -- or when the counters
    // cannot be provided (first use under capture) -- one workgroup per row.
    constexpr int kMaxWideRows = kWsCounters / 4;
    if (n >= 16384 && n % 8 == 0 && aligned(logits, 16) && rows <= kMaxWideRows) {
        if (unsigned* c = ws_counters(nullptr, st)) {
            const int slice = int(((n + 63) / 64 + 2047) / 2048 * 2048);  // at most 64 slices, multiples of 2048
            const int groups = int((n + slice - 1) / slice);
            unsigned long long* keys = reinterpret_cast<unsigned long long*>(c + kWsCounters / 2);
            argmax_wide_kernel<<<dim3(unsigned(groups), unsigned(rows)), dim3(256), 0, st>>>(
                out, static_cast<const uint16_t*>(logits), n, slice, c, keys);
            return check_launch("eq_argmax");
        }
    }
    argmax_kernel<<<dim3(unsigned(rows)), dim3(1024), 0, st>>>(out, static_cast<const uint16_t*>(logits), n,
                                                              n % 8 == 0 && aligned(logits, 16));
    return check_launch("eq_argmax");
}
