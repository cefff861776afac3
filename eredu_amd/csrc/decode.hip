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

// Decode attention keeps, per query head, kAttnSplits softmax states, state
// y over the 32-position chunks y, y + kAttnSplits, ... of positions 0..pos:
// a row of kAttnStateFloats floats [m, l, o[0..127]] = the maximum scaled
// score, the sum of exp(score - m) and the exp-weighted value rows.  Only the
// first min(chunks, kAttnSplits) states of a head are written and read.
constexpr int kAttnSplits = 64;
constexpr int kAttnStateFloats = kHeadDim + 2;

// DPP lane moves within rows of 16 lanes (quad_perm [1,0,3,2] = 0xB1,
// quad_perm [2,3,0,1] = 0x4E, row_half_mirror = 0x141, row_mirror = 0x140).
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Maximum / sum over each row of 16 lanes, in every lane of the row.
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_move<0xB1>(v));
    v = fmaxf(v, dpp_move<0x4E>(v));
    v = fmaxf(v, dpp_move<0x141>(v));
    return fmaxf(v, dpp_move<0x140>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_move<0xB1>(v);
    v += dpp_move<0x4E>(v);
    v += dpp_move<0x141>(v);
    return v + dpp_move<0x140>(v);
}
__device__ __forceinline__ float lane_value(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// Grid (n_kv_heads, kAttnSplits), 256 threads (4 waves; wave h = query head
// g * group + h of KV head g).  Split y walks its chunks: each chunk's keys
// and values go through registers into LDS (the first chunk's are requested
// before the position is known, bounded by max_seq; each next chunk's while
// the current one is computed), the group's queries are rotated once (the 64
// angles' sines and cosines computed once per workgroup), and the chunk that
// holds pos rotates the new key and writes it and the new value into the
// cache (no other chunk reads row pos).  Per query head the split keeps a
// running softmax state merged chunk by chunk (m' = max(m, m_c); l, o scaled
// by e^(m - m') and e^(m_c - m')) and writes it to states[head][y].
// Scores: lane = position (lane / 2) x half of the dimensions (lane % 2), the
// query half in registers, the key half-row in 16-byte LDS reads; maxima and
// sums by DPP within rows of 16 lanes and lane reads across the rows.
//
// pos_p, when not null, names the position in device memory (read when the
// kernel runs); a position outside [0, max_seq) writes nothing.
__global__ __launch_bounds__(256) void attn_states_kernel(float* __restrict__ states, const uint16_t* __restrict__ q,
                                                          const uint16_t* __restrict__ k_new,
                                                          const uint16_t* __restrict__ v_new,
                                                          uint16_t* __restrict__ k_cache,
                                                          uint16_t* __restrict__ v_cache,
                                                          const float* __restrict__ freqs, int pos_arg,
                                                          const int32_t* __restrict__ pos_p, int max_seq,
                                                          int group, float scale) {
    __shared__ __attribute__((aligned(16))) float qs[4][kHeadDim];  // rotated queries of this group
    __shared__ __attribute__((aligned(16))) uint16_t ks[kAttnChunk][kRowPad];
    __shared__ __attribute__((aligned(16))) uint16_t vs[kAttnChunk][kRowPad];
    __shared__ float knew[kHeadDim];
    __shared__ float rot[2][kHeadDim / 2];  // cos, sin of the angles pos / freqs[i]
    // Every load of the prologue is requested before any is waited for, so
    // that they cost one memory round trip: the position by a vector load
    // (a scalar one would be waited for together with the argument loads
    // the addresses below need), then the group's queries, the new key, the
    // frequencies and the split's first chunk, each at an in-range index
    // with dead lanes' values selected away afterwards (a load behind a
    // per-lane branch is waited for where the branch joins).
    const uint32_t pos_v = __builtin_amdgcn_raw_buffer_load_b32(raw_rsrc(pos_p, pos_p ? 4u : 0u), 0u, 0u, 0);
    const int g = blockIdx.x, split = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint16_t* kc = k_cache + int64_t(g) * max_seq * kHeadDim;
    uint16_t* vc = v_cache + int64_t(g) * max_seq * kHeadDim;

    float qv[2];
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int i = tid + 256 * r;
        const bool live = i < group * kHeadDim;
        const float v = bf16_bits_to_f32(q[int64_t(g) * group * kHeadDim + (live ? i : 0)]);
        qv[r] = live ? v : 0.f;
    }
    const float kn_v = bf16_bits_to_f32(k_new[int64_t(g) * kHeadDim + (tid & (kHeadDim - 1))]);
    const float fr_v = freqs[tid & (kHeadDim / 2 - 1)];
    const float kn = tid < kHeadDim ? kn_v : 0.f;
    const float fr = tid < kHeadDim / 2 ? fr_v : 1.f;
    // this thread's two 16-byte pieces of a chunk's keys and of its values:
    // piece i = tid + 256 r is position i / 16, dimensions 8 (i % 16) ..;
    // pieces past `limit` read row 0 and are replaced by zeros
    uint4 kr[2], vr[2];
    auto fetch = [&](int c, int limit) __attribute__((always_inline)) {
        const int p0 = c * kAttnChunk;
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int i = tid + 256 * r, p = p0 + i / (kHeadDim / 8), v = i % (kHeadDim / 8);
            const bool live = p < limit;
            const int64_t row = live ? int64_t(p) * kHeadDim : 0;
            const uint4 kx = reinterpret_cast<const uint4*>(kc + row)[v];
            const uint4 vx = reinterpret_cast<const uint4*>(vc + row)[v];
            kr[r] = live ? kx : make_uint4(0u, 0u, 0u, 0u);
            vr[r] = live ? vx : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    fetch(split, max_seq);  // rows past pos are masked out below
    const int pos = pos_p ? int(__builtin_amdgcn_readfirstlane(pos_v)) : pos_arg;
    const bool valid = pos >= 0 && pos < max_seq;
    const int nch = valid ? pos / kAttnChunk + 1 : 0;
    if (split >= nch) return;
    const float fpos = float(pos);
    const int c_new = pos / kAttnChunk;  // the chunk holding pos
    const bool mine_new = c_new % kAttnSplits == split;

#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int i = tid + 256 * r;
        if (i < group * kHeadDim) qs[i / kHeadDim][i % kHeadDim] = qv[r];
    }
    if (tid < kHeadDim) knew[tid] = kn;
    if (tid < kHeadDim / 2) {
        float sn, cs;
        sincosf(fpos / fr, &sn, &cs);
        rot[0][tid] = cs;
        rot[1][tid] = sn;
    }
    __syncthreads();
    // non-traditional (half-split) rotation, Llama3Rope::forward: pairs
    // (d, d + 64) of each query head, and of the new key in its chunk's split
    for (int i = tid; i < (group + (mine_new ? 1 : 0)) * (kHeadDim / 2); i += 256) {
        const int hh = i / (kHeadDim / 2), d = i % (kHeadDim / 2);
        float* head = hh < group ? qs[hh] : knew;
        const float cs = rot[0][d], sn = rot[1][d];
        const float x1 = head[d], x2 = head[d + kHeadDim / 2];
        head[d] = x1 * cs - x2 * sn;
        head[d + kHeadDim / 2] = x2 * cs + x1 * sn;
    }
    __syncthreads();
    // position pos: the rotated new key rounded to bf16, and the new value,
    // into the cache (and into LDS when its chunk is staged)
    uint4 kk_new = make_uint4(0u, 0u, 0u, 0u), vv_new = make_uint4(0u, 0u, 0u, 0u);
    if (mine_new && tid < kHeadDim / 8) {
        const int v = tid;
        uint32_t* pk = reinterpret_cast<uint32_t*>(&kk_new);
#pragma unroll
        for (int e = 0; e < 4; e++)
            pk[e] = f32_to_bf16_bits(knew[8 * v + 2 * e]) | (f32_to_bf16_bits(knew[8 * v + 2 * e + 1]) << 16);
        vv_new = reinterpret_cast<const uint4*>(v_new + int64_t(g) * kHeadDim)[v];
        reinterpret_cast<uint4*>(kc + int64_t(pos) * kHeadDim)[v] = kk_new;
        reinterpret_cast<uint4*>(vc + int64_t(pos) * kHeadDim)[v] = vv_new;
    }
    const int h = wave, p = lane >> 1, half = lane & 1;
    float qreg[kHeadDim / 2];
    if (h < group) {
#pragma unroll
        for (int j = 0; j < kHeadDim / 8; j++) {
            const float4 t = reinterpret_cast<const float4*>(&qs[h][half * (kHeadDim / 2)])[j];
            qreg[4 * j] = t.x;
            qreg[4 * j + 1] = t.y;
            qreg[4 * j + 2] = t.z;
            qreg[4 * j + 3] = t.w;
        }
    }

    float m_run = -INFINITY, l_run = 0.f, o0 = 0.f, o1 = 0.f;
    for (int c = split; c < nch; c += kAttnSplits) {
        const int p0 = c * kAttnChunk, np = min(kAttnChunk, pos + 1 - p0);
        __syncthreads();  // the previous chunk's LDS reads are done
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int i = tid + 256 * r, pr = i / (kHeadDim / 8), v = i % (kHeadDim / 8);
            reinterpret_cast<uint4*>(&ks[pr][0])[v] = kr[r];
            reinterpret_cast<uint4*>(&vs[pr][0])[v] = vr[r];
        }
        if (c == c_new && tid < kHeadDim / 8) {
            reinterpret_cast<uint4*>(&ks[pos - p0][0])[tid] = kk_new;
            reinterpret_cast<uint4*>(&vs[pos - p0][0])[tid] = vv_new;
        }
        __syncthreads();
        if (c + kAttnSplits < nch) fetch(c + kAttnSplits, pos);  // in flight while this chunk is computed
        if (h < group) {
            float sa = 0.f, sb = 0.f;
            if (p < np) {
                const uint4* kr4 = reinterpret_cast<const uint4*>(&ks[p][half * (kHeadDim / 2)]);
#pragma unroll
                for (int j = 0; j < kHeadDim / 16; j++) {
                    const uint4 kk = kr4[j];
                    const uint32_t w4[4] = {kk.x, kk.y, kk.z, kk.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        sa = fmaf(qreg[8 * j + 2 * e], bf16_bits_to_f32(w4[e] & 0xffffu), sa);
                        sb = fmaf(qreg[8 * j + 2 * e + 1], bf16_bits_to_f32(w4[e] >> 16), sb);
                    }
                }
            }
            float sc = sa + sb;
            sc += dpp_move<0xB1>(sc);  // the other half of the dimensions
            sc = p < np ? sc * scale : -INFINITY;
            const float rm = row16_max(sc);
            const float mc = fmaxf(fmaxf(lane_value(rm, 0), lane_value(rm, 16)),
                                   fmaxf(lane_value(rm, 32), lane_value(rm, 48)));
            const float e = p < np ? expf(sc - mc) : 0.f;
            const float rs = row16_sum(half == 0 ? e : 0.f);
            const float lc = (lane_value(rs, 0) + lane_value(rs, 16)) + (lane_value(rs, 32) + lane_value(rs, 48));
            // weighted values: lane owns dimensions 2 lane, 2 lane + 1; every
            // row is read (rows past np hold finite or stale data, skipped)
            uint32_t vv[kAttnChunk];
#pragma unroll
            for (int pp = 0; pp < kAttnChunk; pp++) vv[pp] = reinterpret_cast<const uint32_t*>(&vs[pp][0])[lane];
            float c0 = 0.f, c1 = 0.f;
#pragma unroll
            for (int pp = 0; pp < kAttnChunk; pp++) {
                if (pp < np) {
                    const float w = lane_value(e, 2 * pp);
                    c0 = fmaf(w, bf16_bits_to_f32(vv[pp] & 0xffffu), c0);
                    c1 = fmaf(w, bf16_bits_to_f32(vv[pp] >> 16), c1);
                }
            }
            if (c == split) {
                m_run = mc;
                l_run = lc;
                o0 = c0;
                o1 = c1;
            } else {
                const float mn = fmaxf(m_run, mc);
                const float fa = expf(m_run - mn), fb = expf(mc - mn);
                l_run = l_run * fa + lc * fb;
                o0 = o0 * fa + c0 * fb;
                o1 = o1 * fa + c1 * fb;
                m_run = mn;
            }
        }
    }
    if (h < group) {
        float* dst = states + (int64_t(g * group + h) * kAttnSplits + split) * kAttnStateFloats;
        if (lane == 0) {
            dst[0] = m_run;
            dst[1] = l_run;
        }
        reinterpret_cast<float2*>(dst + 2)[lane] = make_float2(o0, o1);
    }
}

// One workgroup of 256 threads per query head, over the first
// ns = min(chunks, kAttnSplits) states: M = max m_y, f_y = e^(m_y - M); wave
// w sums f_y o_y over the states y = w, w + 4, ... (all its loads issued
// together), lane d for dimensions 2 d and 2 d + 1; the waves' sums are added
// in wave order and divided by sum f_y l_y; rounded to bf16.  A position
// outside [0, max_seq) gives zeros.
__global__ __launch_bounds__(256) void attn_states_combine_kernel(uint16_t* __restrict__ out,
                                                                  const float* __restrict__ states, int pos_arg,
                                                                  const int32_t* __restrict__ pos_p, int max_seq) {
    __shared__ float2 part[4][64];
    // The position (a vector load, as in attn_states_kernel) and all 64
    // states of the head are requested together; states past the position's
    // chunk count (stale) are selected away once the position is known.
    const uint32_t pos_v = __builtin_amdgcn_raw_buffer_load_b32(raw_rsrc(pos_p, pos_p ? 4u : 0u), 0u, 0u, 0);
    const int h = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const float* st = states + int64_t(h) * kAttnSplits * kAttnStateFloats;
    float2 ov[kAttnSplits / 4];
#pragma unroll
    for (int k = 0; k < kAttnSplits / 4; k++)
        ov[k] = reinterpret_cast<const float2*>(st + (w + 4 * k) * kAttnStateFloats + 2)[lane];
    const float m_v = st[lane * kAttnStateFloats], l_v = st[lane * kAttnStateFloats + 1];
    const int pos = pos_p ? int(__builtin_amdgcn_readfirstlane(pos_v)) : pos_arg;
    const int nch = pos >= 0 && pos < max_seq ? pos / kAttnChunk + 1 : 0;
    const int ns = min(nch, kAttnSplits);
    uint32_t* dst = reinterpret_cast<uint32_t*>(out + int64_t(h) * kHeadDim) + lane;
    if (ns == 0) {
        if (w == 0) *dst = 0u;
        return;
    }
    float2 o[kAttnSplits / 4];
#pragma unroll
    for (int k = 0; k < kAttnSplits / 4; k++) o[k] = w + 4 * k < ns ? ov[k] : make_float2(0.f, 0.f);
    const float m = lane < ns ? m_v : -INFINITY;
    const float l = lane < ns ? l_v : 0.f;
    float mx = m;
#pragma unroll
    for (int of = 32; of > 0; of >>= 1) mx = fmaxf(mx, __shfl_xor(mx, of));
    const float f = lane < ns ? expf(m - mx) : 0.f;
    const float lsum = wave_sum(f * l);
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int k = 0; k < kAttnSplits / 4; k++) {
        const float fy = lane_value(f, w + 4 * k);  // 0 past ns
        a0 = fmaf(fy, o[k].x, a0);
        a1 = fmaf(fy, o[k].y, a1);
    }
    part[w][lane] = make_float2(a0, a1);
    __syncthreads();
    if (w == 0) {
        float2 t = part[0][lane];
#pragma unroll
        for (int i = 1; i < 4; i++) {
            t.x += part[i][lane].x;
            t.y += part[i][lane].y;
        }
        *dst = f32_to_bf16_bits(t.x / lsum) | (f32_to_bf16_bits(t.y / lsum) << 16);
    }
}

// pos[0] += 1 (the next decode position), one thread.
__global__ void advance_position_kernel(int32_t* pos) { pos[0] += 1; }

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

// Validation shared by the attention entry points (true when the arguments
// are accepted; else the error is set).
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

// The two attention passes: kAttnSplits softmax states per query head into
// `states`, then their combination.  pos_p (device position) or pos.
static void launch_attention(float* states, void* out, const void* q, const void* k_new, const void* v_new,
                             void* k_cache, void* v_cache, const float* freqs, int64_t pos, const int32_t* pos_p,
                             int64_t max_seq, int n_heads, int n_kv_heads, float scale, hipStream_t st) {
    attn_states_kernel<<<dim3(unsigned(n_kv_heads), unsigned(kAttnSplits)), dim3(256), 0, st>>>(
        states, static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k_new),
        static_cast<const uint16_t*>(v_new), static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), freqs,
        int(pos), pos_p, int(max_seq), n_heads / n_kv_heads, scale);
    attn_states_combine_kernel<<<dim3(unsigned(n_heads)), dim3(256), 0, st>>>(static_cast<uint16_t*>(out), states,
                                                                               int(pos), pos_p, int(max_seq));
}

// Bytes of softmax states of one attention call (n_heads * 64 * 520).
static size_t attention_states_bytes(int n_heads) {
    return size_t(n_heads) * kAttnSplits * kAttnStateFloats * sizeof(float);
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
    float* ws = static_cast<float*>(ws_acquire(nullptr, attention_states_bytes(n_heads), st));
    if (!ws) {
        set_error("eq_rope_attention_decode: no workspace (its stream's workspace cannot grow while capturing: "
                  "make one call with this head count on the stream before capturing)");
        return 1;
    }
    launch_attention(ws, out, q, k_new, v_new, k_cache, v_cache, freqs, pos, nullptr, max_seq, n_heads, n_kv_heads,
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
    float* ws = static_cast<float*>(ws_acquire(nullptr, attention_states_bytes(n_heads), st));
    if (!ws) {
        set_error(std::string(who) + ": no workspace (its stream's workspace cannot grow while capturing: make one "
                  "call with this head count on the stream before capturing)");
        return 1;
    }
    launch_attention(ws, out, q, k_new, v_new, k_cache, v_cache, freqs, 0, pos, max_seq, n_heads, n_kv_heads, scale,
                     st);
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

// Scratch of eq_rope_attention_decode_noalloc: the attention softmax states
// (n_heads * 64 * 520 bytes, at most 252 heads).  Every GPU the library runs on holds its own
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
    const size_t ws_bytes = attention_states_bytes(n_heads);
    if (ws_bytes > kAttnScratchBytes) {
        set_error("eq_rope_attention_decode_noalloc: n_heads * 64 * 520 = " + std::to_string(ws_bytes) +
                  " bytes of scratch, more than the " + std::to_string(kAttnScratchBytes) +
                  " this entry point holds (use eq_rope_attention_decode)");
        return 1;
    }
    void* ws = attention_scratch_address();
    if (!ws) return 1;
    launch_attention(static_cast<float*>(ws), out, q, k_new, v_new, k_cache, v_cache, freqs, pos, nullptr, max_seq,
                     n_heads, n_kv_heads, scale, reinterpret_cast<hipStream_t>(stream));
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
