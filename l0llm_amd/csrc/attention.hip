// GQA decode attention over the KV cache for gfx950 (Attention.Execute / ExecutePrefill,
// LlmDecoderLayer.cs:325-327, :369-371).
//
// Split-K over the sequence ("flash decoding"): block (split, kv head, batch) reads its slice
// of the K and V rows of one kv head once and serves all the q heads of that group from it.
// Layout: cache [batch, max_seq, n_kv * head_dim] (LlmKvCache.cs:5-8). A lane owns 8 dims of a
// row (one 16-byte fp16 load), head_dim/8 lanes cover a row, so a wave instruction reads 4
// (head_dim 128) or 8 (head_dim 64) positions of 256/128 contiguous bytes. Scores and
// probabilities are staged in LDS, softmax is fp32 in the log2 domain, and each block writes its
// (max, sum, acc) partial; a second small kernel merges the splits with a log-sum-exp combine.
// The kernel boundary publishes the partials, so no block waits on another and no device-scope
// fence is needed (on gfx950 such a fence writes back the L2).
#include "kernels.h"

#include <cmath>

namespace l0h {
namespace {

constexpr int kBlock = 256;
constexpr int kGroupMax = 8;   // q heads per kv head
constexpr int kChunkMax = 1024;  // positions per block (scores staged in LDS)
constexpr int kUnroll = 4;
constexpr int kMergeBlock = 256;

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_src(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

// Sum over the LPP lanes that share a position (2, 4 or 8 lanes of a row, or the full
// 16-lane row), left in every lane of the group.
template <int LPP>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp_src<0xB1, 0xf>(v);  // quad_perm [1,0,3,2]
    if constexpr (LPP >= 4) v += dpp_src<0x4E, 0xf>(v);  // quad_perm [2,3,0,1]
    if constexpr (LPP == 8) {
        v += dpp_src<0x141, 0xf>(v);  // row_half_mirror: quad 0 <-> quad 1
    } else if constexpr (LPP == 16) {
        v += dpp_src<0x124, 0xf>(v);  // row_ror:4
        v += dpp_src<0x128, 0xf>(v);  // row_ror:8
    }
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

template <int CT>
struct CacheRow;
template <>
struct CacheRow<L0H_F16> {
    using T = uint16_t;
    uint4 raw;
    __device__ __forceinline__ void load(const T* p) { raw = ld_nt16(p); }
    __device__ __forceinline__ void zero() { raw = make_uint4(0u, 0u, 0u, 0u); }
    __device__ __forceinline__ void get(float* f) const {
        const uint32_t d[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float2 t = __half22float2(__builtin_bit_cast(__half2, d[j]));
            f[2 * j] = t.x;
            f[2 * j + 1] = t.y;
        }
    }
};
template <>
struct CacheRow<L0H_F32> {
    using T = float;
    float4 a, b;
    __device__ __forceinline__ void load(const T* p) {
        uint4 t0 = ld_nt16(p);
        a = make_float4(__uint_as_float(t0.x), __uint_as_float(t0.y), __uint_as_float(t0.z), __uint_as_float(t0.w));
        uint4 t1 = ld_nt16(p + 4);
        b = make_float4(__uint_as_float(t1.x), __uint_as_float(t1.y), __uint_as_float(t1.z), __uint_as_float(t1.w));
    }
    __device__ __forceinline__ void zero() { a = b = make_float4(0.f, 0.f, 0.f, 0.f); }
    __device__ __forceinline__ void get(float* f) const {
        f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
        f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    }
};

template <int HD, int CT>
__global__ __launch_bounds__(kBlock) void attn_decode_kernel(const AttnParams p, int seq_len_step,
                                                             size_t cache_batch_stride) {
    constexpr int LPP = HD / 8;     // lanes per position
    constexpr int PPW = 64 / LPP;   // positions per wave instruction
    constexpr int NG = 4 * PPW;     // lane groups per block
    using T = typename CacheRow<CT>::T;
    __shared__ float s_scores[kGroupMax * kChunkMax];
    __shared__ float s_acc[4][kGroupMax][HD];
    __shared__ float s_m[kGroupMax], s_l[kGroupMax];

    const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int G = p.nh / p.nkv;
    const int kv_dim = p.nkv * HD;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lg = lane % LPP;
    const int grp = wave * PPW + lane / LPP;

    int len = (p.seq_len_device ? *p.seq_len_device + p.seq_len_add : p.seq_len) + b * seq_len_step;
    len = min(len, p.max_seq_len);
    const int chunk = (len + p.splits - 1) / p.splits;
    const int lo = split * chunk;
    const int n = max(0, min(len, lo + chunk) - lo);

    // q for this lane's 8 dims of every head of the group, scaled by log2(e) / sqrt(HD).
    float qr[kGroupMax][8];
    const float qscale = 1.4426950408889634f / sqrtf((float)HD);
#pragma unroll
    for (int h = 0; h < kGroupMax; h++) {
#pragma unroll
        for (int d = 0; d < 8; d++)
            qr[h][d] = h < G ? load_act(p.q, p.q_dtype, (size_t)b * p.nh * HD + (size_t)(g * G + h) * HD + lg * 8 + d) * qscale
                             : 0.f;
    }
    const T* kbase = static_cast<const T*>(p.kc) + (size_t)b * cache_batch_stride + (size_t)g * HD + lg * 8;
    const T* vbase = static_cast<const T*>(p.vc) + (size_t)b * cache_batch_stride + (size_t)g * HD + lg * 8;

    // The first batch of V rows is requested together with the K rows, so a chunk that fits one
    // batch (the decode case) costs a single HBM round trip.
    CacheRow<CT> vpre[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
        const int t = grp + u * NG;
        if (t < n) vpre[u].load(vbase + (size_t)(lo + t) * kv_dim);
        else vpre[u].zero();
    }

    // Phase A: scores of this block's positions into LDS.
    for (int t0 = grp; t0 < n; t0 += NG * kUnroll) {
        CacheRow<CT> kr[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int t = t0 + u * NG;
            if (t < n) kr[u].load(kbase + (size_t)(lo + t) * kv_dim);
            else kr[u].zero();
        }
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int t = t0 + u * NG;
            float kf[8];
            kr[u].get(kf);
#pragma unroll
            for (int h = 0; h < kGroupMax; h++) {
                if (h < G) {
                    float s = 0.f;
#pragma unroll
                    for (int d = 0; d < 8; d++) s = fmaf(qr[h][d], kf[d], s);
                    s = group_sum<LPP>(s);
                    if (lg == h % LPP && t < n) s_scores[h * kChunkMax + t] = s;
                }
            }
        }
    }
    __syncthreads();

    // Phase B: per-head max and exp (wave w handles heads w, w+4).
    for (int h = wave; h < G; h += 4) {
        float m = -INFINITY;
        for (int t = lane; t < n; t += 64) m = fmaxf(m, s_scores[h * kChunkMax + t]);
        m = wave_max(m);
        float l = 0.f;
        for (int t = lane; t < n; t += 64) {
            const float e = exp2f(s_scores[h * kChunkMax + t] - m);
            s_scores[h * kChunkMax + t] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) {
            s_m[h] = m;
            s_l[h] = l;
        }
    }
    __syncthreads();

    // Phase C: P . V per lane group, then across the groups of the wave.
    float acc[kGroupMax][8];
#pragma unroll
    for (int h = 0; h < kGroupMax; h++)
#pragma unroll
        for (int d = 0; d < 8; d++) acc[h][d] = 0.f;
    for (int t0 = grp; t0 < n; t0 += NG * kUnroll) {
        CacheRow<CT> vr[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int t = t0 + u * NG;
            if (t0 == grp) vr[u] = vpre[u];
            else if (t < n) vr[u].load(vbase + (size_t)(lo + t) * kv_dim);
            else vr[u].zero();
        }
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int t = t0 + u * NG;
            if (t < n) {
                float vf[8];
                vr[u].get(vf);
#pragma unroll
                for (int h = 0; h < kGroupMax; h++) {
                    if (h < G) {
                        const float pr = s_scores[h * kChunkMax + t];
#pragma unroll
                        for (int d = 0; d < 8; d++) acc[h][d] = fmaf(pr, vf[d], acc[h][d]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int h = 0; h < kGroupMax; h++) {
        if (h < G) {
#pragma unroll
            for (int d = 0; d < 8; d++) {
                float v = acc[h][d];
#pragma unroll
                for (int off = LPP; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
                acc[h][d] = v;
            }
        }
    }
    if (lane < LPP) {
#pragma unroll
        for (int h = 0; h < kGroupMax; h++)
            if (h < G)
#pragma unroll
                for (int d = 0; d < 8; d++) s_acc[wave][h][lg * 8 + d] = acc[h][d];
    }
    __syncthreads();

    // Block partial -> workspace.
    const size_t pbase = (((size_t)b * p.nkv + g) * p.splits + split) * (size_t)G * (HD + 2);
    float* part = p.partials + pbase;
    for (int idx = threadIdx.x; idx < G * HD; idx += kBlock) {
        const int h = idx / HD, d = idx - h * HD;
        part[idx] = s_acc[0][h][d] + s_acc[1][h][d] + s_acc[2][h][d] + s_acc[3][h][d];
    }
    if (threadIdx.x < G) {
        part[G * HD + threadIdx.x] = n > 0 ? s_m[threadIdx.x] : -INFINITY;
        part[G * HD + G + threadIdx.x] = n > 0 ? s_l[threadIdx.x] : 0.f;
    }
}

// Log-sum-exp merge of the splits' partials: one block per (q head of the group, kv head,
// batch). Wave w folds splits w, w+4, ... against its own running max (lane owns dims lane,
// lane+64), then the four wave results are combined in a fixed order, so the output does not
// depend on timing.
template <int HD>
__global__ __launch_bounds__(kMergeBlock) void attn_merge_kernel(const AttnParams p) {
    constexpr int kWavesM = kMergeBlock / 64;
    constexpr int DPL = (HD + 63) / 64;  // dims per lane
    __shared__ float s_num[kWavesM][HD];
    __shared__ float s_wm[kWavesM], s_wden[kWavesM];
    const int h = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int G = p.nh / p.nkv;
    const size_t stride = (size_t)G * (HD + 2);
    const float* all = p.partials + ((size_t)b * p.nkv + g) * p.splits * stride;
    float M = -INFINITY;
    for (int s = wave; s < p.splits; s += kWavesM) M = fmaxf(M, all[s * stride + G * HD + h]);
    float num[DPL], den = 0.f;
#pragma unroll
    for (int j = 0; j < DPL; j++) num[j] = 0.f;
    if (M != -INFINITY) {
#pragma unroll 4
        for (int s = wave; s < p.splits; s += kWavesM) {
            const float* ps = all + s * stride;
            const float ms = ps[G * HD + h];
            const float w = ms == -INFINITY ? 0.f : exp2f(ms - M);
            den = fmaf(w, ps[G * HD + G + h], den);
#pragma unroll
            for (int j = 0; j < DPL; j++)
                if (lane + 64 * j < HD) num[j] = fmaf(w, ps[h * HD + lane + 64 * j], num[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < DPL; j++)
        if (lane + 64 * j < HD) s_num[wave][lane + 64 * j] = num[j];
    if (lane == 0) {
        s_wm[wave] = M;
        s_wden[wave] = den;
    }
    __syncthreads();
    float Mt = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWavesM; w++) Mt = fmaxf(Mt, s_wm[w]);
    for (int d = threadIdx.x; d < HD; d += kMergeBlock) {
        float n = 0.f, dd = 0.f;
        if (Mt != -INFINITY) {
#pragma unroll
            for (int w = 0; w < kWavesM; w++) {
                const float sc = s_wm[w] == -INFINITY ? 0.f : exp2f(s_wm[w] - Mt);
                n = fmaf(sc, s_num[w][d], n);
                dd = fmaf(sc, s_wden[w], dd);
            }
        }
        store_act(p.out, p.out_dtype, (size_t)b * p.nh * HD + (size_t)(g * G + h) * HD + d, dd > 0.f ? n / dd : 0.f);
    }
}

template <int HD>
int launch_hd(hipStream_t s, const AttnParams& p, int seq_len_step, size_t cache_batch_stride) {
    dim3 grid(p.splits, p.nkv, p.batch);
    if (p.cache_dtype == L0H_F16)
        attn_decode_kernel<HD, L0H_F16><<<grid, kBlock, 0, s>>>(p, seq_len_step, cache_batch_stride);
    else
        attn_decode_kernel<HD, L0H_F32><<<grid, kBlock, 0, s>>>(p, seq_len_step, cache_batch_stride);
    int st = launch_status("attention");
    if (st) return st;
    attn_merge_kernel<HD><<<dim3(p.nh / p.nkv, p.nkv, p.batch), kMergeBlock, 0, s>>>(p);
    return launch_status("attention merge");
}

int launch_any(hipStream_t s, const AttnParams& p, int seq_len_step, size_t cache_batch_stride) {
    if (p.head_dim != 16 && p.head_dim != 32 && p.head_dim != 64 && p.head_dim != 128)
        return fail(L0H_ERR_UNSUPPORTED, "attention supports head_dim 16, 32, 64 and 128");
    if (p.nkv <= 0 || p.nh % p.nkv != 0 || p.nh / p.nkv > kGroupMax)
        return fail(L0H_ERR_UNSUPPORTED, "attention needs n_heads a multiple of n_kv_heads, at most 8 per group");
    if (p.cache_dtype != L0H_F16 && p.cache_dtype != L0H_F32)
        return fail(L0H_ERR_INVALID_ARG, "cache dtype must be F16 or F32");
    if (p.splits < 1 || (size_t)p.max_seq_len > (size_t)p.splits * kChunkMax)
        return fail(L0H_ERR_INVALID_ARG, "too few splits for the sequence length");
    if (!p.partials) return fail(L0H_ERR_INVALID_ARG, "attention workspace missing");
    switch (p.head_dim) {
    case 16: return launch_hd<16>(s, p, seq_len_step, cache_batch_stride);
    case 32: return launch_hd<32>(s, p, seq_len_step, cache_batch_stride);
    case 64: return launch_hd<64>(s, p, seq_len_step, cache_batch_stride);
    default: return launch_hd<128>(s, p, seq_len_step, cache_batch_stride);
    }
}

}  // namespace

int attention_default_splits(int batch, int nkv, int max_len, int compute_units) {
    const int min_splits = (int)ceil_div((size_t)std::max(max_len, 1), kChunkMax);
    const int target = (int)ceil_div((size_t)2 * std::max(compute_units, 1), (size_t)std::max(batch * nkv, 1));
    const int by_len = (int)ceil_div((size_t)std::max(max_len, 1), 64);
    return std::max(min_splits, std::max(1, std::min(target, by_len)));
}

size_t attention_partials_bytes(const AttnParams& p) {
    const int G = p.nkv > 0 ? p.nh / p.nkv : 1;
    return (size_t)p.batch * p.nkv * p.splits * G * (p.head_dim + 2) * sizeof(float);
}

int launch_attention_decode(hipStream_t s, const AttnParams& p) {
    return launch_any(s, p, 0, (size_t)p.max_seq_len * p.nkv * p.head_dim);
}

// Prefill: token t of the chunk is batch entry t with length pos0 + t + 1 over the shared cache.
int launch_attention_prefill(hipStream_t s, AttnParams p, int pos0, int tokens) {
    p.batch = tokens;
    p.seq_len = pos0 + 1;
    p.seq_len_device = nullptr;
    return launch_any(s, p, 1, 0);
}

}  // namespace l0h
