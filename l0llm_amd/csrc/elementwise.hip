// Element-wise and small operators of the decode step for gfx950: RMSNorm (with fused
// residual), SwiGLU, residual add, bias add, RoPE, KV-cache store, embedding gather, copy,
// greedy argmax, and the device-side random initialiser used for synthetic weights.
// Reference call sites: LlmDecoderLayer.cs:167-194, :301-322, :411-425; LlmModel.cs:360-398.
#include "kernels.h"

namespace l0h {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ float warp_reduce_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ float block_reduce_sum(float v, float* red) {
    v = warp_reduce_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) t += red[i];
    return t;
}

// RMSNorm.Execute (LlmDecoderLayer.cs:167, :183-184): one block per row.
__global__ __launch_bounds__(kBlock) void rmsnorm_kernel(float* x, const float* residual,
                                                         const float* w, float* out, float eps,
                                                         int n, int add_residual) {
    __shared__ float red[kBlock / 64];
    const size_t row = blockIdx.x;
    float* xr = x + row * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += kBlock) {
        float v = xr[i];
        if (add_residual) {
            v += residual[row * n + i];
            xr[i] = v;
        }
        ss += v * v;
    }
    ss = block_reduce_sum(ss, red);
    const float inv = rsqrtf(ss / (float)n + eps);
    float* o = out + row * n;
    for (int i = threadIdx.x; i < n; i += kBlock) o[i] = xr[i] * inv * w[i];
}

__global__ void swiglu_kernel(float* gate, const float* up, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        float g = gate[i];
        gate[i] = g / (1.0f + __expf(-g)) * up[i];
    }
}

__global__ void add_kernel(float* a, const float* b, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) a[i] += b[i];
}

__global__ void bias_add_kernel(float* x, const float* bias, int n, size_t total) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < total) x[i] += bias[i % n];
}

// RoPE (LlmDecoderLayer.cs:411-425), HF rotate-half pairs (i, i + rot/2). One thread per pair.
__global__ void rope_kernel(float* q, float* k, const int* positions, const float* inv_freq,
                            float theta, int head_dim, int nh, int nkv, float attn_scale,
                            int rotary_dim) {
    const int half = rotary_dim / 2;
    const int t = blockIdx.y;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;  // over (head, pair)
    const int heads = nh + nkv;
    if (idx >= heads * half) return;
    const int head = idx / half, i = idx - head * half;
    float* v = head < nh ? q + ((size_t)t * nh + head) * head_dim
                         : k + ((size_t)t * nkv + (head - nh)) * head_dim;
    const float f = inv_freq ? inv_freq[i] : (float)(1.0 / pow((double)theta, 2.0 * i / head_dim));
    const float angle = (float)positions[t] * f;
    float sn, cs;
    sincosf(angle, &sn, &cs);
    cs *= attn_scale;
    sn *= attn_scale;
    const float x0 = v[i], x1 = v[i + half];
    v[i] = x0 * cs - x1 * sn;
    v[i + half] = x1 * cs + x0 * sn;
}

// KvCacheStore (LlmDecoderLayer.cs:322, :368): slot = position (LlmKvCache.cs:5-8).
__global__ void kv_store_kernel(const float* k, const float* v, void* kc, void* vc, int cache_dtype,
                                const int* pos_device, int pos0, int kv_dim, int tokens) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)kv_dim * tokens) return;
    const int base = pos_device ? *pos_device : pos0;
    const size_t dst = (size_t)base * kv_dim + i;
    if (cache_dtype == L0H_F16) {
        static_cast<uint16_t*>(kc)[dst] = __half_as_ushort(__float2half_rn(k[i]));
        static_cast<uint16_t*>(vc)[dst] = __half_as_ushort(__float2half_rn(v[i]));
    } else {
        static_cast<float*>(kc)[dst] = k[i];
        static_cast<float*>(vc)[dst] = v[i];
    }
}

// Also clears `clear[0 .. nclear)` (the decode step's per-layer range flags: the embedding is the
// step's first kernel).
__global__ void embedding_kernel(const int* ids, const float* table, float* out, int h, size_t n, unsigned* clear,
                                 int nclear) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = table[(size_t)ids[i / h] * h + i % h];
    if (i < (size_t)nclear) clear[i] = 0u;
}

__global__ void copy_kernel(const float* src, float* dst, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

// 16-byte copy for aligned buffers: grid-stride over groups of 4 float4 chunks per thread (four
// loads in flight before the stores), the remaining chunks and the scalar tail (n % 4) after.
__global__ __launch_bounds__(kBlock) void copy16_kernel(const float4* src, float4* dst, size_t chunks,
                                                        const float* src_tail, float* dst_tail, int tail) {
    const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t nthreads = (size_t)gridDim.x * blockDim.x;
    const size_t groups = chunks / (4 * nthreads);
    for (size_t g = 0; g < groups; g++) {
        const size_t base = g * 4 * nthreads + tid;
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = src[base + u * nthreads];
#pragma unroll
        for (int u = 0; u < 4; u++) dst[base + u * nthreads] = v[u];
    }
    for (size_t i = groups * 4 * nthreads + tid; i < chunks; i += nthreads) dst[i] = src[i];
    if (blockIdx.x == 0 && (int)threadIdx.x < tail) dst_tail[threadIdx.x] = src_tail[threadIdx.x];
}

__global__ void fill_kernel(float* dst, float value, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) dst[i] = value;
}

// ---- greedy argmax --------------------------------------------------------------------------
// Keys: greedy_key (larger value first, then the smaller index).

__device__ unsigned long long block_max_key(unsigned long long key, unsigned long long* red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) key = greedy_max(key, __shfl_xor(key, off, 64));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = key;
    __syncthreads();
    unsigned long long t = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) t = greedy_max(t, red[i]);
    return t;
}

constexpr int kArgmaxPerBlock = 4096;

// The sampled index of key `best`, and the device-side feedback of a greedy loop: next token,
// recorded ids, position + 1.
__device__ void write_sample(unsigned long long best, int* sampled, const ArgmaxFeed& feed) {
    const int idx = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffull));
    *sampled = idx;
    if (feed.token) *feed.token = idx;
    if (feed.out_list) {
        const int s = *feed.step;
        if (s >= 0 && s < feed.capacity) feed.out_list[s] = idx;
        *feed.step = s + 1;
    }
    if (feed.position) *feed.position += 1;
}

__global__ __launch_bounds__(kBlock) void argmax_kernel(const float* logits, int vocab, int* sampled,
                                                        unsigned long long* partials,
                                                        unsigned* ticket, ArgmaxFeed feed) {
    __shared__ unsigned long long red[kBlock / 64];
    __shared__ bool last;
    const int begin = blockIdx.x * kArgmaxPerBlock;
    const int end = min(vocab, begin + kArgmaxPerBlock);
    unsigned long long key = 0ull;
    for (int i = begin + threadIdx.x; i < end; i += kBlock) key = greedy_max(key, greedy_key(logits[i], i));
    key = block_max_key(key, red);
    if (threadIdx.x == 0) {
        __hip_atomic_store(&partials[blockIdx.x], key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __threadfence();
        const unsigned t = atomicAdd(ticket, 1u);
        last = (t == gridDim.x - 1);
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    unsigned long long best = 0ull;
    for (int b = threadIdx.x; b < (int)gridDim.x; b += kBlock)
        best = greedy_max(best, __hip_atomic_load(&partials[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    best = block_max_key(best, red);
    if (threadIdx.x == 0) {
        write_sample(best, sampled, feed);
        *ticket = 0u;  // ready for the next launch (graph replay)
    }
}

// The argmax over per-wave keys that the lm_head GEMV wrote (one block): the largest key, then the
// same outputs and device-side feedback as argmax_kernel.
__global__ __launch_bounds__(kBlock) void argmax_keys_kernel(const unsigned long long* keys, int count, int* sampled,
                                                             ArgmaxFeed feed) {
    __shared__ unsigned long long red[kBlock / 64];
    unsigned long long best = 0ull;
    for (int i = threadIdx.x; i < count; i += kBlock) best = greedy_max(best, keys[i]);
    best = block_max_key(best, red);
    if (threadIdx.x == 0) write_sample(best, sampled, feed);
}

// ---- random initialisation (synthetic weights) ---------------------------------------------
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t rng64(uint64_t seed, uint64_t idx) {
    return mix64(seed * 0x9E3779B97F4A7C15ull + idx * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull);
}

// Box-Muller from two 24-bit uniforms of the counter stream.
__device__ __forceinline__ float rng_normal(uint64_t seed, uint64_t i) {
    const float u1 = (float)((rng64(seed, 2 * i) >> 40) + 1) * 0x1p-24f;  // (0, 1]
    const float u2 = (float)(rng64(seed, 2 * i + 1) >> 40) * 0x1p-24f;    // [0, 1)
    return sqrtf(-2.0f * logf(u1)) * cosf(6.28318530717958647692f * u2);
}

__global__ void init_normal_kernel(void* dst, int dtype, size_t n, uint64_t seed, float stddev) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) store_act(dst, dtype, i, rng_normal(seed, i) * stddev);
}

// One block per row: pass 1 finds max|w|, pass 2 regenerates and quantizes (no staging).
__global__ __launch_bounds__(kBlock) void init_i8pc_kernel(int8_t* q, uint16_t* scales, int k,
                                                           uint64_t seed, float stddev) {
    __shared__ float red[kBlock / 64];
    const size_t row = blockIdx.x;
    const size_t base = row * (size_t)k;
    float amax = 0.f;
    for (int i = threadIdx.x; i < k; i += kBlock) amax = fmaxf(amax, fabsf(rng_normal(seed, base + i) * stddev));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    uint16_t sh = __half_as_ushort(__float2half_rn(amax / 127.0f));
    if ((sh & 0x7fffu) == 0 && amax > 0.f) sh = 0x0001u;  // non-zero row: scale 2^-24 at least
    if ((sh & 0x7fffu) >= 0x7c00u) sh = 0x7bffu;          // and 65504 at most
    const float s = __half2float(__ushort_as_half(sh));
    if (threadIdx.x == 0) scales[row] = sh;
    for (int i = threadIdx.x; i < k; i += kBlock) {
        float v = s > 0.f ? rintf(rng_normal(seed, base + i) * stddev / s) : 0.f;
        v = fminf(127.f, fmaxf(-127.f, v));
        q[base + i] = (int8_t)v;
    }
}

}  // namespace

int launch_rmsnorm(hipStream_t s, float* x, const float* residual, const float* w, float* out,
                   float eps, int n, int rows, int add_residual) {
    if (n <= 0 || rows <= 0) return fail(L0H_ERR_INVALID_ARG, "RMSNorm sizes must be positive");
    rmsnorm_kernel<<<rows, kBlock, 0, s>>>(x, residual, w, out, eps, n, add_residual);
    return launch_status("rmsnorm");
}

int launch_swiglu(hipStream_t s, float* gate, const float* up, int n) {
    if (n <= 0) return L0H_OK;
    swiglu_kernel<<<ceil_div(n, kBlock), kBlock, 0, s>>>(gate, up, n);
    return launch_status("swiglu");
}

int launch_add(hipStream_t s, float* a, const float* b, int n) {
    if (n <= 0) return L0H_OK;
    add_kernel<<<ceil_div(n, kBlock), kBlock, 0, s>>>(a, b, n);
    return launch_status("add");
}

int launch_bias_add(hipStream_t s, float* x, const float* bias, int n, int rows) {
    if (n <= 0 || rows <= 0) return L0H_OK;
    const size_t total = (size_t)n * rows;
    bias_add_kernel<<<ceil_div(total, kBlock), kBlock, 0, s>>>(x, bias, n, total);
    return launch_status("bias_add");
}

int launch_rope(hipStream_t s, float* q, float* k, const int* positions, const float* inv_freq,
                float theta, int head_dim, int nh, int nkv, float attn_scale, int tokens,
                int rotary_dim) {
    if (tokens <= 0) return L0H_OK;
    const int pairs = (nh + nkv) * (rotary_dim / 2);
    dim3 grid(ceil_div(pairs, kBlock), tokens);
    rope_kernel<<<grid, kBlock, 0, s>>>(q, k, positions, inv_freq, theta, head_dim, nh, nkv,
                                        attn_scale, rotary_dim);
    return launch_status("rope");
}

int launch_kv_store(hipStream_t s, const float* k, const float* v, void* kc, void* vc,
                    int cache_dtype, const int* pos_device, int pos0, int kv_dim, int tokens) {
    const size_t n = (size_t)kv_dim * tokens;
    if (n == 0) return L0H_OK;
    kv_store_kernel<<<ceil_div(n, kBlock), kBlock, 0, s>>>(k, v, kc, vc, cache_dtype, pos_device,
                                                           pos0, kv_dim, tokens);
    return launch_status("kv_store");
}

int launch_embedding(hipStream_t s, const int* ids, const float* table, float* out, int h, size_t n, unsigned* clear,
                     int nclear) {
    if (n == 0 && nclear <= 0) return L0H_OK;
    const size_t threads = std::max(n, (size_t)std::max(nclear, 0));
    embedding_kernel<<<ceil_div(threads, kBlock), kBlock, 0, s>>>(ids, table, out, h, n, clear, clear ? nclear : 0);
    return launch_status("embedding");
}

int launch_copy(hipStream_t s, const float* src, float* dst, size_t n) {
    if (n == 0) return L0H_OK;
    if ((((uintptr_t)src | (uintptr_t)dst) & 15) == 0 && n >= 4 * kBlock) {
        const size_t chunks = n / 4;
        const unsigned blocks = (unsigned)std::min<size_t>(ceil_div(chunks, kBlock), 8192);
        copy16_kernel<<<blocks, kBlock, 0, s>>>(reinterpret_cast<const float4*>(src), reinterpret_cast<float4*>(dst),
                                                chunks, src + 4 * chunks, dst + 4 * chunks, (int)(n % 4));
    } else {
        copy_kernel<<<ceil_div(n, kBlock), kBlock, 0, s>>>(src, dst, n);
    }
    return launch_status("copy");
}

int launch_fill(hipStream_t s, float* dst, float value, size_t n) {
    if (n == 0) return L0H_OK;
    const unsigned blocks = (unsigned)std::min<size_t>(ceil_div(n, kBlock), 8192);
    fill_kernel<<<blocks, kBlock, 0, s>>>(dst, value, n);
    return launch_status("fill");
}

int argmax_blocks(int vocab) { return (int)ceil_div((size_t)vocab, kArgmaxPerBlock); }

int launch_argmax(hipStream_t s, const float* logits, int vocab, int* sampled,
                  unsigned long long* partials, unsigned* ticket, const ArgmaxFeed& feed) {
    if (vocab <= 0) return fail(L0H_ERR_INVALID_ARG, "vocab must be positive");
    argmax_kernel<<<argmax_blocks(vocab), kBlock, 0, s>>>(logits, vocab, sampled, partials, ticket, feed);
    return launch_status("argmax");
}

int launch_argmax_keys(hipStream_t s, const unsigned long long* keys, int count, int* sampled, const ArgmaxFeed& feed) {
    if (count <= 0) return fail(L0H_ERR_INVALID_ARG, "argmax key count must be positive");
    argmax_keys_kernel<<<1, kBlock, 0, s>>>(keys, count, sampled, feed);
    return launch_status("argmax keys");
}

int launch_init_normal(hipStream_t s, void* dst, int dtype, size_t count, uint64_t seed, float stddev) {
    if (count == 0) return L0H_OK;
    const unsigned blocks = (unsigned)std::min<size_t>(ceil_div(count, kBlock), 16384);
    init_normal_kernel<<<blocks, kBlock, 0, s>>>(dst, dtype, count, seed, stddev);
    return launch_status("init_normal");
}

int launch_init_normal_i8pc(hipStream_t s, int8_t* q, uint16_t* scales, int n, int k, uint64_t seed,
                            float stddev) {
    if (n <= 0 || k <= 0) return L0H_OK;
    init_i8pc_kernel<<<n, kBlock, 0, s>>>(q, scales, k, seed, stddev);
    return launch_status("init_i8pc");
}

}  // namespace l0h
