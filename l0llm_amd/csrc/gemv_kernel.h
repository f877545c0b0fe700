// Weight-streaming GEMV kernel template for gfx950 (decode, M = 1 .. 8 activation rows), shared
// by the per-weight-type translation units gemv_i8.hip, gemv_f16.hip, gemv_bf16.hip and
// gemv_f32.hip (compiled in parallel).
//
// Replaces LlmKernelSuite.Gemv / GemvQ8 (call sites LlmMatrix.cs:122-171, :231-241) for the
// weight formats of this path. Weights are [N, K] row-major (HuggingFace [out, in]).
//
// Work: the N rows are cut into row groups of R rows and each row group's K extent into batches
// of 64 * U chunks of 16 bytes. Wave w of the grid walks the items (row group, batch) of row
// groups w, w + W, w + 2W, ... (W waves in the grid) in order; in an item, lane l reads chunk
// batch * 64U + u * 64 + l of each of the R rows, so one wave instruction reads 1 KiB of one
// row. The loads of item i+1 (its R * U weight chunks and the per-row values its epilogue needs)
// are issued before item i is computed. Every load is unconditional: rows past N and chunks past
// K are clamped to the last valid ones, and the activations staged in LDS are zero past K, so a
// clamped chunk adds nothing. The load stream is therefore straight-line and the in-order memory
// counter waits for exactly the item being computed (a conditional load, or a use of a load
// issued after the prefetch, would make that wait cover the prefetched item too).
//
// Activations are staged once per block in LDS as fp32, times the RMSNorm weights when the norm is
// fused (its scale, one scalar per row, multiplies the row sums in the epilogue). Every wave
// issues its activation loads, then the block meets at a barrier before the first weight item is
// requested: a CU's memory pipeline returns data in order, so the activations come back ahead of
// the weight stream and are staged while it is in flight; the staging barrier waits on LDS only,
// never on the weight loads. Dequantisation
// happens in registers (int8: bytes biased by +128 and converted with v_cvt_f32_ubyteN; the bias
// is removed chunk by chunk: the dot product of every 16-byte chunk starts from -128 times the
// sum of its 16 activations, staged in LDS next to them, so the accumulator only ever holds
// sum(q * x) and a large activation mean cannot cancel it; the per-row scale is applied once),
// accumulation is fp32, and the cross-lane sum uses DPP.
#pragma once

#include <cstdlib>

#include "dpp.h"
#include "kernels.h"

namespace l0h {
namespace {

constexpr int kWaves = 4;
constexpr int kBlock = 64 * kWaves;
// Activation tile per block: up to 16384 fp32 values, plus for int8 weights one bias term per
// 16 values (two blocks per CU still fit the 160 KiB of LDS).
constexpr size_t kLdsBudget = 72 * 1024;
constexpr int kMaxRotaryHalf = 128;       // cos/sin table entries per block (rotary_dim <= 256)

// Block-wide sum (all threads of a kBlock block must call it). Returns the sum to all.
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kWaves; i++) t += red[i];
    return t;
}

// Workgroup barrier that orders LDS only: the wave's LDS operations complete, then s_barrier. Unlike
// __syncthreads it does not wait for outstanding global loads, so a weight stream issued before it
// stays in flight.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int WT>
struct WTraits;
template <>
struct WTraits<L0H_I8PC> {
    static constexpr int kElems = 16;
    static constexpr int kBytes = 1;
};
template <>
struct WTraits<L0H_F16> {
    static constexpr int kElems = 8;
    static constexpr int kBytes = 2;
};
template <>
struct WTraits<L0H_BF16> {
    static constexpr int kElems = 8;
    static constexpr int kBytes = 2;
};
template <>
struct WTraits<L0H_F32> {
    static constexpr int kElems = 4;
    static constexpr int kBytes = 4;
};

// acc += dot(chunk, x). For int8 the bytes are biased by +128 and converted with
// v_cvt_f32_ubyteN; the caller starts acc at -128 * sum(x) of the chunk.
template <int WT>
__device__ __forceinline__ void chunk_fma(const uint4& w, const float* x, float& acc) {
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
    if constexpr (WT == L0H_I8PC) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            uint32_t u = d[j] ^ 0x80808080u;
            acc = fmaf((float)(u & 0xffu), x[4 * j + 0], acc);
            acc = fmaf((float)((u >> 8) & 0xffu), x[4 * j + 1], acc);
            acc = fmaf((float)((u >> 16) & 0xffu), x[4 * j + 2], acc);
            acc = fmaf((float)(u >> 24), x[4 * j + 3], acc);
        }
    } else if constexpr (WT == L0H_F16) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            __half2 h = __builtin_bit_cast(__half2, d[j]);
            float2 f = __half22float2(h);
            acc = fmaf(f.x, x[2 * j + 0], acc);
            acc = fmaf(f.y, x[2 * j + 1], acc);
        }
    } else if constexpr (WT == L0H_BF16) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            acc = fmaf(__uint_as_float(d[j] << 16), x[2 * j + 0], acc);
            acc = fmaf(__uint_as_float(d[j] & 0xffff0000u), x[2 * j + 1], acc);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; j++) acc = fmaf(__uint_as_float(d[j]), x[j], acc);
    }
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// acc += dot(int8 chunk, x) with x staged as fp16 (XH): each weight byte becomes an exact fp16
// integer (byte ^ 0x80 placed under the exponent of 1024 by v_perm_b32 is 1152 + q; a packed fp16
// add of -1152 leaves q) and v_dot2_f32_f16 multiplies pairs into the fp32 accumulator (products of
// two fp16 values are exact in fp32). xa / xb: the chunk's 16 activations, 8 per 16 bytes, each 4
// stored as (x0, x2), (x1, x3): the order of the weight bytes that one v_perm_b32 pairs up.
__device__ __forceinline__ float chunk_dot_h(const uint4& w, const uint4& xa, const uint4& xb, float acc) {
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
    const uint32_t xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    const half2_t bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t u = d[j] ^ 0x80808080u;
        const half2_t lo = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, u, 0x04020400u)) + bias;
        const half2_t hi = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, u, 0x04030401u)) + bias;
        acc = __builtin_amdgcn_fdot2(lo, __builtin_bit_cast(half2_t, xv[2 * j]), acc, false);
        acc = __builtin_amdgcn_fdot2(hi, __builtin_bit_cast(half2_t, xv[2 * j + 1]), acc, false);
    }
    return acc;
}

// 8 fp16 activations (x0 .. x7 in two-byte order) rearranged for chunk_dot_h: (x0, x2), (x1, x3),
// (x4, x6), (x5, x7).
__device__ __forceinline__ uint4 pair_halves(const uint4& c) {
    return make_uint4(__builtin_amdgcn_perm(c.y, c.x, 0x05040100u), __builtin_amdgcn_perm(c.y, c.x, 0x07060302u),
                      __builtin_amdgcn_perm(c.w, c.z, 0x05040100u), __builtin_amdgcn_perm(c.w, c.z, 0x07060302u));
}

// The 16 bytes of an activation chunk as fp32 (4 fp32 values or 8 fp16 / bf16 values).
__device__ __forceinline__ int chunk_to_float(const uint4& c, int dt, float* f) {
    const uint32_t d[4] = {c.x, c.y, c.z, c.w};
    if (dt == L0H_F32) {
#pragma unroll
        for (int j = 0; j < 4; j++) f[j] = __uint_as_float(d[j]);
        return 4;
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        if (dt == L0H_F16) {
            float2 t = __half22float2(__builtin_bit_cast(__half2, d[j]));
            f[2 * j] = t.x;
            f[2 * j + 1] = t.y;
        } else {
            f[2 * j] = __uint_as_float(d[j] << 16);
            f[2 * j + 1] = __uint_as_float(d[j] & 0xffff0000u);
        }
    }
    return 8;
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

__device__ __forceinline__ float half_bits(uint32_t b) { return __half2float(__ushort_as_half((uint16_t)b)); }

__device__ __forceinline__ void store_cache(void* cache, int dt, size_t idx, float v) {
    if (dt == L0H_F16)
        static_cast<uint16_t*>(cache)[idx] = __half_as_ushort(__float2half_rn(v));
    else
        static_cast<float*>(cache)[idx] = v;
}

// Epilogue for the RoPE-paired rows (row, row+1) of the fused q|k|v matrix; cs/sn hold
// cos/sin(pos * inv_freq[i]) * scale for this launch's position.
// rope(i, cs, sn) gives cos/sin * scale of rotated pair i.
template <class Rope>
__device__ __forceinline__ void qkv_pair_with(const GemvParams& p, int row, float v0, float v1, int pos, Rope&& rope) {
    const int hd = p.head_dim, rot = p.rotary_dim;
    if (row >= p.q_dim + p.kv_dim) {  // v rows: natural order
        const int off = row - p.q_dim - p.kv_dim;
        size_t base = (size_t)pos * p.kv_dim + off;
        store_cache(p.v_cache, p.cache_dtype, base, v0);
        store_cache(p.v_cache, p.cache_dtype, base + 1, v1);
        return;
    }
    const bool is_q = row < p.q_dim;
    const int off = is_q ? row : row - p.q_dim;
    const int head = off / hd, j = off - head * hd;
    int d0, d1;
    float o0, o1;
    if (j < rot) {
        const int i = j >> 1;
        d0 = i;
        d1 = i + (rot >> 1);
        float cs, sn;
        rope(i, cs, sn);
        o0 = v0 * cs - v1 * sn;
        o1 = v1 * cs + v0 * sn;
    } else {
        d0 = j;
        d1 = j + 1;
        o0 = v0;
        o1 = v1;
    }
    if (is_q) {
        p.q_out[head * hd + d0] = o0;
        p.q_out[head * hd + d1] = o1;
    } else {
        size_t base = (size_t)pos * p.kv_dim + (size_t)head * hd;
        store_cache(p.k_cache, p.cache_dtype, base + d0, o0);
        store_cache(p.k_cache, p.cache_dtype, base + d1, o1);
    }
}

__device__ __forceinline__ void qkv_pair(const GemvParams& p, int row, float v0, float v1, int pos,
                                         const float* cs_tab, const float* sn_tab) {
    qkv_pair_with(p, row, v0, v1, pos, [&](int i, float& cs, float& sn) {
        cs = cs_tab[i];
        sn = sn_tab[i];
    });
}

// Per-row values an item's epilogue needs, loaded with the item's weights. A lane holds the
// values of the rows it finalises: row r0 + r for lane mr * R + r (store / residual), or rows
// r0 + 2j and r0 + 2j + 1 for lane j (SwiGLU and q|k|v pairs). Absent operands are read from a
// valid address and multiplied by 0, so the load count never depends on the arguments.
struct Side {
    uint32_t s0 = 0, s1 = 0;  // fp16 scale bits (int8 weights)
    float b0 = 0.f, b1 = 0.f;  // bias
    float res = 0.f;           // residual
};

template <int WT, int R, int MR, int EPI>
__device__ __forceinline__ Side load_side(const GemvParams& p, int group, int lane, const float* any) {
    Side sd;
    const float has_bias = p.bias ? 1.f : 0.f;
    if constexpr (EPI == EPI_STORE) {
        const int r = lane % R, mr = min(lane / R, MR - 1);
        const int row = min(group * R + r, p.n - 1);
        if constexpr (WT == L0H_I8PC) sd.s0 = p.scales[row];
        sd.b0 = *(p.bias ? p.bias + row : any) * has_bias;
        sd.res = *(p.resid ? p.resid + (size_t)mr * p.n + row : any) * (p.resid ? 1.f : 0.f);
    } else {
        const int j = min(lane, R / 2 - 1);
        const int row = min(group * R + 2 * j, p.n - 2);
        if constexpr (WT == L0H_I8PC) {
            sd.s0 = p.scales[row];
            sd.s1 = p.scales[row + 1];
        }
        sd.b0 = *(p.bias ? p.bias + row : any) * has_bias;
        sd.b1 = *(p.bias ? p.bias + row + 1 : any) * has_bias;
    }
    return sd;
}

// WT weight type, R rows per wave item, U chunks per row per lane in an item, MR activation
// rows, KX 16-byte activation chunks staged per thread (MR == 1), NORM: RMSNorm prologue,
// EPI: EPI_STORE (store or residual, chosen at run time), EPI_SWIGLU or EPI_QKV.
// Sum of v over aligned groups of G lanes (G = 1, 2, 4 or 16), left in every lane of the group.
template <int G>
__device__ __forceinline__ float lane_group_sum(float v) {
    if constexpr (G == 2 || G == 4) v += dpp_src<0xB1, 0xf>(v);  // quad_perm [1,0,3,2]
    if constexpr (G == 4) v += dpp_src<0x4E, 0xf>(v);            // quad_perm [2,3,0,1]
    if constexpr (G == 16) {
        v += dpp_src<0x128, 0xf>(v);  // row_ror:8
        v += dpp_src<0x124, 0xf>(v);  // row_ror:4
        v += dpp_src<0x122, 0xf>(v);  // row_ror:2
        v += dpp_src<0x121, 0xf>(v);  // row_ror:1
    }
    return v;
}

// Issue priority from progress: 3 for the first quarter of a wave's items, then 2, 1 and 0.
__device__ __forceinline__ void progress_priority(int done, int items) {
    const int q = (4 * done) / max(items, 1);
    if (q <= 0)
        __builtin_amdgcn_s_setprio(3);
    else if (q == 1)
        __builtin_amdgcn_s_setprio(2);
    else if (q == 2)
        __builtin_amdgcn_s_setprio(1);
    else
        __builtin_amdgcn_s_setprio(0);
}

// XH (int8 weights, one fp16 activation row, no RMSNorm, store / residual epilogue): the row is
// staged as fp16 in two planes of k_pad / 16 slots of 16 bytes, the first 8 and the last 8
// activations of every weight chunk (pair_halves order), and chunks are computed by chunk_dot_h;
// there are no bias terms. DX (with XH, for launches of one or two row groups a wave): no staging
// and no block barrier; each lane reads the 32 bytes of x under each of its weight chunks with the
// chunk (from L1 / L2: every wave reads the same row), and a clamped chunk past K adds 0. XHW (with
// XH): the row has an fp32 twin (p.x_wide) and a range flag; a launch whose flag is set stages the
// twin as fp32 and computes as the fp32 path does, otherwise it is XH (the LDS holds either tile).
// PRIO (one activation row): each wave steps its instruction-issue priority down with its
// progress (progress_priority).
template <int WT, int R, int U, int MR, int KX, bool NORM, int EPI, bool XH = false, bool DX = false, bool XHW = false,
          bool PRIO = false>
__global__ __launch_bounds__(kBlock) void gemv_nk_kernel(const GemvParams p, int k_pad) {
    static_assert(!XH || (WT == L0H_I8PC && MR == 1 && !NORM && EPI == EPI_STORE), "fp16-row int8 GEMV");
    static_assert(!DX || (XH && !XHW), "direct x reads: the fp16-row int8 GEMV without a twin");
    static_assert(!XHW || XH, "the fp32 twin of an fp16-row int8 GEMV");
    // PRIO: each wave steps its instruction-issue priority down (s_setprio 3 -> 0) as it works
    // through its items, so the waves that started later or fell behind win the SIMD's arbitration
    // and the launch's waves end closer together.
    static_assert(!PRIO || MR == 1, "progress priority: one activation row");
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(3);
    extern __shared__ float4 smem4[];
    float* xs = reinterpret_cast<float*>(smem4);  // [MR, k_pad], zero past K
    uint4* xh = reinterpret_cast<uint4*>(smem4);  // XH: [2, k_pad / 16] slots, zero past K
    // int8: [MR, k_pad / 16] bias terms, -128 * (sum of the 16 activations of each weight chunk)
    float* xc = xs + (size_t)MR * k_pad;
    const int kc_pad = k_pad / 16;
    __shared__ float red[2 * kWaves];
    __shared__ float rope_cs[EPI == EPI_QKV ? kMaxRotaryHalf : 1];
    __shared__ float rope_sn[EPI == EPI_QKV ? kMaxRotaryHalf : 1];
    constexpr int EPC = WTraits<WT>::kElems;
    constexpr int KB = 64 * U;  // chunks per batch
    const int K = p.k, N = p.n;
    const int C = K / EPC;
    const int nb = (C + KB - 1) / KB;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar control flow
    const int W = gridDim.x * kWaves;
    const int ngroups = (N + R - 1) / R;
    const char* wbase = static_cast<const char*>(p.w);
    const size_t row_bytes = (size_t)K * WTraits<WT>::kBytes;
    const float* any = static_cast<const float*>(p.x);

    // DX: xq[u] = the 16 fp16 activations of weight chunk batch * KB + u * 64 + lane (clamped)
    auto load_w = [&](uint4 (&w)[U][R], uint4 (&xq)[DX ? U : 1][2], int group, int batch) {
        const int grp = min(group, ngroups - 1);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint4* rp = reinterpret_cast<const uint4*>(wbase + (size_t)min(grp * R + r, N - 1) * row_bytes);
#pragma unroll
            for (int u = 0; u < U; u++) w[u][r] = ld_nt16(rp + min(batch * KB + u * 64 + lane, C - 1));
        }
        if constexpr (DX) {
            const uint4* xp = static_cast<const uint4*>(p.x);
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int c = min(batch * KB + u * 64 + lane, C - 1);
                xq[u][0] = xp[2 * c];
                xq[u][1] = xp[2 * c + 1];
            }
        }
    };

    // ---- several activation rows: staged before any weight load (not the decode path) ----
    if constexpr (MR > 1) {
#pragma unroll
        for (int mr = 0; mr < MR; mr++) {
            float* dst = xs + (size_t)mr * k_pad;
            for (int i = tid; i < k_pad; i += kBlock) {  // k_pad is a multiple of kBlock
                const float v = i < K ? load_act(p.x, p.x_dtype, (size_t)mr * K + i) : 0.f;
                dst[i] = v;
                if constexpr (WT == L0H_I8PC) {  // the 16 values of chunk i / 16 sit in one DPP row
                    const float cs = lane_group_sum<16>(v);
                    if ((i & 15) == 0) xc[(size_t)mr * kc_pad + (i >> 4)] = -128.0f * cs;
                }
            }
        }
    }

    // ---- one activation row: prologue loads first (x, norm weights, RoPE frequencies) ----
    // A 16-bit row with an fp32 twin (p.x_wide) whose writer flagged a value beyond the 16-bit
    // range is staged from the twin instead; the flag is read alongside the row's loads, so the
    // common case waits for nothing more. The read is unconditional (from x, masked to 0, when there
    // is no twin): a branch here would split the kernel's argument loads into two dependent rounds.
    unsigned wide = 0u;
    if constexpr (MR == 1) {
        const bool twin = p.x_wide != nullptr;
        const unsigned* wf = twin ? p.range_flag : static_cast<const unsigned*>(p.x);
        wide = *wf & (twin ? 0xffffffffu : 0u);
    }
    uint4 xr[KX], nr[NORM ? KX : 1];
    const int xdt = p.x_dtype;
    const int nxc = (int)((size_t)K * dtype_size(xdt) / 16);  // 16-byte chunks of x
    if constexpr (MR == 1 && !DX) {
        const uint4* xp = static_cast<const uint4*>(p.x);
#pragma unroll
        for (int i = 0; i < KX; i++) xr[i] = xp[min(i * kBlock + tid, nxc - 1)];
        if constexpr (NORM) {
            const uint4* np = reinterpret_cast<const uint4*>(p.norm_w);
#pragma unroll
            for (int i = 0; i < KX; i++) nr[i] = np[min(i * kBlock + tid, K / 4 - 1)];
        }
    }
    float inv_f = 0.f;
    int pos = 0;
    if constexpr (EPI == EPI_QKV) {
        inv_f = p.inv_freq[min(tid, p.rotary_dim / 2 - 1)];
        pos = *p.position;
    }

    // ---- first weight item, issued once every wave of the block has issued its activation loads:
    // a CU's memory pipeline returns data in order, so the activations come back ahead of the
    // block's weight stream and are staged while the weights are in flight ----
    if constexpr (!DX) __builtin_amdgcn_s_barrier();
    int g = blockIdx.x * kWaves + wave;
    uint4 wa[U][R], wb[U][R];
    uint4 xqa[DX ? U : 1][2], xqb[DX ? U : 1][2];
    Side sa, sb;
    sa = load_side<WT, R, MR, EPI>(p, min(g, ngroups - 1), lane, any);
    load_w(wa, xqa, g, 0);

    // ---- stage the one activation row (and RMSNorm) in LDS ----
    // RMSNorm: x * w goes to LDS at once; the row's scale 1 / rms(x), one scalar, multiplies the
    // row sums in the epilogue. Each wave leaves the sum of squares of its chunks (x is fp32 here:
    // 4 values per chunk, matching the 4 norm weights) in `red`, and the barrier that publishes the
    // staged row publishes those too, so no block reduction waits before the stream starts.
    float norm_scale = 1.f;
    if constexpr (MR == 1 && !DX) {
        if constexpr (NORM) {
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < KX; i++) {
                float f[8];
                (void)chunk_to_float(xr[i], xdt, f);
                if (i * kBlock + tid < nxc) {
#pragma unroll
                    for (int e = 0; e < 4; e++) ss += f[e] * f[e];
                }
            }
            ss = wave_sum(ss);
            if (lane == 0) red[wave] = ss;
        }
        if (XH && !(XHW && wide)) {
            // chunk idx of x is 8 fp16 activations: half idx & 1 of weight chunk idx >> 1
#pragma unroll
            for (int i = 0; i < KX; i++) {
                const int idx = i * kBlock + tid;
                if (idx < nxc) xh[(idx & 1) * kc_pad + (idx >> 1)] = pair_halves(xr[i]);
            }
        } else if (wide) {
            // the fp32 twin, in groups of 16 values (K % 16 == 0 where a twin is given)
            const float4* xw = reinterpret_cast<const float4*>(p.x_wide);
            for (int g16 = tid; g16 < K / 16; g16 += kBlock) {
                float cs = 0.f;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 v = xw[g16 * 4 + q];
                    *reinterpret_cast<float4*>(xs + g16 * 16 + 4 * q) = v;
                    cs += (v.x + v.y) + (v.z + v.w);
                }
                if constexpr (WT == L0H_I8PC) xc[g16] = -128.0f * cs;
            }
        } else {
#pragma unroll
            for (int i = 0; i < KX; i++) {
                const int idx = i * kBlock + tid;
                float f[8];
                const int n = chunk_to_float(xr[i], xdt, f);
                if constexpr (NORM) {
                    f[0] *= __uint_as_float(nr[i].x);
                    f[1] *= __uint_as_float(nr[i].y);
                    f[2] *= __uint_as_float(nr[i].z);
                    f[3] *= __uint_as_float(nr[i].w);
                }
                if (idx < nxc) {
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        if (e < n) xs[idx * n + e] = f[e];
                }
                if constexpr (WT == L0H_I8PC) {
                    // A weight chunk covers 16 activations: 4 fp32 or 2 16-bit activation chunks, held
                    // by that many adjacent lanes (every lane takes part in the DPP sum).
                    float cs = 0.f;
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        if (e < n) cs += f[e];
                    cs = idx < nxc ? cs : 0.f;
                    if (xdt == L0H_F32) {
                        cs = lane_group_sum<4>(cs);
                        if (idx < nxc && (idx & 3) == 0) xc[idx >> 2] = -128.0f * cs;
                    } else {
                        cs = lane_group_sum<2>(cs);
                        if (idx < nxc && (idx & 1) == 0) xc[idx >> 1] = -128.0f * cs;
                    }
                }
            }
        }
        if (XH && !(XHW && wide)) {
            for (int c = K / 16 + tid; c < kc_pad; c += kBlock) {
                xh[c] = make_uint4(0u, 0u, 0u, 0u);
                xh[kc_pad + c] = make_uint4(0u, 0u, 0u, 0u);
            }
        } else {
            for (int i = K + tid; i < k_pad; i += kBlock) xs[i] = 0.f;
            if constexpr (WT == L0H_I8PC)
                for (int c = K / 16 + tid; c < kc_pad; c += kBlock) xc[c] = 0.f;
        }
    }
    if constexpr (EPI == EPI_QKV) {
        // cos/sin of this position for every rotated pair, once per block (accurate sincos of
        // the fp32 product pos * inv_freq[i]).
        if (tid < p.rotary_dim / 2) {
            float sn, cs;
            sincosf((float)pos * inv_f, &sn, &cs);
            rope_cs[tid] = cs * p.rope_scale;
            rope_sn[tid] = sn * p.rope_scale;
        }
    }
    if constexpr (!DX) lds_barrier();
    if constexpr (NORM && MR == 1) {  // the waves' sums of squares in a fixed order
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < kWaves; i++) t += red[i];
        norm_scale = rsqrtf(t / (float)K + p.eps);
    }

    // ---- stream: no barrier below this point, waves run independently ----
    float acc[MR][R];
#pragma unroll
    for (int mr = 0; mr < MR; mr++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[mr][r] = 0.f;

    auto compute = [&](const uint4 (&w)[U][R], const uint4 (&xq)[DX ? U : 1][2], int batch) {
        if constexpr (DX) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                const bool in = batch * KB + u * 64 + lane < C;
                const uint4 xa = pair_halves(xq[u][0]), xb = pair_halves(xq[u][1]);
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const float t = chunk_dot_h(w[u][r], xa, xb, 0.f);
                    acc[0][r] += in ? t : 0.f;
                }
            }
            return;
        }
        if (XH && !(XHW && wide)) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int c = batch * KB + u * 64 + lane;  // < nb * KB: x is zero past K
                const uint4 xa = xh[c], xb = xh[kc_pad + c];
#pragma unroll
                for (int r = 0; r < R; r++) acc[0][r] = chunk_dot_h(w[u][r], xa, xb, acc[0][r]);
            }
            return;
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int c = batch * KB + u * 64 + lane;  // < nb * KB: x is zero past K
#pragma unroll
            for (int mr = 0; mr < MR; mr++) {
                float xv[EPC];
                const float4* xp = reinterpret_cast<const float4*>(xs + (size_t)mr * k_pad + (size_t)c * EPC);
#pragma unroll
                for (int q = 0; q < EPC / 4; q++) {
                    float4 t = xp[q];
                    xv[4 * q + 0] = t.x;
                    xv[4 * q + 1] = t.y;
                    xv[4 * q + 2] = t.z;
                    xv[4 * q + 3] = t.w;
                }
                if constexpr (WT == L0H_I8PC) {
                    const float corr = xc[(size_t)mr * kc_pad + c];
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        float t = corr;
                        chunk_fma<WT>(w[u][r], xv, t);
                        acc[mr][r] += t;
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < R; r++) chunk_fma<WT>(w[u][r], xv, acc[mr][r]);
                }
            }
        }
    };

    // Largest greedy key of the values this lane stored (argmax_keys, one activation row).
    unsigned long long best = 0ull;
    // Wave reduction and epilogue of row group `group`; resets the accumulators. No loads.
    auto finish = [&](int group, const Side& sd) {
        const int r0 = group * R;
        float sums[MR][R];
#pragma unroll
        for (int mr = 0; mr < MR; mr++)
#pragma unroll
            for (int r = 0; r < R; r++) {
                sums[mr][r] = wave_sum(acc[mr][r]);
                if constexpr (NORM) sums[mr][r] *= norm_scale;
                acc[mr][r] = 0.f;
            }
        if constexpr (EPI == EPI_STORE) {
#pragma unroll
            for (int mr = 0; mr < MR; mr++)
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const int row = r0 + r;
                    if (lane == mr * R + r && row < N) {
                        float v = sums[mr][r];
                        if constexpr (WT == L0H_I8PC) v *= half_bits(sd.s0);
                        v += sd.b0;
                        if (p.epilogue == EPI_STORE) {
                            store_act(p.y, p.y_dtype, (size_t)mr * N + row, v);
                            if constexpr (MR == 1)
                                if (p.argmax_keys) best = greedy_max(best, greedy_key(v, row));
                        } else {
                            p.resid[(size_t)mr * N + row] = sd.res + v;
                        }
                    }
                }
        } else {
#pragma unroll
            for (int j = 0; j < R / 2; j++) {
                const int row = r0 + 2 * j;
                if (lane == j && row + 1 < N) {
                    float v0 = sums[0][2 * j], v1 = sums[0][2 * j + 1];
                    if constexpr (WT == L0H_I8PC) {
                        v0 *= half_bits(sd.s0);
                        v1 *= half_bits(sd.s1);
                    }
                    v0 += sd.b0;
                    v1 += sd.b1;
                    if constexpr (EPI == EPI_SWIGLU) {
                        const float o = silu(v0) * v1;
                        store_act(p.y, p.y_dtype, (size_t)(row >> 1), o);
                        if (p.y16) {  // the 16-bit copy; a value it cannot hold flags the row
                            store_act_sat(p.y16, L0H_F16, (size_t)(row >> 1), o);
                            if (!(fabsf(o) <= 65504.f)) *p.range_flag = 1u;
                        }
                    } else
                        qkv_pair(p, row, v0, v1, pos, rope_cs, rope_sn);
                }
            }
        }
    };

    // Items of this wave: every batch of row groups g, g + W, ... < ngroups. Each pipeline step
    // issues item i+1 into the other buffer, then computes item i and finishes its row group after
    // its last batch; the last item is computed with nothing issued behind it (no re-read past the
    // end). The branch to the last item comes before any load of its step, so the two paths never
    // merge between a load and its use.
    const int items = g < ngroups ? ((ngroups - 1 - g) / W + 1) * nb : 0;
    int b = 0;  // batch of the current item
    auto advance = [&](int& gg, int& bb) {
        if (++bb == nb) {
            bb = 0;
            gg += W;
        }
    };
    if (items > 0) {
        int i = 0;
        for (;;) {
            if (i + 1 == items) {
                compute(wa, xqa, b);
                finish(g, sa);
                break;
            }
            {
                int gn = g, bn = b;
                advance(gn, bn);
                sb = load_side<WT, R, MR, EPI>(p, gn, lane, any);
                load_w(wb, xqb, gn, bn);
                compute(wa, xqa, b);
                if (b == nb - 1) finish(g, sa);
                g = gn;
                b = bn;
                i++;
                if constexpr (PRIO) progress_priority(i, items);
            }
            if (i + 1 == items) {
                compute(wb, xqb, b);
                finish(g, sb);
                break;
            }
            {
                int gn = g, bn = b;
                advance(gn, bn);
                sa = load_side<WT, R, MR, EPI>(p, gn, lane, any);
                load_w(wa, xqa, gn, bn);
                compute(wb, xqb, b);
                if (b == nb - 1) finish(g, sb);
                g = gn;
                b = bn;
                i++;
                if constexpr (PRIO) progress_priority(i, items);
            }
        }
    }
    if constexpr (MR == 1 && EPI == EPI_STORE) {
        if (p.argmax_keys) {  // every wave of the grid writes its key (0 when it stored nothing)
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) best = greedy_max(best, __shfl_xor(best, off, 64));
            if (lane == 0) p.argmax_keys[(size_t)blockIdx.x * kWaves + wave] = best;
        }
    }
}

// Zero-padded activation tile of the fast kernel: K rounded up to whole batches.
template <int WT, int U>
int padded_k(int k) {
    constexpr int EPC = WTraits<WT>::kElems, KB = 64 * U;
    const int nb = (k / EPC + KB - 1) / KB;
    return nb * KB * EPC;
}

// Dynamic LDS of the fast kernel: the activation tile (+ the int8 bias terms, one per 16 values).
template <int WT>
size_t tile_bytes(int mr, int k_pad) {
    const size_t per_row = (size_t)k_pad + (WT == L0H_I8PC ? k_pad / 16 : 0);
    return (size_t)mr * per_row * sizeof(float);
}

template <int WT, int R, int U, int MR, int KX, bool NORM, int EPI, bool XH = false, bool DX = false, bool XHW = false,
          bool PRIO = false>
int launch_fast(hipStream_t s, const GemvParams& p) {
    const int k_pad = padded_k<WT, U>(p.k);
    const size_t shmem = DX ? 0 : (XH && !XHW) ? (size_t)k_pad * 2 : tile_bytes<WT>(MR, k_pad);
    if (shmem > kLdsBudget) return fail(L0H_ERR_UNSUPPORTED, "GEMV activation tile exceeds LDS");
    auto kern = gemv_nk_kernel<WT, R, U, MR, KX, NORM, EPI, XH, DX, XHW, PRIO>;
    // The dynamic tile may reach kLdsBudget on top of the static LDS: raise the limit once.
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsBudget);
    if (attr != hipSuccess) return fail(L0H_ERR_DEVICE, std::string("hipFuncSetAttribute: ") + hipGetErrorString(attr));
    const unsigned groups = ceil_div(p.n, R);
    unsigned grid = ceil_div(groups, kWaves);
    if (p.max_blocks > 0) {
        // A persistent grid must be resident in one round: at most as many blocks per CU as the
        // kernel's registers and this launch's LDS allow (queried once per instantiation and
        // tile size).
        static thread_local int occ_shmem = -1, occ_blocks = 0;
        if (occ_shmem != (int)shmem) {
            int nb = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void*>(kern), kBlock, shmem) != hipSuccess)
                nb = 1;
            occ_shmem = (int)shmem;
            occ_blocks = std::max(1, nb);
        }
        // Rows of at most 64 chunks (int8 K <= 1024) take twice the blocks: their items are short
        // and their small LDS tile leaves room. Measured (int8, K = 896, graph replay, cold
        // weights, four blocks per CU against two): 896 -> 151936 28.5 -> 27.3 us, 896 -> 9728 4.23
        // -> 3.84, 896 -> 4864 3.30 -> 3.23, 896 -> 1152 and 896 -> 896 unchanged.
        const int per = MR == 1 && p.k / WTraits<WT>::kElems <= 64 ? 2 * p.max_blocks : p.max_blocks;
        const unsigned cap = std::min<unsigned>((unsigned)per, (unsigned)(occ_blocks * std::max(1, p.compute_units)));
        grid = std::min(grid, cap);
    }
    if (p.argmax_keys && (size_t)grid * kWaves > (size_t)std::max(0, p.argmax_capacity))
        return fail(L0H_ERR_INVALID_OP, "GEMV greedy keys: the launch has more waves than the key buffer holds");
    if (p.launched_waves) *p.launched_waves = (int)(grid * kWaves);
    kern<<<grid, kBlock, shmem, s>>>(p, k_pad);
    return launch_status("gemv_nk");
}

// One activation row: the fused epilogues and the RMSNorm prologue live here.
// L0H_GEMV_XH=0 keeps fp16 activation rows of int8 GEMVs on the fp32 staging (A/B measurements).
inline bool xh_enabled() {
    static const bool on = [] {
        const char* e = std::getenv("L0H_GEMV_XH");
        return !e || std::atoi(e) != 0;
    }();
    return on;
}

// int8 weights against one fp16 activation row without a fused prologue or an fp32 twin: the fp16
// staging and v_dot2 compute (XH).
inline bool use_xh(const GemvParams& p) {
    return p.w_dtype == L0H_I8PC && p.m == 1 && p.x_dtype == L0H_F16 && !p.norm_w && !p.x_wide &&
           (p.epilogue == EPI_STORE || p.epilogue == EPI_RESIDUAL) && xh_enabled();
}

// int8 weights against an fp16 row with an fp32 twin (the decode step's down projection): XH unless
// the twin's range flag is set (XHW). L0H_GEMV_XHW=0 keeps such rows on the fp32 staging.
inline bool use_xhw(const GemvParams& p) {
    static const bool on = [] {
        const char* e = std::getenv("L0H_GEMV_XHW");
        return !e || std::atoi(e) != 0;
    }();
    return on && p.w_dtype == L0H_I8PC && p.m == 1 && p.x_dtype == L0H_F16 && !p.norm_w && p.x_wide &&
           p.range_flag && (p.epilogue == EPI_STORE || p.epilogue == EPI_RESIDUAL) && xh_enabled();
}

// XH launches of rows of at most 64 chunks (K <= 1024) with at most two row groups a wave read x
// with their weight chunks instead of staging it (DX). Measured (graph replay, cold weights, two
// interleaved runs each): 896 -> 4864 3.24 -> 3.08 us, 896 -> 1152 and 896 -> 896 unchanged; longer
// rows lose (4864 -> 896 3.47 -> 3.72 us; the 8B step with DX on its 4096-wide O projection 544.6
// -> 541.1 tokens/s). L0H_GEMV_DX=0 keeps the staging (A/B measurements).
inline bool use_dx(const GemvParams& p, int r) {
    static const bool on = [] {
        const char* e = std::getenv("L0H_GEMV_DX");
        return !e || std::atoi(e) != 0;
    }();
    const long groups = (p.n + r - 1) / r;
    const long blocks = p.max_blocks > 0 ? std::min<long>(p.max_blocks, (groups + kWaves - 1) / kWaves)
                                         : (groups + kWaves - 1) / kWaves;
    return on && p.k / 16 <= 64 && groups <= 2 * blocks * kWaves;
}

template <int WT, int R, int U, int KX, bool PRIO = false>
int dispatch_one(hipStream_t s, const GemvParams& p) {
    if constexpr (WT == L0H_I8PC) {
        if (use_xh(p))
            return use_dx(p, R) ? launch_fast<WT, R, U, 1, 1, false, EPI_STORE, true, true, false, PRIO>(s, p)
                                : launch_fast<WT, R, U, 1, KX, false, EPI_STORE, true, false, false, PRIO>(s, p);
        if (use_xhw(p)) return launch_fast<WT, R, U, 1, KX, false, EPI_STORE, true, false, true, PRIO>(s, p);
    }
    switch (p.epilogue) {
    case EPI_SWIGLU: return launch_fast<WT, R, U, 1, KX, true, EPI_SWIGLU, false, false, false, PRIO>(s, p);
    case EPI_QKV: return launch_fast<WT, R, U, 1, KX, true, EPI_QKV, false, false, false, PRIO>(s, p);
    default:
        return p.norm_w ? launch_fast<WT, R, U, 1, KX, true, EPI_STORE, false, false, false, PRIO>(s, p)
                        : launch_fast<WT, R, U, 1, KX, false, EPI_STORE, false, false, false, PRIO>(s, p);
    }
}

// Activation chunks per thread of a 256-thread block, rounded up to a power of two (<= 16).
int staged_chunks(const GemvParams& p) {
    const size_t chunks = (size_t)p.k * dtype_size(p.x_dtype) / 16;
    const size_t per = (chunks + kBlock - 1) / kBlock;
    int kx = 1;
    while ((size_t)kx < per) kx <<= 1;
    return kx;
}

template <int WT, int R, int U, bool PRIO = false>
int dispatch_mr(hipStream_t s, const GemvParams& p, int mr) {
    if (mr == 1) {
        switch (staged_chunks(p)) {
        case 1: return dispatch_one<WT, R, U, 1, PRIO>(s, p);
        case 2: return dispatch_one<WT, R, U, 2, PRIO>(s, p);
        case 4: return dispatch_one<WT, R, U, 4, PRIO>(s, p);
        case 8: return dispatch_one<WT, R, U, 8, PRIO>(s, p);
        case 16: return dispatch_one<WT, R, U, 16, PRIO>(s, p);
        default: return fail(L0H_ERR_UNSUPPORTED, "GEMV activation row exceeds the LDS tile");
        }
    }
    if (mr == 2) return launch_fast<WT, R, U, 2, 1, false, EPI_STORE>(s, p);
    if (mr == 4) return launch_fast<WT, R, U, 4, 1, false, EPI_STORE>(s, p);
    return launch_fast<WT, R, U, 8, 1, false, EPI_STORE>(s, p);
}

// Rows per wave item (R) and 16-byte chunks per row per lane (U), chosen by the row length: C <= 64
// chunks per row -> 4 rows x 1 chunk per lane (4 KiB of int8 weights an item), C <= 128 -> 4 x 2,
// else 2 x 4 (8 KiB); short rows of a matrix with few rows take 2-row
// items (2 x 1, 2 x 2), or 1-row ones (1 x 1) where the matrix has at most one row per wave, long
// ones 1-row items (1 x 4). Several activation rows use 2 x 4.
template <int WT>
int dispatch_wt(hipStream_t s, const GemvParams& p, int mr) {
    const int C = p.k / WTraits<WT>::kElems;
    // Short rows (at most 128 chunks): the 4-row items below suit long streams (matrices with at
    // least four 8- or 4-row groups per wave of the grid); fewer rows leave most of the grid idle,
    // so those take 2-row items, one item per wave or a few. Measured (int8, K = 896, graph replay,
    // cold weights, 2-row items against 8-row ones): 896 -> 4864 4.30 -> 3.45 us, 896 -> 1152 3.96
    // -> 2.55, 896 -> 9728 5.43 -> 4.45.
    if (mr == 1 && C <= 128) {
        const long waves = (long)(p.max_blocks > 0 ? p.max_blocks : 512) * kWaves;
        const int r_long = C <= 64 ? 8 : 4;
        if (ceil_div(p.n, r_long) < 4 * waves) {
            // At most one row per wave of the grid (plain store or residual epilogue, no fused
            // norm): 1-row items, twice the waves of 2-row items, each waiting on one row. Measured
            // (int8, K = 896, fp16 row, graph replay, cold weights, three interleaved pairs): 896 ->
            // 1152 2.45 -> 2.37 us, 896 -> 896 2.44 -> 2.33 us; with more rows than waves 2-row items
            // stay ahead (896 -> 4864 3.07 against 3.08, 896 -> 9728 3.89 against 4.12).
            if (C <= 64 && p.n <= waves && !p.norm_w && staged_chunks(p) == 1 &&
                (p.epilogue == EPI_STORE || p.epilogue == EPI_RESIDUAL)) {
                if constexpr (WT == L0H_I8PC) {
                    if (use_xh(p))
                        return use_dx(p, 1) ? launch_fast<WT, 1, 1, 1, 1, false, EPI_STORE, true, true>(s, p)
                                            : launch_fast<WT, 1, 1, 1, 1, false, EPI_STORE, true>(s, p);
                    if (use_xhw(p)) return launch_fast<WT, 1, 1, 1, 1, false, EPI_STORE, true, false, true>(s, p);
                }
                return launch_fast<WT, 1, 1, 1, 1, false, EPI_STORE>(s, p);
            }
            if (C <= 64) return dispatch_mr<WT, 2, 1>(s, p, mr);
            return dispatch_mr<WT, 2, 2>(s, p, mr);
        }
    }
    // Long rows with 1-row items, each wave's rows pipelined one behind the other instead of a 2-row
    // item with both rows in flight at once: a plain store with fewer than two rows per wave of the
    // grid, and int8 weights against an fp16 row (XH, XHW; store or residual) with at most two.
    // Measured (graph replay, cold weights): 4864 -> 896 (plain store) int8 5.21 -> 4.59 us, fp16
    // 4.87 -> 4.52 us, 1 x 2 and 1 x 1 items slower; in the 8B int8 decode step (two interleaved runs
    // each) O 4096 -> 4096 5.3-5.7 -> 4.9 us, down 14336 -> 4096 12.2-12.3 -> 11.6-11.7 us, 544.7-
    // 545.1 -> 553.5-554.9 tokens/s. With an fp32 row (staged as fp32: a 1-row item reads twice the
    // LDS bytes per weight byte) the same O and down shapes in the operator sequence of the drop-in
    // path ran 293-296 against 300-303 tokens/s (three interleaved pairs), so they keep 2-row items;
    // so does the 8B lm_head (fused norm; 1-row items 83-90 against 81-83 us, the step unchanged).
    if (mr == 1 && C > 128 && (p.epilogue == EPI_STORE || p.epilogue == EPI_RESIDUAL) && !p.norm_w) {
        const long waves = (long)(p.max_blocks > 0 ? p.max_blocks : 512) * kWaves;
        bool x16 = false;
        if constexpr (WT == L0H_I8PC) x16 = use_xh(p) || use_xhw(p);
        if ((p.epilogue == EPI_STORE && ceil_div(p.n, 2) < waves) || (x16 && ceil_div(p.n, 2) <= waves)) {
            if constexpr (WT == L0H_I8PC) {
                if (use_xh(p)) {
                    switch (staged_chunks(p)) {
                    case 1: return launch_fast<WT, 1, 4, 1, 1, false, EPI_STORE, true>(s, p);
                    case 2: return launch_fast<WT, 1, 4, 1, 2, false, EPI_STORE, true>(s, p);
                    case 4: return launch_fast<WT, 1, 4, 1, 4, false, EPI_STORE, true>(s, p);
                    case 8: return launch_fast<WT, 1, 4, 1, 8, false, EPI_STORE, true>(s, p);
                    default: return fail(L0H_ERR_UNSUPPORTED, "GEMV activation row exceeds the LDS tile");
                    }
                }
                if (use_xhw(p)) {
                    switch (staged_chunks(p)) {
                    case 1: return launch_fast<WT, 1, 4, 1, 1, false, EPI_STORE, true, false, true>(s, p);
                    case 2: return launch_fast<WT, 1, 4, 1, 2, false, EPI_STORE, true, false, true>(s, p);
                    case 4: return launch_fast<WT, 1, 4, 1, 4, false, EPI_STORE, true, false, true>(s, p);
                    case 8: return launch_fast<WT, 1, 4, 1, 8, false, EPI_STORE, true, false, true>(s, p);
                    default: return fail(L0H_ERR_UNSUPPORTED, "GEMV activation row exceeds the LDS tile");
                    }
                }
            }
            switch (staged_chunks(p)) {
            case 1: return launch_fast<WT, 1, 4, 1, 1, false, EPI_STORE>(s, p);
            case 2: return launch_fast<WT, 1, 4, 1, 2, false, EPI_STORE>(s, p);
            case 4: return launch_fast<WT, 1, 4, 1, 4, false, EPI_STORE>(s, p);
            case 8: return launch_fast<WT, 1, 4, 1, 8, false, EPI_STORE>(s, p);
            case 16: return launch_fast<WT, 1, 4, 1, 16, false, EPI_STORE>(s, p);
            default: return fail(L0H_ERR_UNSUPPORTED, "GEMV activation row exceeds the LDS tile");
            }
        }
    }
    // Rows of at most 64 chunks in a tall matrix: 4-row items (90 registers: 4 blocks per CU fit),
    // not 8-row ones (142 registers: 3 blocks per CU). Measured (int8, 896 -> 151936, graph replay,
    // cold weights, two runs each): 8 x 1 items at 3 blocks per CU 27.1 us, 4 x 1 at 4 blocks
    // 24.6 us, 4 x 1 at 5 blocks 25.3 us, 2 x 1 at 6 blocks 24.4-24.6 us, at 8 blocks 25.3 us.
    // These launches also lower each wave's issue priority as it progresses: the later-dispatched
    // blocks of a CU otherwise lose the arbitration to the older waves and end ~4 us after them.
    // Measured (896 -> 151936, graph replay, cold weights, three interleaved pairs): fp16 row 24.62-
    // 24.68 -> 23.79-23.87 us, fp32 row 24.74-24.92 -> 24.32-24.44 us; the 8B shapes showed no
    // change in a timing copy, and in the 8B decode step every wave starting at priority 3 cost
    // 0.7 % (538.6 against 542.2 tokens/s, three interleaved pairs), so they keep the priority flat.
    if (mr == 1 && C <= 64) return dispatch_mr<WT, 4, 1, true>(s, p, mr);
    if (mr == 1 && C <= 128) return dispatch_mr<WT, 4, 2>(s, p, mr);
    return dispatch_mr<WT, 2, 4>(s, p, mr);
}

}  // namespace

// One-row / multi-row dispatch for one weight type (defined in gemv_<type>.hip).
int gemv_dispatch_i8(hipStream_t s, const GemvParams& p, int mr);
int gemv_dispatch_f16(hipStream_t s, const GemvParams& p, int mr);
int gemv_dispatch_bf16(hipStream_t s, const GemvParams& p, int mr);
int gemv_dispatch_f32(hipStream_t s, const GemvParams& p, int mr);

}  // namespace l0h
