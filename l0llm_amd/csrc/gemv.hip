// Weight-streaming GEMV kernels for gfx950 (decode, M = 1 .. 8 activation rows).
//
// Replaces LlmKernelSuite.Gemv / GemvQ8 (call sites LlmMatrix.cs:122-171, :231-241) for the
// BASELINE weight formats. Weights are [N, K] row-major (HuggingFace [out, in]); each wave owns
// R consecutive rows and streams them with 16-byte non-temporal loads, 64 lanes side by side
// along K, so a wave instruction covers 1 KiB of one row. Activations are staged once per block
// in LDS as fp32 (with the RMSNorm prologue applied there when fused), dequantisation happens in
// registers (int8 per-row scale folded in after the reduction), accumulation is fp32, and the
// cross-lane sum uses DPP (quad_perm, row mirrors, row_bcast15/31).
#include <cstdlib>

#include "kernels.h"

namespace l0h {
namespace {

constexpr int kWaves = 4;
constexpr int kBlock = 64 * kWaves;

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_src(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

// Sum over the 64 lanes of a wave, returned to every lane (wave-uniform).
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_src<0xB1, 0xf>(v);   // quad_perm [1,0,3,2]
    v += dpp_src<0x4E, 0xf>(v);   // quad_perm [2,3,0,1]
    v += dpp_src<0x141, 0xf>(v);  // row_half_mirror
    v += dpp_src<0x140, 0xf>(v);  // row_mirror
    v += dpp_src<0x142, 0xa>(v);  // row_bcast15 into rows 1, 3
    v += dpp_src<0x143, 0xc>(v);  // row_bcast31 into rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

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
// v_cvt_f32_ubyteN; the bias is removed after the reduction using sum(x).
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

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

__device__ __forceinline__ void store_cache(void* cache, int dt, size_t idx, float v) {
    if (dt == L0H_F16)
        static_cast<uint16_t*>(cache)[idx] = __half_as_ushort(__float2half_rn(v));
    else
        static_cast<float*>(cache)[idx] = v;
}

constexpr int kMaxRotaryHalf = 128;  // cos/sin table entries per block (rotary_dim <= 256)

// Epilogue for the RoPE-paired rows (r0, r0+1) of the fused q|k|v matrix; cs/sn hold
// cos/sin(pos * inv_freq[i]) * scale for this launch's position.
__device__ __forceinline__ void qkv_pair(const GemvParams& p, int row, float v0, float v1, int pos,
                                         const float* cs_tab, const float* sn_tab) {
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
        const float cs = cs_tab[i], sn = sn_tab[i];
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

// R rows per wave, U chunks in flight per row per lane, MR activation rows, XLDS: x staged in
// LDS, EPI: EPI_STORE (store or residual, chosen at run time), EPI_SWIGLU or EPI_QKV.
template <int WT, int R, int U, int MR, bool XLDS, int EPI>
__global__ __launch_bounds__(kBlock) void gemv_nk_kernel(const GemvParams p) {
    extern __shared__ float4 smem4[];
    float* xs = reinterpret_cast<float*>(smem4);  // [MR, K] when XLDS
    __shared__ float red[kWaves];
    __shared__ float xsum_s[MR];
    __shared__ float rope_cs[EPI == EPI_QKV ? kMaxRotaryHalf : 1];
    __shared__ float rope_sn[EPI == EPI_QKV ? kMaxRotaryHalf : 1];
    int pos = 0;
    constexpr int EPC = WTraits<WT>::kElems;
    const int K = p.k, N = p.n;
    const int C = K / EPC;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // Persistent waves: wave w of block b owns row groups (b * kWaves + w) + i * (all waves).
    const int wave_stride = gridDim.x * kWaves * R;
    int row0 = (blockIdx.x * kWaves + wave) * R;

    auto row_ptr = [&](int row) {
        return reinterpret_cast<const uint4*>(static_cast<const char*>(p.w) +
                                              (size_t)min(row, N - 1) * K * WTraits<WT>::kBytes);
    };
    uint4 wa[U][R], wb[U][R];  // double buffer: item i computes from one while item i+1 loads
    auto load_into = [&](uint4 (&w)[U][R], int r0, int c0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int c = c0 + 64 * u;
#pragma unroll
            for (int r = 0; r < R; r++) w[u][r] = c < C ? ld_nt16(row_ptr(r0 + r) + c) : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    const int nb = (C + 64 * U - 1) / (64 * U);  // batches per row group, the same for every lane
    // The first batch of weight loads goes out before the activations are staged, so the
    // prologue overlaps their HBM latency.
    // Per-row values the epilogue needs (int8 scale, bias, residual), fetched with the row group's
    // first weight batch so the epilogue issues no dependent global load. A lane holds the values
    // of the rows it finalizes: row r0 + r for lane mr * R + r (store / residual), or rows
    // r0 + 2j and r0 + 2j + 1 for lane j (SwiGLU and q|k|v pairs).
    struct Side {
        float s0 = 1.f, s1 = 1.f, b0 = 0.f, b1 = 0.f, res = 0.f;
    };
    auto load_side = [&](int r0) {
        Side sd;
        if constexpr (EPI == EPI_STORE) {
            const int r = lane % R, mr = lane / R;
            if (mr < MR) {
                const int row = min(r0 + r, N - 1);
                if constexpr (WT == L0H_I8PC) sd.s0 = __half2float(__ushort_as_half(p.scales[row]));
                if (p.bias) sd.b0 = p.bias[row];
                if (p.epilogue == EPI_RESIDUAL) sd.res = p.resid[(size_t)mr * N + row];
            }
        } else if (lane < R / 2) {
            const int row = min(r0 + 2 * lane, N - 2);
            if constexpr (WT == L0H_I8PC) {
                sd.s0 = __half2float(__ushort_as_half(p.scales[row]));
                sd.s1 = __half2float(__ushort_as_half(p.scales[row + 1]));
            }
            if (p.bias) {
                sd.b0 = p.bias[row];
                sd.b1 = p.bias[row + 1];
            }
        }
        return sd;
    };
    Side side_cur, side_next;
    if (row0 < N) {
        load_into(wa, row0, lane);
        side_cur = load_side(row0);
    }

    if constexpr (EPI == EPI_QKV) {
        pos = *p.position;
        // cos/sin of this position for every rotated pair, once per block (accurate sincos of
        // the fp32 product pos * inv_freq[i]); published by the staging barrier below.
        for (int i = threadIdx.x; i < p.rotary_dim / 2; i += kBlock) {
            float sn, cs;
            sincosf((float)pos * p.inv_freq[i], &sn, &cs);
            rope_cs[i] = cs * p.rope_scale;
            rope_sn[i] = sn * p.rope_scale;
        }
    }

    // Stage activations (and RMSNorm) in LDS.
    if constexpr (XLDS) {
#pragma unroll
        for (int mr = 0; mr < MR; mr++) {
            float* dst = xs + (size_t)mr * K;
            float ss = 0.f;
            if (p.x_dtype == L0H_F32) {
                const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(p.x) + (size_t)mr * K);
                for (int i = threadIdx.x; i < K / 4; i += kBlock) {
                    float4 v = src[i];
                    reinterpret_cast<float4*>(dst)[i] = v;
                    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                }
            } else {
                for (int i = threadIdx.x; i < K; i += kBlock) {
                    float v = load_act(p.x, p.x_dtype, (size_t)mr * K + i);
                    dst[i] = v;
                    ss += v * v;
                }
            }
            __syncthreads();  // other threads read these LDS elements below
            float scale = 1.f;
            if (p.norm_w) {
                ss = block_sum(ss, red);
                scale = rsqrtf(ss / (float)K + p.eps);
            }
            float xsum = 0.f;
            if (p.norm_w || WT == L0H_I8PC) {
                for (int i = threadIdx.x; i < K; i += kBlock) {
                    float v = dst[i];
                    if (p.norm_w) {
                        v = v * scale * p.norm_w[i];
                        dst[i] = v;
                    }
                    xsum += v;
                }
            }
            if constexpr (WT == L0H_I8PC) {
                xsum = block_sum(xsum, red);
                if (threadIdx.x == 0) xsum_s[mr] = xsum;
            }
        }
        __syncthreads();
    } else {
        if constexpr (WT == L0H_I8PC) {
#pragma unroll
            for (int mr = 0; mr < MR; mr++) {
                const float* src = static_cast<const float*>(p.x) + (size_t)mr * K;
                float xsum = 0.f;
                for (int i = threadIdx.x; i < K; i += kBlock) xsum += src[i];
                xsum = block_sum(xsum, red);
                if (threadIdx.x == 0) xsum_s[mr] = xsum;
            }
            __syncthreads();
        }
    }
    const float* xg = static_cast<const float*>(p.x);
    // Pipelined stream over this wave's (row group, batch) items: the loads of item i+1 are issued
    // before item i is computed, across row-group boundaries, so every HBM round trip overlaps
    // compute. No barrier below this point: waves run independently.
    float acc[MR][R];
#pragma unroll
    for (int mr = 0; mr < MR; mr++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[mr][r] = 0.f;

    auto compute = [&](const uint4 (&w)[U][R], int c0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int c = c0 + 64 * u;
            if (c < C) {
#pragma unroll
                for (int mr = 0; mr < MR; mr++) {
                    float xv[EPC];
                    const float4* xp = reinterpret_cast<const float4*>(
                        (XLDS ? xs : xg) + (size_t)mr * K + (size_t)c * EPC);
#pragma unroll
                    for (int q = 0; q < EPC / 4; q++) {
                        float4 t = xp[q];
                        xv[4 * q + 0] = t.x;
                        xv[4 * q + 1] = t.y;
                        xv[4 * q + 2] = t.z;
                        xv[4 * q + 3] = t.w;
                    }
#pragma unroll
                    for (int r = 0; r < R; r++) chunk_fma<WT>(w[u][r], xv, acc[mr][r]);
                }
            }
        }
    };

    // Wave reduction and epilogue of the row group starting at r0; resets the accumulators.
    auto finish = [&](int r0, const Side& sd) {
        float sums[MR][R];
#pragma unroll
        for (int mr = 0; mr < MR; mr++)
#pragma unroll
            for (int r = 0; r < R; r++) {
                sums[mr][r] = wave_sum(acc[mr][r]);
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
                        if constexpr (WT == L0H_I8PC) v = (v - 128.0f * xsum_s[mr]) * sd.s0;
                        v += sd.b0;
                        if (p.epilogue == EPI_STORE)
                            store_act(p.y, p.y_dtype, (size_t)mr * N + row, v);
                        else
                            p.resid[(size_t)mr * N + row] = sd.res + v;
                    }
                }
        } else {
#pragma unroll
            for (int j = 0; j < R / 2; j++) {
                const int row = r0 + 2 * j;
                if (lane == j && row + 1 < N) {
                    float v0 = sums[0][2 * j], v1 = sums[0][2 * j + 1];
                    if constexpr (WT == L0H_I8PC) {
                        v0 = (v0 - 128.0f * xsum_s[0]) * sd.s0;
                        v1 = (v1 - 128.0f * xsum_s[0]) * sd.s1;
                    }
                    v0 += sd.b0;
                    v1 += sd.b1;
                    if constexpr (EPI == EPI_SWIGLU)
                        store_act(p.y, p.y_dtype, (size_t)(row >> 1), silu(v0) * v1);
                    else
                        qkv_pair(p, row, v0, v1, pos, rope_cs, rope_sn);
                }
            }
        }
    };

    int b = 0;  // batch of the current row group
    auto step = [&](uint4 (&cur)[U][R], uint4 (&nxt)[U][R]) -> bool {
        int n_row0 = row0, n_b = b + 1;
        if (n_b == nb) {
            n_b = 0;
            n_row0 += wave_stride;
        }
        const bool more = n_row0 < N;
        if (more) {
            load_into(nxt, n_row0, lane + 64 * U * n_b);
            if (n_b == 0) side_next = load_side(n_row0);
        }
        compute(cur, lane + 64 * U * b);
        if (b == nb - 1) {
            finish(row0, side_cur);
            side_cur = side_next;
        }
        row0 = n_row0;
        b = n_b;
        return more;
    };
    if (row0 < N) {
        while (step(wa, wb) && step(wb, wa)) {
        }
    }
}

// Any shape: one wave per (activation row, output row), scalar loads. STORE / RESIDUAL only.
__global__ __launch_bounds__(kBlock) void gemv_nk_generic_kernel(const GemvParams p) {
    const int lane = threadIdx.x & 63;
    const size_t task = (size_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (task >= (size_t)p.m * p.n) return;
    const int mr = (int)(task / p.n), row = (int)(task % p.n);
    const int K = p.k;
    float acc = 0.f;
    for (int k = lane; k < K; k += 64) {
        float w;
        size_t idx = (size_t)row * K + k;
        switch (p.w_dtype) {
        case L0H_I8PC: w = (float)static_cast<const int8_t*>(p.w)[idx]; break;
        case L0H_F16: w = __half2float(__ushort_as_half(static_cast<const uint16_t*>(p.w)[idx])); break;
        case L0H_BF16: w = bf16_bits_to_float(static_cast<const uint16_t*>(p.w)[idx]); break;
        default: w = static_cast<const float*>(p.w)[idx]; break;
        }
        acc = fmaf(w, load_act(p.x, p.x_dtype, (size_t)mr * K + k), acc);
    }
    acc = wave_sum(acc);
    if (p.w_dtype == L0H_I8PC) acc *= __half2float(__ushort_as_half(p.scales[row]));
    if (lane == 0) {
        if (p.bias) acc += p.bias[row];
        if (p.epilogue == EPI_RESIDUAL)
            p.resid[(size_t)mr * p.n + row] += acc;
        else
            store_act(p.y, p.y_dtype, (size_t)mr * p.n + row, acc);
    }
}

template <int WT, int R, int U, int MR, bool XLDS, int EPI = EPI_STORE>
int launch_fast(hipStream_t s, const GemvParams& p) {
    const unsigned rows_per_block = kWaves * R;
    unsigned grid = ceil_div(p.n, rows_per_block);
    if (p.max_blocks > 0) grid = std::min<unsigned>(grid, (unsigned)p.max_blocks);
    const size_t shmem = XLDS ? (size_t)MR * p.k * sizeof(float) : 0;
    auto kern = gemv_nk_kernel<WT, R, U, MR, XLDS, EPI>;
    if (shmem > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem);
        if (e != hipSuccess) return fail(L0H_ERR_UNSUPPORTED, "GEMV activation tile exceeds LDS");
    }
    kern<<<grid, kBlock, shmem, s>>>(p);
    return launch_status("gemv_nk");
}

constexpr size_t kLdsBudget = 64 * 1024;

// One activation row with x in LDS: the fused epilogues live here.
template <int WT, int R, int U>
int dispatch_one(hipStream_t s, const GemvParams& p) {
    switch (p.epilogue) {
    case EPI_SWIGLU: return launch_fast<WT, R, U, 1, true, EPI_SWIGLU>(s, p);
    case EPI_QKV: return launch_fast<WT, R, U, 1, true, EPI_QKV>(s, p);
    default: return launch_fast<WT, R, U, 1, true, EPI_STORE>(s, p);
    }
}

template <int WT, int R, int U>
int dispatch_mr(hipStream_t s, const GemvParams& p, int mr) {
    const bool fits = (size_t)mr * p.k * sizeof(float) <= kLdsBudget;
    if (mr == 1) return fits ? dispatch_one<WT, R, U>(s, p) : launch_fast<WT, R, U, 1, false>(s, p);
    if (mr == 2) return fits ? launch_fast<WT, R, U, 2, true>(s, p) : launch_fast<WT, R, U, 2, false>(s, p);
    if (mr == 4) return fits ? launch_fast<WT, R, U, 4, true>(s, p) : launch_fast<WT, R, U, 4, false>(s, p);
    return fits ? launch_fast<WT, R, U, 8, true>(s, p) : launch_fast<WT, R, U, 8, false>(s, p);
}

// Rows per wave (R) and 16-byte chunks in flight per row per lane (U) for the one-row int8
// kernel: R * U loads of 1 KiB per wave are outstanding. L0H_GEMV_RU="RU" selects another
// instantiation (for tuning sweeps); the default is the measured best.
int int8_ru_choice() {
    static const int v = [] {
        const char* e = std::getenv("L0H_GEMV_RU");
        return e ? std::atoi(e) : 0;
    }();
    return v;
}

template <int WT>
int dispatch_wt(hipStream_t s, const GemvParams& p, int mr) {
    if constexpr (WT == L0H_I8PC) {
        if (mr == 1 && (size_t)p.k * sizeof(float) <= kLdsBudget) {
            switch (int8_ru_choice()) {
            case 22: return dispatch_one<WT, 2, 2>(s, p);
            case 42: return dispatch_one<WT, 4, 2>(s, p);
            case 44: return dispatch_one<WT, 4, 4>(s, p);
            case 82: return dispatch_one<WT, 8, 2>(s, p);
            default: break;
            }
        }
    }
    // Rows per wave and chunks in flight, chosen per weight width.
    // (R, U) = (2, 4): 2 rows per wave, 4 x 1 KiB loads per row in flight, double-buffered
    // (the fastest of the measured shapes at the Llama-3.1-8B decode sizes).
    return dispatch_mr<WT, 2, 4>(s, p, mr);
}

}  // namespace

int gemv_max_blocks(int compute_units) {
    // L0H_GEMV_BLOCKS_PER_CU overrides the default (0: one block per row group, no cap).
    static const int per_cu = [] {
        const char* e = std::getenv("L0H_GEMV_BLOCKS_PER_CU");
        const int v = e ? std::atoi(e) : 4;
        return v >= 0 ? v : 4;
    }();
    return per_cu == 0 ? 0 : std::max(1, compute_units) * per_cu;
}

int launch_gemv_nk(hipStream_t s, const GemvParams& p0) {
    const int epc = p0.w_dtype == L0H_I8PC ? 16 : (p0.w_dtype == L0H_F32 ? 4 : 8);
    const bool fused = p0.epilogue == EPI_SWIGLU || p0.epilogue == EPI_QKV || p0.norm_w;
    const bool aligned = p0.k % epc == 0 && ((uintptr_t)p0.w & 15) == 0 &&
                         (p0.x_dtype != L0H_F32 || ((uintptr_t)p0.x & 15) == 0);
    if (p0.n <= 0 || p0.k <= 0 || p0.m <= 0) return fail(L0H_ERR_INVALID_ARG, "GEMV sizes must be positive");
    if (fused && (!aligned || p0.m != 1 || (size_t)p0.k * 4 > kLdsBudget))
        return fail(L0H_ERR_UNSUPPORTED, "fused GEMV needs one row, K a multiple of the load width and K*4 <= 64 KiB");
    if (!aligned || (p0.x_dtype != L0H_F32 && (size_t)p0.k * 4 > kLdsBudget)) {
        if (fused) return fail(L0H_ERR_UNSUPPORTED, "fused GEMV shape not supported");
        GemvParams p = p0;
        const size_t tasks = (size_t)p.m * p.n;
        gemv_nk_generic_kernel<<<ceil_div(tasks, kWaves), kBlock, 0, s>>>(p);
        return launch_status("gemv_nk_generic");
    }
    // Activation rows in groups of 8/4/2/1 (each group reads W once).
    int done = 0;
    while (done < p0.m) {
        const int left = p0.m - done;
        const int mr = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
        GemvParams p = p0;
        p.m = mr;
        const bool need_lds = p.x_dtype != L0H_F32;
        if (need_lds && (size_t)mr * p.k * 4 > kLdsBudget && mr > 1) {
            // activations that must be converted have to fit LDS: take a smaller group
            int smaller = mr;
            while (smaller > 1 && (size_t)smaller * p.k * 4 > kLdsBudget) smaller >>= 1;
            p.m = smaller;
        }
        const size_t xsz = (size_t)dtype_size(p.x_dtype);
        p.x = static_cast<const char*>(p0.x) + (size_t)done * p.k * xsz;
        if (p.y) p.y = static_cast<char*>(p0.y) + (size_t)done * p.n * dtype_size(p.y_dtype);
        if (p.resid) p.resid = p0.resid + (size_t)done * p.n;
        int st;
        switch (p.w_dtype) {
        case L0H_I8PC: st = dispatch_wt<L0H_I8PC>(s, p, p.m); break;
        case L0H_F16: st = dispatch_wt<L0H_F16>(s, p, p.m); break;
        case L0H_BF16: st = dispatch_wt<L0H_BF16>(s, p, p.m); break;
        case L0H_F32: st = dispatch_wt<L0H_F32>(s, p, p.m); break;
        default: return fail(L0H_ERR_INVALID_ARG, "unknown weight dtype");
        }
        if (st) return st;
        done += p.m;
    }
    return L0H_OK;
}

// ---------------------------------------------------------------------------------------------
// Reference [K, N] layout (Gemv.Execute / Gemm.Execute): y[r, n] = sum_k x[r, k] * W[k, n].
// Each thread owns 4 adjacent columns; the 4 waves of a block split K and reduce in LDS.
// ---------------------------------------------------------------------------------------------
namespace {
template <int WT>
__global__ __launch_bounds__(kBlock) void gemv_kn_kernel(int rows, int N, int K, const float* x,
                                                         const void* w, float* y) {
    __shared__ float4 part[kWaves][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = (blockIdx.x * 64 + lane) * 4;
    const int r = blockIdx.y;
    const int kper = (K + kWaves - 1) / kWaves;
    const int k0 = wave * kper, k1 = min(K, k0 + kper);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    const float* xr = x + (size_t)r * K;
    if (col < N) {
        for (int k = k0; k < k1; k++) {
            const float xv = xr[k];
            float wv[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int c = col + j;
                const size_t idx = (size_t)k * N + min(c, N - 1);
                float t = WT == L0H_F16 ? __half2float(__ushort_as_half(static_cast<const uint16_t*>(w)[idx]))
                                        : static_cast<const float*>(w)[idx];
                wv[j] = c < N ? t : 0.f;
            }
            acc.x = fmaf(xv, wv[0], acc.x);
            acc.y = fmaf(xv, wv[1], acc.y);
            acc.z = fmaf(xv, wv[2], acc.z);
            acc.w = fmaf(xv, wv[3], acc.w);
        }
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && col < N) {
        float4 t = part[0][lane];
        for (int i = 1; i < kWaves; i++) {
            t.x += part[i][lane].x;
            t.y += part[i][lane].y;
            t.z += part[i][lane].z;
            t.w += part[i][lane].w;
        }
        float* yr = y + (size_t)r * N;
        const float tv[4] = {t.x, t.y, t.z, t.w};
        for (int j = 0; j < 4; j++)
            if (col + j < N) yr[col + j] = tv[j];
    }
}
}  // namespace

int launch_gemv_kn(hipStream_t s, int rows, int n, int k, const float* x, const void* w,
                   int w_dtype, float* y) {
    if (rows <= 0 || n <= 0 || k <= 0) return fail(L0H_ERR_INVALID_ARG, "sizes must be positive");
    dim3 grid(ceil_div(n, 256), rows);
    if (w_dtype == L0H_F16)
        gemv_kn_kernel<L0H_F16><<<grid, kBlock, 0, s>>>(rows, n, k, x, w, y);
    else if (w_dtype == L0H_F32)
        gemv_kn_kernel<L0H_F32><<<grid, kBlock, 0, s>>>(rows, n, k, x, w, y);
    else
        return fail(L0H_ERR_INVALID_ARG, "Gemv.Execute weights are F32 or F16");
    return launch_status("gemv_kn");
}

}  // namespace l0h
