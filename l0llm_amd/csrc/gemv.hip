// Weight-streaming GEMV entry (launch_gemv_nk): shape checks, the fallback kernel for shapes the
// fast kernel does not take, and the split of activation rows into groups; the fast kernel is
// in gemv_kernel.h. Also the reference-layout [K, N] GEMV (Gemv.Execute / Gemm.Execute).
#include "gemv_kernel.h"

namespace l0h {
namespace {

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

}  // namespace

int gemv_max_blocks(int compute_units, int per_cu) {
    // L0H_GEMV_BLOCKS_PER_CU overrides every launch's value (tuning; 0: one block per 4 row
    // groups, no cap).
    static const int env = [] {
        const char* e = std::getenv("L0H_GEMV_BLOCKS_PER_CU");
        const int v = e ? std::atoi(e) : -1;
        return v >= 0 ? v : -1;
    }();
    const int n = env >= 0 ? env : per_cu;
    return n == 0 ? 0 : std::max(1, compute_units) * n;
}

int launch_gemv_nk(hipStream_t s, const GemvParams& p0) {
    if (p0.n <= 0 || p0.k <= 0 || p0.m <= 0) return fail(L0H_ERR_INVALID_ARG, "GEMV sizes must be positive");
    const int epc = p0.w_dtype == L0H_I8PC ? 16 : (p0.w_dtype == L0H_F32 ? 4 : 8);
    const int xsize = dtype_size(p0.x_dtype);
    const bool fused = p0.epilogue == EPI_SWIGLU || p0.epilogue == EPI_QKV || p0.norm_w;
    // Fast path: whole 16-byte weight chunks, aligned rows, and activation rows that fit the
    // zero-padded LDS tile (padding up to 64 * 4 chunks of the weight row).
    const size_t k_pad_max = (size_t)((p0.k / epc + 255) / 256) * 256 * epc;
    const bool aligned = p0.k % epc == 0 && ((uintptr_t)p0.w & 15) == 0 && ((uintptr_t)p0.x & 15) == 0 &&
                         ((uintptr_t)p0.norm_w & 15) == 0 && ((size_t)p0.k * xsize) % 16 == 0;
    const bool pairs = p0.epilogue == EPI_SWIGLU || p0.epilogue == EPI_QKV;
    if (pairs && p0.n % 2) return fail(L0H_ERR_INVALID_ARG, "paired-row epilogues need an even row count");
    const bool fits = k_pad_max * sizeof(float) <= kLdsBudget;
    if (fused) {
        if (!aligned || !fits || p0.m != 1 || p0.x_dtype != L0H_F32 || (p0.epilogue != EPI_STORE && !p0.norm_w) ||
            (p0.epilogue == EPI_QKV && (p0.rotary_dim > 2 * kMaxRotaryHalf || p0.rotary_dim < 2)))
            return fail(L0H_ERR_UNSUPPORTED,
                        "fused GEMV needs one fp32 activation row with the RMSNorm prologue, K a multiple of the "
                        "load width and a zero-padded row of at most 64 KiB");
    }
    if (!aligned || !fits) {
        if (fused) return fail(L0H_ERR_UNSUPPORTED, "fused GEMV shape not supported");
        GemvParams p = p0;
        const size_t tasks = (size_t)p.m * p.n;
        gemv_nk_generic_kernel<<<ceil_div(tasks, kWaves), kBlock, 0, s>>>(p);
        return launch_status("gemv_nk_generic");
    }
    // Activation rows in groups of 8/4/2/1 (each group reads W once), as many as fit the tile.
    int done = 0;
    while (done < p0.m) {
        const int left = p0.m - done;
        int mr = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
        while (mr > 1 && (size_t)mr * k_pad_max * sizeof(float) > kLdsBudget) mr >>= 1;
        GemvParams p = p0;
        p.m = mr;
        p.x = static_cast<const char*>(p0.x) + (size_t)done * p.k * xsize;
        if (p.y) p.y = static_cast<char*>(p0.y) + (size_t)done * p.n * dtype_size(p.y_dtype);
        if (p.resid) p.resid = p0.resid + (size_t)done * p.n;
        int st;
        switch (p.w_dtype) {
        case L0H_I8PC: st = gemv_dispatch_i8(s, p, mr); break;
        case L0H_F16: st = gemv_dispatch_f16(s, p, mr); break;
        case L0H_BF16: st = gemv_dispatch_bf16(s, p, mr); break;
        case L0H_F32: st = gemv_dispatch_f32(s, p, mr); break;
        default: return fail(L0H_ERR_INVALID_ARG, "unknown weight dtype");
        }
        if (st) return st;
        done += mr;
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
