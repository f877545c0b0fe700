// Weight-streaming GEMV entry (launch_gemv_nk): shape checks, the fallback kernel for shapes the
// fast kernel does not take, and the split of activation rows into groups; the fast kernel is
// in gemv_kernel.h. Also the reference-layout [K, N] GEMV (Gemv.Execute / Gemm.Execute).
#include "gemv_kernel.h"

namespace l0h {
namespace {

// Any shape: one wave per (activation row, output row), scalar loads. STORE / RESIDUAL only.
__device__ void generic_task(const GemvParams& p, int lane, int mr, int row) {
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

__global__ __launch_bounds__(kBlock) void gemv_nk_generic_kernel(const GemvParams p) {
    if (p.run_flag && ((*p.run_flag != 0u) != (p.run_when_set != 0))) return;  // gated launch
    const int lane = threadIdx.x & 63;
    // one wave per (activation row, output) task, grid-stride over the tasks
    for (size_t task = (size_t)blockIdx.x * kWaves + (threadIdx.x >> 6); task < (size_t)p.m * p.n;
         task += (size_t)gridDim.x * kWaves)
        generic_task(p, lane, (int)(task / p.n), (int)(task % p.n));
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
    // Per activation row: the fp32 tile, plus one int8 bias term per 16 values.
    const size_t row_tile = (k_pad_max + (p0.w_dtype == L0H_I8PC ? k_pad_max / 16 : 0)) * sizeof(float);
    const bool fits = row_tile <= kLdsBudget;
    if (p0.y16 && (!p0.range_flag || p0.epilogue != EPI_SWIGLU))
        return fail(L0H_ERR_INVALID_ARG, "a 16-bit copy of the output is written by the SwiGLU epilogue, with its range flag");
    if (p0.x_wide) {  // a 16-bit row with an fp32 twin: the fast kernel chooses between them
        if (!p0.range_flag || p0.norm_w || fused || p0.m != 1 || p0.x_dtype == L0H_F32)
            return fail(L0H_ERR_INVALID_ARG, "an fp32 twin row needs its range flag, one 16-bit row and no fused epilogue");
        if (!aligned || !fits || p0.k % 16 || ((uintptr_t)p0.x_wide & 15)) {  // other kernels read the twin itself
            GemvParams p = p0;
            p.x = p0.x_wide;
            p.x_dtype = L0H_F32;
            p.x_wide = nullptr;
            p.range_flag = nullptr;
            return launch_gemv_nk(s, p);
        }
    }
    if (fused) {
        if (!aligned || !fits || p0.m != 1 || p0.x_dtype != L0H_F32 || (p0.epilogue != EPI_STORE && !p0.norm_w) ||
            (p0.epilogue == EPI_QKV && (p0.rotary_dim > 2 * kMaxRotaryHalf || p0.rotary_dim < 2)))
            return fail(L0H_ERR_UNSUPPORTED,
                        "fused GEMV needs one fp32 activation row with the RMSNorm prologue, K a multiple of the "
                        "load width and a zero-padded row that fits the LDS tile (16384 values)");
    }
    if (p0.argmax_keys && (p0.m != 1 || p0.epilogue != EPI_STORE))
        return fail(L0H_ERR_INVALID_ARG, "per-wave argmax keys need one activation row and the store epilogue");
    // A gated launch (a rarely taken fallback decided on the device) is one launch of the generic
    // kernel over every activation row: the fast path below issues one launch per group of rows.
    if (!aligned || !fits || p0.run_flag) {
        if (fused || p0.argmax_keys) return fail(L0H_ERR_UNSUPPORTED, "fused GEMV shape not supported");
        GemvParams p = p0;
        const size_t tasks = (size_t)p.m * p.n;
        // at most 8 blocks per CU, striding over the tasks (a gated launch that does nothing
        // dispatches no more than that)
        const size_t cap = (size_t)8 * std::max(1, p.compute_units > 0 ? p.compute_units : 256);
        gemv_nk_generic_kernel<<<(unsigned)std::min<size_t>(ceil_div(tasks, kWaves), cap), kBlock, 0, s>>>(p);
        return launch_status("gemv_nk_generic");
    }
    // Activation rows in groups of 8/4/2/1 (each group reads W once), as many as fit the tile.
    int done = 0;
    while (done < p0.m) {
        const int left = p0.m - done;
        int mr = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
        while (mr > 1 && (size_t)mr * row_tile > kLdsBudget) mr >>= 1;
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
// Reference [K, N] layout (Gemv.Execute / ExecuteRows, Gemm.Execute): y[r, n] = sum_k x[r, k] W[k, n].
//
// Fast path (N a multiple of the load width, 16-byte aligned W): lane l of a wave reads the
// 16-byte chunk t * 64 + l of a weight row, i.e. EPC = 8 fp16 (4 fp32) adjacent columns, so one
// wave instruction streams 1 KiB of one row. Block (column tile t, K slice s) covers 64 chunks
// of columns and the rows [s * KS, (s + 1) * KS); its 4 waves take every fourth row of the slice,
// with U rows in flight per lane. The slice's activations are staged in LDS (zero past K; the
// clamped rows there add nothing), the waves reduce through LDS in a fixed order, and a split K
// leaves per-slice partials [S, rows, N] that a second kernel sums in slice order. The slice
// count fills the GPU: about two blocks per CU over the column tiles.
// ---------------------------------------------------------------------------------------------
namespace {
constexpr int kKnUnroll = 8;           // weight rows in flight per lane
constexpr int kKnLds = 160 * 1024;  // LDS bytes a block may use

template <int WT, int MR>
__global__ __launch_bounds__(kBlock) void gemv_kn_tile_kernel(int N, int K, int ks, const float* x, const void* w,
                                                              float* out) {
    constexpr int EPC = WT == L0H_F16 ? 8 : 4;
    extern __shared__ float kn_smem[];
    float* xs = kn_smem;                   // [MR][ks]
    float* red = kn_smem + (size_t)MR * ks;  // [kWaves][MR * EPC][64]
    const int CN = N / EPC;
    const int t = blockIdx.x, sl = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int k0 = sl * ks;
    const int c = t * 64 + lane;
    const int cc = min(c, CN - 1);
    for (int i = threadIdx.x; i < MR * ks; i += kBlock) {
        const int mr = i / ks, kk = k0 + (i - mr * ks);
        xs[i] = kk < K ? x[(size_t)mr * K + kk] : 0.f;
    }
    __syncthreads();
    float acc[MR][EPC];
#pragma unroll
    for (int mr = 0; mr < MR; mr++)
#pragma unroll
        for (int e = 0; e < EPC; e++) acc[mr][e] = 0.f;
    const uint4* wp = static_cast<const uint4*>(w) + cc;
    const int rows = ks / kWaves;  // rows of this wave (ks is a multiple of kWaves * kKnUnroll)
    for (int j0 = 0; j0 < rows; j0 += kKnUnroll) {
        uint4 wv[kKnUnroll];
#pragma unroll
        for (int u = 0; u < kKnUnroll; u++) {
            const int kk = min(k0 + (j0 + u) * kWaves + wave, K - 1);
            wv[u] = ld_nt16(wp + (size_t)kk * CN);
        }
#pragma unroll
        for (int u = 0; u < kKnUnroll; u++) {
            float f[EPC];
            const uint32_t d[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
            if constexpr (WT == L0H_F16) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float2 h = __half22float2(__builtin_bit_cast(__half2, d[q]));
                    f[2 * q] = h.x;
                    f[2 * q + 1] = h.y;
                }
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++) f[q] = __uint_as_float(d[q]);
            }
            const int j = (j0 + u) * kWaves + wave;
#pragma unroll
            for (int mr = 0; mr < MR; mr++) {
                const float xv = xs[mr * ks + j];
#pragma unroll
                for (int e = 0; e < EPC; e++) acc[mr][e] = fmaf(xv, f[e], acc[mr][e]);
            }
        }
    }
#pragma unroll
    for (int mr = 0; mr < MR; mr++)
#pragma unroll
        for (int e = 0; e < EPC; e++) red[((size_t)wave * MR * EPC + mr * EPC + e) * 64 + lane] = acc[mr][e];
    __syncthreads();
    // Fixed-order sum of the four waves; thread i finishes (row, column) pairs i, i + 256, ...
    for (int i = threadIdx.x; i < MR * EPC * 64; i += kBlock) {
        const int l = i & 63, me = i >> 6, mr = me / EPC, e = me - mr * EPC;
        float v = red[(size_t)me * 64 + l];
#pragma unroll
        for (int ww = 1; ww < kWaves; ww++) v += red[((size_t)ww * MR * EPC + me) * 64 + l];
        const int col = (t * 64 + l) * EPC + e;
        if (t * 64 + l < CN) out[((size_t)sl * MR + mr) * N + col] = v;
    }
}

// y[r, n] = sum over slices of part[s, r, n] in a fixed order: four running sums over the slices
// s = 4 j + q (their loads independent, so four are in flight), added as (s0 + s1) + (s2 + s3).
__global__ void kn_slice_sum_kernel(const float* part, float* y, int splits, size_t count) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    int s = 0;
    for (; s + 4 <= splits; s += 4) {
#pragma unroll
        for (int q = 0; q < 4; q++) a[q] += part[(size_t)(s + q) * count + i];
    }
    for (int q = 0; s + q < splits; q++) a[q] += part[(size_t)(s + q) * count + i];
    y[i] = (a[0] + a[1]) + (a[2] + a[3]);
}

// One activation row in narrow column tiles: block (tile t of 8 chunks = 128 bytes of every weight
// row, K slice s). Lane l reads chunk l % 8 of row l / 8 of each group of 8 rows, so one wave
// instruction covers 8 whole 128-byte row segments and the block's NW waves take rows 8 * NW apart.
// The slice's rows go in batches of kNarrowU per lane, the next batch requested before the current
// one is computed; x comes from LDS (zero past the slice, where the clamped rows add nothing). The
// 8 lanes of a chunk are summed over DPP and row swaps, the waves through LDS in a fixed order.
constexpr int kNarrowU = 8;      // row groups per lane per batch
constexpr int kNarrowLds = kKnLds - 16384;  // dynamic LDS for x (the wave reduction is static)

template <int WT, int NW>
__global__ __launch_bounds__(NW * 64) void gemv_kn_narrow_kernel(int N, int K, int ks, const float* x, const void* w,
                                                                 float* out) {
    constexpr int EPC = WT == L0H_F16 ? 8 : 4;  // columns per 16-byte chunk
    constexpr int TC = 8 * EPC;                 // columns per tile
    constexpr int kNarrowRPS = 8 * NW;          // rows per block step (8 per wave instruction)
    extern __shared__ float kn_smem[];
    float* xs = kn_smem;                         // [steps rounded to batches * kNarrowRPS]
    __shared__ float red[NW][TC];
    const int CN = N / EPC;
    const int t = blockIdx.x, sl = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane >> 3, cj = lane & 7;
    const int k0 = sl * ks, k1 = min(K, k0 + ks);
    const int steps = (k1 - k0 + kNarrowRPS - 1) / kNarrowRPS;
    const int batches = (steps + kNarrowU - 1) / kNarrowU;
    const int nx = batches * kNarrowU * kNarrowRPS;
    for (int i = threadIdx.x; i < nx; i += NW * 64) xs[i] = k0 + i < k1 ? x[k0 + i] : 0.f;
    __syncthreads();
    const uint4* wp = static_cast<const uint4*>(w) + min(t * 8 + cj, CN - 1);
    float acc[EPC];
#pragma unroll
    for (int e = 0; e < EPC; e++) acc[e] = 0.f;
    auto load = [&](uint4 (&v)[kNarrowU], int b) {
#pragma unroll
        for (int u = 0; u < kNarrowU; u++) {
            const int row = k0 + (b * kNarrowU + u) * kNarrowRPS + wave * 8 + r;
            v[u] = ld_nt16(wp + (size_t)min(row, K - 1) * CN);
        }
    };
    auto compute = [&](const uint4 (&v)[kNarrowU], int b) {
#pragma unroll
        for (int u = 0; u < kNarrowU; u++) {
            const float xv = xs[(b * kNarrowU + u) * kNarrowRPS + wave * 8 + r];
            const uint32_t d[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
            if constexpr (WT == L0H_F16) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float2 h = __half22float2(__builtin_bit_cast(__half2, d[q]));
                    acc[2 * q] = fmaf(xv, h.x, acc[2 * q]);
                    acc[2 * q + 1] = fmaf(xv, h.y, acc[2 * q + 1]);
                }
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++) acc[q] = fmaf(xv, __uint_as_float(d[q]), acc[q]);
            }
        }
    };
    // Batch b: request batch b + 1, compute batch b (the last one with nothing behind it).
    uint4 va[kNarrowU], vb[kNarrowU];
    if (batches > 0) {
        load(va, 0);
        int b = 0;
        for (;;) {
            if (b + 1 == batches) {
                compute(va, b);
                break;
            }
            load(vb, b + 1);
            compute(va, b);
            if (++b + 1 == batches) {
                compute(vb, b);
                break;
            }
            load(va, b + 1);
            compute(vb, b);
            b++;
        }
    }
#pragma unroll
    for (int e = 0; e < EPC; e++) acc[e] = slot_reduce<8, false>(acc[e]);  // the 8 row lanes of chunk cj
    if (r == 0) {
#pragma unroll
        for (int e = 0; e < EPC; e++) red[wave][cj * EPC + e] = acc[e];
    }
    __syncthreads();
    if (threadIdx.x < TC) {
        const int c = t * TC + threadIdx.x;
        float v = red[0][threadIdx.x];
#pragma unroll
        for (int ww = 1; ww < NW; ww++) v += red[ww][threadIdx.x];
        if (c < N) out[(size_t)sl * N + c] = v;
    }
}

// Any shape (N not a multiple of the load width, unaligned buffers): each thread owns 4
// adjacent columns, the 4 waves of a block split K and reduce in LDS.
template <int WT>
__global__ __launch_bounds__(kBlock) void gemv_kn_generic_kernel(int N, int K, const float* x, const void* w,
                                                                 float* y) {
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

template <int WT, int MR>
int launch_kn_tile(hipStream_t s, int n, int k, int ks, int splits, const float* x, const void* w, float* out) {
    constexpr int EPC = WT == L0H_F16 ? 8 : 4;
    const unsigned tiles = ceil_div((size_t)(n / EPC), 64);
    const size_t shmem = ((size_t)MR * ks + (size_t)kWaves * MR * EPC * 64) * sizeof(float);
    auto kern = gemv_kn_tile_kernel<WT, MR>;
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, kKnLds);
    if (attr != hipSuccess) return fail(L0H_ERR_DEVICE, std::string("hipFuncSetAttribute: ") + hipGetErrorString(attr));
    kern<<<dim3(tiles, splits), kBlock, shmem, s>>>(n, k, ks, x, w, out);
    return launch_status("gemv_kn_tile");
}

template <int WT, int NW>
int launch_kn_narrow_nw(hipStream_t s, int n, int k, int ks, int splits, const float* x, const void* w, float* out) {
    constexpr int EPC = WT == L0H_F16 ? 8 : 4;
    constexpr int kNarrowRPS = 8 * NW;
    const unsigned tiles = ceil_div((size_t)(n / EPC), 8);
    const int steps = (ks + kNarrowRPS - 1) / kNarrowRPS;
    const size_t shmem = (size_t)((steps + kNarrowU - 1) / kNarrowU) * kNarrowU * kNarrowRPS * sizeof(float);
    if (shmem > (size_t)kNarrowLds) return fail(L0H_ERR_UNSUPPORTED, "GEMV K slice exceeds the LDS tile");
    auto kern = gemv_kn_narrow_kernel<WT, NW>;
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, kNarrowLds);
    if (attr != hipSuccess) return fail(L0H_ERR_DEVICE, std::string("hipFuncSetAttribute: ") + hipGetErrorString(attr));
    kern<<<dim3(tiles, splits), NW * 64, shmem, s>>>(n, k, ks, x, w, out);
    return launch_status("gemv_kn_narrow");
}

template <int WT>
int launch_kn_narrow(hipStream_t s, int nw, int n, int k, int ks, int splits, const float* x, const void* w,
                     float* out) {
    return nw == 16 ? launch_kn_narrow_nw<WT, 16>(s, n, k, ks, splits, x, w, out)
                    : launch_kn_narrow_nw<WT, 4>(s, n, k, ks, splits, x, w, out);
}

template <int WT>
int launch_kn_rows(hipStream_t s, int mr, int n, int k, int ks, int splits, const float* x, const void* w, float* out) {
    switch (mr) {
    case 1: return launch_kn_tile<WT, 1>(s, n, k, ks, splits, x, w, out);
    case 2: return launch_kn_tile<WT, 2>(s, n, k, ks, splits, x, w, out);
    case 4: return launch_kn_tile<WT, 4>(s, n, k, ks, splits, x, w, out);
    default: return launch_kn_tile<WT, 8>(s, n, k, ks, splits, x, w, out);
    }
}
}  // namespace

KnPlan plan_gemv_kn(int rows, int n, int k, int w_dtype, int compute_units, size_t ws_bytes) {
    const int epc = w_dtype == L0H_F16 ? 8 : 4;
    if (rows == 1) {
        // Narrow tiles: no K split from min_tiles tiles up (a K split costs a second launch for the
        // slice sum); else slices of whole batches (at least 256 or 1024 rows) up to about one block
        // per CU.
        KnPlan pl;
        pl.narrow = true;
        const int tiles = (int)ceil_div((size_t)(n / epc), 8);
        static const int nw_env = [] {  // waves per block, 4 or 16 (tuning)
            const char* e = std::getenv("L0H_GEMV_KN_NW");
            return e ? std::atoi(e) : 0;
        }();
        // 16 waves when all of K is one batch of theirs (1024 rows) and the tiles are few: each
        // wave then has one batch to stream. Measured (fp16, graph replay, cold weights): Qwen2.5-0.5B
        // O 896 -> 896 5.6 (split in 3 + slice sum) -> 4.5 us, q|k|v 4.9 -> 4.5, 896 -> 4864 5.4 -> 5.2,
        // gate|up 6.7 -> 6.4; longer K (down 4864 -> 896: 7.4 -> 9.7) and many tiles (lm_head, 2374
        // tiles: 45.3 -> 49.3) stay at 4.
        pl.nw = nw_env == 4 || nw_env == 16 ? nw_env : k <= kNarrowU * 8 * 16 && tiles <= 512 ? 16 : 4;
        const int rps = 8 * pl.nw;
        const int batch_rows = kNarrowU * rps;
        const int max_ks = (kNarrowLds / 4) / batch_rows * batch_rows;  // the slice's x fits the LDS
        static const int min_tiles_env = [] {  // tiles from which no K split is made (tuning)
            const char* e = std::getenv("L0H_GEMV_KN_TILES");
            return e ? std::atoi(e) : 0;
        }();
        // 16 tiles (1024 fp16 columns) measured best on MI355X: Qwen2.5-0.5B q|k|v (18 tiles) 4.9 us
        // unsplit against 5.7 us in slices; 896 -> 4864 (76 tiles) 5.4 against 6.6 us.
        const int min_tiles = min_tiles_env > 0 ? min_tiles_env : 16;
        int splits = tiles >= min_tiles ? 1 : (int)ceil_div((size_t)std::max(compute_units, 1), (size_t)tiles);
        splits = std::min(splits, std::max(1, k / batch_rows));
        splits = std::max(splits, (int)ceil_div((size_t)k, (size_t)max_ks));
        const size_t per_split = (size_t)n * sizeof(float);
        if (splits > 1 && (size_t)splits * per_split > ws_bytes)
            splits = std::max((int)ceil_div((size_t)k, (size_t)max_ks), (int)std::min<size_t>(splits, ws_bytes / per_split));
        pl.ks = (int)ceil_div((size_t)ceil_div((size_t)k, (size_t)std::max(splits, 1)), (size_t)rps) * rps;
        pl.ks = std::min(pl.ks, max_ks);
        pl.splits = (int)ceil_div((size_t)k, (size_t)pl.ks);
        return pl;
    }
    const int tiles = (int)ceil_div((size_t)(n / epc), 64);
    constexpr int step = kWaves * kKnUnroll;  // rows of a slice come in whole unrolled steps
    // About two blocks per CU over the column tiles.
    const int target = (int)ceil_div((size_t)2 * std::max(compute_units, 1), (size_t)std::max(tiles, 1));
    KnPlan pl;
    for (int mr = rows >= 8 ? 8 : rows >= 4 ? 4 : rows >= 2 ? 2 : 1;; mr >>= 1) {
        // The slice's activations and the wave reduction share the block's LDS.
        const int max_ks = ((kKnLds / 4 - kWaves * mr * epc * 64) / mr) / step * step;
        const int min_splits = (int)ceil_div((size_t)k, (size_t)max_ks);
        const size_t per_split = (size_t)mr * n * sizeof(float);
        const int cap = (int)std::min<size_t>(ws_bytes / per_split, 1 << 20);  // slices the workspace holds
        if (min_splits > 1 && min_splits > cap && mr > 1) continue;  // fewer rows per launch
        int splits = std::max(1, std::min(target, (k + step - 1) / step));
        if (splits > 1 && splits > cap) splits = std::max(1, cap);
        splits = std::max(splits, min_splits);
        pl.mr = mr;
        pl.ks = std::min(max_ks, (int)ceil_div((size_t)ceil_div((size_t)k, (size_t)splits), (size_t)step) * step);
        pl.splits = (int)ceil_div((size_t)k, (size_t)pl.ks);
        return pl;
    }
}

size_t gemv_kn_workspace_bytes(const KnPlan& pl, int n) {
    return pl.splits > 1 ? (size_t)pl.splits * pl.mr * n * sizeof(float) : 0;
}

bool gemv_kn_fast(int n, int w_dtype, const void* w, const float* x) {
    const int epc = w_dtype == L0H_F16 ? 8 : 4;
    return n % epc == 0 && ((uintptr_t)w & 15) == 0 && ((uintptr_t)x & 3) == 0;
}

int launch_gemv_kn(hipStream_t s, int rows, int n, int k, const float* x, const void* w, int w_dtype, float* y,
                   float* ws, size_t ws_bytes, int compute_units) {
    if (rows <= 0 || n <= 0 || k <= 0) return fail(L0H_ERR_INVALID_ARG, "sizes must be positive");
    if (w_dtype != L0H_F16 && w_dtype != L0H_F32) return fail(L0H_ERR_INVALID_ARG, "Gemv.Execute weights are F32 or F16");
    if (!gemv_kn_fast(n, w_dtype, w, x)) {
        dim3 grid(ceil_div(n, 256), rows);
        if (w_dtype == L0H_F16)
            gemv_kn_generic_kernel<L0H_F16><<<grid, kBlock, 0, s>>>(n, k, x, w, y);
        else
            gemv_kn_generic_kernel<L0H_F32><<<grid, kBlock, 0, s>>>(n, k, x, w, y);
        return launch_status("gemv_kn_generic");
    }
    for (int done = 0; done < rows;) {
        // Slices beyond what the workspace holds are merged (or fewer rows run per launch).
        const KnPlan pl = plan_gemv_kn(rows - done, n, k, w_dtype, compute_units, ws ? ws_bytes : 0);
        if (gemv_kn_workspace_bytes(pl, n) > (ws ? ws_bytes : 0))
            return fail(L0H_ERR_INVALID_OP, "the split-reduction workspace cannot hold this [K, N] GEMV's partials");
        const float* xr = x + (size_t)done * k;
        float* yr = y + (size_t)done * n;
        float* out = pl.splits > 1 ? ws : yr;
        int st;
        if (pl.narrow)
            st = w_dtype == L0H_F16 ? launch_kn_narrow<L0H_F16>(s, pl.nw, n, k, pl.ks, pl.splits, xr, w, out)
                                    : launch_kn_narrow<L0H_F32>(s, pl.nw, n, k, pl.ks, pl.splits, xr, w, out);
        else
            st = w_dtype == L0H_F16 ? launch_kn_rows<L0H_F16>(s, pl.mr, n, k, pl.ks, pl.splits, xr, w, out)
                                    : launch_kn_rows<L0H_F32>(s, pl.mr, n, k, pl.ks, pl.splits, xr, w, out);
        if (st) return st;
        if (pl.splits > 1) {
            const size_t count = (size_t)pl.mr * n;
            kn_slice_sum_kernel<<<ceil_div(count, 256), 256, 0, s>>>(ws, yr, pl.splits, count);
            if ((st = launch_status("gemv_kn slice sum"))) return st;
        }
        done += pl.mr;
    }
    return L0H_OK;
}

}  // namespace l0h
