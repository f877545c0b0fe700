// Prefill GEMM on gfx950 MFMA: Y[M, N] = X[M, K] * W[N, K]^T, fp16 or bf16 operands, fp32
// accumulation (the role of LlmMatrix.ProjectRows, LlmMatrix.cs:149-171, for M >= 64).
//
// Both operands are K-contiguous, which is the layout v_mfma_f32_16x16x32_{bf16,f16} wants:
// lane l holds A[l % 16][8 (l / 16) .. +7] and B[8 (l / 16) .. +7][l % 16] and receives
// D[4 (l / 16) + r][l % 16], r < 4. A block of 4 waves (2 x 2) computes a BM x BN tile; tiles
// of BM x 64 and BN x 64 are staged in LDS (rows padded by 16 bytes against bank conflicts),
// double-buffered so the next tile's global loads overlap the current tile's MFMAs. Small-M
// shapes split K across blocks into fp32 partials that a second pass sums.
#include "kernels.h"

namespace l0h {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;

constexpr int BK = 64;
constexpr int kPad = 8;  // elements of padding per LDS row
constexpr int kLds = BK + kPad;

template <int DT>
__device__ __forceinline__ f32x4 mfma(const uint4& a, const uint4& b, f32x4 c) {
    if constexpr (DT == L0H_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// BM x BN block tile, 2 x 2 waves, each (BM/2) x (BN/2) = TM x TN MFMA tiles.
template <int DT, int BM, int BN>
__global__ __launch_bounds__(256) void gemm_nk_kernel(int M, int N, int K, int k_per_split,
                                                      const uint16_t* __restrict__ X,
                                                      const uint16_t* __restrict__ W, void* Y,
                                                      int y_dtype, float* partial) {
    constexpr int TM = BM / 32, TN = BN / 32;
    constexpr int A_CHUNKS = BM * BK / 8 / 256;  // 16-byte chunks per thread per tile
    constexpr int B_CHUNKS = BN * BK / 8 / 256;
    __shared__ __attribute__((aligned(16))) uint16_t sa[2][BM * kLds];
    __shared__ __attribute__((aligned(16))) uint16_t sb[2][BN * kLds];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int kbeg = blockIdx.z * k_per_split;
    const int kend = min(K, kbeg + k_per_split);
    const int ntiles = (kend - kbeg) / BK;

    uint4 ra[A_CHUNKS], rb[B_CHUNKS];
    auto gload = [&](int kt) {
        const int k0 = kbeg + kt * BK;
#pragma unroll
        for (int c = 0; c < A_CHUNKS; c++) {
            const int idx = tid + c * 256;
            const int r = idx >> 3, kc = (idx & 7) * 8;
            const int row = m0 + r;
            ra[c] = row < M ? *reinterpret_cast<const uint4*>(X + (size_t)row * K + k0 + kc) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int c = 0; c < B_CHUNKS; c++) {
            const int idx = tid + c * 256;
            const int r = idx >> 3, kc = (idx & 7) * 8;
            const int row = n0 + r;
            rb[c] = row < N ? ld_nt16(W + (size_t)row * K + k0 + kc)
                            : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int c = 0; c < A_CHUNKS; c++) {
            const int idx = tid + c * 256;
            const int r = idx >> 3, kc = (idx & 7) * 8;
            *reinterpret_cast<uint4*>(&sa[buf][r * kLds + kc]) = ra[c];
        }
#pragma unroll
        for (int c = 0; c < B_CHUNKS; c++) {
            const int idx = tid + c * 256;
            const int r = idx >> 3, kc = (idx & 7) * 8;
            *reinterpret_cast<uint4*>(&sb[buf][r * kLds + kc]) = rb[c];
        }
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int li = lane & 15, lk = (lane >> 4) * 8;
    if (ntiles > 0) {
        gload(0);
        sstore(0);
        __syncthreads();
        for (int kt = 0; kt < ntiles; kt++) {
            const int buf = kt & 1;
            if (kt + 1 < ntiles) gload(kt + 1);
#pragma unroll
            for (int ks = 0; ks < BK; ks += 32) {
                uint4 af[TM], bf[TN];
#pragma unroll
                for (int i = 0; i < TM; i++)
                    af[i] = *reinterpret_cast<const uint4*>(&sa[buf][(wm * (BM / 2) + i * 16 + li) * kLds + ks + lk]);
#pragma unroll
                for (int j = 0; j < TN; j++)
                    bf[j] = *reinterpret_cast<const uint4*>(&sb[buf][(wn * (BN / 2) + j * 16 + li) * kLds + ks + lk]);
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++) acc[i][j] = mfma<DT>(af[i], bf[j], acc[i][j]);
            }
            if (kt + 1 < ntiles) sstore(buf ^ 1);
            __syncthreads();
        }
    }

    // D[4 (l/16) + r][l % 16] of each 16 x 16 tile.
    const int rq = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < TM; i++) {
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int col = n0 + wn * (BN / 2) + j * 16 + li;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = m0 + wm * (BM / 2) + i * 16 + rq + r;
                if (row < M && col < N) {
                    const float v = acc[i][j][r];
                    if (partial)
                        partial[((size_t)blockIdx.z * M + row) * N + col] = v;
                    else
                        store_act(Y, y_dtype, (size_t)row * N + col, v);
                }
            }
        }
    }
}

__global__ void splitk_reduce_kernel(const float* partial, int splits, size_t mn, void* Y, int y_dtype) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= mn) return;
    float s = 0.f;
    for (int z = 0; z < splits; z++) s += partial[(size_t)z * mn + i];
    store_act(Y, y_dtype, i, s);
}

// Any shape (K not a multiple of 64): one thread per output, fp32 accumulation.
__global__ void gemm_nk_generic_kernel(int dt, int M, int N, int K, const uint16_t* X, const uint16_t* W,
                                       void* Y, int y_dtype) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)M * N) return;
    const int row = (int)(i / N), col = (int)(i % N);
    float acc = 0.f;
    for (int k = 0; k < K; k++) {
        const uint16_t a = X[(size_t)row * K + k], b = W[(size_t)col * K + k];
        const float fa = dt == L0H_BF16 ? bf16_bits_to_float(a) : __half2float(__ushort_as_half(a));
        const float fb = dt == L0H_BF16 ? bf16_bits_to_float(b) : __half2float(__ushort_as_half(b));
        acc = fmaf(fa, fb, acc);
    }
    store_act(Y, y_dtype, i, acc);
}

template <int DT, int BM, int BN>
int launch_tiles(hipStream_t s, int m, int n, int k, const void* x, const void* w, void* y, int y_dtype,
                 int splits, float* ws) {
    const int k_per_split = (k / BK + splits - 1) / splits * BK;
    dim3 grid(ceil_div(n, BN), ceil_div(m, BM), splits);
    gemm_nk_kernel<DT, BM, BN><<<grid, 256, 0, s>>>(m, n, k, k_per_split, static_cast<const uint16_t*>(x),
                                                    static_cast<const uint16_t*>(w), y, y_dtype,
                                                    splits > 1 ? ws : nullptr);
    int st = launch_status("gemm_nk");
    if (st || splits == 1) return st;
    const size_t mn = (size_t)m * n;
    splitk_reduce_kernel<<<ceil_div(mn, 256), 256, 0, s>>>(ws, splits, mn, y, y_dtype);
    return launch_status("gemm splitk reduce");
}

template <int DT>
int dispatch(hipStream_t s, int m, int n, int k, const void* x, const void* w, void* y, int y_dtype,
             float* ws, size_t ws_bytes, int cus) {
    // Tile choice: large M uses 128 x 128; small M 64 x 64 tiles with split-K to fill the CUs.
    if (m >= 256) {
        return launch_tiles<DT, 128, 128>(s, m, n, k, x, w, y, y_dtype, 1, ws);
    }
    const size_t blocks = (size_t)ceil_div(n, 64) * ceil_div(m, 64);
    int splits = 1;
    while (blocks * splits < (size_t)cus * 2 && (k / BK) / (splits * 2) >= 4) splits *= 2;
    while (splits > 1 && (size_t)splits * m * n * sizeof(float) > ws_bytes) splits /= 2;
    return launch_tiles<DT, 64, 64>(s, m, n, k, x, w, y, y_dtype, splits, ws);
}

}  // namespace

size_t gemm_workspace_bytes(int m, int n, int k) {
    if (m >= 256 || k % BK) return 0;
    return (size_t)16 * m * n * sizeof(float);
}

int launch_gemm_nk(hipStream_t s, int dtype, int m, int n, int k, const void* x, const void* w,
                   void* y, int y_dtype, float* ws, size_t ws_bytes, int cus) {
    if (m <= 0 || n <= 0 || k <= 0) return fail(L0H_ERR_INVALID_ARG, "GEMM sizes must be positive");
    if (dtype != L0H_BF16 && dtype != L0H_F16) return fail(L0H_ERR_INVALID_ARG, "GEMM operands are F16 or BF16");
    const bool aligned = k % BK == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0;
    if (!aligned) {
        const size_t mn = (size_t)m * n;
        gemm_nk_generic_kernel<<<ceil_div(mn, 256), 256, 0, s>>>(dtype, m, n, k, static_cast<const uint16_t*>(x),
                                                                 static_cast<const uint16_t*>(w), y, y_dtype);
        return launch_status("gemm_nk_generic");
    }
    return dtype == L0H_BF16 ? dispatch<L0H_BF16>(s, m, n, k, x, w, y, y_dtype, ws, ws_bytes, cus)
                             : dispatch<L0H_F16>(s, m, n, k, x, w, y, y_dtype, ws, ws_bytes, cus);
}

}  // namespace l0h
